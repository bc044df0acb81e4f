// tsp_tiling.hip -- CSR -> tiles on the GPU (the csr2tile conversion of
// src/csr2tile.h:15-379,724-795 moved onto MI355X), bit-exact with the host
// conversion (tilespmm_amd/host/tiles.cpp):
//   1. segmented radix sort (rocPRIM) of every row-block's column indices;
//   2. first-of-run flags + exclusive scan -> the block's sorted distinct
//      columns and their count d;
//   3. ceil(d/BN) tiles per block, exclusive scan -> tile_ptr; tile_colidx is
//      the distinct list cut into BN-wide tiles, padded with the last column;
//   4. one thread per CSR row places its entries in CSR order: rank by binary
//      search in the block's distinct list, atomic per-tile entry count,
//      atomic bitmap OR, and a sequential add into the canonical row-major
//      tile slot with the value type's rounding after every add (fp16: exact
//      fp32 add then round to half) -- only that thread ever touches a slot of
//      its row, so duplicate entries accumulate in CSR order exactly as on the
//      host;
//   5. exclusive scan of the per-tile counts -> tile_nnz.
#include <cstring>
#include <hip/hip_runtime.h>
#include <rocprim/rocprim.hpp>
#include <stdint.h>

#include "../../include/tilespmm_hip.h"

namespace {

constexpr int kThreads = 256;

inline unsigned nblocks(long long n) { return (unsigned)((n + kThreads - 1) / kThreads); }

// off[b] = ptr[min(rows, b*stride + shift)] for b <= nseg (segment b covers
// rows [b*stride+shift, min(rows, b*stride+shift+len))); end[b] likewise.
__global__ void seg_bounds_kernel(const int *__restrict__ ptr, int rows, int nseg, int stride,
                                  int shift, int len, int *__restrict__ beg, int *__restrict__ end)
{
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nseg) return;
    const long long r0 = (long long)b * stride + shift;
    const long long r1 = r0 + len;
    beg[b] = ptr[r0 < rows ? r0 : rows];
    end[b] = ptr[r1 < rows ? r1 : rows];
}

// head[i] = 1 at the first entry of every non-empty segment
__global__ void head_kernel(const int *__restrict__ beg, const int *__restrict__ end, int nseg,
                            uint8_t *__restrict__ head)
{
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nseg) return;
    if (end[b] > beg[b]) head[beg[b]] = 1;
}

// flag[i] = 1 where a new distinct column starts within its segment
__global__ void flag_kernel(const int *__restrict__ sorted, const uint8_t *__restrict__ head, long long n,
                            int *__restrict__ flag)
{
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    flag[i] = (head[i] || sorted[i] != sorted[i - 1]) ? 1 : 0;
}

__global__ void distinct_scatter_kernel(const int *__restrict__ sorted, const int *__restrict__ flag,
                                        const int *__restrict__ pos, long long n, int *__restrict__ dcols)
{
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    if (flag[i]) dcols[pos[i]] = sorted[i];
}

// per segment: distinct count d = pos[end] - pos[beg] (pos has n+1 entries)
__global__ void seg_distinct_kernel(const int *__restrict__ beg, const int *__restrict__ end,
                                    const int *__restrict__ pos, int nseg, int *__restrict__ dstart,
                                    int *__restrict__ dcount)
{
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nseg) return;
    const int s = pos[beg[b]], e = pos[end[b]];
    if (dstart) dstart[b] = s;
    dcount[b] = e - s;
}

__global__ void ntiles_kernel(const int *__restrict__ dcount, int nseg, int bn, int *__restrict__ nt)
{
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nseg) return;
    nt[b] = (dcount[b] + bn - 1) / bn;
}

// one work-group per row-block writes its padded column indices
__global__ void colidx_kernel(const int *__restrict__ tile_ptr, const int *__restrict__ dstart,
                              const int *__restrict__ dcount, const int *__restrict__ dcols, int bn,
                              int *__restrict__ colidx)
{
    const int b = blockIdx.x;
    const int t0 = tile_ptr[b], nt = tile_ptr[b + 1] - t0;
    const int d = dcount[b], s = dstart[b];
    for (int k = threadIdx.x; k < nt * bn; k += blockDim.x)
        colidx[(size_t)t0 * bn + k] = dcols[s + (k < d ? k : d - 1)];
}

template <typename V>
__device__ __forceinline__ V add_round(V a, V b)
{
    if constexpr (sizeof(V) == 2) return (V)((float)a + (float)b);
    else return a + b;
}

// one thread per row of the sub-CSR; a column index that is not in its
// row-block's distinct list (out of [0, colA), so the key sort could not
// place it) is counted in cnt[tilenum] and written nowhere
template <typename V>
__global__ void fill_kernel(const int *__restrict__ ptr, const int *__restrict__ idx, const V *__restrict__ val,
                            int rows, int bm, int bn, int words, const int *__restrict__ tile_ptr,
                            const int *__restrict__ dstart, const int *__restrict__ dcount,
                            const int *__restrict__ dcols, int *__restrict__ cnt, int *__restrict__ bad,
                            V *__restrict__ dense, unsigned long long *__restrict__ bitmap)
{
    const int r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= rows) return;
    const int b = r / bm, lr = r - b * bm;
    const int *dl = dcols + dstart[b];
    const int d = dcount[b];
    const int t0 = tile_ptr[b];
    for (int j = ptr[r]; j < ptr[r + 1]; ++j) {
        const int c = idx[j];
        int lo = 0, hi = d;                       // lower_bound in the sorted distinct list
        while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if (dl[mid] < c) lo = mid + 1;
            else hi = mid;
        }
        if (lo >= d || dl[lo] != c) {
            atomicAdd(bad, 1);
            continue;
        }
        const int tile = t0 + lo / bn;
        const int slot = lr * bn + lo % bn;
        atomicAdd(&cnt[tile], 1);
        atomicOr(&bitmap[(size_t)tile * words + slot / 64], 1ull << (slot % 64));
        V *dst = dense + (size_t)tile * bm * bn + slot;
        *dst = add_round(*dst, val[j]);
    }
}

// ---- bitmap-packed A -------------------------------------------------------
__global__ void popcount_kernel(const unsigned long long *__restrict__ bmp, int tilenum, int words,
                                int *__restrict__ cnt)
{
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= tilenum) return;
    int k = 0;
    for (int w = 0; w < words; ++w) k += __popcll(bmp[(size_t)t * words + w]);
    cnt[t] = k;
}

// one thread per tile: the values at the set bits, in bit (row-major) order
template <typename V>
__global__ void pack_kernel(const V *__restrict__ dense, const unsigned long long *__restrict__ bmp,
                            const int *__restrict__ vptr, int tilenum, int words, int slots,
                            V *__restrict__ pval)
{
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= tilenum) return;
    int o = vptr[t];
    const V *src = dense + (size_t)t * slots;
    for (int w = 0; w < words; ++w) {
        unsigned long long m = bmp[(size_t)t * words + w];
        while (m) {
            const int b = __ffsll((long long)m) - 1;
            pval[o++] = src[w * 64 + b];
            m &= m - 1;
        }
    }
}

struct Scratch {
    void *p = nullptr;
    size_t bytes = 0;
    hipError_t grow(size_t n)
    {
        if (n <= bytes) return hipSuccess;
        if (p) (void)hipFree(p);
        bytes = 0;
        hipError_t e = hipMalloc(&p, n ? n : 16);
        if (e == hipSuccess) bytes = n;
        return e;
    }
    ~Scratch()
    {
        if (p) (void)hipFree(p);
    }
};

int bits_for(int colA)
{
    int b = 1;
    while (b < 31 && (1ll << b) < (long long)colA) ++b;
    return b;
}

#define TCHK(x)                                     \
    do {                                            \
        hipError_t e_ = (x);                        \
        if (e_ != hipSuccess) return (int)e_;       \
    } while (0)

// Distinct columns of every segment [beg, end): sorted keys + flags + scan.
// Outputs (device): pos (n+1 ints, exclusive scan of flags), dcols (<= n).
struct DistinctWork {
    int *sorted = nullptr, *flag = nullptr, *pos = nullptr, *dcols = nullptr;
    uint8_t *head = nullptr;
    ~DistinctWork()
    {
        (void)hipFree(sorted);
        (void)hipFree(flag);
        (void)hipFree(pos);
        (void)hipFree(dcols);
        (void)hipFree(head);
    }
};

int distinct_segments(const int *d_idx, long long n, int colA, int nseg, const int *beg, const int *end,
                      DistinctWork &w, Scratch &tmp, hipStream_t s)
{
    const size_t nn = (size_t)(n > 0 ? n : 1);
    if (!w.sorted) {
        TCHK(hipMalloc(&w.sorted, nn * sizeof(int)));
        TCHK(hipMalloc(&w.flag, (nn + 1) * sizeof(int)));
        TCHK(hipMalloc(&w.pos, (nn + 1) * sizeof(int)));
        TCHK(hipMalloc(&w.dcols, nn * sizeof(int)));
        TCHK(hipMalloc(&w.head, nn));
    }
    if (n == 0) return (int)hipMemsetAsync(w.pos, 0, sizeof(int), s);
    size_t need = 0;
    TCHK(rocprim::segmented_radix_sort_keys(nullptr, need, d_idx, w.sorted, (unsigned)n, (unsigned)nseg, beg,
                                            end, 0, (unsigned)bits_for(colA), s));
    TCHK(tmp.grow(need));
    TCHK(rocprim::segmented_radix_sort_keys(tmp.p, need, d_idx, w.sorted, (unsigned)n, (unsigned)nseg, beg,
                                            end, 0, (unsigned)bits_for(colA), s));
    TCHK(hipMemsetAsync(w.head, 0, nn, s));
    TCHK(hipMemsetAsync(w.flag + n, 0, sizeof(int), s));
    head_kernel<<<nblocks(nseg), kThreads, 0, s>>>(beg, end, nseg, w.head);
    flag_kernel<<<nblocks(n), kThreads, 0, s>>>(w.sorted, w.head, n, w.flag);
    // exclusive scan over n+1 flags (the last is 0): pos[n] = distinct total
    need = 0;
    TCHK(rocprim::exclusive_scan(nullptr, need, w.flag, w.pos, 0, (size_t)n + 1, rocprim::plus<int>(), s));
    TCHK(tmp.grow(need));
    TCHK(rocprim::exclusive_scan(tmp.p, need, w.flag, w.pos, 0, (size_t)n + 1, rocprim::plus<int>(), s));
    distinct_scatter_kernel<<<nblocks(n), kThreads, 0, s>>>(w.sorted, w.flag, w.pos, n, w.dcols);
    return (int)hipGetLastError();
}

int tile_create_device(tsp_dev_tiles *out, int rows, int colA, long long nnz, const int *d_ptr,
                           const int *d_idx, const void *d_val, int BM, int BN, int prec, void *stream)
{
    if (!out || rows < 0 || colA <= 0 || nnz < 0 || nnz > 0x7ffffff0LL) return TSP_EINVAL;
    if ((BM != 64 && BM != 16 && BM != 8) || BN <= 0 || BN > 32) return TSP_EINVAL;
    if (prec != TSP_PREC_FP16 && prec != TSP_PREC_TF32) return TSP_EINVAL;
    if (rows > 0 && (!d_ptr || (nnz > 0 && (!d_idx || !d_val)))) return TSP_EINVAL;
    hipStream_t s = (hipStream_t)stream;
    memset(out, 0, sizeof *out);
    out->bm = BM;
    out->bn = BN;
    out->prec = prec;
    out->bitmap_words = (BM * BN + 63) / 64;
    const int tilem = (rows + BM - 1) / BM;
    out->tilem = tilem;
    TCHK(hipMalloc(&out->d_tile_ptr, sizeof(int) * ((size_t)tilem + 1)));
    if (tilem == 0) {
        TCHK(hipMemsetAsync(out->d_tile_ptr, 0, sizeof(int), s));
        return (int)hipStreamSynchronize(s);
    }
    int *beg = nullptr, *end = nullptr, *dstart = nullptr, *dcount = nullptr, *nt = nullptr;
    Scratch tmp;
    DistinctWork w;
    struct Free {
        int **a[5];
        ~Free()
        {
            for (int **p : a) (void)hipFree(*p);
        }
    } fr{{&beg, &end, &dstart, &dcount, &nt}};
    TCHK(hipMalloc(&beg, sizeof(int) * (size_t)tilem));
    TCHK(hipMalloc(&end, sizeof(int) * (size_t)tilem));
    TCHK(hipMalloc(&dstart, sizeof(int) * (size_t)tilem));
    TCHK(hipMalloc(&dcount, sizeof(int) * (size_t)tilem));
    TCHK(hipMalloc(&nt, sizeof(int) * ((size_t)tilem + 1)));
    seg_bounds_kernel<<<nblocks(tilem), kThreads, 0, s>>>(d_ptr, rows, tilem, BM, 0, BM, beg, end);
    int st = distinct_segments(d_idx, nnz, colA, tilem, beg, end, w, tmp, s);
    if (st) return st;
    seg_distinct_kernel<<<nblocks(tilem), kThreads, 0, s>>>(beg, end, w.pos, tilem, dstart, dcount);
    TCHK(hipMemsetAsync(nt + tilem, 0, sizeof(int), s));
    ntiles_kernel<<<nblocks(tilem), kThreads, 0, s>>>(dcount, tilem, BN, nt);
    size_t need = 0;
    TCHK(rocprim::exclusive_scan(nullptr, need, nt, out->d_tile_ptr, 0, (size_t)tilem + 1,
                                 rocprim::plus<int>(), s));
    TCHK(tmp.grow(need));
    TCHK(rocprim::exclusive_scan(tmp.p, need, nt, out->d_tile_ptr, 0, (size_t)tilem + 1,
                                 rocprim::plus<int>(), s));
    // every tile holds at least one CSR entry, so tilenum <= nnz < 2^31
    int tilenum = 0;
    TCHK(hipMemcpyAsync(&tilenum, out->d_tile_ptr + tilem, sizeof(int), hipMemcpyDeviceToHost, s));
    TCHK(hipStreamSynchronize(s));
    out->tilenum = tilenum;
    const size_t vs = prec == TSP_PREC_FP16 ? 2 : 4;
    const size_t tn = (size_t)(tilenum > 0 ? tilenum : 1);
    TCHK(hipMalloc(&out->d_tile_colidx, sizeof(int) * tn * BN));
    TCHK(hipMalloc(&out->d_tile_nnz, sizeof(int) * (tn + 1)));
    TCHK(hipMalloc(&out->d_val, vs * tn * BM * BN));
    TCHK(hipMalloc((void **)&out->d_bitmap, sizeof(uint64_t) * tn * out->bitmap_words));
    int *cnt = nullptr;
    TCHK(hipMalloc(&cnt, sizeof(int) * (tn + 2)));    // + the invalid-column counter
    struct FreeCnt {
        int *p;
        ~FreeCnt() { (void)hipFree(p); }
    } fc{cnt};
    TCHK(hipMemsetAsync(cnt, 0, sizeof(int) * (tn + 2), s));
    int *bad = cnt + tn + 1;
    TCHK(hipMemsetAsync(out->d_val, 0, vs * tn * BM * BN, s));
    TCHK(hipMemsetAsync(out->d_bitmap, 0, sizeof(uint64_t) * tn * out->bitmap_words, s));
    if (tilenum > 0) {
        colidx_kernel<<<tilem, kThreads, 0, s>>>(out->d_tile_ptr, dstart, dcount, w.dcols, BN, out->d_tile_colidx);
        if (prec == TSP_PREC_FP16)
            fill_kernel<_Float16><<<nblocks(rows), kThreads, 0, s>>>(
                d_ptr, d_idx, (const _Float16 *)d_val, rows, BM, BN, out->bitmap_words, out->d_tile_ptr, dstart,
                dcount, w.dcols, cnt, bad, (_Float16 *)out->d_val, (unsigned long long *)out->d_bitmap);
        else
            fill_kernel<float><<<nblocks(rows), kThreads, 0, s>>>(
                d_ptr, d_idx, (const float *)d_val, rows, BM, BN, out->bitmap_words, out->d_tile_ptr, dstart,
                dcount, w.dcols, cnt, bad, (float *)out->d_val, (unsigned long long *)out->d_bitmap);
        TCHK(hipGetLastError());
        need = 0;
        TCHK(rocprim::exclusive_scan(nullptr, need, cnt, out->d_tile_nnz, 0, (size_t)tilenum + 1,
                                     rocprim::plus<int>(), s));
        TCHK(tmp.grow(need));
        TCHK(rocprim::exclusive_scan(tmp.p, need, cnt, out->d_tile_nnz, 0, (size_t)tilenum + 1,
                                     rocprim::plus<int>(), s));
    } else {
        TCHK(hipMemsetAsync(out->d_tile_nnz, 0, sizeof(int), s));
    }
    int nbad = 0;
    TCHK(hipMemcpyAsync(&nbad, bad, sizeof(int), hipMemcpyDeviceToHost, s));
    TCHK(hipStreamSynchronize(s));
    return nbad ? TSP_EINVAL : TSP_OK;
}

}  // namespace

extern "C" {

int tsp_tile_create_device(tsp_dev_tiles *out, int rows, int colA, long long nnz, const int *d_ptr,
                           const int *d_idx, const void *d_val, int BM, int BN, int prec, void *stream)
{
    if (!out) return TSP_EINVAL;
    memset(out, 0, sizeof *out);
    const int st = tile_create_device(out, rows, colA, nnz, d_ptr, d_idx, d_val, BM, BN, prec, stream);
    if (st != TSP_OK) tsp_dev_tiles_free(out);
    return st;
}

int tsp_tiles_pack_device(int tilenum, int bm, int bn, int prec, const void *d_val,
                          const unsigned long long *d_bitmap, long long *nvals, void **d_pval, int **d_vptr,
                          void *stream)
{
    if (tilenum < 0 || !nvals || (bm != 64 && bm != 16 && bm != 8) || bn <= 0 || bn > 32) return TSP_EINVAL;
    if (prec != TSP_PREC_FP16 && prec != TSP_PREC_TF32) return TSP_EINVAL;
    if ((d_pval == nullptr) != (d_vptr == nullptr)) return TSP_EINVAL;
    if (tilenum > 0 && (!d_bitmap || (d_pval && !d_val))) return TSP_EINVAL;
    hipStream_t s = (hipStream_t)stream;
    const int words = (bm * bn + 63) / 64;
    int *vptr = nullptr, *cnt = nullptr;
    Scratch tmp;
    TCHK(hipMalloc(&cnt, sizeof(int) * ((size_t)tilenum + 1)));
    struct FreeCnt {
        int *p;
        ~FreeCnt() { (void)hipFree(p); }
    } fc{cnt};
    hipError_t e = hipMalloc(&vptr, sizeof(int) * ((size_t)tilenum + 1));
    if (e != hipSuccess) return (int)e;
    auto fail = [&](int st) {
        (void)hipFree(vptr);
        return st;
    };
    if ((e = hipMemsetAsync(cnt + tilenum, 0, sizeof(int), s)) != hipSuccess) return fail((int)e);
    if (tilenum > 0) popcount_kernel<<<nblocks(tilenum), kThreads, 0, s>>>(d_bitmap, tilenum, words, cnt);
    size_t need = 0;
    if ((e = rocprim::exclusive_scan(nullptr, need, cnt, vptr, 0, (size_t)tilenum + 1, rocprim::plus<int>(), s)) !=
        hipSuccess)
        return fail((int)e);
    if ((e = tmp.grow(need)) != hipSuccess) return fail((int)e);
    if ((e = rocprim::exclusive_scan(tmp.p, need, cnt, vptr, 0, (size_t)tilenum + 1, rocprim::plus<int>(), s)) !=
        hipSuccess)
        return fail((int)e);
    int total = 0;   // <= slots of all tiles; a class's nnz bounds it below 2^31
    if ((e = hipMemcpyAsync(&total, vptr + tilenum, sizeof(int), hipMemcpyDeviceToHost, s)) != hipSuccess)
        return fail((int)e);
    if ((e = hipStreamSynchronize(s)) != hipSuccess) return fail((int)e);
    *nvals = total;
    if (!d_pval) return fail(TSP_OK);
    // 4 elements of zero padding: the kernels' packed loads may read past the last value
    const size_t vs = prec == TSP_PREC_FP16 ? 2 : 4;
    void *pv = nullptr;
    if ((e = hipMalloc(&pv, vs * ((size_t)total + 4))) != hipSuccess) return fail((int)e);
    if ((e = hipMemsetAsync((char *)pv + vs * (size_t)total, 0, vs * 4, s)) != hipSuccess) {
        (void)hipFree(pv);
        return fail((int)e);
    }
    if (tilenum > 0) {
        if (prec == TSP_PREC_FP16)
            pack_kernel<uint16_t><<<nblocks(tilenum), kThreads, 0, s>>>(
                (const uint16_t *)d_val, d_bitmap, vptr, tilenum, words, bm * bn, (uint16_t *)pv);
        else
            pack_kernel<uint32_t><<<nblocks(tilenum), kThreads, 0, s>>>(
                (const uint32_t *)d_val, d_bitmap, vptr, tilenum, words, bm * bn, (uint32_t *)pv);
    }
    if ((e = hipGetLastError()) != hipSuccess || (e = hipStreamSynchronize(s)) != hipSuccess) {
        (void)hipFree(pv);
        return fail((int)e);
    }
    *d_pval = pv;
    *d_vptr = vptr;
    return TSP_OK;
}

int tsp_dev_tiles_free(tsp_dev_tiles *t)
{
    if (!t) return TSP_OK;
    (void)hipFree(t->d_tile_ptr);
    (void)hipFree(t->d_tile_nnz);
    (void)hipFree(t->d_tile_colidx);
    (void)hipFree(t->d_val);
    (void)hipFree(t->d_bitmap);
    memset(t, 0, sizeof *t);
    return TSP_OK;
}

}  // extern "C"

// tsp_tiling.hip -- CSR -> tiles on the GPU (the csr2tile conversion of
// src/csr2tile.h:15-379,724-795 moved onto MI355X), bit-exact with the host
// conversion (tilespmm_amd/host/tiles.cpp).
//
//   1. key[e] = (row-block of entry e, column), value = e; one stable LSD
//      radix sort (rocPRIM) of all pairs.  Entries of one (block, column)
//      pair become a contiguous run that keeps the CSR order.
//   2. run heads -> exclusive scan -> run ids.  A block's runs are its sorted
//      distinct columns; the rank of a run inside its block is its run id
//      minus the run id at the block's first entry, and the block's distinct
//      count d is the difference at its ends (the sort keeps blocks in place,
//      so block b's entries still start at ptr[b*BM]).
//   3. ceil(d/BN) tiles per block, exclusive scan -> tile_ptr; tile_colidx is
//      the distinct list cut into BN-wide tiles, padded with the last column.
//   4. one thread per run walks its entries in CSR order: slot
//      (local row, rank % BN) of tile rank / BN, per-tile entry count, bitmap
//      bit, and a sequential add into the canonical row-major slot with the
//      value type's rounding after every add (fp16: fp32 add then round to
//      half).  A slot belongs to exactly one run, so duplicates accumulate in
//      CSR order exactly as on the host.
//   5. exclusive scan of the per-tile counts -> tile_nnz.
// Work is O(nnz) with no per-row serial loop, so hub rows of power-law
// matrices cost no more than their entries.
#include <cstring>
#include <hip/hip_runtime.h>
#include <rocprim/rocprim.hpp>
#include <stdint.h>

#include <mutex>

#include "../../include/tilespmm_hip.h"
#include "tsp_kernels.h"

// Scratch of the allocation-free packing entry point
// (tsp_tiles_pack_device_noalloc): per-block partial sums of the per-tile
// value counts, one int per kPackBlockTiles tiles, plus the total, and the
// 64-bit total in the last two ints (checked before any offset is formed,
// so the int offsets never wrap).  Every
// GPU the library runs on holds one copy for the life of the process; host
// code uses only its per-device address from hipGetSymbolAddress
// (tsp::scratch_init_current_device), never this name.
constexpr int kScratchInts = 1 << 18;                 // 1 MiB
static __device__ __align__(256) int scratch[kScratchInts];

namespace {

constexpr int kThreads = 256;

inline unsigned nblocks(long long n) { return (unsigned)((n + kThreads - 1) / kThreads); }

int bits_for(long long v)     // bits to hold values 0 .. v-1
{
    int b = 1;
    while (b < 62 && (1ll << b) < v) ++b;
    return b;
}

// bptr[b] = ptr[min(rows, b*BM)], b = 0..tilem
__global__ void block_ptr_kernel(const int *__restrict__ ptr, int rows, int tilem, int bm, int *__restrict__ bptr)
{
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b > tilem) return;
    const long long r = (long long)b * bm;
    bptr[b] = ptr[r < rows ? r : rows];
}

// one thread per entry: key = (block << cbits) | col, value = entry index,
// lrow = row inside the block.  The row comes from a binary search of ptr.
__global__ void key_kernel(const int *__restrict__ ptr, const int *__restrict__ idx, int rows, long long nnz,
                           int bm, int cbits, int colA, unsigned long long *__restrict__ key,
                           int *__restrict__ ent, uint8_t *__restrict__ lrow, int *__restrict__ bad)
{
    const long long e = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= nnz) return;
    int lo = 0, hi = rows - 1;                 // last row r with ptr[r] <= e
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (ptr[mid] <= e) lo = mid;
        else hi = mid - 1;
    }
    const int c = idx[e];
    if (c < 0 || c >= colA) atomicAdd(bad, 1);
    const unsigned cc = (unsigned)c & ((1u << cbits) - 1u);
    key[e] = ((unsigned long long)(lo / bm) << cbits) | cc;
    ent[e] = (int)e;
    lrow[e] = (uint8_t)(lo % bm);
}

__global__ void head_kernel(const unsigned long long *__restrict__ key, long long n, int *__restrict__ flag)
{
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    flag[i] = (i == 0 || key[i] != key[i - 1]) ? 1 : 0;
}

// run r starts at sorted position i; its column goes to dcols[r]
__global__ void run_scatter_kernel(const unsigned long long *__restrict__ key, const int *__restrict__ flag,
                                   const int *__restrict__ run, long long n, unsigned cmask,
                                   int *__restrict__ run_start, int *__restrict__ dcols)
{
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    if (flag[i]) {
        run_start[run[i]] = (int)i;
        dcols[run[i]] = (int)(key[i] & cmask);
    }
}

// per block: first run id and distinct count; tiles ceil(d/BN)
__global__ void block_runs_kernel(const int *__restrict__ bptr, const int *__restrict__ run, int tilem, int bn,
                                  int *__restrict__ dstart, int *__restrict__ nt)
{
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= tilem) return;
    const int s = run[bptr[b]], e = run[bptr[b + 1]];
    dstart[b] = s;
    nt[b] = (e - s + bn - 1) / bn;
}

// one work-group per row-block writes its padded column indices
__global__ void colidx_kernel(const int *__restrict__ tile_ptr, const int *__restrict__ dstart,
                              const int *__restrict__ dcols, int bn, int *__restrict__ colidx)
{
    const int b = blockIdx.x;
    const int t0 = tile_ptr[b], nt = tile_ptr[b + 1] - t0;
    if (nt == 0) return;
    const int s = dstart[b], d = dstart[b + 1] - s;
    for (int k = threadIdx.x; k < nt * bn; k += blockDim.x)
        colidx[(size_t)t0 * bn + k] = dcols[s + (k < d ? k : d - 1)];
}

template <typename V>
__device__ __forceinline__ V add_round(V a, V b)
{
    if constexpr (sizeof(V) == 2) return (V)((float)a + (float)b);
    else return a + b;
}

// one thread per run (distinct column of a block)
template <typename V>
__global__ void fill_kernel(const unsigned long long *__restrict__ key, const int *__restrict__ ent,
                            const uint8_t *__restrict__ lrow, const V *__restrict__ val,
                            const int *__restrict__ run_start, int nruns, long long n, int cbits, int bm, int bn,
                            int words, const int *__restrict__ tile_ptr, const int *__restrict__ dstart,
                            int *__restrict__ cnt, V *__restrict__ dense, unsigned long long *__restrict__ bitmap)
{
    const int r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= nruns) return;
    const long long i0 = run_start[r];
    const long long i1 = r + 1 < nruns ? run_start[r + 1] : n;
    const int b = (int)(key[i0] >> cbits);
    const int rank = r - dstart[b];
    const int tile = tile_ptr[b] + rank / bn, col = rank % bn;
    V *tv = dense + (size_t)tile * bm * bn;
    unsigned long long *tb = bitmap + (size_t)tile * words;
    for (long long i = i0; i < i1; ++i) {
        const int e = ent[i];
        const int slot = lrow[e] * bn + col;
        atomicOr(&tb[slot / 64], 1ull << (slot % 64));
        tv[slot] = add_round(tv[slot], val[e]);
    }
    atomicAdd(&cnt[tile], (int)(i1 - i0));
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

// one thread per tile: the values at the set bits, in bit (row-major) order;
// writes at or past `cap` elements are dropped
template <typename V>
__global__ void pack_kernel(const V *__restrict__ dense, const unsigned long long *__restrict__ bmp,
                            const int *__restrict__ vptr, int tilenum, int words, int slots,
                            V *__restrict__ pval, long long cap)
{
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= tilenum) return;
    long long o = vptr[t];
    const V *src = dense + (size_t)t * slots;
    for (int w = 0; w < words; ++w) {
        unsigned long long m = bmp[(size_t)t * words + w];
        while (m) {
            const int b = __ffsll((long long)m) - 1;
            if (o < cap) pval[o] = src[w * 64 + b];
            ++o;
            m &= m - 1;
        }
    }
}

// ---- allocation-free packing: a three-pass scan through `scratch` -----------
// Tiles are taken in blocks of kPackBlockTiles (kPackPer consecutive tiles per
// thread).  Pass 1 stores each tile's value count in vptr[t] and each block's
// sum in sums[b]; pass 2 (one workgroup) turns sums[0..nb) into exclusive
// block offsets and stores the total in sums[nb]; pass 3 turns the counts of
// each block into exclusive offsets.  The output array vptr doubles as the
// count buffer, so the only scratch is nb + 1 ints.
constexpr int kPackPer = 8;
constexpr int kPackBlockTiles = kThreads * kPackPer;

__global__ __launch_bounds__(kThreads) void pack_count_kernel(const unsigned long long *__restrict__ bmp, int tilenum,
                                                              int words, int *__restrict__ vptr,
                                                              int *__restrict__ sums)
{
    using BR = rocprim::block_reduce<int, kThreads>;
    __shared__ typename BR::storage_type st;
    const long long base = (long long)blockIdx.x * kPackBlockTiles + (long long)threadIdx.x * kPackPer;
    int s = 0;
    for (int j = 0; j < kPackPer; ++j) {
        const long long t = base + j;
        if (t >= tilenum) break;
        int k = 0;
        for (int w = 0; w < words; ++w) k += __popcll(bmp[(size_t)t * words + w]);
        vptr[t] = k;
        s += k;
    }
    int total = 0;
    BR().reduce(s, total, st, rocprim::plus<int>());
    if (threadIdx.x == 0) sums[blockIdx.x] = total;
}

// The block offsets are scanned in 64 bits; the int copies in sums[] are
// only used (pass 3) when the 64-bit total stored in *total64 leaves room
// for the padding within INT_MAX, which the host checks first.
__global__ __launch_bounds__(kThreads) void pack_block_scan_kernel(int *__restrict__ sums, int nb,
                                                                   long long *__restrict__ total64)
{
    using BS = rocprim::block_scan<long long, kThreads>;
    __shared__ typename BS::storage_type st;
    long long carry = 0;
    for (int base = 0; base < nb; base += kThreads) {
        const int i = base + (int)threadIdx.x;
        const long long v = i < nb ? sums[i] : 0;
        long long ex = 0, agg = 0;
        BS().exclusive_scan(v, ex, 0ll, agg, st, rocprim::plus<long long>());
        if (i < nb) sums[i] = (int)min(carry + ex, (long long)INT_MAX);
        carry += agg;
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        sums[nb] = (int)min(carry, (long long)INT_MAX);
        *total64 = carry;
    }
}

// 64-bit sum of the per-tile value counts (the allocating entry point's
// overflow check before its int scan)
__global__ __launch_bounds__(kThreads) void count_total_kernel(const int *__restrict__ cnt, int n,
                                                               unsigned long long *__restrict__ total)
{
    using BR = rocprim::block_reduce<long long, kThreads>;
    __shared__ typename BR::storage_type st;
    long long s = 0;
    for (long long i = (long long)blockIdx.x * kThreads + threadIdx.x; i < n; i += (long long)gridDim.x * kThreads)
        s += cnt[i];
    long long b = 0;
    BR().reduce(s, b, st, rocprim::plus<long long>());
    if (threadIdx.x == 0) atomicAdd(total, (unsigned long long)b);
}

__global__ __launch_bounds__(kThreads) void pack_offsets_kernel(int *__restrict__ vptr, int tilenum,
                                                                const int *__restrict__ sums)
{
    using BS = rocprim::block_scan<int, kThreads>;
    __shared__ typename BS::storage_type st;
    const long long base = (long long)blockIdx.x * kPackBlockTiles + (long long)threadIdx.x * kPackPer;
    int c[kPackPer];
    int s = 0;
    for (int j = 0; j < kPackPer; ++j) {
        const long long t = base + j;
        c[j] = t < tilenum ? vptr[t] : 0;
        s += c[j];
    }
    int ex = 0;
    BS().exclusive_scan(s, ex, 0, st, rocprim::plus<int>());
    int o = sums[blockIdx.x] + ex;
    for (int j = 0; j < kPackPer; ++j) {
        const long long t = base + j;
        if (t < tilenum) vptr[t] = o;
        o += c[j];
    }
}

// vptr[tilenum] = total; zero the nz padding elements after the last value
template <typename V>
__global__ void pack_tail_kernel(int *__restrict__ vptr, int tilenum, const int *__restrict__ sums, int nb,
                                 V *__restrict__ pval, long long cap, int nz)
{
    const int total = sums[nb];
    if (threadIdx.x == 0) vptr[tilenum] = total;
    if ((int)threadIdx.x < nz && (long long)total + threadIdx.x < cap) pval[(long long)total + threadIdx.x] = V(0);
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

// device buffers freed at scope exit
struct DevBufs {
    void *p[16] = {};
    int n = 0;
    template <typename T>
    hipError_t get(T **out, size_t bytes)
    {
        void *q = nullptr;
        hipError_t e = hipMalloc(&q, bytes ? bytes : 16);
        if (e == hipSuccess) p[n++] = q;
        *out = (T *)q;
        return e;
    }
    ~DevBufs()
    {
        for (int i = 0; i < n; ++i) (void)hipFree(p[i]);
    }
};

#define TCHK(x)                                     \
    do {                                            \
        hipError_t e_ = (x);                        \
        if (e_ != hipSuccess) return (int)e_;       \
    } while (0)

template <typename T>
int scan_excl(Scratch &tmp, const T *in, T *out, size_t n, hipStream_t s)
{
    size_t need = 0;
    TCHK(rocprim::exclusive_scan(nullptr, need, in, out, T(0), n, rocprim::plus<T>(), s));
    TCHK(tmp.grow(need));
    TCHK(rocprim::exclusive_scan(tmp.p, need, in, out, T(0), n, rocprim::plus<T>(), s));
    return 0;
}

int tile_create_device(tsp_dev_tiles *out, int rows, int colA, long long nnz, const int *d_ptr, const int *d_idx,
                       const void *d_val, int BM, int BN, int prec, void *stream)
{
    if (!out || rows < 0 || colA <= 0 || nnz < 0 || nnz > 0x7ffffff0LL) return TSP_EINVAL;
    if ((BM != 64 && BM != 16 && BM != 8) || BN <= 0 || BN > 32) return TSP_EINVAL;
    if (prec != TSP_PREC_FP16 && prec != TSP_PREC_TF32) return TSP_EINVAL;
    if (rows > 0 && (!d_ptr || (nnz > 0 && (!d_idx || !d_val)))) return TSP_EINVAL;
    hipStream_t s = (hipStream_t)stream;
    out->bm = BM;
    out->bn = BN;
    out->prec = prec;
    out->bitmap_words = (BM * BN + 63) / 64;
    const int tilem = (rows + BM - 1) / BM;
    out->tilem = tilem;
    const size_t vs = prec == TSP_PREC_FP16 ? 2 : 4;
    TCHK(hipMalloc(&out->d_tile_ptr, sizeof(int) * ((size_t)tilem + 1)));
    if (tilem == 0 || nnz == 0) {
        // no entries: every row-block has zero tiles
        TCHK(hipMemsetAsync(out->d_tile_ptr, 0, sizeof(int) * ((size_t)tilem + 1), s));
        TCHK(hipMalloc(&out->d_tile_colidx, 16));
        TCHK(hipMalloc(&out->d_val, 16));
        TCHK(hipMalloc((void **)&out->d_bitmap, 16));
        TCHK(hipMalloc(&out->d_tile_nnz, sizeof(int)));
        TCHK(hipMemsetAsync(out->d_tile_nnz, 0, sizeof(int), s));
        return (int)hipStreamSynchronize(s);
    }
    const int cbits = bits_for(colA);
    const int bbits = bits_for(tilem);
    const size_t n = (size_t)nnz;
    DevBufs db;
    Scratch tmp;
    unsigned long long *key = nullptr, *key2 = nullptr;
    int *ent = nullptr, *ent2 = nullptr, *flag = nullptr, *run = nullptr, *run_start = nullptr, *dcols = nullptr;
    int *bptr = nullptr, *dstart = nullptr, *nt = nullptr, *bad = nullptr;
    uint8_t *lrow = nullptr;
    TCHK(db.get(&key, n * 8));
    TCHK(db.get(&key2, n * 8));
    TCHK(db.get(&ent, n * 4));
    TCHK(db.get(&ent2, n * 4));
    TCHK(db.get(&lrow, n));
    TCHK(db.get(&flag, (n + 1) * 4));
    TCHK(db.get(&run, (n + 1) * 4));
    TCHK(db.get(&run_start, n * 4));
    TCHK(db.get(&dcols, n * 4));
    TCHK(db.get(&bptr, ((size_t)tilem + 1) * 4));
    TCHK(db.get(&dstart, ((size_t)tilem + 1) * 4));
    TCHK(db.get(&nt, ((size_t)tilem + 1) * 4));
    TCHK(db.get(&bad, 4));
    TCHK(hipMemsetAsync(bad, 0, 4, s));
    block_ptr_kernel<<<nblocks(tilem + 1), kThreads, 0, s>>>(d_ptr, rows, tilem, BM, bptr);
    key_kernel<<<nblocks(nnz), kThreads, 0, s>>>(d_ptr, d_idx, rows, nnz, BM, cbits, colA, key, ent, lrow, bad);
    // 1. stable sort by (block, column)
    size_t need = 0;
    TCHK(rocprim::radix_sort_pairs(nullptr, need, key, key2, ent, ent2, n, 0, cbits + bbits, s));
    TCHK(tmp.grow(need));
    TCHK(rocprim::radix_sort_pairs(tmp.p, need, key, key2, ent, ent2, n, 0, cbits + bbits, s));
    // 2. runs
    TCHK(hipMemsetAsync(flag + n, 0, 4, s));
    head_kernel<<<nblocks(nnz), kThreads, 0, s>>>(key2, nnz, flag);
    if (int st = scan_excl(tmp, flag, run, n + 1, s)) return st;
    run_scatter_kernel<<<nblocks(nnz), kThreads, 0, s>>>(key2, flag, run, nnz, (1u << cbits) - 1u, run_start,
                                                        dcols);
    // 3. tiles per block, tile_ptr
    TCHK(hipMemsetAsync(nt + tilem, 0, 4, s));
    block_runs_kernel<<<nblocks(tilem), kThreads, 0, s>>>(bptr, run, tilem, BN, dstart, nt);
    int nruns = 0;
    TCHK(hipMemcpyAsync(&nruns, run + n, 4, hipMemcpyDeviceToHost, s));
    TCHK(hipMemcpyAsync(dstart + tilem, run + n, 4, hipMemcpyDeviceToDevice, s));
    if (int st = scan_excl(tmp, nt, out->d_tile_ptr, (size_t)tilem + 1, s)) return st;
    int tilenum = 0, nbad = 0;
    TCHK(hipMemcpyAsync(&tilenum, out->d_tile_ptr + tilem, 4, hipMemcpyDeviceToHost, s));
    TCHK(hipMemcpyAsync(&nbad, bad, 4, hipMemcpyDeviceToHost, s));
    TCHK(hipStreamSynchronize(s));
    if (nbad) return TSP_EINVAL;        // a column outside [0, colA)
    // every tile holds at least one entry, so tilenum <= nnz < 2^31
    out->tilenum = tilenum;
    const size_t tn = (size_t)tilenum;
    TCHK(hipMalloc(&out->d_tile_colidx, 4 * tn * BN));
    TCHK(hipMalloc(&out->d_tile_nnz, 4 * (tn + 1)));
    TCHK(hipMalloc(&out->d_val, vs * tn * BM * BN));
    TCHK(hipMalloc((void **)&out->d_bitmap, 8 * tn * out->bitmap_words));
    int *cnt = nullptr;
    TCHK(db.get(&cnt, 4 * (tn + 1)));
    TCHK(hipMemsetAsync(cnt, 0, 4 * (tn + 1), s));
    TCHK(hipMemsetAsync(out->d_val, 0, vs * tn * BM * BN, s));
    TCHK(hipMemsetAsync(out->d_bitmap, 0, 8 * tn * out->bitmap_words, s));
    colidx_kernel<<<tilem, kThreads, 0, s>>>(out->d_tile_ptr, dstart, dcols, BN, out->d_tile_colidx);
    // 4. values, counts, bitmaps
    if (prec == TSP_PREC_FP16)
        fill_kernel<_Float16><<<nblocks(nruns), kThreads, 0, s>>>(
            key2, ent2, lrow, (const _Float16 *)d_val, run_start, nruns, nnz, cbits, BM, BN, out->bitmap_words,
            out->d_tile_ptr, dstart, cnt, (_Float16 *)out->d_val, (unsigned long long *)out->d_bitmap);
    else
        fill_kernel<float><<<nblocks(nruns), kThreads, 0, s>>>(
            key2, ent2, lrow, (const float *)d_val, run_start, nruns, nnz, cbits, BM, BN, out->bitmap_words,
            out->d_tile_ptr, dstart, cnt, (float *)out->d_val, (unsigned long long *)out->d_bitmap);
    TCHK(hipGetLastError());
    // 5. tile_nnz
    if (int st = scan_excl(tmp, cnt, out->d_tile_nnz, tn + 1, s)) return st;
    return (int)hipStreamSynchronize(s);
}

}  // namespace

namespace tsp {

bool pack_total_fits(long long total) { return total >= 0 && total <= (long long)INT_MAX - 4; }

// Per-device address of `scratch`, looked up with the device current (each
// GPU holds its own copy at its own address).
constexpr int kScratchDevices = 64;
static std::mutex g_scratch_mu;
static int *g_scratch_ptr[kScratchDevices];

int scratch_init_current_device(int **ptr)
{
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    if (dev < 0 || dev >= kScratchDevices) return TSP_EINVAL;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return (int)e;
        if (!p) return TSP_EINVAL;
        g_scratch_ptr[dev] = (int *)p;
    }
    if (ptr) *ptr = g_scratch_ptr[dev];
    return TSP_OK;
}

}  // namespace tsp

extern "C" {

int tsp_tiles_pack_device_noalloc(int tilenum, int bm, int bn, int prec, const void *d_val,
                                  const unsigned long long *d_bitmap, void *d_pval, long long pval_capacity,
                                  int *d_vptr, long long *nvals, void *stream)
{
    if (tilenum < 0 || !nvals || !d_vptr || pval_capacity < 0 || (bm != 64 && bm != 16 && bm != 8) || bn <= 0 ||
        bn > 32)
        return TSP_EINVAL;
    if (prec != TSP_PREC_FP16 && prec != TSP_PREC_TF32) return TSP_EINVAL;
    if (pval_capacity > 0 && !d_pval) return TSP_EINVAL;
    if (tilenum > 0 && (!d_bitmap || !d_val)) return TSP_EINVAL;
    if ((long long)tilenum > TSP_PACK_NOALLOC_MAX_TILES) return TSP_EINVAL;
    int *sums = nullptr;
    int st = tsp::scratch_init_current_device(&sums);
    if (st) return st;
    long long *total64 = (long long *)(sums + kScratchInts - 2);
    hipStream_t s = (hipStream_t)stream;
    const int words = (bm * bn + 63) / 64;
    const int nb = (int)(((long long)tilenum + kPackBlockTiles - 1) / kPackBlockTiles);
    if (nb > 0) pack_count_kernel<<<nb, kThreads, 0, s>>>(d_bitmap, tilenum, words, d_vptr, sums);
    pack_block_scan_kernel<<<1, kThreads, 0, s>>>(sums, nb, total64);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
    long long total = 0;
    if ((e = hipMemcpyAsync(&total, total64, sizeof total, hipMemcpyDeviceToHost, s)) != hipSuccess) return (int)e;
    if ((e = hipStreamSynchronize(s)) != hipSuccess) return (int)e;
    *nvals = total;
    // the values plus 4 elements of zero padding (the kernels' packed loads
    // may read past the last value) must fit, and the offsets are ints
    if (!tsp::pack_total_fits(total) || total + 4 > pval_capacity) return TSP_EINVAL;
    if (nb > 0) pack_offsets_kernel<<<nb, kThreads, 0, s>>>(d_vptr, tilenum, sums);
    if (prec == TSP_PREC_FP16) {
        pack_tail_kernel<uint16_t><<<1, 64, 0, s>>>(d_vptr, tilenum, sums, nb, (uint16_t *)d_pval, pval_capacity, 4);
        if (tilenum > 0)
            pack_kernel<uint16_t><<<nblocks(tilenum), kThreads, 0, s>>>(
                (const uint16_t *)d_val, d_bitmap, d_vptr, tilenum, words, bm * bn, (uint16_t *)d_pval, pval_capacity);
    } else {
        pack_tail_kernel<uint32_t><<<1, 64, 0, s>>>(d_vptr, tilenum, sums, nb, (uint32_t *)d_pval, pval_capacity, 4);
        if (tilenum > 0)
            pack_kernel<uint32_t><<<nblocks(tilenum), kThreads, 0, s>>>(
                (const uint32_t *)d_val, d_bitmap, d_vptr, tilenum, words, bm * bn, (uint32_t *)d_pval, pval_capacity);
    }
    if ((e = hipGetLastError()) != hipSuccess || (e = hipStreamSynchronize(s)) != hipSuccess) return (int)e;
    return TSP_OK;
}


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
    // the counts, then (8-byte aligned) their 64-bit total
    const size_t cnt_bytes = (sizeof(int) * ((size_t)tilenum + 1) + 7) / 8 * 8;
    TCHK(hipMalloc(&cnt, cnt_bytes + sizeof(unsigned long long)));
    unsigned long long *total64 = (unsigned long long *)((char *)cnt + cnt_bytes);
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
    if ((e = hipMemsetAsync(total64, 0, sizeof *total64, s)) != hipSuccess) return fail((int)e);
    if (tilenum > 0) {
        popcount_kernel<<<nblocks(tilenum), kThreads, 0, s>>>(d_bitmap, tilenum, words, cnt);
        count_total_kernel<<<min(1024u, nblocks(tilenum)), kThreads, 0, s>>>(cnt, tilenum, total64);
    }
    unsigned long long total_u = 0;
    if ((e = hipMemcpyAsync(&total_u, total64, sizeof total_u, hipMemcpyDeviceToHost, s)) != hipSuccess)
        return fail((int)e);
    if ((e = hipStreamSynchronize(s)) != hipSuccess) return fail((int)e);
    *nvals = (long long)total_u;
    // the int scan below and the kernels' int offsets need the values plus
    // the padding to stay within INT_MAX
    if (!tsp::pack_total_fits((long long)total_u)) return fail(TSP_EINVAL);
    size_t need = 0;
    if ((e = rocprim::exclusive_scan(nullptr, need, cnt, vptr, 0, (size_t)tilenum + 1, rocprim::plus<int>(), s)) !=
        hipSuccess)
        return fail((int)e);
    if ((e = tmp.grow(need)) != hipSuccess) return fail((int)e);
    if ((e = rocprim::exclusive_scan(tmp.p, need, cnt, vptr, 0, (size_t)tilenum + 1, rocprim::plus<int>(), s)) !=
        hipSuccess)
        return fail((int)e);
    const int total = (int)total_u;
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
                (const uint16_t *)d_val, d_bitmap, vptr, tilenum, words, bm * bn, (uint16_t *)pv, total);
        else
            pack_kernel<uint32_t><<<nblocks(tilenum), kThreads, 0, s>>>(
                (const uint32_t *)d_val, d_bitmap, vptr, tilenum, words, bm * bn, (uint32_t *)pv, total);
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

// tiles.cpp -- CSR -> variable-height tiles, and the task schedule.
//
// Tile format (Tile_create, src/csr2tile.h:724-795): row-block b covers rows
// [b*BM, min((b+1)*BM, rows)) of the class's sub-CSR.  Its distinct columns,
// sorted ascending, are cut into ceil(distinct/BN) tiles of BN columns; the
// last tile's unused slots repeat the largest column (src/csr2tile.h:117-132).
// A CSR entry (r, c) lands in tile rank(c)/BN at (r - b*BM, rank(c)%BN);
// entries that land on the same slot are summed in CSR order with the value
// type's rounding after every add (fp16: exact float add, then round to
// half, as the reference's host half arithmetic does).
//
// This implementation is organised differently from the reference's three
// OpenMP passes: one counting pass stores each row-block's distinct columns
// (at most its entry count, so they fit in an nnz-sized scratch array), and
// one fill pass sorts them, writes column indices, per-tile entry counts,
// canonical ROW-MAJOR dense tiles (the layout the MI355X kernels read) and the
// occupancy bitmaps.
#include <omp.h>
#include <string.h>

#include <algorithm>
#include <type_traits>
#include <vector>

#include "common.hpp"

namespace {

template <bool F16>
int fill_tiles(Tile_matrix *m, int rows, int colA, const int *ptr, const int *idx, const void *val_,
               const std::vector<int> &dist, const std::vector<int> &ndist)
{
    const int BM = m->bm, BN = m->bn, W = m->bitmap_words;
    const int tilem = m->tilem;
    int *tile_nnz = m->tile_nnz;
    int *tile_colidx = m->tile_colidx;
    uint64_t *bitmap = m->tile_bitmap;
    const int *tile_ptr = m->tile_ptr;
    typedef typename std::conditional<F16, uint16_t, float>::type V;
    V *dense = (V *)m->Blockdense_Val;
    const V *val = (const V *)val_;
#pragma omp parallel
    {
        std::vector<int> rank((size_t)(colA > 0 ? colA : 1));
        std::vector<int> sorted;
#pragma omp for schedule(dynamic, 64)
        for (int b = 0; b < tilem; ++b) {
            const int t0 = tile_ptr[b], nt = tile_ptr[b + 1] - t0;
            if (nt == 0) continue;
            const int start = b * BM, end = std::min(rows, start + BM);
            const int d = ndist[(size_t)b];
            sorted.assign(dist.begin() + ptr[start], dist.begin() + ptr[start] + d);
            std::sort(sorted.begin(), sorted.end());
            int *ci = tile_colidx + (size_t)t0 * BN;
            for (int k = 0; k < nt * BN; ++k) ci[k] = sorted[(size_t)std::min(k, d - 1)];
            for (int k = 0; k < d; ++k) rank[(size_t)sorted[(size_t)k]] = k;
            V *tiles = dense + (size_t)t0 * BM * BN;
            memset(tiles, 0, sizeof(V) * (size_t)nt * BM * BN);
            memset(bitmap + (size_t)t0 * W, 0, sizeof(uint64_t) * (size_t)nt * W);
            for (int t = 0; t < nt; ++t) tile_nnz[t0 + t] = 0;
            for (int r = start; r < end; ++r) {
                const int lr = r - start;
                for (int k = ptr[r]; k < ptr[r + 1]; ++k) {
                    const int rk = rank[(size_t)idx[k]];
                    const int tl = rk / BN, slot = lr * BN + rk % BN;
                    tile_nnz[t0 + tl]++;
                    bitmap[(size_t)(t0 + tl) * W + slot / 64] |= 1ull << (slot % 64);
                    V &dst = tiles[(size_t)tl * BM * BN + slot];
                    if constexpr (F16) dst = tsph::f2h(tsph::h2f(dst) + tsph::h2f(val[k]));
                    else dst = dst + val[k];
                }
            }
        }
    }
    return 0;
}

}  // namespace

extern "C" int tsp_tile_bn(int bm, int prec)
{
    if (prec == TSP_PREC_FP16) return bm == 64 ? 32 : (bm == 16 || bm == 8) ? 16 : -1;
    return bm == 64 ? 16 : (bm == 16 || bm == 8) ? 8 : -1;
}

extern "C" void tsp_tile_destroy(Tile_matrix *m)
{
    if (!m) return;
    free(m->tile_ptr);
    free(m->tile_nnz);
    free(m->tile_colidx);
    free(m->Blockdense_Val);
    free(m->blkcoostylerowidx);
    free(m->blkcoostylerowidx_colstart);
    free(m->orig_tile_row_idx);
    free(m->tile_bitmap);
    memset(m, 0, sizeof *m);
}

extern "C" int tsp_tile_create(Tile_matrix *m, int rows, int colA, long long nnz, const int *ptr,
                               const int *idx, const void *val, const int *orig_row, int BM, int BN,
                               int prec)
{
    if (!m || rows < 0 || colA < 0 || (rows > 0 && (!ptr || !orig_row))) return TSP_EINVAL;
    if (BM != 64 && BM != 16 && BM != 8) return TSP_EINVAL;
    if (BN <= 0 || BN > 32 || (prec != TSP_PREC_FP16 && prec != TSP_PREC_TF32)) return TSP_EINVAL;
    if (rows > 0 && (long long)ptr[rows] != nnz) return TSP_EINVAL;
    memset(m, 0, sizeof *m);
    m->bm = BM;
    m->bn = BN;
    m->prec = prec;
    m->bitmap_words = (BM * BN + 63) / 64;
    const int tilem = (rows + BM - 1) / BM;
    m->tilem = tilem;
    m->tilen = (colA + BN - 1) / BN;
    m->tile_ptr = tsph::alloc_n<int>((size_t)tilem + 1);
    m->orig_tile_row_idx = tsph::alloc_n<int>((size_t)tilem);
    if (!m->tile_ptr || !m->orig_tile_row_idx) { tsp_tile_destroy(m); return TSP_ENOMEM; }
    for (int b = 0; b < tilem; ++b) m->orig_tile_row_idx[b] = orig_row[(size_t)b * BM];

    // Pass 1: distinct columns of every row-block, stored at the block's own
    // CSR offset (distinct <= entries).
    std::vector<int> dist((size_t)(nnz > 0 ? nnz : 1));
    std::vector<int> ndist((size_t)(tilem > 0 ? tilem : 1), 0);
#pragma omp parallel
    {
        std::vector<int> stamp((size_t)(colA > 0 ? colA : 1), -1);
#pragma omp for schedule(dynamic, 64)
        for (int b = 0; b < tilem; ++b) {
            const int start = b * BM, end = std::min(rows, start + BM);
            int d = 0;
            int *out = dist.data() + ptr[start];
            for (int k = ptr[start]; k < ptr[end]; ++k) {
                const int c = idx[k];
                if (stamp[(size_t)c] != b) { stamp[(size_t)c] = b; out[d++] = c; }
            }
            ndist[(size_t)b] = d;
        }
    }
    long long run = 0;
    for (int b = 0; b < tilem; ++b) {
        m->tile_ptr[b] = (int)run;
        run += (ndist[(size_t)b] + BN - 1) / BN;
    }
    if (run > 0x7fffffffLL) { tsp_tile_destroy(m); return TSP_EINVAL; }
    m->tile_ptr[tilem] = (int)run;
    const int tilenum = (int)run;
    m->tilenum = tilenum;
    m->dnssize = (size_t)tilenum * BM * BN;
    m->tile_nnz = tsph::alloc_n<int>((size_t)tilenum + 1);
    m->tile_colidx = tsph::alloc_n<int>((size_t)tilenum * BN);
    m->Blockdense_Val = malloc(tsph::val_size(prec) * (m->dnssize ? m->dnssize : 1));
    m->tile_bitmap = tsph::alloc_n<uint64_t>((size_t)tilenum * m->bitmap_words);
    if (!m->tile_nnz || !m->tile_colidx || !m->Blockdense_Val || !m->tile_bitmap) {
        tsp_tile_destroy(m);
        return TSP_ENOMEM;
    }
    if (prec == TSP_PREC_FP16) fill_tiles<true>(m, rows, colA, ptr, idx, val, dist, ndist);
    else fill_tiles<false>(m, rows, colA, ptr, idx, val, dist, ndist);
    // per-tile counts -> exclusive prefix sum with tilenum+1 entries
    int acc = 0;
    for (int t = 0; t < tilenum; ++t) {
        const int c = m->tile_nnz[t];
        m->tile_nnz[t] = acc;
        acc += c;
    }
    m->tile_nnz[tilenum] = acc;
    return TSP_OK;
}

// tile_pretreatment (src/csr2tile.h:383-434): a row-block with L tiles is one
// task when L <= TH, else n = ceil(L/TH) tasks of ceil(L/n) tiles each (the
// last takes the remainder), all flagged with bit 31 so the kernel
// accumulates them atomically.
extern "C" int tsp_tile_pretreatment(const Tile_matrix *m, int TH, int *rowblkblock,
                                     unsigned **rows_out, int **colstart_out)
{
    if (!m || TH <= 0 || !rowblkblock || !rows_out || !colstart_out) return TSP_EINVAL;
    const int tilem = m->tilem;
    const int *tp = m->tile_ptr;
    long long n = 0;
    for (int b = 0; b < tilem; ++b) {
        const int L = tp[b + 1] - tp[b];
        n += L <= TH ? 1 : (L + TH - 1) / TH;
    }
    if (n > 0x7fffffffLL) return TSP_EINVAL;
    unsigned *rows = tsph::alloc_n<unsigned>((size_t)n);
    int *cs = tsph::alloc_n<int>((size_t)n + 1);
    if (!rows || !cs) { free(rows); free(cs); return TSP_ENOMEM; }
    cs[0] = tilem > 0 ? tp[0] : 0;
    int k = 0;
    for (int b = 0; b < tilem; ++b) {
        const int L = tp[b + 1] - tp[b];
        const unsigned r0 = (unsigned)m->orig_tile_row_idx[b];
        if (L <= TH) {
            rows[k] = r0;
            cs[++k] = tp[b + 1];
        } else {
            const int parts = (L + TH - 1) / TH, len = (L + parts - 1) / parts;
            for (int p = 0; p < parts; ++p) {
                rows[k] = r0 | 0x80000000u;
                cs[++k] = p == parts - 1 ? tp[b] + L : tp[b] + (p + 1) * len;
            }
        }
    }
    *rowblkblock = (int)n;
    *rows_out = rows;
    *colstart_out = cs;
    return TSP_OK;
}

// split.cpp -- heterogeneous row split into 64-, 16- and 8-row groups.
//
// Decision rule (matrix_split, src/hetero_split.h:144-291), scanning row i in
// steps of 8:
//   64 rows  if gamma < 4, i+64 <= rows, N64 > 0 and the running sum of the
//            four 16-row windows' distinct-column counts exceeds gamma*N64
//            (float product, strict '>', checked after each window);
//   16 rows  else if delta <= 0, or delta <= 2, i+16 <= rows, N16 > 0 and the
//            running sum of the two 8-row windows' counts reaches delta*N16
//            (float product, '>=');
//   8 rows   otherwise.
// Shortcuts: gamma <= 0 -> all rows 64; gamma >= 4 and delta <= 0 -> all 16;
// gamma >= 4 and delta > 2 -> all 8 (src/hetero_split.h:152-169).
//
// Every window the scan can look at starts at a multiple of 8, so instead of
// the reference's serial lazily-cached counting this file computes all 8-,
// 16- and 64-row window counts up front in parallel -- 8/16-row windows with
// per-thread stamp arrays, 64-row windows with a sliding window per thread
// range (each entry enters and leaves once) -- and then runs the scan as a
// cheap serial walk over those arrays.  The counts are exact, so the decisions
// are identical.
#include <omp.h>
#include <string.h>

#include <algorithm>
#include <vector>

#include "common.hpp"

namespace {

// Distinct columns of rows [8j, 8j+len) for every j with 8j+len <= rows
// (len = 8 or 16), stamps avoid clearing.
void window_counts_small(int rows, int cols, const int *ptr, const int *idx, int len,
                         std::vector<int> &out)
{
    const int nj = (rows + 7) / 8;
    out.assign((size_t)nj, -1);
#pragma omp parallel
    {
        std::vector<int> stamp((size_t)(cols > 0 ? cols : 1), -1);
#pragma omp for schedule(dynamic, 256)
        for (int j = 0; j < nj; ++j) {
            const int s = 8 * j;
            if (s + len > rows) continue;
            int d = 0;
            for (int k = ptr[s]; k < ptr[s + len]; ++k) {
                const int c = idx[k];
                if (stamp[(size_t)c] != j) { stamp[(size_t)c] = j; ++d; }
            }
            out[(size_t)j] = d;
        }
    }
}

// Distinct columns of rows [8j, 8j+64) for every j with 8j+64 <= rows, by a
// sliding window over each thread's contiguous range of j.
void window_counts_64(int rows, int cols, const int *ptr, const int *idx, std::vector<int> &out)
{
    const int nj = (rows + 7) / 8;
    out.assign((size_t)nj, -1);
    const int last = rows >= 64 ? (rows - 64) / 8 : -1;   // last valid j
    if (last < 0) return;
#pragma omp parallel
    {
        const int nt = omp_get_num_threads(), tid = omp_get_thread_num();
        const int per = (last + 1 + nt - 1) / nt;
        const int j0 = tid * per, j1 = std::min(last + 1, j0 + per);
        if (j0 < j1) {
            std::vector<int> cnt((size_t)(cols > 0 ? cols : 1), 0);
            int d = 0;
            for (int k = ptr[8 * j0]; k < ptr[8 * j0 + 64]; ++k)
                if (cnt[(size_t)idx[k]]++ == 0) ++d;
            out[(size_t)j0] = d;
            for (int j = j0 + 1; j < j1; ++j) {
                const int drop = 8 * (j - 1), add = 8 * j + 56;
                for (int k = ptr[drop]; k < ptr[drop + 8]; ++k)
                    if (--cnt[(size_t)idx[k]] == 0) --d;
                for (int k = ptr[add]; k < ptr[add + 8]; ++k)
                    if (cnt[(size_t)idx[k]]++ == 0) ++d;
                out[(size_t)j] = d;
            }
        }
    }
}

void build_sub(int rows, const int *ptr, const int *idx, const void *val, size_t vsz,
               const std::vector<int> &group, tsp_sub_csr *out)
{
    memset(out, 0, sizeof *out);
    const int n = (int)group.size();
    out->rows = n;
    if (n == 0) return;
    out->ptr = tsph::alloc_n<int>((size_t)n + 1);
    out->orig_row = tsph::alloc_n<int>((size_t)n);
    long long nz = 0;
    out->ptr[0] = 0;
    for (int r = 0; r < n; ++r) {
        out->orig_row[r] = group[(size_t)r];
        nz += ptr[group[(size_t)r] + 1] - ptr[group[(size_t)r]];
        out->ptr[r + 1] = (int)nz;
    }
    out->nnz = nz;
    if (nz == 0) return;
    out->idx = tsph::alloc_n<int>((size_t)nz);
    out->val = malloc(vsz * (size_t)nz);
    char *vdst = (char *)out->val;
    const char *vsrc = (const char *)val;
#pragma omp parallel for schedule(static)
    for (int r = 0; r < n; ++r) {
        const int o = group[(size_t)r];
        const int len = ptr[o + 1] - ptr[o];
        if (len <= 0) continue;
        memcpy(out->idx + out->ptr[r], idx + ptr[o], sizeof(int) * (size_t)len);
        if (vsrc) memcpy(vdst + vsz * (size_t)out->ptr[r], vsrc + vsz * (size_t)ptr[o], vsz * (size_t)len);
    }
    (void)rows;
}

}  // namespace

extern "C" int tsp_split_classes(int rowA, int colA, const int *ptr, const int *idx, float gamma,
                                 float delta, int *cls)
{
    if (rowA < 0 || colA < 0 || (!ptr && rowA) || !cls) return TSP_EINVAL;
    if (gamma <= 0.0f) { std::fill(cls, cls + rowA, 0); return TSP_OK; }
    if (gamma >= 4.0f && delta <= 0.0f) { std::fill(cls, cls + rowA, 1); return TSP_OK; }
    if (gamma >= 4.0f && delta > 2.0f) { std::fill(cls, cls + rowA, 2); return TSP_OK; }

    const bool need64 = gamma < 4.0f;
    const bool need16 = delta > 0.0f && !(delta > 2.0f);
    std::vector<int> c8, c16, c64;
    if (need64 || need16) window_counts_small(rowA, colA, ptr, idx, 16, c16);
    if (need16) window_counts_small(rowA, colA, ptr, idx, 8, c8);
    if (need64) window_counts_64(rowA, colA, ptr, idx, c64);

    int i = 0;
    while (i < rowA) {
        const int j = i / 8;
        if (need64 && i + 64 <= rowA) {
            const int n64 = c64[(size_t)j];
            if (n64 > 0) {
                const float th = gamma * (float)n64;
                int s = 0;
                bool is64 = false;
                for (int w = 0; w < 4 && !is64; ++w) {
                    s += c16[(size_t)(j + 2 * w)];
                    if ((float)s > th) is64 = true;
                }
                if (is64) {
                    std::fill(cls + i, cls + i + 64, 0);
                    i += 64;
                    continue;
                }
            }
        }
        bool is16 = false;
        if (delta <= 0.0f) {
            is16 = true;
        } else if (need16 && i + 16 <= rowA) {
            const int n16 = c16[(size_t)j];
            if (n16 > 0) {
                const float th = delta * (float)n16;
                int s = c8[(size_t)j];
                if ((float)s >= th) is16 = true;
                else if ((float)(s + c8[(size_t)j + 1]) >= th) is16 = true;
            }
        }
        if (is16) {
            std::fill(cls + i, cls + std::min(i + 16, rowA), 1);
            i += 16;
            continue;
        }
        std::fill(cls + i, cls + std::min(i + 8, rowA), 2);
        i += 8;
    }
    return TSP_OK;
}

extern "C" int tsp_matrix_split(int rowA, int colA, long long nnzA, const int *ptr, const int *idx,
                                const void *val, int prec, float gamma, float delta,
                                tsp_sub_csr *out64, tsp_sub_csr *out16, tsp_sub_csr *out8)
{
    if (!out64 || !out16 || !out8) return TSP_EINVAL;
    if (rowA > 0 && (long long)ptr[rowA] != nnzA) return TSP_EINVAL;
    std::vector<int> cls((size_t)(rowA > 0 ? rowA : 1));
    int st = tsp_split_classes(rowA, colA, ptr, idx, gamma, delta, cls.data());
    if (st) return st;
    std::vector<int> g[3];
    for (int r = 0; r < rowA; ++r) g[cls[(size_t)r]].push_back(r);
    const size_t vsz = tsph::val_size(prec);
    build_sub(rowA, ptr, idx, val, vsz, g[0], out64);
    build_sub(rowA, ptr, idx, val, vsz, g[1], out16);
    build_sub(rowA, ptr, idx, val, vsz, g[2], out8);
    return TSP_OK;
}

extern "C" void tsp_sub_csr_free(tsp_sub_csr *s)
{
    if (!s) return;
    free(s->ptr);
    free(s->idx);
    free(s->val);
    free(s->orig_row);
    memset(s, 0, sizeof *s);
}

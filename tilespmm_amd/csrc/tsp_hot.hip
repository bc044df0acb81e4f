// tsp_hot.hip -- hot B rows: the most-gathered rows of B copied into one
// contiguous region appended to B.
//
// A row-wise tiled SpMM gathers one B row (segment) per tile column.  When
// the column indices are skewed -- RMAT graphs without a vertex relabelling,
// whose hub columns are the indices with few set bits -- the hot rows sit at
// addresses that share their low bits, so their lines pile onto a few L2 and
// memory channels and the gathers run below the uniform-random rate (on
// MI355X: 24 G 256-byte rows/s against 27 G/s for uniform rows).  Copying the
// hottest rows (a few MB) into consecutive rows spreads their lines over
// every channel and keeps them in L2: the same gather stream then runs at
// 37 G rows/s.  The plan owns B with spare rows after row colA; a remapped
// column index colA + s names hot slot s, so the kernels need no change.
//
// Three device helpers, each a grid-stride loop with every access bounds
// checked against the sizes the host passes:
//   count  -- gathers per column over a class's tile column indices;
//   remap  -- rewrite tile column indices through a column -> slot map
//             (decoding slots of an earlier map first, so maps can change);
//   gather -- copy B[hot[s]] into row colA + s, once per SpMM step.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/tilespmm_hip.h"
#include "tsp_kernels.h"

namespace tsp {

typedef uint32_t hu4 __attribute__((ext_vector_type(4)));

// canonical column of a (possibly remapped) tile column index
__device__ __forceinline__ int hot_decode(int c, int colA, const int *__restrict__ hot, int nhot)
{
    return (c >= colA && c - colA < nhot) ? hot[c - colA] : c;
}

__global__ __launch_bounds__(256) void colidx_count_kernel(const int *__restrict__ colidx, long long n, int colA,
                                                           const int *__restrict__ hot, int nhot,
                                                           unsigned *__restrict__ counts)
{
    const long long stride = (long long)gridDim.x * blockDim.x;
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const int c = hot_decode(colidx[i], colA, hot, nhot);
        if (c >= 0 && c < colA) atomicAdd(counts + c, 1u);
    }
}

__global__ __launch_bounds__(256) void colidx_remap_kernel(int *__restrict__ colidx, long long n, int colA,
                                                           const int *__restrict__ old_hot, int old_nhot,
                                                           const int *__restrict__ map)
{
    const long long stride = (long long)gridDim.x * blockDim.x;
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        int c = hot_decode(colidx[i], colA, old_hot, old_nhot);
        if (map && c >= 0 && c < colA) c = map[c];
        colidx[i] = c;
    }
}

__global__ __launch_bounds__(256) void hot_gather_kernel(hu4 *__restrict__ B, int colA, int vpr,
                                                         const int *__restrict__ hot, int nhot)
{
    const long long n = (long long)nhot * vpr;
    const long long stride = (long long)gridDim.x * blockDim.x;
    for (long long v = (long long)blockIdx.x * blockDim.x + threadIdx.x; v < n; v += stride) {
        const int s = (int)(v / vpr), j = (int)(v - (long long)s * vpr);
        const int c = hot[s];
        if (c < 0 || c >= colA) continue;
        B[((size_t)colA + s) * vpr + j] = B[(size_t)c * vpr + j];
    }
}

static unsigned grid_for(long long n)
{
    const long long b = (n + 255) / 256;
    return (unsigned)(b < 1 ? 1 : (b > 8192 ? 8192 : b));
}

}  // namespace tsp

extern "C" {

int tsp_colidx_count(const int *d_colidx, long long n, int colA, const int *d_hot, int nhot, unsigned *d_counts,
                     void *stream)
{
    if (n < 0 || colA < 0 || nhot < 0 || (n > 0 && (!d_colidx || !d_counts)) || (nhot > 0 && !d_hot))
        return TSP_EINVAL;
    if (n == 0) return TSP_OK;
    tsp::colidx_count_kernel<<<tsp::grid_for(n), 256, 0, (hipStream_t)stream>>>(d_colidx, n, colA, d_hot, nhot,
                                                                                  d_counts);
    return (int)hipGetLastError();
}

int tsp_colidx_remap(int *d_colidx, long long n, int colA, const int *d_old_hot, int old_nhot, const int *d_map,
                     void *stream)
{
    if (n < 0 || colA < 0 || old_nhot < 0 || (n > 0 && !d_colidx) || (old_nhot > 0 && !d_old_hot)) return TSP_EINVAL;
    if (n == 0) return TSP_OK;
    tsp::colidx_remap_kernel<<<tsp::grid_for(n), 256, 0, (hipStream_t)stream>>>(d_colidx, n, colA, d_old_hot,
                                                                                  old_nhot, d_map);
    return (int)hipGetLastError();
}

int tsp_hot_rows_gather(void *d_B, int colA, long long row_bytes, const int *d_hot, int nhot, void *stream)
{
    if (colA < 0 || nhot < 0 || row_bytes <= 0 || row_bytes % 16 || row_bytes / 16 > 0x7fffffffLL) return TSP_EINVAL;
    if (nhot == 0) return TSP_OK;
    if (!d_B || !d_hot || ((uintptr_t)d_B & 15)) return TSP_EINVAL;
    const int vpr = (int)(row_bytes / 16);
    tsp::hot_gather_kernel<<<tsp::grid_for((long long)nhot * vpr), 256, 0, (hipStream_t)stream>>>(
        (tsp::hu4 *)d_B, colA, vpr, d_hot, nhot);
    return (int)hipGetLastError();
}

}  // extern "C"

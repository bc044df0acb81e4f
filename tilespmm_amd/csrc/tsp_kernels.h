// tsp_kernels.h -- internal declarations shared by the kernel and C-ABI
// translation units of libtilespmm_hip.so.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>

namespace tsp {

constexpr int kWavesPerBlock = 4;
constexpr int kBlockThreads = 64 * kWavesPerBlock;

// Tile width BN for a row-block height BM and precision (fp16: 64->32,
// 16->16, 8->16; tf32: 64->16, 16->8, 8->8), as src/main.cu:267-275 fixes it.
constexpr __host__ __device__ int tile_bn(int bm, int prec)
{
    return prec == 0 ? (bm == 64 ? 32 : 16) : (bm == 64 ? 16 : 8);
}

// Placement of a launch's workgroups on the XCDs.  The hardware deals
// workgroups to the XCDs round-robin (workgroup b -> XCD b % kXcds), and each
// XCD has its own L2.  kPlaceContiguous gives each XCD one contiguous eighth
// of the logical blocks (neighbouring task ranges, which share B rows, share
// an L2); kPlaceInterleaved deals runs of kXcdRun consecutive logical blocks
// to the XCDs in turn, which keeps skewed matrices (hub rows at one end)
// balanced across the XCDs.
constexpr int kXcds = 8;
constexpr int kXcdRun = 4;
constexpr int kPlaceContiguous = 0;
constexpr int kPlaceInterleaved = 1;

// Kernel variant = (chunk width W, pipeline stages S, tasks per wave).
int default_chunk_width(int bm, int colB_p);
int default_stages(int bm, int prec, int w);
bool valid_variant(int bm, int w, int s);
const void *select_kernel(int bm, int prec, int w, int s, bool packed);
// w, s, tpw <= 0 select the defaults; order 0 = default, 1 = chunks of one
// task range adjacent, 2 = chunk-major.  bmp != nullptr selects the
// bitmap-packed A format (val = packed values, vptr = per-tile offsets).
int launch(int bm, int prec, int ntasks, int colB_p, const void *val, const uint64_t *bmp,
           const int *vptr, const unsigned *rows, const int *colstart, const void *B, float *C,
           const int *colidx, int c_rows, hipStream_t st, int w, int s, int tpw, int order,
           int placement = kPlaceContiguous);
int launch_copy(void *dst, const void *src, size_t bytes, hipStream_t s);
constexpr int kGatherBlocks = 8192;      // gather probe grid: 8192 x 256 threads
int launch_gather(const void *table, size_t table_bytes, int row_bytes, int iters, unsigned seed, void *sink,
                  hipStream_t s);

// Address of the allocation-free entry points' `scratch` array on the current
// device (looked up once per device; tsp_device_init calls it).
int scratch_init_current_device(int **ptr);

}  // namespace tsp

// tsp_kernels.h -- internal declarations shared by the kernel and C-ABI
// translation units of libtilespmm_hip.so.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace tsp {

constexpr int kWavesPerBlock = 4;
constexpr int kBlockThreads = 64 * kWavesPerBlock;

// Tile width BN for a row-block height BM and precision (fp16: 64->32,
// 16->16, 8->16; tf32: 64->16, 16->8, 8->8), as src/main.cu:267-275 fixes it.
// Internal precision code of tf32 launches whose operands are tf32 values
// already (the kernels then skip the per-operand rounding); tile shapes are
// those of TSP_PREC_TF32.
constexpr int kPrecTf32Exact = 2;

constexpr __host__ __device__ int tile_bn(int bm, int prec)
{
    return prec == 0 ? (bm == 64 ? 32 : 16) : (bm == 64 ? 16 : 8);
}

// fp32 bits rounded to tf32 (10 mantissa bits), nearest-even.  Inf and NaN
// pass unchanged: adding the rounding bias to a NaN would carry its payload
// into the exponent or the sign (0x7f800001 -> Inf, 0x7fffffff -> -0), while
// the reference's tensor cores see the raw NaN and propagate it.  Shared by
// the kernels and the host-callable tsp_round_tf32_bits.
__host__ __device__ inline uint32_t round_tf32_bits(uint32_t x)
{
    const uint32_t r = (x + 0xfffu + ((x >> 13) & 1u)) & 0xffffe000u;
    return (x & 0x7f800000u) == 0x7f800000u ? x : r;
}

// Placement of a launch's workgroups on the XCDs.  The hardware deals
// workgroups to the XCDs round-robin (workgroup b -> XCD b % kXcds), and each
// XCD has its own L2.  kPlaceContiguous gives each XCD one contiguous eighth
// of the logical blocks (neighbouring task ranges, which share B rows, share
// an L2); kPlaceInterleaved deals runs of kXcdRun consecutive logical blocks
// to the XCDs in turn, which keeps skewed matrices (hub rows at one end)
// balanced across the XCDs.
// kPlaceChunkXcd gives each group of 8 / nchunks XCDs one column chunk (for
// 2, 4 or 8 chunks), dealt in runs of kXcdRun inside the group: every XCD's
// L2 then holds B segments of one chunk only, so it covers nchunks times as
// many B rows.
constexpr int kXcds = 8;
constexpr int kXcdRun = 4;
constexpr int kPlaceContiguous = 0;
constexpr int kPlaceInterleaved = 1;
constexpr int kPlaceChunkXcd = 2;

// Kernel variant = (chunk width W, pipeline stages S, tasks per wave).
int default_chunk_width(int bm, int colB_p);
int default_stages(int bm, int prec, int w);
bool valid_variant(int bm, int w, int s);
const void *select_kernel(int bm, int prec, int w, int s, bool packed, bool lane_idx = false);
// w, s, tpw <= 0 select the defaults; order 0 = default, 1 = chunks of one
// task range adjacent, 2 = chunk-major.  bmp != nullptr selects the
// bitmap-packed A format (val = packed values, vptr = per-tile offsets).
int launch(int bm, int prec, int ntasks, int colB_p, const void *val, const uint64_t *bmp,
           const int *vptr, const unsigned *rows, const int *colstart, const void *B, float *C,
           const int *colidx, int c_rows, hipStream_t st, int w, int s, int tpw, int order,
           int placement = kPlaceContiguous, bool lane_idx = false);
int launch_copy(void *dst, const void *src, size_t bytes, hipStream_t s);
constexpr int kGatherBlocks = 8192;      // gather probe grid: 8192 x 256 threads
int launch_gather(const void *table, size_t table_bytes, int row_bytes, int iters, unsigned seed, void *sink,
                  hipStream_t s);

// Address of the allocation-free entry points' `scratch` array on the current
// device (looked up once per device; tsp_device_init calls it).
int scratch_init_current_device(int **ptr);

}  // namespace tsp

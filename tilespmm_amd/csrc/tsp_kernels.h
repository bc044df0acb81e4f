// tsp_kernels.h -- internal declarations shared by the kernel and C-ABI
// translation units of libtilespmm_hip.so.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace tsp {

constexpr int kWavesPerBlock = 4;
constexpr int kBlockThreads = 64 * kWavesPerBlock;

// Internal precision code of tf32 launches whose operands are tf32 values
// already (the kernels then skip the per-operand rounding); tile shapes are
// those of TSP_PREC_TF32.
constexpr int kPrecTf32Exact = 2;
// The same, with B's rows in the 3-byte form of pack_3byte_bits (row stride
// colB_p * 3 bytes): 25% fewer bytes per gathered row, lossless for tf32
// values.  Built without tile pairs or the panel sweep.
constexpr int kPrecTf32B3 = 3;

// Tile width BN for a row-block height BM and precision (fp16: 64->32,
// 16->16, 8->16; tf32: 64->16, 16->8, 8->8), as src/main.cu:267-275 fixes it.
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

// A tf32 value split into two bf16 halves that sum to it exactly, packed in
// one 32-bit word: high half = the value truncated to bf16 (its top 16
// bits), low half = the rest (at most 3 significant bits, so exact in
// bf16).  The tile-pair tf32 kernels multiply such words on bf16 MFMAs.
// Inf keeps its high half and gets a zero low half; NaN becomes a quiet NaN
// in both halves (a payload only in the low bits would otherwise leave an
// Inf high half).  The input must be a tf32 value (low 13 mantissa bits
// zero), as the plan's rounded copies are.
__host__ __device__ inline uint32_t split_bf16_bits(uint32_t x)
{
    if ((x & 0x7f800000u) == 0x7f800000u) return (x & 0x007fffffu) ? 0x7fc07fc0u : (x & 0xffff0000u);
    const uint32_t hi = x & 0xffff0000u;
    float fx, fh;
    __builtin_memcpy(&fx, &x, 4);
    __builtin_memcpy(&fh, &hi, 4);
    const float lo = fx - fh;
    uint32_t lb;
    __builtin_memcpy(&lb, &lo, 4);
    return hi | (lb >> 16);
}

// A tf32 value in 3 bytes: the top 24 bits of its fp32 word (sign, exponent,
// the 10 tf32 mantissa bits and 5 zero bits), which keep every tf32 value
// exactly; 4 values pack into 12 bytes, little-endian.  A NaN whose payload
// lies only in the dropped low byte gets the quiet bit, so that it stays a
// NaN.  The kernels widen a lane's 12 bytes back into 4 fp32 words
// (widen_3byte).
__host__ __device__ inline uint32_t pack_3byte_bits(uint32_t x)
{
    const bool nan_low_payload = (x & 0x7f800000u) == 0x7f800000u && (x & 0x007fffffu) && !(x & 0x007fff00u);
    return (nan_low_payload ? x | 0x00400000u : x) >> 8;
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

// Kernel option bits (the `opts` argument).
constexpr int kOptSkipZeroStores = 1;   // do not store exact-zero results (C holds them already)

// Panel-synchronised sweep (optional).  The B rows are cut into panels of
// 2^pshift rows; the waves that one XCD runs in one generation of the grid
// step through the panels together, so the B rows they gather stay in that
// XCD's L2.  Per (generation g, XCD x) the counters hold the waves
// registered for g (a wave registers when its work item of g starts) and
// one count per panel, each striped over kSyncStripes cache lines.  A wave announces a panel when it issues the loads of
// its first tile at or past it, and before it loads from panel q it waits
// until as many waves have announced panel q - lag as have registered, for at
// most `spin` wall-clock ticks: the wait only shapes the timing, never the
// result.  The grid holds at most the waves that fit on the device at once;
// each wave runs one work item per generation (ngen generations).  Every
// registered wave announces every panel by the end of its item, so a launch
// leaves each panel count equal to its registration count: the counters
// carry over to the next launch with the same layout and are zeroed only
// when the layout changes.  cnt == nullptr: no synchronisation, one
// generation over a grid of every work item.
constexpr int kSyncStripes = 16;   // words per count, one per 128-byte line
constexpr int kSyncLine = 32;      // ints per 128-byte line
struct SyncArgs {
    int *cnt;        // [ngen][kXcds][npanels + 1][kSyncStripes][kSyncLine]
    int pshift;
    int npanels;
    int brows;       // canonical B rows: tiles whose first column lies past them (hot-row copies) are not gated
    int ngen;
    int lag;         // a wave loads from panel q once all have reached q - lag
    long long spin;  // longest wait per panel, wall-clock ticks
};

// Kernel variant = (chunk width W, pipeline stages S, tasks per wave).
int default_chunk_width(int bm, int colB_p);
int default_stages(int bm, int prec, int w);
bool valid_variant(int bm, int w, int s);
const void *select_kernel(int bm, int prec, int w, int s, bool packed, bool lane_idx = false, bool sync = false,
                          bool pair = false);
// The instantiations of one row-block class (tsp_spmm_bm{64,16,8}.hip);
// nullptr for a variant that is not built.  prec: TSP_PREC_FP16,
// TSP_PREC_TF32, kPrecTf32Exact or kPrecTf32B3.  pair: the tile-pair form
// (fp16 8- and 16-row tiles at 64- and 128-column chunks; kPrecTf32Exact
// 8-row tiles at 64-column chunks).
const void *select_kernel_bm64(int prec, int w, int s, bool packed, bool lane_idx, bool sync, bool pair);
const void *select_kernel_bm16(int prec, int w, int s, bool packed, bool lane_idx, bool sync, bool pair);
const void *select_kernel_bm8(int prec, int w, int s, bool packed, bool lane_idx, bool sync, bool pair);
// w, s, tpw <= 0 select the defaults; order 0 = default, 1 = chunks of one
// task range adjacent, 2 = chunk-major.  bmp != nullptr selects the
// bitmap-packed A format (val = packed values, vptr = per-tile offsets).
// b_rows, panel_rows, panel_lag, sync, sync_ints, sync_reset: the
// panel-synchronised sweep (sync != nullptr; see SyncArgs) with a buffer of
// sync_ints counters, zeroed first when sync_reset is set.  pair: tile pairs
// (TSP_LAUNCH_TILE_PAIRS).  opts: kOpt* bits.
int launch(int bm, int prec, int ntasks, int colB_p, const void *val, const uint64_t *bmp,
           const int *vptr, const unsigned *rows, const int *colstart, const void *B, float *C,
           const int *colidx, int c_rows, hipStream_t st, int w, int s, int tpw, int order,
           int placement = kPlaceContiguous, bool lane_idx = false, int b_rows = 0, int panel_rows = 0,
           int panel_lag = 1, int *sync = nullptr, long long sync_ints = 0, bool sync_reset = false,
           bool pair = false, int opts = 0);
int launch_copy(void *dst, const void *src, size_t bytes, hipStream_t s);
constexpr int kGatherBlocks = 8192;      // gather probe grid: 8192 x 256 threads
int launch_gather(const void *table, size_t table_bytes, int row_bytes, int iters, unsigned seed, void *sink,
                  hipStream_t s);
int launch_stream_gather(const void *table, long long nrows, int row_bytes, const int *idx, long long n, void *sink,
                         hipStream_t s);

// Address of the allocation-free entry points' `scratch` array on the current
// device (looked up once per device; tsp_device_init calls it).
int scratch_init_current_device(int **ptr);
// whether a packed-value total plus the 4 padding elements fits the int offsets
bool pack_total_fits(long long total);

}  // namespace tsp

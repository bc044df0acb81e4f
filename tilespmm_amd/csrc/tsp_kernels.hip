// tsp_kernels.hip -- kernel selection and launch for the tile SpMM kernel
// template (tsp_spmm.hpp, instantiated per row-block class in
// tsp_spmm_bm{64,16,8}.hip), plus the copy and random-gather probe kernels
// the benchmark calibrates against.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <utility>

#include "../../include/tilespmm_hip.h"
#include "tsp_kernels.h"

namespace tsp {

typedef uint32_t u4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void copy_kernel(u4 *__restrict__ dst, const u4 *__restrict__ src, size_t n)
{
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (; i < n; i += stride) dst[i] = src[i];
}

// Zeroes n ints (the panel sweep's counters when their layout changes; a
// kernel rather than a memset so that a captured stream holds no memset
// node).
__global__ __launch_bounds__(256) void fill_kernel(int *__restrict__ p, long long n)
{
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long long)gridDim.x * blockDim.x)
        p[i] = 0;
}

// ---------------------------------------------------------------------------
// Dispatch.
// ---------------------------------------------------------------------------
// Defaults from the MI355X variant sweep (bench.py --sweep over configs 1-5):
// 64-column chunks for 8- and 64-row tiles, 128-column chunks for 16-row
// tiles at widths that are multiples of 128, one prefetch stage (with the
// column indices prefetched S tiles ahead, more stages cost occupancy for no
// gain), one task per wave and the chunks of a task range side by side.  The
// plan's runtime tuning revisits the order, the tasks per wave, the XCD
// placement and the chunk width per class.
int default_chunk_width(int bm, int colB_p)
{
    if (colB_p == 32) return 32;
    if (bm == 16 && colB_p % 128 == 0) return 128;
    return 64;
}

int default_stages(int bm, int prec, int w)
{
    (void)bm;
    (void)prec;
    (void)w;
    return 1;
}

bool valid_variant(int bm, int w, int s)
{
    if (s < 1 || s > 3) return false;
    if (bm == 64) return w == 32 || w == 64;
    if (w == 256) return s <= 2;
    return w == 32 || w == 64 || w == 128;
}

const void *select_kernel(int bm, int prec, int w, int s, bool packed, bool lane_idx, bool sync, bool pair)
{
    if (bm == 64) return select_kernel_bm64(prec, w, s, packed, lane_idx, sync, pair);
    if (bm == 16) return select_kernel_bm16(prec, w, s, packed, lane_idx, sync, pair);
    if (bm == 8) return select_kernel_bm8(prec, w, s, packed, lane_idx, sync, pair);
    return nullptr;
}

// Resolves the variant defaults of a launch; false if the variant is invalid.
static bool resolve_variant(int bm, int prec, int colB_p, int &w, int &s, int &nchunks, int &tpw, int order,
                            int &cm)
{
    if (w <= 0) w = default_chunk_width(bm, colB_p);
    if (colB_p % w != 0) return false;
    if (s <= 0) s = default_stages(bm, prec, w);
    if (!valid_variant(bm, w, s)) return false;
    nchunks = colB_p / w;
    if (tpw <= 0) tpw = 1;
    cm = order == 2 ? 1 : 0;
    return true;
}

// Workgroups of the kernel `k` that fit on the device at once (0 if unknown),
// looked up once per kernel.
static long long resident_blocks(const void *k)
{
    static std::mutex mu;
    static std::map<std::pair<int, const void *>, long long> cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    std::lock_guard<std::mutex> lock(mu);
    auto it = cache.find({dev, k});
    if (it != cache.end()) return it->second;
    int per_cu = 0, cus = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k, kBlockThreads, 0) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return 0;
    return cache[{dev, k}] = (long long)per_cu * cus;
}

// Wall-clock ticks in `us` microseconds on the current device.
static long long wall_ticks(int us)
{
    int dev = 0, khz = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev) != hipSuccess || khz <= 0)
        khz = 100000;
    return (long long)khz * us / 1000;
}

// Longest wait of a synchronised wave for the waves of its XCD, per panel.
constexpr int kSyncSpinUs = 20;

int launch(int bm, int prec, int ntasks, int colB_p, const void *val, const uint64_t *bmp,
           const int *vptr, const unsigned *rows, const int *colstart, const void *B, float *C,
           const int *colidx, int c_rows, hipStream_t st, int w, int s, int tpw, int order,
           int placement, bool lane_idx, int b_rows, int panel_rows, int panel_lag, int *sync, long long sync_ints,
           bool sync_reset, bool pair, int opts)
{
    const bool packed = bmp != nullptr;
    if (packed && (bm == 64 || !vptr)) return TSP_EINVAL;
    if (placement != kPlaceContiguous && placement != kPlaceInterleaved && placement != kPlaceChunkXcd)
        return TSP_EINVAL;
    int nchunks = 0, cm = 0;
    if (!resolve_variant(bm, prec, colB_p, w, s, nchunks, tpw, order, cm)) return TSP_EINVAL;
    if (placement == kPlaceChunkXcd && (nchunks < 2 || kXcds % nchunks != 0)) return TSP_EINVAL;
    const void *k = select_kernel(bm, prec, w, s, packed, lane_idx, sync != nullptr, pair);
    if (!k) return TSP_EINVAL;
    const long long ranges = ((long long)ntasks + tpw - 1) / tpw;
    const long long waves = ranges * nchunks;
    long long blocks = (waves + kWavesPerBlock - 1) / kWavesPerBlock;
    if (blocks <= 0) return 0;
    SyncArgs sy{nullptr, 0, 1, 0, 1, 1, 0};
    if (sync) {
        // panel-synchronised sweep: at most the resident workgroups, in whole
        // runs of kXcds * kXcdRun (every XCD holds the same number of waves)
        if (placement == kPlaceChunkXcd || b_rows <= 0 || panel_rows < 64 || (panel_rows & (panel_rows - 1)) ||
            panel_lag < 1)
            return TSP_EINVAL;
        const long long run = (long long)kXcds * kXcdRun;
        const long long cap = resident_blocks(k) / run * run;
        if (cap <= 0) return TSP_ENODEV;
        blocks = std::min((blocks + run - 1) / run * run, cap);
        const long long gen = (waves + blocks * kWavesPerBlock - 1) / (blocks * kWavesPerBlock);
        const long long np = ((long long)b_rows + panel_rows - 1) / panel_rows;
        const long long n = gen * kXcds * (np + 1) * kSyncStripes * kSyncLine;
        if (n > sync_ints) return TSP_EINVAL;
        sy.cnt = sync;
        sy.pshift = __builtin_ctz((unsigned)panel_rows);
        sy.npanels = (int)np;
        sy.brows = b_rows;
        sy.ngen = (int)gen;
        sy.spin = wall_ticks(kSyncSpinUs);
        sy.lag = panel_lag;
        if (sync_reset) {
            fill_kernel<<<(unsigned)std::min<long long>((n + 255) / 256, 1024), 256, 0, st>>>(sync, n);
            const hipError_t fe = hipGetLastError();
            if (fe != hipSuccess) return (int)fe;
        }
    } else if (placement == kPlaceInterleaved) {
        // whole runs on every XCD (workgroups past the last logical block
        // find no task range and exit)
        const long long run = (long long)kXcds * kXcdRun;
        blocks = (blocks + run - 1) / run * run;
    } else if (placement == kPlaceChunkXcd) {
        // per XCD: enough whole runs for its share of one chunk's ranges
        const long long per_chunk = (ranges + kWavesPerBlock - 1) / kWavesPerBlock;
        const long long nx = kXcds / nchunks;
        const long long per_xcd = (per_chunk + nx * kXcdRun - 1) / (nx * kXcdRun) * kXcdRun;
        blocks = per_xcd * kXcds;
    }
    if (blocks > 0x7fffffffLL) return TSP_EINVAL;
    const int ld = colB_p;
    void *args[] = {&ntasks, &nchunks, &tpw, &cm, &val, &bmp, &vptr, &rows, &colstart, &B, &C, &colidx, (void *)&ld,
                    &c_rows, &placement, &opts, &sy};
    const hipError_t e = hipLaunchKernel(k, dim3((unsigned)blocks), dim3(kBlockThreads), args, 0, st);
    return e != hipSuccess ? (int)e : (int)hipGetLastError();
}

// Random row gathers from a table: each group of ROWB/16 lanes reads one
// ROWB-byte row (16 bytes per lane) per iteration, rows drawn uniformly by an
// integer hash.  The XOR of everything read is stored only when an
// improbable bit pattern appears, which keeps the loads live without output
// traffic.  Measures the gather bandwidth ceiling of row-wise SpMM.
__device__ __forceinline__ uint32_t hash32(uint32_t x)
{
    x ^= x >> 16;
    x *= 0x7feb352du;
    x ^= x >> 15;
    x *= 0x846ca68bu;
    x ^= x >> 16;
    return x;
}

template <int ROWB>
__global__ __launch_bounds__(256) void gather_kernel(const u4 *__restrict__ tab, uint32_t nrows, int iters,
                                                     uint32_t seed, uint32_t *__restrict__ sink)
{
    constexpr int RL = ROWB / 16;
    const uint32_t tid = blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t grp = tid / RL, sub = tid % RL;
    u4 acc = {0u, 0u, 0u, 0u};
#pragma unroll 8
    for (int i = 0; i < iters; ++i) {
        const uint32_t r = hash32(grp * 2654435761u + (uint32_t)i * 40503u + seed) % nrows;
        acc ^= tab[(size_t)r * RL + sub];
    }
    if ((acc.x & 0xfffffu) == 0x12345u) sink[tid] = acc.x ^ acc.y ^ acc.z ^ acc.w;
}

int launch_gather(const void *table, size_t table_bytes, int row_bytes, int iters, unsigned seed, void *sink,
                  hipStream_t s)
{
    const uint32_t nrows = (uint32_t)(table_bytes / (size_t)row_bytes);
    const u4 *t = (const u4 *)table;
    uint32_t *k = (uint32_t *)sink;
    switch (row_bytes) {
    case 16: gather_kernel<16><<<kGatherBlocks, 256, 0, s>>>(t, nrows, iters, seed, k); break;
    case 32: gather_kernel<32><<<kGatherBlocks, 256, 0, s>>>(t, nrows, iters, seed, k); break;
    case 64: gather_kernel<64><<<kGatherBlocks, 256, 0, s>>>(t, nrows, iters, seed, k); break;
    case 128: gather_kernel<128><<<kGatherBlocks, 256, 0, s>>>(t, nrows, iters, seed, k); break;
    case 256: gather_kernel<256><<<kGatherBlocks, 256, 0, s>>>(t, nrows, iters, seed, k); break;
    default: return TSP_EINVAL;
    }
    return (int)hipGetLastError();
}

// Row gathers in the order of a given index stream (a class's tile column
// indices, canonical or hot-remapped): wave w reads rows idx[w*per_wave ..],
// each group of ROWB/16 lanes one row (16 bytes per lane), 8 loads in flight
// per lane.  Indices are clamped to the table.  Measures the gather rate of
// the kernels' own B-row stream with nothing else in the loop.
template <int ROWB>
__global__ __launch_bounds__(256) void stream_gather_kernel(const u4 *__restrict__ tab, long long nrows,
                                                            const int *__restrict__ idx, long long n,
                                                            long long per_wave, uint32_t *__restrict__ sink)
{
    constexpr int RL = ROWB / 16, RPW = 64 / RL;   // lanes per row, rows per wave instruction
    const long long wave = ((long long)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int lane = threadIdx.x & 63, q = lane / RL, sub = lane % RL;
    const long long b = wave * per_wave, e = min(b + per_wave, n);
    u4 acc = {0u, 0u, 0u, 0u};
    for (long long i = b; i < e; i += 8 * RPW) {
        u4 v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const long long j = i + (long long)u * RPW + q;
            long long r = j < e ? (long long)idx[j] : 0;
            r = r < 0 ? 0 : (r >= nrows ? nrows - 1 : r);
            v[u] = j < e ? tab[(size_t)r * RL + sub] : u4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) acc ^= v[u];
    }
    if ((acc.x & 0xfffffu) == 0x12345u) sink[threadIdx.x] = acc.x ^ acc.y ^ acc.z ^ acc.w;
}

// The same for rows of 3-byte tf32 values (kPrecTf32B3's B): 12 bytes per
// lane, as the kernels load them.
template <int ROWB>
__global__ __launch_bounds__(256) void stream_gather3_kernel(const uint32_t *__restrict__ tab, long long nrows,
                                                             const int *__restrict__ idx, long long n,
                                                             long long per_wave, uint32_t *__restrict__ sink)
{
    constexpr int RL = ROWB / 12, RPW = 64 / RL;   // lanes per row, rows per wave instruction
    const long long wave = ((long long)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int lane = threadIdx.x & 63, q = lane / RL, sub = lane % RL;
    const long long b = wave * per_wave, e = min(b + per_wave, n);
    uint32_t acc = 0u;
    for (long long i = b; i < e; i += 8 * RPW) {
        uint32_t v[8][3];
        bool in[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const long long j = i + (long long)u * RPW + q;
            in[u] = j < e;
            long long r = in[u] ? (long long)idx[j] : 0;
            r = r < 0 ? 0 : (r >= nrows ? nrows - 1 : r);
            // always a valid row: the three words load as one 3-dword load
            const uint32_t *p = tab + (size_t)r * (ROWB / 4) + 3 * sub;
            v[u][0] = p[0];
            v[u][1] = p[1];
            v[u][2] = p[2];
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) acc ^= in[u] ? v[u][0] ^ v[u][1] ^ v[u][2] : 0u;
    }
    if ((acc & 0xfffffu) == 0x12345u) sink[threadIdx.x] = acc;
}

int launch_stream_gather(const void *table, long long nrows, int row_bytes, const int *idx, long long n, void *sink,
                         hipStream_t s)
{
    if (n <= 0) return 0;
    const u4 *t = (const u4 *)table;
    const uint32_t *t3 = (const uint32_t *)table;
    uint32_t *k = (uint32_t *)sink;
    const long long waves = (long long)kGatherBlocks * 4;
    const int rpw = 64 / (row_bytes % 16 ? row_bytes / 12 : row_bytes / 16);
    const long long per = ((n + waves - 1) / waves + 8 * rpw - 1) / (8 * rpw) * (8 * rpw);
    switch (row_bytes) {
    case 64: stream_gather_kernel<64><<<kGatherBlocks, 256, 0, s>>>(t, nrows, idx, n, per, k); break;
    case 128: stream_gather_kernel<128><<<kGatherBlocks, 256, 0, s>>>(t, nrows, idx, n, per, k); break;
    case 256: stream_gather_kernel<256><<<kGatherBlocks, 256, 0, s>>>(t, nrows, idx, n, per, k); break;
    case 512: stream_gather_kernel<512><<<kGatherBlocks, 256, 0, s>>>(t, nrows, idx, n, per, k); break;
    case 96: stream_gather3_kernel<96><<<kGatherBlocks, 256, 0, s>>>(t3, nrows, idx, n, per, k); break;
    case 192: stream_gather3_kernel<192><<<kGatherBlocks, 256, 0, s>>>(t3, nrows, idx, n, per, k); break;
    case 384: stream_gather3_kernel<384><<<kGatherBlocks, 256, 0, s>>>(t3, nrows, idx, n, per, k); break;
    default: return TSP_EINVAL;
    }
    return (int)hipGetLastError();
}

int launch_copy(void *dst, const void *src, size_t bytes, hipStream_t s)
{
    const size_t n = bytes / 16;
    unsigned blocks = (unsigned)((n + 255) / 256);
    if (blocks > 65536u * 4u) blocks = 65536u * 4u;
    if (blocks == 0) return 0;
    copy_kernel<<<blocks, 256, 0, s>>>((u4 *)dst, (const u4 *)src, n);
    return (int)hipGetLastError();
}

}  // namespace tsp

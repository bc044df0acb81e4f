// tsp_spmm.hpp -- MI355X (gfx950, CDNA4) tile SpMM kernel template.
//
// One kernel template serves the three row-block classes (BM = 64, 16, 8) of
// both precisions.  It computes, for every task of the schedule,
//     C[start .. start+BM)[cols] (= or atomically +=)
//         sum over the task's tiles of  A_tile(BM x BN) * B[colidx[tile]][cols]
// which is what the reference's stir_spmm_cuda_kernel_v{8,16,64}[_tf32][_32]
// compute (src/tilespmm_cuda.h:12-1632).  The design is CDNA4-first, not a
// translation:
//   * a wave64 owns a contiguous RANGE of tasks for one column chunk of W
//     columns.  The tiles of consecutive tasks are contiguous in memory, so
//     the wave streams them through one software pipeline that never drains
//     at task boundaries; at a boundary it only flushes its accumulators to C
//     and clears them.  Consecutive tasks of one split row-block keep
//     accumulating.  A split task is flushed with fp32 atomics whose lanes
//     cover whole rows (the slab is transposed through LDS first), unless
//     the wave ran every task of its row-block; then, like an unsplit task,
//     with plain vector stores.  A 256-thread block runs four independent
//     waves: there is no block barrier;
//   * S tiles are in flight per wave: the B row panel (BN rows x W columns,
//     16-byte vector loads) and the A fragment of tile t+S are loaded while
//     tile t is computed, and the column indices of tile t+2S (they feed the
//     B addresses) S steps earlier still;
//   * the B panel is staged in a wave-private LDS slice (one wave's LDS
//     operations execute in issue order, so one buffer is safe).  MFMA
//     column n of 16-column block c is chunk column n*CB + c (CB = W/16
//     blocks), so a lane reads CB adjacent values of a B row with one LDS
//     read and owns CB adjacent output columns (one vector store per row).
//     Dense fp16 tiles read the panel with LDS transpose reads instead, and
//     tf32 tiles with 64-column chunks gather their MFMA operands straight
//     into registers (no LDS panel);
//   * A tiles are canonical row-major BM x BN blocks read straight into MFMA
//     operand registers (8 or 16 bytes per lane);
//   * fp16: v_mfma_f32_16x16x16_f16 (BN = 16) and v_mfma_f32_16x16x32_f16
//     (BN = 32), fp32 accumulate; 8-row tiles occupy rows 0-7 of the 16-row
//     MFMA block;
//   * tf32: operands are rounded to tf32 (nearest-even, 10 mantissa bits) in
//     registers and multiplied with v_mfma_f32_16x16x4_f32 -- a tf32 product
//     is exact in fp32, so this is tf32 arithmetic with fp32 accumulate
//     (CDNA4 has no xf32 MFMA); B may also come in a 3-byte form
//     (kPrecTf32B3: 12-byte loads, widened in registers);
//   * workgroups are placed on the 8 XCDs (each with its own L2) either as
//     8 contiguous ranges of task ranges (neighbouring row-blocks share B
//     rows) or as runs of 4 workgroups dealt to the XCDs in turn (skewed
//     matrices stay balanced); the plan's runtime tuning picks per class.
//
// The MFMA K index of (lane group q = lane/16, operand element j) is a free
// permutation as long as A and B use the same one; this file uses
//   fp16: k = 4q + j (j < 4), k = 16 + 4q + (j - 4) (j >= 4)
//   tf32: k = (BN/4) q + s for MFMA step s
// so that A fragments are contiguous in the row-major tile and the four lane
// groups read LDS rows that fall in disjoint bank ranges.
//
// The template is instantiated per row-block class in tsp_spmm_bm{64,16,8}.hip
// (so the instantiations compile in parallel); tsp_kernels.hip selects and
// launches them.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <type_traits>

#include "../../include/tilespmm_hip.h"
#include "tsp_kernels.h"

namespace tsp {

typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));

// Wave-uniform read-only data (schedule, column indices) is read through the
// constant address space so the loads become scalar (SMEM) loads into SGPRs:
// they are counted by lgkmcnt and never make a wave wait on its in-flight
// vector loads.
template <typename T>
using cptr = const __attribute__((address_space(4))) T *;

template <typename T>
__device__ __forceinline__ T uload(const T *p, size_t i)
{
    return ((cptr<T>)p)[i];
}

// Workgroup b of nb -> logical block.  Contiguous: each XCD receives one
// contiguous range of logical blocks.  Interleaved: runs of kXcdRun logical
// blocks go to the XCDs in turn (nb is then a multiple of kXcds * kXcdRun).
__device__ __forceinline__ int place_block(int b, int nb, int placement)
{
    const int x = b % kXcds, k = b / kXcds;
    if (placement == kPlaceInterleaved) return ((k / kXcdRun) * kXcds + x) * kXcdRun + k % kXcdRun;
    const int q = nb / kXcds, r = nb % kXcds;
    return x < r ? x * (q + 1) + k : r * (q + 1) + (x - r) * q + k;
}

// 4 tf32 values in the 3-byte form of pack_3byte_bits (bytes 0-11 of p,
// 3 per value, little-endian) -> their fp32 words.  v_perm_b32 takes bytes
// 0-3 from its second operand and 4-7 from its first; selector 0x0c gives a
// zero byte.
__device__ __forceinline__ u4 widen_3byte(u4 p)
{
    return u4{p.x << 8, __builtin_amdgcn_perm(p.y, p.x, 0x0504030cu), __builtin_amdgcn_perm(p.z, p.y, 0x0403020cu),
              p.z & 0xffffff00u};
}

// PK selects the bitmap-packed A format (8- and 16-row classes): per tile a
// row-major occupancy bitmap (BM*BN bits, bit r*BN+c) in `bmp`, and the values
// of its set bits, in bit order, at `val_` + vptr[tile].  Each lane expands its
// slice of the tile into MFMA operand registers.  Without PK, `val_` holds
// dense canonical tiles and `bmp` / `vptr` are unused.
// Waves per SIMD the register allocation must leave room for, where the
// compiler's own choice lands a few registers past a step in occupancy: the
// 64-row kernel with 64-column chunks fits 3 waves in 168 registers, the
// synchronised fp16 16-row and 8-row kernels with 128-column chunks
// (configuration 4's) 5 waves in 96, the dense fp16 8-row kernel with
// 256-column chunks 4 waves in 128; elsewhere the compiler decides.
// With tile pairs, the synchronised 64-column kernels are held to 5 waves in
// 96 registers (the compiler's own choice lands one register past it); the
// 128-column pair kernels are limited to 4 waves by their LDS panels anyway.
// The 64-column 3-byte B kernels are held to the waves of their 4-byte
// counterparts at depth 3 (8- and 16-row: 5 in 96 registers) and 2 (8-row: 7
// in 72): their widening's temporaries cost up to 6 registers more.  (The
// LDS-panel ones widen before the LDS write and need fewer registers than
// their 4-byte counterparts.)
template <int BM, int W, int PREC, int S, bool PK, bool SY, bool PR>
constexpr int kMinWaves = PR ? (SY && W == 64 && S == 1 ? 5 : 1)
                          : PREC == kPrecTf32B3 && BM <= 16 && W == 64 ? (S == 3 ? 5 : S == 2 && BM == 8 ? 7 : 1)
                          : BM == 64 && W == 64 && S == 1 && !SY                                      ? 3
                          : SY && PREC == TSP_PREC_FP16 && BM == 16 && W == 128 && S == 1 ? 5
                          : SY && PREC == TSP_PREC_FP16 && BM == 8 && W == 128 && S == 1  ? 5
                          : !SY && !PK && PREC == TSP_PREC_FP16 && BM == 8 && W == 256 && S == 1 ? 4
                                                                                           : 1;

// SY: the panel-synchronised sweep (SyncArgs) is compiled in; without it the
// kernel runs one generation and the sync arguments are ignored.
// PR: tile pairs.  The wave's unit of work is two consecutive tiles of one
// task.  fp16 tiles with BN = 16 are multiplied together as one 16 x 32 tile
// with v_mfma_f32_16x16x32_f16 (MFMA K index 16 + k is the second tile's
// column k): half the MFMAs of the K = 16 form (which runs at half the fp16
// rate), half the loop iterations, and twice the B rows in flight per
// iteration.  tf32 8-row tiles (BN = 8, operands already tf32 values) use
// split-bf16 products on v_mfma_f32_16x16x32_bf16 (SPL below).  A task with
// an odd number of tiles ends with a unit whose second half has zero A
// values and zeroed B rows.
template <int BM, int W, int PREC, int S, bool PK, bool LI, bool SY, bool PR = false>
__global__ __launch_bounds__(kBlockThreads) __attribute__((amdgpu_waves_per_eu(kMinWaves<BM, W, PREC, S, PK, SY, PR>))) void spmm_kernel(
    int ntasks, int nchunks, int tasks_per_wave, int chunk_major, const void *__restrict__ val_,
    const uint64_t *__restrict__ bmp, const int *__restrict__ vptr,
    const unsigned *__restrict__ rows, const int *__restrict__ colstart,
    const void *__restrict__ B_, float *__restrict__ C, const int *__restrict__ colidx, int ld,
    int c_rows, int placement, int opts, SyncArgs sy)
{
    constexpr bool F16 = PREC == TSP_PREC_FP16;
    // fp16 dense tiles read their B operands with LDS transpose reads and
    // keep MFMA block c on chunk columns 16c .. 16c + 15; fp16 packed and tf32
    // tiles map MFMA column n of block c to chunk column n*CB + c (the
    // packed kernels are gather-bound, and at the occupancy the transpose
    // reads allow they ran 1-2% slower)
    constexpr bool TR = F16 && !PK;
    // tf32 operands are rounded in registers, unless the launch guarantees
    // they are tf32 values already (kPrecTf32Exact: the plan rounds its copies
    // of A and B once when they enter it)
    constexpr bool RND = PREC == TSP_PREC_TF32;
    auto rnd = [](uint32_t x) { return RND ? round_tf32_bits(x) : x; };
    constexpr int BN = tile_bn(BM, PREC);
    static_assert(!PR || (F16 && BN == 16) || (PREC == kPrecTf32Exact && BM == 8 && W == 64 && !SY),
                  "tile pairs: fp16 tiles 16 columns wide, or tf32 8-row tiles at 64-column chunks");
    // tf32 tile pairs: split-bf16 products (v_mfma_f32_16x16x32_bf16) on B
    // words in the split form of split_bf16_bits
    constexpr bool SPL = PR && !F16;
    constexpr int BNU = PR ? 2 * BN : BN;    // B rows per unit of work (a tile or a pair)
    constexpr int VV = F16 ? 8 : 4;          // values per 16-byte vector
    constexpr int VPR = W / VV;              // vectors per panel row
    constexpr int NV = BNU * VPR / 64;       // vectors per lane per unit
    static_assert(NV >= 1 && (BNU * VPR) % 64 == 0, "panel does not tile the wave");
    // LDS row stride: a multiple of the CB-value vectors the MFMA operand
    // reads use (up to 32 bytes), padded so consecutive rows shift banks
    constexpr int LDSW = W + 8;
    constexpr int RG = BM >= 16 ? BM / 16 : 1;   // 16-row MFMA row groups
    constexpr int CB = W / 16;                   // 16-column MFMA blocks
    constexpr int KS = F16 ? 1 : BN / 4;         // tf32 MFMA steps per tile
    // tf32 with 64-column chunks: lane (n, q) gathers panel row KS*q + i,
    // columns 4n .. 4n+3 with its load i, which is exactly its B operand of
    // MFMA step i (CB = 4 adjacent columns of row KS*q + i), so the gathered
    // registers feed the MFMAs directly and the panel never passes through
    // LDS.  Each load instruction still covers 4 whole 256-byte rows (192
    // with B3).
    constexpr bool DB = !F16 && VPR == 16 && CB == VV && (SPL ? NV == 4 : NV == KS);
    // B rows in the 3-byte form: a lane's 4 values are 12 bytes at 3 bytes
    // per value, widened just before the MFMAs that use them (DB) or before
    // they are written to the LDS panel
    constexpr bool B3 = PREC == kPrecTf32B3;
    static_assert(!B3 || (!PR && !SY), "3-byte B: single tiles, no panel sweep");
    constexpr int AW = F16 ? (BNU == 32 ? 4 : 2) : SPL ? 4 : KS;   // A words per row group
    using VT = typename std::conditional<F16, _Float16, float>::type;
    using RV = VT __attribute__((ext_vector_type(CB)));     // CB values of one B row
    constexpr int PWD = PK ? BM * BN / 64 : 1;               // packed: bitmap words per tile
    constexpr int NT = PR ? 2 : 1;                           // tiles per unit
    struct PMeta {
        uint64_t bw[NT][PWD];
        int vbase[NT];
    };
    using FV = float __attribute__((ext_vector_type(CB)));  // CB output columns

    __shared__ __attribute__((aligned(32))) VT lds_all[kWavesPerBlock][BNU * LDSW];
    // fp16 packed A: per wave, the v_perm_b32 byte selectors that expand a
    // lane's 4 raw values into its 4 operand slots, for each of the 16
    // occupancy patterns (slot j takes value rank_j = set bits below j, or 0)
    __shared__ u2 lut_all[kWavesPerBlock][F16 && PK ? 16 : 1];

    const int lane = threadIdx.x & 63;
    const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // uniform per wave
    if constexpr (F16 && PK) {
        // selector byte pairs: value r's halves are bytes 2r, 2r+1 of the
        // lane's 8 raw bytes (lo dword: values 0-1, hi dword: values 2-3);
        // 0x0c selects a zero byte.  One wave's LDS operations execute in
        // issue order, so its own later reads see the table.
        if (lane < 16) {
            unsigned sel[4];
            unsigned r = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const bool b = (lane >> j) & 1;
                sel[j] = b ? 0x0100u + 0x0202u * r : 0x0c0cu;
                r += b ? 1u : 0u;
            }
            lut_all[wid][lane] = u2{sel[0] | sel[1] << 16, sel[2] | sel[3] << 16};
        }
    }
    // (one task per wave and one chunk, the common launch of small plans,
    // skip the 64-bit divisions: each costs dozens of scalar instructions,
    // which a launch-bound kernel pays in full)
    const long long nranges =
        tasks_per_wave == 1 ? (long long)ntasks : ((long long)ntasks + tasks_per_wave - 1) / tasks_per_wave;
    const bool sync = SY && sy.cnt != nullptr;
    const int xcd = blockIdx.x % kXcds;
    // Counters of generation g on this XCD: the waves registered for it, then
    // one announcement count per panel.  Each count is striped over
    // kSyncStripes words in separate 128-byte lines (wave w of the XCD adds
    // to stripe w % kSyncStripes): one word taking an atomic from each of
    // the XCD's hundreds of waves would serialise in the L2 atomic unit for
    // longer than the waits it gates.  Only this XCD's waves touch them, so
    // the adds are L2 atomics, and a poll reads the stripes from L2 with one
    // device-scope vector load (it skips the CU's L1, whose copy would be
    // stale) and sums them.
    const int stripe = ((blockIdx.x / kXcds) * kWavesPerBlock + wid) % kSyncStripes;
    auto cell = [&](int g, int i, int st) {
        return sy.cnt + ((((size_t)g * kXcds + xcd) * (sy.npanels + 1) + i) * kSyncStripes + st) * kSyncLine;
    };
    auto bump = [&](int g, int i) {
        __hip_atomic_fetch_add(cell(g, i, stripe), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    };
    auto total = [&](int g, int i) {
        int v = 0;
        if (lane < kSyncStripes) v = __hip_atomic_load(cell(g, i, lane), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
        for (int o = kSyncStripes / 2; o >= 1; o >>= 1) v += __shfl_xor(v, o, kSyncStripes);
        return __builtin_amdgcn_readfirstlane(v);
    };
    // Panel announcements from..to of generation g (lane 0 only).
    auto announce = [&](int g, int from, int to) {
        if (lane == 0)
            for (int i = from; i <= to; ++i) bump(g, 1 + i);
    };

    // One work item: the task range `range` on column chunk `chunk`.
    auto run = [&](int g, int range, int chunk) {
        int lp = -1;                     // last panel this wave announced (sync)
        const int k0 = range * tasks_per_wave;
        const int k1 = min(ntasks, k0 + tasks_per_wave);
        // One batch of scalar loads: the range's tile bounds, the first task's
        // end and its schedule word (first row, split flag; a task's word is
        // read when the task starts, so that a flush never waits for it).
        const int tb = uload(colstart, k0), te = uload(colstart, k1);
        int kend = uload(colstart, k0 + 1);
        unsigned rwk = uload(rows, k0);
        if (tb >= te) return;                        // every task of the range is empty
        // a wave waits only for the waves that registered before it looks, so
        // a wave that is not resident (yet) holds nobody back
        if (sync && lane == 0) bump(g, 0);
        int k = k0;
        int gfirst = k0;                 // first task of the accumulation group
        // Skip leading empty tasks.  Called once the first column-index loads
        // are in flight, so that the common case (none) adds no round trip
        // before them.
        auto skip_empty = [&]() {
            if (kend > tb) return;
            while (kend <= tb) kend = uload(colstart, ++k + 1);
            gfirst = k;
            rwk = uload(rows, k);
        };
        const int col0 = chunk * W;
        // Before the B loads of a tile whose first column is fc: announce its
        // panel q and wait (bounded) until every registered wave of this XCD
        // has reached panel q - lag.  The tiles of one task run in ascending
        // column order, so with one task per wave a wave's panels only grow
        // (later tasks of a longer range are simply not held back).  A tile
        // whose first column is a hot-row copy (past the canonical rows) is
        // not gated.
        auto gate = [&](int fc) {
            if (!sync || fc >= sy.brows) return;
            const int q = fc >> sy.pshift;
            if (q <= lp) return;
            announce(g, lp + 1, q);
            lp = q;
            if (q < sy.lag) return;
            const long long t0 = wall_clock64();
            // the counts carry over from earlier launches, which leave every
            // panel's count equal to the registrations: compare differences
            while ((int)(total(g, 1 + q - sy.lag) - total(g, 0)) < 0 && wall_clock64() - t0 < sy.spin)
                __builtin_amdgcn_s_sleep(2);
        };

        VT *lds = lds_all[wid];
        const VT *val = (const VT *)val_;
        const char *Bb = (const char *)B_;
        const int ln = lane & 15;        // MFMA row (A) / column (B, D) index
        const int lq = lane >> 4;        // MFMA lane group

        // Panel rows of the lane's NV B loads.  Scalar column indices (LI
        // false): load i covers rows i*RPI .. i*RPI+RPI-1, row i*RPI + lane/VPR
        // for this lane.  Lane-loaded indices (LI), and the direct tf32
        // operands (DB): the lane's rows are the NV consecutive rows
        // (lane/VPR)*NV + i (with LI their column indices are consecutive in
        // the tile's index list: one vector load).
        int prow[NV], pcol[NV];
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int v = lane + 64 * i;
            prow[i] = LI || DB ? (lane / VPR) * NV + i : v / VPR;
            pcol[i] = (v % VPR) * VV;
        }

        f4 acc[RG][CB];
#pragma unroll
        for (int g = 0; g < RG; ++g)
#pragma unroll
            for (int c = 0; c < CB; ++c) acc[g][c] = f4{0.f, 0.f, 0.f, 0.f};

        // Packed-format metadata of one tile (bitmap words, value offset): wave-
        // uniform scalar loads, prefetched S tiles ahead like the column indices
        // because the value addresses depend on them.
        // With tile pairs, a unit without a second tile gets an empty bitmap
        // (its values decode to zeros) and the first tile's value offset (a
        // valid address).
        auto load_meta = [&](int t, PMeta &m, bool two = false) {
            if constexpr (PK) {
#pragma unroll
                for (int w = 0; w < PWD; ++w) m.bw[0][w] = uload(bmp, (size_t)t * PWD + w);
                m.vbase[0] = uload(vptr, t);
                if constexpr (PR) {
#pragma unroll
                    for (int w = 0; w < PWD; ++w) m.bw[1][w] = two ? uload(bmp, (size_t)(t + 1) * PWD + w) : 0ull;
                    m.vbase[1] = two ? uload(vptr, t + 1) : m.vbase[0];
                }
            }
        };
        // Packed A in two halves, so a wave never waits for a load it has just
        // issued: issue_a_packed (S tiles ahead) computes the lane's position in
        // the packed stream from the scalar bitmap words, loads its NVAL
        // consecutive values raw and looks up how to expand them (fp16: the
        // byte selectors of its occupancy pattern; tf32: the occupancy bits);
        // finish_a_packed (just before the tile's MFMAs) expands them into
        // operand registers.
        constexpr int NVAL = F16 || SPL ? 4 : KS;    // packed: operand values per lane
        using DecT = typename std::conditional<F16, u2, uint32_t>::type;
        // the lane's first slot bit, the bitmap word holding its NVAL bits
        // (NVAL-bit groups never straddle words) and the bits below it there
        const int pbit = ln * BN + NVAL * lq;
        const int pword = pbit >> 6, poff = pbit & 63;
        const uint64_t below = (1ull << poff) - 1ull;
        const u2 *lut = lut_all[wid];
        auto issue_a_packed = [&](const PMeta &m, int h, VT (&raw)[NVAL], DecT &dec) {
            static_assert(!PK || BM <= 16, "packed tiles are 8- or 16-row");
            constexpr int WD = PWD;                  // bitmap words per tile
            const uint64_t *bw = m.bw[h];
            if (BM == 8 && ln >= 8) {
#pragma unroll
                for (int j = 0; j < NVAL; ++j) raw[j] = (VT)0;
                if constexpr (F16) dec = u2{0x0c0c0c0cu, 0x0c0c0c0cu};
                else dec = 0u;
                return;
            }
            // whole-word prefix counts are wave-uniform (scalar unit); the lane
            // picks its word and counts the bits below its slots in it
            uint64_t word = bw[0];
            int pre = 0, whole = 0;
#pragma unroll
            for (int w = 1; w < WD; ++w) {
                whole += __popcll(bw[w - 1]);
                if (pword == w) {
                    word = bw[w];
                    pre = whole;
                }
            }
            pre += __popcll(word & below);
            const unsigned nib = (unsigned)(word >> poff) & ((1u << NVAL) - 1u);
            // the lane's values are consecutive in the packed stream (the value
            // array is padded, so reading NVAL of them is always in bounds)
            const VT *pv = val + m.vbase[h] + pre;
#pragma unroll
            for (int j = 0; j < NVAL; ++j) raw[j] = pv[j];
            if constexpr (F16) dec = lut[nib];
            else dec = nib;
        };
        // h: which tile of a pair (its words are MFMA K slots 16h .. 16h + 15)
        // Split-bf16 A (tf32 tile pairs): lane (ln, lq) holds row ln & 7 of
        // tile lq >> 1 of the pair, columns 4 (lq & 1) .. +3 -- the high bf16
        // halves in MFMA rows 0-7, the low halves in rows 8-15, each value
        // doubled into a bf16 pair so that it multiplies both halves of a B
        // split word (K slots 2d, 2d + 1 of lane group lq are B row 4 lq + d
        // of the pair's 16 rows, which is tile column 4 (lq & 1) + d).
        const int sbit = (ln & 7) * 8 + 4 * (lq & 1);
        const uint64_t sbelow = (1ull << sbit) - 1ull;
        const uint32_t ssel = ln < 8 ? 0x07060706u : 0x05040504u;
        // an infinite A value keeps its high half only in the K slot of the B
        // high halves (slot 2d + 1), so that it never meets a zero low half
        // of a finite B value (Inf * 0 would turn its row's product into NaN)
        const uint32_t sinf = (ssel & 0xffff0000u) | 0x0c0cu;
        auto issue_a_split = [&](const PMeta &m, VT (&raw)[NVAL], DecT &dec) {
            if constexpr (SPL && PK) {
                const uint64_t word = lq >= 2 ? m.bw[1][0] : m.bw[0][0];
                const int vb = lq >= 2 ? m.vbase[1] : m.vbase[0];
                const int pre = __popcll(word & sbelow);
                dec = (uint32_t)(word >> sbit) & 15u;
                const VT *pv = val + vb + pre;       // padded: 4 values are always readable
#pragma unroll
                for (int j = 0; j < NVAL; ++j) raw[j] = pv[j];
            }
        };
        // values (fp32 bits, tf32) -> operand words: dst[0][j] is the lane's
        // half of value j, doubled
        auto split_words = [&](const uint32_t (&v)[4], uint32_t (&dst)[RG][AW]) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t w = split_bf16_bits(v[j]);
                dst[0][j] = __builtin_amdgcn_perm(w, w, (v[j] & 0x7fffffffu) == 0x7f800000u ? sinf : ssel);
            }
        };
        auto finish_a_packed = [&](const VT (&v)[NVAL], const DecT &dec, uint32_t (&dst)[RG][AW], int h = 0) {
            if constexpr (F16) {
                const u2 bits = __builtin_bit_cast(u2, h4{v[0], v[1], v[2], v[3]});
                dst[0][2 * h] = __builtin_amdgcn_perm(bits.y, bits.x, dec.x);
                dst[0][2 * h + 1] = __builtin_amdgcn_perm(bits.y, bits.x, dec.y);
            } else {
                VT o[NVAL];
                int idx = 0;
#pragma unroll
                for (int j = 0; j < NVAL; ++j) {
                    const bool b = (dec >> j) & 1u;
                    VT x = v[0];
#pragma unroll
                    for (int q = 1; q < NVAL; ++q) x = idx == q ? v[q] : x;
                    o[j] = b ? x : (VT)0;
                    idx += b ? 1 : 0;
                }
#pragma unroll
                for (int j = 0; j < NVAL; ++j) dst[0][j] = rnd(__float_as_uint(o[j]));
            }
        };
        // dense A of tile t; with tile pairs (two: the unit holds tile t + 1
        // too) the second tile's words follow as MFMA K slots 16 .. 31
        auto load_a = [&](int t, uint32_t (&dst)[RG][AW], bool two = false) {
            const VT *tile = val + (size_t)t * (BM * BN);
#pragma unroll
            for (int g = 0; g < RG; ++g) {
                const int r = 16 * g + ln;
                if (BM == 8 && ln >= 8 && !SPL) {
#pragma unroll
                    for (int w = 0; w < AW; ++w) dst[g][w] = 0u;
                    continue;
                }
                if constexpr (F16) {
                    const u2 lo = *(const u2 *)(tile + r * BN + 4 * lq);
                    dst[g][0] = lo.x; dst[g][1] = lo.y;
                    if constexpr (PR) {
                        u2 hi = u2{0u, 0u};
                        if (two) hi = *(const u2 *)(tile + BM * BN + r * BN + 4 * lq);
                        dst[g][2] = hi.x; dst[g][3] = hi.y;
                    } else if constexpr (BN == 32) {
                        const u2 hi = *(const u2 *)(tile + r * BN + 16 + 4 * lq);
                        dst[g][2] = hi.x; dst[g][3] = hi.y;
                    }
                } else if constexpr (SPL) {
                    // raw values of tile t + (lq >> 1), row ln & 7, columns 4 (lq & 1) .. +3
                    u4 x = u4{0u, 0u, 0u, 0u};
                    if (lq < 2 || two) x = *(const u4 *)(tile + (lq >> 1) * (BM * BN) + (ln & 7) * BN + 4 * (lq & 1));
                    dst[g][0] = x.x; dst[g][1] = x.y; dst[g][2] = x.z; dst[g][3] = x.w;
                } else {
                    const float *p = tile + r * BN + KS * lq;
                    if constexpr (KS == 2) {
                        const u2 x = *(const u2 *)p;
                        dst[g][0] = rnd(x.x); dst[g][1] = rnd(x.y);
                    } else {
                        const u4 x = *(const u4 *)p;
                        dst[g][0] = rnd(x.x); dst[g][1] = rnd(x.y);
                        dst[g][2] = rnd(x.z); dst[g][3] = rnd(x.w);
                    }
                }
            }
        };
        // Column indices.  Scalar (LI false): the tile's BN indices are
        // wave-uniform; they are read with scalar loads (counted by lgkmcnt, so
        // waiting for them never waits for the vector loads of the B/A ring),
        // then each lane picks the index of each of its panel rows with a select
        // chain (RPI - 1 selects per load).  Lane-loaded (LI): each lane reads
        // its NV consecutive indices with one vector load and needs no selects,
        // at the cost of a vector memory instruction per tile.  Either way the
        // indices of tile t+S are read S tiles before the B gathers that use them.
        constexpr int RPI = 64 / VPR;                // panel rows one vector instruction covers
        const int lrow = lane / VPR;
        using CSV = int __attribute__((ext_vector_type(LI ? NV : BNU)));
        // a unit's BNU indices: its tile's, then (tile pairs) the second
        // tile's, or the first tile's again when the unit has no second tile
        auto load_cs = [&](int t, CSV &cs, bool two = false) {
            if constexpr (LI) {
                int off = lrow * NV;
                if (PR && !two && off >= BN) off -= BN;
                cs = *(const CSV *)(colidx + (size_t)t * BN + off);
            } else if constexpr (PR) {
                using CSH = int __attribute__((ext_vector_type(BN)));
                const CSH lo = *(cptr<CSH>)(colidx + (size_t)t * BN);
                const CSH hi = *(cptr<CSH>)(colidx + (size_t)(two ? t + 1 : t) * BN);
#pragma unroll
                for (int j = 0; j < BN; ++j) {
                    cs[j] = lo[j];
                    cs[BN + j] = hi[j];
                }
            } else {
                cs = *(cptr<CSV>)(colidx + (size_t)t * BN);
            }
        };
        auto select_cid = [&](const CSV &cs, int (&dst)[NV]) {
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                if constexpr (LI) {
                    dst[i] = cs[i];
                } else {
                    // the lane's row: i*RPI + lrow, or KS*lrow + i when the
                    // gathered registers are the MFMA operands
                    auto row = [&](int r) { return DB ? NV * r + i : i * RPI + r; };
                    int v = cs[row(0)];
#pragma unroll
                    for (int r = 1; r < RPI; ++r) v = lrow == r ? cs[row(r)] : v;
                    dst[i] = v;
                }
            }
        };
        auto load_b = [&](const int (&cid)[NV], u4 (&dst)[NV]) {
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                if constexpr (B3) {
                    // 12 bytes, 4-byte aligned (rows and chunk columns are
                    // multiples of 4 values): one 3-dword load
                    const uint32_t *q = (const uint32_t *)(Bb + ((size_t)cid[i] * ld + col0 + pcol[i]) * 3);
                    dst[i] = u4{q[0], q[1], q[2], 0u};
                } else {
                    dst[i] = *(const u4 *)(Bb + ((size_t)cid[i] * ld + col0 + pcol[i]) * sizeof(VT));
                }
            }
        };
        // Flush the accumulators of tasks first..last, which this wave ran back
        // to back and which share one row-block.  A split task (bit 31) is added
        // atomically, as the reference does, whatever the order of the schedule.
        // Only a group of several tasks of one split row-block may store: when
        // the tasks just before and after the group belong to other row-blocks,
        // this wave ran every task of it (a split row-block's tasks are
        // consecutive, as tile_pretreatment emits them).
        // kOptSkipZeroStores: C already holds zero (or this same result)
        // wherever the launch would store an exact zero -- a plan's own C,
        // zeroed when the plan is made and written only by its launches --
        // so those stores are skipped (a row-block's empty rows, 43% of the
        // RMAT matrices' rows, cost no write).  NaN compares unequal to zero
        // and is stored (the test per stored value or vector cost nothing
        // measurable on configurations 2 and 4, which have no empty rows).
        const bool skip0 = (opts & kOptSkipZeroStores) != 0;
        auto flush = [&](int first, int last, unsigned rw) {   // rw = rows[last]
            if constexpr (SPL) {
                // rows 8-15 of each MFMA block hold the low-half products of
                // rows 0-7: lane l (< 32) adds lane l + 32's sums.  Where an
                // infinite B value meets a zero low half of A, the low-half sum
                // is NaN (0 * Inf) while the high-half sum holds the row's true
                // infinite result (a zero A value makes the high half NaN too):
                // an infinite high-half sum is the result.
#pragma unroll
                for (int c = 0; c < CB; ++c)
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const float o = __shfl_xor(acc[0][c][j], 32);
                        acc[0][c][j] = __builtin_isinf(acc[0][c][j]) ? acc[0][c][j] : acc[0][c][j] + o;
                    }
            }
            const int row0 = (int)(rw & 0x7fffffffu);
            bool split = (rw & 0x80000000u) != 0;
            if (split && first < last) {
                const bool from_start = first == 0 || (int)(uload(rows, first - 1) & 0x7fffffffu) != row0;
                const bool to_end = last + 1 >= ntasks || (int)(uload(rows, last + 1) & 0x7fffffffu) != row0;
                split = !(from_start && to_end);
            }
            if (!split) {
#pragma unroll
                for (int g = 0; g < RG; ++g) {
                    if (BM == 8 && lq >= 2) break;
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const int r = row0 + 16 * g + 4 * lq + j;
                        if (r >= c_rows) continue;
                        float *crow = C + (size_t)r * ld + col0;
                        if constexpr (TR) {
                            // MFMA column n of block c is output column 16c + n:
                            // the 16 lanes of a group store 64 contiguous bytes
#pragma unroll
                            for (int c = 0; c < CB; ++c)
                                if (!skip0 || acc[g][c][j] != 0.f)
                                    __builtin_nontemporal_store(acc[g][c][j], crow + 16 * c + ln);
                        } else {
                            // MFMA column n of block c is output column n*CB + c:
                            // the lane owns CB adjacent columns (one vector store)
                            FV v;
                            bool nz = !skip0;
#pragma unroll
                            for (int c = 0; c < CB; ++c) {
                                v[c] = acc[g][c][j];
                                nz |= v[c] != 0.f;
                            }
                            if (nz) __builtin_nontemporal_store(v, (FV *)(crow + ln * CB));
                        }
                    }
                }
            } else {
                // fp32 atomics are issued per lane: transpose each 8-row slab
                // through the wave's (now idle) B panel in LDS so that every
                // atomic instruction covers whole rows of consecutive columns
                static_assert(BNU * LDSW * sizeof(VT) >= 8 * W * sizeof(float), "panel too small for a slab");
                float *tr = (float *)lds;
#pragma unroll
                for (int h = 0; h < BM / 8; ++h) {
                    if ((lq >> 1) == (h & 1)) {
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            float *trow = tr + (4 * (lq & 1) + j) * W;
                            if constexpr (TR) {
#pragma unroll
                                for (int c = 0; c < CB; ++c) trow[16 * c + ln] = acc[h >> 1][c][j];
                            } else {
                                FV v;
#pragma unroll
                                for (int c = 0; c < CB; ++c) v[c] = acc[h >> 1][c][j];
                                *(FV *)(trow + ln * CB) = v;
                            }
                        }
                    }
                    __builtin_amdgcn_wave_barrier();
#pragma unroll
                    for (int i = 0; i < 8 * W / 64; ++i) {
                        const int idx = lane + 64 * i;
                        const int rr = idx / W, col = idx % W;
                        const int r = row0 + 8 * h + rr;
                        const float x = tr[rr * W + col];
                        if (r < c_rows && (!skip0 || x != 0.f)) unsafeAtomicAdd(C + (size_t)r * ld + col0 + col, x);
                    }
                    __builtin_amdgcn_wave_barrier();
                }
            }
#pragma unroll
            for (int g = 0; g < RG; ++g)
#pragma unroll
                for (int c = 0; c < CB; ++c) acc[g][c] = f4{0.f, 0.f, 0.f, 0.f};
        };
        // B operand of MFMA block c at lane (n = ln, group lq).  Dense fp16
        // (TR): column 16c + n of the chunk, read with LDS transpose reads
        // (ds_read_b64_tr_b16): within a 16-lane group, lane j receives
        // element j % 4 of the 8 bytes that lanes 4k + j / 4 (k = 0..3) point
        // at, so lane L pointing at columns 16c + 4(L % 4) .. +3 of panel row
        // 4 lq + (L % 16) / 4 hands lane (n, lq) rows 4 lq .. 4 lq + 3 of
        // column 16c + n -- the K-ordered operand, with no VALU shuffling.
        // Otherwise column n*CB + c of the chunk, so one LDS read of CB
        // adjacent values per B row serves all CB blocks (fp16 packed: four
        // rows' reads are then shuffled into K order); with DB those CB
        // values are the lane's gathered registers `bd` instead.
        auto compute = [&](const uint32_t (&a)[RG][AW], const u4 (&bd)[NV]) {
            if constexpr (TR) {
                typedef short s4 __attribute__((ext_vector_type(4)));
                using lds_s4 = __attribute__((address_space(3))) s4 *;
                const VT *tb = lds + (4 * lq + (ln >> 2)) * LDSW + 4 * (ln & 3);
#pragma unroll
                for (int c = 0; c < CB; ++c) {
                    const h4 b0 = __builtin_bit_cast(h4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4)(tb + 16 * c)));
                    if constexpr (BNU == 16) {
#pragma unroll
                        for (int g = 0; g < RG; ++g) {
                            const h4 av = __builtin_bit_cast(h4, u2{a[g][0], a[g][1]});
                            acc[g][c] = __builtin_amdgcn_mfma_f32_16x16x16f16(av, b0, acc[g][c], 0, 0, 0);
                        }
                    } else {
                        const h4 b1 =
                            __builtin_bit_cast(h4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4)(tb + 16 * LDSW + 16 * c)));
                        const h8 b = h8{b0[0], b0[1], b0[2], b0[3], b1[0], b1[1], b1[2], b1[3]};
#pragma unroll
                        for (int g = 0; g < RG; ++g) {
                            const h8 av = __builtin_bit_cast(h8, u4{a[g][0], a[g][1], a[g][2], a[g][3]});
                            acc[g][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, b, acc[g][c], 0, 0, 0);
                        }
                    }
                }
            } else if constexpr (F16) {
                const VT *lb = lds + ln * CB;
                constexpr int KR = BNU == 16 ? 4 : 8;    // B rows of one lane
                RV rv[KR];
#pragma unroll
                for (int j = 0; j < 4; ++j) rv[j] = *(const RV *)(lb + (4 * lq + j) * LDSW);
                if constexpr (BNU == 32) {
#pragma unroll
                    for (int j = 0; j < 4; ++j) rv[4 + j] = *(const RV *)(lb + (16 + 4 * lq + j) * LDSW);
                }
#pragma unroll
                for (int c = 0; c < CB; ++c) {
                    if constexpr (BNU == 16) {
                        const h4 b = h4{rv[0][c], rv[1][c], rv[2][c], rv[3][c]};
#pragma unroll
                        for (int g = 0; g < RG; ++g) {
                            const h4 av = __builtin_bit_cast(h4, u2{a[g][0], a[g][1]});
                            acc[g][c] = __builtin_amdgcn_mfma_f32_16x16x16f16(av, b, acc[g][c], 0, 0, 0);
                        }
                    } else {
                        const h8 b = h8{rv[0][c], rv[1][c], rv[2][c], rv[3][c], rv[4][c], rv[5][c], rv[6][c], rv[7][c]};
#pragma unroll
                        for (int g = 0; g < RG; ++g) {
                            const h8 av = __builtin_bit_cast(h8, u4{a[g][0], a[g][1], a[g][2], a[g][3]});
                            acc[g][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, b, acc[g][c], 0, 0, 0);
                        }
                    }
                }
            } else if constexpr (SPL) {
                // block c: the split words of the lane's 4 B rows at chunk
                // column 4 ln + c (its gathered registers), one K = 32 bf16
                // MFMA covering both tiles of the unit
                typedef __bf16 bf8 __attribute__((ext_vector_type(8)));
                const bf8 av = __builtin_bit_cast(bf8, u4{a[0][0], a[0][1], a[0][2], a[0][3]});
#pragma unroll
                for (int c = 0; c < CB; ++c) {
                    const bf8 bt = __builtin_bit_cast(bf8, u4{bd[0][c], bd[1][c], bd[2][c], bd[3][c]});
                    acc[0][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bt, acc[0][c], 0, 0, 0);
                }
            } else {
                const VT *lb = lds + ln * CB;
#pragma unroll
                for (int s = 0; s < KS; ++s) {
                    RV rv;
                    if constexpr (DB) {
                        u4 x = bd[s];
                        if constexpr (B3) x = widen_3byte(x);
                        if constexpr (RND) {
                            x.x = rnd(x.x); x.y = rnd(x.y);
                            x.z = rnd(x.z); x.w = rnd(x.w);
                        }
                        rv = __builtin_bit_cast(RV, x);
                    } else {
                        rv = *(const RV *)(lb + (KS * lq + s) * LDSW);
                    }
#pragma unroll
                    for (int c = 0; c < CB; ++c)
#pragma unroll
                        for (int g = 0; g < RG; ++g)
                            acc[g][c] = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a[g][s]), rv[c],
                                                                              acc[g][c], 0, 0, 0);
                }
            }
        };
        auto stage_b = [&](const u4 (&src)[NV]) {
            if constexpr (DB) return;
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                u4 x = src[i];
                if constexpr (B3) x = widen_3byte(x);
                if constexpr (RND) {
                    x.x = rnd(x.x); x.y = rnd(x.y);
                    x.z = rnd(x.z); x.w = rnd(x.w);
                }
                VT *d = lds + prow[i] * LDSW + pcol[i];
                if constexpr (F16) {
                    *(u2 *)d = u2{x.x, x.y};
                    *(u2 *)(d + 4) = u2{x.z, x.w};
                } else {
                    *(u4 *)d = x;
                }
            }
        };

        // Prologue: B panels and A fragments of the first S tiles in flight, and
        // a ring of S column-index sets in SGPRs: slot s holds the indices of
        // tile t+S when tile t = s (mod S) is computed, so each scalar load has S
        // tile periods to arrive before its B addresses are formed (the indices
        // stream from HBM; one period is not enough to hide that latency).
        u4 bv[S][NV];
        uint32_t ar[S][RG][AW];          // dense A: operand words
        VT araw[S][NT][NVAL];             // packed A: raw values and occupancy bits
        DecT anib[S][NT];
        CSV cs[S];
        PMeta pm[S];
        int cid[NV];
        auto issue_a = [&](int t, int s, bool two = false) {
            if constexpr (SPL && PK) {
                issue_a_split(pm[s], araw[s][0], anib[s][0]);
            } else if constexpr (PK) {
#pragma unroll
                for (int h = 0; h < NT; ++h) issue_a_packed(pm[s], h, araw[s][h], anib[s][h]);
            } else {
                load_a(t, ar[s], two);
            }
        };
        auto take_a = [&](int s, uint32_t (&acur)[RG][AW]) {
            if constexpr (SPL) {
                uint32_t raw4[RG][AW];
                if constexpr (PK) {
                    finish_a_packed(araw[s][0], anib[s][0], raw4);
                } else {
#pragma unroll
                    for (int w = 0; w < AW; ++w) raw4[0][w] = ar[s][0][w];
                }
                const uint32_t v[4] = {raw4[0][0], raw4[0][1], raw4[0][2], raw4[0][3]};
                split_words(v, acur);
            } else if constexpr (PK) {
#pragma unroll
                for (int h = 0; h < NT; ++h) finish_a_packed(araw[s][h], anib[s][h], acur, h);
            } else {
#pragma unroll
                for (int g = 0; g < RG; ++g)
#pragma unroll
                    for (int w = 0; w < AW; ++w) acur[g][w] = ar[s][g][w];
            }
        };
        // Task bookkeeping when the compute front reaches tile t: at the end
        // of task k, flush unless the next task continues the same row-block.
        auto advance_task = [&](int t) {
            if (t >= kend) {                 // task k is complete
                int kn = k;
                do kend = uload(colstart, ++kn + 1);
                while (kend <= t);           // skip empty tasks
                // the next task continues the same row-block: keep
                // accumulating instead of flushing partial sums
                const unsigned rn = uload(rows, kn);
                if ((rn & 0x7fffffffu) != (rwk & 0x7fffffffu)) {
                    flush(gfirst, k, rwk);
                    gfirst = kn;
                }
                k = kn;
                rwk = rn;
            }
        };
        if constexpr (PR) {
            // Units: two consecutive tiles of one task, or the last tile of a
            // task with an odd count alone.  The unit cursor (ut, in task uk
            // ending at ukend) runs 2S units ahead of the compute front; a
            // slot's descriptors follow its unit from the index load (dI) to
            // the B/A loads and the compute (dB).
            skip_empty();
            int ut = tb, uk = k, ukend = kend;
            auto next_unit = [&](int &first, bool &two) {
                first = ut;
                two = false;
                if (ut >= te) return;
                two = ut + 1 < ukend;
                ut += two ? 2 : 1;
                while (ut < te && ut >= ukend) ukend = uload(colstart, ++uk + 1);
            };
            int dIt[S], dBt[S];
            bool dI2[S], dB2[S];
#pragma unroll
            for (int s = 0; s < S; ++s) {
                next_unit(dIt[s], dI2[s]);
                if (dIt[s] < te) {
                    load_cs(dIt[s], cs[s], dI2[s]);
                    load_meta(dIt[s], pm[s], dI2[s]);
                }
            }
#pragma unroll
            for (int s = 0; s < S; ++s) {
                dBt[s] = dIt[s];
                dB2[s] = dI2[s];
                if (dBt[s] < te) {
                    gate(__builtin_amdgcn_readfirstlane(cs[s][0]));
                    select_cid(cs[s], cid);
                    load_b(cid, bv[s]);
                    issue_a(dBt[s], s, dB2[s]);
                }
            }
#pragma unroll
            for (int s = 0; s < S; ++s) {
                next_unit(dIt[s], dI2[s]);
                if (dIt[s] < te) {
                    load_cs(dIt[s], cs[s], dI2[s]);
                    load_meta(dIt[s], pm[s], dI2[s]);
                }
            }
            bool more = dBt[0] < te;
            while (more) {
#pragma unroll
                for (int s = 0; s < S; ++s) {
                    if (more && dBt[s] < te) {
                        advance_task(dBt[s]);
                        if (!dB2[s]) {
                            // a unit without a second tile gathered the first
                            // tile's B rows again for its second half: zero them,
                            // so that its zero A values meet no Inf or NaN
#pragma unroll
                            for (int i = 0; i < NV; ++i)
                                if (prow[i] >= BN) bv[s][i] = u4{0u, 0u, 0u, 0u};
                        }
                        stage_b(bv[s]);
                        u4 bcur[NV];
#pragma unroll
                        for (int i = 0; i < NV; ++i) bcur[i] = DB ? bv[s][i] : u4{0u, 0u, 0u, 0u};
                        uint32_t acur[RG][AW];
                        take_a(s, acur);
                        if (dIt[s] < te) {
                            gate(__builtin_amdgcn_readfirstlane(cs[s][0]));
                            select_cid(cs[s], cid);
                            load_b(cid, bv[s]);
                            dBt[s] = dIt[s];
                            dB2[s] = dI2[s];
                            issue_a(dBt[s], s, dB2[s]);
                            next_unit(dIt[s], dI2[s]);
                            if (dIt[s] < te) {
                                load_cs(dIt[s], cs[s], dI2[s]);
                                load_meta(dIt[s], pm[s], dI2[s]);
                            }
                        } else {
                            dBt[s] = te;
                        }
                        compute(acur, bcur);
                    } else {
                        more = false;
                    }
                }
            }
            flush(gfirst, k, rwk);
            if (sync && lp < sy.npanels - 1) announce(g, lp + 1, sy.npanels - 1);
            return;
        }
#pragma unroll
        for (int s = 0; s < S; ++s)
            if (tb + s < te) {
                load_cs(tb + s, cs[s]);
                load_meta(tb + s, pm[s]);
            }
        skip_empty();
#pragma unroll
        for (int s = 0; s < S; ++s)
            if (tb + s < te) {
                gate(__builtin_amdgcn_readfirstlane(cs[s][0]));
                select_cid(cs[s], cid);
                load_b(cid, bv[s]);
                issue_a(tb + s, s);
            }
#pragma unroll
        for (int s = 0; s < S; ++s)
            if (tb + S + s < te) {
                load_cs(tb + S + s, cs[s]);
                load_meta(tb + S + s, pm[s]);
            }

        for (int t0 = tb; t0 < te; t0 += S) {
#pragma unroll
            for (int s = 0; s < S; ++s) {
                const int t = t0 + s;
                if (t < te) {
                    advance_task(t);
                    stage_b(bv[s]);
                    u4 bcur[NV];
#pragma unroll
                    for (int i = 0; i < NV; ++i) bcur[i] = DB ? bv[s][i] : u4{0u, 0u, 0u, 0u};
                    uint32_t acur[RG][AW];
                    take_a(s, acur);
                    if (t + S < te) {
                        gate(__builtin_amdgcn_readfirstlane(cs[s][0]));
                        select_cid(cs[s], cid);
                        load_b(cid, bv[s]);
                        issue_a(t + S, s);
                        if (t + 2 * S < te) {
                            load_cs(t + 2 * S, cs[s]);
                            load_meta(t + 2 * S, pm[s]);
                        }
                    }
                    compute(acur, bcur);
                }
            }
        }
        flush(gfirst, k, rwk);
        if (sync && lp < sy.npanels - 1) announce(g, lp + 1, sy.npanels - 1);
    };

    // Work item of this wave in each generation (one generation unless the
    // sweep is synchronised).
    for (int g = 0; g < (SY ? sy.ngen : 1); ++g) {
        long long r = -1;
        int chunk = 0;
        if (placement == kPlaceChunkXcd) {
            // XCD x (workgroup b runs on XCD b % 8) serves chunk x % nchunks;
            // the group's 8 / nchunks XCDs take runs of kXcdRun workgroups in
            // turn (never synchronised)
            const int x = blockIdx.x % kXcds, kk = blockIdx.x / kXcds, nx = kXcds / nchunks;
            const long long j = ((long long)(kk / kXcdRun) * nx + x / nchunks) * kXcdRun + kk % kXcdRun;
            const long long rr = j * kWavesPerBlock + wid;
            if (rr < nranges) {
                r = rr;
                chunk = x % nchunks;
            }
        } else {
            const int lb = place_block(blockIdx.x, gridDim.x, placement);
            const long long gw = ((long long)g * gridDim.x + lb) * kWavesPerBlock + wid;
            if (gw < nranges * nchunks) {
                // chunk_major: all task ranges of chunk 0, then chunk 1, ...
                // (the live B working set of a phase is one chunk's columns);
                // otherwise the chunks of one range are neighbours (the A
                // tiles are reused from L2).
                if (nchunks == 1) {
                    r = gw;
                } else {
                    r = chunk_major ? gw % nranges : gw / nchunks;
                    chunk = chunk_major ? (int)(gw / nranges) : (int)(gw - r * nchunks);
                }
            }
        }
        if (r >= 0) run(g, (int)r, chunk);
    }
}

// Host-side address of one instantiation for a launch precision
// (TSP_PREC_FP16, TSP_PREC_TF32, kPrecTf32Exact, or kPrecTf32B3 without the
// panel sweep -- nullptr with it); taking it instantiates the kernel.
template <int BM, int W, int S, bool PK, bool LI, bool SY>
const void *pick_kernel(int prec)
{
    if (prec == TSP_PREC_FP16) return (const void *)&spmm_kernel<BM, W, TSP_PREC_FP16, S, PK, LI, SY>;
    if (prec == kPrecTf32Exact) return (const void *)&spmm_kernel<BM, W, kPrecTf32Exact, S, PK, LI, SY>;
    if (prec == kPrecTf32B3) {
        if constexpr (!SY) return (const void *)&spmm_kernel<BM, W, kPrecTf32B3, S, PK, LI, SY>;
        return nullptr;
    }
    return (const void *)&spmm_kernel<BM, W, TSP_PREC_TF32, S, PK, LI, SY>;
}

// Tile-pair instantiations: fp16, and tf32 operands that are tf32 values
// already for 8-row tiles at 64-column chunks (nullptr otherwise).
template <int BM, int W, int S, bool PK, bool LI, bool SY>
const void *pick_pair_kernel(int prec)
{
    if (prec == TSP_PREC_FP16) return (const void *)&spmm_kernel<BM, W, TSP_PREC_FP16, S, PK, LI, SY, true>;
    if constexpr (BM == 8 && W == 64 && !SY)
        if (prec == kPrecTf32Exact) return (const void *)&spmm_kernel<BM, W, kPrecTf32Exact, S, PK, LI, SY, true>;
    return nullptr;
}

}  // namespace tsp

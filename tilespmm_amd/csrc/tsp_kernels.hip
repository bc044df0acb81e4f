// tsp_kernels.hip -- MI355X (gfx950, CDNA4) tile SpMM kernels.
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
//     read and owns CB adjacent output columns (one vector store per row);
//   * A tiles are canonical row-major BM x BN blocks read straight into MFMA
//     operand registers (8 or 16 bytes per lane);
//   * fp16: v_mfma_f32_16x16x16_f16 (BN = 16) and v_mfma_f32_16x16x32_f16
//     (BN = 32), fp32 accumulate; 8-row tiles occupy rows 0-7 of the 16-row
//     MFMA block;
//   * tf32: operands are rounded to tf32 (nearest-even, 10 mantissa bits) in
//     registers and multiplied with v_mfma_f32_16x16x4_f32 -- a tf32 product
//     is exact in fp32, so this is tf32 arithmetic with fp32 accumulate
//     (CDNA4 has no xf32 MFMA);
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

// PK selects the bitmap-packed A format (8- and 16-row classes): per tile a
// row-major occupancy bitmap (BM*BN bits, bit r*BN+c) in `bmp`, and the values
// of its set bits, in bit order, at `val_` + vptr[tile].  Each lane expands its
// slice of the tile into MFMA operand registers.  Without PK, `val_` holds
// dense canonical tiles and `bmp` / `vptr` are unused.
template <int BM, int W, int PREC, int S, bool PK, bool LI>
__global__ __launch_bounds__(kBlockThreads) void spmm_kernel(
    int ntasks, int nchunks, int tasks_per_wave, int chunk_major, const void *__restrict__ val_,
    const uint64_t *__restrict__ bmp, const int *__restrict__ vptr,
    const unsigned *__restrict__ rows, const int *__restrict__ colstart,
    const void *__restrict__ B_, float *__restrict__ C, const int *__restrict__ colidx, int ld,
    int c_rows, int placement)
{
    constexpr bool F16 = PREC == TSP_PREC_FP16;
    // tf32 operands are rounded in registers, unless the launch guarantees
    // they are tf32 values already (kPrecTf32Exact: the plan rounds its copies
    // of A and B once when they enter it)
    constexpr bool RND = PREC == TSP_PREC_TF32;
    auto rnd = [](uint32_t x) { return RND ? round_tf32_bits(x) : x; };
    constexpr int BN = tile_bn(BM, PREC);
    constexpr int VV = F16 ? 8 : 4;          // values per 16-byte vector
    constexpr int VPR = W / VV;              // vectors per panel row
    constexpr int NV = BN * VPR / 64;        // vectors per lane per tile
    static_assert(NV >= 1 && (BN * VPR) % 64 == 0, "panel does not tile the wave");
    // LDS row stride: a multiple of the CB-value vectors the MFMA operand
    // reads use (up to 32 bytes), padded so consecutive rows shift banks
    constexpr int LDSW = W + 8;
    constexpr int RG = BM >= 16 ? BM / 16 : 1;   // 16-row MFMA row groups
    constexpr int CB = W / 16;                   // 16-column MFMA blocks
    constexpr int KS = F16 ? 1 : BN / 4;         // tf32 MFMA steps per tile
    constexpr int AW = F16 ? (BN == 32 ? 4 : 2) : KS;   // A words per row group
    using VT = typename std::conditional<F16, _Float16, float>::type;
    using RV = VT __attribute__((ext_vector_type(CB)));     // CB values of one B row
    constexpr int PWD = PK ? BM * BN / 64 : 1;               // packed: bitmap words per tile
    struct PMeta {
        uint64_t bw[PWD];
        int vbase;
    };
    using FV = float __attribute__((ext_vector_type(CB)));  // CB output columns

    __shared__ __attribute__((aligned(32))) VT lds_all[kWavesPerBlock][BN * LDSW];

    const int lane = threadIdx.x & 63;
    const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // uniform per wave
    const long long nranges = ((long long)ntasks + tasks_per_wave - 1) / tasks_per_wave;
    int range, chunk;
    if (placement == kPlaceChunkXcd) {
        // XCD x (workgroup b runs on XCD b % 8) serves chunk x % nchunks; the
        // group's 8 / nchunks XCDs take runs of kXcdRun workgroups in turn
        const int x = blockIdx.x % kXcds, k = blockIdx.x / kXcds, nx = kXcds / nchunks;
        const long long j = ((long long)(k / kXcdRun) * nx + x / nchunks) * kXcdRun + k % kXcdRun;
        const long long r = j * kWavesPerBlock + wid;
        if (r >= nranges) return;
        range = (int)r;
        chunk = x % nchunks;
    } else {
        const int lb = place_block(blockIdx.x, gridDim.x, placement);
        const long long gw = (long long)lb * kWavesPerBlock + wid;
        if (gw >= nranges * nchunks) return;
        // chunk_major: all task ranges of chunk 0, then chunk 1, ... (the
        // live B working set of a phase is one chunk's columns); otherwise
        // the chunks of one range are neighbours (the A tiles are reused
        // from L2).
        range = chunk_major ? (int)(gw % nranges) : (int)(gw / nchunks);
        chunk = chunk_major ? (int)(gw / nranges) : (int)(gw - (long long)range * nchunks);
    }
    const int k0 = range * tasks_per_wave;
    const int k1 = min(ntasks, k0 + tasks_per_wave);
    const int tb = uload(colstart, k0), te = uload(colstart, k1);
    if (tb >= te) return;                        // every task of the range is empty
    int k = k0;
    int kend = uload(colstart, k0 + 1);
    while (kend <= tb) kend = uload(colstart, ++k + 1);  // skip leading empty tasks
    int gfirst = k;                  // first task of the accumulation group
    const int col0 = chunk * W;

    VT *lds = lds_all[wid];
    const VT *val = (const VT *)val_;
    const char *Bb = (const char *)B_;
    const int ln = lane & 15;        // MFMA row (A) / column (B, D) index
    const int lq = lane >> 4;        // MFMA lane group

    // Panel rows of the lane's NV B loads.  Scalar column indices (LI
    // false): load i covers rows i*RPI .. i*RPI+RPI-1, row i*RPI + lane/VPR
    // for this lane.  Lane-loaded indices (LI): the lane's rows are the NV
    // consecutive rows (lane/VPR)*NV + i, whose column indices are
    // consecutive in the tile's index list (one vector load).
    int prow[NV], pcol[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int v = lane + 64 * i;
        prow[i] = LI ? (lane / VPR) * NV + i : v / VPR;
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
    auto load_meta = [&](int t, PMeta &m) {
        if constexpr (PK) {
#pragma unroll
            for (int w = 0; w < PWD; ++w) m.bw[w] = uload(bmp, (size_t)t * PWD + w);
            m.vbase = uload(vptr, t);
        }
    };
    // Packed A in two halves, so a wave never waits for a load it has just
    // issued: issue_a_packed (S tiles ahead) computes the lane's position in
    // the packed stream from the scalar bitmap words, loads its NVAL
    // consecutive values raw and keeps its NVAL occupancy bits; finish_a_packed
    // (just before the tile's MFMAs) expands them into operand registers.
    constexpr int NVAL = F16 ? 4 : KS;           // packed: operand values per lane
    auto issue_a_packed = [&](const PMeta &m, VT (&raw)[NVAL], uint32_t &nib) {
        static_assert(!PK || BM <= 16, "packed tiles are 8- or 16-row");
        constexpr int WD = PWD;                  // bitmap words per tile
        const uint64_t *bw = m.bw;
        const int vbase = m.vbase;
        if (BM == 8 && ln >= 8) {
#pragma unroll
            for (int j = 0; j < NVAL; ++j) raw[j] = (VT)0;
            nib = 0u;
            return;
        }
        // first bit of this lane's slots; NVAL-bit groups never straddle words
        const int p = ln * BN + NVAL * lq;
        int pre = 0;
        uint64_t word = bw[0];
#pragma unroll
        for (int w = 0; w < WD; ++w) {
            const int lo = 64 * w;
            const uint64_t m = p >= lo + 64 ? ~0ull : (p <= lo ? 0ull : ((1ull << (p - lo)) - 1ull));
            pre += __popcll(bw[w] & m);
            if (p >= lo && p < lo + 64) word = bw[w];
        }
        nib = (unsigned)(word >> (p & 63)) & ((1u << NVAL) - 1u);
        // the lane's values are consecutive in the packed stream (the value
        // array is padded, so reading NVAL of them is always in bounds)
        const VT *pv = val + vbase + pre;
#pragma unroll
        for (int j = 0; j < NVAL; ++j) raw[j] = pv[j];
    };
    auto finish_a_packed = [&](const VT (&v)[NVAL], uint32_t nib, uint32_t (&dst)[RG][AW]) {
        VT o[NVAL];
        int idx = 0;
#pragma unroll
        for (int j = 0; j < NVAL; ++j) {
            const bool b = (nib >> j) & 1u;
            VT x = v[0];
#pragma unroll
            for (int q = 1; q < NVAL; ++q) x = idx == q ? v[q] : x;
            o[j] = b ? x : (VT)0;
            idx += b ? 1 : 0;
        }
        if constexpr (F16) {
            const h4 hv = h4{o[0], o[1], o[2], o[3]};
            const u2 bits = __builtin_bit_cast(u2, hv);
            dst[0][0] = bits.x;
            dst[0][1] = bits.y;
        } else {
#pragma unroll
            for (int j = 0; j < NVAL; ++j) dst[0][j] = rnd(__float_as_uint(o[j]));
        }
    };
    auto load_a = [&](int t, uint32_t (&dst)[RG][AW]) {
        const VT *tile = val + (size_t)t * (BM * BN);
#pragma unroll
        for (int g = 0; g < RG; ++g) {
            const int r = 16 * g + ln;
            if (BM == 8 && ln >= 8) {
#pragma unroll
                for (int w = 0; w < AW; ++w) dst[g][w] = 0u;
                continue;
            }
            if constexpr (F16) {
                const u2 lo = *(const u2 *)(tile + r * BN + 4 * lq);
                dst[g][0] = lo.x; dst[g][1] = lo.y;
                if constexpr (BN == 32) {
                    const u2 hi = *(const u2 *)(tile + r * BN + 16 + 4 * lq);
                    dst[g][2] = hi.x; dst[g][3] = hi.y;
                }
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
    using CSV = int __attribute__((ext_vector_type(LI ? NV : BN)));
    auto load_cs = [&](int t, CSV &cs) {
        if constexpr (LI) cs = *(const CSV *)(colidx + (size_t)t * BN + lrow * NV);
        else cs = *(cptr<CSV>)(colidx + (size_t)t * BN);
    };
    auto select_cid = [&](const CSV &cs, int (&dst)[NV]) {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            if constexpr (LI) {
                dst[i] = cs[i];
            } else {
                int v = cs[i * RPI];
#pragma unroll
                for (int r = 1; r < RPI; ++r) v = lrow == r ? cs[i * RPI + r] : v;
                dst[i] = v;
            }
        }
    };
    auto load_b = [&](const int (&cid)[NV], u4 (&dst)[NV]) {
#pragma unroll
        for (int i = 0; i < NV; ++i)
            dst[i] = *(const u4 *)(Bb + ((size_t)cid[i] * ld + col0 + pcol[i]) * sizeof(VT));
    };
    // Flush the accumulators of tasks first..last, which this wave ran back
    // to back and which share one row-block.  A split task (bit 31) is added
    // atomically, as the reference does, whatever the order of the schedule.
    // Only a group of several tasks of one split row-block may store: when
    // the tasks just before and after the group belong to other row-blocks,
    // this wave ran every task of it (a split row-block's tasks are
    // consecutive, as tile_pretreatment emits them).
    auto flush = [&](int first, int last) {
        const unsigned rw = uload(rows, last);
        const int row0 = (int)(rw & 0x7fffffffu);
        bool split = (rw & 0x80000000u) != 0;
        if (split && first < last) {
            const bool from_start = first == 0 || (int)(uload(rows, first - 1) & 0x7fffffffu) != row0;
            const bool to_end = last + 1 >= ntasks || (int)(uload(rows, last + 1) & 0x7fffffffu) != row0;
            split = !(from_start && to_end);
        }
        if (!split) {
            // MFMA column n of block c is output column n*CB + c: the lane
            // owns CB adjacent columns of each of its rows (one vector store)
#pragma unroll
            for (int g = 0; g < RG; ++g) {
                if (BM == 8 && lq >= 2) break;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int r = row0 + 16 * g + 4 * lq + j;
                    if (r >= c_rows) continue;
                    FV v;
#pragma unroll
                    for (int c = 0; c < CB; ++c) v[c] = acc[g][c][j];
                    __builtin_nontemporal_store(v, (FV *)(C + (size_t)r * ld + col0 + ln * CB));
                }
            }
        } else {
            // fp32 atomics are issued per lane: transpose each 8-row slab
            // through the wave's (now idle) B panel in LDS so that every
            // atomic instruction covers whole rows of consecutive columns
            static_assert(BN * LDSW * sizeof(VT) >= 8 * W * sizeof(float), "panel too small for a slab");
            float *tr = (float *)lds;
#pragma unroll
            for (int h = 0; h < BM / 8; ++h) {
                if ((lq >> 1) == (h & 1)) {
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        FV v;
#pragma unroll
                        for (int c = 0; c < CB; ++c) v[c] = acc[h >> 1][c][j];
                        *(FV *)(tr + (4 * (lq & 1) + j) * W + ln * CB) = v;
                    }
                }
                __builtin_amdgcn_wave_barrier();
#pragma unroll
                for (int i = 0; i < 8 * W / 64; ++i) {
                    const int idx = lane + 64 * i;
                    const int rr = idx / W, col = idx % W;
                    const int r = row0 + 8 * h + rr;
                    const float x = tr[rr * W + col];
                    if (r < c_rows) unsafeAtomicAdd(C + (size_t)r * ld + col0 + col, x);
                }
                __builtin_amdgcn_wave_barrier();
            }
        }
#pragma unroll
        for (int g = 0; g < RG; ++g)
#pragma unroll
            for (int c = 0; c < CB; ++c) acc[g][c] = f4{0.f, 0.f, 0.f, 0.f};
    };
    // B operand of MFMA block c at lane (n = ln, group lq): column n*CB + c
    // of the chunk, so one LDS read of CB adjacent values per B row serves
    // all CB blocks.
    auto compute = [&](const uint32_t (&a)[RG][AW]) {
        const VT *lb = lds + ln * CB;
        if constexpr (F16) {
            constexpr int KR = BN == 16 ? 4 : 8;     // B rows of one lane
            RV rv[KR];
#pragma unroll
            for (int j = 0; j < 4; ++j) rv[j] = *(const RV *)(lb + (4 * lq + j) * LDSW);
            if constexpr (BN == 32) {
#pragma unroll
                for (int j = 0; j < 4; ++j) rv[4 + j] = *(const RV *)(lb + (16 + 4 * lq + j) * LDSW);
            }
#pragma unroll
            for (int c = 0; c < CB; ++c) {
                if constexpr (BN == 16) {
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
        } else {
#pragma unroll
            for (int s = 0; s < KS; ++s) {
                const RV rv = *(const RV *)(lb + (KS * lq + s) * LDSW);
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
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            u4 x = src[i];
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
    VT araw[S][NVAL];                 // packed A: raw values and occupancy bits
    uint32_t anib[S];
    CSV cs[S];
    PMeta pm[S];
    int cid[NV];
    auto issue_a = [&](int t, int s) {
        if constexpr (PK) issue_a_packed(pm[s], araw[s], anib[s]);
        else load_a(t, ar[s]);
    };
#pragma unroll
    for (int s = 0; s < S; ++s)
        if (tb + s < te) {
            load_cs(tb + s, cs[s]);
            load_meta(tb + s, pm[s]);
        }
#pragma unroll
    for (int s = 0; s < S; ++s)
        if (tb + s < te) {
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
                if (t >= kend) {                 // task k is complete
                    int kn = k;
                    do kend = uload(colstart, ++kn + 1);
                    while (kend <= t);           // skip empty tasks
                    // the next task continues the same row-block: keep
                    // accumulating instead of flushing partial sums
                    const bool same = (uload(rows, kn) & 0x7fffffffu) == (uload(rows, k) & 0x7fffffffu);
                    if (!same) {
                        flush(gfirst, k);
                        gfirst = kn;
                    }
                    k = kn;
                }
                stage_b(bv[s]);
                uint32_t acur[RG][AW];
                if constexpr (PK) {
                    finish_a_packed(araw[s], anib[s], acur);
                } else {
#pragma unroll
                    for (int g = 0; g < RG; ++g)
#pragma unroll
                        for (int w = 0; w < AW; ++w) acur[g][w] = ar[s][g][w];
                }
                if (t + S < te) {
                    select_cid(cs[s], cid);
                    load_b(cid, bv[s]);
                    issue_a(t + S, s);
                    if (t + 2 * S < te) {
                        load_cs(t + 2 * S, cs[s]);
                        load_meta(t + 2 * S, pm[s]);
                    }
                }
                compute(acur);
            }
        }
    }
    flush(gfirst, k);
}

__global__ __launch_bounds__(256) void copy_kernel(u4 *__restrict__ dst, const u4 *__restrict__ src, size_t n)
{
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (; i < n; i += stride) dst[i] = src[i];
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
    return w == 32 || w == 64 || w == 128;
}

#define TSP_FOR_EACH_VARIANT(X)                                                                \
    X(64, 32, 1) X(64, 32, 2) X(64, 32, 3)                                                     \
    X(64, 64, 1) X(64, 64, 2) X(64, 64, 3)                                                     \
    X(16, 32, 1) X(16, 32, 2) X(16, 32, 3)                                                     \
    X(16, 64, 1) X(16, 64, 2) X(16, 64, 3)                                                     \
    X(16, 128, 1) X(16, 128, 2) X(16, 128, 3)                                                  \
    X(8, 32, 1) X(8, 32, 2) X(8, 32, 3)                                                        \
    X(8, 64, 1) X(8, 64, 2) X(8, 64, 3)                                                        \
    X(8, 128, 1) X(8, 128, 2) X(8, 128, 3)

#define TSP_FOR_EACH_PACKED_VARIANT(X)                                                         \
    X(16, 32, 1) X(16, 32, 2) X(16, 32, 3)                                                     \
    X(16, 64, 1) X(16, 64, 2) X(16, 64, 3)                                                     \
    X(16, 128, 1) X(16, 128, 2) X(16, 128, 3)                                                  \
    X(8, 32, 1) X(8, 32, 2) X(8, 32, 3)                                                        \
    X(8, 64, 1) X(8, 64, 2) X(8, 64, 3)                                                        \
    X(8, 128, 1) X(8, 128, 2) X(8, 128, 3)

const void *select_kernel(int bm, int prec, int w, int s, bool packed, bool lane_idx)
{
#define TSP_K(BMv, Wv, Sv, PKv, LIv)                                                                    \
    if (packed == PKv && lane_idx == LIv && bm == BMv && w == Wv && s == Sv)                            \
        return prec == TSP_PREC_FP16   ? (const void *)&spmm_kernel<BMv, Wv, TSP_PREC_FP16, Sv, PKv, LIv>  \
               : prec == kPrecTf32Exact ? (const void *)&spmm_kernel<BMv, Wv, kPrecTf32Exact, Sv, PKv, LIv> \
                                       : (const void *)&spmm_kernel<BMv, Wv, TSP_PREC_TF32, Sv, PKv, LIv>;
#define TSP_KD(BMv, Wv, Sv) TSP_K(BMv, Wv, Sv, false, false)
#define TSP_KP(BMv, Wv, Sv) TSP_K(BMv, Wv, Sv, true, false)
#define TSP_KL(BMv, Wv, Sv) TSP_K(BMv, Wv, Sv, true, true)
    TSP_FOR_EACH_VARIANT(TSP_KD)
    TSP_FOR_EACH_PACKED_VARIANT(TSP_KP)
    TSP_FOR_EACH_PACKED_VARIANT(TSP_KL)
#undef TSP_KD
#undef TSP_KP
#undef TSP_KL
#undef TSP_K
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

int launch(int bm, int prec, int ntasks, int colB_p, const void *val, const uint64_t *bmp,
           const int *vptr, const unsigned *rows, const int *colstart, const void *B, float *C,
           const int *colidx, int c_rows, hipStream_t st, int w, int s, int tpw, int order,
           int placement, bool lane_idx)
{
    const bool packed = bmp != nullptr;
    if (packed && (bm == 64 || !vptr)) return TSP_EINVAL;
    if (lane_idx && !packed) return TSP_EINVAL;          // lane-loaded indices: packed kernels only
    if (placement != kPlaceContiguous && placement != kPlaceInterleaved && placement != kPlaceChunkXcd)
        return TSP_EINVAL;
    int nchunks = 0, cm = 0;
    if (!resolve_variant(bm, prec, colB_p, w, s, nchunks, tpw, order, cm)) return TSP_EINVAL;
    if (placement == kPlaceChunkXcd && (nchunks < 2 || kXcds % nchunks != 0)) return TSP_EINVAL;
    const long long ranges = ((long long)ntasks + tpw - 1) / tpw;
    const long long waves = ranges * nchunks;
    long long blocks = (waves + kWavesPerBlock - 1) / kWavesPerBlock;
    if (blocks <= 0) return 0;
    if (placement == kPlaceInterleaved) {
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
    const dim3 grid3((unsigned)blocks);
#define TSP_L(BMv, Wv, Sv, PKv, LIv)                                                            \
    if (packed == PKv && lane_idx == LIv && bm == BMv && w == Wv && s == Sv) {                  \
        if (prec == TSP_PREC_FP16)                                                              \
            spmm_kernel<BMv, Wv, TSP_PREC_FP16, Sv, PKv, LIv><<<grid3, kBlockThreads, 0, st>>>(  \
                ntasks, nchunks, tpw, cm, val, bmp, vptr, rows, colstart, B, C, colidx, colB_p, \
                c_rows, placement);                                                             \
        else if (prec == kPrecTf32Exact)                                                        \
            spmm_kernel<BMv, Wv, kPrecTf32Exact, Sv, PKv, LIv><<<grid3, kBlockThreads, 0, st>>>( \
                ntasks, nchunks, tpw, cm, val, bmp, vptr, rows, colstart, B, C, colidx, colB_p, \
                c_rows, placement);                                                             \
        else                                                                                    \
            spmm_kernel<BMv, Wv, TSP_PREC_TF32, Sv, PKv, LIv><<<grid3, kBlockThreads, 0, st>>>(  \
                ntasks, nchunks, tpw, cm, val, bmp, vptr, rows, colstart, B, C, colidx, colB_p, \
                c_rows, placement);                                                             \
        return (int)hipGetLastError();                                                          \
    }
#define TSP_LD(BMv, Wv, Sv) TSP_L(BMv, Wv, Sv, false, false)
#define TSP_LP(BMv, Wv, Sv) TSP_L(BMv, Wv, Sv, true, false)
#define TSP_LL(BMv, Wv, Sv) TSP_L(BMv, Wv, Sv, true, true)
    TSP_FOR_EACH_VARIANT(TSP_LD)
    TSP_FOR_EACH_PACKED_VARIANT(TSP_LP)
    TSP_FOR_EACH_PACKED_VARIANT(TSP_LL)
#undef TSP_LD
#undef TSP_LP
#undef TSP_LL
#undef TSP_L
    return TSP_EINVAL;
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

// tsp_kernels.hip -- MI355X (gfx950, CDNA4) tile SpMM kernels.
//
// One kernel template serves the three row-block classes (BM = 64, 16, 8) of
// both precisions.  It computes, for every task of the schedule,
//     C[start .. start+BM)[cols] (= or atomically +=)
//         sum over the task's tiles of  A_tile(BM x BN) * B[colidx[tile]][cols]
// which is what the reference's stir_spmm_cuda_kernel_v{8,16,64}[_tf32][_32]
// compute (src/tilespmm_cuda.h:12-1632).  The design is CDNA4-first, not a
// translation:
//   * one wave64 owns one (task, column chunk of W columns); a 256-thread
//     block runs four independent waves, so no block barrier exists at all;
//   * the gathered B row panel (BN rows x W columns) is loaded with 16-byte
//     vector loads and staged in a wave-private LDS slice; one wave's LDS
//     operations execute in issue order, so a single buffer is safe;
//   * A tiles are canonical row-major BM x BN blocks read straight into MFMA
//     operand registers (8 or 16 bytes per lane);
//   * fp16: v_mfma_f32_16x16x16_f16 (BN = 16) and v_mfma_f32_16x16x32_f16
//     (BN = 32), fp32 accumulate; 8-row tiles occupy rows 0-7 of the 16-row
//     MFMA block;
//   * tf32: operands are rounded to tf32 (nearest-even, 10 mantissa bits) in
//     registers and multiplied with v_mfma_f32_16x16x4_f32 -- a tf32 product
//     is exact in fp32, so this is tf32 arithmetic with fp32 accumulate
//     (CDNA4 has no xf32 MFMA);
//   * the column indices of tile t+1 are loaded while tile t is computed, the
//     B panel and A fragment of tile t+1 are in flight during tile t's MFMAs;
//   * block ids are remapped so that consecutive tasks (which tend to share B
//     rows) run on the same XCD and share its L2.
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
typedef float f2 __attribute__((ext_vector_type(2)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t round_tf32_bits(uint32_t x)
{
    return (x + 0xfffu + ((x >> 13) & 1u)) & 0xffffe000u;
}

__device__ __forceinline__ float round_tf32(float f)
{
    return __uint_as_float(round_tf32_bits(__float_as_uint(f)));
}

// Block id -> logical block id such that each XCD (blocks are dealt to the 8
// XCDs round-robin) receives one contiguous range of logical blocks.
__device__ __forceinline__ int xcd_remap(int b, int nb)
{
    const int q = nb >> 3, r = nb & 7;
    const int x = b & 7, k = b >> 3;
    return x < r ? x * (q + 1) + k : r * (q + 1) + (x - r) * q + k;
}

template <int BM, int W, int PREC>
__global__ __launch_bounds__(kBlockThreads) void spmm_kernel(
    int ntasks, int nchunks, const void *__restrict__ val_, const unsigned *__restrict__ rows,
    const int *__restrict__ colstart, const void *__restrict__ B_, float *__restrict__ C,
    const int *__restrict__ colidx, int ld, int c_rows)
{
    constexpr bool F16 = PREC == TSP_PREC_FP16;
    constexpr int BN = tile_bn(BM, PREC);
    constexpr int VV = F16 ? 8 : 4;          // values per 16-byte vector
    constexpr int VPR = W / VV;              // vectors per panel row
    constexpr int NV = BN * VPR / 64;        // vectors per lane per tile
    static_assert(NV >= 1 && (BN * VPR) % 64 == 0, "panel does not tile the wave");
    constexpr int LDSW = F16 ? W + 4 : W + (BN == 8 ? 8 : 4);
    constexpr int RG = BM >= 16 ? BM / 16 : 1;   // 16-row MFMA row groups
    constexpr int CB = W / 16;                   // 16-column MFMA blocks
    constexpr int KS = F16 ? 1 : BN / 4;         // tf32 MFMA steps per tile
    using VT = typename std::conditional<F16, _Float16, float>::type;

    __shared__ __attribute__((aligned(16))) VT lds_all[kWavesPerBlock][BN * LDSW];

    const int lane = threadIdx.x & 63;
    const int wid = threadIdx.x >> 6;
    const int lb = xcd_remap(blockIdx.x, gridDim.x);
    const long long gw = (long long)lb * kWavesPerBlock + wid;
    if (gw >= (long long)ntasks * nchunks) return;
    const int task = (int)(gw / nchunks);
    const int chunk = (int)(gw - (long long)task * nchunks);
    const int ts = colstart[task], te = colstart[task + 1];
    if (ts >= te) return;
    const unsigned rw = rows[task];
    const bool split = (rw & 0x80000000u) != 0;
    const int row0 = (int)(rw & 0x7fffffffu);
    const int col0 = chunk * W;

    VT *lds = lds_all[wid];
    const VT *val = (const VT *)val_;
    const char *Bb = (const char *)B_;
    const int ln = lane & 15;        // MFMA row (A) / column (B, D) index
    const int lq = lane >> 4;        // MFMA lane group

    // Per-lane geometry of the B panel vectors.
    int prow[NV], pcol[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int v = lane + 64 * i;
        prow[i] = v / VPR;
        pcol[i] = (v % VPR) * VV;
    }

    f4 acc[RG][CB];
#pragma unroll
    for (int g = 0; g < RG; ++g)
#pragma unroll
        for (int c = 0; c < CB; ++c) acc[g][c] = f4{0.f, 0.f, 0.f, 0.f};

    // A operand registers: fp16 -> 4 halves (BN=16) or 8 halves (BN=32) per
    // row group; tf32 -> KS floats per row group.
    constexpr int AW = F16 ? (BN == 32 ? 4 : 2) : KS;   // 32-bit words per row group
    uint32_t areg[RG][AW];

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
                    dst[g][0] = round_tf32_bits(x.x); dst[g][1] = round_tf32_bits(x.y);
                } else {
                    const u4 x = *(const u4 *)p;
                    dst[g][0] = round_tf32_bits(x.x); dst[g][1] = round_tf32_bits(x.y);
                    dst[g][2] = round_tf32_bits(x.z); dst[g][3] = round_tf32_bits(x.w);
                }
            }
        }
    };

    int cid[NV];
    u4 bv[NV];
    auto load_cid = [&](int t) {
#pragma unroll
        for (int i = 0; i < NV; ++i) cid[i] = colidx[(size_t)t * BN + prow[i]];
    };
    auto load_b = [&]() {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const char *p = Bb + ((size_t)cid[i] * ld + col0 + pcol[i]) * sizeof(VT);
            bv[i] = *(const u4 *)p;
        }
    };

    // Prologue: tile ts in flight, column indices of ts+1 in flight.
    load_cid(ts);
    load_b();
    load_a(ts, areg);
    if (ts + 1 < te) load_cid(ts + 1);

    for (int t = ts; t < te; ++t) {
        // Stage tile t's B panel in LDS (tf32 operands rounded on the way).
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            u4 x = bv[i];
            if constexpr (!F16) {
                x.x = round_tf32_bits(x.x); x.y = round_tf32_bits(x.y);
                x.z = round_tf32_bits(x.z); x.w = round_tf32_bits(x.w);
            }
            VT *d = lds + prow[i] * LDSW + pcol[i];
            if constexpr (F16) {
                *(u2 *)d = u2{x.x, x.y};
                *(u2 *)(d + 4) = u2{x.z, x.w};
            } else {
                *(u4 *)d = x;
            }
        }
        uint32_t acur[RG][AW];
#pragma unroll
        for (int g = 0; g < RG; ++g)
#pragma unroll
            for (int w = 0; w < AW; ++w) acur[g][w] = areg[g][w];

        // Issue tile t+1's loads, and the column indices of t+2.
        if (t + 1 < te) {
            load_b();
            load_a(t + 1, areg);
            if (t + 2 < te) load_cid(t + 2);
        }

        // MFMAs on tile t.
#pragma unroll
        for (int c = 0; c < CB; ++c) {
            const int col = 16 * c + ln;
            if constexpr (F16) {
                if constexpr (BN == 16) {
                    h4 b;
#pragma unroll
                    for (int j = 0; j < 4; ++j) b[j] = lds[(4 * lq + j) * LDSW + col];
#pragma unroll
                    for (int g = 0; g < RG; ++g) {
                        h4 a;
                        u2 ab = u2{acur[g][0], acur[g][1]};
                        a = __builtin_bit_cast(h4, ab);
                        acc[g][c] = __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, acc[g][c], 0, 0, 0);
                    }
                } else {
                    h8 b;
#pragma unroll
                    for (int j = 0; j < 4; ++j) b[j] = lds[(4 * lq + j) * LDSW + col];
#pragma unroll
                    for (int j = 0; j < 4; ++j) b[4 + j] = lds[(16 + 4 * lq + j) * LDSW + col];
#pragma unroll
                    for (int g = 0; g < RG; ++g) {
                        u4 ab = u4{acur[g][0], acur[g][1], acur[g][2], acur[g][3]};
                        h8 a = __builtin_bit_cast(h8, ab);
                        acc[g][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc[g][c], 0, 0, 0);
                    }
                }
            } else {
#pragma unroll
                for (int s = 0; s < KS; ++s) {
                    const float b = lds[(KS * lq + s) * LDSW + col];
#pragma unroll
                    for (int g = 0; g < RG; ++g) {
                        acc[g][c] = __builtin_amdgcn_mfma_f32_16x16x4f32(
                            __uint_as_float(acur[g][s]), b, acc[g][c], 0, 0, 0);
                    }
                }
            }
        }
    }

    // Epilogue: lane (ln, lq) holds D[4*lq + j][ln] of every 16x16 block.
#pragma unroll
    for (int g = 0; g < RG; ++g) {
        if (BM == 8 && lq >= 2) break;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int r = row0 + 16 * g + 4 * lq + j;
            if (r >= c_rows) continue;
            float *crow = C + (size_t)r * ld + col0 + ln;
#pragma unroll
            for (int c = 0; c < CB; ++c) {
                if (split) unsafeAtomicAdd(crow + 16 * c, acc[g][c][j]);
                else crow[16 * c] = acc[g][c][j];
            }
        }
    }
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
int chunk_width(int bm, int colB_p)
{
    if (colB_p == 32) return 32;
    if (bm == 64) return 64;
    return (colB_p % 128 == 0) ? 128 : 64;
}

template <int BM, int W, int PREC>
static const void *kernel_ptr()
{
    return (const void *)&spmm_kernel<BM, W, PREC>;
}

const void *select_kernel(int bm, int prec, int w)
{
#define TSP_K(BMv, Wv)                                                              \
    if (bm == BMv && w == Wv)                                                      \
        return prec == TSP_PREC_FP16 ? kernel_ptr<BMv, Wv, TSP_PREC_FP16>()        \
                                     : kernel_ptr<BMv, Wv, TSP_PREC_TF32>();
    TSP_K(64, 32) TSP_K(64, 64)
    TSP_K(16, 32) TSP_K(16, 64) TSP_K(16, 128)
    TSP_K(8, 32) TSP_K(8, 64) TSP_K(8, 128)
#undef TSP_K
    return nullptr;
}

template <int BM, int W, int PREC>
static void launch_t(dim3 grid, hipStream_t s, int ntasks, int nchunks, const void *val,
                     const unsigned *rows, const int *colstart, const void *B, float *C,
                     const int *colidx, int ld, int c_rows)
{
    spmm_kernel<BM, W, PREC><<<grid, kBlockThreads, 0, s>>>(ntasks, nchunks, val, rows, colstart,
                                                            B, C, colidx, ld, c_rows);
}

int launch(int bm, int prec, int ntasks, int colB_p, const void *val, const unsigned *rows,
           const int *colstart, const void *B, float *C, const int *colidx, int c_rows,
           hipStream_t s)
{
    const int w = chunk_width(bm, colB_p);
    const int nchunks = colB_p / w;
    const long long waves = (long long)ntasks * nchunks;
    const long long blocks = (waves + kWavesPerBlock - 1) / kWavesPerBlock;
    if (blocks <= 0) return 0;
    if (blocks > 0x7fffffffLL) return TSP_EINVAL;
    dim3 grid((unsigned)blocks);
#define TSP_L(BMv, Wv)                                                                         \
    if (bm == BMv && w == Wv) {                                                                \
        if (prec == TSP_PREC_FP16)                                                             \
            launch_t<BMv, Wv, TSP_PREC_FP16>(grid, s, ntasks, nchunks, val, rows, colstart, B, C, \
                                            colidx, colB_p, c_rows);                          \
        else                                                                                   \
            launch_t<BMv, Wv, TSP_PREC_TF32>(grid, s, ntasks, nchunks, val, rows, colstart, B, C, \
                                            colidx, colB_p, c_rows);                          \
        return (int)hipGetLastError();                                                         \
    }
    TSP_L(64, 32) TSP_L(64, 64)
    TSP_L(16, 32) TSP_L(16, 64) TSP_L(16, 128)
    TSP_L(8, 32) TSP_L(8, 64) TSP_L(8, 128)
#undef TSP_L
    return TSP_EINVAL;
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

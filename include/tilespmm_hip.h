/*
 * tilespmm_hip.h -- C ABI of the MI355X (gfx950) TileSpMM device library,
 * libtilespmm_hip.so.  Plain pointers and sizes only; every function returns
 * an int status (0 = success, otherwise a hipError_t value or one of the
 * TSP_E* codes below) instead of exiting, so a caller maps failures to its
 * own policy.  The CLI maps any non-zero status to exit(1), which is the
 * reference's fail-fast behaviour (src/common.h:75-94).
 *
 * Data layout expected in device memory (all row-major, 4-byte indices):
 *   B    [colA][colB_p]            value type (fp16 bits or fp32)
 *   C    [c_rows][colB_p]          fp32
 *   val  [tilenum][BM][BN]         value type, canonical row-major tiles
 *   colidx [tilenum][BN]           int32, sorted distinct columns per row-block
 *   rows [rowblkblock]             uint32 start row, bit 31 = split task
 *   colstart [rowblkblock + 1]     int32 tile range of each task
 * colB_p is 32 or a multiple of 64, as the reference pads it
 * (src/main.cu:173).  BN is fixed by (BM, precision): fp16 64->32, 16->16,
 * 8->16; tf32 64->16, 16->8, 8->8 (src/main.cu:267-275).
 */
#ifndef TILESPMM_HIP_H
#define TILESPMM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TSP_PREC_FP16 0
#define TSP_PREC_TF32 1

#define TSP_OK 0
#define TSP_EINVAL 1001      /* bad argument (class, width, pointer) */
#define TSP_ENODEV 1002      /* no usable gfx950 device */

/* Library version string and the offload target it was built for. */
const char *tsp_hip_version(void);

/* Last error text of this thread (static storage). */
const char *tsp_hip_error_string(int status);

/* Select the device and check that it is a gfx950 part.
 * Replaces cudaSetDevice + cudaGetDeviceProperties + prefetch_device_matches
 * (src/main.cu:210-219). */
int tsp_device_init(int device_id);

/* Device resource probe: the fields the reference's generated
 * PrefetchDeviceInfo carries (pre/prefetch_probe.cu:62-95), read from
 * hipDeviceProp_t.  Any pointer may be NULL. */
typedef struct {
    int cu_count;               /* multiProcessorCount */
    int max_threads_per_cu;
    int regs_per_cu;            /* 32-bit registers per CU */
    int max_blocks_per_cu;
    long long lds_bytes_per_cu;
    long long l2_bytes;
    int wavefront_size;
    int clock_khz;
    int memory_clock_khz;
    int memory_bus_width;
    char name[256];
    char gcn_arch[64];
} tsp_device_info;
int tsp_device_probe(int device_id, tsp_device_info *out);

/* Kernel resource probe for one (BM, precision, colB_p) kernel: the fields of
 * the reference's PrefetchKernelInfo (pre/prefetch_probe.cu:15-27), read with
 * hipFuncGetAttributes.  iteration_bytes = tasks per block x
 * (BM*BN + BN*cols) x value size. */
typedef struct {
    int threads;                /* threads per block */
    int tasks_per_block;        /* independent tasks one block runs */
    int registers_per_thread;   /* VGPRs (arch + acc) per lane */
    long long shared_bytes;     /* static LDS per block */
    int iteration_bytes;
    int cols_per_task;          /* output columns one task covers */
} tsp_kernel_info;
int tsp_kernel_probe(int bm, int prec, int colB_p, tsp_kernel_info *out);

/* Current and maximum GFX clock of a device in MHz, read through AMD SMI
 * (libamd_smi.so, loaded on first use).  Replaces get_gpu_clock
 * (src/common.h:96-119), which reads the SM clock through NVML.  *mhz = 0
 * (status TSP_OK) when the clock cannot be read. */
int tsp_gpu_clock_mhz(int device_id, unsigned *mhz, unsigned *max_mhz);

/* Memory and copies (hipMalloc / hipMemcpy / hipMemset wrappers). */
int tsp_malloc(void **ptr, size_t bytes);
int tsp_free(void *ptr);
int tsp_memcpy_h2d(void *dst, const void *src, size_t bytes);
int tsp_memcpy_d2h(void *dst, const void *src, size_t bytes);
int tsp_memcpy_h2d_async(void *dst, const void *src, size_t bytes, void *stream);
int tsp_memset(void *dst, int value, size_t bytes);
int tsp_memset_async(void *dst, int value, size_t bytes, void *stream);

/* Streams and events.  Streams are created at the default priority. */
int tsp_stream_create(void **stream);
int tsp_stream_destroy(void *stream);
int tsp_stream_sync(void *stream);
int tsp_device_sync(void);
int tsp_event_create(void **event);
int tsp_event_destroy(void *event);
int tsp_event_record(void *event, void *stream);   /* stream NULL = null stream */
int tsp_event_sync(void *event);
int tsp_event_elapsed_ms(float *ms, void *start, void *stop);
/* Non-blocking stream (no implicit ordering with the null stream) and an
 * explicit stream -> event dependency, used to join class streams. */
int tsp_stream_create_nonblocking(void **stream);
int tsp_stream_wait_event(void *stream, void *event);
/* HIP graphs (no counterpart in the reference, which launches every kernel
 * from the host): tsp_stream_begin_capture starts a thread-local capture of
 * `stream` (work recorded on other streams that wait on its events joins
 * it); tsp_stream_end_capture ends it and instantiates the graph into
 * *graph_exec (NULL on failure; the capture is ended either way);
 * tsp_graph_launch replays it on a stream; tsp_graph_destroy frees it. */
int tsp_stream_begin_capture(void *stream);
int tsp_stream_end_capture(void *stream, void **graph_exec);
int tsp_graph_launch(void *graph_exec, void *stream);
int tsp_graph_destroy(void *graph_exec);

/* Tile SpMM launch, one row-block class:
 *   C[rows of task][cols] (=, or += atomically for split tasks)
 *       sum over the task's tiles of  A_tile (BM x BN) * B[colidx[tile]][cols]
 * Replaces switch_tilespmm_cuda_v64 / _v16 / _v8
 * (src/tilespmm_cuda.h:1634-1744); same arguments plus c_rows, the number of
 * rows of C that may be written (rows >= c_rows of a short last row-block are
 * skipped instead of relying on padding rows).  Asynchronous on `stream`;
 * returns the launch status.  C must be zeroed first when any task is split
 * (bit 31 of its row word); split tasks are added atomically, in any order of
 * the schedule, as in the reference. */
int tsp_spmm_launch(int bm, int prec, int rowblkblock, int colB_p,
                    const void *d_val, const unsigned *d_rows, const int *d_colstart,
                    const void *d_B, float *d_C, const int *d_colidx,
                    int c_rows, void *stream);

/* Same launch with an explicit kernel variant, for tuning drivers: chunk
 * width w (output columns per wave: 32, 64 or 128; 64-row tiles 32 or 64),
 * software-pipeline depth stages (1-3 tiles in flight per wave) and
 * tasks_per_wave (consecutive tasks one wave streams) and the order of the
 * column chunks (1: the chunks of one task range run side by side, 2:
 * chunk-major, every range of chunk 0 first).  Values <= 0 pick the defaults
 * tsp_spmm_launch uses.  With tasks_per_wave > 1 the tasks of a split
 * row-block must be consecutive in the schedule (tsp_tile_pretreatment's
 * always are): a wave that runs all of them stores their sum without
 * atomics.  No counterpart in the reference (its kernels have one fixed
 * shape per class). */
int tsp_spmm_launch_variant(int bm, int prec, int rowblkblock, int colB_p,
                            const void *d_val, const unsigned *d_rows, const int *d_colstart,
                            const void *d_B, float *d_C, const int *d_colidx,
                            int c_rows, void *stream, int w, int stages, int tasks_per_wave,
                            int order);

/* Launch on the bitmap-packed A format (8- and 16-row classes only): for
 * tile t, bit r*BN+c of d_bitmap[t*BM*BN/64 ...] marks slot (r, c), and the
 * values of its set bits, in bit order, start at element d_vptr[t] of d_pval
 * (d_pval must hold 4 readable elements past the last value).  Same result
 * as tsp_spmm_launch on the dense tiles; variant arguments as in
 * tsp_spmm_launch_variant.  No counterpart in the reference (it always
 * streams dense zero-padded tiles). */
int tsp_spmm_launch_packed(int bm, int prec, int rowblkblock, int colB_p, const void *d_pval,
                           const uint64_t *d_bitmap, const int *d_vptr, const unsigned *d_rows,
                           const int *d_colstart, const void *d_B, float *d_C,
                           const int *d_colidx, int c_rows, void *stream, int w, int stages,
                           int tasks_per_wave, int order);

/* Workgroup placement on the XCDs.  Each of the 8 XCDs of an MI355X has its
 * own L2 and receives every 8th workgroup of a launch.  The launches above
 * use TSP_PLACE_CONTIGUOUS: each XCD runs one contiguous eighth of the task
 * ranges, so neighbouring row-blocks, which share B rows, share an L2.
 * TSP_PLACE_INTERLEAVED deals runs of 4 workgroups to the XCDs in turn,
 * which keeps matrices whose heavy rows sit together (graphs with hub
 * vertices at one end) balanced across the XCDs.  tsp_spmm_launch_placed
 * takes the placement with the variant arguments of tsp_spmm_launch_variant
 * (d_bitmap NULL: dense A tiles in d_val; else the packed format of
 * tsp_spmm_launch_packed, with d_val the packed values).  No counterpart in
 * the reference (NVIDIA GPUs have one L2). */
#define TSP_PLACE_CONTIGUOUS 0
#define TSP_PLACE_INTERLEAVED 1
/* TSP_PLACE_CHUNK_XCD (2, 4 or 8 column chunks of w columns): each group of
 * 8 / chunks XCDs serves one chunk, with runs of 4 workgroups dealt in turn
 * inside the group, so an XCD's L2 holds the B segments of one chunk only
 * (the chunk order argument is then ignored). */
#define TSP_PLACE_CHUNK_XCD 2
int tsp_spmm_launch_placed(int bm, int prec, int rowblkblock, int colB_p, const void *d_val,
                           const uint64_t *d_bitmap, const int *d_vptr, const unsigned *d_rows,
                           const int *d_colstart, const void *d_B, float *d_C, const int *d_colidx,
                           int c_rows, void *stream, int w, int stages, int tasks_per_wave, int order,
                           int placement);

/* tsp_spmm_launch_placed with flags.  TSP_LAUNCH_OPERANDS_TF32 (tf32 only):
 * the caller guarantees that every A value and every B value the launch
 * reads is a tf32 value already (low 13 mantissa bits zero, or Inf/NaN),
 * e.g. after tsp_round_tf32_device; the kernels then skip their
 * per-operand rounding and give the same result as the rounding launch.
 * The plan rounds its copies of A and B once when they enter it and
 * launches this way.  No counterpart in the reference. */
#define TSP_LAUNCH_OPERANDS_TF32 1
/* TSP_LAUNCH_LANE_INDICES (8- and 16-row classes: every packed-format
 * variant; dense tiles at chunk widths up to 128, without tile pairs or the
 * panel sweep): each lane reads the column indices of its B rows with one
 * vector load instead of the scalar loads plus a per-lane select chain; same
 * result, fewer VALU instructions per tile, one more vector memory
 * instruction.  The plan's tuning picks per class (faster on the
 * gather-bound RMAT and power-law fp16 classes and on small launch-bound
 * plans, slower on banded and block-sparse ones).  Other launches with the
 * flag fail with TSP_EINVAL. */
#define TSP_LAUNCH_LANE_INDICES 2
/* TSP_LAUNCH_TILE_PAIRS (fp16 8- and 16-row tiles, chunk width w 64 or 128;
 * tf32 8-row tiles, w 64): each wave multiplies two consecutive tiles of a
 * task at a time; a task with an odd tile count ends with a single tile.
 * fp16: one 16 x 32 tile on v_mfma_f32_16x16x32_f16 (the K = 16 form runs at
 * half the fp16 rate).  tf32 (needs TSP_LAUNCH_OPERANDS_TF32): split-bf16
 * products on v_mfma_f32_16x16x32_bf16 -- the high and low bf16 halves of
 * each A value in MFMA rows 0-7 and 8-15, each B value as the split word of
 * tsp_split_bf16_device, so d_B must hold those words (B values as split
 * words, same layout); every product is exact, as in the fp32 MFMA path
 * (but for values below 2^-116, whose low halves lose bits).
 * Same products, accumulated in another order (fp32).
 * tsp_pairs_supported(bm, prec, w) says whether a launch with chunk width w
 * may pass it (a launch given w <= 0 checks its default width).  No
 * counterpart in the reference (its 16-row kernel covers both k-halves of
 * one 16 x 16 tile with two m16n8k16 steps). */
#define TSP_LAUNCH_TILE_PAIRS 8
/* TSP_LAUNCH_SKIP_ZERO_STORES: the caller guarantees that C already holds
 * zero wherever the launch's result is an exact zero (a zero-filled C that
 * only launches of the same matrix and B write, as a plan's is); the kernels
 * then skip storing (and atomically adding) exact zeros -- a row-block's
 * empty rows, for instance, cost no write.  NaN is stored.  No counterpart
 * in the reference, whose kernels store every row of every tile. */
#define TSP_LAUNCH_SKIP_ZERO_STORES 16
/* TSP_LAUNCH_B_3BYTE (tf32 with TSP_LAUNCH_OPERANDS_TF32, no tile pairs; not
 * for the panel sweep): d_B holds B's rows in the 3-byte form of
 * tsp_pack_3byte_device -- each tf32 value as the top 3 bytes of its fp32
 * word, row r at byte offset r * colB_p * 3 -- which the kernels gather with
 * 12-byte loads and widen in registers (64-column chunks) or before their
 * LDS panel (other widths).  Every tf32 value is kept
 * exactly, so the result is bit for bit that of the 4-byte launch, while each
 * gathered row is a quarter smaller (and rows no longer start at multiples
 * of a power of two, which spread the most gathered rows unevenly over the
 * memory channels).  Other launches with the flag fail with TSP_EINVAL.  No
 * counterpart in the reference. */
#define TSP_LAUNCH_B_3BYTE 32
int tsp_pairs_supported(int bm, int prec, int w);
int tsp_spmm_launch_ex(int bm, int prec, int rowblkblock, int colB_p, const void *d_val,
                       const uint64_t *d_bitmap, const int *d_vptr, const unsigned *d_rows,
                       const int *d_colstart, const void *d_B, float *d_C, const int *d_colidx,
                       int c_rows, void *stream, int w, int stages, int tasks_per_wave, int order,
                       int placement, int flags);

/* Panel-synchronised sweep: tsp_spmm_launch_ex whose waves step through
 * the B rows in panels of panel_rows rows (a power of two, at least 64;
 * b_rows = rows of B that panels cover; a tile whose first column index is
 * b_rows or more, such as a hot-row copy, is not held back).  The grid holds at most
 * the workgroups that fit on the device at once, each wave running one task
 * range per generation.  Within a generation, a wave about to load from
 * panel q first waits (at most 20 us) until every wave of its XCD that has
 * started has reached panel q - panel_lag, so the waves of one XCD gather
 * from a window of about panel_lag + 1 panels, which that XCD's L2 holds.
 * With one task per wave the tiles of a task come in ascending column
 * order.  The result is the same as tsp_spmm_launch_ex's with the same
 * arguments; only the timing changes.  d_sync: sync_ints ints of device
 * memory for the wave counters; a launch needs generations x 8 x (panels +
 * 1) x 512 of them (TSP_EINVAL if sync_ints is smaller, for
 * TSP_PLACE_CHUNK_XCD, for a bad panel_rows or for panel_lag < 1).  A launch
 * leaves the counters ready for the next launch with the same arguments; the
 * first launch on a buffer, and the first after any argument changes, passes
 * TSP_LAUNCH_SYNC_RESET in flags, which zeroes them on the stream first
 * (with stale counters the waits only run into their time limit).  Launches
 * that share d_sync must not overlap.  No counterpart in the reference (its
 * grid is one block per task). */
#define TSP_LAUNCH_SYNC_RESET 4
int tsp_spmm_launch_panels(int bm, int prec, int rowblkblock, int colB_p, const void *d_val,
                           const uint64_t *d_bitmap, const int *d_vptr, const unsigned *d_rows,
                           const int *d_colstart, const void *d_B, float *d_C, const int *d_colidx,
                           int c_rows, void *stream, int w, int stages, int tasks_per_wave, int order,
                           int placement, int flags, int b_rows, int panel_rows, int panel_lag, int *d_sync,
                           long long sync_ints);

/* Per-class entry points with the reference dispatcher names
 * (src/tilespmm_cuda.h:1634, :1672, :1710) and argument order. */
int tsp_switch_v64(int prec, int rowblkblock, int colB_p, const void *d_val,
                   const unsigned *d_rows, const int *d_colstart, const void *d_B,
                   float *d_C, const int *d_colidx, int c_rows, void *stream);
int tsp_switch_v16(int prec, int rowblkblock, int colB_p, const void *d_val,
                   const unsigned *d_rows, const int *d_colstart, const void *d_B,
                   float *d_C, const int *d_colidx, int c_rows, void *stream);
int tsp_switch_v8(int prec, int rowblkblock, int colB_p, const void *d_val,
                  const unsigned *d_rows, const int *d_colstart, const void *d_B,
                  float *d_C, const int *d_colidx, int c_rows, void *stream);

/* Vendor SpMM baseline on rocSPARSE, the counterpart of cusparse_spmm_all
 * (src/main.cu:16-134): host CSR A (prec values), host B [k][ldb] row-major
 * (first n columns used), host C [m][n] fp32 out.  pre_ms = descriptor and
 * buffer set-up (wall clock), ms = mean of `repeat` timed calls after
 * `warmup` untimed ones.  Allocates and frees its own device memory. */
int tsp_vendor_spmm(int prec, int m, int k, long long nnz, const int *rowptr, const int *colidx,
                    const void *val, int n, int ldb, const void *h_B, float *h_C, int warmup,
                    int repeat, double *pre_ms, double *ms);

/* The kernels' tf32 operand rounding, run on the host over n fp32 bit
 * patterns: nearest-even to 10 mantissa bits; Inf and NaN unchanged.  The
 * reference gives raw fp32 bits to its tf32 tensor-core instructions
 * (src/utils.h:233-246); this build rounds explicitly, and NaN still
 * propagates. */
int tsp_round_tf32_bits(const uint32_t *in, uint32_t *out, size_t n);
/* The same rounding in place over n fp32 values in device memory,
 * asynchronous on `stream`. */
int tsp_round_tf32_device(void *d_x, size_t n, void *stream);

/* tf32 values as split-bf16 words: high half = the value truncated to bf16,
 * low half = the rest, exact for magnitudes of at least 2^-116 (below, the
 * rest is an fp32 subnormal truncated to 16 bits: error < 2^-126); these are
 * the words the tf32 tile-pair kernels read as B.  Inf keeps a zero low
 * half, NaN becomes a quiet NaN in both halves.
 * Inputs must be tf32 values (e.g. after tsp_round_tf32_device).  The host
 * form converts n values; the device form converts n values of d_src into
 * d_dst (may be equal), asynchronously on `stream`.  No counterpart in the
 * reference (its tensor cores take tf32 operands directly). */
int tsp_split_bf16_bits(const uint32_t *in, uint32_t *out, size_t n);
int tsp_split_bf16_device(const void *d_src, void *d_dst, size_t n, void *stream);

/* tf32 values in 3 bytes each (the B form of TSP_LAUNCH_B_3BYTE): the top 24
 * bits of each fp32 word, little-endian, 4 values in 12 bytes; a NaN whose
 * payload lies only in the dropped low byte gets the quiet bit.  Lossless
 * for tf32 values (low 13 mantissa bits zero, e.g. after
 * tsp_round_tf32_device).  n (a multiple of 4) values of `in` / d_src to
 * 3 n bytes of `out` / d_dst; the device form runs asynchronously on
 * `stream` (d_dst must not overlap d_src).  No counterpart in the
 * reference. */
int tsp_pack_3byte_bits(const uint32_t *in, void *out, size_t n);
int tsp_pack_3byte_device(const void *d_src, void *d_dst, size_t n, void *stream);

/* A plain streaming copy kernel (dst = src, 16-byte vectors), used to
 * calibrate HBM byte counters and the achievable copy bandwidth. */
int tsp_copy_kernel(void *dst, const void *src, size_t bytes, void *stream);
/* Random row gathers (the access pattern of SpMM's B rows): 8192 x 256
 * threads, each group of row_bytes/16 lanes reads `iters` uniformly random
 * rows of row_bytes (16, 32, 64, 128 or 256) from `table`; one launch reads
 * 8192 * 256 * 16 * iters bytes.  sink: 8192 * 256 uint32 of device memory
 * (written only on an improbable value pattern).  Calibrates the gather
 * bandwidth ceiling; no reference counterpart. */
int tsp_gather_kernel(const void *table, size_t table_bytes, int row_bytes, int iters, unsigned seed,
                      void *sink, void *stream);
/* Row gathers in the order of an index stream: reads row d_idx[i] (row_bytes
 * 64, 128, 256 or 512, 16 bytes per lane; or 96, 192 or 384, 12 bytes per
 * lane, the rows of TSP_LAUNCH_B_3BYTE) of a table of table_rows rows for
 * i = 0..n-1, the stream cut into contiguous pieces, one per wave, with 8
 * loads in flight per lane; indices outside the table are clamped to it.
 * Nothing is written unless an improbable bit pattern is read (d_sink, 256
 * words).  Given a class's tile column indices it measures the gather rate
 * of the kernels' own B-row stream with no other work; no reference
 * counterpart. */
int tsp_gather_index_stream(const void *d_table, long long table_rows, int row_bytes, const int *d_idx, long long n,
                            void *d_sink, void *stream);

/* ---- Hot B rows ------------------------------------------------------------
 * B is allocated with spare rows after row colA; hot slot s is row colA + s
 * and holds a copy of B row hot[s].  A tile column index colA + s then reads
 * the copy.  Copying the most-gathered rows of a skewed matrix into
 * consecutive rows spreads their cache lines over every L2 and memory
 * channel.  No counterpart in the reference (it gathers every row from its
 * place in B).
 *
 * tsp_colidx_count: counts[c] += number of entries of d_colidx[n] naming
 *   column c (entries >= colA are first decoded through d_hot[nhot]).
 *   d_counts[colA] must be zeroed by the caller.
 * tsp_colidx_remap: d_colidx[i] = map[decode(d_colidx[i])], where decode
 *   undoes an earlier remap through d_old_hot[old_nhot] and d_map[colA] names
 *   each column's new index (itself or colA + slot); d_map NULL restores the
 *   canonical column indices.
 * tsp_hot_rows_gather: rows colA + s = rows d_hot[s] of d_B (row_bytes per
 *   row, a multiple of 16), s < nhot; d_B must hold colA + nhot rows.
 * All three are asynchronous on `stream`. */
int tsp_colidx_count(const int *d_colidx, long long n, int colA, const int *d_hot, int nhot,
                     unsigned *d_counts, void *stream);
int tsp_colidx_remap(int *d_colidx, long long n, int colA, const int *d_old_hot, int old_nhot,
                     const int *d_map, void *stream);
int tsp_hot_rows_gather(void *d_B, int colA, long long row_bytes, const int *d_hot, int nhot,
                        void *stream);

/* ---- CSR -> tiles on the device ------------------------------------------
 * Device counterpart of Tile_create (src/csr2tile.h:724-795, convert_step1-3
 * at :15-379) producing the same arrays as the host tsp_tile_create, bit for
 * bit: tile_ptr[tilem+1], tile_nnz[tilenum+1], tile_colidx[tilenum*BN]
 * (sorted distinct columns, last tile padded with the last column), val
 * (canonical row-major BM x BN tiles, duplicates summed in CSR order with the
 * value type's rounding per add) and the occupancy bitmap.  The schedule and
 * orig_tile_row_idx stay host work (tsp_tile_pretreatment). */
typedef struct {
    int tilem, tilenum, bm, bn, prec, bitmap_words;
    int *d_tile_ptr;
    int *d_tile_nnz;
    int *d_tile_colidx;
    void *d_val;                /* fp16 or fp32 (tf32 values) */
    unsigned long long *d_bitmap;
} tsp_dev_tiles;

/* d_ptr[rows+1], d_idx[nnz], d_val[nnz] (prec-typed) are the class sub-CSR
 * on the device.  Allocates the output arrays (free with tsp_dev_tiles_free)
 * and its scratch; synchronises `stream` before returning.  On failure the
 * outputs are already freed. */
int tsp_tile_create_device(tsp_dev_tiles *out, int rows, int colA, long long nnz, const int *d_ptr,
                           const int *d_idx, const void *d_val, int BM, int BN, int prec,
                           void *stream);
int tsp_dev_tiles_free(tsp_dev_tiles *t);

/* Bitmap-packed A on the device (the format tsp_spmm_launch_packed reads):
 * *nvals = set bits over all tiles; when d_pval/d_vptr are non-NULL also
 * allocates and fills d_vptr[tilenum+1] (per-tile offsets) and d_pval
 * (values at the set bits in row-major bit order, + 4 zero elements).
 * d_val/d_bitmap as in tsp_dev_tiles.  The offsets are ints: when the set
 * bits plus the 4 padding elements exceed INT_MAX the call returns
 * TSP_EINVAL (before any offset is formed) with *nvals = the 64-bit count.
 * No reference counterpart (the reference has no packed format). */
int tsp_tiles_pack_device(int tilenum, int bm, int bn, int prec, const void *d_val,
                          const unsigned long long *d_bitmap, long long *nvals, void **d_pval,
                          int **d_vptr, void *stream);

/* Allocation-free variant of tsp_tiles_pack_device.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, serving loops, harnesses that forbid hipMalloc).
 * The caller passes the outputs: d_vptr [tilenum + 1] ints and d_pval, room
 * for pval_capacity elements of the value type, which must hold the packed
 * values plus 4 padding elements.  *nvals = number of packed values (also
 * on failure for lack of room, which returns TSP_EINVAL, so the caller can
 * size the buffer).  As in tsp_tiles_pack_device, a count whose values plus
 * padding exceed INT_MAX returns TSP_EINVAL (d_vptr then holds the per-tile
 * counts, not offsets).  The scan's per-block sums live in a static 1 MiB
 * device array, so tilenum is limited to TSP_PACK_NOALLOC_MAX_TILES (larger
 * requests return TSP_EINVAL).  Calls no hipMalloc/hipFree; synchronises
 * `stream`.  Every call on one GPU shares that array: calls that overlap on
 * the same GPU (other threads, other streams) race and must be serialised
 * by the caller. */
#define TSP_PACK_NOALLOC_MAX_TILES (((1LL << 18) - 3) * 2048)
int tsp_tiles_pack_device_noalloc(int tilenum, int bm, int bn, int prec, const void *d_val,
                                  const unsigned long long *d_bitmap, void *d_pval,
                                  long long pval_capacity, int *d_vptr, long long *nvals,
                                  void *stream);

#ifdef __cplusplus
}
#endif

#endif /* TILESPMM_HIP_H */

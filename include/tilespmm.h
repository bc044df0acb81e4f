/*
 * tilespmm.h -- C ABI of the TileSpMM host library, libtilespmm_host.so.
 *
 * This is the reference's host-side surface (CSR -> matrix_split -> csr2tile
 * tiles -> task schedule -> launch), kept with the reference's names and
 * argument meanings so code written against it drops in.  Values travel as
 * raw bit patterns of the precision's storage type: binary16 (uint16) for
 * TSP_PREC_FP16, binary32 (float) for TSP_PREC_TF32.
 *
 * Errors: every function returns an int status (0 = success; TSP_E* codes or
 * a HIP status from tilespmm_hip.h otherwise) instead of calling exit(); the
 * CLI turns a non-zero status into exit(1) as src/common.h:75-94 does.
 */
#ifndef TILESPMM_H
#define TILESPMM_H

#include <stddef.h>
#include <stdint.h>
#include <stdio.h>

#include "tilespmm_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

#define TSP_ENOMEM 1003     /* host allocation failed */
#define TSP_EIO 1004        /* file missing or malformed */

/* Tile format of one row-block class.  Field names and meanings follow the
 * reference's Tile_matrix (src/format.h:4-21):
 *   tile_ptr[tilem+1]       tiles per row-block, exclusive prefix sum
 *   tile_nnz[tilenum+1]     CSR entries per tile, exclusive prefix sum
 *   tile_colidx[tilenum*BN] sorted distinct columns, last tile padded with
 *                           the last valid column
 *   Blockdense_Val          tilenum * BM * BN values.  Layout differs from the
 *                           reference on purpose: canonical ROW-MAJOR tiles
 *                           (the reference stores NVIDIA mma.sync fragment
 *                           order, src/csr2tile.h:255-372); the values are the
 *                           same bits once that permutation is inverted.
 *   rowblkblock, blkcoostylerowidx, blkcoostylerowidx_colstart: the current
 *                           task schedule (tile_pretreatment).
 *   orig_tile_row_idx[tilem] first original row of each row-block.
 * Added for MI355X: bm, bn, prec, and the occupancy bitmap (bit r*BN+c of a
 * tile is set when some CSR entry lands at row r, slot c; bitmap_words
 * uint64 words per tile). */
typedef struct {
    int tilem;
    int tilen;
    int tilenum;
    int *tile_ptr;
    int *tile_nnz;
    int *tile_colidx;
    void *Blockdense_Val;
    size_t dnssize;
    int rowblkblock;
    unsigned int *blkcoostylerowidx;
    int *blkcoostylerowidx_colstart;
    int *orig_tile_row_idx;
    int bm, bn, prec;
    int bitmap_words;
    uint64_t *tile_bitmap;
} Tile_matrix;

/* One row class of the split (build_sub_csr outputs, src/hetero_split.h:86). */
typedef struct {
    int rows;
    long long nnz;
    int *ptr;
    int *idx;
    void *val;
    int *orig_row;
} tsp_sub_csr;

/* ---- Matrix Market ------------------------------------------------------
 * mmio_allinone semantics (src/mmio_highlevel.h:307-480): COO -> CSR in file
 * order, symmetric/hermitian mirrored (diagonal once), pattern -> 1,
 * complex -> real part, no sort, no dedupe.  Unlike the reference, a missing
 * or malformed file is an error (TSP_EIO), not silently ignored.
 * Values are returned as doubles; free arrays with tsp_free_host. */
int tsp_mm_read(const char *path, int *rows, int *cols, long long *nnz, int *is_symmetric,
                int **rowptr, int **colidx, double **val);
void tsp_free_host(void *p);

/* ---- Row split (matrix_split, src/hetero_split.h:144-291) --------------- */
int tsp_matrix_split(int rowA, int colA, long long nnzA, const int *rowptr, const int *colidx,
                     const void *val, int prec, float gamma, float delta,
                     tsp_sub_csr *out64, tsp_sub_csr *out16, tsp_sub_csr *out8);
/* Only the per-row class (0 = 64-row, 1 = 16-row, 2 = 8-row). */
int tsp_split_classes(int rowA, int colA, const int *rowptr, const int *colidx, float gamma,
                      float delta, int *row_class);
void tsp_sub_csr_free(tsp_sub_csr *s);

/* ---- CSR -> tiles (Tile_create, src/csr2tile.h:724-795) ----------------- */
int tsp_tile_create(Tile_matrix *m, int rows, int colA, long long nnz, const int *ptr,
                    const int *idx, const void *val, const int *orig_row, int BM, int BN,
                    int prec);
/* Frees every array of the tile matrix (including orig_tile_row_idx, which
 * the reference frees separately) and zeroes the struct. */
void tsp_tile_destroy(Tile_matrix *m);
/* BN the reference uses for (BM, precision) (src/main.cu:267-275). */
int tsp_tile_bn(int bm, int prec);

/* ---- Task schedule (tile_pretreatment, src/csr2tile.h:383-434) ---------
 * Writes a fresh schedule into *rows / *colstart (malloc'd; caller frees
 * with tsp_free_host) and the task count into *rowblkblock. */
int tsp_tile_pretreatment(const Tile_matrix *m, int TH, int *rowblkblock, unsigned **rows,
                          int **colstart);

/* ---- Threshold cost model (get_optimal_prefetch_th, :437-642) ----------
 * Resource inputs of the analytic model; tsp_th_params_probe fills them
 * from the device and the kernel that will run (hipDeviceProp_t +
 * hipFuncGetAttributes), lambda_atom from the MI355X calibration table. */
typedef struct {
    int sm_count, threads_per_sm, registers_per_sm, blocks_per_sm;
    long long shared_bytes_per_sm, l2_bytes;
    int kernel_threads, kernel_registers;
    long long kernel_shared_bytes;
    int iteration_bytes;
    float lambda_atom;
    /* launch geometry: tasks one block runs, output columns one task
     * covers.  The reference's CUDA kernels are (4, 32) for 8/16-row tiles
     * at colB_p = 32, (1, 32) for 64-row tiles at 32, and (1, 64) otherwise
     * (src/csr2tile.h:588-601); the MI355X kernels report theirs through
     * tsp_kernel_probe. */
    int tasks_per_block, cols_per_task;
    /* weight of the L2 re-read term: lambda_L2 = lambda_l2_scale *
     * iteration_bytes * cap / l2_bytes.  1.0 is the reference's model;
     * the probe fills the MI355X calibration. */
    float lambda_l2_scale;
} tsp_th_params;
int tsp_th_params_probe(int device_id, int bm, int prec, int colB_p, tsp_th_params *out);
/* The MI355X calibration the probe applies: lambda_atom and lambda_l2_scale
 * for (class, precision, padded colB).  No device needed. */
int tsp_th_weights(int bm, int prec, int colB_p, float *lambda_atom, float *lambda_l2_scale);
/* Fills top4 (cheapest first); returns the number of distinct candidates
 * evaluated (>= 1), or a negative value when the resources do not fit. */
int tsp_optimal_th(int BM, int colB, int tilem, const int *tile_ptr, const tsp_th_params *p,
                   int top4[4]);

/* ---- Threshold policy (src/model_features.h, src/ml_predict.h:8-15) ----
 * 11 features: [0, 0, rows, cols, nnz, 1-nnz/(rows*cols), nnz/rows,
 * max_row_nnz, min_row_nnz, capability, colB].  On MI355X the capability
 * slot holds the gfx target as major + minor/10 (gfx950 -> 9.5). */
#define TILESPMM_ML_FEATURE_COUNT 11
int tsp_features_from_csr(int rows, int cols, long long nnz, const int *rowptr,
                          double capability, int colB, double *features);
void tilespmm_predict_fp16(const double *features, float *gamma, float *delta);
void tilespmm_predict_tf32(const double *features, float *gamma, float *delta);

/* ---- Synthetic inputs (the five benchmark configurations) ---------------
 * config 1..5 as in the benchmark definition; prec/colB < 0 select the
 * configuration's own; seed 0 selects 20260000 + config.  Produces CSR A
 * (values in prec's storage type) and row-major B [cols][colB_p] with the
 * padded columns zero.  Arrays are malloc'd; free with tsp_free_host. */
int tsp_gen_config(int config, int prec, int colB, unsigned long long seed, int *rows, int *cols,
                   long long *nnz, int **rowptr, int **colidx, void **val, int *colB_p,
                   void **B);
/* Only the structure of config (no values). */
int tsp_gen_structure(int config, unsigned long long seed, int *rows, int *cols, long long *nnz,
                      int **rowptr, int **colidx);
/* The configuration-5 RMAT generator at any scale: 2^scale vertices, `edges`
 * directed edges with quadrant probabilities (a, b, c, d) = (.57, .19, .19,
 * .05), symmetrised, duplicates removed, self-loops kept, columns ascending;
 * values 1/deg(row) in prec's storage type.  Configuration 5 is scale 22,
 * 2^26 edges, seed 20260005.  Free the arrays with tsp_free_host. */
int tsp_gen_rmat(int scale, long long edges, unsigned long long seed, int prec, int *rows,
                 long long *nnz, int **rowptr, int **colidx, void **val);
/* Fill n values of prec from seed: dist 0 = U[-1,1), 1 = N(0,1). */
int tsp_gen_values(int prec, int dist, unsigned long long seed, size_t n, void *out);
/* padded width the kernels see: colB <= 32 ? 32 : roundup(colB, 64). */
int tsp_colB_padded(int colB);

/* ---- Device plan: the orchestration of call_tilespmm_cuda -------------
 * (src/csr2tile.h:826-1093) split into steps so both the CLI and benchmark
 * drivers use it.  A plan owns device copies of the three classes, B, C, one
 * stream per class and the timing events. */
typedef struct tsp_plan tsp_plan;
int tsp_plan_create(tsp_plan **plan, int device_id, Tile_matrix *m64, Tile_matrix *m16,
                    Tile_matrix *m8, int rowA, int colA, int colB_p, int prec, const void *h_B);
/* The same plan from the three class sub-CSRs (matrix_split outputs, NULL
 * or rows == 0 for an empty class): Tile_create runs on the device
 * (tsp_tile_create_device, bit-identical to tsp_tile_create) instead of the
 * host, and only tile_ptr / orig_tile_row_idx / the schedule stay on the
 * host.  *tile_ms (optional) = wall time of the sub-CSR upload + device
 * conversion. */
int tsp_plan_create_csr(tsp_plan **plan, int device_id, const tsp_sub_csr *s64,
                        const tsp_sub_csr *s16, const tsp_sub_csr *s8, int rowA, int colA,
                        int colB_p, int prec, const void *h_B, double *tile_ms);
/* Build + upload schedules for the three classes (a TH <= 0 keeps the
 * current one). */
int tsp_plan_set_th(tsp_plan *plan, int th64, int th16, int th8);
/* Cost-model top-4 per class, then runtime tuning over the cross product
 * (5 untimed + 10 timed runs each, src/csr2tile.h:962-1014).  With tune != 0
 * it then tunes each class's kernel variant (A format, chunk order and
 * width, tasks per wave, XCD placement, pipeline depth, index loads, tile
 * pairs, 3-byte B, panel sweep), the hot B rows, and each class's threshold once more
 * with its tuned variant.  Leaves the best schedule installed; outputs the
 * thresholds and the two timing parts. */
int tsp_plan_tune(tsp_plan *plan, int tune, int th_out[3], double *model_ms, double *tune_ms);
/* Pin the kernel variant one class launches with (see
 * tsp_spmm_launch_variant); zeros restore the library default. */
int tsp_plan_set_variant(tsp_plan *plan, int bm, int w, int stages, int tasks_per_wave,
                         int order);
/* A-tile format of one class on the device: 1 = dense canonical tiles,
 * 2 = bitmap-packed (8- and 16-row classes), 0 = keep.  tsp_plan_create picks
 * packed when it moves at most 3/4 of the dense bytes.  get returns the
 * current format (0 for an empty class, -1 on a bad argument). */
int tsp_plan_set_format(tsp_plan *plan, int bm, int fmt);
int tsp_plan_get_format(tsp_plan *plan, int bm);
/* The variant a class is pinned to (0 = library default), e.g. after
 * tsp_plan_tune picked the chunk width and order. */
int tsp_plan_get_variant(tsp_plan *plan, int bm, int *w, int *stages, int *tasks_per_wave, int *order);
/* Workgroup placement of one class on the XCDs (TSP_PLACE_CONTIGUOUS or
 * TSP_PLACE_INTERLEAVED, see tsp_spmm_launch_placed); tsp_plan_tune times
 * both.  get returns -1 on a bad argument. */
/* Lane-loaded column indices (TSP_LAUNCH_LANE_INDICES) for a class: 1 on,
 * 0 off (64-row classes: off only); tsp_plan_tune picks.  The setting applies
 * to the launches that have a lane-loaded kernel: every packed-format
 * variant, and dense variants at chunks of up to 128 columns without tile
 * pairs or the panel sweep.  get returns whether the class's launches load
 * indices per lane (1 / 0), or -1 on a bad argument. */
int tsp_plan_set_lane_indices(tsp_plan *plan, int bm, int on);
int tsp_plan_get_lane_indices(tsp_plan *plan, int bm);
/* Tile pairs (TSP_LAUNCH_TILE_PAIRS) for one class: 1 on, 0 off; fp16 8- and
 * 16-row classes with 64- or 128-column chunks, tf32 8-row classes with
 * 64-column chunks (a launch with another width fails; tf32 pairs read a
 * split-bf16 copy of B that the plan makes when they are first switched
 * on).  tsp_plan_tune picks.  No counterpart in the reference. */
int tsp_plan_set_pairs(tsp_plan *plan, int bm, int on);
int tsp_plan_get_pairs(tsp_plan *plan, int bm);
/* B in the 3-byte form (TSP_LAUNCH_B_3BYTE) for one class of a tf32 plan: 1
 * on, 0 off (fp16 plans: TSP_EINVAL for on).  Switching it on makes the
 * plan's 3-byte copy of B (colB_p * 3 bytes per row plus the hot-row
 * slots) if it has none.  The setting applies to the class's launches
 * without tile pairs or the panel sweep; the results are bit for bit those
 * of the 4-byte form.  get returns whether the class's
 * launches read the 3-byte form (1 / 0), or -1 on a bad argument.
 * tsp_plan_tune picks, and frees the copy when no class keeps it.  No
 * counterpart in the reference. */
int tsp_plan_set_b_3byte(tsp_plan *plan, int bm, int on);
int tsp_plan_get_b_3byte(tsp_plan *plan, int bm);
int tsp_plan_set_placement(tsp_plan *plan, int bm, int placement);
int tsp_plan_get_placement(tsp_plan *plan, int bm);
/* Panel-synchronised sweep (tsp_spmm_launch_panels) for one class on the
 * dense format: B rows per panel (a power of two, at least 64; 0 = off) and
 * the lead in panels a wave may have on the slowest wave of its XCD (at
 * least 1).  The plan allocates the class's 4 MB of counters on first use;
 * tsp_plan_tune tries it for classes whose work fills the device a few
 * times at most.  No counterpart in the reference. */
int tsp_plan_set_panels(tsp_plan *plan, int bm, int panel_rows, int lag);
int tsp_plan_get_panels(tsp_plan *plan, int bm, int *panel_rows, int *lag);
/* Hot B rows (see tsp_hot_rows_gather): copy the most-gathered B rows, at
 * most budget_bytes of them (and at most TSP_HOT_MAX_BYTES), into spare rows
 * of the plan's B and point every class's tile columns at the copies; every
 * step then re-copies them before the class kernels run.  Only columns
 * gathered at least TSP_HOT_MIN_GATHERS times qualify.  budget_bytes 0
 * restores the canonical column indices.  tsp_plan_tune times steps with
 * no hot rows against 16 MB of them and keeps the hot rows when they are 2%
 * faster.  get: the current slot count and bytes.  No counterpart in the
 * reference. */
#define TSP_HOT_MAX_BYTES (64LL << 20)
/* What tsp_plan_tune optimises.  TSP_TUNE_BACK_TO_BACK (the default): steps
 * run back to back, as the reference times its 1000 repetitions, so data
 * that fits in L2 or the 256 MB MALL carries over between steps.
 * TSP_TUNE_COLD: single steps from a cold cache (each measurement follows a
 * copy that evicts L2 and the MALL), for callers that run the product once
 * between other work; setting it allocates 1 GB of eviction buffer, which
 * TSP_TUNE_BACK_TO_BACK or tsp_plan_destroy frees.  No counterpart in the
 * reference. */
#define TSP_TUNE_BACK_TO_BACK 0
#define TSP_TUNE_COLD 1
int tsp_plan_set_tune_mode(tsp_plan *plan, int mode);
int tsp_plan_get_tune_mode(tsp_plan *plan);
#define TSP_HOT_MIN_GATHERS 4
int tsp_plan_set_hot_rows(tsp_plan *plan, long long budget_bytes);
int tsp_plan_get_hot_rows(tsp_plan *plan, int *nhot, long long *bytes);
/* Launch the classes once (each on its own stream, forked from and joined on
 * the plan's main stream; a plan with one class launches it on the main
 * stream).  zero_c != 0 clears C first. */
int tsp_plan_run(tsp_plan *plan, int zero_c);
/* Warm-up before timing, replacing warmup_gpu (src/csr2tile.h:798-823):
 * steps in batches of 20, then 50, reading the GFX clock
 * (tsp_gpu_clock_mhz) while each batch runs, until -- after at least 20 ms
 * of steps -- two successive readings agree within 2% and are at least 95%
 * of the maximum clock, or three successive readings agree within 2%
 * (MI355X power management can settle a memory-bound load below 95% of the
 * maximum); at most max_iters steps.
 * Without a readable clock it runs min(max_iters, 100) steps, the
 * reference's fallback.  *iters_run / *clock_mhz (may be NULL): steps run and
 * the last clock reading. */
int tsp_plan_warmup_clock(tsp_plan *plan, int max_iters, int *iters_run, unsigned *clock_mhz);
int tsp_plan_warmup(tsp_plan *plan, int max_iters);
/* Time `reps` back-to-back runs bracketed by events on the plan's main stream. */
int tsp_plan_time(tsp_plan *plan, int reps, double *ms_per_iter);
/* The same, plus *submit_ms_per_iter (may be NULL): the host's wall time per
 * run to submit the runs, until the last launch call returns.  When it is
 * about the event time per run, the runs are bound by the host's launch
 * rate (a few microseconds per HIP launch) rather than by the kernels.  No
 * counterpart in the reference. */
int tsp_plan_time_ex(tsp_plan *plan, int reps, double *ms_per_iter, double *submit_ms_per_iter);
/* Steps replayed from a HIP graph.  No counterpart in the reference, which
 * launches every kernel from the host; for callers that repeat the product
 * many times (iterative methods, serving), where steps of a few
 * microseconds are bound by the host's launch rate.
 * tsp_plan_graph_capture runs one step, then captures `steps` steps (1 to
 * 100000: the hot-row copy, the class kernels and their fork/join) into a
 * graph on the plan's main stream; tsp_plan_graph_run replays it `replays`
 * times there (asynchronously); tsp_plan_graph_time times replays as
 * tsp_plan_time does, per step.  Every call that changes the configuration
 * (tsp_plan_set_th / _variant / _format / _lane_indices / _placement /
 * _panels / _hot_rows, tsp_plan_tune) makes the graph stale: run and time
 * then return TSP_EINVAL until it is captured again.  Steps do not zero C
 * (as with tsp_plan_time): with split tasks C accumulates across steps.
 * tsp_plan_graph_free releases the graph (tsp_plan_destroy does too). */
int tsp_plan_graph_capture(tsp_plan *plan, int steps);
int tsp_plan_graph_run(tsp_plan *plan, int replays);
int tsp_plan_graph_time(tsp_plan *plan, int replays, double *ms_per_step);
int tsp_plan_graph_free(tsp_plan *plan);
/* Time one class alone (reps launches) on the stream a step launches it on:
   its own stream, or the main stream when it is the plan's only class. */
int tsp_plan_time_class(tsp_plan *plan, int bm, int reps, double *ms_per_launch);
int tsp_plan_download_c(tsp_plan *plan, float *h_C);
/* Device pointers of the plan (for external drivers).  A plan's C is zeroed
 * when the plan is made and written only by the plan's launches, which
 * therefore skip storing results that are exact zeros (empty rows of a
 * row-block cost no write; TSP_LAUNCH_SKIP_ZERO_STORES).  Once the caller
 * has taken C's device pointer it may write into C, so from then on the
 * plan stores every result (and a graph captured before is stale). */
int tsp_plan_device_c(tsp_plan *plan, float **d_C);
int tsp_plan_destroy(tsp_plan *plan);

/* ---- One-call orchestration (call_tilespmm_cuda) -----------------------
 * Plan + tune + warmup + result run + download + timed loop.  Writes CSV
 * fields 11-16 to csv when non-NULL, with the reference's formats. */
typedef struct {
    int th64, th16, th8;
    double pre_time_ms;      /* cpu_pre_time + model + tuning */
    double time_ms;          /* per iteration */
    double tflops;           /* 2 * nnz * logical_colB / t */
    double model_ms, tune_ms;
    int warmup_iters;        /* steps of the last clock-stable warm-up */
    unsigned clock_mhz;      /* GFX clock at its end (0: not readable) */
} tsp_run_result;
int tsp_call_tilespmm(int device_id, Tile_matrix *m64, Tile_matrix *m16, Tile_matrix *m8, int rowA,
                      int colA, int colB_p, long long total_nnz, int prec, const void *h_B,
                      float *h_C, double cpu_pre_time_ms, int logical_colB, int repeat, int tune,
                      FILE *csv, tsp_run_result *out);
/* The steps of tsp_call_tilespmm after the plan exists (tune, warmup,
 * result run, download, timed loop, CSV fields 11-16), for a plan from
 * tsp_plan_create or tsp_plan_create_csr.  cpu_pre_time_ms is the caller's
 * preprocessing time, to which the plan adds its model and tuning time. */
int tsp_plan_execute(tsp_plan *plan, long long total_nnz, float *h_C, double cpu_pre_time_ms,
                     int logical_colB, int repeat, int tune, FILE *csv, tsp_run_result *out);
/* Tile count of one class of the plan (-1 on a bad argument). */
int tsp_plan_tilenum(tsp_plan *plan, int bm);

#ifdef __cplusplus
}
#endif

#endif /* TILESPMM_H */

// plan.cpp -- device orchestration of one SpMM problem (call_tilespmm_cuda,
// src/csr2tile.h:826-1093), split into steps that the CLI and the benchmark
// driver share.  All device work goes through the C ABI of
// libtilespmm_hip.so; this file never touches the HIP runtime directly.
//
// Per row-block class the plan holds the tiles (values + column indices) and
// the current schedule in device memory, a host-side cache of schedules by
// threshold (the reference caches four, src/csr2tile.h:657-711), and one
// stream.  The three classes write disjoint rows of C and run concurrently;
// a run forks from and joins on the plan's main stream through events (the
// reference orders its class streams with legacy null-stream events).
#include <string.h>

#include <algorithm>
#include <array>
#include <cmath>
#include <chrono>
#include <map>
#include <memory>
#include <utility>
#include <vector>

#include "common.hpp"

namespace {

struct ClassDev {
    Tile_matrix *m = nullptr;
    int bm = 0;
    void *d_val = nullptr;
    int *d_colidx = nullptr;
    unsigned *d_rows = nullptr;
    int *d_colstart = nullptr;
    long long cap_tasks = 0;
    int th = 0;
    int ntasks = 0;
    int var_w = 0, var_s = 0, var_tpw = 0, var_order = 0;   // kernel variant, 0 = library default
    int var_li = 0;               // lane-loaded column indices (TSP_LAUNCH_LANE_INDICES), where a kernel has them
    int wdef = 0;                 // the library's default chunk width for this class
    int var_pr = 0;               // tile pairs (TSP_LAUNCH_TILE_PAIRS; fp16 8-/16-row, 64-/128-column chunks)
    int var_b3 = 0;               // tf32: B in the 3-byte form (TSP_LAUNCH_B_3BYTE), where a kernel has it
    int fmt = 1;                  // A format on the device: 1 dense tiles, 2 bitmap-packed
    bool pack_ok = false;         // packed format is worth trying (fewer bytes)
    void *d_pval = nullptr;       // packed values (+4 elements of padding)
    uint64_t *d_bmp = nullptr;    // per-tile occupancy bitmaps
    int *d_vptr = nullptr;        // per-tile offset into d_pval
    void *stream = nullptr;
    bool dev_built = false;       // tiles made on the device: `own` holds the host-side view
    Tile_matrix own{};            // tile_ptr, orig_tile_row_idx, schedule; no value arrays
    std::map<int, std::pair<std::vector<unsigned>, std::vector<int>>> cache;
    int place = TSP_PLACE_CONTIGUOUS;   // workgroup placement on the XCDs
    int panel = 0;                // panel-synchronised sweep: B rows per panel (0 = off)
    int panel_lag = 1;            // ... and how many panels a wave may lead the slowest by
    int *d_sync = nullptr;        // its wave counters (kSyncInts)
    std::vector<long long> sync_sig;   // launch arguments the counters are balanced for
    bool active() const { return m && m->tilenum > 0; }
};

// Counters of a class's panel-synchronised sweep: generations x 8 XCDs x
// (panels + 1) x 16 striped 128-byte lines must fit (4 MB per class that
// uses it).
constexpr long long kSyncInts = 1LL << 20;

double now_ms()
{
    return std::chrono::duration<double, std::milli>(
               std::chrono::steady_clock::now().time_since_epoch())
        .count();
}

}  // namespace

// Streams: one non-blocking stream per class plus a non-blocking "main"
// stream.  A run records a start event on main, every class stream waits for
// it, launches, records its own done event, and main waits for all three done
// events -- an explicit fork/join that never touches the null stream, so no
// launch pays an implicit null-stream synchronisation.
struct tsp_plan {
    int dev = 0, prec = 0, rowA = 0, colA = 0, colB_p = 0;
    void *d_B = nullptr;          // colA rows of B, then hot_cap spare rows for hot-row copies
    // C is zeroed when the plan is made and written only by its launches, so
    // they skip storing exact zeros (TSP_LAUNCH_SKIP_ZERO_STORES: a
    // row-block's empty rows cost no write) -- until the caller takes C's
    // device pointer and may write into it, from then on every result is
    // stored
    bool c_shared = false;
    void *d_Bs = nullptr;         // tf32 plans: the same rows as split-bf16 words, made when a class first
                                  // uses tile pairs (their kernels read B in that form)
    void *d_B3 = nullptr;         // tf32 plans: the same rows in the 3-byte form (colB_p * 3 bytes per row),
                                  // made when a class first reads B that way
    int hot_cap = 0;              // spare rows after row colA
    int nhot = 0;                 // hot slots in use: row colA + s copies B row d_hot[s]
    int *d_hot = nullptr;
    std::vector<unsigned> col_gathers;   // gathers per column over every class (canonical indices)
    int tune_mode = TSP_TUNE_BACK_TO_BACK;
    void *d_flush = nullptr;      // cold tuning: 2 x kFlushBytes of other memory, copied to evict the caches
    float *d_C = nullptr;
    ClassDev cls[3];
    void *main = nullptr;
    void *ev0 = nullptr, *ev1 = nullptr;
    void *done[3] = {nullptr, nullptr, nullptr};
    // A captured HIP graph of graph_steps steps; it holds the kernel
    // arguments of the configuration it was captured under (version), and
    // every call that changes the configuration bumps the version.
    void *graph = nullptr;
    int graph_steps = 0;
    unsigned long long version = 0, graph_version = 0;
};

#define TSP_TRY(x)                  \
    do {                            \
        int st_ = (x);              \
        if (st_) return st_;        \
    } while (0)

static int upload_schedule(tsp_plan *p, ClassDev &c, int th)
{
    auto it = c.cache.find(th);
    if (it == c.cache.end()) {
        int n = 0;
        unsigned *rows = nullptr;
        int *cs = nullptr;
        TSP_TRY(tsp_tile_pretreatment(c.m, th, &n, &rows, &cs));
        std::pair<std::vector<unsigned>, std::vector<int>> e;
        e.first.assign(rows, rows + n);
        e.second.assign(cs, cs + n + 1);
        free(rows);
        free(cs);
        it = c.cache.emplace(th, std::move(e)).first;
    }
    const int n = (int)it->second.first.size();
    if (n > c.cap_tasks) return TSP_EINVAL;
    // kernels of an earlier run may still read the schedule buffers
    TSP_TRY(tsp_device_sync());
    TSP_TRY(tsp_memcpy_h2d(c.d_rows, it->second.first.data(), sizeof(unsigned) * (size_t)n));
    TSP_TRY(tsp_memcpy_h2d(c.d_colstart, it->second.second.data(), sizeof(int) * ((size_t)n + 1)));
    c.th = th;
    c.ntasks = n;
    // Mirror the schedule into the tile matrix, as update_metadata does.
    free(c.m->blkcoostylerowidx);
    free(c.m->blkcoostylerowidx_colstart);
    c.m->blkcoostylerowidx = tsph::alloc_n<unsigned>((size_t)n);
    c.m->blkcoostylerowidx_colstart = tsph::alloc_n<int>((size_t)n + 1);
    memcpy(c.m->blkcoostylerowidx, it->second.first.data(), sizeof(unsigned) * (size_t)n);
    memcpy(c.m->blkcoostylerowidx_colstart, it->second.second.data(), sizeof(int) * ((size_t)n + 1));
    c.m->rowblkblock = n;
    (void)p;
    return TSP_OK;
}

// Bitmap-packed A: per tile the canonical tile's occupancy bitmap plus the
// values at its set bits in bit (row-major) order.  Chosen for 8- and 16-row
// classes when it moves fewer bytes than the dense zero-padded tiles.
static long long packed_values(const Tile_matrix *m)
{
    const size_t words = (size_t)m->tilenum * m->bitmap_words;
    long long n = 0;
#pragma omp parallel for reduction(+ : n)
    for (long long i = 0; i < (long long)words; ++i) n += __builtin_popcountll(m->tile_bitmap[i]);
    return n;
}

// tf32 plans keep their copies of A and B as tf32 values: rounded once here
// (nearest-even, Inf/NaN unchanged), so the kernels launch with
// TSP_LAUNCH_OPERANDS_TF32 and skip the per-operand rounding.
static int round_tf32_copy(const tsp_plan *p, void *d, size_t n)
{
    if (p->prec != TSP_PREC_TF32 || n == 0) return TSP_OK;
    TSP_TRY(tsp_round_tf32_device(d, n, nullptr));
    return tsp_device_sync();
}

static int upload_packed(tsp_plan *p, ClassDev &c)
{
    if (c.d_pval) return TSP_OK;
    if (c.dev_built) {
        // packed from the (already rounded) dense tiles
        long long n = 0;
        return tsp_tiles_pack_device(c.m->tilenum, c.m->bm, c.m->bn, p->prec, c.d_val,
                                     (const unsigned long long *)c.d_bmp, &n, &c.d_pval, &c.d_vptr, nullptr);
    }
    const Tile_matrix *m = c.m;
    const size_t vs = tsph::val_size(p->prec);
    const int nt = m->tilenum, wd = m->bitmap_words, slots = m->bm * m->bn;
    std::vector<int> vptr((size_t)nt + 1);
    std::vector<int> cnt((size_t)nt);
#pragma omp parallel for
    for (int t = 0; t < nt; ++t) {
        int k = 0;
        for (int w = 0; w < wd; ++w) k += __builtin_popcountll(m->tile_bitmap[(size_t)t * wd + w]);
        cnt[(size_t)t] = k;
    }
    long long run = 0;
    for (int t = 0; t < nt; ++t) {
        vptr[(size_t)t] = (int)run;
        run += cnt[(size_t)t];
    }
    if (run > 0x7ffffff0LL) return TSP_EINVAL;
    vptr[(size_t)nt] = (int)run;
    std::vector<char> pv(vs * ((size_t)run + 4), 0);
    const char *dense = (const char *)m->Blockdense_Val;
#pragma omp parallel for schedule(dynamic, 1024)
    for (int t = 0; t < nt; ++t) {
        size_t o = (size_t)vptr[(size_t)t];
        for (int s = 0; s < slots; ++s)
            if ((m->tile_bitmap[(size_t)t * wd + s / 64] >> (s % 64)) & 1ull) {
                memcpy(pv.data() + vs * o, dense + vs * ((size_t)t * slots + s), vs);
                ++o;
            }
    }
    TSP_TRY(tsp_malloc(&c.d_pval, pv.size()));
    TSP_TRY(tsp_memcpy_h2d(c.d_pval, pv.data(), pv.size()));
    TSP_TRY(round_tf32_copy(p, c.d_pval, pv.size() / vs));
    TSP_TRY(tsp_malloc((void **)&c.d_bmp, sizeof(uint64_t) * (size_t)nt * wd));
    TSP_TRY(tsp_memcpy_h2d(c.d_bmp, m->tile_bitmap, sizeof(uint64_t) * (size_t)nt * wd));
    TSP_TRY(tsp_malloc((void **)&c.d_vptr, sizeof(int) * ((size_t)nt + 1)));
    TSP_TRY(tsp_memcpy_h2d(c.d_vptr, vptr.data(), sizeof(int) * ((size_t)nt + 1)));
    return TSP_OK;
}

static int upload_dense(tsp_plan *p, ClassDev &c)
{
    if (c.d_val) return TSP_OK;
    const size_t vs = tsph::val_size(p->prec);
    TSP_TRY(tsp_malloc(&c.d_val, vs * c.m->dnssize));
    TSP_TRY(tsp_memcpy_h2d(c.d_val, c.m->Blockdense_Val, vs * c.m->dnssize));
    return round_tf32_copy(p, c.d_val, c.m->dnssize);
}

// A class reads B as split-bf16 words (tf32 tile pairs) or as values.
static bool reads_split_b(const tsp_plan *p, const ClassDev &c)
{
    return p->prec == TSP_PREC_TF32 && c.var_pr;
}

// The class's launches read B in the 3-byte form: asked for, and a kernel
// exists for the variant (tf32, single tiles, no panel sweep).
static bool b3_on(const tsp_plan *p, const ClassDev &c)
{
    return p->prec == TSP_PREC_TF32 && c.var_b3 && !c.var_pr && c.panel == 0;
}

// The class's launches load column indices per lane: asked for, and a
// lane-loaded kernel exists for the variant (every packed one; dense ones at
// chunks of up to 128 columns, without tile pairs or the panel sweep).
static bool lane_indices_on(const ClassDev &c)
{
    if (!c.var_li || c.bm == 64) return false;
    return c.fmt == 2 || ((c.var_w ? c.var_w : c.wdef) <= 128 && !c.var_pr && c.panel == 0);
}

// Launch one class on `stream` (its own stream unless given another).
static int launch_class(tsp_plan *p, ClassDev &c, void *stream = nullptr)
{
    if (!c.active() || c.ntasks == 0) return TSP_OK;
    const bool pk = c.fmt == 2;
    const bool b3 = b3_on(p, c);
    const int flags = (p->prec == TSP_PREC_TF32 ? TSP_LAUNCH_OPERANDS_TF32 : 0) |
                      (lane_indices_on(c) ? TSP_LAUNCH_LANE_INDICES : 0) | (c.var_pr ? TSP_LAUNCH_TILE_PAIRS : 0) |
                      (p->c_shared ? 0 : TSP_LAUNCH_SKIP_ZERO_STORES) | (b3 ? TSP_LAUNCH_B_3BYTE : 0);
    if (c.panel > 0) {
        // the counters are zeroed whenever the launch arguments change
        const std::vector<long long> sig{c.ntasks, c.var_w, c.var_s, c.var_tpw, c.var_order, c.place,
                                         c.panel, c.panel_lag, p->colA, c.fmt, c.var_pr};
        const int reset = sig != c.sync_sig ? TSP_LAUNCH_SYNC_RESET : 0;
        const int st = tsp_spmm_launch_panels(c.bm, p->prec, c.ntasks, p->colB_p, pk ? c.d_pval : c.d_val,
                                              pk ? c.d_bmp : nullptr, pk ? c.d_vptr : nullptr, c.d_rows,
                                              c.d_colstart, p->d_B, p->d_C, c.d_colidx, p->rowA,
                                              stream ? stream : c.stream, c.var_w, c.var_s, c.var_tpw, c.var_order,
                                              c.place, flags | reset, p->colA, c.panel, c.panel_lag,
                                              c.d_sync, kSyncInts);
        c.sync_sig = st == TSP_OK ? sig : std::vector<long long>();
        return st;
    }
    return tsp_spmm_launch_ex(c.bm, p->prec, c.ntasks, p->colB_p, pk ? c.d_pval : c.d_val, pk ? c.d_bmp : nullptr,
                              pk ? c.d_vptr : nullptr, c.d_rows, c.d_colstart,
                              reads_split_b(p, c) ? p->d_Bs : b3 ? p->d_B3 : p->d_B,
                              p->d_C, c.d_colidx, p->rowA,
                              stream ? stream : c.stream, c.var_w, c.var_s, c.var_tpw, c.var_order, c.place, flags);
}

extern "C" int tsp_plan_set_panels(tsp_plan *p, int bm, int panel_rows, int lag)
{
    if (p) ++p->version;          // any captured graph is stale now
    if (!p || panel_rows < 0 || (panel_rows > 0 && (panel_rows < 64 || (panel_rows & (panel_rows - 1)) || lag < 1)))
        return TSP_EINVAL;
    for (ClassDev &c : p->cls)
        if (c.bm == bm) {
            if (panel_rows > 0 && !c.d_sync) {
                void *d = nullptr;
                TSP_TRY(tsp_malloc(&d, sizeof(int) * (size_t)kSyncInts));
                c.d_sync = (int *)d;
                c.sync_sig.clear();      // the first launch zeroes the counters
            }
            c.panel = panel_rows;
            c.panel_lag = panel_rows > 0 ? lag : 1;
            return TSP_OK;
        }
    return TSP_EINVAL;
}

extern "C" int tsp_plan_get_panels(tsp_plan *p, int bm, int *panel_rows, int *lag)
{
    if (!p || !panel_rows || !lag) return TSP_EINVAL;
    for (ClassDev &c : p->cls)
        if (c.bm == bm) {
            *panel_rows = c.panel;
            *lag = c.panel_lag;
            return TSP_OK;
        }
    return TSP_EINVAL;
}

extern "C" int tsp_plan_set_format(tsp_plan *p, int bm, int fmt)
{
    if (p) ++p->version;          // any captured graph is stale now
    if (!p || fmt < 0 || fmt > 2) return TSP_EINVAL;
    for (ClassDev &c : p->cls)
        if (c.bm == bm) {
            if (!c.active()) return TSP_OK;
            if (fmt == 0) fmt = c.fmt;
            if (fmt == 2 && bm == 64) return TSP_EINVAL;
            TSP_TRY(tsp_device_sync());
            TSP_TRY(fmt == 2 ? upload_packed(p, c) : upload_dense(p, c));
            c.fmt = fmt;
            return TSP_OK;
        }
    return TSP_EINVAL;
}

extern "C" int tsp_plan_get_format(tsp_plan *p, int bm)
{
    if (!p) return -1;
    for (ClassDev &c : p->cls)
        if (c.bm == bm) return c.active() ? c.fmt : 0;
    return -1;
}

extern "C" int tsp_plan_set_variant(tsp_plan *p, int bm, int w, int stages, int tasks_per_wave,
                                    int order)
{
    if (p) ++p->version;          // any captured graph is stale now
    if (!p) return TSP_EINVAL;
    for (ClassDev &c : p->cls)
        if (c.bm == bm) {
            if (w > 0 && p->colB_p % w != 0) return TSP_EINVAL;
            c.var_w = w;
            c.var_s = stages;
            c.var_tpw = tasks_per_wave;
            c.var_order = order;
            return TSP_OK;
        }
    return TSP_EINVAL;
}

extern "C" int tsp_plan_set_lane_indices(tsp_plan *p, int bm, int on)
{
    if (p) ++p->version;          // any captured graph is stale now
    if (!p || (on != 0 && on != 1)) return TSP_EINVAL;
    for (ClassDev &c : p->cls)
        if (c.bm == bm) {
            if (on && bm == 64) return TSP_EINVAL;
            c.var_li = on;
            return TSP_OK;
        }
    return TSP_EINVAL;
}

extern "C" int tsp_plan_get_lane_indices(tsp_plan *p, int bm)
{
    if (!p) return -1;
    for (ClassDev &c : p->cls)
        if (c.bm == bm) return lane_indices_on(c) ? 1 : 0;
    return -1;
}

// The split-bf16 form of a tf32 plan's B (tf32 tile pairs read it): its
// canonical rows, converted once, and the spare hot-row slots, which every
// step refills from those rows.
static int ensure_split_b(tsp_plan *p)
{
    if (p->d_Bs) return TSP_OK;
    const size_t n = ((size_t)p->colA + (size_t)p->hot_cap) * (size_t)p->colB_p;
    TSP_TRY(tsp_device_sync());
    void *bs = nullptr;
    TSP_TRY(tsp_malloc(&bs, n * sizeof(float)));
    int st = tsp_split_bf16_device(p->d_B, bs, (size_t)p->colA * (size_t)p->colB_p, nullptr);
    if (st == TSP_OK && p->nhot)
        st = tsp_hot_rows_gather(bs, p->colA, (long long)sizeof(float) * p->colB_p, p->d_hot, p->nhot, nullptr);
    if (st == TSP_OK) st = tsp_device_sync();
    if (st != TSP_OK) {               // never keep a half-made copy
        tsp_free(bs);
        return st;
    }
    p->d_Bs = bs;
    return TSP_OK;
}

// The 3-byte form of a tf32 plan's B (TSP_LAUNCH_B_3BYTE): its canonical
// rows, converted once, and the spare hot-row slots, which every step
// refills from those rows.
static long long b3_row_bytes(const tsp_plan *p) { return 3LL * p->colB_p; }
static int ensure_b3(tsp_plan *p)
{
    if (p->d_B3) return TSP_OK;
    const size_t n = ((size_t)p->colA + (size_t)p->hot_cap) * (size_t)p->colB_p;
    TSP_TRY(tsp_device_sync());
    void *b3 = nullptr;
    TSP_TRY(tsp_malloc(&b3, n * 3));
    int st = tsp_pack_3byte_device(p->d_B, b3, (size_t)p->colA * (size_t)p->colB_p, nullptr);
    if (st == TSP_OK && p->nhot) st = tsp_hot_rows_gather(b3, p->colA, b3_row_bytes(p), p->d_hot, p->nhot, nullptr);
    if (st == TSP_OK) st = tsp_device_sync();
    if (st != TSP_OK) {               // never keep a half-made copy
        tsp_free(b3);
        return st;
    }
    p->d_B3 = b3;
    return TSP_OK;
}

extern "C" int tsp_plan_set_b_3byte(tsp_plan *p, int bm, int on)
{
    if (p) ++p->version;          // any captured graph is stale now
    if (!p || (on != 0 && on != 1)) return TSP_EINVAL;
    for (ClassDev &c : p->cls)
        if (c.bm == bm) {
            if (on && p->prec != TSP_PREC_TF32) return TSP_EINVAL;
            if (on) TSP_TRY(ensure_b3(p));
            c.var_b3 = on;
            return TSP_OK;
        }
    return TSP_EINVAL;
}

extern "C" int tsp_plan_get_b_3byte(tsp_plan *p, int bm)
{
    if (!p) return -1;
    for (ClassDev &c : p->cls)
        if (c.bm == bm) return b3_on(p, c) ? 1 : 0;
    return -1;
}

extern "C" int tsp_plan_set_pairs(tsp_plan *p, int bm, int on)
{
    if (p) ++p->version;          // any captured graph is stale now
    if (!p || (on != 0 && on != 1)) return TSP_EINVAL;
    for (ClassDev &c : p->cls)
        if (c.bm == bm) {
            if (on && (bm == 64 || (p->prec == TSP_PREC_TF32 && bm != 8))) return TSP_EINVAL;
            if (on && p->prec == TSP_PREC_TF32) TSP_TRY(ensure_split_b(p));
            c.var_pr = on;
            return TSP_OK;
        }
    return TSP_EINVAL;
}

extern "C" int tsp_plan_get_pairs(tsp_plan *p, int bm)
{
    if (!p) return -1;
    for (ClassDev &c : p->cls)
        if (c.bm == bm) return c.var_pr;
    return -1;
}

extern "C" int tsp_plan_set_placement(tsp_plan *p, int bm, int placement)
{
    if (p) ++p->version;          // any captured graph is stale now
    if (!p || (placement != TSP_PLACE_CONTIGUOUS && placement != TSP_PLACE_INTERLEAVED &&
               placement != TSP_PLACE_CHUNK_XCD))
        return TSP_EINVAL;
    for (ClassDev &c : p->cls)
        if (c.bm == bm) {
            c.place = placement;
            return TSP_OK;
        }
    return TSP_EINVAL;
}

extern "C" int tsp_plan_get_placement(tsp_plan *p, int bm)
{
    if (!p) return -1;
    for (ClassDev &c : p->cls)
        if (c.bm == bm) return c.place;
    return -1;
}

extern "C" int tsp_plan_get_variant(tsp_plan *p, int bm, int *w, int *stages, int *tasks_per_wave, int *order)
{
    if (!p || !w || !stages || !tasks_per_wave || !order) return TSP_EINVAL;
    for (ClassDev &c : p->cls)
        if (c.bm == bm) {
            *w = c.var_w;
            *stages = c.var_s;
            *tasks_per_wave = c.var_tpw;
            *order = c.var_order;
            return TSP_OK;
        }
    return TSP_EINVAL;
}

extern "C" int tsp_plan_destroy(tsp_plan *p)
{
    if (!p) return TSP_OK;
    tsp_device_sync();
    tsp_graph_destroy(p->graph);
    for (ClassDev &c : p->cls) {
        tsp_free(c.d_val);
        tsp_free(c.d_pval);
        tsp_free(c.d_bmp);
        tsp_free(c.d_vptr);
        tsp_free(c.d_colidx);
        tsp_free(c.d_rows);
        tsp_free(c.d_colstart);
        tsp_free(c.d_sync);
        tsp_stream_destroy(c.stream);
        if (c.dev_built) tsp_tile_destroy(&c.own);
    }
    tsp_free(p->d_B);
    tsp_free(p->d_Bs);
    tsp_free(p->d_B3);
    tsp_free(p->d_hot);
    tsp_free(p->d_flush);
    tsp_free(p->d_C);
    tsp_event_destroy(p->ev0);
    tsp_event_destroy(p->ev1);
    for (void *e : p->done) tsp_event_destroy(e);
    tsp_stream_destroy(p->main);
    delete p;
    return TSP_OK;
}

// Plan shell: B, C.  Classes are filled by the caller.
static int plan_begin(std::unique_ptr<tsp_plan> &p, int device_id, int rowA, int colA, int colB_p, int prec,
                      const void *h_B)
{
    if (rowA < 0 || colA < 0 || (prec != 0 && prec != 1)) return TSP_EINVAL;
    if (colB_p != 32 && (colB_p <= 0 || colB_p % 64)) return TSP_EINVAL;
    TSP_TRY(tsp_device_init(device_id));
    p.reset(new tsp_plan);
    p->dev = device_id;
    p->prec = prec;
    p->rowA = rowA;
    p->colA = colA;
    p->colB_p = colB_p;
    TSP_TRY(tsp_stream_create_nonblocking(&p->main));
    const size_t vs = tsph::val_size(prec);
    const size_t bbytes = vs * (size_t)colA * colB_p, cbytes = sizeof(float) * (size_t)rowA * colB_p;
    // spare rows for hot-row copies (tsp_plan_set_hot_rows); slot indices
    // colA + s must stay valid int column indices
    const long long row_bytes = (long long)vs * colB_p;
    p->hot_cap = (int)std::min<long long>({(long long)colA, TSP_HOT_MAX_BYTES / row_bytes, 0x7fffffffLL - colA});
    TSP_TRY(tsp_malloc(&p->d_B, bbytes + (size_t)row_bytes * p->hot_cap));
    if (p->hot_cap > 0) TSP_TRY(tsp_malloc((void **)&p->d_hot, sizeof(int) * (size_t)p->hot_cap));
    TSP_TRY(tsp_malloc((void **)&p->d_C, cbytes));
    if (h_B) TSP_TRY(tsp_memcpy_h2d(p->d_B, h_B, bbytes));
    TSP_TRY(round_tf32_copy(p.get(), p->d_B, (size_t)colA * colB_p));
    return tsp_memset(p->d_C, 0, cbytes);
}

// Per active class: schedule buffers (a row-block splits into at most its
// tile count of tasks) and the class stream.
static int class_finish(tsp_plan *p, ClassDev &c)
{
    tsp_kernel_info k;
    TSP_TRY(tsp_kernel_probe(c.bm, p->prec, p->colB_p, &k));
    c.wdef = k.cols_per_task;
    c.cap_tasks = (long long)c.m->tilem + c.m->tilenum;
    TSP_TRY(tsp_malloc((void **)&c.d_rows, sizeof(unsigned) * (size_t)c.cap_tasks));
    TSP_TRY(tsp_malloc((void **)&c.d_colstart, sizeof(int) * ((size_t)c.cap_tasks + 1)));
    return tsp_stream_create_nonblocking(&c.stream);
}

static int plan_end(tsp_plan *p)
{
    TSP_TRY(tsp_event_create(&p->ev0));
    TSP_TRY(tsp_event_create(&p->ev1));
    for (void *&e : p->done) TSP_TRY(tsp_event_create(&e));
    return TSP_OK;
}

// The bitmap-packed format is a tuning candidate for the 8/16-row classes
// when it moves at most 3/4 of the dense bytes.
static bool packed_pays(const Tile_matrix *m, size_t vs, long long nvals)
{
    const size_t pbytes = (size_t)nvals * vs + (size_t)m->tilenum * m->bitmap_words * 8 + (size_t)m->tilenum * 4;
    return m->bm != 64 && pbytes * 4 <= vs * m->dnssize * 3;
}

extern "C" int tsp_plan_create(tsp_plan **out, int device_id, Tile_matrix *m64, Tile_matrix *m16,
                               Tile_matrix *m8, int rowA, int colA, int colB_p, int prec,
                               const void *h_B)
{
    if (!out) return TSP_EINVAL;
    *out = nullptr;
    std::unique_ptr<tsp_plan> p;
    int st = plan_begin(p, device_id, rowA, colA, colB_p, prec, h_B);
    auto fail = [&](int s) { tsp_plan_destroy(p.release()); return s; };
    if (st) return fail(st);
    const size_t vs = tsph::val_size(prec);
    Tile_matrix *ms[3] = {m64, m16, m8};
    const int bms[3] = {64, 16, 8};
    for (int i = 0; i < 3; ++i) {
        ClassDev &c = p->cls[i];
        c.m = ms[i];
        c.bm = bms[i];
        if (!c.active()) continue;
        if (c.m->bm != bms[i] || c.m->prec != prec || c.m->bn != tsp_tile_bn(bms[i], prec)) return fail(TSP_EINVAL);
        const size_t nt = (size_t)c.m->tilenum;
        c.pack_ok = c.bm != 64 && packed_pays(c.m, vs, packed_values(c.m));
        c.fmt = 1;
        if ((st = upload_dense(p.get(), c))) return fail(st);
        if ((st = tsp_malloc((void **)&c.d_colidx, sizeof(int) * nt * c.m->bn))) return fail(st);
        if ((st = tsp_memcpy_h2d(c.d_colidx, c.m->tile_colidx, sizeof(int) * nt * c.m->bn))) return fail(st);
        if ((st = class_finish(p.get(), c))) return fail(st);
    }
    if ((st = plan_end(p.get()))) return fail(st);
    *out = p.release();
    return TSP_OK;
}

// Device-built class: upload the sub-CSR, convert on the device, keep the
// device arrays the kernels read and only tile_ptr / orig_tile_row_idx on
// the host.
static int class_from_csr(tsp_plan *p, ClassDev &c, const tsp_sub_csr *s)
{
    const int BM = c.bm, BN = tsp_tile_bn(BM, p->prec);
    Tile_matrix &m = c.own;
    memset(&m, 0, sizeof m);
    c.dev_built = true;
    c.m = &m;
    m.bm = BM;
    m.bn = BN;
    m.prec = p->prec;
    m.bitmap_words = (BM * BN + 63) / 64;
    const int rows = s ? s->rows : 0;
    m.tilem = (rows + BM - 1) / BM;
    m.tilen = (p->colA + BN - 1) / BN;
    m.tile_ptr = tsph::alloc_n<int>((size_t)m.tilem + 1);
    m.orig_tile_row_idx = tsph::alloc_n<int>((size_t)(m.tilem > 0 ? m.tilem : 1));
    if (!m.tile_ptr || !m.orig_tile_row_idx) return TSP_ENOMEM;
    m.tile_ptr[0] = 0;
    if (rows == 0) return TSP_OK;
    if (!s->ptr || !s->orig_row || (s->nnz > 0 && (!s->idx || !s->val))) return TSP_EINVAL;
    if ((long long)s->ptr[rows] != s->nnz) return TSP_EINVAL;
    for (int b = 0; b < m.tilem; ++b) m.orig_tile_row_idx[b] = s->orig_row[(size_t)b * BM];
    const size_t vs = tsph::val_size(p->prec), nnz = (size_t)s->nnz;
    void *d_ptr = nullptr, *d_idx = nullptr, *d_v = nullptr;
    struct FreeIn {
        void **a[3];
        ~FreeIn()
        {
            for (void **x : a) tsp_free(*x);
        }
    } fin{{&d_ptr, &d_idx, &d_v}};
    TSP_TRY(tsp_malloc(&d_ptr, sizeof(int) * ((size_t)rows + 1)));
    TSP_TRY(tsp_malloc(&d_idx, sizeof(int) * (nnz ? nnz : 1)));
    TSP_TRY(tsp_malloc(&d_v, vs * (nnz ? nnz : 1)));
    TSP_TRY(tsp_memcpy_h2d(d_ptr, s->ptr, sizeof(int) * ((size_t)rows + 1)));
    if (nnz) {
        TSP_TRY(tsp_memcpy_h2d(d_idx, s->idx, sizeof(int) * nnz));
        TSP_TRY(tsp_memcpy_h2d(d_v, s->val, vs * nnz));
    }
    tsp_dev_tiles dt;
    TSP_TRY(tsp_tile_create_device(&dt, rows, p->colA, s->nnz, (const int *)d_ptr, (const int *)d_idx, d_v, BM, BN,
                                   p->prec, nullptr));
    // adopt the arrays the kernels read; the plan frees them
    c.d_val = dt.d_val;
    c.d_colidx = dt.d_tile_colidx;
    c.d_bmp = (uint64_t *)dt.d_bitmap;
    m.tilenum = dt.tilenum;
    m.dnssize = (size_t)dt.tilenum * BM * BN;
    int st = tsp_memcpy_d2h(m.tile_ptr, dt.d_tile_ptr, sizeof(int) * ((size_t)m.tilem + 1));
    tsp_free(dt.d_tile_ptr);
    tsp_free(dt.d_tile_nnz);
    if (st) return st;
    TSP_TRY(round_tf32_copy(p, c.d_val, m.dnssize));
    if (c.bm != 64 && m.tilenum > 0) {
        long long nvals = 0;
        TSP_TRY(tsp_tiles_pack_device(m.tilenum, BM, BN, p->prec, nullptr, dt.d_bitmap, &nvals, nullptr, nullptr,
                                      nullptr));
        c.pack_ok = packed_pays(&m, vs, nvals);
    }
    c.fmt = 1;
    return TSP_OK;
}

extern "C" int tsp_plan_create_csr(tsp_plan **out, int device_id, const tsp_sub_csr *s64, const tsp_sub_csr *s16,
                                   const tsp_sub_csr *s8, int rowA, int colA, int colB_p, int prec,
                                   const void *h_B, double *tile_ms)
{
    if (!out) return TSP_EINVAL;
    *out = nullptr;
    std::unique_ptr<tsp_plan> p;
    int st = plan_begin(p, device_id, rowA, colA, colB_p, prec, h_B);
    auto fail = [&](int s) { tsp_plan_destroy(p.release()); return s; };
    if (st) return fail(st);
    const tsp_sub_csr *ss[3] = {s64, s16, s8};
    const int bms[3] = {64, 16, 8};
    const double t0 = now_ms();
    for (int i = 0; i < 3; ++i) {
        ClassDev &c = p->cls[i];
        c.bm = bms[i];
        if ((st = class_from_csr(p.get(), c, ss[i]))) return fail(st);
        if (c.active() && (st = class_finish(p.get(), c))) return fail(st);
    }
    if (tile_ms) *tile_ms = now_ms() - t0;
    if ((st = plan_end(p.get()))) return fail(st);
    *out = p.release();
    return TSP_OK;
}

extern "C" int tsp_plan_set_th(tsp_plan *p, int th64, int th16, int th8)
{
    if (p) ++p->version;          // any captured graph is stale now
    if (!p) return TSP_EINVAL;
    const int th[3] = {th64, th16, th8};
    for (int i = 0; i < 3; ++i) {
        ClassDev &c = p->cls[i];
        if (!c.active() || th[i] <= 0) continue;
        TSP_TRY(upload_schedule(p, c, th[i]));
    }
    return TSP_OK;
}

// Fork from main (event ev0), `reps` launches per class on its own stream,
// join back on main.
// The class a plan launches alone, or nullptr when several classes have
// tasks.  A plan with one active class launches it on the main stream: there
// is nothing to overlap, and the cross-stream fork and join cost about a
// microsecond per step on the small matrices.
static ClassDev *only_class(tsp_plan *p)
{
    ClassDev *only = nullptr;
    int active = 0;
    for (ClassDev &c : p->cls)
        if (c.active() && c.ntasks > 0) {
            ++active;
            only = &c;
        }
    return active == 1 ? only : nullptr;
}

static long long b_row_bytes(const tsp_plan *p) { return (long long)tsph::val_size(p->prec) * p->colB_p; }

// Copy the hot B rows into their slots (on main, ahead of the class kernels).
// Hot-row copies into the spare rows of each form of B that an active class
// reads.
static int hot_gather(tsp_plan *p)
{
    if (!p->nhot) return TSP_OK;
    bool plain = false, split = false, b3 = false;
    for (const ClassDev &c : p->cls)
        if (c.active() && c.ntasks > 0) (reads_split_b(p, c) ? split : b3_on(p, c) ? b3 : plain) = true;
    if (plain || (!split && !b3))
        TSP_TRY(tsp_hot_rows_gather(p->d_B, p->colA, b_row_bytes(p), p->d_hot, p->nhot, p->main));
    if (split && p->d_Bs)
        TSP_TRY(tsp_hot_rows_gather(p->d_Bs, p->colA, b_row_bytes(p), p->d_hot, p->nhot, p->main));
    if (b3 && p->d_B3)
        TSP_TRY(tsp_hot_rows_gather(p->d_B3, p->colA, b3_row_bytes(p), p->d_hot, p->nhot, p->main));
    return TSP_OK;
}

// A class of at most kTinyTiles tiles and at most 1/kTinyShare of the tiles
// of the step's largest one runs on the main stream ahead of the others:
// forked beside a class that fills the device it only starts as that
// class's waves retire, and the join then waits for its tail (configuration
// 5 with a 2-tile 16-row class beside 15.2M 8-row tiles: 3.473 ms forked,
// 3.455 ms ahead).  A larger small class overlaps enough to stay forked
// (configuration 5 in fp16 at colB 128, 20790 16-row tiles beside 7.7M
// 8-row ones: 3.478 ms forked, 3.513 ms ahead).  A single class left after
// them runs on the main stream too.
static constexpr long long kTinyShare = 128;
static constexpr long long kTinyTiles = 1024;
static bool tiny_class(const tsp_plan *p, const ClassDev &c)
{
    long long most = 0;
    for (const ClassDev &x : p->cls)
        if (x.active() && x.ntasks > 0) most = std::max<long long>(most, x.m->tilenum);
    return c.active() && c.ntasks > 0 && c.m->tilenum <= kTinyTiles && (long long)c.m->tilenum * kTinyShare <= most;
}

// The stream a step launches class c on.
static void *step_stream(tsp_plan *p, const ClassDev &c)
{
    if (tiny_class(p, c)) return p->main;
    int forked = 0;
    for (const ClassDev &x : p->cls) forked += x.active() && x.ntasks > 0 && !tiny_class(p, x);
    return forked == 1 ? p->main : c.stream;
}

static int fork_join_once(tsp_plan *p, int reps)
{
    if (ClassDev *only = only_class(p)) {
        for (int r = 0; r < reps; ++r) TSP_TRY(launch_class(p, *only, p->main));
        return TSP_OK;
    }
    // tiny classes first, then the rest: on main, or forked over the class
    // streams when several remain
    bool fork = false;
    for (int pass = 0; pass < 2; ++pass)
        for (ClassDev &c : p->cls) {
            if (!c.active() || c.ntasks == 0 || tiny_class(p, c) != (pass == 0)) continue;
            if (step_stream(p, c) != p->main) {
                fork = true;
                continue;
            }
            for (int r = 0; r < reps; ++r) TSP_TRY(launch_class(p, c, p->main));
        }
    if (!fork) return TSP_OK;
    TSP_TRY(tsp_event_record(p->ev0, p->main));
    for (int i = 0; i < 3; ++i) {
        ClassDev &c = p->cls[i];
        if (!c.active() || c.ntasks == 0 || step_stream(p, c) == p->main) continue;
        TSP_TRY(tsp_stream_wait_event(c.stream, p->ev0));
        for (int r = 0; r < reps; ++r) TSP_TRY(launch_class(p, c));
        TSP_TRY(tsp_event_record(p->done[i], c.stream));
        TSP_TRY(tsp_stream_wait_event(p->main, p->done[i]));
    }
    return TSP_OK;
}

// `reps` steps.  With hot rows every step first re-copies them (B may have
// changed since the last step), and the class kernels of one step finish
// before the next step's copy rewrites the slots they read.
static int fork_join(tsp_plan *p, int reps)
{
    if (!p->nhot) return fork_join_once(p, reps);
    for (int r = 0; r < reps; ++r) {
        TSP_TRY(hot_gather(p));
        TSP_TRY(fork_join_once(p, 1));
    }
    return TSP_OK;
}

// Gathers per column over every class's tile column indices (what each
// kernel launch reads from B), counted once on the canonical indices.
static int count_gathers(tsp_plan *p)
{
    if (!p->col_gathers.empty() || p->colA == 0) return TSP_OK;
    unsigned *d_cnt = nullptr;
    TSP_TRY(tsp_malloc((void **)&d_cnt, sizeof(unsigned) * (size_t)p->colA));
    std::unique_ptr<void, int (*)(void *)> guard(d_cnt, tsp_free);
    TSP_TRY(tsp_memset(d_cnt, 0, sizeof(unsigned) * (size_t)p->colA));
    for (ClassDev &c : p->cls)
        if (c.active())
            TSP_TRY(tsp_colidx_count(c.d_colidx, (long long)c.m->tilenum * c.m->bn, p->colA, p->d_hot, p->nhot,
                                     d_cnt, p->main));
    TSP_TRY(tsp_stream_sync(p->main));
    p->col_gathers.resize((size_t)p->colA);
    return tsp_memcpy_d2h(p->col_gathers.data(), d_cnt, sizeof(unsigned) * (size_t)p->colA);
}

extern "C" int tsp_plan_set_hot_rows(tsp_plan *p, long long budget_bytes)
{
    if (p) ++p->version;          // any captured graph is stale now
    if (!p || budget_bytes < 0) return TSP_EINVAL;
    const long long rb = b_row_bytes(p);
    const long long want = std::min<long long>(p->hot_cap, std::min(budget_bytes, TSP_HOT_MAX_BYTES) / rb);
    std::vector<int> hot;
    if (want > 0) {
        TSP_TRY(count_gathers(p));
        std::vector<int> cand;
        for (int col = 0; col < p->colA; ++col)
            if (p->col_gathers[(size_t)col] >= TSP_HOT_MIN_GATHERS) cand.push_back(col);
        if ((long long)cand.size() > want) {
            const auto more = [&](int a, int b) {
                const unsigned ga = p->col_gathers[(size_t)a], gb = p->col_gathers[(size_t)b];
                return ga != gb ? ga > gb : a < b;
            };
            std::nth_element(cand.begin(), cand.begin() + want, cand.end(), more);
            cand.resize((size_t)want);
        }
        std::sort(cand.begin(), cand.end());
        hot.swap(cand);
    }
    // kernels of an earlier run may still read the column indices and slots
    TSP_TRY(tsp_device_sync());
    int *d_map = nullptr;
    std::unique_ptr<void, int (*)(void *)> guard(nullptr, tsp_free);
    if (!hot.empty()) {
        std::vector<int> map((size_t)p->colA);
        for (int col = 0; col < p->colA; ++col) map[(size_t)col] = col;
        for (size_t s = 0; s < hot.size(); ++s) map[(size_t)hot[s]] = p->colA + (int)s;
        TSP_TRY(tsp_malloc((void **)&d_map, sizeof(int) * (size_t)p->colA));
        guard.reset(d_map);
        TSP_TRY(tsp_memcpy_h2d(d_map, map.data(), sizeof(int) * (size_t)p->colA));
    }
    for (ClassDev &c : p->cls)
        if (c.active())
            TSP_TRY(tsp_colidx_remap(c.d_colidx, (long long)c.m->tilenum * c.m->bn, p->colA, p->d_hot, p->nhot,
                                     d_map, p->main));
    TSP_TRY(tsp_stream_sync(p->main));
    p->nhot = (int)hot.size();
    if (p->nhot) TSP_TRY(tsp_memcpy_h2d(p->d_hot, hot.data(), sizeof(int) * hot.size()));
    TSP_TRY(hot_gather(p));
    return tsp_stream_sync(p->main);
}

extern "C" int tsp_plan_get_hot_rows(tsp_plan *p, int *nhot, long long *bytes)
{
    if (!p) return TSP_EINVAL;
    if (nhot) *nhot = p->nhot;
    if (bytes) *bytes = (long long)p->nhot * b_row_bytes(p);
    return TSP_OK;
}

extern "C" int tsp_plan_run(tsp_plan *p, int zero_c)
{
    if (!p) return TSP_EINVAL;
    if (zero_c) TSP_TRY(tsp_memset_async(p->d_C, 0, sizeof(float) * (size_t)p->rowA * p->colB_p, p->main));
    return fork_join(p, 1);
}

// K steps: the three classes each run K back-to-back launches concurrently,
// bracketed by events on main (as the reference times 1000 repetitions of
// the three class streams between two events, src/csr2tile.h:1043-1055).
extern "C" int tsp_plan_time(tsp_plan *p, int reps, double *ms)
{
    return tsp_plan_time_ex(p, reps, ms, nullptr);
}

// The same, plus the host's wall time to submit the steps (until the last
// launch call returns): when it is about the event time per step, the steps
// are bound by the host's launch rate rather than by the kernels.
extern "C" int tsp_plan_time_ex(tsp_plan *p, int reps, double *ms, double *submit_ms)
{
    if (!p || reps <= 0 || !ms) return TSP_EINVAL;
    void *start = nullptr;
    TSP_TRY(tsp_event_create(&start));
    std::unique_ptr<void, int (*)(void *)> guard(start, tsp_event_destroy);
    TSP_TRY(tsp_event_record(start, p->main));
    const double t0 = now_ms();
    TSP_TRY(fork_join(p, reps));
    const double t1 = now_ms();
    TSP_TRY(tsp_event_record(p->ev1, p->main));
    TSP_TRY(tsp_event_sync(p->ev1));
    float t = 0.f;
    TSP_TRY(tsp_event_elapsed_ms(&t, start, p->ev1));
    *ms = (double)t / reps;
    if (submit_ms) *submit_ms = (t1 - t0) / reps;
    return TSP_OK;
}

// HIP graph of `steps` steps: one graph launch replays them with a single
// submission, so back-to-back steps of a few microseconds are no longer
// bound by the host's per-kernel launch rate.  One step runs eagerly first
// (it settles the per-class launch state, e.g. the first launch of a
// synchronised sweep zeroes its counters), then the steps are captured on
// the main stream; the class streams join the capture through the step's
// own fork and join events.
extern "C" int tsp_plan_graph_capture(tsp_plan *p, int steps)
{
    if (!p || steps < 1 || steps > 100000) return TSP_EINVAL;
    TSP_TRY(tsp_plan_graph_free(p));
    TSP_TRY(fork_join(p, 1));
    TSP_TRY(tsp_stream_sync(p->main));
    TSP_TRY(tsp_stream_begin_capture(p->main));
    const int st = fork_join(p, steps);
    void *g = nullptr;
    const int se = tsp_stream_end_capture(p->main, st == TSP_OK ? &g : nullptr);
    if (st != TSP_OK || se != TSP_OK) {
        tsp_graph_destroy(g);
        return st != TSP_OK ? st : se;
    }
    p->graph = g;
    p->graph_steps = steps;
    p->graph_version = p->version;
    return TSP_OK;
}

extern "C" int tsp_plan_graph_free(tsp_plan *p)
{
    if (!p) return TSP_EINVAL;
    if (p->graph) {
        TSP_TRY(tsp_stream_sync(p->main));
        TSP_TRY(tsp_graph_destroy(p->graph));
    }
    p->graph = nullptr;
    p->graph_steps = 0;
    return TSP_OK;
}

extern "C" int tsp_plan_graph_run(tsp_plan *p, int replays)
{
    if (!p || replays < 0) return TSP_EINVAL;
    if (!p->graph || p->graph_version != p->version) return TSP_EINVAL;   // none, or stale
    for (int r = 0; r < replays; ++r) TSP_TRY(tsp_graph_launch(p->graph, p->main));
    return TSP_OK;
}

extern "C" int tsp_plan_graph_time(tsp_plan *p, int replays, double *ms_per_step)
{
    if (!p || replays <= 0 || !ms_per_step) return TSP_EINVAL;
    void *start = nullptr;
    TSP_TRY(tsp_event_create(&start));
    std::unique_ptr<void, int (*)(void *)> guard(start, tsp_event_destroy);
    TSP_TRY(tsp_event_record(start, p->main));
    TSP_TRY(tsp_plan_graph_run(p, replays));
    TSP_TRY(tsp_event_record(p->ev1, p->main));
    TSP_TRY(tsp_event_sync(p->ev1));
    float t = 0.f;
    TSP_TRY(tsp_event_elapsed_ms(&t, start, p->ev1));
    *ms_per_step = (double)t / ((double)replays * p->graph_steps);
    return TSP_OK;
}

extern "C" int tsp_plan_time_class(tsp_plan *p, int bm, int reps, double *ms)
{
    if (!p || reps <= 0 || !ms) return TSP_EINVAL;
    ClassDev *c = nullptr;
    for (ClassDev &x : p->cls)
        if (x.bm == bm) c = &x;
    if (!c || !c->active()) { *ms = 0.0; return TSP_OK; }
    // on the stream a step launches the class on (launches of a few
    // microseconds have timed up to twice as long on a class stream as on the
    // main stream)
    void *s = step_stream(p, *c);
    if (p->nhot) {                   // slots valid before the class runs alone
        TSP_TRY(hot_gather(p));
        TSP_TRY(tsp_stream_sync(p->main));
    }
    TSP_TRY(tsp_event_record(p->ev0, s));
    for (int r = 0; r < reps; ++r) TSP_TRY(launch_class(p, *c, s));
    TSP_TRY(tsp_event_record(p->ev1, s));
    TSP_TRY(tsp_event_sync(p->ev1));
    float t = 0.f;
    TSP_TRY(tsp_event_elapsed_ms(&t, p->ev0, p->ev1));
    *ms = (double)t / reps;
    return TSP_OK;
}

// warmup_gpu (src/csr2tile.h:798-823) with the clock read through AMD SMI.
// The clock is read right after a batch is enqueued, while its steps run (a
// reading after the batch has drained sees the idle clock), and stability is
// accepted only after at least kWarmupMinMs of steps, so batches of a few
// microseconds-long steps cannot stop the warm-up while the clock still ramps.
static constexpr double kWarmupMinMs = 20.0;

extern "C" int tsp_plan_warmup_clock(tsp_plan *p, int max_iters, int *iters_run, unsigned *clock_mhz)
{
    if (!p || max_iters < 0) return TSP_EINVAL;
    unsigned cur = 0, maxc = 0;
    TSP_TRY(tsp_gpu_clock_mhz(p->dev, &cur, &maxc));
    const bool clocked = cur > 0;
    const int limit = clocked ? max_iters : std::min(max_iters, 100);
    const auto agree = [](unsigned a, unsigned b) { return a && b && std::fabs((double)a / b - 1.0) <= 0.02; };
    unsigned prev = 0, prev2 = 0;
    int total = 0;
    const double t0 = now_ms();
    while (total < limit) {
        const int count = std::min(total == 0 ? 20 : 50, limit - total);
        for (int i = 0; i < count; ++i) TSP_TRY(tsp_plan_run(p, 0));
        if (clocked) TSP_TRY(tsp_gpu_clock_mhz(p->dev, &cur, nullptr));
        TSP_TRY(tsp_stream_sync(p->main));
        total += count;
        if (!clocked || now_ms() - t0 < kWarmupMinMs) {
            prev2 = prev;
            prev = cur;
            continue;
        }
        const bool high = maxc == 0 || (cur >= 0.95 * maxc && prev >= 0.95 * maxc);
        if (agree(cur, prev) && (high || agree(prev, prev2))) break;
        prev2 = prev;
        prev = cur;
    }
    if (iters_run) *iters_run = total;
    if (clock_mhz) *clock_mhz = clocked ? cur : 0;
    return tsp_device_sync();
}

extern "C" int tsp_plan_warmup(tsp_plan *p, int max_iters)
{
    return tsp_plan_warmup_clock(p, max_iters, nullptr, nullptr);
}

// Cold-cache tuning (TSP_TUNE_COLD): every measurement is the median of
// single launches (or steps), each after a copy over 2 x 512 MB of other
// memory, which evicts L2 (8 x 4 MB) and the 256 MB MALL.
static constexpr size_t kFlushBytes = 512ull << 20;
static constexpr int kColdReps = 7;

static int evict_caches(tsp_plan *p)
{
    TSP_TRY(tsp_copy_kernel((char *)p->d_flush + kFlushBytes, p->d_flush, kFlushBytes, p->main));
    return tsp_stream_sync(p->main);
}

static double median(std::vector<double> v)
{
    std::sort(v.begin(), v.end());
    return v[v.size() / 2];
}

static int cold_time(tsp_plan *p, int bm, double *ms)
{
    std::vector<double> t;
    for (int r = 0; r < kColdReps; ++r) {
        TSP_TRY(evict_caches(p));
        double x = 0;
        TSP_TRY(bm ? tsp_plan_time_class(p, bm, 1, &x) : tsp_plan_time(p, 1, &x));
        t.push_back(x);
    }
    *ms = median(t);
    return TSP_OK;
}

extern "C" int tsp_plan_set_tune_mode(tsp_plan *p, int mode)
{
    if (!p || (mode != TSP_TUNE_BACK_TO_BACK && mode != TSP_TUNE_COLD)) return TSP_EINVAL;
    if (mode == TSP_TUNE_COLD && !p->d_flush) TSP_TRY(tsp_malloc(&p->d_flush, 2 * kFlushBytes));
    if (mode == TSP_TUNE_BACK_TO_BACK && p->d_flush) {
        TSP_TRY(tsp_device_sync());
        TSP_TRY(tsp_free(p->d_flush));
        p->d_flush = nullptr;
    }
    p->tune_mode = mode;
    return TSP_OK;
}

extern "C" int tsp_plan_get_tune_mode(tsp_plan *p) { return p ? p->tune_mode : -1; }

// One tuning measurement of a class: a warm-up launch, then enough launches
// to span about 2 ms (at least 3, at most 200), so that short kernels are not
// decided by timer noise and long ones cost little.
static int tune_time_class(tsp_plan *p, int bm, double *ms)
{
    if (p->tune_mode == TSP_TUNE_COLD) return cold_time(p, bm, ms);
    double warm = 0;
    TSP_TRY(tsp_plan_time_class(p, bm, 1, &warm));
    const int reps = (int)std::min(200.0, std::max(3.0, 2.0 / std::max(warm, 1e-4)));
    return tsp_plan_time_class(p, bm, reps, ms);
}

// MI355X additions to the runtime tuning, measured for one class with its
// threshold fixed (each option timed on the stream a step launches the class
// on, best of two interleaved rounds, so a drift of the clock cannot decide a
// pick):
//   1. A format (dense tiles, or bitmap-packed: fewer bytes against a per-lane
//      decode) x chunk order (chunks of one task side by side share A tiles in
//      L2; chunk-major shrinks the live B working set per phase) x tasks per
//      wave (1, or 4 when row-blocks are split: consecutive tasks of a split
//      row-block then merge into one flush instead of several atomic ones);
//   2. the two best of step 1 under each XCD placement (contiguous eighths
//      keep neighbouring row-blocks, which share B rows, on one L2; runs dealt
//      round-robin balance matrices whose heavy row-blocks sit together; with
//      2, 4 or 8 column chunks, one chunk per XCD group shrinks each L2's B
//      working set);
//   3. every chunk width (32, 64, 128, 256 columns; 32 or 64 for 64-row tiles),
//      each with both chunk orders, under each placement: wider chunks mean
//      fewer waves and longer B row segments, narrower ones a smaller B
//      working set per wave and more waves (tf32 RMAT gains 11% at 32 when
//      interleaved).  Step 2's choice stays unless another is 1% faster;
//   4. the pipeline depth (1-3 tiles in flight per wave; 1-2 for 256-column
//      chunks);
//   5. the panel-synchronised sweep (tune_panels).
// A class whose variant was pinned with tsp_plan_set_variant is left alone.
static int tune_panels(tsp_plan *p, ClassDev &c, double kept_ms);
static int tune_time_step(tsp_plan *p, double min_ms, double *ms);
static int tune_class(tsp_plan *p, ClassDev &c)
{
    if (!c.active() || c.ntasks == 0 || c.var_w || c.var_order || c.var_tpw) return TSP_OK;
    c.var_pr = 0;                 // steps 1-3 without tile pairs or 3-byte B (step 4 tries them)
    c.var_b3 = 0;
    tsp_kernel_info k;
    TSP_TRY(tsp_kernel_probe(c.bm, p->prec, p->colB_p, &k));
    const bool chunks = p->colB_p / k.cols_per_task >= 2;
    bool any_split = false;
    for (int i = 0; i < c.ntasks && !any_split; ++i) any_split = (c.m->blkcoostylerowidx[i] & 0x80000000u) != 0;
    struct Opt {
        int fmt, order, tpw, place;
    };
    auto time_options = [&](const std::vector<Opt> &opts, std::vector<double> &best_of) -> int {
        best_of.assign(opts.size(), 1e30);
        for (int round = 0; round < (opts.size() > 1 ? 2 : 0); ++round)
            for (size_t j = 0; j < opts.size(); ++j) {
                TSP_TRY(tsp_plan_set_format(p, c.bm, opts[j].fmt));
                c.var_order = opts[j].order;
                c.var_tpw = opts[j].tpw;
                c.place = opts[j].place;
                double ms = 0;
                TSP_TRY(tune_time_class(p, c.bm, &ms));
                best_of[j] = std::min(best_of[j], ms);
            }
        return TSP_OK;
    };
    const bool log = getenv("TSP_TUNE_LOG") != nullptr;

    std::vector<Opt> cand;
    for (int fmt = 1; fmt <= (c.pack_ok ? 2 : 1); ++fmt)
        for (int o = chunks ? 1 : 0; o <= (chunks ? 2 : 0); ++o)
            for (int tpw = 1; tpw <= (any_split ? 4 : 1); tpw += 3) cand.push_back({fmt, o, tpw, TSP_PLACE_CONTIGUOUS});
    std::vector<double> cand_ms;
    TSP_TRY(time_options(cand, cand_ms));
    std::vector<size_t> rank(cand.size());
    for (size_t j = 0; j < cand.size(); ++j) rank[j] = j;
    std::sort(rank.begin(), rank.end(), [&](size_t a, size_t b) { return cand_ms[a] < cand_ms[b]; });
    if (log)
        for (size_t j = 0; j < cand.size(); ++j)
            fprintf(stderr, "tune bm=%d th=%d format=%d order=%d tasks/wave=%d: %.5f ms\n", c.bm, c.th, cand[j].fmt,
                    cand[j].order, cand[j].tpw, cand_ms[j]);

    // placements a launch with `nch` column chunks can use
    const auto places = [](int nch) {
        std::vector<int> v{TSP_PLACE_CONTIGUOUS, TSP_PLACE_INTERLEAVED};
        if (nch == 2 || nch == 4 || nch == 8) v.push_back(TSP_PLACE_CHUNK_XCD);
        return v;
    };
    const char *place_name[3] = {"contiguous", "interleaved", "chunk-xcd"};
    std::vector<Opt> pl;
    for (size_t j = 0; j < std::min<size_t>(2, rank.size()); ++j)
        for (int place : places(p->colB_p / k.cols_per_task)) {
            Opt o = cand[rank[j]];
            o.place = place;
            if (place == TSP_PLACE_CHUNK_XCD && o.order == 2) continue;   // order has no effect there
            pl.push_back(o);
        }
    std::vector<double> pl_ms;
    TSP_TRY(time_options(pl, pl_ms));
    size_t best = 0;
    for (size_t j = 1; j < pl.size(); ++j)
        if (pl_ms[j] < pl_ms[best]) best = j;
    if (log)
        for (size_t j = 0; j < pl.size(); ++j)
            fprintf(stderr, "tune bm=%d format=%d order=%d tasks/wave=%d placement=%s: %.5f ms%s\n", c.bm, pl[j].fmt,
                    pl[j].order, pl[j].tpw, place_name[pl[j].place], pl_ms[j],
                    j == best ? "  <- kept" : "");
    TSP_TRY(tsp_plan_set_format(p, c.bm, pl[best].fmt));
    c.var_order = pl[best].order;
    c.var_tpw = pl[best].tpw == 1 ? 0 : pl[best].tpw;
    c.place = pl[best].place;

    // 3. every chunk width, each with both chunk orders when it leaves
    //    several chunks, under both placements (width and placement interact:
    //    narrow chunks gain most when interleaved); format and tasks per wave
    //    stay as kept.  tf32 classes time every option with B in both forms:
    //    the 3-byte form moves the best width (configuration 3: 64-column
    //    chunks with 4-byte rows, 128-column ones with 3-byte rows, 3% ahead
    //    of 64) and placement (its chunks share lines that only one XCD's L2
    //    can reuse)
    struct WOpt {
        int w, order, place, b3;
    };
    // the 3-byte copy of B; without room for it that form is not tried
    const bool b3_ok = p->prec == TSP_PREC_TF32 && ensure_b3(p) == TSP_OK;
    std::vector<WOpt> wo;
    WOpt runner{-1, 0, 0, 0};            // the next best of step 3, when close
    for (int place = TSP_PLACE_CONTIGUOUS; place <= TSP_PLACE_CHUNK_XCD; ++place) {
        const auto add = [&](int w, int order) {
            wo.push_back({w, order, place, 0});
            if (b3_ok) wo.push_back({w, order, place, 1});
        };
        const std::vector<int> dp = places(p->colB_p / k.cols_per_task);
        if (std::find(dp.begin(), dp.end(), place) != dp.end())
            add(0, place == TSP_PLACE_CHUNK_XCD ? 1 : c.var_order);
        for (int w : {32, 64, 128, 256}) {
            if (w == k.cols_per_task || p->colB_p % w != 0 || (c.bm == 64 && w >= 128)) continue;
            const std::vector<int> wp = places(p->colB_p / w);
            if (std::find(wp.begin(), wp.end(), place) == wp.end()) continue;
            if (place == TSP_PLACE_CHUNK_XCD) {
                add(w, 1);
            } else if (p->colB_p / w >= 2) {
                add(w, 1);
                add(w, 2);
            } else {
                add(w, 0);
            }
        }
    }
    if (wo.size() > 2) {
        std::vector<double> wms(wo.size(), 1e30);
        for (int round = 0; round < 2; ++round)
            for (size_t j = 0; j < wo.size(); ++j) {
                c.var_w = wo[j].w;
                c.var_order = wo[j].order;
                c.place = wo[j].place;
                c.var_b3 = wo[j].b3;
                double t = 0;
                TSP_TRY(tune_time_class(p, c.bm, &t));
                wms[j] = std::min(wms[j], t);
            }
        size_t bw = 0;
        for (size_t j = 1; j < wo.size(); ++j)
            if (wms[j] < wms[bw]) bw = j;
        // keep the step-2 choice unless another option is clearly faster
        const WOpt keep{0, pl[best].order, pl[best].place, 0};
        size_t kj = 0;
        for (size_t j = 0; j < wo.size(); ++j)
            if (wo[j].w == 0 && wo[j].place == keep.place && wo[j].b3 == 0) kj = j;
        if (wms[bw] > 0.99 * wms[kj]) bw = kj;
        size_t br = bw;
        for (size_t j = 0; j < wo.size(); ++j)
            if (j != bw && (br == bw || wms[j] < wms[br])) br = j;
        if (br != bw && wms[br] < 1.03 * wms[bw]) runner = wo[br];
        c.var_w = wo[bw].w;
        c.var_order = wo[bw].order;
        c.place = wo[bw].place;
        c.var_b3 = wo[bw].b3;
        if (log)
            for (size_t j = 0; j < wo.size(); ++j)
                fprintf(stderr, "tune bm=%d chunk width %d order=%d placement=%s%s: %.5f ms%s\n", c.bm,
                        wo[j].w ? wo[j].w : k.cols_per_task, wo[j].order, place_name[wo[j].place],
                        wo[j].b3 ? " 3-byte B" : "", wms[j], j == bw ? "  <- kept" : "");
    }

    // 4. pipeline depth (1-3 tiles in flight per wave) x scalar or
    //    lane-loaded column indices (packed format, or dense tiles at chunks
    //    of up to 128 columns), for step 3's choice and
    //    for its runner-up when that was within 3% (a width that wins at
    //    depth 1 can lose once both are tuned); the rest as kept.  A deeper
    //    pipeline holds more B gathers in flight per wave but costs registers
    //    (occupancy); lane-loaded indices save the select chain for a vector
    //    load.  fp16 8- and 16-row classes also try tile pairs (two tiles per
    //    K = 32 MFMA) at 64- and 128-column chunks, tf32 8-row classes at 64
    //    (split-bf16 products), with the same depths and index modes (depth
    //    1-2 on dense tiles).  tf32 classes also try B in the 3-byte form
    //    (every width, depth and index mode).  The fastest option wins
    //    unless it is within 1% of step 3's choice at depth 1 with scalar
    //    indices (comparing each option with the best so far instead would
    //    make the pick depend on the order).
    struct DOpt {
        int w, order, place, st, li, pr, b3;
        double ms;
    };
    std::vector<WOpt> dw{{c.var_w, c.var_order, c.place, c.var_b3}};
    if (runner.w >= 0) dw.push_back(runner);
    const int nli = c.fmt == 2 ? 2 : 1;
    std::vector<DOpt> dopt;
    for (const WOpt &d : dw) {
        const int wd = d.w ? d.w : k.cols_per_task;
        for (int f = 0; f <= (b3_ok ? 1 : 0); ++f) {
            const int b3 = f ? 1 - d.b3 : d.b3;      // step 3's form first
            for (int li = 0; li < (c.fmt == 2 || (wd <= 128 && c.bm != 64) ? 2 : 1); ++li)
                for (int st = 1; st <= (wd == 256 ? 2 : 3); ++st)
                    dopt.push_back({d.w, d.order, d.place, st, li, 0, b3, 1e30});
        }
    }
    bool pair_ok = p->prec == TSP_PREC_FP16 ? c.bm != 64 : c.bm == 8;
    // tf32 pairs read a split copy of B; without room for it they are not tried
    if (pair_ok && p->prec == TSP_PREC_TF32 && ensure_split_b(p) != TSP_OK) pair_ok = false;
    if (pair_ok)
        for (int w : {64, 128}) {
            if (p->colB_p % w != 0 || !tsp_pairs_supported(c.bm, p->prec, w)) continue;
            const int nch = p->colB_p / w;
            // the kept order and placement, where this width allows them
            int place = c.place, order = nch >= 2 ? (c.var_order ? c.var_order : 1) : 0;
            if (place == TSP_PLACE_CHUNK_XCD && !(nch == 2 || nch == 4 || nch == 8)) place = TSP_PLACE_INTERLEAVED;
            for (int li = 0; li < nli; ++li)
                for (int st = 1; st <= (c.fmt == 2 ? 3 : 2); ++st) dopt.push_back({w, order, place, st, li, 1, 0, 1e30});
        }
    for (int round = 0; round < 2; ++round)
        for (DOpt &o : dopt) {
            c.var_w = o.w;
            c.var_order = o.order;
            c.place = o.place;
            c.var_s = o.st;
            c.var_li = o.li;
            c.var_pr = o.pr;
            c.var_b3 = o.b3;
            double t = 0;
            TSP_TRY(tune_time_class(p, c.bm, &t));
            o.ms = std::min(o.ms, t);
        }
    size_t db = 0;
    for (size_t j = 1; j < dopt.size(); ++j)
        if (dopt[j].ms < dopt[db].ms) db = j;
    if (dopt[db].ms > 0.99 * dopt[0].ms) db = 0;     // dopt[0]: step 3's choice, depth 1, scalar indices
    c.var_w = dopt[db].w;
    c.var_order = dopt[db].order;
    c.place = dopt[db].place;
    c.var_s = dopt[db].st;
    c.var_li = dopt[db].li;
    c.var_pr = dopt[db].pr;
    c.var_b3 = dopt[db].b3;
    if (log)
        for (size_t j = 0; j < dopt.size(); ++j)
            fprintf(stderr, "tune bm=%d chunk width %d order=%d placement=%s stages %d %s indices%s%s: %.5f ms%s\n",
                    c.bm, dopt[j].w ? dopt[j].w : k.cols_per_task, dopt[j].order, place_name[dopt[j].place],
                    dopt[j].st, dopt[j].li ? "lane" : "scalar", dopt[j].pr ? " tile pairs" : "",
                    dopt[j].b3 ? " 3-byte B" : "", dopt[j].ms, j == db ? "  <- kept" : "");
    return tune_panels(p, c, dopt[db].ms);
}

// 5. The panel-synchronised sweep (tsp_spmm_launch_panels) on the dense
//    format, one task per wave: chunk widths x both chunk orders x panels of
//    1 and 2 MB of B row segments x a lead of 2, 3 or 4 panels, then pipeline
//    depth 2 for the best of them.  Tried only when the class's work items
//    fill the device a few times at most (each generation re-reads the B
//    panels).  It stays when it is 2% faster than `kept_ms`, the time of
//    the variant steps 1-4 kept, and, when other classes run beside this one
//    in a step, when whole steps are 2% faster with it.
static int tune_panels(tsp_plan *p, ClassDev &c, double kept_ms)
{
    if (c.fmt != 1 || (long long)c.ntasks * p->colB_p / 128 > 16384) return TSP_OK;
    const bool log = getenv("TSP_TUNE_LOG") != nullptr;
    const int w0 = c.var_w, s0 = c.var_s, tpw0 = c.var_tpw, o0 = c.var_order, pl0 = c.place, pr0 = c.var_pr;
    const int vs = p->prec == TSP_PREC_FP16 ? 2 : 4;
    struct P {
        int w, order, rows, lag, s, pr;
        double ms;
    };
    std::vector<P> opts;
    const bool pairs = p->prec == TSP_PREC_FP16 && c.bm != 64;
    for (int w : {64, 128, 256}) {
        if (p->colB_p % w != 0 || (c.bm == 64 && w != 64)) continue;
        for (int pr = 0; pr <= (pairs && w <= 128 ? 1 : 0); ++pr)
            for (int order = 1; order <= (p->colB_p / w >= 2 ? 2 : 1); ++order)
                for (long long bytes : {1LL << 20, 2LL << 20}) {
                    int rows = 64;
                    while ((long long)rows * 2 * w * vs <= bytes) rows *= 2;
                    for (int lag : {2, 3, 4}) opts.push_back({w, order, rows, lag, 1, pr, 1e30});
                }
    }
    if (opts.empty()) return TSP_OK;
    const int place = pl0 == TSP_PLACE_CHUNK_XCD ? TSP_PLACE_INTERLEAVED : pl0;
    auto time_opt = [&](P &o) -> int {
        c.var_w = o.w;
        c.var_s = o.s;
        c.var_tpw = 0;
        c.var_order = o.order;
        c.place = place;
        c.var_pr = o.pr;
        TSP_TRY(tsp_plan_set_panels(p, c.bm, o.rows, o.lag));
        double t = 0;
        const int st = tune_time_class(p, c.bm, &t);
        if (st == TSP_EINVAL) return TSP_OK;          // too many generations x panels for the counters
        TSP_TRY(st);
        o.ms = std::min(o.ms, t);
        return TSP_OK;
    };
    for (int round = 0; round < 2; ++round)
        for (P &o : opts) TSP_TRY(time_opt(o));
    size_t best = 0;
    for (size_t j = 1; j < opts.size(); ++j)
        if (opts[j].ms < opts[best].ms) best = j;
    P deep = opts[best];
    deep.s = 2;
    deep.ms = 1e30;
    for (int round = 0; round < 2; ++round) TSP_TRY(time_opt(deep));
    opts.push_back(deep);
    if (deep.ms < 0.99 * opts[best].ms) best = opts.size() - 1;
    bool keep = opts[best].ms < 0.98 * kept_ms;
    if (log)
        for (size_t j = 0; j < opts.size(); ++j)
            fprintf(stderr, "tune bm=%d panels of %d rows lead %d, chunk width %d order=%d stages %d%s: %.5f ms%s\n",
                    c.bm, opts[j].rows, opts[j].lag, opts[j].w, opts[j].order, opts[j].s,
                    opts[j].pr ? " tile pairs" : "", opts[j].ms, keep && j == best ? "  <- kept" : "");
    auto apply_best = [&]() -> int {
        c.var_w = opts[best].w;
        c.var_s = opts[best].s;
        c.var_tpw = 0;
        c.var_order = opts[best].order;
        c.place = place;
        c.var_pr = opts[best].pr;
        return tsp_plan_set_panels(p, c.bm, opts[best].rows, opts[best].lag);
    };
    auto restore = [&]() -> int {
        c.var_w = w0;
        c.var_s = s0;
        c.var_tpw = tpw0;
        c.var_order = o0;
        c.place = pl0;
        c.var_pr = pr0;
        return tsp_plan_set_panels(p, c.bm, 0, 1);
    };
    // The capped grid assumes the device to itself: when other classes run
    // beside this one in a step, the sweep must also win whole steps.
    bool others = false;
    for (const ClassDev &o : p->cls) others |= &o != &c && o.active() && o.ntasks > 0;
    if (keep && others) {
        double with = 1e30, without = 1e30;
        for (int round = 0; round < 2; ++round) {
            double t = 0;
            TSP_TRY(apply_best());
            TSP_TRY(tune_time_step(p, 20.0, &t));
            with = std::min(with, t);
            TSP_TRY(restore());
            TSP_TRY(tune_time_step(p, 20.0, &t));
            without = std::min(without, t);
        }
        keep = with < 0.98 * without;
        if (log)
            fprintf(stderr, "tune bm=%d panel sweep in whole steps: %.5f ms against %.5f ms%s\n", c.bm, with, without,
                    keep ? "  <- kept" : "");
    }
    return keep ? apply_best() : restore();
}

// One tuning measurement of whole steps: a warm-up step, then enough steps to
// span about min_ms (at least 3, at most 1000).
static int tune_time_step(tsp_plan *p, double min_ms, double *ms)
{
    if (p->tune_mode == TSP_TUNE_COLD) return cold_time(p, 0, ms);
    double warm = 0;
    TSP_TRY(tsp_plan_time(p, 1, &warm));
    const int reps = (int)std::min(1000.0, std::max(3.0, min_ms / std::max(warm, 1e-4)));
    return tsp_plan_time(p, reps, ms);
}

// Hot B rows during tuning.  The thresholds and class variants are tuned
// with kHotTuneBytes of hot rows whenever any column is gathered at least
// TSP_HOT_MIN_GATHERS times; then whole steps are timed without hot rows and
// with them (best of three interleaved rounds, each 3 untimed steps after
// the switch and then at least 30 ms) and the hot rows stay when they are
// faster (each measurement includes their refill).  (With two rounds of
// 20 ms straight after the switch, configuration 5 in tf32 with B in the
// 3-byte form measured 3.55 ms with them and 3.53 without, where single runs
// of each give 3.44 and 3.61 ms.)  On the skewed MI355X cases
// the step time is flat from 8 to 64 MB of hot rows (RMAT scale 22: within
// 0.4% tf32 and 1% fp16) and 1-3% slower at 4 MB, so one budget in the middle
// of that plateau is timed instead of a noisy search over several.  Deciding
// before the variants are tuned is not enough: with the default variants the
// hot rows may miss the bar, and variants tuned without them then hide
// their gain (RMAT fp16 colB 128 ran 4.8 instead of 3.9 ms that way).
// TSP_HOT_BYTES=<bytes> pins the budget instead.
static constexpr long long kHotTuneBytes = 16LL << 20;

static int hot_candidates(tsp_plan *p, long long *ncand)
{
    *ncand = 0;
    if (p->hot_cap == 0) return TSP_OK;
    TSP_TRY(count_gathers(p));
    for (unsigned g : p->col_gathers) *ncand += g >= TSP_HOT_MIN_GATHERS;
    return TSP_OK;
}

// A class's tuned variant, to compare two tunings and reinstall one.
struct ClassVariant {
    int fmt, w, s, tpw, order, li, pr, b3, place, panel, lag;
};
static ClassVariant save_variant(const ClassDev &c)
{
    return {c.fmt, c.var_w, c.var_s, c.var_tpw, c.var_order, c.var_li, c.var_pr, c.var_b3, c.place, c.panel,
            c.panel_lag};
}
static int restore_variant(tsp_plan *p, ClassDev &c, const ClassVariant &v)
{
    if (!c.active()) return TSP_OK;
    TSP_TRY(tsp_plan_set_format(p, c.bm, v.fmt));
    TSP_TRY(tsp_plan_set_panels(p, c.bm, v.panel, v.panel > 0 ? v.lag : 1));
    c.var_w = v.w;
    c.var_s = v.s;
    c.var_tpw = v.tpw;
    c.var_order = v.order;
    c.var_li = v.li;
    c.var_pr = v.pr;
    c.var_b3 = v.b3;
    c.place = v.place;
    ++p->version;
    return TSP_OK;
}

static int decide_hot_rows(tsp_plan *p, bool *kept)
{
    const long long budgets[2] = {0, kHotTuneBytes};
    double best[2] = {1e30, 1e30};
    for (int round = 0; round < 3; ++round)
        for (int j = 0; j < 2; ++j) {
            TSP_TRY(tsp_plan_set_hot_rows(p, budgets[j]));
            double ms = 0;
            if (p->tune_mode != TSP_TUNE_COLD) TSP_TRY(tsp_plan_time(p, 3, &ms));
            TSP_TRY(tune_time_step(p, 30.0, &ms));
            best[j] = std::min(best[j], ms);
        }
    *kept = best[1] < best[0];
    if (getenv("TSP_TUNE_LOG"))
        for (int j = 0; j < 2; ++j)
            fprintf(stderr, "tune hot rows %lld MB: %.5f ms%s\n", budgets[j] >> 20, best[j],
                    (j == 1) == *kept ? "  <- kept" : "");
    return tsp_plan_set_hot_rows(p, budgets[*kept ? 1 : 0]);
}

extern "C" int tsp_plan_tune(tsp_plan *p, int tune, int th_out[3], double *model_ms, double *tune_ms)
{
    if (p) ++p->version;          // any captured graph is stale now
    if (!p) return TSP_EINVAL;
    const double t0 = now_ms();
    std::vector<int> opts[3];
    for (int i = 0; i < 3; ++i) {
        ClassDev &c = p->cls[i];
        if (!c.active()) { opts[i].push_back(0); continue; }
        tsp_th_params prm;
        TSP_TRY(tsp_th_params_probe(p->dev, c.bm, p->prec, p->colB_p, &prm));
        int top4[4];
        if (tsp_optimal_th(c.bm, p->colB_p, c.m->tilem, c.m->tile_ptr, &prm, top4) < 0) return TSP_EINVAL;
        for (int k = 0; k < 4; ++k) {
            bool dup = false;
            for (int v : opts[i]) dup |= v == top4[k];
            if (!dup) opts[i].push_back(top4[k]);
        }
    }
    const double t1 = now_ms();
    if (model_ms) *model_ms = t1 - t0;
    int best[3] = {opts[0][0], opts[1][0], opts[2][0]};
    TSP_TRY(tsp_plan_set_th(p, best[0], best[1], best[2]));
    double t2 = now_ms(), t3 = t2;
    // bring the clock up before the first option is timed: right after plan
    // creation the GPU can still be ramping, which made the first options
    // of the first step (the dense format of an 8-row class: 3.95 and 4.54
    // us against 3.56 us later) look slower than they are
    // (at most about 100 ms of steps)
    if (tune && p->tune_mode == TSP_TUNE_BACK_TO_BACK) {
        double one = 0;
        TSP_TRY(tsp_plan_time(p, 1, &one));
        const int iters = (int)std::min(20000.0, std::max(20.0, 100.0 / std::max(one, 1e-3)));
        TSP_TRY(tsp_plan_warmup_clock(p, iters, nullptr, nullptr));
    }
    bool hot_tuning = false;
    if (const char *pin = getenv("TSP_HOT_BYTES")) {
        TSP_TRY(tsp_plan_set_hot_rows(p, atoll(pin)));
    } else if (tune) {
        long long ncand = 0;
        TSP_TRY(hot_candidates(p, &ncand));
        if (ncand > 0) {
            TSP_TRY(tsp_plan_set_hot_rows(p, kHotTuneBytes));
            hot_tuning = true;
        }
    }
    const size_t combos = opts[0].size() * opts[1].size() * opts[2].size();
    if (tune && combos > 1) {
        double best_ms = 1e30;
        for (int a : opts[0])
            for (int b : opts[1])
                for (int c : opts[2]) {
                    TSP_TRY(tsp_plan_set_th(p, a, b, c));
                    double ms = 0;
                    if (p->tune_mode == TSP_TUNE_COLD) {
                        TSP_TRY(cold_time(p, 0, &ms));
                    } else {
                        for (int w = 0; w < 5; ++w) TSP_TRY(tsp_plan_run(p, 0));
                        TSP_TRY(tsp_plan_time(p, 10, &ms));
                    }
                    if (ms < best_ms) {
                        best_ms = ms;
                        best[0] = a; best[1] = b; best[2] = c;
                    }
                }
        TSP_TRY(tsp_plan_set_th(p, best[0], best[1], best[2]));
        t3 = now_ms();
    }
    if (tune) {
        for (ClassDev &c : p->cls) TSP_TRY(tune_class(p, c));
        bool kept = false;
        if (hot_tuning) TSP_TRY(decide_hot_rows(p, &kept));
        if (hot_tuning && !kept) {
            // the variants were tuned for the hot rows: tune them again
            // without, and keep the new set only if it runs the step faster
            // without hot rows than the first set does (a tuning from
            // scratch can settle elsewhere: configuration 5 in tf32 went
            // from 3.63 ms with the first set to 4.74 ms)
            ClassVariant first[3], second[3];
            for (int i = 0; i < 3; ++i) first[i] = save_variant(p->cls[i]);
            for (ClassDev &c : p->cls) {
                c.var_w = c.var_s = c.var_tpw = c.var_order = c.var_li = c.var_pr = c.var_b3 = 0;
                c.place = TSP_PLACE_CONTIGUOUS;
                TSP_TRY(tsp_plan_set_panels(p, c.bm, 0, 1));
                TSP_TRY(tune_class(p, c));
            }
            for (int i = 0; i < 3; ++i) second[i] = save_variant(p->cls[i]);
            double t[2] = {1e30, 1e30};
            for (int round = 0; round < 2; ++round)
                for (int j = 0; j < 2; ++j) {
                    for (int i = 0; i < 3; ++i) TSP_TRY(restore_variant(p, p->cls[i], j ? second[i] : first[i]));
                    double ms = 0;
                    TSP_TRY(tune_time_step(p, 20.0, &ms));
                    t[j] = std::min(t[j], ms);
                }
            const bool retuned = t[1] <= t[0];
            for (int i = 0; i < 3; ++i) TSP_TRY(restore_variant(p, p->cls[i], retuned ? second[i] : first[i]));
            if (getenv("TSP_TUNE_LOG"))
                fprintf(stderr, "tune without hot rows: variants tuned with them %.5f ms, re-tuned %.5f ms%s\n", t[0],
                        t[1], retuned ? "  <- re-tuned kept" : "  <- first kept");
        }
        // The thresholds again, with the tuned variants: the cross product
        // above timed them with the library's default variants, and a
        // class's best threshold can move with its variant (configuration 5
        // in fp16 at colB 128 kept 8 with the defaults and then ran 5% slower
        // than at 16 with its tuned variant).  One class at a time over its
        // cost-model candidates, the others as kept; whole steps of at least
        // 20 ms, best of two interleaved rounds; the cross product's pick
        // stays unless another is 1% faster.
        const bool log = getenv("TSP_TUNE_LOG") != nullptr;
        for (int i = 0; i < 3; ++i) {
            if (opts[i].size() < 2 || !p->cls[i].active()) continue;
            std::vector<double> ms(opts[i].size(), 1e30);
            for (int round = 0; round < 2; ++round)
                for (size_t j = 0; j < opts[i].size(); ++j) {
                    int th[3] = {best[0], best[1], best[2]};
                    th[i] = opts[i][j];
                    TSP_TRY(tsp_plan_set_th(p, th[0], th[1], th[2]));
                    double t = 0;
                    TSP_TRY(tune_time_step(p, 20.0, &t));
                    ms[j] = std::min(ms[j], t);
                }
            size_t bj = 0, kj = 0;
            for (size_t j = 0; j < opts[i].size(); ++j) {
                if (ms[j] < ms[bj]) bj = j;
                if (opts[i][j] == best[i]) kj = j;
            }
            if (ms[bj] > 0.99 * ms[kj]) bj = kj;
            if (log)
                for (size_t j = 0; j < opts[i].size(); ++j)
                    fprintf(stderr, "tune bm=%d threshold %d with the tuned variant: %.5f ms%s\n", p->cls[i].bm,
                            opts[i][j], ms[j], j == bj ? "  <- kept" : "");
            best[i] = opts[i][bj];
        }
        TSP_TRY(tsp_plan_set_th(p, best[0], best[1], best[2]));
        // the split and 3-byte forms of B stay only if a tuned class reads them
        bool split = false, b3 = false;
        for (ClassDev &c : p->cls) {
            split |= c.active() && reads_split_b(p, c);
            b3 |= c.active() && b3_on(p, c);
        }
        if (p->d_Bs && !split) {
            TSP_TRY(tsp_device_sync());
            TSP_TRY(tsp_free(p->d_Bs));
            p->d_Bs = nullptr;
        }
        if (p->d_B3 && !b3) {
            TSP_TRY(tsp_device_sync());
            TSP_TRY(tsp_free(p->d_B3));
            p->d_B3 = nullptr;
            for (ClassDev &c : p->cls) c.var_b3 = 0;
        }
        t3 = now_ms();
    }
    if (tune_ms) *tune_ms = t3 - t2;
    if (th_out) for (int i = 0; i < 3; ++i) th_out[i] = best[i];
    return TSP_OK;
}

extern "C" int tsp_plan_download_c(tsp_plan *p, float *h_C)
{
    if (!p || !h_C) return TSP_EINVAL;
    TSP_TRY(tsp_device_sync());
    return tsp_memcpy_d2h(h_C, p->d_C, sizeof(float) * (size_t)p->rowA * p->colB_p);
}

extern "C" int tsp_plan_device_c(tsp_plan *p, float **d_C)
{
    if (!p || !d_C) return TSP_EINVAL;
    *d_C = p->d_C;
    if (!p->c_shared) {
        p->c_shared = true;
        ++p->version;             // a graph captured with zero stores skipped is stale
    }
    return TSP_OK;
}

extern "C" int tsp_plan_tilenum(tsp_plan *p, int bm)
{
    if (!p) return -1;
    for (ClassDev &c : p->cls)
        if (c.bm == bm) return c.m ? c.m->tilenum : 0;
    return -1;
}

// tune + warmup + result run + download + timed loop + CSV fields 11-16
extern "C" int tsp_plan_execute(tsp_plan *p, long long total_nnz, float *h_C, double cpu_pre_ms,
                                int logical_colB, int repeat, int tune, FILE *csv, tsp_run_result *out)
{
    if (!p) return TSP_EINVAL;
    int th[3];
    double model_ms = 0, tune_ms = 0;
    TSP_TRY(tsp_plan_tune(p, tune, th, &model_ms, &tune_ms));
    // as call_tilespmm_cuda: warm-up (up to 1000 steps with a readable
    // clock), result run, download, warm-up again, then the timed loop
    int wit = 0;
    unsigned mhz = 0;
    TSP_TRY(tsp_plan_warmup_clock(p, 1000, &wit, &mhz));
    TSP_TRY(tsp_plan_run(p, 1));
    if (h_C) TSP_TRY(tsp_plan_download_c(p, h_C));
    TSP_TRY(tsp_plan_warmup_clock(p, 1000, &wit, &mhz));
    TSP_TRY(tsp_plan_run(p, 1));
    double ms = 0;
    TSP_TRY(tsp_plan_time(p, repeat > 0 ? repeat : 1000, &ms));
    const double tflops = 2.0 * (double)total_nnz * 1.0e-6 / ms * logical_colB / 1000.0;
    const double pre = cpu_pre_ms + model_ms + tune_ms;
    if (csv) {
        fprintf(csv, "%d,%d,%d,%.9g,%.9g,%.9g,", th[0], th[1], th[2], pre, ms, tflops);
        fflush(csv);
    }
    if (out) {
        out->th64 = th[0]; out->th16 = th[1]; out->th8 = th[2];
        out->pre_time_ms = pre;
        out->time_ms = ms;
        out->tflops = tflops;
        out->model_ms = model_ms;
        out->tune_ms = tune_ms;
        out->warmup_iters = wit;
        out->clock_mhz = mhz;
    }
    return TSP_OK;
}

extern "C" int tsp_call_tilespmm(int device_id, Tile_matrix *m64, Tile_matrix *m16, Tile_matrix *m8,
                                 int rowA, int colA, int colB_p, long long total_nnz, int prec,
                                 const void *h_B, float *h_C, double cpu_pre_ms, int logical_colB,
                                 int repeat, int tune, FILE *csv, tsp_run_result *out)
{
    tsp_plan *p = nullptr;
    TSP_TRY(tsp_plan_create(&p, device_id, m64, m16, m8, rowA, colA, colB_p, prec, h_B));
    std::unique_ptr<tsp_plan, int (*)(tsp_plan *)> guard(p, tsp_plan_destroy);
    return tsp_plan_execute(p, total_nnz, h_C, cpu_pre_ms, logical_colB, repeat, tune, csv, out);
}

// cost_model.cpp -- analytic split-threshold model and its resource inputs.
//
// Model (get_optimal_prefetch_th, src/csr2tile.h:437-642).  For each
// candidate TH = 8, 16, ..., min(128, roundup8(max row-block length)):
//   tasks(L)    = ceil(L / TH), tiles per task ceil(L / tasks(L))
//   cost(TH)    = blocks / cap * TH            (throughput)
//               + max tiles per task           (tail)
//               + sum_L cnt(L)(1 - 1/tasks(L)) * lambda_L2
//               + atom_pen * extra tasks       (atomic traffic)
//   cap         = resident blocks per CU * CUs
//   lambda_L2   = lambda_l2_scale * iteration_bytes * cap / L2 bytes
//                 (scale 1 in the reference's model)
//   atom_pen    = lambda_atom / 32 * colB, x0.04 when max length > 5 x mean
// consecutive thresholds with the same task count are skipped; the four
// cheapest survive (stable on ties).  The float arithmetic keeps this order.
//
// What is re-derived for MI355X: cap, lambda_L2 and the block count come from
// the MI355X kernels' real launch geometry (four independent wave64 tasks per
// 256-thread block, W output columns per task) and from hipDeviceProp_t /
// hipFuncGetAttributes on the device, instead of a build-time CUDA probe.
#include <math.h>
#include <string.h>

#include <vector>

#include "common.hpp"
#include "th_calibration.h"

namespace {

// Weights of the atomic and L2 terms for (class, precision, width): the
// MI355X calibration in th_calibration.h (regret-minimising fit of the
// model's top-4 against exhaustive per-threshold timings).  On gfx950 the
// re-read penalty of split row-blocks is close to zero and fp32 global
// atomics are cheap, so the fitted weights make small thresholds (16-32)
// win where the reference's weights pick 96-128.
void th_weights_mi355x(int bm, int prec, int colB_p, float *lambda_atom, float *l2_scale)
{
    const int wide = colB_p == 32 ? 0 : 1;
    *lambda_atom = 0.004f;
    *l2_scale = 1.0f;
    for (const tsp_th_weight &w : tsp_th_weight_table)
        if (w.bm == bm && w.prec == prec && w.wide == wide) {
            *lambda_atom = w.lambda_atom;
            *l2_scale = w.lambda_l2_scale;
        }
}

}  // namespace

extern "C" int tsp_optimal_th(int BM, int colB, int tilem, const int *tile_ptr,
                              const tsp_th_params *p, int top4[4])
{
    if (!p || !top4 || (tilem > 0 && !tile_ptr)) return -1;
    if (p->kernel_threads <= 0 || p->kernel_registers <= 0 || p->tasks_per_block <= 0 ||
        p->cols_per_task <= 0 || p->l2_bytes <= 0)
        return -1;
    const int th_blk = p->kernel_threads;
    const int blk_reg = p->registers_per_sm / (p->kernel_registers * th_blk);
    const int blk_smem = p->kernel_shared_bytes > 0
                             ? (int)(p->shared_bytes_per_sm / p->kernel_shared_bytes)
                             : p->blocks_per_sm;
    int blk_sm = p->threads_per_sm / th_blk;
    if (blk_reg < blk_sm) blk_sm = blk_reg;
    if (blk_smem < blk_sm) blk_sm = blk_smem;
    if (blk_sm > p->blocks_per_sm) blk_sm = p->blocks_per_sm;
    if (blk_sm <= 0) return -1;
    const float cap = (float)(blk_sm * p->sm_count);
    const float lambda_L2 = p->lambda_l2_scale * (float)(p->iteration_bytes * cap) / (float)p->l2_bytes;
    const float atom_per_col = p->lambda_atom * (1.0f / 32.0f);

    int max_len = 0;
    long long total_len = 0;
    for (int i = 0; i < tilem; ++i) {
        const int len = tile_ptr[i + 1] - tile_ptr[i];
        if (len > max_len) max_len = len;
        total_len += len;
    }
    if (max_len == 0 || tilem == 0) {
        for (int i = 0; i < 4; ++i) top4[i] = 32;
        return 1;
    }
    // Histogram of non-empty row-block lengths, walked over its occupied bins.
    std::vector<int> hist((size_t)max_len + 1, 0);
    for (int i = 0; i < tilem; ++i) {
        const int len = tile_ptr[i + 1] - tile_ptr[i];
        if (len > 0) hist[(size_t)len]++;
    }
    std::vector<int> lens;
    for (int len = 1; len <= max_len; ++len)
        if (hist[(size_t)len]) lens.push_back(len);

    const float avg_len = (float)total_len / tilem;
    float atom_pen = atom_per_col * (float)colB;
    if (max_len > avg_len * 5.0f) atom_pen *= 0.04f;
    int Tmax = (max_len + 7) / 8 * 8;
    if (Tmax > 128) Tmax = 128;
    const long long chunks = (colB + p->cols_per_task - 1) / p->cols_per_task;

    struct Cand { int th; float cost; };
    std::vector<Cand> c;
    long long prev_total = -1;
    for (int TH = 8; TH <= Tmax; TH += 8) {
        long long atom_ops = 0, total_chunk = 0;
        int max_chunk = 0;
        float l2_pen = 0.0f;
        for (int len : lens) {
            const int cnt = hist[(size_t)len];
            const int blk = (len + TH - 1) / TH;
            const int per = (len + blk - 1) / blk;
            atom_ops += (long long)(blk - 1) * cnt;
            total_chunk += (long long)blk * cnt;
            if (per > max_chunk) max_chunk = per;
            if (blk > 1) l2_pen += (1.0f - 1.0f / (float)blk) * cnt;
        }
        if (total_chunk == prev_total) continue;
        prev_total = total_chunk;
        const long long total_block = (total_chunk * chunks + p->tasks_per_block - 1) / p->tasks_per_block;
        const float cost_base = (float)total_block / cap * TH;
        const float cost_tail = (float)max_chunk;
        const float cost_l2 = l2_pen * lambda_L2;
        const float cost_comp = cost_base + cost_tail + cost_l2;
        const float cost_atom = atom_pen * atom_ops;
        c.push_back({TH, cost_comp + cost_atom});
    }
    // Stable selection of the four cheapest.
    for (size_t i = 0; i + 1 < c.size(); ++i)
        for (size_t j = 0; j + 1 < c.size() - i; ++j)
            if (c[j].cost > c[j + 1].cost) std::swap(c[j], c[j + 1]);
    for (int i = 0; i < 4; ++i) top4[i] = i < (int)c.size() ? c[(size_t)i].th : c[0].th;
    return (int)c.size();
}

extern "C" int tsp_th_weights(int bm, int prec, int colB_p, float *lambda_atom, float *lambda_l2_scale)
{
    if (!lambda_atom || !lambda_l2_scale || (bm != 64 && bm != 16 && bm != 8)) return TSP_EINVAL;
    th_weights_mi355x(bm, prec, colB_p, lambda_atom, lambda_l2_scale);
    return TSP_OK;
}

extern "C" int tsp_th_params_probe(int device_id, int bm, int prec, int colB_p, tsp_th_params *out)
{
    if (!out) return TSP_EINVAL;
    tsp_device_info d;
    int st = tsp_device_probe(device_id, &d);
    if (st) return st;
    tsp_kernel_info k;
    st = tsp_kernel_probe(bm, prec, colB_p, &k);
    if (st) return st;
    memset(out, 0, sizeof *out);
    out->sm_count = d.cu_count;
    out->threads_per_sm = d.max_threads_per_cu;
    out->registers_per_sm = d.regs_per_cu;
    out->blocks_per_sm = d.max_blocks_per_cu > 0 ? d.max_blocks_per_cu : 32;
    out->shared_bytes_per_sm = d.lds_bytes_per_cu;
    out->l2_bytes = d.l2_bytes;
    out->kernel_threads = k.threads;
    out->kernel_registers = k.registers_per_thread > 0 ? k.registers_per_thread : 1;
    out->kernel_shared_bytes = k.shared_bytes;
    out->iteration_bytes = k.iteration_bytes;
    th_weights_mi355x(bm, prec, colB_p, &out->lambda_atom, &out->lambda_l2_scale);
    out->tasks_per_block = k.tasks_per_block;
    out->cols_per_task = k.cols_per_task;
    return TSP_OK;
}

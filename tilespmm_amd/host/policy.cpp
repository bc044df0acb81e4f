// policy.cpp -- matrix features and the (gamma, delta) threshold policy.
//
// Features (features_from_stats / features_from_csr,
// src/model_features.h:9-57): [0, 0, rows, cols, nnz, 1 - nnz/(rows*cols),
// nnz/rows, max row nnz, min row nnz (empty rows count), capability, colB].
// The capability slot carries the GPU generation; on MI355X it is the gfx
// target written as major + minor/10 (gfx950 -> 9.5).
//
// Candidate action space: three fixed-group actions, a grid of ten gammas x
// six deltas, and three extra pairs -- 66 actions in the same order as the
// reference's candidate list (src/model.h:14-38), so tables trained for
// either build index the same (gamma, delta) pairs.
#include <math.h>
#include <omp.h>

#include <vector>

#include "common.hpp"
#include "policy_model.h"

namespace {

struct Cands {
    float g[66], d[66];
    int n = 0;
    Cands()
    {
        auto add = [&](float gg, float dd) { g[n] = gg; d[n] = dd; ++n; };
        add(0.0f, 1.5f);   // everything in 64-row tiles
        add(5.0f, 0.0f);   // everything in 16-row tiles
        add(5.0f, 3.0f);   // everything in 8-row tiles
        const float gammas[10] = {1.0f, 1.4f, 1.8f, 2.0f, 2.4f, 2.8f, 3.0f, 3.4f, 3.8f, 4.0f};
        const float deltas[6] = {1.0f, 1.2f, 1.4f, 1.5f, 1.8f, 2.0f};
        for (float gg : gammas)
            for (float dd : deltas) add(gg, dd);
        add(2.5f, 1.0f);
        add(2.5f, 1.2f);
        add(3.5f, 1.0f);
    }
};

const Cands &cands()
{
    static const Cands c;
    return c;
}

void select(const double *f, int index, float *gamma, float *delta)
{
    while (index >= 0) {
        const tsp_policy_node &n = tsp_policy_nodes[index];
        float v = (float)f[n.feature + 2];
        bool left = isnan(v) ? (n.missing_left_mask & 1) != 0 : v < n.cut;
        if (left) {
            if (n.left_feature < 0) index = n.child0;
            else {
                v = (float)f[n.left_feature + 2];
                left = isnan(v) ? (n.missing_left_mask & 2) != 0 : v < n.left_cut;
                index = left ? n.child0 : n.child1;
            }
        } else {
            if (n.right_feature < 0) index = n.child2;
            else {
                v = (float)f[n.right_feature + 2];
                left = isnan(v) ? (n.missing_left_mask & 4) != 0 : v < n.right_cut;
                index = left ? n.child2 : n.child3;
            }
        }
    }
    const int a = -1 - index;
    *gamma = cands().g[a];
    *delta = cands().d[a];
}

}  // namespace

extern "C" int tsp_features_from_csr(int rows, int cols, long long nnz, const int *rowptr,
                                     double capability, int colB, double *f)
{
    if (!rowptr || !f || rows <= 0 || rowptr[0] != 0 || (long long)rowptr[rows] != nnz) return 0;
    int mn = 0x7fffffff, mx = 0, bad = 0;
#pragma omp parallel for reduction(min : mn) reduction(max : mx) reduction(| : bad)
    for (int r = 0; r < rows; ++r) {
        const long long c = (long long)rowptr[r + 1] - rowptr[r];
        if (c < 0 || c > 0x7fffffffLL) bad = 1;
        else {
            if (c < mn) mn = (int)c;
            if (c > mx) mx = (int)c;
        }
    }
    if (bad || cols <= 0 || nnz < 0 || !isfinite(capability) || capability <= 0.0 || colB <= 0) return 0;
    f[0] = 0.0;
    f[1] = 0.0;
    f[2] = (double)rows;
    f[3] = (double)cols;
    f[4] = (double)nnz;
    f[5] = 1.0 - (double)nnz / ((double)rows * (double)cols);
    f[6] = (double)nnz / (double)rows;
    f[7] = (double)mx;
    f[8] = (double)mn;
    f[9] = capability;
    f[10] = (double)colB;
    return 1;
}

extern "C" void tilespmm_predict_fp16(const double *f, float *gamma, float *delta)
{
    select(f, tsp_policy_root_fp16, gamma, delta);
}

extern "C" void tilespmm_predict_tf32(const double *f, float *gamma, float *delta)
{
    select(f, tsp_policy_root_tf32, gamma, delta);
}

// Candidate list access for tuning drivers.
extern "C" int tsp_policy_candidates(float *gamma, float *delta)
{
    const Cands &c = cands();
    for (int i = 0; i < c.n; ++i) {
        if (gamma) gamma[i] = c.g[i];
        if (delta) delta[i] = c.d[i];
    }
    return c.n;
}

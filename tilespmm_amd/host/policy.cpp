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
// either build index the same (gamma, delta) pairs.  The table and its walk
// live in the generated model.h, which the reference's src/ml_predict.c
// also builds against (lib/model.so, the CPU-only policy library).
#include <math.h>
#include <omp.h>

#include <vector>

#include "common.hpp"
// the retrained table, in the format of the reference's src/model.h
// (tilespmm_shared_nodes, tilespmm_model_candidates, predictparams_*)
#include "model.h"

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
    predictparams_fp16(f, gamma, delta);
}

extern "C" void tilespmm_predict_tf32(const double *f, float *gamma, float *delta)
{
    predictparams_tf32(f, gamma, delta);
}

// Candidate list access for tuning drivers.
extern "C" int tsp_policy_candidates(float *gamma, float *delta)
{
    constexpr int n = (int)(sizeof tilespmm_model_candidates / sizeof tilespmm_model_candidates[0]);
    for (int i = 0; i < n; ++i) {
        if (gamma) gamma[i] = tilespmm_model_candidates[i][0];
        if (delta) delta[i] = tilespmm_model_candidates[i][1];
    }
    return n;
}

// cli.cpp -- the tilespmm_fp16 / tilespmm_tf32 command line.
//
//   tilespmm_fp16 -d <device> <matrix.mtx> <colB>
//   tilespmm_tf32 -d <device> <matrix.mtx> <colB>
//
// Same surface and behaviour as the reference driver (src/main.cu:136-352):
//   * A's values are replaced by 1 + rand()%3 after srand(1325), then B
//     [colA][colB_padded] is drawn the same way in row order with the padded
//     columns zero (src/main.cu:176-207), so only A's structure matters and
//     every C entry is an exact integer in fp32;
//   * colB_padded = colB <= 32 ? 32 : roundup(colB, 64) (src/main.cu:173);
//   * features -> policy (gamma, delta) -> matrix_split -> tiles, timed as
//     the preprocessing time.  The tiles are built on the GPU from the class
//     sub-CSRs (upload + device conversion, included in that time); with
//     TSP_TILING=host in the environment they are built by the host library
//     instead, as the reference does;
//   * one 19-field row is appended to ./TileSpMM-FP16.csv or
//     ./TileSpMM-TF32.csv (README.md:89-97): matrix, rows, cols, nnz, colB,
//     tilenum64/16/8, gamma, delta, TH64/16/8, pre-time, runtime, TFLOPS,
//     vendor pre-time, vendor runtime, vendor TFLOPS;
//   * the result is checked element-wise (|diff| <= 1e-3) against an
//     independent SpMM; a failed check prints NO PASS and still exits 0,
//     usage/IO/device errors exit 1.
// Differences: the independent SpMM for the check and the vendor columns is
// rocSPARSE (the reference uses cuSPARSE), and a missing or malformed .mtx
// file is an error instead of being ignored.
#include <limits.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/time.h>

#include <vector>

#include "common.hpp"

#ifndef TSP_CLI_PREC
#define TSP_CLI_PREC TSP_PREC_FP16
#endif

extern "C" int tsp_vendor_spmm(int prec, int m, int k, long long nnz, const int *rowptr,
                               const int *colidx, const void *val, int n, int ldb, const void *h_B,
                               float *h_C, int warmup, int repeat, double *pre_ms, double *ms);

static double wall_ms()
{
    struct timeval t;
    gettimeofday(&t, nullptr);
    return t.tv_sec * 1000.0 + t.tv_usec / 1000.0;
}

static int die(const char *what, int st)
{
    fprintf(stderr, "%s failed: %s (%d)\n", what, tsp_hip_error_string(st), st);
    return EXIT_FAILURE;
}

int main(int argc, char **argv)
{
    if (argc < 5 || strcmp(argv[1], "-d") != 0) {
        printf("Usage: %s -d device_id matrix.mtx colB\n", argv[0]);
        return EXIT_FAILURE;
    }
    const int prec = TSP_CLI_PREC;
    const int device_id = atoi(argv[2]);
    const char *filename = argv[3];
    printf("device_id = %i\n", device_id);
    printf("MAT: -------------- %s --------------\n", filename);

    int rowA = 0, colA = 0, is_sym = 0;
    long long nnzA = 0;
    int *rowptr = nullptr, *colidx = nullptr;
    double *dval = nullptr;
    double t1 = wall_ms();
    int st = tsp_mm_read(filename, &rowA, &colA, &nnzA, &is_sym, &rowptr, &colidx, &dval);
    if (st) {
        fprintf(stderr, "Cannot read Matrix Market file %s\n", filename);
        return EXIT_FAILURE;
    }
    double t2 = wall_ms();
    printf("  input matrix A: ( %i, %i ) nnz = %lld\n  loadfile time    = %4.5f sec\n", rowA, colA,
           nnzA, (t2 - t1) / 1000.0);
    const long long colB_ll = atoll(argv[4]);
    if (colB_ll <= 0 || colB_ll > INT_MAX - 63) {
        fprintf(stderr, "colB must be positive and fit the padded kernel width.\n");
        return EXIT_FAILURE;
    }
    const int colB = (int)colB_ll;
    const int colB_p = tsp_colB_padded(colB);
    printf("  colB = %d, padded colB = %d\n", colB, colB_p);

    // Integer value stream (src/main.cu:176-207).
    const size_t vs = tsph::val_size(prec);
    std::vector<char> aval(vs * (size_t)(nnzA ? nnzA : 1));
    srand(1325);
    for (long long i = 0; i < nnzA; ++i) {
        const float v = (float)(1 + rand() % 3);
        if (prec == TSP_PREC_FP16) ((uint16_t *)aval.data())[i] = tsph::f2h(v);
        else ((float *)aval.data())[i] = v;
    }
    const size_t nb = (size_t)colA * colB_p;
    std::vector<char> B(vs * (nb ? nb : 1));
    for (int r = 0; r < colA; ++r)
        for (int c = 0; c < colB_p; ++c) {
            const float v = c < colB ? (float)(1 + rand() % 3) : 0.0f;
            const size_t i = (size_t)r * colB_p + c;
            if (prec == TSP_PREC_FP16) ((uint16_t *)B.data())[i] = tsph::f2h(v);
            else ((float *)B.data())[i] = v;
        }
    free(dval);

    if ((st = tsp_device_init(device_id))) {
        fprintf(stderr, "Device %d is not a usable gfx950 (MI355X) GPU: %s\n", device_id,
                tsp_hip_error_string(st));
        return EXIT_FAILURE;
    }
    tsp_device_info dev;
    if ((st = tsp_device_probe(device_id, &dev))) return die("device probe", st);
    printf("---------------------------------------------------------------------------------------------\n");
    printf("  Device [ %i ] %s (%s, %d CUs) @ %4.2f MHz\n", device_id, dev.name, dev.gcn_arch,
           dev.cu_count, dev.clock_khz * 1e-3f);

    t1 = wall_ms();
    double feat[TILESPMM_ML_FEATURE_COUNT];
    const double capability = 9.5;   // gfx950
    if (!tsp_features_from_csr(rowA, colA, nnzA, rowptr, capability, colB, feat)) {
        fprintf(stderr, "Cannot extract model features from the input CSR matrix.\n");
        return EXIT_FAILURE;
    }
    float gamma = 0.f, delta = 0.f;
    if (prec == TSP_PREC_FP16) tilespmm_predict_fp16(feat, &gamma, &delta);
    else tilespmm_predict_tf32(feat, &gamma, &delta);
    tsp_sub_csr s64, s16, s8;
    if ((st = tsp_matrix_split(rowA, colA, nnzA, rowptr, colidx, aval.data(), prec, gamma, delta, &s64,
                               &s16, &s8)))
        return die("matrix_split", st);
    Tile_matrix m64, m16, m8;
    memset(&m64, 0, sizeof m64);
    memset(&m16, 0, sizeof m16);
    memset(&m8, 0, sizeof m8);
    tsp_sub_csr *subs[3] = {&s64, &s16, &s8};
    Tile_matrix *ms[3] = {&m64, &m16, &m8};
    const int bms[3] = {64, 16, 8};
    const char *tiling = getenv("TSP_TILING");
    const bool host_tiles = tiling && strcmp(tiling, "host") == 0;
    tsp_plan *plan = nullptr;
    if (host_tiles) {
        for (int i = 0; i < 3; ++i) {
            if (subs[i]->rows <= 0) continue;
            if ((st = tsp_tile_create(ms[i], subs[i]->rows, colA, subs[i]->nnz, subs[i]->ptr, subs[i]->idx,
                                      subs[i]->val, subs[i]->orig_row, bms[i], tsp_tile_bn(bms[i], prec), prec)))
                return die("Tile_create", st);
        }
        t2 = wall_ms();
        if ((st = tsp_plan_create(&plan, device_id, &m64, &m16, &m8, rowA, colA, colB_p, prec, B.data())))
            return die("plan", st);
    } else {
        // B's upload is not preprocessing: the host path uploads it outside the timed span too
        const double t_split = wall_ms();
        double tile_ms = 0;
        if ((st = tsp_plan_create_csr(&plan, device_id, &s64, &s16, &s8, rowA, colA, colB_p, prec, B.data(),
                                      &tile_ms)))
            return die("Tile_create (device)", st);
        t2 = t_split + tile_ms;
        for (int i = 0; i < 3; ++i) ms[i]->tilenum = tsp_plan_tilenum(plan, bms[i]);
    }
    const double pre_ms = t2 - t1;
    printf("  %s preprocessing time = %4.5f s\n", host_tiles ? "CPU" : "CPU+GPU", pre_ms / 1000.0);

    const char *csv_path = prec == TSP_PREC_FP16 ? "TileSpMM-FP16.csv" : "TileSpMM-TF32.csv";
    FILE *fout = fopen(csv_path, "a");
    if (!fout) {
        printf("Writing results fails.\n");
        return EXIT_FAILURE;
    }
    fprintf(fout, "%s,%d,%d,%lld,%d,%d,%d,%d,%.1f,%.1f,", filename, rowA, colA, nnzA, colB,
            m64.tilenum, m16.tilenum, m8.tilenum, gamma, delta);
    fflush(fout);

    std::vector<float> C((size_t)rowA * colB_p);
    tsp_run_result res;
    st = tsp_plan_execute(plan, nnzA, C.data(), pre_ms, colB, 1000, 1, fout, &res);
    tsp_plan_destroy(plan);
    if (st) return die("TileSpMM", st);
    printf("  TileSpMM runtime %4.3f ms, %4.3f TFlops\n", res.time_ms, res.tflops);

    std::vector<float> Cv((size_t)rowA * colB);
    double vpre = 0, vms = 0;
    if ((st = tsp_vendor_spmm(prec, rowA, colA, nnzA, rowptr, colidx, aval.data(), colB, colB_p, B.data(),
                              Cv.data(), 100, 1000, &vpre, &vms)))
        return die("rocSPARSE SpMM", st);
    const double vtf = 2.0 * (double)nnzA * colB / (vms / 1000.0) / 1e12;
    printf("  rocSPARSE runtime %4.3f ms, %4.3f Tflops\n", vms, vtf);
    fprintf(fout, "%.9g,%.9g,%.9g\n", vpre, vms, vtf);
    fclose(fout);

    size_t errors = 0;
    for (int r = 0; r < rowA; ++r)
        for (int c = 0; c < colB; ++c) {
            const double t = C[(size_t)r * colB_p + c], v = Cv[(size_t)r * colB + c];
            if (!std::isfinite(t) || !std::isfinite(v) || fabs(v - t) > 1e-3) {
                if (errors < 10) printf("  c[%d][%d], tilespmm: %lf, rocsparse: %lf\n", r, c, t, v);
                ++errors;
            }
        }
    if (errors == 0) printf("  Check... PASS!\n");
    else printf("  Check... NO PASS! error_count = %zu\n", errors);

    for (int i = 0; i < 3; ++i) {
        tsp_tile_destroy(ms[i]);
        tsp_sub_csr_free(subs[i]);
    }
    free(rowptr);
    free(colidx);
    return EXIT_SUCCESS;
}

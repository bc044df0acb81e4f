// Host preprocessing under AddressSanitizer + UndefinedBehaviorSanitizer.
//
// tests/test_host_sanitize.py builds this driver together with the host
// library sources (mmio, split, tiles, cost model, policy, generators) with
// -fsanitize=address,undefined and runs it; any sanitizer report aborts
// with a non-zero status.  The driver only exercises host code (no device
// calls), on random ragged matrices with duplicate entries and empty rows,
// every (gamma, delta) shortcut, every class and precision, several split
// thresholds, the cost model, the policy and a small Matrix Market file.
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <random>
#include <vector>

#include "../include/tilespmm.h"
#include "../include/tilespmm_hip.h"

// The cost model's device probes live in the HIP library, which this host-only
// build does not link; the driver never calls them.
extern "C" int tsp_device_probe(int, tsp_device_info *) { return TSP_ENODEV; }
extern "C" int tsp_kernel_probe(int, int, int, tsp_kernel_info *) { return TSP_ENODEV; }

static int fail(const char *what, int st)
{
    fprintf(stderr, "%s failed with status %d\n", what, st);
    return 1;
}

struct Csr {
    int rows = 0, cols = 0;
    std::vector<int> ptr, idx;
    std::vector<float> v32;
    std::vector<uint16_t> v16;
};

// Ragged rows (some empty, a few long), columns with repeats.
static Csr random_csr(std::mt19937_64 &rng, int rows, int cols, int maxlen)
{
    Csr a;
    a.rows = rows;
    a.cols = cols;
    a.ptr.assign(rows + 1, 0);
    std::uniform_int_distribution<int> len(0, maxlen), col(0, cols - 1), pick(0, 9);
    for (int r = 0; r < rows; ++r) {
        int l = pick(rng) == 0 ? 0 : len(rng);
        if (pick(rng) == 1) l = maxlen * 8;
        for (int k = 0; k < l; ++k) a.idx.push_back(col(rng));
        a.ptr[r + 1] = (int)a.idx.size();
    }
    std::uniform_real_distribution<float> val(-1.f, 1.f);
    for (size_t k = 0; k < a.idx.size(); ++k) {
        const float x = val(rng);
        a.v32.push_back(x);
        a.v16.push_back((uint16_t)(0x3c00u + (uint16_t)(k % 1024)));   // any finite fp16 pattern
    }
    return a;
}

static int exercise(const Csr &a)
{
    const long long nnz = (long long)a.idx.size();
    const float gd[][2] = {{0.f, 1.5f}, {5.f, 0.f}, {5.f, 3.f}, {2.f, 1.5f}, {1.4f, 1.8f}, {1.f, 1.f}};
    for (int prec = 0; prec < 2; ++prec) {
        const void *val = prec == 0 ? (const void *)a.v16.data() : (const void *)a.v32.data();
        double feat[TILESPMM_ML_FEATURE_COUNT];
        if (!tsp_features_from_csr(a.rows, a.cols, nnz, a.ptr.data(), 9.5, 128, feat))
            return fail("features", 0);
        float g = 0, d = 0;
        if (prec == 0) tilespmm_predict_fp16(feat, &g, &d);
        else tilespmm_predict_tf32(feat, &g, &d);
        for (const auto &p : gd) {
            tsp_sub_csr s[3];
            int st = tsp_matrix_split(a.rows, a.cols, nnz, a.ptr.data(), a.idx.data(), val, prec, p[0], p[1], &s[0],
                                      &s[1], &s[2]);
            if (st) return fail("matrix_split", st);
            const int bms[3] = {64, 16, 8};
            for (int c = 0; c < 3; ++c) {
                if (s[c].rows <= 0) continue;
                Tile_matrix m;
                memset(&m, 0, sizeof m);
                st = tsp_tile_create(&m, s[c].rows, a.cols, s[c].nnz, s[c].ptr, s[c].idx, s[c].val, s[c].orig_row,
                                     bms[c], tsp_tile_bn(bms[c], prec), prec);
                if (st) return fail("tile_create", st);
                for (int th : {1, 8, 32, 128}) {
                    int n = 0;
                    unsigned *rows = nullptr;
                    int *cs = nullptr;
                    st = tsp_tile_pretreatment(&m, th, &n, &rows, &cs);
                    if (st) return fail("tile_pretreatment", st);
                    tsp_free_host(rows);
                    tsp_free_host(cs);
                }
                tsp_th_params prm;
                memset(&prm, 0, sizeof prm);
                prm.sm_count = 256;
                prm.threads_per_sm = 2048;
                prm.registers_per_sm = 524288;
                prm.blocks_per_sm = 32;
                prm.shared_bytes_per_sm = 160 * 1024;
                prm.l2_bytes = 4 << 20;
                prm.kernel_threads = 256;
                prm.kernel_registers = 64;
                prm.kernel_shared_bytes = 9216;
                prm.iteration_bytes = 4 * (bms[c] * tsp_tile_bn(bms[c], prec) + tsp_tile_bn(bms[c], prec) * 64) * 2;
                prm.tasks_per_block = 4;
                prm.cols_per_task = 64;
                if ((st = tsp_th_weights(bms[c], prec, 128, &prm.lambda_atom, &prm.lambda_l2_scale)))
                    return fail("th_weights", st);
                int top4[4];
                if (tsp_optimal_th(bms[c], 128, m.tilem, m.tile_ptr, &prm, top4) < 0) return fail("optimal_th", -1);
                tsp_tile_destroy(&m);
            }
            for (auto &x : s) tsp_sub_csr_free(&x);
        }
    }
    return 0;
}

static int matrix_market(const char *dir)
{
    const char *files[][2] = {
        {"general.mtx", "%%MatrixMarket matrix coordinate real general\n% c\n5 4 6\n1 1 1.5\n2 3 -2\n5 4 1e-3\n3 2 4\n3 2 4\n4 1 .5\n"},
        {"sym.mtx", "%%MatrixMarket matrix coordinate real symmetric\n4 4 4\n1 1 2\n2 1 3\n4 3 -1\n4 4 7\n"},
        {"pat.mtx", "%%MatrixMarket matrix coordinate pattern general\n3 3 3\n1 2\n2 3\n3 1\n"},
        {"int.mtx", "%%MatrixMarket matrix coordinate integer skew-symmetric\n3 3 2\n2 1 5\n3 2 -4\n"},
    };
    for (auto &f : files) {
        char path[4096];
        snprintf(path, sizeof path, "%s/%s", dir, f[0]);
        FILE *fp = fopen(path, "w");
        if (!fp) return fail("fopen", 0);
        fputs(f[1], fp);
        fclose(fp);
        int rows = 0, cols = 0, sym = 0;
        long long nnz = 0;
        int *rp = nullptr, *ci = nullptr;
        double *v = nullptr;
        const int st = tsp_mm_read(path, &rows, &cols, &nnz, &sym, &rp, &ci, &v);
        if (st) return fail(f[0], st);
        tsp_free_host(rp);
        tsp_free_host(ci);
        tsp_free_host(v);
    }
    return 0;
}

int main(int argc, char **argv)
{
    std::mt19937_64 rng(20260101);
    const int shapes[][3] = {{1, 1, 1}, {7, 3, 3}, {129, 17, 17}, {777, 613, 40}, {2000, 5000, 12}};
    for (const auto &sh : shapes)
        for (int rep = 0; rep < 2; ++rep) {
            const Csr a = random_csr(rng, sh[0], sh[1], sh[2]);
            if (exercise(a)) return 1;
        }
    // a generated benchmark structure (configuration 1, 32K nonzeros)
    int rows = 0, cols = 0;
    long long nnz = 0;
    int *rp = nullptr, *ci = nullptr;
    if (int st = tsp_gen_structure(1, 0, &rows, &cols, &nnz, &rp, &ci)) return fail("gen_structure", st);
    Csr g;
    g.rows = rows;
    g.cols = cols;
    g.ptr.assign(rp, rp + rows + 1);
    g.idx.assign(ci, ci + nnz);
    g.v32.assign((size_t)nnz, 0.5f);
    g.v16.assign((size_t)nnz, (uint16_t)0x3800u);
    tsp_free_host(rp);
    tsp_free_host(ci);
    if (exercise(g)) return 1;
    if (matrix_market(argc > 1 ? argv[1] : ".")) return 1;
    printf("sanitize_host: ok\n");
    return 0;
}

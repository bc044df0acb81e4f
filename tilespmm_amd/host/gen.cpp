// gen.cpp -- seeded synthetic inputs for the five benchmark configurations.
//
//   1  uniform 4096 x 4096, exactly 8 distinct uniform columns per row,
//      A and B U[-1,1), colB 32, fp16
//   2  5-point Laplacian on a 512 x 512 grid (row y*512+x; diagonal 4,
//      neighbours -1, columns ascending), B U[-1,1), colB 128, fp16
//   3  power law, 2^20 rows, row length clip(round(xmin * u^(-1/1.1)), 1,
//      10000) (pdf ~ x^-2.1) with xmin bisected so the mean length is
//      16 +- 0.05, distinct uniform columns; A and B U[-1,1), colB 128, tf32
//   4  block-sparse 65536^2: round(0.02 * 4096^2) distinct 16x16 dense blocks
//      at random block coordinates plus round(1e-4 * 65536^2) singletons
//      (collisions dropped); A and B N(0,1), colB 256, fp16
//   5  RMAT scale 22, 2^26 edges, (a,b,c,d) = (.57,.19,.19,.05), symmetrised,
//      duplicates removed, self-loops kept; A = 1/deg(row), B U[-1,1),
//      colB 64, tf32
// Random streams: xoshiro256** seeded through splitmix64; every parallel
// chunk draws from its own stream derived from (seed, tag, chunk), so the
// output does not depend on the thread count.  fp16 values are the nearest
// half of an fp32 draw, tf32 values the nearest tf32 (both ties-to-even).
#include <math.h>
#include <omp.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <vector>

#include "common.hpp"

namespace {

inline uint64_t splitmix64(uint64_t &x)
{
    uint64_t z = (x += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

struct Rng {
    uint64_t s[4];
    explicit Rng(uint64_t seed)
    {
        uint64_t x = seed;
        for (int i = 0; i < 4; ++i) s[i] = splitmix64(x);
    }
    static uint64_t rotl(uint64_t v, int k) { return (v << k) | (v >> (64 - k)); }
    uint64_t next()
    {
        const uint64_t r = rotl(s[1] * 5, 7) * 9;
        const uint64_t t = s[1] << 17;
        s[2] ^= s[0];
        s[3] ^= s[1];
        s[1] ^= s[2];
        s[0] ^= s[3];
        s[2] ^= t;
        s[3] = rotl(s[3], 45);
        return r;
    }
    double u01() { return (double)(next() >> 11) * 0x1.0p-53; }           // [0,1)
    double u01_open() { return ((double)(next() >> 11) + 0.5) * 0x1.0p-53; }  // (0,1)
    float upm1() { return (float)((double)(next() >> 40) * 0x1.0p-23 - 1.0); }  // [-1,1), 24-bit grid
    uint32_t below(uint32_t n) { return (uint32_t)(((next() >> 32) * (uint64_t)n) >> 32); }
    float normal()
    {
        const double u1 = u01_open(), u2 = u01();
        return (float)(sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2));
    }
};

uint64_t stream_seed(uint64_t seed, uint64_t tag, uint64_t chunk)
{
    uint64_t x = seed ^ (tag * 0xd1b54a32d192ed03ull);
    uint64_t a = splitmix64(x);
    x = a ^ (chunk * 0x9e3779b97f4a7c15ull);
    return splitmix64(x);
}

enum : uint64_t { TAG_STRUCT = 1, TAG_AVAL = 2, TAG_BVAL = 3, TAG_LEN = 4 };

struct Csr {
    int rows = 0, cols = 0;
    std::vector<int> ptr, idx;
};

// k distinct sorted values in [0, n) (k <= n), by sampling with rejection.
void sample_distinct(Rng &g, uint32_t n, int k, std::vector<int> &out)
{
    out.clear();
    if (k <= 0) return;
    if ((uint64_t)k * 2 > n) {  // dense: partial Fisher-Yates on an index list
        std::vector<int> all(n);
        for (uint32_t i = 0; i < n; ++i) all[i] = (int)i;
        for (int i = 0; i < k; ++i) std::swap(all[(size_t)i], all[i + g.below(n - (uint32_t)i)]);
        out.assign(all.begin(), all.begin() + k);
        std::sort(out.begin(), out.end());
        return;
    }
    while ((int)out.size() < k) {
        const size_t need = (size_t)k - out.size();
        for (size_t i = 0; i < need; ++i) out.push_back((int)g.below(n));
        std::sort(out.begin(), out.end());
        out.erase(std::unique(out.begin(), out.end()), out.end());
    }
}

void gen_uniform8(uint64_t seed, Csr &a)
{
    a.rows = a.cols = 4096;
    a.ptr.resize(4097);
    a.idx.resize(4096 * 8);
    for (int r = 0; r <= 4096; ++r) a.ptr[(size_t)r] = 8 * r;
#pragma omp parallel
    {
        std::vector<int> row;
#pragma omp for schedule(static)
        for (int r = 0; r < 4096; ++r) {
            Rng g(stream_seed(seed, TAG_STRUCT, (uint64_t)r));
            sample_distinct(g, 4096, 8, row);
            std::copy(row.begin(), row.end(), a.idx.begin() + 8 * r);
        }
    }
}

void gen_laplacian(int nx, Csr &a, std::vector<float> &vals)
{
    const int n = nx * nx;
    a.rows = a.cols = n;
    a.ptr.assign((size_t)n + 1, 0);
    a.idx.clear();
    vals.clear();
    a.idx.reserve((size_t)n * 5);
    vals.reserve((size_t)n * 5);
    for (int y = 0; y < nx; ++y)
        for (int x = 0; x < nx; ++x) {
            const int r = y * nx + x;
            if (y > 0) { a.idx.push_back(r - nx); vals.push_back(-1.0f); }
            if (x > 0) { a.idx.push_back(r - 1); vals.push_back(-1.0f); }
            a.idx.push_back(r); vals.push_back(4.0f);
            if (x < nx - 1) { a.idx.push_back(r + 1); vals.push_back(-1.0f); }
            if (y < nx - 1) { a.idx.push_back(r + nx); vals.push_back(-1.0f); }
            a.ptr[(size_t)r + 1] = (int)a.idx.size();
        }
}

void gen_powerlaw(uint64_t seed, Csr &a)
{
    const int n = 1 << 20;
    a.rows = a.cols = n;
    // Row lengths: one uniform draw per row, then xmin bisected on the
    // realised sample so that the mean length is 16 (+- 0.05).
    std::vector<double> u((size_t)n);
    {
        const int chunks = 256, per = n / chunks;
#pragma omp parallel for schedule(static)
        for (int c = 0; c < chunks; ++c) {
            Rng g(stream_seed(seed, TAG_LEN, (uint64_t)c));
            for (int i = c * per; i < (c + 1) * per; ++i) u[(size_t)i] = g.u01_open();
        }
    }
    auto len_of = [](double xmin, double uu) {
        double x = floor(xmin * pow(uu, -1.0 / 1.1) + 0.5);
        if (x < 1) x = 1;
        if (x > 10000) x = 10000;
        return (int)x;
    };
    auto mean_for = [&](double xmin) {
        double s = 0;
#pragma omp parallel for reduction(+ : s)
        for (int i = 0; i < n; ++i) s += len_of(xmin, u[(size_t)i]);
        return s / n;
    };
    double lo = 0.1, hi = 16.0;
    for (int it = 0; it < 80; ++it) {
        const double mid = 0.5 * (lo + hi);
        if (mean_for(mid) < 16.0) lo = mid;
        else hi = mid;
        if (fabs(mean_for(0.5 * (lo + hi)) - 16.0) < 0.01) break;
    }
    const double xmin = 0.5 * (lo + hi);
    a.ptr.assign((size_t)n + 1, 0);
    for (int i = 0; i < n; ++i) a.ptr[(size_t)i + 1] = a.ptr[(size_t)i] + len_of(xmin, u[(size_t)i]);
    a.idx.resize((size_t)a.ptr[(size_t)n]);
#pragma omp parallel
    {
        std::vector<int> row;
#pragma omp for schedule(dynamic, 1024)
        for (int r = 0; r < n; ++r) {
            Rng g(stream_seed(seed, TAG_STRUCT, (uint64_t)r));
            const int L = a.ptr[(size_t)r + 1] - a.ptr[(size_t)r];
            sample_distinct(g, (uint32_t)n, L, row);
            std::copy(row.begin(), row.end(), a.idx.begin() + a.ptr[(size_t)r]);
        }
    }
}

void gen_blocksparse(uint64_t seed, Csr &a)
{
    const int n = 65536, nb = n / 16;                 // 4096 x 4096 block grid
    const long long nblocks = llround(0.02 * (double)nb * nb);       // 335,544
    const long long nsingle = llround(1e-4 * (double)n * n);         // 429,497
    a.rows = a.cols = n;
    // Distinct block ids in [0, nb*nb).
    std::vector<uint32_t> blk;
    {
        Rng g(stream_seed(seed, TAG_STRUCT, 0));
        while ((long long)blk.size() < nblocks) {
            const long long need = nblocks - (long long)blk.size();
            for (long long i = 0; i < need; ++i) blk.push_back((uint32_t)(g.next() >> 40));   // 24 bits = nb*nb
            std::sort(blk.begin(), blk.end());
            blk.erase(std::unique(blk.begin(), blk.end()), blk.end());
        }
    }
    std::vector<std::vector<int>> brow((size_t)nb);     // block columns per block row
    for (uint32_t id : blk) brow[id >> 12].push_back((int)(id & 4095));
    // Singletons: (row, col) uniform; collisions with blocks or each other dropped.
    std::vector<uint64_t> single((size_t)nsingle);
    {
        Rng g(stream_seed(seed, TAG_STRUCT, 1));
        for (long long i = 0; i < nsingle; ++i) {
            const uint64_t r = g.below((uint32_t)n), c = g.below((uint32_t)n);
            single[(size_t)i] = (r << 32) | c;
        }
        std::sort(single.begin(), single.end());
        single.erase(std::unique(single.begin(), single.end()), single.end());
    }
    std::vector<int> scnt((size_t)n, 0);
    std::vector<long long> sstart((size_t)n + 1, 0);
    for (uint64_t s : single) scnt[(size_t)(s >> 32)]++;
    for (int r = 0; r < n; ++r) sstart[(size_t)r + 1] = sstart[(size_t)r] + scnt[(size_t)r];
    // Row lengths, then fill.
    std::vector<int> len((size_t)n);
#pragma omp parallel for schedule(static)
    for (int r = 0; r < n; ++r) {
        const std::vector<int> &bc = brow[(size_t)(r / 16)];
        int l = 16 * (int)bc.size();
        for (long long k = sstart[(size_t)r]; k < sstart[(size_t)r + 1]; ++k) {
            const int c = (int)(single[(size_t)k] & 0xffffffffu);
            if (!std::binary_search(bc.begin(), bc.end(), c / 16)) ++l;
        }
        len[(size_t)r] = l;
    }
    a.ptr.assign((size_t)n + 1, 0);
    for (int r = 0; r < n; ++r) a.ptr[(size_t)r + 1] = a.ptr[(size_t)r] + len[(size_t)r];
    a.idx.resize((size_t)a.ptr[(size_t)n]);
#pragma omp parallel for schedule(static)
    for (int r = 0; r < n; ++r) {
        const std::vector<int> &bc = brow[(size_t)(r / 16)];
        int *o = a.idx.data() + a.ptr[(size_t)r];
        int k = 0;
        for (int b : bc)
            for (int j = 0; j < 16; ++j) o[k++] = 16 * b + j;
        for (long long s = sstart[(size_t)r]; s < sstart[(size_t)r + 1]; ++s) {
            const int c = (int)(single[(size_t)s] & 0xffffffffu);
            if (!std::binary_search(bc.begin(), bc.end(), c / 16)) o[k++] = c;
        }
        std::sort(o, o + k);
    }
}

void gen_rmat(uint64_t seed, int scale, long long edges, Csr &a)
{
    const int n = 1 << scale;
    a.rows = a.cols = n;
    std::vector<uint32_t> eu((size_t)edges), ev((size_t)edges);
    const int chunks = 1024;
    const long long per = (edges + chunks - 1) / chunks;
    // Quadrant thresholds: a=.57 (0,0), b=.19 (0,1), c=.19 (1,0), d=.05 (1,1).
#pragma omp parallel for schedule(dynamic, 4)
    for (int c = 0; c < chunks; ++c) {
        Rng g(stream_seed(seed, TAG_STRUCT, (uint64_t)c));
        const long long e0 = c * per, e1 = std::min(edges, e0 + per);
        for (long long e = e0; e < e1; ++e) {
            uint32_t u = 0, v = 0;
            for (int l = 0; l < scale; ++l) {
                const double p = g.u01();
                const uint32_t bu = p >= 0.76 ? 1u : 0u;                 // c or d
                const uint32_t bv = (p >= 0.57 && p < 0.76) || p >= 0.95 ? 1u : 0u;   // b or d
                u = (u << 1) | bu;
                v = (v << 1) | bv;
            }
            eu[(size_t)e] = u;
            ev[(size_t)e] = v;
        }
    }
    // Symmetrise into per-row buckets, then sort + dedupe each row.
    std::vector<std::atomic<int>> deg((size_t)n);
    for (auto &d : deg) d.store(0, std::memory_order_relaxed);
#pragma omp parallel for schedule(static)
    for (long long e = 0; e < edges; ++e) {
        deg[eu[(size_t)e]].fetch_add(1, std::memory_order_relaxed);
        deg[ev[(size_t)e]].fetch_add(1, std::memory_order_relaxed);
    }
    std::vector<long long> bstart((size_t)n + 1, 0);
    for (int r = 0; r < n; ++r) bstart[(size_t)r + 1] = bstart[(size_t)r] + deg[(size_t)r].load();
    std::vector<int> tmp((size_t)bstart[(size_t)n]);
    for (auto &d : deg) d.store(0, std::memory_order_relaxed);
#pragma omp parallel for schedule(static)
    for (long long e = 0; e < edges; ++e) {
        const uint32_t u = eu[(size_t)e], v = ev[(size_t)e];
        tmp[(size_t)(bstart[u] + deg[u].fetch_add(1, std::memory_order_relaxed))] = (int)v;
        tmp[(size_t)(bstart[v] + deg[v].fetch_add(1, std::memory_order_relaxed))] = (int)u;
    }
    eu.clear(); eu.shrink_to_fit();
    ev.clear(); ev.shrink_to_fit();
    std::vector<int> len((size_t)n);
#pragma omp parallel for schedule(dynamic, 1024)
    for (int r = 0; r < n; ++r) {
        int *b = tmp.data() + bstart[(size_t)r], *e = tmp.data() + bstart[(size_t)r + 1];
        std::sort(b, e);
        len[(size_t)r] = (int)(std::unique(b, e) - b);
    }
    a.ptr.assign((size_t)n + 1, 0);
    for (int r = 0; r < n; ++r) a.ptr[(size_t)r + 1] = a.ptr[(size_t)r] + len[(size_t)r];
    a.idx.resize((size_t)a.ptr[(size_t)n]);
#pragma omp parallel for schedule(static)
    for (int r = 0; r < n; ++r)
        std::copy(tmp.begin() + bstart[(size_t)r], tmp.begin() + bstart[(size_t)r] + len[(size_t)r],
                  a.idx.begin() + a.ptr[(size_t)r]);
}

int structure(int config, uint64_t seed, Csr &a, std::vector<float> *fixed_vals)
{
    switch (config) {
    case 1: gen_uniform8(seed, a); return 0;
    case 2: {
        std::vector<float> v;
        gen_laplacian(512, a, v);
        if (fixed_vals) fixed_vals->swap(v);
        return 0;
    }
    case 3: gen_powerlaw(seed, a); return 0;
    case 4: gen_blocksparse(seed, a); return 0;
    case 5: gen_rmat(seed, 22, 1ll << 26, a); return 0;
    default: return -1;
    }
}

void fill_values(int prec, int dist, uint64_t seed, uint64_t tag, size_t n, void *out)
{
    const size_t chunk = 1u << 16;
    const long long nch = (long long)((n + chunk - 1) / chunk);
#pragma omp parallel for schedule(static)
    for (long long c = 0; c < nch; ++c) {
        Rng g(stream_seed(seed, tag, (uint64_t)c));
        const size_t i0 = (size_t)c * chunk, i1 = std::min(n, i0 + chunk);
        for (size_t i = i0; i < i1; ++i) {
            const float x = dist == 1 ? g.normal() : g.upm1();
            if (prec == TSP_PREC_FP16) ((uint16_t *)out)[i] = tsph::f2h(x);
            else ((float *)out)[i] = tsph::round_tf32(x);
        }
    }
}

const int kDefaultPrec[6] = {0, TSP_PREC_FP16, TSP_PREC_FP16, TSP_PREC_TF32, TSP_PREC_FP16, TSP_PREC_TF32};
const int kDefaultColB[6] = {0, 32, 128, 128, 256, 64};
const int kADist[6] = {0, 0, -1, 0, 1, -2};     // -1 fixed stencil, -2 1/deg
const int kBDist[6] = {0, 0, 0, 0, 1, 0};

}  // namespace

extern "C" int tsp_colB_padded(int colB) { return colB <= 32 ? 32 : (colB + 63) / 64 * 64; }

extern "C" int tsp_gen_values(int prec, int dist, unsigned long long seed, size_t n, void *out)
{
    if ((prec != 0 && prec != 1) || (dist != 0 && dist != 1) || (!out && n)) return TSP_EINVAL;
    fill_values(prec, dist, seed, TAG_AVAL, n, out);
    return TSP_OK;
}

extern "C" int tsp_gen_structure(int config, unsigned long long seed, int *rows, int *cols,
                                 long long *nnz, int **rowptr, int **colidx)
{
    if (config < 1 || config > 5 || !rows || !cols || !nnz || !rowptr || !colidx) return TSP_EINVAL;
    if (seed == 0) seed = 20260000ull + (unsigned)config;
    Csr a;
    if (structure(config, seed, a, nullptr)) return TSP_EINVAL;
    *rows = a.rows;
    *cols = a.cols;
    *nnz = (long long)a.idx.size();
    *rowptr = tsph::alloc_n<int>(a.ptr.size());
    *colidx = tsph::alloc_n<int>(a.idx.size());
    if (!*rowptr || !*colidx) return TSP_ENOMEM;
    memcpy(*rowptr, a.ptr.data(), sizeof(int) * a.ptr.size());
    memcpy(*colidx, a.idx.data(), sizeof(int) * a.idx.size());
    return TSP_OK;
}

extern "C" int tsp_gen_rmat(int scale, long long edges, unsigned long long seed, int prec, int *rows,
                            long long *nnz, int **rowptr, int **colidx, void **val)
{
    if (scale < 1 || scale > 30 || edges < 0 || (prec != 0 && prec != 1) || !rows || !nnz || !rowptr || !colidx ||
        !val)
        return TSP_EINVAL;
    Csr a;
    gen_rmat(seed, scale, edges, a);
    const size_t nz = a.idx.size();
    *rows = a.rows;
    *nnz = (long long)nz;
    *rowptr = tsph::alloc_n<int>(a.ptr.size());
    *colidx = tsph::alloc_n<int>(nz ? nz : 1);
    *val = malloc(tsph::val_size(prec) * (nz ? nz : 1));
    if (!*rowptr || !*colidx || !*val) return TSP_ENOMEM;
    memcpy(*rowptr, a.ptr.data(), sizeof(int) * a.ptr.size());
    if (nz) memcpy(*colidx, a.idx.data(), sizeof(int) * nz);
#pragma omp parallel for schedule(static)
    for (int r = 0; r < a.rows; ++r) {
        const int deg = a.ptr[(size_t)r + 1] - a.ptr[(size_t)r];
        for (int k = a.ptr[(size_t)r]; k < a.ptr[(size_t)r + 1]; ++k) {
            const float x = 1.0f / (float)deg;
            if (prec == TSP_PREC_FP16) ((uint16_t *)*val)[k] = tsph::f2h(x);
            else ((float *)*val)[k] = tsph::round_tf32(x);
        }
    }
    return TSP_OK;
}

extern "C" int tsp_gen_config(int config, int prec, int colB, unsigned long long seed, int *rows,
                              int *cols, long long *nnz, int **rowptr, int **colidx, void **val,
                              int *colB_p_out, void **B)
{
    if (config < 1 || config > 5 || !rows || !cols || !nnz || !rowptr || !colidx || !val ||
        !colB_p_out || !B)
        return TSP_EINVAL;
    if (seed == 0) seed = 20260000ull + (unsigned)config;
    if (prec < 0) prec = kDefaultPrec[config];
    if (colB <= 0) colB = kDefaultColB[config];
    if (prec != 0 && prec != 1) return TSP_EINVAL;
    Csr a;
    std::vector<float> fixed;
    if (structure(config, seed, a, &fixed)) return TSP_EINVAL;
    const size_t nz = a.idx.size(), vs = tsph::val_size(prec);
    void *v = malloc(vs * (nz ? nz : 1));
    if (!v) return TSP_ENOMEM;
    const int adist = kADist[config];
    if (adist >= 0) {
        fill_values(prec, adist, seed, TAG_AVAL, nz, v);
    } else {
#pragma omp parallel for schedule(static)
        for (int r = 0; r < a.rows; ++r) {
            const int deg = a.ptr[(size_t)r + 1] - a.ptr[(size_t)r];
            for (int k = a.ptr[(size_t)r]; k < a.ptr[(size_t)r + 1]; ++k) {
                const float x = adist == -1 ? fixed[(size_t)k] : 1.0f / (float)deg;
                if (prec == TSP_PREC_FP16) ((uint16_t *)v)[k] = tsph::f2h(x);
                else ((float *)v)[k] = tsph::round_tf32(x);
            }
        }
    }
    const int colB_p = tsp_colB_padded(colB);
    const size_t nb = (size_t)a.cols * colB_p;
    void *b = malloc(vs * (nb ? nb : 1));
    if (!b) { free(v); return TSP_ENOMEM; }
    // Draw colB values per B row (row-major), padded columns zero.
    {
        const int bdist = kBDist[config];
        const int rows_per_chunk = std::max(1, (1 << 16) / std::max(colB, 1));
        const long long nch = (a.cols + rows_per_chunk - 1) / rows_per_chunk;
#pragma omp parallel for schedule(static)
        for (long long c = 0; c < nch; ++c) {
            Rng g(stream_seed(seed, TAG_BVAL, (uint64_t)c));
            const int r0 = (int)(c * rows_per_chunk), r1 = std::min(a.cols, r0 + rows_per_chunk);
            for (int r = r0; r < r1; ++r)
                for (int j = 0; j < colB_p; ++j) {
                    const size_t o = (size_t)r * colB_p + j;
                    float x = 0.0f;
                    if (j < colB) x = bdist == 1 ? g.normal() : g.upm1();
                    if (prec == TSP_PREC_FP16) ((uint16_t *)b)[o] = tsph::f2h(x);
                    else ((float *)b)[o] = tsph::round_tf32(x);
                }
        }
    }
    *rows = a.rows;
    *cols = a.cols;
    *nnz = (long long)nz;
    *rowptr = tsph::alloc_n<int>(a.ptr.size());
    *colidx = tsph::alloc_n<int>(nz);
    if (!*rowptr || !*colidx) { free(v); free(b); return TSP_ENOMEM; }
    memcpy(*rowptr, a.ptr.data(), sizeof(int) * a.ptr.size());
    memcpy(*colidx, a.idx.data(), sizeof(int) * nz);
    *val = v;
    *colB_p_out = colB_p;
    *B = b;
    return TSP_OK;
}

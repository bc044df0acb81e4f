// mmio.cpp -- Matrix Market coordinate reader with the reference's semantics
// (mmio_allinone, src/mmio_highlevel.h:307-480; banner and size line,
// src/mmio.h:394-480, 564-590): entries kept in file order inside each row,
// symmetric and hermitian files mirrored (diagonal once), pattern -> 1.0,
// integer -> its value, complex -> real part, no sorting, no duplicate
// merging.  The file is read in one pass into memory and parsed by hand,
// which is several times faster than fscanf for GB-sized inputs.
#include <ctype.h>
#include <errno.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <strings.h>

#include <string>
#include <vector>

#include "common.hpp"

namespace {

struct Cursor {
    const char *p, *end;
    void skip_ws()
    {
        while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) ++p;
    }
    bool read_long(long long *v)
    {
        skip_ws();
        if (p >= end) return false;
        char *e = nullptr;
        errno = 0;
        long long x = strtoll(p, &e, 10);
        if (e == p || errno) return false;
        p = e;
        *v = x;
        return true;
    }
    bool read_double(double *v)
    {
        skip_ws();
        if (p >= end) return false;
        char *e = nullptr;
        double x = strtod(p, &e);
        if (e == p) return false;
        p = e;
        *v = x;
        return true;
    }
};

}  // namespace

extern "C" int tsp_mm_read(const char *path, int *rows_out, int *cols_out, long long *nnz_out,
                           int *is_sym_out, int **rowptr_out, int **colidx_out, double **val_out)
{
    FILE *f = fopen(path, "rb");
    if (!f) return TSP_EIO;
    if (fseek(f, 0, SEEK_END) != 0) { fclose(f); return TSP_EIO; }
    long long fsize = ftell(f);
    rewind(f);
    if (fsize <= 0) { fclose(f); return TSP_EIO; }
    std::vector<char> buf((size_t)fsize + 1);
    if (fread(buf.data(), 1, (size_t)fsize, f) != (size_t)fsize) { fclose(f); return TSP_EIO; }
    fclose(f);
    buf[(size_t)fsize] = '\0';
    const char *p = buf.data(), *end = buf.data() + fsize;

    // Banner: %%MatrixMarket matrix coordinate <type> <symmetry>
    const char *nl = (const char *)memchr(p, '\n', (size_t)(end - p));
    if (!nl) return TSP_EIO;
    char banner[64], mtx[64], crd[64], dtype[64], storage[64];
    std::string first(p, nl);
    if (sscanf(first.c_str(), "%63s %63s %63s %63s %63s", banner, mtx, crd, dtype, storage) != 5)
        return TSP_EIO;
    if (strncmp(banner, "%%MatrixMarket", 14) != 0) return TSP_EIO;
    if (strcasecmp(mtx, "matrix") != 0 || strcasecmp(crd, "coordinate") != 0) return TSP_EIO;
    enum { REAL, CPLX, INTG, PATT } ty;
    if (!strcasecmp(dtype, "real")) ty = REAL;
    else if (!strcasecmp(dtype, "complex")) ty = CPLX;
    else if (!strcasecmp(dtype, "integer")) ty = INTG;
    else if (!strcasecmp(dtype, "pattern")) ty = PATT;
    else return TSP_EIO;
    const bool sym = !strcasecmp(storage, "symmetric") || !strcasecmp(storage, "hermitian");
    if (!sym && strcasecmp(storage, "general") && strcasecmp(storage, "skew-symmetric")) return TSP_EIO;
    p = nl + 1;
    // Comment lines, then the size line.
    while (p < end && *p == '%') {
        const char *q = (const char *)memchr(p, '\n', (size_t)(end - p));
        p = q ? q + 1 : end;
    }
    Cursor cur{p, end};
    long long m, n, nz;
    if (!cur.read_long(&m) || !cur.read_long(&n) || !cur.read_long(&nz)) return TSP_EIO;
    if (m < 0 || n < 0 || nz < 0 || m > 0x7ffffffe || n > 0x7ffffffe) return TSP_EIO;

    std::vector<int> ri((size_t)nz), ci((size_t)nz);
    std::vector<double> vv((size_t)nz);
    std::vector<long long> cnt((size_t)m + 1, 0);
    for (long long k = 0; k < nz; ++k) {
        long long i, j;
        double re = 1.0, im;
        if (!cur.read_long(&i) || !cur.read_long(&j)) return TSP_EIO;
        if (ty == REAL || ty == CPLX) {
            if (!cur.read_double(&re)) return TSP_EIO;
            if (ty == CPLX && !cur.read_double(&im)) return TSP_EIO;
        } else if (ty == INTG) {
            long long iv;
            if (!cur.read_long(&iv)) return TSP_EIO;
            re = (double)iv;
        }
        if (i < 1 || i > m || j < 1 || j > n) return TSP_EIO;
        ri[(size_t)k] = (int)(i - 1);
        ci[(size_t)k] = (int)(j - 1);
        vv[(size_t)k] = re;
        cnt[(size_t)(i - 1)]++;
    }
    if (sym)
        for (long long k = 0; k < nz; ++k)
            if (ri[(size_t)k] != ci[(size_t)k]) cnt[(size_t)ci[(size_t)k]]++;
    long long run = 0;
    for (long long r = 0; r <= m; ++r) {
        long long c = cnt[(size_t)r];
        cnt[(size_t)r] = run;
        run += c;
    }
    if (run > 0x7fffffffLL) return TSP_EINVAL;
    int *rowptr = tsph::alloc_n<int>((size_t)m + 1);
    int *col = tsph::alloc_n<int>((size_t)run);
    double *val = tsph::alloc_n<double>((size_t)run);
    if (!rowptr || !col || !val) { free(rowptr); free(col); free(val); return TSP_ENOMEM; }
    for (long long r = 0; r <= m; ++r) rowptr[r] = (int)cnt[(size_t)r];
    std::vector<long long> fill((size_t)m + 1, 0);
    for (long long k = 0; k < nz; ++k) {
        const int a = ri[(size_t)k], b = ci[(size_t)k];
        long long o = cnt[(size_t)a] + fill[(size_t)a]++;
        col[o] = b;
        val[o] = vv[(size_t)k];
        if (sym && a != b) {
            o = cnt[(size_t)b] + fill[(size_t)b]++;
            col[o] = a;
            val[o] = vv[(size_t)k];
        }
    }
    *rows_out = (int)m;
    *cols_out = (int)n;
    *nnz_out = run;
    *is_sym_out = sym ? 1 : 0;
    *rowptr_out = rowptr;
    *colidx_out = col;
    *val_out = val;
    return TSP_OK;
}

extern "C" void tsp_free_host(void *p) { free(p); }

// mmio.cpp -- Matrix Market coordinate reader with the reference's semantics
// (mmio_allinone, src/mmio_highlevel.h:307-480; banner and size line,
// src/mmio.h:394-480, 564-590): entries kept in file order inside each row,
// symmetric and hermitian files mirrored (diagonal once), pattern -> 1.0,
// integer -> its value, complex -> real part, no sorting, no duplicate
// merging.  The file is read in one pass into memory and the entry lines are
// parsed in parallel: the data section is cut into chunks at line
// boundaries, every thread parses its chunks into local arrays, and the
// chunks are concatenated in file order.  A file whose entries do not sit one
// per line (legal for fscanf-style readers) is parsed again sequentially.
#include <ctype.h>
#include <errno.h>
#include <omp.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <strings.h>

#include <memory>
#include <string>
#include <vector>

#include "common.hpp"

namespace {

// Decimal -> double, correctly rounded: Clinger's fast path (at most 19
// significant digits with mantissa <= 2^53 and a power of ten in
// [1e-22, 1e22], where one exact multiply or divide rounds once), strtod
// for everything else.  Returns the end of the token or nullptr.
const double kPow10[23] = {1e0,  1e1,  1e2,  1e3,  1e4,  1e5,  1e6,  1e7,  1e8,  1e9,  1e10, 1e11,
                           1e12, 1e13, 1e14, 1e15, 1e16, 1e17, 1e18, 1e19, 1e20, 1e21, 1e22};

const char *parse_double(const char *p, double *out)
{
    const char *s = p;
    bool neg = false;
    if (*p == '+' || *p == '-') neg = *p++ == '-';
    unsigned long long mant = 0;
    int digits = 0, exp10 = 0;
    bool any = false, slow = false;
    while (*p >= '0' && *p <= '9') {
        any = true;
        if (mant == 0 && *p == '0') { ++p; continue; }
        if (digits < 19) { mant = mant * 10 + (unsigned)(*p - '0'); ++digits; }
        else { slow = true; ++exp10; }
        ++p;
    }
    if (*p == '.') {
        ++p;
        while (*p >= '0' && *p <= '9') {
            any = true;
            if (mant == 0 && *p == '0') { --exp10; ++p; continue; }
            if (digits < 19) { mant = mant * 10 + (unsigned)(*p - '0'); ++digits; --exp10; }
            else slow = true;
            ++p;
        }
    }
    if (!any) slow = true;                       // inf, nan, hex, or not a number
    if (!slow && (*p == 'e' || *p == 'E')) {
        const char *q = p + 1;
        bool eneg = false;
        if (*q == '+' || *q == '-') eneg = *q++ == '-';
        if (*q < '0' || *q > '9') slow = true;
        int e = 0;
        while (*q >= '0' && *q <= '9') {
            if (e < 100000) e = e * 10 + (*q - '0');
            ++q;
        }
        exp10 += eneg ? -e : e;
        p = q;
    }
    if (!slow && (*p == 'x' || *p == 'X' || (*p >= 'a' && *p <= 'z') || (*p >= 'A' && *p <= 'Z'))) slow = true;
    if (!slow && mant <= (1ull << 53) && exp10 >= -22 && exp10 <= 22) {
        double v = (double)mant;
        v = exp10 >= 0 ? v * kPow10[exp10] : v / kPow10[-exp10];
        *out = neg ? -v : v;
        return p;
    }
    char *e = nullptr;
    const double v = strtod(s, &e);
    if (e == s) return nullptr;
    *out = v;
    return e;
}

// Decimal integer with optional sign; nullptr if none or out of range.
const char *parse_long(const char *p, long long *out)
{
    bool neg = false;
    if (*p == '+' || *p == '-') neg = *p++ == '-';
    if (*p < '0' || *p > '9') return nullptr;
    unsigned long long v = 0;
    while (*p >= '0' && *p <= '9') {
        if (v > (1ull << 62)) return nullptr;
        v = v * 10 + (unsigned)(*p++ - '0');
    }
    if (v > (1ull << 62)) return nullptr;
    *out = neg ? -(long long)v : (long long)v;
    return p;
}

inline bool is_blank(char c) { return c == ' ' || c == '\t' || c == '\r'; }

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
        const char *e = parse_long(p, v);
        if (!e || e > end) return false;
        p = e;
        return true;
    }
    bool read_double(double *v)
    {
        skip_ws();
        if (p >= end) return false;
        const char *e = parse_double(p, v);
        if (!e || e > end) return false;
        p = e;
        return true;
    }
};

enum ValType { REAL, CPLX, INTG, PATT };

// One entry from cur; false if malformed or out of range.
inline bool parse_entry(Cursor &cur, ValType ty, long long m, long long n, int *r, int *c, double *v)
{
    long long i, j;
    double re = 1.0, im;
    if (!cur.read_long(&i) || !cur.read_long(&j)) return false;
    if (ty == REAL || ty == CPLX) {
        if (!cur.read_double(&re)) return false;
        if (ty == CPLX && !cur.read_double(&im)) return false;
    } else if (ty == INTG) {
        long long iv;
        if (!cur.read_long(&iv)) return false;
        re = (double)iv;
    }
    if (i < 1 || i > m || j < 1 || j > n) return false;
    *r = (int)(i - 1);
    *c = (int)(j - 1);
    *v = re;
    return true;
}

// Sequential reader: exactly nz entries, whitespace (newlines included)
// between tokens, as fscanf reads them; anything after them is ignored.
bool parse_sequential(Cursor cur, ValType ty, long long m, long long n, long long nz, int *ri, int *ci, double *vv)
{
    for (long long k = 0; k < nz; ++k)
        if (!parse_entry(cur, ty, m, n, ri + k, ci + k, vv + k)) return false;
    return true;
}

// Parallel reader for files with one entry per line: the data section
// [p, end) is cut into chunks after a newline; pass 1 counts the non-blank
// lines of each chunk, pass 2 parses each chunk straight into its slice of
// the output.  Returns false (and the sequential reader decides) unless there
// are exactly nz non-blank lines, each holding exactly one entry.
bool parse_parallel(const char *p, const char *end, ValType ty, long long m, long long n, long long nz, int *ri,
                    int *ci, double *vv)
{
    const size_t bytes = (size_t)(end - p);
    const size_t nchunk = bytes < ((size_t)1 << 20) ? 1 : (size_t)omp_get_max_threads() * 8;
    std::vector<const char *> cut(nchunk + 1);
    cut[0] = p;
    cut[nchunk] = end;
    for (size_t c = 1; c < nchunk; ++c) {
        const char *q = p + bytes / nchunk * c;
        if (q < cut[c - 1]) q = cut[c - 1];
        const char *nl = q < end ? (const char *)memchr(q, '\n', (size_t)(end - q)) : nullptr;
        cut[c] = nl ? nl + 1 : end;
    }
    std::vector<long long> lines(nchunk + 1, 0);
#pragma omp parallel for schedule(dynamic, 1)
    for (long long c = 0; c < (long long)nchunk; ++c) {
        long long k = 0;
        for (const char *q = cut[(size_t)c]; q < cut[(size_t)c + 1];) {
            const char *nl = (const char *)memchr(q, '\n', (size_t)(cut[(size_t)c + 1] - q));
            const char *le = nl ? nl : cut[(size_t)c + 1];
            const char *t = q;
            while (t < le && is_blank(*t)) ++t;
            if (t < le) ++k;
            q = nl ? nl + 1 : le;
        }
        lines[(size_t)c + 1] = k;
    }
    for (size_t c = 0; c < nchunk; ++c) lines[c + 1] += lines[c];
    if (lines[nchunk] != nz) return false;
    int ok = 1;
#pragma omp parallel for schedule(dynamic, 1) reduction(& : ok)
    for (long long c = 0; c < (long long)nchunk; ++c) {
        long long k = lines[(size_t)c];
        const char *ce = cut[(size_t)c + 1];
        for (const char *q = cut[(size_t)c]; q < ce && ok;) {
            const char *nl = (const char *)memchr(q, '\n', (size_t)(ce - q));
            const char *le = nl ? nl : ce;
            const char *t = q;
            while (t < le && is_blank(*t)) ++t;
            if (t < le) {
                Cursor cur{t, le};
                if (!parse_entry(cur, ty, m, n, ri + k, ci + k, vv + k)) ok = 0;
                while (cur.p < le && is_blank(*cur.p)) ++cur.p;
                if (cur.p != le) ok = 0;         // more than one entry on the line
                ++k;
            }
            q = nl ? nl + 1 : le;
        }
    }
    return ok != 0;
}

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
    std::unique_ptr<char, void (*)(void *)> buf((char *)malloc((size_t)fsize + 1), free);
    if (!buf) { fclose(f); return TSP_ENOMEM; }
    if (fread(buf.get(), 1, (size_t)fsize, f) != (size_t)fsize) { fclose(f); return TSP_EIO; }
    fclose(f);
    buf.get()[(size_t)fsize] = '\0';      // token parsers stop at the terminator
    const char *p = buf.get(), *end = buf.get() + fsize;

    // Banner: %%MatrixMarket matrix coordinate <type> <symmetry>
    const char *nl = (const char *)memchr(p, '\n', (size_t)(end - p));
    if (!nl) return TSP_EIO;
    char banner[64], mtx[64], crd[64], dtype[64], storage[64];
    std::string first(p, nl);
    if (sscanf(first.c_str(), "%63s %63s %63s %63s %63s", banner, mtx, crd, dtype, storage) != 5)
        return TSP_EIO;
    if (strncmp(banner, "%%MatrixMarket", 14) != 0) return TSP_EIO;
    if (strcasecmp(mtx, "matrix") != 0 || strcasecmp(crd, "coordinate") != 0) return TSP_EIO;
    ValType ty;
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

    std::unique_ptr<int, void (*)(void *)> ri_((int *)malloc(sizeof(int) * (size_t)(nz ? nz : 1)), free);
    std::unique_ptr<int, void (*)(void *)> ci_((int *)malloc(sizeof(int) * (size_t)(nz ? nz : 1)), free);
    std::unique_ptr<double, void (*)(void *)> vv_((double *)malloc(sizeof(double) * (size_t)(nz ? nz : 1)), free);
    if (!ri_ || !ci_ || !vv_) return TSP_ENOMEM;
    int *ri = ri_.get(), *ci = ci_.get();
    double *vv = vv_.get();
    // the entries start on the line after the size line (which may end with
    // blanks); anything else on that line goes to the sequential reader
    const char *q = cur.p;
    while (q < end && is_blank(*q)) ++q;
    const bool line_start = q >= end || *q == '\n';
    if (!line_start || !parse_parallel(q, end, ty, m, n, nz, ri, ci, vv))
        if (!parse_sequential(cur, ty, m, n, nz, ri, ci, vv)) return TSP_EIO;
    std::vector<long long> cnt((size_t)m + 1, 0);
    for (long long k = 0; k < nz; ++k) cnt[(size_t)ri[k]]++;
    if (sym)
        for (long long k = 0; k < nz; ++k)
            if (ri[k] != ci[k]) cnt[(size_t)ci[k]]++;
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
        const int a = ri[k], b = ci[k];
        long long o = cnt[(size_t)a] + fill[(size_t)a]++;
        col[o] = b;
        val[o] = vv[k];
        if (sym && a != b) {
            o = cnt[(size_t)b] + fill[(size_t)b]++;
            col[o] = a;
            val[o] = vv[k];
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

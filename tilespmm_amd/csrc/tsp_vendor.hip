// tsp_vendor.hip -- vendor SpMM baseline on rocSPARSE, the counterpart of the
// reference's cusparse_spmm_all (src/main.cu:16-134): CSR A (fp16 or fp32
// values, 32-bit indices), row-major B with leading dimension ldb, row-major
// fp32 C [m][n], fp32 compute, default algorithm; pre-time covers handle,
// descriptors and buffer query/allocation (host wall clock, H2D copies
// excluded), then `warmup` untimed and `repeat` timed calls bracketed by
// events.  C is copied back after timing (beta = 0, so it holds one product).
#include <hip/hip_runtime.h>
#include <rocsparse/rocsparse.h>
#include <sys/time.h>

#include "../../include/tilespmm_hip.h"

namespace {
double wall_ms()
{
    struct timeval t;
    gettimeofday(&t, nullptr);
    return t.tv_sec * 1000.0 + t.tv_usec / 1000.0;
}
}  // namespace

extern "C" int tsp_vendor_spmm(int prec, int m, int k, long long nnz, const int *rowptr,
                               const int *colidx, const void *val, int n, int ldb, const void *h_B,
                               float *h_C, int warmup, int repeat, double *pre_ms, double *ms)
{
    if (m < 0 || k < 0 || n <= 0 || ldb < n || nnz < 0 || !rowptr || repeat <= 0) return TSP_EINVAL;
    const size_t vs = prec == TSP_PREC_FP16 ? 2 : 4;
    const rocsparse_datatype vt = prec == TSP_PREC_FP16 ? rocsparse_datatype_f16_r : rocsparse_datatype_f32_r;
    int *d_ptr = nullptr, *d_idx = nullptr;
    void *d_val = nullptr, *d_B = nullptr, *d_buf = nullptr;
    float *d_C = nullptr;
    hipError_t he = hipSuccess;
    int status = TSP_OK;
    rocsparse_handle h = nullptr;
    rocsparse_spmat_descr A = nullptr;
    rocsparse_dnmat_descr Bd = nullptr, Cd = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    size_t bufsz = 0;
    const float alpha = 1.0f, beta = 0.0f;
    double t0, t1;
    float tms = 0.f;
#define HCHK(x) do { he = (x); if (he != hipSuccess) { status = (int)he; goto done; } } while (0)
#define SCHK(x) do { if ((x) != rocsparse_status_success) { status = TSP_EINVAL; goto done; } } while (0)
    HCHK(hipMalloc(&d_ptr, sizeof(int) * ((size_t)m + 1)));
    HCHK(hipMalloc(&d_idx, sizeof(int) * (size_t)(nnz ? nnz : 1)));
    HCHK(hipMalloc(&d_val, vs * (size_t)(nnz ? nnz : 1)));
    HCHK(hipMalloc(&d_B, vs * (size_t)k * ldb + 16));
    HCHK(hipMalloc(&d_C, sizeof(float) * (size_t)m * n + 16));
    HCHK(hipMemcpy(d_ptr, rowptr, sizeof(int) * ((size_t)m + 1), hipMemcpyHostToDevice));
    if (nnz) {
        HCHK(hipMemcpy(d_idx, colidx, sizeof(int) * (size_t)nnz, hipMemcpyHostToDevice));
        HCHK(hipMemcpy(d_val, val, vs * (size_t)nnz, hipMemcpyHostToDevice));
    }
    HCHK(hipMemcpy(d_B, h_B, vs * (size_t)k * ldb, hipMemcpyHostToDevice));
    HCHK(hipMemset(d_C, 0, sizeof(float) * (size_t)m * n));
    t0 = wall_ms();
    SCHK(rocsparse_create_handle(&h));
    SCHK(rocsparse_create_csr_descr(&A, m, k, nnz, d_ptr, d_idx, d_val, rocsparse_indextype_i32,
                                    rocsparse_indextype_i32, rocsparse_index_base_zero, vt));
    SCHK(rocsparse_create_dnmat_descr(&Bd, k, n, ldb, d_B, vt, rocsparse_order_row));
    SCHK(rocsparse_create_dnmat_descr(&Cd, m, n, n, d_C, rocsparse_datatype_f32_r, rocsparse_order_row));
    SCHK(rocsparse_spmm(h, rocsparse_operation_none, rocsparse_operation_none, &alpha, A, Bd, &beta, Cd,
                        rocsparse_datatype_f32_r, rocsparse_spmm_alg_default,
                        rocsparse_spmm_stage_buffer_size, &bufsz, nullptr));
    HCHK(hipMalloc(&d_buf, bufsz ? bufsz : 16));
    SCHK(rocsparse_spmm(h, rocsparse_operation_none, rocsparse_operation_none, &alpha, A, Bd, &beta, Cd,
                        rocsparse_datatype_f32_r, rocsparse_spmm_alg_default,
                        rocsparse_spmm_stage_preprocess, &bufsz, d_buf));
    HCHK(hipDeviceSynchronize());
    t1 = wall_ms();
    if (pre_ms) *pre_ms = t1 - t0;
    for (int i = 0; i < warmup; ++i)
        SCHK(rocsparse_spmm(h, rocsparse_operation_none, rocsparse_operation_none, &alpha, A, Bd, &beta,
                            Cd, rocsparse_datatype_f32_r, rocsparse_spmm_alg_default,
                            rocsparse_spmm_stage_compute, &bufsz, d_buf));
    HCHK(hipDeviceSynchronize());
    HCHK(hipEventCreate(&e0));
    HCHK(hipEventCreate(&e1));
    HCHK(hipEventRecord(e0, nullptr));
    for (int i = 0; i < repeat; ++i)
        SCHK(rocsparse_spmm(h, rocsparse_operation_none, rocsparse_operation_none, &alpha, A, Bd, &beta,
                            Cd, rocsparse_datatype_f32_r, rocsparse_spmm_alg_default,
                            rocsparse_spmm_stage_compute, &bufsz, d_buf));
    HCHK(hipEventRecord(e1, nullptr));
    HCHK(hipEventSynchronize(e1));
    HCHK(hipEventElapsedTime(&tms, e0, e1));
    if (ms) *ms = (double)tms / repeat;
    if (h_C) HCHK(hipMemcpy(h_C, d_C, sizeof(float) * (size_t)m * n, hipMemcpyDeviceToHost));
done:
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (A) (void)rocsparse_destroy_spmat_descr(A);
    if (Bd) (void)rocsparse_destroy_dnmat_descr(Bd);
    if (Cd) (void)rocsparse_destroy_dnmat_descr(Cd);
    if (h) (void)rocsparse_destroy_handle(h);
    (void)hipFree(d_ptr);
    (void)hipFree(d_idx);
    (void)hipFree(d_val);
    (void)hipFree(d_B);
    (void)hipFree(d_C);
    (void)hipFree(d_buf);
#undef HCHK
#undef SCHK
    return status;
}

// tsp_capi.hip -- the extern "C" boundary of libtilespmm_hip.so.
//
// Thin wrappers over the HIP runtime plus the kernel dispatch.  Every entry
// point returns an int status; none of them exits the process.  Argument
// checks happen here, on the host, before anything is launched: a launch whose
// shapes do not match what the kernels assume is refused with TSP_EINVAL.
#include <amd_smi/amdsmi.h>
#include <dlfcn.h>
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <string.h>

#include <mutex>

#include "../../include/tilespmm_hip.h"
#include "tsp_kernels.h"

#ifndef TSP_VERSION
#define TSP_VERSION "0.1.0"
#endif

extern "C" {

const char *tsp_hip_version(void) { return "tilespmm_hip " TSP_VERSION " gfx950"; }

const char *tsp_hip_error_string(int status)
{
    switch (status) {
    case TSP_OK: return "success";
    case TSP_EINVAL: return "invalid argument (class, width or pointer)";
    case TSP_ENODEV: return "no usable gfx950 device";
    default: return hipGetErrorString((hipError_t)status);
    }
}

int tsp_device_init(int device_id)
{
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess) return (int)e;
    if (device_id < 0 || device_id >= n) return TSP_ENODEV;
    e = hipSetDevice(device_id);
    if (e != hipSuccess) return (int)e;
    hipDeviceProp_t p;
    e = hipGetDeviceProperties(&p, device_id);
    if (e != hipSuccess) return (int)e;
    if (strncmp(p.gcnArchName, "gfx950", 6) != 0) return TSP_ENODEV;
    // per-device address of the allocation-free entry points' scratch
    return tsp::scratch_init_current_device(nullptr);
}

int tsp_device_probe(int device_id, tsp_device_info *out)
{
    if (!out) return TSP_EINVAL;
    hipDeviceProp_t p;
    hipError_t e = hipGetDeviceProperties(&p, device_id);
    if (e != hipSuccess) return (int)e;
    memset(out, 0, sizeof *out);
    out->cu_count = p.multiProcessorCount;
    out->max_threads_per_cu = p.maxThreadsPerMultiProcessor;
    out->regs_per_cu = p.regsPerMultiprocessor;
    out->max_blocks_per_cu = p.maxBlocksPerMultiProcessor;
    out->lds_bytes_per_cu = (long long)p.maxSharedMemoryPerMultiProcessor;
    out->l2_bytes = (long long)p.l2CacheSize;
    out->wavefront_size = p.warpSize;
    out->clock_khz = p.clockRate;
    out->memory_clock_khz = p.memoryClockRate;
    out->memory_bus_width = p.memoryBusWidth;
    strncpy(out->name, p.name, sizeof out->name - 1);
    strncpy(out->gcn_arch, p.gcnArchName, sizeof out->gcn_arch - 1);
    return TSP_OK;
}

int tsp_kernel_probe(int bm, int prec, int colB_p, tsp_kernel_info *out)
{
    if (!out || (bm != 64 && bm != 16 && bm != 8) || (prec != 0 && prec != 1)) return TSP_EINVAL;
    if (colB_p != 32 && (colB_p <= 0 || colB_p % 64)) return TSP_EINVAL;
    const int w = tsp::default_chunk_width(bm, colB_p);
    const void *k = tsp::select_kernel(bm, prec, w, tsp::default_stages(bm, prec, w), false);
    if (!k) return TSP_EINVAL;
    hipFuncAttributes a;
    hipError_t e = hipFuncGetAttributes(&a, k);
    if (e != hipSuccess) return (int)e;
    const int bn = tsp::tile_bn(bm, prec);
    out->threads = tsp::kBlockThreads;
    out->tasks_per_block = tsp::kWavesPerBlock;
    out->registers_per_thread = a.numRegs;
    out->shared_bytes = (long long)a.sharedSizeBytes;
    out->cols_per_task = w;
    out->iteration_bytes = tsp::kWavesPerBlock * (bm * bn + bn * w) * (prec == TSP_PREC_FP16 ? 2 : 4);
    return TSP_OK;
}

// GFX clock through AMD SMI, loaded at run time (as the reference loads NVML
// for its warm-up, src/common.h:96-119) so the library does not depend on it.
// The device is matched to its SMI handle by PCI bus id.
namespace {
struct Smi {
    std::mutex mu;
    bool tried = false;
    decltype(&amdsmi_get_processor_handle_from_bdf) from_bdf = nullptr;
    decltype(&amdsmi_get_clock_info) clock_info = nullptr;
    static constexpr int kMaxDev = 64;
    amdsmi_processor_handle handle[kMaxDev] = {};
    bool looked[kMaxDev] = {};
};
Smi g_smi;
}  // namespace

int tsp_gpu_clock_mhz(int device_id, unsigned *mhz, unsigned *max_mhz)
{
    if (!mhz) return TSP_EINVAL;
    *mhz = 0;
    if (max_mhz) *max_mhz = 0;
    if (device_id < 0 || device_id >= Smi::kMaxDev) return TSP_EINVAL;
    std::lock_guard<std::mutex> lk(g_smi.mu);
    if (!g_smi.tried) {
        g_smi.tried = true;
        void *lib = dlopen("libamd_smi.so", RTLD_LAZY | RTLD_LOCAL);
        if (!lib) lib = dlopen("/opt/rocm/lib/libamd_smi.so", RTLD_LAZY | RTLD_LOCAL);
        auto init = lib ? (decltype(&amdsmi_init))dlsym(lib, "amdsmi_init") : nullptr;
        g_smi.from_bdf = lib ? (decltype(g_smi.from_bdf))dlsym(lib, "amdsmi_get_processor_handle_from_bdf") : nullptr;
        g_smi.clock_info = lib ? (decltype(g_smi.clock_info))dlsym(lib, "amdsmi_get_clock_info") : nullptr;
        if (!init || !g_smi.from_bdf || !g_smi.clock_info || init(AMDSMI_INIT_AMD_GPUS) != AMDSMI_STATUS_SUCCESS)
            g_smi.clock_info = nullptr;
    }
    if (!g_smi.clock_info) return TSP_OK;
    if (!g_smi.looked[device_id]) {
        g_smi.looked[device_id] = true;
        char pci[64] = {0};
        unsigned dom = 0, bus = 0, dv = 0, fn = 0;
        if (hipDeviceGetPCIBusId(pci, sizeof pci, device_id) == hipSuccess &&
            sscanf(pci, "%x:%x:%x.%x", &dom, &bus, &dv, &fn) == 4) {
            amdsmi_bdf_t bdf;
            bdf.as_uint = 0;
            bdf.domain_number = dom;
            bdf.bus_number = bus;
            bdf.device_number = dv;
            bdf.function_number = fn;
            amdsmi_processor_handle h = nullptr;
            if (g_smi.from_bdf(bdf, &h) == AMDSMI_STATUS_SUCCESS) g_smi.handle[device_id] = h;
        }
    }
    if (!g_smi.handle[device_id]) return TSP_OK;
    amdsmi_clk_info_t info;
    memset(&info, 0, sizeof info);
    if (g_smi.clock_info(g_smi.handle[device_id], AMDSMI_CLK_TYPE_GFX, &info) != AMDSMI_STATUS_SUCCESS) return TSP_OK;
    *mhz = info.clk;
    if (max_mhz) *max_mhz = info.max_clk;
    return TSP_OK;
}

int tsp_malloc(void **ptr, size_t bytes)
{
    if (!ptr) return TSP_EINVAL;
    *ptr = nullptr;
    if (bytes == 0) return TSP_OK;
    const hipError_t e = hipMalloc(ptr, bytes);
    // a failed allocation must not surface later as the error of an
    // unrelated launch (launches report hipGetLastError)
    if (e != hipSuccess) (void)hipGetLastError();
    return (int)e;
}
int tsp_free(void *ptr) { return ptr ? (int)hipFree(ptr) : TSP_OK; }
int tsp_memcpy_h2d(void *dst, const void *src, size_t bytes)
{
    return bytes ? (int)hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice) : TSP_OK;
}
int tsp_memcpy_d2h(void *dst, const void *src, size_t bytes)
{
    return bytes ? (int)hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost) : TSP_OK;
}
int tsp_memcpy_h2d_async(void *dst, const void *src, size_t bytes, void *stream)
{
    return bytes ? (int)hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, (hipStream_t)stream)
                 : TSP_OK;
}
int tsp_memset(void *dst, int value, size_t bytes)
{
    return bytes ? (int)hipMemset(dst, value, bytes) : TSP_OK;
}
int tsp_memset_async(void *dst, int value, size_t bytes, void *stream)
{
    return bytes ? (int)hipMemsetAsync(dst, value, bytes, (hipStream_t)stream) : TSP_OK;
}

int tsp_stream_create(void **stream)
{
    if (!stream) return TSP_EINVAL;
    hipStream_t s = nullptr;
    hipError_t e = hipStreamCreate(&s);
    *stream = (void *)s;
    return (int)e;
}
int tsp_stream_destroy(void *stream) { return stream ? (int)hipStreamDestroy((hipStream_t)stream) : TSP_OK; }
int tsp_stream_sync(void *stream) { return (int)hipStreamSynchronize((hipStream_t)stream); }
int tsp_device_sync(void) { return (int)hipDeviceSynchronize(); }
int tsp_event_create(void **event)
{
    if (!event) return TSP_EINVAL;
    hipEvent_t ev = nullptr;
    hipError_t e = hipEventCreate(&ev);
    *event = (void *)ev;
    return (int)e;
}
int tsp_event_destroy(void *event) { return event ? (int)hipEventDestroy((hipEvent_t)event) : TSP_OK; }
int tsp_event_record(void *event, void *stream)
{
    return (int)hipEventRecord((hipEvent_t)event, (hipStream_t)stream);
}
int tsp_event_sync(void *event) { return (int)hipEventSynchronize((hipEvent_t)event); }
int tsp_stream_create_nonblocking(void **stream)
{
    if (!stream) return TSP_EINVAL;
    hipStream_t s = nullptr;
    hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
    *stream = (void *)s;
    return (int)e;
}
int tsp_stream_wait_event(void *stream, void *event)
{
    return (int)hipStreamWaitEvent((hipStream_t)stream, (hipEvent_t)event, 0);
}
int tsp_event_elapsed_ms(float *ms, void *start, void *stop)
{
    if (!ms) return TSP_EINVAL;
    return (int)hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop);
}
int tsp_stream_begin_capture(void *stream)
{
    if (!stream) return TSP_EINVAL;       // the null stream cannot be captured
    return (int)hipStreamBeginCapture((hipStream_t)stream, hipStreamCaptureModeThreadLocal);
}
int tsp_stream_end_capture(void *stream, void **graph_exec)
{
    if (!stream) return TSP_EINVAL;
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture((hipStream_t)stream, &g);
    if (graph_exec) *graph_exec = nullptr;
    if (e == hipSuccess && graph_exec) {
        hipGraphExec_t x = nullptr;
        e = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
        if (e == hipSuccess) *graph_exec = (void *)x;
    }
    if (g) (void)hipGraphDestroy(g);
    return (int)e;
}
int tsp_graph_launch(void *graph_exec, void *stream)
{
    if (!graph_exec) return TSP_EINVAL;
    return (int)hipGraphLaunch((hipGraphExec_t)graph_exec, (hipStream_t)stream);
}
int tsp_graph_destroy(void *graph_exec)
{
    return graph_exec ? (int)hipGraphExecDestroy((hipGraphExec_t)graph_exec) : TSP_OK;
}

int tsp_spmm_launch(int bm, int prec, int rowblkblock, int colB_p, const void *d_val,
                    const unsigned *d_rows, const int *d_colstart, const void *d_B, float *d_C,
                    const int *d_colidx, int c_rows, void *stream)
{
    if (bm != 64 && bm != 16 && bm != 8) return TSP_EINVAL;
    if (prec != TSP_PREC_FP16 && prec != TSP_PREC_TF32) return TSP_EINVAL;
    if (colB_p != 32 && (colB_p <= 0 || colB_p % 64 != 0)) return TSP_EINVAL;
    if (rowblkblock < 0 || c_rows < 0) return TSP_EINVAL;
    if (rowblkblock == 0) return TSP_OK;
    if (!d_val || !d_rows || !d_colstart || !d_B || !d_C || !d_colidx) return TSP_EINVAL;
    return tsp::launch(bm, prec, rowblkblock, colB_p, d_val, nullptr, nullptr, d_rows, d_colstart,
                       d_B, d_C, d_colidx, c_rows, (hipStream_t)stream, 0, 0, 0, 0);
}

int tsp_spmm_launch_packed(int bm, int prec, int rowblkblock, int colB_p, const void *d_pval,
                           const uint64_t *d_bitmap, const int *d_vptr, const unsigned *d_rows,
                           const int *d_colstart, const void *d_B, float *d_C, const int *d_colidx,
                           int c_rows, void *stream, int w, int stages, int tasks_per_wave, int order)
{
    if (bm != 16 && bm != 8) return TSP_EINVAL;
    if (prec != TSP_PREC_FP16 && prec != TSP_PREC_TF32) return TSP_EINVAL;
    if (colB_p != 32 && (colB_p <= 0 || colB_p % 64 != 0)) return TSP_EINVAL;
    if (rowblkblock < 0 || c_rows < 0) return TSP_EINVAL;
    if (w > 0 && (colB_p % w != 0 || !tsp::valid_variant(bm, w, stages > 0 ? stages : 1))) return TSP_EINVAL;
    if (rowblkblock == 0) return TSP_OK;
    if (!d_pval || !d_bitmap || !d_vptr || !d_rows || !d_colstart || !d_B || !d_C || !d_colidx)
        return TSP_EINVAL;
    return tsp::launch(bm, prec, rowblkblock, colB_p, d_pval, d_bitmap, d_vptr, d_rows, d_colstart,
                       d_B, d_C, d_colidx, c_rows, (hipStream_t)stream, w, stages, tasks_per_wave,
                       order);
}

int tsp_spmm_launch_placed(int bm, int prec, int rowblkblock, int colB_p, const void *d_val,
                           const uint64_t *d_bitmap, const int *d_vptr, const unsigned *d_rows,
                           const int *d_colstart, const void *d_B, float *d_C, const int *d_colidx,
                           int c_rows, void *stream, int w, int stages, int tasks_per_wave, int order,
                           int placement)
{
    return tsp_spmm_launch_ex(bm, prec, rowblkblock, colB_p, d_val, d_bitmap, d_vptr, d_rows, d_colstart, d_B, d_C,
                              d_colidx, c_rows, stream, w, stages, tasks_per_wave, order, placement, 0);
}

int tsp_pairs_supported(int bm, int prec, int w)
{
    if (prec == TSP_PREC_TF32) return bm == 8 && w == 64;
    return prec == TSP_PREC_FP16 && (bm == 8 || bm == 16) && (w == 64 || w == 128);
}

int tsp_spmm_launch_ex(int bm, int prec, int rowblkblock, int colB_p, const void *d_val,
                       const uint64_t *d_bitmap, const int *d_vptr, const unsigned *d_rows,
                       const int *d_colstart, const void *d_B, float *d_C, const int *d_colidx,
                       int c_rows, void *stream, int w, int stages, int tasks_per_wave, int order,
                       int placement, int flags)
{
    if (flags & ~(TSP_LAUNCH_OPERANDS_TF32 | TSP_LAUNCH_LANE_INDICES | TSP_LAUNCH_TILE_PAIRS |
                  TSP_LAUNCH_SKIP_ZERO_STORES | TSP_LAUNCH_B_3BYTE))
        return TSP_EINVAL;
    if ((flags & TSP_LAUNCH_TILE_PAIRS) &&
        (!tsp_pairs_supported(bm, prec, w > 0 ? w : tsp::default_chunk_width(bm, colB_p)) ||
         (prec == TSP_PREC_TF32 && !(flags & TSP_LAUNCH_OPERANDS_TF32))))
        return TSP_EINVAL;
    // 3-byte B: tf32 values only, single tiles (and no panel sweep: the
    // panel launch does not accept the flag)
    if ((flags & TSP_LAUNCH_B_3BYTE) && (prec != TSP_PREC_TF32 || !(flags & TSP_LAUNCH_OPERANDS_TF32) ||
                                         (flags & TSP_LAUNCH_TILE_PAIRS)))
        return TSP_EINVAL;
    if (bm != 64 && bm != 16 && bm != 8) return TSP_EINVAL;
    if (prec != TSP_PREC_FP16 && prec != TSP_PREC_TF32) return TSP_EINVAL;
    if (colB_p != 32 && (colB_p <= 0 || colB_p % 64 != 0)) return TSP_EINVAL;
    if (rowblkblock < 0 || c_rows < 0) return TSP_EINVAL;
    if (d_bitmap && (bm == 64 || !d_vptr)) return TSP_EINVAL;
    if (placement != TSP_PLACE_CONTIGUOUS && placement != TSP_PLACE_INTERLEAVED && placement != TSP_PLACE_CHUNK_XCD)
        return TSP_EINVAL;
    if (w > 0 && (colB_p % w != 0 || !tsp::valid_variant(bm, w, stages > 0 ? stages : 1))) return TSP_EINVAL;
    if (rowblkblock == 0) return TSP_OK;
    if (!d_val || !d_rows || !d_colstart || !d_B || !d_C || !d_colidx) return TSP_EINVAL;
    const int kprec = (flags & TSP_LAUNCH_B_3BYTE)                                   ? tsp::kPrecTf32B3
                      : prec == TSP_PREC_TF32 && (flags & TSP_LAUNCH_OPERANDS_TF32) ? tsp::kPrecTf32Exact
                                                                                    : prec;
    return tsp::launch(bm, kprec, rowblkblock, colB_p, d_val, d_bitmap, d_vptr, d_rows, d_colstart, d_B,
                       d_C, d_colidx, c_rows, (hipStream_t)stream, w, stages, tasks_per_wave, order,
                       placement, (flags & TSP_LAUNCH_LANE_INDICES) != 0, 0, 0, 1, nullptr, 0, false,
                       (flags & TSP_LAUNCH_TILE_PAIRS) != 0,
                       (flags & TSP_LAUNCH_SKIP_ZERO_STORES) ? tsp::kOptSkipZeroStores : 0);
}

int tsp_spmm_launch_panels(int bm, int prec, int rowblkblock, int colB_p, const void *d_val,
                           const uint64_t *d_bitmap, const int *d_vptr, const unsigned *d_rows,
                           const int *d_colstart, const void *d_B, float *d_C, const int *d_colidx,
                           int c_rows, void *stream, int w, int stages, int tasks_per_wave, int order,
                           int placement, int flags, int b_rows, int panel_rows, int panel_lag, int *d_sync,
                           long long sync_ints)
{
    if (flags & ~(TSP_LAUNCH_OPERANDS_TF32 | TSP_LAUNCH_LANE_INDICES | TSP_LAUNCH_SYNC_RESET | TSP_LAUNCH_TILE_PAIRS |
                  TSP_LAUNCH_SKIP_ZERO_STORES))
        return TSP_EINVAL;
    if ((flags & TSP_LAUNCH_TILE_PAIRS) &&
        (!tsp_pairs_supported(bm, prec, w > 0 ? w : tsp::default_chunk_width(bm, colB_p)) ||
         (prec == TSP_PREC_TF32 && !(flags & TSP_LAUNCH_OPERANDS_TF32))))
        return TSP_EINVAL;
    if (bm != 64 && bm != 16 && bm != 8) return TSP_EINVAL;
    if (prec != TSP_PREC_FP16 && prec != TSP_PREC_TF32) return TSP_EINVAL;
    if (colB_p != 32 && (colB_p <= 0 || colB_p % 64 != 0)) return TSP_EINVAL;
    if (rowblkblock < 0 || c_rows < 0 || b_rows <= 0 || sync_ints <= 0) return TSP_EINVAL;
    if (d_bitmap && (bm == 64 || !d_vptr)) return TSP_EINVAL;
    if (placement != TSP_PLACE_CONTIGUOUS && placement != TSP_PLACE_INTERLEAVED) return TSP_EINVAL;
    if (panel_rows < 64 || (panel_rows & (panel_rows - 1)) || panel_lag < 1) return TSP_EINVAL;
    if (w > 0 && (colB_p % w != 0 || !tsp::valid_variant(bm, w, stages > 0 ? stages : 1))) return TSP_EINVAL;
    if (rowblkblock == 0) return TSP_OK;
    if (!d_val || !d_rows || !d_colstart || !d_B || !d_C || !d_colidx || !d_sync) return TSP_EINVAL;
    const int kprec = prec == TSP_PREC_TF32 && (flags & TSP_LAUNCH_OPERANDS_TF32) ? tsp::kPrecTf32Exact : prec;
    return tsp::launch(bm, kprec, rowblkblock, colB_p, d_val, d_bitmap, d_vptr, d_rows, d_colstart, d_B,
                       d_C, d_colidx, c_rows, (hipStream_t)stream, w, stages, tasks_per_wave, order,
                       placement, (flags & TSP_LAUNCH_LANE_INDICES) != 0, b_rows, panel_rows, panel_lag, d_sync,
                       sync_ints, (flags & TSP_LAUNCH_SYNC_RESET) != 0, (flags & TSP_LAUNCH_TILE_PAIRS) != 0,
                       (flags & TSP_LAUNCH_SKIP_ZERO_STORES) ? tsp::kOptSkipZeroStores : 0);
}

int tsp_spmm_launch_variant(int bm, int prec, int rowblkblock, int colB_p, const void *d_val,
                            const unsigned *d_rows, const int *d_colstart, const void *d_B,
                            float *d_C, const int *d_colidx, int c_rows, void *stream, int w,
                            int stages, int tasks_per_wave, int order)
{
    if (bm != 64 && bm != 16 && bm != 8) return TSP_EINVAL;
    if (prec != TSP_PREC_FP16 && prec != TSP_PREC_TF32) return TSP_EINVAL;
    if (colB_p != 32 && (colB_p <= 0 || colB_p % 64 != 0)) return TSP_EINVAL;
    if (rowblkblock < 0 || c_rows < 0) return TSP_EINVAL;
    if (w > 0 && (colB_p % w != 0 || !tsp::valid_variant(bm, w, stages > 0 ? stages : 1))) return TSP_EINVAL;
    if (rowblkblock == 0) return TSP_OK;
    if (!d_val || !d_rows || !d_colstart || !d_B || !d_C || !d_colidx) return TSP_EINVAL;
    return tsp::launch(bm, prec, rowblkblock, colB_p, d_val, nullptr, nullptr, d_rows, d_colstart,
                       d_B, d_C, d_colidx, c_rows, (hipStream_t)stream, w, stages, tasks_per_wave,
                       order);
}

int tsp_switch_v64(int prec, int rowblkblock, int colB_p, const void *d_val, const unsigned *d_rows,
                   const int *d_colstart, const void *d_B, float *d_C, const int *d_colidx,
                   int c_rows, void *stream)
{
    return tsp_spmm_launch(64, prec, rowblkblock, colB_p, d_val, d_rows, d_colstart, d_B, d_C,
                           d_colidx, c_rows, stream);
}
int tsp_switch_v16(int prec, int rowblkblock, int colB_p, const void *d_val, const unsigned *d_rows,
                   const int *d_colstart, const void *d_B, float *d_C, const int *d_colidx,
                   int c_rows, void *stream)
{
    return tsp_spmm_launch(16, prec, rowblkblock, colB_p, d_val, d_rows, d_colstart, d_B, d_C,
                           d_colidx, c_rows, stream);
}
int tsp_switch_v8(int prec, int rowblkblock, int colB_p, const void *d_val, const unsigned *d_rows,
                  const int *d_colstart, const void *d_B, float *d_C, const int *d_colidx,
                  int c_rows, void *stream)
{
    return tsp_spmm_launch(8, prec, rowblkblock, colB_p, d_val, d_rows, d_colstart, d_B, d_C,
                           d_colidx, c_rows, stream);
}

namespace tsp {
__global__ __launch_bounds__(256) void round_tf32_kernel(uint32_t *__restrict__ x, size_t n)
{
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) x[i] = round_tf32_bits(x[i]);
}
// 4 values (16 bytes in) -> 12 bytes out per thread
__global__ __launch_bounds__(256) void pack_3byte_kernel(const uint32_t *__restrict__ x, uint32_t *__restrict__ y,
                                                         size_t groups)
{
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < groups; i += stride) {
        const uint32_t a = pack_3byte_bits(x[4 * i]), b = pack_3byte_bits(x[4 * i + 1]),
                       c = pack_3byte_bits(x[4 * i + 2]), d = pack_3byte_bits(x[4 * i + 3]);
        y[3 * i] = a | b << 24;
        y[3 * i + 1] = b >> 8 | c << 16;
        y[3 * i + 2] = c >> 16 | d << 8;
    }
}
__global__ __launch_bounds__(256) void split_bf16_kernel(const uint32_t *__restrict__ x, uint32_t *__restrict__ y,
                                                        size_t n)
{
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) y[i] = split_bf16_bits(x[i]);
}
}  // namespace tsp

int tsp_split_bf16_device(const void *d_src, void *d_dst, size_t n, void *stream)
{
    if (n && (!d_src || !d_dst)) return TSP_EINVAL;
    if (n == 0) return TSP_OK;
    const size_t b = (n + 255) / 256;
    tsp::split_bf16_kernel<<<(unsigned)(b < 16384 ? b : 16384), 256, 0, (hipStream_t)stream>>>(
        (const uint32_t *)d_src, (uint32_t *)d_dst, n);
    return (int)hipGetLastError();
}

int tsp_split_bf16_bits(const uint32_t *in, uint32_t *out, size_t n)
{
    if (n && (!in || !out)) return TSP_EINVAL;
    for (size_t i = 0; i < n; ++i) out[i] = tsp::split_bf16_bits(in[i]);
    return TSP_OK;
}

int tsp_pack_3byte_device(const void *d_src, void *d_dst, size_t n, void *stream)
{
    if (n % 4 || (n && (!d_src || !d_dst))) return TSP_EINVAL;
    if (n == 0) return TSP_OK;
    if (((uintptr_t)d_src | (uintptr_t)d_dst) & 3) return TSP_EINVAL;
    const char *s0 = (const char *)d_src, *d0 = (const char *)d_dst;
    if (d0 < s0 + 4 * n && s0 < d0 + 3 * n) return TSP_EINVAL;   // overlapping
    const size_t g = n / 4, b = (g + 255) / 256;
    tsp::pack_3byte_kernel<<<(unsigned)(b < 16384 ? b : 16384), 256, 0, (hipStream_t)stream>>>(
        (const uint32_t *)d_src, (uint32_t *)d_dst, g);
    return (int)hipGetLastError();
}

int tsp_pack_3byte_bits(const uint32_t *in, void *out, size_t n)
{
    if (n % 4 || (n && (!in || !out))) return TSP_EINVAL;
    unsigned char *o = (unsigned char *)out;
    for (size_t i = 0; i < n; ++i) {
        const uint32_t v = tsp::pack_3byte_bits(in[i]);
        o[3 * i] = (unsigned char)v;
        o[3 * i + 1] = (unsigned char)(v >> 8);
        o[3 * i + 2] = (unsigned char)(v >> 16);
    }
    return TSP_OK;
}

int tsp_round_tf32_device(void *d_x, size_t n, void *stream)
{
    if (n && !d_x) return TSP_EINVAL;
    if (n == 0) return TSP_OK;
    const size_t b = (n + 255) / 256;
    tsp::round_tf32_kernel<<<(unsigned)(b < 16384 ? b : 16384), 256, 0, (hipStream_t)stream>>>((uint32_t *)d_x, n);
    return (int)hipGetLastError();
}

int tsp_round_tf32_bits(const uint32_t *in, uint32_t *out, size_t n)
{
    if (n && (!in || !out)) return TSP_EINVAL;
    for (size_t i = 0; i < n; ++i) out[i] = tsp::round_tf32_bits(in[i]);
    return TSP_OK;
}

int tsp_copy_kernel(void *dst, const void *src, size_t bytes, void *stream)
{
    if ((!dst || !src) && bytes) return TSP_EINVAL;
    if (((uintptr_t)dst | (uintptr_t)src | bytes) & 15) return TSP_EINVAL;
    return tsp::launch_copy(dst, src, bytes, (hipStream_t)stream);
}

int tsp_gather_kernel(const void *table, size_t table_bytes, int row_bytes, int iters, unsigned seed,
                      void *sink, void *stream)
{
    const bool rb_ok = row_bytes == 16 || row_bytes == 32 || row_bytes == 64 || row_bytes == 128 || row_bytes == 256;
    if (!table || !sink || !rb_ok || iters <= 0) return TSP_EINVAL;
    if (table_bytes < (size_t)row_bytes || table_bytes / (size_t)row_bytes > 0xffffffffull) return TSP_EINVAL;
    if ((uintptr_t)table & 15) return TSP_EINVAL;
    return tsp::launch_gather(table, table_bytes, row_bytes, iters, seed, sink, (hipStream_t)stream);
}

int tsp_gather_index_stream(const void *d_table, long long table_rows, int row_bytes, const int *d_idx, long long n,
                            void *d_sink, void *stream)
{
    const bool rb_ok = row_bytes == 64 || row_bytes == 128 || row_bytes == 256 || row_bytes == 512 ||
                       row_bytes == 96 || row_bytes == 192 || row_bytes == 384;
    if (!rb_ok || n < 0 || (n > 0 && (!d_table || !d_idx || !d_sink || table_rows <= 0))) return TSP_EINVAL;
    if ((uintptr_t)d_table & 15) return TSP_EINVAL;
    return tsp::launch_stream_gather(d_table, table_rows, row_bytes, d_idx, n, d_sink, (hipStream_t)stream);
}

}  // extern "C"

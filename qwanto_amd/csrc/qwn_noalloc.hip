// Allocation-free Q8-KV attention (qwn_hip_ext_kv_attention_device_noalloc):
// the device attention entry point with its split partials kept in a
// file-scope device array instead of a caller-supplied workspace, for
// callers that cannot allocate (code under HIP graph capture, serving loops
// that forbid hipMalloc).
//
// The array is a host-side name only: kernels get its device address,
// looked up once per device with hipGetSymbolAddress (noalloc_init_device,
// called at context creation with the device current).  Every call on one
// GPU shares that GPU's array: calls that overlap on a GPU race.  The split
// kernel writes every partial the merge reads, so nothing needs clearing
// between calls.
#include "qwn_context.h"
#include "qwn_hip_ext.h"
#include "qwn_internal.h"

#include <mutex>

namespace {

constexpr size_t kScratchFloats = size_t{1} << 20;  // 4 MiB of partials per GPU
constexpr int kMaxScratchDevices = 64;

__device__ __align__(256) float scratch[kScratchFloats];

std::mutex g_scratch_mutex;
float *g_scratch[kMaxScratchDevices] = {};

}  // namespace

namespace qwn {

// The device address of `scratch` on `device`, which must be current.
hipError_t noalloc_init_device(int device) {
    if (device < 0 || device >= kMaxScratchDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch[device]) return hipSuccess;
    void *ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    g_scratch[device] = static_cast<float *>(ptr);
    return hipSuccess;
}

}  // namespace qwn

using namespace qwn;

extern "C" {

QWN_CUDA_ABI_API int qwn_hip_ext_kv_attention_device_noalloc(QwnCudaContextHandle *handle,
                                                             QwnCudaKvCacheHandle *h, const float *query,
                                                             float *output, uint32_t query_heads,
                                                             uint32_t position, float scale, void *stream) {
    Context *ctx = context_of(handle);
    if (!ctx || !h || !query || !output || query_heads == 0) {
        set_error("invalid allocation-free attention request");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    std::lock_guard<std::mutex> lock(ctx->mutex);
    ResidentKv *rk = cache_of(ctx, *h);
    if (!rk || position >= rk->c.tokens) {
        set_error("invalid allocation-free attention request");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    const size_t need = attention_workspace_floats(rk->c, query_heads, position);
    if (need > kScratchFloats) {
        set_error("allocation-free attention needs %llu bytes of partials; its device array holds %llu",
                  static_cast<unsigned long long>(need * sizeof(float)),
                  static_cast<unsigned long long>(kScratchFloats * sizeof(float)));
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    float *partials = nullptr;
    {
        std::lock_guard<std::mutex> slock(g_scratch_mutex);
        partials = ctx->device >= 0 && ctx->device < kMaxScratchDevices ? g_scratch[ctx->device] : nullptr;
    }
    if (!partials) {
        set_error("allocation-free attention: no device array address for device %d", ctx->device);
        return QWN_CUDA_STATUS_RUNTIME_ERROR;
    }
    AttentionLaunch a{};
    a.cache = &rk->c;
    a.query = query;
    a.output = output;
    a.query_heads = query_heads;
    a.position = position;
    a.scale = scale;
    a.partials = partials;
    hipStream_t s = stream ? static_cast<hipStream_t>(stream) : ctx->stream;
    const hipError_t e = launch_attention(a, s);
    if (e != hipSuccess) return hip_fail("allocation-free attention launch", e);
    ctx->telemetry.kv_cache_kernel_count++;
    return QWN_CUDA_STATUS_OK;
}

}  // extern "C"

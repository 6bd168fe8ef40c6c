// Allocation-free Q8-KV attention (qwn_hip_ext_kv_attention_device_noalloc):
// the device attention entry point with its split partials kept in a
// file-scope device array instead of a caller-supplied workspace, for
// callers that cannot allocate (code under HIP graph capture, serving loops
// that forbid hipMalloc).
//
// The array is a host-side name only: kernels get its device address,
// looked up once per device with hipGetSymbolAddress (noalloc_init_device,
// called at context creation with the device current).  Every call on one
// GPU shares that GPU's array, so two calls that run at the same time on a
// GPU would race: a call is refused (QWN_CUDA_STATUS_UNAVAILABLE) while the
// previous call on that GPU, enqueued on another stream, has not finished
// (a per-device event recorded behind each call; calls on one stream are
// ordered and always accepted).  Calls recorded into a HIP graph are not
// tracked: their ordering is the graph's.  The split kernel writes every
// partial the merge reads, so nothing needs clearing between calls.
#include "qwn_context.h"
#include "qwn_hip_ext.h"
#include "qwn_internal.h"

#include <mutex>

namespace {

constexpr size_t kScratchFloats = size_t{1} << 20;  // 4 MiB of partials per GPU
constexpr int kMaxScratchDevices = 64;

__device__ __align__(256) float scratch[kScratchFloats];

// Per device: the array's address, and the last call outside graph
// capture (the stream it was enqueued on, an event recorded behind it).
struct ScratchUse {
    float *ptr = nullptr;
    hipEvent_t done = nullptr;
    hipStream_t stream = nullptr;
    bool live = false;
};
std::mutex g_scratch_mutex;  // held across each call's check, launch and record
ScratchUse g_scratch[kMaxScratchDevices];

}  // namespace

namespace qwn {

// The device address of `scratch` on `device`, which must be current.
hipError_t noalloc_init_device(int device) {
    if (device < 0 || device >= kMaxScratchDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    ScratchUse &u = g_scratch[device];
    if (u.ptr) return hipSuccess;
    void *ptr = nullptr;
    hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if ((e = hipEventCreateWithFlags(&u.done, hipEventDisableTiming)) != hipSuccess) return e;
    u.ptr = static_cast<float *>(ptr);
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
    hipStream_t s = stream ? static_cast<hipStream_t>(stream) : ctx->stream;
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    hipError_t e = hipStreamIsCapturing(s, &capture);
    if (e != hipSuccess) return hip_fail("allocation-free attention stream query", e);
    std::lock_guard<std::mutex> slock(g_scratch_mutex);
    ScratchUse *u = ctx->device >= 0 && ctx->device < kMaxScratchDevices ? &g_scratch[ctx->device] : nullptr;
    if (!u || !u->ptr) {
        set_error("allocation-free attention: no device array address for device %d", ctx->device);
        return QWN_CUDA_STATUS_RUNTIME_ERROR;
    }
    if (capture == hipStreamCaptureStatusNone && u->live && u->stream != s) {
        e = hipEventQuery(u->done);
        if (e == hipErrorNotReady) {
            set_error("allocation-free attention: the previous call on device %d (another stream) has not "
                      "finished; its device array is in use", ctx->device);
            return QWN_CUDA_STATUS_UNAVAILABLE;
        }
        if (e != hipSuccess) return hip_fail("allocation-free attention event query", e);
    }
    AttentionLaunch a{};
    a.cache = &rk->c;
    a.query = query;
    a.output = output;
    a.query_heads = query_heads;
    a.position = position;
    a.scale = scale;
    a.partials = u->ptr;
    if ((e = launch_attention(a, s)) != hipSuccess) return hip_fail("allocation-free attention launch", e);
    if (capture == hipStreamCaptureStatusNone) {
        if ((e = hipEventRecord(u->done, s)) != hipSuccess) return hip_fail("allocation-free attention event", e);
        u->stream = s;
        u->live = true;
    }
    ctx->telemetry.kv_cache_kernel_count++;
    return QWN_CUDA_STATUS_OK;
}

}  // extern "C"

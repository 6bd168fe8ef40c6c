// qwn_hip: the qwnrun GPU ABI (qwn_cuda_abi.h) on one MI355X.
//
// Replaces c/cuda/qwn_hypervsq2_cuda_abi.cu.  Same contract: versioned
// struct headers validated on every call, resident weights charged against
// a memory budget, synchronous host-pointer GEMV/GEMM and Q8-KV calls,
// cumulative telemetry copied out on every call, one process-wide last
// error string.  Different machinery: weights are repacked on upload into
// the wave-tile layout of qwn_internal.h, activations are turned into an
// activation image on the device, host buffers are staged through pinned memory,
// every call runs on the context's own non-blocking stream, and each
// context has its own lock.
#include "qwn_context.h"
#include "qwn_cuda_abi.h"
#include "qwn_hip_ext.h"
#include "qwn_internal.h"

#include <algorithm>
#include <chrono>
#include <cstdarg>
#include <cstdlib>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <thread>
#include <new>
#include <string>
#include <vector>

namespace qwn {

std::mutex g_error_mutex;
std::string g_last_error;

void set_error(const char *fmt, ...) {
    char buffer[512];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buffer, sizeof(buffer), fmt, ap);
    va_end(ap);
    std::lock_guard<std::mutex> lock(g_error_mutex);
    g_last_error = buffer;
}

int hip_fail(const char *what, hipError_t e, int status) {
    set_error("%s: %s", what, hipGetErrorString(e));
    return status;
}

Context *context_of(const QwnCudaContextHandle *h) {
    if (!h || !header_ok(*h) || !h->opaque) return nullptr;
    return static_cast<Context *>(h->opaque);
}

ResidentTensor *tensor_of(Context *ctx, const QwnCudaTensorHandle &h) {
    if (!header_ok(h) || !h.opaque) return nullptr;
    auto *t = static_cast<ResidentTensor *>(h.opaque);
    // only handles this context issued are accepted
    return std::find(ctx->tensors.begin(), ctx->tensors.end(), t) != ctx->tensors.end() ? t : nullptr;
}

ResidentKv *cache_of(Context *ctx, const QwnCudaKvCacheHandle &h) {
    if (!header_ok(h) || !h.opaque) return nullptr;
    auto *c = static_cast<ResidentKv *>(h.opaque);
    return std::find(ctx->caches.begin(), ctx->caches.end(), c) != ctx->caches.end() ? c : nullptr;
}

}  // namespace qwn

namespace {

using namespace qwn;

double ms_since(std::chrono::steady_clock::time_point t0) {
    return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
}

void copy_telemetry(const Context *ctx, QwnCudaTelemetry *out) {
    if (out) *out = ctx->telemetry;
}

const char *kernel_name(const qwn::DeviceTensor &t) {
    switch (t.kind) {
    case qwn::kHvsq2: return "hvsq2-74-q8-gfx950";
    case qwn::kQ4_0: return "q4_0-18-q8-gfx950";
    case qwn::kF16: return t.bf16 ? "bf16-f32-gfx950" : "f16-f32-gfx950";
    default: return "none";
    }
}

// Validates a GEMV/GEMM request against a resident tensor; returns the
// tensor or null (error set).
ResidentTensor *check_request(Context *ctx, const QwnCudaGemmRequest *r) {
    if (!r || !header_ok(*r) || !r->input_q8 || !r->output || r->batch == 0 || r->rows == 0 ||
        r->cols == 0) {
        set_error("invalid GEMV/GEMM request");
        return nullptr;
    }
    ResidentTensor *rt = tensor_of(ctx, r->tensor);
    if (!rt || rt->t.rows != r->rows || rt->t.cols != r->cols) {
        set_error("tensor handle unknown or dimensions do not match the request");
        return nullptr;
    }
    const uint32_t in_stride = r->input_stride ? r->input_stride : r->cols;
    const uint32_t out_stride = r->output_stride ? r->output_stride : r->rows;
    if (in_stride < r->cols || out_stride < r->rows) {
        set_error("input/output stride smaller than the tensor shape");
        return nullptr;
    }
    const bool f16 = rt->t.kind == qwn::kF16;
    // F16 tensors take fp32 activations; quantized tensors take int8 tokens
    // with their scales, or fp32 activations quantized on the device.
    if (r->input_mode != QWN_CUDA_INPUT_F32 && (f16 || r->input_mode != QWN_CUDA_INPUT_Q8)) {
        set_error("input mode %u does not match the tensor dtype", r->input_mode);
        return nullptr;
    }
    return rt;
}

int execute_gemm(Context *ctx, const QwnCudaGemmRequest *r, QwnCudaTelemetry *telemetry) {
    ResidentTensor *rt = check_request(ctx, r);
    if (!rt) return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    const DeviceTensor &t = rt->t;
    hipError_t e = hipSetDevice(ctx->device);
    if (e != hipSuccess) return hip_fail("hipSetDevice", e);

    const bool f16 = t.kind == qwn::kF16;
    const bool f32_in = r->input_mode == QWN_CUDA_INPUT_F32;
    const bool quantize = f32_in && !f16;  // per-token int8 quantization on the device
    const size_t elem = f32_in ? 4 : 1;
    const uint32_t in_stride = r->input_stride ? r->input_stride : r->cols;
    const uint32_t out_stride = r->output_stride ? r->output_stride : r->rows;
    // device copy of the activations with a 16-byte aligned row stride
    const uint32_t dev_stride = (r->cols + 255u) & ~255u;
    const size_t in_bytes = static_cast<size_t>(r->batch) * dev_stride * elem;
    const size_t scale_bytes = static_cast<size_t>(r->batch) * sizeof(float);
    const size_t out_bytes = static_cast<size_t>(r->batch) * r->rows * sizeof(float);
    const uint32_t img_stride = static_cast<uint32_t>(qwn::image_bytes(t.kind, t.units));
    const size_t img_bytes = static_cast<size_t>(r->batch) * img_stride;
    if ((e = ctx->host_in.ensure(in_bytes + scale_bytes)) != hipSuccess ||
        (e = ctx->host_out.ensure(out_bytes)) != hipSuccess ||
        (e = ctx->dev_in.ensure(in_bytes)) != hipSuccess ||
        (e = ctx->dev_scales.ensure(scale_bytes)) != hipSuccess ||
        (e = ctx->dev_out.ensure(out_bytes)) != hipSuccess ||
        (e = ctx->dev_img.ensure(img_bytes)) != hipSuccess)
        return hip_fail("GEMV workspace allocation", e, QWN_CUDA_STATUS_OUT_OF_MEMORY);

    const auto t_transfer = std::chrono::steady_clock::now();
    uint8_t *hin = static_cast<uint8_t *>(ctx->host_in.ptr);
    const uint8_t *src = reinterpret_cast<const uint8_t *>(r->input_q8);
    for (uint32_t b = 0; b < r->batch; ++b) {
        std::memcpy(hin + static_cast<size_t>(b) * dev_stride * elem,
                    src + static_cast<size_t>(b) * in_stride * elem, static_cast<size_t>(r->cols) * elem);
        std::memset(hin + (static_cast<size_t>(b) * dev_stride + r->cols) * elem, 0,
                    static_cast<size_t>(dev_stride - r->cols) * elem);
    }
    float *hscales = reinterpret_cast<float *>(hin + in_bytes);
    for (uint32_t b = 0; b < r->batch; ++b) hscales[b] = r->input_scales ? r->input_scales[b] : r->input_scale;
    // int8 MFMA tiles of 16 tokens (mfma_batch: from 2 HyperVSQ-2 / 3 Q4_0
    // tokens on the MFMA-order copy, from 3 / 6 without it)
    const bool mfma = qwn::mfma_batch(t.kind, r->batch, t.mfma_payload != nullptr);
    // Small requests skip the copy engines: the image kernel reads the
    // activations (and the GEMV its scales) straight from the pinned staging
    // buffer, and the GEMV epilogue stores into the pinned output buffer, so a
    // call is two kernels and one synchronisation instead of three DMA
    // transfers around them.  Outputs of 64K+ rows (the LM head) and the MFMA
    // path keep the device buffers and DMA.
    const bool zero_copy = !mfma && r->rows < 65536;
    if (!zero_copy &&
        ((e = hipMemcpyAsync(ctx->dev_in.ptr, hin, in_bytes, hipMemcpyHostToDevice, ctx->stream)) != hipSuccess ||
         (!quantize && (e = hipMemcpyAsync(ctx->dev_scales.ptr, hscales, scale_bytes, hipMemcpyHostToDevice,
                                           ctx->stream)) != hipSuccess)))
        return hip_fail("activation upload", e);
    const void *act = zero_copy ? static_cast<const void *>(hin) : ctx->dev_in.ptr;
    float *scales_dev = zero_copy ? (quantize ? static_cast<float *>(ctx->dev_scales.ptr) : hscales)
                                  : static_cast<float *>(ctx->dev_scales.ptr);
    float *out_dev = zero_copy ? static_cast<float *>(ctx->host_out.ptr) : static_cast<float *>(ctx->dev_out.ptr);
    const double transfer_ms = ms_since(t_transfer);

    qwn::GemvLaunch g{};
    g.tensor = &t;
    g.image = ctx->dev_img.ptr;
    g.image_stride = img_stride;
    g.scales = scales_dev;
    g.scale = r->input_scale;
    g.output = out_dev;
    g.batch = r->batch;
    g.output_stride = r->rows;
    const size_t mfma_img = qwn::mfma_image_bytes(t);
    if (mfma && ((e = ctx->dev_work.ensure(mfma_img + (quantize ? in_bytes / 4 : 0))) != hipSuccess))
        return hip_fail("MFMA workspace allocation", e, QWN_CUDA_STATUS_OUT_OF_MEMORY);
    (void)hipEventRecord(ctx->ev_start, ctx->stream);
    if (mfma) {
        // int8 tokens on the device: as given, or quantized from fp32 per token
        const int8_t *q8 = static_cast<const int8_t *>(ctx->dev_in.ptr);
        if (quantize) {
            int8_t *dq = reinterpret_cast<int8_t *>(static_cast<uint8_t *>(ctx->dev_work.ptr) + mfma_img);
            e = qwn::launch_quantize_image(t, static_cast<const float *>(ctx->dev_in.ptr), r->batch, dev_stride,
                                           nullptr, 0, static_cast<float *>(ctx->dev_scales.ptr), dq, dev_stride,
                                           ctx->stream);
            if (e != hipSuccess) return hip_fail("activation quantize launch", e);
            q8 = dq;
        }
        uint8_t *img = static_cast<uint8_t *>(ctx->dev_work.ptr);
        for (uint32_t t0 = 0; t0 < r->batch; t0 += 16) {
            const uint32_t nt = std::min<uint32_t>(16, r->batch - t0);
            if ((e = qwn::launch_mfma_image(t, q8 + static_cast<size_t>(t0) * dev_stride, nt, dev_stride, img,
                                            ctx->stream)) != hipSuccess ||
                (e = qwn::launch_gemm_mfma(t, img, static_cast<const float *>(ctx->dev_scales.ptr) + t0,
                                           static_cast<float *>(ctx->dev_out.ptr) + static_cast<size_t>(t0) * r->rows,
                                           nt, r->rows, ctx->stream)) != hipSuccess)
                return hip_fail("MFMA GEMM launch", e);
        }
    } else {
        if (quantize)
            e = qwn::launch_quantize_image(t, static_cast<const float *>(act), r->batch, dev_stride,
                                           static_cast<uint8_t *>(ctx->dev_img.ptr), img_stride,
                                           static_cast<float *>(ctx->dev_scales.ptr), nullptr, 0, ctx->stream);
        else
            e = qwn::launch_image(t, act, r->batch, dev_stride, static_cast<uint8_t *>(ctx->dev_img.ptr), img_stride,
                                  ctx->stream);
        if (e != hipSuccess) return hip_fail("activation image launch", e);
        if ((e = qwn::launch_gemv(g, ctx->stream)) != hipSuccess) return hip_fail("GEMV launch", e);
    }
    (void)hipEventRecord(ctx->ev_end, ctx->stream);
    if (!zero_copy && (e = hipMemcpyAsync(ctx->host_out.ptr, ctx->dev_out.ptr, out_bytes, hipMemcpyDeviceToHost,
                                          ctx->stream)) != hipSuccess)
        return hip_fail("result download", e);
    const auto t_sync = std::chrono::steady_clock::now();
    if ((e = hipStreamSynchronize(ctx->stream)) != hipSuccess) return hip_fail("GEMV synchronize", e);
    const double sync_ms = ms_since(t_sync);
    const float *hout = static_cast<const float *>(ctx->host_out.ptr);
    for (uint32_t b = 0; b < r->batch; ++b)
        std::memcpy(r->output + static_cast<size_t>(b) * out_stride, hout + static_cast<size_t>(b) * r->rows,
                    static_cast<size_t>(r->rows) * sizeof(float));
    float kernel_ms = 0.0f;
    if (hipEventElapsedTime(&kernel_ms, ctx->ev_start, ctx->ev_end) != hipSuccess) kernel_ms = 0.0f;

    QwnCudaTelemetry &tm = ctx->telemetry;
    tm.gpu_matmul_count++;
    tm.gpu_kernel_launch_count += 1 + (r->batch + qwn::kMaxTokensPerLaunch - 1) / qwn::kMaxTokensPerLaunch;
    tm.gpu_projection_count++;
    tm.gpu_kernel_ms += kernel_ms;
    tm.gpu_transfer_ms += transfer_ms;
    tm.gpu_sync_ms += sync_ms;
    tm.gpu_resident_bytes = ctx->resident;
    tm.device_id = ctx->device;
    std::snprintf(tm.kernel_type, sizeof(tm.kernel_type), "%s", kernel_name(t));
    copy_telemetry(ctx, telemetry);
    return QWN_CUDA_STATUS_OK;
}

void free_tensor(ResidentTensor *rt) {
    if (rt->allocation) (void)hipFree(rt->allocation);
    if (rt->mfma_allocation) (void)hipFree(rt->mfma_allocation);
    delete rt;
}

// The MFMA-order copy of a HyperVSQ-2 or Q4_0 tensor (qwn::launch_mfma_copy),
// which the batched GEMM reads directly instead of staging the wave tiles.
// Its bytes are charged to the context like the tensor's own (the budget
// caps every device byte a tensor holds, c/cuda/qwn_hypervsq2_cuda_abi.cu:
// 554-562) and reported in gpu_resident_bytes.  The copy is optional, so it
// never takes room a tensor needs:
//  - under a budget it is made only in a batch upload (`batch`), from the
//    budget left after every tensor of the batch (`pending`: this upload's
//    tensors, not yet charged) and the copies already made (`copies`), and
//    only while a tenth of the device stays free; an upload of one tensor at
//    a time (the reference host's lazy upload) gets no copy, since a later
//    tensor would otherwise be refused for the room it took;
//  - without a budget it is made while half the device stays free.
// A model too large for that gets copies for its first tensors only, or
// none; a group of tensors that are not all copied runs the staged GEMM.
// QWN_HIP_MFMA_COPY=0 turns the copies off.
void attach_mfma_copy(Context *ctx, ResidentTensor *rt, uint64_t pending, uint64_t copies, bool batch) {
    const size_t cb = qwn::mfma_copy_bytes(rt->t);
    if (!cb) return;
    const char *env = std::getenv("QWN_HIP_MFMA_COPY");
    if (env && env[0] == '0') return;
    size_t free_b = 0, total_b = 0;
    if (hipMemGetInfo(&free_b, &total_b) != hipSuccess) return;
    uint64_t reserve = total_b / 2;
    if (ctx->budget) {
        const uint64_t charged = ctx->resident + pending + copies;
        if (!batch || charged > ctx->budget || ctx->budget - charged < cb) return;
        reserve = total_b / 10;
    }
    if (free_b < cb + reserve) return;
    if (hipMalloc(&rt->mfma_allocation, cb) != hipSuccess) {
        rt->mfma_allocation = nullptr;
        return;
    }
    rt->copy_bytes = cb;
    const size_t groups = (rt->t.rows + 15) / 16;
    rt->t.mfma_payload = static_cast<uint8_t *>(rt->mfma_allocation);
    rt->t.mfma_meta = rt->t.mfma_payload + groups * rt->t.units * 1024;
}

void free_cache(ResidentKv *rk) {
    if (rk->allocation) (void)hipFree(rk->allocation);
    delete rk;
}

bool budget_allows(Context *ctx, uint64_t bytes, uint64_t device_bytes) {
    size_t free_b = 0, total_b = 0;
    if (hipMemGetInfo(&free_b, &total_b) != hipSuccess) return false;
    if (ctx->budget && ctx->resident + bytes > ctx->budget) return false;
    return device_bytes <= free_b;
}

}  // namespace

extern "C" {

QWN_CUDA_ABI_API int qwn_cuda_abi_query(QwnCudaAbiInfo *info) {
    if (!info || !header_ok(*info)) {
        set_error("invalid ABI query structure");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    std::memset(info, 0, sizeof(*info));
    qwn_cuda_abi_header_init(&info->header, sizeof(*info));
    info->capability_bits = QWN_CUDA_CAP_HYPERVSQ2_GEMV | QWN_CUDA_CAP_HYPERVSQ2_GEMM |
                            QWN_CUDA_CAP_RESIDENT_WEIGHTS | QWN_CUDA_CAP_TELEMETRY |
                            QWN_CUDA_CAP_DEVICE_ENUMERATION | QWN_CUDA_CAP_Q8_KV |
                            QWN_CUDA_CAP_Q4_0_GEMV | QWN_CUDA_CAP_F16_GEMV |
                            QWN_CUDA_CAP_DEVICE_POINTERS | QWN_CUDA_CAP_BF16_GEMV;
    info->max_devices = 16;
    info->max_resident_tensors = QWN_CUDA_MAX_RESIDENT_TENSORS;
    info->hypervsq2_block_bytes = QWN_CUDA_HYPERVSQ2_BLOCK_BYTES;
    info->hypervsq2_block_elements = QWN_CUDA_HYPERVSQ2_BLOCK_ELEMENTS;
    std::snprintf(info->abi_name, sizeof(info->abi_name), "%s", QWN_CUDA_ABI_NAME);
    return QWN_CUDA_STATUS_OK;
}

QWN_CUDA_ABI_API int qwn_cuda_abi_get_capabilities(QwnCudaAbiInfo *info) {
    return qwn_cuda_abi_query(info);
}

QWN_CUDA_ABI_API int qwn_cuda_abi_enumerate_devices(QwnCudaDeviceInfo *devices, uint32_t capacity,
                                                    uint32_t *count) {
    if (!count) {
        set_error("enumerate_devices: null count");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess) {
        *count = 0;
        return hip_fail("hipGetDeviceCount", e, QWN_CUDA_STATUS_UNAVAILABLE);
    }
    *count = static_cast<uint32_t>(n);
    if (!devices || capacity == 0) return QWN_CUDA_STATUS_OK;
    int driver = 0;
    (void)hipDriverGetVersion(&driver);
    int current = 0;
    (void)hipGetDevice(&current);
    const uint32_t limit = std::min<uint32_t>(capacity, *count);
    for (uint32_t i = 0; i < limit; ++i) {
        QwnCudaDeviceInfo &d = devices[i];
        std::memset(&d, 0, sizeof(d));
        qwn_cuda_abi_header_init(&d.header, sizeof(d));
        hipDeviceProp_t p{};
        if (hipGetDeviceProperties(&p, static_cast<int>(i)) != hipSuccess) continue;
        d.device_id = static_cast<int32_t>(i);
        // gfx950 -> compute 9.5 (the gfx major/minor digits)
        d.compute_major = p.major;
        d.compute_minor = p.minor;
        d.total_vram_bytes = p.totalGlobalMem;
        size_t free_b = 0, total_b = 0;
        if (hipSetDevice(static_cast<int>(i)) == hipSuccess && hipMemGetInfo(&free_b, &total_b) == hipSuccess)
            d.free_vram_bytes = free_b;
        std::snprintf(d.name, sizeof(d.name), "%s (%s)", p.name, p.gcnArchName);
        std::snprintf(d.driver, sizeof(d.driver), "hip %d", driver);
    }
    (void)hipSetDevice(current);
    return QWN_CUDA_STATUS_OK;
}

QWN_CUDA_ABI_API int qwn_cuda_abi_context_create(const QwnCudaContextOptions *options,
                                                 QwnCudaContextHandle *handle) {
    if (!options || !handle || !header_ok(*options) || !header_ok(*handle) || options->device_id < 0) {
        set_error("invalid context options");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || options->device_id >= n) {
        set_error("device %d is not available", options->device_id);
        return QWN_CUDA_STATUS_UNAVAILABLE;
    }
    {
        // the kernels are gfx950 code objects and the MFMA GEMM stages up to
        // kMfmaLdsLimit bytes of LDS per workgroup
        hipDeviceProp_t dp{};
        if (hipGetDeviceProperties(&dp, options->device_id) != hipSuccess ||
            std::strncmp(dp.gcnArchName, "gfx950", 6) != 0 || dp.sharedMemPerBlock < qwn::kMfmaLdsLimit) {
            set_error("device %d (%s) is not a gfx950 device with %llu bytes of LDS per workgroup", options->device_id,
                      dp.gcnArchName, static_cast<unsigned long long>(qwn::kMfmaLdsLimit));
            return QWN_CUDA_STATUS_UNSUPPORTED;
        }
    }
    auto *ctx = new (std::nothrow) Context();
    if (!ctx) return QWN_CUDA_STATUS_OUT_OF_MEMORY;
    ctx->device = options->device_id;
    ctx->budget = options->memory_budget_bytes;
    hipError_t e = hipSetDevice(ctx->device);
    if (e == hipSuccess) e = qwn::noalloc_init_device(ctx->device);
    // A blocking stream: work on it is ordered with work on the null stream
    // (torch's default stream), which callers of the device-pointer entry
    // points pass as NULL = this stream; a non-blocking stream let a null-stream
    // fill of an output buffer land after the library's kernel had written it.
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&ctx->stream, hipStreamDefault);
    if (e == hipSuccess) e = hipEventCreate(&ctx->ev_start);
    if (e == hipSuccess) e = hipEventCreate(&ctx->ev_end);
    if (e != hipSuccess) {
        if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
        delete ctx;
        return hip_fail("context creation", e, QWN_CUDA_STATUS_UNAVAILABLE);
    }
    QwnCudaTelemetry &tm = ctx->telemetry;
    std::memset(&tm, 0, sizeof(tm));
    qwn_cuda_abi_header_init(&tm.header, sizeof(tm));
    tm.device_id = ctx->device;
    hipDeviceProp_t p{};
    if (hipGetDeviceProperties(&p, ctx->device) == hipSuccess)
        std::snprintf(tm.device_name, sizeof(tm.device_name), "%s (%s)", p.name, p.gcnArchName);
    std::snprintf(tm.kernel_type, sizeof(tm.kernel_type), "%s", "hvsq2-74-q8-gfx950");
    std::snprintf(tm.kv_cache_kernel_type, sizeof(tm.kv_cache_kernel_type), "Unavailable");
    std::memset(handle, 0, sizeof(*handle));
    qwn_cuda_abi_header_init(&handle->header, sizeof(*handle));
    handle->opaque = ctx;
    return QWN_CUDA_STATUS_OK;
}

QWN_CUDA_ABI_API int qwn_cuda_abi_context_destroy(QwnCudaContextHandle *handle) {
    Context *ctx = context_of(handle);
    if (!ctx) {
        set_error("invalid context handle");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    {
        std::lock_guard<std::mutex> lock(ctx->mutex);
        (void)hipSetDevice(ctx->device);
        (void)hipStreamSynchronize(ctx->stream);
        for (Decoder *d : ctx->decoders) destroy_decoder(d);
        ctx->decoders.clear();
        for (ResidentTensor *t : ctx->tensors) free_tensor(t);
        for (ResidentKv *c : ctx->caches) free_cache(c);
        ctx->tensors.clear();
        ctx->caches.clear();
        ctx->host_in.release();
        ctx->host_out.release();
        ctx->dev_in.release();
        ctx->dev_out.release();
        ctx->dev_scales.release();
        ctx->dev_work.release();
        ctx->dev_img.release();
        for (int i = 0; i < 2; ++i) {
            ctx->upload.host[i].release();
            ctx->upload.dev[i].release();
            if (ctx->upload.done[i]) (void)hipEventDestroy(ctx->upload.done[i]);
        }
        (void)hipEventDestroy(ctx->ev_start);
        (void)hipEventDestroy(ctx->ev_end);
        (void)hipStreamDestroy(ctx->stream);
    }
    delete ctx;
    handle->opaque = nullptr;
    return QWN_CUDA_STATUS_OK;
}

namespace {

// Validates an upload and lays the tensor out (no device memory yet).
int describe_upload(const QwnCudaTensorUpload *up, DeviceTensor &t) {
    if (!up || !header_ok(*up) || !up->host_data || up->rows == 0 || up->cols == 0) {
        set_error("invalid tensor upload request");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    t = DeviceTensor{};
    t.rows = up->rows;
    t.cols = up->cols;
    switch (up->dtype) {
    case QWN_CUDA_TENSOR_HYPERVSQ2_74:
        if (up->block_bytes != QWN_CUDA_HYPERVSQ2_BLOCK_BYTES) break;
        t.kind = qwn::kHvsq2;
        t.logical_bytes = static_cast<uint64_t>(up->rows) * ((up->cols + 255u) / 256u) * 74u;
        break;
    case QWN_CUDA_TENSOR_Q4_0_18:
        if (up->block_bytes != QWN_CUDA_Q4_0_BLOCK_BYTES) break;
        t.kind = qwn::kQ4_0;
        t.logical_bytes = static_cast<uint64_t>(up->rows) * ((up->cols + 31u) / 32u) * 18u;
        break;
    case QWN_CUDA_TENSOR_F16:
    case QWN_CUDA_TENSOR_BF16:
        if (up->block_bytes != 2) break;
        t.kind = qwn::kF16;
        t.bf16 = up->dtype == QWN_CUDA_TENSOR_BF16;
        t.logical_bytes = static_cast<uint64_t>(up->rows) * up->cols * 2u;
        break;
    default:
        break;
    }
    if (t.kind == 0) {
        set_error("unsupported tensor dtype %u / block_bytes %u", up->dtype, up->block_bytes);
        return QWN_CUDA_STATUS_UNSUPPORTED;
    }
    if (up->data_bytes < t.logical_bytes) {
        set_error("tensor upload is shorter than its shape (%llu < %llu bytes)",
                  static_cast<unsigned long long>(up->data_bytes),
                  static_cast<unsigned long long>(t.logical_bytes));
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    if (!qwn::layout_tensor(t)) {
        set_error("tensor rows of %u columns exceed the GEMV lane plan", up->cols);
        return QWN_CUDA_STATUS_UNSUPPORTED;
    }
    return QWN_CUDA_STATUS_OK;
}

// Host copy into a pinned slot, split over up to 8 threads for large chunks
// (one core's copy rate is below what the DMA engines take).
void copy_parallel(void *dst, const uint8_t *src, size_t bytes) {
    constexpr size_t kPerThread = 4u << 20;
    const unsigned hw = std::max(1u, std::thread::hardware_concurrency() / 2);
    const size_t n = std::min<size_t>({8, hw, (bytes + kPerThread - 1) / kPerThread});
    if (n <= 1) {
        std::memcpy(dst, src, bytes);
        return;
    }
    const size_t part = (bytes / n + 63) & ~static_cast<size_t>(63);
    std::vector<std::thread> workers;
    for (size_t i = 1; i < n; ++i) {
        const size_t off = i * part;
        if (off >= bytes) break;
        workers.emplace_back([=] { std::memcpy(static_cast<uint8_t *>(dst) + off, src + off, std::min(part, bytes - off)); });
    }
    std::memcpy(dst, src, std::min(part, bytes));
    for (auto &w : workers) w.join();
}

// Enqueues the upload of one allocated tensor through the pipeline (context
// lock held): the layout is zeroed, then chunks of whole rows go host ->
// pinned slot (CPU copy, after that slot's previous DMA and repack ended)
// -> device slot (DMA) -> wave-tile layout (repack kernel), alternating
// slots so the CPU copy of one chunk overlaps the DMA and repack of the
// previous one.  Nothing here waits for the last chunk.
hipError_t enqueue_upload(Context *ctx, const DeviceTensor &t, const uint8_t *host) {
    UploadPipe &p = ctx->upload;
    hipError_t e = hipSuccess;
    for (int i = 0; i < 2 && e == hipSuccess; ++i) {
        if (!p.done[i]) e = hipEventCreateWithFlags(&p.done[i], hipEventDisableTiming);
        if (e == hipSuccess) e = p.host[i].ensure(kUploadSlotBytes);
        if (e == hipSuccess) e = p.dev[i].ensure(kUploadSlotBytes);
    }
    if (e == hipSuccess) e = qwn::clear_tensor(t, ctx->stream);
    const uint64_t row_bytes = t.logical_bytes / t.rows;
    const uint32_t per_chunk = static_cast<uint32_t>(std::max<uint64_t>(1, kUploadSlotBytes / row_bytes));
    if (row_bytes > kUploadSlotBytes) {
        for (int i = 0; i < 2 && e == hipSuccess; ++i) {
            if (p.pending[i]) e = hipEventSynchronize(p.done[i]);
            p.pending[i] = false;
            if (e == hipSuccess) e = p.host[i].ensure(row_bytes);
            if (e == hipSuccess) e = p.dev[i].ensure(row_bytes);
        }
    }
    for (uint32_t r0 = 0; e == hipSuccess && r0 < t.rows; r0 += per_chunk) {
        const int s = p.next;
        p.next ^= 1;
        const uint32_t n = std::min(per_chunk, t.rows - r0);
        const size_t bytes = static_cast<size_t>(n) * row_bytes;
        if (p.pending[s] && (e = hipEventSynchronize(p.done[s])) != hipSuccess) break;
        p.pending[s] = false;
        copy_parallel(p.host[s].ptr, host + static_cast<size_t>(r0) * row_bytes, bytes);
        if ((e = hipMemcpyAsync(p.dev[s].ptr, p.host[s].ptr, bytes, hipMemcpyHostToDevice, ctx->stream)) !=
                hipSuccess ||
            (e = qwn::repack_rows(t, static_cast<const uint8_t *>(p.dev[s].ptr), r0, n, ctx->stream)) !=
                hipSuccess ||
            (e = hipEventRecord(p.done[s], ctx->stream)) != hipSuccess)
            break;
        p.pending[s] = true;
    }
    return e;
}

// Uploads `count` tensors (context lock held): describe and allocate all,
// pipeline all, one synchronisation; on failure none stays resident.
// `batch`: the caller handed over its tensors together
// (qwn_hip_ext_upload_batch), so under a budget MFMA-order copies may use
// what the budget leaves after all of them.
int upload_tensors(Context *ctx, const QwnCudaTensorUpload *ups, uint32_t count, QwnCudaTensorHandle *out,
                   bool batch) {
    std::vector<ResidentTensor *> made;
    uint64_t bytes = 0, device_bytes = 0;
    auto fail = [&](int status) {
        (void)hipStreamSynchronize(ctx->stream);
        for (ResidentTensor *rt : made) free_tensor(rt);
        return status;
    };
    if (ctx->tensors.size() + count > QWN_CUDA_MAX_RESIDENT_TENSORS) {
        set_error("resident tensor limit (%u) reached", QWN_CUDA_MAX_RESIDENT_TENSORS);
        return QWN_CUDA_STATUS_OUT_OF_MEMORY;
    }
    hipError_t e = hipSetDevice(ctx->device);
    if (e != hipSuccess) return hip_fail("hipSetDevice", e);
    for (uint32_t i = 0; i < count; ++i) {
        if (!header_ok(out[i])) {
            set_error("invalid tensor handle %u", i);
            return fail(QWN_CUDA_STATUS_INVALID_ARGUMENT);
        }
        DeviceTensor t;
        const int st = describe_upload(&ups[i], t);
        if (st != QWN_CUDA_STATUS_OK) return fail(st);
        bytes += t.logical_bytes;
        device_bytes += t.device_bytes;
        if (!budget_allows(ctx, bytes, device_bytes)) {
            set_error("tensor upload does not fit the configured GPU memory budget");
            return fail(QWN_CUDA_STATUS_OUT_OF_MEMORY);
        }
        auto *rt = new (std::nothrow) ResidentTensor();
        if (!rt) return fail(QWN_CUDA_STATUS_OUT_OF_MEMORY);
        if ((e = hipMalloc(&rt->allocation, t.device_bytes)) != hipSuccess) {
            delete rt;
            (void)hip_fail("tensor allocation", e, QWN_CUDA_STATUS_OUT_OF_MEMORY);
            return fail(QWN_CUDA_STATUS_OUT_OF_MEMORY);
        }
        t.payload = static_cast<uint8_t *>(rt->allocation);
        const size_t meta_off = (t.tile_payload_bytes * t.tiles + 255) & ~static_cast<size_t>(255);
        t.meta = t.tile_meta_bytes ? t.payload + meta_off : nullptr;
        rt->t = t;
        made.push_back(rt);
    }
    const auto t0 = std::chrono::steady_clock::now();
    uint64_t pending = 0, copies = 0;
    for (uint32_t i = 0; i < count; ++i) pending += made[i]->t.logical_bytes;
    for (uint32_t i = 0; i < count; ++i) {
        if ((e = enqueue_upload(ctx, made[i]->t, static_cast<const uint8_t *>(ups[i].host_data))) != hipSuccess) {
            (void)hip_fail("tensor upload", e);
            return fail(QWN_CUDA_STATUS_RUNTIME_ERROR);
        }
        attach_mfma_copy(ctx, made[i], pending, copies, batch);
        copies += made[i]->copy_bytes;
        if (made[i]->t.mfma_payload && (e = qwn::launch_mfma_copy(made[i]->t, ctx->stream)) != hipSuccess) {
            (void)hip_fail("MFMA-order copy", e);
            return fail(QWN_CUDA_STATUS_RUNTIME_ERROR);
        }
    }
    if ((e = hipStreamSynchronize(ctx->stream)) != hipSuccess) {
        (void)hip_fail("tensor upload", e);
        return fail(QWN_CUDA_STATUS_RUNTIME_ERROR);
    }
    ctx->upload.pending[0] = ctx->upload.pending[1] = false;
    QwnCudaTelemetry &tm = ctx->telemetry;
    for (uint32_t i = 0; i < count; ++i) {
        ctx->tensors.push_back(made[i]);
        ctx->resident += made[i]->t.logical_bytes + made[i]->copy_bytes;
        tm.gpu_upload_count++;
        tm.gpu_upload_bytes += made[i]->t.logical_bytes;
        std::memset(&out[i], 0, sizeof(out[i]));
        qwn_cuda_abi_header_init(&out[i].header, sizeof(out[i]));
        out[i].opaque = made[i];
    }
    tm.gpu_resident_bytes = ctx->resident;
    tm.gpu_transfer_ms += ms_since(t0);
    return QWN_CUDA_STATUS_OK;
}

}  // namespace

QWN_CUDA_ABI_API int qwn_cuda_abi_upload_tensor(QwnCudaContextHandle *handle,
                                                const QwnCudaTensorUpload *up,
                                                QwnCudaTensorHandle *out) {
    Context *ctx = context_of(handle);
    if (!ctx || !up || !out || !header_ok(*up) || !header_ok(*out)) {
        set_error("invalid tensor upload request");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    std::lock_guard<std::mutex> lock(ctx->mutex);
    return upload_tensors(ctx, up, 1, out, false);
}

QWN_CUDA_ABI_API int qwn_hip_ext_upload_batch(QwnCudaContextHandle *handle, const QwnCudaTensorUpload *uploads,
                                              uint32_t count, QwnCudaTensorHandle *out) {
    Context *ctx = context_of(handle);
    if (!ctx || !uploads || !out || count == 0) {
        set_error("invalid batch upload request");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    std::lock_guard<std::mutex> lock(ctx->mutex);
    return upload_tensors(ctx, uploads, count, out, true);
}

QWN_CUDA_ABI_API int qwn_cuda_abi_release_tensor(QwnCudaContextHandle *handle, QwnCudaTensorHandle *h) {
    Context *ctx = context_of(handle);
    if (!ctx || !h) {
        set_error("invalid release request");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    std::lock_guard<std::mutex> lock(ctx->mutex);
    ResidentTensor *rt = tensor_of(ctx, *h);
    if (!rt) {
        set_error("tensor handle is not resident in this context");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    ctx->resident -= std::min(ctx->resident, rt->t.logical_bytes + rt->copy_bytes);
    ctx->tensors.erase(std::find(ctx->tensors.begin(), ctx->tensors.end(), rt));
    free_tensor(rt);
    ctx->telemetry.gpu_resident_bytes = ctx->resident;
    h->opaque = nullptr;
    return QWN_CUDA_STATUS_OK;
}

QWN_CUDA_ABI_API int qwn_cuda_abi_kv_cache_create(QwnCudaContextHandle *handle,
                                                  const QwnCudaKvCacheOptions *opt,
                                                  QwnCudaKvCacheHandle *out) {
    Context *ctx = context_of(handle);
    if (!ctx || !opt || !out || !header_ok(*opt) || !header_ok(*out) || opt->max_tokens == 0 ||
        opt->kv_heads == 0 || opt->head_dim == 0) {
        set_error("invalid Q8 KV-cache options");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    KvCache c;
    c.max_tokens = opt->max_tokens;
    c.kv_heads = opt->kv_heads;
    c.head_dim = opt->head_dim;
    const size_t total = qwn::kv_cache_layout(c, nullptr);
    // charged like the reference (c/cuda/qwn_hypervsq2_cuda_abi.cu:624-626)
    c.bytes = static_cast<uint64_t>(c.max_tokens) * c.channels * 2u +
              static_cast<uint64_t>(c.max_tokens) * c.groups * sizeof(float) * 2u;
    std::lock_guard<std::mutex> lock(ctx->mutex);
    if (ctx->caches.size() >= QWN_CUDA_MAX_RESIDENT_KV_CACHES) {
        set_error("resident KV-cache limit reached");
        return QWN_CUDA_STATUS_OUT_OF_MEMORY;
    }
    hipError_t e = hipSetDevice(ctx->device);
    if (e != hipSuccess) return hip_fail("hipSetDevice", e);
    if (!budget_allows(ctx, c.bytes, total)) {
        set_error("Q8 KV-cache does not fit the configured GPU memory budget");
        return QWN_CUDA_STATUS_OUT_OF_MEMORY;
    }
    auto *rk = new (std::nothrow) ResidentKv();
    if (!rk) return QWN_CUDA_STATUS_OUT_OF_MEMORY;
    if ((e = hipMalloc(&rk->allocation, total)) != hipSuccess) {
        delete rk;
        return hip_fail("Q8 KV-cache allocation", e, QWN_CUDA_STATUS_OUT_OF_MEMORY);
    }
    uint8_t *base = static_cast<uint8_t *>(rk->allocation);
    qwn::kv_cache_layout(c, base);
    if ((e = hipMemsetAsync(base, 0, total, ctx->stream)) != hipSuccess ||
        (e = hipStreamSynchronize(ctx->stream)) != hipSuccess) {
        free_cache(rk);
        return hip_fail("Q8 KV-cache clear", e);
    }
    rk->c = c;
    ctx->caches.push_back(rk);
    ctx->resident += c.bytes;
    ctx->telemetry.kv_cache_resident_bytes += c.bytes;
    std::memset(out, 0, sizeof(*out));
    qwn_cuda_abi_header_init(&out->header, sizeof(*out));
    out->opaque = rk;
    return QWN_CUDA_STATUS_OK;
}

QWN_CUDA_ABI_API int qwn_cuda_abi_kv_cache_destroy(QwnCudaContextHandle *handle, QwnCudaKvCacheHandle *h) {
    Context *ctx = context_of(handle);
    if (!ctx || !h) {
        set_error("invalid KV-cache destroy request");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    std::lock_guard<std::mutex> lock(ctx->mutex);
    ResidentKv *rk = cache_of(ctx, *h);
    if (!rk) {
        set_error("KV-cache handle is not resident in this context");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    const uint64_t bytes = rk->c.bytes;
    ctx->caches.erase(std::find(ctx->caches.begin(), ctx->caches.end(), rk));
    free_cache(rk);
    ctx->resident -= std::min(ctx->resident, bytes);
    ctx->telemetry.kv_cache_resident_bytes -= std::min(ctx->telemetry.kv_cache_resident_bytes, bytes);
    h->opaque = nullptr;
    return QWN_CUDA_STATUS_OK;
}

QWN_CUDA_ABI_API int qwn_cuda_abi_kv_cache_append(QwnCudaContextHandle *handle,
                                                  const QwnCudaKvAppendRequest *r,
                                                  QwnCudaTelemetry *telemetry) {
    Context *ctx = context_of(handle);
    if (!ctx || !r || !header_ok(*r) || !r->host_key || !r->host_value) {
        set_error("invalid Q8 KV-cache append request");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    std::lock_guard<std::mutex> lock(ctx->mutex);
    ResidentKv *rk = cache_of(ctx, r->cache);
    if (!rk || r->n_channels != rk->c.channels || r->token != rk->c.tokens || r->token >= rk->c.max_tokens) {
        set_error("invalid Q8 KV-cache append request");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    KvCache &c = rk->c;
    hipError_t e = hipSetDevice(ctx->device);
    if (e != hipSuccess) return hip_fail("hipSetDevice", e);
    const size_t bytes = static_cast<size_t>(c.channels) * sizeof(float);
    if ((e = ctx->host_in.ensure(2 * bytes)) != hipSuccess)
        return hip_fail("KV workspace allocation", e, QWN_CUDA_STATUS_OUT_OF_MEMORY);
    const auto t0 = std::chrono::steady_clock::now();
    // the quantize kernel reads K and V straight from the pinned staging buffer
    uint8_t *hin = static_cast<uint8_t *>(ctx->host_in.ptr);
    std::memcpy(hin, r->host_key, bytes);
    std::memcpy(hin + bytes, r->host_value, bytes);
    const float *dk = reinterpret_cast<const float *>(hin);
    const float *dv = reinterpret_cast<const float *>(hin + bytes);
    (void)hipEventRecord(ctx->ev_start, ctx->stream);
    if ((e = qwn::launch_kv_append(c, dk, dv, c.tokens, ctx->stream)) != hipSuccess)
        return hip_fail("Q8 KV quantize launch", e);
    (void)hipEventRecord(ctx->ev_end, ctx->stream);
    if ((e = hipStreamSynchronize(ctx->stream)) != hipSuccess) return hip_fail("Q8 KV quantize", e);
    float kms = 0.0f;
    if (hipEventElapsedTime(&kms, ctx->ev_start, ctx->ev_end) != hipSuccess) kms = 0.0f;
    c.tokens++;
    QwnCudaTelemetry &tm = ctx->telemetry;
    tm.kv_cache_kernel_count += 2;  // one quantization each for K and V (one fused launch)
    tm.kv_cache_upload_bytes += 2 * bytes;
    tm.kv_cache_kernel_ms += kms;
    tm.kv_cache_transfer_ms += ms_since(t0) - kms;
    std::snprintf(tm.kv_cache_kernel_type, sizeof(tm.kv_cache_kernel_type), "q8-paged-gfx950");
    copy_telemetry(ctx, telemetry);
    return QWN_CUDA_STATUS_OK;
}

QWN_CUDA_ABI_API int qwn_cuda_abi_kv_cache_attention(QwnCudaContextHandle *handle,
                                                     const QwnCudaKvAttentionRequest *r,
                                                     QwnCudaTelemetry *telemetry) {
    Context *ctx = context_of(handle);
    if (!ctx || !r || !header_ok(*r) || !r->host_query || !r->host_output || r->query_heads == 0) {
        set_error("invalid Q8 KV-cache attention request");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    std::lock_guard<std::mutex> lock(ctx->mutex);
    ResidentKv *rk = cache_of(ctx, r->cache);
    // any query/KV head ratio: query head h reads KV head h * kv_heads / query_heads
    // (c/cuda/qwn_hypervsq2_cuda_abi.cu:184)
    if (!rk || r->kv_heads != rk->c.kv_heads || r->head_dim != rk->c.head_dim || r->position >= rk->c.tokens) {
        set_error("invalid Q8 KV-cache attention request");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    const KvCache &c = rk->c;
    hipError_t e = hipSetDevice(ctx->device);
    if (e != hipSuccess) return hip_fail("hipSetDevice", e);
    const size_t qbytes = static_cast<size_t>(r->query_heads) * c.head_dim * sizeof(float);
    const size_t work = qwn::attention_workspace_floats(c, r->query_heads, r->position) * sizeof(float);
    if ((e = ctx->host_in.ensure(qbytes)) != hipSuccess || (e = ctx->host_out.ensure(qbytes)) != hipSuccess ||
        (e = ctx->dev_work.ensure(work)) != hipSuccess)
        return hip_fail("attention workspace allocation", e, QWN_CUDA_STATUS_OUT_OF_MEMORY);
    const auto t0 = std::chrono::steady_clock::now();
    // the kernels read the query from and write the output to the pinned
    // staging buffers directly (no copy-engine transfers around them)
    std::memcpy(ctx->host_in.ptr, r->host_query, qbytes);
    qwn::AttentionLaunch a{};
    a.cache = &c;
    a.query = static_cast<const float *>(ctx->host_in.ptr);
    a.output = static_cast<float *>(ctx->host_out.ptr);
    a.query_heads = r->query_heads;
    a.position = r->position;
    a.scale = r->scale;
    a.partials = static_cast<float *>(ctx->dev_work.ptr);
    (void)hipEventRecord(ctx->ev_start, ctx->stream);
    if ((e = qwn::launch_attention(a, ctx->stream)) != hipSuccess) return hip_fail("Q8 KV attention launch", e);
    (void)hipEventRecord(ctx->ev_end, ctx->stream);
    if ((e = hipStreamSynchronize(ctx->stream)) != hipSuccess) return hip_fail("Q8 KV attention", e);
    std::memcpy(r->host_output, ctx->host_out.ptr, qbytes);
    float kms = 0.0f;
    if (hipEventElapsedTime(&kms, ctx->ev_start, ctx->ev_end) != hipSuccess) kms = 0.0f;
    QwnCudaTelemetry &tm = ctx->telemetry;
    tm.kv_cache_kernel_count++;
    tm.kv_cache_kernel_ms += kms;
    tm.kv_cache_transfer_ms += ms_since(t0) - kms;
    std::snprintf(tm.kv_cache_kernel_type, sizeof(tm.kv_cache_kernel_type), "q8-paged-gfx950");
    copy_telemetry(ctx, telemetry);
    return QWN_CUDA_STATUS_OK;
}

QWN_CUDA_ABI_API int qwn_cuda_abi_kv_cache_reset(QwnCudaContextHandle *handle, QwnCudaKvCacheHandle *h) {
    Context *ctx = context_of(handle);
    if (!ctx || !h) {
        set_error("invalid KV-cache reset request");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    std::lock_guard<std::mutex> lock(ctx->mutex);
    ResidentKv *rk = cache_of(ctx, *h);
    if (!rk) {
        set_error("KV-cache handle is not resident in this context");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    rk->c.tokens = 0;
    return QWN_CUDA_STATUS_OK;
}

QWN_CUDA_ABI_API int qwn_cuda_abi_hypervsq2_gemv(QwnCudaContextHandle *handle, const QwnCudaGemmRequest *r,
                                                 QwnCudaTelemetry *telemetry) {
    Context *ctx = context_of(handle);
    if (!ctx || !r || r->batch != 1) {
        set_error("hypervsq2_gemv needs a context and batch == 1");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    std::lock_guard<std::mutex> lock(ctx->mutex);
    return execute_gemm(ctx, r, telemetry);
}

QWN_CUDA_ABI_API int qwn_cuda_abi_hypervsq2_gemm(QwnCudaContextHandle *handle, const QwnCudaGemmRequest *r,
                                                 QwnCudaTelemetry *telemetry) {
    Context *ctx = context_of(handle);
    if (!ctx) {
        set_error("invalid context handle");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    std::lock_guard<std::mutex> lock(ctx->mutex);
    return execute_gemm(ctx, r, telemetry);
}

QWN_CUDA_ABI_API int qwn_cuda_abi_synchronize(QwnCudaContextHandle *handle) {
    Context *ctx = context_of(handle);
    if (!ctx) {
        set_error("invalid context handle");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    (void)hipSetDevice(ctx->device);
    hipError_t e = hipStreamSynchronize(ctx->stream);
    return e == hipSuccess ? QWN_CUDA_STATUS_OK : hip_fail("stream synchronize", e);
}

QWN_CUDA_ABI_API int qwn_cuda_abi_get_telemetry(QwnCudaContextHandle *handle, QwnCudaTelemetry *telemetry) {
    Context *ctx = context_of(handle);
    if (!ctx || !telemetry || !header_ok(*telemetry)) {
        set_error("invalid telemetry request");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    std::lock_guard<std::mutex> lock(ctx->mutex);
    *telemetry = ctx->telemetry;
    return QWN_CUDA_STATUS_OK;
}

QWN_CUDA_ABI_API int qwn_cuda_abi_last_error(char *buffer, uint32_t size) {
    if (!buffer || size == 0) return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    std::lock_guard<std::mutex> lock(g_error_mutex);
    std::snprintf(buffer, size, "%s", g_last_error.c_str());
    return QWN_CUDA_STATUS_OK;
}

// ---- extensions (qwn_hip_ext.h) --------------------------------------------

QWN_CUDA_ABI_API int qwn_hip_ext_tensor_info(const QwnCudaTensorHandle *h, QwnHipTensorInfo *info) {
    if (!h || !header_ok(*h) || !h->opaque || !info || !header_ok(*info)) {
        set_error("invalid tensor info request");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    const ResidentTensor *rt = static_cast<const ResidentTensor *>(h->opaque);
    const DeviceTensor &t = rt->t;
    std::memset(info, 0, sizeof(*info));
    qwn_cuda_abi_header_init(&info->header, sizeof(*info));
    info->dtype = t.kind == qwn::kHvsq2 ? QWN_CUDA_TENSOR_HYPERVSQ2_74
                  : t.kind == qwn::kQ4_0 ? QWN_CUDA_TENSOR_Q4_0_18
                  : t.bf16               ? QWN_CUDA_TENSOR_BF16
                                         : QWN_CUDA_TENSOR_F16;
    info->rows = t.rows;
    info->cols = t.cols;
    info->units_per_row = t.units;
    info->logical_bytes = t.logical_bytes;
    info->device_bytes = t.device_bytes;
    info->lanes_per_row = t.lanes;
    info->units_per_lane = t.upl;
    info->rows_per_wave = t.rows_per_wave;
    info->grid = static_cast<uint32_t>(qwn::plan_gemv(t, 1).grid);
    info->mfma_copy_bytes = rt->copy_bytes;
    return QWN_CUDA_STATUS_OK;
}

QWN_CUDA_ABI_API uint64_t qwn_hip_ext_activation_image_bytes(const QwnCudaTensorHandle *h) {
    if (!h || !header_ok(*h) || !h->opaque) return 0;
    const DeviceTensor &t = static_cast<const ResidentTensor *>(h->opaque)->t;
    return qwn::image_bytes(t.kind, t.units);
}

namespace {
// Tensor of a handle issued by this context (lock held by the caller).
ResidentTensor *ext_tensor(Context *ctx, const QwnCudaTensorHandle *h) {
    return h ? tensor_of(ctx, *h) : nullptr;
}
}  // namespace

QWN_CUDA_ABI_API int qwn_hip_ext_prepare_image_device(QwnCudaContextHandle *handle, const QwnCudaTensorHandle *th,
                                                      const void *x, uint32_t batch, uint32_t x_stride,
                                                      void *image, uint32_t image_stride, void *stream) {
    Context *ctx = context_of(handle);
    if (!ctx || !x || !image || batch == 0) {
        set_error("invalid image request");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    std::lock_guard<std::mutex> lock(ctx->mutex);
    ResidentTensor *rt = ext_tensor(ctx, th);
    if (!rt || x_stride < rt->t.cols || image_stride < qwn::image_bytes(rt->t.kind, rt->t.units) ||
        (image_stride & 15u) || (reinterpret_cast<uintptr_t>(image) & 15u)) {
        set_error("image request does not fit the tensor (strides, 16-byte alignment)");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    hipStream_t s = stream ? static_cast<hipStream_t>(stream) : ctx->stream;
    hipError_t e = qwn::launch_image(rt->t, x, batch, x_stride, static_cast<uint8_t *>(image), image_stride, s);
    return e == hipSuccess ? QWN_CUDA_STATUS_OK : hip_fail("image launch", e);
}

QWN_CUDA_ABI_API int qwn_hip_ext_quantize_image_device(QwnCudaContextHandle *handle,
                                                       const QwnCudaTensorHandle *th, const float *x,
                                                       uint32_t batch, uint32_t x_stride, void *image,
                                                       uint32_t image_stride, float *scales, int8_t *q8,
                                                       uint32_t q8_stride, void *stream) {
    Context *ctx = context_of(handle);
    if (!ctx || !x || !image || !scales || batch == 0) {
        set_error("invalid quantize-image request");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    std::lock_guard<std::mutex> lock(ctx->mutex);
    ResidentTensor *rt = ext_tensor(ctx, th);
    if (!rt || rt->t.kind == qwn::kF16 || x_stride < rt->t.cols ||
        image_stride < qwn::image_bytes(rt->t.kind, rt->t.units) || (image_stride & 15u) ||
        (reinterpret_cast<uintptr_t>(image) & 15u) || (q8 && q8_stride < rt->t.cols)) {
        set_error("quantize-image request does not fit the tensor");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    hipStream_t s = stream ? static_cast<hipStream_t>(stream) : ctx->stream;
    hipError_t e = qwn::launch_quantize_image(rt->t, x, batch, x_stride, static_cast<uint8_t *>(image),
                                              image_stride, scales, q8, q8_stride, s);
    return e == hipSuccess ? QWN_CUDA_STATUS_OK : hip_fail("quantize-image launch", e);
}

QWN_CUDA_ABI_API int qwn_hip_ext_gemm_image_device(QwnCudaContextHandle *handle, const QwnCudaTensorHandle *th,
                                                   const void *image, uint32_t image_stride,
                                                   const float *scales, float scale, float *output,
                                                   uint32_t batch, uint32_t output_stride, void *stream) {
    Context *ctx = context_of(handle);
    if (!ctx || !image || !output || batch == 0) {
        set_error("invalid image GEMV request");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    std::lock_guard<std::mutex> lock(ctx->mutex);
    ResidentTensor *rt = ext_tensor(ctx, th);
    if (!rt || image_stride < qwn::image_bytes(rt->t.kind, rt->t.units) || (image_stride & 15u) ||
        (reinterpret_cast<uintptr_t>(image) & 15u) || (output_stride && output_stride < rt->t.rows)) {
        set_error("image GEMV request does not fit the tensor");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    qwn::GemvLaunch g{};
    g.tensor = &rt->t;
    g.image = image;
    g.image_stride = image_stride;
    g.scales = scales;
    g.scale = scale;
    g.output = output;
    g.batch = batch;
    g.output_stride = output_stride ? output_stride : rt->t.rows;
    hipStream_t s = stream ? static_cast<hipStream_t>(stream) : ctx->stream;
    hipError_t e = qwn::launch_gemv(g, s);
    if (e != hipSuccess) return hip_fail("image GEMV launch", e);
    ctx->telemetry.gpu_matmul_count++;
    ctx->telemetry.gpu_kernel_launch_count++;
    ctx->telemetry.gpu_projection_count++;
    return QWN_CUDA_STATUS_OK;
}

namespace {
// Translates a group request (context lock held); false with the error set.
bool group_of(Context *ctx, const QwnHipGemvGroupRequest *r, qwn::GemvGroupLaunch &g) {
    if (!r || !header_ok(*r) || !r->tensors || !r->outputs || r->count == 0 || r->count > QWN_HIP_GEMV_MAX_GROUP ||
        r->input_mode > QWN_HIP_GEMV_INPUT_SWIGLU || r->output_mode > QWN_HIP_GEMV_OUTPUT_SWIGLU) {
        set_error("invalid grouped GEMV request");
        return false;
    }
    g = qwn::GemvGroupLaunch();
    g.njobs = static_cast<int>(r->count);
    for (uint32_t i = 0; i < r->count; ++i) {
        ResidentTensor *rt = tensor_of(ctx, r->tensors[i]);
        if (!rt || !r->outputs[i]) {
            set_error("grouped GEMV: unknown tensor handle or null output %u", i);
            return false;
        }
        g.tensors[i] = &rt->t;
        g.outputs[i] = r->outputs[i];
    }
    g.input_mode = r->input_mode;
    g.output_mode = r->output_mode;
    g.batch = r->input_mode == QWN_HIP_GEMV_INPUT_IMAGE ? r->batch : 1u;
    g.image = r->image;
    g.image_stride = r->image_stride;
    g.scales = r->scales;
    g.scale = r->scale;
    g.x = r->x;
    g.x2 = r->x2;
    g.norm = r->norm;
    g.eps = r->eps;
    g.scale_out = r->scale_out;
    g.argmax_partials = r->argmax_partials;
    for (uint32_t i = 0; i < r->count; ++i) g.output_stride[i] = r->output_stride;  // 0: each tensor's rows
    const qwn::DeviceTensor &t0 = *g.tensors[0];
    if (r->input_mode == QWN_HIP_GEMV_INPUT_IMAGE &&
        (r->batch == 0 || r->image_stride < qwn::image_bytes(t0.kind, t0.units) || (r->image_stride & 15u) ||
         (reinterpret_cast<uintptr_t>(r->image) & 15u))) {
        set_error("grouped GEMV: image does not fit the tensors (strides, 16-byte alignment)");
        return false;
    }
    if (r->input_mode != QWN_HIP_GEMV_INPUT_IMAGE &&
        ((reinterpret_cast<uintptr_t>(r->x) & 15u) || (reinterpret_cast<uintptr_t>(r->x2) & 15u) ||
         (reinterpret_cast<uintptr_t>(r->norm) & 15u))) {
        set_error("grouped GEMV: fp32 inputs must be 16-byte aligned");
        return false;
    }
    for (uint32_t i = 0; i < r->count; ++i)
        if (r->output_stride && r->output_stride < g.tensors[i]->rows) {
            set_error("grouped GEMV: output stride below the rows of tensor %u", i);
            return false;
        }
    if (qwn::gemv_group_grid(g) == 0) {
        set_error("grouped GEMV: tensors differ in dtype/columns, or the mode does not fit them "
                  "(fp32 input needs one token and columns a multiple of 32; SwiGLU output needs two "
                  "tensors of one shape)");
        return false;
    }
    return true;
}
}  // namespace

QWN_CUDA_ABI_API uint32_t qwn_hip_ext_gemv_group_partials(QwnCudaContextHandle *handle,
                                                          const QwnHipGemvGroupRequest *r) {
    Context *ctx = context_of(handle);
    if (!ctx) return 0;
    std::lock_guard<std::mutex> lock(ctx->mutex);
    qwn::GemvGroupLaunch g;
    if (!group_of(ctx, r, g)) return 0;
    return qwn::gemv_group_grid(g);
}

QWN_CUDA_ABI_API int qwn_hip_ext_gemv_group_device(QwnCudaContextHandle *handle, const QwnHipGemvGroupRequest *r,
                                                   void *stream) {
    Context *ctx = context_of(handle);
    if (!ctx) {
        set_error("invalid context handle");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    std::lock_guard<std::mutex> lock(ctx->mutex);
    qwn::GemvGroupLaunch g;
    if (!group_of(ctx, r, g)) return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    hipStream_t s = stream ? static_cast<hipStream_t>(stream) : ctx->stream;
    hipError_t e = qwn::launch_gemv_group(g, s);
    if (e != hipSuccess) return hip_fail("grouped GEMV launch", e);
    ctx->telemetry.gpu_matmul_count += r->count;
    ctx->telemetry.gpu_kernel_launch_count++;
    ctx->telemetry.gpu_projection_count += r->count;
    return QWN_CUDA_STATUS_OK;
}

QWN_CUDA_ABI_API int qwn_hip_ext_argmax_device(QwnCudaContextHandle *handle, const uint64_t *partials,
                                               uint32_t count, int32_t *index, void *stream) {
    Context *ctx = context_of(handle);
    if (!ctx || !partials || !index || count == 0) {
        set_error("invalid argmax request");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    hipStream_t s = stream ? static_cast<hipStream_t>(stream) : ctx->stream;
    hipError_t e = qwn::launch_argmax_finish(partials, count, index, s);
    return e == hipSuccess ? QWN_CUDA_STATUS_OK : hip_fail("argmax launch", e);
}

QWN_CUDA_ABI_API uint64_t qwn_hip_ext_mfma_image_bytes(const QwnCudaTensorHandle *h) {
    if (!h || !header_ok(*h) || !h->opaque) return 0;
    const DeviceTensor &t = static_cast<const ResidentTensor *>(h->opaque)->t;
    return qwn::mfma_image_bytes(t);
}

QWN_CUDA_ABI_API int qwn_hip_ext_mfma_image_device(QwnCudaContextHandle *handle, const QwnCudaTensorHandle *th,
                                                   const int8_t *q8, uint32_t batch, uint32_t q8_stride,
                                                   void *image, void *stream) {
    Context *ctx = context_of(handle);
    if (!ctx || !q8 || !image || batch == 0 || batch > 16) {
        set_error("invalid MFMA image request");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    std::lock_guard<std::mutex> lock(ctx->mutex);
    ResidentTensor *rt = ext_tensor(ctx, th);
    if (!rt || (rt->t.kind != qwn::kHvsq2 && rt->t.kind != qwn::kQ4_0) || q8_stride < rt->t.cols ||
        (reinterpret_cast<uintptr_t>(image) & 15u)) {
        set_error("MFMA image request does not fit the tensor (HyperVSQ-2 or Q4_0)");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    hipStream_t s = stream ? static_cast<hipStream_t>(stream) : ctx->stream;
    hipError_t e = qwn::launch_mfma_image(rt->t, q8, batch, q8_stride, static_cast<uint8_t *>(image), s);
    return e == hipSuccess ? QWN_CUDA_STATUS_OK : hip_fail("MFMA image launch", e);
}

QWN_CUDA_ABI_API int qwn_hip_ext_gemm_mfma_device(QwnCudaContextHandle *handle, const QwnCudaTensorHandle *th,
                                                  const void *image, const float *scales, float *output,
                                                  uint32_t batch, uint32_t output_stride, void *stream) {
    Context *ctx = context_of(handle);
    if (!ctx || !image || !scales || !output || batch == 0 || batch > 16) {
        set_error("invalid MFMA GEMM request");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    std::lock_guard<std::mutex> lock(ctx->mutex);
    ResidentTensor *rt = ext_tensor(ctx, th);
    if (!rt || (rt->t.kind != qwn::kHvsq2 && rt->t.kind != qwn::kQ4_0) ||
        (output_stride && output_stride < rt->t.rows)) {
        set_error("MFMA GEMM request does not fit the tensor (HyperVSQ-2 or Q4_0)");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    hipStream_t s = stream ? static_cast<hipStream_t>(stream) : ctx->stream;
    hipError_t e = qwn::launch_gemm_mfma(rt->t, static_cast<const uint8_t *>(image), scales, output, batch,
                                         output_stride, s);
    if (e != hipSuccess) return hip_fail("MFMA GEMM launch", e);
    ctx->telemetry.gpu_matmul_count++;
    ctx->telemetry.gpu_kernel_launch_count++;
    ctx->telemetry.gpu_projection_count++;
    return QWN_CUDA_STATUS_OK;
}

QWN_CUDA_ABI_API int qwn_hip_ext_gemm_mfma_group_device(QwnCudaContextHandle *handle,
                                                        const QwnCudaTensorHandle *tensors, uint32_t count,
                                                        const void *image, const float *scales,
                                                        float *const *outputs, uint32_t batch,
                                                        uint32_t output_stride, uint32_t accumulate,
                                                        void *stream) {
    Context *ctx = context_of(handle);
    if (!ctx || !tensors || !outputs || !image || !scales || count == 0 || count > qwn::kMaxGroup || batch == 0 ||
        batch > 16 || (reinterpret_cast<uintptr_t>(image) & 15u)) {
        set_error("invalid MFMA group GEMM request");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    std::lock_guard<std::mutex> lock(ctx->mutex);
    const DeviceTensor *ts[qwn::kMaxGroup] = {};
    uint32_t strides[qwn::kMaxGroup] = {};
    for (uint32_t i = 0; i < count; ++i) {
        ResidentTensor *rt = ext_tensor(ctx, &tensors[i]);
        if (!rt || (rt->t.kind != qwn::kHvsq2 && rt->t.kind != qwn::kQ4_0) || !outputs[i] ||
            (output_stride && output_stride < rt->t.rows) ||
            (i > 0 && (rt->t.cols != ts[0]->cols || rt->t.kind != ts[0]->kind))) {
            set_error("MFMA group GEMM tensor %u does not fit (HyperVSQ-2 or Q4_0, one kind, equal columns, "
                      "output stride)", i);
            return QWN_CUDA_STATUS_INVALID_ARGUMENT;
        }
        ts[i] = &rt->t;
        strides[i] = output_stride;
    }
    hipStream_t s = stream ? static_cast<hipStream_t>(stream) : ctx->stream;
    hipError_t e = qwn::launch_gemm_mfma_group(ts, outputs, count, static_cast<const uint8_t *>(image), scales, batch,
                                               strides, s, accumulate != 0);
    if (e != hipSuccess) return hip_fail("MFMA group GEMM launch", e);
    ctx->telemetry.gpu_matmul_count += count;
    ctx->telemetry.gpu_kernel_launch_count++;
    ctx->telemetry.gpu_projection_count += count;
    return QWN_CUDA_STATUS_OK;
}

namespace {

uint64_t fnv1a64(const char *s) {
    uint64_t h = 0xcbf29ce484222325ull;  // FNV-1a 64 offset basis
    for (; *s; ++s) {
        h ^= static_cast<uint8_t>(*s);
        h *= 0x100000001b3ull;  // FNV-1a 64 prime
    }
    return h;
}

// Placement priority of a tensor name (c/qwanto_native.c:379-389).
uint8_t name_priority(const char *n) {
    auto has = [n](const char *p) { return std::strstr(n, p) != nullptr; };
    if (has("embed") || has("lm_head")) return 255;
    if (has("norm")) return 245;
    if (has("q_proj") || has("k_proj") || has("v_proj") || has("o_proj") || has("attn")) return 230;
    if (has("gate") && !has("expert")) return 210;
    if (has("expert")) return 80;
    return 160;
}

}  // namespace

QWN_CUDA_ABI_API int qwn_hip_ext_plan_residency(QwnCudaContextHandle *handle, const char *const *names,
                                                const uint64_t *byte_offsets, const uint64_t *byte_sizes,
                                                uint32_t count, uint64_t gpu_budget, uint64_t ram_budget,
                                                QwnHipPlacement *items, uint64_t *totals) {
    if (!names || !byte_offsets || !byte_sizes || !items || !totals || (count && !names)) {
        set_error("invalid residency plan request");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    for (uint32_t i = 0; i < count; ++i)
        if (!names[i]) {
            set_error("tensor %u has no name", i);
            return QWN_CUDA_STATUS_INVALID_ARGUMENT;
        }
    if (gpu_budget == QWN_HIP_GPU_BUDGET_AUTO) {
        Context *ctx = context_of(handle);
        if (!ctx) {
            set_error("an automatic GPU budget needs a context");
            return QWN_CUDA_STATUS_INVALID_ARGUMENT;
        }
        std::lock_guard<std::mutex> lock(ctx->mutex);
        size_t free_b = 0, total_b = 0;
        hipError_t e = hipSetDevice(ctx->device);
        if (e == hipSuccess) e = hipMemGetInfo(&free_b, &total_b);
        if (e != hipSuccess) return hip_fail("device memory query", e);
        gpu_budget = static_cast<uint64_t>(static_cast<double>(free_b) * 0.90);
        if (ctx->budget) gpu_budget = std::min(gpu_budget, ctx->budget - std::min(ctx->budget, ctx->resident));
    }
    for (uint32_t i = 0; i < count; ++i) {
        QwnHipPlacement &p = items[i];
        std::memset(&p, 0, sizeof(p));
        p.name_hash = fnv1a64(names[i]);
        p.byte_offset = byte_offsets[i];
        p.byte_size = byte_sizes[i];
        p.tensor_index = i;
        p.priority = name_priority(names[i]);
        p.tier = QWN_HIP_TIER_FILE;
    }
    // a total order (priority desc, size asc, index asc): any sort gives the
    // reference's qsort result
    std::sort(items, items + count, [](const QwnHipPlacement &x, const QwnHipPlacement &y) {
        if (x.priority != y.priority) return x.priority > y.priority;
        if (x.byte_size != y.byte_size) return x.byte_size < y.byte_size;
        return x.tensor_index < y.tensor_index;
    });
    uint64_t gpu = 0, ram = 0, file = 0;
    for (uint32_t i = 0; i < count; ++i) {
        QwnHipPlacement &p = items[i];
        if (gpu <= gpu_budget && p.byte_size <= gpu_budget - gpu) {
            p.tier = QWN_HIP_TIER_GPU;
            gpu += p.byte_size;
        } else if (ram <= ram_budget && p.byte_size <= ram_budget - ram) {
            p.tier = QWN_HIP_TIER_RAM;
            ram += p.byte_size;
        } else {
            p.tier = QWN_HIP_TIER_FILE;
            file += p.byte_size;
        }
    }
    totals[0] = gpu;
    totals[1] = ram;
    totals[2] = file;
    return QWN_CUDA_STATUS_OK;
}

QWN_CUDA_ABI_API int qwn_hip_ext_quantize_device(QwnCudaContextHandle *handle, const float *x, uint32_t batch,
                                                 uint32_t cols, uint32_t x_stride, int8_t *q8,
                                                 uint32_t q8_stride, float *scales, void *stream) {
    Context *ctx = context_of(handle);
    if (!ctx || !x || !q8 || !scales || batch == 0 || cols == 0 || x_stride < cols || q8_stride < cols) {
        set_error("invalid device quantize request");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    hipStream_t s = stream ? static_cast<hipStream_t>(stream) : ctx->stream;
    DeviceTensor shape;  // only the padding width matters without an image
    shape.kind = qwn::kHvsq2;
    shape.cols = cols;
    shape.units = (cols + 255u) / 256u;
    hipError_t e = qwn::launch_quantize_image(shape, x, batch, x_stride, nullptr, 0, scales, q8, q8_stride, s);
    return e == hipSuccess ? QWN_CUDA_STATUS_OK : hip_fail("quantize launch", e);
}

QWN_CUDA_ABI_API int qwn_hip_ext_kv_append_device(QwnCudaContextHandle *handle, QwnCudaKvCacheHandle *h,
                                                  const float *keys, const float *values, uint32_t count,
                                                  void *stream) {
    Context *ctx = context_of(handle);
    if (!ctx || !h || !keys || !values || count == 0) {
        set_error("invalid device KV append request");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    std::lock_guard<std::mutex> lock(ctx->mutex);
    ResidentKv *rk = cache_of(ctx, *h);
    if (!rk || rk->c.tokens + count > rk->c.max_tokens) {
        set_error("device KV append exceeds the cache");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    hipStream_t s = stream ? static_cast<hipStream_t>(stream) : ctx->stream;
    KvCache &c = rk->c;
    hipError_t e = qwn::launch_kv_append(c, keys, values, c.tokens, s, count);
    if (e != hipSuccess) return hip_fail("device KV append launch", e);
    c.tokens += count;
    // launches issued (one per 32768 tokens), counted twice as the ABI
    // append counts its one fused K and V launch
    ctx->telemetry.kv_cache_kernel_count += 2ull * ((count + 32767u) / 32768u);
    return QWN_CUDA_STATUS_OK;
}

QWN_CUDA_ABI_API uint64_t qwn_hip_ext_attention_workspace_bytes(QwnCudaKvCacheHandle *h, uint32_t query_heads,
                                                                 uint32_t position) {
    if (!h || !header_ok(*h) || !h->opaque) return 0;
    const KvCache &c = static_cast<ResidentKv *>(h->opaque)->c;
    return qwn::attention_workspace_floats(c, query_heads, position) * sizeof(float);
}

QWN_CUDA_ABI_API int qwn_hip_ext_kv_attention_device(QwnCudaContextHandle *handle, QwnCudaKvCacheHandle *h,
                                                     const float *query, float *output, uint32_t query_heads,
                                                     uint32_t position, float scale, void *workspace,
                                                     void *stream) {
    Context *ctx = context_of(handle);
    if (!ctx || !h || !query || !output || !workspace || query_heads == 0) {
        set_error("invalid device attention request");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    std::lock_guard<std::mutex> lock(ctx->mutex);
    ResidentKv *rk = cache_of(ctx, *h);
    if (!rk || position >= rk->c.tokens) {
        set_error("invalid device attention request");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    qwn::AttentionLaunch a{};
    a.cache = &rk->c;
    a.query = query;
    a.output = output;
    a.query_heads = query_heads;
    a.position = position;
    a.scale = scale;
    a.partials = static_cast<float *>(workspace);
    hipStream_t s = stream ? static_cast<hipStream_t>(stream) : ctx->stream;
    hipError_t e = qwn::launch_attention(a, s);
    if (e != hipSuccess) return hip_fail("device attention launch", e);
    ctx->telemetry.kv_cache_kernel_count++;
    return QWN_CUDA_STATUS_OK;
}

QWN_CUDA_ABI_API int qwn_hip_ext_debug_int_sums(QwnCudaContextHandle *handle, const QwnCudaTensorHandle *th,
                                                const int8_t *host_q8, int32_t *host_out,
                                                uint64_t out_capacity) {
    Context *ctx = context_of(handle);
    if (!ctx || !th || !host_q8 || !host_out) {
        set_error("invalid debug request");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    std::lock_guard<std::mutex> lock(ctx->mutex);
    ResidentTensor *rt = tensor_of(ctx, *th);
    if (!rt || rt->t.kind == qwn::kF16) {
        set_error("debug sums need a resident HyperVSQ-2 or Q4_0 tensor");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    const DeviceTensor &t = rt->t;
    const uint64_t per_row = t.kind == qwn::kHvsq2 ? t.units * 8ull : (t.cols + 31ull) / 32ull;
    const uint64_t n = per_row * t.rows;
    if (out_capacity < n) {
        set_error("debug output needs %llu int32 values", static_cast<unsigned long long>(n));
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    hipError_t e = hipSetDevice(ctx->device);
    const uint32_t stride = (t.cols + 255u) & ~255u;
    const size_t img = qwn::image_bytes(t.kind, t.units);
    void *dx = nullptr, *dimg = nullptr, *dout = nullptr;
    if (e == hipSuccess) e = hipMalloc(&dx, stride);
    if (e == hipSuccess) e = hipMalloc(&dimg, img);
    if (e == hipSuccess) e = hipMalloc(&dout, n * sizeof(int32_t));
    if (e == hipSuccess) e = hipMemsetAsync(dx, 0, stride, ctx->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(dx, host_q8, t.cols, hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess)
        e = qwn::launch_image(t, dx, 1, stride, static_cast<uint8_t *>(dimg), static_cast<uint32_t>(img), ctx->stream);
    if (e == hipSuccess) {
        qwn::GemvLaunch g{};
        g.tensor = &t;
        g.image = dimg;
        g.image_stride = static_cast<uint32_t>(img);
        g.batch = 1;
        g.debug_sums = static_cast<int32_t *>(dout);
        e = qwn::launch_gemv(g, ctx->stream);
    }
    if (e == hipSuccess)
        e = hipMemcpyAsync(host_out, dout, n * sizeof(int32_t), hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (dx) (void)hipFree(dx);
    if (dimg) (void)hipFree(dimg);
    if (dout) (void)hipFree(dout);
    return e == hipSuccess ? QWN_CUDA_STATUS_OK : hip_fail("debug integer sums", e);
}

QWN_CUDA_ABI_API int qwn_hip_ext_debug_mfma_int_sums(QwnCudaContextHandle *handle, const QwnCudaTensorHandle *th,
                                                     const int8_t *host_q8, uint32_t batch, int32_t *host_out,
                                                     uint64_t out_capacity) {
    Context *ctx = context_of(handle);
    if (!ctx || !th || !host_q8 || !host_out || batch == 0 || batch > 16) {
        set_error("invalid MFMA debug request");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    std::lock_guard<std::mutex> lock(ctx->mutex);
    ResidentTensor *rt = tensor_of(ctx, *th);
    if (!rt || rt->t.kind == qwn::kF16) {
        set_error("MFMA debug sums need a resident HyperVSQ-2 or Q4_0 tensor");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    const DeviceTensor &t = rt->t;
    const uint64_t nblk = t.kind == qwn::kHvsq2 ? t.units : (t.cols + 31ull) / 32ull;
    const uint64_t n = static_cast<uint64_t>(batch) * t.rows * nblk;
    if (out_capacity < n) {
        set_error("MFMA debug output needs %llu int32 values", static_cast<unsigned long long>(n));
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    hipError_t e = hipSetDevice(ctx->device);
    const uint32_t stride = (t.cols + 255u) & ~255u;
    const size_t img = qwn::mfma_image_bytes(t);
    void *dx = nullptr, *dimg = nullptr, *dout = nullptr, *dy = nullptr, *dsc = nullptr;
    if (e == hipSuccess) e = hipMalloc(&dx, static_cast<size_t>(stride) * batch);
    if (e == hipSuccess) e = hipMalloc(&dimg, img);
    if (e == hipSuccess) e = hipMalloc(&dout, n * sizeof(int32_t));
    if (e == hipSuccess) e = hipMalloc(&dy, static_cast<size_t>(batch) * t.rows * sizeof(float));
    if (e == hipSuccess) e = hipMalloc(&dsc, 16 * sizeof(float));
    if (e == hipSuccess) e = hipMemsetAsync(dx, 0, static_cast<size_t>(stride) * batch, ctx->stream);
    if (e == hipSuccess) e = hipMemsetAsync(dsc, 0, 16 * sizeof(float), ctx->stream);
    if (e == hipSuccess)
        e = hipMemcpy2DAsync(dx, stride, host_q8, t.cols, t.cols, batch, hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess)
        e = qwn::launch_mfma_image(t, static_cast<const int8_t *>(dx), batch, stride, static_cast<uint8_t *>(dimg),
                                   ctx->stream);
    if (e == hipSuccess) {
        const DeviceTensor *ts[1] = {&t};
        float *outs[1] = {static_cast<float *>(dy)};
        e = qwn::launch_gemm_mfma_group(ts, outs, 1, static_cast<const uint8_t *>(dimg),
                                        static_cast<const float *>(dsc), batch, nullptr, ctx->stream, false,
                                        static_cast<int32_t *>(dout));
    }
    if (e == hipSuccess)
        e = hipMemcpyAsync(host_out, dout, n * sizeof(int32_t), hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    for (void *p : {dx, dimg, dout, dy, dsc})
        if (p) (void)hipFree(p);
    return e == hipSuccess ? QWN_CUDA_STATUS_OK : hip_fail("MFMA debug integer sums", e);
}

QWN_CUDA_ABI_API int qwn_hip_ext_debug_kv_read(QwnCudaContextHandle *handle, const QwnCudaKvCacheHandle *h,
                                               uint32_t first, uint32_t count, int8_t *host_keys,
                                               int8_t *host_values, float *host_key_scales,
                                               float *host_value_scales) {
    Context *ctx = context_of(handle);
    if (!ctx || !h || !host_keys || !host_values || !host_key_scales || !host_value_scales || count == 0) {
        set_error("invalid KV debug read");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    std::lock_guard<std::mutex> lock(ctx->mutex);
    ResidentKv *rk = cache_of(ctx, *h);
    if (!rk || first > rk->c.tokens || count > rk->c.tokens - first) {
        set_error("KV debug read beyond the appended tokens");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    const KvCache &c = rk->c;
    const size_t vb = static_cast<size_t>(count) * c.channels, sb = static_cast<size_t>(count) * c.groups * 4;
    hipError_t e = hipSetDevice(ctx->device);
    void *dk = nullptr, *dv = nullptr, *dks = nullptr, *dvs = nullptr;
    if (e == hipSuccess) e = hipMalloc(&dk, vb);
    if (e == hipSuccess) e = hipMalloc(&dv, vb);
    if (e == hipSuccess) e = hipMalloc(&dks, sb);
    if (e == hipSuccess) e = hipMalloc(&dvs, sb);
    if (e == hipSuccess)
        e = qwn::launch_kv_gather(c, first, count, static_cast<int8_t *>(dk), static_cast<int8_t *>(dv),
                                  static_cast<float *>(dks), static_cast<float *>(dvs), ctx->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(host_keys, dk, vb, hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(host_values, dv, vb, hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(host_key_scales, dks, sb, hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(host_value_scales, dvs, sb, hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    for (void *p : {dk, dv, dks, dvs})
        if (p) (void)hipFree(p);
    return e == hipSuccess ? QWN_CUDA_STATUS_OK : hip_fail("KV debug read", e);
}

}  // extern "C"

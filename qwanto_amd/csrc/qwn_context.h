// Host-side state of a qwn_hip context, shared by the ABI translation units
// (qwn_runtime.hip: the qwn_cuda ABI and the device-pointer extensions;
// qwn_decoder.hip: the resident decoder).
#pragma once

#include "qwn_cuda_abi.h"
#include "qwn_internal.h"

#include <algorithm>
#include <mutex>
#include <vector>

namespace qwn {

struct PinnedBuffer {
    void *ptr = nullptr;
    size_t bytes = 0;
    hipError_t ensure(size_t want) {
        if (want <= bytes) return hipSuccess;
        if (ptr) (void)hipHostFree(ptr);
        ptr = nullptr;
        bytes = 0;
        hipError_t e = hipHostMalloc(&ptr, want, hipHostMallocDefault);
        if (e == hipSuccess) bytes = want;
        return e;
    }
    void release() {
        if (ptr) (void)hipHostFree(ptr);
        ptr = nullptr;
        bytes = 0;
    }
};

struct DeviceBuffer {
    void *ptr = nullptr;
    size_t bytes = 0;
    hipError_t ensure(size_t want) {
        if (want <= bytes) return hipSuccess;
        if (ptr) (void)hipFree(ptr);
        ptr = nullptr;
        bytes = 0;
        hipError_t e = hipMalloc(&ptr, want);
        if (e == hipSuccess) bytes = want;
        return e;
    }
    void release() {
        if (ptr) (void)hipFree(ptr);
        ptr = nullptr;
        bytes = 0;
    }
};

struct ResidentTensor {
    DeviceTensor t;
    void *allocation = nullptr;
    void *mfma_allocation = nullptr;  // the MFMA-order copy (HyperVSQ-2, Q4_0), if any
    uint64_t copy_bytes = 0;          // its size, charged to the context like the tensor's own bytes
};

struct ResidentKv {
    KvCache c;
    void *allocation = nullptr;
};

struct Decoder;  // qwn_decoder.hip

// Weight upload pipeline: whole-row chunks of a host buffer are copied into
// one of two pinned slots while the other slot's DMA and repack run.
constexpr size_t kUploadSlotBytes = 32u << 20;
struct UploadPipe {
    PinnedBuffer host[2];
    DeviceBuffer dev[2];
    hipEvent_t done[2] = {nullptr, nullptr};
    bool pending[2] = {false, false};
    int next = 0;
};

struct Context {
    std::mutex mutex;
    int device = -1;
    uint64_t budget = 0;
    uint64_t resident = 0;  // bytes charged against the budget: tensors' logical bytes, their
                            // MFMA-order copies, Q8 KV caches (gpu_resident_bytes reports it)
    hipStream_t stream = nullptr;
    hipEvent_t ev_start = nullptr, ev_end = nullptr;
    PinnedBuffer host_in, host_out;
    DeviceBuffer dev_in, dev_out, dev_scales, dev_work, dev_img;
    std::vector<ResidentTensor *> tensors;
    std::vector<ResidentKv *> caches;
    std::vector<Decoder *> decoders;
    UploadPipe upload;
    QwnCudaTelemetry telemetry{};
};

// Process-wide last error (qwn_cuda_abi_last_error).
void set_error(const char *fmt, ...);
int hip_fail(const char *what, hipError_t e, int status = QWN_CUDA_STATUS_RUNTIME_ERROR);

template <typename T>
bool header_ok(const T &s) {
    return s.header.abi_version == QWN_CUDA_ABI_VERSION && s.header.struct_size >= sizeof(T);
}

Context *context_of(const QwnCudaContextHandle *h);
// Handles this context issued (lock held by the caller); null otherwise.
ResidentTensor *tensor_of(Context *ctx, const QwnCudaTensorHandle &h);
ResidentKv *cache_of(Context *ctx, const QwnCudaKvCacheHandle &h);

// Releases a decoder's device memory and graph (context lock held).
void destroy_decoder(Decoder *d);

}  // namespace qwn

// tms_chain.hip -- chained device-resident decode: the pieces that let n
// decode steps be enqueued at once, each step's sampled ids feeding the next
// step's embedding on the device while the host watches the ids land
// (gpu_chain_begin / gpu_chain_poll, tensormark/llama.h:6047-6130, and the
// token-slot peek, tensormark/metal.h:3216-3228).
//
//   * tms_token_slot: host memory the device writes (hipHostMalloc, mapped
//     and coherent), one int32 entry per (step, row), filled with a
//     sentinel; the host reads entries with acquire loads and never waits.
//   * tms_embed_gather: x[b][:] = table[tokens[b]][:] for the next step's
//     input, tokens read from device memory (the sampler's out_tokens), and
//     the same ids published into the slot by system-scope release stores:
//     the host sees each id once its store lands, while the later steps of
//     the chain keep running.  With table NULL it only publishes (the last
//     step of a chain).
//
// The model's forward pass between the gather and the sampler is the
// caller's (out of this library's scope).

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/tmsample_hip.h"
#include "tms_device.h"

struct tms_token_slot {
    int device;
    int capacity;
    int32_t* host;
    int32_t* dev;
};

namespace tms {

// One workgroup per row: 16-byte vectors of the row's embedding, then one
// lane publishes the id.
__global__ __launch_bounds__(256) void embed_gather_kernel(const uint8_t* table, int64_t rows, int64_t row_bytes,
                                                           const int32_t* tokens, uint8_t* x, int32_t* slot_out) {
    const int b = blockIdx.x;
    const int32_t id = tokens[b];
    if (table) {
        const bool ok = id >= 0 && (int64_t)id < rows;
        const uint4* src = (const uint4*)(table + (ok ? (int64_t)id : 0) * row_bytes);
        uint4* dst = (uint4*)(x + (int64_t)b * row_bytes);
        const int64_t nv = row_bytes / 16;
        for (int64_t i = threadIdx.x; i < nv; i += blockDim.x) dst[i] = ok ? src[i] : make_uint4(0, 0, 0, 0);
    }
    if (slot_out && threadIdx.x == 0)   // -1 is the slot's "pending": a row without a token is -2
        __hip_atomic_store(&slot_out[b], id >= 0 ? id : -2, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

}  // namespace tms

extern "C" tms_token_slot* tms_token_slot_create(int device, int capacity) {
    if (capacity <= 0) return nullptr;
    int prev = 0;
    if (hipGetDevice(&prev) != hipSuccess || hipSetDevice(device) != hipSuccess) return nullptr;
    auto* s = new tms_token_slot{device, capacity, nullptr, nullptr};
    bool ok = hipHostMalloc((void**)&s->host, sizeof(int32_t) * (size_t)capacity,
                            hipHostMallocMapped | hipHostMallocCoherent) == hipSuccess;
    ok = ok && hipHostGetDevicePointer((void**)&s->dev, s->host, 0) == hipSuccess;
    (void)hipSetDevice(prev);
    if (!ok) {
        if (s->host) (void)hipHostFree(s->host);
        delete s;
        return nullptr;
    }
    for (int i = 0; i < capacity; ++i) __atomic_store_n(&s->host[i], -1, __ATOMIC_RELAXED);
    __atomic_thread_fence(__ATOMIC_SEQ_CST);
    return s;
}

extern "C" void tms_token_slot_free(tms_token_slot* s) {
    if (!s) return;
    int prev = 0;
    (void)hipGetDevice(&prev);
    (void)hipSetDevice(s->device);
    (void)hipHostFree(s->host);
    (void)hipSetDevice(prev);
    delete s;
}

extern "C" int32_t* tms_token_slot_device(tms_token_slot* s) { return s ? s->dev : nullptr; }

extern "C" int tms_token_slot_capacity(const tms_token_slot* s) { return s ? s->capacity : 0; }

// Host side, no device work in flight on the slot: every entry := value.
extern "C" int tms_token_slot_fill(tms_token_slot* s, int32_t value) {
    if (!s) return TMS_ERR_INVALID_ARG;
    for (int i = 0; i < s->capacity; ++i) __atomic_store_n(&s->host[i], value, __ATOMIC_RELAXED);
    __atomic_thread_fence(__ATOMIC_SEQ_CST);
    return TMS_OK;
}

extern "C" int32_t tms_token_slot_peek(const tms_token_slot* s, int i) {
    if (!s || i < 0 || i >= s->capacity) return -1;
    return __atomic_load_n(&s->host[i], __ATOMIC_ACQUIRE);
}

extern "C" int tms_embed_gather(const void* table, int dtype, int64_t rows, int64_t dim, const int32_t* tokens,
                                int batch, void* x, int32_t* slot_out, hipStream_t stream) {
    if (!tokens || batch <= 0) return TMS_ERR_INVALID_ARG;
    int esz = 0;
    switch (dtype) {
        case TMS_DTYPE_F32: esz = 4; break;
        case TMS_DTYPE_F16:
        case TMS_DTYPE_BF16: esz = 2; break;
        default: return TMS_ERR_INVALID_ARG;
    }
    const int64_t row_bytes = dim * esz;
    if (table) {
        if (!x || rows <= 0 || dim <= 0 || row_bytes % 16 != 0 || (uintptr_t)table % 16 != 0 ||
            (uintptr_t)x % 16 != 0)
            return TMS_ERR_INVALID_ARG;
    } else if (!slot_out) {
        return TMS_ERR_INVALID_ARG;
    }
    hipLaunchKernelGGL(tms::embed_gather_kernel, dim3((unsigned)batch), dim3(256), 0, stream,
                       (const uint8_t*)table, rows, row_bytes, tokens, (uint8_t*)x, slot_out);
    return hipGetLastError() == hipSuccess ? TMS_OK : TMS_ERR_HIP;
}

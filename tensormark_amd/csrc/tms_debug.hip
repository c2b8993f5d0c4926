// tms_debug.hip -- test hooks: run the device Philox, the device double
// exp and the reciprocal-based division on caller inputs so the tests can pin them against the host checker,
// and check the ordering properties of the device that the library's
// cross-workgroup protocols rely on.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

#include "../../include/tmsample_hip.h"
#include "tms_device.h"

namespace tms {

__global__ void philox_kernel(const uint32_t* in6, uint32_t* out4, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    uint32_t c[4] = {in6[6 * i], in6[6 * i + 1], in6[6 * i + 2], in6[6 * i + 3]};
    philox4x32_10(c, in6[6 * i + 4], in6[6 * i + 5]);
    for (int j = 0; j < 4; ++j) out4[4 * i + j] = c[j];
}

__constant__ double kExpTab[64] = {TMS_EXP2_64THS};

__global__ void exp_kernel(const double* in, double* out, int n, int which) {
    __shared__ double tab[64];
    if (threadIdx.x < 64) tab[threadIdx.x] = kExpTab[threadIdx.x];
    __syncthreads();
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (which == 3) {   // quotients of the pairs (in[2i], in[2i + 1]) into out[i]
        if (2 * i + 1 < n) out[i] = div_rn(in[2 * i], in[2 * i + 1], 1.0 / in[2 * i + 1]);
        return;
    }
    if (i >= n) return;
    out[i] = which == 2 ? (double)q44_exp_nonpos(in[i], tab) : which ? exp64(in[i], tab) : exp(in[i]);
}

// ---- ordering checks (tms_debug_ordering)

// The XCD (XCC) this wave runs on: hardware register XCC_ID, bits 3:0.
__device__ __forceinline__ int xcc_id() {
    return __builtin_amdgcn_s_getreg(20 | (0 << 6) | (3 << 11)) & 0xF;
}

// The first workgroup of the grid found running on XCD `who` claims the role.
__device__ __forceinline__ bool claims(int who, int* claim) {
    return xcc_id() == who && atomicCAS(&claim[who], 0, 1) == 0;
}

// One line of 16 words: the claimant on XCD `who` sums it (plain loads).
__global__ void line_read(const uint64_t* p, int who, int* claim, uint64_t* out) {
    if (threadIdx.x != 0 || !claims(who, claim)) return;
    uint64_t s = 0;
    for (int i = 0; i < 16; ++i) s += p[i];
    out[0] = s;
}

// XCD `a` writes the even words, XCD `b` the odd words of the line (plain
// stores), in one kernel; with a == b XCD a writes every word.
__global__ void line_write(uint64_t* p, uint64_t v, int a, int b, int* claim) {
    if (threadIdx.x != 0) return;
    int off = -1, step = a == b ? 1 : 2;
    if (claims(a, claim)) off = 0;
    else if (a != b && claims(b, claim)) off = 1;
    if (off < 0) return;
    for (int i = off; i < 16; i += step) p[i] = v;
}

// As line_write, but each writer first reads the whole line (plain loads,
// the line then valid in its XCD's L2) and writes only after its reads
// returned: the access pattern of a workgroup that reads its neighbours'
// records of a line and then stores its own.
__global__ void line_read_write(uint64_t* p, uint64_t v, int a, int b, int* claim, uint64_t* sink) {
    if (threadIdx.x != 0) return;
    int off = -1;
    if (claims(a, claim)) off = 0;
    else if (claims(b, claim)) off = 1;
    if (off < 0) return;
    uint64_t s = 0;
    for (int i = 0; i < 16; ++i) s += p[i];
    const uint64_t w = v + (s == 0x5EEDull ? 1u : 0u);   // the stores wait for the loads
    for (int i = off; i < 16; i += 2) p[i] = w;
    if (s == 0x5EEDull) sink[0] = s;
}

// Back to back on one stream: every workgroup of the first kernel counts
// itself after a short bounded pause; the second reads the count at once.
__global__ void count_in(unsigned* ctr, int pause) {
    if (threadIdx.x != 0) return;
    for (int i = 0; i < pause; ++i) __builtin_amdgcn_s_sleep(10);
    __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__global__ void count_seen(unsigned* ctr, unsigned want, int* bad) {
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    if (__hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != want) atomicAdd(bad, 1);
    __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__global__ void xcc_of(int* ids) {
    if (threadIdx.x == 0) ids[blockIdx.x] = xcc_id();
}

}  // namespace tms

// counts[0]: reads on XCD 1 that missed a line written on XCD 0 by the
//            previous kernel, after XCD 1 had read (cached) the line;
// counts[1]: lines written half by XCD 0 and half by XCD 1 in one kernel
//            that the next kernel (XCD 2) read with a word lost;
// counts[2]: kernels that started before the previous kernel on the stream
//            had finished;
// counts[3]: workgroups w of a 64-workgroup grid not on XCD w mod (XCD
//            count), the placement the sampler's row mapping assumes;
// counts[4]: the XCD count seen;
// counts[5]: trials of (a), (b) and (d) not run because no workgroup of a
//            grid landed on an XCD a role needs (the reader's result keeps
//            its sentinel); they count as neither stale nor lost;
// counts[6]: (d) as (b), but each writer reads the whole line before it
//            writes its half: lines the next kernel read with a word lost.
//            No sampler kernel stores into a line it has read with plain
//            accesses while another workgroup stores into the same line, so
//            this is reported, not required to be 0.
// Synchronous; `trials` of each.
extern "C" int tms_debug_ordering(int trials, int32_t* counts) {
    if (!counts || trials <= 0) return TMS_ERR_INVALID_ARG;
    constexpr int kGrid = 64;
    uint64_t* line = nullptr;
    uint64_t* out = nullptr;
    int* claim = nullptr;
    int* ids = nullptr;
    int* bad = nullptr;
    unsigned* ctr = nullptr;
    int rc = TMS_OK;
    hipStream_t s = nullptr;
    if (hipMalloc(&line, 128) != hipSuccess || hipMalloc(&out, 8) != hipSuccess ||
        hipMalloc(&claim, 16 * sizeof(int)) != hipSuccess || hipMalloc(&ids, kGrid * sizeof(int)) != hipSuccess ||
        hipMalloc(&bad, sizeof(int)) != hipSuccess || hipMalloc(&ctr, sizeof(unsigned)) != hipSuccess ||
        hipStreamCreate(&s) != hipSuccess)
        rc = TMS_ERR_HIP;
    int hid[kGrid] = {0};
    int nx = 1;
    if (rc == TMS_OK) {
        hipLaunchKernelGGL(tms::xcc_of, dim3(kGrid), dim3(64), 0, s, ids);
        if (hipMemcpyAsync(hid, ids, sizeof(hid), hipMemcpyDeviceToHost, s) != hipSuccess ||
            hipStreamSynchronize(s) != hipSuccess)
            rc = TMS_ERR_HIP;
        for (int i = 0; i < kGrid; ++i) nx = std::max(nx, hid[i] + 1);
    }
    int stale = 0, lost = 0, overlap = 0, placed = 0, not_run = 0, lost_rw = 0;
    constexpr uint64_t kSentinel = ~0ull;   // `out` before a read: no reader ran
    if (rc == TMS_OK) {
        for (int i = 0; i < kGrid; ++i) placed += hid[i] != i % nx;
        const int b = nx > 1 ? 1 : 0, c2 = nx > 2 ? 2 : 0;
        for (int it = 1; it <= trials && rc == TMS_OK; ++it) {
            uint64_t sum = 0;
            // (a) XCD b caches the line; XCD 0 writes it; XCD b reads it again
            (void)hipMemsetAsync(claim, 0, 16 * sizeof(int), s);
            hipLaunchKernelGGL(tms::line_read, dim3(kGrid), dim3(64), 0, s, line, b, claim, out);
            (void)hipMemsetAsync(claim, 0, 16 * sizeof(int), s);
            hipLaunchKernelGGL(tms::line_write, dim3(kGrid), dim3(64), 0, s, line, (uint64_t)it, 0, 0, claim);
            (void)hipMemsetAsync(claim, 0, 16 * sizeof(int), s);
            (void)hipMemsetAsync(out, 0xFF, 8, s);
            hipLaunchKernelGGL(tms::line_read, dim3(kGrid), dim3(64), 0, s, line, b, claim, out);
            if (hipMemcpyAsync(&sum, out, 8, hipMemcpyDeviceToHost, s) != hipSuccess ||
                hipStreamSynchronize(s) != hipSuccess) rc = TMS_ERR_HIP;
            if (sum == kSentinel) ++not_run;
            else stale += sum != 16ull * (uint64_t)it;
            // (b) XCDs 0 and b write alternate words in one kernel; XCD c2 reads
            (void)hipMemsetAsync(claim, 0, 16 * sizeof(int), s);
            hipLaunchKernelGGL(tms::line_write, dim3(kGrid), dim3(64), 0, s, line, (uint64_t)it + 1000000, 0, b, claim);
            (void)hipMemsetAsync(claim, 0, 16 * sizeof(int), s);
            (void)hipMemsetAsync(out, 0xFF, 8, s);
            hipLaunchKernelGGL(tms::line_read, dim3(kGrid), dim3(64), 0, s, line, c2, claim, out);
            if (hipMemcpyAsync(&sum, out, 8, hipMemcpyDeviceToHost, s) != hipSuccess ||
                hipStreamSynchronize(s) != hipSuccess) rc = TMS_ERR_HIP;
            if (sum == kSentinel) ++not_run;
            else lost += sum != 16ull * ((uint64_t)it + 1000000);
            // (d) as (b), each writer reading the line first
            (void)hipMemsetAsync(claim, 0, 16 * sizeof(int), s);
            hipLaunchKernelGGL(tms::line_read_write, dim3(kGrid), dim3(64), 0, s, line, (uint64_t)it + 2000000, 0,
                               b, claim, out);
            (void)hipMemsetAsync(claim, 0, 16 * sizeof(int), s);
            (void)hipMemsetAsync(out, 0xFF, 8, s);
            hipLaunchKernelGGL(tms::line_read, dim3(kGrid), dim3(64), 0, s, line, c2, claim, out);
            if (hipMemcpyAsync(&sum, out, 8, hipMemcpyDeviceToHost, s) != hipSuccess ||
                hipStreamSynchronize(s) != hipSuccess) rc = TMS_ERR_HIP;
            if (sum == kSentinel) ++not_run;
            else lost_rw += sum != 16ull * ((uint64_t)it + 2000000);
        }
        // (c) back-to-back kernels
        if (rc == TMS_OK) {
            (void)hipMemsetAsync(ctr, 0, sizeof(unsigned), s);
            (void)hipMemsetAsync(bad, 0, sizeof(int), s);
            for (int it = 0; it < trials; ++it) {
                hipLaunchKernelGGL(tms::count_in, dim3(1024), dim3(64), 0, s, ctr, 1 + (it % 7) * 20);
                hipLaunchKernelGGL(tms::count_seen, dim3(8), dim3(64), 0, s, ctr, 1024u, bad);
            }
            if (hipMemcpyAsync(&overlap, bad, sizeof(int), hipMemcpyDeviceToHost, s) != hipSuccess ||
                hipStreamSynchronize(s) != hipSuccess) rc = TMS_ERR_HIP;
        }
    }
    if (hipGetLastError() != hipSuccess) rc = TMS_ERR_HIP;
    counts[0] = stale;
    counts[1] = lost;
    counts[2] = overlap;
    counts[3] = placed;
    counts[4] = nx;
    counts[5] = not_run;
    counts[6] = lost_rw;
    if (s) (void)hipStreamDestroy(s);
    for (void* q : {(void*)line, (void*)out, (void*)claim, (void*)ids, (void*)bad, (void*)ctr})
        if (q) (void)hipFree(q);
    return rc;
}

extern "C" int tms_debug_philox(const uint32_t* in6, uint32_t* out4, int n, hipStream_t stream) {
    if (!in6 || !out4 || n < 0) return TMS_ERR_INVALID_ARG;
    if (n == 0) return TMS_OK;
    hipLaunchKernelGGL(tms::philox_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, in6, out4, n);
    return hipGetLastError() == hipSuccess ? TMS_OK : TMS_ERR_HIP;
}

extern "C" int tms_debug_exp(const double* in, double* out, int n, int which, hipStream_t stream) {
    if (!in || !out || n < 0 || which < 0 || which > 3) return TMS_ERR_INVALID_ARG;
    if (n == 0) return TMS_OK;
    hipLaunchKernelGGL(tms::exp_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, in, out, n, which);
    return hipGetLastError() == hipSuccess ? TMS_OK : TMS_ERR_HIP;
}

// tms_debug.hip -- test hooks: run the device Philox and the device double
// exp on caller inputs so the tests can pin them against the host checker.

#include <hip/hip_runtime.h>
#include <stdint.h>

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
    if (i >= n) return;
    out[i] = which ? exp64(in[i], tab) : exp(in[i]);
}

}  // namespace tms

extern "C" int tms_debug_philox(const uint32_t* in6, uint32_t* out4, int n, hipStream_t stream) {
    if (!in6 || !out4 || n < 0) return TMS_ERR_INVALID_ARG;
    if (n == 0) return TMS_OK;
    hipLaunchKernelGGL(tms::philox_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, in6, out4, n);
    return hipGetLastError() == hipSuccess ? TMS_OK : TMS_ERR_HIP;
}

extern "C" int tms_debug_exp(const double* in, double* out, int n, int which, hipStream_t stream) {
    if (!in || !out || n < 0 || (which != 0 && which != 1)) return TMS_ERR_INVALID_ARG;
    if (n == 0) return TMS_OK;
    hipLaunchKernelGGL(tms::exp_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, in, out, n, which);
    return hipGetLastError() == hipSuccess ? TMS_OK : TMS_ERR_HIP;
}

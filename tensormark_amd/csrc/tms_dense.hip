// tms_dense.hip -- the whole-row pass of tms_sample_batch: samples the rows
// that the chunked kernels queued (dense top-p rows, draws past the held
// entries, rows that break the top-k kernel's hint) by the exact full-row
// form of tmsample::sample (tensormark/tmsample.h:177-200) in tms_dense.h.
//
// It runs right after the chunked kernel on the same stream, so the queue
// (count, rows) that kernel wrote is complete when it starts.  Each
// workgroup takes queued rows one at a time with an agent-scope counter and
// works in its own region of the workspace; the last workgroup to finish
// returns the queue's three counters to zero for the next call.  With an
// empty queue every workgroup reads the count and exits.

#include "tms_dense.h"

namespace tms {

template <typename T>
__global__ __launch_bounds__(kBlock) void dense_kernel(KArgs a) {
    __shared__ DenseLds L;
    __shared__ uint32_t take;
    const uint32_t queued = ld_agent(&a.dqueue[0]);
    if (queued == 0) return;   // nothing queued: nothing taken, nothing to reset
    uint64_t* ws = a.dense + (int64_t)blockIdx.x * 2 * a.dense_stride;
    for (;;) {
        if (threadIdx.x == 0)
            take = __hip_atomic_fetch_add(&a.dqueue[1], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        const uint32_t i = take;
        __syncthreads();
        if (i >= queued) break;
        const int row = (int)a.dqueue[kDenseQueueHead + i];
        const tms_row_params P = a.params[row];
        const int V = a.V;
        const int K = (P.top_k <= 0 || P.top_k > V) ? V : P.top_k;
        dense_row<T>(a, row, P, K, ws, L);
        __syncthreads();   // L and ws are free for the next row
    }
    if (threadIdx.x == 0) {
        const uint32_t done =
            __hip_atomic_fetch_add(&a.dqueue[2], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (done == gridDim.x - 1) {
            // every other workgroup has taken its last row
            st_agent(&a.dqueue[0], 0u);
            st_agent(&a.dqueue[1], 0u);
            st_agent(&a.dqueue[2], 0u);
        }
    }
}

}  // namespace tms

int tms_launch_dense(const tms::KArgs& k, int dtype, int workgroups, hipStream_t stream) {
    const dim3 grid((unsigned)workgroups), block(tms::kBlock);
    switch (dtype) {
        case TMS_DTYPE_F32: hipLaunchKernelGGL((tms::dense_kernel<float>), grid, block, 0, stream, k); break;
        case TMS_DTYPE_F16: hipLaunchKernelGGL((tms::dense_kernel<_Float16>), grid, block, 0, stream, k); break;
        default: hipLaunchKernelGGL((tms::dense_kernel<tms::Bf16>), grid, block, 0, stream, k); break;
    }
    return hipGetLastError() == hipSuccess ? TMS_OK : TMS_ERR_HIP;
}

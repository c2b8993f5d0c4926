// tms_spec.hip -- speculative verify (placeholder until the kernel lands).
#include <hip/hip_runtime.h>
#include "../../include/tmsample_hip.h"
extern "C" int tms_spec_verify(tms_context*, const tms_spec_args*, hipStream_t) {
    return TMS_ERR_INVALID_ARG;
}

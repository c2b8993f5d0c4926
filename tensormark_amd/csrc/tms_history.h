// tms_history.h -- the device pre-pass's own DRY penalty scale
// (tms_hist.hip), for calls that bring no table of the reference's powf
// values (tms_sample_args.dry_scale).
#pragma once

#ifdef __HIP__
#define TMS_HD __host__ __device__
#else
#define TMS_HD
#endif

// base^k for an integer k >= 0 by binary powering in double, then one
// rounding to float.  The double products carry at most ~2 log2(k) roundings
// of 2^-53, so the float result is the correctly rounded power except when
// the exact power lies within ~2^-48 (relative) of a float rounding
// boundary.  tensormark/tmsample.h:168 calls powf(base, (float)k); glibc's
// powf is not correctly rounded (0.82 ulp bound) and differs from this by one
// ulp for about 0.1% of (base, k) pairs (base 1.75: first at k = 83), which
// is why callers that need the reference's bits pass the table.
static inline TMS_HD float tms_dry_scale(float base, int k) {
    double r = 1.0, x = (double)base;
    for (unsigned e = (unsigned)k; e != 0u; e >>= 1) {
        if (e & 1u) r *= x;
        x *= x;
    }
    return (float)r;
}

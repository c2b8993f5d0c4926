// tms_device.h -- device helpers shared by the sampler and the speculative
// verify kernels: order keys, Philox4x32-10, the canonical uniform, the
// library's own double exp, and wave/block reductions for 64-wide waves.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tms {

constexpr int kBlock = 256;   // threads per workgroup: four 64-wide waves
constexpr int kWaves = kBlock / 64;

// ------------------------------------------------------------- order keys

// Order-preserving 32-bit key of a float under IEEE `>`: -0 and +0 map to
// one key (x + 0.0f turns -0 into +0), so equal values stay equal and the id
// decides.  NaN never reaches a key: rows holding one are rejected first.
__device__ __forceinline__ uint32_t okey(float x) {
    const uint32_t u = __float_as_uint(x + 0.0f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float okey_inv(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

// 64-bit candidate key: value order first, then lower id first.  Larger key
// is the better candidate; 0 means "no candidate".
__device__ __forceinline__ uint64_t ckey(float v, uint32_t id) {
    return ((uint64_t)okey(v) << 32) | (uint64_t)(0xFFFFFFFFu - id);
}
__device__ __forceinline__ uint32_t ckey_id(uint64_t k) { return 0xFFFFFFFFu - (uint32_t)k; }
__device__ __forceinline__ float ckey_val(uint64_t k) { return okey_inv((uint32_t)(k >> 32)); }

// ----------------------------------------------------------------- Philox

// Philox4x32-10 (Salmon et al., SC'11): ten rounds, key bumped by the Weyl
// constants between rounds.
__device__ __forceinline__ void philox4x32_10(uint32_t c[4], uint32_t k0, uint32_t k1) {
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        const uint32_t lo0 = 0xD2511F53u * c[0];
        const uint32_t hi0 = __umulhi(0xD2511F53u, c[0]);
        const uint32_t lo1 = 0xCD9E8D57u * c[2];
        const uint32_t hi1 = __umulhi(0xCD9E8D57u, c[2]);
        const uint32_t n0 = hi1 ^ c[1] ^ k0;
        const uint32_t n2 = hi0 ^ c[3] ^ k1;
        c[0] = n0;
        c[1] = lo1;
        c[2] = n2;
        c[3] = lo0;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
}

// Words (w0, w1) of a row's draw: key = seed, counter = (offset, stream, 0).
__device__ __forceinline__ void row_words(uint64_t seed, uint64_t offset, uint32_t stream,
                                          uint32_t& w0, uint32_t& w1) {
    uint32_t c[4] = {(uint32_t)offset, (uint32_t)(offset >> 32), stream, 0u};
    philox4x32_10(c, (uint32_t)seed, (uint32_t)(seed >> 32));
    w0 = c[0];
    w1 = c[1];
}

// Uniform in [0, 1) from two 32-bit words, with the arithmetic of libstdc++'s
// generate_canonical<double, 53> over a 32-bit engine: sum = w0 + w1 * 2^32
// rounded to double, divided by 2^64, clamped below 1.
__device__ __forceinline__ double canonical(uint32_t w0, uint32_t w1) {
    double sum = 0.0;
    sum += (double)w0 * 1.0;
    sum += (double)w1 * 4294967296.0;
    double r = sum / 18446744073709551616.0;
    if (r >= 1.0) r = 0x1.fffffffffffffp-1;
    return r;
}

// ------------------------------------------------------------------- exp

// exp(x) by Cody-Waite reduction and a degree-13 Taylor polynomial, one IEEE
// operation per step, so the host checker evaluates the same bits.  Used by
// the speculative verify, whose weights are build-defined.
__device__ __forceinline__ double exp64(double x) {
    if (x != x) return x;
    if (x < -746.0) return 0.0;
    if (x > 709.782712893384) return __builtin_huge_val();
    const double inv_ln2 = 1.4426950408889634;
    const double ln2_hi = 0x1.62e42fefa39efp-1;
    const double ln2_lo = 0x1.abc9e3b39803fp-56;
    const double kd = floor(x * inv_ln2 + 0.5);
    double r = fma(-kd, ln2_hi, x);
    r = fma(-kd, ln2_lo, r);
    double q = 1.0 / 6227020800.0;
    q = fma(q, r, 1.0 / 479001600);
    q = fma(q, r, 1.0 / 39916800);
    q = fma(q, r, 1.0 / 3628800);
    q = fma(q, r, 1.0 / 362880);
    q = fma(q, r, 1.0 / 40320);
    q = fma(q, r, 1.0 / 5040);
    q = fma(q, r, 1.0 / 720);
    q = fma(q, r, 1.0 / 120);
    q = fma(q, r, 1.0 / 24);
    q = fma(q, r, 1.0 / 6);
    q = fma(q, r, 1.0 / 2);
    q = fma(q, r, 1.0);
    q = fma(q, r, 1.0);
    int k = (int)kd;
    if (k > 1023) {
        q = q * 2.0;
        k -= 1;
    }
    if (k < -1020) {
        q = q * 0x1p-200;
        k += 200;
    }
    return q * __longlong_as_double((long long)(k + 1023) << 52);
}

__device__ __forceinline__ int64_t q44(double y) {
    return (int64_t)floor(y * 17592186044416.0 + 0.5);
}

// ------------------------------------------------------------ reductions

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int m) {
    const uint32_t lo = __shfl_xor((uint32_t)v, m, 64);
    const uint32_t hi = __shfl_xor((uint32_t)(v >> 32), m, 64);
    return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        const uint64_t o = shfl_xor_u64(v, m);
        v = o > v ? o : v;
    }
    return v;
}

__device__ __forceinline__ float wave_max_f32(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
    return v;
}

__device__ __forceinline__ float wave_min_f32(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = fminf(v, __shfl_xor(v, m, 64));
    return v;
}

__device__ __forceinline__ int wave_sum_i32(int v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}

__device__ __forceinline__ int64_t wave_sum_i64(int64_t v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += (int64_t)shfl_xor_u64((uint64_t)v, m);
    return v;
}

// DPP lane moves (row_shr:n within 16-lane rows, row_bcast:15/31 across
// rows).  `old` fills lanes whose source is outside the row or masked.
template <int CTRL, int ROW_MASK, bool BOUND_ZERO>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t old, uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp((int)old, (int)v, CTRL, ROW_MASK, 0xF, BOUND_ZERO);
}

// Inclusive prefix sum across the 64 lanes of a wave (DPP, no LDS).
__device__ __forceinline__ int wave_incl_scan_i32(int v) {
    uint32_t u = (uint32_t)v;
    u += dpp_u32<0x111, 0xF, true>(0u, u);   // row_shr:1
    u += dpp_u32<0x112, 0xF, true>(0u, u);   // row_shr:2
    u += dpp_u32<0x114, 0xF, true>(0u, u);   // row_shr:4
    u += dpp_u32<0x118, 0xF, true>(0u, u);   // row_shr:8
    u += dpp_u32<0x142, 0xA, false>(0u, u);  // row_bcast:15 into rows 1 and 3
    u += dpp_u32<0x143, 0xC, false>(0u, u);  // row_bcast:31 into rows 2 and 3
    return (int)u;
}

__device__ __forceinline__ int wave_sum_dpp(int v) {
    return __builtin_amdgcn_readlane(wave_incl_scan_i32(v), 63);
}

// Maximum over the wave of u64 keys, by DPP steps towards lane 63.
__device__ __forceinline__ uint64_t wave_max_u64_dpp(uint64_t v) {
#define TMS_MAXSTEP(CTRL, RM, BZ)                                                   \
    {                                                                             \
        const uint32_t lo = dpp_u32<CTRL, RM, BZ>(0u, (uint32_t)v);               \
        const uint32_t hi = dpp_u32<CTRL, RM, BZ>(0u, (uint32_t)(v >> 32));       \
        const uint64_t o = ((uint64_t)hi << 32) | lo;                              \
        v = o > v ? o : v;                                                        \
    }
    TMS_MAXSTEP(0x111, 0xF, true)
    TMS_MAXSTEP(0x112, 0xF, true)
    TMS_MAXSTEP(0x114, 0xF, true)
    TMS_MAXSTEP(0x118, 0xF, true)
    TMS_MAXSTEP(0x142, 0xA, false)
    TMS_MAXSTEP(0x143, 0xC, false)
#undef TMS_MAXSTEP
    const uint32_t lo = __builtin_amdgcn_readlane((int)(uint32_t)v, 63);
    const uint32_t hi = __builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), 63);
    return ((uint64_t)hi << 32) | lo;
}

// Maximum over the wave of floats (no NaN), by DPP steps towards lane 63.
__device__ __forceinline__ float wave_max_f32_dpp(float v) {
    const uint32_t ninf = 0xFF800000u;
#define TMS_FMAXSTEP(CTRL, RM, BZ) \
    v = fmaxf(v, __uint_as_float(dpp_u32<CTRL, RM, BZ>(ninf, __float_as_uint(v))));
    TMS_FMAXSTEP(0x111, 0xF, false)
    TMS_FMAXSTEP(0x112, 0xF, false)
    TMS_FMAXSTEP(0x114, 0xF, false)
    TMS_FMAXSTEP(0x118, 0xF, false)
    TMS_FMAXSTEP(0x142, 0xA, false)
    TMS_FMAXSTEP(0x143, 0xC, false)
#undef TMS_FMAXSTEP
    return __uint_as_float(__builtin_amdgcn_readlane((int)__float_as_uint(v), 63));
}

__device__ __forceinline__ int64_t wave_incl_scan_i64(int64_t v) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const uint32_t lo = __shfl_up((uint32_t)v, d, 64);
        const uint32_t hi = __shfl_up((uint32_t)((uint64_t)v >> 32), d, 64);
        const int64_t o = (int64_t)(((uint64_t)hi << 32) | lo);
        if (lane >= d) v += o;
    }
    return v;
}

// Sort 64 floats across a wave, descending (lane 0 holds the largest):
// bitonic network on lane pairs exchanged by shuffles.
__device__ __forceinline__ float wave_sort_desc_f32(float v) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int k = 2; k <= 64; k <<= 1) {
#pragma unroll
        for (int j = k >> 1; j >= 1; j >>= 1) {
            const float o = __shfl_xor(v, j, 64);
            const bool lower = (lane & j) == 0;
            const bool desc = (lane & k) == 0;
            // Lower lane of a descending pair keeps the max.
            const bool take_max = (lower == desc);
            v = take_max ? fmaxf(v, o) : fminf(v, o);
        }
    }
    return v;
}

// Sort 64 u64 keys across a wave, descending.
__device__ __forceinline__ uint64_t wave_sort_desc_u64(uint64_t v) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int k = 2; k <= 64; k <<= 1) {
#pragma unroll
        for (int j = k >> 1; j >= 1; j >>= 1) {
            const uint64_t o = shfl_xor_u64(v, j);
            const bool lower = (lane & j) == 0;
            const bool desc = (lane & k) == 0;
            const bool take_max = (lower == desc);
            const uint64_t mx = o > v ? o : v;
            const uint64_t mn = o > v ? v : o;
            v = take_max ? mx : mn;
        }
    }
    return v;
}

}  // namespace tms

namespace tms {

// Sort 128 u64 keys held two per lane (entry i = lane + 64 * slot) across a
// wave, descending.
__device__ __forceinline__ void wave_sort_desc_u64x2(uint64_t& a0, uint64_t& a1) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int k = 2; k <= 128; k <<= 1) {
#pragma unroll
        for (int j = k >> 1; j >= 1; j >>= 1) {
            if (j == 64) {
                // Partners are the two slots of one lane; entry index bit 6
                // is the slot, so the block direction comes from k alone.
                const bool desc = true;   // k == 128: one descending block
                const uint64_t mx = a0 > a1 ? a0 : a1;
                const uint64_t mn = a0 > a1 ? a1 : a0;
                a0 = desc ? mx : mn;
                a1 = desc ? mn : mx;
            } else {
                const uint64_t o0 = shfl_xor_u64(a0, j);
                const uint64_t o1 = shfl_xor_u64(a1, j);
                const bool lower = (lane & j) == 0;
                // entry index of slot s: lane + 64 s; block direction bit k.
                const bool desc0 = (lane & k) == 0;
                const bool desc1 = ((lane + 64) & k) == 0;
                const bool tmax0 = (lower == desc0);
                const bool tmax1 = (lower == desc1);
                const uint64_t mx0 = o0 > a0 ? o0 : a0, mn0 = o0 > a0 ? a0 : o0;
                const uint64_t mx1 = o1 > a1 ? o1 : a1, mn1 = o1 > a1 ? a1 : o1;
                a0 = tmax0 ? mx0 : mn0;
                a1 = tmax1 ? mx1 : mn1;
            }
        }
    }
}

__device__ __forceinline__ double readlane_f64(double v, int lane) {
    const uint64_t u = (uint64_t)__double_as_longlong(v);
    const uint32_t lo = __builtin_amdgcn_readlane((int)(uint32_t)u, lane);
    const uint32_t hi = __builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), lane);
    return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

// The largest float below x (x finite, not -FLT_MAX): one step down in the
// order of IEEE values, by integer arithmetic on the bits.
__device__ __forceinline__ float float_below(float x) {
    const uint32_t u = __float_as_uint(x);
    if ((u & 0x7FFFFFFFu) == 0) return __uint_as_float(0x80000001u);   // +-0 -> -min subnormal
    return __uint_as_float((u & 0x80000000u) ? u + 1u : u - 1u);
}

}  // namespace tms

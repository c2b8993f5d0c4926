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

// 2^(j/64), j = 0..63, each the double nearest the exact value.
#define TMS_EXP2_64THS \
    0x1.0000000000000p+0, 0x1.02c9a3e778061p+0, 0x1.059b0d3158574p+0, 0x1.0874518759bc8p+0, \
    0x1.0b5586cf9890fp+0, 0x1.0e3ec32d3d1a2p+0, 0x1.11301d0125b51p+0, 0x1.1429aaea92de0p+0, \
    0x1.172b83c7d517bp+0, 0x1.1a35beb6fcb75p+0, 0x1.1d4873168b9aap+0, 0x1.2063b88628cd6p+0, \
    0x1.2387a6e756238p+0, 0x1.26b4565e27cddp+0, 0x1.29e9df51fdee1p+0, 0x1.2d285a6e4030bp+0, \
    0x1.306fe0a31b715p+0, 0x1.33c08b26416ffp+0, 0x1.371a7373aa9cbp+0, 0x1.3a7db34e59ff7p+0, \
    0x1.3dea64c123422p+0, 0x1.4160a21f72e2ap+0, 0x1.44e086061892dp+0, 0x1.486a2b5c13cd0p+0, \
    0x1.4bfdad5362a27p+0, 0x1.4f9b2769d2ca7p+0, 0x1.5342b569d4f82p+0, 0x1.56f4736b527dap+0, \
    0x1.5ab07dd485429p+0, 0x1.5e76f15ad2148p+0, 0x1.6247eb03a5585p+0, 0x1.6623882552225p+0, \
    0x1.6a09e667f3bcdp+0, 0x1.6dfb23c651a2fp+0, 0x1.71f75e8ec5f74p+0, 0x1.75feb564267c9p+0, \
    0x1.7a11473eb0187p+0, 0x1.7e2f336cf4e62p+0, 0x1.82589994cce13p+0, 0x1.868d99b4492edp+0, \
    0x1.8ace5422aa0dbp+0, 0x1.8f1ae99157736p+0, 0x1.93737b0cdc5e5p+0, 0x1.97d829fde4e50p+0, \
    0x1.9c49182a3f090p+0, 0x1.a0c667b5de565p+0, 0x1.a5503b23e255dp+0, 0x1.a9e6b5579fdbfp+0, \
    0x1.ae89f995ad3adp+0, 0x1.b33a2b84f15fbp+0, 0x1.b7f76f2fb5e47p+0, 0x1.bcc1e904bc1d2p+0, \
    0x1.c199bdd85529cp+0, 0x1.c67f12e57d14bp+0, 0x1.cb720dcef9069p+0, 0x1.d072d4a07897cp+0, \
    0x1.d5818dcfba487p+0, 0x1.da9e603db3285p+0, 0x1.dfc97337b9b5fp+0, 0x1.e502ee78b3ff6p+0, \
    0x1.ea4afa2a490dap+0, 0x1.efa1bee615a27p+0, 0x1.f50765b6e4540p+0, 0x1.fa7c1819e90d8p+0,

// exp(x) by table-driven range reduction (Tang, "Table-driven implementation
// of the exponential function in IEEE floating-point arithmetic", ACM TOMS
// 15(2), 1989): x = (64m + j) ln2/64 + r with |r| <= ln2/128, ln2/64 split
// into a double and its residual, e^r by its Taylor series to degree 5 in
// Horner form, times 2^(j/64) from the table `tab` (64 doubles, in LDS), times
// 2^m.  Every step is one IEEE operation, so the host checker evaluates the
// identical function.  Used for the speculative verify's weights.
__device__ __forceinline__ double exp64(double x, const double* tab) {
    if (x != x) return x;
    if (x < -746.0) return 0.0;
    if (x > 709.782712893384) return __builtin_huge_val();
    const double kd = rint(x * 0x1.71547652b82fep+6);
    double r = fma(-kd, 0x1.62e42fefa39efp-7, x);
    r = fma(-kd, 0x1.abc9e3b39803fp-62, r);
    double p = 1.0 / 120;
    p = fma(p, r, 1.0 / 24);
    p = fma(p, r, 1.0 / 6);
    p = fma(p, r, 0.5);
    p = fma(p, r, 1.0);
    p = fma(p, r, 1.0);
    const int ki = (int)kd;
    int m = ki >> 6;
    double y = tab[ki & 63] * p;
    if (m > 1023) {
        y = y * 2.0;
        m -= 1;
    }
    if (m < -1020) {
        y = y * 0x1p-200;
        m += 200;
    }
    return y * __longlong_as_double((long long)(m + 1023) << 52);
}

// y in [0, 1] (a probability): rint(y * 2^44), the nearest multiple of
// 2^-44 in units of 2^-44 (ties to even), is a whole number below 2^52, so
// adding 2^52 holds it exactly in the mantissa, and the difference of the
// bit patterns is that integer (two operations, where a general double ->
// int64 conversion takes several).
__device__ __forceinline__ int64_t q44(double y) {
    const double f = rint(y * 17592186044416.0);
    return __double_as_longlong(f + 0x1p52) - __double_as_longlong(0x1p52);
}

// q44(exp64(x)) for x <= 0, bit-identical to the pair above, as a double
// holding the whole number (at most 2^44, so sums of up to 128 of them stay
// exact and below 2^52).  Below -40 the weight is 0: exp64(x) < e^-40 <
// 2^-57, which rounds to 0 on the 2^-44 grid; the argument is clamped at -41, where the same
// holds, so no select is needed (a NaN clamps to -41 too).  On [-41, 0]
// exp64 takes none of its special cases (2^m is normal, m >= -60), and its
// final scaling by 2^m and q44's by 2^44 are both exact, so they fold into
// one ldexp by m + 44.
__device__ __forceinline__ double q44_exp_nonpos_f(double x, const double* tab) {
    const double xc = fmax(x, -41.0);
    const double kd = rint(xc * 0x1.71547652b82fep+6);
    double r = fma(-kd, 0x1.62e42fefa39efp-7, xc);
    r = fma(-kd, 0x1.abc9e3b39803fp-62, r);
    double p = 1.0 / 120;
    p = fma(p, r, 1.0 / 24);
    p = fma(p, r, 1.0 / 6);
    p = fma(p, r, 0.5);
    p = fma(p, r, 1.0);
    p = fma(p, r, 1.0);
    const int ki = (int)kd;
    const double y = tab[ki & 63] * p;
    return rint(ldexp(y, (ki >> 6) + 44));
}

// a / b correctly rounded, given y = RN(1/b) (one division per divisor in
// place of one per element).  q0 = RN(a * y) is within 1.5 ulp of a / b; the
// remainder a - b * q0 is exact by fma, and q1 = RN(q0 + r0 * y) is within
// an ulp (faithful); from a faithful quotient and the correctly rounded
// reciprocal, one more correction returns RN(a / b) (Markstein, IBM J. Res.
// Dev. 34(1), 1990).  For finite a, b whose quotient, remainders and
// reciprocal neither overflow nor fall below the normal range.
__device__ __forceinline__ double div_rn(double a, double b, double y) {
    double q = a * y;
    double r = fma(-b, q, a);
    q = fma(r, y, q);
    r = fma(-b, q, a);
    return fma(r, y, q);
}

// The same weight as an int64 (the bit-pattern difference of q44).
__device__ __forceinline__ int64_t q44_exp_nonpos(double x, const double* tab) {
    const double f = q44_exp_nonpos_f(x, tab);
    return __double_as_longlong(f + 0x1p52) - __double_as_longlong(0x1p52);
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

// Inclusive prefix sums of non-negative doubles across the wave (DPP, a
// tree of depth 6; lanes without a source add +0.0, which is exact).
__device__ __forceinline__ double wave_incl_scan_f64(double v) {
#define TMS_FSCAN(CTRL, RM, BZ)                                                            \
    {                                                                                      \
        const uint64_t b = (uint64_t)__double_as_longlong(v);                              \
        const uint32_t lo = dpp_u32<CTRL, RM, BZ>(0u, (uint32_t)b);                        \
        const uint32_t hi = dpp_u32<CTRL, RM, BZ>(0u, (uint32_t)(b >> 32));                \
        v += __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));                 \
    }
    TMS_FSCAN(0x111, 0xF, true)
    TMS_FSCAN(0x112, 0xF, true)
    TMS_FSCAN(0x114, 0xF, true)
    TMS_FSCAN(0x118, 0xF, true)
    TMS_FSCAN(0x142, 0xA, false)
    TMS_FSCAN(0x143, 0xC, false)
#undef TMS_FSCAN
    return v;
}

// Inclusive prefix sums of int64 across the wave (DPP; lanes without a
// source add 0).
__device__ __forceinline__ int64_t wave_incl_scan_i64_dpp(int64_t v) {
#define TMS_ISCAN(CTRL, RM, BZ)                                                            \
    {                                                                                      \
        const uint64_t b = (uint64_t)v;                                                    \
        const uint32_t lo = dpp_u32<CTRL, RM, BZ>(0u, (uint32_t)b);                        \
        const uint32_t hi = dpp_u32<CTRL, RM, BZ>(0u, (uint32_t)(b >> 32));                \
        v += (int64_t)(((uint64_t)hi << 32) | lo);                                         \
    }
    TMS_ISCAN(0x111, 0xF, true)
    TMS_ISCAN(0x112, 0xF, true)
    TMS_ISCAN(0x114, 0xF, true)
    TMS_ISCAN(0x118, 0xF, true)
    TMS_ISCAN(0x142, 0xA, false)
    TMS_ISCAN(0x143, 0xC, false)
#undef TMS_ISCAN
    return v;
}

__device__ __forceinline__ int64_t readlane_i64(int64_t v, int l) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, l);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)((uint64_t)v >> 32), l);
    return (int64_t)(((uint64_t)hi << 32) | lo);
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

// bf16 storage: the high half of an fp32.
struct Bf16 {
    uint16_t bits;
};

// Element types: vector width of a 16-byte load, exact widening to fp32.
template <typename T>
struct Elt;
template <>
struct Elt<float> {
    static constexpr int kVec = 4;
    static constexpr uint32_t kNegInfWord = 0xFF800000u;   // -inf in each element of a word
    __device__ static void widen(const uint4& q, float (&f)[4]) {
        f[0] = __uint_as_float(q.x);
        f[1] = __uint_as_float(q.y);
        f[2] = __uint_as_float(q.z);
        f[3] = __uint_as_float(q.w);
    }
    __device__ static float scalar(const float* p) { return *p; }
};
template <>
struct Elt<_Float16> {
    static constexpr int kVec = 8;
    static constexpr uint32_t kNegInfWord = 0xFC00FC00u;
    __device__ static float h2f(uint32_t h) {
        _Float16 v;
        const uint16_t b = (uint16_t)h;
        __builtin_memcpy(&v, &b, 2);
        return (float)v;
    }
    __device__ static void widen(const uint4& q, float (&f)[8]) {
        const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            f[2 * i] = h2f(w[i] & 0xFFFFu);
            f[2 * i + 1] = h2f(w[i] >> 16);
        }
    }
    __device__ static float scalar(const _Float16* p) { return (float)*p; }
};
template <>
struct Elt<Bf16> {
    static constexpr int kVec = 8;
    static constexpr uint32_t kNegInfWord = 0xFF80FF80u;
    __device__ static void widen(const uint4& q, float (&f)[8]) {
        const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            f[2 * i] = __uint_as_float(w[i] << 16);
            f[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
        }
    }
    __device__ static float scalar(const Bf16* p) { return __uint_as_float((uint32_t)p->bits << 16); }
};

// Relaxed agent-scope accesses: coherent across the XCDs' L2 caches.
template <typename U>
__device__ __forceinline__ void st_agent(U* p, U v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename U>
__device__ __forceinline__ U ld_agent(const U* p) {
    return __hip_atomic_load(const_cast<U*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Workgroup barrier for LDS traffic only.  __syncthreads() also waits for
// this wave's global stores still in flight (a device round trip after a
// store); every exchange between the threads of a workgroup here goes
// through LDS, so only LDS is ordered.
__device__ __forceinline__ void lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// 16-byte nontemporal load: the logits are read exactly once per call.
__device__ __forceinline__ uint4 ld_nt(const void* p) {
    typedef unsigned u4v __attribute__((ext_vector_type(4)));
    const u4v q = __builtin_nontemporal_load((const u4v*)p);
    return make_uint4(q.x, q.y, q.z, q.w);
}

// Element e of a 16-byte slot, widened exactly to fp32.
template <typename T>
__device__ __forceinline__ float elt(const uint4& q, int e) {
    if constexpr (sizeof(T) == 4) {
        return __uint_as_float(e == 0 ? q.x : e == 1 ? q.y : e == 2 ? q.z : q.w);
    } else {
        const uint32_t w = (e >> 1) == 0 ? q.x : (e >> 1) == 1 ? q.y : (e >> 1) == 2 ? q.z : q.w;
        const uint32_t h = (e & 1) ? (w >> 16) : (w & 0xFFFFu);
        if constexpr (__is_same(T, Bf16)) return __uint_as_float(h << 16);
        else return Elt<_Float16>::h2f(h);
    }
}

// The entries of a 16-byte slot whose bit in `bits` is clear become the
// -inf pattern of their type (two instructions a 32-bit word).
template <typename T>
__device__ __forceinline__ uint4 fold_bits(const uint4& q, uint32_t bits) {
    constexpr int VEC = Elt<T>::kVec;
    uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        uint32_t keep;
        if constexpr (VEC == 4) {
            keep = (uint32_t)__builtin_amdgcn_sbfe((int)bits, i, 1);
        } else {
            keep = ((uint32_t)__builtin_amdgcn_sbfe((int)bits, 2 * i, 1) & 0xFFFFu) |
                   ((uint32_t)__builtin_amdgcn_sbfe((int)bits, 2 * i + 1, 1) << 16);
        }
        w[i] = (w[i] & keep) | (Elt<T>::kNegInfWord & ~keep);
    }
    return make_uint4(w[0], w[1], w[2], w[3]);
}


}  // namespace tms

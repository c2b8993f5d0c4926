// tms_spec.hip -- speculative accept/reject (stochastic verify) for gfx950.
//
// Two launches per call, both stream-ordered:
//
//   statistics    one record per row (the k + 1 target rows and the k draft
//                 rows of every sequence): m = max(v / T), the exact integer
//                 sum Z of the row's weights q44(exp64(v / T - m)), and the
//                 weight of the row's draft token.  16-byte aligned rows of
//                 up to 64K fp32 (32K fp16/bf16) ids: spec_row_kernel, one
//                 1024-thread workgroup per row holding the row in registers
//                 (one read); other rows: spec_stats_kernel, two passes.
//   spec_resolve  B x P workgroups.  Every workgroup of a sequence evaluates
//                 the accept tests u_i < p_t(x_i) / p_d(x_i) from the row
//                 statistics (the same decision in each), then sums the
//                 weights of its 1/P of the vocabulary for the distribution
//                 the final draw uses: the residual max(p_t - p_d, 0) at the
//                 first rejection, else the target row k (the bonus token).
//                 It publishes the partial sums, takes a ticket, and the last
//                 arriver finds the part holding the draw's threshold,
//                 recomputes that part's weights and locates the token.
//
// The weights are build-defined (no reference counterpart): exp64 is the
// table-driven exponential of tms_device.h, q44 rounds to multiples of 2^-44,
// so every sum is an exact int64 and independent of summation order.  The
// greedy limit (one-hot p_t and p_d) is the argmax-match rule of
// spec_generate_greedy (tensormark/llama.h:5127-5131).

#include <float.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

#include "../../include/tmsample_hip.h"
#include "tms_context.h"
#include "tms_device.h"

namespace tms {

__constant__ double kSpecExpTab[64] = {TMS_EXP2_64THS};
constexpr uint64_t kPartReady = 1ull << 63;   // published partial sum is complete
constexpr int kPartPoll = 1 << 20;            // bound on the finisher's wait per part

constexpr int kRowT = 1024;          // threads of the row kernel
constexpr int kRowW = kRowT / 64;

struct SArgs {
    const void* target;
    const void* draft;
    int B, k, V;
    bool fast;   // rows 16-byte aligned and V a multiple of the vector width
    int P, Lp;   // vocabulary parts of the two-launch resolve and their length
    bool lazy;   // the row kernel leaves the bonus rows (target row k) to the resolve
    const int32_t* tokens;
    const tms_row_params* params;
    const uint32_t* draws;
    int32_t* out_acc;
    int32_t* out_tok;
    int32_t* out_status;
    tms_spec_stat* stats;
    uint64_t* parts;
    uint32_t* tickets;   // [B][kCounterStride]: resolve parts, or rows of the row kernel
#ifdef TMS_TRACE
    uint64_t* trace;     // trace builds: 8 stamps per workgroup
#endif
};

#ifdef TMS_TRACE
#define SPEC_TR(i)                                                                                         \
    do {                                                                                                   \
        if (threadIdx.x == 0 && a.trace) a.trace[blockIdx.x * 8 + (i)] = __builtin_amdgcn_s_memrealtime(); \
    } while (0)
#else
#define SPEC_TR(i) ((void)0)
#endif

// LDS of a verify workgroup (up to 16 waves).
struct SpecLds {
    double tab[64];
    float shf[kRowW];
    int64_t shl[2 * kRowW];
    int64_t part_w[kSpecParts];
    int64_t part_t[kSpecParts];
    int misc[kRowW];
    tms_spec_stat srow[2 * kSpecMaxK + 1];
    int stok[kSpecMaxK];
    double su[kSpecMaxK];
};

__device__ __forceinline__ void load_exp_table(double* tab) {
    if (threadIdx.x < 64) tab[threadIdx.x] = kSpecExpTab[threadIdx.x];
}

// Row i of sequence b: i <= k is target row i, i > k is draft row i - k - 1.
template <typename T>
__device__ __forceinline__ const T* spec_row(const SArgs& a, int b, int i) {
    if (i <= a.k) return (const T*)a.target + ((int64_t)b * (a.k + 1) + i) * a.V;
    return (const T*)a.draft + ((int64_t)b * a.k + (i - a.k - 1)) * a.V;
}

// f(id, value) over ids [lo, hi) of a row, strided over the workgroup.  The
// vector path needs lo and hi multiples of the vector width.
template <typename T, typename F>
__device__ __forceinline__ void for_range(const T* row, int lo, int hi, bool fast, F&& f) {
    constexpr int VEC = Elt<T>::kVec;
    if (fast) {
#pragma unroll 4
        for (int v = lo / VEC + (int)threadIdx.x; v < hi / VEC; v += kBlock) {
            const uint4 q = *(const uint4*)(row + (int64_t)v * VEC);
            float x[VEC];
            Elt<T>::widen(q, x);
#pragma unroll
            for (int e = 0; e < VEC; ++e) f(v * VEC + e, x[e]);
        }
    } else {
        for (int i = lo + (int)threadIdx.x; i < hi; i += kBlock) f(i, Elt<T>::scalar(row + i));
    }
}

// The same over two rows at once: f(id, value of r0, value of r1).
template <typename T, typename F>
__device__ __forceinline__ void for_range2(const T* r0, const T* r1, int lo, int hi, bool fast, F&& f) {
    constexpr int VEC = Elt<T>::kVec;
    if (fast) {
#pragma unroll 2
        for (int v = lo / VEC + (int)threadIdx.x; v < hi / VEC; v += kBlock) {
            const uint4 q0 = *(const uint4*)(r0 + (int64_t)v * VEC);
            const uint4 q1 = *(const uint4*)(r1 + (int64_t)v * VEC);
            float x0[VEC], x1[VEC];
            Elt<T>::widen(q0, x0);
            Elt<T>::widen(q1, x1);
#pragma unroll
            for (int e = 0; e < VEC; ++e) f(v * VEC + e, x0[e], x1[e]);
        }
    } else {
        for (int i = lo + (int)threadIdx.x; i < hi; i += kBlock)
            f(i, Elt<T>::scalar(r0 + i), Elt<T>::scalar(r1 + i));
    }
}

template <int NW = kWaves>
__device__ __forceinline__ float block_max_f32(float v, float* sh) {
    v = wave_max_f32(v);
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
    __syncthreads();
    float r = sh[0];
#pragma unroll
    for (int i = 1; i < NW; ++i) r = fmaxf(r, sh[i]);
    __syncthreads();
    return r;
}

template <int NW = kWaves>
__device__ __forceinline__ int64_t block_sum_i64(int64_t v, int64_t* sh) {
    v = wave_sum_i64(v);
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
    __syncthreads();
    int64_t r = 0;
#pragma unroll
    for (int i = 0; i < NW; ++i) r += sh[i];
    __syncthreads();
    return r;
}

template <int NW = kWaves>
__device__ __forceinline__ int block_or(int v, int* sh) {
    v = __any(v) ? 1 : 0;
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
    __syncthreads();
    int r = 0;
#pragma unroll
    for (int i = 0; i < NW; ++i) r |= sh[i];
    __syncthreads();
    return r;
}

// v / T.  The hot loops are instantiated twice, DIV false for T = 1 (where
// the division is the identity) and true otherwise, and pick one per row:
// a per-element test compiles to a select that still divides.
template <bool DIV = true>
__device__ __forceinline__ float scaled(float v, float temp) { return DIV ? v / temp : v; }

// Weight of a scaled logit on the 2^-44 grid: q44(exp64(v / T - m)), where m
// is the maximum of v / T over the row, so the argument is never positive.
template <bool DIV = true>
__device__ __forceinline__ int64_t weight(float v, float temp, double m, const double* tab) {
    return q44_exp_nonpos((double)scaled<DIV>(v, temp) - m, tab);
}

// The same weight as a double holding the whole number.
template <bool DIV = true>
__device__ __forceinline__ double weight_f(float v, float temp, double m, const double* tab) {
    return q44_exp_nonpos_f((double)scaled<DIV>(v, temp) - m, tab);
}

// Residual weight q44(max(p_t - p_d, 0)) from the two rows' weights (whole
// numbers as doubles), p = e / (double)Z.  The divisors' reciprocals are
// formed once (Resid), and div_rn returns the correctly rounded quotients,
// the same as dividing per element.  Z >= 2^44 for a row that reaches here
// (its maximum has weight 2^44), so nothing overflows or is subnormal.
struct Resid {
    double zt, zd, yt, yd;
    __device__ __forceinline__ Resid(int64_t Zt, int64_t Zd)
        : zt((double)Zt), zd((double)Zd), yt(1.0 / (double)Zt), yd(1.0 / (double)Zd) {}
    __device__ __forceinline__ int64_t operator()(double et, double ed) const {
        const double d = div_rn(et, zt, yt) - div_rn(ed, zd, yd);
        return d > 0.0 ? q44(d) : 0;
    }
};

__device__ __forceinline__ int64_t as_i64(double f) {
    return __double_as_longlong(f + 0x1p52) - __double_as_longlong(0x1p52);
}

template <typename T>
__global__ __launch_bounds__(kBlock) void spec_stats_kernel(SArgs a) {
    __shared__ double tab[64];
    __shared__ float shf[kWaves];
    __shared__ int64_t shl[kWaves];
    __shared__ int shi[kWaves];
    load_exp_table(tab);
    const int R = 2 * a.k + 1;
    const int g = blockIdx.x;
    const int b = g / R, i = g - b * R;
    const T* row = spec_row<T>(a, b, i);
    const float temp = a.params[b].temperature;

    float mx = -__builtin_huge_valf();
    int nf = 0;
    for_range(row, 0, a.V, a.fast, [&](int, float v) {
        nf |= __builtin_amdgcn_class(v, 0x203);   // NaN or +inf
        mx = fmaxf(mx, scaled(v, temp));
    });
    mx = block_max_f32(mx, shf);   // also orders the table's LDS writes
    nf = block_or(nf, shi);
    int st = TMS_ROW_OK;
    if (nf) st = TMS_ROW_NONFINITE;
    else if (mx == -__builtin_huge_valf()) st = TMS_ROW_ALL_MASKED;
    else if (mx == __builtin_huge_valf()) st = TMS_ROW_NONFINITE;
    const double md = (double)mx;
    int64_t z = 0;
    if (st == TMS_ROW_OK) {
        for_range(row, 0, a.V, a.fast, [&](int, float v) { z += weight(v, temp, md, tab); });
        z = block_sum_i64(z, shl);
    }
    if (threadIdx.x == 0) {
        const int di = i < a.k ? i : (i > a.k ? i - a.k - 1 : -1);
        int64_t ex = 0;
        if (st == TMS_ROW_OK && di >= 0) {
            const int x = a.tokens[(int64_t)b * a.k + di];
            if (x >= 0 && x < a.V) ex = weight(Elt<T>::scalar(row + x), temp, md, tab);
        }
        // Agent-scope stores, as the chunked statistics write theirs: rows on
        // different XCDs share cache lines of the record array.
        uint64_t* w = (uint64_t*)(a.stats + g);
        st_agent(&w[0], (uint64_t)__float_as_uint(mx) | ((uint64_t)(uint32_t)st << 32));
        st_agent(&w[1], (uint64_t)z);
        st_agent(&w[2], (uint64_t)ex);
        st_agent(&w[3], (uint64_t)0);
    }
}

// Loops over a thread's registers (slot sl holds vector t + sl * NT, in
// while below nv): the max of v / T and the NaN/+inf flag, then the share
// of Z.
template <typename T, int NS, int NT, bool DIV>
__device__ __forceinline__ void row_max(const uint4 (&q)[NS], int nv, float temp, float& mx, int& nf) {
    constexpr int VEC = Elt<T>::kVec;
    const int t = threadIdx.x;
#pragma unroll
    for (int sl = 0; sl < NS; ++sl) {
        const bool in = t + sl * NT < nv;
        float x[VEC];
        Elt<T>::widen(q[sl], x);
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
            nf |= in ? __builtin_amdgcn_class(x[e], 0x203) : 0;   // NaN or +inf
            mx = in ? fmaxf(mx, scaled<DIV>(x[e], temp)) : mx;
        }
    }
}
template <typename T, int NS, int NT, bool DIV>
__device__ __forceinline__ int64_t row_z(const uint4 (&q)[NS], int nv, float temp, double md, const double* tab) {
    constexpr int VEC = Elt<T>::kVec;
    const int t = threadIdx.x;
    // whole numbers of at most 2^44 each, at most 128 of them: the double
    // sum is exact
    static_assert(NS * VEC <= 128, "exact double sum");
    double z = 0.0;
#pragma unroll
    for (int sl = 0; sl < NS; ++sl) {
        float x[VEC];
        Elt<T>::widen(q[sl], x);
        if (t + sl * NT < nv) {
#pragma unroll
            for (int e = 0; e < VEC; ++e) z += q44_exp_nonpos_f((double)scaled<DIV>(x[e], temp) - md, tab);
        }
    }
    return __double_as_longlong(z + 0x1p52) - __double_as_longlong(0x1p52);
}

// The sequence's statistics, draft tokens and accept uniforms staged in LDS
// (one load or Philox draw per thread), then the accept tests
// u_i < (e_t * Z_d) / (e_d * Z_t), evaluated identically by every workgroup
// that runs them.  rej < 0: every draft accepted (the bonus draw).
template <typename T>
__device__ void accept_tests(const SArgs& a, int b, SpecLds& L, int& status, int& acc, int& rej) {
    const int t = threadIdx.x;
    const int R = 2 * a.k + 1;
    const tms_row_params P = a.params[b];
    const int g0 = b * R;
    const uint32_t* dw = a.draws ? a.draws + (int64_t)b * (a.k + 1) * 2 : nullptr;
    if (t < R) {
        const uint64_t* w = (const uint64_t*)(a.stats + g0 + t);
        const uint64_t w0 = ld_agent(&w[0]);
        L.srow[t].m = __uint_as_float((uint32_t)w0);
        L.srow[t].status = (int32_t)(w0 >> 32);
        L.srow[t].Z = (int64_t)ld_agent(&w[1]);
        L.srow[t].ex = (int64_t)ld_agent(&w[2]);
        L.srow[t].pad = 0;
    }
    if (t < a.k) {
        L.stok[t] = a.tokens[(int64_t)b * a.k + t];
        uint32_t w0, w1;
        if (dw) { w0 = dw[2 * t]; w1 = dw[2 * t + 1]; }
        else row_words(P.seed, P.offset, (uint32_t)t, w0, w1);
        L.su[t] = canonical(w0, w1);
    }
    __syncthreads();
    status = TMS_ROW_OK;
    acc = 0;
    rej = -1;
    if (!(P.temperature > 0.0f && P.temperature <= FLT_MAX)) {
        status = TMS_ROW_BAD_PARAMS;
        return;
    }
    acc = a.k;
    // Lane i < k of every wave evaluates position i (the same operations as
    // a loop over i would); the lowest position that is not an accept
    // decides, as the first exit of that loop would.
    const int lane = t & 63;
    int code = 0;   // 0: accepted, 1: rejected, 2: the row's status sv
    int sv = TMS_ROW_OK;
    if (lane < a.k) {
        const tms_spec_stat ts = L.srow[lane], ds = L.srow[a.k + 1 + lane];
        const int x = L.stok[lane];
        if (ts.status) {
            code = 2;
            sv = ts.status;
        } else if (ds.status) {
            code = 2;
            sv = ds.status;
        } else if (x < 0 || x >= a.V) {
            code = 2;
            sv = TMS_ROW_BAD_PARAMS;
        } else {
            double r;
            if (ds.ex == 0) r = ts.ex > 0 ? 1.0 : 0.0;
            else r = ((double)ts.ex * (double)ds.Z) / ((double)ds.ex * (double)ts.Z);
            code = L.su[lane] < r ? 0 : 1;
        }
    }
    const uint64_t stop = __ballot(lane < a.k && code != 0);
    if (stop) {
        const int i = __builtin_ctzll(stop);
        const int ci = __shfl(code, i, 64);
        if (ci == 2) {
            status = __shfl(sv, i, 64);
            return;
        }
        acc = i;
        rej = i;
    }
    if (rej < 0 && !a.lazy && L.srow[a.k].status) status = L.srow[a.k].status;
}

// Part p of sequence b's resolution.
// WAIT (the whole grid resident at once, runs of at most kRunMax ids): every
// workgroup keeps its part's weights in registers, reads every part's sums
// (bounded wait), and the one whose part holds the draw's threshold locates
// the token from its registers; the last reader (by a done counter) zeroes
// the parts.  Otherwise the last arriver by ticket gathers the parts and
// recomputes the weights of the part holding the threshold.
constexpr int kRunMax = 16;
template <typename T, bool WAIT>
__device__ void resolve_part(const SArgs& a, int b, int p, SpecLds& L) {
    const double* tab = L.tab;
    int64_t* shl = L.shl;
    int64_t* part_w = L.part_w;
    int64_t* part_t = L.part_t;
    int* misc = L.misc;
    const tms_spec_stat* srow = L.srow;
    const int t = threadIdx.x;
    const tms_row_params P = a.params[b];
    const uint32_t* dw = a.draws ? a.draws + (int64_t)b * (a.k + 1) * 2 : nullptr;
    int status, acc, rej;
    SPEC_TR(0);
    accept_tests<T>(a, b, L, status, acc, rej);
    SPEC_TR(1);
    if (status != TMS_ROW_OK) {
        if (p == 0 && t == 0) {
            a.out_acc[b] = 0;
            a.out_tok[b] = -1;
            a.out_status[b] = status;
        }
        return;   // every workgroup of the sequence returns here: no ticket
    }

    // ---- this part's sums: the draw's weights (w) and the target's (et).
    const int ti = rej < 0 ? a.k : rej;
    const T* rt = spec_row<T>(a, b, ti);
    const T* rd = spec_row<T>(a, b, rej < 0 ? ti : a.k + 1 + rej);
    const tms_spec_stat ts = srow[ti];
    const tms_spec_stat ds = rej < 0 ? ts : srow[a.k + 1 + rej];
    const float temp = P.temperature;
    const double mt = (double)ts.m, md = (double)ds.m;
    const Resid res(ts.Z, ds.Z);
    __syncthreads();   // exp table in LDS
    const int lo = p * a.Lp, hi = min(a.V, lo + a.Lp);
    int64_t wsum = 0, tsum = 0;
    int64_t wr[kRunMax], er[kRunMax];   // WAIT: the run's draw and target weights
    if constexpr (WAIT) {
        // a contiguous run of ids per thread, every load issued at once
        const int E = (hi - lo + kBlock - 1) / kBlock;
        const int r_lo = min(hi, lo + t * E), r_hi = min(hi, r_lo + E);
        float xt[kRunMax], xd[kRunMax];
#pragma unroll
        for (int j = 0; j < kRunMax; ++j) {
            const int id = min(r_lo + j, hi - 1);
            xt[j] = j < E ? Elt<T>::scalar(rt + id) : 0.0f;
            xd[j] = (j < E && rej >= 0) ? Elt<T>::scalar(rd + id) : 0.0f;
        }
        double mtu = mt;
        if (a.lazy && rej < 0) {
            // The bonus row's statistics (the row kernel left them): each
            // part's max of v / T and NaN / +inf flag, exchanged between the
            // sequence's workgroups; the status rules of the statistics
            // kernels (tmo_spec_weights).
            float pm = -__builtin_huge_valf();
            int pnf = 0;
#pragma unroll
            for (int j = 0; j < kRunMax; ++j) {
                if (r_lo + j < r_hi) {
                    const float v = xt[j];
                    pnf |= (__builtin_isnan(v) || v == __builtin_huge_valf()) ? 1 : 0;
                    pm = fmaxf(pm, scaled(v, temp));
                }
            }
            pm = block_max_f32(pm, L.shf);
            pnf = block_or(pnf, misc);
            uint64_t* mw = a.parts + ((int64_t)b * kSpecParts + p) * kPartWords + 2;
            if (t == 0) st_agent(mw, kPartReady | ((uint64_t)pnf << 32) | okey(pm));
            int bad = 0;
            uint32_t km = 0;
            int knf = 0;
            if (t < a.P) {
                const uint64_t* q = a.parts + ((int64_t)b * kSpecParts + t) * kPartWords + 2;
                uint64_t h = 0;
                for (int it = 0; it < kPartPoll; ++it) {
                    h = ld_agent(q);
                    if (h & kPartReady) break;
                    __builtin_amdgcn_s_sleep(1);
                }
                bad = (h & kPartReady) ? 0 : 1;
                km = (uint32_t)h;
                knf = (int)((h >> 32) & 1u);
            }
            // the bonus maxima's readers: the last zeroes the words and its
            // counter.  The waves' maxima meet in part_w, whose next writes
            // (the part sums' gather) come after the sums' barriers; shl is
            // the sums' own scratch.
            km = (uint32_t)wave_max_u64(km);
            if ((t & 63) == 0) part_w[t >> 6] = (int64_t)km;
            bad = block_or(bad, misc);
            knf = block_or(knf, misc);
            if (t == 0) {
                const uint32_t done = __hip_atomic_fetch_add(&a.tickets[b * kCounterStride + 1], 1u,
                                                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                misc[2] = done == (uint32_t)(a.P - 1) ? 1 : 0;
            }
            __syncthreads();
            uint32_t kmax = (uint32_t)part_w[0];
            for (int w = 1; w < kWaves; ++w) kmax = max(kmax, (uint32_t)part_w[w]);
            if (misc[2]) {
                if (t < a.P) st_agent(a.parts + ((int64_t)b * kSpecParts + t) * kPartWords + 2, (uint64_t)0);
                if (t == 0) st_agent(&a.tickets[b * kCounterStride + 1], 0u);
            }
            const float gm = okey_inv(kmax);
            int st = TMS_ROW_OK;
            if (bad) st = TMS_ROW_INTERNAL;
            else if (knf) st = TMS_ROW_NONFINITE;
            else if (gm == -__builtin_huge_valf()) st = TMS_ROW_ALL_MASKED;
            else if (gm == __builtin_huge_valf()) st = TMS_ROW_NONFINITE;
            if (st != TMS_ROW_OK) {
                if (p == 0 && t == 0) {
                    a.out_acc[b] = 0;
                    a.out_tok[b] = -1;
                    a.out_status[b] = st;
                }
                return;   // every workgroup of the sequence: no parts published
            }
            mtu = (double)gm;
        }
#pragma unroll
        for (int j = 0; j < kRunMax; ++j) {
            er[j] = 0;
            wr[j] = 0;
            if (r_lo + j < r_hi) {
                const double etf = weight_f(xt[j], temp, mtu, tab);
                er[j] = as_i64(etf);
                wr[j] = rej < 0 ? er[j] : res(etf, weight_f(xd[j], temp, md, tab));
            }
            tsum += er[j];
            wsum += wr[j];
        }
    } else if (rej < 0) {
        for_range(rt, lo, hi, a.fast, [&](int, float v) { tsum += weight(v, temp, mt, tab); });
        wsum = tsum;
    } else {
        for_range2(rt, rd, lo, hi, a.fast, [&](int, float vt, float vd) {
            const double et = weight_f(vt, temp, mt, tab);
            tsum += as_i64(et);
            wsum += res(et, weight_f(vd, temp, md, tab));
        });
    }
    wsum = block_sum_i64(wsum, shl);
    tsum = block_sum_i64(tsum, shl + kWaves);
    SPEC_TR(2);
    uint64_t* pw = a.parts + ((int64_t)b * kSpecParts + p) * kPartWords;
    if constexpr (WAIT) {
        if (t == 0) {
            st_agent(&pw[0], kPartReady | (uint64_t)wsum);
            st_agent(&pw[1], kPartReady | (uint64_t)tsum);
        }
    } else {
        uint32_t ticket = 0;
        if (t == 0) {
            st_agent(&pw[0], kPartReady | (uint64_t)wsum);
            st_agent(&pw[1], kPartReady | (uint64_t)tsum);
            ticket = __hip_atomic_fetch_add(&a.tickets[b * kCounterStride], 1u, __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_AGENT);
            misc[0] = (int)ticket;
        }
        __syncthreads();
        SPEC_TR(3);
        if (misc[0] != a.P - 1) return;
        // the last arriver: its ticket for the next call
        if (t == 0) st_agent(&a.tickets[b * kCounterStride], 0u);
    }

    // ---- gather the parts (bounded wait on their ready bits); the reader
    //      that is last zeroes them for the next call.
    int timed_out = 0;
    if (t < a.P) {
        uint64_t* q = a.parts + ((int64_t)b * kSpecParts + t) * kPartWords;
        uint64_t w = 0, u = 0;
        for (int it = 0; it < kPartPoll; ++it) {
            w = ld_agent(&q[0]);
            u = ld_agent(&q[1]);
            if ((w & kPartReady) && (u & kPartReady)) break;
            __builtin_amdgcn_s_sleep(1);
        }
        timed_out = !((w & kPartReady) && (u & kPartReady));
        part_w[t] = (int64_t)(w & ~kPartReady);
        part_t[t] = (int64_t)(u & ~kPartReady);
        if (!WAIT) {
            st_agent(&q[0], (uint64_t)0);
            st_agent(&q[1], (uint64_t)0);
        }
    }
    timed_out = block_or(timed_out, misc);
    if constexpr (WAIT) {
        // every word read: the last of the P readers (a relaxed counter; each
        // adds after its loads returned) zeroes the parts and the counter
        if (t == 0) {
            const uint32_t done = __hip_atomic_fetch_add(&a.tickets[b * kCounterStride], 1u, __ATOMIC_RELAXED,
                                                         __HIP_MEMORY_SCOPE_AGENT);
            misc[1] = done == (uint32_t)(a.P - 1) ? 1 : 0;
        }
        __syncthreads();
        if (misc[1]) {
            if (t < a.P) {
                uint64_t* q = a.parts + ((int64_t)b * kSpecParts + t) * kPartWords;
                st_agent(&q[0], (uint64_t)0);
                st_agent(&q[1], (uint64_t)0);
            }
            if (t == 0) st_agent(&a.tickets[b * kCounterStride], 0u);
        }
    }
    SPEC_TR(4);
    if (timed_out) {
        if (t == 0 && (!WAIT || p == 0)) {
            a.out_acc[b] = 0;
            a.out_tok[b] = -1;
            a.out_status[b] = TMS_ROW_INTERNAL;
        }
        return;
    }
    // The parts' sums across the lanes of each wave (P <= 64), by integer
    // scans: exact, so W, the threshold's part and the sum before it equal
    // the sequential sums.  Residual mass 0 (p_t <= p_d everywhere on the
    // grid): draw from p_t.
    static_assert(kSpecParts <= 64, "one part per lane");
    const int pl = t & 63;
    const int64_t sw = wave_incl_scan_i64_dpp(pl < a.P ? part_w[pl] : 0);
    const int64_t st = wave_incl_scan_i64_dpp(pl < a.P ? part_t[pl] : 0);
    int64_t W = readlane_i64(sw, 63);
    const bool use_t = rej < 0 || W == 0;
    if (use_t) W = readlane_i64(st, 63);
    uint32_t w0, w1;
    if (dw) { w0 = dw[2 * a.k]; w1 = dw[2 * a.k + 1]; }
    else row_words(P.seed, P.offset, (uint32_t)a.k, w0, w1);
    const double uf = canonical(w0, w1);
    int64_t thr = (int64_t)floor(uf * (double)W);
    if (thr > W - 1) thr = W - 1;
    // the first part whose inclusive sum exceeds thr (the last one does:
    // thr < W), and the sum of the parts before it
    const int64_t sc = use_t ? st : sw;
    const uint64_t over = __ballot(pl < a.P && sc > thr);
    const int ps = over ? __ffsll((unsigned long long)over) - 1 : a.P - 1;
    const int64_t base = ps > 0 ? readlane_i64(sc, ps - 1) : 0;
    if (WAIT && ps != p) return;   // another workgroup holds the threshold's part
    SPEC_TR(6);
    // The part's weights, a contiguous run of ids per thread.
    const int plo = ps * a.Lp, phi = min(a.V, plo + a.Lp);
    const int E = (phi - plo + kBlock - 1) / kBlock;
    const int my_lo = min(phi, plo + t * E), my_hi = min(phi, my_lo + E);
    auto w_at = [&](int id) -> int64_t {
        const double et = weight_f(Elt<T>::scalar(rt + id), temp, mt, tab);
        if (use_t) return as_i64(et);
        return res(et, weight_f(Elt<T>::scalar(rd + id), temp, md, tab));
    };
    // Runs of up to kRunMax ids: every load issued at once (clamped
    // addresses), the weights kept in registers for the scan and the search;
    // longer runs walk the ids one by one.  WAIT: this workgroup's own run
    // weights, still in registers.
    const bool cached = WAIT || E <= kRunMax;
    int64_t wc[kRunMax];
    int64_t mine = 0;
    if constexpr (WAIT) {
#pragma unroll
        for (int j = 0; j < kRunMax; ++j) {
            wc[j] = use_t ? er[j] : wr[j];
            mine += wc[j];
        }
    } else if (cached) {
        float xt[kRunMax], xd[kRunMax];
#pragma unroll
        for (int j = 0; j < kRunMax; ++j) {
            const int id = min(my_lo + j, phi - 1);
            xt[j] = Elt<T>::scalar(rt + id);
            xd[j] = use_t ? 0.0f : Elt<T>::scalar(rd + id);
        }
#pragma unroll
        for (int j = 0; j < kRunMax; ++j) {
            wc[j] = 0;
            if (my_lo + j < my_hi) {
                const double et = weight_f(xt[j], temp, mt, tab);
                wc[j] = use_t ? as_i64(et) : res(et, weight_f(xd[j], temp, md, tab));
            }
            mine += wc[j];
        }
    } else {
        for (int id = my_lo; id < my_hi; ++id) mine += w_at(id);
    }
    SPEC_TR(7);
    // Exclusive scan of the threads' sums.
    const int lane = t & 63, wv = t >> 6;
    const int64_t inc = wave_incl_scan_i64(mine);
    if (lane == 63) shl[wv] = inc;
    __syncthreads();
    SPEC_TR(5);
    int64_t pre = base;
    for (int i = 0; i < wv; ++i) pre += shl[i];
    pre += inc - mine;
    if (mine > 0 && pre <= thr && thr < pre + mine) {
        int64_t acc_w = pre;
        int tok = my_hi - 1;
        if (cached) {
            bool found = false;
#pragma unroll
            for (int j = 0; j < kRunMax; ++j) {
                acc_w += wc[j];
                if (!found && my_lo + j < my_hi && acc_w > thr) {
                    tok = my_lo + j;
                    found = true;
                }
            }
        } else {
            for (int id = my_lo; id < my_hi; ++id) {
                acc_w += w_at(id);
                if (acc_w > thr) { tok = id; break; }
            }
        }
        a.out_acc[b] = acc;
        a.out_tok[b] = tok;
        a.out_status[b] = TMS_ROW_OK;
    }
}


#ifdef TMS_TRACE
static uint64_t* g_spec_trace;
extern "C" int tms_spec_trace_set(uint64_t* buf) {
    g_spec_trace = buf;
    return 0;
}
#endif

template <typename T, bool WAIT>
__global__ __launch_bounds__(kBlock) void spec_resolve_kernel(SArgs a) {
    __shared__ SpecLds L;
    load_exp_table(L.tab);
    resolve_part<T, WAIT>(a, blockIdx.x / a.P, blockIdx.x % a.P, L);
}

// Row statistics for 16-byte aligned rows of at most kRowT x NS vectors:
// one 1024-thread workgroup per row holds the row in registers (one read)
// and writes the row's record: m = max(v / T), the status,
// Z = sum of q44(exp64(v / T - m)) and the draft token's weight, equal to
// spec_stats_kernel's.  Two workgroups per CU (64 registers a thread) up to
// 8 vectors a thread.  The parts-wise resolve follows on the stream.
template <typename T, int NS>
__global__ __launch_bounds__(kRowT) __attribute__((amdgpu_waves_per_eu(NS <= 8 ? 8 : 4, 8)))
void spec_row_kernel(SArgs a) {
    constexpr int VEC = Elt<T>::kVec;
    __shared__ SpecLds L;
    load_exp_table(L.tab);
    const int t = threadIdx.x;
    // lazy: 2k rows a sequence (the bonus row k left to the resolve)
    const int R = a.lazy ? 2 * a.k : 2 * a.k + 1;
    const int g = blockIdx.x;
    const int b = g / R;
    int i = g - b * R;
    if (a.lazy && i >= a.k) ++i;
    const T* row = spec_row<T>(a, b, i);
    const float temp = a.params[b].temperature;
    const bool div = temp != 1.0f;
    const int nv = a.V / VEC;
    uint4 q[NS];
#pragma unroll
    for (int sl = 0; sl < NS; ++sl) q[sl] = *(const uint4*)(row + (int64_t)min(t + sl * kRowT, nv - 1) * VEC);
    // The draft token's logit (draft rows; target row i takes draft i's
    // token), loaded now, after the stream's loads: it is in flight under
    // the max and the sums, and its weight is formed at the end.
    const int di = i < a.k ? i : (i > a.k ? i - a.k - 1 : -1);
    bool xin = false;
    float xv = 0.0f;
    if (t == 0 && di >= 0) {
        const int x = a.tokens[(int64_t)b * a.k + di];
        xin = x >= 0 && x < a.V;
        if (xin) xv = Elt<T>::scalar(row + x);
    }
    float mx = -__builtin_huge_valf();
    int nf = 0;
    if (div) row_max<T, NS, kRowT, true>(q, nv, temp, mx, nf);
    else row_max<T, NS, kRowT, false>(q, nv, temp, mx, nf);
    // The row's maximum and NaN/+inf flag in one exchange: each wave's pair
    // in LDS words written once, so one barrier (which also orders the
    // table's LDS writes) and none after the reads.
    {
        const float wm = wave_max_f32(mx);
        const int wn = __any(nf) ? 1 : 0;
        if ((t & 63) == 0) {
            L.shf[t >> 6] = wm;
            L.misc[t >> 6] = wn;
        }
        lds_sync();
        mx = L.shf[0];
        nf = L.misc[0];
#pragma unroll
        for (int i = 1; i < kRowW; ++i) {
            mx = fmaxf(mx, L.shf[i]);
            nf |= L.misc[i];
        }
    }
    int st = TMS_ROW_OK;
    if (nf) st = TMS_ROW_NONFINITE;
    else if (mx == -__builtin_huge_valf()) st = TMS_ROW_ALL_MASKED;
    else if (mx == __builtin_huge_valf()) st = TMS_ROW_NONFINITE;
    const double md = (double)mx;
    int64_t z = 0;
    if (st == TMS_ROW_OK)
        z = div ? row_z<T, NS, kRowT, true>(q, nv, temp, md, L.tab) : row_z<T, NS, kRowT, false>(q, nv, temp, md, L.tab);
    {   // Z: each wave's share in LDS words written once (one barrier)
        const int64_t wz = wave_sum_i64(z);
        if ((t & 63) == 0) L.shl[t >> 6] = wz;
        lds_sync();
        z = 0;
        if (t == 0)
#pragma unroll
            for (int i = 0; i < kRowW; ++i) z += L.shl[i];
    }
    if (t == 0) {
        const int64_t ex = (st == TMS_ROW_OK && xin) ? weight(xv, temp, md, L.tab) : 0;
        uint64_t* w = (uint64_t*)(a.stats + (int64_t)b * (2 * a.k + 1) + i);
        st_agent(&w[0], (uint64_t)__float_as_uint(mx) | ((uint64_t)(uint32_t)st << 32));
        st_agent(&w[1], (uint64_t)z);
        st_agent(&w[2], (uint64_t)ex);
        st_agent(&w[3], (uint64_t)0);
    }
}

}  // namespace tms

// Whether a resolve grid of n workgroups is resident at once on the current
// device (occupancy of the waiting form x compute units, looked up once per
// device and type): the waiting form's workgroups wait on each other.
template <typename T>
static bool resolve_resident(int n) {
    constexpr int kMaxDevices = 64;
    static std::atomic<int> cap[kMaxDevices];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return false;
    int c = cap[dev].load(std::memory_order_relaxed);
    if (c == 0) {
        int per_cu = 0, cus = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, tms::spec_resolve_kernel<T, true>, tms::kBlock, 0) !=
                hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            return false;
        c = per_cu * cus > 0 ? per_cu * cus : -1;
        cap[dev].store(c, std::memory_order_relaxed);
    }
    return c > 0 && n <= c;
}

extern "C" int tms_spec_verify(tms_context* ctx, const tms_spec_args* a, hipStream_t stream) {
    if (!ctx || !a || !a->target_logits || !a->draft_logits || !a->draft_tokens || !a->params ||
        !a->out_accepted || !a->out_token || !a->out_status)
        return TMS_ERR_INVALID_ARG;
    if (a->batch <= 0 || a->k < 1 || a->k > tms::kSpecMaxK || a->vocab <= 0)
        return TMS_ERR_INVALID_ARG;
    if (a->batch > ctx->max_batch || a->vocab > ctx->max_vocab) return TMS_ERR_CAPACITY;
    int esz;
    switch (a->dtype) {
        case TMS_DTYPE_F32: esz = 4; break;
        case TMS_DTYPE_F16:
        case TMS_DTYPE_BF16: esz = 2; break;
        default: return TMS_ERR_INVALID_ARG;
    }
    const int vec = 16 / esz;
    tms::SArgs s{};
    s.target = a->target_logits;
    s.draft = a->draft_logits;
    s.B = a->batch;
    s.k = a->k;
    s.V = a->vocab;
    s.fast = ((uintptr_t)a->target_logits % 16 == 0) && ((uintptr_t)a->draft_logits % 16 == 0) &&
             (a->vocab % vec == 0);
    // Parts of about 2K ids, at most kSpecParts, each a multiple of 8 ids.
    int P = (a->vocab + 2047) / 2048;
    P = P < 1 ? 1 : (P > tms::kSpecParts ? tms::kSpecParts : P);
    s.Lp = ((a->vocab + P - 1) / P + 7) / 8 * 8;
    s.P = (a->vocab + s.Lp - 1) / s.Lp;
    s.tokens = a->draft_tokens;
    s.params = a->params;
    s.draws = a->draws;
    s.out_acc = a->out_accepted;
    s.out_tok = a->out_token;
    s.out_status = a->out_status;
    s.stats = ctx->spec_stats;
    s.parts = ctx->spec_parts;
    s.tickets = ctx->spec_tickets;
#ifdef TMS_TRACE
    s.trace = tms::g_spec_trace;
#endif
    // 16-byte aligned rows of at most kRowT x 16 vectors (fp32) or x 4
    // (fp16, bf16: 8 spill): the row kernel (two workgroups per CU up to 8
    // vectors a thread); others: the per-row statistics.  Then the resolve.
    const int R = 2 * a->k + 1;
    const int slots = (a->vocab / vec + tms::kRowT - 1) / tms::kRowT;
    const int max_ns = esz == 4 ? 16 : 4;
    const int row_ns = (!s.fast || slots > max_ns) ? 0 : slots <= 4 ? 4 : slots <= 8 ? 8 : 16;
    const dim3 block(tms::kBlock);
    const dim3 g2((unsigned)(a->batch * s.P));
    const dim3 brow(tms::kRowT);
    // The waiting resolve (its grid resident at once, runs of at most
    // kRunMax ids) takes the bonus rows' statistics itself when the row
    // kernel runs: 2k rows a sequence there (config 4: 512 rows, one round
    // of two workgroups per CU, in place of 544).
#define TMS_SPEC_LAUNCH(T, NS2, NS3)                                                       \
    do {                                                                                   \
        const bool wait = resolve_resident<T>(a->batch * s.P) &&                          \
                          (s.Lp + tms::kBlock - 1) / tms::kBlock <= tms::kRunMax;          \
        s.lazy = wait && row_ns > 0;                                                       \
        const dim3 g1((unsigned)(a->batch * (s.lazy ? R - 1 : R)));                        \
        if (row_ns > 0) {                                                                  \
            if (row_ns == 4)                                                               \
                hipLaunchKernelGGL((tms::spec_row_kernel<T, 4>), g1, brow, 0, stream, s);  \
            else if (row_ns == 8)                                                          \
                hipLaunchKernelGGL((tms::spec_row_kernel<T, NS2>), g1, brow, 0, stream, s);\
            else                                                                           \
                hipLaunchKernelGGL((tms::spec_row_kernel<T, NS3>), g1, brow, 0, stream, s);\
        } else {                                                                           \
            hipLaunchKernelGGL(tms::spec_stats_kernel<T>, g1, block, 0, stream, s);        \
        }                                                                                  \
        if (wait)                                                                          \
            hipLaunchKernelGGL((tms::spec_resolve_kernel<T, true>), g2, block, 0, stream, s);  \
        else                                                                               \
            hipLaunchKernelGGL((tms::spec_resolve_kernel<T, false>), g2, block, 0, stream, s); \
    } while (0)
    switch (a->dtype) {
        case TMS_DTYPE_F32: TMS_SPEC_LAUNCH(float, 8, 16); break;
        case TMS_DTYPE_F16: TMS_SPEC_LAUNCH(_Float16, 4, 4); break;   // row_ns is 4 or 0
        default: TMS_SPEC_LAUNCH(tms::Bf16, 4, 4); break;              // row_ns is 4 or 0
    }
#undef TMS_SPEC_LAUNCH
    return hipGetLastError() == hipSuccess ? TMS_OK : TMS_ERR_HIP;
}

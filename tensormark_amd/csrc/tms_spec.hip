// tms_spec.hip -- speculative accept/reject (stochastic verify) for gfx950.
//
// Two launches per call, both stream-ordered:
//
//   spec_stats    one workgroup per row (the k + 1 target rows and the k draft
//                 rows of every sequence): m = max(v / T), the exact integer
//                 sum Z of the row's weights q44(exp64(v / T - m)), and the
//                 weight of the row's draft token.  Two passes over the row;
//                 the second re-reads it from cache.
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

#include "../../include/tmsample_hip.h"
#include "tms_context.h"
#include "tms_device.h"

namespace tms {

__constant__ double kSpecExpTab[64] = {TMS_EXP2_64THS};
constexpr uint64_t kPartReady = 1ull << 63;   // published partial sum is complete
constexpr int kPartPoll = 1 << 20;            // bound on the finisher's wait per part

constexpr int kSpecChunk = 4096;   // ids per chunk of the chunked statistics

// One chunk's statistics: max of v / T, NaN/+inf flag, share of Z.
struct SpecPart {
    float m;
    int nf;
    int64_t z;
};

struct SArgs {
    const void* target;
    const void* draft;
    int B, k, V;
    bool fast;   // rows 16-byte aligned and V a multiple of the vector width
    int P, Lp;   // vocabulary parts of the draw and their length
    const int32_t* tokens;
    const tms_row_params* params;
    const uint32_t* draws;
    int32_t* out_acc;
    int32_t* out_tok;
    int32_t* out_status;
    tms_spec_stat* stats;
    uint64_t* parts;
    uint32_t* tickets;
    SpecPart* zparts;   // [B * (2k + 1)][C] chunk statistics
    int C;              // chunks per row of the chunked statistics (0: spec_stats_kernel)
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

__device__ __forceinline__ float block_max_f32(float v, float* sh) {
    v = wave_max_f32(v);
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
    __syncthreads();
    float r = sh[0];
#pragma unroll
    for (int i = 1; i < kWaves; ++i) r = fmaxf(r, sh[i]);
    __syncthreads();
    return r;
}

__device__ __forceinline__ int64_t block_sum_i64(int64_t v, int64_t* sh) {
    v = wave_sum_i64(v);
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
    __syncthreads();
    int64_t r = 0;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) r += sh[i];
    __syncthreads();
    return r;
}

__device__ __forceinline__ int block_or(int v, int* sh) {
    v = __any(v) ? 1 : 0;
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
    __syncthreads();
    int r = 0;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) r |= sh[i];
    __syncthreads();
    return r;
}

// Weight of a scaled logit on the 2^-44 grid.
__device__ __forceinline__ int64_t weight(float v, float temp, double m, const double* tab) {
    const float l = v / temp;
    return q44(exp64((double)l - m, tab));
}

// Residual weight q44(max(p_t - p_d, 0)) from the two rows' weights.
__device__ __forceinline__ int64_t residual(int64_t et, int64_t ed, int64_t Zt, int64_t Zd) {
    const double pt = (double)et / (double)Zt;
    const double pd = (double)ed / (double)Zd;
    const double d = pt - pd;
    return d > 0.0 ? q44(d) : 0;
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
        mx = fmaxf(mx, v / temp);
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

// Chunked statistics (16-byte aligned rows): the vocabulary in chunks of
// kSpecChunk ids, one workgroup per (row, chunk), in two launches.  Whole
// rows as work units left a CU in 8 with a third row while the rest idled
// (544 rows of exp64 work on 256 CUs).
//   spec_chunk_max_kernel: the chunk's max of v / T and NaN/+inf flag.
//   spec_chunk_z_kernel:   the row's max and status from its chunks' parts,
//                          then the chunk's share of Z (exact int64); chunk 0
//                          writes the row's record: m, status and the draft
//                          token's weight ex.
// The resolve kernel sums a row's Z shares (exact in any order).  m, status,
// Z and ex equal those of spec_stats_kernel.
template <typename T>
__global__ __launch_bounds__(kBlock) void spec_chunk_max_kernel(SArgs a) {
    constexpr int VEC = Elt<T>::kVec;
    constexpr int NS = kSpecChunk / VEC / kBlock;   // vectors per thread
    __shared__ float shf[kWaves];
    __shared__ int shi[kWaves];
    const int t = threadIdx.x;
    const int g = blockIdx.x / a.C, c = blockIdx.x - g * a.C;
    const int R = 2 * a.k + 1;
    const int b = g / R, i = g - b * R;
    const T* row = spec_row<T>(a, b, i);
    const float temp = a.params[b].temperature;
    const int nv = a.V / VEC;
    const int v0 = c * (kSpecChunk / VEC);
    uint4 q[NS];
#pragma unroll
    for (int sl = 0; sl < NS; ++sl) q[sl] = *(const uint4*)(row + (int64_t)min(v0 + t + sl * kBlock, nv - 1) * VEC);
    float mx = -__builtin_huge_valf();
    int nf = 0;
#pragma unroll
    for (int sl = 0; sl < NS; ++sl) {
        const bool in = v0 + t + sl * kBlock < nv;
        float x[VEC];
        Elt<T>::widen(q[sl], x);
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
            nf |= in ? __builtin_amdgcn_class(x[e], 0x203) : 0;   // NaN or +inf
            mx = in ? fmaxf(mx, x[e] / temp) : mx;
        }
    }
    mx = block_max_f32(mx, shf);
    nf = block_or(nf, shi);
    if (t == 0) {
        // Agent-scope stores: workgroups on different XCDs write neighbouring
        // records of one cache line, read by the next kernel.
        uint64_t* w = (uint64_t*)(a.zparts + (int64_t)g * a.C + c);
        st_agent(&w[0], (uint64_t)__float_as_uint(mx) | ((uint64_t)(uint32_t)nf << 32));
        st_agent(&w[1], (uint64_t)0);
    }
}

template <typename T>
__global__ __launch_bounds__(kBlock) void spec_chunk_z_kernel(SArgs a) {
    constexpr int VEC = Elt<T>::kVec;
    constexpr int NS = kSpecChunk / VEC / kBlock;
    __shared__ double tab[64];
    __shared__ int64_t shl[kWaves];
    load_exp_table(tab);
    const int t = threadIdx.x;
    const int g = blockIdx.x / a.C, c = blockIdx.x - g * a.C;
    const int R = 2 * a.k + 1;
    const int b = g / R, i = g - b * R;
    const T* row = spec_row<T>(a, b, i);
    const float temp = a.params[b].temperature;
    const int nv = a.V / VEC;
    const int v0 = c * (kSpecChunk / VEC);
    uint4 q[NS];
#pragma unroll
    for (int sl = 0; sl < NS; ++sl) q[sl] = *(const uint4*)(row + (int64_t)min(v0 + t + sl * kBlock, nv - 1) * VEC);
    // The row's max and flag from its chunks (every thread reads them all).
    const SpecPart* parts = a.zparts + (int64_t)g * a.C;
    float mx = -__builtin_huge_valf();
    int nf = 0;
    for (int u = 0; u < a.C; ++u) {
        const uint64_t w = ld_agent((uint64_t*)(parts + u));
        mx = fmaxf(mx, __uint_as_float((uint32_t)w));
        nf |= (int)(w >> 32);
    }
    int st = TMS_ROW_OK;
    if (nf) st = TMS_ROW_NONFINITE;
    else if (mx == -__builtin_huge_valf()) st = TMS_ROW_ALL_MASKED;
    else if (mx == __builtin_huge_valf()) st = TMS_ROW_NONFINITE;
    const double md = (double)mx;
    int64_t z = 0;
    if (st == TMS_ROW_OK) {
#pragma unroll
        for (int sl = 0; sl < NS; ++sl) {
            float x[VEC];
            Elt<T>::widen(q[sl], x);
            if (v0 + t + sl * kBlock < nv) {
#pragma unroll
                for (int e = 0; e < VEC; ++e) z += weight(x[e], temp, md, tab);
            }
        }
        z = block_sum_i64(z, shl);
    } else {
        __syncthreads();   // the table's LDS writes, as block_sum_i64 orders them
    }
    if (t == 0) {
        st_agent((uint64_t*)(a.zparts + (int64_t)g * a.C + c) + 1, (uint64_t)z);
        const int di = i < a.k ? i : (i > a.k ? i - a.k - 1 : -1);
        const int x = di >= 0 ? a.tokens[(int64_t)b * a.k + di] : -1;
        const bool xin = x >= 0 && x < a.V;
        if (c == 0) {
            // The whole record from one workgroup (the token's weight by one
            // scalar load), so no two workgroups write parts of it.
            const int64_t ex = (st == TMS_ROW_OK && xin) ? weight(Elt<T>::scalar(row + x), temp, md, tab) : 0;
            uint64_t* w = (uint64_t*)(a.stats + g);
            st_agent(&w[0], (uint64_t)__float_as_uint(mx) | ((uint64_t)(uint32_t)st << 32));
            st_agent(&w[1], (uint64_t)0);
            st_agent(&w[2], (uint64_t)ex);
            st_agent(&w[3], (uint64_t)0);
        }
    }
}

template <typename T>
__global__ __launch_bounds__(kBlock) void spec_resolve_kernel(SArgs a) {
    __shared__ double tab[64];
    __shared__ int64_t shl[2 * kWaves];
    __shared__ int64_t part_w[kSpecParts];
    __shared__ int64_t part_t[kSpecParts];
    __shared__ int misc[4];
    load_exp_table(tab);
    const int t = threadIdx.x;
    const int b = blockIdx.x / a.P, p = blockIdx.x - b * a.P;
    const tms_row_params P = a.params[b];
    const int g0 = b * (2 * a.k + 1);
    const uint32_t* dw = a.draws ? a.draws + (int64_t)b * (a.k + 1) * 2 : nullptr;
    // The sequence's statistics, draft tokens and accept uniforms, staged in
    // LDS with one load (or Philox draw) per thread, so the sequential accept
    // loop below waits on no memory.  With chunked statistics Z is the sum
    // of the chunks' shares, gathered the same way.
    __shared__ tms_spec_stat srow[2 * kSpecMaxK + 1];
    __shared__ int64_t zrow[2 * kSpecMaxK + 1];
    __shared__ int stok[kSpecMaxK];
    __shared__ double su[kSpecMaxK];
    {
        const int R = 2 * a.k + 1;
        if (t < R) {
            const uint64_t* w = (const uint64_t*)(a.stats + g0 + t);
            const uint64_t w0 = ld_agent(&w[0]);
            srow[t].m = __uint_as_float((uint32_t)w0);
            srow[t].status = (int32_t)(w0 >> 32);
            srow[t].Z = (int64_t)ld_agent(&w[1]);
            srow[t].ex = (int64_t)ld_agent(&w[2]);
            srow[t].pad = 0;
            zrow[t] = 0;
        }
        if (t < a.k) {
            stok[t] = a.tokens[(int64_t)b * a.k + t];
            uint32_t w0, w1;
            if (dw) { w0 = dw[2 * t]; w1 = dw[2 * t + 1]; }
            else row_words(P.seed, P.offset, (uint32_t)t, w0, w1);
            su[t] = canonical(w0, w1);
        }
        __syncthreads();
        if (a.C > 0) {
            for (int idx = t; idx < R * a.C; idx += kBlock)
                atomicAdd((unsigned long long*)&zrow[idx / a.C],
                          (unsigned long long)ld_agent((const uint64_t*)(a.zparts + (int64_t)g0 * a.C + idx) + 1));
            __syncthreads();
            if (t < R) srow[t].Z = zrow[t];
            __syncthreads();
        }
    }

    // ---- the accept tests, evaluated identically by every workgroup.
    int status = TMS_ROW_OK, acc = 0, rej = -1;   // rej < 0: all accepted, bonus draw
    if (!(P.temperature > 0.0f && P.temperature <= FLT_MAX)) {
        status = TMS_ROW_BAD_PARAMS;
    } else {
        acc = a.k;
        for (int i = 0; i < a.k; ++i) {
            const tms_spec_stat ts = srow[i], ds = srow[a.k + 1 + i];
            if (ts.status) { status = ts.status; break; }
            if (ds.status) { status = ds.status; break; }
            const int x = stok[i];
            if (x < 0 || x >= a.V) { status = TMS_ROW_BAD_PARAMS; break; }
            double r;
            if (ds.ex == 0) r = ts.ex > 0 ? 1.0 : 0.0;
            else r = ((double)ts.ex * (double)ds.Z) / ((double)ds.ex * (double)ts.Z);
            if (su[i] < r) continue;
            acc = i;
            rej = i;
            break;
        }
        if (status == TMS_ROW_OK && rej < 0 && srow[a.k].status) status = srow[a.k].status;
    }
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
    __syncthreads();   // exp table in LDS
    const int lo = p * a.Lp, hi = min(a.V, lo + a.Lp);
    int64_t wsum = 0, tsum = 0;
    if (rej < 0) {
        for_range(rt, lo, hi, a.fast, [&](int, float v) { tsum += weight(v, temp, mt, tab); });
        wsum = tsum;
    } else {
        for_range2(rt, rd, lo, hi, a.fast, [&](int, float vt, float vd) {
            const int64_t et = weight(vt, temp, mt, tab);
            const int64_t ed = weight(vd, temp, md, tab);
            tsum += et;
            wsum += residual(et, ed, ts.Z, ds.Z);
        });
    }
    wsum = block_sum_i64(wsum, shl);
    tsum = block_sum_i64(tsum, shl + kWaves);
    uint64_t* pw = a.parts + ((int64_t)b * kSpecParts + p) * 2;
    uint32_t ticket = 0;
    if (t == 0) {
        st_agent(&pw[0], kPartReady | (uint64_t)wsum);
        st_agent(&pw[1], kPartReady | (uint64_t)tsum);
        ticket = __hip_atomic_fetch_add(&a.tickets[b * kCounterStride], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        misc[0] = (int)ticket;
    }
    __syncthreads();
    if (misc[0] != a.P - 1) return;

    // ---- the last arriver: gather the parts (bounded wait on their ready
    //      bits), zero them and the ticket for the next call.
    if (t == 0) st_agent(&a.tickets[b * kCounterStride], 0u);
    int timed_out = 0;
    if (t < a.P) {
        uint64_t* q = a.parts + ((int64_t)b * kSpecParts + t) * 2;
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
        st_agent(&q[0], (uint64_t)0);
        st_agent(&q[1], (uint64_t)0);
    }
    timed_out = block_or(timed_out, misc);
    if (timed_out) {
        if (t == 0) {
            a.out_acc[b] = 0;
            a.out_tok[b] = -1;
            a.out_status[b] = TMS_ROW_INTERNAL;
        }
        return;
    }
    // Residual mass 0 (p_t <= p_d everywhere on the grid): draw from p_t.
    int64_t W = 0;
    for (int i = 0; i < a.P; ++i) W += part_w[i];
    const bool use_t = rej < 0 || W == 0;
    if (use_t) {
        W = 0;
        for (int i = 0; i < a.P; ++i) W += part_t[i];
    }
    uint32_t w0, w1;
    if (dw) { w0 = dw[2 * a.k]; w1 = dw[2 * a.k + 1]; }
    else row_words(P.seed, P.offset, (uint32_t)a.k, w0, w1);
    const double uf = canonical(w0, w1);
    int64_t thr = (int64_t)floor(uf * (double)W);
    if (thr > W - 1) thr = W - 1;
    int ps = a.P - 1;
    int64_t base = 0;
    for (int i = 0; i < a.P; ++i) {
        const int64_t wi = use_t ? part_t[i] : part_w[i];
        if (base + wi > thr) { ps = i; break; }
        base += wi;
    }
    // The part's weights, a contiguous run of ids per thread.
    const int plo = ps * a.Lp, phi = min(a.V, plo + a.Lp);
    const int E = (phi - plo + kBlock - 1) / kBlock;
    const int my_lo = min(phi, plo + t * E), my_hi = min(phi, my_lo + E);
    auto w_at = [&](int id) -> int64_t {
        const int64_t et = weight(Elt<T>::scalar(rt + id), temp, mt, tab);
        if (use_t) return et;
        const int64_t ed = weight(Elt<T>::scalar(rd + id), temp, md, tab);
        return residual(et, ed, ts.Z, ds.Z);
    };
    // Runs of up to kRunMax ids: every load issued at once (clamped
    // addresses), the weights kept in registers for the scan and the search;
    // longer runs walk the ids one by one.
    constexpr int kRunMax = 16;
    const bool cached = E <= kRunMax;
    int64_t wc[kRunMax];
    int64_t mine = 0;
    if (cached) {
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
                const int64_t et = weight(xt[j], temp, mt, tab);
                wc[j] = use_t ? et : residual(et, weight(xd[j], temp, md, tab), ts.Z, ds.Z);
            }
            mine += wc[j];
        }
    } else {
        for (int id = my_lo; id < my_hi; ++id) mine += w_at(id);
    }
    // Exclusive scan of the threads' sums.
    const int lane = t & 63, wv = t >> 6;
    const int64_t inc = wave_incl_scan_i64(mine);
    if (lane == 63) shl[wv] = inc;
    __syncthreads();
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

}  // namespace tms

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
    s.zparts = (tms::SpecPart*)ctx->spec_zparts;
    s.C = s.fast ? (a->vocab + tms::kSpecChunk - 1) / tms::kSpecChunk : 0;
    static_assert(sizeof(tms::SpecPart) == 2 * sizeof(uint64_t), "chunk statistics layout");
    const dim3 block(tms::kBlock);
    const dim3 g1((unsigned)(a->batch * (2 * a->k + 1))), g2((unsigned)(a->batch * s.P));
    // 16-byte aligned rows take the chunked statistics; others the per-row
    // kernel.
    const dim3 gc((unsigned)(a->batch * (2 * a->k + 1) * (s.C > 0 ? s.C : 1)));
#define TMS_SPEC_LAUNCH(T)                                                                 \
    do {                                                                                   \
        if (s.C > 0) {                                                                     \
            hipLaunchKernelGGL(tms::spec_chunk_max_kernel<T>, gc, block, 0, stream, s);    \
            hipLaunchKernelGGL(tms::spec_chunk_z_kernel<T>, gc, block, 0, stream, s);      \
        } else {                                                                           \
            hipLaunchKernelGGL(tms::spec_stats_kernel<T>, g1, block, 0, stream, s);        \
        }                                                                                  \
        hipLaunchKernelGGL(tms::spec_resolve_kernel<T>, g2, block, 0, stream, s);         \
    } while (0)
    switch (a->dtype) {
        case TMS_DTYPE_F32: TMS_SPEC_LAUNCH(float); break;
        case TMS_DTYPE_F16: TMS_SPEC_LAUNCH(_Float16); break;
        default: TMS_SPEC_LAUNCH(tms::Bf16); break;
    }
#undef TMS_SPEC_LAUNCH
    return hipGetLastError() == hipSuccess ? TMS_OK : TMS_ERR_HIP;
}

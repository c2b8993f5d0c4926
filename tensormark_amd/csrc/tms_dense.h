// tms_dense.h -- the exact full-row form of tmsample::sample
// (tensormark/tmsample.h:177-200) for the rows the general kernel cannot
// finish from its candidate lists: top-p rows (top_k = 0 or large) whose
// significant entries (v / T within 40 of the maximum) outnumber the list
// capacity, a draw that lands past the last significant entry, id lists
// longer than the held entries.
//
// The row's merger samples such a row itself, right where it finds it needs
// the whole row (no second launch): 256 threads of its workgroup, over a
// region of the context's workspace (2 x vocab 64-bit words) taken by a
// lock (dense_inline):
//
//   1. window counts per id (global atomics into the second half);
//   2. the row maximum of lg = penalised value / T;
//   3. a stable compaction, in id order, of the keys okey(lg) << 32 | ~id of
//      the significant entries (or of every entry, when the answer needs
//      the order past them);
//   4. a stable LSD radix sort, descending, on the 32-bit order keys, four
//      8-bit passes, each wave scattering a contiguous quarter in order, so
//      equal values keep ascending ids (the lowest-id tie rule);
//   5. the fp64 tail: pr = exp(lg - mx) in parallel into the second half,
//      prefix sums by thread blocks plus a block scan, and the top-p cut,
//      min-p cut and draw decided from them within a proven margin of the
//      reference's left-to-right sums; a decision inside the margin runs
//      the sequential sums (one thread, in the reference's order).
//
// Entries outside the 40 span change no sum: pr <= e^-40 < 2^-57 while every
// running sum of pr is >= pr_0 = 1 (and every running sum of pr / z is
// >= pr_0 / z), so each such addition rounds back to the running sum.  Only
// the draw's index, the top-k id list and a min-p threshold at or below
// e^-40 can reach past them; those cases sort the whole row.
#pragma once

#include "tms_sample_common.h"

namespace tms {

// LDS of the dense path, laid over the caller's (dead) merge staging.
struct DenseLds {
    uint32_t base[kWaves][256];   // per wave: digit counts, then scatter positions
    double wave_d[kWaves];
    int wave_i[kWaves];
    float wave_f[kWaves];
    int wave_any[kWaves];
    int misc[8];
};

__device__ __forceinline__ void dense_sync() { __syncthreads(); }

__device__ __forceinline__ int dense_block_sum(int v, DenseLds& L) {
    v = wave_sum_dpp(v);
    if ((threadIdx.x & 63) == 0) L.wave_i[threadIdx.x >> 6] = v;
    dense_sync();
    int s = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) s += L.wave_i[w];
    dense_sync();
    return s;
}

__device__ __forceinline__ int dense_block_min(int v, DenseLds& L) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = min(v, __shfl_xor(v, m, 64));
    if ((threadIdx.x & 63) == 0) L.wave_i[threadIdx.x >> 6] = v;
    dense_sync();
    int s = L.wave_i[0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) s = min(s, L.wave_i[w]);
    dense_sync();
    return s;
}

__device__ __forceinline__ float dense_block_max(float v, DenseLds& L) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
    if ((threadIdx.x & 63) == 0) L.wave_f[threadIdx.x >> 6] = v;
    dense_sync();
    float s = L.wave_f[0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) s = fmaxf(s, L.wave_f[w]);
    dense_sync();
    return s;
}

// Exclusive prefix of non-negative doubles over the workgroup's threads in
// thread order; `total` gets the sum.  Depth: the 6-step wave scan plus the
// preceding waves' totals (3 additions).
__device__ __forceinline__ double dense_block_excl_f64(double v, double& total, DenseLds& L) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const double inc = wave_incl_scan_f64(v);
    if (lane == 63) L.wave_d[w] = inc;
    dense_sync();
    double before = 0.0;
    total = 0.0;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) {
        const double x = L.wave_d[i];
        before += i < w ? x : 0.0;
        total += x;
    }
    dense_sync();
    // this wave's lanes before this one: the inclusive scan one lane up
    uint64_t up = __shfl_up((unsigned long long)__double_as_longlong(inc), 1, 64);
    const double prev = lane ? __longlong_as_double((long long)up) : 0.0;
    return before + prev;
}

// The value of id after the mask and the history penalties (counts in C),
// divided by the temperature: the lg that tmsample::sample ranks by.
template <typename T>
__device__ __forceinline__ float dense_lg(const T* base, const uint32_t* mrow, const uint32_t* C, int id,
                                          const Pen& pn, float temp, bool divide) {
    float v = Elt<T>::scalar(base + id);
    if (!((mrow[id >> 5] >> (id & 31)) & 1u)) return -__builtin_huge_valf();
    if (pn.on) {
        const uint32_t c = C[id];
        if (c) v = apply_pen(v, c, pn);
    }
    return divide ? v / temp : v;
}

// Stable LSD radix sort of n keys, descending by bits 32..63, between the
// two halves; returns the half that holds the result.  Wave w scatters
// the w-th quarter of the input in order, 64 keys per step, each lane's
// place among the equal digits of its step found with eight ballots.
__device__ __forceinline__ uint64_t* dense_sort(uint64_t* src, uint64_t* dst, int n, DenseLds& L) {
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int seg = ((n + kWaves - 1) / kWaves + 63) & ~63;
    const int s0 = min(n, w * seg), s1 = min(n, s0 + seg);
    const uint64_t lt = lane ? (~0ull >> (64 - lane)) : 0ull;
    for (int shift = 32; shift < 64; shift += 8) {
        for (int d = lane; d < 256; d += 64) L.base[w][d] = 0;
        __builtin_amdgcn_wave_barrier();
        for (int i = s0 + lane; i < s1; i += 64) {
            const uint32_t d = 255u - (uint32_t)((src[i] >> shift) & 0xFFu);
            atomicAdd(&L.base[w][d], 1u);
        }
        dense_sync();
        // thread t owns digit t: bases of every wave for it, after the scan
        // of the digits' totals
        uint32_t cw[kWaves];
        int tot = 0;
#pragma unroll
        for (int q = 0; q < kWaves; ++q) {
            cw[q] = L.base[q][t];
            tot += (int)cw[q];
        }
        const int inc = wave_incl_scan_i32(tot);
        if (lane == 63) L.wave_i[w] = inc;
        dense_sync();
        int start = inc - tot;
#pragma unroll
        for (int q = 0; q < kWaves; ++q) start += q < w ? L.wave_i[q] : 0;
        const bool any = __any(tot == n);
        if (lane == 0) L.wave_any[w] = any;
        dense_sync();
        bool one_digit = false;
#pragma unroll
        for (int q = 0; q < kWaves; ++q) one_digit |= L.wave_any[q] != 0;
        if (one_digit) continue;   // every key has this digit: order unchanged
        uint32_t b = (uint32_t)start;
#pragma unroll
        for (int q = 0; q < kWaves; ++q) {
            L.base[q][t] = b;
            b += cw[q];
        }
        dense_sync();
        for (int i0 = s0; i0 < s1; i0 += 64) {
            const int i = i0 + lane;
            const bool valid = i < s1;
            const uint64_t k = valid ? src[i] : 0ull;
            const uint32_t d = 255u - (uint32_t)((k >> shift) & 0xFFu);
            uint64_t peers = __ballot(valid);
#pragma unroll
            for (int bit = 0; bit < 8; ++bit) {
                const uint64_t m = __ballot(valid && ((d >> bit) & 1u));
                peers &= ((d >> bit) & 1u) ? m : ~m;
            }
            const uint32_t pos = L.base[w][d] + (uint32_t)__popcll(peers & lt);
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
            if (valid) {
                dst[pos] = k;
                if ((peers & lt) == 0ull) L.base[w][d] = pos + (uint32_t)__popcll(peers);
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
        }
        dense_sync();
        uint64_t* x = src;
        src = dst;
        dst = x;
    }
    return src;
}

// Stable compaction, in id order, of the keys of the entries with
// (double)lg - mx >= -kSigSpan (every entry when `all`) into out[]; returns
// the count.  Wave w walks the w-th quarter of the ids twice: once to count,
// once to store at its offset.
template <typename T>
__device__ __forceinline__ int dense_compact(const T* base, const uint32_t* mrow, const uint32_t* C, int V, const Pen& pn,
                             float temp, bool divide, double mx, bool all, uint64_t* out, DenseLds& L) {
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int seg = ((V + kWaves - 1) / kWaves + 63) & ~63;
    const int s0 = min(V, w * seg), s1 = min(V, s0 + seg);
    auto take = [&](float lg) { return all || ((double)lg - mx >= -(double)kSigSpan); };
    int cnt = 0;
    for (int i = s0 + lane; i < s1; i += 64) cnt += take(dense_lg(base, mrow, C, i, pn, temp, divide)) ? 1 : 0;
    cnt = wave_sum_dpp(cnt);
    if (lane == 0) L.wave_i[w] = cnt;
    dense_sync();
    int off = 0, n = 0;
#pragma unroll
    for (int q = 0; q < kWaves; ++q) {
        off += q < w ? L.wave_i[q] : 0;
        n += L.wave_i[q];
    }
    dense_sync();
    const uint64_t lt = lane ? (~0ull >> (64 - lane)) : 0ull;
    for (int i0 = s0; i0 < s1; i0 += 64) {
        const int i = i0 + lane;
        const float lg = i < s1 ? dense_lg(base, mrow, C, i, pn, temp, divide) : 0.0f;
        const bool p = i < s1 && take(lg);
        const uint64_t m = __ballot(p);
        if (p) out[off + __popcll(m & lt)] = ckey(lg, (uint32_t)i);
        off += __popcll(m);
    }
    dense_sync();
    return n;
}

// Window counts per id; with `positions` (the history pre-pass's list of
// distinct ids) the list position + 1 instead.
__device__ __forceinline__ void dense_count_window(uint32_t* C, int V, const int32_t* hist, int from, int nrec,
                                                   bool positions) {
    for (int i = threadIdx.x; i < V; i += kBlock) C[i] = 0u;
    dense_sync();
    for (int p = from + (int)threadIdx.x; p < nrec; p += kBlock) {
        const int id = hist[p];
        if (id >= 0 && id < V) atomicAdd(&C[id], positions ? (uint32_t)(p + 1) : 1u);
    }
    dense_sync();
}

constexpr int kDenseNone = 0x7FFFFFFF;

// First index i < lim whose prefix of pr[] divided by D is >= thr: above the
// margin (fd) or within it (fm), kDenseNone when there is none.  Thread t
// holds entries [b0, b1) and `excl`, the sum of the entries before them.
__device__ __forceinline__ void dense_first_ge(const double* pr, int b0, int b1, double excl, double D,
                                               double thr, int lim, double kRel, int& fd, int& fm,
                                               DenseLds& L) {
    int d = kDenseNone, m = kDenseNone;
    double c = excl;
    const int e = min(b1, lim);
    for (int i = b0; i < e; ++i) {
        c += pr[i];
        const double v = c / D;
        const double mg = (v + fabs(thr)) * kRel + 1e-300;
        if (v > thr + mg) {
            d = i;
            break;
        }
        if (!(v < thr - mg) && m == kDenseNone) m = i;
    }
    fd = dense_block_min(d, L);
    fm = dense_block_min(m, L);
}

// The whole-row sample of row `row` into the outputs.  K as tmsample::sample
// takes it (1 <= K <= V); the row is known to be finite after the mask and
// penalties, not all masked, with valid parameters, and not greedy.
// `ws` is the row's 2 * V words of workspace; without one the row reports
// TMS_ROW_UNSUPPORTED.
template <typename T>
__device__ __forceinline__ void dense_row(const KArgs& a, int row, tms_row_params P, int K, uint64_t* ws,
                                       DenseLds& L) {
    const int t = threadIdx.x;
    if (!ws) {
        write_row_error(a, row, TMS_ROW_UNSUPPORTED);
        return;
    }
    const int V = a.V;
    const T* base = (const T*)a.logits + (int64_t)row * a.row_stride;
    const uint32_t* mrow = a.mask + (int64_t)row * a.mask_stride;
    uint64_t* A = ws;
    uint64_t* B = ws + V;
    uint32_t* C = (uint32_t*)B;   // window counts per id, while the keys are formed
    // ---- history: counts per id over the window (tmsample.h:55-61)
    int nrec = 0;
    if (a.recent) {
        nrec = a.n_recent ? a.n_recent[row] : (int)a.recent_stride;
        if (nrec > (int)a.recent_stride) nrec = (int)a.recent_stride;
    }
    nrec = max(nrec, 0);   // -1 (pre-pass overflow) never reaches this pass
    const bool ovm = a.ov_vals != nullptr;
    Pen pn;
    pn.rep_on = !(P.repeat_penalty <= 1.0f);
    pn.fp_on = P.frequency_penalty != 0.0f || P.presence_penalty != 0.0f;
    pn.on = nrec > 0 && (ovm || (P.repeat_last_n > 0 && (pn.rep_on || pn.fp_on)));
    pn.rep = P.repeat_penalty;
    pn.freq = P.frequency_penalty;
    pn.pres = P.presence_penalty;
    if (ovm) pn.ov = a.ov_vals + (int64_t)row * kHistMax;
    // C shares its words with the sort's second half, so it is counted
    // again before each compaction.
    const int from = (!ovm && nrec > P.repeat_last_n) ? nrec - P.repeat_last_n : 0;
    const int32_t* hist = a.recent + (int64_t)row * a.recent_stride;
    if (pn.on) dense_count_window(C, V, hist, from, nrec, ovm);
    const float temp = P.temperature;
    const bool divide = temp != 1.0f;
    // ---- the row maximum of lg
    float mxf = -__builtin_huge_valf();
    for (int i = t; i < V; i += kBlock) mxf = fmaxf(mxf, dense_lg(base, mrow, C, i, pn, temp, divide));
    mxf = dense_block_max(mxf, L);
    if (mxf == __builtin_huge_valf() || mxf == -__builtin_huge_valf()) {
        // v / T overflowed (the reference's mx is +inf), or nothing is left
        write_row_error(a, row, mxf > 0.0f ? TMS_ROW_NONFINITE : TMS_ROW_ALL_MASKED);
        return;
    }
    const double mx = (double)mxf;
    uint32_t w0, w1;
    row_uniform(a, row, P, w0, w1);
    const double u = canonical(w0, w1);
    int32_t* ids = a.out_topk_ids ? a.out_topk_ids + (int64_t)row * a.topk_cap : nullptr;
    float* probs = a.out_topk_probs ? a.out_topk_probs + (int64_t)row * a.topk_cap : nullptr;

    for (int pass = 0; pass < 2; ++pass) {
        const bool all = pass == 1;
        if (all && pn.on) dense_count_window(C, V, hist, from, nrec, ovm);
        const int n = dense_compact(base, mrow, C, V, pn, temp, divide, mx, all, A, L);
        const uint64_t* S = dense_sort(A, B, n, L);
        double* pr = (double*)(S == A ? B : A);   // the other half
        const int nu = min(n, K);                 // entries tmsample::sample sums
        // a span-only pass must know the order past its entries when the
        // caller wants more ids than it holds
        bool need_all = !all && nu < K && a.topk_cap > nu && (ids || probs);
        // ---- pr, block prefix sums
        const int per = (nu + kBlock - 1) / kBlock;
        const int b0 = min(nu, t * per), b1 = min(nu, b0 + per);
        double loc = 0.0;
        for (int i = b0; i < b1; ++i) {
            const double p = exp((double)ckey_val(S[i]) - mx);
            pr[i] = p;
            loc += p;
        }
        double z;
        const double excl = dense_block_excl_f64(loc, z, L);
        dense_sync();   // pr[] complete
        // First index i < lim whose prefix / D is >= thr: above the margin
        // (fd) or within it (fm).  Against the reference's left-to-right sums
        // of quotients: a prefix here takes at most per - 1 + 9 roundings,
        // the reference's sums and quotients at most 2 nu + 1, the divisors
        // differ by at most (nu + per + 9) roundings, so the margin
        // (4 nu + 256) * 2^-53 relative covers every rounding with room.
        const double kRel = (4.0 * (double)nu + 256.0) * 0x1p-53;
        int fd, fm;
        dense_first_ge(pr, b0, b1, excl, z, (double)P.top_p, nu, kRel, fd, fm, L);
        bool ok = fm > fd || (fm == kDenseNone && fd == kDenseNone);
        int kp = fd < nu ? fd + 1 : K;
        if (ok && P.min_p > 0.0f) {
            // min-p: the first entry (from 1) below min_p ends the kept prefix
            const double mp = (double)P.min_p;
            int fl = kDenseNone;
            for (int i = max(b0, 1); i < b1; ++i)
                if (pr[i] < mp) {
                    fl = i;
                    break;
                }
            fl = dense_block_min(fl, L);
            if (fl < nu) kp = min(kp, fl);
            else if (nu < K && kp > nu) {
                // past the held entries pr <= e^-40: below a larger min_p
                if (mp > 4.3e-18) kp = nu;
                else need_all = need_all || !all;
            }
        }
        const int keep = kp;
        int tok = 0;
        if (ok && keep >= 2) {
            const int e = min(keep, nu) - 1;   // the draw's sum runs to entry keep - 1
            // prefix at e, from the thread holding it
            if (e >= b0 && e < b1) {
                double c = excl;
                for (int i = b0; i <= e; ++i) c += pr[i];
                L.wave_d[0] = c;
            }
            dense_sync();
            const double sum = L.wave_d[0];
            dense_sync();
            const int dl = min(nu, keep - 1);   // cp at keep - 1 is 1.0 (> u)
            int gd, gm;
            dense_first_ge(pr, b0, b1, excl, sum, u, dl, kRel, gd, gm, L);
            ok = gm > gd || (gm == kDenseNone && gd == kDenseNone);
            tok = gd < dl ? gd : keep - 1;
        }
        if (!ok && t == 0) {
            L.misc[1] = 0;
            // ---- sequential sums, the reference's order (tmsample.h:186-199,
            //      random.tcc:2656-2712)
            double zs = 0.0;
            for (int i = 0; i < nu; ++i) zs += pr[i];
            double cum = 0.0;
            int k2 = K;
            for (int i = 0; i < nu; ++i) {
                cum += pr[i] / zs;
                if (cum >= (double)P.top_p) {
                    k2 = i + 1;
                    break;
                }
            }
            if (P.min_p > 0.0f) {
                const double mp = (double)P.min_p;
                int m = 1;
                while (m < k2 && m < nu && pr[m] >= mp) ++m;
                if (m < k2 && m >= nu) {   // past the held entries (m == nu < K)
                    if (mp > 4.3e-18) k2 = m;
                    else L.misc[1] = 1;    // needs the whole row
                } else {
                    k2 = m;
                }
            }
            int j = 0;
            if (k2 >= 2) {
                const int lim = min(k2, nu);
                double sum = 0.0;
                for (int i = 0; i < lim; ++i) sum += pr[i];
                double cp = 0.0;
                j = k2 - 1;
                for (int i = 0; i < lim; ++i) {
                    const double q = pr[i] / sum;
                    cp = i == 0 ? q : cp + q;
                    const double cc = i == k2 - 1 ? 1.0 : cp;
                    if (!(cc < u)) {
                        j = i;
                        break;
                    }
                }
            }
            L.misc[0] = k2;
            L.misc[2] = j;
            L.wave_d[1] = zs;
        }
        if (t == 0 && ok) L.misc[1] = 0;
        dense_sync();
        int keep_f = keep, tok_f = tok;
        if (!ok) {
            keep_f = L.misc[0];
            tok_f = L.misc[2];
            z = L.wave_d[1];
            need_all = need_all || (L.misc[1] != 0 && !all);
        }
        dense_sync();
        if (!all && (need_all || tok_f >= nu)) continue;   // the order past the span is needed
        if (t == 0) {
            a.out_tokens[row] = (int)ckey_id(S[tok_f]);
            a.out_status[row] = TMS_ROW_OK;
            if (a.out_keep) a.out_keep[row] = keep_f;
        }
        for (int i = t; i < a.topk_cap; i += kBlock) {
            const bool have = i < nu;
            if (ids) ids[i] = have ? (int)ckey_id(S[i]) : -1;
            if (probs) probs[i] = have ? (float)(pr[i] / z) : 0.0f;
        }
        return;
    }
}

// A region of the workspace for the whole-row path: slot row mod n first,
// then the next ones, each taken by an agent-scope compare-and-swap on its
// lock word (0 free, 1 taken).  A slot is held only by a workgroup already
// running the path, which frees it when done, so the wait ends; it is still
// bounded (-1: none taken).
__device__ __forceinline__ int take_dense_slot(uint32_t* locks, int n, int row) {
    int s = row % n;
    for (int spins = 0; spins < kPollCap; ++spins) {
        uint32_t expect = 0u;
        if (__hip_atomic_compare_exchange_strong(&locks[s], &expect, 1u, __ATOMIC_ACQUIRE, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT))
            return s;
        s = s + 1 == n ? 0 : s + 1;
        if (s == row % n) __builtin_amdgcn_s_sleep(8);   // a full round without a free slot
    }
    return -1;
}

// The whole-row path for row `row`, run by the first 256 threads of the
// calling workgroup (every one of them calls it, and no other thread of the
// workgroup is left waiting at a barrier), its LDS in L: a region of the
// workspace is taken, the row sampled by dense_row, the region freed (a
// release store, after every store of the path).  Without a region the row
// reports TMS_ROW_UNSUPPORTED.
template <typename T>
__device__ void dense_inline(const KArgs& a, int row, DenseLds& L) {
    if (!a.dense) {
        write_row_error(a, row, TMS_ROW_UNSUPPORTED);
        return;
    }
    if (threadIdx.x == 0) L.misc[7] = take_dense_slot(a.dlocks, a.dense_slots, row);
    dense_sync();
    const int slot = L.misc[7];
    dense_sync();
    if (slot < 0) {
        write_row_error(a, row, TMS_ROW_INTERNAL);
        return;
    }
    const tms_row_params P = a.params[row];
    const int V = a.V;
    const int K = (P.top_k <= 0 || P.top_k > V) ? V : P.top_k;
    dense_row<T>(a, row, P, K, a.dense + (int64_t)slot * 2 * a.dense_stride, L);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    dense_sync();
    if (threadIdx.x == 0) __hip_atomic_store(&a.dlocks[slot], 0u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
}

// Greedy over the whole row, for a kernel that cannot hold the row's
// candidates: the largest key of the penalised value (no temperature),
// lowest id among equals, NaN / +inf and all-masked rows reported; window
// counts (positions [from, nrec) of the row's history) in a region of the
// workspace taken by its lock.  The first 256 threads of the workgroup.
template <typename T>
__device__ void dense_greedy(const KArgs& a, int row, const Pen& pn0, int from, int nrec, DenseLds& L) {
    const int t = threadIdx.x;
    const int V = a.V;
    const T* base = (const T*)a.logits + (int64_t)row * a.row_stride;
    const uint32_t* mrow = a.mask + (int64_t)row * a.mask_stride;
    Pen pn = pn0;
    int slot = -1;
    if (pn.on) {
        if (!a.dense) {
            write_row_error(a, row, TMS_ROW_UNSUPPORTED);
            return;
        }
        if (t == 0) L.misc[7] = take_dense_slot(a.dlocks, a.dense_slots, row);
        dense_sync();
        slot = L.misc[7];
        dense_sync();
        if (slot < 0) {
            write_row_error(a, row, TMS_ROW_INTERNAL);
            return;
        }
    }
    uint32_t* C = pn.on ? (uint32_t*)(a.dense + (int64_t)slot * 2 * a.dense_stride) : nullptr;
    if (pn.on) dense_count_window(C, V, a.recent + (int64_t)row * a.recent_stride, from, nrec, false);
    uint64_t best = 0ull;
    int bad = 0;
    for (int i = t; i < V; i += kBlock) {
        const float v = dense_lg(base, mrow, C, i, pn, 1.0f, false);
        bad |= __builtin_amdgcn_class(v, 0x203);   // NaN or +inf
        if (v != -__builtin_huge_valf()) {
            const uint64_t k = ckey(v, (uint32_t)i);
            best = k > best ? k : best;
        }
    }
    if (pn.on) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        dense_sync();
        if (t == 0) __hip_atomic_store(&a.dlocks[slot], 0u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
    }
    best = wave_max_u64_dpp(best);
    bad = __any(bad != 0);
    if ((t & 63) == 0) {
        L.wave_d[t >> 6] = __longlong_as_double((long long)best);
        L.wave_i[t >> 6] = bad;
    }
    dense_sync();
    uint64_t b = 0ull;
    int anyb = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
        const uint64_t x = (uint64_t)__double_as_longlong(L.wave_d[w]);
        b = x > b ? x : b;
        anyb |= L.wave_i[w];
    }
    if (anyb || b == 0ull) {
        write_row_error(a, row, anyb ? TMS_ROW_NONFINITE : TMS_ROW_ALL_MASKED);
        return;
    }
    const int tok = (int)ckey_id(b);
    if (t == 0) {
        a.out_tokens[row] = tok;
        a.out_status[row] = TMS_ROW_OK;
        if (a.out_keep) a.out_keep[row] = 0;
    }
    for (int i = t; i < a.topk_cap; i += kBlock) {
        if (a.out_topk_ids) a.out_topk_ids[(int64_t)row * a.topk_cap + i] = i == 0 ? tok : -1;
        if (a.out_topk_probs) a.out_topk_probs[(int64_t)row * a.topk_cap + i] = i == 0 ? 1.0f : 0.0f;
    }
}

}  // namespace tms

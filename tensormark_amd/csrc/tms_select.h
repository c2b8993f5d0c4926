// tms_select.h -- the ranking and the top-p block tail that the general
// kernel's row merger (tms_sample.hip) and the sparse-mask kernel
// (tms_sparse.hip) share: bucket_rank orders a row's candidate keys,
// tail_topp_block runs the fp64 tail of tmsample::sample
// (tensormark/tmsample.h:184-199) on a top-p row's sorted entries.  Both
// take the caller's LDS struct, which provides wave_f, wave_k, wave_i, hist
// and theta.
#pragma once

#include "tms_sample_common.h"

namespace tms {

// Ranks of the n distinct keys keys[0..n) (n <= kUni, any order; the
// whole workgroup): every key whose rank r (the number of larger keys) is
// below nkeep lands at out[r].  Each key goes to one of kBuckets buckets by
// a monotone function of its quotient (fl((q - qmin) * scale), truncated),
// so every key of a higher bucket is larger; counts per bucket (LDS
// atomics), a descending scan for each bucket's start, the keys scattered
// to their buckets in place, and each key ranked within its own bucket
// only.  A few barriers and a handful of reads a key, where binary searches
// over sorted lists cost dependent reads at conflicting addresses.  keys is
// reordered; cnt holds kBuckets ints of scratch.  Correct for any keys;
// massive ties (one bucket holding most keys) only cost time.  Keys equal
// to 0 (never a real key) are absent: unranked and not counted.
//
// kGiven: the caller passes the keys' quotient range [qmin, qmax] (any
// range keeps the bucket function monotone; the true one spreads the keys)
// and has zeroed cnt[0..kBuckets) before a barrier, which saves the range's
// reduction and its barrier.
constexpr int kBuckets = 2 * kBlock;
template <int kPer, bool kGiven = false, typename SM>   // keys per thread: n <= kPer * kBlock
__device__ void bucket_rank(uint64_t* keys, int n, int nkeep, uint64_t* out, int* cnt, SM& sm,
                            float qmax_in = 0.0f, float qmin_in = 0.0f) {
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    if constexpr (!kGiven) {
#pragma unroll
        for (int u = 0; u < kBuckets / kBlock; ++u) cnt[t * (kBuckets / kBlock) + u] = 0;
    }
    uint64_t k[kPer];
    float qhi = -__builtin_huge_valf(), qlo_neg = -__builtin_huge_valf();
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
        const int i = t + u * kBlock;
        k[u] = i < n ? keys[i] : 0ull;
        if (!kGiven && k[u] != 0ull) {
            const float q = ckey_val(k[u]);
            qhi = fmaxf(qhi, q);
            qlo_neg = fmaxf(qlo_neg, -q);
        }
    }
    float qmax = qmax_in, qmin = qmin_in;
    if constexpr (!kGiven) {
        qhi = wave_max_f32_dpp(qhi);
        qlo_neg = wave_max_f32_dpp(qlo_neg);
        if (lane == 0) {
            sm.wave_f[wv] = qhi;
            sm.wave_k[wv] = __float_as_uint(qlo_neg);
        }
        lds_sync();
        float qmin_neg = __uint_as_float((uint32_t)sm.wave_k[0]);
        qmax = sm.wave_f[0];
#pragma unroll
        for (int i = 1; i < kWaves; ++i) {
            qmax = fmaxf(qmax, sm.wave_f[i]);
            qmin_neg = fmaxf(qmin_neg, __uint_as_float((uint32_t)sm.wave_k[i]));
        }
        qmin = -qmin_neg;
    }
    const float span = qmax - qmin;
    // a span that is 0, or not finite, puts every key in bucket 0
    const float scale = (span > 0.0f && span <= FLT_MAX) ? (float)(kBuckets - 1) / span : 0.0f;
    int b[kPer], slot[kPer];
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
        const int i = t + u * kBlock;
        b[u] = 0;
        slot[u] = 0;
        if (k[u] != 0ull) {
            const float f = (ckey_val(k[u]) - qmin) * scale;   // NaN (inf * 0) and below 0 -> bucket 0
            b[u] = f >= (float)(kBuckets - 1) ? kBuckets - 1 : (f >= 1.0f ? (int)f : 0);
            slot[u] = atomicAdd(&cnt[b[u]], 1);
        }
    }
    lds_sync();
    // descending exclusive scan: start[b] = keys in buckets above b
    int tot;   // keys present
    {
        constexpr int kB = kBuckets / kBlock;   // buckets per thread
        int cb[kB], loc = 0;
#pragma unroll
        for (int u = 0; u < kB; ++u) {
            cb[u] = cnt[kBuckets - 1 - (t * kB + u)];
            loc += cb[u];
        }
        int st = block_excl_scan(loc, tot, sm);
#pragma unroll
        for (int u = 0; u < kB; ++u) {
            cnt[kBuckets - 1 - (t * kB + u)] = st;
            st += cb[u];
        }
    }
    lds_sync();
    // every key was read into registers above: scatter in place
#pragma unroll
    for (int u = 0; u < kPer; ++u)
        if (k[u] != 0ull) keys[cnt[b[u]] + slot[u]] = k[u];
    lds_sync();
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
        if (k[u] != 0ull) {
            const int lo = cnt[b[u]], hi = b[u] > 0 ? cnt[b[u] - 1] : tot;
            int r = lo;
            for (int j = lo; j < hi; ++j) r += keys[j] > k[u] ? 1 : 0;
            if (r < nkeep) out[r] = k[u];
        }
    }
}

// The top-p tail from block prefix sums (every thread of the workgroup),
// for n <= kToppCap entries pr[0..n) in LDS (srt, K, P as in tail_topp).
// Every prefix also goes to pre[0..n) (LDS, room for n doubles, apart
// from pr). Thread t holds the entries [t * per, t * per + per), per =
// ceil(n / kBlock) rounded up to odd (<= 5: an odd stride keeps the
// threads' 8-byte reads on distinct banks), and a prefix is its sequential
// partial sum within the thread, plus the exclusive scan of the thread
// totals within its wave, plus the totals of the waves before it (added in
// order).  Against the reference's sequential sums of the quotients
// pr_j / D (tmsample.h:186-199): a prefix takes at most 15 roundings (4 in
// the thread, 6 in the scan, 3 across the waves, 2 to combine), the scaling
// two (a prefix times the rounded reciprocal of the divisor), our divisor
// (a prefix) 15 and the reference's n - 1, its quotients and additions
// 2n + 1, so the two differ by at most (3n + 32) * 2^-53 relative
// (3104 * 2^-53 at n = 1024) plus subnormal units, inside the margin
// kRelP = 4160 * 2^-53.  A cut or draw decided within the margin of its
// threshold, and any call that returns per-entry probabilities, takes the
// sequential tail_topp.  The min-p cut compares the same pr values, so it is
// exact here.  The decisions (first index at or above a threshold,
// definitely or within the margin) meet in LDS: three barriers in place of
// one wave's serial chains.  Returns 0 when the row is written, 1 when the
// answer needs the order past the held entries (the whole-row path), 2 when
// only tail_topp can decide.  Every thread gets the same value.
template <typename SM>
__device__ __forceinline__ int tail_topp_block(const KArgs& a, int row, const tms_row_params& P, const uint64_t* srt, int n,
                               int K, const double* pr, double* pre, uint32_t w0, uint32_t w1, SM& sm) {
    static_assert(kToppCap <= kBlock * 4, "thread blocks of at most 5 entries");
    if (a.topk_cap && a.out_topk_probs) return 2;
    if (n < K && a.topk_cap > n && a.out_topk_ids) return 1;
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    const int per = ((n + kBlock - 1) / kBlock) | 1;
    const int b0 = t * per;
    double c[5];
    double acc = 0.0;
#pragma unroll
    for (int j = 0; j < 5; ++j) {
        const int i = b0 + j;
        acc += (j < per && i < n) ? pr[i] : 0.0;   // adding 0 is exact
        c[j] = acc;
    }
    const double incl = wave_incl_scan_f64(acc);
    double excl = __builtin_bit_cast(double, __shfl_up((unsigned long long)__builtin_bit_cast(uint64_t, incl), 1, 64));
    if (lane == 0) excl = 0.0;
    double* wt = (double*)sm.wave_k;   // the waves' totals
    if (lane == 63) wt[wv] = incl;
    lds_sync();
    double base = 0.0, z = 0.0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
        const double v = wt[w];
        if (w < wv) base += v;
        z += v;
    }
#pragma unroll
    for (int j = 0; j < 5; ++j) {
        c[j] = base + (excl + c[j]);
        if (j < per && b0 + j < n) pre[b0 + j] = c[j];   // read after the next barrier
    }
    constexpr double kRelP = (4.0 * kToppCap + 64.0) * 0x1p-53;
    constexpr double kAbs = 1e-300;
    constexpr int kNone = 1 << 30;
    // this thread's first index i < lim whose prefix / D is >= thr,
    // definitely (fd) or within the margin (fm)
    auto first_ge = [&](double D, double thr, int lim) {
        int fd = kNone, fm = kNone;
        const double rD = 1.0 / D;
#pragma unroll
        for (int j = 4; j >= 0; --j) {
            const int i = b0 + j;
            if (j < per && i < lim) {
                const double v = c[j] * rD;
                const double m = (v + fabs(thr)) * kRelP + kAbs;
                if (v > thr + m) fd = i;
                else if (!(v < thr - m)) fm = i;
            }
        }
        return make_int2(wave_min_nonneg(fd), wave_min_nonneg(fm));
    };
    // the block minima of up to three per-wave values, in slots of hist
    auto block_min3 = [&](int s0, int3 v) {
        if (lane == 0) {
            sm.hist[s0 + wv] = v.x;
            sm.hist[s0 + kWaves + wv] = v.y;
            sm.hist[s0 + 2 * kWaves + wv] = v.z;
        }
        lds_sync();
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            v.x = min(v.x, sm.hist[s0 + w]);
            v.y = min(v.y, sm.hist[s0 + kWaves + w]);
            v.z = min(v.z, sm.hist[s0 + 2 * kWaves + w]);
        }
        return v;
    };
    const int2 f1 = first_ge(z, (double)P.top_p, n);
    int fl = kNone;   // first index >= 1 with pr < min_p
    const bool minp = P.min_p > 0.0f;
    if (minp) {
        const double mp = (double)P.min_p;
#pragma unroll
        for (int j = 4; j >= 0; --j) {
            const int i = b0 + j;
            if (j < per && i >= 1 && i < n && pr[i] < mp) fl = i;
        }
        fl = wave_min_nonneg(fl);
    }
    const int3 m1 = block_min3(0, make_int3(f1.x, f1.y, fl));
    const int fd = m1.x, fm = m1.y;
    fl = m1.z;
    bool ok = fm > fd || (fm == kNone && fd == kNone);
    int kp = fd < n ? fd + 1 : K;
    if (ok && minp) {
        if (fl >= n && n < kp && !((double)P.min_p > 4.3e-18)) return 1;   // as in tail_topp
        const int m = min(fl, min(kp, n));
        if (m < kp) kp = m;
    }
    const int keep = kp;
    const int lim = keep < n ? keep : n;
    int tokidx = 0;
    if (ok && keep >= 2) {
        // sum = the prefix at lim - 1 (every prefix went to pre before
        // block_min3's barrier)
        const double u = canonical(w0, w1);
        const double sum = pre[lim - 1];
        // cp at keep - 1 is 1.0 exactly (> u): only indices before it are
        // decided from the prefixes
        const int dl = min(lim, keep - 1);
        const int2 f2 = first_ge(sum, u, dl);
        const int3 m2 = block_min3(3 * kWaves, make_int3(f2.x, f2.y, kNone));
        const int gd = m2.x, gm = m2.y;
        ok = gm > gd || (gm == kNone && gd == kNone);
        tokidx = gd < dl ? gd : keep - 1;
    }
    if (!ok) return 2;
    // tokidx >= n: the draw fell past the last entry that moves the sums
    if (tokidx >= n) return 1;
    if (t == 0) {
        a.out_tokens[row] = (int)ckey_id(srt[tokidx]);
        a.out_status[row] = TMS_ROW_OK;
        if (a.out_keep) a.out_keep[row] = keep;
    }
    if (a.topk_cap && a.out_topk_ids)
        for (int i = t; i < a.topk_cap; i += kBlock)
            a.out_topk_ids[(int64_t)row * a.topk_cap + i] = i < n ? (int)ckey_id(srt[i]) : -1;
    return 0;
}

}  // namespace tms

/*
 * tms_oracle.c -- CPU restatement of TensorMark's token-sampling path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP library, never part of
 * it.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * may load it.  Built with -O2 -ffp-contract=off so every float and double
 * operation below is one IEEE operation in source order.
 *
 * What pins each function (checked in tests/test_oracle.py):
 *   tmo_philox4x32_10       Random123 known-answer vectors (Salmon et al., SC'11).
 *   tmo_canonical           libstdc++ std::generate_canonical<double,53> driven by
 *                           a scripted generator, through oracle/_ref.
 *   tmo_apply_mask          bitmask <-> allowed-list invariant; the -inf rule of
 *                           GrammarFilter::restrict (llama_chat.cpp:206-207).
 *   tmo_apply_repeat_penalty  compiled reference apply_repeat_penalty (oracle/_ref)
 *                           and the closed form for counts 1..3.
 *   tmo_apply_freq_presence closed form v - (c*freq + presence); brute force.
 *                           No reference counterpart: parity unpinned by the
 *                           reference, pinned by the closed form only.
 *   tmo_no_repeat_ngram, tmo_dry  the reference's own outputs: committed golden
 *                           vectors of the compiled tmsample.h
 *                           (tests/golden/history_golden.npz), oracle/_ref on
 *                           random histories, closed forms.
 *   tmo_sample_batch_h      composition of the pinned steps in sample_token's
 *                           order (llama_chat.cpp:148-151).
 *   tmo_sample_row          compiled reference tmsample::sample (oracle/_ref) on
 *                           tie-free rows (token, keep); committed golden vectors
 *                           (tests/golden/); brute-force enumeration on tiny V.
 *                           min-p: closed form only (absent from the reference).
 *   tmo_exp64, tmo_q44, tmo_spec_*  build-defined (no reference counterpart):
 *                           exp64 against glibc exp within 2 ulp; spec verify
 *                           against its one-hot (greedy) limit, p_t == p_d
 *                           (always accept), brute-force rejection sampling
 *                           marginals on V <= 8.
 */
#include "tms_oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

enum { ROW_OK = 0, ROW_BAD_PARAMS = 1, ROW_ALL_MASKED = 2, ROW_NONFINITE = 3 };

/* ------------------------------------------------------------------ Philox */

/* Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as
 * easy as 1, 2, 3", SC'11): ten rounds of two 32x32->64 multiplies with the
 * key bumped by the Weyl constants between rounds. */
void tmo_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]) {
    uint32_t c0 = ctr[0], c1 = ctr[1], c2 = ctr[2], c3 = ctr[3];
    uint32_t k0 = key[0], k1 = key[1];
    for (int r = 0; r < 10; ++r) {
        const uint64_t p0 = (uint64_t)0xD2511F53u * c0;
        const uint64_t p1 = (uint64_t)0xCD9E8D57u * c2;
        const uint32_t n0 = (uint32_t)(p1 >> 32) ^ c1 ^ k0;
        const uint32_t n1 = (uint32_t)p1;
        const uint32_t n2 = (uint32_t)(p0 >> 32) ^ c3 ^ k1;
        const uint32_t n3 = (uint32_t)p0;
        c0 = n0; c1 = n1; c2 = n2; c3 = n3;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
    out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

/* The two words a row's draw uses: key = seed, counter = (offset, stream, 0). */
void tmo_row_words(uint64_t seed, uint64_t offset, uint32_t stream, uint32_t* w0, uint32_t* w1) {
    const uint32_t ctr[4] = {(uint32_t)offset, (uint32_t)(offset >> 32), stream, 0u};
    const uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
    uint32_t o[4];
    tmo_philox4x32_10(ctr, key, o);
    *w0 = o[0];
    *w1 = o[1];
}

/* std::generate_canonical<double, 53> over a 32-bit engine, as libstdc++
 * computes it (/usr/include/c++/11/bits/random.tcc:3348-3380): two draws,
 * sum = 0 + w0 * 1, sum += w1 * 2^32, ret = sum / 2^64, clamped below 1. */
double tmo_canonical(uint32_t w0, uint32_t w1) {
    double sum = 0.0;
    sum += (double)w0 * 1.0;
    sum += (double)w1 * 4294967296.0;
    double ret = sum / 18446744073709551616.0;
    if (ret >= 1.0) ret = nextafter(1.0, 0.0);
    return ret;
}

/* ------------------------------------------------------------- transforms */

/* GrammarFilter::restrict (tensormark/llama_chat.cpp:184-209): every id the
 * allowed set lacks becomes -inf.  The allowed set travels as a bitmask,
 * bit (id & 31) of word id >> 5.  The stall narrowing (llama_chat.cpp:
 * 193-205) stays with the host that builds the mask. */
void tmo_apply_mask(float* row, int V, const uint32_t* mask) {
    if (!mask) return;
    for (int i = 0; i < V; ++i)
        if (!((mask[i >> 5] >> (i & 31)) & 1u)) row[i] = -INFINITY;
}

/* tmsample::apply_repeat_penalty (tensormark/tmsample.h:52-63): for each of the
 * last `window` ids in range, v = v > 0 ? v / p : v * p, once per occurrence. */
void tmo_apply_repeat_penalty(float* row, int V, const int32_t* recent, int n_recent,
                              int window, float penalty) {
    if (penalty <= 1.0f || window <= 0 || n_recent <= 0) return;
    const int from = n_recent > window ? n_recent - window : 0;
    for (int i = from; i < n_recent; ++i) {
        const int t = recent[i];
        if (t < 0 || t >= V) continue;
        const float v = row[t];
        row[t] = v > 0.f ? v / penalty : v * penalty;
    }
}

/* Frequency/presence penalty (no reference counterpart; the llama.cpp
 * convention): v -= (float)count * freq + presence over the same window. */
void tmo_apply_freq_presence(float* row, int V, const int32_t* recent, int n_recent,
                             int window, float freq, float presence) {
    if ((freq == 0.0f && presence == 0.0f) || window <= 0 || n_recent <= 0) return;
    const int from = n_recent > window ? n_recent - window : 0;
    int* cnt = (int*)calloc((size_t)V, sizeof(int));
    for (int i = from; i < n_recent; ++i) {
        const int t = recent[i];
        if (t >= 0 && t < V) cnt[t]++;
    }
    for (int i = 0; i < V; ++i)
        if (cnt[i] > 0) {
            const float t1 = (float)cnt[i] * freq;
            const float t = t1 + presence;
            row[i] = row[i] - t;
        }
    free(cnt);
}

/* tmsample::apply_no_repeat_ngram (tensormark/tmsample.h:81-114): the id
 * after each earlier occurrence of the last ngram - 1 ids becomes -inf (its
 * value saved the first time); when the row's std::max scan from -inf then
 * finds nothing above -inf, the saved values go back. */
void tmo_no_repeat_ngram(float* row, int V, const int32_t* recent, int n_recent, int ngram) {
    if (ngram < 2 || n_recent < ngram) return;
    const int m = ngram - 1, s = n_recent - m;
    int* bid = (int*)malloc((size_t)s * sizeof(int) + 1);
    float* bv = (float*)malloc((size_t)s * sizeof(float) + 1);
    int nb = 0;
    for (int i = 0; i < s; ++i) {
        int k = 0;
        while (k < m && recent[i + k] == recent[s + k]) ++k;
        if (k < m) continue;
        const int t = recent[i + m];
        if (t < 0 || t >= V) continue;
        if (row[t] == -INFINITY) continue;
        bid[nb] = t;
        bv[nb] = row[t];
        ++nb;
        row[t] = -INFINITY;
    }
    if (nb > 0) {
        float best = -INFINITY;
        for (int i = 0; i < V; ++i) best = (best < row[i]) ? row[i] : best;   /* std::max */
        if (best == -INFINITY)
            for (int j = 0; j < nb; ++j) row[bid[j]] = bv[j];
    }
    free(bid);
    free(bv);
}

/* tmsample::apply_dry (tensormark/tmsample.h:148-170), with the reference's
 * powf.  Breaker lookups of ids outside [0, V) read as "not a breaker" (the
 * reference indexes is_breaker with them unchecked). */
static int tmo_brk(const uint8_t* brk, int V, int id) { return brk && id >= 0 && id < V && brk[id]; }

void tmo_dry(float* row, int V, const int32_t* recent, int n_recent, float multiplier, float base,
             int allowed_length, int penalty_last_n, const uint8_t* is_breaker) {
    if (multiplier <= 0.0f || allowed_length < 1) return;
    if (n_recent < allowed_length + 1) return;
    const int n = n_recent < penalty_last_n ? n_recent : penalty_last_n;
    if (n < allowed_length + 1) return;
    const int32_t* s = recent + (n_recent - n);
    const int last = n - 1;
    for (int i = 0; i < last; ++i) {
        int L = 0;
        while (L <= i && s[i - L] == s[last - L] &&
               !(tmo_brk(is_breaker, V, s[i - L]) || tmo_brk(is_breaker, V, s[last - L])))
            ++L;
        if (L < allowed_length) continue;
        const int nxt = s[i + 1];
        if (nxt < 0 || nxt >= V) continue;
        if (tmo_brk(is_breaker, V, nxt)) continue;
        row[nxt] -= multiplier * powf(base, (float)(L - allowed_length));
    }
}

/* --------------------------------------------------------------- sampling */

typedef struct { float v; int id; } ent;

/* The reference's order (tmsample.h:181-183: lg[a] > lg[b]) made total:
 * equal values go lowest id first. */
static int better(const ent* a, const ent* b) {
    return a->v > b->v || (a->v == b->v && a->id < b->id);
}

static int cmp_ent(const void* pa, const void* pb) {
    const ent* a = (const ent*)pa;
    const ent* b = (const ent*)pb;
    if (better(a, b)) return -1;
    if (better(b, a)) return 1;
    return 0;
}

/* The K best of lg[0..V) in order; nth_element + sort of the prefix in the
 * reference (tmsample.h:179-183). */
static void select_topk(const float* lg, int V, int K, ent* out) {
    if ((long)K * 8 < V) {
        int n = 0;
        for (int i = 0; i < V; ++i) {
            ent e = {lg[i], i};
            if (n == K && !better(&e, &out[K - 1])) continue;
            int pos = n < K ? n : K - 1;
            while (pos > 0 && better(&e, &out[pos - 1])) {
                out[pos] = out[pos - 1];
                --pos;
            }
            out[pos] = e;
            if (n < K) ++n;
        }
        return;
    }
    ent* all = (ent*)malloc((size_t)V * sizeof(ent));
    for (int i = 0; i < V; ++i) { all[i].v = lg[i]; all[i].id = i; }
    qsort(all, (size_t)V, sizeof(ent), cmp_ent);
    memcpy(out, all, (size_t)K * sizeof(ent));
    free(all);
}

/* tmsample::sample (tensormark/tmsample.h:173-200), with the draw of
 * std::discrete_distribution (/usr/include/c++/11/bits/random.tcc:2656-2712)
 * spelled out: sum = accumulate(pr[0..keep)), p = pr / sum,
 * cp = partial_sum(p), cp.back() = 1, j = lower_bound(cp, u); keep == 1
 * draws nothing.  Additions: the row status codes, the lowest-id tie order,
 * top_k <= 0 meaning V, and the min-p cut. */
int tmo_sample_row(const float* row, int V, const tmo_row_params* p, uint32_t w0, uint32_t w1,
                   int32_t* token, int32_t* keep, int32_t* topk_ids, float* topk_probs,
                   int topk_cap) {
    *token = -1;
    *keep = 0;
    for (int j = 0; j < topk_cap; ++j) {
        if (topk_ids) topk_ids[j] = -1;
        if (topk_probs) topk_probs[j] = 0.0f;
    }
    if (!p->greedy && !(p->temperature > 0.0f && p->temperature <= FLT_MAX))
        return ROW_BAD_PARAMS;
    int nfin = 0;
    for (int i = 0; i < V; ++i) {
        const float v = row[i];
        if (isnan(v) || v == INFINITY) return ROW_NONFINITE;
        if (v != -INFINITY) ++nfin;
    }
    if (nfin == 0) return ROW_ALL_MASKED;

    if (p->greedy) {
        /* std::max_element: the first maximum (tmsample.h:175-176). */
        int best = 0;
        for (int i = 1; i < V; ++i)
            if (row[best] < row[i]) best = i;
        *token = best;
        if (topk_cap > 0) {
            if (topk_ids) topk_ids[0] = best;
            if (topk_probs) topk_probs[0] = 1.0f;
        }
        return ROW_OK;
    }

    const int K = (p->top_k <= 0 || p->top_k > V) ? V : p->top_k;
    float* lg = (float*)malloc((size_t)V * sizeof(float));
    for (int i = 0; i < V; ++i) lg[i] = row[i] / p->temperature;
    ent* top = (ent*)malloc((size_t)K * sizeof(ent));
    select_topk(lg, V, K, top);
    free(lg);

    const float mx = top[0].v;
    if (mx == INFINITY) { free(top); return ROW_NONFINITE; }
    double* pr = (double*)malloc((size_t)K * sizeof(double));
    double* zp = (double*)malloc((size_t)K * sizeof(double));
    double z = 0;
    for (int k = 0; k < K; ++k) {
        pr[k] = exp((double)top[k].v - (double)mx);
        z += pr[k];
        zp[k] = z;
    }
    double cum = 0;
    int kp = K;
    for (int k = 0; k < K; ++k) {
        cum += pr[k] / z;
        if (cum >= (double)p->top_p) { kp = k + 1; break; }
    }
    if (p->min_p > 0.0f) {
        int m = 1;
        while (m < kp && pr[m] >= (double)p->min_p) ++m;
        kp = m;
    }
    *keep = kp;
    int j = 0;
    if (kp >= 2) {
        const double sum = zp[kp - 1];
        const double u = tmo_canonical(w0, w1);
        double cp = 0;
        j = kp - 1;
        for (int i = 0; i < kp; ++i) {
            const double q = pr[i] / sum;
            cp = (i == 0) ? q : cp + q;
            const double c = (i == kp - 1) ? 1.0 : cp;
            if (!(c < u)) { j = i; break; }
        }
    }
    *token = top[j].id;
    const int n = topk_cap < K ? topk_cap : K;
    for (int i = 0; i < n; ++i) {
        if (topk_ids) topk_ids[i] = top[i].id;
        if (topk_probs) topk_probs[i] = (float)(pr[i] / z);
    }
    free(pr);
    free(zp);
    free(top);
    return ROW_OK;
}

/* The per-row composition of sample_token with the grammar restriction
 * (tensormark/llama_chat.cpp:787-791 then 146-153): mask, repetition
 * penalty, frequency/presence, sample. */
void tmo_sample_batch(const float* logits, int B, int V, int64_t row_stride,
                      const tmo_row_params* params, const int32_t* recent,
                      const int32_t* n_recent, int64_t recent_stride, const uint32_t* mask,
                      int64_t mask_stride, const uint32_t* draws, int32_t* tokens,
                      int32_t* status, int32_t* keep, int32_t* topk_ids, float* topk_probs,
                      int topk_cap) {
    float* row = (float*)malloc((size_t)V * sizeof(float));
    for (int b = 0; b < B; ++b) {
        const tmo_row_params* p = &params[b];
        memcpy(row, logits + (int64_t)b * row_stride, (size_t)V * sizeof(float));
        if (mask) tmo_apply_mask(row, V, mask + (int64_t)b * mask_stride);
        if (recent) {
            const int32_t* r = recent + (int64_t)b * recent_stride;
            const int n = n_recent ? n_recent[b] : (int)recent_stride;
            tmo_apply_repeat_penalty(row, V, r, n, p->repeat_last_n, p->repeat_penalty);
            tmo_apply_freq_presence(row, V, r, n, p->repeat_last_n, p->frequency_penalty,
                                    p->presence_penalty);
        }
        uint32_t w0, w1;
        if (draws) {
            w0 = draws[2 * b];
            w1 = draws[2 * b + 1];
        } else {
            tmo_row_words(p->seed, p->offset, 0u, &w0, &w1);
        }
        int32_t kp = 0;
        status[b] = tmo_sample_row(row, V, p, w0, w1, &tokens[b], &kp,
                                   topk_ids ? topk_ids + (int64_t)b * topk_cap : NULL,
                                   topk_probs ? topk_probs + (int64_t)b * topk_cap : NULL,
                                   topk_cap);
        if (keep) keep[b] = kp;
    }
    free(row);
}

/* sample_token with the grammar restriction in front (llama_chat.cpp:
 * 787-791, then 148-151): mask, repetition penalty, frequency/presence,
 * n-gram ban, DRY, sample.  A NaN or +inf left by the mask makes the row
 * ROW_NONFINITE whatever the history steps do to it (the library's row
 * contract).  hp may be NULL (then this is tmo_sample_batch). */
void tmo_sample_batch_h(const float* logits, int B, int V, int64_t row_stride,
                        const tmo_row_params* params, const tmo_history_params* hp,
                        const uint8_t* breaker, const int32_t* recent, const int32_t* n_recent,
                        int64_t recent_stride, const uint32_t* mask, int64_t mask_stride,
                        const uint32_t* draws, int32_t* tokens, int32_t* status, int32_t* keep,
                        int32_t* topk_ids, float* topk_probs, int topk_cap) {
    float* row = (float*)malloc((size_t)V * sizeof(float));
    for (int b = 0; b < B; ++b) {
        const tmo_row_params* p = &params[b];
        memcpy(row, logits + (int64_t)b * row_stride, (size_t)V * sizeof(float));
        if (mask) tmo_apply_mask(row, V, mask + (int64_t)b * mask_stride);
        int nonfinite = 0;
        for (int i = 0; i < V; ++i) nonfinite |= isnan(row[i]) || row[i] == INFINITY;
        if (recent) {
            const int32_t* r = recent + (int64_t)b * recent_stride;
            int n = n_recent ? n_recent[b] : (int)recent_stride;
            if (n > (int)recent_stride) n = (int)recent_stride;
            if (n < 0) n = 0;
            tmo_apply_repeat_penalty(row, V, r, n, p->repeat_last_n, p->repeat_penalty);
            tmo_apply_freq_presence(row, V, r, n, p->repeat_last_n, p->frequency_penalty,
                                    p->presence_penalty);
            if (hp) {
                tmo_no_repeat_ngram(row, V, r, n, hp[b].no_repeat_ngram);
                tmo_dry(row, V, r, n, hp[b].dry_multiplier, hp[b].dry_base,
                        hp[b].dry_allowed_length, hp[b].dry_penalty_last_n, breaker);
            }
        }
        uint32_t w0, w1;
        if (draws) {
            w0 = draws[2 * b];
            w1 = draws[2 * b + 1];
        } else {
            tmo_row_words(p->seed, p->offset, 0u, &w0, &w1);
        }
        int32_t kp = 0;
        int32_t* ids = topk_ids ? topk_ids + (int64_t)b * topk_cap : NULL;
        float* probs = topk_probs ? topk_probs + (int64_t)b * topk_cap : NULL;
        status[b] = tmo_sample_row(row, V, p, w0, w1, &tokens[b], &kp, ids, probs, topk_cap);
        if (nonfinite && status[b] != ROW_BAD_PARAMS) {
            status[b] = ROW_NONFINITE;
            tokens[b] = -1;
            kp = 0;
            for (int j = 0; j < topk_cap; ++j) {
                if (ids) ids[j] = -1;
                if (probs) probs[j] = 0.0f;
            }
        }
        if (keep) keep[b] = kp;
    }
    free(row);
}

/* ---------------------------------------------------- speculative verify */

/* 2^(j/64), j = 0..63, each the double nearest the exact value (computed
 * with 60-digit decimal arithmetic). */
static const double kExp2_64ths[64] = {
    0x1.0000000000000p+0, 0x1.02c9a3e778061p+0, 0x1.059b0d3158574p+0, 0x1.0874518759bc8p+0,
    0x1.0b5586cf9890fp+0, 0x1.0e3ec32d3d1a2p+0, 0x1.11301d0125b51p+0, 0x1.1429aaea92de0p+0,
    0x1.172b83c7d517bp+0, 0x1.1a35beb6fcb75p+0, 0x1.1d4873168b9aap+0, 0x1.2063b88628cd6p+0,
    0x1.2387a6e756238p+0, 0x1.26b4565e27cddp+0, 0x1.29e9df51fdee1p+0, 0x1.2d285a6e4030bp+0,
    0x1.306fe0a31b715p+0, 0x1.33c08b26416ffp+0, 0x1.371a7373aa9cbp+0, 0x1.3a7db34e59ff7p+0,
    0x1.3dea64c123422p+0, 0x1.4160a21f72e2ap+0, 0x1.44e086061892dp+0, 0x1.486a2b5c13cd0p+0,
    0x1.4bfdad5362a27p+0, 0x1.4f9b2769d2ca7p+0, 0x1.5342b569d4f82p+0, 0x1.56f4736b527dap+0,
    0x1.5ab07dd485429p+0, 0x1.5e76f15ad2148p+0, 0x1.6247eb03a5585p+0, 0x1.6623882552225p+0,
    0x1.6a09e667f3bcdp+0, 0x1.6dfb23c651a2fp+0, 0x1.71f75e8ec5f74p+0, 0x1.75feb564267c9p+0,
    0x1.7a11473eb0187p+0, 0x1.7e2f336cf4e62p+0, 0x1.82589994cce13p+0, 0x1.868d99b4492edp+0,
    0x1.8ace5422aa0dbp+0, 0x1.8f1ae99157736p+0, 0x1.93737b0cdc5e5p+0, 0x1.97d829fde4e50p+0,
    0x1.9c49182a3f090p+0, 0x1.a0c667b5de565p+0, 0x1.a5503b23e255dp+0, 0x1.a9e6b5579fdbfp+0,
    0x1.ae89f995ad3adp+0, 0x1.b33a2b84f15fbp+0, 0x1.b7f76f2fb5e47p+0, 0x1.bcc1e904bc1d2p+0,
    0x1.c199bdd85529cp+0, 0x1.c67f12e57d14bp+0, 0x1.cb720dcef9069p+0, 0x1.d072d4a07897cp+0,
    0x1.d5818dcfba487p+0, 0x1.da9e603db3285p+0, 0x1.dfc97337b9b5fp+0, 0x1.e502ee78b3ff6p+0,
    0x1.ea4afa2a490dap+0, 0x1.efa1bee615a27p+0, 0x1.f50765b6e4540p+0, 0x1.fa7c1819e90d8p+0,
};

/* exp(x) by table-driven range reduction (Tang, ACM TOMS 15(2), 1989):
 * x = (64m + j) ln2/64 + r with |r| <= ln2/128, ln2/64 split into a double
 * and its residual, e^r by its Taylor series to degree 5 in Horner form,
 * times 2^(j/64), times 2^m.  Used by the build-defined speculative verify so
 * that the device and this oracle evaluate bit-identical weights; every step
 * is one IEEE operation. */
double tmo_exp64(double x) {
    if (isnan(x)) return x;
    if (x < -746.0) return 0.0;
    if (x > 709.782712893384) return INFINITY;
    const double kd = nearbyint(x * 0x1.71547652b82fep+6);   /* ties to even */
    double r = fma(-kd, 0x1.62e42fefa39efp-7, x);
    r = fma(-kd, 0x1.abc9e3b39803fp-62, r);
    double p = 1.0 / 120;
    p = fma(p, r, 1.0 / 24);
    p = fma(p, r, 1.0 / 6);
    p = fma(p, r, 0.5);
    p = fma(p, r, 1.0);
    p = fma(p, r, 1.0);
    const int ki = (int)kd;
    int m = ki >> 6;   /* floor division: arithmetic shift */
    double y = kExp2_64ths[ki & 63] * p;
    if (m > 1023) {
        y = y * 2.0;
        m -= 1;
    }
    if (m < -1020) {
        y = y * 0x1p-200;
        m += 200;
    }
    union { double d; uint64_t u; } s;
    s.u = (uint64_t)(int64_t)(m + 1023) << 52;
    return y * s.d;
}

/* Weights on a 2^-44 grid: y * 2^44 rounded to the nearest whole number,
 * ties to even (one IEEE operation on the device). */
int64_t tmo_q44(double y) {
    return (int64_t)nearbyint(y * 17592186044416.0);
}

/* Softmax weights of one row: lg = v / T, m = max lg,
 * e_i = q44(exp64(lg_i - m)), Z = sum e_i (exact). */
int tmo_spec_weights(const float* row, int V, float temperature, int64_t* e, int64_t* Z,
                     float* m) {
    float mx = -INFINITY;
    for (int i = 0; i < V; ++i) {
        const float v = row[i];
        if (isnan(v) || v == INFINITY) return ROW_NONFINITE;
        const float l = v / temperature;
        if (l > mx) mx = l;
    }
    if (mx == -INFINITY) return ROW_ALL_MASKED;
    if (mx == INFINITY) return ROW_NONFINITE;
    int64_t z = 0;
    for (int i = 0; i < V; ++i) {
        const float l = row[i] / temperature;
        e[i] = tmo_q44(tmo_exp64((double)l - (double)mx));
        z += e[i];
    }
    *Z = z;
    *m = mx;
    return ROW_OK;
}

/* Smallest id whose inclusive prefix weight exceeds floor(u * W). */
static int inverse_cdf(const int64_t* w, int V, int64_t W, double u) {
    int64_t t = (int64_t)floor(u * (double)W);
    if (t > W - 1) t = W - 1;
    int64_t acc = 0;
    for (int i = 0; i < V; ++i) {
        acc += w[i];
        if (acc > t) return i;
    }
    return V - 1;
}

/* Speculative accept/reject for one sequence (Leviathan, Kalman, Matias,
 * "Fast Inference from Transformers via Speculative Decoding", 2023; Chen et
 * al. 2023).  No reference counterpart beyond the greedy limit
 * (tensormark/llama.h:5127-5131).  words holds k + 1 word pairs: pair i
 * (i < k) is the accept test of draft i, pair k the final draw. */
int tmo_spec_verify_seq(const float* target, const float* draft, int V, int k,
                        const int32_t* draft_tokens, float temperature,
                        const uint32_t* words, int32_t* accepted, int32_t* token) {
    *accepted = 0;
    *token = -1;
    if (!(temperature > 0.0f && temperature <= FLT_MAX)) return ROW_BAD_PARAMS;
    int64_t* et = (int64_t*)malloc((size_t)V * sizeof(int64_t));
    int64_t* ed = (int64_t*)malloc((size_t)V * sizeof(int64_t));
    int64_t Zt = 0, Zd = 0;
    float mt, md;
    const double uf = tmo_canonical(words[2 * k], words[2 * k + 1]);
    int st = ROW_OK;
    for (int i = 0; i < k; ++i) {
        st = tmo_spec_weights(target + (int64_t)i * V, V, temperature, et, &Zt, &mt);
        if (st) goto out;
        st = tmo_spec_weights(draft + (int64_t)i * V, V, temperature, ed, &Zd, &md);
        if (st) goto out;
        const int x = draft_tokens[i];
        if (x < 0 || x >= V) { st = ROW_BAD_PARAMS; goto out; }
        double r;
        if (ed[x] == 0) r = et[x] > 0 ? 1.0 : 0.0;
        else r = ((double)et[x] * (double)Zd) / ((double)ed[x] * (double)Zt);
        const double u = tmo_canonical(words[2 * i], words[2 * i + 1]);
        if (u < r) continue;
        /* First rejection: residual max(p_t - p_d, 0) on the 2^-44 grid. */
        int64_t R = 0;
        for (int v = 0; v < V; ++v) {
            const double pt = (double)et[v] / (double)Zt;
            const double pd = (double)ed[v] / (double)Zd;
            const double d = pt - pd;
            ed[v] = d > 0.0 ? tmo_q44(d) : 0;
            R += ed[v];
        }
        *accepted = i;
        *token = R > 0 ? inverse_cdf(ed, V, R, uf) : inverse_cdf(et, V, Zt, uf);
        goto out;
    }
    st = tmo_spec_weights(target + (int64_t)k * V, V, temperature, et, &Zt, &mt);
    if (st) goto out;
    *accepted = k;
    *token = inverse_cdf(et, V, Zt, uf);
out:
    free(et);
    free(ed);
    return st;
}

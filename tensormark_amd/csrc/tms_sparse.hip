// tms_sparse.hip -- the sampler kernel for calls whose grammar masks allow
// few ids a row (tms_sample_args.row_kinds = TMS_ROWS_SPARSE_MASK): only the
// allowed logits are read.
//
// A masked-out id is -inf before anything else (tensormark/llama_chat.cpp
// GrammarFilter::apply, then tmsample::sample), so it takes no part in the
// penalties, the top-k, the softmax sums or the draw except as a -inf entry:
// the row's answer depends on the allowed ids' logits alone.  One
// 1024-thread workgroup a row:
//
//   mask      the row's mask words into registers (thread t: words t,
//             t + 1024, ..., at most kWpt, every load issued at once); each
//             thread's allowed count and a 16-wave scan give every entry's
//             index;
//   ids       each wave's non-zero words expanded half-wave by half-wave
//             (lane j of a half takes bit j), two words a step, into the
//             allowed ids in LDS; then their logits, at most kGpt loads a
//             thread issued together;
//   window    history counts per allowed entry (an id's entry index from its
//             word's prefix and a popcount), the compounding penalty
//             (tmsample.h:58-61), then frequency/presence;
//   select    greedy: the largest key; sampled rows, on waves 0-3 (the
//             others leave): keys (v / T, then lowest id) ranked by
//             bucket_rank, then the fp64 tail of tmsample::sample
//             (tmsample.h:184-199): tail_topk for top-k <= 128, else the
//             top-p block tail.
//
// A row with more than kSparseCap allowed ids, a top-p row with more than
// kToppCap finite entries, or an answer that needs the order past the held
// entries is sampled whole (tms_dense.h) by the same workgroup, so every row
// gets the reference's answer; only the speed depends on the hint.
#include "tms_dense.h"
#include "tms_select.h"

namespace tms {
namespace sparse {

constexpr int kNT = 1024;                             // threads of the gather phases
constexpr int kNW = kNT / 64;
constexpr int kSparseCap = kUni;                      // allowed ids a row held in LDS
constexpr int kPer = kSparseCap / kBlock;             // keys a thread of the rank holds
constexpr int kGpt = kSparseCap / kNT;                // entries a thread gathers
constexpr int kMaxWords = kSparseMaxVocab / 32;       // mask words a row
constexpr int kWpt = kMaxWords / kNT;                 // mask words a thread holds

struct Smem {
    uint32_t mw[kMaxWords];          // the row's mask (bits past the vocabulary cleared)
    uint16_t wpre[kMaxWords];        // entry index of each word's first allowed id
    alignas(16) uint64_t keys[kSparseCap + 16];   // the entries' keys (0: absent)
    alignas(16) uint64_t srt[kSparseCap + 16];    // ranked keys
    alignas(16) double pr[kToppCap];              // fp64 tail: weights
    alignas(16) double q[kToppCap];               // fp64 tail: quotients
    uint32_t ids[kSparseCap];        // allowed ids, in entry order
    uint32_t cnt[kSparseCap];        // window occurrences per entry
    int pbits[kBuckets];             // bucket_rank's counts
    int hist[8 * kWaves];            // tail_topp_block's per-wave minima
    uint64_t wave_k[kNW];
    float wave_f[kWaves];
    int wave_i[kNW];
    int wave_s[kNW];                 // the mask scan's per-wave counts (written once)
    int wave_z[kNW];                 //   and non-zero words
    float wave_q[kNW];               // the least finite key quotient per wave
    uint64_t theta;
    int misc[4];
};
static_assert(sizeof(DenseLds) <= sizeof(uint32_t) * kMaxWords, "the whole-row path's LDS lies over the mask");

// Whether any allowed entry of the row is NaN or +inf (the whole-row path
// takes finite rows only): one pass over the row.
template <typename T>
__device__ bool row_nonfinite(const KArgs& a, int row, Smem& sm) {
    const int t = threadIdx.x;
    const T* base = (const T*)a.logits + (int64_t)row * a.row_stride;
    const uint32_t* mrow = a.mask + (int64_t)row * a.mask_stride;
    int bad = 0;
    for (int i = t; i < a.V; i += kBlock)
        if ((mrow[i >> 5] >> (i & 31)) & 1u) bad |= __builtin_amdgcn_class(Elt<T>::scalar(base + i), 0x203);
    bad = __any(bad != 0);
    if ((t & 63) == 0) sm.wave_i[t >> 6] = bad;
    lds_sync();
    int any = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) any |= sm.wave_i[w];
    lds_sync();
    return any != 0;
}

template <typename T>
__global__ __launch_bounds__(kNT) void sparse_kernel(KArgs a) {
    __shared__ Smem sm;
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    const int row = blockIdx.x;
    const int V = a.V;
    const int W = (V + 31) >> 5;
    const T* base = (const T*)a.logits + (int64_t)row * a.row_stride;
    const uint32_t* mrow = a.mask + (int64_t)row * a.mask_stride;
    const tms_row_params P = a.params[row];

    // ---- the mask: thread t holds words t, t + 1024, ... in registers (all
    //      loads issued at once); each thread's allowed count.  The gather
    //      phases run on 16 waves (four a SIMD, so their dependent chains
    //      interleave); the rank and the tails on waves 0-3, the others
    //      leaving after the keys.
    const uint32_t tail_bits = (V & 31) ? (1u << (V & 31)) - 1u : ~0u;
    uint32_t mwr[kWpt];
    int c = 0, cz = 0;
#pragma unroll
    for (int i = 0; i < kWpt; ++i) {
        const int w = t + i * kNT;
        uint32_t x = w < W ? mrow[w] : 0u;
        if (w == W - 1) x &= tail_bits;
        mwr[i] = x;
        c += __popc(x);
        cz += x ? 1 : 0;
    }
    // the thread's first entry index and its first slot in the list of
    // non-zero words: scans over the 16 waves
    int n = 0, tb = 0, nzw = 0, zb = 0;
    {
        const int inc = wave_incl_scan_i32(c);
        const int incz = wave_incl_scan_i32(cz);
        if (lane == 63) {
            sm.wave_s[wv] = inc;
            sm.wave_z[wv] = incz;
        }
        lds_sync();
#pragma unroll
        for (int i = 0; i < kNW; ++i) {
            const int x = sm.wave_s[i], z = sm.wave_z[i];
            tb += i < wv ? x : 0;
            zb += i < wv ? z : 0;
            n += x;
            nzw += z;
        }
        tb += inc - c;
        zb += incz - cz;
        // no barrier: nothing writes wave_s or wave_z again
    }

    const bool greedy = P.greedy != 0;
    const float temp = P.temperature;
    const bool bad_params = !greedy && !(temp > 0.0f && temp <= FLT_MAX);
    const int K = greedy ? 1 : ((P.top_k <= 0 || P.top_k > V) ? V : P.top_k);
    const int mode = greedy ? MODE_GREEDY : (K <= kTopkFast ? MODE_TOPK : MODE_TOPP);
    const bool divide = !greedy && temp != 1.0f;
    int nrec = 0;
    if (a.recent) {
        nrec = a.n_recent ? a.n_recent[row] : (int)a.recent_stride;
        nrec = min(max(nrec, 0), (int)a.recent_stride);
    }
    Pen pn;
    pn.rep_on = !(P.repeat_penalty <= 1.0f);
    pn.fp_on = P.frequency_penalty != 0.0f || P.presence_penalty != 0.0f;
    pn.on = nrec > 0 && P.repeat_last_n > 0 && (pn.rep_on || pn.fp_on);
    pn.rep = P.repeat_penalty;
    pn.freq = P.frequency_penalty;
    pn.pres = P.presence_penalty;
    const int from = pn.on ? (nrec > P.repeat_last_n ? nrec - P.repeat_last_n : 0) : 0;
    const int32_t* hist = a.recent ? a.recent + (int64_t)row * a.recent_stride : nullptr;

    if (bad_params || n == 0) {
        if (t < kBlock) write_row_error(a, row, bad_params ? TMS_ROW_BAD_PARAMS : TMS_ROW_ALL_MASKED);
        return;
    }
    DenseLds& L = *reinterpret_cast<DenseLds*>(sm.mw);   // the mask is dead when the whole row is sampled
    if (n > kSparseCap) {
        if (t >= kBlock) return;   // the whole-row path runs on waves 0-3
        // more allowed ids than the LDS holds: the whole row
        if (greedy) {
            [[clang::always_inline]] dense_greedy<T>(a, row, pn, from, nrec, L);
        } else if ([&]() { bool r; [[clang::always_inline]] r = row_nonfinite<T>(a, row, sm); return r; }()) {
            write_row_error(a, row, TMS_ROW_NONFINITE);
        } else {
            [[clang::always_inline]] dense_inline<T>(a, row, L);
        }
        return;
    }

    // ---- the allowed ids in entry order (thread, then word), then their
    //      logits.  The non-zero words go to a list (word, its index, its
    //      first entry index), and the workgroup's 32 half-waves expand the
    //      list's words in turn (lane j of a half takes bit j), so no lane
    //      loops over its bits or its zero words.  With a window, each word
    //      and its first entry index go to LDS for the history lookups.
    {
        // n <= kSparseCap here, so at most that many non-zero words, each
        // entry index below 2^11 and each word index below 2^13
        static_assert(kSparseCap <= 2048 && kMaxWords <= 8192, "list word packing");
        uint64_t* wl = sm.keys;   // dead until the keys are formed
        int e = tb, z = zb;
#pragma unroll
        for (int i = 0; i < kWpt; ++i) {
            const int w = t + i * kNT;
            const uint32_t x = mwr[i];
            if (pn.on && w < W) {
                sm.mw[w] = x;
                sm.wpre[w] = (uint16_t)e;
            }
            if (x) wl[z++] = ((uint64_t)x << 32) | (uint32_t)((w << 11) | e);
            e += __popc(x);
        }
        lds_sync();
        const int bitj = lane & 31;
        for (int q = t >> 5; q < nzw; q += kNT / 32) {
            const uint64_t d = wl[q];
            const uint32_t x = (uint32_t)(d >> 32), we = (uint32_t)d;
            if ((x >> bitj) & 1u)
                sm.ids[(we & 2047u) + __popc(x & ((1u << bitj) - 1u))] = ((we >> 11) << 5) + (uint32_t)bitj;
        }
    }
    if (pn.on)
        for (int e = t; e < n; e += kNT) sm.cnt[e] = 0u;
    lds_sync();
    float v[kGpt];
#pragma unroll
    for (int j = 0; j < kGpt; ++j) {
        const int e = t + j * kNT;
        v[j] = e < n ? Elt<T>::scalar(base + sm.ids[e]) : -__builtin_huge_valf();
    }
    // ---- window counts per allowed entry (ids outside the vocabulary and
    //      masked ids have no entry)
    if (pn.on) {
        for (int p = from + t; p < nrec; p += kNT) {
            const int id = hist[p];
            if (id >= 0 && id < V) {
                const uint32_t x = sm.mw[id >> 5];
                if ((x >> (id & 31)) & 1u) {
                    const int e = sm.wpre[id >> 5] + __popc(x & ((1u << (id & 31)) - 1u));
                    atomicAdd(&sm.cnt[e], 1u);
                }
            }
        }
        lds_sync();
    }
    int bad = 0, fin = 0;
    uint64_t gbest = 0ull;
    float qlo = __builtin_huge_valf();
#pragma unroll
    for (int j = 0; j < kGpt; ++j) {
        const int e = t + j * kNT;
        if (e < n) {
            float x = v[j];
            bad |= __builtin_amdgcn_class(x, 0x203);
            if (pn.on) {
                const uint32_t k = sm.cnt[e];
                if (k && x != -__builtin_huge_valf()) {
                    x = apply_pen(x, k, pn);
                    bad |= __builtin_amdgcn_class(x, 0x203);
                }
            }
            uint64_t key = 0ull;
            if (x != -__builtin_huge_valf()) {
                key = ckey(divide ? x / temp : x, sm.ids[e]);
                qlo = fminf(qlo, ckey_val(key));
                ++fin;
            }
            gbest = key > gbest ? key : gbest;
            sm.keys[e] = key;
        }
    }
    // block totals: NaN / +inf, finite entries, the largest key
    bad = __any(bad != 0);
    fin = wave_sum_dpp(fin);
    gbest = wave_max_u64_dpp(gbest);
    qlo = -wave_max_f32_dpp(-qlo);
    if (lane == 0) {
        sm.wave_i[wv] = bad ? -1 : fin;
        sm.wave_k[wv] = gbest;
        sm.wave_q[wv] = qlo;
    }
    if (t < kBuckets) sm.pbits[t] = 0;   // bucket_rank's counts, zeroed before its atomics
    lds_sync();
    int N = 0;
    bool nonfin = false;
    uint64_t best = 0ull;
    float qmin = __builtin_huge_valf();
#pragma unroll
    for (int w = 0; w < kNW; ++w) {
        const int x = sm.wave_i[w];
        nonfin |= x < 0;
        N += x < 0 ? 0 : x;
        best = sm.wave_k[w] > best ? sm.wave_k[w] : best;
        qmin = fminf(qmin, sm.wave_q[w]);
    }
    if (t >= kBlock) return;   // from here waves 0-3 (the leavers drop out of the barriers)
    lds_sync();   // the totals are read before bucket_rank writes wave_k again
    if (nonfin) {
        write_row_error(a, row, TMS_ROW_NONFINITE);
        return;
    }
    if (N == 0) {
        write_row_error(a, row, TMS_ROW_ALL_MASKED);
        return;
    }
    if (mode == MODE_GREEDY) {
        const int tok = (int)ckey_id(best);
        if (t == 0) {
            a.out_tokens[row] = tok;
            a.out_status[row] = TMS_ROW_OK;
            if (a.out_keep) a.out_keep[row] = 0;
        }
        for (int i = t; i < a.topk_cap; i += kBlock) {
            if (a.out_topk_ids) a.out_topk_ids[(int64_t)row * a.topk_cap + i] = i == 0 ? tok : -1;
            if (a.out_topk_probs) a.out_topk_probs[(int64_t)row * a.topk_cap + i] = i == 0 ? 1.0f : 0.0f;
        }
        return;
    }
    if (ckey_val(best) == __builtin_huge_valf()) {   // v / T overflowed
        write_row_error(a, row, TMS_ROW_NONFINITE);
        return;
    }
    bool whole = false;
    if (mode == MODE_TOPP && min(N, K) > kToppCap) {
        whole = true;
    } else {
        // ---- rank: the top min(N, K) keys (zero keys are absent) into srt
        const int nkeep = min(N, K);
        sm.keys[n] = 0ull;   // bucket_rank reads whole 16-byte words
        // the range of the finite keys' quotients, from the block totals
        const float qmax = ckey_val(best);
        if (n <= 2 * kBlock) {
            [[clang::always_inline]] bucket_rank<2, true>(sm.keys, n, nkeep, sm.srt, sm.pbits, sm, qmax, qmin);
        } else if (n <= 4 * kBlock) {
            [[clang::always_inline]] bucket_rank<4, true>(sm.keys, n, nkeep, sm.srt, sm.pbits, sm, qmax, qmin);
        } else {
            [[clang::always_inline]] bucket_rank<kPer, true>(sm.keys, n, nkeep, sm.srt, sm.pbits, sm, qmax, qmin);
        }
        lds_sync();
        uint32_t w0, w1;
        if (mode == MODE_TOPK) {
            if (N < K) {
                // Fewer than K finite ids: the top-k goes on with -inf entries
                // in ascending id order, the ids in [0, K + N) outside the
                // finite set (K + N <= 2 * kTopkFast <= kBlock).
                const int q = t;
                int member = 0;
                if (q < K + N)
                    for (int i = 0; i < N; ++i) member |= (int)ckey_id(sm.srt[i]) == q;
                const int gap = (q < K + N && !member && q < V) ? 1 : 0;
                int tot;
                const int p = block_excl_scan(gap, tot, sm);
                if (gap && p < K - N) sm.srt[N + p] = ckey(-__builtin_huge_valf(), (uint32_t)q);
                lds_sync();
            }
            if (wv == 0) {
                row_uniform(a, row, P, w0, w1);
                [[clang::always_inline]] tail_topk(a, row, P, sm.srt, K, K, sm.pr, sm.q, w0, w1);
            }
            return;
        }
        // ---- top-p: the entries within kSigSpan of the maximum, their
        //      weights; the block tail, else the sequential one
        const double mx = (double)ckey_val(sm.srt[0]);
        int sig = 0;
        for (int i = t; i < nkeep; i += kBlock) {
            const double d = (double)ckey_val(sm.srt[i]) - mx;
            sig += d >= -(double)kSigSpan ? 1 : 0;
            sm.pr[i] = exp(d);
        }
        sig = wave_sum_dpp(sig);
        if (lane == 0) sm.wave_i[wv] = sig;
        lds_sync();
        int ns = 0;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) ns += sm.wave_i[w];
        ns = min(ns, K);
        lds_sync();
        row_uniform(a, row, P, w0, w1);
        const int tp = tail_topp_block(a, row, P, sm.srt, ns, K, sm.pr, sm.q, w0, w1, sm);
        if (tp == 2) {
            if (wv == 0) {
                bool lost;
                [[clang::always_inline]] lost = tail_topp(a, row, P, sm.srt, ns, K, sm.pr, sm.q);
                if (lane == 0) sm.misc[0] = lost ? 1 : 0;
            }
        } else if (t == 0) {
            sm.misc[0] = tp;
        }
        lds_sync();
        whole = sm.misc[0] != 0;
        lds_sync();
    }
    if (whole) {
        [[clang::always_inline]] dense_inline<T>(a, row, L);
    }
}

}  // namespace sparse
}  // namespace tms

// Launch of the sparse-mask kernel for tms_sample_batch: one workgroup a
// row; the host checks vocab <= kSparseMaxVocab and a mask.
int tms_launch_sparse(const tms::KArgs& k, int dtype, int batch, hipStream_t stream) {
    const dim3 grid((unsigned)batch), block(tms::sparse::kNT);
    switch (dtype) {
        case TMS_DTYPE_F32:
            hipLaunchKernelGGL((tms::sparse::sparse_kernel<float>), grid, block, 0, stream, k);
            break;
        case TMS_DTYPE_F16:
            hipLaunchKernelGGL((tms::sparse::sparse_kernel<_Float16>), grid, block, 0, stream, k);
            break;
        default:
            hipLaunchKernelGGL((tms::sparse::sparse_kernel<tms::Bf16>), grid, block, 0, stream, k);
            break;
    }
    return hipGetLastError() == hipSuccess ? TMS_OK : TMS_ERR_HIP;
}

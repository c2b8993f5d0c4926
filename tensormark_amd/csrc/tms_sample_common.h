// tms_sample_common.h -- device code shared by the sampler kernels: limits,
// the kernel argument block, the history penalty, the exact radix fallback
// of a chunk's top-K, and the sequential fp64 tail of tmsample::sample
// (tensormark/tmsample.h:184-199) in its top-k and top-p forms.
#pragma once

#include <float.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/tmsample_hip.h"
#include "tms_device.h"
#include "tms_context.h"

#ifdef TMS_TRACE
// Trace-only builds: lane 0 of each wave stamps the 100 MHz real-time
// counter at phase boundaries, 24 slots per wave, into a buffer passed as a
// kernel argument (no memory read on the traced path).
#define TMS_TR(i)                                                                   \
    do {                                                                            \
        asm volatile("; trace point " #i);                                          \
        if ((threadIdx.x & 63) == 0 && a.trace)                                     \
            a.trace[(blockIdx.x * 4 + (threadIdx.x >> 6)) * 24 + (i)] =             \
                __builtin_amdgcn_s_memrealtime();                                   \
    } while (0)
#define TMS_TV(i, val)                                                              \
    do {                                                                            \
        if ((threadIdx.x & 63) == 0 && a.trace)                                     \
            a.trace[(blockIdx.x * 4 + (threadIdx.x >> 6)) * 24 + (i)] = (uint64_t)(val); \
    } while (0)
#else
#define TMS_TR(i) ((void)0)
#define TMS_TV(i, val) ((void)0)
#endif

namespace tms {

constexpr int kEpt = 64;                   // logits per thread held in registers
constexpr int kChunk = kBlock * kEpt;      // ids per workgroup
constexpr int kEptPacked = 80;             // the same for the packed stream (2-byte rows, no window)
constexpr int kTopkFast = 128;             // largest K on the threshold path
constexpr int kCand = 512;                 // chunk candidates held in LDS
constexpr int kListStride = kCand + 2;     // u64 per published list: header + entries
constexpr int kUni = 2048;                 // merge staging (u64)
constexpr int kToppCap = 1024;             // candidates per top-p row
constexpr int kMaxChunks = 64;             // chunks per row (vocab <= 1,048,576)
constexpr int kWideMaxChunksHost = 16;     // chunks per row of the wide top-k kernel
constexpr int kWideChunkVecs = 4096;       // 16-byte vectors per chunk of the wide kernel
constexpr int kWideMaxWindow = 1024;       // history positions the wide kernel holds (one per thread)
constexpr int kWideListStride = 136;       // u64 per (row, chunk) list of the wide kernel: header + 128 keys, padded
constexpr int kRankLists = 16;             // most chunk lists the sampled merge reads in one round
constexpr float kSigSpan = 40.0f;          // exp(-40) < 2^-57: below this, no effect
constexpr uint64_t kReady = 1ull << 63;    // header bit: the list is complete
constexpr int kPollCap = 1 << 20;          // bound on the merger's wait per list
constexpr int kReadRounds = 64;            // bound on the merger's re-reads of a sample
constexpr int kDenseSlotsMax = 256;        // whole-row regions of a context
constexpr int kHistMax = TMS_HISTORY_MAX_IDS; // ids one row's history pre-pass may list
constexpr int kSparseMaxVocab = TMS_SPARSE_MAX_VOCAB;   // vocab of the sparse-mask kernel (its mask in LDS)
static_assert(kUni == TMS_SPARSE_MAX_IDS, "the sparse-mask kernel holds kUni ids");

enum : int { MODE_GREEDY = 0, MODE_TOPK = 1, MODE_TOPP = 2 };
enum : int { FLAG_NONFINITE = 1, FLAG_OVERFLOW = 2 };

struct KArgs {
    const void* logits;
    int64_t row_stride;
    int V;
    int S;            // chunks per row
    int CE;           // ids per chunk (multiple of the vector width)
    const tms_row_params* params;
    const int32_t* recent;
    const int32_t* n_recent;
    int64_t recent_stride;
    const uint32_t* mask;     // never null: an all-ones row when the caller has none
    int64_t mask_stride;      // 0 with the all-ones row
    const uint32_t* draws;
    int32_t* out_tokens;
    int32_t* out_status;
    int32_t* out_keep;
    int32_t* out_topk_ids;
    float* out_topk_probs;
    int topk_cap;
    // workspace
    uint32_t* counters;    // [B] arrival tickets, reset by the merger
    uint64_t* lists;       // [B][S][kListStride]: header, entries; headers reset by the merger
    uint64_t* tlists;      // [B][S][kWideListStride]: the wide kernel's lists, zeroed by the merger
    uint64_t* dense;       // [dense_slots][2 * dense_stride]: the whole-row path's keys and
                           // sums; null when the call has no whole-row path
    int64_t dense_stride;  // >= V
    uint32_t* dlocks;      // [dense_slots]: 1 while a workgroup works in the region, else 0
    int dense_slots;
    const float* ov_vals;  // [B][kHistMax] the history pre-pass's values, with `recent`,
                           // `n_recent` its id lists (n_recent -1: the row overflowed);
                           // null when the call has no pre-pass
#ifdef TMS_TRACE
    uint64_t* trace;
#endif
};

// History penalties of one row.  With `ov` (calls with the history
// pre-pass) the window holds the pre-pass's list of distinct ids instead of
// the history, each window word holds the id's list position + 1 instead of
// a count, and ov[] holds the ids' final values.
struct Pen {
    bool on, rep_on, fp_on;
    float rep, freq, pres;
    const float* ov = nullptr;
};

// Repetition penalty applied `cnt` times (tmsample.h:61), then frequency and
// presence: v -= (float)cnt * freq + presence.  With pn.ov, the pre-pass's
// value of list entry cnt - 1.
__device__ __forceinline__ float apply_pen(float v, uint32_t cnt, const Pen& pn) {
    if (pn.ov) return pn.ov[cnt - 1];
    if (pn.rep_on)
        for (uint32_t r = 0; r < cnt; ++r) v = v > 0.f ? v / pn.rep : v * pn.rep;
    if (pn.fp_on) {
        const float t1 = (float)cnt * pn.freq;
        const float tt = t1 + pn.pres;
        v = v - tt;
    }
    return v;
}

// Shared memory of one workgroup.  `big` holds the chunk's window counts
// (16 bits per id) during the scan and the merge's lists afterwards.
struct Smem {
    union {
        uint32_t cnt[kChunk / 2];
        struct {
            uint64_t uni[kUni];    // the lists of a merge round; pr[] of the top-p tail
            uint64_t surv[kUni];   // the merged, sorted entries; q[] of the top-p tail
        } m;
    } big;
    uint64_t cand[kCand];
    // One region for two phases (lds_syncs between them): pbits, per thread
    // its penalised entries (bit = slot * VEC + e), read once after the
    // window and reused by the merge's buckets; tkey, the order keys of the
    // thread maxima, during the selection.  Keeping the workgroup's LDS at
    // most 40 KB lets four workgroups share a CU.
    union {
        uint32_t pbits[2 * kBlock];
        uint32_t tkey[kBlock];
    };
    int wave_i[kWaves];
    uint64_t wave_k[kWaves];
    float wave_f[kWaves];
    int list_src[kMaxChunks + 1];
    int list_n[kMaxChunks];        // entries of each chunk list
    int list_s[kMaxChunks];        // survivors of each chunk list
    int hist[256];
    int ncand;
    int nvalid;                    // top-p tail: the row takes the whole-row path
    int misc[8];
    uint64_t theta;
};

template <typename SM>
__device__ __forceinline__ int block_excl_scan(int v, int& total, SM& sm) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int inc = wave_incl_scan_i32(v);
    if (lane == 63) sm.wave_i[w] = inc;
    lds_sync();
    int base = 0;
    total = 0;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) {
        const int t = sm.wave_i[i];
        base += i < w ? t : 0;
        total += t;
    }
    lds_sync();
    return base + inc - v;
}

// Sort sm.cand[0..n) descending in place (n <= kCand) by ranking: each key's
// rank is the number of larger keys, counted with broadcast LDS reads.
template <typename SM>
__device__ void sort_cand(int n, SM& sm) {
    const int t = threadIdx.x;
    if (n <= 1) return;
    if (n <= 64) {
        // One wave; its LDS operations complete in order, so the reads of
        // the loop finish before the scatter.
        if (t < 64) {
            const uint64_t mine = t < n ? sm.cand[t] : 0ull;
            int rank = 0;
#pragma unroll 8
            for (int j = 0; j < n; ++j) rank += sm.cand[j] > mine ? 1 : 0;
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
            if (t < n) sm.cand[rank] = mine;
        }
        lds_sync();
        return;
    }
    constexpr int R = kCand / kBlock;
    uint64_t mine[R];
    int rank[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int i = t + r * kBlock;
        mine[r] = i < n ? sm.cand[i] : 0ull;
        rank[r] = 0;
    }
    if (n <= kBlock) {
#pragma unroll 8
        for (int j = 0; j < n; ++j) rank[0] += sm.cand[j] > mine[0] ? 1 : 0;
    } else {
#pragma unroll 4
        for (int j = 0; j < n; ++j) {
            const uint64_t o = sm.cand[j];
#pragma unroll
            for (int r = 0; r < R; ++r) rank[r] += o > mine[r] ? 1 : 0;
        }
    }
    lds_sync();
#pragma unroll
    for (int r = 0; r < R; ++r)
        if (t + r * kBlock < n) sm.cand[rank[r]] = mine[r];
    lds_sync();
}

// The final value of chunk id `id` (mask, then penalties from the LDS
// window counts), read again from memory: the slow paths use it.
template <typename T, typename SM>
__device__ float slow_value(const T* base, const uint32_t* mrow, int id, int e0, const Pen& pn,
                            const SM& sm) {
    float v = Elt<T>::scalar(base + id);
    if (!((mrow[id >> 5] >> (id & 31)) & 1u)) return -__builtin_huge_valf();
    if (pn.on) {
        const int off = id - e0;
        const uint32_t c = (sm.big.cnt[off >> 1] >> ((off & 1) * 16)) & 0xFFFFu;
        if (c) v = apply_pen(v, c, pn);
    }
    return v;
}

// Exact top-K of the chunk's finite entries by candidate key, for chunks
// where the threshold admits too many: a radix select over the keys of
// v / T (8 bits per pass) with the chunk re-read from memory, then the
// strictly greater entries and the lowest-id ties.  Writes sm.cand, unsorted;
// returns the count (<= K).  The penalties come as scalars: a Pen argument
// (by reference, or by value once it holds a pointer) put the caller's Pen in
// scratch memory, and a kernel with any scratch launched its workgroups
// measurably slower (B = 1024, V = 256000: 256 -> 244 us).
template <typename T, typename SM>
__device__ __noinline__ int radix_slow(const T* base, const uint32_t* mrow, int e0, int e1, int K,
                                       float temp, bool divide, bool pen_on, bool pen_rep_on, bool pen_fp_on,
                                       float pen_rep, float pen_freq, float pen_pres, const float* pen_ov,
                                       SM& sm) {
    Pen pn;
    pn.on = pen_on;
    pn.rep_on = pen_rep_on;
    pn.fp_on = pen_fp_on;
    pn.rep = pen_rep;
    pn.freq = pen_freq;
    pn.pres = pen_pres;
    pn.ov = pen_ov;
    const int t = threadIdx.x;
    const float NEG_INF = -__builtin_huge_valf();
    uint32_t prefix = 0, pmask = 0;
    int remaining = K;
    for (int shift = 24; shift >= 0; shift -= 8) {
        sm.hist[t] = 0;
        if (t == 0) {
        sm.ncand = 0;
        sm.misc[2] = 0;   // the merger's read found an incomplete list
    }
        lds_sync();
        for (int id = e0 + t; id < e1; id += kBlock) {
            const float v = slow_value(base, mrow, id, e0, pn, sm);
            if (v == NEG_INF) continue;
            const uint32_t k = okey(divide ? v / temp : v);
            if ((k & pmask) == prefix) atomicAdd(&sm.hist[(k >> shift) & 0xFF], 1);
        }
        lds_sync();
        const int h = sm.hist[255 - t];   // thread t holds digit 255 - t
        int total;
        const int above = block_excl_scan(h, total, sm);
        if (shift == 24 && total <= K) {
            // At most K finite entries: all of them.
            for (int id = e0 + t; id < e1; id += kBlock) {
                const float v = slow_value(base, mrow, id, e0, pn, sm);
                if (v == NEG_INF) continue;
                const int pos = atomicAdd(&sm.ncand, 1);
                sm.cand[pos] = ckey(divide ? v / temp : v, (uint32_t)id);
            }
            lds_sync();
            return sm.ncand;
        }
        if (above < remaining && above + h >= remaining) {
            sm.misc[0] = 255 - t;
            sm.misc[1] = above;
        }
        lds_sync();
        remaining -= sm.misc[1];
        prefix |= (uint32_t)sm.misc[0] << shift;
        pmask |= 0xFFu << shift;
        lds_sync();
    }
    // prefix is the K-th largest key; K - remaining keys are strictly greater.
    for (int id = e0 + t; id < e1; id += kBlock) {
        const float v = slow_value(base, mrow, id, e0, pn, sm);
        if (v == NEG_INF) continue;
        const float lg = divide ? v / temp : v;
        if (okey(lg) > prefix) {
            const int pos = atomicAdd(&sm.ncand, 1);
            sm.cand[pos] = ckey(lg, (uint32_t)id);
        }
    }
    lds_sync();
    const int g = sm.ncand;
    // Ties in id order, 256 consecutive ids per step.
    int taken = 0;
    for (int b0 = e0; b0 < e1 && taken < remaining; b0 += kBlock) {
        const int id = b0 + t;
        float lg = NEG_INF;
        int tie = 0;
        if (id < e1) {
            const float v = slow_value(base, mrow, id, e0, pn, sm);
            if (v != NEG_INF) {
                lg = divide ? v / temp : v;
                tie = okey(lg) == prefix;
            }
        }
        int tot;
        const int p = block_excl_scan(tie, tot, sm);
        if (tie && taken + p < remaining) sm.cand[g + taken + p] = ckey(lg, (uint32_t)id);
        taken += tot;
    }
    lds_sync();
    return g + (taken < remaining ? taken : remaining);
}

// Number of keys in the descending list L[0..n) that are greater than k.
__device__ __forceinline__ int count_greater(const uint64_t* L, int n, uint64_t k) {
    int lo = 0, hi = n;
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (L[mid] > k) lo = mid + 1;
        else hi = mid;
    }
    return lo;
}


__device__ __forceinline__ void write_row_error(const KArgs& a, int row, int status) {
    const int t = threadIdx.x;
    if (t == 0) {
        a.out_tokens[row] = -1;
        a.out_status[row] = status;
        if (a.out_keep) a.out_keep[row] = 0;
    }
    int32_t* ids = a.out_topk_ids ? a.out_topk_ids + (int64_t)row * a.topk_cap : nullptr;
    float* probs = a.out_topk_probs ? a.out_topk_probs + (int64_t)row * a.topk_cap : nullptr;
    for (int i = t; i < a.topk_cap; i += kBlock) {
        if (ids) ids[i] = -1;
        if (probs) probs[i] = 0.0f;
    }
}

__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
}

__device__ __forceinline__ void row_uniform(const KArgs& a, int row, const tms_row_params& P,
                                            uint32_t& w0, uint32_t& w1) {
    if (a.draws) {
        w0 = a.draws[2 * row];
        w1 = a.draws[2 * row + 1];
    } else {
        row_words(P.seed, P.offset, 0u, w0, w1);
    }
}

// Workgroup b of a B x S grid -> (row, chunk).  Workgroups are handed to
// the 8 XCDs round-robin by index, so rows are kept whole on one XCD: in the
// first 8 * floor(B / 8) rows, row r's chunks are the workgroups with
// b % 8 == r % 8, in order.  Each XCD then merges its own rows; with
// consecutive workgroups of a row on different XCDs, an XCD that ran a
// little behind held the last chunk, and so the merge, of nearly every row
// and fell further behind (B = 1024, S = 16: 501 of 515 merges on one XCD,
// 717 us against 290 us for the others).  The mapping is a bijection
// whatever the placement is.
__device__ __forceinline__ void wg_row_chunk(int S, int& row, int& c) {
    const int b = (int)blockIdx.x;
    const int B = (int)gridDim.x / S;
    const int whole = (B >> 3) << 3;
    if (b < whole * S) {
        const int s = b >> 3;
        row = (b & 7) + 8 * (s / S);
        c = s - (s / S) * S;
    } else {
        const int r = b - whole * S;
        row = whole + r / S;
        c = r - (r / S) * S;
    }
}

// Count of keys > k in the descending list L[0..n), n < P (P a power of
// two): a fixed number of halving steps, so searches in several lists can
// proceed in lock step.
__device__ __forceinline__ int count_gt_fixed(const uint64_t* L, int n, uint64_t k, int P) {
    int lo = 0;
    for (int step = P >> 1; step >= 1; step >>= 1) {
        const int nx = lo + step;
        const bool in = nx <= n;
        const uint64_t v = L[in ? nx - 1 : 0];
        lo = (in && v > k) ? nx : lo;
    }
    return lo;
}

// The sequential fp64 tail for top-k rows: n = K <= 128 sorted entries in
// `srt`, run by one wave.  pr, q and p live in LDS so every lane walks them
// in order (broadcast reads) and forms each sum exactly as tmsample::sample
// forms it, one dependent fp64 add per step; lane i & 63 keeps the partial
// sum at step i in a register.  The partial sums only grow (the terms are
// >= 0), so the top-p cut and the drawn index are counts of partial sums
// below the threshold.
// Zero the published lists of a row (header, entries and padding up to r of
// every chunk), threads tid0 .. nthr-1 of the workgroup: one index space of
// S lists x W words (W the longest list's words), so the lengths are
// independent reads rather than one list after another.
__device__ __forceinline__ void zero_lists(uint64_t* row_lists, int S, int r, const int* list_n,
                                           int tid0, int nthr) {
    int W = 1 + r;
    for (int cc = 0; cc < S; ++cc) W = max(W, 1 + list_n[cc]);
    for (int idx = tid0; idx < S * W; idx += nthr) {
        const int cc = idx / W, jj = idx - cc * W;
        if (jj < 1 + max(list_n[cc], r)) st_agent(&row_lists[(int64_t)cc * kListStride + jj], (uint64_t)0);
    }
}

// Eight doubles from LDS (16-byte reads; v + i 16-byte aligned).  Blocks of
// eight keep the sequential sums within the register budget of kernels that
// run two 1024-thread workgroups per CU.
__device__ __forceinline__ void ld8(const double* v, int i, double (&c)[8]) {
    const double2* v2 = (const double2*)(v + i);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const double2 d = v2[u];
        c[2 * u] = d.x;
        c[2 * u + 1] = d.y;
    }
}

// Left-to-right prefix sums of v[0..n) as a scalar loop computes them; v
// holds zeros from n up to the next multiple of 16 (x + 0.0 == x for
// x >= 0).  Lane 0 stores every prefix to pre[] (off the dependent chain);
// returns the total.
__device__ __forceinline__ double seq_prefix_sums(const double* v, int n, double* pre) {
    double s = 0.0;
    for (int i = 0; i < n; i += 8) {
        double c[8];
        ld8(v, i, c);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            s += c[e];
            c[e] = s;
        }
        if ((threadIdx.x & 63) == 0) {
            double2* p2 = (double2*)(pre + i);
#pragma unroll
            for (int u = 0; u < 4; ++u) p2[u] = make_double2(c[2 * u], c[2 * u + 1]);
        }
    }
    return s;
}

// First i in [0, n) whose left-to-right prefix sum v[0] + ... + v[i] is >=
// thr, or n (v >= 0 and zero-padded as above, so the prefixes never
// decrease).  Eight prefixes at a time stay in registers; the chain stops
// at the block that crosses.
__device__ __forceinline__ int first_prefix_ge(const double* v, int n, double thr) {
    double s = 0.0;
    for (int i = 0; i < n; i += 8) {
        double c[8];
        ld8(v, i, c);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            s += c[e];
            c[e] = s;
        }
        if (s >= thr) {
            int below = 0;
#pragma unroll
            for (int e = 0; e < 8; ++e) below += c[e] < thr ? 1 : 0;
            return i + below;
        }
    }
    return n;
}

// fp64 tail of tmsample::sample (tensormark/tmsample.h:185-199) for top-k
// rows, one wave, n = K <= 2 * 64 sorted entries in srt: pr = exp(lg - mx),
// z, the top-p and min-p cuts and the std::discrete_distribution draw, with
// every sum in the reference's order (uniform chains over LDS).
__device__ void tail_topk_exact(const KArgs& a, int row, const tms_row_params& P,
                                const uint64_t* srt, int n, int K, double* pr, double* q,
                                uint32_t w0, uint32_t w1) {
    const int lane = threadIdx.x & 63;
    const double u = canonical(w0, w1);
    const double mx = (double)ckey_val(srt[0]);
    const bool h0 = lane < n, h1 = lane + 64 < n;
    const double pr0 = h0 ? exp((double)ckey_val(srt[lane]) - mx) : 0.0;
    const double pr1 = h1 ? exp((double)ckey_val(srt[lane + 64]) - mx) : 0.0;
    // pr, q and p in LDS, each zero from n up to a multiple of 16
    double* zpre = pr + 256;   // the prefixes of z
    pr[lane] = pr0;
    pr[lane + 64] = pr1;
    wave_lds_sync();
    const double z = seq_prefix_sums(pr, n, zpre);   // tmsample.h:186-191
    const double q0 = pr0 / z, q1 = pr1 / z;
    q[lane] = q0;
    q[lane + 64] = q1;
    wave_lds_sync();
    // keep = first index with cum >= top_p, + 1, else K (tmsample.h:192-197;
    // a NaN top_p never compares true).
    const int fi = first_prefix_ge(q, n, (double)P.top_p);
    int kp = fi < n ? fi + 1 : K;
    if (P.min_p > 0.0f) {
        // min-p: the first entry below min_p ends the kept prefix.
        const double mp = (double)P.min_p;
        const uint64_t b0 = __ballot(lane >= 1 && h0 && pr0 < mp);
        const uint64_t b1 = __ballot(h1 && pr1 < mp);
        const int m = b0 ? __ffsll((unsigned long long)b0) - 1
                         : (b1 ? 64 + __ffsll((unsigned long long)b1) - 1 : K);
        if (m < kp) kp = m;
    }
    const int keep = kp;
    int tokidx = 0;
    if (keep >= 2) {
        // std::discrete_distribution over pr[0..keep): sum = accumulate(),
        // p = pr / sum, partial sums with the last forced to 1, then
        // lower_bound(u) = the first j < keep - 1 with cp_j >= u, else keep - 1.
        const double sum = zpre[keep - 1];
        const double p0 = pr0 / sum, p1 = pr1 / sum;
        pr[lane] = lane < keep - 1 ? p0 : 0.0;
        pr[lane + 64] = lane + 64 < keep - 1 ? p1 : 0.0;
        wave_lds_sync();
        tokidx = first_prefix_ge(pr, keep - 1, u);
    }
    if (lane == 0) {
        a.out_tokens[row] = (int)ckey_id(srt[tokidx]);
        a.out_status[row] = TMS_ROW_OK;
        if (a.out_keep) a.out_keep[row] = keep;
    }
    if (a.topk_cap) {
        int32_t* ids = a.out_topk_ids ? a.out_topk_ids + (int64_t)row * a.topk_cap : nullptr;
        float* probs = a.out_topk_probs ? a.out_topk_probs + (int64_t)row * a.topk_cap : nullptr;
        for (int i = lane; i < a.topk_cap; i += 64) {
            const bool have = i < n;
            const double qq = i < 64 ? q0 : q1;
            if (ids) ids[i] = have ? (int)ckey_id(srt[i]) : -1;
            if (probs) probs[i] = have ? (float)qq : 0.0f;
        }
    }
}

// Whether the reference's left-to-right prefix sums of quotients pr_j / D
// decide "first index k < m whose prefix is >= thr" the same way as the
// prefixes c (lane k in c0, lane k - 64 in c1) computed here as (tree
// prefix sum of pr) * fl(1 / D'), D' the tree's value of the divisor.  For
// n <= 128 non-negative terms: the tree prefixes carry at most 7 roundings
// per term (a 6-step DPP scan plus one addition), the scaling two (the
// reciprocal and the product), the reference's quotients and sequential
// additions 2n + 1, and the two divisors differ by at most (n + 7) * 2^-53
// relative, so the two differ by at most (3n + 17) * 2^-53 relative
// (401 * 2^-53 at n = 128), plus a few subnormal units; the margin below is
// 576 * 2^-53.  Returns false when some prefix up
// to the decision lies within the margin of thr (or thr is NaN): only the
// sequential sums decide it.
__device__ __forceinline__ bool decide_first_ge(double c0, double c1, double thr, int m, int& idx) {
    const int lane = threadIdx.x & 63;
    constexpr double kRel = (4.0 * 2 * 64 + 64.0) * 0x1p-53;
    constexpr double kAbs = 1e-300;
    const double m0 = (c0 + fabs(thr)) * kRel + kAbs, m1 = (c1 + fabs(thr)) * kRel + kAbs;
    const bool v0 = lane < m, v1 = lane + 64 < m;
    const uint64_t g0 = __ballot(v0 && c0 > thr + m0), g1 = __ballot(v1 && c1 > thr + m1);
    const uint64_t l0 = __ballot(!v0 || c0 < thr - m0), l1 = __ballot(!v1 || c1 < thr - m1);
    const int first = g0 ? __ffsll((unsigned long long)g0) - 1
                         : (g1 ? 64 + __ffsll((unsigned long long)g1) - 1 : m);
    idx = first;
    const auto below = [](int b) { return b >= 64 ? ~0ull : ((1ull << b) - 1ull); };
    if (first <= 64) return (l0 | ~below(first)) == ~0ull;
    return l0 == ~0ull && (l1 | ~below(first - 64)) == ~0ull;
}

// fp64 tail of tmsample::sample (tensormark/tmsample.h:185-199) for top-k
// rows, one wave, n = K <= 2 * 64 sorted entries in srt.  The top-p cut and
// the drawn index are decided from tree prefix sums within a proven error
// margin of the reference's sequential ones; a decision inside the margin
// (and any call that returns the per-entry probabilities) takes the
// sequential path, tail_topk_exact.
__device__ void tail_topk(const KArgs& a, int row, const tms_row_params& P, const uint64_t* srt,
                          int n, int K, double* pr, double* q, uint32_t w0, uint32_t w1) {
    if (a.topk_cap && a.out_topk_probs) {
        tail_topk_exact(a, row, P, srt, n, K, pr, q, w0, w1);
        return;
    }
    const int lane = threadIdx.x & 63;
    const double u = canonical(w0, w1);
    const double mx = (double)ckey_val(srt[0]);
    const bool h0 = lane < n, h1 = lane + 64 < n;
    const double pr0 = h0 ? exp((double)ckey_val(srt[lane]) - mx) : 0.0;
    const double pr1 = h1 ? exp((double)ckey_val(srt[lane + 64]) - mx) : 0.0;
    const double s0 = wave_incl_scan_f64(pr0);
    const double s1 = wave_incl_scan_f64(pr1) + readlane_f64(s0, 63);
    const double z = readlane_f64(s1, 63);
    // cum = prefix of q = pr / z: from the prefixes of pr (decide_first_ge
    // bounds the difference from the reference's sums of quotients)
    const double rz = 1.0 / z;
    const double c0 = s0 * rz, c1 = s1 * rz;
    int fi;
    bool ok = decide_first_ge(c0, c1, (double)P.top_p, n, fi);
    int kp = fi < n ? fi + 1 : K;
    if (P.min_p > 0.0f) {
        const double mp = (double)P.min_p;
        const uint64_t b0 = __ballot(lane >= 1 && h0 && pr0 < mp);
        const uint64_t b1 = __ballot(h1 && pr1 < mp);
        const int m = b0 ? __ffsll((unsigned long long)b0) - 1
                         : (b1 ? 64 + __ffsll((unsigned long long)b1) - 1 : K);
        if (m < kp) kp = m;
    }
    const int keep = kp;
    int tokidx = 0;
    if (ok && keep >= 2) {
        const int e = keep - 1;   // the sum runs over entries 0 .. keep - 1
        const double sum = e < 64 ? readlane_f64(s0, e) : readlane_f64(s1, e - 64);
        // cp = prefix of p = pr / sum, likewise from the prefixes of pr
        const double rs = 1.0 / sum;
        ok = decide_first_ge(s0 * rs, s1 * rs, u, keep - 1, tokidx);
    }
    if (!ok) {
        TMS_TV(16, 1);
        tail_topk_exact(a, row, P, srt, n, K, pr, q, w0, w1);
        return;
    }
    if (lane == 0) {
        a.out_tokens[row] = (int)ckey_id(srt[tokidx]);
        a.out_status[row] = TMS_ROW_OK;
        if (a.out_keep) a.out_keep[row] = keep;
    }
    if (a.topk_cap && a.out_topk_ids)
        for (int i = lane; i < a.topk_cap; i += 64)
            a.out_topk_ids[(int64_t)row * a.topk_cap + i] = i < n ? (int)ckey_id(srt[i]) : -1;
}

// The same tail for top-p rows (n = min(K, significant entries) <= kToppCap
// entries in LDS), one wave reading the entries from LDS in order.  Returns
// true, having written nothing, when the answer needs the order past the
// held entries (the draw or a min-p threshold of at most e^-40 reaching past
// them, or more top-k ids asked for than are held): the caller then runs
// the whole-row path.
__device__ bool tail_topp(const KArgs& a, int row, const tms_row_params& P, const uint64_t* srt,
                          int n, int K, double* pr, double* q) {
    const int lane = threadIdx.x & 63;
    if (n < K && a.topk_cap > n && (a.out_topk_ids || a.out_topk_probs)) return true;
    double z = 0;
#pragma unroll 8
    for (int i = 0; i < n; ++i) z += pr[i];
    for (int i = lane; i < n; i += 64) q[i] = pr[i] / z;
    wave_lds_sync();
    int kp = K;
    {
        double cum = 0;
        const double tp = (double)P.top_p;
        for (int i = 0; i < n; ++i) {
            cum += q[i];
            if (cum >= tp) {
                kp = i + 1;
                break;
            }
        }
    }
    if (P.min_p > 0.0f) {
        const double mp = (double)P.min_p;
        int m = 1;
        while (m < kp && m < n && pr[m] >= mp) ++m;
        // Past the held entries pr <= e^-40 (4.2484e-18): below a larger
        // min_p; a smaller one needs the entries themselves.
        if (m == n && m < kp && !(mp > 4.3e-18)) return true;
        kp = m;
    }
    const int keep = kp;
    const int lim = keep < n ? keep : n;
    int tokidx = 0;
    if (keep >= 2) {
        double sum = 0;
#pragma unroll 8
        for (int i = 0; i < lim; ++i) sum += pr[i];
        wave_lds_sync();
        for (int i = lane; i < lim; i += 64) q[i] = pr[i] / sum;
        wave_lds_sync();
        uint32_t w0, w1;
        row_uniform(a, row, P, w0, w1);
        const double u = canonical(w0, w1);
        double cp = 0;
        tokidx = keep - 1;
        for (int i = 0; i < lim; ++i) {
            cp = i == 0 ? q[i] : cp + q[i];
            const double cc = (i == keep - 1) ? 1.0 : cp;
            if (!(cc < u)) {
                tokidx = i;
                break;
            }
        }
    }
    // tokidx >= n: the draw fell past the last entry that moves the sums; the
    // reference returns its entry at that rank, which this row does not hold.
    if (tokidx >= n) return true;
    if (lane == 0) {
        a.out_tokens[row] = (int)ckey_id(srt[tokidx]);
        a.out_status[row] = TMS_ROW_OK;
        if (a.out_keep) a.out_keep[row] = keep;
    }
    int32_t* ids = a.out_topk_ids ? a.out_topk_ids + (int64_t)row * a.topk_cap : nullptr;
    float* probs = a.out_topk_probs ? a.out_topk_probs + (int64_t)row * a.topk_cap : nullptr;
    for (int i = lane; i < a.topk_cap; i += 64) {
        const bool have = i < n;
        if (ids) ids[i] = have ? (int)ckey_id(srt[i]) : -1;
        if (probs) probs[i] = have ? (float)(pr[i] / z) : 0.0f;
    }
    return false;
}

// Minimum of non-negative ints across the wave (DPP steps towards lane 63;
// lanes without a source see INT_MAX).
__device__ __forceinline__ int wave_min_nonneg(int v) {
    constexpr uint32_t kBig = 0x7FFFFFFFu;
    uint32_t u = (uint32_t)v;
    u = min(u, dpp_u32<0x111, 0xF, false>(kBig, u));
    u = min(u, dpp_u32<0x112, 0xF, false>(kBig, u));
    u = min(u, dpp_u32<0x114, 0xF, false>(kBig, u));
    u = min(u, dpp_u32<0x118, 0xF, false>(kBig, u));
    u = min(u, dpp_u32<0x142, 0xA, false>(kBig, u));
    u = min(u, dpp_u32<0x143, 0xC, false>(kBig, u));
    return __builtin_amdgcn_readlane((int)u, 63);
}

}  // namespace tms

// Launches the wide top-k kernel (tms_wide.hip) over `batch` rows.
int tms_launch_wide(const tms::KArgs& k, int dtype, bool fast, int batch, int slots, hipStream_t stream);
// Launches the row-stream kernel (tms_rows.hip), one workgroup a row.
int tms_launch_rows(const tms::KArgs& k, int dtype, int batch, hipStream_t stream);
// Launches the sparse-mask kernel (tms_sparse.hip), one workgroup a row.
int tms_launch_sparse(const tms::KArgs& k, int dtype, int batch, hipStream_t stream);
int tms_launch_history(const tms::KArgs& k, const tms_history_params* hp, const uint8_t* breaker,
                       const float* dry_scale, int64_t dry_scale_stride, int dtype, int batch,
                       int32_t* ov_n, int32_t* ov_ids, float* ov_vals, hipStream_t stream);

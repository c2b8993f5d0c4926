// tms_topk.hip -- the sampler kernel for batches whose rows are all greedy or
// top-k with k <= 128 (the host picks it from the caller's row-kind hint).
//
// One launch per call.  Row b is cut into S chunks of at most 16K ids and
// workgroup (b, c) streams its chunk once (nontemporal 16-byte loads, 64
// values per thread).  A chunk selects nothing: each thread keeps its three
// largest entries (with ids) and its fourth value, and the chunk publishes
// the keys, its history-penalised entries and the largest fourth value the
// moment its stream is in.  The last workgroup of the row to take a ticket
// merges: it bounds the row's K-th value from below by the 256 "group
// maxima" (group j = thread j of every chunk), gathers every published key
// above the bound, ranks them and runs the fp64 tail of tmsample::sample
// (tensormark/tmsample.h:184-199).  Every entry >= the bound is one of a
// thread's three entries or a penalised window entry, unless the chunk's
// largest fourth value reaches the bound: such a chunk (very rare) is read
// again.
//
//   pass 1     mask (bit extract + select; history ids masked out, counted
//              while the stream is in flight), running top three values
//              with ids and the fourth value, per thread.
//   penalties  the thread that counted a window id first loaded its logit
//              with the stream; it forms the compounding penalty
//              (tmsample.h:58-61, then frequency/presence) and publishes the
//              entry.
//   publish    header, 3 x 256 keys, penalised entries: every word non-zero
//              (keys never are); the merger reads each word before zeroing
//              it, so a word still in flight reads 0 and is read again, and
//              no store waits.
//   merge      bound (bisection on order keys), gather from registers, rank
//              by counting, tail on wave 0.
// A row that is not greedy and not top-k <= 128 breaks the hint: it goes to
// the whole-row pass (tms_dense.hip) when the call runs one, else it reports
// TMS_ROW_UNSUPPORTED.

#include "tms_sample_common.h"

namespace tms {

constexpr int kLeanMaxChunks = kLeanMaxChunksHost;   // vocab <= 262,144
constexpr int kPendRead = 64;                        // penalised entries per chunk in the first read
constexpr int kWordKeys = 1;                         // list words: [0] header, [1, 769) keys (key j
constexpr int kWordPend = kWordKeys + 3 * kBlock;    // of thread t at 1 + j * 256 + t), [769,
                                                     // kTopkListStride) penalised entries
constexpr int kPendCap = kTopkListStride - kWordPend;
constexpr int kLate = 1024;                          // window ids past the preloaded positions
static_assert(kPendCap > kPendRead, "list layout");
static_assert(8 * kPendRead % kBlock == 0, "pending-entry read layout");
static_assert(4 * kTopkFast >= kBlock, "gather junk slots");

// Header word: ready bit, flags (bits 56-62), penalised entries (bits
// 32-47), order key of the chunk's largest fourth value (bits 0-31).
__device__ __forceinline__ uint64_t lean_header(int flags, int npen, uint32_t t4key) {
    return kReady | ((uint64_t)(flags & 0x7F) << 56) | ((uint64_t)(npen & 0xFFFF) << 32) | t4key;
}
__device__ __forceinline__ int hdr_npen(uint64_t h) { return (int)((h >> 32) & 0xFFFF); }
__device__ __forceinline__ int hdr_flags(uint64_t h) { return (int)((h >> 56) & 0x7F); }

// Read in place of the caller's draws when there are none (never written).
__device__ uint64_t kDeadWord = 1;

struct LeanSmem {
    union {
        uint32_t cnt[kChunk / 2];   // window counts (16 bits per id), chunk phase
        struct {
            uint64_t keys[kCand + 8];   // candidate keys
            uint64_t srt[kCand + 8];    // the sorted top-K
            double pr[4 * kTopkFast];   // fp64 tail scratch
        } m;
        uint32_t wbits[kChunk / 32];    // a re-read chunk's window ids (merge)
    } big;
    uint64_t cand[kCand + 8];       // merge candidates (raw value bits, id)
    uint64_t pend[kPendCap];        // this chunk's penalised window entries (keys)
    uint32_t mw[kWaves * 128];      // per wave: the mask words of its slots
    uint32_t gkey[kBlock];          // merge: group maxima order keys
    int late[kLate];                // window ids past the preloaded positions
    alignas(16) uint64_t hdr[kLeanMaxChunks];   // merge: the chunks' headers (1 past S)
    int wave_i[kWaves];
    uint32_t wave_u[kWaves];
    alignas(16) int hist[256];
    alignas(16) int hist2[256];
    int ncand;
    int npen, nlate;
    int misc[8];
#ifdef TMS_TRACE
    uint64_t trs[kWaves * 24];   // trace stamps, written out at exit
#endif
};

#ifdef TMS_TRACE
// Trace builds of this kernel stamp into LDS and write the stamps out when
// the workgroup exits, so no trace store is outstanding at a vmcnt wait.
#undef TMS_TR
#undef TMS_TV
#define TMS_TR(i)                                                                   \
    do {                                                                            \
        asm volatile("; trace point " #i);                                          \
        if ((threadIdx.x & 63) == 0) sm.trs[(threadIdx.x >> 6) * 24 + (i)] = __builtin_amdgcn_s_memrealtime(); \
    } while (0)
#define TMS_TV(i, val)                                                              \
    do {                                                                            \
        if ((threadIdx.x & 63) == 0) sm.trs[(threadIdx.x >> 6) * 24 + (i)] = (uint64_t)(val); \
    } while (0)
#define TK_TRACE_INIT()                                                             \
    do {                                                                            \
        if ((threadIdx.x & 63) < 24) sm.trs[(threadIdx.x >> 6) * 24 + (threadIdx.x & 63)] = 0; \
    } while (0)
#define TK_TRACE_FLUSH()                                                            \
    do {                                                                            \
        if ((threadIdx.x & 63) < 24 && a.trace)                                     \
            a.trace[(blockIdx.x * 4 + (threadIdx.x >> 6)) * 24 + (threadIdx.x & 63)] = \
                sm.trs[(threadIdx.x >> 6) * 24 + (threadIdx.x & 63)];               \
    } while (0)
#else
#define TK_TRACE_INIT() ((void)0)
#define TK_TRACE_FLUSH() ((void)0)
#endif

// Maximum over the 64 lanes of a wave of u32 values (DPP steps towards lane 63).
__device__ __forceinline__ uint32_t wave_max_u32_dpp(uint32_t v) {
    v = max(v, dpp_u32<0x111, 0xF, true>(0u, v));
    v = max(v, dpp_u32<0x112, 0xF, true>(0u, v));
    v = max(v, dpp_u32<0x114, 0xF, true>(0u, v));
    v = max(v, dpp_u32<0x118, 0xF, true>(0u, v));
    v = max(v, dpp_u32<0x142, 0xA, false>(0u, v));
    v = max(v, dpp_u32<0x143, 0xC, false>(0u, v));
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// 16-byte nontemporal load: the logits are read exactly once per call.
template <typename T>
__device__ __forceinline__ uint4 ld_stream(const T* p) {
    typedef unsigned u4v __attribute__((ext_vector_type(4)));
    const u4v q = __builtin_nontemporal_load((const u4v*)p);
    return make_uint4(q.x, q.y, q.z, q.w);
}

// Rank-sort the distinct keys keys[0..n) (n <= kCand; keys has room for 8
// more) descending into out[0..min(n, lim)): a key's rank is the number of
// larger keys, counted with 16-byte broadcast reads of the list zero-padded
// to a multiple of 8.
__device__ __forceinline__ void rank_sort(uint64_t* keys, int n, uint64_t* out, int lim) {
    const int t = threadIdx.x;
    if (t < 8) keys[n + t] = 0ull;
    lds_sync();
    const uint4* k4 = (const uint4*)keys;
    for (int i = t; i < n; i += kBlock) {
        const uint64_t k = keys[i];
        int r0 = 0, r1 = 0;
        for (int j = 0; j < n; j += 8) {
            uint4 q[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) q[u] = k4[(j >> 1) + u];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                r0 += (((uint64_t)q[u].y << 32) | q[u].x) > k ? 1 : 0;
                r1 += (((uint64_t)q[u].w << 32) | q[u].z) > k ? 1 : 0;
            }
        }
        if (r0 + r1 < lim) out[r0 + r1] = k;
    }
    lds_sync();
}

// Id of entry q (slot q / vec, element q % vec) of thread j of the chunk at e0.
template <int VEC>
__device__ __forceinline__ uint32_t id_of(int j, int q, int e0) {
    return (uint32_t)(e0 + (j + (q / VEC) * kBlock) * VEC + q % VEC);
}

// Appends `key` where `take` holds to sm.cand after the first base0 entries
// (one ballot and one LDS atomic per wave, counted in sm.ncand); past kCand
// the count still grows and nothing is stored.
template <typename SM>
__device__ __forceinline__ void append_cand(SM& sm, bool take, uint64_t key, int base0) {
    const uint64_t m = __ballot(take);
    if (!m) return;
    int wb = 0;
    if ((threadIdx.x & 63) == 0) wb = atomicAdd(&sm.ncand, __popcll(m));
    wb = __builtin_amdgcn_readfirstlane(wb);
    const int pos = base0 + wb + __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                                   __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
    if (take && pos < kCand) sm.cand[pos] = key;
}

// The key value of id in a row (the logit divided by the temperature when
// `divide`): a window entry's penalised value as published (in `pend`, np
// entries, already divided), else the logit masked.
template <typename T>
__device__ __forceinline__ float row_value(const T* base, const uint32_t* mrow, const uint64_t* pend,
                                           int np, int id, float temp, bool divide) {
    for (int i = 0; i < np; ++i)
        if ((int)ckey_id(pend[i]) == id) return ckey_val(pend[i]);
    if (!((mrow[id >> 5] >> (id & 31)) & 1u)) return -__builtin_huge_valf();
    const float x = Elt<T>::scalar(base + id);
    return divide ? x / temp : x;
}

// The exact top-K of a whole row by (lg desc, id asc), for rows the bound
// cannot narrow (massive ties, or more penalised entries than a list holds):
// a radix select over the keys of lg = v / T, 8 bits a pass, with the row
// read again from memory (row_value).  `pend` holds every penalised entry of
// the row (np of them, read from the lists).  Writes sm.cand as ckey(lg,
// id), unsorted; returns the count (<= K).
template <typename T, typename SM>
__device__ __noinline__ int lean_row_radix(const T* base, const uint32_t* mrow, const uint64_t* pend,
                                           int np, int V, int K, float temp, bool divide, SM& sm) {
    const int t = threadIdx.x;
    const float NEG_INF = -__builtin_huge_valf();
    auto lkey = [](float v) { return okey(v); };
    uint32_t prefix = 0, pmask = 0;
    int remaining = K;
    for (int shift = 24; shift >= 0; shift -= 8) {
        sm.hist[t] = 0;
        if (t == 0) sm.ncand = 0;
        lds_sync();
        for (int id = t; id < V; id += kBlock) {
            const float v = row_value(base, mrow, pend, np, id, temp, divide);
            if (v == NEG_INF) continue;
            const uint32_t k = lkey(v);
            if ((k & pmask) == prefix) atomicAdd(&sm.hist[(k >> shift) & 0xFF], 1);
        }
        lds_sync();
        const int h = sm.hist[255 - t];   // thread t holds digit 255 - t
        int total;
        const int above = block_excl_scan(h, total, sm);
        if (shift == 24 && total <= K) {
            // At most K finite entries: all of them.
            for (int id = t; id < V; id += kBlock) {
                const float v = row_value(base, mrow, pend, np, id, temp, divide);
                if (v == NEG_INF) continue;
                const int pos = atomicAdd(&sm.ncand, 1);
                sm.cand[pos] = ckey(v, (uint32_t)id);
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
    for (int id = t; id < V; id += kBlock) {
        const float v = row_value(base, mrow, pend, np, id, temp, divide);
        if (v == NEG_INF) continue;
        if (lkey(v) > prefix) {
            const int pos = atomicAdd(&sm.ncand, 1);
            sm.cand[pos] = ckey(v, (uint32_t)id);
        }
    }
    lds_sync();
    const int g = sm.ncand;
    // Ties in id order, kBlock consecutive ids per step.
    int taken = 0;
    for (int b0 = 0; b0 < V && taken < remaining; b0 += kBlock) {
        const int id = b0 + t;
        float v = NEG_INF;
        int tie = 0;
        if (id < V) {
            v = row_value(base, mrow, pend, np, id, temp, divide);
            tie = v != NEG_INF && lkey(v) == prefix;
        }
        int tot;
        const int p = block_excl_scan(tie, tot, sm);
        if (tie && taken + p < remaining)
            sm.cand[g + taken + p] = ckey(v, (uint32_t)id);
        taken += tot;
    }
    lds_sync();
    return g + (taken < remaining ? taken : remaining);
}

// Wave 0: the digit d of the K-th largest count in the 256-bin histogram
// h (K >= 1, at least K counted) and the count in the bins above d, into
// sm.misc[4] and sm.misc[5].  Lane l sums bins 255-4l .. 252-4l; the lane
// whose running sum crosses K finds the bin.
template <typename SM>
__device__ __forceinline__ void pick_digit(const int* h, int K, SM& sm) {
    const int l = threadIdx.x & 63;
    const int4 q = ((const int4*)h)[63 - l];   // bins 252-4l .. 255-4l
    const int c[4] = {q.w, q.z, q.y, q.x};     // descending bin order
    const int s = c[0] + c[1] + c[2] + c[3];
    const int incl = wave_incl_scan_i32(s);
    int cum = incl - s;
    if (cum < K && incl >= K) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (cum + c[j] >= K) {
                sm.misc[4] = 255 - 4 * l - j;
                sm.misc[5] = cum;
                break;
            }
            cum += c[j];
        }
    }
}

// A chunk read again by the merger (its largest fourth value reaches the
// bound kb): the whole chunk [ce0, ce1) in one round of loads (pass 1's
// layout), every entry whose key (lg) is >= kb and that is not a window id
// of the chunk (bitmap
// sm.big.wbits, chunk-relative) appended to sm.cand after the first base0
// entries (one LDS atomic per wave on sm.ncand).
template <typename T, bool FAST>
__device__ __noinline__ void reread_chunk(const T* base, const uint32_t* mrow, int ce0, int ce1, uint32_t kb,
                                          float temp, bool divide, int base0, LeanSmem& sm) {
    constexpr int VEC = Elt<T>::kVec;
    constexpr int NVT = kEpt / VEC;
    const int t = threadIdx.x, lane = t & 63;
    const int cnv = (ce1 - ce0 + VEC - 1) / VEC;
    float f[kEpt];
    uint32_t mk[NVT];
#pragma unroll
    for (int j = 0; j < NVT; ++j) {
        const int v = min(t + j * kBlock, cnv - 1);
        const int eb = ce0 + v * VEC;
        mk[j] = mrow[eb >> 5];
        if constexpr (FAST) {
            const uint4 q = *(const uint4*)(base + eb);
            float g[VEC];
            Elt<T>::widen(q, g);
#pragma unroll
            for (int e = 0; e < VEC; ++e) f[j * VEC + e] = g[e];
        } else {
#pragma unroll
            for (int e = 0; e < VEC; ++e) f[j * VEC + e] = Elt<T>::scalar(base + min(eb + e, ce1 - 1));
        }
    }
    if (divide) {
#pragma unroll
        for (int q = 0; q < kEpt; ++q) f[q] = f[q] / temp;
    }
    uint64_t take = 0;   // bit q: entry q of this thread
#pragma unroll
    for (int j = 0; j < NVT; ++j) {
        const int v = t + j * kBlock;
        const int eb = ce0 + v * VEC;
        const uint32_t wb = v < cnv ? sm.big.wbits[(eb - ce0) >> 5] : 0u;
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
            const int id = eb + e;
            const bool ok = v < cnv && id < ce1 && ((mk[j] >> (id & 31)) & 1u) && !((wb >> (id & 31)) & 1u) &&
                            okey(f[j * VEC + e]) >= kb;
            take |= (uint64_t)ok << (j * VEC + e);
        }
    }
    const int m = __popcll(take);
    const int inc = wave_incl_scan_i32(m);
    int wb0 = 0;
    if (lane == 63 && inc) wb0 = atomicAdd(&sm.ncand, inc);
    int q = base0 + __builtin_amdgcn_readlane(wb0, 63) + inc - m;
#pragma unroll
    for (int b = 0; b < kEpt; ++b) {
        if ((take >> b) & 1u) {
            const int id = ce0 + (t + (b / VEC) * kBlock) * VEC + b % VEC;
            if (q < kCand) sm.cand[q] = ckey(f[b], (uint32_t)id);
            ++q;
        }
    }
}

// MS: the merge's chunk slots, 8 or 16 (>= S).
template <typename T, bool FAST, int MS>
__global__ __launch_bounds__(kBlock, 2) void topk_kernel(KArgs a) {
    static_assert(MS == 8 || MS == 16, "merge slots");
    constexpr int VEC = Elt<T>::kVec;
    constexpr int NVT = kEpt / VEC;
    constexpr int kWin = 4;   // history ids loaded per thread with the stream
    __shared__ LeanSmem sm;
    const float NEG_INF = -__builtin_huge_valf();
    const int t = threadIdx.x;
    const int lane = t & 63, wv = t >> 6;
    const int S = a.S;
    int row, c;
    wg_row_chunk(S, row, c);
    const int V = a.V;
    const int e0 = c * a.CE;   // a multiple of 32: the chunk starts on a mask word
    const int e1 = min(e0 + a.CE, V);
    const int nvec = (e1 - e0 + VEC - 1) / VEC;
    TK_TRACE_INIT();
    TMS_TR(0);

    // ---- loads in the order they are needed: history window, row
    //      parameters, this wave's mask words, then the stream, then the
    //      logits of the window ids in this chunk (their owners' loads).
    const int32_t* hist = a.recent + (int64_t)row * a.recent_stride;
    int wid[kWin];
    if (a.recent) {
        const int rs = (int)a.recent_stride;
#pragma unroll
        for (int i = 0; i < kWin; ++i) wid[i] = hist[min(t + i * kBlock, rs - 1)];
    }
    const tms_row_params P = a.params[row];
    // the caller's draw for the row, if given, loaded now (no branch: a
    // dummy word otherwise) so the merge never waits for it
    const uint32_t* dp = a.draws ? a.draws + 2 * row : (const uint32_t*)&kDeadWord;
    const uint32_t dw0 = dp[0], dw1 = dp[1];
    int nrec = 0;
    if (a.recent) {
        nrec = a.n_recent ? a.n_recent[row] : (int)a.recent_stride;
        nrec = min(max(nrec, 0), (int)a.recent_stride);
    }
    // Slot j of thread t covers ids e0 + (t + j * kBlock) * VEC ..: its mask
    // word is (t + j * kBlock) * VEC / 32.  A wave's 64 threads over NVT
    // slots need kWaveWords words, kWpS per slot; lane l loads two of them.
    constexpr int kWpS = 64 * VEC / 32;            // words per wave slot
    constexpr int kWaveWords = kWpS * NVT;         // 128 for either width
    const uint32_t* mrow = a.mask + (int64_t)row * a.mask_stride;
    const int nwords = (e1 - e0 + 31) >> 5;
    uint32_t mwd[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int k = 2 * lane + u;                // this wave's word k: slot k / kWpS
        const int w = (k / kWpS) * (kBlock * VEC / 32) + wv * kWpS + k % kWpS;
        mwd[u] = mrow[(e0 >> 5) + min(w, nwords - 1)];
    }
    __builtin_amdgcn_sched_barrier(0);
    const T* base = (const T*)a.logits + (int64_t)row * a.row_stride;
    // 16-byte slots: the first kLook now, slot j + kLook once slot j is
    // worked (the queue of a CU's loads is full while the row streams, so a
    // wave that issued everything first would wait there and then work
    // every slot after the data is in).
#ifdef TMS_TOPK_LOOK
    constexpr int kLook = TMS_TOPK_LOOK < NVT ? TMS_TOPK_LOOK : NVT;
#else
    constexpr int kLook = NVT < 4 ? NVT : 4;
#endif
    uint4 raw[NVT];
    float sx[FAST ? 1 : kEpt];
    auto issue = [&](int j) {
        const int v = min(t + j * kBlock, nvec - 1);
        raw[j] = ld_stream(base + e0 + v * VEC);
    };
#pragma unroll
    for (int j = 0; j < NVT; ++j) {
        const int v = min(t + j * kBlock, nvec - 1);
        const int eb = e0 + v * VEC;
        if constexpr (FAST) {
            if (j < kLook) issue(j);
        } else {
#pragma unroll
            for (int e = 0; e < VEC; ++e) sx[j * VEC + e] = Elt<T>::scalar(base + min(eb + e, V - 1));
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    float own_v[kWin];
    uint32_t own_m[kWin];
#pragma unroll
    for (int i = 0; i < kWin; ++i) {
        const int id = a.recent ? wid[i] : -1;
        const bool in = id >= e0 && id < e1;
        own_v[i] = in ? Elt<T>::scalar(base + id) : 0.0f;
        own_m[i] = in ? mrow[id >> 5] : 0u;
    }
    TMS_TR(1);

    Pen pn;
    pn.rep_on = !(P.repeat_penalty <= 1.0f);
    pn.fp_on = P.frequency_penalty != 0.0f || P.presence_penalty != 0.0f;
    pn.on = nrec > 0 && P.repeat_last_n > 0 && (pn.rep_on || pn.fp_on);
    pn.rep = P.repeat_penalty;
    pn.freq = P.frequency_penalty;
    pn.pres = P.presence_penalty;
    const int from = pn.on ? (nrec > P.repeat_last_n ? nrec - P.repeat_last_n : 0) : 0;

    // ---- while the stream is in flight: this wave's mask words into its
    //      LDS words, and the window count table cleared.
    uint32_t* mw = sm.mw + wv * kWaveWords;
    mw[2 * lane] = mwd[0];
    mw[2 * lane + 1] = mwd[1];
    if (pn.on) {
        uint4* c4 = (uint4*)sm.big.cnt;
        for (int i = t; i < kChunk / 8; i += kBlock) c4[i] = make_uint4(0, 0, 0, 0);
    }
    if (t == 0) {
        sm.npen = 0;
        sm.nlate = 0;
    }
    if (pn.on) lds_sync();
    else wave_lds_sync();
    TMS_TR(2);

    // ---- pass 1, as each slot lands: widen and mask (mask bit -> value,
    //      else -inf), with the thread's running top
    //      three values and their slot indices and its fourth value.  Ids grow
    //      with the index, so a strict > keeps the lowest id.  t1 propagates
    //      NaN (IEEE maximum): a NaN or +inf anywhere in the chunk shows in
    //      t1.
    float t1 = NEG_INF, t2 = NEG_INF, t3 = NEG_INF, t4 = NEG_INF;
    int i1 = 0, i2 = 0, i3 = 0;
    // The window's first kWin * kBlock positions are counted while the
    // stream lands (after slot 1: the ids were loaded first), each count's
    // old value kept for after pass 1 (the barrier that follows pass 1 makes
    // every count final before it is read).
    // The ticket is taken with the last kLook slots of the stream still to
    // come: its round trip overlaps them, the window and the publish, and
    // the last of the row to get there merges.  A chunk with an earlier
    // ticket may still be publishing when the merger reads; the merger reads
    // such words again.
    uint32_t ticket = 0;
    bool win_in[kWin];
    uint32_t win_old[kWin];
#pragma unroll
    for (int i = 0; i < kWin; ++i) {
        win_in[i] = false;
        win_old[i] = 1u;
    }
#pragma unroll
    for (int j = 0; j < NVT; ++j) {
        if constexpr (FAST) {
            if (j + kLook < NVT) issue(j + kLook);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (j == NVT - kLook && t == 0)
            ticket = __hip_atomic_fetch_add(&a.counters[row * kCounterStride], 1u, __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_AGENT);
        if (j == 1 && pn.on) {
#pragma unroll
            for (int i = 0; i < kWin; ++i) {
                const int p = t + i * kBlock;
                const int id = (p < from || p >= nrec) ? -1 : wid[i];
                win_in[i] = id >= e0 && id < e1;
                if (win_in[i]) {
                    const int off = id - e0;
                    const uint32_t sh = (off & 1) * 16;
                    win_old[i] = (atomicAdd(&sm.big.cnt[off >> 1], 1u << sh) >> sh) & 0xFFFFu;
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        const int v = t + j * kBlock;
        float f[VEC];
        if constexpr (FAST) {
            Elt<T>::widen(raw[j], f);
        } else {
#pragma unroll
            for (int e = 0; e < VEC; ++e) f[e] = sx[j * VEC + e];
        }
        // this lane's word of slot j: (lane * VEC / 32) within the slot's run
        uint32_t mb = v < nvec ? mw[j * kWpS + ((lane * VEC) >> 5)] >> ((v * VEC) & 31) : 0u;
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
            const uint32_t sel = (uint32_t)__builtin_amdgcn_sbfe((int)mb, e, 1);
            uint32_t bits = (__float_as_uint(f[e]) & sel) | (0xFF800000u & ~sel);
            if constexpr (!FAST) bits = (e0 + v * VEC + e < e1) ? bits : 0xFF800000u;
            const float g = __uint_as_float(bits);
            const int q = j * VEC + e;
            const bool c1 = g > t1, c2 = g > t2, c3 = g > t3;
            i3 = c2 ? i2 : (c3 ? q : i3);
            i2 = c1 ? i1 : (c2 ? q : i2);
            i1 = c1 ? q : i1;
            // t(k+1) <= t(k): the median of the two and g is the new t(k+1)
            t4 = __builtin_amdgcn_fmed3f(t3, t4, g);
            t3 = __builtin_amdgcn_fmed3f(t2, t3, g);
            t2 = __builtin_amdgcn_fmed3f(t1, t2, g);
            t1 = __builtin_elementwise_maximum(t1, g);
        }
        // The running state is complete after each slot, so none of this
        // slot's work is deferred past the next slot's wait.
        asm volatile("" : "+v"(t1), "+v"(t2), "+v"(t3), "+v"(t4), "+v"(i1), "+v"(i2), "+v"(i3));
        __builtin_amdgcn_sched_barrier(0);
    }
    TMS_TR(3);
#ifdef TMS_PROBE_PASS1ONLY
    // Measurement builds stop here, to time the stream and pass 1 alone.
    if (t1 == 12345.0f && t2 == 1.0f && i1 == 7 && t3 == 2.0f && i2 == 3 && t4 == 0.5f && i3 == 1)
        a.out_tokens[row] = 0;
    return;
#endif


    // ---- the history window: each window id in this chunk is counted (16
    //      bits per id) and the position that counted it first owns it (the
    //      first kWin * kBlock positions were counted during pass 1).  Pass
    //      1 saw window ids with their raw logits; a thread leaves them out
    //      of what it publishes (every entry it does not publish stays <= its
    //      fourth value, so the bound test is unchanged).
    bool first[kWin];
#pragma unroll
    for (int i = 0; i < kWin; ++i) first[i] = win_in[i] && win_old[i] == 0u;
    if (pn.on) {
        for (int p0 = kWin * kBlock; p0 < nrec; p0 += kWin * kBlock) {   // long windows
#pragma unroll
            for (int i = 0; i < kWin; ++i) {
                const int p = p0 + t + i * kBlock;
                const int id = (p < from || p >= nrec) ? -1 : hist[p];
                if (id >= e0 && id < e1) {
                    const int off = id - e0;
                    const uint32_t sh = (off & 1) * 16;
                    const uint32_t old = atomicAdd(&sm.big.cnt[off >> 1], 1u << sh);
                    if (((old >> sh) & 0xFFFFu) == 0) {   // its logit is loaded late
                        const int k = atomicAdd(&sm.nlate, 1);
                        if (k < kLate) sm.late[k] = id;
                    }
                }
            }
        }
        lds_sync();
    }
    TMS_TR(19);

    // Published keys are of lg = value / temperature (the quotient the tail
    // ranks by; for greedy rows and invalid temperatures the value itself).
    const bool cdiv = !P.greedy && P.temperature != 1.0f && P.temperature > 0.0f && P.temperature <= FLT_MAX;
    auto lgof = [&](float x) { return cdiv ? x / P.temperature : x; };

    // ---- penalised window entries, from their owners
    bool my_nf = !(t1 < __builtin_huge_valf());   // +inf or NaN among this thread's entries
    if (pn.on) {
#pragma unroll
        for (int i = 0; i < kWin; ++i) {
            if (first[i]) {
                const int id = wid[i];
                const int off = id - e0;
                const uint32_t cnt = (sm.big.cnt[off >> 1] >> ((off & 1) * 16)) & 0xFFFFu;
                float g = ((own_m[i] >> (id & 31)) & 1u) ? own_v[i] : NEG_INF;
                g = apply_pen(g, cnt, pn);
                my_nf |= !(g < __builtin_huge_valf()) && g != NEG_INF;   // NaN or +inf
                const int k = atomicAdd(&sm.npen, 1);
                if (k < kPendCap) sm.pend[k] = ckey(lgof(g), (uint32_t)id);
            }
        }
        const int nlate = min(sm.nlate, kLate);
        for (int k0 = 0; k0 < nlate; k0 += kBlock) {   // long windows only
            const int k = k0 + t;
            if (k < nlate) {
                const int id = sm.late[k];
                const int off = id - e0;
                const uint32_t cnt = (sm.big.cnt[off >> 1] >> ((off & 1) * 16)) & 0xFFFFu;
                float g = ((mrow[id >> 5] >> (id & 31)) & 1u) ? Elt<T>::scalar(base + id) : NEG_INF;
                g = apply_pen(g, cnt, pn);
                my_nf |= !(g < __builtin_huge_valf()) && g != NEG_INF;
                const int q = atomicAdd(&sm.npen, 1);
                if (q < kPendCap) sm.pend[q] = ckey(lgof(g), (uint32_t)id);
            }
        }
    }
    TMS_TR(20);
    // per wave: any non-finite entry, and the largest fourth value's key
    const uint32_t t4k = okey(lgof(t4));
    const bool wnf = __any(my_nf);
    const uint32_t wt4 = wave_max_u32_dpp(t4k);
    if (lane == 0) {
        sm.wave_i[wv] = wnf;
        sm.wave_u[wv] = wt4;
    }
    lds_sync();
    TMS_TR(13);
    int flags = (sm.wave_i[0] | sm.wave_i[1] | sm.wave_i[2] | sm.wave_i[3]) ? FLAG_NONFINITE : 0;
    const uint32_t t4max = max(max(sm.wave_u[0], sm.wave_u[1]), max(sm.wave_u[2], sm.wave_u[3]));
    const int npen_all = sm.npen;
    if (npen_all > kPendCap) flags |= FLAG_OVERFLOW;
    const int npen = min(npen_all, kPendCap);
    const uint64_t hdr = lean_header(flags, npen, t4max);

    // ---- publish (no store waits).  Thread t stores its
    //      three keys, thread i % kBlock penalised entry i, thread 0 the
    //      header; the same lanes zero them if this workgroup merges (one
    //      lane stores each word, so its zero lands after it).
    const uint32_t id1 = id_of<VEC>(t, i1, e0), id2 = id_of<VEC>(t, i2, e0), id3 = id_of<VEC>(t, i3, e0);
    auto windowed = [&](uint32_t id) {
        const int off = (int)id - e0;
        return pn.on && ((sm.big.cnt[off >> 1] >> ((off & 1) * 16)) & 0xFFFFu) != 0;
    };
    // a window entry's key is 1: never 0 (data as flag), below every bound
    const uint64_t k1 = windowed(id1) ? 1ull : ckey(lgof(t1), id1);
    const uint64_t k2 = windowed(id2) ? 1ull : ckey(lgof(t2), id2);
    const uint64_t k3 = windowed(id3) ? 1ull : ckey(lgof(t3), id3);
    uint64_t* row_lists = a.tlists + (int64_t)row * S * kTopkListStride;
    uint64_t* my_list = row_lists + (int64_t)c * kTopkListStride;
    st_agent(&my_list[kWordKeys + t], k1);
    st_agent(&my_list[kWordKeys + kBlock + t], k2);
    st_agent(&my_list[kWordKeys + 2 * kBlock + t], k3);
    for (int i = t; i < npen; i += kBlock) st_agent(&my_list[kWordPend + i], sm.pend[i]);
    if (t == 0) {
        st_agent(&my_list[0], hdr);
        sm.misc[0] = ticket == (uint32_t)(S - 1) ? 1 : 0;
    }
    TMS_TR(4);
    lds_sync();
    if (!sm.misc[0]) {
        TK_TRACE_FLUSH();
        return;
    }
    TMS_TR(5);
    TMS_TV(21, __builtin_amdgcn_s_memtime());

    // ================= merge: the last workgroup of the row =================
    // Thread t reads the three keys of thread t of every other chunk and the
    // first kPendRead penalised entries of each chunk (a share of them);
    // threads < S read the headers.  A word still 0 is read again.
    if (t == 64) st_agent(&a.counters[row * kCounterStride], 0u);   // ready for the next launch
    const bool greedy = P.greedy != 0;
    const bool bad_params = !greedy && !(P.temperature > 0.0f && P.temperature <= FLT_MAX);
    const int K = greedy ? 1 : ((P.top_k <= 0 || P.top_k > V) ? V : P.top_k);
    const bool unsupported = K > kTopkFast;   // the caller's hint does not hold for this row
    const float temp = P.temperature;
    const bool divide = !greedy && temp != 1.0f;
    // Every word is loaded without a branch (a load under a condition makes
    // the compiler wait for it where the paths join): slots S..MS-1 read
    // chunk S-1's words again and are left out where the words are used,
    // and this workgroup reads its own list back like the others.  Keys and
    // headers first, then the penalised entries, then the third keys, which
    // the gather is the first to need.
    const uint32_t slots = (1u << S) - 1u;   // S <= 16
    // (tid: the thread index, passed opaque on the rare re-read paths so the
    // compiler recomputes these addresses there rather than keeping them)
    auto key_at = [&](int cc, int j, int tid) -> const uint64_t* {
        return &row_lists[(int64_t)min(cc, S - 1) * kTopkListStride + kWordKeys + j * kBlock + tid];
    };
    auto pend_at = [&](int idx) -> const uint64_t* {
        return &row_lists[(int64_t)min(idx / kPendRead, S - 1) * kTopkListStride + kWordPend + idx % kPendRead];
    };
    auto opaque = [](int v) {
        asm volatile("" : "+v"(v));
        return v;
    };
    const uint64_t* const hdr_at = &row_lists[(int64_t)min(t, S - 1) * kTopkListStride];
    uint64_t kk[2 * MS];
#pragma unroll
    for (int cc = 0; cc < MS; ++cc) {
        kk[2 * cc] = ld_agent(key_at(cc, 0, t));
        kk[2 * cc + 1] = ld_agent(key_at(cc, 1, t));
    }
    uint64_t h = ld_agent(hdr_at);   // this workgroup's own: from hdr below (another lane stored it)
    constexpr int kPendPer = MS * kPendRead / kBlock;
    uint64_t pw[kPendPer];
#pragma unroll
    for (int u = 0; u < kPendPer; ++u) pw[u] = ld_agent(pend_at(t + u * kBlock));
    uint64_t kt[MS];
#pragma unroll
    for (int cc = 0; cc < MS; ++cc) kt[cc] = ld_agent(key_at(cc, 2, t));
    uint32_t w0 = 0, w1 = 0;
    if (wv == 0) {   // the row's uniform, while the reads are in flight
        if (a.draws) {
            w0 = dw0;
            w1 = dw1;
        } else {
            row_words(P.seed, P.offset, 0u, w0, w1);
        }
    }
    // A word still 0 is in flight: the thread reads all of its words again
    // (a non-zero word does not change until this workgroup zeroes it), a
    // bounded number of times; spins reaching kPollCap marks the row lost.
    h = t == c ? hdr : h;
    int spins = 0;
    bool zero = h == 0;
#pragma unroll
    for (int i = 0; i < 2 * MS; ++i) zero |= kk[i] == 0;
    for (; zero && spins < kPollCap; ++spins) {   // rare
        __builtin_amdgcn_s_sleep(1);
        const int tid = opaque(t);
#pragma unroll
        for (int cc = 0; cc < MS; ++cc) {
            kk[2 * cc] = ld_agent(key_at(cc, 0, tid));
            kk[2 * cc + 1] = ld_agent(key_at(cc, 1, tid));
        }
        h = tid == c ? hdr : ld_agent(&row_lists[(int64_t)min(tid, S - 1) * kTopkListStride]);
        zero = h == 0;
#pragma unroll
        for (int i = 0; i < 2 * MS; ++i) zero |= kk[i] == 0;
    }
    if (zero) spins = kPollCap;
    auto settle = [&](uint64_t& v, const uint64_t* p) {   // one word, on the rare paths
        while (v == 0 && spins < kPollCap) {
            __builtin_amdgcn_s_sleep(1);
            v = ld_agent(p);
            ++spins;
        }
    };
    if (t < kLeanMaxChunks) sm.hdr[t] = t < S ? h : 1ull;   // 1: no flags, entries or fourth value
    if (t == 0) {
        sm.misc[3] = 0;   // a key or header word never arrived
        sm.misc[7] = 0;   // a later word never arrived (misc[3] is read for the status)
        sm.ncand = 0;
    }
    // group maxima: the largest first key of thread t over the chunks
    uint32_t gm = 0;
#pragma unroll
    for (int cc = 0; cc < MS; ++cc) gm = max(gm, cc < S ? (uint32_t)(kk[2 * cc] >> 32) : 0u);
    sm.gkey[t] = gm;
    sm.hist[t] = 0;
    sm.hist2[t] = 0;
    lds_sync();
    TMS_TR(6);
    // the penalised entries read with the keys; past kPendRead (rare) below
    bool plive[kPendPer];
#pragma unroll
    for (int u = 0; u < kPendPer; ++u) {
        const int idx = t + u * kBlock;
        const int cc = idx / kPendRead;
        plive[u] = cc < S && cc != c && idx % kPendRead < hdr_npen(sm.hdr[cc]);
    }
    // The third keys and penalised entries, first needed by the gather:
    // waited for there (their loads stay in flight through the bound), and
    // on an error row before the words are zeroed.
    auto late_zero = [&]() {
        bool z = false;
#pragma unroll
        for (int u = 0; u < kPendPer; ++u) z |= plive[u] && pw[u] == 0;
#pragma unroll
        for (int cc = 0; cc < MS; ++cc) z |= kt[cc] == 0;
        return z;
    };
    auto settle_late = [&]() {
        bool z = late_zero();
        for (; z && spins < kPollCap; ++spins) {   // rare: read them all again
            __builtin_amdgcn_s_sleep(1);
            const int tid = opaque(t);
#pragma unroll
            for (int cc = 0; cc < MS; ++cc) kt[cc] = ld_agent(key_at(cc, 2, tid));
#pragma unroll
            for (int u = 0; u < kPendPer; ++u) pw[u] = ld_agent(pend_at(tid + u * kBlock));
            z = late_zero();
        }
        if (z) spins = kPollCap;
        if (spins >= kPollCap) sm.misc[7] = 1;
    };
    if (spins >= kPollCap) sm.misc[3] = 1;
    // the headers (1 past S): flags, largest fourth values, penalised
    // entries past the first read
    int fo = 0;
    uint32_t t4all = 0;
    int pextra = 0;
    {
        const uint4* h4 = (const uint4*)sm.hdr;
#pragma unroll
        for (int i = 0; i < kLeanMaxChunks / 2; ++i) {
            const uint4 q = h4[i];
            const uint64_t hh[2] = {((uint64_t)q.y << 32) | q.x, ((uint64_t)q.w << 32) | q.z};
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                fo |= hdr_flags(hh[e]);
                t4all = max(t4all, (uint32_t)hh[e]);
                pextra += 2 * i + e == c ? 0 : max(hdr_npen(hh[e]) - kPendRead, 0);
            }
        }
    }
    lds_sync();   // misc[3]
    TMS_TR(10);
    int status = TMS_ROW_OK;
    if (sm.misc[3]) status = TMS_ROW_INTERNAL;
    else if (bad_params) status = TMS_ROW_BAD_PARAMS;
    else if (fo & FLAG_NONFINITE) status = TMS_ROW_NONFINITE;
    else if (unsupported) status = TMS_ROW_UNSUPPORTED;   // the whole-row path below

    uint64_t* srt = sm.big.m.srt;
    int n = 0;        // candidates gathered, then the sorted top-K kept
    int N = 0;        // finite entries of the row when fewer than K, else >= K
    bool all_finite = false;
    int ngath = 0;    // keys placed by the gather's scan
    bool late_done = false;   // third keys and penalised entries waited for
    if (status == TMS_ROW_OK) {
        // ---- the bound: the K-th largest of the 256 group maxima (K groups
        //      hold an entry >= it, so it bounds the row's K-th key from
        //      below), on the sixteen high bits of the order keys: two
        //      rounds of an 8-bit histogram in LDS, wave 0 picking the digit.
        atomicAdd(&sm.hist[gm >> 24], 1);
        lds_sync();
        if (wv == 0) pick_digit(sm.hist, K, sm);
        lds_sync();
        const uint32_t d1 = (uint32_t)sm.misc[4];
        const int above1 = sm.misc[5];
        if ((gm >> 24) == d1) atomicAdd(&sm.hist2[(gm >> 16) & 0xFFu], 1);
        lds_sync();
        if (wv == 0) pick_digit(sm.hist2, K - above1, sm);
        lds_sync();
        const uint32_t pre = (d1 << 24) | ((uint32_t)sm.misc[4] << 16);
        TMS_TR(11);
        // Keys below okey(-FLT_MAX) decode to -inf or NaN: every finite entry.
        all_finite = pre < 0x00800000u;
        const bool radix = (fo & FLAG_OVERFLOW) != 0;
        const uint32_t kb = all_finite ? 0x00800000u : pre;
        settle_late();
        late_done = true;
        TMS_TR(9);
        // Chunks whose largest fourth value reaches the bound are read again
        // whole; their published keys are left out.
        uint32_t reread = 0;
        if (t4all >= kb)
            for (int cc = 0; cc < S; ++cc)
                if ((uint32_t)sm.hdr[cc] >= kb) reread |= 1u << cc;
        const uint32_t use = slots & ~reread;   // chunk slots whose keys are gathered
        TMS_TV(14, __popc(reread) + 1);
        // ---- the gather from registers: each thread counts the keys it
        //      takes (its three keys of every chunk not read again, its share
        //      of the first penalised reads, this workgroup's penalised entry
        //      t), one block scan places them, and every key is stored, the
        //      ones not taken to a slot of this thread's own (no branches);
        //      sm.ncand then counts what the rare paths below append.
                auto above = [&](uint64_t k) { return (uint32_t)(k >> 32) >= kb; };
        int mine = 0;
#pragma unroll
        for (int i = 0; i < 2 * MS; ++i) mine += (int)(((use >> (i / 2)) & 1u) && above(kk[i]));
#pragma unroll
        for (int i = 0; i < MS; ++i) mine += (int)(((use >> i) & 1u) && above(kt[i]));
        bool pl[kPendPer];
#pragma unroll
        for (int u = 0; u < kPendPer; ++u) {
            pl[u] = plive[u] && above(pw[u]);
            mine += (int)pl[u];
        }
        const uint64_t op = t < npen ? sm.pend[t] : 0ull;
        const bool ownp = t < npen && above(op);
        mine += (int)ownp;
        int pos = block_excl_scan(mine, ngath, sm);
        uint64_t* const junk = (uint64_t*)sm.big.m.pr + t;   // the tail's scratch, free until then
        auto put = [&](bool take, uint64_t k) {
            *(take && pos < kCand ? &sm.cand[pos] : junk) = k;
            pos += (int)take;
        };
#pragma unroll
        for (int i = 0; i < 2 * MS; ++i) put(((use >> (i / 2)) & 1u) && above(kk[i]), kk[i]);
#pragma unroll
        for (int i = 0; i < MS; ++i) put(((use >> i) & 1u) && above(kt[i]), kt[i]);
#pragma unroll
        for (int u = 0; u < kPendPer; ++u) put(pl[u], pw[u]);
        put(ownp, op);
        TMS_TR(18);
        for (int i0 = kBlock; i0 < npen; i0 += kBlock) {   // this workgroup's own past kBlock
            const int i = i0 + t;
            const uint64_t v = i < npen ? sm.pend[i] : 0ull;
            append_cand(sm, i < npen && above(v), v, ngath);
        }
        if (pextra) {
            // penalised entries past the first read (more than kPendRead
            // window ids in a chunk)
            for (int cc = 0; cc < S; ++cc) {
                if (cc == c) continue;
                const int npc = hdr_npen(sm.hdr[cc]);
                for (int i0 = kPendRead; i0 < npc; i0 += kBlock) {
                    const int i = i0 + t;
                    uint64_t v = 0;
                    if (i < npc) {
                        const uint64_t* p = &row_lists[(int64_t)cc * kTopkListStride + kWordPend + i];
                        v = ld_agent(p);
                        settle(v, p);
                    }
                    append_cand(sm, i < npc && above(v), v, ngath);
                }
            }
            if (spins >= kPollCap) sm.misc[7] = 1;
        }
        // ---- chunks read again (rare): the whole chunk in one round of
        //      loads (pass 1's layout), every entry >= the bound that is not
        //      a window id of the chunk (a bitmap from its penalised entries)
        for (int cc = 0; cc < S && !radix; ++cc) {
            if (!((reread >> cc) & 1u)) continue;
            // the chunk's window ids as a bitmap: from registers, the list
            // past the first read
            const int ce0 = cc * a.CE;
            auto mark = [&](uint64_t pe) {
                const int off = (int)ckey_id(pe) - ce0;
                atomicOr(&sm.big.wbits[off >> 5], 1u << (off & 31));
            };
            lds_sync();
            for (int i = t; i < kChunk / 32; i += kBlock) sm.big.wbits[i] = 0;
            lds_sync();
            const int npc = hdr_npen(sm.hdr[cc]);
            if (cc == c) {
                for (int i = t; i < npen; i += kBlock) mark(sm.pend[i]);
            } else {
#pragma unroll
                for (int u = 0; u < kPendPer; ++u) {
                    const int idx = t + u * kBlock;
                    if (idx / kPendRead == cc && idx % kPendRead < npc) mark(pw[u]);
                }
                for (int i = kPendRead + t; i < npc; i += kBlock)
                    mark(ld_agent(&row_lists[(int64_t)cc * kTopkListStride + kWordPend + i]));
            }
            lds_sync();
            reread_chunk<T, FAST>(base, mrow, ce0, min(ce0 + a.CE, V), kb, temp, divide, ngath, sm);
        }
        lds_sync();
        TMS_TR(12);
        n = ngath + sm.ncand;
        TMS_TV(17, n + 1);
        if (sm.misc[7]) {
            status = TMS_ROW_INTERNAL;
        } else if (radix || n > kCand) {
            // Massive ties (or too many penalised entries for the lists): the
            // exact top-K by a radix select over the whole row read again,
            // with every penalised entry of the row in sm.big.m.keys.
            if (t == 0) sm.ncand = 0;
            lds_sync();
            for (int cc = 0; cc < S; ++cc) {
                const int npc = hdr_npen(sm.hdr[cc]);
                for (int i = t; i < npc; i += kBlock) {
                    const uint64_t pe = cc == c ? sm.pend[i]
                                                : ld_agent(&row_lists[(int64_t)cc * kTopkListStride + kWordPend + i]);
                    const int pos = atomicAdd(&sm.ncand, 1);
                    if (pos < kCand) sm.big.m.keys[pos] = pe;
                }
            }
            lds_sync();
            const int np = min(sm.ncand, kCand);
            lds_sync();
            if ((fo & FLAG_OVERFLOW) || sm.ncand > kCand) {
                status = TMS_ROW_UNSUPPORTED;   // more window ids in the row than staging holds
            } else {
                n = lean_row_radix<T>(base, mrow, sm.big.m.keys, np, V, K, temp, divide, sm);
                all_finite = n < K;
                TMS_TV(16, 2);
            }
        }
        if (status == TMS_ROW_OK) {
            // Rank the candidates' keys by counting; the row's sorted top
            // min(n, K) lands in srt.
            rank_sort(sm.cand, n, srt, K);
            // With the bound at "every finite entry" the gather holds every
            // finite entry of the row.
            N = all_finite ? n : K;
            if (N == 0) status = TMS_ROW_ALL_MASKED;
            n = min(n, K);
        }
    }
    // Every word read goes back to zero for the next call: the other
    // chunks' headers, keys and penalised entries; this workgroup's own by
    // the lanes that stored them.  Waves 1-3 zero the other chunks' words
    // while wave 0 runs a sampled row's tail.
    auto zero_own = [&]() {
        st_agent(&my_list[kWordKeys + t], (uint64_t)0);
        st_agent(&my_list[kWordKeys + kBlock + t], (uint64_t)0);
        st_agent(&my_list[kWordKeys + 2 * kBlock + t], (uint64_t)0);
        for (int i = t; i < npen; i += kBlock) st_agent(&my_list[kWordPend + i], (uint64_t)0);
        if (t == 0) st_agent(&my_list[0], (uint64_t)0);
    };
    auto zero_others = [&](int tid0, int nthr) {
        for (int cc = 0; cc < S; ++cc) {
            if (cc == c) continue;
            uint64_t* L = row_lists + (int64_t)cc * kTopkListStride;
            const int npc = hdr_npen(sm.hdr[cc]);
            for (int i = tid0; i < kWordPend; i += nthr) st_agent(&L[i], (uint64_t)0);
            for (int i = tid0; i < npc; i += nthr) st_agent(&L[kWordPend + i], (uint64_t)0);
        }
    };
    if (!late_done) {   // a row that ended before the bound (uniform)
        if (!sm.misc[3]) settle_late();
        lds_sync();
    }
    const bool lost = sm.misc[3] != 0 || sm.misc[7] != 0;   // uniform: written before a barrier
    if (!lost && pextra && status != TMS_ROW_OK) {
        // penalised words past the first read: read (once written) before
        // they are zeroed
        for (int cc = 0; cc < S; ++cc) {
            if (cc == c) continue;
            const int npc = hdr_npen(sm.hdr[cc]);
            for (int i = kPendRead + t; i < npc; i += kBlock) {
                const uint64_t* p = &row_lists[(int64_t)cc * kTopkListStride + kWordPend + i];
                uint64_t v = ld_agent(p);
                settle(v, p);
            }
        }
    }
    if (!lost) zero_own();
    const bool sampled_ok = status == TMS_ROW_OK && !greedy;
    if (!lost && !sampled_ok) zero_others(t, kBlock);
    if (status == TMS_ROW_UNSUPPORTED) {
        // A row outside this kernel's kinds (top_k = 0 or > 128), or more
        // window ids than the lists stage: the exact whole-row path.
        if (a.dense) defer_dense(a, row);
        else write_row_error(a, row, TMS_ROW_UNSUPPORTED);
        TK_TRACE_FLUSH();
        return;
    }
    if (status != TMS_ROW_OK) {
        write_row_error(a, row, status);
        TK_TRACE_FLUSH();
        return;
    }
    TMS_TR(7);
    if (greedy) {
        const int tok = (int)ckey_id(srt[0]);
        if (t == 0) {
            a.out_tokens[row] = tok;
            a.out_status[row] = TMS_ROW_OK;
            if (a.out_keep) a.out_keep[row] = 0;
        }
        for (int i = t; i < a.topk_cap; i += kBlock) {
            if (a.out_topk_ids) a.out_topk_ids[(int64_t)row * a.topk_cap + i] = i == 0 ? tok : -1;
            if (a.out_topk_probs) a.out_topk_probs[(int64_t)row * a.topk_cap + i] = i == 0 ? 1.0f : 0.0f;
        }
        TK_TRACE_FLUSH();
        return;
    }
    if (N < K) {
        // Fewer than K finite ids: the tail goes on with -inf entries in
        // ascending id order, i.e. the ids in [0, K + N) missing from the
        // (then complete) finite set; K + N < 2 * kTopkFast <= kBlock.
        const int q = t;
        int member = 0;
        if (q < K + N)
            for (int i = 0; i < N; ++i) member |= (int)ckey_id(srt[i]) == q;
        const int gap = (q < K + N && !member && q < V) ? 1 : 0;
        int tot;
        const int p = block_excl_scan(gap, tot, sm);
        if (gap && p < K - N) srt[N + p] = ckey(NEG_INF, (uint32_t)q);
        lds_sync();
        n = K;
    }
    if (wv == 0) {
        tail_topk(a, row, P, srt, n, K, sm.big.m.pr, (double*)sm.cand, w0, w1);
        TMS_TR(8);
        TMS_TV(22, __builtin_amdgcn_s_memtime());
    } else {
        zero_others(t - 64, kBlock - 64);
    }
    TK_TRACE_FLUSH();
}

}  // namespace tms

// Launch of the top-k kernel for tms_sample_batch (declared in
// tms_sample_common.h): same argument block as the general kernel.
int tms_launch_topk(const tms::KArgs& k, int dtype, bool fast, int batch, hipStream_t stream) {
    const dim3 grid((unsigned)(batch * k.S)), block(tms::kBlock);
#define TMS_LAUNCH(T, F)                                                                  \
    do {                                                                                  \
        if (k.S <= 8) hipLaunchKernelGGL((tms::topk_kernel<T, F, 8>), grid, block, 0, stream, k); \
        else hipLaunchKernelGGL((tms::topk_kernel<T, F, 16>), grid, block, 0, stream, k);        \
    } while (0)
    switch (dtype) {
        case TMS_DTYPE_F32:
            if (fast) TMS_LAUNCH(float, true);
            else TMS_LAUNCH(float, false);
            break;
        case TMS_DTYPE_F16:
            if (fast) TMS_LAUNCH(_Float16, true);
            else TMS_LAUNCH(_Float16, false);
            break;
        default:
            if (fast) TMS_LAUNCH(tms::Bf16, true);
            else TMS_LAUNCH(tms::Bf16, false);
            break;
    }
#undef TMS_LAUNCH
    return hipGetLastError() == hipSuccess ? TMS_OK : TMS_ERR_HIP;
}

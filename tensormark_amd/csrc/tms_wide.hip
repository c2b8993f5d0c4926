// tms_wide.hip -- the sampler kernel for batches whose rows are all greedy or
// top-k with k <= 128 (the host picks it from the caller's row-kind hint),
// with 1024-thread workgroups whose grid is resident at once.
//
// One launch per call.  Row b is cut into S <= 16 chunks; workgroup (b, c)
// streams chunk c once, each thread kSlots nontemporal 16-byte loads: 8 for
// fp32 rows at one workgroup per CU (config 2: S = 4), else 4 at two per CU.
// A bare stream of 33 MB measured 8.7 us with 512 x 256-thread workgroups and
// 5.9 us with 512 x 1024.
//
//   window    while the stream is in flight: the row's history ids that fall
//             in the chunk go into an LDS bitmap and a hash table; the first
//             position holding an id owns it, counts its occurrences and
//             loads the id's logit and mask word itself.  The stream leaves
//             those ids out; after the bound the owners bring them back
//             penalised (tmsample.h:52-63 compounding, then
//             frequency/presence).
//   pass 1    per 16-byte slot: mask bit (and not a window id) -> value,
//             else -inf; the thread's maximum; NaN / +inf flagged.
//   bound     the maxima of 128 groups of lanes (DPP), ranked by counting on
//             every lane (eight lanes a group maximum); the K-th largest
//             bounds the chunk's K-th value from below (K groups, each with a
//             distinct entry, reach it); the ceil(K / S)-th largest gives the
//             merger's pruning bound.
//   select    every entry whose v / T can reach the bound's quotient is a
//             candidate (the division runs on candidates only): hot lanes
//             stage their words in LDS and each wave appends its takes.  Up
//             to 128 candidates are published unranked; more are ranked and
//             the top K published; over 1024 (massive ties) take an exact
//             radix select over the keys.  The list header carries both
//             bounds.
//   merge     the last chunk of the row to take a ticket reads the other
//             lists (a word still in flight reads 0 and is read again; the
//             merger returns every word it read to 0), keeps the keys at or
//             above the quotient of the larger of the two bounds, ranks them
//             together, and runs the fp64 tail of tmsample::sample
//             (tensormark/tmsample.h:184-199) on one wave.
#include "tms_sample_common.h"

namespace tms {
namespace wide {

constexpr int kTMax = 1024;         // threads per workgroup, at most
constexpr int kWMax = kTMax / 64;   // waves per workgroup, at most
constexpr int kWaveSlots = 128;     // waves x slots per thread, at most (32768 ids a chunk in fp32)
constexpr int kMaxS = kWideMaxChunksHost;
constexpr int kKMax = kTopkFast;    // largest K
constexpr int kLStride = kWideListStride;   // u64 per (row, chunk) list: header + kKMax keys, padded
constexpr int kHash = 2048;         // window table slots (at most 1024 ids: half full)
constexpr int kCntBits = 11;        // occurrence count bits of a table word (<= 1024)
constexpr uint32_t kEmpty = 0xFFFFFFFFu;
constexpr int kHot = 8;             // lanes a wave examines from LDS (more: every entry in place)
constexpr int kCap = 1024;          // chunk candidates held in LDS
constexpr int kPad = 256;           // slack after a ranked list (rank_place reads past it)
constexpr int kList = 128;          // a chunk's candidates published unranked up to this many
constexpr int kMW = 8;             // waves of the merge after the compaction (two a SIMD)
static_assert(kLStride >= 1 + kKMax && kLStride >= 1 + kList && kList >= kKMax && kList <= 128, "list layout");

// Header word: ready bit, flags (bits 48-55), list length (bits 32-47),
// the chunk's two bounds as the top 16 bits of their order keys (bits
// 16-31: K groups; bits 0-15: ceil(K / S) groups).
__device__ __forceinline__ uint64_t header(int flags, int n, uint32_t bound) {
    return kReady | ((uint64_t)(flags & 0xFF) << 48) | ((uint64_t)(n & 0xFFFF) << 32) | bound;
}
__device__ __forceinline__ uint32_t hdr_bound(uint64_t h) { return (uint32_t)h; }
__device__ __forceinline__ int hdr_n(uint64_t h) { return (int)((h >> 32) & 0xFFFF); }
__device__ __forceinline__ int hdr_flags(uint64_t h) { return (int)((h >> 48) & 0xFF); }

// Where the window bitmap keeps chunk offset `off`: thread-major, so that the
// thread that streams an id finds all of its ids' bits in one word.  Slot j,
// thread t, entry e (off = VEC (j NT + t) + e) is bit j VEC + e of word t.
template <int VEC, int NT>
__device__ __forceinline__ void wbit_pos(uint32_t off, uint32_t& word, uint32_t& bit) {
    const uint32_t r = off % (VEC * NT);
    word = r / VEC;
    bit = (off / (VEC * NT)) * VEC + r % VEC;
}

// First table slot of a chunk offset (multiplicative hash, 11 bits).
__device__ __forceinline__ int hash_slot(uint32_t off) { return (int)((off * 0x9E3779B1u) >> 21); }

// Read in place of the caller's draws and history when there are none
// (never written), so those loads need no branch.
__device__ uint32_t kNoDraws[2] = {0u, 0u};
__device__ int32_t kNoHistory[1] = {-1};

struct Smem {
    uint32_t wbits[1024];           // window ids of the chunk, thread-major (wbit_pos)
    uint32_t wtab[kHash];           // window ids: chunk offset << kCntBits | occurrences, or kEmpty
    alignas(16) union {
        struct {
            uint64_t cand[kCap + kPad];     // the chunk's candidates: value bits << 32 | id, then keys
        } c;
        uint64_t surv[kMaxS * kKMax + kPad];   // merge: the keys that can place
        struct {
            double pr[4 * kKMax];   // fp64 tail: pr, then the prefixes of z at +256
            double q[kKMax];
        } tail;
    } u;
    alignas(16) uint64_t slist[kKMax + 8];    // this chunk's sorted top keys
    alignas(16) uint64_t srt[kKMax + 8];      // the row's sorted top-K
    alignas(16) uint32_t gmax[128];           // order keys of the 128 lane-group maxima
    alignas(16) uint4 hot[kHot * kWaveSlots]; // per wave: the words of its hot lanes
    int hotlane[kWMax * kHot];                // per wave: the lane of each hot slot
    uint32_t tkey;                            // the chunk's bound (order key)
    uint32_t tkey_rm;                         // the same for ceil(K / S) groups
    float vlo;                                // the least value that can be a candidate
    alignas(16) uint32_t wnf[kWMax];          // per wave: a NaN or +inf seen
    alignas(16) int hist[256];
    alignas(16) uint32_t mt[kMaxS]; // merge: each chunk's bound (order key)
    alignas(16) int mn[kMaxS];      // merge: list lengths
    alignas(16) int mf[kMaxS];      // merge: list flags
    int ncand, nsurv, lost, onf;
    uint32_t ticket;
    uint32_t draw[2];               // the merger's draw words
    int flags;
    int misc[4];
};

#ifdef TMS_TRACE
// Trace builds: lane 0 of every wave stamps the 100 MHz real-time counter at
// phase boundaries, 32 slots per wave.
#define WTR(i)                                                                          \
    do {                                                                                \
        if ((threadIdx.x & 63) == 0 && a.trace)                                         \
            a.trace[(blockIdx.x * kWMax + (threadIdx.x >> 6)) * 32 + (i)] =                \
                __builtin_amdgcn_s_memrealtime();                                       \
    } while (0)
// A stamp that waits for `dep` (a value computed from the stream), so the
// compiler cannot move it ahead of the data it follows.
#define WTRD(i, dep)                                                                    \
    do {                                                                                \
        if ((threadIdx.x & 63) == 0 && a.trace && __float_as_uint(dep) != 0x7FC0ABCDu)     \
            a.trace[(blockIdx.x * kWMax + (threadIdx.x >> 6)) * 32 + (i)] =                \
                __builtin_amdgcn_s_memrealtime();                                       \
    } while (0)
#define WTV(i, val)                                                                     \
    do {                                                                                \
        if ((threadIdx.x & 63) == 0 && a.trace)                                         \
            a.trace[(blockIdx.x * kWMax + (threadIdx.x >> 6)) * 32 + (i)] = (uint64_t)(val); \
    } while (0)
#else
#define WTR(i) ((void)0)
#define WTRD(i, dep) ((void)0)
#define WTV(i, val) ((void)0)
#endif

// Reductions over the 64 lanes of a wave by DPP (no LDS round trips):
// butterflies within 16-lane rows (quad_perm, half-row and row mirrors),
// then across rows (row_bcast:15 and :31 towards lane 63, read there).
template <int CTRL, int RM = 0xF>
__device__ __forceinline__ uint32_t dpp_mov(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, CTRL, RM, 0xF, false);
}
constexpr int kQxor1 = 0xB1;   // quad_perm [1, 0, 3, 2]
constexpr int kQxor2 = 0x4E;   // quad_perm [2, 3, 0, 1]
constexpr int kHalfMirror = 0x141;
constexpr int kMirror = 0x140;
__device__ __forceinline__ int wave_or_i32(int v) {
    uint32_t u = (uint32_t)v;
    u |= dpp_mov<kQxor1>(u);
    u |= dpp_mov<kQxor2>(u);
    u |= dpp_mov<kHalfMirror>(u);
    u |= dpp_mov<kMirror>(u);
    u |= dpp_u32<0x142, 0xA, false>(0u, u);   // row_bcast:15
    u |= dpp_u32<0x143, 0xC, false>(0u, u);   // row_bcast:31
    return __builtin_amdgcn_readlane((int)u, 63);
}
// The maximum over lanes 0 .. 15 (DPP row shifts within row 0).
__device__ __forceinline__ uint32_t lanes16_max(uint32_t v) {
    v = max(v, dpp_u32<0x111, 0xF, true>(0u, v));   // row_shr:1
    v = max(v, dpp_u32<0x112, 0xF, true>(0u, v));   // row_shr:2
    v = max(v, dpp_u32<0x114, 0xF, true>(0u, v));   // row_shr:4
    v = max(v, dpp_u32<0x118, 0xF, true>(0u, v));   // row_shr:8
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 15);
}

// Sum over each aligned group of P lanes (P a power of two <= 16), every
// lane of the group receiving it.
__device__ __forceinline__ int group_sum(int v, int P) {
    uint32_t u = (uint32_t)v;
    if (P >= 2) u += dpp_mov<kQxor1>(u);
    if (P >= 4) u += dpp_mov<kQxor2>(u);
    if (P >= 8) u += dpp_mov<kHalfMirror>(u);
    if (P >= 16) u += dpp_mov<kMirror>(u);
    return (int)u;
}

// The digit of the 64-bit key radix select: wave 0 finds, among the 256
// bins of hist (digit values), the one holding the `remaining`-th largest key
// and how many keys lie in higher bins.
__device__ __forceinline__ void pick_digit(const int* hist, int remaining, int* out) {
    const int lane = threadIdx.x & 63;
    int h[4], s = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        h[i] = hist[255 - (4 * lane + i)];   // lane 0 holds the top bins
        s += h[i];
    }
    int above = wave_incl_scan_i32(s) - s;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if (above < remaining && above + h[i] >= remaining) {
            out[0] = 255 - (4 * lane + i);
            out[1] = above;
        }
        above += h[i];
    }
}

// Every thread of the workgroup: the keys keys[0..n) (distinct, 16-byte
// aligned, readable up to n + 32) whose rank (the number of larger keys)
// is below K land at out[rank].  P neighbouring lanes share a key,
// each counting the larger keys in its share of the list, and their counts
// are summed across the P lanes (DPP): P = NT / n rounded down to a power of
// two (at most 16), so a short list is ranked in a few steps by every wave
// instead of n steps by a few.
template <int NT>
__device__ __forceinline__ void rank_place(const uint64_t* keys, int n, int K, uint64_t* out,
                                           uint64_t* gout = nullptr) {
    const int t = threadIdx.x;
    int P = 16;
    while (P > 1 && P * n > NT) P >>= 1;
    // lane `part` of a key's P counts the keys [part * L, part * L + L) below
    // n, L even, in 16-byte reads (P * L <= n + 2P)
    const int L = ((n + P - 1) / P + 1) & ~1;
    const int per_pass = NT / P;
    for (int base = 0; base < n; base += per_pass) {
        const int i = base + t / P, part = t & (P - 1);
        const uint64_t k = i < n ? keys[i] : ~0ull;
        const ulonglong2* c2 = (const ulonglong2*)(keys + part * L);
        int cnt = 0;
#pragma unroll 2
        for (int q = 0; q < (L >> 1); ++q) {
            const ulonglong2 y = c2[q];
            const int j = part * L + 2 * q;
            cnt += (j < n && y.x > k ? 1 : 0) + (j + 1 < n && y.y > k ? 1 : 0);
        }
        cnt = group_sum(cnt, P);
        if (part == 0 && i < n && cnt < K) {
            out[cnt] = k;
            if (gout) st_agent(&gout[cnt], k);
        }
    }
}

// Every thread of the first ceil(n / 64) waves of NT: key t of keys[0..n)
// (distinct, 16-byte aligned) lands at out[rank] when its rank (the number
// of larger keys) is below K.  Each lane scans the whole list at addresses
// common to the wave (broadcast reads), eight keys a step into eight
// independent counts, so the compares do not wait on one another.
template <int NT>
__device__ __forceinline__ void rank_scan(const uint64_t* keys, int n, int K, uint64_t* out) {
    const int t = threadIdx.x;
    const ulonglong2* k2 = (const ulonglong2*)keys;
    for (int base = 0; base < n; base += NT) {
        const int i = base + t;
        if (base + (t & ~63) >= n) break;   // whole waves past the list
        const uint64_t x = i < n ? keys[i] : ~0ull;
        int c[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        const int n8 = n >> 3;
#pragma unroll 1
        for (int q = 0; q < n8; ++q) {
            ulonglong2 y[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) y[u] = k2[4 * q + u];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                c[2 * u] += y[u].x > x ? 1 : 0;
                c[2 * u + 1] += y[u].y > x ? 1 : 0;
            }
        }
        for (int j = n8 * 8; j < n; ++j) c[j & 7] += keys[j] > x ? 1 : 0;
        const int r = ((c[0] + c[1]) + (c[2] + c[3])) + ((c[4] + c[5]) + (c[6] + c[7]));
        if (i < n && r < K) out[r] = x;
    }
}

// The exact top-K keys of a chunk whose bound admits more than kCap
// candidates (massive ties): a radix select over the 64-bit keys (v / T,
// then lowest id), 8 bits a pass, with the chunk read again from memory
// (mask bit, window ids left to their owners, whose values come in as
// arguments).  Writes the K keys, unsorted, to sm.u.c.cand and returns K
// (the chunk holds more than kCap >= K finite entries).  Reading the chunk
// again, rather than from the registers of the stream, keeps the kernel's
// registers at what two workgroups per CU allow.
template <typename T, int NT>
__device__ __forceinline__ int radix_chunk(const T* base, const uint32_t* mrow, int e0, int e1, int K,
                                        float temp, bool divide, bool win, bool owner, float own_v,
                                        uint32_t own_id, Smem& sm) {
    const int t = threadIdx.x;
    const float NEG_INF = -__builtin_huge_valf();
    auto key_at = [&](int id, uint64_t& k) {
        if (!((mrow[id >> 5] >> (id & 31)) & 1u)) return false;
        if (win) {
            uint32_t wd, bt;
            wbit_pos<16 / sizeof(T), NT>((uint32_t)(id - e0), wd, bt);
            if ((sm.wbits[wd] >> bt) & 1u) return false;
        }
        const float v = Elt<T>::scalar(base + id);
        if (!(v > NEG_INF)) return false;
        k = ckey(divide ? v / temp : v, (uint32_t)id);
        return true;
    };
    const bool own = owner && own_v > NEG_INF;
    const uint64_t own_key = own ? ckey(divide ? own_v / temp : own_v, own_id) : 0ull;
    uint64_t prefix = 0, pmask = 0;
    int remaining = K;
    for (int shift = 56; shift >= 0; shift -= 8) {
        if (t < 256) sm.hist[t] = 0;
        lds_sync();
        for (int id = e0 + t; id < e1; id += NT) {
            uint64_t k;
            if (key_at(id, k) && (k & pmask) == prefix) atomicAdd(&sm.hist[(k >> shift) & 0xFF], 1);
        }
        if (own && (own_key & pmask) == prefix) atomicAdd(&sm.hist[(own_key >> shift) & 0xFF], 1);
        lds_sync();
        if (t < 64) pick_digit(sm.hist, remaining, sm.misc);
        lds_sync();
        remaining -= sm.misc[1];
        prefix |= (uint64_t)sm.misc[0] << shift;
        pmask |= 0xFFull << shift;
        lds_sync();
    }
    // prefix is the K-th largest key (keys are distinct): the K keys >= it
    if (t == 0) sm.ncand = 0;
    lds_sync();
    for (int id = e0 + t; id < e1; id += NT) {
        uint64_t k;
        if (key_at(id, k) && k >= prefix) {
            const int p = atomicAdd(&sm.ncand, 1);
            if (p < K) sm.u.c.cand[p] = k;
        }
    }
    if (own && own_key >= prefix) {
        const int p = atomicAdd(&sm.ncand, 1);
        if (p < K) sm.u.c.cand[p] = own_key;
    }
    lds_sync();
    return min(sm.ncand, K);
}

// NT threads of kSlots 16-byte slots each: (1024, 4) two workgroups per
// CU; (1024, 8), fp32, one workgroup per CU.
template <typename T, bool FAST, int kSlots, int NT>
__global__ __launch_bounds__(NT)
__attribute__((amdgpu_waves_per_eu(kSlots == 4 ? 8 : NT / 256, 8))) void topk_wide_kernel(KArgs a) {
    constexpr int kT = NT, kW = NT / 64;
    static_assert(kW * kSlots <= kWaveSlots, "hot-lane staging");
    constexpr int VEC = Elt<T>::kVec;
    constexpr int NV = kSlots * VEC;         // stream values per thread
    static_assert(kT <= 1024 && kSlots * VEC <= 32, "window bitmap: a word a thread");
    static_assert(kT == 1024, "bound: eight lanes a group maximum");
    __shared__ Smem sm;
    const float NEG_INF = -__builtin_huge_valf();
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    const int S = a.S, V = a.V;
    int row, c;
    wg_row_chunk(S, row, c);
    const int e0 = c * a.CE;   // a multiple of 32: the chunk starts on a mask word
    const int e1 = min(e0 + a.CE, V);
    const T* base = (const T*)a.logits + (int64_t)row * a.row_stride;
    const uint32_t* mrow = a.mask + (int64_t)row * a.mask_stride;

    // ---- loads in the order they are needed: history position t, then the
    //      mask words and the stream; the row's parameters and draw words
    //      come through the scalar path meanwhile.
    const int rs = a.recent ? (int)a.recent_stride : 1;
    const int32_t* hrow = a.recent ? a.recent + (int64_t)row * a.recent_stride : kNoHistory;
    const int wid_raw = hrow[min(t, rs - 1)];
    uint32_t mw[kSlots];
#pragma unroll
    for (int j = 0; j < kSlots; ++j) {
        const int off = VEC * (j * kT + t);
        mw[j] = mrow[(e0 + min(off, e1 - e0 - 1)) >> 5];
    }
    // Slot j holds the VEC entries from e0 + off in one 16-byte word group:
    // one nontemporal load when the row is 16-byte aligned, else VEC element
    // loads packed the same way.
    uint4 raw[kSlots];
#pragma unroll
    for (int j = 0; j < kSlots; ++j) {
        const int off = VEC * (j * kT + t);
        if constexpr (FAST) {
            raw[j] = ld_nt(base + e0 + min(off, e1 - e0 - VEC));
        } else {
            uint32_t w[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if constexpr (VEC == 4) {
                    w[i] = ((const uint32_t*)base)[min(e0 + off + i, e1 - 1)];
                } else {
                    const uint16_t* h = (const uint16_t*)base;
                    w[i] = (uint32_t)h[min(e0 + off + 2 * i, e1 - 1)] |
                           ((uint32_t)h[min(e0 + off + 2 * i + 1, e1 - 1)] << 16);
                }
            }
            raw[j] = make_uint4(w[0], w[1], w[2], w[3]);
        }
    }
    WTR(0);
    const tms_row_params P = a.params[row];
    const uint32_t* dp = a.draws ? a.draws + 2 * row : kNoDraws;
    const uint32_t dw0 = dp[0], dw1 = dp[1];
    int nrec = 0;
    if (a.recent) {
        nrec = a.n_recent ? a.n_recent[row] : rs;
        nrec = min(max(nrec, 0), rs);
    }

    const bool greedy = P.greedy != 0;
    const int K = greedy ? 1 : min(P.top_k, V);
    const bool unsupported = !greedy && !(P.top_k >= 1 && P.top_k <= kKMax);
    const float temp = P.temperature;
    const bool bad_params = !greedy && !(temp > 0.0f && temp <= FLT_MAX);
    const bool divide = !greedy && temp != 1.0f;
    const bool skip = unsupported || bad_params;   // the row needs no selection

    Pen pn;
    pn.rep_on = !(P.repeat_penalty <= 1.0f);
    pn.fp_on = P.frequency_penalty != 0.0f || P.presence_penalty != 0.0f;
    pn.on = nrec > 0 && P.repeat_last_n > 0 && (pn.rep_on || pn.fp_on);
    pn.rep = P.repeat_penalty;
    pn.freq = P.frequency_penalty;
    pn.pres = P.presence_penalty;
    const int from = pn.on ? (nrec > P.repeat_last_n ? nrec - P.repeat_last_n : 0) : 0;

    // ---- window, while the stream is in flight: the row's history ids in
    //      this chunk go into an LDS bitmap and a hash table keyed by chunk
    //      offset that counts their occurrences.  The entry that inserts a
    //      key owns the id.  The thread that streams the id writes its
    //      (masked) value into the table in pass 1, and after the bound the
    //      owner forms the penalised value (tmsample.h:58-61 once per
    //      occurrence, then frequency/presence) and offers it as a candidate.
    //      No load beyond the stream.
    if (pn.on) {
        sm.wbits[t] = 0u;
        for (int i = t; i < kHash; i += kT) sm.wtab[i] = kEmpty;
    }
    if (t == 0) {
        sm.lost = 0;
        sm.onf = 0;
        sm.ncand = 0;
        sm.nsurv = 0;
    }
    lds_sync();
    const bool in_chunk = pn.on && t >= from && t < nrec && wid_raw >= e0 && wid_raw < e1;
    // Every window position in the chunk loads its id's mask word and logit
    // now, both at once and before the insert, so the owner's copy is in
    // flight under the insert and the stream (the owner is known only after
    // the insert; the other positions drop theirs).
    uint32_t wmw = 0u;
    float wx = NEG_INF;
    if (in_chunk) {
        wmw = mrow[wid_raw >> 5];
        wx = Elt<T>::scalar(base + wid_raw);
    }
    bool owner = false;
    int wslot = 0;
    if (in_chunk) {
        const uint32_t off = (uint32_t)(wid_raw - e0);
        uint32_t wd, bt;
        wbit_pos<VEC, kT>(off, wd, bt);
        atomicOr(&sm.wbits[wd], 1u << bt);
        int sl = hash_slot(off);
        for (int probe = 0; probe < kHash; ++probe) {   // 2048 slots for at most 1024 ids
            const uint32_t old = atomicCAS(&sm.wtab[sl], kEmpty, off << kCntBits);
            if (old == kEmpty) {
                owner = true;
                break;
            }
            if ((old >> kCntBits) == off) break;
            sl = (sl + 1) & (kHash - 1);
        }
        atomicAdd(&sm.wtab[sl], 1u);
        wslot = sl;
    }
    // The window table is complete before the stream lands (the history
    // positions were loaded first): each thread reads the bits of its own
    // entries once, and pass 1 takes window ids out with the mask.
    uint32_t wt = 0u;
    if (pn.on) {
        lds_sync();
        wt = sm.wbits[t];   // bits past the chunk stay 0
    }
    WTR(1);

    // ---- pass 1, per slot as it lands: the mask and the window ids folded
    //      into the words (an entry the mask leaves out, or a window id,
    //      becomes the -inf pattern of its type in place; a window id's owner
    //      forms its penalised value from its own load), and the thread's
    //      IEEE maximum, which keeps a NaN, so one test of it finds any NaN
    //      or +inf.  Two to three instructions an entry.
    float m = NEG_INF;
#pragma unroll
    for (int j = 0; j < kSlots; ++j) {
        const int off = VEC * (j * kT + t);
        const int lim = e1 - e0 - off;   // ids of this slot inside the chunk
        const uint32_t vmask = lim > 0 ? (1u << min(lim, VEC)) - 1u : 0u;
        raw[j] = fold_bits<T>(raw[j], (mw[j] >> (off & 31)) & vmask & ~(wt >> (j * VEC)));
#pragma unroll
        for (int e = 0; e < VEC; e += 2)
            m = __builtin_elementwise_maximum(m, __builtin_elementwise_maximum(elt<T>(raw[j], e), elt<T>(raw[j], e + 1)));
    }
    WTRD(16, m);
    WTRD(17, m);
    // The owner's own copy of its id's masked logit, used after the bound
    // (its load was issued after the stream's, so it is read after pass 1).
    const float own_x = (owner && ((wmw >> (wid_raw & 31)) & 1u)) ? wx : NEG_INF;
    const bool nf = !(m < __builtin_huge_valf()) && m != NEG_INF;   // NaN or +inf
    // The row's ticket, now that the chunk's data is in: its round trip
    // overlaps the selection.  The last chunk of the row to get here merges;
    // a chunk with an earlier ticket may still be publishing when the merger
    // reads, and the merger reads such words again.
    uint32_t ticket = 0;
    if (S > 1 && t == 0)
        ticket = __hip_atomic_fetch_add(&a.counters[row * kCounterStride], 1u, __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_AGENT);
    WTR(2);
    // The widened values are formed again from the raw words where they are
    // used next: holding 32 widened 16-bit values across the bound would
    // take twice the registers of the words.
#pragma unroll
    for (int j = 0; j < kSlots; ++j)
        asm volatile("" : "+v"(raw[j].x), "+v"(raw[j].y), "+v"(raw[j].z), "+v"(raw[j].w));

    // ---- bound: the maxima of the 128 groups of G = NT / 128 lanes (DPP,
    //      on order keys), then the K-th largest of those, found by rank
    //      counting over every lane.  K groups, each with a distinct entry at
    //      or above it, bound the chunk's K-th value from below.  The group
    //      maxima are stored with their low 7 key bits replaced by 127 - the
    //      group's index, so they are distinct, ties going to the lower
    //      index; clearing those bits again leaves the K-th largest group
    //      maximum rounded down by under 2^7 key units, still a lower bound.
    const uint32_t mkey = nf ? 0u : okey(m);
    {
        constexpr int G = kT / 128;
        uint32_t g = mkey;
        if constexpr (G >= 2) g = max(g, dpp_u32<0x111, 0xF, true>(0u, g));   // row_shr:1
        if constexpr (G >= 4) g = max(g, dpp_u32<0x112, 0xF, true>(0u, g));   // row_shr:2
        if constexpr (G >= 8) g = max(g, dpp_u32<0x114, 0xF, true>(0u, g));   // row_shr:4
        const int gi = wv * (64 / G) + lane / G;
        if ((lane & (G - 1)) == G - 1) sm.gmax[gi] = (g & ~127u) | (uint32_t)(127 - gi);   // lanes Gq .. Gq + G - 1
    }
    const uint64_t nfw = __ballot(nf);
    if (lane == 0) sm.wnf[wv] = nfw ? 1 : 0;
    lds_sync();
    int flags = 0;
    {
        const uint4* f4 = (const uint4*)sm.wnf;
#pragma unroll
        for (int i = 0; i < kW / 4; ++i) {
            const uint4 q = f4[i];
            flags |= (q.x | q.y | q.z | q.w) ? FLAG_NONFINITE : 0;
        }
    }
    if (!skip) {
        // group maximum i = t / 8 is ranked by its eight lanes, lane p
        // counting the larger ones among groups 16p .. 16p + 15; the one of
        // rank K - 1 is the bound (and the one of rank ceil(K / S) - 1, to
        // 16 bits, the bound for ceil(K / S) groups, which only the
        // merger's pruning uses)
        const int gi = t >> 3, p = t & 7;
        const uint32_t x = sm.gmax[gi];
        const uint4* g4 = (const uint4*)(sm.gmax + 16 * p);
        uint4 y[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) y[q] = g4[q];
        int r = 0;
#pragma unroll
        for (int q = 0; q < 4; ++q)
            r += (y[q].x > x ? 1 : 0) + (y[q].y > x ? 1 : 0) + (y[q].z > x ? 1 : 0) + (y[q].w > x ? 1 : 0);
        r = group_sum(r, 8);
        if (p == 0) {
            if (r == K - 1) sm.tkey = x & ~127u;
            if (S > 1 && r == (K + S - 1) / S - 1) sm.tkey_rm = x & 0xFFFF0000u;
        }
    }
    lds_sync();
    const uint32_t tkey = sm.tkey;
    // the owners' penalised values (the table is complete: pass 1 came
    // before the barrier); they are left out of the bound, which K other
    // entries already meet
    float own_v = NEG_INF;
    if (owner) {
        own_v = apply_pen(own_x, sm.wtab[wslot] & ((1u << kCntBits) - 1u), pn);
        if (!(own_v < __builtin_huge_valf()) && own_v != NEG_INF) atomicOr(&sm.onf, 1);
    }
    WTR(3);

    // ---- select: candidates are the entries at or above vlo, whose
    //      quotient can reach the bound's.
    //      v < vlo implies fl(v / T) < fl(tau / T) (a relative gap of
    //      2^-19 exceeds two roundings; the absolute term covers subnormal
    //      quotients), so every entry below it has a key below K entries at
    //      or above tau.  -inf entries are never candidates (vlo >= -FLT_MAX).
    const bool select = !skip && !(flags & FLAG_NONFINITE);
    const float tau = okey_inv(tkey);
    float vlo = tau;
    if (divide && tau != NEG_INF) {
        if (fabsf(tau) >= temp * 0x1p-100f) {
            // normal quotients: tau - |tau| 2^-18 rounds to at most
            // tau (1 - 2^-19)
            vlo = tau - fabsf(tau) * 0x1p-18f;
        } else {
            const double lo = (double)tau - (fabs((double)tau) * 0x1p-19 + (double)temp * 0x1p-140);
            float f = (float)lo;
            if ((double)f > lo) f = float_below(f);
            vlo = f;
        }
    }
    vlo = fmaxf(vlo, -FLT_MAX);
    auto key_of = [&](float v, uint32_t id) { return ckey(divide ? v / temp : v, id); };
    // Candidates are appended as (value bits, id) to one LDS array: a
    // ballot per pass and one LDS atomic per wave and round.
    if (select) {
        // A lane holds candidates only if its maximum reaches vlo ("hot").
        const bool hot = m >= vlo;
        const uint64_t hb = __ballot(hot);
        const int nh = __popcll(hb);
        // The hot lanes' words go to LDS, kHot lanes a round, and the wave
        // examines only those entries, 64 a pass; the owner's value joins
        // the last round.
        const int hs = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(hb >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)hb, 0u));
        uint4* hw = sm.hot + (wv * kHot) * kSlots;
        const T* hv = (const T*)hw;   // hot slot s, entry q: hv[s * NV + q] with q = j * VEC + e
        constexpr int kPass = kHot * NV / 64;
        for (int g0 = 0; g0 == 0 || g0 < nh; g0 += kHot) {
            const int ng = max(0, min(nh - g0, kHot));
            const bool last = g0 + kHot >= nh;
            if (ng) {
                if (hot && hs >= g0 && hs < g0 + kHot) {
#pragma unroll
                    for (int j = 0; j < kSlots; ++j) hw[(hs - g0) * kSlots + j] = raw[j];
                    sm.hotlane[wv * kHot + hs - g0] = lane;
                }
                wave_lds_sync();
            }
            uint64_t bits[kPass];
            float xs[kPass];
            uint32_t ids[kPass];
            int total = 0;
#pragma unroll
            for (int pi = 0; pi < kPass; ++pi) {
                bits[pi] = 0ull;
                xs[pi] = NEG_INF;
                ids[pi] = 0u;
                if (pi * 64 < ng * NV) {
                    const int q = pi * 64 + lane, sidx = q / NV, qi = q % NV;
                    if (sidx < ng) {
                        xs[pi] = Elt<T>::scalar(hv + q);
                        ids[pi] = (uint32_t)(e0 + VEC * ((qi / VEC) * kT + wv * 64 + sm.hotlane[wv * kHot + sidx]) +
                                             qi % VEC);
                    }
                    bits[pi] = __ballot(xs[pi] >= vlo);
                    total += __popcll(bits[pi]);
                }
            }
            const bool ot = last && owner && own_v >= vlo;
            const uint64_t ob = __ballot(ot);
            total += __popcll(ob);
            if (total) {
                int base = 0;
                if (lane == 0) base = atomicAdd(&sm.ncand, total);
                base = __builtin_amdgcn_readfirstlane(base);
#pragma unroll
                for (int pi = 0; pi < kPass; ++pi) {
                    const uint64_t b = bits[pi];
                    const int p = base + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(b >> 32),
                                                                       __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0u));
                    if (((b >> lane) & 1ull) && p < kCap)
                        sm.u.c.cand[p] = ((uint64_t)__float_as_uint(xs[pi]) << 32) | ids[pi];
                    base += __popcll(b);
                }
                const int p = base + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(ob >> 32),
                                                                   __builtin_amdgcn_mbcnt_lo((uint32_t)ob, 0u));
                if (ot && p < kCap) sm.u.c.cand[p] = ((uint64_t)__float_as_uint(own_v) << 32) | (uint32_t)wid_raw;
            }
            if (ng) wave_lds_sync();   // the next round writes over these slots
        }
    }
    WTR(6);
    if (t == 0) sm.ticket = ticket;
    lds_sync();
    int ncand = select ? sm.ncand : 0;
    const bool merger = S == 1 || (int)sm.ticket == S - 1;   // the last chunk of the row to arrive
    WTR(4);
    const bool radixed = ncand > kCap;
    if (radixed) {
        // ---- exact radix select (every wave): the chunk's K keys
        ncand = radix_chunk<T, kT>(base, mrow, e0, e1, K, temp, divide, pn.on, owner, own_v,
                               (uint32_t)wid_raw, sm);
    }
    WTV(15, ncand);
    uint64_t* rl = a.tlists + (int64_t)row * S * kLStride;   // this row's lists
    uint64_t* my = rl + (int64_t)c * kLStride;
    // Merger waves 1 .. S - 1 hold the other lists (wave w: entry i in key0
    // of lane i, entry 64 + i in key1); wave 0 holds this chunk's own.
    uint64_t key0 = 0, key1 = 0;
    int ncc = 0;
    // ---- the keys (the division, one per candidate) and the publish
    //      (every word is non-zero; the merger reads a word again while it
    //      reads 0).  Up to kList candidates go out as they are, unranked;
    //      more are ranked first and their top K go out.  The header
    //      carries the chunk's bound, from which the merger prunes.  The
    //      merger's own list stays in LDS.
    if (sm.onf) flags |= FLAG_NONFINITE;     // a penalised window value
    const bool ranked = ncand > kList;
    const int nlist = ranked ? K : ncand;
    // the two bounds, each rounded down to 16 bits (still lower bounds)
    const uint32_t bound = select ? ((tkey >> 16) << 16) | (S > 1 ? sm.tkey_rm >> 16 : 0u) : 0u;
    for (int i = t; i < ncand; i += kT) {
        uint64_t key = sm.u.c.cand[i];
        if (!radixed) {
            key = key_of(__uint_as_float((uint32_t)(key >> 32)), (uint32_t)key);
            sm.u.c.cand[i] = key;
        }
        if (!merger && !ranked) st_agent(&my[1 + i], key);
    }
    WTR(10);
    if (ranked) {
        lds_sync();
        rank_place<kT>(sm.u.c.cand, ncand, K, sm.slist, merger ? nullptr : my + 1);
    }
    WTR(11);
    if (!merger) {
        if (t == 0) st_agent(&my[0], header(flags, nlist, bound));
        return;
    }
    lds_sync();   // the own list (keys or ranked) is in LDS
    if (wv == 0) {
        const uint64_t* own = ranked ? sm.slist : sm.u.c.cand;
        key0 = lane < nlist ? own[lane] : 0ull;
        key1 = lane + 64 < nlist ? own[lane + 64] : 0ull;
        ncc = nlist;
        if (lane == 0) {
            sm.mf[0] = flags;
            sm.mt[0] = bound;
        }
    } else if (wv == kW - 1 && S < kW) {
        // an idle merger wave: the row's draw words meanwhile
        uint32_t w0 = dw0, w1 = dw1;
        if (!a.draws && !greedy) row_words(P.seed, P.offset, 0u, w0, w1);
        if (lane == 0) {
            sm.draw[0] = w0;
            sm.draw[1] = w1;
        }
    } else if (wv < S) {
        // other list number wv - 1 (skipping this chunk's own)
        const int cc = wv - 1 < c ? wv - 1 : wv;
        uint64_t* L = rl + (int64_t)cc * kLStride;
        // header and keys at once; a word still in flight reads 0
        uint64_t h = ld_agent(&L[0]);
        uint64_t k0 = ld_agent(&L[1 + lane]);
        uint64_t k1 = ld_agent(&L[65 + lane]);   // unranked lists hold up to kList
        int spins = 0;
        while (!(h & kReady) && spins < kPollCap) {
            h = ld_agent(&L[0]);
            ++spins;
        }
        const int n = (h & kReady) ? hdr_n(h) : 0;
        while (lane < n && k0 == 0 && spins < kPollCap) {
            k0 = ld_agent(&L[1 + lane]);
            ++spins;
        }
        while (lane + 64 < n && k1 == 0 && spins < kPollCap) {
            k1 = ld_agent(&L[65 + lane]);
            ++spins;
        }
        const bool lost = !(h & kReady) || (lane < n && k0 == 0) || (lane + 64 < n && k1 == 0);
        if (__ballot(lost) && lane == 0) sm.lost = 1;
        key0 = lane < n ? k0 : 0ull;
        key1 = lane + 64 < n ? k1 : 0ull;
        ncc = n;
        if (lane == 0) {
            sm.mf[wv] = hdr_flags(h);
            sm.mt[wv] = hdr_bound(h);
        }
        // every word read goes back to zero for the next call
        if (!lost) {
            if (lane < n) st_agent(&L[1 + lane], (uint64_t)0);
            if (lane + 64 < n) st_agent(&L[65 + lane], (uint64_t)0);
            if (lane == 0) st_agent(&L[0], (uint64_t)0);
        }
    }
    WTR(5);

    // ================= merge (the last chunk of the row)
    if (t == 0 && S > 1) st_agent(&a.counters[row * kCounterStride], 0u);
    if (wv < S && lane == 0) sm.mn[wv] = ncc;
    lds_sync();
    // From here the merge runs on waves 0 .. max(S, kMW) - 1 (the list
    // holders for the compaction, eight for the rank), then on waves
    // 0 .. kMW - 1: the others leave, so each instruction of the merge is
    // issued by two waves or so a SIMD instead of four.  Eight rank a short
    // list in half the dependent LDS reads of four (0.15 us on config 2);
    // all sixteen were slower again.
    if (wv >= (S > kMW ? S : kMW)) return;

    WTR(7);
    // the lists' flags, lengths and bounds: lane l reads list l, and wave
    // reductions give each wave the totals and the largest bound
    int fo, ntot;
    uint32_t tmax;
    {
        const bool in = lane < S;
        const int f = in ? sm.mf[lane] : 0, n = in ? sm.mn[lane] : 0;
        fo = wave_or_i32(f);
        ntot = wave_sum_dpp(n);
        const uint32_t b = in ? sm.mt[lane] : 0u;
        // the largest K-group bound, and the least ceil(K / S)-group bound
        const uint32_t bk = lanes16_max(in ? b & 0xFFFF0000u : 0u);
        const uint32_t brm = ~lanes16_max(in ? ~(b << 16) : 0u);
        tmax = max(bk, brm);
    }
    WTR(12);
    int status = TMS_ROW_OK;
    if (sm.lost) status = TMS_ROW_INTERNAL;
    else if (bad_params) status = TMS_ROW_BAD_PARAMS;
    else if (fo & FLAG_NONFINITE) status = TMS_ROW_NONFINITE;
    else if (unsupported) status = TMS_ROW_UNSUPPORTED;
    else if (ntot == 0) status = TMS_ROW_ALL_MASKED;
    if (status != TMS_ROW_OK) {
        if (t == 0) {
            a.out_tokens[row] = -1;
            a.out_status[row] = status;
            if (a.out_keep) a.out_keep[row] = 0;
        }
        for (int i = t; i < a.topk_cap; i += kMW * 64) {
            if (t >= kMW * 64) break;
            if (a.out_topk_ids) a.out_topk_ids[(int64_t)row * a.topk_cap + i] = -1;
            if (a.out_topk_probs) a.out_topk_probs[(int64_t)row * a.topk_cap + i] = 0.0f;
        }
        return;
    }

    // ---- rank merge.  Chunk c holds K entries at or above its bound tau_c
    //      (K groups, each with a distinct entry at or above it) and
    //      ceil(K / S) at or above its bound rho_c, so the row's K-th largest
    //      value is at least T = max(max_c tau_c, min_c rho_c), and each of
    //      the row's top K keys has a quotient at least fl(T / temp) (the
    //      division is monotone).  Each of the row's top K keys is in its
    //      chunk's list: fewer than K keys of its chunk are above it, so it
    //      is at or above the chunk's bound (a candidate) and in a ranked
    //      list's top K.  The keys at or above that quotient are compacted
    //      and ranked among themselves: they hold the row's top K, so a key
    //      ranks below K there exactly when it does in the row, at the same
    //      rank.  A bound below -FLT_MAX prunes nothing.
    {
        uint64_t tg = 0ull;
        if (tmax >= okey(-FLT_MAX)) {
            const float tb = okey_inv(tmax);
            tg = (uint64_t)okey(divide ? tb / temp : tb) << 32;
        }
        const bool s0 = wv < S && lane < ncc && key0 >= tg;
        const bool s1 = wv < S && lane + 64 < ncc && key1 >= tg;
        // in any order (the rank counts): one LDS atomic per list wave
        const uint64_t b0 = __ballot(s0), b1 = __ballot(s1);
        if (wv < S && (b0 | b1)) {
            int off = 0;
            if (lane == 0) off = atomicAdd(&sm.nsurv, __popcll(b0) + __popcll(b1));
            off = __builtin_amdgcn_readfirstlane(off);
            const int r0 = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(b0 >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)b0, 0u));
            const int r1 = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(b1 >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)b1, 0u));
            if (s0) sm.u.surv[off + r0] = key0;
            if (s1) sm.u.surv[off + __popcll(b0) + r1] = key1;
        }
        lds_sync();
        if (wv >= kMW) return;
        const int nsurv = sm.nsurv;
        WTR(13);
        WTV(14, nsurv);
        rank_place<kMW * 64>(sm.u.surv, nsurv, K, sm.srt);
    }
    lds_sync();
    WTR(8);
    const int N = min(ntot, K);

    if (greedy) {
        const int tok = (int)ckey_id(sm.srt[0]);
        if (t == 0) {
            a.out_tokens[row] = tok;
            a.out_status[row] = TMS_ROW_OK;
            if (a.out_keep) a.out_keep[row] = 0;
        }
        for (int i = t; i < a.topk_cap; i += kMW * 64) {
            if (a.out_topk_ids) a.out_topk_ids[(int64_t)row * a.topk_cap + i] = i == 0 ? tok : -1;
            if (a.out_topk_probs) a.out_topk_probs[(int64_t)row * a.topk_cap + i] = i == 0 ? 1.0f : 0.0f;
        }
        return;
    }
    if (wv != 0) return;
    // ---- one wave from here: fewer than K finite ids -> the top-K goes on
    //      with -inf entries in ascending id order (the ids in [0, K + N)
    //      missing from the finite set).
    if (N < K) {
        int filled = 0;
        for (int q0 = 0; q0 < K + N && filled < K - N; q0 += 64) {
            const int q = q0 + lane;
            bool member = false;
            for (int i = 0; i < N; ++i) member |= (int)ckey_id(sm.srt[i]) == q;
            const bool gap = q < K + N && q < V && !member;
            const uint64_t b = __ballot(gap);
            const int p = filled + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(b >> 32),
                                                                  __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0u));
            if (gap && p < K - N) sm.srt[N + p] = ckey(NEG_INF, (uint32_t)q);
            filled += __popcll(b);
        }
        wave_lds_sync();
    }
    if (ckey_val(sm.srt[0]) == __builtin_huge_valf()) {   // v / T overflowed
        if (lane == 0) {
            a.out_tokens[row] = -1;
            a.out_status[row] = TMS_ROW_NONFINITE;
            if (a.out_keep) a.out_keep[row] = 0;
        }
        for (int i = lane; i < a.topk_cap; i += 64) {
            if (a.out_topk_ids) a.out_topk_ids[(int64_t)row * a.topk_cap + i] = -1;
            if (a.out_topk_probs) a.out_topk_probs[(int64_t)row * a.topk_cap + i] = 0.0f;
        }
        return;
    }
    uint32_t w0 = dw0, w1 = dw1;
    if (S < kW) {   // formed by the idle merger wave (the barriers since order its store)
        w0 = sm.draw[0];
        w1 = sm.draw[1];
    } else if (!a.draws) {
        row_words(P.seed, P.offset, 0u, w0, w1);
    }
    tail_topk(a, row, P, sm.srt, K, K, sm.u.tail.pr, sm.u.tail.q, w0, w1);
    WTR(9);
}

}  // namespace wide
}  // namespace tms

// Launch of the wide top-k kernel for tms_sample_batch (declared in
// tms_sample_common.h): same argument block as the general kernel, with
// k.S <= kWideMaxChunksHost chunks of k.CE ids (a multiple of 32, at most
// 4096 * the vector width).
int tms_launch_wide(const tms::KArgs& k, int dtype, bool fast, int batch, int slots, hipStream_t stream) {
    const dim3 grid((unsigned)(batch * k.S));
#define TMS_LAUNCH(T, F, SL, NT) \
    hipLaunchKernelGGL((tms::wide::topk_wide_kernel<T, F, SL, NT>), grid, dim3(NT), 0, stream, k)
    switch (dtype) {
        case TMS_DTYPE_F32:
            if (slots == 8) {
                if (fast) TMS_LAUNCH(float, true, 8, 1024);
                else TMS_LAUNCH(float, false, 8, 1024);
            } else if (fast) TMS_LAUNCH(float, true, 4, 1024);
            else TMS_LAUNCH(float, false, 4, 1024);
            break;
        case TMS_DTYPE_F16:
            if (fast) TMS_LAUNCH(_Float16, true, 4, 1024);
            else TMS_LAUNCH(_Float16, false, 4, 1024);
            break;
        default:
            if (fast) TMS_LAUNCH(tms::Bf16, true, 4, 1024);
            else TMS_LAUNCH(tms::Bf16, false, 4, 1024);
            break;
    }
#undef TMS_LAUNCH
    return hipGetLastError() == hipSuccess ? TMS_OK : TMS_ERR_HIP;
}

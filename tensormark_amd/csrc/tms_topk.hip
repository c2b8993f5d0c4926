// tms_topk.hip -- the sampler kernel for batches whose rows are all greedy or
// top-k with k <= 128 (the host picks it from the caller's row-kind hint).
//
// One launch per call, as the general kernel: row b is cut into S chunks of
// at most 16K ids, workgroup (b, c) streams its chunk once (nontemporal
// 16-byte loads) and reduces it to its sorted top-K, and the last workgroup
// of the row to take a ticket merges the S lists and runs the fp64 tail of
// tmsample::sample (tensormark/tmsample.h:184-199).  What differs is that
// every step is shaped for latency: the path has no top-p branch, so the
// whole chunk stays in registers and the compiler keeps the per-slot work
// where each slot's data lands.
//
//   pass 1     mask (bit extract + select), history penalties on the entries
//              this thread holds (marked in LDS while the stream is in
//              flight), and the running top two values per thread with the
//              index of the first.
//   threshold  the K-th largest of the 256 thread maxima by bisection on
//              their order keys, four compares a round into separate masks.
//   candidates a thread whose second value is below the threshold offers its
//              maximum (one ballot); a thread holding several stages its
//              values in LDS and the wave tests them an entry per lane.
//   ticket     taken right after pass 1, so its round trip overlaps the
//              selection; the last chunk of the row to take one merges, the
//              others publish their sorted lists.  Keys are never 0 and the
//              merger zeroes what it read, so a word still in flight reads 0
//              and is read again.
//   merge      keys above a proven lower bound of the row's K-th key are
//              gathered and ranked by counting; wave 0 runs the tail while
//              waves 1-3 zero the lists.
// A row that is not greedy and not top-k <= 128 breaks the hint and reports
// TMS_ROW_UNSUPPORTED.

#include "tms_sample_common.h"

namespace tms {

constexpr int kLeanMaxChunks = kLeanMaxChunksHost;       // vocab <= 262,144
constexpr int kLeanUni = kLeanMaxChunks * (kTopkFast + 1);   // every list, header + K entries
constexpr int kStage = 4;                                // threads a wave stages at a time
constexpr int kLate = kWaves * kStage * kEpt;           // window ids past the preloaded positions

struct LeanSmem {
    union {
        uint32_t cnt[kChunk / 2];   // window counts (16 bits per id) during pass 1
        struct {
            uint64_t uni[kLeanUni];     // the lists of the row (merger); candidate keys (chunk)
            uint64_t srt[kCand + 8];    // the merged, sorted top-K
        } m;
    } big;
    uint64_t cand[kCand + 8];       // chunk candidates, then the chunk's sorted list
    union {
        float stage[kWaves][kStage * kEpt];   // per wave: the values of threads holding several candidates
        int late[kLate];                      // window ids past the preloaded positions (before that)
    } sl;
    uint32_t mw[kWaves * 128];      // per wave: the mask words of its slots
    uint32_t wbits[kChunk / 32];    // ids of the chunk in the history window
    uint64_t pend[kCand];           // penalised window entries: (value, id)
    int npen, nlate;
    uint32_t tkey[kBlock];          // order keys of the thread maxima
    uint64_t wave_k[kWaves];
    int wave_i[kWaves];
    int wave_m[kWaves];
    int list_n[kLeanMaxChunks];
    int list_s[kLeanMaxChunks + 2];
    int list_src[kLeanMaxChunks + 1];
    int hist[256];
    int ncand;
    int misc[8];
    uint64_t theta;
};

// Bitwise OR over the 64 lanes of a wave (DPP steps towards lane 63).
__device__ __forceinline__ uint64_t wave_or_u64_dpp(uint64_t v) {
#define TMS_ORSTEP(CTRL, RM, BZ)                                                  \
    {                                                                             \
        const uint32_t lo = dpp_u32<CTRL, RM, BZ>(0u, (uint32_t)v);               \
        const uint32_t hi = dpp_u32<CTRL, RM, BZ>(0u, (uint32_t)(v >> 32));       \
        v |= ((uint64_t)hi << 32) | lo;                                           \
    }
    TMS_ORSTEP(0x111, 0xF, true)
    TMS_ORSTEP(0x112, 0xF, true)
    TMS_ORSTEP(0x114, 0xF, true)
    TMS_ORSTEP(0x118, 0xF, true)
    TMS_ORSTEP(0x142, 0xA, false)
    TMS_ORSTEP(0x143, 0xC, false)
#undef TMS_ORSTEP
    const uint32_t lo = __builtin_amdgcn_readlane((int)(uint32_t)v, 63);
    const uint32_t hi = __builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), 63);
    return ((uint64_t)hi << 32) | lo;
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

// List index of word idx when lists are R1 words long: (idx + 1/2) / R1 in
// float, exact for idx < 4096 and R1 <= 129 (the product is at least
// 1/(2 R1) away from an integer, far beyond the float error).
__device__ __forceinline__ int list_of(int idx, float rcp_r1) {
    return (int)(((float)idx + 0.5f) * rcp_r1);
}

// Zero every word of the row's lists the merger read (header and r entries
// of every list but its own, which it never publishes), threads tid0 ..
// nthr-1 of the workgroup.  Each word was read as written first, so its zero
// is ordered after its key.
__device__ __forceinline__ void zero_lean_lists(uint64_t* row_lists, int S, int r, int c, int tid0,
                                                int nthr) {
    for (int cc = 0; cc < S; ++cc) {
        if (cc == c) continue;
        uint64_t* L = row_lists + (int64_t)cc * kListStride;
        for (int jj = tid0; jj <= r; jj += nthr) st_agent(&L[jj], (uint64_t)0);
    }
}

// Id of entry q (slot q / vec, element q % vec) of thread t in the chunk at e0.
template <int VEC>
__device__ __forceinline__ uint32_t id_of(int t, int q, int e0) {
    return (uint32_t)(e0 + (t + (q / VEC) * kBlock) * VEC + q % VEC);
}

template <typename T, bool FAST>
__global__ __launch_bounds__(kBlock, 2) void topk_kernel(KArgs a) {
    constexpr int VEC = Elt<T>::kVec;
    constexpr int NVT = kEpt / VEC;
    constexpr uint64_t kLaneMask = (1ull << VEC) - 1ull;
    constexpr int kWin = 4;   // history ids loaded per thread with the stream
    __shared__ LeanSmem sm;
    const float NEG_INF = -__builtin_huge_valf();
    const int t = threadIdx.x;
    const int lane = t & 63, wv = t >> 6;
    const int S = a.S;
    const int row = blockIdx.x / S;
    const int c = blockIdx.x - row * S;
    const int V = a.V;
    const int e0 = c * a.CE;   // a multiple of 32: the chunk starts on a mask word
    const int e1 = min(e0 + a.CE, V);
    const int nvec = (e1 - e0 + VEC - 1) / VEC;
    TMS_TR(0);

    // ---- loads in the order they are needed: history window, row
    //      parameters, this wave's mask words, then the stream.
    const int32_t* hist = a.recent + (int64_t)row * a.recent_stride;
    int wid[kWin];
    if (a.recent) {
        const int rs = (int)a.recent_stride;
#pragma unroll
        for (int i = 0; i < kWin; ++i) wid[i] = hist[min(t + i * kBlock, rs - 1)];
    }
    const tms_row_params P = a.params[row];
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
    uint4 raw[NVT];
    float sx[FAST ? 1 : kEpt];
#pragma unroll
    for (int j = 0; j < NVT; ++j) {
        const int v = min(t + j * kBlock, nvec - 1);
        const int eb = e0 + v * VEC;
        if constexpr (FAST) {
            raw[j] = ld_stream(base + eb);
        } else {
#pragma unroll
            for (int e = 0; e < VEC; ++e) sx[j * VEC + e] = Elt<T>::scalar(base + min(eb + e, V - 1));
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    // The owners' loads: the logit and mask word of each preloaded window id
    // in this chunk (returned in order after this thread's stream).
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
    // While the stream is in flight: this wave's mask words into its own LDS
    // words (a wave-level sync, no workgroup barrier), and the window count
    // table zeroed for the count after pass 1.
    uint32_t* mw = sm.mw + wv * kWaveWords;
    mw[2 * lane] = mwd[0];
    mw[2 * lane + 1] = mwd[1];
    if (pn.on) {
        uint4* c4 = (uint4*)sm.big.cnt;
        for (int i = t; i < kChunk / 8; i += kBlock) c4[i] = make_uint4(0, 0, 0, 0);
        sm.wbits[2 * t] = 0;
        sm.wbits[2 * t + 1] = 0;
    }
    if (t == 0) {
        sm.ncand = 0;
        sm.npen = 0;
        sm.nlate = 0;
        sm.misc[2] = 0;   // the merger's read found an incomplete list
    }
    wave_lds_sync();
    TMS_TR(2);

    // ---- pass 1, as each slot lands: widen and mask (bit -> value or -inf),
    //      kept as the chunk's values in registers, with the thread's running
    //      top two values and the slot index of the first maximum (ids grow
    //      with the index, so a strict > keeps the lowest id).  The maxima
    //      propagate NaN (IEEE maximum): a NaN or +inf anywhere in the chunk
    //      shows in t1.  History penalties come after, on the few entries
    //      they touch.
    float xv[kEpt];
    float t1 = NEG_INF, t2 = NEG_INF;
    int i1 = 0;
#pragma unroll
    for (int j = 0; j < NVT; ++j) {
        const int v = t + j * kBlock;
        float f[VEC];
        if constexpr (FAST) {
            Elt<T>::widen(raw[j], f);
        } else {
#pragma unroll
            for (int e = 0; e < VEC; ++e) f[e] = sx[j * VEC + e];
        }
        // this lane's word of slot j: (lane * VEC / 32) within the slot's run
        const uint32_t mb = v < nvec ? mw[j * kWpS + ((lane * VEC) >> 5)] >> ((v * VEC) & 31) : 0u;
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
            const uint32_t sel = (uint32_t)__builtin_amdgcn_sbfe((int)mb, e, 1);
            uint32_t bits = (__float_as_uint(f[e]) & sel) | (0xFF800000u & ~sel);
            if constexpr (!FAST) bits = (e0 + v * VEC + e < e1) ? bits : 0xFF800000u;
            const float g = __uint_as_float(bits);
            i1 = g > t1 ? j * VEC + e : i1;
            t2 = __builtin_elementwise_maximum(t2, __builtin_elementwise_minimum(t1, g));
            t1 = __builtin_elementwise_maximum(t1, g);
            xv[j * VEC + e] = g;
        }
        // The running state is complete after each slot, so none of this
        // slot's work is deferred past the next slot's wait.
        asm volatile("" : "+v"(t1), "+v"(t2), "+v"(i1));
        __builtin_amdgcn_sched_barrier(0);
    }
    TMS_TR(3);
#ifdef TMS_PROBE_PASS1ONLY
    // Measurement builds stop here, to time the stream and pass 1 alone.
    if (t1 == 12345.0f && t2 == 1.0f && i1 == 7) a.out_tokens[row] = 0;   // keep the work live
    return;
#endif

    // ---- history penalties.  A chunk entry whose id is in the row's window
    //      is taken out of the holders' selection (a bitmap of window ids) and
    //      offered instead, with its penalised value, by the thread that
    //      counted that id first: the "owner", which loaded the logit with the
    //      stream.  The compounding penalty (tmsample.h:58-61) needs the id's
    //      count, from a 16-bit count table.
    int n_pen = 0;      // penalised candidates in sm.pend (all >= -inf; filtered by thr below)
    int m_win = 0;      // threads whose maximum is a window entry (the threshold skips them)
    bool pen_nf = false;
    if (pn.on) {
        lds_sync();   // the count table and bitmap are zeroed
        bool first[kWin];
#pragma unroll
        for (int i = 0; i < kWin; ++i) first[i] = false;
        for (int p0 = 0; p0 < nrec; p0 += kWin * kBlock) {
#pragma unroll
            for (int i = 0; i < kWin; ++i) {
                const int p = p0 + t + i * kBlock;
                const int id = (p < from || p >= nrec) ? -1 : (p0 == 0 ? wid[i] : hist[p]);
                if (id >= e0 && id < e1) {
                    const int off = id - e0;
                    atomicAdd(&sm.big.cnt[off >> 1], 1u << ((off & 1) * 16));
                    const uint32_t old = atomicOr(&sm.wbits[off >> 5], 1u << (off & 31));
                    if (!((old >> (off & 31)) & 1u)) {
                        if (p0 == 0) {
                            first[i] = true;
                        } else {
                            // past the preloaded positions (windows over
                            // kWin * kBlock ids): remembered for a late load
                            const int k = atomicAdd(&sm.nlate, 1);
                            if (k < kLate) sm.sl.late[k] = id;
                        }
                    }
                }
            }
        }
        lds_sync();
        // owners of the preloaded positions
        uint32_t flags_nf = 0;
#pragma unroll
        for (int i = 0; i < kWin; ++i) {
            if (first[i]) {
                const int id = wid[i];
                const int off = id - e0;
                const uint32_t cnt = (sm.big.cnt[off >> 1] >> ((off & 1) * 16)) & 0xFFFFu;
                float g = ((own_m[i] >> (id & 31)) & 1u) ? own_v[i] : NEG_INF;
                g = apply_pen(g, cnt, pn);
                flags_nf |= !(g < __builtin_huge_valf()) && g == g ? 1u : 0u;   // +inf after the penalty
                flags_nf |= g != g ? 1u : 0u;
                const int k = atomicAdd(&sm.npen, 1);
                if (k < kCand) sm.pend[k] = ((uint64_t)__float_as_uint(g) << 32) | (uint32_t)id;
            }
        }
        // owners past the preloaded positions (long windows only)
        const int nlate = min(sm.nlate, kLate);
        for (int k0 = 0; k0 < nlate; k0 += kBlock) {
            const int k = k0 + t;
            if (k < nlate) {
                const int id = sm.sl.late[k];
                const int off = id - e0;
                const uint32_t cnt = (sm.big.cnt[off >> 1] >> ((off & 1) * 16)) & 0xFFFFu;
                float g = slow_value(base, mrow, id, e0, Pen{false, false, false, 0.f, 0.f, 0.f}, sm);
                g = apply_pen(g, cnt, pn);
                flags_nf |= !(g < __builtin_huge_valf()) ? 1u : 0u;
                const int q = atomicAdd(&sm.npen, 1);
                if (q < kCand) sm.pend[q] = ((uint64_t)__float_as_uint(g) << 32) | (uint32_t)id;
            }
        }
        pen_nf = flags_nf != 0;
        // threads whose maximum is a window entry
        const int off1 = (int)id_of<VEC>(t, i1, e0) - e0;
        const bool w1 = t1 != NEG_INF && ((sm.wbits[off1 >> 5] >> (off1 & 31)) & 1u);
        m_win = __popcll(__ballot(w1));
    }
    TMS_TR(18);

    // ---- row mode
    const bool greedy = P.greedy != 0;
    const bool bad_params = !greedy && !(P.temperature > 0.0f && P.temperature <= FLT_MAX);
    const int K = greedy ? 1 : ((P.top_k <= 0 || P.top_k > V) ? V : P.top_k);
    const bool unsupported = K > kTopkFast;   // the caller's hint does not hold for this row
    const float temp = P.temperature;
    const bool divide = !greedy && temp != 1.0f;
    const uint32_t id1 = id_of<VEC>(t, i1, e0);
    const bool nf = __any(!(t1 < __builtin_huge_valf()));   // +inf or NaN in this wave's entries

    if (lane == 0) {
        sm.wave_i[wv] = nf || __any(pen_nf);
        sm.wave_m[wv] = m_win;
    }
    sm.tkey[t] = okey(t1);
    // Greedy rows without penalties take the chunk's best key directly;
    // others go through the selection below (greedy as K = 1).
    const bool greedy_fast = greedy && !pn.on;
    if (greedy_fast) {
        const uint64_t gb = wave_max_u64_dpp(t1 != NEG_INF ? ckey(t1, id1) : 0ull);
        if (lane == 0) sm.wave_k[wv] = gb;
    }
    // The row ticket, taken as soon as this chunk's stream is in: its round
    // trip overlaps the selection below.  The last chunk of the row to get
    // here merges; every other chunk publishes its list (and those all took
    // their tickets earlier, so none of them waits on the merger).
    uint32_t ticket = 0;
    if (t == 0)
        ticket = __hip_atomic_fetch_add(&a.counters[row * kCounterStride], 1u, __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_AGENT);
    lds_sync();
    TMS_TR(13);

    // ---- selection: the chunk's candidates, sorted, into sm.cand[0..nout).
    int flags = 0;
    int nout = 0;
    const bool anynf = (sm.wave_i[0] | sm.wave_i[1] | sm.wave_i[2] | sm.wave_i[3]) != 0;
    if (anynf) flags |= FLAG_NONFINITE;
    if (greedy_fast) {
        uint64_t b = sm.wave_k[0];
#pragma unroll
        for (int i = 1; i < kWaves; ++i) b = sm.wave_k[i] > b ? sm.wave_k[i] : b;
        if (t == 0 && b) sm.cand[0] = b;
        nout = (b && !anynf) ? 1 : 0;
    } else if (!anynf && !bad_params && !unsupported) {
        // The (K + M)-th largest of the 256 thread maxima, M the threads
        // whose maximum is a window entry: K threads then hold a non-window
        // entry >= it, so it bounds the K-th value from below.  Found bit by
        // bit on the sixteen high bits of their order keys: `pre` stays a
        // lower bound, and the few extra candidates it admits are ranked away.
        const int Kt = K + sm.wave_m[0] + sm.wave_m[1] + sm.wave_m[2] + sm.wave_m[3];
        const uint4 k4 = ((const uint4*)sm.tkey)[lane];   // 4 keys per lane, all 256
        uint32_t pre = 0;
        for (int bit = 31; bit >= 16; --bit) {
            const uint32_t cand = pre | (1u << bit);
            const uint64_t m0 = __builtin_amdgcn_uicmp(k4.x, cand, 35);   // unsigned >=
            const uint64_t m1 = __builtin_amdgcn_uicmp(k4.y, cand, 35);
            const uint64_t m2 = __builtin_amdgcn_uicmp(k4.z, cand, 35);
            const uint64_t m3 = __builtin_amdgcn_uicmp(k4.w, cand, 35);
            if (__popcll(m0) + __popcll(m1) + __popcll(m2) + __popcll(m3) >= Kt) pre = cand;
        }
        // Keys below okey(-FLT_MAX) decode to -inf or NaN: every finite entry.
        float thr = pre < 0x00800000u ? -FLT_MAX : okey_inv(pre);
        // Division can merge neighbouring values: lower the threshold to the
        // smallest float with the same quotient, so every entry tying the
        // K-th quotient is a candidate.
        bool fallback = false;
        if (divide && thr != NEG_INF) {
            const float qt = thr / temp;
            int it = 0;
            for (; it < 64; ++it) {
                const float p = float_below(thr);
                if (p / temp == qt) thr = p;
                else break;
            }
            fallback = it == 64;
        }
        if (thr == NEG_INF) thr = -FLT_MAX;   // every finite entry
        TMS_TR(9);
        int n = kCand + 1;
        if (!fallback) {
            // A thread whose second value is below thr holds at most one
            // entry >= thr, its maximum: one ballot places those.  A thread
            // holding several stages its values in LDS, and the wave tests
            // one staged thread per step, an entry per lane.
            auto in_window = [&](uint32_t id) -> bool {
                const int off = (int)id - e0;
                return pn.on && ((sm.wbits[off >> 5] >> (off & 31)) & 1u);
            };
            const bool multi = t2 >= thr;
            const bool one = t1 >= thr && !multi && !in_window(id1);
            const uint64_t m1 = __ballot(one);
            int wbase = 0;
            if (lane == 0 && m1) wbase = atomicAdd(&sm.ncand, __popcll(m1));
            wbase = __builtin_amdgcn_readfirstlane(wbase);
            const int r1 = __builtin_amdgcn_mbcnt_hi((uint32_t)(m1 >> 32),
                                                     __builtin_amdgcn_mbcnt_lo((uint32_t)m1, 0u));
            if (one && wbase + r1 < kCand)
                sm.cand[wbase + r1] = ((uint64_t)__float_as_uint(t1) << 32) | id1;
            uint64_t mm = __ballot(multi);
            float* stage = sm.sl.stage[wv];
            while (mm) {
                // up to kStage threads of the wave at a time
                const int rank = __builtin_amdgcn_mbcnt_hi((uint32_t)(mm >> 32),
                                                           __builtin_amdgcn_mbcnt_lo((uint32_t)mm, 0u));
                const bool mine = ((mm >> lane) & 1ull) && rank < kStage;
                if (mine) {
                    float4* dst = (float4*)(stage + rank * kEpt);
#pragma unroll
                    for (int q = 0; q < kEpt / 4; ++q)
                        dst[q] = make_float4(xv[4 * q], xv[4 * q + 1], xv[4 * q + 2], xv[4 * q + 3]);
                }
                const uint64_t taken = __ballot(mine);
                wave_lds_sync();
                uint64_t tk = taken;
                for (int si = 0; tk; ++si) {
                    const int L = __builtin_ctzll(tk);   // the staged thread: wave lane L
                    tk &= tk - 1;
                    // lane q tests entry q of thread L (slot q / VEC, element q % VEC)
                    const float f = stage[si * kEpt + lane];
                    const int tt = wv * 64 + L;
                    const uint32_t idq = id_of<VEC>(tt, lane, e0);
                    const bool hit = f >= thr && !in_window(idq);
                    const uint64_t mh = __ballot(hit);
                    int hb = 0;
                    if (lane == 0) hb = atomicAdd(&sm.ncand, __popcll(mh));
                    hb = __builtin_amdgcn_readfirstlane(hb);
                    const int pos = hb + __builtin_amdgcn_mbcnt_hi((uint32_t)(mh >> 32),
                                                                   __builtin_amdgcn_mbcnt_lo((uint32_t)mh, 0u));
                    if (hit && pos < kCand) sm.cand[pos] = ((uint64_t)__float_as_uint(f) << 32) | idq;
                }
                mm &= ~taken;
                wave_lds_sync();
            }
            if (pn.on) {
                // the window entries, with their penalised values
                const int np = min(sm.npen, kCand);
                for (int i0 = 0; i0 < np; i0 += kBlock) {
                    const int i = i0 + t;
                    const uint64_t pe = i < np ? sm.pend[i] : 0ull;
                    const bool hit = i < np && __uint_as_float((uint32_t)(pe >> 32)) >= thr;
                    const uint64_t mh = __ballot(hit);
                    int hb = 0;
                    if (lane == 0 && mh) hb = atomicAdd(&sm.ncand, __popcll(mh));
                    hb = __builtin_amdgcn_readfirstlane(hb);
                    const int pos = hb + __builtin_amdgcn_mbcnt_hi((uint32_t)(mh >> 32),
                                                                   __builtin_amdgcn_mbcnt_lo((uint32_t)mh, 0u));
                    if (hit && pos < kCand) sm.cand[pos] = pe;
                }
                if (sm.npen > kCand && t == 0) atomicAdd(&sm.ncand, kCand);   // overflow: the fallback
            }
            lds_sync();
            n = sm.ncand;
        }
        TMS_TR(10);
        TMS_TV(15, n + 1);
        if (n <= kCand) {
            // Divide the candidates and form their keys, then rank them by
            // counting; the chunk's list is its top min(n, K).
            uint64_t* keys = sm.big.m.uni;
            for (int i = t; i < n; i += kBlock) {
                const uint64_t rw = sm.cand[i];
                const float f = __uint_as_float((uint32_t)(rw >> 32));
                keys[i] = ckey(divide ? f / temp : f, (uint32_t)rw);
            }
            TMS_TR(11);
            rank_sort(keys, n, sm.cand, K);
            nout = n < K ? n : K;
        } else {
            nout = radix_slow<T>(base, mrow, e0, e1, K, temp, divide, pn, sm);
            sort_cand(nout, sm);
        }
    }
    TMS_TR(4);

    // ---- publish, or merge.  Each list is a ready header and K entries (key
    //      1 past nout), all non-zero; the merger zeroes what it read, so a
    //      word still in flight reads 0 and is read again.
    const int r = K > kTopkFast ? 0 : K;
    const int R1 = r + 1;
    const int NW = S * R1;
    const float rcp_r1 = 1.0f / (float)R1;
    const uint64_t hdr = kReady | ((uint64_t)flags << 32) | (uint64_t)(uint32_t)nout;
    uint64_t* row_lists = a.lists + (int64_t)row * S * kListStride;
    if (t == 0) sm.misc[0] = ticket == (uint32_t)(S - 1) ? 1 : 0;
    lds_sync();
    if (!sm.misc[0]) {
        uint64_t* my_list = row_lists + (int64_t)c * kListStride;
        for (int i = t; i <= r; i += kBlock)
            st_agent(&my_list[i], i == 0 ? hdr : (i <= nout ? sm.cand[i - 1] : (uint64_t)1));
        return;
    }
    TMS_TR(5);

    // ================= merge: the last workgroup of the row =================
    // Read every other list whole (waves 0-3), the row's uniform formed by
    // wave 0 meanwhile.
    constexpr int kReadPer = (kLeanUni + kBlock - 1) / kBlock;
    uint64_t sp[kReadPer];
#pragma unroll
    for (int u = 0; u < kReadPer; ++u) {
        const int idx = t + u * kBlock;
        sp[u] = 0;
        if (idx < NW) {
            const int cc = list_of(idx, rcp_r1);
            if (cc != c) sp[u] = ld_agent(&row_lists[(int64_t)cc * kListStride + (idx - cc * R1)]);
        }
    }
    uint32_t w0 = 0, w1 = 0;
    if (wv == 0) row_uniform(a, row, P, w0, w1);
    if (t == 64) st_agent(&a.counters[row * kCounterStride], 0u);   // ready for the next launch
    uint64_t* uni = sm.big.m.uni;
    if (t == 0) {
        sm.theta = 0;     // lists to read again (bit per list)
        sm.misc[3] = 0;   // a list never arrived
    }
    {
        // Every word read must be set: a ready header, non-zero entries.
        int bad = 0;
#pragma unroll
        for (int u = 0; u < kReadPer; ++u) {
            const int idx = t + u * kBlock;
            if (idx < NW) {
                const int cc = list_of(idx, rcp_r1), jj = idx - cc * R1;
                uint64_t v = sp[u];
                if (cc == c) v = jj == 0 ? hdr : (jj <= nout ? sm.cand[jj - 1] : (uint64_t)1);
                else bad |= (jj == 0 ? !(v & kReady) : v == 0) ? 1 : 0;
                uni[idx] = v;
            }
        }
        if (__ballot(bad) && lane == 0) atomicOr(&sm.misc[2], 1);
        lds_sync();
        // Lists read before they were complete are read again in rounds:
        // wave 0 waits (bounded) for their ready headers, then every thread
        // re-reads their entries at once.
        int rounds = 0;
        for (int round = 0; sm.misc[2]; ++round) {
            rounds = round + 1;
            for (int idx = t; idx < NW; idx += kBlock) {
                const int cc = list_of(idx, rcp_r1), jj = idx - cc * R1;
                const uint64_t h = uni[cc * R1];
                if (!(h & kReady) || (jj >= 1 && uni[idx] == 0))
                    atomicOr((unsigned long long*)&sm.theta, 1ull << cc);
            }
            lds_sync();
            const uint64_t redo = sm.theta;
            if (redo == 0 || sm.misc[3]) break;
            if (round == kReadRounds) {
                if (t == 0) sm.misc[3] = 1;
                lds_sync();
                break;
            }
            lds_sync();   // every thread has read theta
            if (t == 0) sm.theta = 0;
            if (wv == 0 && lane < S && ((redo >> lane) & 1)) {
                uint64_t h = 0;
                for (int it = 0; it < kPollCap; ++it) {
                    h = ld_agent(&row_lists[(int64_t)lane * kListStride]);
                    if (h & kReady) break;
                    __builtin_amdgcn_s_sleep(1);
                }
                uni[lane * R1] = h;
                if (!(h & kReady)) sm.misc[3] = 1;
            }
            lds_sync();
            for (int idx = t; idx < NW; idx += kBlock) {
                const int cc = list_of(idx, rcp_r1), jj = idx - cc * R1;
                if (jj == 0 || !((redo >> cc) & 1)) continue;
                uni[idx] = ld_agent(&row_lists[(int64_t)cc * kListStride + jj]);
            }
            lds_sync();
        }
        TMS_TV(14, rounds + 1);
    }
    TMS_TR(6);
    // Headers: counts and flags; lower bounds tau on the row's K-th key: a
    // list's K-th entry (that list alone holds K keys >= it), or the
    // smallest m-th entry over all lists, m = ceil(K / S) (the S lists hold
    // S * m >= K keys >= it).  Every wave forms them, so no barrier follows.
    int n_c = 0, f_c = 0;
    uint64_t kth = 0, mth = ~0ull;
    if (lane < S) {
        const uint64_t h = uni[lane * R1];
        n_c = (int)(uint32_t)h;
        f_c = (int)((h >> 32) & 0xFF);
        const int m = (K + S - 1) / S;
        kth = (r > 0 && n_c >= K) ? uni[lane * R1 + K] : 0ull;
        mth = (r > 0 && n_c >= m) ? uni[lane * R1 + m] : 0ull;
        if (wv == 0) sm.list_n[lane] = n_c;
    }
    const int N = wave_sum_dpp(n_c);
    const bool any_nf = __ballot(lane < S && (f_c & FLAG_NONFINITE)) != 0;
    const uint64_t tau = max(wave_max_u64_dpp(kth), ~wave_max_u64_dpp(~mth));
    int status = TMS_ROW_OK;
    if (sm.misc[3]) status = TMS_ROW_INTERNAL;
    else if (unsupported) status = TMS_ROW_UNSUPPORTED;
    else if (bad_params) status = TMS_ROW_BAD_PARAMS;
    else if (any_nf) status = TMS_ROW_NONFINITE;
    else if (N == 0) status = TMS_ROW_ALL_MASKED;

    uint64_t* srt = sm.big.m.srt;
    const int n_acc = min(N, K);
    bool whole = false;
    if (status == TMS_ROW_OK) {
        // Every key >= tau, gathered in parallel (unordered), then ranked by
        // counting within that set: it is closed upward, so ranks are exact.
        if (t == 0) sm.ncand = 0;
        lds_sync();
        for (int i0 = 0; i0 < NW; i0 += kBlock) {
            const int idx = i0 + t;
            bool keepit = false;
            uint64_t k = 0;
            if (idx < NW) {
                const int cc = list_of(idx, rcp_r1), jj = idx - cc * R1;
                k = uni[idx];
                keepit = jj >= 1 && jj <= (int)(uint32_t)uni[cc * R1] && k >= tau;
            }
            const uint64_t m = __ballot(keepit);
            int wb = 0;
            if (lane == 0 && m) wb = atomicAdd(&sm.ncand, __popcll(m));
            wb = __builtin_amdgcn_readfirstlane(wb);
            const int pos = wb + __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                                           __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
            if (keepit && pos < kCand) sm.cand[pos] = k;
        }
        lds_sync();
        TMS_TR(12);
        const int nc = sm.ncand;
        TMS_TV(17, nc + 1);
        if (nc <= kCand) {
            rank_sort(sm.cand, nc, srt, n_acc);
        } else {
            // A weak tau (rare): rank every list entry by binary search in
            // the other lists, all of them in LDS (uni).
            whole = true;
            for (int idx = t; idx < NW; idx += kBlock) {
                const int cc = list_of(idx, rcp_r1), jj = idx - cc * R1;
                if (jj == 0 || jj > sm.list_n[cc]) continue;
                const uint64_t k = uni[idx];
                int rank = jj - 1;
                for (int o = 0; o < S; ++o)
                    if (o != cc) rank += count_greater(uni + o * R1 + 1, sm.list_n[o], k);
                if (rank < n_acc) srt[rank] = k;
            }
            lds_sync();
        }
    }
    (void)whole;
    // Every word of this call's lists goes back to zero for the next call;
    // on a sampled row's success path waves 1-3 do it while wave 0 runs the
    // tail.
    const bool defer_zero = status == TMS_ROW_OK && !greedy && !sm.misc[3];
    if (!defer_zero && !sm.misc[3]) zero_lean_lists(row_lists, S, r, c, t, kBlock);
    if (status != TMS_ROW_OK) {
        write_row_error(a, row, status);
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
        return;
    }

    int n = n_acc;
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
    if (ckey_val(srt[0]) == __builtin_huge_valf()) {
        zero_lean_lists(row_lists, S, r, c, t, kBlock);
        write_row_error(a, row, TMS_ROW_NONFINITE);
        return;
    }
    if (wv == 0) {
        tail_topk(a, row, P, srt, n, K, (double*)sm.big.m.uni, (double*)sm.cand, w0, w1);
        TMS_TR(8);
    } else {
        zero_lean_lists(row_lists, S, r, c, t - 64, kBlock - 64);
    }
}

}  // namespace tms

// Launch of the top-k kernel for tms_sample_batch (declared in
// tms_sample_common.h): same argument block as the general kernel.
int tms_launch_topk(const tms::KArgs& k, int dtype, bool fast, int batch, hipStream_t stream) {
    const dim3 grid((unsigned)(batch * k.S)), block(tms::kBlock);
#define TMS_LAUNCH(T, F) hipLaunchKernelGGL((tms::topk_kernel<T, F>), grid, block, 0, stream, k)
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

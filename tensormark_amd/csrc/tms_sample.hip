// tms_sample.hip -- batched token sampler for gfx950 (MI355X).
//
// One launch per call.  Row b of the batch is cut into S chunks of at most
// 16K ids; workgroup (b, c) streams its chunk from HBM once with 16-byte
// loads into registers (64 values per thread), applies the grammar mask and
// the history penalties there, and reduces the chunk to a short sorted
// candidate list.  The last workgroup of the row to finish its stream merges
// the S lists (top-k rows from a pruned sample of them; whole lists ranked by
// value buckets otherwise) and runs the fp64 tail of tmsample::sample
// (tensormark/tmsample.h:184-199): softmax over the top-k, top-p and min-p
// cuts, and the inverse-CDF draw.
//
// Row modes (uniform per workgroup):
//   greedy  the chunk's best (value, lowest id); the merge takes the best.
//   top-k   K <= kTopkFast: the chunk's exact top-K by (v / T desc, id asc).
//           The K-th largest of the 256 thread maxima bounds the candidates
//           (about K of them), so only they are divided by T.  An exact
//           radix select over the chunk (re-read from L2) is the fallback
//           when the bound admits too many.
//   top-p   K > kTopkFast (top_k = 0 or large): every chunk entry whose
//           probability can change the fp64 sums, i.e. v / T within 40 of
//           the chunk maximum (exp(-40) < 2^-57); rows past the capacity
//           are sampled whole by their merger (tms_dense.h).
//
// Timeline of a workgroup: the stream's loads are the kernel's first
// instructions and are issued unconditionally (clamped addresses, an all-ones
// mask row when the caller gives none), so each slot is processed as it
// lands.  The history window is counted in LDS before the stream lands: each
// penalised entry is masked out of the stream like a grammar-masked one and
// comes back as an extra candidate from the thread that counted its id first
// (that thread read the logit separately and applies the compounding penalty
// once).  The workgroup then selects its candidates and takes a
// ticket from the row's arrival counter.  The last ticket holder merges; the
// others publish their list and set a ready bit in its header.  All
// cross-workgroup words are relaxed
// agent-scope atomics, coherent across the XCDs' L2 caches, with stores
// drained (s_waitcnt) before the header that announces them; the merger's
// wait for the headers is bounded.

#include <algorithm>
#include <atomic>
#include <mutex>

#include "tms_dense.h"
#include "tms_select.h"

namespace tms {

// Every thread of the workgroup: out[r] = keys[i] for every i < n, r the
// number of larger keys (keys 16-byte aligned, readable up to n + 16).  P
// neighbouring lanes share a key (P = kBlock / n rounded down to a power of
// two, at most 8), each counting the larger keys in its share of the list in
// 16-byte reads; the shares meet by DPP within the group.  Equal keys (the
// zero keys of dropped top-p entries) land on one slot.
__device__ __forceinline__ void rank_all(const uint64_t* keys, int n, uint64_t* out) {
    const int t = threadIdx.x;
    int P = 8;
    while (P > 1 && P * n > kBlock) P >>= 1;
    const int L = ((n + P - 1) / P + 1) & ~1;
    for (int b0 = 0; b0 < n; b0 += kBlock / P) {
        const int i = b0 + t / P, part = t & (P - 1);
        const uint64_t k = i < n ? keys[i] : ~0ull;
        const ulonglong2* c2 = (const ulonglong2*)(keys + part * L);
        int cnt = 0;
#pragma unroll 4
        for (int q = 0; q < (L >> 1); ++q) {
            const ulonglong2 y = c2[q];
            const int j = part * L + 2 * q;
            cnt += (j < n && y.x > k ? 1 : 0) + (j + 1 < n && y.y > k ? 1 : 0);
        }
        uint32_t u = (uint32_t)cnt;
        if (P >= 2) u += dpp_u32<0xB1, 0xF, false>(0u, u);    // quad_perm [1, 0, 3, 2]
        if (P >= 4) u += dpp_u32<0x4E, 0xF, false>(0u, u);    // quad_perm [2, 3, 0, 1]
        if (P >= 8) u += dpp_u32<0x141, 0xF, false>(0u, u);   // row_half_mirror
        if (part == 0 && i < n) out[u] = k;
    }
}

// log2 of the words per list (header + entries) a whole-list merger reads
// with the headers: the largest power of two that kUni holds for S lists,
// at most 128.
__device__ __forceinline__ int stage_log2(int S) {
    int l = 7;
    while (l > 0 && (S << l) > kUni) --l;
    return l;
}

// NV logits a thread: kEpt, or kEptPacked for calls without a history
// window on 16-byte-aligned 2-byte rows, whose stream stays in registers as
// the masked raw vectors (half the registers of widened values), so a
// chunk holds 20480 ids and fewer workgroups cover a row.
template <typename T, bool FAST, int NV>
__global__ __launch_bounds__(kBlock, 3) void sample_kernel(KArgs a) {
    constexpr int VEC = Elt<T>::kVec;
    constexpr int NVT = NV / VEC;
    constexpr bool kPacked = NV != kEpt;
    static_assert(!kPacked || (FAST && VEC == 8), "the packed stream: 2-byte, aligned rows");
    __shared__ Smem sm;
    static_assert(sizeof(DenseLds) <= sizeof(sm.big), "the whole-row path's LDS over the merge staging");
    const float NEG_INF = -__builtin_huge_valf();
    const int t = threadIdx.x;
    const int lane = t & 63, wv = t >> 6;
    const int S = a.S;
    int row, c;
    wg_row_chunk(S, row, c);
    const int V = a.V;
    const int e0 = c * a.CE;
    const int e1 = min(e0 + a.CE, V);
    const int nvec = (e1 - e0 + VEC - 1) / VEC;
    TMS_TR(0);

    // ---- history ids first (the row's first 4 * kBlock; positions are
    //      checked against the window once the parameters are in), then the
    //      stream: one mask word and one 16-byte vector per slot, every slot
    //      loaded (clamped to the chunk's last vector), in slot order.
    constexpr int kWin = 4;   // history ids per thread per pass
    const int32_t* hist = a.recent + (int64_t)row * a.recent_stride;
    int wid[kWin];
    if (a.recent) {
        const int rs = (int)a.recent_stride;
#pragma unroll
        for (int i = 0; i < kWin; ++i) wid[i] = hist[min(t + i * kBlock, rs - 1)];
    }
    // Row parameters: scalar loads, independent of the vector stream.
    const tms_row_params P = a.params[row];
    int nrec = 0;
    if (a.recent) {
        nrec = a.n_recent ? a.n_recent[row] : (int)a.recent_stride;
        if (nrec > (int)a.recent_stride) nrec = (int)a.recent_stride;
    }
    // With the history pre-pass the window is its list; -1: the row touched
    // more ids than the list holds.
    const bool ovm = a.ov_vals != nullptr;
    const bool hist_over = ovm && nrec < 0;
    nrec = max(nrec, 0);
    __builtin_amdgcn_sched_barrier(0);
    const T* base = (const T*)a.logits + (int64_t)row * a.row_stride;
    const uint32_t* mrow = a.mask + (int64_t)row * a.mask_stride;
    uint4 raw[NVT];
    uint32_t mw[NVT];
    float sx[FAST ? 1 : NV];
#pragma unroll
    for (int j = 0; j < NVT; ++j) {
        const int v = min(t + j * kBlock, nvec - 1);
        const int eb = e0 + v * VEC;
        mw[j] = mrow[eb >> 5];
        if constexpr (FAST) {
            raw[j] = *(const uint4*)(base + eb);
        } else {
#pragma unroll
            for (int e = 0; e < VEC; ++e) sx[j * VEC + e] = Elt<T>::scalar(base + min(eb + e, V - 1));
        }
        __builtin_amdgcn_sched_barrier(0);
    }

    // ---- history penalties, before the stream lands.  Every window id in
    //      this chunk is counted in LDS; the thread that counts an id first
    //      owns it: it marks the entry in its holder's bit set (pass 1 then
    //      masks it like a grammar-masked entry) and, after pass 1, applies
    //      the penalty to the logit it read for it and carries the result as
    //      an extra candidate.  Windows past kWin * kBlock positions take the
    //      register pass below instead.
    Pen pn;
    pn.rep_on = !(P.repeat_penalty <= 1.0f);
    pn.fp_on = P.frequency_penalty != 0.0f || P.presence_penalty != 0.0f;
    pn.on = !kPacked && nrec > 0 && (ovm || (P.repeat_last_n > 0 && (pn.rep_on || pn.fp_on)));
    pn.rep = P.repeat_penalty;
    pn.freq = P.frequency_penalty;
    pn.pres = P.presence_penalty;
    if (ovm) pn.ov = a.ov_vals + (int64_t)row * kHistMax;
    const int from = (pn.on && !ovm) ? (nrec > P.repeat_last_n ? nrec - P.repeat_last_n : 0) : 0;
    const bool pen_own = pn.on && nrec <= kWin * kBlock;
    if (pn.on) {
        uint4* c4 = (uint4*)sm.big.cnt;
        for (int i = t; i < kChunk / 8; i += kBlock) c4[i] = make_uint4(0, 0, 0, 0);
        sm.pbits[2 * t] = 0;
        sm.pbits[2 * t + 1] = 0;
        lds_sync();
    }
    int own_off[kWin];
    float own_v[kWin];
    uint32_t own_m[kWin];
    uint64_t penbits = 0;
#pragma unroll
    for (int i = 0; i < kWin; ++i) own_off[i] = -1;
    if (pen_own) {
        // The counts first, all four positions' atomics issued before any
        // result is used (a branch on each result would wait out one LDS
        // round trip per position), then the owners mark their entries.
        int woff[kWin];
        uint32_t wold[kWin];
#pragma unroll
        for (int i = 0; i < kWin; ++i) {
            const int p = t + i * kBlock;
            const int id = (p >= from && p < nrec) ? wid[i] : -1;
            const bool in = id >= e0 && id < e1;
            const int off = in ? id - e0 : 0;
            woff[i] = in ? off : -1;
            // read for every slot (clamped): the logit and its mask word
            own_v[i] = Elt<T>::scalar(base + e0 + off);
            own_m[i] = mrow[(e0 + off) >> 5];
            const uint32_t sh = (off & 1) * 16;
            const uint32_t add = ovm ? (uint32_t)(p + 1) : 1u;   // list position + 1, or a count
            wold[i] = 0u;
            if (in) wold[i] = atomicAdd(&sm.big.cnt[off >> 1], add << sh);
        }
#pragma unroll
        for (int i = 0; i < kWin; ++i) {
            const int off = woff[i];
            if (off >= 0 && ((wold[i] >> ((off & 1) * 16)) & 0xFFFFu) == 0) {
                own_off[i] = off;
                const int vv = off / VEC;
                const int bit = (vv / kBlock) * VEC + off % VEC;
                atomicOr(&sm.pbits[2 * (vv % kBlock) + (bit >> 5)], 1u << (bit & 31));
            }
        }
        lds_sync();
        penbits = ((uint64_t)sm.pbits[2 * t + 1] << 32) | sm.pbits[2 * t];
    }

    // ---- pass 1, as each slot lands: widen, mask, NaN/+inf check, slot max.
    //      The packed form keeps the masked raw vector (a masked entry holds
    //      the type's -inf) and widens it again where it is read.
    float x[kPacked ? 1 : NV];
    uint4 xr[kPacked ? NVT : 1];
    float vmax[NVT];
    int nonfinite = 0;
#pragma unroll
    for (int j = 0; j < NVT; ++j) {
        const int v = t + j * kBlock;
        const int eb = e0 + v * VEC;
        uint32_t mb = (v < nvec) ? (mw[j] >> (eb & 31)) : 0u;
        if constexpr (!kPacked) mb &= ~(uint32_t)(penbits >> (j * VEC));
        float vm = NEG_INF;
        if constexpr (kPacked) {
            uint32_t wd[4] = {raw[j].x, raw[j].y, raw[j].z, raw[j].w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t m = (((mb >> (2 * i)) & 1u) ? 0x0000FFFFu : 0u) |
                                   (((mb >> (2 * i + 1)) & 1u) ? 0xFFFF0000u : 0u);
                wd[i] = (wd[i] & m) | (Elt<T>::kNegInfWord & ~m);
            }
            xr[j] = make_uint4(wd[0], wd[1], wd[2], wd[3]);
            float f[VEC];
            Elt<T>::widen(xr[j], f);
#pragma unroll
            for (int e = 0; e < VEC; ++e) vm = __builtin_elementwise_maximum(vm, f[e]);
        } else {
            float f[VEC];
            if constexpr (FAST) {
                Elt<T>::widen(raw[j], f);
            } else {
#pragma unroll
                for (int e = 0; e < VEC; ++e) f[e] = sx[j * VEC + e];
            }
#pragma unroll
            for (int e = 0; e < VEC; ++e) {
                // bit e of mb, sign-extended, selects the value or -inf
                const uint32_t sel = (uint32_t)((int)(mb << (31 - e)) >> 31);
                uint32_t bits = (__float_as_uint(f[e]) & sel) | (0xFF800000u & ~sel);
                if constexpr (!FAST) bits = (eb + e < e1) ? bits : 0xFF800000u;
                const float g = __uint_as_float(bits);
                // IEEE maximum (v_maximum3_f32) keeps a NaN, so one class test
                // of the slot maximum finds any NaN or +inf of the slot.
                vm = __builtin_elementwise_maximum(vm, g);
                x[j * VEC + e] = g;
            }
        }
        nonfinite |= __builtin_amdgcn_class(vm, 0x203);   // NaN or +inf
        vmax[j] = vm;
    }
    // The stream values of slot j, widened (masked entries -inf).
    auto slot_vals = [&](int j, float (&f)[VEC]) {
        if constexpr (kPacked) {
            Elt<T>::widen(xr[j], f);
        } else {
#pragma unroll
            for (int e = 0; e < VEC; ++e) f[e] = x[j * VEC + e];
        }
    };

    __builtin_amdgcn_sched_barrier(0);
    TMS_TR(3);
    // ---- row parameters and history window (the parameters' load was issued
    //      before pass 1 and is first waited for here).
    const bool greedy = P.greedy != 0;
    const bool bad_params = !greedy && !(P.temperature > 0.0f && P.temperature <= FLT_MAX);
    const int K = greedy ? 1 : ((P.top_k <= 0 || P.top_k > V) ? V : P.top_k);
    const int mode = greedy ? MODE_GREEDY : (K <= kTopkFast ? MODE_TOPK : MODE_TOPP);
    const float temp = P.temperature;
    const bool divide = !greedy && temp != 1.0f;
    if (t == 0) {
        sm.ncand = 0;
        sm.misc[2] = 0;   // the merger's read found an incomplete list
    }

    // ---- the owned penalised entries: count, mask bit, penalty.
    float xo[kWin];
    uint32_t io[kWin];
#pragma unroll
    for (int i = 0; i < kWin; ++i) {
        xo[i] = NEG_INF;
        io[i] = 0;
        if (own_off[i] >= 0) {
            const int off = own_off[i];
            const uint32_t cnt = (sm.big.cnt[off >> 1] >> ((off & 1) * 16)) & 0xFFFFu;
            const bool allowed = (own_m[i] >> ((e0 + off) & 31)) & 1u;
            float g = allowed ? own_v[i] : NEG_INF;
            nonfinite |= __builtin_amdgcn_class(g, 0x203);
            if (allowed) {
                g = apply_pen(g, cnt, pn);
                nonfinite |= __builtin_amdgcn_class(g, 0x203);
            }
            xo[i] = g;
            io[i] = (uint32_t)(e0 + off);
        }
    }

    // ---- pass 2 (long windows only): history penalties from the counts.
    if constexpr (!kPacked) if (pn.on && !pen_own) {
        // Positions [0, kWin * kBlock) came with the stream; later ones are
        // read now.
        for (int p0 = 0; p0 < nrec; p0 += kBlock * kWin) {
#pragma unroll
            for (int i = 0; i < kWin; ++i) {
                const int p = p0 + t + i * kBlock;
                const int id = (p < from || p >= nrec) ? -1 : (p0 == 0 ? wid[i] : hist[p]);
                if (id >= e0 && id < e1) {
                    const int off = id - e0;
                    const uint32_t add = ovm ? (uint32_t)(p + 1) : 1u;
                    atomicAdd(&sm.big.cnt[off >> 1], add << ((off & 1) * 16));
                }
            }
        }
        lds_sync();
#pragma unroll
        for (int j = 0; j < NVT; ++j) {
            const int v = t + j * kBlock;
            const int off = min(v * VEC, kChunk - VEC);
            uint32_t cw[VEC / 2];
            uint32_t any = 0;
#pragma unroll
            for (int i = 0; i < VEC / 2; ++i) {
                cw[i] = sm.big.cnt[(off >> 1) + i];
                any |= cw[i];
            }
            if (any && v < nvec) {
                float vm = NEG_INF;
#pragma unroll
                for (int e = 0; e < VEC; ++e) {
                    const uint32_t cnt = (cw[e >> 1] >> ((e & 1) * 16)) & 0xFFFFu;
                    float g = x[j * VEC + e];
                    if (cnt) {
                        g = apply_pen(g, cnt, pn);
                        nonfinite |= __builtin_amdgcn_class(g, 0x203);
                        x[j * VEC + e] = g;
                    }
                    vm = fmaxf(vm, g);
                }
                vmax[j] = vm;
            }
        }
    }
    float tmax = vmax[0];
#pragma unroll
    for (int j = 1; j < NVT; ++j) tmax = fmaxf(tmax, vmax[j]);
#pragma unroll
    for (int i = 0; i < kWin; ++i) tmax = fmaxf(tmax, xo[i]);

    TMS_TR(13);
    // ---- selection: the chunk's candidates, sorted, into sm.cand[0..nout).
    int flags = 0;
    int nout = 0;
    if (mode == MODE_GREEDY) {
        // The thread's best stream entry: its largest value and, among the
        // entries equal to it (equal values share a key, -0 and +0 too), the
        // first position, whose id is the lowest (ids grow with j, then e).
        float smax = vmax[0];
#pragma unroll
        for (int j = 1; j < NVT; ++j) smax = fmaxf(smax, vmax[j]);
        int q = 0;
#pragma unroll
        for (int j = NVT - 1; j >= 0; --j) {
            float f[VEC];
            slot_vals(j, f);
#pragma unroll
            for (int e = VEC - 1; e >= 0; --e) q = f[e] == smax ? j * VEC + e : q;
        }
        uint64_t gb = smax != NEG_INF
                          ? ckey(smax, (uint32_t)(e0 + (t + (q / VEC) * kBlock) * VEC + q % VEC))
                          : 0ull;
#pragma unroll
        for (int i = 0; i < kWin; ++i) {
            const uint64_t k = xo[i] != NEG_INF ? ckey(xo[i], io[i]) : 0ull;
            gb = k > gb ? k : gb;
        }
        gb = wave_max_u64_dpp(gb);
        const bool nf = __any(nonfinite != 0);
        if (lane == 0) {
            sm.wave_k[wv] = gb;
            sm.wave_i[wv] = nf;
        }
        lds_sync();
        uint64_t b = sm.wave_k[0];
        int anynf = sm.wave_i[0];
#pragma unroll
        for (int i = 1; i < kWaves; ++i) {
            b = sm.wave_k[i] > b ? sm.wave_k[i] : b;
            anynf |= sm.wave_i[i];
        }
        if (anynf) flags |= FLAG_NONFINITE;
        if (t == 0 && b) sm.cand[0] = b;
        nout = (b && !anynf) ? 1 : 0;
    } else {
        // Threshold thr in v.  top-k: the K-th largest of the 256 thread
        // maxima (K threads hold an entry >= it), found bit by bit on their
        // order keys with ballots.  top-p: the chunk maximum less the
        // significance span, generously, in v.
        const bool nf = __any(nonfinite != 0);
        sm.tkey[t] = okey(tmax);
        if (lane == 0) sm.wave_i[wv] = nf;
        lds_sync();
        int anynf = 0;
#pragma unroll
        for (int i = 0; i < kWaves; ++i) anynf |= sm.wave_i[i];
        if (anynf) flags |= FLAG_NONFINITE;
        const uint4 k4 = ((const uint4*)sm.tkey)[lane];   // 4 keys per lane, all 256
        float thr;
        double lthr = 0.0;
        bool fallback = false;
        if (mode == MODE_TOPK) {
            // Sixteen high bits suffice: `pre` stays a lower bound of the K-th
            // key, and the few extra candidates it admits are ranked away.
            uint32_t pre = 0;
            for (int bit = 31; bit >= 16; --bit) {
                const uint32_t cand = pre | (1u << bit);
                const int cnt = __popcll(__ballot(k4.x >= cand)) + __popcll(__ballot(k4.y >= cand)) +
                                __popcll(__ballot(k4.z >= cand)) + __popcll(__ballot(k4.w >= cand));
                if (cnt >= K) pre = cand;
            }
            // Keys below okey(-FLT_MAX) decode to -inf or NaN: every finite entry.
            thr = pre < 0x00800000u ? -FLT_MAX : okey_inv(pre);
            // Division can merge neighbouring values: lower the threshold to
            // the smallest float with the same quotient, so every entry tying
            // the K-th quotient is a candidate.
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
        } else {
            const uint32_t km = max(max(k4.x, k4.y), max(k4.z, k4.w));
            uint32_t kmax = km;
#pragma unroll
            for (int m = 32; m >= 1; m >>= 1) kmax = max(kmax, (uint32_t)__shfl_xor((int)kmax, m, 64));
            const float cm = okey_inv(kmax);
            const float lmax = divide ? cm / temp : cm;
            lthr = (double)lmax - (double)kSigSpan;
            thr = cm == NEG_INF ? __builtin_huge_valf()
                                : __double2float_rd(((double)lmax - (double)kSigSpan - 1.0 -
                                                     fabs((double)lmax) * 0x1p-20) *
                                                    (double)temp);
            if (thr == NEG_INF) thr = -FLT_MAX;
        }
        TMS_TR(20);
        int n = 0;
        if (!anynf && !bad_params && !fallback) {
            // Each wave compacts its candidates with ballots into its own
            // segment of cand (kCand / kWaves entries), as raw (value, id).
            constexpr int kSeg = kCand / kWaves;
            uint64_t* seg = sm.cand + wv * kSeg;
            int wcnt = 0;
            // Stage 1: each slot whose maximum reaches thr is copied whole
            // (VEC values, then its slot index) into the wave's staging area
            // in sm.big (the window counts are dead now): one ballot per slot.
            // Stage 2: the wave compacts the staged values 64 at a time.  A
            // wave with more than kStage such slots compacts entry by entry.
            constexpr int kStageWords = (int)(sizeof(sm.big) / 4) / kWaves;
            constexpr int kStage = kStageWords / (VEC + 1);
            float* stv = (float*)sm.big.cnt + wv * kStageWords;
            int* sts = (int*)(stv + kStage * VEC);
            int ns = 0;
#pragma unroll
            for (int j = 0; j < NVT; ++j) {
                const bool sj = vmax[j] >= thr;
                const uint64_t m = __ballot(sj);
                if (m) {
                    const int pos = ns + __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                                                   __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
                    if (sj && pos < kStage) {
                        float f[VEC];
                        slot_vals(j, f);
#pragma unroll
                        for (int e = 0; e < VEC; e += 4)
                            *(float4*)(stv + pos * VEC + e) = make_float4(f[e], f[e + 1], f[e + 2], f[e + 3]);
                        sts[pos] = t + j * kBlock;
                    }
                    ns += __popcll(m);
                }
            }
            if (ns <= kStage) {
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                const int total = ns * VEC;
                for (int b = 0; b < total; b += 64) {
                    const int i = b + lane;
                    const int ic = min(i, total - 1);
                    const float f = i < total ? stv[ic] : NEG_INF;
                    const uint32_t id = (uint32_t)(e0 + sts[ic / VEC] * VEC + ic % VEC);
                    const bool p = f >= thr;
                    const uint64_t m = __ballot(p);
                    const int pos = wcnt + __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                                                     __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
                    if (p && pos < kSeg) seg[pos] = ((uint64_t)__float_as_uint(f) << 32) | id;
                    wcnt += __popcll(m);
                }
            } else {
#pragma unroll
                for (int j = 0; j < NVT; ++j) {
                    if (__any(vmax[j] >= thr)) {
                        float fv[VEC];
                        slot_vals(j, fv);
#pragma unroll
                        for (int e = 0; e < VEC; ++e) {
                            const float f = fv[e];
                            const bool p = f >= thr;
                            const uint64_t m = __ballot(p);
                            if (m) {
                                const int pos = wcnt + __builtin_amdgcn_mbcnt_hi(
                                                           (uint32_t)(m >> 32),
                                                           __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
                                if (p && pos < kSeg)
                                    seg[pos] = ((uint64_t)__float_as_uint(f) << 32) |
                                               (uint32_t)(e0 + (t + j * kBlock) * VEC + e);
                                wcnt += __popcll(m);
                            }
                        }
                    }
                }
            }
#pragma unroll
            for (int i = 0; i < kWin; ++i) {
                const bool p = xo[i] >= thr;
                const uint64_t m = __ballot(p);
                if (m) {
                    const int pos = wcnt + __builtin_amdgcn_mbcnt_hi(
                                               (uint32_t)(m >> 32),
                                               __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
                    if (p && pos < kSeg) seg[pos] = ((uint64_t)__float_as_uint(xo[i]) << 32) | io[i];
                    wcnt += __popcll(m);
                }
            }
            if (lane == 0) sm.wave_i[wv] = wcnt;
            lds_sync();
            int cw[kWaves];
            int over = 0;
            n = 0;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) {
                cw[w] = sm.wave_i[w];
                over |= cw[w] > kSeg;
                n += cw[w];
            }
            if (over) {
                // A wave's segment overflowed: compact again, contiguously.
                if (t == 0) {
        sm.ncand = 0;
        sm.misc[2] = 0;   // the merger's read found an incomplete list
    }
                lds_sync();
#pragma unroll
                for (int j = 0; j < NVT; ++j) {
                    if (vmax[j] >= thr) {
                        float fv[VEC];
                        slot_vals(j, fv);
#pragma unroll
                        for (int e = 0; e < VEC; ++e) {
                            const float f = fv[e];
                            if (f >= thr) {
                                const int pos = atomicAdd(&sm.ncand, 1);
                                if (pos < kCand)
                                    sm.cand[pos] = ((uint64_t)__float_as_uint(f) << 32) |
                                                   (uint32_t)(e0 + (t + j * kBlock) * VEC + e);
                            }
                        }
                    }
                }
#pragma unroll
                for (int i = 0; i < kWin; ++i) {
                    if (xo[i] >= thr) {
                        const int pos = atomicAdd(&sm.ncand, 1);
                        if (pos < kCand) sm.cand[pos] = ((uint64_t)__float_as_uint(xo[i]) << 32) | io[i];
                    }
                }
                lds_sync();
                n = sm.ncand;
                cw[0] = n;
#pragma unroll
                for (int w = 1; w < kWaves; ++w) cw[w] = 0;
            }
            TMS_TR(21);
            // The raw candidate i, divided: its key (value, id) and whether
            // a top-p row keeps it (within the exact span).
            auto cand_key = [&](int i, bool& keepit) {
                // the wave segment holding i (static indices into cw)
                int w = 0, base_i = 0, acc = 0;
#pragma unroll
                for (int u = 0; u < kWaves - 1; ++u) {
                    acc += cw[u];
                    if (i >= acc) {
                        w = u + 1;
                        base_i = acc;
                    }
                }
                const uint64_t rw = sm.cand[(over ? 0 : w * kSeg) + (i - base_i)];
                const float f = __uint_as_float((uint32_t)(rw >> 32));
                const uint32_t id = (uint32_t)rw;
                const float lg = divide ? f / temp : f;
                keepit = mode == MODE_TOPK || (double)lg >= lthr;
                return ckey(lg, id);
            };
            if (n <= kCand && mode == MODE_TOPP) {
                // Top-p lists are merged whole and ranked by the merger, so
                // the chunk only compacts the kept keys into cand, in
                // candidate order (two candidates a thread at most).
                static_assert(kCand <= 2 * kBlock, "two candidates a thread");
                bool kp0 = false, kp1 = false;
                const uint64_t kk0 = t < n ? cand_key(t, kp0) : 0ull;
                const uint64_t kk1 = t + kBlock < n ? cand_key(t + kBlock, kp1) : 0ull;
                kp0 = kp0 && t < n;
                kp1 = kp1 && t + kBlock < n;
                const uint64_t bm0 = __ballot(kp0), bm1 = __ballot(kp1);
                if (lane == 0) {
                    sm.list_src[wv] = __popcll(bm0);
                    sm.list_src[kWaves + wv] = __popcll(bm1);
                }
                lds_sync();   // every raw candidate read, every wave counted
                TMS_TR(17);
                TMS_TV(19, n + 1);
                int off0 = 0, off1 = 0;
                nout = 0;
#pragma unroll
                for (int w = 0; w < kWaves; ++w) {
                    const int c0 = sm.list_src[w], c1 = sm.list_src[kWaves + w];
                    off0 += w < wv ? c0 : 0;
                    off1 += w < wv ? c1 : 0;
                    nout += c0;
                }
                off1 += nout;
#pragma unroll
                for (int w = 0; w < kWaves; ++w) nout += sm.list_src[kWaves + w];
                if (kp0)
                    sm.cand[off0 + __builtin_amdgcn_mbcnt_hi((uint32_t)(bm0 >> 32),
                                                             __builtin_amdgcn_mbcnt_lo((uint32_t)bm0, 0u))] = kk0;
                if (kp1)
                    sm.cand[off1 + __builtin_amdgcn_mbcnt_hi((uint32_t)(bm1 >> 32),
                                                             __builtin_amdgcn_mbcnt_lo((uint32_t)bm1, 0u))] = kk1;
                lds_sync();
                TMS_TR(18);
            } else if (n <= kCand) {
                // Top-k: the candidates' keys contiguously in uni (the window
                // counts are dead now), then ranked by counting into cand.
                uint64_t* keys = sm.big.m.uni;
                for (int i = t; i < n; i += kBlock) {
                    bool keepit;
                    keys[i] = cand_key(i, keepit);
                }
                lds_sync();
                TMS_TR(17);
                TMS_TV(19, n + 1);
                nout = n < K ? n : K;
                rank_all(keys, n, sm.cand);
                lds_sync();
                TMS_TR(18);
            }
        }
        if (!anynf && !bad_params && (fallback || n > kCand)) {
            if (mode == MODE_TOPK) {
                if (pn.on) {
                    // The candidate staging wrote over the window counts in
                    // sm.big; the radix select reads the penalised values
                    // through them, so they are counted again.
                    uint4* c4 = (uint4*)sm.big.cnt;
                    lds_sync();
                    for (int i = t; i < kChunk / 8; i += kBlock) c4[i] = make_uint4(0, 0, 0, 0);
                    lds_sync();
                    for (int p = from + t; p < nrec; p += kBlock) {
                        const int id = hist[p];
                        if (id >= e0 && id < e1) {
                            const int off = id - e0;
                            const uint32_t add = ovm ? (uint32_t)(p + 1) : 1u;
                            atomicAdd(&sm.big.cnt[off >> 1], add << ((off & 1) * 16));
                        }
                    }
                    lds_sync();
                }
                nout = radix_slow<T>(base, mrow, e0, e1, K, temp, divide, pn.on, pn.rep_on, pn.fp_on, pn.rep,
                                     pn.freq, pn.pres, pn.ov, sm);
                [[clang::always_inline]] sort_cand(nout, sm);
            } else {
                flags |= FLAG_OVERFLOW;
                nout = 0;
            }
        }
    }

    TMS_TR(4);
    // ---- publish, then take a ticket: the row's last workgroup to publish
    //      merges, and every other list is complete by then.
    // Header and entries are stored together and complete before the
    // ticket, so a reader that reads after its own ticket sees them all.
    // The merger reads the first r entries of every list at once (top-k and
    // greedy rows); slots past nout hold key 1, below every real key, so
    // every word it reads is non-zero once written.  That read is issued
    // with the ticket, before the ticket tells whether this workgroup
    // merges: it may see a list still in flight, which the merger checks
    // word by word and reads again.
    const int r = (mode == MODE_TOPP || S > kRankLists) ? 0 : min(K, kUni / S - 1);
    const int R1 = r + 1;   // words per list in uni: header, r entries
    const bool spec = r > 0;
    const uint64_t hdr = kReady | ((uint64_t)flags << 32) | (uint64_t)(uint32_t)nout;
    uint64_t* row_lists = a.lists + (int64_t)row * S * kListStride;
    if (wv == 0) {
        uint64_t* my_list = row_lists + (int64_t)c * kListStride;
        for (int i = lane; i <= max(nout, r); i += 64)
            st_agent(&my_list[i], i == 0 ? hdr : (i <= nout ? sm.cand[i - 1] : (uint64_t)1));
        __builtin_amdgcn_s_waitcnt(0);   // the list is complete before the ticket
    }
    lds_sync();
    // Waves 1-3 read; wave 0 takes the ticket alone (a wave's loads return
    // in order, so its own loads would hold the ticket back).
    constexpr int kSpecThreads = kBlock - 64;
    constexpr int kSpecPer = (kUni + kSpecThreads - 1) / kSpecThreads;
    const int ts = t - 64;
    uint64_t sp[kSpecPer];
#pragma unroll
    for (int u = 0; u < kSpecPer; ++u) {
        const int idx = ts + u * kSpecThreads;
        sp[u] = 0;
        if (spec && wv != 0 && idx < S * R1) {
            const int cc = idx / R1;
            if (cc != c) sp[u] = ld_agent(&row_lists[(int64_t)cc * kListStride + (idx - cc * R1)]);
        }
    }
    if (t == 0) {
        const uint32_t ticket = __hip_atomic_fetch_add(&a.counters[row * kCounterStride], 1u, __ATOMIC_RELAXED,
                                                       __HIP_MEMORY_SCOPE_AGENT);
        sm.misc[0] = ticket == (uint32_t)(S - 1) ? 1 : 0;
    }
    lds_sync();
    if (!sm.misc[0]) return;
    TMS_TR(5);
    // The row's draw words, formed while the lists are read.
    uint32_t rw0 = 0, rw1 = 0;

    // ================= merge: the last workgroup of the row =================
    // Top-k rows took each list's header and first r entries (r = K where
    // it fits) with the ticket.  A header not yet ready or an entry still 0
    // (the merger of the previous call zeroed every word it consumed; keys
    // are never 0) is read again, boundedly.  The K best of the sample are
    // the row's K best unless some list's last sampled entry is among them
    // while the list holds more; only then, and for top-p rows, are whole
    // lists merged.
    if (t == 64) st_agent(&a.counters[row * kCounterStride], 0u);   // ready for the next launch (wave 0 keeps no store in flight)
    uint64_t* uni = sm.big.m.uni;
    if (t == 0) {
        sm.theta = 0;     // lists to read again (bit per list)
        sm.misc[3] = 0;   // a list never arrived
    }
    uint64_t* srt = sm.big.m.surv;
    const int RL = stage_log2(S), RT = 1 << RL;   // staged words per list (whole lists)
    uint64_t hv[kUni / kBlock];
    if (spec) {
        if (mode != MODE_GREEDY) row_uniform(a, row, P, rw0, rw1);
        // Every word read must be set: a ready header, non-zero entries (the
        // writer padded its r slots).  Each thread checks its own words.
        int bad = 0;
#pragma unroll
        for (int u = 0; u < kSpecPer; ++u) {
            const int idx = ts + u * kSpecThreads;
            if (wv != 0 && idx < S * R1) {
                const int cc = idx / R1, jj = idx - cc * R1;
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
        // re-reads their sampled entries at once.
        for (int round = 0; sm.misc[2]; ++round) {
            for (int idx = t; idx < S * R1; idx += kBlock) {
                const int cc = idx / R1, jj = idx - cc * R1;
                const uint64_t h = uni[cc * R1];
                const int m = min((int)(uint32_t)h, r);
                if (!(h & kReady) || (jj >= 1 && jj <= m && uni[idx] == 0))
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
            for (int idx = t; idx < S * R1; idx += kBlock) {
                const int cc = idx / R1, jj = idx - cc * R1;
                if (jj == 0 || !((redo >> cc) & 1)) continue;
                if (jj <= min((int)(uint32_t)uni[cc * R1], r))
                    uni[idx] = ld_agent(&row_lists[(int64_t)cc * kListStride + jj]);
            }
            lds_sync();
        }
    } else {
        // Whole lists (top-p rows, top-k rows over many lists): every
        // list's header and first RT - 1 entries in one round of loads, all
        // issued before any is used, kept in registers (hv); the headers go
        // to srt (free until a merge ranks into it).  When every list fits,
        // its entries are stored packed and ranked; otherwise the merge
        // rounds below read the lists again.
#pragma unroll
        for (int u = 0; u < kUni / kBlock; ++u) {
            const int idx = t + u * kBlock;
            const int cc = idx >> RL, jj = idx & (RT - 1);
            hv[u] = (cc < S && cc != c) ? ld_agent(&row_lists[(int64_t)cc * kListStride + jj]) : 0ull;
            if (cc == c) hv[u] = jj == 0 ? hdr : (jj <= nout ? sm.cand[jj - 1] : 0ull);
        }
        if (mode != MODE_GREEDY) row_uniform(a, row, P, rw0, rw1);
#pragma unroll
        for (int u = 0; u < kUni / kBlock; ++u) {
            const int idx = t + u * kBlock;
            const int cc = idx >> RL, jj = idx & (RT - 1);
            if (cc < S && jj == 0) srt[cc] = hv[u];
        }
        lds_sync();
    }
    uint64_t* hdrs = spec ? uni : srt;   // the headers, stride HW
    const int HW = spec ? R1 : 1;
    if (wv == 0) {
        // Whole-list mode: wait (bounded) for the headers not yet ready
        // (read from srt after the barrier above; one wave, no atomics).
        const uint64_t redo = spec ? 0ull : __ballot(lane < S && !(hdrs[lane] & kReady));
        if (lane < S && ((redo >> lane) & 1)) {
            uint64_t h = 0;
            for (int it = 0; it < kPollCap; ++it) {
                h = ld_agent(&row_lists[(int64_t)lane * kListStride]);
                if (h & kReady) break;
                __builtin_amdgcn_s_sleep(1);
            }
            hdrs[lane * HW] = h;
            if (!(h & kReady)) sm.misc[3] = 1;
        }
        int n_c = 0, f_c = 0, m_c = 0;
        if (lane < S) {
            const uint64_t h = hdrs[lane * HW];
            n_c = (int)(uint32_t)h;
            f_c = (int)((h >> 32) & 0xFF);
            m_c = min(n_c, r);
            sm.list_n[lane] = n_c;
            sm.list_s[lane] = m_c;
        }
        const int incl = wave_incl_scan_i32(n_c);
        const int N = __shfl(incl, 63, 64);
        int fo = f_c;
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) fo |= __shfl_xor(fo, m, 64);
        // Staged whole lists are ranked in place when no header was read
        // again and every list fits its staged words.
        const bool fits = lane >= S || n_c <= RT - 1;
        const bool staged = !spec && redo == 0 && __ballot(!fits) == 0ull;
        if (lane < S) sm.hist[lane] = incl - n_c;   // packed offset of each list
        if (lane == 0) {
            sm.misc[5] = N;
            sm.misc[4] = fo;
            sm.misc[1] = 0;   // "a list ran out"
            sm.misc[6] = staged;
        }
    }
    lds_sync();
    TMS_TR(6);
    const int N = sm.misc[5];
    const int fo = sm.misc[4];
    int status = TMS_ROW_OK;
    if (sm.misc[3]) status = TMS_ROW_INTERNAL;
    else if (hist_over) status = TMS_ROW_UNSUPPORTED;
    else if (bad_params) status = TMS_ROW_BAD_PARAMS;
    else if (fo & FLAG_NONFINITE) status = TMS_ROW_NONFINITE;
    else if (N == 0 && !(fo & FLAG_OVERFLOW)) status = TMS_ROW_ALL_MASKED;   // an overflowed list holds 0
    // Top-p rows whose lists overflowed, or whose top min(N, K) exceed the
    // merge capacity, take the whole-row path (tms_dense.h).
    const bool go_dense = status == TMS_ROW_OK && mode == MODE_TOPP &&
                          ((fo & FLAG_OVERFLOW) || min(N, K) > kToppCap);

    int n_acc = 0;
    bool full = !spec;
    if (status == TMS_ROW_OK && spec) {
        // Prune with a lower bound tau on the row's K-th key: the largest
        // K-th entry of any list (that list alone holds K keys >= it), or
        // the smallest m-th entry over all lists, m = ceil(K / S) (the S
        // lists hold S * m >= K keys >= it).  Only keys >= tau can rank
        // below K, and every key larger than one of them is >= tau too, so
        // counting within that set ranks it exactly.
        n_acc = min(N, K);
        if (wv == 0) {
            const int m = (K + S - 1) / S;
            const int ls = lane < S ? sm.list_s[lane] : 0;
            const uint64_t kth = (lane < S && ls >= K) ? uni[lane * R1 + K] : 0ull;
            const uint64_t mth = lane >= S ? ~0ull : (ls >= m ? uni[lane * R1 + m] : 0ull);
            const uint64_t tau = max(wave_max_u64_dpp(kth), ~wave_max_u64_dpp(~mth));
            // Each sorted list's keys >= tau are a prefix: its length by
            // binary search, its place among the candidates by a scan.
            int p = 0;
            if (lane < S) {
                int hi = ls;
                while (p < hi) {
                    const int mid = (p + hi) >> 1;
                    if (uni[lane * R1 + 1 + mid] >= tau) p = mid + 1;
                    else hi = mid;
                }
            }
            const int incl = wave_incl_scan_i32(p);
            const int tot = __shfl(incl, 63, 64);
            if (lane < S && tot <= kCand) {
                // Copy the prefix into cand.  A list whose whole sample is
                // in (only possible when fewer than K entries were sampled)
                // while it holds more sends the row to the whole-list merge.
#pragma unroll 4
                for (int j = 0; j < p; ++j) sm.cand[incl - p + j] = uni[lane * R1 + 1 + j];
                if (r < K && p == ls && sm.list_n[lane] > ls) sm.misc[1] = 1;
            }
            if (lane == 0) {
                sm.ncand = tot;
                if (tot > kCand) sm.misc[1] = 1;   // rare (a weak tau): whole lists below
            }
        }
        lds_sync();
        const int nc = sm.ncand;
        if (nc <= kCand) {
            // Zero-pad to a multiple of 8 (keys are never 0), then count in
            // blocks of eight keys read 16 bytes at a time.
            if (t < 8 && nc + t < kCand) sm.cand[nc + t] = 0ull;
            lds_sync();
            const uint4* c4 = (const uint4*)sm.cand;
            for (int i = t; i < nc; i += kBlock) {
                const uint64_t k = sm.cand[i];
                int r0 = 0, r1 = 0;
                for (int j = 0; j < nc; j += 8) {
                    uint4 q[4];
#pragma unroll
                    for (int u = 0; u < 4; ++u) q[u] = c4[(j >> 1) + u];
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        r0 += (((uint64_t)q[u].y << 32) | q[u].x) > k ? 1 : 0;
                        r1 += (((uint64_t)q[u].w << 32) | q[u].z) > k ? 1 : 0;
                    }
                }
                if (r0 + r1 < n_acc) srt[r0 + r1] = k;
            }
        }
        lds_sync();
        full = sm.misc[1] != 0;
    }
    const int keep_cap = mode == MODE_TOPP ? min(kToppCap, K) : K;
    bool merged = false, zeroed = false;
    if (status == TMS_ROW_OK && !spec && !go_dense && sm.misc[6]) {
        // The staged lists, packed in list order into uni; a word inside a
        // list that still reads 0 sends the row to the merge rounds.
        int bad = 0;
#pragma unroll
        for (int u = 0; u < kUni / kBlock; ++u) {
            const int idx = t + u * kBlock;
            const int cc = idx >> RL, jj = idx & (RT - 1);
            if (cc < S && jj >= 1 && jj <= sm.list_n[cc]) {
                bad |= hv[u] == 0ull;
                uni[sm.hist[cc] + jj - 1] = hv[u];
            }
        }
        if (__ballot(bad) && lane == 0) atomicOr(&sm.misc[2], 1);
        lds_sync();
        TMS_TR(11);
        if (!sm.misc[2]) {
            // Every word read is consumed: back to zero for the next call
            // now (the stores complete under the rank and the tail).
#pragma unroll
            for (int u = 0; u < kUni / kBlock; ++u) {
                const int idx = t + u * kBlock;
                const int cc = idx >> RL, jj = idx & (RT - 1);
                if (cc < S && jj <= sm.list_n[cc]) st_agent(&row_lists[(int64_t)cc * kListStride + jj], (uint64_t)0);
            }
            zeroed = true;
            n_acc = min(N, keep_cap);
            if (N <= 2 * kBlock) {
                [[clang::always_inline]] bucket_rank<2>(uni, N, n_acc, srt, (int*)sm.pbits, sm);
            } else if (N <= 4 * kBlock) {
                bucket_rank<4>(uni, N, n_acc, srt, (int*)sm.pbits, sm);
            } else {
                bucket_rank<kUni / kBlock>(uni, N, n_acc, srt, (int*)sm.pbits, sm);
            }
            merged = true;
            lds_sync();
            TMS_TR(12);
        }
    }
    if (status == TMS_ROW_OK && full && !go_dense && !merged) {
        // Whole lists, in rounds: the running top list (surv[0..n_acc)) plus
        // as many chunk lists as fit in kUni, ranked by binary search against
        // each other.  Top-k rows read at most K entries a list.
        if (t < S) sm.list_s[t] = mode == MODE_TOPP ? sm.list_n[t] : min(sm.list_n[t], K);
        n_acc = 0;
        int c_next = 0;
        lds_sync();
        while (c_next < S) {
            if (t == 0) {
                int off = n_acc, g = 1, cc = c_next;
                sm.hist[0] = 0;   // this round's list offsets
                sm.hist[1] = n_acc;
                sm.list_src[0] = -1;
                while (cc < S && off + sm.list_s[cc] <= kUni) {
                    off += sm.list_s[cc];
                    sm.list_src[g] = cc;
                    sm.hist[++g] = off;
                    ++cc;
                }
                sm.misc[6] = g;
                sm.misc[7] = cc;
            }
            lds_sync();
            const int ng = sm.misc[6];
            const int total = sm.hist[ng];
            // The list of staged entry i: the last g >= 1 whose start is at
            // or below i (independent reads, not a dependent walk).
            auto list_of = [&](int i) {
                int lc = 0;
                for (int g = 1; g < ng; ++g) lc += sm.hist[g] <= i ? 1 : 0;
                return lc;
            };
            for (int i = t; i < total; i += kBlock) {
                const int lc = list_of(i);
                const int src = sm.list_src[lc];
                const int jj = i - sm.hist[lc];
                uni[i] = src < 0 ? srt[i]
                         : (src == c ? sm.cand[jj]
                                     : ld_agent(&row_lists[(int64_t)src * kListStride + 1 + jj]));
            }
            lds_sync();
            TMS_TR(11);
            const int nkeep = total < keep_cap ? total : keep_cap;
            // The staged lists' keys ranked together (the bucket counts go
            // to pbits, dead since the chunk phase).
            if (total <= 2 * kBlock) {
                [[clang::always_inline]] bucket_rank<2>(uni, total, nkeep, srt, (int*)sm.pbits, sm);
            } else {
                bucket_rank<kUni / kBlock>(uni, total, nkeep, srt, (int*)sm.pbits, sm);
            }
            TMS_TR(12);
            c_next = sm.misc[7];
            n_acc = nkeep;
            lds_sync();
        }
    }
    // Every word the other chunks wrote this call (headers, entries) goes
    // back to zero for the next call; on a top-k or top-p row's success path
    // waves 1-3 do it while wave 0 runs the tail.
    TMS_TR(9);
    const bool defer_zero = status == TMS_ROW_OK && (mode == MODE_TOPK || (mode == MODE_TOPP && !go_dense)) &&
                            !sm.misc[3];
    if (!defer_zero && !sm.misc[3] && !zeroed) zero_lists(row_lists, S, r, sm.list_n, t, kBlock);
    TMS_TR(10);
    if (status != TMS_ROW_OK) {
        write_row_error(a, row, status);
        return;
    }
    // One place runs the whole-row path (the lists are done with): rows
    // that need it from the start, and top-p rows whose answer turns out to
    // need the order past the held entries.
    bool whole = go_dense;
    if (!go_dense) {
        if (mode == MODE_GREEDY) {
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
        if (mode == MODE_TOPK && N < K) {
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
        TMS_TR(7);
        const float mx = ckey_val(srt[0]);
        if (mx == __builtin_huge_valf()) {
            if (defer_zero && !zeroed) zero_lists(row_lists, S, r, sm.list_n, t, kBlock);
            write_row_error(a, row, TMS_ROW_NONFINITE);
            return;
        }
        if (mode == MODE_TOPK) {
            if (wv == 0) {
                [[clang::always_inline]] tail_topk(a, row, P, srt, n, K, (double*)sm.big.m.uni, (double*)sm.cand, rw0, rw1);
            }
            else if (!zeroed)
                zero_lists(row_lists, S, r, sm.list_n, t - 64, kBlock - 64);
            return;
        }
        // Top-p rows: only the prefix within kSigSpan of the maximum is exact.
        // The count of that prefix and every held entry's pr in one pass (pr
        // past the prefix is never read).
        double* pr = (double*)sm.big.m.uni;               // staging no longer needed
        double* q = (double*)(sm.big.m.surv + kToppCap);  // past the sorted entries
        {
            int sig = 0;
            for (int i = t; i < n; i += kBlock) {
                const double d = (double)ckey_val(srt[i]) - (double)mx;
                sig += d >= -(double)kSigSpan ? 1 : 0;
                pr[i] = exp(d);
            }
            sig = wave_sum_dpp(sig);
            if (lane == 0) sm.wave_i[wv] = sig;
            if (t == 0) sm.nvalid = 0;
            lds_sync();
            n = sm.wave_i[0] + sm.wave_i[1] + sm.wave_i[2] + sm.wave_i[3];
            n = min(n, K);   // tmsample::sample sums over the top K only (tmsample.h:185-191)
        }
        TMS_TR(14);
        const int tp = tail_topp_block(a, row, P, srt, n, K, pr, q, rw0, rw1, sm);
        TMS_TR(15);
        if (tp == 2) {
            // the sequential tail decides (or returns the probabilities)
            if (wv == 0) {
                TMS_TV(16, 1);
                bool lost;
                [[clang::always_inline]] lost = tail_topp(a, row, P, srt, n, K, pr, q);
                if (lane == 0) sm.nvalid = lost;
            } else if (!zeroed) {
                zero_lists(row_lists, S, r, sm.list_n, t - 64, kBlock - 64);
            }
        } else {
            if (t == 0) sm.nvalid = tp;
            if (!zeroed) zero_lists(row_lists, S, r, sm.list_n, t, kBlock);
        }
        TMS_TR(8);
        lds_sync();
        whole = sm.nvalid != 0;
    }
    if (__builtin_expect(whole, 0)) {
        [[clang::always_inline]] dense_inline<T>(a, row, *reinterpret_cast<DenseLds*>(&sm.big));
    }
}

}  // namespace tms

// ============================================================== C ABI


extern "C" int tms_abi_version(void) { return TMS_ABI_VERSION; }

#ifdef TMS_TRACE
// Trace-only builds: the buffer the kernels stamp (24 slots per wave).
static uint64_t* g_tms_trace_host;
extern "C" int tms_trace_set(uint64_t* buf) {
    g_tms_trace_host = buf;
    return 0;
}
#endif

extern "C" const char* tms_status_string(int code) {
    switch (code) {
        case TMS_OK: return "ok";
        case TMS_ERR_INVALID_ARG: return "invalid argument";
        case TMS_ERR_CAPACITY: return "batch or vocab above the context capacity";
        case TMS_ERR_HIP: return "HIP runtime error";
        case TMS_ERR_NO_DEVICE: return "no HIP device";
        default: return "unknown";
    }
}

static int chunks_for(int V) { return (V + tms::kChunk - 1) / tms::kChunk; }

extern "C" int tms_create(int device, int max_batch, int max_vocab, tms_context** out) {
    if (!out || max_batch <= 0 || max_vocab <= 0 ||
        max_vocab > tms::kMaxChunks * tms::kChunk)
        return TMS_ERR_INVALID_ARG;
    *out = nullptr;
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev <= 0) return TMS_ERR_NO_DEVICE;
    if (device < 0 || device >= ndev) return TMS_ERR_INVALID_ARG;
    int prev = 0;
    if (hipGetDevice(&prev) != hipSuccess) return TMS_ERR_HIP;
    if (hipSetDevice(device) != hipSuccess) return TMS_ERR_HIP;
    tms_context* ctx = new tms_context{};
    ctx->device = device;
    ctx->max_batch = max_batch;
    ctx->max_vocab = max_vocab;
    ctx->max_chunks = chunks_for(max_vocab);
    const size_t nb = (size_t)max_batch;
    const size_t nc = nb * (size_t)ctx->max_chunks;
    const size_t ones_words = ((size_t)max_vocab + 31) / 32;
    const size_t off_ones = nb * tms::kCounterStride * 4;   // one 256-byte line per row counter
    const size_t off_l = off_ones + 256 * ((ones_words * 4 + 255) / 256);
    const size_t off_st = off_l + nc * tms::kListStride * sizeof(uint64_t);
    const size_t off_sp = off_st + nb * tms::kCounterStride * 4;   // one 256-byte line per ticket
    const size_t off_ss = off_sp + nb * tms::kSpecParts * tms::kPartWords * sizeof(uint64_t);
    const size_t off_tl = off_ss + nb * (2 * tms::kSpecMaxK + 1) * sizeof(tms_spec_stat);
    const size_t tl_chunks = (size_t)std::min(ctx->max_chunks, tms::kWideMaxChunksHost);
    const size_t off_dq = off_tl + nb * tl_chunks * tms::kWideListStride * sizeof(uint64_t);
    const size_t off_hn = off_dq + 256 * (((size_t)tms::kDenseSlotsMax * sizeof(uint32_t) + 255) / 256);
    const size_t off_hi = off_hn + 256 * ((nb * sizeof(int32_t) + 255) / 256);
    const size_t off_hv = off_hi + nb * tms::kHistMax * sizeof(int32_t);
    ctx->bytes = off_hv + nb * tms::kHistMax * sizeof(float);
    int rc = TMS_OK;
    if (hipMalloc(&ctx->ws, ctx->bytes) != hipSuccess) rc = TMS_ERR_HIP;
    else if (hipMemset(ctx->ws, 0, ctx->bytes) != hipSuccess) rc = TMS_ERR_HIP;   // lists start zeroed
    else if (hipMemset((char*)ctx->ws + off_ones, 0xFF, ones_words * 4) != hipSuccess) rc = TMS_ERR_HIP;
    else if (hipDeviceSynchronize() != hipSuccess) rc = TMS_ERR_HIP;
    // The whole-row path's region: never read before it is written, so not
    // cleared.
    ctx->dense_slots = std::min(max_batch, tms::kDenseSlotsMax);
    ctx->dense_bytes = (size_t)ctx->dense_slots * 2 * (size_t)max_vocab * sizeof(uint64_t);
    if (rc == TMS_OK && hipMalloc(&ctx->dense, ctx->dense_bytes) != hipSuccess) {
        ctx->dense = nullptr;
        rc = TMS_ERR_HIP;
    }
    if (rc != TMS_OK) {
        if (ctx->ws) (void)hipFree(ctx->ws);
        delete ctx;
        (void)hipSetDevice(prev);
        return rc;
    }
    char* p = (char*)ctx->ws;
    ctx->counters = (uint32_t*)p;
    ctx->ones = (uint32_t*)(p + off_ones);
    ctx->lists = (uint64_t*)(p + off_l);
    ctx->spec_tickets = (uint32_t*)(p + off_st);
    ctx->spec_parts = (uint64_t*)(p + off_sp);
    ctx->spec_stats = (tms_spec_stat*)(p + off_ss);
    ctx->tlists = (uint64_t*)(p + off_tl);
    ctx->dlocks = (uint32_t*)(p + off_dq);
    ctx->ov_n = (int32_t*)(p + off_hn);
    ctx->ov_ids = (int32_t*)(p + off_hi);
    ctx->ov_vals = (float*)(p + off_hv);
    ctx->ones_begin = off_ones;
    ctx->ones_end = off_l;
    (void)hipSetDevice(prev);
    *out = ctx;
    return TMS_OK;
}

extern "C" int tms_destroy(tms_context* ctx) {
    if (!ctx) return TMS_ERR_INVALID_ARG;
    int prev = 0;
    (void)hipGetDevice(&prev);
    (void)hipSetDevice(ctx->device);
    hipError_t e = hipFree(ctx->ws);
    if (ctx->dense && hipFree(ctx->dense) != hipSuccess) e = hipErrorUnknown;
    (void)hipSetDevice(prev);
    delete ctx;
    return e == hipSuccess ? TMS_OK : TMS_ERR_HIP;
}

extern "C" size_t tms_workspace_bytes(const tms_context* ctx) {
    return ctx ? ctx->bytes + ctx->dense_bytes : 0;
}

// Zero every workspace word the cross-workgroup protocols expect at zero
// (counters, tickets, list and part words, the region locks), keeping the all-ones
// mask row.  For recovery after a TMS_ROW_INTERNAL row, whose late words
// may otherwise be taken as the next call's.
static int reset_regions(void* ws, size_t ones_begin, size_t ones_end, size_t bytes, hipStream_t stream) {
    if (hipMemsetAsync(ws, 0, ones_begin, stream) != hipSuccess) return TMS_ERR_HIP;
    if (hipMemsetAsync((char*)ws + ones_end, 0, bytes - ones_end, stream) != hipSuccess) return TMS_ERR_HIP;
    return TMS_OK;
}

// Compute units of the current device (looked up once per device).
static int device_cus() {
    constexpr int kMaxDevices = 64;
    static std::atomic<int> cus[kMaxDevices];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 0;
    int n = cus[dev].load(std::memory_order_relaxed);
    if (n == 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
        cus[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

// The workspace regions one sampling call uses, and their capacities.
struct SampleWs {
    int max_batch, max_vocab;
    uint32_t* counters;
    uint32_t* ones;
    uint64_t* lists;
    uint64_t* tlists;
    uint32_t* dlocks;
    uint64_t* dense;
    int dense_slots;
    int32_t* ov_n;         // the history pre-pass's lists
    int32_t* ov_ids;
    float* ov_vals;
};

// tms_sample_batch over workspace w (a context's, or the allocation-free
// entry point's static one).
static int sample_launch(const SampleWs& w, const tms_sample_args* a, hipStream_t stream) {
    if (!a || !a->logits || !a->params || !a->out_tokens || !a->out_status)
        return TMS_ERR_INVALID_ARG;
    if (a->batch <= 0 || a->vocab <= 0 || a->row_stride < a->vocab) return TMS_ERR_INVALID_ARG;
    if (a->batch > w.max_batch || a->vocab > w.max_vocab) return TMS_ERR_CAPACITY;
    if (a->mask && a->mask_stride < (a->vocab + 31) / 32) return TMS_ERR_INVALID_ARG;
    // Window counts are 16-bit per id in LDS.
    if (a->recent && (a->recent_stride <= 0 || a->recent_stride > 65535)) return TMS_ERR_INVALID_ARG;
    if ((a->out_topk_ids || a->out_topk_probs) && a->topk_cap <= 0) return TMS_ERR_INVALID_ARG;
    if (a->row_kinds != TMS_ROWS_ANY && a->row_kinds != TMS_ROWS_TOPK && a->row_kinds != TMS_ROWS_SPARSE_MASK)
        return TMS_ERR_INVALID_ARG;
    int esz;
    switch (a->dtype) {
        case TMS_DTYPE_F32: esz = 4; break;
        case TMS_DTYPE_F16:
        case TMS_DTYPE_BF16: esz = 2; break;
        default: return TMS_ERR_INVALID_ARG;
    }
    const int vec = 16 / esz;
    tms::KArgs k{};
    k.logits = a->logits;
    k.row_stride = a->row_stride;
    k.V = a->vocab;
    k.S = chunks_for(a->vocab);
    const int per = (a->vocab + k.S - 1) / k.S;
    k.CE = (per + vec - 1) / vec * vec;
    const bool fast = ((uintptr_t)a->logits % 16 == 0) && ((a->row_stride * esz) % 16 == 0) &&
                      (a->vocab % vec == 0);
    k.params = a->params;
    k.recent = a->recent;
    k.n_recent = a->n_recent;
    k.recent_stride = a->recent_stride;
    k.mask = a->mask ? a->mask : w.ones;
    k.mask_stride = a->mask ? a->mask_stride : 0;
    k.draws = a->draws;
    k.out_tokens = a->out_tokens;
    k.out_status = a->out_status;
    k.out_keep = a->out_keep;
    k.out_topk_ids = a->out_topk_ids;
    k.out_topk_probs = a->out_topk_probs;
    k.topk_cap = (a->out_topk_ids || a->out_topk_probs) ? a->topk_cap : 0;
    k.counters = w.counters;
    k.lists = w.lists;
    k.tlists = w.tlists;
    // Any row a chunked kernel cannot finish from its candidate lists is
    // sampled whole by its own merger, in a region of the workspace taken
    // by a lock (no second launch).
    k.dense = w.dense;
    k.dense_stride = w.max_vocab;
    k.dlocks = w.dlocks;
    k.dense_slots = w.dense_slots;
#ifdef TMS_TRACE
    k.trace = g_tms_trace_host;
#endif
    if (a->history && a->recent) {
        // The history pre-pass lists every row's touched ids with their
        // final values; the general kernel and its whole-row path take the
        // list as the window (tms_hist.hip).
        if (a->dry_scale && a->dry_scale_stride <= 0) return TMS_ERR_INVALID_ARG;
        const int rc = tms_launch_history(k, a->history, a->dry_breaker, a->dry_scale, a->dry_scale_stride,
                                          a->dtype, a->batch, w.ov_n, w.ov_ids, w.ov_vals, stream);
        if (rc != TMS_OK) return rc;
        k.recent = w.ov_ids;
        k.n_recent = w.ov_n;
        k.recent_stride = tms::kHistMax;
        k.ov_vals = w.ov_vals;
        k.dense = w.dense;
        const dim3 grid((unsigned)(a->batch * k.S)), block(tms::kBlock);
#define TMS_LAUNCH(T, F) hipLaunchKernelGGL((tms::sample_kernel<T, F, tms::kEpt>), grid, block, 0, stream, k)
        switch (a->dtype) {
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
    if (a->row_kinds == TMS_ROWS_SPARSE_MASK && a->mask && a->vocab <= tms::kSparseMaxVocab) {
        // Few allowed ids a row (the caller's hint): one workgroup a row
        // reads the mask and only the allowed logits.
        return tms_launch_sparse(k, a->dtype, a->batch, stream);
    }
    if (a->row_kinds == TMS_ROWS_TOPK && (!a->recent || a->recent_stride <= tms::kWideMaxWindow)) {
        // Every row greedy or top-k <= 128 (the caller's promise): the wide
        // top-k kernel, S chunks of at most 4096 16-byte vectors, CE a
        // multiple of 32 so each chunk starts on a mask word, when the grid
        // is resident at once (two 1024-thread workgroups per CU).  A grid
        // that runs in several rounds keeps each workgroup (16 waves) through
        // its serial tail; there the general kernel is faster (B = 1024,
        // V = 256000 bf16: 336 us against 234 us).
        // fp32 rows whose grid fits one workgroup per CU with 8 vectors a
        // thread take that form: half the waves to start and half the lists
        // to merge.  (512 threads of 16 vectors were slower: 18.5 against
        // 16.9 us at B = 64, V = 128256; the stream and the hot-lane select
        // take longer with fewer waves.)
        const int cus = device_cus();
        struct Form { int slots, nt, per_cu; };
        for (const Form f : {Form{8, 1024, 1}, Form{4, 1024, 2}}) {
            if (f.slots > 4 && esz != 4) continue;
            if (a->recent && a->recent_stride > f.nt) continue;
            const int cap = f.nt * f.slots * vec;
            const int s_w = (a->vocab + cap - 1) / cap;
            const int per_w = (a->vocab + s_w - 1) / s_w;
            const int ce = (per_w + 31) / 32 * 32;
            if (s_w <= f.nt / 64 && ce <= cap && a->batch * s_w <= f.per_cu * cus) {
                const int slots = f.slots;
                tms::KArgs kw = k;
                kw.CE = ce;
                kw.S = (a->vocab + ce - 1) / ce;
                return tms_launch_wide(kw, a->dtype, fast, a->batch, slots, stream);
            }
        }
    }
    if (a->row_kinds == TMS_ROWS_TOPK && fast && (!a->recent || a->recent_stride <= 512) &&
        a->batch >= device_cus()) {
        // Top-k batches with a row for every CU: one workgroup a row streams
        // the whole row (B = 1024, V = 256000 bf16: no chunk merges).
        return tms_launch_rows(k, a->dtype, a->batch, stream);
    }
    // Everything else, including top-k batches whose grid does not fit the
    // wide kernel's residency: the general kernel.  Aligned 2-byte rows
    // without a history window take its packed form when that needs fewer
    // chunks a row (config 3's shape, B = 128 and V = 151936: 8 chunks
    // instead of 10, so the 1,024 workgroups are resident at once).
    const int s_packed = (a->vocab + tms::kBlock * tms::kEptPacked - 1) / (tms::kBlock * tms::kEptPacked);
    const bool packed = fast && esz == 2 && !a->recent && s_packed < k.S;
    if (packed) {
        k.S = s_packed;
        const int per_p = (a->vocab + k.S - 1) / k.S;
        k.CE = (per_p + vec - 1) / vec * vec;
    }
    const dim3 grid((unsigned)(a->batch * k.S)), block(tms::kBlock);
#define TMS_LAUNCH(T, F) hipLaunchKernelGGL((tms::sample_kernel<T, F, tms::kEpt>), grid, block, 0, stream, k)
#define TMS_LAUNCH_PACKED(T) hipLaunchKernelGGL((tms::sample_kernel<T, true, tms::kEptPacked>), grid, block, 0, stream, k)
    switch (a->dtype) {
        case TMS_DTYPE_F32:
            if (fast) TMS_LAUNCH(float, true);
            else TMS_LAUNCH(float, false);
            break;
        case TMS_DTYPE_F16:
            if (packed) TMS_LAUNCH_PACKED(_Float16);
            else if (fast) TMS_LAUNCH(_Float16, true);
            else TMS_LAUNCH(_Float16, false);
            break;
        default:
            if (packed) TMS_LAUNCH_PACKED(tms::Bf16);
            else if (fast) TMS_LAUNCH(tms::Bf16, true);
            else TMS_LAUNCH(tms::Bf16, false);
            break;
    }
#undef TMS_LAUNCH_PACKED
#undef TMS_LAUNCH
    return hipGetLastError() == hipSuccess ? TMS_OK : TMS_ERR_HIP;
}

extern "C" int tms_sample_batch(tms_context* ctx, const tms_sample_args* a, hipStream_t stream) {
    if (!ctx) return TMS_ERR_INVALID_ARG;
    SampleWs w;
    w.max_batch = ctx->max_batch;
    w.max_vocab = ctx->max_vocab;
    w.counters = ctx->counters;
    w.ones = ctx->ones;
    w.lists = ctx->lists;
    w.tlists = ctx->tlists;
    w.dlocks = ctx->dlocks;
    w.dense = ctx->dense;
    w.dense_slots = ctx->dense_slots;
    w.ov_n = ctx->ov_n;
    w.ov_ids = ctx->ov_ids;
    w.ov_vals = ctx->ov_vals;
    return sample_launch(w, a, stream);
}

// ============================================= allocation-free entry point
//
// tms_sample_batch_noalloc runs the same kernels over `scratch`, a
// file-scope device array of fixed size, instead of a context's workspace:
// batches of up to kNoAllocRows rows of up to kNoAllocVocab ids, and one
// region for the whole-row path (taken by a lock: rows that need it run one
// after another).
// The array starts zeroed when the code object loads, and every launch
// leaves its counters, lists and lock at zero again, as a context's
// workspace does.  The all-ones mask row (for calls without a mask) is set
// once per device.  In host code `scratch` names a host-side stand-in, so
// its device address is looked up once per device (hipGetSymbolAddress,
// with that device current) and only that address reaches the kernels and
// the memset.

namespace {
constexpr int kNoAllocRows = 64;
constexpr int kNoAllocVocab = 262144;
constexpr size_t kNoAllocChunks = kNoAllocVocab / tms::kChunk;   // 16
constexpr size_t align32(size_t words) { return (words + 31) / 32 * 32; }   // u64 words: 256 bytes
constexpr size_t kNaCounters = 0;
constexpr size_t kNaLists = kNaCounters + align32((size_t)kNoAllocRows * tms::kCounterStride / 2);
constexpr size_t kNaTlists = kNaLists + align32((size_t)kNoAllocRows * kNoAllocChunks * tms::kListStride);
constexpr size_t kNaLocks = kNaTlists + align32((size_t)kNoAllocRows * kNoAllocChunks * tms::kWideListStride);
constexpr size_t kNaHistN = kNaLocks + align32(1);   // one whole-row region lock
constexpr size_t kNaHistIds = kNaHistN + align32(kNoAllocRows / 2);
constexpr size_t kNaHistVals = kNaHistIds + (size_t)kNoAllocRows * tms::kHistMax / 2;
constexpr size_t kNaOnes = kNaHistVals + (size_t)kNoAllocRows * tms::kHistMax / 2;
constexpr size_t kNaDense = kNaOnes + align32(kNoAllocVocab / 64);
constexpr size_t kNaWords = kNaDense + 2 * (size_t)kNoAllocVocab;   // 21.0 MB
}  // namespace

static __device__ __align__(256) uint64_t scratch[kNaWords];

namespace {
constexpr int kNoAllocMaxDevices = 64;
std::mutex g_noalloc_mu;
uint64_t* g_noalloc_scratch[kNoAllocMaxDevices];   // device address of `scratch`, per device
}  // namespace

extern "C" int tms_workspace_reset(tms_context* ctx, hipStream_t stream) {
    int prev = 0;
    if (hipGetDevice(&prev) != hipSuccess) return TMS_ERR_NO_DEVICE;
    if (!ctx) {
        // the allocation-free entry point's scratch on the current device
        uint64_t* base = nullptr;
        {
            std::lock_guard<std::mutex> lock(g_noalloc_mu);
            if (prev >= 0 && prev < kNoAllocMaxDevices) base = g_noalloc_scratch[prev];
        }
        if (!base) return TMS_OK;   // never used on this device: still zero
        return reset_regions(base, kNaOnes * 8, kNaDense * 8, kNaDense * 8, stream);
    }
    if (hipSetDevice(ctx->device) != hipSuccess) return TMS_ERR_HIP;
    const int rc = reset_regions(ctx->ws, ctx->ones_begin, ctx->ones_end, ctx->bytes, stream);
    (void)hipSetDevice(prev);
    return rc;
}

extern "C" int tms_sample_batch_noalloc(const tms_sample_args* a, hipStream_t stream) {
    if (!a) return TMS_ERR_INVALID_ARG;
    if (a->batch > kNoAllocRows || a->vocab > kNoAllocVocab) return TMS_ERR_CAPACITY;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return TMS_ERR_NO_DEVICE;
    if (dev < 0 || dev >= kNoAllocMaxDevices) return TMS_ERR_NO_DEVICE;
    uint64_t* base;
    {
        std::lock_guard<std::mutex> lock(g_noalloc_mu);
        if (!g_noalloc_scratch[dev]) {
            void* p = nullptr;
            if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return TMS_ERR_HIP;
            uint64_t* q = (uint64_t*)p;
            // the all-ones row, once (synchronous: before any launch uses it)
            if (hipMemset(q + kNaOnes, 0xFF, kNoAllocVocab / 8) != hipSuccess) return TMS_ERR_HIP;
            if (hipDeviceSynchronize() != hipSuccess) return TMS_ERR_HIP;
            g_noalloc_scratch[dev] = q;
        }
        base = g_noalloc_scratch[dev];
    }
    SampleWs w;
    w.max_batch = kNoAllocRows;
    w.max_vocab = kNoAllocVocab;
    w.counters = (uint32_t*)(base + kNaCounters);
    w.ones = (uint32_t*)(base + kNaOnes);
    w.lists = base + kNaLists;
    w.tlists = base + kNaTlists;
    w.dlocks = (uint32_t*)(base + kNaLocks);
    w.dense = base + kNaDense;
    w.dense_slots = 1;
    w.ov_n = (int32_t*)(base + kNaHistN);
    w.ov_ids = (int32_t*)(base + kNaHistIds);
    w.ov_vals = (float*)(base + kNaHistVals);
    return sample_launch(w, a, stream);
}

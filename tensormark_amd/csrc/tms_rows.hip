// tms_rows.hip -- the sampler kernel for top-k batches with a row for every
// workgroup slot (row_kinds = TMS_ROWS_TOPK, batch >= the device's CUs):
// one 256-thread workgroup a row streams the whole row in passes, with no
// cross-workgroup merge.
//
// Config 5's shape (B = 1024, V = 256000 bf16) runs 16,384 chunk workgroups
// in the general kernel, each paying a chunk's selection and a share of a
// row merge after its 32 KB stream.  Here the 1,024 workgroups are resident
// at once (four a CU), each keeps two passes of loads in flight (double
// buffering in registers: 2 x 3 slots of 16 bytes a thread),
// and a row's selection work runs while the other workgroups of its CU
// stream.
//
//   window    history positions (at most 512) into an LDS hash keyed by id
//             that counts occurrences; the first position holding an id
//             owns it, loads the id's logit and mask word, and offers the
//             penalised value (tmsample.h:58-61, then frequency/presence) as
//             a candidate.  The stream's copies of window ids leave pass 0
//             through a thread-major bitmap and later passes at each
//             compaction (a hash lookup per candidate).
//   pass      per 16-byte slot: the mask folded in (-inf in place), the
//             thread's IEEE maximum (NaN / +inf); greedy rows without a
//             window keep each thread's best (value, lowest id); other rows
//             (greedy ones as K = 1) stage the slots
//             whose maximum reaches vlo in LDS, and after the next pass's
//             loads are issued append their entries at or above vlo to an
//             LDS buffer.
//   bound     after pass 0: the K-th largest of its 128 group maxima (two
//             lanes a group), by rank counting, bounds the row's K-th value
//             from below; vlo is that bound less the margin that keeps every
//             entry whose quotient by T can tie with it.
//   compact   after every pair of passes once the buffer is a quarter full,
//             and after the last pass:
//             two 8-bit histogram levels of the candidates' order keys find
//             a value with at least K candidates at or above it, which
//             raises vlo; entries below the new vlo leave.
//   select    the survivors' keys (v / T, then lowest id) ranked by
//             bucket_rank, the top K into the fp64 tail of tmsample::sample
//             (tail_topk, tmsample.h:184-199).
//
// A row that breaks the promise (top_k outside 1..128, not greedy) or whose
// candidates overflow the buffer (massive ties) is sampled whole
// (tms_dense.h) by the same workgroup, so every row gets the reference's
// answer.
#include "tms_dense.h"
#include "tms_select.h"

namespace tms {
namespace rows {

constexpr int kBuf = 1024;          // candidate buffer
constexpr int kCompactAt = kBuf / 4;
constexpr int kHashR = 2048;        // window table slots (at most 1024 ids)
constexpr int kCntR = 11;           // occurrence count bits of a table word
constexpr uint32_t kEmptyR = 0xFFFFFFFFu;
constexpr uint32_t kOwnerBit = 0x80000000u;   // candidate id word: an owner's penalised entry
constexpr int kMaxWindow = 512;
constexpr int kStg = 64;            // hot slots a wave stages (a full area is drained at once)
constexpr int kKMax = kTopkFast;    // the top-k promise: 1 <= top_k <= 128

struct Smem {
    alignas(16) uint64_t cand[kBuf + 16];    // value bits << 32 | id (kOwnerBit: an owner's entry)
    alignas(16) uint64_t srt[kKMax + 8];     // the row's sorted top-K
    alignas(16) double pr[4 * kKMax];        // fp64 tail
    alignas(16) double q[kKMax];
    uint32_t wtab[kHashR];                   // id << kCntR | occurrences, or kEmptyR
    uint32_t wbits[kBlock];                  // pass 0 window ids, thread-major
    alignas(16) uint32_t gmax[128];          // pass 0 group maxima (order keys)
    int hist[256];                           // compaction level 1 (zero between compactions)
    int hist2[256];                          //   and level 2
    int pbits[kBuckets];                     // bucket_rank's counts
    uint64_t wave_k[kWaves];
    float wave_f[kWaves];
    int wave_i[kWaves];
    uint64_t theta;
    alignas(16) uint4 stg[kWaves][kStg];     // per wave: the words of its hot slots
    uint32_t sid[kWaves][kStg];              // and each one's first id
    int ncand, onf, over;
    uint32_t tkey;
    int misc[4];
};
static_assert(sizeof(DenseLds) <= sizeof(uint64_t) * kBuf, "the whole-row path's LDS lies over the buffer");

__device__ __forceinline__ int hash_r(uint32_t id) { return (int)((id * 0x9E3779B1u) >> 21); }

// Table slot of id, or -1 when it is not a window id.
__device__ __forceinline__ int window_find(const uint32_t* tab, uint32_t id) {
    int sl = hash_r(id);
    for (int probe = 0; probe < kHashR; ++probe) {
        const uint32_t w = tab[sl];
        if (w == kEmptyR) return -1;
        if ((w >> kCntR) == id) return sl;
        sl = (sl + 1) & (kHashR - 1);
    }
    return -1;
}

// The least value v that can still place given a lower bound tau on the
// K-th value: v < vlo implies fl(v / T) < fl(tau / T) (a 2^-19 relative gap
// exceeds two roundings; the absolute term covers subnormal quotients).
__device__ __forceinline__ float vlo_of(float tau, float temp, bool divide) {
    float vlo = tau;
    if (divide && tau != -__builtin_huge_valf()) {
        if (fabsf(tau) >= temp * 0x1p-100f) {
            vlo = tau - fabsf(tau) * 0x1p-18f;   // rounds to at most tau (1 - 2^-19)
        } else {
            const double lo = (double)tau - (fabs((double)tau) * 0x1p-19 + (double)temp * 0x1p-140);
            float f = (float)lo;
            if ((double)f > lo) f = float_below(f);
            vlo = f;
        }
    }
    return fmaxf(vlo, -FLT_MAX);   // NaN (a bound below -inf) -> every finite entry
}

template <typename T>
__global__ __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(4, 8))) void row_kernel(KArgs a) {
    __shared__ Smem sm;
    constexpr int VEC = Elt<T>::kVec;
    // 16-byte slots a thread per pass (per buffer), within the 128
    // registers of four workgroups a CU (four spill with the staging)
    constexpr int PS = 3;
    constexpr int PI = kBlock * PS * VEC;   // ids a pass
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    const int row = blockIdx.x;
    const int V = a.V;
    const int NP = (V + PI - 1) / PI;
    const T* base = (const T*)a.logits + (int64_t)row * a.row_stride;
    const uint32_t* mrow = a.mask + (int64_t)row * a.mask_stride;
    const float NEG_INF = -__builtin_huge_valf();

    // ---- loads first: history positions, then passes 0 and 1
    const int rs = a.recent ? (int)a.recent_stride : 1;
    const int32_t* hrow = a.recent ? a.recent + (int64_t)row * a.recent_stride : nullptr;
    int hid[kMaxWindow / kBlock];
#pragma unroll
    for (int i = 0; i < kMaxWindow / kBlock; ++i) {
        const int p = t + i * kBlock;
        hid[i] = (hrow && p < rs) ? hrow[p] : -1;
    }
    uint4 A[PS], B[PS];
    uint32_t mA[PS], mB[PS];
    const bool masked = a.mask_stride != 0;   // 0: no caller mask (the all-ones row)
    auto load = [&](uint4 (&buf)[PS], uint32_t (&mw)[PS], int p) {
#pragma unroll
        for (int j = 0; j < PS; ++j) {
            const int off = p * PI + VEC * (j * kBlock + t);
            mw[j] = masked ? mrow[min(off, V - 1) >> 5] : ~0u;
            buf[j] = ld_nt(base + min(off, V - VEC));
        }
    };
    load(A, mA, 0);
    if (NP > 1) load(B, mB, 1);

    const tms_row_params P = a.params[row];
    const bool greedy = P.greedy != 0;
    const bool promise = greedy || (P.top_k >= 1 && P.top_k <= kKMax);
    const int K = greedy ? 1 : min(P.top_k, V);
    const float temp = P.temperature;
    const bool bad_params = !greedy && !(temp > 0.0f && temp <= FLT_MAX);
    const bool divide = !greedy && temp != 1.0f;
    int nrec = 0;
    if (a.recent) {
        nrec = a.n_recent ? a.n_recent[row] : rs;
        nrec = min(max(nrec, 0), rs);
    }
    Pen pn;
    pn.rep_on = !(P.repeat_penalty <= 1.0f);
    pn.fp_on = P.frequency_penalty != 0.0f || P.presence_penalty != 0.0f;
    pn.on = nrec > 0 && P.repeat_last_n > 0 && (pn.rep_on || pn.fp_on);
    pn.rep = P.repeat_penalty;
    pn.freq = P.frequency_penalty;
    pn.pres = P.presence_penalty;
    const int from = pn.on ? (nrec > P.repeat_last_n ? nrec - P.repeat_last_n : 0) : 0;
    // Greedy rows without a window keep each thread's best entry; every other
    // row in the promise selects candidates (a greedy row with a window as
    // top-1, so the stream's copies of window ids leave at a compaction).
    const bool track = greedy && !pn.on;
    const bool select = promise && !bad_params && !track;

    // ---- window: inserts (the first position of an id owns it), the
    //      owners' loads of their logit and mask word
    if (t == 0) {
        sm.ncand = 0;
        sm.onf = 0;
        sm.over = 0;
    }
    sm.hist[t] = 0;
    sm.hist2[t] = 0;
    if (pn.on) {
        sm.wbits[t] = 0u;
        for (int i = t; i < kHashR; i += kBlock) sm.wtab[i] = kEmptyR;
    }
    lds_sync();
    bool owner[kMaxWindow / kBlock];
    int oslot[kMaxWindow / kBlock];
    float ox[kMaxWindow / kBlock];
    uint32_t omw[kMaxWindow / kBlock];
#pragma unroll
    for (int i = 0; i < kMaxWindow / kBlock; ++i) {
        owner[i] = false;
        oslot[i] = 0;
        ox[i] = NEG_INF;
        omw[i] = 0u;
        const int p = t + i * kBlock;
        const int id = hid[i];
        if (pn.on && p >= from && p < nrec && id >= 0 && id < V) {
            ox[i] = Elt<T>::scalar(base + id);
            omw[i] = mrow[id >> 5];
            if (id < PI) {   // pass 0: the streaming thread's bit
                const int jj = id / (VEC * kBlock), r = id % (VEC * kBlock);
                atomicOr(&sm.wbits[r / VEC], 1u << (jj * VEC + r % VEC));
            }
            int sl = hash_r((uint32_t)id);
            for (int probe = 0; probe < kHashR; ++probe) {
                const uint32_t old = atomicCAS(&sm.wtab[sl], kEmptyR, (uint32_t)id << kCntR);
                if (old == kEmptyR) {
                    owner[i] = true;
                    break;
                }
                if ((old >> kCntR) == (uint32_t)id) break;
                sl = (sl + 1) & (kHashR - 1);
            }
            atomicAdd(&sm.wtab[sl], 1u);
            oslot[i] = sl;
        }
    }
    uint32_t wt = 0u;
    if (pn.on) {
        lds_sync();
        wt = sm.wbits[t];
    }

    // ---- the stream
    float m = NEG_INF;                  // IEEE maximum: a NaN stays
    float gbv = NEG_INF;                // greedy: the thread's best value
    uint32_t gbi = 0xFFFFFFFFu;         //   and its (lowest) id
    float vlo = __builtin_huge_valf();  // top-k: no candidate before the bound
    int nstg = 0;                       // the wave's staged hot slots (uniform)
    // The staged slots' entries at or above vlo into the buffer: the wave
    // takes 64 entries a step, one LDS atomic for all of a step's takes.
    auto drain = [&]() {
        if (!nstg) return;
        __builtin_amdgcn_wave_barrier();
        const T* hv = (const T*)&sm.stg[wv][0];
        for (int q = lane; q < nstg * VEC; q += 64) {
            const float x = Elt<T>::scalar(hv + q);
            if (x >= vlo) {
                const int at = atomicAdd(&sm.ncand, 1);
                if (at < kBuf) sm.cand[at] = ((uint64_t)__float_as_uint(x) << 32) | (sm.sid[wv][q / VEC] + (uint32_t)(q % VEC));
            }
        }
        nstg = 0;
        __builtin_amdgcn_wave_barrier();
    };

    auto process = [&](uint4 (&buf)[PS], uint32_t (&mw)[PS], int p) {
        const bool first = p == 0;   // pass 0: window bits, the bound
        float pm = NEG_INF;
        float smx[PS];   // each slot's maximum
#pragma unroll
        for (int j = 0; j < PS; ++j) {
            const int off = p * PI + VEC * (j * kBlock + t);
            const int lim = V - off;
            // the fold only where a bit can be clear: a caller mask, pass 0's
            // window ids, the row's last pass
            if (masked || (first && wt) || p == NP - 1) {
                uint32_t bits = lim > 0 ? (mw[j] >> (off & 31)) & ((1u << min(lim, VEC)) - 1u) : 0u;
                if (first) bits &= ~(wt >> (j * VEC));
                buf[j] = fold_bits<T>(buf[j], bits);
            }
            float sx = NEG_INF;
#pragma unroll
            for (int e = 0; e < VEC; e += 2)
                sx = __builtin_elementwise_maximum(sx, __builtin_elementwise_maximum(elt<T>(buf[j], e), elt<T>(buf[j], e + 1)));
            pm = __builtin_elementwise_maximum(pm, sx);
            smx[j] = sx;
            if (track && sx > gbv) {   // rare once the best has risen
#pragma unroll
                for (int e = VEC - 1; e >= 0; --e) {
                    // the slot's first entry equal to its maximum: its lowest id
                    if (elt<T>(buf[j], e) == sx) gbi = (uint32_t)(off + e);
                }
                gbv = sx;
            }
        }
        m = __builtin_elementwise_maximum(m, pm);
        if (!select) return;
        // The widened values are formed again from the words where they are
        // used next (holding 2-byte entries widened would double their
        // registers).
#pragma unroll
        for (int j = 0; j < PS; ++j)
            asm volatile("" : "+v"(buf[j].x), "+v"(buf[j].y), "+v"(buf[j].z), "+v"(buf[j].w));
        if (first) {
            // ---- bound: the K-th largest of the 128 group maxima (two lanes
            //      a group, order keys with the low 7 bits replaced by 127 -
            //      the group, so they are distinct), by rank counting
            const bool nf = !(pm < __builtin_huge_valf()) && pm != NEG_INF;
            uint32_t g = nf ? 0u : okey(pm);
            g = max(g, dpp_u32<0x111, 0xF, true>(0u, g));   // row_shr:1
            const int gi = t >> 1;
            if (t & 1) sm.gmax[gi] = (g & ~127u) | (uint32_t)(127 - gi);
            lds_sync();
            const int gx = t >> 1, part = t & 1;
            const uint32_t x = sm.gmax[gx];
            const uint4* g4 = (const uint4*)(sm.gmax + 64 * part);
            int r = 0;
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const uint4 y = g4[q];
                r += (y.x > x ? 1 : 0) + (y.y > x ? 1 : 0) + (y.z > x ? 1 : 0) + (y.w > x ? 1 : 0);
            }
            r += __shfl_xor(r, 1, 64);
            if (part == 0 && r == K - 1) sm.tkey = x & ~127u;
            lds_sync();
            const uint32_t tk = sm.tkey;
            vlo = vlo_of(tk < 0x00800000u ? NEG_INF : okey_inv(tk), temp, divide);
        }
        // ---- candidates: the slots whose maximum reaches vlo go to the
        //      wave's staging area (no wait), and drain() appends their
        //      entries after the next pass's loads are issued (or at once,
        //      when a slot's hot lanes would not fit the area).
        if (__ballot(pm >= vlo)) {
#pragma unroll
            for (int jj = 0; jj < PS; ++jj) {
                const bool hot = smx[jj] >= vlo;
                const uint64_t hb = __ballot(hot);
                if (!hb) continue;
                if (nstg + __popcll(hb) > kStg) drain();   // the area is full: empty it first
                const int off = p * PI + VEC * (jj * kBlock + t);
                const int pos = nstg + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(hb >> 32),
                                                                     __builtin_amdgcn_mbcnt_lo((uint32_t)hb, 0u));
                if (hot) {
                    sm.stg[wv][pos] = buf[jj];
                    sm.sid[wv][pos] = (uint32_t)off;
                }
                nstg += __popcll(hb);
            }
        }
    };

    // ---- compaction: two 8-bit histogram levels over the candidates'
    //      order keys find tau with at least K candidates at or above it;
    //      vlo rises to vlo_of(tau) and the entries below leave.  Stream
    //      copies of window ids leave too (their owners' entries stay).
    //      The histograms are zero on entry (each is cleared after its last
    //      read), and the count is cleared once every thread has read it.
    auto compact = [&](bool synced) {
        if (!synced) lds_sync();
        const int nc = min(sm.ncand, kBuf);
        if (sm.ncand > kBuf && t == 0) sm.over = 1;
        uint64_t c[kBuf / kBlock];
        uint32_t kk[kBuf / kBlock];
#pragma unroll
        for (int u = 0; u < kBuf / kBlock; ++u) {
            const int i = t + u * kBlock;
            c[u] = i < nc ? sm.cand[i] : 0ull;
            kk[u] = 0u;
            if (i < nc) {
                const uint32_t idw = (uint32_t)c[u];
                const bool dup = pn.on && !(idw & kOwnerBit) && window_find(sm.wtab, idw) >= 0;
                if (!dup) kk[u] = okey(__uint_as_float((uint32_t)(c[u] >> 32)));
                if (dup) c[u] = 0ull;
            }
        }
#pragma unroll
        for (int u = 0; u < kBuf / kBlock; ++u)
            if (kk[u]) atomicAdd(&sm.hist[kk[u] >> 24], 1);
        lds_sync();
        if (t == 0) sm.ncand = 0;   // read by every thread before the barrier
        // wave 0: the bin where the count from the top first reaches K
        auto pick = [&](int above0, int* out, const int* hist) {
            int h[4], s = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                h[i] = hist[255 - (4 * lane + i)];
                s += h[i];
            }
            int above = above0 + wave_incl_scan_i32(s) - s;
            const int total = above0 + __builtin_amdgcn_readlane(wave_incl_scan_i32(s), 63);
            if (lane == 0 && total < K) {   // fewer than K: every candidate stays
                out[0] = -1;
                out[1] = total;
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if (above < K && above + h[i] >= K) {
                    out[0] = 255 - (4 * lane + i);
                    out[1] = above;
                }
                above += h[i];
            }
        };
        if (wv == 0) pick(0, sm.misc, sm.hist);
        lds_sync();
        const int b1 = sm.misc[0], above1 = sm.misc[1];
        sm.hist[t] = 0;   // read by pick before the barrier
        uint32_t tau = 0u;
        if (b1 >= 0) {
#pragma unroll
            for (int u = 0; u < kBuf / kBlock; ++u)
                if (kk[u] && (int)(kk[u] >> 24) == b1) atomicAdd(&sm.hist2[(kk[u] >> 16) & 0xFF], 1);
            lds_sync();
            if (wv == 0) pick(above1, sm.misc + 2, sm.hist2);
            lds_sync();
            tau = ((uint32_t)b1 << 24) | ((uint32_t)max(sm.misc[2], 0) << 16);
            sm.hist2[t] = 0;
        }
        // at least K candidates have a key >= tau, so the row's K-th value is
        // at least okey_inv(tau); keys below 0x00800000 decode to -inf or NaN
        const float nv = vlo_of(tau < 0x00800000u ? NEG_INF : okey_inv(tau), temp, divide);
        vlo = fmaxf(vlo, nv);
        // the count was cleared before the last barrier
#pragma unroll
        for (int u = 0; u < kBuf / kBlock; ++u) {
            if (c[u] && __uint_as_float((uint32_t)(c[u] >> 32)) >= vlo) {
                const int at = atomicAdd(&sm.ncand, 1);
                sm.cand[at] = c[u];
            }
        }
        lds_sync();
    };

    // A compaction check after every pair of passes (a barrier), at a
    // quarter of the buffer: pass 0's bound keeps about 2-6% of its 8192
    // entries (bf16 ties included), so the first pair appends up to about
    // 500 (config 5's worst row: 492) and is compacted at once; later bounds
    // keep far fewer.  Compacting at half the buffer let that row reach 1041
    // candidates after its second pair, and the whole-row path (1.8 ms for
    // the call).
    auto check = [&]() {
        if (select) {
            lds_sync();
            if (sm.ncand > kCompactAt) compact(true);
        }
    };
    for (int p = 0; p < NP; p += 2) {
        process(A, mA, p);
        if (p + 2 < NP) load(A, mA, p + 2);
        drain();
        if (p + 1 < NP) {
            process(B, mB, p + 1);
            if (p + 3 < NP) load(B, mB, p + 3);
            drain();
        }
        if (p == 0) {
            // the owners' penalised values (their loads were issued after
            // passes 0 and 1, which are in now)
#pragma unroll
            for (int i = 0; i < kMaxWindow / kBlock; ++i) {
                if (owner[i]) {
                    const int id = hid[i];
                    float v = ((omw[i] >> (id & 31)) & 1u) ? ox[i] : NEG_INF;
                    if (v != NEG_INF) v = apply_pen(v, sm.wtab[oslot[i]] & ((1u << kCntR) - 1u), pn);
                    if (!(v < __builtin_huge_valf()) && v != NEG_INF) atomicOr(&sm.onf, 1);
                    if (select && v >= vlo) {
                        const int at = atomicAdd(&sm.ncand, 1);
                        if (at < kBuf) sm.cand[at] = ((uint64_t)__float_as_uint(v) << 32) | (kOwnerBit | (uint32_t)id);
                    }
                }
            }
        }
        check();
    }

    // ---- row totals: NaN / +inf, the greedy best
    const bool nf = !(m < __builtin_huge_valf()) && m != NEG_INF;
    const uint64_t gk = gbv != NEG_INF ? ckey(gbv, gbi) : 0ull;
    const uint64_t best = wave_max_u64_dpp(gk);
    const bool anynf = __any(nf);
    const bool anyfin = __any(m != NEG_INF);
    if (lane == 0) {
        sm.wave_k[wv] = best;
        sm.wave_i[wv] = (anynf ? 1 : 0) | (anyfin ? 2 : 0);
    }
    if (select) compact(false);
    lds_sync();
    uint64_t gb = 0ull;
    int fl = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
        gb = sm.wave_k[w] > gb ? sm.wave_k[w] : gb;
        fl |= sm.wave_i[w];
    }
    const bool nonfin = (fl & 1) || sm.onf;
    const bool overflow = sm.over != 0;
    lds_sync();
    if (bad_params) {
        write_row_error(a, row, TMS_ROW_BAD_PARAMS);
        return;
    }
    if (nonfin) {
        write_row_error(a, row, TMS_ROW_NONFINITE);
        return;
    }
    auto greedy_out = [&](int tok) {
        if (t == 0) {
            a.out_tokens[row] = tok;
            a.out_status[row] = TMS_ROW_OK;
            if (a.out_keep) a.out_keep[row] = 0;
        }
        for (int i = t; i < a.topk_cap; i += kBlock) {
            if (a.out_topk_ids) a.out_topk_ids[(int64_t)row * a.topk_cap + i] = i == 0 ? tok : -1;
            if (a.out_topk_probs) a.out_topk_probs[(int64_t)row * a.topk_cap + i] = i == 0 ? 1.0f : 0.0f;
        }
    };
    if (track) {
        if (gb == 0ull) write_row_error(a, row, TMS_ROW_ALL_MASKED);
        else greedy_out((int)ckey_id(gb));
        return;
    }
    const bool anyf = (fl & 2) != 0 || sm.ncand > 0;
    if (!anyf) {
        write_row_error(a, row, TMS_ROW_ALL_MASKED);
        return;
    }
    DenseLds& L = *reinterpret_cast<DenseLds*>(sm.cand);
    if (greedy && overflow) {
        // a greedy row with a window whose top ties overflow the buffer
        [[clang::always_inline]] dense_greedy<T>(a, row, pn, from, nrec, L);
        return;
    }
    if (!promise || overflow) {
        // outside the top-k promise, or massive ties: the whole row
        [[clang::always_inline]] dense_inline<T>(a, row, L);
        return;
    }

    // ---- select: the survivors' keys ranked, the top K into the tail
    const int n = sm.ncand;
    uint64_t* keys = sm.cand;
    for (int i = t; i < n; i += kBlock) {
        const uint64_t c = keys[i];
        const float v = __uint_as_float((uint32_t)(c >> 32));
        const uint32_t id = (uint32_t)c & ~kOwnerBit;
        keys[i] = v != NEG_INF ? ckey(divide ? v / temp : v, id) : 0ull;
    }
    lds_sync();
    int N = 0;
    {
        int f = 0;
        for (int i = t; i < n; i += kBlock) f += keys[i] != 0ull ? 1 : 0;
        int tot;
        block_excl_scan(f, tot, sm);
        N = tot;
    }
    if (N == 0) {
        write_row_error(a, row, TMS_ROW_ALL_MASKED);
        return;
    }
    const int nkeep = min(N, K);
    keys[n] = 0ull;
    if (n <= 2 * kBlock) {
        [[clang::always_inline]] bucket_rank<2>(keys, n, nkeep, sm.srt, sm.pbits, sm);
    } else {
        [[clang::always_inline]] bucket_rank<kBuf / kBlock>(keys, n, nkeep, sm.srt, sm.pbits, sm);
    }
    lds_sync();
    if (greedy) {   // with a window: the top-1 of the candidates
        greedy_out((int)ckey_id(sm.srt[0]));
        return;
    }
    if (ckey_val(sm.srt[0]) == __builtin_huge_valf()) {   // v / T overflowed
        write_row_error(a, row, TMS_ROW_NONFINITE);
        return;
    }
    if (N < K) {
        // Fewer than K finite ids: the top-k goes on with -inf entries in
        // ascending id order, the ids in [0, K + N) outside the finite set
        // (K + N <= 2 * kKMax <= kBlock).
        const int q = t;
        int member = 0;
        if (q < K + N)
            for (int i = 0; i < N; ++i) member |= (int)ckey_id(sm.srt[i]) == q;
        const int gap = (q < K + N && !member && q < V) ? 1 : 0;
        int tot;
        const int p = block_excl_scan(gap, tot, sm);
        if (gap && p < K - N) sm.srt[N + p] = ckey(NEG_INF, (uint32_t)q);
        lds_sync();
    }
    if (wv == 0) {
        uint32_t w0, w1;
        row_uniform(a, row, P, w0, w1);
        [[clang::always_inline]] tail_topk(a, row, P, sm.srt, K, K, sm.pr, sm.q, w0, w1);
    }
}

}  // namespace rows
}  // namespace tms

// Launch of the row-stream kernel for tms_sample_batch: one workgroup a row
// (16-byte aligned rows, vocab a multiple of the vector width, a window of
// at most kMaxWindow = 512 positions; the host checks).
int tms_launch_rows(const tms::KArgs& k, int dtype, int batch, hipStream_t stream) {
    const dim3 grid((unsigned)batch), block(tms::kBlock);
    switch (dtype) {
        case TMS_DTYPE_F32:
            hipLaunchKernelGGL((tms::rows::row_kernel<float>), grid, block, 0, stream, k);
            break;
        case TMS_DTYPE_F16:
            hipLaunchKernelGGL((tms::rows::row_kernel<_Float16>), grid, block, 0, stream, k);
            break;
        default:
            hipLaunchKernelGGL((tms::rows::row_kernel<tms::Bf16>), grid, block, 0, stream, k);
            break;
    }
    return hipGetLastError() == hipSuccess ? TMS_OK : TMS_ERR_HIP;
}

// tms_hist.hip -- the history pre-pass of tms_sample_batch calls that carry
// tms_sample_args.history: the steps of sample_token before the sampler
// (tensormark/llama_chat.cpp:148-150) for every row, on the device.
//
// One workgroup per row turns the row's history into a list of the distinct
// ids it touches, each with its final value after
//   the grammar mask                    (llama_chat.cpp:184-209),
//   the repetition penalty              (tmsample.h:52-63),
//   the frequency/presence penalty,
//   the no-repeat n-gram ban            (tmsample.h:81-114),
//   DRY                                 (tmsample.h:148-170, with the caller's
//                                        table of the reference's powf values),
// and the general sampling kernel and its whole-row path then take those
// values in place of the logits of those ids (the window machinery they use
// for the repetition penalty, fed with the list instead of the history).
// Every other id keeps its masked logit, which is what the reference's
// transforms leave it.
//
// Per row, in LDS: an open-addressing hash of the touched ids (2 *
// kHistMax slots: id + 1, or 0) with a word of facts per slot (window
// count, banned, DRY target); the slots are then numbered in slot order
// (the list's order), the values formed per entry, and DRY's subtractions
// applied in the reference's position order.  The list goes to the
// workspace: ov_n[row] (-1 when the row touches more than kHistMax ids),
// ov_ids[row][e], ov_vals[row][e].
//
// DRY's match lengths come from the window staged in LDS (reversed, so the
// run ending at position i against the tail is the common prefix of r and
// r[last - i ..]): every position compares up to kDryDirect ids directly,
// in parallel; when some position reaches that many, one wave computes
// every length again with the Z-function (linear in the window: each
// extension step compares 64 ids by ballot), so a repetitive window costs
// O(n) and not O(n^2).
//
// The n-gram ban's restore rule (the banned ids get their values back when
// nothing above -inf is left) needs the row's maximum outside the list:
// an entry that is not banned and above -inf settles it at once; otherwise
// the row is scanned (mask word by mask word) for an allowed id outside the
// list whose logit is above -inf, stopping at the first.

#include "tms_history.h"
#include "tms_sample_common.h"

namespace tms {

constexpr int kHBlock = 256;
constexpr int kHSlots = 2 * kHistMax;
constexpr uint32_t kHCount = 0xFFFFu;     // window count
constexpr uint32_t kHDry = 1u << 30;      // a DRY target
constexpr uint32_t kHBan = 1u << 31;      // banned by the n-gram rule
constexpr int kDryMax = TMS_DRY_MAX_WINDOW;   // DRY window positions held in LDS
constexpr int kDryDirect = 64;            // ids a position compares before the Z-function pass
static_assert(kDryMax <= 2 * kHistMax, "the staged window lies over the table's keys");

struct HistArgs {
    const void* logits;
    int64_t row_stride;
    int V;
    const tms_row_params* params;
    const tms_history_params* hp;
    const uint8_t* breaker;
    const int32_t* recent;
    const int32_t* n_recent;
    int64_t recent_stride;
    const uint32_t* mask;      // never null (the all-ones row)
    int64_t mask_stride;
    const float* dry_scale;    // [B][dry_scale_stride] or null
    int64_t dry_scale_stride;
    int32_t* ov_n;             // [B]
    int32_t* ov_ids;           // [B][kHistMax]
    float* ov_vals;            // [B][kHistMax]
};

struct HistLds {
    uint32_t key[kHSlots];     // id + 1; 0 = empty (before the table: DRY's staged window)
    uint32_t info[kHSlots];    // kHCount | kHDry | kHBan
    uint16_t ent[kHSlots];     // the slot's entry
    uint16_t eslot[kHistMax];  // the entry's slot
    float val[kHistMax];
    int32_t tslot[kHBlock];    // DRY: one tile of target slots, in position order
    int32_t tk[kHBlock];       //      and their exponents L - allowed_length
    uint16_t dlen[kDryMax];    // DRY: the match length at each window position
    uint32_t dbrk[kDryMax / 32];   // DRY: staged window positions holding a breaker
    int wave_i[kHBlock / 64];
    int flag;                  // overflow
    int found;
};

__device__ __forceinline__ uint32_t hslot0(int id) {
    return ((uint32_t)id * 2654435761u) >> (32 - 13);   // 13 bits: kHSlots = 8192
}
static_assert(kHSlots == 8192, "hslot0 takes 13 bits");

// Slot of id, inserting it; -1 when the table is full.
__device__ __forceinline__ int hinsert(HistLds& L, int id) {
    const uint32_t h = hslot0(id), k = (uint32_t)id + 1u;
    for (int p = 0; p < kHSlots; ++p) {
        const int s = (int)((h + (uint32_t)p) & (kHSlots - 1));
        const uint32_t old = atomicCAS(&L.key[s], 0u, k);
        if (old == 0u || old == k) return s;
    }
    return -1;
}

// Slot of id, or -1.
__device__ __forceinline__ int hfind(const HistLds& L, int id) {
    const uint32_t h = hslot0(id), k = (uint32_t)id + 1u;
    for (int p = 0; p < kHSlots; ++p) {
        const int s = (int)((h + (uint32_t)p) & (kHSlots - 1));
        const uint32_t x = L.key[s];
        if (x == k) return s;
        if (x == 0u) return -1;
    }
    return -1;
}

__device__ __forceinline__ int block_or(int v, HistLds& L) {
    v = __any(v) ? 1 : 0;
    if ((threadIdx.x & 63) == 0) L.wave_i[threadIdx.x >> 6] = v;
    __syncthreads();
    int r = 0;
#pragma unroll
    for (int w = 0; w < kHBlock / 64; ++w) r |= L.wave_i[w];
    __syncthreads();
    return r;
}

// Exclusive prefix over the workgroup in thread order; `total` gets the sum.
__device__ __forceinline__ int hist_excl_scan(int v, int& total, HistLds& L) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int inc = wave_incl_scan_i32(v);
    if (lane == 63) L.wave_i[w] = inc;
    __syncthreads();
    int before = 0;
    total = 0;
#pragma unroll
    for (int i = 0; i < kHBlock / 64; ++i) {
        const int x = L.wave_i[i];
        before += i < w ? x : 0;
        total += x;
    }
    __syncthreads();
    return before + inc - v;
}

__device__ __forceinline__ bool is_breaker(const uint8_t* brk, int V, int id) {
    return brk && id >= 0 && id < V && brk[id] != 0;
}

// DRY match lengths (tmsample.h:159-163) of every window position i <
// last = dn - 1: how far the runs ending at i and at last agree, never
// across a breaker.  r[j] is the window's id at last - j (staged in the
// table's key array), bit j of dbrk marks a breaker there; the length at i
// is the common prefix of r and r[last - i ..], which stops at the window's
// start (position d + k <= last).  Lengths go to L.dlen[i].
__device__ __forceinline__ bool dry_eq(const int32_t* r, const uint32_t* brk, int a, int b) {
    return r[a] == r[b] && !((brk[a >> 5] >> (a & 31)) & 1u) && !((brk[b >> 5] >> (b & 31)) & 1u);
}

__device__ void dry_lengths(const int32_t* dw, int dn, const uint8_t* breaker, int V, HistLds& L) {
    const int t = threadIdx.x, lane = t & 63;
    const int last = dn - 1;
    int32_t* r = (int32_t*)L.key;
    for (int i = t; i < kDryMax / 32; i += kHBlock) L.dbrk[i] = 0u;
    __syncthreads();
    for (int j = t; j < dn; j += kHBlock) {
        const int id = dw[last - j];
        r[j] = id;
        if (is_breaker(breaker, V, id)) atomicOr(&L.dbrk[j >> 5], 1u << (j & 31));
    }
    __syncthreads();
    int over = 0;
    for (int i = t; i < last; i += kHBlock) {
        const int d = last - i;
        int k = 0;
        while (k < kDryDirect && d + k < dn && dry_eq(r, L.dbrk, k, d + k)) ++k;
        over |= k == kDryDirect ? 1 : 0;
        L.dlen[i] = (uint16_t)k;
    }
    if (!block_or(over, L)) return;
    // Z-function over r, one wave: z(d) = common prefix of r and r[d ..],
    // kept at dlen[last - d]; [lo, hi) is the rightmost match found so far.
    if (t < 64) {
        int lo = 0, hi = 0;
        for (int d = 1; d < dn; ++d) {
            int k = d < hi ? min(hi - d, (int)L.dlen[last - (d - lo)]) : 0;
            if (d + k >= hi) {
                for (;;) {
                    const int b = d + k + lane;
                    const bool eq = b < dn && dry_eq(r, L.dbrk, k + lane, b);
                    const uint64_t ne = __ballot(!eq);
                    if (ne) {
                        k += __ffsll((unsigned long long)ne) - 1;
                        break;
                    }
                    k += 64;
                }
                lo = d;
                hi = d + k;
            }
            if (lane == 0) L.dlen[last - d] = (uint16_t)k;
            wave_lds_sync();
        }
    }
    __syncthreads();
}

template <typename T>
__global__ __launch_bounds__(kHBlock) void history_kernel(HistArgs a) {
    __shared__ HistLds L;
    const int row = blockIdx.x, t = threadIdx.x;
    const int V = a.V;
    const tms_row_params P = a.params[row];
    const tms_history_params H = a.hp[row];
    int nrec = a.n_recent ? a.n_recent[row] : (int)a.recent_stride;
    nrec = max(0, min(nrec, (int)a.recent_stride));
    const int32_t* rec = a.recent + (int64_t)row * a.recent_stride;
    const T* base = (const T*)a.logits + (int64_t)row * a.row_stride;
    const uint32_t* mrow = a.mask + (int64_t)row * a.mask_stride;

    // ---- DRY's window and every position's match length, first: the
    //      window is staged over the table's keys, which are cleared after
    const bool dry_on = H.dry_multiplier > 0.0f && H.dry_allowed_length >= 1 &&
                        nrec >= H.dry_allowed_length + 1 &&
                        min(nrec, H.dry_penalty_last_n) >= H.dry_allowed_length + 1;
    const int dn = dry_on ? min(nrec, H.dry_penalty_last_n) : 0;
    const int32_t* dw = rec + (nrec - dn);
    const int dlast = dn - 1;
    // every exponent L - allowed_length is below dn - allowed_length
    if (dry_on && (dn > kDryMax || (a.dry_scale && a.dry_scale_stride < dn - H.dry_allowed_length))) {
        if (t == 0) a.ov_n[row] = -1;   // the row reports TMS_ROW_UNSUPPORTED
        return;
    }
    if (dry_on) dry_lengths(dw, dn, a.breaker, V, L);

    {
        uint4* k4 = (uint4*)L.key;
        uint4* i4 = (uint4*)L.info;
        for (int i = t; i < kHSlots / 4; i += kHBlock) {
            k4[i] = make_uint4(0, 0, 0, 0);
            i4[i] = make_uint4(0, 0, 0, 0);
        }
        if (t == 0) {
            L.flag = 0;
            L.found = 0;
        }
    }
    __syncthreads();
    int full = 0;

    // ---- repetition / frequency / presence window: counts per id
    Pen pn;
    pn.rep_on = !(P.repeat_penalty <= 1.0f);
    pn.fp_on = P.frequency_penalty != 0.0f || P.presence_penalty != 0.0f;
    pn.on = nrec > 0 && P.repeat_last_n > 0 && (pn.rep_on || pn.fp_on);
    pn.rep = P.repeat_penalty;
    pn.freq = P.frequency_penalty;
    pn.pres = P.presence_penalty;
    if (pn.on) {
        const int from = nrec > P.repeat_last_n ? nrec - P.repeat_last_n : 0;
        for (int p = from + t; p < nrec; p += kHBlock) {
            const int id = rec[p];
            if (id < 0 || id >= V) continue;
            const int s = hinsert(L, id);
            if (s < 0) full = 1;
            else atomicAdd(&L.info[s], 1u);
        }
    }

    // ---- n-gram ban (tmsample.h:83-101): the id after every earlier
    //      occurrence of the last m = ngram - 1 ids
    const int ng = H.no_repeat_ngram;
    if (ng >= 2 && nrec >= ng) {
        const int m = ng - 1, s0 = nrec - m;
        for (int i = t; i < s0; i += kHBlock) {
            bool same = true;
            for (int k = 0; k < m && same; ++k) same = rec[i + k] == rec[s0 + k];
            if (!same) continue;
            const int id = rec[i + m];
            if (id < 0 || id >= V) continue;
            const int s = hinsert(L, id);
            if (s < 0) full = 1;
            else atomicOr(&L.info[s], kHBan);
        }
    }

    // ---- DRY targets (tmsample.h:150-169)
    if (dry_on) {
        for (int i = t; i < dlast; i += kHBlock) {
            if (L.dlen[i] < H.dry_allowed_length) continue;
            const int id = dw[i + 1];
            if (id < 0 || id >= V || is_breaker(a.breaker, V, id)) continue;
            const int s = hinsert(L, id);
            if (s < 0) full = 1;
            else atomicOr(&L.info[s], kHDry);
        }
    }
    if (full) L.flag = 1;
    __syncthreads();

    // ---- number the slots (the list, in slot order)
    constexpr int kPer = kHSlots / kHBlock;   // 32 consecutive slots per thread
    int mine = 0;
#pragma unroll 8
    for (int j = 0; j < kPer; ++j) mine += L.key[t * kPer + j] != 0u ? 1 : 0;
    int n = 0;
    int e = hist_excl_scan(mine, n, L);
    if (L.flag || n > kHistMax) {
        if (t == 0) a.ov_n[row] = -1;   // the row reports TMS_ROW_UNSUPPORTED
        return;
    }
    for (int j = 0; j < kPer; ++j) {
        const int s = t * kPer + j;
        if (L.key[s] != 0u) {
            L.ent[s] = (uint16_t)e;
            L.eslot[e] = (uint16_t)s;
            ++e;
        }
    }
    __syncthreads();

    // ---- values after mask and penalties; is anything left after the ban?
    const float NEG_INF = -__builtin_huge_valf();
    int alive = 0, banned = 0;
    for (int i = t; i < n; i += kHBlock) {
        const int s = L.eslot[i];
        const int id = (int)L.key[s] - 1;
        const uint32_t f = L.info[s];
        const bool allowed = (mrow[id >> 5] >> (id & 31)) & 1u;
        float v = allowed ? Elt<T>::scalar(base + id) : NEG_INF;
        const uint32_t c = f & kHCount;
        if (allowed && c) v = apply_pen(v, c, pn);
        L.val[i] = v;
        if (f & kHBan) banned = 1;
        else if (v > NEG_INF) alive = 1;
    }
    banned = block_or(banned, L);
    bool restore = false;
    if (banned) {
        alive = block_or(alive, L);
        if (!alive) {
            // an allowed id outside the list with a logit above -inf?
            const int words = (V + 31) >> 5;
            for (int w0 = 0; w0 < words; w0 += kHBlock) {
                const int w = w0 + t;
                int hit = 0;
                if (w < words) {
                    uint32_t bits = mrow[w];
                    if (w == words - 1 && (V & 31)) bits &= (1u << (V & 31)) - 1u;
                    while (bits && !hit) {
                        const int id = w * 32 + __builtin_ctz(bits);
                        bits &= bits - 1u;
                        if (Elt<T>::scalar(base + id) > NEG_INF && hfind(L, id) < 0) hit = 1;
                    }
                }
                if (block_or(hit, L)) {
                    alive = 1;
                    break;
                }
            }
            restore = !alive;
        }
    }
    if (!restore) {
        for (int i = t; i < n; i += kHBlock)
            if (L.info[L.eslot[i]] & kHBan) L.val[i] = NEG_INF;
    }
    __syncthreads();

    // ---- DRY, in the reference's position order: tiles of kHBlock
    //      positions; each tile's hits are listed in order, then every DRY
    //      target entry subtracts its hits in that order.
    if (dry_on) {
        const float mult = H.dry_multiplier, dbase = H.dry_base;
        const float* scale = a.dry_scale ? a.dry_scale + (int64_t)row * a.dry_scale_stride : nullptr;
        for (int i0 = 0; i0 < dlast; i0 += kHBlock) {
            const int i = i0 + t;
            int slot = -1, k = 0;
            if (i < dlast) {
                const int Lr = L.dlen[i];
                if (Lr >= H.dry_allowed_length) {
                    const int id = dw[i + 1];
                    if (id >= 0 && id < V && !is_breaker(a.breaker, V, id)) {
                        slot = hfind(L, id);
                        k = Lr - H.dry_allowed_length;
                    }
                }
            }
            int nh = 0;
            const int pos = hist_excl_scan(slot >= 0 ? 1 : 0, nh, L);
            if (slot >= 0) {
                L.tslot[pos] = slot;
                L.tk[pos] = k;
            }
            __syncthreads();
            if (nh) {
                for (int q = t; q < n; q += kHBlock) {
                    const int s = L.eslot[q];
                    if (!(L.info[s] & kHDry)) continue;
                    float v = L.val[q];
                    for (int j = 0; j < nh; ++j)
                        if (L.tslot[j] == s)
                            v -= mult * (scale ? scale[L.tk[j]] : tms_dry_scale(dbase, L.tk[j]));
                    L.val[q] = v;
                }
            }
            __syncthreads();
        }
    }

    // ---- the list
    int32_t* oid = a.ov_ids + (int64_t)row * kHistMax;
    float* ovl = a.ov_vals + (int64_t)row * kHistMax;
    for (int i = t; i < n; i += kHBlock) {
        oid[i] = (int32_t)L.key[L.eslot[i]] - 1;
        ovl[i] = L.val[i];
    }
    if (t == 0) a.ov_n[row] = n;
}

}  // namespace tms

int tms_launch_history(const tms::KArgs& k, const tms_history_params* hp, const uint8_t* breaker,
                       const float* dry_scale, int64_t dry_scale_stride, int dtype, int batch,
                       int32_t* ov_n, int32_t* ov_ids, float* ov_vals, hipStream_t stream) {
    tms::HistArgs h;
    h.logits = k.logits;
    h.row_stride = k.row_stride;
    h.V = k.V;
    h.params = k.params;
    h.hp = hp;
    h.breaker = breaker;
    h.recent = k.recent;
    h.n_recent = k.n_recent;
    h.recent_stride = k.recent_stride;
    h.mask = k.mask;
    h.mask_stride = k.mask_stride;
    h.dry_scale = dry_scale;
    h.dry_scale_stride = dry_scale_stride;
    h.ov_n = ov_n;
    h.ov_ids = ov_ids;
    h.ov_vals = ov_vals;
    const dim3 grid((unsigned)batch), block(tms::kHBlock);
    switch (dtype) {
        case TMS_DTYPE_F32: hipLaunchKernelGGL((tms::history_kernel<float>), grid, block, 0, stream, h); break;
        case TMS_DTYPE_F16: hipLaunchKernelGGL((tms::history_kernel<_Float16>), grid, block, 0, stream, h); break;
        default: hipLaunchKernelGGL((tms::history_kernel<tms::Bf16>), grid, block, 0, stream, h); break;
    }
    return hipGetLastError() == hipSuccess ? TMS_OK : TMS_ERR_HIP;
}

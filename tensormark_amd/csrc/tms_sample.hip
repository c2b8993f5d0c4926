// tms_sample.hip -- batched token sampler for gfx950 (MI355X).
//
// One launch per call.  Row b of the batch is cut into S chunks of at most
// 16K ids; workgroup (b, c) streams its chunk from HBM once with 16-byte
// loads into registers (64 values per thread), applies the grammar mask and
// the history penalties there, and reduces the chunk to a short sorted
// candidate list in the workspace.  The last workgroup of the row to arrive
// (a per-row counter) merges the S lists and runs the sequential fp64 tail
// of tmsample::sample (tensormark/tmsample.h:184-199): softmax over the
// top-k, top-p and min-p cuts, and the inverse-CDF draw.
//
// Row modes (uniform per workgroup):
//   greedy  the chunk's best (value, lowest id); the merge takes the best.
//   top-k   K <= kTopkFast: the chunk's exact top-K by (v / T desc, id asc).
//           A threshold from the per-thread maxima bounds the candidates,
//           so only they are divided by T.  An exact radix select over the
//           chunk (re-read from L2) is the fallback when it admits too many.
//   top-p   K > kTopkFast (top_k = 0 or large): every chunk entry whose
//           probability can change the fp64 sums, i.e. v / T within 40 of
//           the chunk maximum (exp(-40) < 2^-57); rows with more than the
//           capacity report TMS_ROW_UNSUPPORTED.
//
// Cross-workgroup traffic (lists, counts, the arrival counter) uses relaxed
// agent-scope atomics, which are coherent across the XCDs' L2 caches, with
// the stores drained (s_waitcnt) before the arrival is counted; no L2
// write-back or invalidate is needed.

#include <float.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/tmsample_hip.h"
#include "tms_device.h"

namespace tms {

constexpr int kEpt = 64;                   // logits per thread held in registers
constexpr int kChunk = kBlock * kEpt;      // ids per workgroup
constexpr int kTopkFast = 128;             // largest K on the threshold path
constexpr int kCand = 512;                 // chunk candidates held in LDS
constexpr int kMergeCap = 1024;            // candidates per merge round
constexpr int kMaxChunks = 64;             // chunks per row (vocab <= 1,048,576)
constexpr float kSigSpan = 40.0f;          // exp(-40) < 2^-57: below this, no effect

enum : int { MODE_GREEDY = 0, MODE_TOPK = 1, MODE_TOPP = 2 };
enum : int { FLAG_NONFINITE = 1, FLAG_OVERFLOW = 2 };

struct KArgs {
    const void* logits;
    int64_t row_stride;
    int V;
    int S;            // chunks per row
    int CE;           // ids per chunk (multiple of the vector width)
    int aligned;      // rows start on 16-byte boundaries
    const tms_row_params* params;
    const int32_t* recent;
    const int32_t* n_recent;
    int64_t recent_stride;
    const uint32_t* mask;
    int64_t mask_stride;
    const uint32_t* draws;
    int32_t* out_tokens;
    int32_t* out_status;
    int32_t* out_keep;
    int32_t* out_topk_ids;
    float* out_topk_probs;
    int topk_cap;
    // workspace
    uint32_t* counters;    // [B] arrival counters, self-resetting
    int32_t* chunk_n;      // [B][S] entries per chunk list
    int32_t* chunk_flags;  // [B][S]
    uint64_t* lists;       // [B][S][kCand]
};

struct Bf16 {
    uint16_t bits;
};

// Element types: vector width of a 16-byte load, exact widening to fp32.
template <typename T>
struct Elt;
template <>
struct Elt<float> {
    static constexpr int kVec = 4;
    __device__ static void widen(const uint4& q, float (&f)[4]) {
        f[0] = __uint_as_float(q.x);
        f[1] = __uint_as_float(q.y);
        f[2] = __uint_as_float(q.z);
        f[3] = __uint_as_float(q.w);
    }
    __device__ static float scalar(const float* p) { return *p; }
};
template <>
struct Elt<_Float16> {
    static constexpr int kVec = 8;
    __device__ static float h2f(uint32_t h) {
        _Float16 v;
        const uint16_t b = (uint16_t)h;
        __builtin_memcpy(&v, &b, 2);
        return (float)v;
    }
    __device__ static void widen(const uint4& q, float (&f)[8]) {
        const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            f[2 * i] = h2f(w[i] & 0xFFFFu);
            f[2 * i + 1] = h2f(w[i] >> 16);
        }
    }
    __device__ static float scalar(const _Float16* p) { return (float)*p; }
};
template <>
struct Elt<Bf16> {
    static constexpr int kVec = 8;
    __device__ static void widen(const uint4& q, float (&f)[8]) {
        const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            f[2 * i] = __uint_as_float(w[i] << 16);
            f[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
        }
    }
    __device__ static float scalar(const Bf16* p) { return __uint_as_float((uint32_t)p->bits << 16); }
};

// History penalties of one row.
struct Pen {
    bool on, rep_on, fp_on;
    float rep, freq, pres;
};

// Repetition penalty applied `cnt` times (tmsample.h:61), then frequency and
// presence: v -= (float)cnt * freq + presence.
__device__ __forceinline__ float apply_pen(float v, uint32_t cnt, const Pen& pn) {
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
            uint64_t uni[kMergeCap];      // the round's lists; then pr[] of the tail
            uint64_t sorted[kMergeCap];
            double q[kMergeCap];
        } m;
    } big;
    uint64_t cand[kCand];
    int wave_i[kWaves];
    float wave_f[kWaves];
    uint64_t wave_k[kWaves];
    int list_off[kMaxChunks + 2];
    int list_src[kMaxChunks + 1];
    int list_n[kMaxChunks];
    int hist[256];
    int ncand;
    int misc[8];
};

__device__ __forceinline__ int block_excl_scan(int v, int& total, Smem& sm) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int inc = wave_incl_scan_i32(v);
    if (lane == 63) sm.wave_i[w] = inc;
    __syncthreads();
    int base = 0;
    total = 0;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) {
        const int t = sm.wave_i[i];
        base += i < w ? t : 0;
        total += t;
    }
    __syncthreads();
    return base + inc - v;
}

__device__ __forceinline__ uint64_t block_max_u64(uint64_t v, Smem& sm) {
    v = wave_max_u64(v);
    if ((threadIdx.x & 63) == 0) sm.wave_k[threadIdx.x >> 6] = v;
    __syncthreads();
    uint64_t r = sm.wave_k[0];
#pragma unroll
    for (int i = 1; i < kWaves; ++i) r = sm.wave_k[i] > r ? sm.wave_k[i] : r;
    __syncthreads();
    return r;
}

__device__ __forceinline__ float block_max_f32(float v, Smem& sm) {
    v = wave_max_f32(v);
    if ((threadIdx.x & 63) == 0) sm.wave_f[threadIdx.x >> 6] = v;
    __syncthreads();
    float r = sm.wave_f[0];
#pragma unroll
    for (int i = 1; i < kWaves; ++i) r = fmaxf(r, sm.wave_f[i]);
    __syncthreads();
    return r;
}

__device__ __forceinline__ int block_or(int v, Smem& sm) {
    const bool any = __any(v != 0);
    if ((threadIdx.x & 63) == 0) sm.wave_i[threadIdx.x >> 6] = any ? 1 : 0;
    __syncthreads();
    int r = 0;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) r |= sm.wave_i[i];
    __syncthreads();
    return r;
}

// Sort sm.cand[0..n) descending in place (n <= kCand): one wave's bitonic
// network for n <= 64, ranking by counting otherwise.
__device__ void sort_cand(int n, Smem& sm) {
    const int t = threadIdx.x;
    if (n <= 1) return;
    if (n <= 64) {
        if (t < 64) {
            uint64_t k = t < n ? sm.cand[t] : 0ull;
            k = wave_sort_desc_u64(k);
            if (t < n) sm.cand[t] = k;
        }
        __syncthreads();
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
#pragma unroll 4
        for (int j = 0; j < n; ++j) rank[0] += sm.cand[j] > mine[0] ? 1 : 0;
    } else {
#pragma unroll 4
        for (int j = 0; j < n; ++j) {
            const uint64_t o = sm.cand[j];
#pragma unroll
            for (int r = 0; r < R; ++r) rank[r] += o > mine[r] ? 1 : 0;
        }
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < R; ++r)
        if (t + r * kBlock < n) sm.cand[rank[r]] = mine[r];
    __syncthreads();
}

// The final value of chunk id `id` (mask, then penalties from the LDS
// window counts), read again from memory: the slow paths use it.
template <typename T>
__device__ float slow_value(const T* base, const uint32_t* mrow, int id, int e0, const Pen& pn,
                            const Smem& sm) {
    float v = Elt<T>::scalar(base + id);
    if (mrow && !((mrow[id >> 5] >> (id & 31)) & 1u)) return -__builtin_huge_valf();
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
// returns the count (<= K).
template <typename T>
__device__ int radix_slow(const T* base, const uint32_t* mrow, int e0, int e1, int K, float temp,
                          bool divide, const Pen& pn, Smem& sm) {
    const int t = threadIdx.x;
    const float NEG_INF = -__builtin_huge_valf();
    uint32_t prefix = 0, pmask = 0;
    int remaining = K;
    for (int shift = 24; shift >= 0; shift -= 8) {
        sm.hist[t] = 0;
        if (t == 0) sm.ncand = 0;
        __syncthreads();
        for (int id = e0 + t; id < e1; id += kBlock) {
            const float v = slow_value(base, mrow, id, e0, pn, sm);
            if (v == NEG_INF) continue;
            const uint32_t k = okey(divide ? v / temp : v);
            if ((k & pmask) == prefix) atomicAdd(&sm.hist[(k >> shift) & 0xFF], 1);
        }
        __syncthreads();
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
            __syncthreads();
            return sm.ncand;
        }
        if (above < remaining && above + h >= remaining) {
            sm.misc[0] = 255 - t;
            sm.misc[1] = above;
        }
        __syncthreads();
        remaining -= sm.misc[1];
        prefix |= (uint32_t)sm.misc[0] << shift;
        pmask |= 0xFFu << shift;
        __syncthreads();
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
    __syncthreads();
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
    __syncthreads();
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

template <typename U>
__device__ __forceinline__ void st_agent(U* p, U v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename U>
__device__ __forceinline__ U ld_agent(const U* p) {
    return __hip_atomic_load(const_cast<U*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <typename T>
__global__ __launch_bounds__(kBlock) void sample_kernel(KArgs a) {
    constexpr int VEC = Elt<T>::kVec;
    constexpr int NVT = kEpt / VEC;
    __shared__ Smem sm;
    const float NEG_INF = -__builtin_huge_valf();
    const int t = threadIdx.x;
    const int lane = t & 63, wv = t >> 6;
    const int S = a.S;
    const int row = blockIdx.x / S;
    const int c = blockIdx.x - row * S;
    const int V = a.V;
    const tms_row_params P = a.params[row];

    const bool greedy = P.greedy != 0;
    const bool bad_params = !greedy && !(P.temperature > 0.0f && P.temperature <= FLT_MAX);
    const int K = greedy ? 1 : ((P.top_k <= 0 || P.top_k > V) ? V : P.top_k);
    const int mode = greedy ? MODE_GREEDY : (K <= kTopkFast ? MODE_TOPK : MODE_TOPP);
    const float temp = P.temperature;
    const bool divide = !greedy && temp != 1.0f;

    // ---- history window: its ids are loaded before the logits so that the
    //      wait for them does not also wait for the logits.
    int nrec = 0;
    if (a.recent) {
        nrec = a.n_recent ? a.n_recent[row] : (int)a.recent_stride;
        if (nrec > (int)a.recent_stride) nrec = (int)a.recent_stride;
    }
    Pen pn;
    pn.rep_on = !(P.repeat_penalty <= 1.0f);
    pn.fp_on = P.frequency_penalty != 0.0f || P.presence_penalty != 0.0f;
    pn.on = nrec > 0 && P.repeat_last_n > 0 && (pn.rep_on || pn.fp_on);
    pn.rep = P.repeat_penalty;
    pn.freq = P.frequency_penalty;
    pn.pres = P.presence_penalty;
    const int from = pn.on ? (nrec > P.repeat_last_n ? nrec - P.repeat_last_n : 0) : 0;
    const int e0 = c * a.CE;
    const int e1 = min(e0 + a.CE, V);
    const int nvec = (e1 - e0 + VEC - 1) / VEC;
    const int32_t* hist = pn.on ? a.recent + (int64_t)row * a.recent_stride : nullptr;
    constexpr int kWin = 4;   // window ids per thread per pass
    int wid[kWin];
#pragma unroll
    for (int i = 0; i < kWin; ++i) {
        const int p = from + t + i * kBlock;
        wid[i] = (pn.on && p < nrec) ? hist[p] : -1;
    }

    // ---- stream the chunk: one mask word and one 16-byte vector per slot.
    const T* base = (const T*)a.logits + (int64_t)row * a.row_stride;
    const uint32_t* mrow = a.mask ? a.mask + (int64_t)row * a.mask_stride : nullptr;
    uint4 raw[NVT];
    uint32_t mw[NVT];
#pragma unroll
    for (int j = 0; j < NVT; ++j) {
        const int v = t + j * kBlock;
        const int eb = e0 + v * VEC;
        mw[j] = 0xFFFFFFFFu;
        raw[j] = make_uint4(0, 0, 0, 0);
        if (v < nvec) {
            if (mrow) mw[j] = mrow[eb >> 5];
            if (a.aligned && eb + VEC <= e1) raw[j] = *(const uint4*)(base + eb);
        }
    }

    // ---- window counts: 16 bits per chunk id in LDS.
    if (t == 0) sm.ncand = 0;
    if (pn.on) {
        uint4* c4 = (uint4*)sm.big.cnt;
        for (int i = t; i < kChunk / 8; i += kBlock) c4[i] = make_uint4(0, 0, 0, 0);
        __syncthreads();
        for (int p0 = from; p0 < nrec; p0 += kBlock * kWin) {
#pragma unroll
            for (int i = 0; i < kWin; ++i) {
                int id;
                if (p0 == from) {
                    id = wid[i];
                } else {
                    const int p = p0 + t + i * kBlock;
                    id = p < nrec ? hist[p] : -1;
                }
                if (id >= e0 && id < e1) {
                    const int off = id - e0;
                    atomicAdd(&sm.big.cnt[off >> 1], 1u << ((off & 1) * 16));
                }
            }
        }
        __syncthreads();
    }

    // ---- per vector: widen, mask, penalties, checks, thread maximum.
    float x[kEpt];
    int nonfinite = 0;
    float tmax = NEG_INF;
#pragma unroll
    for (int j = 0; j < NVT; ++j) {
        const int v = t + j * kBlock;
        const int eb = e0 + v * VEC;
        float f[VEC];
        if (a.aligned && eb + VEC <= e1) {
            Elt<T>::widen(raw[j], f);
        } else {
#pragma unroll
            for (int e = 0; e < VEC; ++e)
                f[e] = (v < nvec && eb + e < e1) ? Elt<T>::scalar(base + eb + e) : NEG_INF;
        }
        const uint32_t mb = mw[j] >> (eb & 31);
#pragma unroll
        for (int e = 0; e < VEC; ++e) f[e] = ((mb >> e) & 1u) ? f[e] : NEG_INF;
        if (pn.on && v < nvec) {
            uint32_t cw[VEC / 2];
            uint32_t any = 0;
#pragma unroll
            for (int i = 0; i < VEC / 2; ++i) {
                cw[i] = sm.big.cnt[((eb - e0) >> 1) + i];
                any |= cw[i];
            }
            if (any) {
#pragma unroll
                for (int e = 0; e < VEC; ++e) {
                    const uint32_t cnt = (cw[e >> 1] >> ((e & 1) * 16)) & 0xFFFFu;
                    if (cnt) f[e] = apply_pen(f[e], cnt, pn);
                }
            }
        }
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
            nonfinite |= (f[e] != f[e]) | (f[e] == __builtin_huge_valf());
            tmax = fmaxf(tmax, f[e]);
            x[j * VEC + e] = f[e];
        }
    }
    const int flags_nf = block_or(nonfinite, sm) ? FLAG_NONFINITE : 0;
    int flags = flags_nf;
    int nout = 0;   // entries of sm.cand this chunk publishes

    if (!bad_params && !flags_nf) {
        if (mode == MODE_GREEDY) {
            uint64_t gb = 0;
#pragma unroll
            for (int j = 0; j < NVT; ++j) {
#pragma unroll
                for (int e = 0; e < VEC; ++e) {
                    const float f = x[j * VEC + e];
                    const uint64_t k =
                        f != NEG_INF ? ckey(f, (uint32_t)(e0 + (t + j * kBlock) * VEC + e)) : 0ull;
                    gb = k > gb ? k : gb;
                }
            }
            const uint64_t b = block_max_u64(gb, sm);
            if (t == 0 && b) sm.cand[0] = b;
            nout = b ? 1 : 0;
            __syncthreads();
        } else if (mode == MODE_TOPK) {
            // tau: at least K chunk entries are >= tau.  Each wave sorts its 64
            // thread maxima; its ceil(K/4)-th is >= tau for 4 * ceil(K/4) >= K
            // threads, each holding an entry >= tau.
            const int kw = (K + kWaves - 1) / kWaves;
            const float srt = wave_sort_desc_f32(tmax);
            const float tw = __shfl(srt, kw - 1, 64);
            if (lane == 0) sm.wave_f[wv] = tw;
            __syncthreads();
            float tau = sm.wave_f[0];
#pragma unroll
            for (int i = 1; i < kWaves; ++i) tau = fminf(tau, sm.wave_f[i]);
            // Division can merge neighbouring values: lower tau to the smallest
            // float with the same quotient, so every entry tying the K-th
            // quotient is a candidate.
            bool fallback = false;
            if (divide && tau != NEG_INF) {
                const float q = tau / temp;
                int it = 0;
                for (; it < 64; ++it) {
                    const float p = nextafterf(tau, NEG_INF);
                    if (p / temp == q) tau = p;
                    else break;
                }
                fallback = it == 64;
            }
            if (!fallback) {
#pragma unroll
                for (int j = 0; j < NVT; ++j) {
                    float vm = x[j * VEC];
#pragma unroll
                    for (int e = 1; e < VEC; ++e) vm = fmaxf(vm, x[j * VEC + e]);
                    if (vm != NEG_INF && vm >= tau) {
#pragma unroll
                        for (int e = 0; e < VEC; ++e) {
                            const float f = x[j * VEC + e];
                            if (f != NEG_INF && f >= tau) {
                                const int pos = atomicAdd(&sm.ncand, 1);
                                if (pos < kCand)
                                    sm.cand[pos] = ckey(divide ? f / temp : f,
                                                        (uint32_t)(e0 + (t + j * kBlock) * VEC + e));
                            }
                        }
                    }
                }
            }
            __syncthreads();
            const int n = sm.ncand;
            __syncthreads();
            if (fallback || n > kCand) {
                nout = radix_slow<T>(base, mrow, e0, e1, K, temp, divide, pn, sm);
                sort_cand(nout, sm);
            } else {
                sort_cand(n, sm);
                nout = n < K ? n : K;
            }
        } else {
            // Top-p only: entries within kSigSpan of the chunk maximum (in v / T).
            const float cmax = block_max_f32(tmax, sm);
            if (cmax != NEG_INF) {
                const float lmax = divide ? cmax / temp : cmax;
                const double lthr = (double)lmax - (double)kSigSpan;
                // Generous prefilter in v, exact test on the quotient.
                const float vthr = __double2float_rd(
                    ((double)lmax - (double)kSigSpan - 1.0 - fabs((double)lmax) * 0x1p-20) *
                    (double)temp);
#pragma unroll
                for (int j = 0; j < NVT; ++j) {
                    float vm = x[j * VEC];
#pragma unroll
                    for (int e = 1; e < VEC; ++e) vm = fmaxf(vm, x[j * VEC + e]);
                    if (vm != NEG_INF && vm >= vthr) {
#pragma unroll
                        for (int e = 0; e < VEC; ++e) {
                            const float f = x[j * VEC + e];
                            if (f != NEG_INF && f >= vthr) {
                                const float lg = divide ? f / temp : f;
                                if ((double)lg >= lthr) {
                                    const int pos = atomicAdd(&sm.ncand, 1);
                                    if (pos < kCand)
                                        sm.cand[pos] =
                                            ckey(lg, (uint32_t)(e0 + (t + j * kBlock) * VEC + e));
                                }
                            }
                        }
                    }
                }
                __syncthreads();
                const int n = sm.ncand;
                __syncthreads();
                if (n > kCand) {
                    flags |= FLAG_OVERFLOW;
                    nout = 0;
                } else {
                    sort_cand(n, sm);
                    nout = n;
                }
            }
        }
    }

    // ---- publish the chunk list (wave 0), then count the row's arrivals.
    if (wv == 0) {
        uint64_t* my_list = a.lists + ((int64_t)row * S + c) * kCand;
        for (int i = lane; i < nout; i += 64) st_agent(&my_list[i], sm.cand[i]);
        if (lane == 0) {
            st_agent(&a.chunk_n[row * S + c], (int32_t)nout);
            st_agent(&a.chunk_flags[row * S + c], (int32_t)flags);
        }
        __builtin_amdgcn_s_waitcnt(0);   // the stores above are complete
        if (lane == 0) {
            const uint32_t prev =
                __hip_atomic_fetch_add(&a.counters[row], 1u, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
            sm.misc[0] = prev == (uint32_t)(S - 1) ? 1 : 0;
        }
    }
    __syncthreads();
    if (!sm.misc[0]) return;

    // ================= merge: the last workgroup of the row =================
    int any_flags = 0;
    if (t < S) {
        sm.list_n[t] = ld_agent(&a.chunk_n[row * S + t]);
        any_flags = ld_agent(&a.chunk_flags[row * S + t]);
    }
    if (t == 0) st_agent(&a.counters[row], 0u);   // ready for the next launch
    const int fl = block_or(any_flags & FLAG_NONFINITE, sm);
    const int ov = block_or(any_flags & FLAG_OVERFLOW, sm);
    if (t == 0) {
        int tot = 0;
        for (int i = 0; i < S; ++i) tot += sm.list_n[i];
        sm.misc[5] = tot;
    }
    __syncthreads();
    const int N = sm.misc[5];   // finite candidates over all chunk lists

    int status = TMS_ROW_OK;
    if (bad_params) status = TMS_ROW_BAD_PARAMS;
    else if (fl) status = TMS_ROW_NONFINITE;
    else if (ov || (mode == MODE_TOPP && N > kMergeCap)) status = TMS_ROW_UNSUPPORTED;
    else if (N == 0) status = TMS_ROW_ALL_MASKED;
    if (status != TMS_ROW_OK) {
        write_row_error(a, row, status);
        return;
    }

    // Merge in rounds: the running top list (sorted[0..n_acc)) plus as many
    // chunk lists as fit in kMergeCap; every entry is ranked against the
    // other lists of the round by binary search.  Top-k rows keep the best
    // K after each round (K + one list always fits); top-p rows have
    // N <= kMergeCap and finish in one round.
    const uint64_t* row_lists = a.lists + (int64_t)row * S * kCand;
    const int keep_cap = mode == MODE_TOPP ? kMergeCap : K;
    int n_acc = 0;
    int c_next = 0;
    while (c_next < S) {
        if (t == 0) {
            int off = n_acc, g = 1, cc = c_next;
            sm.list_off[0] = 0;
            sm.list_off[1] = n_acc;
            sm.list_src[0] = -1;
            while (cc < S && off + sm.list_n[cc] <= kMergeCap) {
                off += sm.list_n[cc];
                sm.list_src[g] = cc;
                sm.list_off[++g] = off;
                ++cc;
            }
            sm.misc[6] = g;
            sm.misc[7] = cc;
        }
        __syncthreads();
        const int ng = sm.misc[6];
        const int total = sm.list_off[ng];
        for (int i = t; i < total; i += kBlock) {
            int lc = 0;
            while (sm.list_off[lc + 1] <= i) ++lc;
            const int src = sm.list_src[lc];
            sm.big.m.uni[i] =
                src < 0 ? sm.big.m.sorted[i]
                        : ld_agent(&row_lists[(int64_t)src * kCand + (i - sm.list_off[lc])]);
        }
        __syncthreads();
        const int nkeep = total < keep_cap ? total : keep_cap;
        for (int i = t; i < total; i += kBlock) {
            int lc = 0;
            while (sm.list_off[lc + 1] <= i) ++lc;
            const uint64_t k = sm.big.m.uni[i];
            int rank = i - sm.list_off[lc];
            for (int o = 0; o < ng; ++o) {
                if (o == lc) continue;
                rank += count_greater(sm.big.m.uni + sm.list_off[o],
                                      sm.list_off[o + 1] - sm.list_off[o], k);
            }
            if (rank < nkeep) sm.big.m.sorted[rank] = k;
        }
        c_next = sm.misc[7];
        n_acc = nkeep;
        __syncthreads();
    }

    int32_t* topk_ids = a.out_topk_ids ? a.out_topk_ids + (int64_t)row * a.topk_cap : nullptr;
    float* topk_probs = a.out_topk_probs ? a.out_topk_probs + (int64_t)row * a.topk_cap : nullptr;
    const uint64_t* srt = sm.big.m.sorted;

    if (mode == MODE_GREEDY) {
        const int tok = (int)ckey_id(srt[0]);
        if (t == 0) {
            a.out_tokens[row] = tok;
            a.out_status[row] = TMS_ROW_OK;
            if (a.out_keep) a.out_keep[row] = 0;
        }
        for (int i = t; i < a.topk_cap; i += kBlock) {
            if (topk_ids) topk_ids[i] = i == 0 ? tok : -1;
            if (topk_probs) topk_probs[i] = i == 0 ? 1.0f : 0.0f;
        }
        return;
    }

    // Entries the tail walks.  Top-k rows with fewer than K finite ids go on
    // with -inf entries in ascending id order: the ids missing from the
    // finite set, which is then complete.
    int n = n_acc;
    if (mode == MODE_TOPK && N < K) {
        // ids in [0, K + N) absent from the N finite ones, lowest first
        // (K + N < 2 * kTopkFast <= kBlock: one id per thread).
        const int q = t;
        int member = 0;
        if (q < K + N)
            for (int i = 0; i < N; ++i) member |= (int)ckey_id(srt[i]) == q;
        const int gap = (q < K + N && !member && q < V) ? 1 : 0;
        int tot;
        const int p = block_excl_scan(gap, tot, sm);
        if (gap && p < K - N) sm.big.m.sorted[N + p] = ckey(NEG_INF, (uint32_t)q);
        __syncthreads();
        n = K;
    }
    const float mx = ckey_val(srt[0]);
    if (mx == __builtin_huge_valf()) {
        write_row_error(a, row, TMS_ROW_NONFINITE);
        return;
    }
    // Top-p rows: only the prefix within kSigSpan of the maximum is exact.
    if (mode == MODE_TOPP) {
        int sig = 0;
        for (int i = t; i < n; i += kBlock)
            sig += ((double)ckey_val(srt[i]) - (double)mx >= -(double)kSigSpan) ? 1 : 0;
        sig = wave_sum_i32(sig);
        if (lane == 0) sm.wave_i[wv] = sig;
        __syncthreads();
        n = sm.wave_i[0] + sm.wave_i[1] + sm.wave_i[2] + sm.wave_i[3];
        __syncthreads();
    }

    // pr[i] = exp(lg_i - mx) in fp64 (tmsample.h:188-189).
    double* pr = (double*)sm.big.m.uni;   // the round's lists are no longer needed
    double* q = sm.big.m.q;
    for (int i = t; i < n; i += kBlock) pr[i] = exp((double)ckey_val(srt[i]) - (double)mx);
    __syncthreads();
    if (wv != 0) return;

    // The sequential fp64 tail runs in wave 0; every lane walks the same
    // LDS entries (broadcast reads), so the sums are formed in the
    // reference's order.
    double z = 0;
#pragma unroll 8
    for (int i = 0; i < n; ++i) z += pr[i];               // tmsample.h:186-191
    for (int i = lane; i < n; i += 64) q[i] = pr[i] / z;
    wave_lds_sync();
    int kp = K;
    {
        double cum = 0;
        const double tp = (double)P.top_p;
        for (int i = 0; i < n; ++i) {                       // tmsample.h:192-197
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
        if (m >= n && n < K && mp <= 4.248354255291589e-18) m = K;   // exp(-40)
        if (m < kp) kp = m;
    }
    const int keep = kp;
    const int lim = keep < n ? keep : n;
    int tokidx = 0;
    if (keep >= 2) {
        // std::discrete_distribution over pr[0..keep): sum, normalise,
        // partial sums with the last forced to 1, lower_bound(u).
        double sum = 0;
#pragma unroll 8
        for (int i = 0; i < lim; ++i) sum += pr[i];
        wave_lds_sync();
        for (int i = lane; i < lim; i += 64) q[i] = pr[i] / sum;
        wave_lds_sync();
        uint32_t w0, w1;
        if (a.draws) {
            w0 = a.draws[2 * row];
            w1 = a.draws[2 * row + 1];
        } else {
            row_words(P.seed, P.offset, 0u, w0, w1);
        }
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
    // tokidx >= n only on top-p rows whose draw fell past the last entry that
    // moves the sums: the reference then returns its K-th entry, which this
    // row does not hold.
    const bool lost = tokidx >= n;
    if (lane == 0) {
        a.out_tokens[row] = lost ? -1 : (int)ckey_id(srt[tokidx]);
        a.out_status[row] = lost ? TMS_ROW_UNSUPPORTED : TMS_ROW_OK;
        if (a.out_keep) a.out_keep[row] = keep;
    }
    for (int i = lane; i < a.topk_cap; i += 64) {
        const bool have = i < n;
        if (topk_ids) topk_ids[i] = have ? (int)ckey_id(srt[i]) : -1;
        if (topk_probs) topk_probs[i] = have ? (float)(pr[i] / z) : 0.0f;
    }
}

}  // namespace tms

// ============================================================== C ABI

struct tms_context {
    int device;
    int max_batch;
    int max_vocab;
    int max_chunks;
    size_t bytes;
    void* ws;
    uint32_t* counters;
    int32_t* chunk_n;
    int32_t* chunk_flags;
    uint64_t* lists;
};

extern "C" int tms_abi_version(void) { return TMS_ABI_VERSION; }

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
    const size_t off_n = 256 * ((nb * 4 + 255) / 256);
    const size_t off_f = off_n + 256 * ((nc * 4 + 255) / 256);
    const size_t off_l = off_f + 256 * ((nc * 4 + 255) / 256);
    ctx->bytes = off_l + nc * tms::kCand * sizeof(uint64_t);
    int rc = TMS_OK;
    if (hipMalloc(&ctx->ws, ctx->bytes) != hipSuccess) rc = TMS_ERR_HIP;
    else if (hipMemset(ctx->ws, 0, off_l) != hipSuccess) rc = TMS_ERR_HIP;
    else if (hipDeviceSynchronize() != hipSuccess) rc = TMS_ERR_HIP;
    if (rc != TMS_OK) {
        if (ctx->ws) (void)hipFree(ctx->ws);
        delete ctx;
        (void)hipSetDevice(prev);
        return rc;
    }
    char* p = (char*)ctx->ws;
    ctx->counters = (uint32_t*)p;
    ctx->chunk_n = (int32_t*)(p + off_n);
    ctx->chunk_flags = (int32_t*)(p + off_f);
    ctx->lists = (uint64_t*)(p + off_l);
    (void)hipSetDevice(prev);
    *out = ctx;
    return TMS_OK;
}

extern "C" int tms_destroy(tms_context* ctx) {
    if (!ctx) return TMS_ERR_INVALID_ARG;
    int prev = 0;
    (void)hipGetDevice(&prev);
    (void)hipSetDevice(ctx->device);
    const hipError_t e = hipFree(ctx->ws);
    (void)hipSetDevice(prev);
    delete ctx;
    return e == hipSuccess ? TMS_OK : TMS_ERR_HIP;
}

extern "C" size_t tms_workspace_bytes(const tms_context* ctx) { return ctx ? ctx->bytes : 0; }

extern "C" int tms_sample_batch(tms_context* ctx, const tms_sample_args* a, hipStream_t stream) {
    if (!ctx || !a || !a->logits || !a->params || !a->out_tokens || !a->out_status)
        return TMS_ERR_INVALID_ARG;
    if (a->batch <= 0 || a->vocab <= 0 || a->row_stride < a->vocab) return TMS_ERR_INVALID_ARG;
    if (a->batch > ctx->max_batch || a->vocab > ctx->max_vocab) return TMS_ERR_CAPACITY;
    if (a->mask && a->mask_stride < (a->vocab + 31) / 32) return TMS_ERR_INVALID_ARG;
    // Window counts are 16-bit per id in LDS.
    if (a->recent && (a->recent_stride <= 0 || a->recent_stride > 65535)) return TMS_ERR_INVALID_ARG;
    if ((a->out_topk_ids || a->out_topk_probs) && a->topk_cap <= 0) return TMS_ERR_INVALID_ARG;
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
    k.aligned = ((uintptr_t)a->logits % 16 == 0) && ((a->row_stride * esz) % 16 == 0);
    k.params = a->params;
    k.recent = a->recent;
    k.n_recent = a->n_recent;
    k.recent_stride = a->recent_stride;
    k.mask = a->mask;
    k.mask_stride = a->mask_stride;
    k.draws = a->draws;
    k.out_tokens = a->out_tokens;
    k.out_status = a->out_status;
    k.out_keep = a->out_keep;
    k.out_topk_ids = a->out_topk_ids;
    k.out_topk_probs = a->out_topk_probs;
    k.topk_cap = (a->out_topk_ids || a->out_topk_probs) ? a->topk_cap : 0;
    k.counters = ctx->counters;
    k.chunk_n = ctx->chunk_n;
    k.chunk_flags = ctx->chunk_flags;
    k.lists = ctx->lists;
    const dim3 grid((unsigned)(a->batch * k.S)), block(tms::kBlock);
    switch (a->dtype) {
        case TMS_DTYPE_F32:
            hipLaunchKernelGGL(tms::sample_kernel<float>, grid, block, 0, stream, k);
            break;
        case TMS_DTYPE_F16:
            hipLaunchKernelGGL(tms::sample_kernel<_Float16>, grid, block, 0, stream, k);
            break;
        default:
            hipLaunchKernelGGL(tms::sample_kernel<tms::Bf16>, grid, block, 0, stream, k);
            break;
    }
    return hipGetLastError() == hipSuccess ? TMS_OK : TMS_ERR_HIP;
}

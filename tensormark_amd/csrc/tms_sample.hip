// tms_sample.hip -- batched token sampler for gfx950 (MI355X).
//
// One launch per call.  Row b of the batch is cut into S chunks of about
// 16K ids; workgroup (b, c) streams its chunk from HBM once with 16-byte
// loads into registers (64 values per thread), applies the grammar mask and
// the history penalties there, and reduces the chunk to a short sorted
// candidate list in the workspace.  The last workgroup of the row to finish
// (a per-row arrival counter) merges the S lists and runs the sequential
// fp64 tail of tmsample::sample (tensormark/tmsample.h:184-199): softmax over
// the top-k, top-p and min-p cuts, and the inverse-CDF draw.
//
// Row modes (uniform per workgroup):
//   greedy  the chunk's best (value, lowest id); merge takes the best.
//   top-k   K <= kTopkFast: the chunk's exact top-K by (v / T desc, id asc).
//           A threshold from the per-thread maxima bounds the candidates,
//           so only they are divided by T; a radix select over the chunk
//           is the fallback when the threshold admits too many.
//   top-p   K > kTopkFast (top_k = 0 or large): every chunk entry whose
//           probability can change the fp64 sums, i.e. v / T within 40 of
//           the chunk maximum (exp(-40) < 2^-57); rows with more than the
//           capacity report TMS_ROW_UNSUPPORTED.

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
constexpr int kMergeCap = 1024;            // candidates per row at the merge
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

// Widen element e of a 16-byte vector (exact for all three types).
template <typename T>
__device__ __forceinline__ float widen(const uint4& q, int e);
template <>
__device__ __forceinline__ float widen<float>(const uint4& q, int e) {
    const uint32_t w = e == 0 ? q.x : e == 1 ? q.y : e == 2 ? q.z : q.w;
    return __uint_as_float(w);
}
template <>
__device__ __forceinline__ float widen<_Float16>(const uint4& q, int e) {
    const uint32_t w = (e >> 1) == 0 ? q.x : (e >> 1) == 1 ? q.y : (e >> 1) == 2 ? q.z : q.w;
    const uint16_t h = (e & 1) ? (uint16_t)(w >> 16) : (uint16_t)w;
    _Float16 f;
    __builtin_memcpy(&f, &h, 2);
    return (float)f;
}
template <>
__device__ __forceinline__ float widen<Bf16>(const uint4& q, int e) {
    const uint32_t w = (e >> 1) == 0 ? q.x : (e >> 1) == 1 ? q.y : (e >> 1) == 2 ? q.z : q.w;
    return __uint_as_float((e & 1) ? (w & 0xFFFF0000u) : (w << 16));
}

template <typename T>
__device__ __forceinline__ float load_scalar(const T* p);
template <>
__device__ __forceinline__ float load_scalar<float>(const float* p) { return *p; }
template <>
__device__ __forceinline__ float load_scalar<_Float16>(const _Float16* p) { return (float)*p; }
template <>
__device__ __forceinline__ float load_scalar<Bf16>(const Bf16* p) {
    return __uint_as_float((uint32_t)p->bits << 16);
}

// Shared memory of one workgroup.  `big` holds the chunk's penalty counts
// (16-bit per id) during the scan and the merge's lists afterwards.
struct Smem {
    union {
        uint32_t cnt[kChunk / 2];
        struct {
            uint64_t uni[kMergeCap];      // the gathered lists; then pr[]
            uint64_t sorted[kMergeCap];
            double q[kMergeCap];
        } m;
    } big;
    uint64_t cand[kCand];
    int wave_i[kWaves * 2];
    float wave_f[kWaves];
    uint64_t wave_k[kWaves];
    int list_off[kMaxChunks + 1];
    int hist[256];
    int misc[8];
    double dmisc[4];
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

// Sort sm.cand[0..n) descending in place (n <= kCand).  One wave sorts up to
// 64 keys in registers; larger sets are ranked by counting.
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
    uint64_t mine[kCand / kBlock];
    int rank[kCand / kBlock];
#pragma unroll
    for (int r = 0; r < kCand / kBlock; ++r) {
        const int i = t + r * kBlock;
        mine[r] = i < n ? sm.cand[i] : 0ull;
        rank[r] = 0;
    }
    for (int j = 0; j < n; ++j) {
        const uint64_t o = sm.cand[j];
#pragma unroll
        for (int r = 0; r < kCand / kBlock; ++r) rank[r] += o > mine[r] ? 1 : 0;
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < kCand / kBlock; ++r)
        if (t + r * kBlock < n) sm.cand[rank[r]] = mine[r];
    __syncthreads();
}

// Exact top-K of the chunk's finite entries by candidate key, for the rare
// chunks where the threshold admits more than kCand: a radix select over the
// keys of v / T (8 bits per pass), then the strictly greater entries plus the
// lowest-id ties, written to sm.cand.  Returns the number written.
template <int NVT, int VEC>
__device__ __forceinline__ int radix_topk(const float (&x)[kEpt], int K, float temp, bool divide, int e0,
                          int nvec, Smem& sm) {
    const int t = threadIdx.x;
    uint32_t prefix = 0, pmask = 0;
    int remaining = K;
    for (int shift = 24; shift >= 0; shift -= 8) {
        sm.hist[t] = 0;
        __syncthreads();
#pragma unroll
        for (int j = 0; j < NVT; ++j) {
            if (t + j * kBlock >= nvec) continue;
#pragma unroll
            for (int e = 0; e < VEC; ++e) {
                const float v = x[j * VEC + e];
                if (v == -__builtin_huge_valf()) continue;
                const uint32_t k = okey(divide ? v / temp : v);
                if ((k & pmask) == prefix) atomicAdd(&sm.hist[(k >> shift) & 0xFF], 1);
            }
        }
        __syncthreads();
        // Digit d: the bin where the count of larger-or-equal keys reaches K.
        const int h = sm.hist[255 - t];   // thread t holds bin 255 - t
        int total;
        const int above = block_excl_scan(h, total, sm);
        if (shift == 24 && total <= K) {
            // At most K finite entries: all of them are the answer.
            int nf = 0;
#pragma unroll
            for (int j = 0; j < NVT; ++j) {
                if (t + j * kBlock >= nvec) continue;
#pragma unroll
                for (int e = 0; e < VEC; ++e) nf += x[j * VEC + e] != -__builtin_huge_valf();
            }
            int tot;
            int pos = block_excl_scan(nf, tot, sm);
#pragma unroll
            for (int j = 0; j < NVT; ++j) {
                if (t + j * kBlock >= nvec) continue;
#pragma unroll
                for (int e = 0; e < VEC; ++e) {
                    const float v = x[j * VEC + e];
                    if (v == -__builtin_huge_valf()) continue;
                    sm.cand[pos++] = ckey(divide ? v / temp : v,
                                          (uint32_t)(e0 + (t + j * kBlock) * VEC + e));
                }
            }
            __syncthreads();
            return tot;
        }
        if (above < remaining && above + h >= remaining) {
            sm.misc[0] = 255 - t;
            sm.misc[1] = above;
        }
        __syncthreads();
        const int d = sm.misc[0];
        remaining -= sm.misc[1];
        prefix |= (uint32_t)d << shift;
        pmask |= 0xFFu << shift;
        __syncthreads();
    }
    // prefix = key of the K-th largest; K - remaining entries are strictly greater.
    const int need_ties = remaining;
    int ng = 0;
#pragma unroll
    for (int j = 0; j < NVT; ++j) {
        if (t + j * kBlock >= nvec) continue;
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
            const float v = x[j * VEC + e];
            if (v == -__builtin_huge_valf()) continue;
            ng += okey(divide ? v / temp : v) > prefix ? 1 : 0;
        }
    }
    int total_g;
    int pos = block_excl_scan(ng, total_g, sm);
#pragma unroll
    for (int j = 0; j < NVT; ++j) {
        if (t + j * kBlock >= nvec) continue;
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
            const float v = x[j * VEC + e];
            if (v == -__builtin_huge_valf()) continue;
            const float lg = divide ? v / temp : v;
            if (okey(lg) > prefix) sm.cand[pos++] = ckey(lg, (uint32_t)(e0 + (t + j * kBlock) * VEC + e));
        }
    }
    // Ties, lowest ids first: ids grow with (slot j, thread, element).
    int taken = 0;
#pragma unroll
    for (int j = 0; j < NVT; ++j) {
        if (taken >= need_ties) continue;   // uniform across the workgroup
        int nt = 0;
        if (t + j * kBlock < nvec) {
#pragma unroll
            for (int e = 0; e < VEC; ++e) {
                const float v = x[j * VEC + e];
                if (v != -__builtin_huge_valf() && okey(divide ? v / temp : v) == prefix) ++nt;
            }
        }
        int tot;
        int p = block_excl_scan(nt, tot, sm);
        if (t + j * kBlock < nvec) {
#pragma unroll
            for (int e = 0; e < VEC; ++e) {
                const float v = x[j * VEC + e];
                if (v == -__builtin_huge_valf()) continue;
                const float lg = divide ? v / temp : v;
                if (okey(lg) == prefix) {
                    if (taken + p < need_ties)
                        sm.cand[total_g + taken + p] =
                            ckey(lg, (uint32_t)(e0 + (t + j * kBlock) * VEC + e));
                    ++p;
                }
            }
        }
        taken += tot;
    }
    __syncthreads();
    return total_g + (taken < need_ties ? taken : need_ties);
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

template <typename T>
__global__ __launch_bounds__(kBlock) void sample_kernel(KArgs a) {
    constexpr int VEC = 16 / (int)sizeof(T);
    constexpr int NVT = kEpt / VEC;
    __shared__ Smem sm;
    const int t = threadIdx.x;
    const int S = a.S;
    const int row = blockIdx.x / S;
    const int c = blockIdx.x - row * S;
    const int V = a.V;
    const tms_row_params P = a.params[row];
    const float NEG_INF = -__builtin_huge_valf();

    const bool greedy = P.greedy != 0;
    const bool bad_params = !greedy && !(P.temperature > 0.0f && P.temperature <= FLT_MAX);
    const int K = greedy ? 1 : ((P.top_k <= 0 || P.top_k > V) ? V : P.top_k);
    const int mode = greedy ? MODE_GREEDY : (K <= kTopkFast ? MODE_TOPK : MODE_TOPP);
    const float temp = P.temperature;
    const bool divide = !greedy && temp != 1.0f;

    // ---- history: load the window ids first so their wait does not cover
    //      the logits loads issued after them.
    int nrec = 0;
    if (a.recent) {
        nrec = a.n_recent ? a.n_recent[row] : (int)a.recent_stride;
        if (nrec > (int)a.recent_stride) nrec = (int)a.recent_stride;
    }
    const bool rep_on = !(P.repeat_penalty <= 1.0f);
    const bool fp_on = P.frequency_penalty != 0.0f || P.presence_penalty != 0.0f;
    const bool pen = nrec > 0 && P.repeat_last_n > 0 && (rep_on || fp_on);
    const int from = pen ? (nrec > P.repeat_last_n ? nrec - P.repeat_last_n : 0) : 0;
    const int e0 = c * a.CE;
    const int e1 = min(e0 + a.CE, V);
    const int nvec = (e1 - e0 + VEC - 1) / VEC;
    const int32_t* hist = pen ? a.recent + (int64_t)row * a.recent_stride : nullptr;
    constexpr int kWin = 4;   // window ids per thread per pass
    int wid[kWin];
#pragma unroll
    for (int i = 0; i < kWin; ++i) {
        const int p = from + t + i * kBlock;
        wid[i] = (pen && p < nrec) ? hist[p] : -1;
    }

    // ---- stream the chunk: mask word + 16-byte logits vector per slot.
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

    // ---- penalty counts: 16-bit count per chunk id in LDS.
    if (pen) {
        for (int i = t; i < kChunk / 2; i += kBlock) sm.big.cnt[i] = 0u;
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

    // ---- per element: widen, mask, penalties, checks, thread maximum.
    float x[kEpt];
    int nonfinite = 0;
    float tmax = NEG_INF;
    uint64_t gbest = 0;
#pragma unroll
    for (int j = 0; j < NVT; ++j) {
        const int v = t + j * kBlock;
        const int eb = e0 + v * VEC;
        const bool full = a.aligned && eb + VEC <= e1;
        uint32_t cw[VEC / 2];
        if (pen && v < nvec) {
#pragma unroll
            for (int i = 0; i < VEC / 2; ++i) cw[i] = sm.big.cnt[((eb - e0) >> 1) + i];
        }
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
            const int id = eb + e;
            float val;
            if (v < nvec && id < e1) {
                val = full ? widen<T>(raw[j], e) : load_scalar<T>(base + id);
                if (!((mw[j] >> (id & 31)) & 1u)) val = NEG_INF;
                if (pen) {
                    const uint32_t cnt = (cw[e >> 1] >> ((e & 1) * 16)) & 0xFFFFu;
                    if (cnt) {
                        if (rep_on)
                            for (uint32_t r = 0; r < cnt; ++r)
                                val = val > 0.f ? val / P.repeat_penalty : val * P.repeat_penalty;
                        if (fp_on) {
                            const float t1 = (float)cnt * P.frequency_penalty;
                            const float tt = t1 + P.presence_penalty;
                            val = val - tt;
                        }
                    }
                }
                nonfinite |= (val != val) | (val == __builtin_huge_valf());
            } else {
                val = NEG_INF;
            }
            x[j * VEC + e] = val;
            tmax = fmaxf(tmax, val);
            if (mode == MODE_GREEDY && val != NEG_INF) {
                const uint64_t k = ckey(val, (uint32_t)id);
                gbest = k > gbest ? k : gbest;
            }
        }
    }
    const int flags_nf = block_or(nonfinite, sm) ? FLAG_NONFINITE : 0;
    int flags = flags_nf;
    int nout = 0;   // entries this chunk writes to its list (from sm.cand)

    if (bad_params || flags_nf) {
        nout = 0;
    } else if (mode == MODE_GREEDY) {
        const uint64_t b = block_max_u64(gbest, sm);
        if (t == 0 && b) sm.cand[0] = b;
        nout = b ? 1 : 0;
        __syncthreads();
    } else if (mode == MODE_TOPK) {
        // tau: a value such that at least K chunk entries are >= tau.  Each
        // wave sorts its 64 thread maxima; the ceil(K/4)-th of every wave
        // gives 4 * ceil(K/4) >= K threads with a maximum >= the smallest.
        const int kw = (K + kWaves - 1) / kWaves;
        const float srt = wave_sort_desc_f32(tmax);
        const float tw = __shfl(srt, kw - 1, 64);
        if ((t & 63) == 0) sm.wave_f[t >> 6] = tw;
        __syncthreads();
        float tau = sm.wave_f[0];
#pragma unroll
        for (int i = 1; i < kWaves; ++i) tau = fminf(tau, sm.wave_f[i]);
        __syncthreads();
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
        int nc = 0;
        if (!fallback) {
#pragma unroll
            for (int i = 0; i < kEpt; ++i) nc += (x[i] != NEG_INF && x[i] >= tau) ? 1 : 0;
        }
        int total;
        int pos = block_excl_scan(nc, total, sm);
        if (fallback || total > kCand) {
            nout = radix_topk<NVT, VEC>(x, K, temp, divide, e0, nvec, sm);
        } else {
#pragma unroll
            for (int j = 0; j < NVT; ++j) {
#pragma unroll
                for (int e = 0; e < VEC; ++e) {
                    const float v = x[j * VEC + e];
                    if (v != NEG_INF && v >= tau) {
                        const float lg = divide ? v / temp : v;
                        sm.cand[pos++] = ckey(lg, (uint32_t)(e0 + (t + j * kBlock) * VEC + e));
                    }
                }
            }
            __syncthreads();
            sort_cand(total, sm);
            nout = total < K ? total : K;
        }
    } else {
        // Top-p only: entries within kSigSpan of the chunk maximum (in v / T).
        const float cmax = block_max_f32(tmax, sm);
        if (cmax != NEG_INF) {
            const float lmax = divide ? cmax / temp : cmax;
            const double lthr = (double)lmax - (double)kSigSpan;
            // Generous prefilter in v, exact test on the quotient.
            const double vthr =
                ((double)lmax - (double)kSigSpan - 1.0 - fabs((double)lmax) * 0x1p-20) * (double)temp;
            int nc = 0;
#pragma unroll
            for (int i = 0; i < kEpt; ++i) {
                const float v = x[i];
                if (v != NEG_INF && (double)v >= vthr) {
                    const float lg = divide ? v / temp : v;
                    nc += (double)lg >= lthr ? 1 : 0;
                }
            }
            int total;
            int pos = block_excl_scan(nc, total, sm);
            if (total > kCand) {
                flags |= FLAG_OVERFLOW;
                nout = 0;
            } else {
#pragma unroll
                for (int j = 0; j < NVT; ++j) {
#pragma unroll
                    for (int e = 0; e < VEC; ++e) {
                        const float v = x[j * VEC + e];
                        if (v != NEG_INF && (double)v >= vthr) {
                            const float lg = divide ? v / temp : v;
                            if ((double)lg >= lthr)
                                sm.cand[pos++] =
                                    ckey(lg, (uint32_t)(e0 + (t + j * kBlock) * VEC + e));
                        }
                    }
                }
                __syncthreads();
                sort_cand(total, sm);
                nout = total;
            }
        }
    }

    // ---- publish the chunk list, then count arrivals for the row.
    uint64_t* my_list = a.lists + ((int64_t)row * S + c) * kCand;
    for (int i = t; i < nout; i += kBlock) my_list[i] = sm.cand[i];
    if (t == 0) {
        a.chunk_n[row * S + c] = nout;
        a.chunk_flags[row * S + c] = flags;
    }
    __threadfence();
    __syncthreads();
    if (t == 0) {
        const uint32_t prev = __hip_atomic_fetch_add(&a.counters[row], 1u, __ATOMIC_ACQ_REL,
                                                     __HIP_MEMORY_SCOPE_AGENT);
        sm.misc[0] = prev == (uint32_t)(S - 1) ? 1 : 0;
    }
    __syncthreads();
    if (!sm.misc[0]) return;
    __threadfence();

    // ================= merge: the last workgroup of the row =================
    if (t == 0) a.counters[row] = 0u;   // ready for the next launch
    int any_flags = 0;
    if (t < S) {
        const int n = a.chunk_n[row * S + t];
        any_flags = a.chunk_flags[row * S + t];
        sm.list_off[t + 1] = n;
    }
    if (t == 0) sm.list_off[0] = 0;
    const int fl = block_or(any_flags & FLAG_NONFINITE, sm);
    const int ov = block_or(any_flags & FLAG_OVERFLOW, sm);
    if (t == 0) {
        for (int i = 0; i < S; ++i) sm.list_off[i + 1] += sm.list_off[i];
    }
    __syncthreads();
    const int N = sm.list_off[S];

    int status = TMS_ROW_OK;
    if (bad_params) status = TMS_ROW_BAD_PARAMS;
    else if (fl) status = TMS_ROW_NONFINITE;
    else if (ov || N > kMergeCap) status = TMS_ROW_UNSUPPORTED;
    else if (N == 0) status = TMS_ROW_ALL_MASKED;

    int32_t* topk_ids = a.out_topk_ids ? a.out_topk_ids + (int64_t)row * a.topk_cap : nullptr;
    float* topk_probs = a.out_topk_probs ? a.out_topk_probs + (int64_t)row * a.topk_cap : nullptr;

    if (status != TMS_ROW_OK) {
        if (t == 0) {
            a.out_tokens[row] = -1;
            a.out_status[row] = status;
            if (a.out_keep) a.out_keep[row] = 0;
        }
        for (int i = t; i < a.topk_cap; i += kBlock) {
            if (topk_ids) topk_ids[i] = -1;
            if (topk_probs) topk_probs[i] = 0.0f;
        }
        return;
    }

    // Gather the lists and rank every entry against the other lists.
    const uint64_t* row_lists = a.lists + (int64_t)row * S * kCand;
    for (int i = t; i < N; i += kBlock) {
        int lc = 0;
        while (sm.list_off[lc + 1] <= i) ++lc;
        sm.big.m.uni[i] = row_lists[(int64_t)lc * kCand + (i - sm.list_off[lc])];
    }
    __syncthreads();
    const int nsort = N < K ? N : K;
    for (int i = t; i < N; i += kBlock) {
        int lc = 0;
        while (sm.list_off[lc + 1] <= i) ++lc;
        const uint64_t k = sm.big.m.uni[i];
        int rank = i - sm.list_off[lc];
        for (int o = 0; o < S; ++o) {
            if (o == lc) continue;
            rank += count_greater(sm.big.m.uni + sm.list_off[o],
                                  sm.list_off[o + 1] - sm.list_off[o], k);
        }
        if (rank < nsort) sm.big.m.sorted[rank] = k;
    }
    __syncthreads();

    if (mode == MODE_GREEDY) {
        if (t == 0) {
            const int tok = (int)ckey_id(sm.big.m.sorted[0]);
            a.out_tokens[row] = tok;
            a.out_status[row] = TMS_ROW_OK;
            if (a.out_keep) a.out_keep[row] = 0;
        }
        for (int i = t; i < a.topk_cap; i += kBlock) {
            if (topk_ids) topk_ids[i] = i == 0 ? (int)ckey_id(sm.big.m.sorted[0]) : -1;
            if (topk_probs) topk_probs[i] = i == 0 ? 1.0f : 0.0f;
        }
        return;
    }

    // Number of entries n the tail walks.  Top-k rows with fewer than K
    // finite ids continue with -inf entries in ascending id order: the ids
    // missing from the finite set (which is then complete).
    int n = nsort;
    if (mode == MODE_TOPK && N < K) {
        // The ids in [0, K + N) that are not among the N finite ones, lowest
        // first (K + N <= 2 * kTopkFast <= kBlock, so one id per thread).
        const int q = t;
        int member = 0;
        if (q < K + N)
            for (int i = 0; i < N; ++i) member |= (int)ckey_id(sm.big.m.sorted[i]) == q;
        const int gap = (q < K + N && !member && q < V) ? 1 : 0;
        int tot;
        const int p = block_excl_scan(gap, tot, sm);
        if (gap && p < K - N) sm.big.m.sorted[N + p] = ckey(NEG_INF, (uint32_t)q);
        __syncthreads();
        n = K;
    }
    const float mx = ckey_val(sm.big.m.sorted[0]);
    if (mx == __builtin_huge_valf()) {
        if (t == 0) {
            a.out_tokens[row] = -1;
            a.out_status[row] = TMS_ROW_NONFINITE;
            if (a.out_keep) a.out_keep[row] = 0;
        }
        for (int i = t; i < a.topk_cap; i += kBlock) {
            if (topk_ids) topk_ids[i] = -1;
            if (topk_probs) topk_probs[i] = 0.0f;
        }
        return;
    }
    // Top-p rows: only the prefix within kSigSpan of the maximum is exact.
    if (mode == MODE_TOPP) {
        int sig = 0;
        for (int i = t; i < n; i += kBlock)
            sig += ((double)ckey_val(sm.big.m.sorted[i]) - (double)mx >= -(double)kSigSpan) ? 1 : 0;
        sig = wave_sum_i32(sig);
        if ((t & 63) == 0) sm.wave_i[t >> 6] = sig;
        __syncthreads();
        n = sm.wave_i[0] + sm.wave_i[1] + sm.wave_i[2] + sm.wave_i[3];
        __syncthreads();
    }

    // pr[j] = exp(lg_j - mx) in fp64, all lanes.
    double* pr = (double*)sm.big.m.uni;   // the gathered lists are no longer needed
    for (int i = t; i < n; i += kBlock)
        pr[i] = exp((double)ckey_val(sm.big.m.sorted[i]) - (double)mx);
    __syncthreads();
    // z: sequential, in sorted order (tmsample.h:186-191).
    if (t == 0) {
        double z = 0;
        for (int i = 0; i < n; ++i) z += pr[i];
        sm.dmisc[0] = z;
    }
    __syncthreads();
    const double z = sm.dmisc[0];
    for (int i = t; i < n; i += kBlock) sm.big.m.q[i] = pr[i] / z;
    __syncthreads();
    if (t == 0) {
        // top-p (tmsample.h:192-197), then min-p.
        double cum = 0;
        int kp = K;
        const double tp = (double)P.top_p;
        for (int i = 0; i < n; ++i) {
            cum += sm.big.m.q[i];
            if (cum >= tp) {
                kp = i + 1;
                break;
            }
        }
        if (P.min_p > 0.0f) {
            const double mp = (double)P.min_p;
            int m = 1;
            while (m < kp && m < n && pr[m] >= mp) ++m;
            if (m >= n && n < K && mp <= 4.248354255291589e-18) m = K;   // exp(-40)
            if (m < kp) kp = m;
        }
        sm.misc[3] = kp;
        // sum of the kept weights, as accumulate() forms it.
        double sum = 0;
        const int lim = kp < n ? kp : n;
        for (int i = 0; i < lim; ++i) sum += pr[i];
        sm.dmisc[1] = sum;
    }
    __syncthreads();
    const int keep = sm.misc[3];
    int tokidx = 0;
    if (keep >= 2) {
        const double sum = sm.dmisc[1];
        const int lim = keep < n ? keep : n;
        for (int i = t; i < lim; i += kBlock) sm.big.m.q[i] = pr[i] / sum;
        __syncthreads();
        if (t == 0) {
            uint32_t w0, w1;
            if (a.draws) {
                w0 = a.draws[2 * row];
                w1 = a.draws[2 * row + 1];
            } else {
                row_words(P.seed, P.offset, 0u, w0, w1);
            }
            const double u = canonical(w0, w1);
            double cp = 0;
            int j = keep - 1;
            for (int i = 0; i < lim; ++i) {
                cp = i == 0 ? sm.big.m.q[i] : cp + sm.big.m.q[i];
                const double cc = (i == keep - 1) ? 1.0 : cp;
                if (!(cc < u)) {
                    j = i;
                    break;
                }
            }
            sm.misc[4] = j;
        }
        __syncthreads();
        tokidx = sm.misc[4];
    }
    // tokidx >= n happens only on top-p rows whose draw fell past the last
    // entry that moves the sums: the reference then returns its K-th entry,
    // which this row does not hold.
    const bool lost = tokidx >= n;
    if (t == 0) {
        a.out_tokens[row] = lost ? -1 : (int)ckey_id(sm.big.m.sorted[tokidx]);
        a.out_status[row] = lost ? TMS_ROW_UNSUPPORTED : TMS_ROW_OK;
        if (a.out_keep) a.out_keep[row] = keep;
    }
    for (int i = t; i < a.topk_cap; i += kBlock) {
        const bool have = i < n;
        if (topk_ids) topk_ids[i] = have ? (int)ckey_id(sm.big.m.sorted[i]) : -1;
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

// tmsample_amd.hpp -- C++ host API of the MI355X sampler, shaped like
// TensorMark's tmsample.h so a caller switches by changing the namespace.
//
// Header-only, over the C ABI of tmsample_hip.h (link libtmsample_hip.so).
//
//   tmsample_amd::Opts                 == tmsample::Opts            (tensormark/tmsample.h:31-35)
//   tmsample_amd::DryOpts              == tmsample::DryOpts         (tensormark/tmsample.h:141-146)
//   tmsample_amd::apply_repeat_penalty == tmsample::apply_repeat_penalty  (tensormark/tmsample.h:52-63)
//   tmsample_amd::apply_no_repeat_ngram== tmsample::apply_no_repeat_ngram (tensormark/tmsample.h:81-114)
//   tmsample_amd::apply_dry            == tmsample::apply_dry             (tensormark/tmsample.h:148-170)
//                                         (host rows, through tms_host_* of the C ABI)
//   Sampler::sample(logits, V, o, greedy, rng)
//                                      == tmsample::sample          (tensormark/tmsample.h:173-200)
//   Sampler::sample_token(...)         == sample_token              (tensormark/llama_chat.cpp:146-153)
//   Sampler::sample_batch / spec_verify   batched device entry points (no reference counterpart)
//
// Errors: the reference's sampler has none (bad knobs are undefined
// behaviour there); here a failed C call or a row status other than OK
// throws tmsample_amd::Error carrying the code.
#pragma once

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <limits>
#include <random>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "tmsample_hip.h"

namespace tmsample_amd {

struct Opts {
    float temperature = 0.7f;
    int top_k = 40;
    float top_p = 0.9f;
};

struct DryOpts {
    float multiplier = 0.0f;   // 0 = disabled
    float base = 1.75f;
    int allowed_length = 2;
    int penalty_last_n = 256;
};

// Knobs of the chat CLI's sample_token (tensormark/llama_chat.cpp:114-126).
struct ChatOpts {
    float temperature = 0.7f;
    int top_k = 40;
    float top_p = 0.9f;
    float repeat_penalty = 1.0f;
    int repeat_last_n = 64;
    int no_repeat_ngram = 0;
    DryOpts dry;
    const unsigned char* dry_breaker = nullptr;
};

class Error : public std::runtime_error {
public:
    Error(const std::string& what, int code) : std::runtime_error(what), code_(code) {}
    int code() const { return code_; }

private:
    int code_;
};

// ---------------------------------------------------------------- host transforms
// The deterministic history transforms of tmsample.h, on a host row.  The
// device sampler applies the repetition penalty itself (from the window);
// these serve callers that transform on the host, and sample_token when an
// n-gram ban or DRY is on (they must follow the repetition penalty).

inline void apply_repeat_penalty(std::vector<float>& logits, const int* recent, int n_recent,
                                 int window, float penalty) {
    tms_host_repeat_penalty(logits.data(), static_cast<int>(logits.size()), recent, n_recent,
                            window, penalty);
}

inline void apply_no_repeat_ngram(std::vector<float>& logits, const int* recent, int n_recent,
                                  int ngram) {
    tms_host_no_repeat_ngram(logits.data(), static_cast<int>(logits.size()), recent, n_recent,
                             ngram);
}

inline void apply_dry(std::vector<float>& logits, const int* recent, int n_recent,
                      const DryOpts& o, const unsigned char* is_breaker = nullptr) {
    tms_host_dry(logits.data(), static_cast<int>(logits.size()), recent, n_recent, o.multiplier,
                 o.base, o.allowed_length, o.penalty_last_n, is_breaker);
}

// ---------------------------------------------------------------- device sampler
class Sampler {
public:
    Sampler(int device, int max_batch, int max_vocab) : device_(device) {
        check(tms_create(device, max_batch, max_vocab, &ctx_), "tms_create");
        int prev = 0;
        hip(hipGetDevice(&prev), "hipGetDevice");
        hip(hipSetDevice(device), "hipSetDevice");
        const size_t words = (static_cast<size_t>(max_vocab) + 31) / 32;
        hip(hipMalloc(&d_logits_, sizeof(float) * static_cast<size_t>(max_vocab)), "hipMalloc");
        hip(hipMalloc(&d_recent_, sizeof(int32_t) * kMaxHistory), "hipMalloc");
        hip(hipMalloc(&d_mask_, sizeof(uint32_t) * words), "hipMalloc");
        hip(hipMalloc(&d_small_, 256), "hipMalloc");
        hip(hipMalloc(&d_breaker_, static_cast<size_t>(max_vocab)), "hipMalloc");
        hip(hipMalloc(&d_scale_, sizeof(float) * TMS_DRY_MAX_WINDOW), "hipMalloc");
        hip(hipStreamCreate(&stream_), "hipStreamCreate");
        (void)hipSetDevice(prev);
        max_vocab_ = max_vocab;
    }
    ~Sampler() {
        int prev = 0;
        (void)hipGetDevice(&prev);
        (void)hipSetDevice(device_);
        if (stream_) (void)hipStreamDestroy(stream_);
        for (void* p : {d_logits_, d_recent_, d_mask_, d_small_, d_breaker_, d_scale_})
            if (p) (void)hipFree(p);
        (void)hipSetDevice(prev);
        if (ctx_) (void)tms_destroy(ctx_);
    }
    Sampler(const Sampler&) = delete;
    Sampler& operator=(const Sampler&) = delete;

    tms_context* context() const { return ctx_; }

    // tmsample::sample on the GPU: greedy argmax, else temperature, top-k,
    // fp64 softmax, top-p and a discrete_distribution draw.  The draw uses
    // the same two mt19937 words the reference would, and `rng` advances
    // exactly as the reference's does (two words when at least two tokens
    // survive the cut, none otherwise).
    [[nodiscard]] int sample(const std::vector<float>& logits, int V, const Opts& o, bool greedy,
                             std::mt19937& rng) {
        tms_row_params p = row_params(o.temperature, o.top_k, o.top_p, greedy);
        return run_row(logits.data(), V, p, nullptr, 0, nullptr, greedy, rng);
    }

    // sample_token (tensormark/llama_chat.cpp:146-153): repetition penalty,
    // n-gram ban, DRY, then sample, all on the GPU.  `mask` (nullable,
    // ceil(V / 32) words, bit id & 31 of word id >> 5) restricts the row
    // first, as GrammarFilter::restrict does (llama_chat.cpp:184-209).  With
    // the ban and DRY off only the repetition window is uploaded; otherwise
    // the whole history (its last 65535 ids), the breaker table and the DRY
    // scales (std::pow(base, (float)k), as tmsample.h:168 computes them) go
    // up and the library's history pre-pass runs; a DRY window longer than
    // the pre-pass holds (TMS_DRY_MAX_WINDOW) runs the three transforms on
    // the host instead.  Unlike the reference, `logits` is left as it was.
    [[nodiscard]] int sample_token(std::vector<float>& logits, int V, const ChatOpts& o,
                                   bool greedy, std::mt19937& rng, const int* recent,
                                   int n_recent, const uint32_t* mask = nullptr) {
        tms_row_params p = row_params(o.temperature, o.top_k, o.top_p, greedy);
        p.repeat_penalty = o.repeat_penalty;
        p.repeat_last_n = o.repeat_last_n;
        const int dry_window = std::min(n_recent, o.dry.penalty_last_n);
        if (o.dry.multiplier > 0.0f && dry_window > TMS_DRY_MAX_WINDOW) {
            std::vector<float> row(logits.begin(), logits.begin() + V);
            if (mask) apply_mask(row, mask);
            tms_host_repeat_penalty(row.data(), V, recent, n_recent, o.repeat_last_n, o.repeat_penalty);
            tms_host_no_repeat_ngram(row.data(), V, recent, n_recent, o.no_repeat_ngram);
            tms_host_dry(row.data(), V, recent, n_recent, o.dry.multiplier, o.dry.base,
                         o.dry.allowed_length, o.dry.penalty_last_n, o.dry_breaker);
            p.repeat_penalty = 1.0f;
            return run_row(row.data(), V, p, nullptr, 0, nullptr, greedy, rng);
        }
        if (o.no_repeat_ngram >= 2 || o.dry.multiplier > 0.0f) {
            tms_history_params h{};
            h.no_repeat_ngram = o.no_repeat_ngram;
            h.dry_multiplier = o.dry.multiplier;
            h.dry_base = o.dry.base;
            h.dry_allowed_length = o.dry.allowed_length;
            h.dry_penalty_last_n = o.dry.penalty_last_n;
            return run_row(logits.data(), V, p, recent, n_recent, mask, greedy, rng, &h,
                           o.dry_breaker);
        }
        // Only the window reaches the device.
        const int from = std::max(0, n_recent - std::max(0, o.repeat_last_n));
        return run_row(logits.data(), V, p, recent + from, n_recent - from, mask, greedy, rng);
    }

    // The batched device path: every pointer in `a` is device memory.
    void sample_batch(const tms_sample_args& a, hipStream_t stream) {
        check(tms_sample_batch(ctx_, &a, stream), "tms_sample_batch");
    }
    void spec_verify(const tms_spec_args& a, hipStream_t stream) {
        check(tms_spec_verify(ctx_, &a, stream), "tms_spec_verify");
    }

private:
    static constexpr int kMaxHistory = 65535;

    static tms_row_params row_params(float T, int k, float p, bool greedy) {
        tms_row_params r{};
        r.temperature = T;
        r.top_k = k;
        r.top_p = p;
        r.repeat_penalty = 1.0f;
        r.greedy = greedy ? 1 : 0;
        return r;
    }
    static void apply_mask(std::vector<float>& logits, const uint32_t* mask) {
        const float ninf = -std::numeric_limits<float>::infinity();
        for (size_t i = 0; i < logits.size(); ++i)
            if (!((mask[i >> 5] >> (i & 31)) & 1u)) logits[i] = ninf;
    }
    static void check(int rc, const char* what) {
        if (rc != TMS_OK) throw Error(std::string(what) + ": " + tms_status_string(rc), rc);
    }
    static void hip(hipError_t e, const char* what) {
        if (e != hipSuccess) throw Error(std::string(what) + ": " + hipGetErrorString(e), TMS_ERR_HIP);
    }

    int run_row(const float* logits, int V, const tms_row_params& p, const int* recent, int n_recent,
                const uint32_t* mask, bool greedy, std::mt19937& rng,
                const tms_history_params* hist = nullptr, const unsigned char* breaker = nullptr) {
        if (V <= 0 || V > max_vocab_) throw Error("row wider than the sampler's vocabulary", TMS_ERR_CAPACITY);
        if (n_recent > kMaxHistory) {
            recent += n_recent - kMaxHistory;
            n_recent = kMaxHistory;
        }
        int prev = 0;
        hip(hipGetDevice(&prev), "hipGetDevice");
        hip(hipSetDevice(device_), "hipSetDevice");
        // The draw's words, from a copy: the caller's generator advances
        // only if the reference would have consumed them.
        std::mt19937 peek = rng;
        uint32_t words[2] = {0, 0};
        if (!greedy) {
            words[0] = static_cast<uint32_t>(peek());
            words[1] = static_cast<uint32_t>(peek());
        }
        struct Small {
            tms_row_params params;
            tms_history_params hist;
            uint32_t draws[2];
            int32_t n_recent, token, status, keep;
        } h{};
        static_assert(sizeof(Small) <= 256, "d_small_ holds 256 bytes");
        if (hist) h.hist = *hist;
        h.params = p;
        h.draws[0] = words[0];
        h.draws[1] = words[1];
        h.n_recent = n_recent;
        auto* d = static_cast<Small*>(d_small_);
        hip(hipMemcpyAsync(d_logits_, logits, sizeof(float) * static_cast<size_t>(V),
                           hipMemcpyHostToDevice, stream_), "hipMemcpyAsync");
        if (n_recent > 0)
            hip(hipMemcpyAsync(d_recent_, recent, sizeof(int32_t) * static_cast<size_t>(n_recent),
                               hipMemcpyHostToDevice, stream_), "hipMemcpyAsync");
        if (mask)
            hip(hipMemcpyAsync(d_mask_, mask, sizeof(uint32_t) * ((static_cast<size_t>(V) + 31) / 32),
                               hipMemcpyHostToDevice, stream_), "hipMemcpyAsync");
        if (hist && breaker)
            hip(hipMemcpyAsync(d_breaker_, breaker, static_cast<size_t>(V), hipMemcpyHostToDevice, stream_),
                "hipMemcpyAsync");
        // the DRY scales of the reference's arithmetic, one per exponent the
        // row's window can need
        int scale_n = 0;
        if (hist && hist->dry_multiplier > 0.0f) {
            scale_n = std::max(1, std::min(hist->dry_penalty_last_n, static_cast<int>(TMS_DRY_MAX_WINDOW)));
            scale_.resize(static_cast<size_t>(scale_n));
            check(tms_dry_scale_table(hist->dry_base, scale_n, scale_.data()), "tms_dry_scale_table");
            hip(hipMemcpyAsync(d_scale_, scale_.data(), sizeof(float) * static_cast<size_t>(scale_n),
                               hipMemcpyHostToDevice, stream_), "hipMemcpyAsync");
        }
        hip(hipMemcpyAsync(d, &h, sizeof(h), hipMemcpyHostToDevice, stream_), "hipMemcpyAsync");
        tms_sample_args a{};
        a.logits = d_logits_;
        a.dtype = TMS_DTYPE_F32;
        a.batch = 1;
        a.vocab = V;
        a.row_stride = V;
        a.params = &d->params;
        a.recent = n_recent > 0 ? static_cast<const int32_t*>(d_recent_) : nullptr;
        a.n_recent = n_recent > 0 ? &d->n_recent : nullptr;
        a.recent_stride = n_recent > 0 ? n_recent : 0;
        a.mask = mask ? static_cast<const uint32_t*>(d_mask_) : nullptr;
        a.mask_stride = mask ? (V + 31) / 32 : 0;
        a.draws = d->draws;
        a.out_tokens = &d->token;
        a.out_status = &d->status;
        a.out_keep = &d->keep;
        a.history = hist ? &d->hist : nullptr;
        a.dry_breaker = (hist && breaker) ? static_cast<const uint8_t*>(d_breaker_) : nullptr;
        a.dry_scale = scale_n ? static_cast<const float*>(d_scale_) : nullptr;
        a.dry_scale_stride = scale_n;
        // The row is known here: a greedy or top-k <= 128 row may take the
        // library's top-k kernel.
        a.row_kinds = (h.params.greedy != 0 || (h.params.top_k >= 1 && h.params.top_k <= 128))
                          ? TMS_ROWS_TOPK : TMS_ROWS_ANY;
        check(tms_sample_batch(ctx_, &a, stream_), "tms_sample_batch");
        hip(hipMemcpyAsync(&h, d, sizeof(h), hipMemcpyDeviceToHost, stream_), "hipMemcpyAsync");
        hip(hipStreamSynchronize(stream_), "hipStreamSynchronize");
        (void)hipSetDevice(prev);
        if (h.status != TMS_ROW_OK)
            throw Error(std::string("row status: ") + row_status_name(h.status), h.status);
        if (!greedy && h.keep >= 2) rng = peek;
        return h.token;
    }
    static const char* row_status_name(int s) {
        switch (s) {
            case TMS_ROW_BAD_PARAMS: return "bad parameters";
            case TMS_ROW_ALL_MASKED: return "every id is masked";
            case TMS_ROW_NONFINITE: return "non-finite logits";
            case TMS_ROW_UNSUPPORTED: return "unsupported row";
            default: return "internal";
        }
    }

    int device_ = 0;
    int max_vocab_ = 0;
    tms_context* ctx_ = nullptr;
    void* d_logits_ = nullptr;
    void* d_recent_ = nullptr;
    void* d_mask_ = nullptr;
    void* d_small_ = nullptr;
    void* d_breaker_ = nullptr;
    void* d_scale_ = nullptr;
    std::vector<float> scale_;
    hipStream_t stream_ = nullptr;
};

}  // namespace tmsample_amd

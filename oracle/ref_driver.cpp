// ref_driver.cpp -- C entry points around the reference's own tmsample.h.
//
// TEST INFRASTRUCTURE ONLY.  Compiled by oracle/Makefile against the header
// where it lies in the reference tree (-I$(REF)); the output goes to
// oracle/_ref/ and is never committed.  It lets the tests pin the C oracle
// against the compiled reference and lets bench.py time the reference
// sampler on the host as the CPU baseline.
//
// The composition below is sample_token with the grammar restriction in
// front (tensormark/llama_chat.cpp:787-791, 146-153, 184-209): the mask
// writes -inf, then tmsample::apply_repeat_penalty, then tmsample::sample.

#include "tmsample.h"

#include <algorithm>
#include <chrono>
#include <cstdint>
#include <cstring>
#include <limits>
#include <random>
#include <sstream>
#include <thread>
#include <vector>

namespace {

// A 32-bit URNG that replays scripted words, for driving libstdc++'s
// distribution code with chosen inputs.
struct Script {
    using result_type = std::uint32_t;
    const std::uint32_t* w;
    int n, i = 0;
    static constexpr result_type min() { return 0; }
    static constexpr result_type max() { return 0xFFFFFFFFu; }
    result_type operator()() { return i < n ? w[i++] : 0u; }
};

void restrict_row(std::vector<float>& lg, const std::uint32_t* mask) {
    if (!mask) return;
    for (std::size_t i = 0; i < lg.size(); ++i)
        if (!((mask[i >> 5] >> (i & 31)) & 1u)) lg[i] = -std::numeric_limits<float>::infinity();
}

int one_row(const float* logits, int V, float T, int top_k, float top_p, int greedy,
            std::mt19937& rng, const std::int32_t* recent, int n_recent, int window,
            float penalty, const std::uint32_t* mask) {
    std::vector<float> lg(logits, logits + V);
    restrict_row(lg, mask);
    if (recent) tmsample::apply_repeat_penalty(lg, recent, n_recent, window, penalty);
    return tmsample::sample(lg, V, tmsample::Opts{T, top_k, top_p}, greedy != 0, rng);
}

// The mt19937 word y such that the engine's tempering gives w.
std::uint32_t untemper(std::uint32_t w) {
    std::uint32_t y = w;
    y ^= y >> 18;
    y ^= (y << 15) & 0xefc60000u;
    std::uint32_t t = y;
    for (int i = 0; i < 5; ++i) t = y ^ ((t << 7) & 0x9d2c5680u);
    y = t;
    y ^= (y >> 11) ^ (y >> 22);
    return y;
}

// An std::mt19937 whose next two outputs are w0, w1: its state, read back
// through the engine's own stream operator, holds the untempered words at
// positions 0 and 1 with the position at 0 (no twist before them).
std::mt19937 engine_giving(std::uint32_t w0, std::uint32_t w1) {
    std::ostringstream os;
    os << untemper(w0) << ' ' << untemper(w1);
    for (int i = 2; i < 624; ++i) os << ' ' << 0x9908b0dfu + i;
    os << ' ' << 0;
    std::istringstream is(os.str());
    std::mt19937 e;
    is >> e;
    return e;
}

}  // namespace

extern "C" {

// tmsample::sample itself (the unmodified header), driven by an mt19937 that
// yields w0 then w1: the reference's token for that uniform, under this
// standard library's nth_element / sort / discrete_distribution.  Returns -1
// if the crafted engine does not give (w0, w1).
int ref_sample_words(const float* logits, int V, float T, int top_k, float top_p, int greedy,
                     std::uint32_t w0, std::uint32_t w1) {
    std::mt19937 check = engine_giving(w0, w1);
    if (check() != w0 || check() != w1) return -1;
    std::mt19937 rng = engine_giving(w0, w1);
    std::vector<float> lg(logits, logits + V);
    return tmsample::sample(lg, V, tmsample::Opts{T, top_k, top_p}, greedy != 0, rng);
}


// std::generate_canonical<double, 53> on the words (w0, w1).
double ref_canonical(std::uint32_t w0, std::uint32_t w1) {
    const std::uint32_t w[2] = {w0, w1};
    Script s{w, 2};
    return std::generate_canonical<double, 53>(s);
}

// std::discrete_distribution<int>(pr, pr + n) drawn with the words (w0, w1);
// *consumed = words the draw took from the generator.
int ref_discrete(const double* pr, int n, std::uint32_t w0, std::uint32_t w1, int* consumed) {
    const std::uint32_t w[2] = {w0, w1};
    Script s{w, 2};
    std::discrete_distribution<int> d(pr, pr + n);
    const int r = d(s);
    *consumed = s.i;
    return r;
}

// tmsample::apply_repeat_penalty on a copy of row, written back.
void ref_apply_repeat_penalty(float* row, int V, const std::int32_t* recent, int n_recent,
                              int window, float penalty) {
    std::vector<float> lg(row, row + V);
    tmsample::apply_repeat_penalty(lg, recent, n_recent, window, penalty);
    std::memcpy(row, lg.data(), sizeof(float) * static_cast<std::size_t>(V));
}

// One sample_token step with an mt19937 seeded by `seed`.  Reports the first
// two words the generator would give (*w0, *w1) and how many it consumed.
int ref_sample(const float* logits, int V, float T, int top_k, float top_p, int greedy,
               std::uint32_t seed, const std::int32_t* recent, int n_recent, int window,
               float penalty, const std::uint32_t* mask, std::uint32_t* w0, std::uint32_t* w1,
               int* consumed) {
    std::mt19937 rng(seed);
    std::mt19937 probe = rng;
    *w0 = probe();
    *w1 = probe();
    std::mt19937 after0 = rng;
    const int tok = one_row(logits, V, T, top_k, top_p, greedy, rng, recent, n_recent, window,
                            penalty, mask);
    int n = 0;
    while (n < 4 && !(after0 == rng)) { after0(); ++n; }
    *consumed = n;
    return tok;
}

// CPU baseline: sample B rows with `threads` workers, `reps` times; returns
// the median wall time of one pass in seconds.  Rows are independent, so they
// are dealt round-robin to the workers.
double ref_bench(const float* logits, int B, int V, float T, int top_k, float top_p, int greedy,
                 const std::int32_t* recent, int recent_stride, int window, float penalty,
                 const std::uint32_t* mask, int mask_stride, int threads, int reps,
                 std::int32_t* tokens) {
    if (threads < 1) threads = 1;
    if (reps < 1) reps = 1;
    std::vector<double> times;
    for (int r = 0; r < reps; ++r) {
        const auto t0 = std::chrono::steady_clock::now();
        std::vector<std::thread> pool;
        for (int w = 0; w < threads; ++w)
            pool.emplace_back([&, w] {
                std::mt19937 rng(1234u + static_cast<unsigned>(w));
                for (int b = w; b < B; b += threads)
                    tokens[b] = one_row(logits + static_cast<std::size_t>(b) * V, V, T, top_k,
                                        top_p, greedy, rng,
                                        recent ? recent + static_cast<std::size_t>(b) * recent_stride
                                               : nullptr,
                                        recent_stride, window, penalty,
                                        mask ? mask + static_cast<std::size_t>(b) * mask_stride
                                             : nullptr);
            });
        for (auto& t : pool) t.join();
        times.push_back(std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count());
    }
    // the median pass (the lower middle one for an even count)
    std::nth_element(times.begin(), times.begin() + (reps - 1) / 2, times.end());
    return times[(reps - 1) / 2];
}

// The reference's no-repeat n-gram ban and DRY on a row, in place
// (tensormark/tmsample.h:81-114, 148-170).
void ref_no_repeat_ngram(float* logits, int V, const std::int32_t* recent, int n_recent, int ngram) {
    std::vector<float> row(logits, logits + V);
    tmsample::apply_no_repeat_ngram(row, recent, n_recent, ngram);
    std::memcpy(logits, row.data(), sizeof(float) * static_cast<std::size_t>(V));
}

void ref_dry(float* logits, int V, const std::int32_t* recent, int n_recent, float multiplier,
             float base, int allowed_length, int penalty_last_n, const unsigned char* is_breaker) {
    std::vector<float> row(logits, logits + V);
    tmsample::DryOpts o;
    o.multiplier = multiplier;
    o.base = base;
    o.allowed_length = allowed_length;
    o.penalty_last_n = penalty_last_n;
    tmsample::apply_dry(row, recent, n_recent, o, is_breaker);
    std::memcpy(logits, row.data(), sizeof(float) * static_cast<std::size_t>(V));
}

}  // extern "C"

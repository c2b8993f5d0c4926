// host_api_check.cpp -- the C++ drop-in (include/tmsample_amd.hpp) on the GPU
// against the C oracle (oracle/tms_oracle.c, compiled into this test
// program as the checker).
//
// For each case the oracle gets the two std::mt19937 words the reference's
// discrete_distribution would draw; the device path must return the same
// token AND leave the caller's generator in the state the reference would
// (two words consumed when at least two tokens survive the cut, none for
// greedy rows or a single survivor).  Prints one line per failure and a
// summary; exit status 0 iff everything matched.

#include <cmath>
#include <cstdio>
#include <random>
#include <vector>

#include "../../oracle/tms_oracle.h"
#include "tmgbnf_amd.hpp"
#include "tmsample_amd.hpp"

namespace {

int failures = 0;

void expect(bool ok, const char* what, int c) {
    if (!ok) {
        ++failures;
        std::printf("FAIL case %d: %s\n", c, what);
    }
}

std::mt19937_64 g64(int a, int b) { return std::mt19937_64(static_cast<uint64_t>(a) * 1000003u + b); }

std::vector<float> make_row(std::mt19937_64& g, int V, float sd) {
    std::normal_distribution<float> n(0.0f, sd);
    std::vector<float> x(static_cast<size_t>(V));
    for (float& v : x) v = n(g);
    return x;
}

std::vector<float> make_row(std::mt19937_64&& g, int V, float sd) { return make_row(g, V, sd); }

tmo_row_params oracle_params(const tmsample_amd::Opts& o, bool greedy) {
    tmo_row_params p{};
    p.temperature = o.temperature;
    p.top_k = o.top_k;
    p.top_p = o.top_p;
    p.repeat_penalty = 1.0f;
    p.greedy = greedy ? 1 : 0;
    return p;
}

// Expected token and generator state for one row through the oracle.
int oracle_sample(const std::vector<float>& row, const tmsample_amd::Opts& o, bool greedy,
                  std::mt19937& rng) {
    std::mt19937 peek = rng;
    const uint32_t w0 = static_cast<uint32_t>(peek());
    const uint32_t w1 = static_cast<uint32_t>(peek());
    const tmo_row_params p = oracle_params(o, greedy);
    int32_t tok = -1, keep = 0;
    tmo_sample_row(row.data(), static_cast<int>(row.size()), &p, w0, w1, &tok, &keep, nullptr,
                   nullptr, 0);
    if (!greedy && keep >= 2) rng = peek;
    return tok;
}

}  // namespace

int main() {
    tmsample_amd::Sampler s(0, 4, 131072);
    std::mt19937_64 g(7);
    int c = 0;

    // tmsample::sample shape: opts, greedy, caller's mt19937.
    const float temps[] = {0.7f, 1.0f, 0.3f, 1.8f};
    const int ks[] = {40, 1, 5, 100, 0};
    const float ps[] = {0.9f, 0.95f, 0.2f, 1.0f};
    for (int i = 0; i < 120; ++i, ++c) {
        const int V = (i % 3 == 0) ? 32000 : (i % 3 == 1 ? 1000 : 128256);
        std::vector<float> row = make_row(g, V, 2.5f);
        tmsample_amd::Opts o{temps[i % 4], ks[i % 5], ps[(i / 5) % 4]};
        if (o.top_k == 0) o.top_k = 40;
        const bool greedy = i % 7 == 0;
        std::mt19937 r1(static_cast<unsigned>(1000 + i)), r2 = r1;
        const int want = oracle_sample(row, o, greedy, r1);
        const int got = s.sample(row, V, o, greedy, r2);
        expect(got == want, "sample: token", c);
        expect(r1 == r2, "sample: generator state", c);
    }

    // sample_token: grammar mask, then the repetition penalty on the device.
    for (int i = 0; i < 40; ++i, ++c) {
        const int V = 32000;
        std::vector<float> row = make_row(g, V, 2.0f);
        std::vector<int> hist(200);
        std::uniform_int_distribution<int> ids(0, 300);   // dense ids: repeats
        for (int& h : hist) h = ids(g);
        std::vector<uint32_t> mask(static_cast<size_t>((V + 31) / 32), 0xFFFFFFFFu);
        if (i % 2) {
            std::uniform_int_distribution<uint32_t> w;
            for (auto& m : mask) m = w(g) | 1u;
        }
        tmsample_amd::ChatOpts o;
        o.repeat_penalty = 1.3f;
        o.repeat_last_n = 64 + i;
        std::vector<float> ref = row;
        tmo_apply_mask(ref.data(), V, mask.data());
        tmo_apply_repeat_penalty(ref.data(), V, hist.data(), static_cast<int>(hist.size()),
                                 o.repeat_last_n, o.repeat_penalty);
        std::mt19937 r1(static_cast<unsigned>(77 + i)), r2 = r1;
        const int want = oracle_sample(ref, tmsample_amd::Opts{o.temperature, o.top_k, o.top_p},
                                       false, r1);
        std::vector<float> mine = row;
        const int got = s.sample_token(mine, V, o, false, r2, hist.data(),
                                       static_cast<int>(hist.size()), mask.data());
        expect(got == want, "sample_token: token", c);
        expect(r1 == r2, "sample_token: generator state", c);
    }

    // sample_token with DRY and an n-gram ban: the device pre-pass, against
    // the oracle's restatement of the reference's steps.
    for (int i = 0; i < 20; ++i, ++c) {
        const int V = 4096;
        std::vector<float> row = make_row(g, V, 2.0f);
        std::vector<int> hist;
        for (int r = 0; r < 30; ++r)
            for (int t : {11, 12, 13, 14}) hist.push_back(t + (r % 3 == 0 ? i : 0));
        tmsample_amd::ChatOpts o;
        o.repeat_penalty = 1.1f;
        o.no_repeat_ngram = 3;
        o.dry.multiplier = 0.8f;
        std::vector<unsigned char> brk(static_cast<size_t>(V), 0);
        if (i % 2) {
            brk[13] = 1;
            o.dry_breaker = brk.data();
        }
        std::vector<float> ref = row;
        const int n = static_cast<int>(hist.size());
        tmo_apply_repeat_penalty(ref.data(), V, hist.data(), n, o.repeat_last_n, o.repeat_penalty);
        tmo_no_repeat_ngram(ref.data(), V, hist.data(), n, o.no_repeat_ngram);
        tmo_dry(ref.data(), V, hist.data(), n, o.dry.multiplier, o.dry.base, o.dry.allowed_length,
                o.dry.penalty_last_n, o.dry_breaker);
        std::mt19937 r1(static_cast<unsigned>(5 + i)), r2 = r1;
        const int want = oracle_sample(ref, tmsample_amd::Opts{o.temperature, o.top_k, o.top_p},
                                       false, r1);
        std::vector<float> mine = row;
        const int got = s.sample_token(mine, V, o, false, r2, hist.data(), n);
        expect(got == want, "sample_token (DRY): token", c);
        expect(r1 == r2, "sample_token (DRY): generator state", c);
    }

    // Constrained decoding: the grammar engine's mask restricts each GPU draw;
    // every sampled id must be allowed, and a sequence ending in EOS must be a
    // sentence of the grammar.
    {
        const char* gtext = R"(root ::= "{" ws pair ("," ws pair)* "}"
pair ::= "\"" [a-z]+ "\"" ":" ws num
num  ::= "-"? [0-9]+
ws   ::= " "?)";
        const auto g = tmgbnf_amd::Grammar::parse(gtext);
        std::vector<std::string> vocab = {"{", "}", ",", ":", " ", "\"", "-", "\"a\"", "\"key\":",
                                          "0", "1", "12", "345", "x", "ab", "z", "{\"", "\":",
                                          "}}", ", ", "9"};
        const int eos = static_cast<int>(vocab.size());
        const int V = eos + 1;
        tmgbnf_amd::TokenMask tm(g, vocab, eos);
        int finished = 0;
        for (int seq = 0; seq < 12; ++seq, ++c) {
            auto st = g.start();
            std::string text;
            std::mt19937 rng(static_cast<unsigned>(900 + seq));
            bool ok = true, ended = false;
            for (int step = 0; step < 40 && ok; ++step) {
                std::vector<uint32_t> words(static_cast<size_t>((V + 31) / 32));
                const int n_allowed = tm.mask(st, words.data(), static_cast<int>(words.size()));
                std::vector<float> row = make_row(g64(seq, step), V, 1.5f);
                tmsample_amd::ChatOpts o;
                o.temperature = 1.0f;
                o.top_k = 40;
                o.top_p = 1.0f;
                const int tok = s.sample_token(row, V, o, false, rng, nullptr, 0, words.data());
                const bool allowed = n_allowed > 0 && ((words[tok >> 5] >> (tok & 31)) & 1u);
                ok = allowed;
                if (!allowed) break;
                if (tok == eos) {
                    ended = true;
                    break;
                }
                text += vocab[static_cast<size_t>(tok)];
                ok = tm.consume(st, tok);
            }
            expect(ok, "constrained decode: every sampled id allowed and consumed", c);
            if (ended) {
                ++finished;
                expect(g.accepts(text), "constrained decode: EOS ends a sentence of the grammar", c);
            }
        }
        expect(finished > 0, "constrained decode: some sequence reached EOS", c++);
    }

    // Errors surface as exceptions with the row status.
    {
        std::vector<float> row(100, 0.0f);
        std::mt19937 r(1);
        bool threw = false;
        try {
            (void)s.sample(row, 100, tmsample_amd::Opts{0.0f, 40, 0.9f}, false, r);
        } catch (const tmsample_amd::Error& e) {
            threw = e.code() == TMS_ROW_BAD_PARAMS;
        }
        expect(threw, "temperature 0 raises BAD_PARAMS", c++);
    }

    std::printf("host_api_check: %d cases, %d failures\n", c, failures);
    return failures == 0 ? 0 : 1;
}

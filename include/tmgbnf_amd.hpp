// tmgbnf_amd.hpp -- C++ view of the host GBNF engine, shaped like TensorMark's
// tmgbnf (tensormark/gbnf.h:345-851) so a caller switches by changing the
// namespace.  Header-only over the tms_grammar_* / tms_vocab_* C ABI
// (include/tmsample_hip.h); link libtmsample_hip.so.
//
//   tmgbnf_amd::Grammar::parse(text)    == tmgbnf::Grammar::parse   (throws std::runtime_error)
//   Grammar::start / advance / can_end / accepts
//   tmgbnf_amd::TokenMask(g, token_text, eos, skip)
//   TokenMask::allowed(state)           == ascending ids, like tmgbnf::TokenMask::allowed
//   TokenMask::mask(state, words, n)    the same set as the sampler's bitmask words
//   TokenMask::consume / clear_cache
#pragma once

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <string_view>
#include <utility>
#include <vector>

#include "tmsample_hip.h"

namespace tmgbnf_amd {

class Grammar;

// A parse state with value semantics (copy before a speculative walk).
class State {
public:
    State() = default;
    State(const State& o) : h_(o.h_ ? tms_gstate_copy(o.h_) : nullptr) {}
    State(State&& o) noexcept : h_(std::exchange(o.h_, nullptr)) {}
    State& operator=(State o) noexcept {
        std::swap(h_, o.h_);
        return *this;
    }
    ~State() {
        if (h_) tms_gstate_free(h_);
    }
    bool operator==(const State& o) const { return tms_gstate_equal(h_, o.h_) != 0; }
    tms_gstate* handle() const { return h_; }

private:
    friend class Grammar;
    explicit State(tms_gstate* h) : h_(h) {}
    tms_gstate* h_ = nullptr;
};

class Grammar {
public:
    static Grammar parse(std::string_view text) {
        char err[512];
        tms_grammar* g = tms_grammar_parse(text.data(), text.size(), err, sizeof err);
        if (!g) throw std::runtime_error(err);
        return Grammar(g);
    }
    Grammar(Grammar&& o) noexcept : h_(std::exchange(o.h_, nullptr)) {}
    Grammar(const Grammar&) = delete;
    Grammar& operator=(const Grammar&) = delete;
    ~Grammar() {
        if (h_) tms_grammar_free(h_);
    }

    int rule_count() const { return tms_grammar_rule_count(h_); }
    State start() const { return State(tms_grammar_start(h_)); }
    [[nodiscard]] bool advance(State& s, unsigned char byte) const {
        return tms_grammar_advance(h_, s.handle(), byte) != 0;
    }
    bool can_end(const State& s) const { return tms_grammar_can_end(h_, s.handle()) != 0; }
    bool accepts(std::string_view text) const {
        return tms_grammar_accepts(h_, text.data(), text.size()) != 0;
    }
    tms_grammar* handle() const { return h_; }

private:
    explicit Grammar(tms_grammar* h) : h_(h) {}
    tms_grammar* h_ = nullptr;
};

class TokenMask {
public:
    TokenMask(const Grammar& g, const std::vector<std::string>& token_text, int eos = -1,
              const std::vector<char>& skip = {})
        : g_(g) {
        std::vector<const char*> p(token_text.size());
        std::vector<size_t> n(token_text.size());
        for (size_t i = 0; i < token_text.size(); ++i) {
            p[i] = token_text[i].data();
            n[i] = token_text[i].size();
        }
        std::vector<unsigned char> sk;
        if (!skip.empty()) {
            sk.assign(token_text.size(), 0);
            for (size_t i = 0; i < skip.size() && i < sk.size(); ++i) sk[i] = skip[i] ? 1 : 0;
        }
        h_ = tms_vocab_create(g.handle(), p.data(), n.data(), static_cast<int>(token_text.size()),
                              eos, sk.empty() ? nullptr : sk.data());
        if (!h_) throw std::runtime_error("gbnf: vocabulary setup failed");
    }
    TokenMask(const TokenMask&) = delete;
    TokenMask& operator=(const TokenMask&) = delete;
    ~TokenMask() {
        if (h_) tms_vocab_free(h_);
    }

    int node_count() const { return tms_vocab_node_count(h_); }

    std::vector<int> allowed(const State& s) const {
        const int n = tms_vocab_allowed(h_, s.handle(), nullptr, 0);
        std::vector<int32_t> ids(static_cast<size_t>(n > 0 ? n : 0));
        if (n > 0) tms_vocab_allowed(h_, s.handle(), ids.data(), n);
        return std::vector<int>(ids.begin(), ids.end());
    }

    // Bit id & 31 of words[id >> 5] for every allowed id; returns the count.
    int mask(const State& s, uint32_t* words, int n_words) const {
        return tms_vocab_mask(h_, s.handle(), words, n_words);
    }

    [[nodiscard]] bool consume(State& s, int id) const {
        return tms_vocab_consume(h_, g_.handle(), s.handle(), id) != 0;
    }
    void clear_cache() const { tms_vocab_clear_cache(h_); }

private:
    const Grammar& g_;
    tms_vocab* h_ = nullptr;
};

}  // namespace tmgbnf_amd

// ref_gbnf.cpp -- C entry points around the reference's own gbnf.h.
//
// TEST INFRASTRUCTURE ONLY.  Compiled by oracle/Makefile against the header
// where it lies in the reference tree (-I$(REF)) into oracle/_ref/, never
// committed.  tests/golden/make_gbnf_golden.py uses it to record allowed-id
// sets along grammar walks, the fixtures the host GBNF engine is pinned on.

#include "gbnf.h"

#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

extern "C" {

// 1 = accepted, 0 = rejected, -1 = the grammar does not parse.
int ref_gbnf_accepts(const char* grammar, const char* text, std::size_t len) {
    try {
        const auto g = tmgbnf::Grammar::parse(grammar);
        return g.accepts(std::string_view(text, len)) ? 1 : 0;
    } catch (const std::exception&) {
        return -1;
    }
}

// Walk `steps` tokens: at each step record the allowed ids (ascending) and
// can_end, then consume the allowed id picked by a 64-bit LCG from `seed`
// (stopping early when nothing is allowed or EOS is picked).  Returns the
// number of steps recorded, -1 if the grammar does not parse, -2 when `cap`
// ids do not fit.  offsets[k]..offsets[k+1] index step k's ids in `ids`.
int ref_gbnf_walk(const char* grammar, const char* const* text, const std::size_t* len,
                  int n_tokens, int eos, const unsigned char* skip, int steps,
                  std::uint64_t seed, std::int32_t* ids, int cap, std::int32_t* offsets,
                  std::int32_t* chosen, std::int32_t* can_end) {
    try {
        const auto g = tmgbnf::Grammar::parse(grammar);
        std::vector<std::string> toks;
        for (int i = 0; i < n_tokens; ++i) toks.emplace_back(text[i], len[i]);
        std::vector<char> sk;
        if (skip) sk.assign(skip, skip + n_tokens);
        tmgbnf::TokenMask mask(g, toks, eos, sk);
        auto s = g.start();
        int used = 0, k = 0;
        offsets[0] = 0;
        for (; k < steps; ++k) {
            const std::vector<int>& a = mask.allowed(s);
            if (used + (int)a.size() > cap) return -2;
            for (int id : a) ids[used++] = id;
            offsets[k + 1] = used;
            can_end[k] = g.can_end(s) ? 1 : 0;
            if (a.empty()) { chosen[k] = -1; ++k; break; }
            seed = seed * 6364136223846793005ull + 1442695040888963407ull;
            const int pick = a[(std::size_t)((seed >> 33) % a.size())];
            chosen[k] = pick;
            if (pick == eos) { ++k; break; }
            if (!mask.consume(s, pick, toks)) { chosen[k] = -2; ++k; break; }
        }
        return k;
    } catch (const std::exception&) {
        return -1;
    }
}

}  // extern "C"

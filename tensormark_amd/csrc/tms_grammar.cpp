// tms_grammar.cpp -- host GBNF engine that produces the sampler's
// allowed-token bitmask (one uint32 word per 32 ids, bit id & 31 of word
// id >> 5), replacing tmgbnf::Grammar / TokenMask (tensormark/gbnf.h:345-851).
//
// Language semantics follow the reference exactly, because the mask must
// allow exactly the ids the reference allows:
//   * GBNF surface: rules `name ::= body`, alternation, literals with escapes,
//     classes with ranges and negation, `.`, groups, `*` `+` `?`, `#` comments;
//     `{m,n}` is a parse error; the entry rule is `root` (gbnf.h:169-343).
//   * A pushdown automaton over codepoints: instructions CHAR / FORK / GOTO /
//     ENTER / LEAVE / ACCEPT; a parse state is the set of (pc, return stack)
//     configurations after the epsilon closure, with the reference's two
//     closure bounds (call depth relative to the incoming depth, and at most
//     2^16 visited configurations, explored in the same depth-first order)
//     (gbnf.h:628-706).
//   * Bytes, not codepoints: a state carries the bytes of an unfinished
//     codepoint; malformed UTF-8 kills the state (gbnf.h:114-167, 442-467).
//   * The token walk: a token is allowed when its whole byte string advances
//     the state and, if it ends inside a codepoint, the grammar still accepts
//     some codepoint with that prefix; EOS when the grammar can end; the
//     first id of each distinct byte string only (gbnf.h:721-851).
//
// Representation (this build's own): return stacks are interned in a tree
// (node = parent + return pc), so a configuration is two ints and a state a
// sorted vector of pairs; the vocabulary is a trie in flat arrays with each
// node's children in one contiguous, byte-sorted run; the per-state memo
// keeps the allowed ids, and the mask is written straight into the caller's
// words.  Single-threaded per grammar, like the reference.

#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <cctype>
#include <memory>
#include <stdexcept>
#include <string>
#include <string_view>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "../../include/tmsample_hip.h"

namespace tmsg {

// ------------------------------------------------------------------ UTF-8

enum class U8 { Complete, Incomplete, Invalid };

// One codepoint from the front of a byte string that holds at most one
// (possibly unfinished) encoded codepoint.
U8 utf8_front(const std::string& b, uint32_t& cp) {
    const unsigned char c0 = (unsigned char)b[0];
    int need;
    if (c0 < 0x80) {
        cp = c0;
        return U8::Complete;
    }
    if ((c0 & 0xE0) == 0xC0) { need = 1; cp = c0 & 0x1Fu; }
    else if ((c0 & 0xF0) == 0xE0) { need = 2; cp = c0 & 0x0Fu; }
    else if ((c0 & 0xF8) == 0xF0) { need = 3; cp = c0 & 0x07u; }
    else return U8::Invalid;
    const int have = std::min((int)b.size() - 1, need);
    for (int k = 1; k <= have; ++k) {
        const unsigned char ck = (unsigned char)b[(size_t)k];
        if ((ck & 0xC0) != 0x80) return U8::Invalid;
        cp = (cp << 6) | (ck & 0x3Fu);
    }
    return have < need ? U8::Incomplete : U8::Complete;
}

// Codepoints whose encoding starts with the unfinished prefix p; lo > hi if p
// does not start with a lead byte.  Over-approximates (ignores overlongs).
void utf8_prefix_span(const std::string& p, uint32_t& lo, uint32_t& hi) {
    const unsigned char c0 = (unsigned char)p[0];
    int need;
    uint32_t v, vmin, vmax;
    if ((c0 & 0xE0) == 0xC0) { need = 1; v = c0 & 0x1Fu; vmin = 0x80; vmax = 0x7FF; }
    else if ((c0 & 0xF0) == 0xE0) { need = 2; v = c0 & 0x0Fu; vmin = 0x800; vmax = 0xFFFF; }
    else if ((c0 & 0xF8) == 0xF0) { need = 3; v = c0 & 0x07u; vmin = 0x10000; vmax = 0x10FFFF; }
    else { lo = 1; hi = 0; return; }
    for (size_t k = 1; k < p.size(); ++k) v = (v << 6) | ((uint32_t)(unsigned char)p[k] & 0x3Fu);
    const int missing = need - (int)(p.size() - 1);
    lo = v << (6 * missing);
    hi = lo | ((1u << (6 * missing)) - 1u);
    lo = std::max(lo, vmin);
    hi = std::min(hi, vmax);
}

// Decode one codepoint of grammar source text (strict).
uint32_t decode_source(std::string_view s, size_t& i) {
    const unsigned char c0 = (unsigned char)s[i];
    if (c0 < 0x80) { ++i; return c0; }
    int need;
    uint32_t v;
    if ((c0 & 0xE0) == 0xC0) { need = 1; v = c0 & 0x1Fu; }
    else if ((c0 & 0xF0) == 0xE0) { need = 2; v = c0 & 0x0Fu; }
    else if ((c0 & 0xF8) == 0xF0) { need = 3; v = c0 & 0x07u; }
    else throw std::runtime_error("gbnf: invalid UTF-8 in grammar");
    ++i;
    for (int k = 0; k < need; ++k, ++i) {
        if (i >= s.size() || ((unsigned char)s[i] & 0xC0) != 0x80)
            throw std::runtime_error("gbnf: truncated UTF-8 in grammar");
        v = (v << 6) | ((unsigned char)s[i] & 0x3Fu);
    }
    return v;
}

void encode_utf8(uint32_t cp, std::string& out) {
    if (cp < 0x80) {
        out += (char)cp;
    } else if (cp < 0x800) {
        out += (char)(0xC0 | (cp >> 6));
        out += (char)(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
        out += (char)(0xE0 | (cp >> 12));
        out += (char)(0x80 | ((cp >> 6) & 0x3F));
        out += (char)(0x80 | (cp & 0x3F));
    } else {
        out += (char)(0xF0 | (cp >> 18));
        out += (char)(0x80 | ((cp >> 12) & 0x3F));
        out += (char)(0x80 | ((cp >> 6) & 0x3F));
        out += (char)(0x80 | (cp & 0x3F));
    }
}

// ------------------------------------------------------------------ syntax tree

struct Span { uint32_t lo, hi; };

struct Term {
    enum Kind { Lit, Set, Any, Rule } kind = Lit;
    std::string text;            // Lit: UTF-8
    std::vector<Span> spans;     // Set
    bool negate = false;         // Set
    std::string name;            // Rule reference (resolved below)
    int rule = -1;
    char rep = 0;                // 0, '*', '+', '?'
};
using Seq = std::vector<Term>;
struct RuleDef {
    std::string name;
    std::vector<Seq> alts;
};

class Reader {
public:
    explicit Reader(std::string_view src) : s_(src) {}

    // rules in source order, then the groups in creation order
    std::vector<RuleDef> read_all() {
        std::vector<RuleDef> out;
        for (;;) {
            blank();
            if (i_ >= s_.size()) break;
            RuleDef r;
            r.name = name();
            owner_ = r.name;
            blank();
            if (s_.compare(i_, 3, "::=") != 0) error("expected '::='");
            i_ += 3;
            r.alts = choice();
            out.push_back(std::move(r));
        }
        for (auto& g : groups_) out.push_back(std::move(g));
        return out;
    }

private:
    [[noreturn]] void error(const std::string& m) const {
        throw std::runtime_error("gbnf: " + m + " at offset " + std::to_string(i_));
    }
    char cur() const { return i_ < s_.size() ? s_[i_] : '\0'; }
    void blank() {
        while (i_ < s_.size()) {
            if (std::isspace((unsigned char)s_[i_])) { ++i_; continue; }
            if (s_[i_] == '#') {
                while (i_ < s_.size() && s_[i_] != '\n') ++i_;
                continue;
            }
            break;
        }
    }
    static bool name_start(char c) { return std::isalpha((unsigned char)c) || c == '_'; }
    static bool name_char(char c) { return std::isalnum((unsigned char)c) || c == '_' || c == '-'; }
    std::string name() {
        blank();
        if (i_ >= s_.size() || !name_start(s_[i_])) error("expected a rule name");
        const size_t b = i_;
        while (i_ < s_.size() && name_char(s_[i_])) ++i_;
        return std::string(s_.substr(b, i_ - b));
    }
    // `name ::=` ahead (nothing consumed)
    bool rule_ahead() {
        const size_t keep = i_;
        blank();
        bool yes = false;
        if (i_ < s_.size() && name_start(s_[i_])) {
            while (i_ < s_.size() && name_char(s_[i_])) ++i_;
            blank();
            yes = s_.compare(i_, 3, "::=") == 0;
        }
        i_ = keep;
        return yes;
    }
    uint32_t escaped() {
        const char c = s_[i_++];
        switch (c) {
            case 'n': return '\n';
            case 'r': return '\r';
            case 't': return '\t';
            case '0': return 0;
            case 'x':
            case 'u': {
                const int digits = c == 'x' ? 2 : 4;
                if (i_ + (size_t)digits > s_.size()) error("short hex escape");
                uint32_t v = 0;
                for (int k = 0; k < digits; ++k) {
                    const char h = s_[i_++];
                    int d;
                    if (h >= '0' && h <= '9') d = h - '0';
                    else if (h >= 'a' && h <= 'f') d = h - 'a' + 10;
                    else if (h >= 'A' && h <= 'F') d = h - 'A' + 10;
                    else error("bad hex digit");
                    v = v * 16 + (uint32_t)d;
                }
                return v;
            }
            default: return (uint32_t)(unsigned char)c;   // \\ \" \' \[ \] and any other
        }
    }
    uint32_t one_char() {
        if (s_[i_] == '\\') {
            ++i_;
            return escaped();
        }
        return decode_source(s_, i_);
    }
    std::vector<Seq> choice() {
        std::vector<Seq> alts;
        alts.push_back(sequence());
        for (;;) {
            blank();
            if (cur() != '|') break;
            ++i_;
            alts.push_back(sequence());
        }
        return alts;
    }
    Seq sequence() {
        Seq seq;
        for (;;) {
            blank();
            const char c = cur();
            if (c == '\0' || c == '|' || c == ')' || rule_ahead()) break;
            Term t = primary();
            blank();
            const char r = cur();
            if (r == '*' || r == '+' || r == '?') {
                t.rep = r;
                ++i_;
            } else if (r == '{') {
                error("counted repetition {m,n} is not supported");
            }
            seq.push_back(std::move(t));
        }
        return seq;
    }
    Term primary() {
        blank();
        Term t;
        const char c = cur();
        if (c == '"') {
            ++i_;
            t.kind = Term::Lit;
            while (i_ < s_.size() && s_[i_] != '"') encode_utf8(one_char(), t.text);
            if (i_ >= s_.size()) error("unterminated literal");
            ++i_;
        } else if (c == '[') {
            ++i_;
            t.kind = Term::Set;
            if (cur() == '^') {
                t.negate = true;
                ++i_;
            }
            while (i_ < s_.size() && s_[i_] != ']') {
                const uint32_t lo = one_char();
                uint32_t hi = lo;
                if (cur() == '-' && i_ + 1 < s_.size() && s_[i_ + 1] != ']') {
                    ++i_;
                    hi = one_char();
                }
                if (hi < lo) error("inverted range in character class");
                t.spans.push_back(Span{lo, hi});
            }
            if (i_ >= s_.size()) error("unterminated character class");
            ++i_;
        } else if (c == '(') {
            ++i_;
            RuleDef g;
            g.name = "group:" + owner_ + ":" + std::to_string(n_groups_++);
            g.alts = choice();
            blank();
            if (cur() != ')') error("expected ')'");
            ++i_;
            t.kind = Term::Rule;
            t.name = g.name;
            groups_.push_back(std::move(g));
        } else if (c == '.') {
            ++i_;
            t.kind = Term::Any;
        } else {
            t.kind = Term::Rule;
            t.name = name();
        }
        return t;
    }

    std::string_view s_;
    size_t i_ = 0;
    std::string owner_;
    int n_groups_ = 0;
    std::vector<RuleDef> groups_;
};

// ------------------------------------------------------------------ automaton

enum class Op : uint8_t { Char, Fork, Goto, Enter, Leave, Accept };

struct Ins {
    Op op = Op::Accept;
    int next = -1;     // Char / Goto: target; Fork: first branch
    int alt = -1;      // Fork: second branch; Enter: return address
    int callee = -1;   // Enter: rule
    int set = -1;      // Char: index into sets (-1 = any codepoint)
};

struct CodeSet {
    std::vector<Span> spans;
    bool negate = false;
    bool has(uint32_t cp) const {
        bool in = false;
        for (const Span& s : spans)
            if (cp >= s.lo && cp <= s.hi) { in = true; break; }
        return negate ? !in : in;
    }
    // Does the set accept some codepoint in [lo, hi]?
    bool meets(uint32_t lo, uint32_t hi) const {
        if (!negate) {
            for (const Span& s : spans)
                if (s.lo <= hi && s.hi >= lo) return true;
            return false;
        }
        // Complement: advance past covering spans until none covers `p`.
        uint32_t p = lo;
        for (bool moved = true; moved && p <= hi;) {
            moved = false;
            for (const Span& s : spans)
                if (s.lo <= p && p <= s.hi) {
                    p = s.hi >= hi ? hi + 1 : s.hi + 1;
                    moved = true;
                }
        }
        return p <= hi;
    }
};

struct Config {
    int pc;
    int stack;   // interned return stack (0 = empty)
    bool operator==(const Config& o) const { return pc == o.pc && stack == o.stack; }
};

struct ConfigHash {
    size_t operator()(const Config& c) const {
        return ((uint64_t)(uint32_t)c.pc << 32 | (uint32_t)c.stack) * 0x9E3779B97F4A7C15ull >> 7;
    }
};

struct State {
    std::vector<Config> cfg;   // canonical order, no duplicates
    std::string pending;       // bytes of an unfinished codepoint
    bool operator==(const State& o) const { return pending == o.pending && cfg == o.cfg; }
};

struct StateHash {
    size_t operator()(const State& s) const {
        uint64_t h = std::hash<std::string>{}(s.pending) ^ 0x51ED27A3u;
        for (const Config& c : s.cfg)
            h = (h ^ ((uint64_t)(uint32_t)c.pc << 32 | (uint32_t)c.stack)) * 0x100000001B3ull;
        return (size_t)(h ^ (h >> 31));
    }
};

class Machine {
public:
    explicit Machine(std::string_view src) {
        Reader rd(src);
        rules_ = rd.read_all();
        std::unordered_map<std::string, int> index;
        for (size_t r = 0; r < rules_.size(); ++r) {
            if (!index.emplace(rules_[r].name, (int)r).second)
                throw std::runtime_error("gbnf: duplicate rule '" + rules_[r].name + "'");
        }
        auto root = index.find("root");
        if (root == index.end()) throw std::runtime_error("gbnf: no 'root' rule");
        root_ = root->second;
        for (RuleDef& r : rules_)
            for (Seq& a : r.alts)
                for (Term& t : a)
                    if (t.kind == Term::Rule) {
                        auto it = index.find(t.name);
                        if (it == index.end())
                            throw std::runtime_error("gbnf: unknown rule '" + t.name + "'");
                        t.rule = it->second;
                    }
        assemble();
        stacks_.push_back(StackNode{-1, -1, 0});   // the empty stack
    }

    int rule_count() const { return (int)rules_.size(); }

    State start() {
        State s;
        s.cfg.push_back(Config{entry_[(size_t)root_], 0});
        close(s);
        return s;
    }

    bool can_end(const State& s) const {
        if (!s.pending.empty()) return false;
        for (const Config& c : s.cfg)
            if (code_[(size_t)c.pc].op == Op::Accept) return true;
        return false;
    }

    bool advance(State& s, unsigned char byte) {
        std::string bytes = s.pending;
        bytes += (char)byte;
        uint32_t cp = 0;
        const U8 r = utf8_front(bytes, cp);
        if (r == U8::Invalid || (r == U8::Incomplete && bytes.size() > 4)) {
            s.cfg.clear();
            return false;
        }
        if (r == U8::Incomplete) {
            s.pending = std::move(bytes);
            return true;
        }
        s.pending.clear();
        std::vector<Config> moved;
        for (const Config& c : s.cfg) {
            const Ins& in = code_[(size_t)c.pc];
            if (in.op == Op::Char && (in.set < 0 || sets_[(size_t)in.set].has(cp)))
                moved.push_back(Config{in.next, c.stack});
        }
        s.cfg = std::move(moved);
        close(s);
        return !s.cfg.empty();
    }

    // May a token that leaves `s` inside a codepoint be taken?
    bool admissible(const State& s) const {
        if (s.pending.empty()) return true;
        uint32_t lo, hi;
        utf8_prefix_span(s.pending, lo, hi);
        if (lo > hi) return false;
        for (const Config& c : s.cfg) {
            const Ins& in = code_[(size_t)c.pc];
            if (in.op != Op::Char) continue;
            if (in.set < 0 || sets_[(size_t)in.set].meets(lo, hi)) return true;
        }
        return false;
    }

private:
    struct StackNode {
        int below;   // stack without the top entry
        int top;     // return pc
        int depth;
    };

    int push(int stack, int ret) {
        const uint64_t key = (uint64_t)(uint32_t)stack << 32 | (uint32_t)ret;
        auto it = intern_.find(key);
        if (it != intern_.end()) return it->second;
        const int id = (int)stacks_.size();
        stacks_.push_back(StackNode{stack, ret, stacks_[(size_t)stack].depth + 1});
        intern_.emplace(key, id);
        return id;
    }

    // Order of configurations: pc, then the return stack compared bottom to
    // top (a shorter stack that is a prefix comes first).
    bool before(const Config& a, const Config& b) const {
        if (a.pc != b.pc) return a.pc < b.pc;
        if (a.stack == b.stack) return false;
        return stack_less(a.stack, b.stack);
    }
    bool stack_less(int x, int y) const {
        std::vector<int> vx, vy;
        for (int n = x; n > 0; n = stacks_[(size_t)n].below) vx.push_back(stacks_[(size_t)n].top);
        for (int n = y; n > 0; n = stacks_[(size_t)n].below) vy.push_back(stacks_[(size_t)n].top);
        return std::lexicographical_compare(vx.rbegin(), vx.rend(), vy.rbegin(), vy.rend());
    }

    // Epsilon closure: follow Fork / Goto / Enter / Leave until only Char and
    // Accept configurations remain.  Depth-first from the last configuration
    // (the visit order fixes which configurations a capped closure keeps);
    // an Enter at depth >= (incoming depth + 2 * rules + 8) is dropped, and
    // at most 2^16 configurations are visited.
    void close(State& s) {
        constexpr size_t kVisitCap = 1u << 16;
        int depth0 = 0;
        for (const Config& c : s.cfg) depth0 = std::max(depth0, stacks_[(size_t)c.stack].depth);
        const int depth_cap = depth0 + 2 * (int)rules_.size() + 8;
        std::vector<Config> todo = s.cfg, keep;
        std::unordered_set<Config, ConfigHash> visited;
        while (!todo.empty() && visited.size() < kVisitCap) {
            const Config c = todo.back();
            todo.pop_back();
            if (!visited.insert(c).second) continue;
            const Ins& in = code_[(size_t)c.pc];
            switch (in.op) {
                case Op::Goto: todo.push_back(Config{in.next, c.stack}); break;
                case Op::Fork:
                    todo.push_back(Config{in.next, c.stack});
                    todo.push_back(Config{in.alt, c.stack});
                    break;
                case Op::Enter:
                    if (stacks_[(size_t)c.stack].depth < depth_cap)
                        todo.push_back(Config{entry_[(size_t)in.callee], push(c.stack, in.alt)});
                    break;
                case Op::Leave:
                    if (c.stack == 0) todo.push_back(Config{accept_pc_, 0});
                    else todo.push_back(Config{stacks_[(size_t)c.stack].top, stacks_[(size_t)c.stack].below});
                    break;
                default: keep.push_back(c); break;
            }
        }
        std::sort(keep.begin(), keep.end(), [this](const Config& a, const Config& b) { return before(a, b); });
        keep.erase(std::unique(keep.begin(), keep.end()), keep.end());
        s.cfg = std::move(keep);
    }

    int emit(const Ins& in) {
        code_.push_back(in);
        return (int)code_.size() - 1;
    }

    // Rule r: a chain of forks reaching every alternative, each alternative
    // followed by a Goto to the rule's Leave.
    void assemble() {
        entry_.assign(rules_.size(), -1);
        for (size_t r = 0; r < rules_.size(); ++r) {
            entry_[r] = (int)code_.size();
            const size_t n = rules_[r].alts.size();
            std::vector<int> forks, starts, exits;
            for (size_t k = 0; k + 1 < n; ++k) forks.push_back(emit(Ins{Op::Fork}));
            for (size_t k = 0; k < n; ++k) {
                starts.push_back((int)code_.size());
                for (const Term& t : rules_[r].alts[k]) term(t);
                exits.push_back(emit(Ins{Op::Goto}));
            }
            const int leave = emit(Ins{Op::Leave});
            for (int e : exits) code_[(size_t)e].next = leave;
            for (size_t k = 0; k + 1 < n; ++k) {
                code_[(size_t)forks[k]].next = starts[k];
                code_[(size_t)forks[k]].alt = k + 2 == n ? starts[k + 1] : forks[k + 1];
            }
        }
        accept_pc_ = emit(Ins{Op::Accept});
    }

    void term(const Term& t) {
        switch (t.rep) {
            case 0: body(t); break;
            case '?': {
                const int f = emit(Ins{Op::Fork});
                code_[(size_t)f].next = (int)code_.size();
                body(t);
                code_[(size_t)f].alt = (int)code_.size();
                break;
            }
            case '*': {
                const int f = emit(Ins{Op::Fork});
                code_[(size_t)f].next = (int)code_.size();
                body(t);
                Ins back{Op::Goto};
                back.next = f;
                emit(back);
                code_[(size_t)f].alt = (int)code_.size();
                break;
            }
            default: {   // '+'
                const int first = (int)code_.size();
                body(t);
                Ins again{Op::Fork};
                again.next = first;
                const int f = emit(again);
                code_[(size_t)f].alt = (int)code_.size();
                break;
            }
        }
    }

    void body(const Term& t) {
        if (t.kind == Term::Lit) {
            size_t i = 0;
            while (i < t.text.size()) {
                const uint32_t cp = decode_source(t.text, i);
                Ins in{Op::Char};
                in.set = (int)sets_.size();
                sets_.push_back(CodeSet{{Span{cp, cp}}, false});
                in.next = (int)code_.size() + 1;
                emit(in);
            }
        } else if (t.kind == Term::Set || t.kind == Term::Any) {
            Ins in{Op::Char};
            if (t.kind == Term::Set) {
                in.set = (int)sets_.size();
                sets_.push_back(CodeSet{t.spans, t.negate});
            }
            in.next = (int)code_.size() + 1;
            emit(in);
        } else {
            Ins in{Op::Enter};
            in.callee = t.rule;
            in.alt = (int)code_.size() + 1;
            emit(in);
        }
    }

    std::vector<RuleDef> rules_;
    std::vector<Ins> code_;
    std::vector<CodeSet> sets_;
    std::vector<int> entry_;
    int root_ = 0;
    int accept_pc_ = 0;
    std::vector<StackNode> stacks_;
    std::unordered_map<uint64_t, int> intern_;
};

// ------------------------------------------------------------------ vocabulary walk

class Vocab {
public:
    Vocab(Machine& m, const char* const* text, const size_t* len, int n, int eos,
          const unsigned char* skip)
        : m_(m), eos_(eos), n_(n) {
        // Build the trie with hash children first, then flatten it.
        struct Tmp {
            std::unordered_map<unsigned char, int> kids;
            int token = -1;
        };
        std::vector<Tmp> tmp(1);
        for (int id = 0; id < n; ++id) {
            if ((skip && skip[id]) || id == eos || len[id] == 0) continue;
            int at = 0;
            for (size_t k = 0; k < len[id]; ++k) {
                const unsigned char b = (unsigned char)text[id][k];
                auto it = tmp[(size_t)at].kids.find(b);
                if (it == tmp[(size_t)at].kids.end()) {
                    tmp.push_back(Tmp{});
                    const int nx = (int)tmp.size() - 1;
                    tmp[(size_t)at].kids.emplace(b, nx);
                    at = nx;
                } else {
                    at = it->second;
                }
            }
            if (tmp[(size_t)at].token < 0) tmp[(size_t)at].token = id;   // first id wins
        }
        // Breadth-first renumbering: every node's children are one run.
        const size_t N = tmp.size();
        std::vector<int> order{0}, newid(N, -1);
        newid[0] = 0;
        first_.assign(N, 0);
        count_.assign(N, 0);
        token_.assign(N, -1);
        byte_.assign(N, 0);
        for (size_t q = 0; q < order.size(); ++q) {
            const int old = order[q];
            std::vector<std::pair<unsigned char, int>> kids(tmp[(size_t)old].kids.begin(),
                                                            tmp[(size_t)old].kids.end());
            std::sort(kids.begin(), kids.end());
            first_[q] = (int)order.size();
            count_[q] = (int)kids.size();
            token_[q] = tmp[(size_t)old].token;
            for (const auto& kb : kids) {
                newid[(size_t)kb.second] = (int)order.size();
                byte_[order.size()] = kb.first;
                order.push_back(kb.second);
            }
        }
    }

    int nodes() const { return (int)token_.size(); }

    const std::vector<int>& allowed(const State& s) {
        auto it = memo_.find(s);
        if (it != memo_.end()) return it->second;
        std::vector<int> ids;
        descend(0, s, ids);
        if (eos_ >= 0 && m_.can_end(s)) ids.push_back(eos_);
        std::sort(ids.begin(), ids.end());
        ids.erase(std::unique(ids.begin(), ids.end()), ids.end());
        return memo_.emplace(s, std::move(ids)).first->second;
    }

    void forget() { memo_.clear(); }
    int eos() const { return eos_; }
    int size() const { return n_; }

private:
    void descend(int node, const State& s, std::vector<int>& ids) {
        if (token_[(size_t)node] >= 0 && m_.admissible(s)) ids.push_back(token_[(size_t)node]);
        for (int c = first_[(size_t)node], e = c + count_[(size_t)node]; c < e; ++c) {
            State t = s;
            if (!m_.advance(t, byte_[(size_t)c])) continue;
            descend(c, t, ids);
        }
    }

    Machine& m_;
    int eos_;
    int n_;
    std::vector<int> first_, count_, token_;
    std::vector<unsigned char> byte_;
    std::unordered_map<State, std::vector<int>, StateHash> memo_;
};

}  // namespace tmsg

// ====================================================================== C ABI

struct tms_grammar {
    std::unique_ptr<tmsg::Machine> m;
};
struct tms_gstate {
    tmsg::State s;
};
struct tms_vocab {
    std::unique_ptr<tmsg::Vocab> v;
    std::vector<std::string> text;   // token bytes, for consume
};

namespace {
void put_error(char* err, size_t cap, const char* msg) {
    if (!err || cap == 0) return;
    const size_t n = strlen(msg) < cap - 1 ? strlen(msg) : cap - 1;
    memcpy(err, msg, n);
    err[n] = '\0';
}
}  // namespace

extern "C" tms_grammar* tms_grammar_parse(const char* text, size_t len, char* err, size_t err_cap) {
    if (!text) {
        put_error(err, err_cap, "gbnf: null grammar text");
        return nullptr;
    }
    try {
        auto* g = new tms_grammar;
        g->m = std::make_unique<tmsg::Machine>(std::string_view(text, len));
        put_error(err, err_cap, "");
        return g;
    } catch (const std::exception& e) {
        put_error(err, err_cap, e.what());
        return nullptr;
    }
}

extern "C" void tms_grammar_free(tms_grammar* g) { delete g; }

extern "C" int tms_grammar_rule_count(const tms_grammar* g) { return g ? g->m->rule_count() : -1; }

extern "C" tms_gstate* tms_grammar_start(tms_grammar* g) {
    if (!g) return nullptr;
    auto* s = new tms_gstate;
    s->s = g->m->start();
    return s;
}

extern "C" tms_gstate* tms_gstate_copy(const tms_gstate* s) { return s ? new tms_gstate(*s) : nullptr; }

extern "C" void tms_gstate_free(tms_gstate* s) { delete s; }

extern "C" int tms_gstate_equal(const tms_gstate* a, const tms_gstate* b) {
    return a && b && a->s == b->s ? 1 : 0;
}

extern "C" int tms_grammar_advance(tms_grammar* g, tms_gstate* s, unsigned char byte) {
    if (!g || !s) return 0;
    return g->m->advance(s->s, byte) ? 1 : 0;
}

extern "C" int tms_grammar_can_end(const tms_grammar* g, const tms_gstate* s) {
    return g && s && g->m->can_end(s->s) ? 1 : 0;
}

extern "C" int tms_grammar_accepts(tms_grammar* g, const char* text, size_t len) {
    if (!g) return 0;
    tmsg::State s = g->m->start();
    for (size_t i = 0; i < len; ++i)
        if (!g->m->advance(s, (unsigned char)text[i])) return 0;
    return g->m->can_end(s) ? 1 : 0;
}

extern "C" tms_vocab* tms_vocab_create(tms_grammar* g, const char* const* text, const size_t* len,
                                       int n_tokens, int eos, const unsigned char* skip) {
    if (!g || n_tokens < 0 || (n_tokens > 0 && (!text || !len))) return nullptr;
    try {
        auto* v = new tms_vocab;
        v->v = std::make_unique<tmsg::Vocab>(*g->m, text, len, n_tokens, eos, skip);
        v->text.reserve((size_t)n_tokens);
        for (int i = 0; i < n_tokens; ++i) v->text.emplace_back(text[i], len[i]);
        return v;
    } catch (const std::exception&) {
        return nullptr;
    }
}

extern "C" void tms_vocab_free(tms_vocab* v) { delete v; }

extern "C" int tms_vocab_node_count(const tms_vocab* v) { return v ? v->v->nodes() : -1; }

extern "C" int tms_vocab_allowed(tms_vocab* v, const tms_gstate* s, int32_t* ids, int cap) {
    if (!v || !s) return -1;
    const std::vector<int>& a = v->v->allowed(s->s);
    const int n = (int)a.size();
    if (ids)
        for (int i = 0; i < n && i < cap; ++i) ids[i] = a[(size_t)i];
    return n;
}

extern "C" int tms_vocab_mask(tms_vocab* v, const tms_gstate* s, uint32_t* words, int n_words) {
    if (!v || !s || !words || n_words < 0) return -1;
    const std::vector<int>& a = v->v->allowed(s->s);
    memset(words, 0, sizeof(uint32_t) * (size_t)n_words);
    int n = 0;
    for (int id : a) {
        if (id < 0 || (id >> 5) >= n_words) continue;
        words[id >> 5] |= 1u << (id & 31);
        ++n;
    }
    return n;
}

extern "C" int tms_vocab_consume(tms_vocab* v, tms_grammar* g, tms_gstate* s, int id) {
    if (!v || !g || !s) return 0;
    if (id == v->v->eos()) return g->m->can_end(s->s) ? 1 : 0;
    if (id < 0 || id >= (int)v->text.size()) return 0;
    for (unsigned char b : v->text[(size_t)id])
        if (!g->m->advance(s->s, b)) return 0;
    return s->s.cfg.empty() ? 0 : 1;
}

extern "C" void tms_vocab_clear_cache(tms_vocab* v) {
    if (v) v->v->forget();
}

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
    else throw std::runtime_error("gbnf: lexer error at byte " + std::to_string(i) + ": not a UTF-8 lead byte");
    ++i;
    for (int k = 0; k < need; ++k, ++i) {
        if (i >= s.size() || ((unsigned char)s[i] & 0xC0) != 0x80)
            throw std::runtime_error("gbnf: lexer error at byte " + std::to_string(i) + ": UTF-8 sequence cut short");
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

// ------------------------------------------------------------------ front end
//
// Two stages.  The lexer turns the source into a flat token list (literal
// and class contents already decoded to codepoints), so every question the
// parser asks is a look at the next one or two tokens.  The parser is a
// loop over that list with an explicit stack of open groups: each frame
// holds the alternatives finished so far and the sequence being built; `(`
// pushes a frame, `)` pops one into a synthetic rule, `|` closes a
// sequence, and a rule name followed by `::=` at depth 0 starts the next
// rule.  Errors are "gbnf: <stage> error at byte N: <what>".

enum class Tk : uint8_t { Name, Define, Literal, Class, Dot, Open, Close, Bar, Star, Plus, Quest, Count, End };

struct Token {
    Tk kind;
    size_t at;                   // byte offset in the source
    std::string text;            // Name: the name; Literal: UTF-8 of the decoded codepoints
    std::vector<Span> spans;     // Class
    bool negate = false;         // Class
};

[[noreturn]] void syntax_fail(const char* stage, size_t at, const std::string& what) {
    throw std::runtime_error(std::string("gbnf: ") + stage + " error at byte " + std::to_string(at) + ": " + what);
}

class Lexer {
public:
    explicit Lexer(std::string_view src) : src_(src) {}

    std::vector<Token> run() {
        std::vector<Token> out;
        for (;;) {
            skip_layout();
            if (pos_ >= src_.size()) break;
            out.push_back(next());
        }
        out.push_back(Token{Tk::End, src_.size(), {}, {}, false});
        return out;
    }

private:
    static bool is_name_head(char c) { return (c >= 'a' && c <= 'z') || (c >= 'A' && c <= 'Z') || c == '_'; }
    static bool is_name_body(char c) { return is_name_head(c) || (c >= '0' && c <= '9') || c == '-'; }

    void skip_layout() {   // whitespace and # comments
        while (pos_ < src_.size()) {
            const char c = src_[pos_];
            if (c == '#') {
                const size_t nl = src_.find('\n', pos_);
                pos_ = nl == std::string_view::npos ? src_.size() : nl;
            } else if (std::isspace((unsigned char)c)) {
                ++pos_;
            } else {
                return;
            }
        }
    }

    static int hex_value(char h) {
        if (h >= '0' && h <= '9') return h - '0';
        const char l = (char)(h | 0x20);
        return (l >= 'a' && l <= 'f') ? l - 'a' + 10 : -1;
    }

    // One codepoint of a literal or class body: an escape or a UTF-8 sequence.
    uint32_t body_codepoint() {
        if (src_[pos_] != '\\') return decode_source(src_, pos_);
        const size_t esc = pos_++;
        if (pos_ >= src_.size()) syntax_fail("lexer", esc, "backslash at the end of the grammar");
        const char c = src_[pos_++];
        static const struct { char key; uint32_t cp; } simple[] = {{'n', '\n'}, {'r', '\r'}, {'t', '\t'}, {'0', 0}};
        for (const auto& e : simple)
            if (e.key == c) return e.cp;
        if (c != 'x' && c != 'u') return (uint32_t)(unsigned char)c;   // \\ \" \' \[ \] and the rest: the character
        const size_t width = c == 'x' ? 2 : 4;
        if (src_.size() - pos_ < width) syntax_fail("lexer", esc, "hex escape cut short");
        uint32_t cp = 0;
        for (size_t k = 0; k < width; ++k) {
            const int d = hex_value(src_[pos_ + k]);
            if (d < 0) syntax_fail("lexer", pos_ + k, "not a hex digit in an escape");
            cp = cp * 16 + (uint32_t)d;
        }
        pos_ += width;
        return cp;
    }

    Token next() {
        const size_t at = pos_;
        const char c = src_[pos_];
        Token t{Tk::End, at, {}, {}, false};
        static const struct { char ch; Tk kind; } single[] = {
            {'.', Tk::Dot}, {'(', Tk::Open}, {')', Tk::Close}, {'|', Tk::Bar},
            {'*', Tk::Star}, {'+', Tk::Plus}, {'?', Tk::Quest}};
        for (const auto& e : single)
            if (e.ch == c) {
                ++pos_;
                t.kind = e.kind;
                return t;
            }
        if (c == '{') {   // {m,n}: one token, which the parser rejects
            const size_t close = src_.find('}', pos_);
            pos_ = close == std::string_view::npos ? src_.size() : close + 1;
            t.kind = Tk::Count;
            return t;
        }
        if (src_.compare(pos_, 3, "::=") == 0) {
            pos_ += 3;
            t.kind = Tk::Define;
            return t;
        }
        if (is_name_head(c)) {
            while (pos_ < src_.size() && is_name_body(src_[pos_])) ++pos_;
            t.kind = Tk::Name;
            t.text.assign(src_.substr(at, pos_ - at));
            return t;
        }
        if (c == '"') {
            ++pos_;
            t.kind = Tk::Literal;
            while (pos_ < src_.size() && src_[pos_] != '"') encode_utf8(body_codepoint(), t.text);
            if (pos_ >= src_.size()) syntax_fail("lexer", at, "string literal never closed");
            ++pos_;
            return t;
        }
        if (c == '[') {
            ++pos_;
            t.kind = Tk::Class;
            if (pos_ < src_.size() && src_[pos_] == '^') {
                t.negate = true;
                ++pos_;
            }
            while (pos_ < src_.size() && src_[pos_] != ']') {
                const size_t item = pos_;
                Span sp;
                sp.lo = sp.hi = body_codepoint();
                // `a-z` is a range unless the '-' is the class's last character
                if (pos_ + 1 < src_.size() && src_[pos_] == '-' && src_[pos_ + 1] != ']') {
                    ++pos_;
                    sp.hi = body_codepoint();
                }
                if (sp.hi < sp.lo) syntax_fail("lexer", item, "character range runs backwards");
                t.spans.push_back(sp);
            }
            if (pos_ >= src_.size()) syntax_fail("lexer", at, "character class never closed");
            ++pos_;
            return t;
        }
        syntax_fail("lexer", at, std::string("unexpected character '") + c + "'");
    }

    std::string_view src_;
    size_t pos_ = 0;
};

// Rules in source order, then the synthetic group rules in the order their
// ')' closed them.
std::vector<RuleDef> parse_grammar(std::string_view src) {
    const std::vector<Token> toks = Lexer(src).run();
    struct Frame {
        std::vector<Seq> alts;
        Seq seq;
        size_t opened_at;
    };
    std::vector<RuleDef> rules, groups;
    std::vector<Frame> open;   // open[0]: the rule body; open[d]: group at depth d
    std::vector<int> group_serial;   // per rule: groups named so far
    auto starts_rule = [&](size_t i) { return toks[i].kind == Tk::Name && toks[i + 1].kind == Tk::Define; };
    auto finish_rule = [&]() {
        Frame& f = open.back();
        f.alts.push_back(std::move(f.seq));
        rules.back().alts = std::move(f.alts);
        open.clear();
    };
    size_t i = 0;
    for (;;) {
        const Token& tk = toks[i];
        if (tk.kind == Tk::End || starts_rule(i)) {
            if (open.size() > 1) syntax_fail("parser", open.back().opened_at, "'(' is never closed");
            if (!open.empty()) finish_rule();
            if (tk.kind == Tk::End) break;
            RuleDef r;
            r.name = tk.text;
            rules.push_back(std::move(r));
            group_serial.push_back(0);
            open.push_back(Frame{{}, {}, tk.at});
            i += 2;
            continue;
        }
        if (open.empty()) syntax_fail("parser", tk.at, "expected a rule: a name followed by '::='");
        Frame& f = open.back();
        switch (tk.kind) {
            case Tk::Bar:
                f.alts.push_back(std::move(f.seq));
                f.seq.clear();
                break;
            case Tk::Open:
                open.push_back(Frame{{}, {}, tk.at});
                break;
            case Tk::Close: {
                if (open.size() == 1) syntax_fail("parser", tk.at, "')' without a matching '('");
                RuleDef g;
                g.name = "(" + rules.back().name + ")#" + std::to_string(group_serial.back()++);
                f.alts.push_back(std::move(f.seq));
                g.alts = std::move(f.alts);
                open.pop_back();
                Term ref;
                ref.kind = Term::Rule;
                ref.name = g.name;
                open.back().seq.push_back(std::move(ref));
                groups.push_back(std::move(g));
                break;
            }
            case Tk::Star:
            case Tk::Plus:
            case Tk::Quest: {
                if (f.seq.empty()) syntax_fail("parser", tk.at, "repetition operator with nothing before it");
                Term& last = f.seq.back();
                if (last.rep) syntax_fail("parser", tk.at, "two repetition operators in a row");
                last.rep = tk.kind == Tk::Star ? '*' : (tk.kind == Tk::Plus ? '+' : '?');
                break;
            }
            case Tk::Count:
                syntax_fail("parser", tk.at, "counted repetition {m,n} is not part of this grammar language");
            case Tk::Define:
                syntax_fail("parser", tk.at, "'::=' without a rule name before it");
            default: {   // an atom
                Term t;
                if (tk.kind == Tk::Literal) {
                    t.kind = Term::Lit;
                    t.text = tk.text;
                } else if (tk.kind == Tk::Class) {
                    t.kind = Term::Set;
                    t.spans = tk.spans;
                    t.negate = tk.negate;
                } else if (tk.kind == Tk::Dot) {
                    t.kind = Term::Any;
                } else {
                    t.kind = Term::Rule;
                    t.name = tk.text;
                }
                f.seq.push_back(std::move(t));
                break;
            }
        }
        ++i;
    }
    for (RuleDef& g : groups) rules.push_back(std::move(g));
    return rules;
}

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
        rules_ = parse_grammar(src);
        std::unordered_map<std::string, int> index;
        for (size_t r = 0; r < rules_.size(); ++r) {
            if (!index.emplace(rules_[r].name, (int)r).second)
                throw std::runtime_error("gbnf: rule error: '" + rules_[r].name + "' is defined twice");
        }
        auto root = index.find("root");
        if (root == index.end()) throw std::runtime_error("gbnf: rule error: the grammar defines no 'root' rule");
        root_ = root->second;
        for (RuleDef& r : rules_)
            for (Seq& a : r.alts)
                for (Term& t : a)
                    if (t.kind == Term::Rule) {
                        auto it = index.find(t.name);
                        if (it == index.end())
                            throw std::runtime_error("gbnf: rule error: '" + t.name + "' is used but never defined");
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

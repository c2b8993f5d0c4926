// tms_filter.cpp -- the host side of grammar-constrained decoding around the
// device sampler:
//
//   * token tables: the bytes each vocabulary id contributes to a running
//     decode, derived from the tokenizer's pieces the way the reference's
//     tokenizers do at load (SentencePiece: sp_tokenizer.h:154-172;
//     byte-level BPE: bpe.h:91-110, 576-586), and the whitespace-only flags
//     the stall narrowing uses (llama_chat.cpp:518-524);
//   * tms_filter: GrammarFilter (llama_chat.cpp:159-223) -- one decode's
//     grammar state, its no-progress counter, and the restriction as mask
//     words, narrowed to non-whitespace ids once the state has stalled for
//     four tokens;
//   * tms_mask_pipe: the next step's masks for a batch of filters, computed
//     on worker threads into pinned staging while the device runs the
//     current step, uploaded on the pipe's own stream (default priority),
//     and ordered before the sampler by an event.  Two slots: step t+1 is
//     produced and uploaded while step t's sampler may still read slot t.

#include <hip/hip_runtime_api.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <condition_variable>
#include <map>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "../../include/tmsample_hip.h"

namespace {

void put_err(char* err, size_t cap, const std::string& msg) {
    if (!err || cap == 0) return;
    const size_t n = std::min(msg.size(), cap - 1);
    memcpy(err, msg.data(), n);
    err[n] = '\0';
}

// GPT-2's byte <-> codepoint table (bytes_to_unicode in OpenAI's encoder.py):
// the printable bytes 33..126, 161..172 and 174..255 stand for themselves,
// the other 68 bytes for codepoints 256, 257, ... in ascending byte order.
struct ByteLevel {
    int16_t byte_of[324];   // codepoint -> byte, -1 when the codepoint is not in the table
    ByteLevel() {
        std::fill(byte_of, byte_of + 324, (int16_t)-1);
        int extra = 0;
        for (int b = 0; b < 256; ++b) {
            const bool self = (b >= 33 && b <= 126) || (b >= 161 && b <= 172) || b >= 174;
            byte_of[self ? b : 256 + extra++] = (int16_t)b;
        }
    }
};
const ByteLevel kByteLevel;

bool is_ws_only(const std::string& s) {
    if (s.empty()) return false;
    for (unsigned char c : s)
        if (c != ' ' && c != '\t' && c != '\n' && c != '\r') return false;
    return true;
}

int hexval(char c) {
    if (c >= '0' && c <= '9') return c - '0';
    if (c >= 'a' && c <= 'f') return c - 'a' + 10;
    if (c >= 'A' && c <= 'F') return c - 'A' + 10;
    return -1;
}

}  // namespace

struct tms_token_table {
    std::vector<std::string> bytes;
    std::vector<unsigned char> ws;
    void finish() {
        ws.resize(bytes.size());
        for (size_t i = 0; i < bytes.size(); ++i) ws[i] = is_ws_only(bytes[i]) ? 1 : 0;
    }
};

// SentencePiece pieces: CONTROL (3) contributes nothing, BYTE (6) "<0xNN>"
// the byte NN (any other length: nothing), every other type the piece with
// each U+2581 (E2 96 81) read as a space.
extern "C" tms_token_table* tms_token_table_spm(const char* const* pieces, const size_t* lens,
                                                const uint8_t* types, int n, char* err, size_t err_cap) {
    if (n < 0 || (n > 0 && (!pieces || !lens || !types))) {
        put_err(err, err_cap, "token table: null argument");
        return nullptr;
    }
    auto* t = new tms_token_table;
    t->bytes.resize((size_t)n);
    static const char kMark[3] = {'\xE2', '\x96', '\x81'};
    for (int id = 0; id < n; ++id) {
        const char* p = pieces[id];
        const size_t L = p ? lens[id] : 0;
        std::string& out = t->bytes[(size_t)id];
        if (types[id] == 3) continue;
        if (types[id] == 6) {
            if (L != 6) continue;
            const int hi = hexval(p[3]), lo = hexval(p[4]);
            if (hi < 0 || lo < 0) {
                put_err(err, err_cap, "token table: id " + std::to_string(id) + ": bad byte piece");
                delete t;
                return nullptr;
            }
            out.assign(1, (char)(hi * 16 + lo));
            continue;
        }
        out.reserve(L);
        for (size_t k = 0; k < L;) {
            if (k + 3 <= L && memcmp(p + k, kMark, 3) == 0) {
                out.push_back(' ');
                k += 3;
            } else {
                out.push_back(p[k++]);
            }
        }
    }
    t->finish();
    put_err(err, err_cap, "");
    return t;
}

// Byte-level BPE pieces: each UTF-8 codepoint (one to three bytes) of the
// piece back to its byte; a NULL piece is an id the vocabulary does not
// hold (no bytes).  A codepoint outside the table, or a truncated or
// four-byte sequence, is an error.
extern "C" tms_token_table* tms_token_table_bpe(const char* const* pieces, const size_t* lens, int n,
                                                char* err, size_t err_cap) {
    if (n < 0 || (n > 0 && (!pieces || !lens))) {
        put_err(err, err_cap, "token table: null argument");
        return nullptr;
    }
    auto* t = new tms_token_table;
    t->bytes.resize((size_t)n);
    for (int id = 0; id < n; ++id) {
        const unsigned char* p = (const unsigned char*)pieces[id];
        if (!p) continue;
        const size_t L = lens[id];
        std::string& out = t->bytes[(size_t)id];
        for (size_t k = 0; k < L;) {
            const unsigned c = p[k];
            const size_t w = c < 0x80 ? 1 : (c & 0xE0) == 0xC0 ? 2 : (c & 0xF0) == 0xE0 ? 3 : 0;
            int cp = -1;
            if (w != 0 && k + w <= L) {
                cp = w == 1 ? (int)c : w == 2 ? (int)(c & 0x1F) : (int)(c & 0x0F);
                for (size_t j = 1; j < w; ++j) cp = (cp << 6) | (p[k + j] & 0x3F);
            }
            if (cp < 0 || cp >= 324 || kByteLevel.byte_of[cp] < 0) {
                put_err(err, err_cap, "token table: id " + std::to_string(id) + ": piece byte " +
                                          std::to_string(k) + " is not a byte-level codepoint");
                delete t;
                return nullptr;
            }
            out.push_back((char)kByteLevel.byte_of[cp]);
            k += w;
        }
    }
    t->finish();
    put_err(err, err_cap, "");
    return t;
}

extern "C" void tms_token_table_free(tms_token_table* t) { delete t; }

extern "C" int tms_token_table_size(const tms_token_table* t) { return t ? (int)t->bytes.size() : -1; }

extern "C" int tms_token_table_bytes(const tms_token_table* t, int id, const char** bytes, size_t* len) {
    if (!t || !bytes || !len) return TMS_ERR_INVALID_ARG;
    static const char kEmpty[1] = {0};
    if (id < 0 || (size_t)id >= t->bytes.size()) {
        *bytes = kEmpty;
        *len = 0;
        return TMS_OK;
    }
    *bytes = t->bytes[(size_t)id].data();
    *len = t->bytes[(size_t)id].size();
    return TMS_OK;
}

extern "C" int tms_token_table_ws_only(const tms_token_table* t, int id) {
    return t && id >= 0 && (size_t)id < t->ws.size() ? t->ws[(size_t)id] : 0;
}

extern "C" tms_vocab* tms_vocab_from_table(tms_grammar* g, const tms_token_table* t, int eos,
                                           const unsigned char* skip) {
    if (!g || !t) return nullptr;
    const size_t n = t->bytes.size();
    std::vector<const char*> ptr(n);
    std::vector<size_t> len(n);
    for (size_t i = 0; i < n; ++i) {
        ptr[i] = t->bytes[i].data();
        len[i] = t->bytes[i].size();
    }
    return tms_vocab_create(g, ptr.data(), len.data(), (int)n, eos, skip);
}

// ------------------------------------------------------------------ filter

struct tms_filter {
    tms_grammar* g;
    tms_vocab* v;
    std::vector<unsigned char> ws;   // whitespace-only ids (empty: none known)
    tms_gstate* st;
    int stall;
};

extern "C" tms_filter* tms_filter_create(tms_grammar* g, tms_vocab* v, const tms_token_table* t) {
    if (!g || !v) return nullptr;
    tms_gstate* s = tms_grammar_start(g);
    if (!s) return nullptr;
    auto* f = new tms_filter{g, v, {}, s, 0};
    if (t) f->ws = t->ws;
    return f;
}

extern "C" void tms_filter_free(tms_filter* f) {
    if (!f) return;
    tms_gstate_free(f->st);
    delete f;
}

extern "C" int tms_filter_reset(tms_filter* f) {
    if (!f) return TMS_ERR_INVALID_ARG;
    tms_gstate* s = tms_grammar_start(f->g);
    if (!s) return TMS_ERR_INVALID_ARG;
    tms_gstate_free(f->st);
    f->st = s;
    f->stall = 0;
    return TMS_OK;
}

// GrammarFilter::restrict (llama_chat.cpp:184-209) as mask words: the
// allowed ids; with stall >= 4 the whitespace-only ids leave the set unless
// nothing else is in it.  No allowed id: every word all ones (the
// restriction fails open) and 0 returned.
extern "C" int tms_filter_mask(tms_filter* f, uint32_t* words, int n_words) {
    if (!f || !words || n_words < 0) return -1;
    int n = tms_vocab_mask(f->v, f->st, words, n_words);
    if (n < 0) return n;
    if (n == 0) {
        for (int w = 0; w < n_words; ++w) words[w] = ~0u;
        return 0;
    }
    if (f->stall >= 4 && !f->ws.empty()) {
        int kept = 0;
        for (int w = 0; w < n_words; ++w) {
            uint32_t bits = words[w];
            for (uint32_t m = bits; m; m &= m - 1) {
                const size_t id = (size_t)w * 32 + (size_t)__builtin_ctz(m);
                if (id < f->ws.size() && f->ws[id]) bits &= ~(1u << (id & 31));
            }
            kept += __builtin_popcount(bits);
        }
        if (kept > 0) {
            for (int w = 0; w < n_words; ++w) {
                uint32_t bits = words[w];
                for (uint32_t m = bits; m; m &= m - 1) {
                    const size_t id = (size_t)w * 32 + (size_t)__builtin_ctz(m);
                    if (id < f->ws.size() && f->ws[id]) bits &= ~(1u << (id & 31));
                }
                words[w] = bits;
            }
            n = kept;
        }
    }
    return n;
}

// GrammarFilter::consume (llama_chat.cpp:216-221): advance by the id's bytes;
// the stall count grows while the state stays the same.
extern "C" int tms_filter_consume(tms_filter* f, int id) {
    if (!f) return 0;
    tms_gstate* before = tms_gstate_copy(f->st);
    const int ok = tms_vocab_consume(f->v, f->g, f->st, id);
    f->stall = tms_gstate_equal(before, f->st) ? f->stall + 1 : 0;
    tms_gstate_free(before);
    return ok;
}

// GrammarFilter::complete (llama_chat.cpp:212-215).
extern "C" int tms_filter_complete(tms_filter* f, int eos) {
    if (!f || !tms_grammar_can_end(f->g, f->st)) return 0;
    int32_t one = -1;
    const int n = tms_vocab_allowed(f->v, f->st, &one, 1);
    return n == 1 && one == eos ? 1 : 0;
}

extern "C" int tms_filter_done(const tms_filter* f) { return f && tms_grammar_can_end(f->g, f->st) ? 1 : 0; }

extern "C" int tms_filter_stall(const tms_filter* f) { return f ? f->stall : -1; }

// ------------------------------------------------------------------ mask pipe

struct tms_mask_pipe {
    int device = 0, batch = 0, n_words = 0;
    size_t bytes = 0;
    uint32_t* host[2] = {nullptr, nullptr};   // pinned staging
    uint32_t* dev[2] = {nullptr, nullptr};
    hipStream_t copy = nullptr;
    hipEvent_t copied[2] = {nullptr, nullptr};    // upload of slot s done
    hipEvent_t consumed[2] = {nullptr, nullptr};  // the sampler that read slot s is done
    bool copied_valid[2] = {false, false};
    bool consumed_valid[2] = {false, false};
    std::vector<tms_filter*> rows;
    std::vector<int32_t> counts;     // allowed ids per row of the slot being produced
    std::vector<int32_t> tokens;

    // workers: each takes whole grammars (a grammar is not safe to share
    // between threads), in groups fixed at submit
    std::vector<std::thread> threads;
    std::vector<std::vector<int>> groups;   // rows per worker for the current step
    std::mutex mu;
    std::condition_variable cv_work, cv_done;
    uint64_t generation = 0;
    int pending = 0;
    bool stop = false;
    int slot = 0;          // slot being produced / last produced
    int acquired = -1;     // slot handed out by acquire and not yet released
    bool in_flight = false;
    int rc = TMS_OK;

    void work(int w) {
        uint64_t seen = 0;
        for (;;) {
            std::vector<int> mine;
            int s;
            {
                std::unique_lock<std::mutex> lk(mu);
                cv_work.wait(lk, [&] { return stop || generation != seen; });
                if (stop) return;
                seen = generation;
                if (w < (int)groups.size()) mine = groups[(size_t)w];
                s = slot;
            }
            for (int b : mine) produce(b, s);
            bool last;
            {
                std::lock_guard<std::mutex> lk(mu);
                last = --pending == 0;
            }
            if (last) finish(s);
        }
    }

    void produce(int b, int s) {
        uint32_t* words = host[s] + (size_t)b * (size_t)n_words;
        tms_filter* f = rows[(size_t)b];
        if (!f) {
            for (int w = 0; w < n_words; ++w) words[w] = ~0u;
            counts[(size_t)b] = -1;
            return;
        }
        if (tokens[(size_t)b] >= 0) (void)tms_filter_consume(f, tokens[(size_t)b]);
        counts[(size_t)b] = tms_filter_mask(f, words, n_words);
    }

    // The last worker of a step: the upload, once the sampler that read this
    // slot two steps ago is done with it.
    void finish(int s) {
        int r = TMS_OK;
        bool wait_consumed;
        {
            std::lock_guard<std::mutex> lk(mu);
            wait_consumed = consumed_valid[s];
        }
        if (hipSetDevice(device) != hipSuccess) r = TMS_ERR_HIP;
        if (r == TMS_OK && wait_consumed && hipStreamWaitEvent(copy, consumed[s], 0) != hipSuccess)
            r = TMS_ERR_HIP;
        if (r == TMS_OK && hipMemcpyAsync(dev[s], host[s], bytes, hipMemcpyHostToDevice, copy) != hipSuccess)
            r = TMS_ERR_HIP;
        if (r == TMS_OK && hipEventRecord(copied[s], copy) != hipSuccess) r = TMS_ERR_HIP;
        std::lock_guard<std::mutex> lk(mu);
        copied_valid[s] = r == TMS_OK;
        rc = r;
        in_flight = false;
        cv_done.notify_all();
    }
};

extern "C" void tms_mask_pipe_free(tms_mask_pipe* p);

extern "C" tms_mask_pipe* tms_mask_pipe_create(int device, int batch, int n_words, int threads) {
    if (batch <= 0 || n_words <= 0 || threads <= 0 || threads > 64) return nullptr;
    int prev = 0;
    if (hipGetDevice(&prev) != hipSuccess || hipSetDevice(device) != hipSuccess) return nullptr;
    auto* p = new tms_mask_pipe;
    p->device = device;
    p->batch = batch;
    p->n_words = n_words;
    p->bytes = (size_t)batch * (size_t)n_words * sizeof(uint32_t);
    p->rows.assign((size_t)batch, nullptr);
    p->counts.assign((size_t)batch, 0);
    p->tokens.assign((size_t)batch, -1);
    bool ok = true;
    for (int s = 0; s < 2 && ok; ++s) {
        ok = hipHostMalloc((void**)&p->host[s], p->bytes, hipHostMallocDefault) == hipSuccess &&
             hipMalloc((void**)&p->dev[s], p->bytes) == hipSuccess &&
             hipEventCreateWithFlags(&p->copied[s], hipEventDisableTiming) == hipSuccess &&
             hipEventCreateWithFlags(&p->consumed[s], hipEventDisableTiming) == hipSuccess;
    }
    ok = ok && hipStreamCreateWithFlags(&p->copy, hipStreamNonBlocking) == hipSuccess;
    (void)hipSetDevice(prev);
    if (!ok) {
        tms_mask_pipe_free(p);
        return nullptr;
    }
    for (int w = 0; w < threads; ++w) p->threads.emplace_back([p, w] { p->work(w); });
    return p;
}

extern "C" void tms_mask_pipe_free(tms_mask_pipe* p) {
    if (!p) return;
    {
        std::unique_lock<std::mutex> lk(p->mu);
        p->cv_done.wait(lk, [&] { return !p->in_flight; });
        p->stop = true;
        p->cv_work.notify_all();
    }
    for (auto& t : p->threads) t.join();
    int prev = 0;
    (void)hipGetDevice(&prev);
    (void)hipSetDevice(p->device);
    if (p->copy) (void)hipStreamSynchronize(p->copy);
    for (int s = 0; s < 2; ++s) {
        if (p->host[s]) (void)hipHostFree(p->host[s]);
        if (p->dev[s]) (void)hipFree(p->dev[s]);
        if (p->copied[s]) (void)hipEventDestroy(p->copied[s]);
        if (p->consumed[s]) (void)hipEventDestroy(p->consumed[s]);
    }
    if (p->copy) (void)hipStreamDestroy(p->copy);
    (void)hipSetDevice(prev);
    delete p;
}

extern "C" int tms_mask_pipe_set_row(tms_mask_pipe* p, int row, tms_filter* f) {
    if (!p || row < 0 || row >= p->batch) return TMS_ERR_INVALID_ARG;
    std::lock_guard<std::mutex> lk(p->mu);
    if (p->in_flight) return TMS_ERR_INVALID_ARG;
    p->rows[(size_t)row] = f;
    return TMS_OK;
}

// Start the next step's masks: each row's filter consumes tokens[row] (if
// >= 0; tokens may be NULL for none), then writes its mask.  Returns at once.
extern "C" int tms_mask_pipe_submit(tms_mask_pipe* p, const int32_t* tokens) {
    if (!p) return TMS_ERR_INVALID_ARG;
    std::unique_lock<std::mutex> lk(p->mu);
    if (p->in_flight) return TMS_ERR_INVALID_ARG;   // acquire the previous step first
    const int s = p->slot ^ 1;
    if (p->acquired == s) return TMS_ERR_INVALID_ARG;   // release the step that slot holds first
    lk.unlock();
    // the staging slot is free once its previous upload has finished
    if (p->copied_valid[s] && hipEventSynchronize(p->copied[s]) != hipSuccess) return TMS_ERR_HIP;
    lk.lock();
    for (int b = 0; b < p->batch; ++b) p->tokens[(size_t)b] = tokens ? tokens[b] : -1;
    // group the rows by grammar; spread the groups over the workers
    std::map<const void*, std::vector<int>> by;
    for (int b = 0; b < p->batch; ++b) {
        tms_filter* f = p->rows[(size_t)b];
        by[f ? (const void*)f->g : nullptr].push_back(b);
    }
    p->groups.assign(p->threads.size(), {});
    size_t w = 0;
    for (auto& kv : by) {
        auto& dst = p->groups[w];
        dst.insert(dst.end(), kv.second.begin(), kv.second.end());
        w = (w + 1) % p->threads.size();
    }
    p->slot = s;
    p->pending = (int)p->threads.size();
    p->in_flight = true;
    p->rc = TMS_OK;
    ++p->generation;
    p->cv_work.notify_all();
    return TMS_OK;
}

// Wait for the submitted step's masks, make `stream` wait for their upload,
// and return the device words [batch][n_words] (and, if `allowed` is not
// NULL, each row's allowed-id count: 0 = the row failed open, -1 = no
// filter).
extern "C" int tms_mask_pipe_acquire(tms_mask_pipe* p, hipStream_t stream, const uint32_t** words,
                                     int32_t* allowed) {
    if (!p || !words) return TMS_ERR_INVALID_ARG;
    std::unique_lock<std::mutex> lk(p->mu);
    p->cv_done.wait(lk, [&] { return !p->in_flight; });
    if (p->rc != TMS_OK || !p->copied_valid[p->slot]) return p->rc != TMS_OK ? p->rc : TMS_ERR_INVALID_ARG;
    const int s = p->slot;
    if (p->acquired >= 0 && p->acquired != s) return TMS_ERR_INVALID_ARG;   // the other slot is still held
    if (hipStreamWaitEvent(stream, p->copied[s], 0) != hipSuccess) return TMS_ERR_HIP;
    p->acquired = s;
    *words = p->dev[s];
    if (allowed) memcpy(allowed, p->counts.data(), sizeof(int32_t) * (size_t)p->batch);
    return TMS_OK;
}

// After enqueueing the launches that read the acquired words on `stream`:
// the slot acquire handed out is refilled only after `stream` has passed
// this point.  The next step may already be submitted (it fills the other
// slot); a release with no acquire outstanding is an error.
extern "C" int tms_mask_pipe_release(tms_mask_pipe* p, hipStream_t stream) {
    if (!p) return TMS_ERR_INVALID_ARG;
    std::lock_guard<std::mutex> lk(p->mu);
    const int s = p->acquired;
    if (s < 0) return TMS_ERR_INVALID_ARG;
    if (hipEventRecord(p->consumed[s], stream) != hipSuccess) return TMS_ERR_HIP;
    p->consumed_valid[s] = true;
    p->acquired = -1;
    return TMS_OK;
}

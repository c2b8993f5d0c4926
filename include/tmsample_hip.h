/*
 * tmsample_hip.h -- C ABI of the MI355X (gfx950) token sampler.
 *
 * This library replaces TensorMark's host sampler and its GPU token kernels
 * with batched HIP kernels.  Every entry point is plain C: device pointers,
 * sizes, a hipStream_t, and an int status.  No exceptions and no C++ types
 * cross this boundary.
 *
 * Interfaces replaced (paths are relative to the TensorMark tree):
 *   tmsample::Opts                  tensormark/tmsample.h:31-35
 *   tmsample::apply_repeat_penalty  tensormark/tmsample.h:52-63
 *   tmsample::sample                tensormark/tmsample.h:173-200
 *   sample_token (mask -> penalty -> sample composition)
 *                                   tensormark/llama_chat.cpp:146-153, 184-209, 787-791
 *   tm_metal_tok_argmax / tm_metal_tok_sample (GPU token kernels)
 *                                   tensormark/llama.h:58-63, tensormark/metal_shim.mm:29-35
 *   spec_generate_greedy's verify rule (greedy limit of tms_spec_verify)
 *                                   tensormark/llama.h:5127-5131
 *
 * Per-row semantics of tms_sample_batch, in order:
 *   1. grammar mask: ids whose bit is clear become -inf
 *      (bit (id & 31) of word id >> 5, LSB first);
 *   2. repetition penalty over the last repeat_last_n ids of the row's
 *      history, compounding once per occurrence (v > 0 ? v / p : v * p);
 *   3. frequency/presence penalty: v -= (float)count * freq + presence;
 *   3a. (with `history`) no-repeat n-gram ban, tensormark/tmsample.h:81-114:
 *      every id that followed an earlier occurrence of the row's last
 *      ngram - 1 ids becomes -inf, unless that leaves no value above -inf
 *      (then the banned ids keep their step-3 values);
 *   3b. (with `history`) DRY, tensormark/tmsample.h:148-170: for each
 *      earlier position of the last penalty_last_n ids whose run agrees with
 *      the tail for L >= allowed_length ids (never across a breaker id), the
 *      id that followed it loses multiplier * base^(L - allowed_length), in
 *      position order (base^k by binary powering in double and one rounding
 *      to float; glibc's powf, which the reference calls, differs from it by
 *      1 ulp for about 0.1% of (base, k) pairs);
 *   4. greedy: the first maximum (lowest id) of the penalised row;
 *   5. otherwise lg = v / temperature (fp32 division), top-k by
 *      (lg descending, id ascending), pr = exp((double)lg - (double)lg_max)
 *      summed in order, top-p cut (cum >= top_p), min-p cut
 *      (pr >= min_p), then an inverse-CDF draw over the survivors with
 *      libstdc++ discrete_distribution arithmetic.  The uniform comes from
 *      two 32-bit words (w0, w1): u = (w0 + w1 * 2^32) / 2^64 in double,
 *      clamped below 1.  The words are Philox4x32-10 outputs 0 and 1 for
 *      key = (seed lo, seed hi) and counter = (offset lo, offset hi, 0, 0),
 *      or caller-supplied (`draws`).
 */
#ifndef TMSAMPLE_HIP_H
#define TMSAMPLE_HIP_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TMS_ABI_VERSION 4

/* Return codes of the entry points. */
enum {
    TMS_OK = 0,
    TMS_ERR_INVALID_ARG = -1,   /* null pointer, bad size, unknown dtype */
    TMS_ERR_CAPACITY = -2,      /* batch or vocab above the context's maxima */
    TMS_ERR_HIP = -3,           /* a HIP runtime call failed */
    TMS_ERR_NO_DEVICE = -4
};

/* Per-row status written to out_status. */
enum {
    TMS_ROW_OK = 0,
    TMS_ROW_BAD_PARAMS = 1,   /* temperature <= 0 or non-finite on a sampled row */
    TMS_ROW_ALL_MASKED = 2,   /* every id is -inf after mask and penalties */
    TMS_ROW_NONFINITE = 3,    /* NaN or +inf after masking, or lg overflowed */
    TMS_ROW_UNSUPPORTED = 4,  /* a row that breaks the TMS_ROWS_TOPK promise (top_k = 0
                                 or > 128, not greedy) in a call the top-k kernel
                                 takes; or, with `history`, a row whose history touches
                                 more than TMS_HISTORY_MAX_IDS distinct ids */
    TMS_ROW_INTERNAL = 5      /* a chunk list never arrived (bounded wait expired) */
};

/* tms_sample_args.row_kinds: what the caller knows of its rows. */
enum {
    TMS_ROWS_ANY = 0,    /* no promise: the general kernel */
    TMS_ROWS_TOPK = 1,   /* every row greedy, or top-k with 1 <= top_k <= 128 */
    TMS_ROWS_SPARSE_MASK = 2   /* the masks allow few ids a row (at most
                                  TMS_SPARSE_MAX_IDS expected): only the allowed
                                  logits are read.  Any row kind; a row with more
                                  allowed ids is still sampled exactly, over the
                                  whole row and more slowly.  Taken when `mask` is
                                  given, `history` is not, and vocab <=
                                  TMS_SPARSE_MAX_VOCAB; otherwise the general
                                  kernel */
};

/* Allowed ids a row the sparse-mask kernel holds, and its largest vocab. */
#define TMS_SPARSE_MAX_IDS 2048
#define TMS_SPARSE_MAX_VOCAB 262144

enum {
    TMS_DTYPE_F32 = 0,
    TMS_DTYPE_F16 = 1,
    TMS_DTYPE_BF16 = 2
};

/*
 * Per-row sampler parameters.  The first three fields are tmsample::Opts
 * (tensormark/tmsample.h:31-35) field for field; repeat_penalty and
 * repeat_last_n are the `penalty` and `window` arguments of
 * apply_repeat_penalty (tensormark/tmsample.h:52-53); `greedy` is the
 * `greedy` argument of tmsample::sample (tensormark/tmsample.h:173-174).
 * min_p, frequency_penalty, presence_penalty, seed and offset have no
 * counterpart in the reference.
 */
typedef struct tms_row_params {
    float temperature;        /* divides the logits; must be > 0 unless greedy */
    int32_t top_k;            /* <= 0 or > vocab means the whole vocabulary */
    float top_p;              /* smallest prefix with cumulative mass >= top_p */
    float min_p;              /* keep pr >= min_p * pr_max; <= 0 disables */
    float repeat_penalty;     /* <= 1 disables, as in the reference */
    int32_t repeat_last_n;    /* window over the row's history */
    float frequency_penalty;  /* 0 disables */
    float presence_penalty;   /* 0 disables */
    int32_t greedy;           /* non-zero: argmax, no temperature, no draw */
    uint32_t flags;           /* reserved, must be 0 */
    uint64_t seed;            /* Philox4x32-10 key */
    uint64_t offset;          /* Philox4x32-10 counter words 0 and 1 */
} tms_row_params;

/* Most distinct ids the history steps (2, 3, 3a, 3b) of one row may touch. */
#define TMS_HISTORY_MAX_IDS 4096
/* Most window positions DRY (step 3b) reads on the device:
 * min(n_recent, dry_penalty_last_n) above this reports TMS_ROW_UNSUPPORTED. */
#define TMS_DRY_MAX_WINDOW 8192

/*
 * Per-row n-gram ban and DRY settings (tms_sample_args.history).
 * no_repeat_ngram is ChatOpts::no_repeat_ngram, the `ngram` argument of
 * apply_no_repeat_ngram (tensormark/tmsample.h:81-82); the dry_* fields are
 * tmsample::DryOpts (tensormark/tmsample.h:141-146) field for field.  The
 * sequence-breaker table (apply_dry's `is_breaker`) is shared by the batch:
 * tms_sample_args.dry_breaker.
 */
typedef struct tms_history_params {
    int32_t no_repeat_ngram;      /* < 2 disables */
    float dry_multiplier;         /* <= 0 disables */
    float dry_base;               /* DryOpts default 1.75 */
    int32_t dry_allowed_length;   /* < 1 disables; DryOpts default 2 */
    int32_t dry_penalty_last_n;   /* DryOpts default 256 */
    int32_t reserved;             /* must be 0 */
} tms_history_params;

/* Opaque context: owns the device workspace for one device. */
typedef struct tms_context tms_context;

typedef struct tms_sample_args {
    const void* logits;       /* device, [batch][row_stride] of dtype */
    int32_t dtype;            /* TMS_DTYPE_* */
    int32_t batch;
    int32_t vocab;
    int32_t topk_cap;         /* columns of out_topk_ids / out_topk_probs */
    int64_t row_stride;       /* elements between rows, >= vocab */
    const tms_row_params* params;   /* device, [batch] */
    const int32_t* recent;    /* device, [batch][recent_stride] token history, nullable */
    const int32_t* n_recent;  /* device, [batch] valid history length, nullable =
                                 every row holds recent_stride ids */
    int64_t recent_stride;
    const uint32_t* mask;     /* device, [batch][mask_stride] allowed bits, nullable */
    int64_t mask_stride;      /* words per row, >= ceil(vocab / 32) */
    const uint32_t* draws;    /* device, [batch][2] words (w0, w1) used instead
                                 of Philox, nullable */
    int32_t* out_tokens;      /* device, [batch]; -1 on a row error */
    int32_t* out_status;      /* device, [batch], TMS_ROW_* */
    int32_t* out_keep;        /* device, [batch], nullable: survivors drawn from
                                 (0 for greedy rows and errors) */
    int32_t* out_topk_ids;    /* device, [batch][topk_cap], nullable: sorted
                                 top-k ids, -1 padded */
    float* out_topk_probs;    /* device, [batch][topk_cap], nullable:
                                 pr / z of the same entries */
    uint32_t row_kinds;       /* TMS_ROWS_SPARSE_MASK: see the enum.
                                 TMS_ROWS_ANY, or TMS_ROWS_TOPK: the caller promises
                                 every row is greedy or has 1 <= top_k <= 128, and
                                 the library may take its top-k kernel (it does when
                                 batch x chunks <= 1024 workgroups).  Every other
                                 call takes the general kernel, whose row mergers
                                 sample whole any row the candidate lists cannot
                                 finish (top-p rows with more than 1024 entries
                                 within 40 of the maximum, draws past those
                                 entries, rows that break the promise) in the same
                                 launch.  In the top-k kernel a row that breaks the
                                 promise gets TMS_ROW_UNSUPPORTED, never a wrong
                                 sample */
    uint32_t reserved;        /* must be 0 */
    const tms_history_params* history;   /* device, [batch], nullable: steps 3a and 3b
                                            (then every row's history steps 2-3b run
                                            in a pre-pass and the general kernel
                                            samples, whatever row_kinds says) */
    const uint8_t* dry_breaker;          /* device, [vocab], nullable: non-zero marks a
                                            DRY sequence breaker; ids outside
                                            [0, vocab) are not breakers */
    const float* dry_scale;              /* device, [batch][dry_scale_stride], nullable:
                                            entry k of row b is the DRY scale base^k as
                                            the reference's std::pow(base, (float)k)
                                            gives it (tmsample.h:168), for the row's
                                            dry_base (tms_dry_scale_table fills one);
                                            a row whose DRY window needs k >=
                                            dry_scale_stride reports
                                            TMS_ROW_UNSUPPORTED.  Null: the library's
                                            own correctly rounded base^k, which differs
                                            from glibc's powf by one ulp for about 0.1%
                                            of (base, k) */
    int64_t dry_scale_stride;            /* floats per row of dry_scale */
} tms_sample_args;

typedef struct tms_spec_args {
    const void* target_logits;    /* device, [batch][k + 1][vocab] of dtype */
    const void* draft_logits;     /* device, [batch][k][vocab] of dtype */
    int32_t dtype;
    int32_t batch;
    int32_t k;                    /* draft tokens per sequence, 1..16 */
    int32_t vocab;
    const int32_t* draft_tokens;  /* device, [batch][k] */
    const tms_row_params* params; /* device, [batch]: temperature, seed, offset */
    const uint32_t* draws;        /* device, [batch][k + 1][2], nullable: words for
                                     the k accept tests and the final draw; when
                                     null, pair i is Philox4x32-10 outputs 0 and 1
                                     for key = seed and counter = (offset lo,
                                     offset hi, i, 0) */
    int32_t* out_accepted;        /* device, [batch]: accepted draft count */
    int32_t* out_token;           /* device, [batch]: residual or bonus token */
    int32_t* out_status;          /* device, [batch], TMS_ROW_* */
} tms_spec_args;

/* Library version (TMS_ABI_VERSION). */
int tms_abi_version(void);

/* Static text for a TMS_* return code or TMS_ROW_* status. */
const char* tms_status_string(int code);

/*
 * Create a context on `device` for batches up to max_batch rows of up to
 * max_vocab ids.  Allocates the workspace (per-row counters and candidate
 * lists) once; the sampling calls allocate nothing.  A context serves one
 * stream at a time: concurrent calls on one context race on its workspace.
 * Replaces the library-owned state the reference keeps in its Metal token
 * slots (tensormark/metal.h:3191-3228).
 */
int tms_create(int device, int max_batch, int max_vocab, tms_context** out);
int tms_destroy(tms_context* ctx);

/* Device bytes the context's workspace holds. */
size_t tms_workspace_bytes(const tms_context* ctx);

/*
 * Zero the words of the workspace that the calls' cross-workgroup protocols
 * expect at zero between calls (arrival counters and tickets, list and part
 * words, the whole-row region locks), stream-ordered.  The calls leave them at zero
 * themselves; a row that reports TMS_ROW_INTERNAL (a bounded wait ran out)
 * may leave late words behind, so a caller that sees that status calls this
 * before the next call on the context.  ctx == NULL resets the current
 * device's tms_sample_batch_noalloc scratch.  Uses hipMemsetAsync: not for
 * graph capture.  No counterpart in the reference (its sampler is host
 * code).
 */
int tms_workspace_reset(tms_context* ctx, hipStream_t stream);

/*
 * Batched mask -> penalties -> temperature -> top-k -> softmax -> top-p /
 * min-p -> draw, one launch, stream-ordered, no host synchronisation.
 * Replaces sample_token (tensormark/llama_chat.cpp:146-153) with the grammar
 * restriction of tensormark/llama_chat.cpp:184-209, i.e. the composition of
 * apply_repeat_penalty (tensormark/tmsample.h:52-63) and tmsample::sample
 * (tensormark/tmsample.h:173-200); greedy rows replace tm_metal_tok_argmax
 * (tensormark/llama.h:58-59).
 */
int tms_sample_batch(tms_context* ctx, const tms_sample_args* args, hipStream_t stream);

/*
 * tms_sample_batch without a context and without any allocation, for
 * callers that cannot call hipMalloc (code under HIP graph capture, tight
 * serving loops, harnesses that forbid allocation).  No counterpart in the
 * reference.  Same arguments, semantics and results as tms_sample_batch;
 * the workspace is a fixed 21.0 MB device array inside the library (one
 * copy per device, held until the process ends), so batch <= 64 rows and
 * vocab <= 262144 ids, else TMS_ERR_CAPACITY.  Runs on the current device
 * (the stream's device must be current).  The first call on each device
 * looks the array's address up (hipGetSymbolAddress): make one call before
 * capturing a graph.  Every call on a device shares that device's array:
 * calls that overlap on one device (two streams, or two threads) race and
 * must be serialised by the caller.  Whole-row-pass rows of one call are
 * sampled one after another.
 */
int tms_sample_batch_noalloc(const tms_sample_args* args, hipStream_t stream);

/*
 * Speculative verify: for each sequence, accept draft i while
 * u_i < p_t(x_i) / p_d(x_i); at the first rejection draw from
 * normalize(max(p_t - p_d, 0)); if all k are accepted draw a bonus token
 * from the target row k.  Softmax weights are exp(lg - max) quantised to
 * multiples of 2^-44 and summed exactly in 64-bit integers.  The greedy
 * limit (one-hot p_t and p_d) is the argmax-match rule of
 * spec_generate_greedy (tensormark/llama.h:5127-5131).
 */
int tms_spec_verify(tms_context* ctx, const tms_spec_args* args, hipStream_t stream);

/*
 * The history transforms on a host row of V fp32 logits, in place, for
 * host-side callers (the device runs them itself with
 * tms_sample_args.history).  tms_host_dry computes base^k as the reference
 * does, std::pow(base, (float)k) of the host's C library.
 *   tms_host_repeat_penalty   tmsample::apply_repeat_penalty  (tensormark/tmsample.h:52-63)
 *   tms_host_no_repeat_ngram  tmsample::apply_no_repeat_ngram (tensormark/tmsample.h:81-114)
 *   tms_host_dry              tmsample::apply_dry             (tensormark/tmsample.h:148-170),
 *                             the DryOpts fields (tensormark/tmsample.h:141-146) passed
 *                             one by one; is_breaker is nullable, indexed by id.
 */
void tms_host_repeat_penalty(float* logits, int V, const int32_t* recent, int n_recent,
                             int window, float penalty);
void tms_host_no_repeat_ngram(float* logits, int V, const int32_t* recent, int n_recent,
                              int ngram);
void tms_host_dry(float* logits, int V, const int32_t* recent, int n_recent, float multiplier,
                  float base, int allowed_length, int penalty_last_n,
                  const unsigned char* is_breaker);
/*
 * out[k] = std::pow(base, (float)k) for k in [0, n): one row of
 * tms_sample_args.dry_scale, the scale apply_dry multiplies by
 * (tensormark/tmsample.h:168), from this host's C library as the
 * reference's own build computes it.  Returns TMS_ERR_INVALID_ARG for a
 * null out or n < 0.
 */
int tms_dry_scale_table(float base, int n, float* out);

/*
 * Host GBNF engine: the producer of the grammar bitmask.  Replaces
 * tmgbnf::Grammar and tmgbnf::TokenMask (tensormark/gbnf.h:345-851) with the
 * same language semantics; the allowed set comes out as the sampler's mask
 * words directly.  Host-only, single-threaded per grammar.
 *
 *   tms_grammar_parse     Grammar::parse (gbnf.h:347-385); NULL on a parse
 *                         error, with the message in err (gbnf: ...)
 *   tms_grammar_start     Grammar::start (gbnf.h:435-440)
 *   tms_grammar_advance   Grammar::advance, one byte (gbnf.h:455-480); 0 =
 *                         rejected (the state is then dead)
 *   tms_grammar_can_end   Grammar::can_end (gbnf.h:443-448)
 *   tms_grammar_accepts   Grammar::accepts (gbnf.h:484-489)
 *   tms_gstate_copy/free/equal   State value semantics (gbnf.h:409-416)
 *   tms_vocab_create      TokenMask(g, token_text, eos, skip) (gbnf.h:729-755);
 *                         text[i]/len[i] = bytes of token i; skip nullable
 *   tms_vocab_allowed     TokenMask::allowed (gbnf.h:759-769): ascending ids,
 *                         returns the count (ids may be NULL to size)
 *   tms_vocab_mask        the same set as bits: words[id >> 5] bit id & 31,
 *                         n_words words cleared first; returns ids written
 *   tms_vocab_consume     TokenMask::consume (gbnf.h:772-778)
 *   tms_vocab_clear_cache TokenMask::clear_cache (gbnf.h:850)
 */
typedef struct tms_grammar tms_grammar;
typedef struct tms_gstate tms_gstate;
typedef struct tms_vocab tms_vocab;

tms_grammar* tms_grammar_parse(const char* text, size_t len, char* err, size_t err_cap);
void tms_grammar_free(tms_grammar* g);
int tms_grammar_rule_count(const tms_grammar* g);
tms_gstate* tms_grammar_start(tms_grammar* g);
int tms_grammar_advance(tms_grammar* g, tms_gstate* s, unsigned char byte);
int tms_grammar_can_end(const tms_grammar* g, const tms_gstate* s);
int tms_grammar_accepts(tms_grammar* g, const char* text, size_t len);
tms_gstate* tms_gstate_copy(const tms_gstate* s);
void tms_gstate_free(tms_gstate* s);
int tms_gstate_equal(const tms_gstate* a, const tms_gstate* b);
tms_vocab* tms_vocab_create(tms_grammar* g, const char* const* text, const size_t* len,
                            int n_tokens, int eos, const unsigned char* skip);
void tms_vocab_free(tms_vocab* v);
int tms_vocab_node_count(const tms_vocab* v);
int tms_vocab_allowed(tms_vocab* v, const tms_gstate* s, int32_t* ids, int cap);
int tms_vocab_mask(tms_vocab* v, const tms_gstate* s, uint32_t* words, int n_words);
int tms_vocab_consume(tms_vocab* v, tms_grammar* g, tms_gstate* s, int id);
void tms_vocab_clear_cache(tms_vocab* v);

/*
 * Vocabulary byte tables: the bytes each id contributes to a running decode,
 * as the reference's tokenizers derive them at load (tensormark/tmtok.h:40-42
 * piece_bytes; llama_chat.cpp:510-524), and the whitespace-only flags of
 * the stall narrowing.
 *   tms_token_table_spm   SentencePiece pieces (sp_tokenizer.h:154-172):
 *                         type 3 (CONTROL) no bytes, type 6 (BYTE) "<0xNN>"
 *                         the byte NN, any other type the piece with U+2581
 *                         read as a space
 *   tms_token_table_bpe   byte-level BPE pieces (bpe.h:91-110, 576-586): each
 *                         codepoint back to its byte through GPT-2's
 *                         bytes_to_unicode table; a NULL piece is an id the
 *                         vocabulary lacks (no bytes).  NULL on an unmapped
 *                         codepoint, with the message in err
 *   tms_token_table_bytes piece_bytes(id): pointer and length (empty for an
 *                         id outside the table)
 *   tms_token_table_ws_only  non-empty and only ' ', '\t', '\n', '\r'
 *                         (llama_chat.cpp:519-524)
 *   tms_vocab_from_table  tms_vocab_create over the table's bytes
 */
typedef struct tms_token_table tms_token_table;
tms_token_table* tms_token_table_spm(const char* const* pieces, const size_t* lens,
                                     const uint8_t* types, int n, char* err, size_t err_cap);
tms_token_table* tms_token_table_bpe(const char* const* pieces, const size_t* lens, int n,
                                     char* err, size_t err_cap);
void tms_token_table_free(tms_token_table* t);
int tms_token_table_size(const tms_token_table* t);
int tms_token_table_bytes(const tms_token_table* t, int id, const char** bytes, size_t* len);
int tms_token_table_ws_only(const tms_token_table* t, int id);
tms_vocab* tms_vocab_from_table(tms_grammar* g, const tms_token_table* t, int eos,
                                const unsigned char* skip);

/*
 * One decode's grammar restriction: GrammarFilter (tensormark/llama_chat.cpp:
 * 159-223).  Host-only; a filter's grammar and vocab are used by one thread
 * at a time.
 *   tms_filter_create    state at the grammar's start, stall 0; the table
 *                        (nullable) gives the whitespace-only ids
 *   tms_filter_reset     reset (llama_chat.cpp:169-179) without the memo drop
 *                        (tms_vocab_clear_cache does that)
 *   tms_filter_mask      restrict (llama_chat.cpp:184-209) as mask words: the
 *                        allowed ids, minus the whitespace-only ones once the
 *                        state has not changed for 4 tokens (unless none
 *                        would be left); returns the ids set.  No allowed id:
 *                        every word all ones (fails open) and 0
 *   tms_filter_consume   consume (llama_chat.cpp:216-221); the stall count
 *                        grows while the state stays the same
 *   tms_filter_complete  complete (llama_chat.cpp:212-215)
 *   tms_filter_done      done (llama_chat.cpp:222)
 */
typedef struct tms_filter tms_filter;
tms_filter* tms_filter_create(tms_grammar* g, tms_vocab* v, const tms_token_table* t);
void tms_filter_free(tms_filter* f);
int tms_filter_reset(tms_filter* f);
int tms_filter_mask(tms_filter* f, uint32_t* words, int n_words);
int tms_filter_consume(tms_filter* f, int id);
int tms_filter_complete(tms_filter* f, int eos);
int tms_filter_done(const tms_filter* f);
int tms_filter_stall(const tms_filter* f);

/*
 * The mask producer overlapped with the device: the per-step restriction of
 * llama_chat.cpp:787-803 (restrict, sample, consume) for a batch of
 * filters, with the next step's masks computed on `threads` worker threads
 * into pinned staging while the device runs the current step, uploaded on
 * the pipe's own stream (default priority) and ordered before the sampler
 * by an event.  Two slots, so one step's upload never overwrites the words
 * the previous step's sampler may still read.  No counterpart in the
 * reference (its restriction runs inline on the host).
 *   tms_mask_pipe_set_row  the row's filter (NULL: unconstrained, all ones);
 *                          rows with one grammar go to one worker
 *   tms_mask_pipe_submit   each filter consumes tokens[row] (host, >= 0;
 *                          NULL or < 0: nothing) and writes its mask; returns
 *                          at once
 *   tms_mask_pipe_acquire  waits for the workers; makes `stream` wait for the
 *                          upload; *words = device [batch][n_words]; allowed
 *                          (nullable) = ids per row (0: failed open, -1: no
 *                          filter).  TMS_ERR_INVALID_ARG while an earlier
 *                          step's words are still acquired and not released
 *   tms_mask_pipe_release  after enqueueing the launches that read the acquired
 *                          words on `stream` (the next step may be submitted
 *                          already); TMS_ERR_INVALID_ARG with nothing acquired.
 *                          A submit whose slot still holds acquired, unreleased
 *                          words returns TMS_ERR_INVALID_ARG
 */
typedef struct tms_mask_pipe tms_mask_pipe;
tms_mask_pipe* tms_mask_pipe_create(int device, int batch, int n_words, int threads);
void tms_mask_pipe_free(tms_mask_pipe* p);
int tms_mask_pipe_set_row(tms_mask_pipe* p, int row, tms_filter* f);
int tms_mask_pipe_submit(tms_mask_pipe* p, const int32_t* tokens);
int tms_mask_pipe_acquire(tms_mask_pipe* p, hipStream_t stream, const uint32_t** words,
                          int32_t* allowed);
int tms_mask_pipe_release(tms_mask_pipe* p, hipStream_t stream);

/*
 * Chained device-resident decode (gpu_chain_begin / gpu_chain_poll,
 * tensormark/llama.h:6047-6130; the token-slot peek, tensormark/metal.h:
 * 3216-3228): n steps enqueued at once, each step's sampled ids gathered
 * into the next step's input on the device, the host polling the ids as
 * they land.
 *   tms_token_slot_create  `capacity` int32 entries of host memory the
 *                          device writes (pinned, mapped, coherent), all -1
 *   tms_token_slot_device  the entries' device address
 *   tms_token_slot_fill    host: every entry := value (no chain in flight)
 *   tms_token_slot_peek    host: entry i with an acquire load, no wait; -1
 *                          while pending, -2 for a row the sampler could not
 *                          sample (its status says why)
 *   tms_embed_gather       x[b][:] = table[tokens[b]][:] (rows x dim of
 *                          dtype; an id outside [0, rows) gives zeros), and
 *                          slot_out[b] = tokens[b] (nullable) by system-scope
 *                          release stores.  table NULL: publish only.  Row
 *                          bytes, table and x 16-byte aligned
 */
typedef struct tms_token_slot tms_token_slot;
tms_token_slot* tms_token_slot_create(int device, int capacity);
void tms_token_slot_free(tms_token_slot* s);
int32_t* tms_token_slot_device(tms_token_slot* s);
int tms_token_slot_capacity(const tms_token_slot* s);
int tms_token_slot_fill(tms_token_slot* s, int32_t value);
int32_t tms_token_slot_peek(const tms_token_slot* s, int i);
int tms_embed_gather(const void* table, int dtype, int64_t rows, int64_t dim, const int32_t* tokens,
                     int batch, void* x, int32_t* slot_out, hipStream_t stream);

/*
 * Test hooks.  Run the device Philox4x32-10 on n (counter[4], key[2])
 * tuples packed as 6 words each and write 4 words each; evaluate the device
 * double exp on n inputs (which = 0: the HIP math library, 1: the
 * library's own exp used by tms_spec_verify, 2: tms_spec_verify's weight
 * q44(exp(x)) for x <= 0 as a double, the integer count of 2^-44 units;
 * 3: the quotients in[2i] / in[2i + 1] by tms_spec_verify's division from
 * a reciprocal, into out[i] for i < n / 2).
 */
int tms_debug_philox(const uint32_t* in6, uint32_t* out4, int n, hipStream_t stream);
/* Checks of the device ordering the cross-workgroup protocols rely on
 * (synchronous; allocates; `trials` of each): counts[0] stale reads of a
 * line written by another XCD in the previous kernel, counts[1] words lost
 * when two XCDs write halves of one line in one kernel, counts[2] kernels
 * started before their predecessor on the stream finished, counts[3]
 * workgroups w of a 64-workgroup grid not on XCD w mod n, counts[4] the XCD
 * count n, counts[5] trials whose roles found no workgroup on their XCD,
 * counts[6] words lost when each of the two writers reads the line before
 * writing its half (counts has at least 7 entries). */
int tms_debug_ordering(int trials, int32_t* counts);
int tms_debug_exp(const double* in, double* out, int n, int which, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* TMSAMPLE_HIP_H */

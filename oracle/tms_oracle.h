/*
 * tms_oracle.h -- CPU restatement of TensorMark's sampling path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load this library, and only as the
 * checker.  The product library (libtmsample_hip.so) never links or calls it.
 *
 * Each function cites the reference lines it restates.  Pins (what checks
 * each function against something other than itself) are listed in the
 * header of tms_oracle.c.
 */
#ifndef TMS_ORACLE_H
#define TMS_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Same layout as tms_row_params in include/tmsample_hip.h. */
typedef struct tmo_row_params {
    float temperature;
    int32_t top_k;
    float top_p;
    float min_p;
    float repeat_penalty;
    int32_t repeat_last_n;
    float frequency_penalty;
    float presence_penalty;
    int32_t greedy;
    uint32_t flags;
    uint64_t seed;
    uint64_t offset;
} tmo_row_params;

/* Same layout as tms_history_params in include/tmsample_hip.h. */
typedef struct tmo_history_params {
    int32_t no_repeat_ngram;
    float dry_multiplier;
    float dry_base;
    int32_t dry_allowed_length;
    int32_t dry_penalty_last_n;
    int32_t reserved;
} tmo_history_params;

void tmo_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);
void tmo_row_words(uint64_t seed, uint64_t offset, uint32_t stream, uint32_t* w0, uint32_t* w1);
double tmo_canonical(uint32_t w0, uint32_t w1);

void tmo_apply_mask(float* row, int V, const uint32_t* mask);
void tmo_apply_repeat_penalty(float* row, int V, const int32_t* recent, int n_recent,
                              int window, float penalty);
void tmo_apply_freq_presence(float* row, int V, const int32_t* recent, int n_recent,
                             int window, float freq, float presence);

void tmo_no_repeat_ngram(float* row, int V, const int32_t* recent, int n_recent, int ngram);
void tmo_dry(float* row, int V, const int32_t* recent, int n_recent, float multiplier, float base,
             int allowed_length, int penalty_last_n, const uint8_t* is_breaker);

/* Sample one already-penalised row; returns a TMS_ROW_* status. */
int tmo_sample_row(const float* row, int V, const tmo_row_params* p, uint32_t w0, uint32_t w1,
                   int32_t* token, int32_t* keep, int32_t* topk_ids, float* topk_probs,
                   int topk_cap);

/* Whole composition for a batch of fp32 rows (mask -> penalties -> sample).
 * recent/n_recent/mask/draws may be NULL, as in tms_sample_args. */
void tmo_sample_batch(const float* logits, int B, int V, int64_t row_stride,
                      const tmo_row_params* params, const int32_t* recent,
                      const int32_t* n_recent, int64_t recent_stride, const uint32_t* mask,
                      int64_t mask_stride, const uint32_t* draws, int32_t* tokens,
                      int32_t* status, int32_t* keep, int32_t* topk_ids, float* topk_probs,
                      int topk_cap);

/* The composition with the n-gram ban and DRY after the penalties
 * (llama_chat.cpp:148-151); hp and breaker may be NULL. */
void tmo_sample_batch_h(const float* logits, int B, int V, int64_t row_stride,
                        const tmo_row_params* params, const tmo_history_params* hp,
                        const uint8_t* breaker, const int32_t* recent, const int32_t* n_recent,
                        int64_t recent_stride, const uint32_t* mask, int64_t mask_stride,
                        const uint32_t* draws, int32_t* tokens, int32_t* status, int32_t* keep,
                        int32_t* topk_ids, float* topk_probs, int topk_cap);

/* Speculative verify (build-defined; see tms_oracle.c). */
double tmo_exp64(double x);
int64_t tmo_q44(double y);
int tmo_spec_weights(const float* row, int V, float temperature, int64_t* e, int64_t* Z,
                     float* m);
int tmo_spec_verify_seq(const float* target, const float* draft, int V, int k,
                        const int32_t* draft_tokens, float temperature,
                        const uint32_t* words, int32_t* accepted, int32_t* token);

#ifdef __cplusplus
}
#endif

#endif

// tms_context.h -- the library's per-device context (internal).
//
// One hipMalloc at creation holds every workspace region; the sampling and
// verify calls allocate nothing.  Every region a kernel reads before writing
// starts zeroed, and the kernels return it to zero (counters, list headers,
// published partial sums) before they exit, so back-to-back calls need no
// clearing launch.
#ifndef TMS_CONTEXT_H
#define TMS_CONTEXT_H

#include <stddef.h>
#include <stdint.h>

namespace tms {
constexpr int kSpecMaxK = 16;      // draft tokens per sequence
constexpr int kSpecParts = 64;     // vocabulary parts of the residual draw
constexpr int kPartWords = 3;      // u64 per part: weight sum, target sum, the bonus row's part max
constexpr int kCounterStride = 64; // u32 between per-row arrival counters: one 256-byte line
                                   // each, so the rows' atomics do not queue on one line
}  // namespace tms

// Statistics of one speculative-verify row (target or draft).
struct tms_spec_stat {
    float m;        // max of v / T
    int32_t status; // TMS_ROW_*
    int64_t Z;      // sum of the row's 2^-44 weights
    int64_t ex;     // weight of the draft token (rows with one), else 0
    int64_t pad;
};

struct tms_context {
    int device;
    int max_batch;
    int max_vocab;
    int max_chunks;
    size_t bytes;
    void* ws;
    size_t ones_begin, ones_end;   // byte range of the all-ones mask row in ws
    uint32_t* counters;        // [max_batch][kCounterStride] sampler arrival counters (word 0)
    uint32_t* ones;            // all-ones mask row, for calls without a grammar mask
    uint64_t* lists;           // [max_batch][max_chunks][kListStride] chunk candidate lists
    uint64_t* tlists;          // [max_batch][min(max_chunks, 16)][136] wide top-k kernel lists
    uint32_t* spec_tickets;    // [max_batch][kCounterStride] verify arrival counters (word 0)
    uint64_t* spec_parts;      // [max_batch][kSpecParts][kPartWords] published partial sums
    tms_spec_stat* spec_stats; // [max_batch][2 * kSpecMaxK + 1]
    uint32_t* dlocks;          // [dense_slots] whole-row region locks
    int32_t* ov_n;             // [max_batch] history pre-pass: list lengths (-1: overflow)
    int32_t* ov_ids;           // [max_batch][TMS_HISTORY_MAX_IDS] listed ids
    float* ov_vals;            // [max_batch][TMS_HISTORY_MAX_IDS] their final values
    uint64_t* dense;           // [dense_slots][2 * max_vocab] the whole-row path (separate allocation)
    int dense_slots;           // min(max_batch, kDenseSlotsMax) regions, each taken by a lock
    size_t dense_bytes;
};

#endif  // TMS_CONTEXT_H

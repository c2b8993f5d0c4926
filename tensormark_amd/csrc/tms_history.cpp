// tms_history.cpp -- the deterministic history transforms of TensorMark's
// sampler on a host row: repetition penalty, no-repeat n-gram ban and DRY.
//
// Host-side forms of what the device pre-pass (tms_hist.hip) does for
// tms_sample_args.history, for callers that hold a host row; the order of
// the reference's sample_token is theirs to keep
// (tensormark/llama_chat.cpp:146-153).

#include <math.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <cmath>
#include <utility>
#include <vector>

#include "../../include/tmsample_hip.h"

// tensormark/tmsample.h:52-63: v > 0 ? v / p : v * p, once per occurrence.
extern "C" void tms_host_repeat_penalty(float* logits, int V, const int32_t* recent, int n_recent,
                                        int window, float penalty) {
    if (!logits || !recent || penalty <= 1.0f || window <= 0 || n_recent <= 0) return;
    for (int i = n_recent > window ? n_recent - window : 0; i < n_recent; ++i) {
        const int id = recent[i];
        if (id < 0 || id >= V) continue;
        const float v = logits[id];
        logits[id] = v > 0.f ? v / penalty : v * penalty;
    }
}

// tensormark/tmsample.h:81-114: every id that followed an earlier occurrence
// of the current (ngram - 1)-id context becomes -inf; if that leaves no
// finite logit the banned ids get their values back.
extern "C" void tms_host_no_repeat_ngram(float* logits, int V, const int32_t* recent, int n_recent,
                                         int ngram) {
    if (!logits || !recent || ngram < 2 || n_recent < ngram) return;
    const float ninf = -INFINITY;
    const int ctx = ngram - 1;
    const int tail = n_recent - ctx;
    std::vector<std::pair<int, float>> undo;
    for (int i = 0; i < tail; ++i) {
        if (memcmp(recent + i, recent + tail, sizeof(int32_t) * (size_t)ctx) != 0) continue;
        const int next = recent[i + ctx];
        if (next < 0 || next >= V) continue;
        if (logits[next] == ninf) continue;   // banned already: keep the first saved value
        undo.emplace_back(next, logits[next]);
        logits[next] = ninf;
    }
    if (undo.empty()) return;
    // the reference's std::max scan from -inf: a NaN never becomes the best
    for (int i = 0; i < V; ++i)
        if (logits[i] > ninf) return;   // something is left
    for (const auto& u : undo) logits[u.first] = u.second;
}

// tensormark/tmsample.h:148-170: for each earlier position whose run agrees
// with the window's tail for L >= allowed_length ids (never across a breaker
// id), subtract multiplier * base^(L - allowed_length) from the id that
// followed the earlier run.
//
// Every position's agreement comes from one linear pass: with the window
// reversed (r[j] = id at last - j), the agreement of the run ending at i
// with the tail is the longest common prefix of r and r[last - i ..], which
// the Z-function gives for every shift at once.  Each breaker occurrence
// becomes a code of its own (below every id), so no match extends across
// one.  The penalties are applied in ascending position order, as the
// reference applies them.
extern "C" void tms_host_dry(float* logits, int V, const int32_t* recent, int n_recent,
                             float multiplier, float base, int allowed_length, int penalty_last_n,
                             const unsigned char* is_breaker) {
    if (!logits || !recent || multiplier <= 0.0f || allowed_length < 1) return;
    const int n = n_recent < penalty_last_n ? n_recent : penalty_last_n;
    if (n_recent < allowed_length + 1 || n < allowed_length + 1) return;
    const int32_t* w = recent + (n_recent - n);
    const int last = n - 1;
    auto breaker = [&](int32_t id) { return is_breaker && id >= 0 && id < V && is_breaker[id]; };
    std::vector<int64_t> r((size_t)n);
    for (int j = 0; j < n; ++j) {
        const int32_t id = w[last - j];
        r[(size_t)j] = breaker(id) ? INT64_MIN + j : (int64_t)id;
    }
    std::vector<int> z((size_t)n, 0);   // z[d]: common prefix of r and r[d..]
    for (int d = 1, lo = 0, hi = 0; d < n; ++d) {
        int k = d < hi ? std::min(hi - d, z[(size_t)(d - lo)]) : 0;
        while (d + k < n && r[(size_t)k] == r[(size_t)(d + k)]) ++k;
        z[(size_t)d] = k;
        if (d + k > hi) {
            lo = d;
            hi = d + k;
        }
    }
    for (int i = 0; i < last; ++i) {
        const int L = z[(size_t)(last - i)];
        if (L < allowed_length) continue;
        const int32_t next = w[i + 1];
        if (next < 0 || next >= V || breaker(next)) continue;
        logits[next] -= multiplier * std::pow(base, (float)(L - allowed_length));
    }
}

extern "C" int tms_dry_scale_table(float base, int n, float* out) {
    if (!out || n < 0) return TMS_ERR_INVALID_ARG;
    for (int k = 0; k < n; ++k) out[k] = std::pow(base, (float)k);
    return TMS_OK;
}

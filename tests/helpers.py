"""Shared helpers for the tests: golden cases and parameter records."""
from __future__ import annotations

import numpy as np

import oracle


def golden_cases(golden):
    """Yield (i, x, params, recent, mask, w0, w1, expected) per golden case."""
    meta = golden["meta"]
    for i, m in enumerate(meta):
        x = golden[f"x{i}"]
        recent = golden[f"recent{i}"] if m["win"] > 0 else None
        mask = golden[f"mask{i}"] if m["has_mask"] else None
        p = np.zeros(1, oracle.ROW_DTYPE)
        p["temperature"] = m["T"]
        p["top_k"] = m["k"]
        p["top_p"] = m["p"]
        p["greedy"] = m["g"]
        p["repeat_penalty"] = m["pen"]
        p["repeat_last_n"] = m["win"]
        yield i, x, p, recent, mask, int(m["w0"]), int(m["w1"]), m


def row_params(**kw) -> oracle.RowParams:
    p = oracle.RowParams()
    p.temperature = kw.get("temperature", 0.7)
    p.top_k = kw.get("top_k", 40)
    p.top_p = kw.get("top_p", 0.9)
    p.min_p = kw.get("min_p", 0.0)
    p.repeat_penalty = kw.get("repeat_penalty", 1.0)
    p.repeat_last_n = kw.get("repeat_last_n", 0)
    p.frequency_penalty = kw.get("frequency_penalty", 0.0)
    p.presence_penalty = kw.get("presence_penalty", 0.0)
    p.greedy = int(kw.get("greedy", 0))
    p.seed = kw.get("seed", 0)
    p.offset = kw.get("offset", 0)
    return p


def params_array(B, **kw) -> np.ndarray:
    p = np.zeros(B, oracle.ROW_DTYPE)
    defaults = dict(temperature=0.7, top_k=40, top_p=0.9, min_p=0.0, repeat_penalty=1.0,
                    repeat_last_n=0, frequency_penalty=0.0, presence_penalty=0.0, greedy=0,
                    seed=0, offset=0)
    defaults.update(kw)
    for k, v in defaults.items():
        p[k] = v
    return p

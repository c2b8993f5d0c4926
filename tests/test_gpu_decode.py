"""GPU decode loops around the sampler:

* grammar-constrained decoding with the asynchronous mask pipeline
  (tms_mask_pipe): the same tokens as the synchronous loop that builds every
  mask on the host before the step (llama_chat.cpp:787-803), every token
  inside the grammar, whitespace narrowing exercised;
* the chained device-resident decode (tms_token_slot + tms_embed_gather):
  n steps enqueued at once give the same ids as the step-by-step loop with a
  host round trip per step, and the host sees every id land in the slot."""
from __future__ import annotations

import time

import numpy as np
import pytest

from tensormark_amd import Sampler
from tensormark_amd.grammar import Filter, Grammar, MaskPipe, TokenMask, TokenTable
from tests.helpers import params_array as make_params

pytestmark = pytest.mark.gpu

GRAMMAR = r'''
root  ::= "{" ws pair ( "," ws pair )* ws "}" ws
pair  ::= "\"" key "\"" ws ":" ws value
key   ::= [a-z]+
value ::= [0-9]+ | "\"" [a-z ]* "\""
ws    ::= [ \t\n]*
'''


def _vocab():
    pieces = ["</s>"] + list("{}\",:") + list("abcdefghijklmnopqrstuvwxyz") + list("0123456789")
    pieces += ["▁", "\n", "▁▁", "\t", "▁\n", "ab", "key", "12", "▁\"", "\":", "▁}", "x▁y", "\"a\""]
    types = [3] + [1] * (len(pieces) - 1)
    return pieces, types


@pytest.fixture(scope="module")
def dev_sampler():
    import torch

    assert torch.cuda.is_available()
    s = Sampler(max_batch=64, max_vocab=4096)
    yield s
    s.close()


def _decode(sampler, mode, steps=48, B=8, seed=3):
    import torch

    pieces, types = _vocab()
    V = len(pieces)
    t = TokenTable.spm(pieces, types)
    grammars = [Grammar.parse(GRAMMAR) for _ in range(2)]   # two grammars: two worker groups
    masks = [TokenMask.from_table(g, t, eos=0) for g in grammars]
    filters = [Filter(grammars[b % 2], masks[b % 2], t) for b in range(B)]
    ws_ids = [i for i in range(V) if t.ws_only(i)]
    rng = np.random.default_rng(seed)
    stream = torch.cuda.current_stream().cuda_stream
    pipe = None
    if mode == "pipe":
        pipe = MaskPipe(B, V, threads=2)
        for b in range(B):
            pipe.set_row(b, filters[b])
        pipe.submit(None)
    done = np.zeros(B, bool)
    out_tokens, used_masks = [], []
    narrowed = 0
    for step in range(steps):
        x = rng.normal(0.0, 1.0, (B, V)).astype(np.float32)
        x[:, ws_ids] += 2.5            # whitespace is attractive: stalls happen
        logits = torch.from_numpy(x).to("cuda:0")     # the step's "forward"
        p = make_params(B, temperature=1.0, top_k=0, top_p=1.0, greedy=(np.arange(B) % 4 == 0),
                        seed=1000 + np.arange(B), offset=step)
        if mode == "pipe":
            ptr, allowed = pipe.acquire(stream)
            out = sampler.sample(logits, p, mask=(ptr, (V + 31) // 32))
            pipe.release(stream)
            words = None
        else:
            ws = [f.mask(V) for f in filters]
            words = np.stack([w for w, _ in ws])
            allowed = np.array([n for _, n in ws], np.int32)
            out = sampler.sample(logits, p, mask=torch.from_numpy(words.view(np.int32)).to("cuda:0"))
        tok = out["tokens"].cpu().numpy()
        st = out["status"].cpu().numpy()
        assert (st[~done] == 0).all(), (step, st)
        nxt = np.where(done, -1, tok).astype(np.int32)
        narrowed += int(sum(filters[b].stall >= 4 for b in range(B) if not done[b]))
        for b in range(B):
            if done[b]:
                continue
            if tok[b] == 0:
                done[b] = True
                nxt[b] = -1
        if mode == "pipe":
            pipe.submit(nxt)           # the filters consume on the workers
        else:
            for b in range(B):
                if nxt[b] >= 0:
                    assert filters[b].consume(int(nxt[b]))
        out_tokens.append(np.where(nxt >= 0, nxt, -1))
        used_masks.append((words, allowed))
        if done.all():
            break
    if pipe is not None:
        pipe.acquire(stream)
        pipe.close()
    return np.array(out_tokens), t, done, narrowed


def test_mask_pipe_acquire_release_order(dev_sampler):
    """release needs an acquire; words stay held until released, so acquiring
    the next step, or submitting the one after it into the held slot, is
    refused; the next step may be submitted while the current one is held."""
    import torch

    from tensormark_amd.grammar import MaskPipe

    stream = torch.cuda.current_stream().cuda_stream
    pipe = MaskPipe(4, 1000, threads=1)
    with pytest.raises(RuntimeError):
        pipe.release(stream)             # nothing acquired
    pipe.submit(None)
    pipe.acquire(stream)                 # step 0 held (slot A)
    pipe.submit(None)                    # step 1 fills slot B: allowed
    with pytest.raises(RuntimeError):
        pipe.acquire(stream)             # step 1 while step 0 is held
    with pytest.raises(RuntimeError):
        pipe.submit(None)                # step 2 would refill slot A, still held
    pipe.release(stream)                 # step 0 done
    pipe.acquire(stream)                 # step 1 (slot B)
    pipe.release(stream)
    with pytest.raises(RuntimeError):
        pipe.release(stream)             # released twice
    pipe.submit(None)                    # step 2 (slot A): allowed now
    pipe.acquire(stream)
    pipe.release(stream)
    pipe.close()


def test_mask_pipe_matches_synchronous_masks(dev_sampler):
    sync, t, done_s, narrowed = _decode(dev_sampler, "sync")
    piped, _, done_p, _ = _decode(dev_sampler, "pipe")
    assert sync.shape == piped.shape
    assert np.array_equal(sync, piped)
    assert np.array_equal(done_s, done_p)
    assert narrowed > 0                       # the stall narrowing ran
    # every finished row is a sentence of the grammar
    g = Grammar.parse(GRAMMAR)
    for b in range(sync.shape[1]):
        if done_s[b]:
            text = b"".join(t.bytes(int(i)) for i in sync[:, b] if i > 0)
            assert g.accepts(text), text
    assert done_s.sum() >= 1


def test_chain_matches_step_by_step(dev_sampler):
    import torch

    from tensormark_amd.chain import Chain, embed_gather

    torch.manual_seed(0)
    B, V, D, n = 4, 3000, 128, 12
    E = torch.randn(V, D, device="cuda:0")
    W = torch.randn(V, D, device="cuda:0") * 0.3
    forward = lambda x: (x @ W.t()).contiguous()
    first = np.array([5, 17, 2999, 0], np.int32)
    params = [make_params(B, temperature=0.9, top_k=50, top_p=0.95, greedy=(np.arange(B) == 3),
                          seed=77 + np.arange(B), offset=i) for i in range(n)]
    # step by step, a host round trip per step
    cur = torch.from_numpy(first).to("cuda:0")
    want = []
    x = torch.empty(B, D, device="cuda:0")
    for i in range(n):
        embed_gather(E, cur, x)
        assert torch.equal(x, E[cur.long()])
        out = dev_sampler.sample(forward(x), params[i])
        ids = out["tokens"].cpu().numpy()
        assert (out["status"].cpu().numpy() == 0).all()
        want.append(ids)
        cur = torch.from_numpy(ids).to("cuda:0")
    want = np.array(want)
    # chained: everything enqueued at once; the host watches the slot
    chain = Chain(dev_sampler, E, forward, batch=B, n_max=32)
    chain.begin(first, n, params)
    seen = np.full((n, B), -1)
    t0 = time.time()
    while (seen < 0).any() and time.time() - t0 < 30.0:
        for i in range(n):
            for b in range(B):
                if seen[i, b] < 0:
                    seen[i, b] = chain.poll(i, b)
    ids, status = chain.end()
    assert (status == 0).all()
    assert np.array_equal(ids, want)
    assert np.array_equal(seen, want)        # every id landed in the slot, as sampled
    assert chain.poll(n, 0) == -1            # beyond the chain


def test_chain_publishes_rows_without_a_token(dev_sampler):
    """A row the sampler cannot sample (temperature 0, not greedy) lands in
    the slot as -2, never as the pending -1."""
    import torch

    from tensormark_amd.chain import Chain

    B, V, D = 2, 1000, 64
    E = torch.randn(V, D, device="cuda:0")
    W = torch.randn(V, D, device="cuda:0")
    chain = Chain(dev_sampler, E, lambda x: (x @ W.t()).contiguous(), batch=B, n_max=4)
    p = make_params(B, temperature=1.0, top_k=10)
    p["temperature"][1] = 0.0
    chain.begin(np.array([1, 2], np.int32), 2, [p, p])
    ids, status = chain.end()
    assert status[0, 1] == 1 and ids[0, 1] == -1
    assert chain.slot.peek(1) == -2 and chain.slot.peek(0) == ids[0, 0]

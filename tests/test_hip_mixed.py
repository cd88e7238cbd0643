"""One continuous-batching step as one pass (axon_model_forward_mixed): a prompt chunk of one
sequence and a decode row for each sequence in decode, through one launch set.

The reference runs the step as two passes (BatchEngine::step, src/engine/batch.cpp:69-156):
forward_prefill of the oldest prompt's next chunk (batch.cpp:71-85, Sequence::prefill_chunk,
sequence.cpp:101-123, which observes the chunk's last row only), then forward_batch of the
sequences in decode (batch.cpp:113-150). The mixed pass must give each row what those two passes
give it, bit for bit: the rows are independent (test_model_batch.cpp:103-157 pins batched rows
to each sequence alone), the prompt rows see their own chunk causally, and the kernels' results
do not depend on how many rows share a launch. Checked here:
* one mixed step against the two passes on the same caches: logits and every cache row, on the
  four fixture models, both cache types, and row counts that take each matmul path (the fused
  decode matvec up to 4 rows, the batched-decode MFMA kernel for 5-64, the tile MFMA kernel
  above);
* the same step against the oracle's two passes (the north star's 1e-4);
* whole continuous-batching schedules on the BASELINE config-4 and config-5 shapes (2 layers):
  the token streams and every observed row of logits equal the two-pass engine's;
* the greedy choice on the device after a mixed pass, and the bounds."""
from dataclasses import replace

import numpy as np
import pytest

from helpers import GOLDEN, OracleModel

pytestmark = pytest.mark.gpu

FIXTURES = ["synthetic-2l.gguf", "synthetic-2l-q8_0.gguf", "synthetic-2l-q4_0.gguf", "synthetic-2l-q4_1.gguf"]


def hip_model(path, **kw):
    import axon_hip as H
    return H.Model(path, **kw)


def prompts(n_vocab, lens, seed):
    rng = np.random.default_rng(seed)
    return [rng.integers(0, n_vocab, n).astype(np.int32) for n in lens]


def prefilled(m, ps):
    out = []
    for p in ps:
        c = m.new_cache()
        m.forward_prefill(c, p)
        out.append(c)
    return out


# (tokens already in the prefill cache, chunk length, decode contexts): 3, 12 and 73 rows.
CASES = [(0, 1, [3, 5]), (5, 9, [3, 7, 11]), (2, 70, [4, 9, 30])]


@pytest.mark.parametrize("cache", ["f32", "f16"])
@pytest.mark.parametrize("name", FIXTURES)
def test_mixed_step_equals_the_two_passes(name, cache):
    path = GOLDEN / "gguf" / name
    m = hip_model(path, max_seq=72, max_ctx=128, max_batch=4, max_caches=10, cache=cache)
    n_vocab = m.info.n_vocab
    for past, chunk_len, ctx in CASES:
        ps = prompts(n_vocab, ctx + [past + chunk_len], seed=past + chunk_len)
        head, chunk = ps[-1][:past], ps[-1][past:]
        nxt = np.random.default_rng(chunk_len).integers(0, n_vocab, len(ctx)).astype(np.int32)
        # The reference's two passes.
        two = prefilled(m, ps[:-1])
        p2 = m.new_cache()
        if past:
            m.forward_prefill(p2, head)
        lp = m.forward_prefill(p2, chunk)
        lb = m.forward_batch(two, nxt)
        # One pass.
        one = prefilled(m, ps[:-1])
        p1 = m.new_cache()
        if past:
            m.forward_prefill(p1, head)
        lm = m.forward_mixed(p1, chunk, one, nxt)
        assert lm.shape == (1 + len(ctx), n_vocab)
        assert np.array_equal(lm[0], lp[-1]), (past, chunk_len)
        assert np.array_equal(lm[1:], lb), (past, chunk_len)
        assert m.cache_pos(p1) == past + chunk_len and [m.cache_pos(c) for c in one] == [n + 1 for n in ctx]
        for layer in range(2):
            for values in (False, True):
                for a, b, n in [(p1, p2, past + chunk_len)] + [(x, y, k + 1) for x, y, k in zip(one, two, ctx)]:
                    assert np.array_equal(m.cache_rows(a, layer, values, n), m.cache_rows(b, layer, values, n))
        # The next step: everyone in decode, the prefilled sequence included.
        t = np.append(nxt, 7).astype(np.int32)
        assert np.array_equal(m.forward_mixed(None, [], one + [p1], t), m.forward_batch(two + [p2], t))
        for c in one + two + [p1, p2]:
            m.free_cache(c)


@pytest.mark.parametrize("name", ["synthetic-2l-q4_0.gguf", "synthetic-2l.gguf"])
def test_mixed_step_matches_the_oracle(name):
    path = GOLDEN / "gguf" / name
    m = hip_model(path, max_seq=72, max_ctx=128, max_batch=4, max_caches=10)
    o = OracleModel(path)
    n_vocab = m.info.n_vocab
    for past, chunk_len, ctx in CASES:
        ps = prompts(n_vocab, ctx + [past + chunk_len], seed=100 + chunk_len)
        head, chunk = ps[-1][:past], ps[-1][past:]
        nxt = np.random.default_rng(chunk_len).integers(0, n_vocab, len(ctx)).astype(np.int32)
        caches = prefilled(m, ps[:-1])
        pc = m.new_cache()
        if past:
            m.forward_prefill(pc, head)
        got = m.forward_mixed(pc, chunk, caches, nxt)
        ocs = []
        for p in ps[:-1]:
            oc = o.new_cache(128)
            o.forward(p, oc)
            ocs.append(oc)
        op = o.new_cache(128)
        if past:
            o.forward(head, op)
        want = np.concatenate([o.forward(chunk, op)[-1:], o.forward_batch(nxt, ocs)])
        assert np.max(np.abs(got - want)) <= 1e-4, (chunk_len, np.max(np.abs(got - want)))
        for c in caches + [pc]:
            m.free_cache(c)


class TwoPass:
    """BatchEngine::step as the reference runs it: the chunk, then the decode batch."""

    def __init__(self, m):
        self.m = m

    def step(self, pc, chunk, caches, toks):
        rows = []
        if chunk is not None:
            rows.append(self.m.forward_prefill(pc, chunk)[-1:])
        if caches:
            rows.append(self.m.forward_batch(caches, toks))
        return np.concatenate(rows)


class OnePass:
    def __init__(self, m):
        self.m = m

    def step(self, pc, chunk, caches, toks):
        return self.m.forward_mixed(pc if chunk is not None else None, [] if chunk is None else chunk, caches, toks)


def run_schedule(engine, m, ps, joins, decode_steps):
    """Continuous batching as BatchEngine::step: each step prefills one chunk (max_seq tokens)
    of the oldest admitted sequence still in prefill and decodes every sequence in decode; a
    sequence moves to decode once its prompt is in, with the greedy choice over the chunk's last
    row. Returns the token streams and every observed row of logits, in order."""
    n = len(ps)
    max_seq = m.info.max_seq
    caches = [None] * n
    fed = [0] * n
    nxt = [None] * n
    out = [[] for _ in range(n)]
    observed = []
    step = 0
    while any(len(o) < decode_steps for o in out):
        for i in range(n):
            if joins[i] == step:
                caches[i] = m.new_cache()
        pre = [i for i in range(n) if caches[i] is not None and fed[i] < len(ps[i])]
        dec = [i for i in range(n) if caches[i] is not None and fed[i] == len(ps[i]) and len(out[i]) < decode_steps]
        pi = min(pre, key=lambda i: (joins[i], i)) if pre else None
        chunk = ps[pi][fed[pi]:fed[pi] + max_seq] if pi is not None else None
        logits = engine.step(caches[pi] if pi is not None else None, chunk, [caches[i] for i in dec],
                             np.array([nxt[i] for i in dec], np.int32))
        observed.append(logits)
        r = 0
        if pi is not None:
            fed[pi] += len(chunk)
            if fed[pi] == len(ps[pi]):
                nxt[pi] = int(np.argmax(logits[0]))
            r = 1
        for j, i in enumerate(dec):
            t = int(np.argmax(logits[r + j]))
            out[i].append(nxt[i])
            nxt[i] = t
            if len(out[i]) == decode_steps:
                m.free_cache(caches[i])
        step += 1
    return out, observed


@pytest.mark.parametrize("cfg", ["c4", "c5"])
def test_mixed_schedule_equals_the_two_pass_engine(cfg, tmp_path_factory):
    """A continuous-batching run on the config-4 (Llama-3.2-1B, Q4_0, tied Q6_K output) and
    config-5 (Qwen2.5-0.5B, Q4_0 with q/k/v bias and NeoX RoPE, Q8_0 output) shapes at 2 layers
    and a 2048-token vocabulary: six sequences with prompts of 3 to 150 tokens (chunked at
    max_seq 64) join over the first steps and decode 12 tokens each. The one-pass engine gives
    the same token streams and the same bits in every observed row as the two-pass engine."""
    import synth
    spec = replace(synth.CONFIGS[cfg], name=f"t-{cfg}-2l", n_layer=2, n_vocab=2048, seed=11)
    path = synth.cached_model(spec, tmp_path_factory.mktemp("models"))
    ps = prompts(spec.n_vocab, [40, 3, 150, 64, 17, 90], seed=3)
    joins = [0, 0, 1, 3, 3, 6]
    outs, obs = [], []
    for engine in (TwoPass, OnePass):
        m = hip_model(path, max_seq=64, max_ctx=256, max_batch=6, max_caches=7)
        o, seen = run_schedule(engine(m), m, ps, joins, 12)
        outs.append(o)
        obs.append(seen)
        m.close()
    assert outs[0] == outs[1]
    assert len(obs[0]) == len(obs[1])
    for a, b in zip(*obs):
        assert np.array_equal(a, b)


def test_greedy_after_a_mixed_pass():
    """The logits left in HBM by a mixed pass feed the device greedy choice: one id for the
    chunk's last row, then one per decode row, equal to the argmax of the host logits."""
    path = GOLDEN / "gguf" / "synthetic-2l-q4_0.gguf"
    m = hip_model(path, max_seq=32, max_ctx=128, max_batch=4, max_caches=10)
    ps = prompts(m.info.n_vocab, [6, 9, 20], seed=9)
    nxt = np.array([5, 6], np.int32)
    a = prefilled(m, ps[:2])
    pa = m.new_cache()
    want = np.argmax(m.forward_mixed(pa, ps[2], a, nxt), axis=1)
    b = prefilled(m, ps[:2])
    pb = m.new_cache()
    assert m.forward_mixed(pb, ps[2], b, nxt, logits=False) is None
    assert np.array_equal(m.greedy(3), want)


def test_mixed_bounds():
    import axon_hip as H
    path = GOLDEN / "gguf" / "synthetic-2l-q4_0.gguf"
    m = hip_model(path, max_seq=8, max_ctx=16, max_batch=2, max_caches=5)
    a, b, c, p = m.new_cache(), m.new_cache(), m.new_cache(), m.new_cache()
    with pytest.raises(H.HipError, match="no rows"):
        m.forward_mixed(None, [], [], [])
    with pytest.raises(H.HipError, match="also in the decode batch"):
        m.forward_mixed(a, [1, 2], [a, b], [1, 2])
    with pytest.raises(H.HipError, match="exceed max_seq"):
        m.forward_mixed(p, np.arange(9), [a], [1])
    with pytest.raises(H.HipError, match="exceed max_batch"):
        m.forward_mixed(p, [1], [a, b, c], [1, 2, 3])
    with pytest.raises(H.HipError, match="unknown cache"):
        m.forward_mixed(99, [1], [a], [1])
    with pytest.raises(ValueError, match="caches for"):
        m.forward_mixed(p, [1], [a, b], [1])
    assert [m.cache_pos(x) for x in (a, b, c, p)] == [0, 0, 0, 0]  # nothing ran
    # The largest pass: a max_seq chunk and max_batch decode rows.
    m.forward_prefill(a, [1])
    m.forward_prefill(b, [2])
    assert m.forward_mixed(p, np.arange(8), [a, b], [3, 4]).shape == (3, m.info.n_vocab)
    m.forward_mixed(p, np.arange(8), [], [])
    with pytest.raises(H.HipError, match="context overflow"):
        m.forward_mixed(p, [1], [], [])
    # Decode rows alone and a chunk alone.
    assert m.forward_mixed(None, [], [a], [5]).shape == (1, m.info.n_vocab)
    assert m.forward_mixed(c, [1, 2, 3], [], []).shape == (1, m.info.n_vocab)

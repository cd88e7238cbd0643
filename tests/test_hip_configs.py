"""The BASELINE model configurations at full depth and vocabulary on the device, against the
reference's own LlamaModel on its scalar table (oracle/_ref, compiled from the reference's
sources, host-threaded), or against the oracle's forward pass where oracle/_ref was not built
(the two are bit-identical: tests/test_oracle_ref.py).

Patterned on the reference's model tests: test_model_kernels.cpp:59-72 (a second kernel table
against the scalar table on whole models) and test_model_batch.cpp:103-157 (batched rows over
caches of different lengths). The north star's bars: logits within 1e-4 max-abs on the prompt
and on every step, and greedy tokens identical over 64 steps. The quantized matmuls are
bit-exact, so in practice nearly every logit is the reference's bit pattern; the fraction is
asserted too, so a path that drifts within tolerance still shows.

  C1  SmolLM2-135M shape, Q8_0, 30 layers, vocabulary 49152: a 128-token prompt, 64 greedy steps.
  C3  TinyLlama-1.1B shape: Q4_0 with a Q4_1 ffn_down, a Q4_0 embedding, an untied Q6_K output,
      GQA group 8: a 512-token prompt, 64 greedy steps.
  C4  Llama-3.2-1B shape (llama3 rope factors, tied Q6_K): a 128-token prompt and 64 greedy
      steps; 32 caches filled with the same random keys and values on both sides at contexts
      drawn from U[64, 2048], then four 32-row forward_batch steps, with either cache type; one
      cache at 3000 positions (past the decode kernels' 2304-position LDS bound), four steps.
  C5  Qwen2.5-0.5B shape (Q/K/V bias, NeoX rotary, Q8_0 output): a 256-token prompt and 32 greedy
      steps; one 64-row forward_batch over random caches at contexts U[32, 1024]; one mixed pass
      (a 128-token chunk and 63 decode rows) against the reference's two passes; and a seeded
      top-k 40 / top-p 0.9 / temperature 0.8 stream drawn on the device path against the oracle
      sampler over the reference's logits.

Models are written by synth.py on first use (under $AXON_MODEL_DIR, default /tmp/axon-models).
"""
import os

import numpy as np
import pytest

from helpers import OracleModel, RefModel, have_ref

pytestmark = pytest.mark.gpu

TOL = 1e-4


def threads():
    try:
        return max(1, min(16, len(os.sched_getaffinity(0))))
    except AttributeError:
        return max(1, min(16, os.cpu_count() or 1))


def model_path(cfg):
    import synth
    return synth.cached_model(synth.CONFIGS[cfg])


class Reference:
    """The reference LlamaModel (oracle/_ref) or, without it, the oracle's forward pass, behind
    one small interface: caches are ints, logits are [rows][n_vocab]."""

    def __init__(self, path, max_seq, max_ctx, max_batch, f16=False):
        self.ref = have_ref()
        # A batch's rows share the reference's max_seq-row activation arena (llama.cpp:326-329).
        max_seq = max(max_seq, max_batch)
        if self.ref:
            self.m = RefModel(path, max_seq=max_seq, max_ctx=max_ctx, max_batch=max_batch, n_threads=threads(), f16=f16)
        else:
            self.m = OracleModel(path)
            self.caches = []
            self.max_ctx, self.f16 = max_ctx, f16

    def new_cache(self):
        if self.ref:
            return self.m.new_cache()
        self.caches.append(self.m.new_cache(self.max_ctx, f16=self.f16))
        return len(self.caches) - 1

    def fill(self, cache, rows):
        """rows [n_layer][2][n][row] float32 at the cache's next positions."""
        rows = np.ascontiguousarray(rows, np.float32)
        n = rows.shape[2]
        if self.ref:
            import ctypes as C
            self.m.lib.ref_cache_fill(C.c_void_p(self.m.h), cache, C.c_void_p(rows.ctypes.data), C.c_size_t(n))
            return
        c = self.caches[cache]
        L, _, _, row = rows.shape
        if self.f16:
            store = c._store.reshape(L, 2, self.max_ctx, row)
            store[:, :, c.pos:c.pos + n] = rows.astype(np.float16).view(np.uint16)
        else:
            store = c._store.reshape(L, 2, self.max_ctx, row)
            store[:, :, c.pos:c.pos + n] = rows
        c.pos += n

    def prefill(self, cache, tokens):
        if self.ref:
            return self.m.forward_prefill(cache, tokens)
        return self.m.forward(tokens, self.caches[cache])

    def batch(self, caches, tokens):
        if self.ref:
            return self.m.forward_batch(caches, tokens)
        return self.m.forward_batch(tokens, [self.caches[c] for c in caches])


def close(got, want, what, min_equal=0.9):
    d = float(np.max(np.abs(got - want)))
    assert d <= TOL, f"{what}: max |logit difference| {d:.3g} > {TOL}"
    eq = float(np.mean(got == want))
    assert eq >= min_equal, f"{what}: only {eq:.3f} of the logits are bit-identical"
    return d


def greedy_run(hm, rm, prompt, steps, what):
    hc, rc = hm.new_cache(), rm.new_cache()
    hl = hm.forward_prefill(hc, prompt)
    rl = rm.prefill(rc, prompt)
    close(hl, rl, f"{what}: prompt logits")
    h_last, r_last = hl[-1], rl[-1]
    for s in range(steps):
        th, tr = int(np.argmax(h_last)), int(np.argmax(r_last))
        assert th == tr, f"{what}: greedy step {s}: {th} != {tr}"
        h_last = hm.forward_prefill(hc, [th])[0]
        r_last = rm.prefill(rc, [tr])[0]
        close(h_last, r_last, f"{what}: step {s}")


def random_rows(info, n, seed):
    rng = np.random.default_rng(seed)
    row = info.n_head_kv * info.head_dim
    return rng.standard_normal((info.n_layer, 2, n, row), dtype=np.float32)


def batch_steps(hm, rm, lens, steps, seed, what):
    """Caches filled with the same random rows on both sides at the given context lengths,
    then `steps` forward_batch steps of every sequence, greedy tokens fed back."""
    hcs, rcs = [], []
    for i, n in enumerate(lens):
        rows = random_rows(hm.info, n, seed + i)
        hc, rc = hm.new_cache(), rm.new_cache()
        hm.cache_fill(hc, rows)
        rm.fill(rc, rows)
        hcs.append(hc)
        rcs.append(rc)
    toks = np.random.default_rng(seed).integers(0, hm.n_vocab, len(lens)).astype(np.int32)
    for s in range(steps):
        hl = hm.forward_batch(hcs, toks)
        rl = rm.batch(rcs, toks)
        close(hl, rl, f"{what}: batch step {s}")
        th, tr = np.argmax(hl, axis=1).astype(np.int32), np.argmax(rl, axis=1).astype(np.int32)
        assert np.array_equal(th, tr), f"{what}: batch step {s} greedy ids differ"
        toks = th
    assert [hm.cache_pos(c) for c in hcs] == [n + steps for n in lens]


def hip(path, **kw):
    import axon_hip as H
    return H.Model(path, **kw)


def test_c1_prompt_128_and_64_greedy_steps():
    path = model_path("c1")
    hm = hip(path, max_seq=128, max_ctx=256)
    rm = Reference(path, max_seq=128, max_ctx=256, max_batch=1)
    prompt = np.random.default_rng(101).integers(0, hm.n_vocab, 128).astype(np.int32)
    greedy_run(hm, rm, prompt, 64, "C1")
    hm.close()


def test_c3_prompt_512_and_64_greedy_steps():
    path = model_path("c3")
    hm = hip(path, max_seq=512, max_ctx=640)
    rm = Reference(path, max_seq=512, max_ctx=640, max_batch=1)
    prompt = np.random.default_rng(103).integers(0, hm.n_vocab, 512).astype(np.int32)
    greedy_run(hm, rm, prompt, 64, "C3")
    hm.close()


def test_c4_prompt_128_and_64_greedy_steps():
    path = model_path("c4")
    hm = hip(path, max_seq=128, max_ctx=256)
    rm = Reference(path, max_seq=128, max_ctx=256, max_batch=1)
    prompt = np.random.default_rng(104).integers(0, hm.n_vocab, 128).astype(np.int32)
    greedy_run(hm, rm, prompt, 64, "C4")
    hm.close()


@pytest.mark.parametrize("cache", ["f32", "f16"])
def test_c4_ragged_32_rows_from_the_same_caches(cache):
    """The ragged-32 workload's step: 32 sequences at contexts U[64, 2048] (the BASELINE draw),
    four forward_batch steps on caches that start from the same random contents on both sides."""
    path = model_path("c4")
    lens = np.random.default_rng(4).integers(64, 2049, 32).tolist()
    hm = hip(path, max_seq=8, max_ctx=2064, max_batch=32, max_caches=33, cache=cache)
    rm = Reference(path, max_seq=8, max_ctx=2064, max_batch=32, f16=cache == "f16")
    batch_steps(hm, rm, lens, 4, 40, f"C4 ragged-32 ({cache} cache)")
    hm.close()


def test_c4_decode_past_the_lds_bound():
    """One sequence at 3000 positions: decode attention beyond 2304 visible positions takes the
    scores-in-global-scratch path."""
    path = model_path("c4")
    hm = hip(path, max_seq=8, max_ctx=3008, max_batch=2, max_caches=3)
    rm = Reference(path, max_seq=8, max_ctx=3008, max_batch=2)
    batch_steps(hm, rm, [3000, 2400], 4, 77, "C4 at 3000 positions")
    hm.close()


def test_c5_prompt_256_and_32_greedy_steps():
    path = model_path("c5")
    hm = hip(path, max_seq=256, max_ctx=320)
    rm = Reference(path, max_seq=256, max_ctx=320, max_batch=1)
    prompt = np.random.default_rng(105).integers(0, hm.n_vocab, 256).astype(np.int32)
    greedy_run(hm, rm, prompt, 32, "C5")
    hm.close()


def test_c5_64_rows_and_a_mixed_pass():
    """A 64-row decode batch over random caches at contexts U[32, 1024] (C5's prompt draw), then
    one continuous-batching step as one pass: a 128-token prompt chunk into a fresh cache and 63
    decode rows, against the reference's two passes (forward_prefill of the chunk, then
    forward_batch of the decode rows)."""
    path = model_path("c5")
    lens = np.random.default_rng(5).integers(32, 1025, 64).tolist()
    hm = hip(path, max_seq=128, max_ctx=1040, max_batch=64, max_caches=130)
    rm = Reference(path, max_seq=128, max_ctx=1040, max_batch=64)
    batch_steps(hm, rm, lens, 1, 50, "C5 64 rows")
    hcs, rcs = [], []
    for i, n in enumerate(lens[:63]):
        rows = random_rows(hm.info, n, 500 + i)
        hc, rc = hm.new_cache(), rm.new_cache()
        hm.cache_fill(hc, rows)
        rm.fill(rc, rows)
        hcs.append(hc)
        rcs.append(rc)
    hp, rp = hm.new_cache(), rm.new_cache()
    chunk = np.random.default_rng(51).integers(0, hm.n_vocab, 128).astype(np.int32)
    toks = np.random.default_rng(52).integers(0, hm.n_vocab, 63).astype(np.int32)
    got = hm.forward_mixed(hp, chunk, hcs, toks)
    want = np.concatenate([rm.prefill(rp, chunk)[-1:], rm.batch(rcs, toks)])
    close(got, want, "C5 mixed pass")
    hm.close()


def test_c5_sampled_stream_matches_the_reference_sampler():
    """Seeded top-k 40 / top-p 0.9 / temperature 0.8 sampling with SamplerConfig's min-p 0.05 and
    repetition penalty 1.1 over the last 64 ids, 32 tokens after a 64-token prompt: the device
    path (penalty and top-k on the device, the draw on the host) draws the same ids as the
    oracle sampler (pinned draw for draw to the reference's Sampler) over the reference's logits."""
    import axon_hip as H
    from test_oracle_sampling import OracleSampler
    path = model_path("c5")
    hm = hip(path, max_seq=64, max_ctx=128)
    rm = Reference(path, max_seq=64, max_ctx=128, max_batch=1)
    cfg = H.SamplerConfig(temperature=0.8, top_k=40, top_p=0.9, min_p=0.05, repeat_penalty=1.1, repeat_last_n=64)
    prompt = np.random.default_rng(106).integers(0, hm.n_vocab, 64).astype(np.int32)
    hc, rc = hm.new_cache(), rm.new_cache()
    hm.forward_prefill(hc, prompt[:-1], logits=False)
    hm.forward_prefill(hc, prompt[-1:], logits=False)  # a pass whose only row is the prompt's last
    rl = rm.prefill(rc, prompt)[-1]
    rng = H.Rng(2024)
    osampler = OracleSampler(hm.n_vocab, temperature=0.8, top_k=40, top_p=0.9, min_p=0.05, repeat_penalty=1.1,
                             repeat_last_n=64, seed=2024)
    hist = list(prompt)
    for s in range(32):
        hid = int(hm.sample([cfg], [rng], [np.array(hist, np.int32)])[0])
        oid = int(osampler.sample(rl, np.array(hist, np.int32)))
        assert hid == oid, f"C5 sampled step {s}: {hid} != {oid}"
        hist.append(hid)
        hm.forward_prefill(hc, [hid], logits=False)
        rl = rm.prefill(rc, [hid])[0]
    hm.close()


@pytest.mark.parametrize("cfg, cache", [("c1", "f32"), ("c3", "f32"), ("c4", "f32"), ("c1", "f16"), ("c4", "f16")])
def test_persistent_decode_equals_launch_by_launch(cfg, cache):
    """The one-kernel decode step (axon_hip_decode_layers) against the same model launching each
    step of a layer on its own: the persistent path is taken (info.persistent_decode), and 48
    greedy steps after a 40-token prompt give bit-identical logits and cache rows. With the fp16
    cache the kernel rounds the new key and value once into the pool and reads every position
    (the new one included) back from fp16, as the per-layer launches do."""
    path = model_path(cfg)
    a = hip(path, max_seq=64, max_ctx=160, cache=cache)
    b = hip(path, max_seq=64, max_ctx=160, persistent=False, cache=cache)
    assert a.info.persistent_decode == 1 and b.info.persistent_decode == 0
    prompt = np.random.default_rng(77).integers(0, a.n_vocab, 40).astype(np.int32)
    ca, cb = a.new_cache(), b.new_cache()
    la, lb = a.forward_prefill(ca, prompt)[-1], b.forward_prefill(cb, prompt)[-1]
    for s in range(48):
        t = int(np.argmax(la))
        la, lb = a.forward_prefill(ca, [t])[0], b.forward_prefill(cb, [t])[0]
        assert np.array_equal(la, lb), f"{cfg} step {s}: max diff {np.max(np.abs(la - lb))}"
    for layer in (0, a.info.n_layer - 1):
        for v in (False, True):
            assert np.array_equal(a.cache_rows(ca, layer, v, 88), b.cache_rows(cb, layer, v, 88))
    a.close()
    b.close()


@pytest.mark.parametrize("cfg, cache", [("c3", "f32"), ("c4", "f32"), ("c4", "f16")])
def test_persistent_decode_at_long_context(cfg, cache):
    """The step kernel past a thousand positions: the scores of each head from 32 workgroups of
    its group, four or more V chunks per mixing workgroup, the score polls in rounds of 2048
    positions. 32 greedy steps from position 1008 (a 1008-token prompt): logits and cache rows
    bit-identical to the per-layer launches."""
    path = model_path(cfg)
    a = hip(path, max_seq=1024, max_ctx=1056, cache=cache)
    b = hip(path, max_seq=1024, max_ctx=1056, persistent=False, cache=cache)
    assert a.info.persistent_decode == 1 and b.info.persistent_decode == 0
    prompt = np.random.default_rng(78).integers(0, a.n_vocab, 1008).astype(np.int32)
    ca, cb = a.new_cache(), b.new_cache()
    a.forward_mixed(ca, prompt, [], [], logits=False)  # logits of the prompt's last row only
    b.forward_mixed(cb, prompt, [], [], logits=False)
    t = int(a.greedy(1)[0])
    assert int(b.greedy(1)[0]) == t
    for s in range(32):
        la, lb = a.forward_prefill(ca, [t])[0], b.forward_prefill(cb, [t])[0]
        assert np.array_equal(la, lb), f"{cfg} position {1008 + s}: max diff {np.max(np.abs(la - lb))}"
        t = int(np.argmax(la))
    for layer in (0, a.info.n_layer - 1):
        for v in (False, True):
            assert np.array_equal(a.cache_rows(ca, layer, v, 1040), b.cache_rows(cb, layer, v, 1040))
    a.close()
    b.close()


@pytest.mark.parametrize("cfg", ["c1", "c4"])
def test_generate_greedy_equals_host_loop(cfg):
    """axon_model_generate_greedy (each step's id kept on the device for the next step's
    embedding) against the host loop of Engine::generate at temperature zero: forward_prefill of
    the previous id, then the greedy choice. 40 steps after a 24-token prompt give the same ids,
    the same K/V rows, and the same logits for the step after, on the persistent path and on
    the per-layer path."""
    path = model_path(cfg)
    for persistent in (True, False):
        a = hip(path, max_seq=64, max_ctx=128, persistent=persistent)
        b = hip(path, max_seq=64, max_ctx=128, persistent=persistent)
        prompt = np.random.default_rng(11).integers(0, a.n_vocab, 24).astype(np.int32)
        ca, cb = a.new_cache(), b.new_cache()
        a.forward_mixed(ca, prompt, [], [], logits=False)  # logits of the prompt's last row only
        t0 = int(a.greedy(1)[0])
        b.forward_mixed(cb, prompt, [], [], logits=False)
        assert int(b.greedy(1)[0]) == t0
        got = a.generate_greedy(ca, t0, 40)
        want, t = [], t0
        for _ in range(40):
            b.forward_prefill(cb, [t], logits=False)
            t = int(b.greedy(1)[0])
            want.append(t)
        assert got.tolist() == want, (cfg, persistent)
        assert a.cache_pos(ca) == b.cache_pos(cb) == 24 + 40
        for layer in (0, a.info.n_layer - 1):
            for v in (False, True):
                assert np.array_equal(a.cache_rows(ca, layer, v, 64), b.cache_rows(cb, layer, v, 64))
        la, lb = a.forward_prefill(ca, [want[-1]])[0], b.forward_prefill(cb, [want[-1]])[0]
        assert np.array_equal(la, lb)
        a.close()
        b.close()


def test_persistent_decode_gives_up_cleanly_and_recovers(tmp_path_factory):
    """The step kernel's bounded waits, forced from the host: with a limit of one poll per
    tagged word and waits that never see their word written, the workgroups of a one-row pass
    give up instead of waiting, the kernel still drains, and the pass is void. With the logits copied the pass fails at once and its cache
    position does not advance; with the logits left in HBM the pass returns, and the next
    synchronization (the greedy choice) fails, names the cache slot and position, and rolls the
    cache back to it. Either way the model turns the persistent kernel off for later one-row
    passes; turned back on, the same model retries the token and decodes on with logits
    bit-identical to the per-layer launches."""
    from dataclasses import replace
    import synth
    import axon_hip as H
    spec = replace(synth.CONFIGS["c4"], name="t-c4-giveup-2l", n_layer=2, n_vocab=2048, seed=41)
    path = synth.cached_model(spec, tmp_path_factory.mktemp("models"))
    a = hip(path, max_seq=32, max_ctx=64)
    b = hip(path, max_seq=32, max_ctx=64, persistent=False)
    assert a.info.persistent_decode == 1
    prompt = np.random.default_rng(9).integers(0, 2048, 12).astype(np.int32)
    ca, cb = a.new_cache(), b.new_cache()
    la, lb = a.forward_prefill(ca, prompt)[-1], b.forward_prefill(cb, prompt)[-1]
    assert np.array_equal(la, lb)
    t = int(np.argmax(la))
    lib = H.lib()
    n0 = len(prompt)
    # Logits copied to the host: the pass itself reports the give-up.
    try:
        assert lib.axon_hip_decode_layers_set_spin_limit(1) == 0
        assert lib.axon_hip_decode_layers_set_fail_waits(1) == 0
        with pytest.raises(H.HipError, match="gave up"):
            a.forward_prefill(ca, [t])
    finally:
        lib.axon_hip_decode_layers_set_fail_waits(0)
        lib.axon_hip_decode_layers_set_spin_limit(0)
    assert a.cache_pos(ca) == n0
    assert not a.persistent_decode()
    a.set_persistent_decode(True)
    assert a.persistent_decode()
    # Logits left in HBM: the pass returns with its cache advanced; the greedy choice's
    # synchronization finds the give-up and rolls the cache back.
    try:
        assert lib.axon_hip_decode_layers_set_spin_limit(1) == 0
        assert lib.axon_hip_decode_layers_set_fail_waits(1) == 0
        a.forward_prefill(ca, [t], logits=False)
    finally:
        lib.axon_hip_decode_layers_set_fail_waits(0)
        lib.axon_hip_decode_layers_set_spin_limit(0)
    assert a.cache_pos(ca) == n0 + 1
    with pytest.raises(H.HipError, match=f"gave up.*position {n0} of the cache in slot {ca}"):
        a.greedy(1)
    assert a.cache_pos(ca) == n0
    assert not a.persistent_decode()
    # Layer by layer now, then on the persistent kernel again: bit-identical throughout.
    for step in range(10):
        if step == 3:
            a.set_persistent_decode(True)
            assert a.persistent_decode()
        la, lb = a.forward_prefill(ca, [t])[0], b.forward_prefill(cb, [t])[0]
        assert np.array_equal(la, lb), f"step {step}"
        t = int(np.argmax(la))
    assert a.cache_pos(ca) == b.cache_pos(cb)
    a.close()
    b.close()

"""The fp16 key/value cache on the device (LoadOptions::cache = CacheType::F16; the rounding
in src/model/llama.cpp:520-563, the reads in attention_kv_heads_f16) against the oracle's fp16
cache, which tests/test_oracle_ref.py pins bit for bit to the reference's own LlamaModel loaded
with the F16 cache.

Patterned on the reference's tests/unit/test_model_cache_f16.cpp:
* the logits of the fp16 cache stay within the locked tolerance of the F32 cache (7e-3 of the
  logit range, test_model_cache_f16.cpp:61-85);
* the fp16 cache keeps its own identities: the same logits however the tokens are split into
  prefill chunks and single steps (test_model_cache_f16.cpp:87-106).
Beyond those: the cache bits against the oracle's (the rounding of every key and value, on
both cache-write paths: the RoPE kernel and the fused q|k|v epilogue), the logits against the
oracle's within the north star's 1e-4, batched rows against each sequence alone, and the
cache-free forward staying float (no cache, nothing rounded)."""
import ctypes as C

import numpy as np
import pytest

from helpers import GOLDEN, OracleModel, golden, oracle

pytestmark = pytest.mark.gpu

FIXTURES = ["synthetic-2l.gguf", "synthetic-2l-q8_0.gguf", "synthetic-2l-q4_0.gguf", "synthetic-2l-q4_1.gguf"]


def hip_model(path, **kw):
    import axon_hip as H
    return H.Model(path, **kw)


@pytest.fixture(scope="module")
def tokens():
    return golden("model/synthetic-2l.tokens.axt").ravel().astype(np.int32)


def stepped(m, tokens, prompt):
    """Prefill `prompt` tokens in max_seq chunks, then one token at a time (the reference's
    stepped(), test_model_cache_f16.cpp:35-50)."""
    c = m.new_cache()
    out = []
    for lo in range(0, prompt, m.info.max_seq):
        out.append(m.forward_prefill(c, tokens[lo:min(prompt, lo + m.info.max_seq)]))
    for t in tokens[prompt:]:
        out.append(m.forward_prefill(c, [t]))
    m.free_cache(c)
    return np.concatenate(out)


def oracle_stepped(o, tokens, prompt, chunk):
    c = o.new_cache(64, f16=True)
    out = []
    for lo in range(0, prompt, chunk):
        out.append(o.forward(tokens[lo:min(prompt, lo + chunk)], c))
    for t in tokens[prompt:]:
        out.append(o.forward(np.array([t], np.int32), c))
    return np.concatenate(out), c


def test_f16_cache_halves_the_pool():
    path = GOLDEN / "gguf" / "synthetic-2l.gguf"
    f32 = hip_model(path, max_seq=8, max_ctx=32)
    f16 = hip_model(path, max_seq=8, max_ctx=32, cache="f16")
    assert f32.info.cache_type == 0 and f16.info.cache_type == 1
    assert f16.info.kv_bytes_per_position * 2 == f32.info.kv_bytes_per_position
    with pytest.raises(ValueError):
        hip_model(path, cache="bf16")


@pytest.mark.parametrize("name", ["synthetic-2l.gguf", "synthetic-2l-q8_0.gguf", "synthetic-2l-q4_0.gguf"])
def test_f16_cache_bits_match_oracle(name, tokens):
    """Every cached key and value, widened back to float, equals the oracle's fp16 cache: a
    10-token prefill (the RoPE kernel's write, rows > 4) then single steps (the fused q|k|v
    epilogue's write on quantized weights)."""
    path = GOLDEN / "gguf" / name
    m = hip_model(path, max_seq=16, max_ctx=64, cache="f16")
    o = OracleModel(path)
    c = m.new_cache()
    m.forward_prefill(c, tokens[:10])
    for t in tokens[10:14]:
        m.forward_prefill(c, [t])
    _, oc = oracle_stepped(o, tokens[:14], 10, 16)
    row = o.cfg.n_head_kv * o.cfg.head_dim
    store = oc._store.reshape(o.cfg.n_layer, 2, 64, row)[:, :, :14]
    want = store.astype(np.uint16).view(np.float16).astype(np.float32)
    for layer in range(o.cfg.n_layer):
        for values in (0, 1):
            got = m.cache_rows(c, layer, bool(values), 14)
            np.testing.assert_array_equal(got.view(np.uint32), want[layer, values].view(np.uint32))


@pytest.mark.parametrize("name", FIXTURES)
def test_f16_cache_logits_match_oracle(name, tokens):
    path = GOLDEN / "gguf" / name
    m = hip_model(path, max_seq=8, max_ctx=64, cache="f16")
    got = stepped(m, tokens, 8)
    want, _ = oracle_stepped(OracleModel(path), tokens, 8, 8)
    # The north star's bar. The fp16 attention reads match the oracle's except where an exp or
    # the double softmax sum rounds differently in its last bit; on the float-weight model such
    # a bit spreads over the rest of its row's logits, hence the looser bit-equal fraction.
    assert np.max(np.abs(got - want)) <= 1e-4, np.max(np.abs(got - want))
    assert np.mean(got == want) > 0.95, np.mean(got == want)


def test_f16_cache_within_the_locked_tolerance_of_f32(tokens):
    """test_model_cache_f16.cpp:61-85: max |f16 - f32| over the F32 logits' range < 7e-3 (four
    times the reference's measurement on these models)."""
    worst = 0.0
    for name in ("synthetic-2l.gguf", "synthetic-2l-q8_0.gguf", "synthetic-2l-q4_0.gguf"):
        path = GOLDEN / "gguf" / name
        full = stepped(hip_model(path, max_seq=8, max_ctx=64), tokens, 8)
        half = stepped(hip_model(path, max_seq=8, max_ctx=64, cache="f16"), tokens, 8)
        worst = max(worst, float(np.max(np.abs(half - full)) / np.max(np.abs(full))))
    assert worst < 7e-3, worst
    assert worst > 0.0  # the rounding is there


@pytest.mark.parametrize("name", ["synthetic-2l.gguf", "synthetic-2l-q4_0.gguf"])
def test_f16_cache_keeps_its_identities(name, tokens):
    """test_model_cache_f16.cpp:87-106: the same bits with prompts of 8, 5 and 16 tokens
    (one chunk, a shorter chunk, two chunks of max_seq)."""
    m = hip_model(GOLDEN / "gguf" / name, max_seq=8, max_ctx=64, cache="f16")
    a = stepped(m, tokens, 8)
    assert np.array_equal(stepped(m, tokens, 5), a)
    assert np.array_equal(stepped(m, tokens, 16), a)


def test_f16_batched_rows_equal_each_sequence_alone(tokens):
    path = GOLDEN / "gguf" / "synthetic-2l-q4_0.gguf"
    m = hip_model(path, max_seq=32, max_ctx=64, max_batch=4, max_caches=8, cache="f16")
    lens = [3, 7, 11]
    caches = []
    for i, n in enumerate(lens):
        c = m.new_cache()
        m.forward_prefill(c, tokens[i:i + n])
        caches.append(c)
    nxt = np.array([tokens[20], tokens[21], tokens[22]], np.int32)
    batch = m.forward_batch(caches, nxt)
    alone = []
    for i, n in enumerate(lens):
        c = m.new_cache()
        m.forward_prefill(c, tokens[i:i + n])
        alone.append(m.forward_prefill(c, [nxt[i]])[0])
    assert np.array_equal(batch, np.stack(alone))
    # The oracle's forward_batch over fp16 caches.
    o = OracleModel(path)
    ocs = []
    for i, n in enumerate(lens):
        oc = o.new_cache(64, f16=True)
        o.forward(tokens[i:i + n], oc)
        ocs.append(oc)
    want = o.forward_batch(nxt, ocs)
    assert np.max(np.abs(batch - want)) <= 1e-4


def test_f16_model_cache_free_forward_stays_float(tokens):
    """llama.cpp:379-383: with no cache the keys and values stay in float, so the cache-free pass
    of an F16-cache model equals the F32 model's bit for bit."""
    path = GOLDEN / "gguf" / "synthetic-2l-q8_0.gguf"
    a = hip_model(path, max_seq=32, max_ctx=64).forward(tokens)
    b = hip_model(path, max_seq=32, max_ctx=64, cache="f16").forward(tokens)
    assert np.array_equal(a, b)


def test_rope_rows_rounds_special_values_into_an_f16_cache():
    """The RoPE kernel's cache write rounds each key and value once, as ora_fp32_to_fp16 does:
    round to nearest even, ties both ways, gradual underflow, overflow to infinity, signed zeros
    and NaN kept NaN."""
    import axon_hip as H
    n_kv, hd = 2, 64
    row = n_kv * hd
    specials = np.array([0.0, -0.0, 1.0, -1.0, 65504.0, 65519.99, 65520.0, 1e9, -1e9, np.inf, -np.inf, np.nan,
                         6.1035156e-05, 6.0975552e-05, 5.9604645e-08, 2.9802322e-08, 2.9802326e-08, 1e-10,
                         1.00048828125, 1.00146484375, 1.0009765625 + 2**-24, -3.1415927], np.float32)
    rng = np.random.default_rng(5)
    v = np.concatenate([specials, rng.standard_normal(row - len(specials)).astype(np.float32) * 1e3])
    v = v.astype(np.float32)[:row]
    k = rng.standard_normal(row).astype(np.float32)
    n_rows = 1
    cache = H.DeviceBuffer(2 * 4 * row * 2)  # [K, V] x 4 positions, fp16
    cache.upload(np.zeros(2 * 4 * row, np.uint16))
    dk, dv = H.DeviceBuffer.of(k), H.DeviceBuffer.of(v)
    ra = H.RopeRowsArgs(k=dk.ptr, v=dv.ptr, pos0=2, k_stride=row, n_kv=n_kv, head_dim=hd, rotary_dim=hd,
                        neox=0, theta=10000.0, cache=cache.ptr, k_layer_off=0, v_layer_off=4 * row, cache_f16=1)
    H.check(H.lib().axon_hip_rope_rows(C.byref(ra), C.c_size_t(n_rows)), "rope_rows")
    got = cache.download(np.uint16, 2 * 4 * row).reshape(2, 4, row)
    k_rot = dk.download(np.float32, row)
    f = oracle().ora_fp32_to_fp16
    want_v = np.array([f(float(x)) for x in v], np.uint16)
    want_k = np.array([f(float(x)) for x in k_rot], np.uint16)
    assert np.array_equal(got[1, 2], want_v)
    assert np.array_equal(got[0, 2], want_k)
    assert not got[:, [0, 1, 3]].any()  # only position 2 is written

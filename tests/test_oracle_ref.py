"""The C restatement against the reference's own code (oracle/_ref, compiled from
/root/reference/src): every table entry and the whole forward pass must agree bit for bit.
Skipped where oracle/_ref was not built (no reference checkout)."""
import numpy as np
import pytest

from helpers import GOLDEN, OracleModel, RefModel, golden, have_ref
from tables import CTable, QUANT_TYPES, random_floats, random_weights

pytestmark = pytest.mark.skipif(not have_ref(), reason="oracle/_ref not built (no reference checkout)")


@pytest.fixture(scope="module")
def both():
    return CTable("oracle"), CTable("ref")


def test_fp16_conversions_bit_exact(both):
    o, r = both
    for h in range(0, 65536, 7):
        a, b = o.lib.ora_fp16_to_fp32(h), r.lib.ref_fp16_to_fp32(h)
        assert a == b or (a != a and b != b)
    for x in random_floats(20000, 9, 70000.0):
        assert o.lib.ora_fp32_to_fp16(float(x)) == r.lib.ref_fp32_to_fp16(float(x))


@pytest.mark.parametrize("n_in", [32, 96, 576, 1536, 2048])
@pytest.mark.parametrize("n_out", [1, 7, 48])
def test_quantized_entries_bit_exact(both, n_in, n_out):
    o, r = both
    x = random_floats(n_in, n_in + 3, 4.0)
    xq = o.quantize_row_q8_0(x)
    assert xq.tobytes() == r.quantize_row_q8_0(x).tobytes()
    xs = random_floats(3 * n_in, n_in + 10, 4.0)
    xsq = np.concatenate([o.quantize_row_q8_0(xs[i * n_in:(i + 1) * n_in]) for i in range(3)])
    for kind in QUANT_TYPES:
        w = random_weights(kind, n_out, n_in, n_in * 11 + n_out)
        for args in ((xq,), ):
            a = o.matmul(f"{kind}_q8", w, *args, n_out, n_in)
            assert np.array_equal(a, r.matmul(f"{kind}_q8", w, *args, n_out, n_in)), kind
        a = o.matmul(f"{kind}_q8", w, xsq, n_out, n_in, n_rows=3, y_stride=n_out + 5)
        assert np.array_equal(a, r.matmul(f"{kind}_q8", w, xsq, n_out, n_in, n_rows=3, y_stride=n_out + 5))
        a = o.matmul(kind, w, x, n_out, n_in)
        assert np.array_equal(a, r.matmul(kind, w, x, n_out, n_in)), kind
        a = o.matmul(kind, w, xs, n_out, n_in, n_rows=3)
        assert np.array_equal(a, r.matmul(kind, w, xs, n_out, n_in, n_rows=3)), kind


@pytest.mark.parametrize("n_in", [256, 2048])
def test_q6_k_and_float_entries_bit_exact(both, n_in):
    o, r = both
    n_out = 9
    w6 = random_weights("q6_k", n_out, n_in, n_in)
    x = random_floats(n_in, 5)
    xs = random_floats(3 * n_in, 6)
    assert np.array_equal(o.matmul("q6_k", w6, x, n_out, n_in), r.matmul("q6_k", w6, x, n_out, n_in))
    assert np.array_equal(o.matmul("q6_k", w6, xs, n_out, n_in, n_rows=3),
                          r.matmul("q6_k", w6, xs, n_out, n_in, n_rows=3))
    wf = random_floats(n_out * n_in, 7)
    w16 = wf.astype(np.float16).view(np.uint16)
    wb = (wf.view(np.uint32) >> 16).astype(np.uint16)
    for kind, w in (("f32", wf), ("f16", w16), ("bf16", wb)):
        assert np.array_equal(o.matmul(kind, w, x, n_out, n_in), r.matmul(kind, w, x, n_out, n_in))
        assert np.array_equal(o.matmul(kind, w, xs, n_out, n_in, n_rows=3),
                              r.matmul(kind, w, xs, n_out, n_in, n_rows=3))


def test_elementwise_entries_bit_exact(both):
    o, r = both
    rng = np.random.default_rng(4)
    for n in (1, 37, 576, 2048, 8192):
        x = rng.normal(0, 2, n).astype(np.float32)
        w = (1 + rng.normal(0, 0.01, n)).astype(np.float32)
        assert np.array_equal(o.rmsnorm(x, w, 1e-5), r.rmsnorm(x, w, 1e-5))
        assert np.array_equal(o.softmax(x * 5), r.softmax(x * 5))
        assert np.array_equal(o.silu_mul(x, w), r.silu_mul(x, w))
    f = np.concatenate([np.ones(8), np.linspace(1.0, 32.0, 16), np.full(8, 32.0)]).astype(np.float32)
    for style, theta, factors in ((0, 10000.0, None), (1, 1e6, None), (0, 5e5, f)):
        for pos in (0, 1, 17, 1000, 4095, 131071):
            x = rng.normal(size=(8, 64)).astype(np.float32)
            assert np.array_equal(o.rope(x, 8, pos, 64, 64, theta, style, factors),
                                  r.rope(x, 8, pos, 64, 64, theta, style, factors))


@pytest.mark.parametrize("n_q,n_past", [(1, 0), (1, 200), (5, 37), (16, 100)])
def test_attention_entries_bit_exact(both, n_q, n_past):
    o, r = both
    rng = np.random.default_rng(n_q * 1000 + n_past)
    nh, nkv, hd = 8, 2, 64
    total = n_past + n_q
    q = rng.normal(size=(n_q, nh, hd)).astype(np.float32)
    k = rng.normal(size=(total, nkv, hd)).astype(np.float32)
    v = rng.normal(size=(total, nkv, hd)).astype(np.float32)
    s = 0.125
    assert np.array_equal(o.attention_kv_heads(q, k, v, n_q, n_past, nh, nkv, hd, s, 0, nh),
                          r.attention_kv_heads(q, k, v, n_q, n_past, nh, nkv, hd, s, 0, nh))
    k16, v16 = k.astype(np.float16).view(np.uint16), v.astype(np.float16).view(np.uint16)
    assert np.array_equal(o.attention_kv_heads(q, k16, v16, n_q, n_past, nh, nkv, hd, s, 2, 5, f16=True),
                          r.attention_kv_heads(q, k16, v16, n_q, n_past, nh, nkv, hd, s, 2, 5, f16=True))


def test_embedding_entries_bit_exact(both):
    o, r = both
    for kind, tid in (("q8_0", 8), ("q4_0", 2), ("q4_1", 3), ("q6_k", 14)):
        table = random_weights(kind, 12, 512, 3)
        for idx in (0, 5, 11):
            assert np.array_equal(o.embedding_row(tid, table, 512, idx), r.embedding_row(tid, table, 512, idx))


MODELS = ["synthetic-2l.gguf", "synthetic-2l-q8_0.gguf", "synthetic-2l-q4_0.gguf", "synthetic-2l-q4_1.gguf"]


@pytest.mark.parametrize("name", MODELS)
def test_model_forward_bit_exact_with_reference(name):
    path = GOLDEN / "gguf" / name
    tokens = golden("model/synthetic-2l.tokens.axt")
    om = OracleModel(path)
    rm = RefModel(path, max_seq=32, max_ctx=128, max_batch=4)
    full = om.forward(tokens)
    assert np.array_equal(full, rm.forward(tokens))
    # Prefill 8, then one token at a time, equals the cache-free pass (test_model_cached.cpp).
    oc = om.new_cache(128)
    rc = rm.new_cache()
    a = om.forward(tokens[:8], oc)
    b = rm.forward_prefill(rc, tokens[:8])
    assert np.array_equal(a, b) and np.array_equal(a, full[:8])
    for i in range(8, len(tokens)):
        a = om.forward(tokens[i:i + 1], oc)
        assert np.array_equal(a, rm.forward_prefill(rc, tokens[i:i + 1]))
        assert np.array_equal(a[0], full[i])
    # forward_batch over caches of different lengths equals decoding each alone.
    caches_o = [om.new_cache(128) for _ in range(3)]
    caches_r = [rm.new_cache() for _ in range(3)]
    for j, n in enumerate((3, 9, 14)):
        om.forward(tokens[:n], caches_o[j])
        rm.forward_prefill(caches_r[j], tokens[:n])
    nxt = np.array([tokens[3], tokens[9], tokens[14]], np.int32)
    a = om.forward_batch(nxt, caches_o)
    assert np.array_equal(a, rm.forward_batch(caches_r, nxt))
    for j, n in enumerate((3, 9, 14)):
        assert np.array_equal(a[j], full[n])


@pytest.mark.parametrize("name", MODELS)
def test_f16_cache_model_bit_exact_with_reference(name):
    """The oracle's fp16 cache (CacheType::F16: keys and values staged in float, rounded once
    into the cache, attention through attention_kv_heads_f16; llama.cpp:379-383, 520-590)
    against the reference's own LlamaModel loaded with LoadOptions::cache = F16: prefill
    chunks, single steps and a ragged forward_batch, bit for bit."""
    path = GOLDEN / "gguf" / name
    tokens = golden("model/synthetic-2l.tokens.axt")
    om = OracleModel(path)
    rm = RefModel(path, max_seq=32, max_ctx=128, max_batch=4, f16=True)
    # The cache-free pass keeps float keys and values (no cache, no rounding).
    assert np.array_equal(om.forward(tokens), rm.forward(tokens))
    oc = om.new_cache(128, f16=True)
    rc = rm.new_cache()
    for lo, hi in ((0, 5), (5, 8), (8, 9), (9, 16), (16, len(tokens))):
        assert np.array_equal(om.forward(tokens[lo:hi], oc), rm.forward_prefill(rc, tokens[lo:hi]))
    caches_o = [om.new_cache(128, f16=True) for _ in range(3)]
    caches_r = [rm.new_cache() for _ in range(3)]
    for j, n in enumerate((3, 9, 14)):
        om.forward(tokens[:n], caches_o[j])
        rm.forward_prefill(caches_r[j], tokens[:n])
    nxt = np.array([tokens[3], tokens[9], tokens[14]], np.int32)
    assert np.array_equal(om.forward_batch(nxt, caches_o), rm.forward_batch(caches_r, nxt))


def test_f16_cache_rounds_keys_and_values_once():
    """Layer 0's keys and values are computed from the same inputs with either cache, so the
    fp16 cache must hold exactly numpy's round-to-nearest-even fp16 of the F32 cache's rows (an
    independent restatement of the rounding), and nothing past the written positions."""
    path = GOLDEN / "gguf" / "synthetic-2l.gguf"
    tokens = golden("model/synthetic-2l.tokens.axt")[:6]
    om = OracleModel(path)
    c16 = om.new_cache(16, f16=True)
    c32 = om.new_cache(16)
    om.forward(tokens, c16)
    om.forward(tokens, c32)
    row = om.cfg.n_head_kv * om.cfg.head_dim
    f32 = c32._store.reshape(om.cfg.n_layer, 2, 16, row)
    f16 = c16._store.reshape(om.cfg.n_layer, 2, 16, row)
    assert np.array_equal(f16[0, :, :6], f32[0, :, :6].astype(np.float16).view(np.uint16))
    assert not f16[:, :, 6:].any()


def test_f32_model_matches_numpy_fixture():
    # tests/unit/test_model_forward.cpp:40-54
    om = OracleModel(GOLDEN / "gguf" / "synthetic-2l.gguf")
    for base in ("synthetic-2l", "synthetic-2l.short"):
        tokens = golden(f"model/{base}.tokens.axt")
        want = golden(f"model/{base}.logits.axt")
        assert np.max(np.abs(om.forward(tokens) - want)) < 1e-4


@pytest.mark.parametrize("cfg", ["c1", "c3", "c4", "c5"])
@pytest.mark.parametrize("f16", [False, True], ids=["f32cache", "f16cache"])
def test_oracle_model_bit_exact_with_reference_on_config_shapes(cfg, f16, tmp_path_factory):
    """The BASELINE model shapes at full width, two layers and a 4096-token vocabulary, through
    the oracle and the reference's own LlamaModel (scalar table): the cache-free pass, a prefill
    chunk then single cached steps, and a ragged forward_batch, bit for bit, with either cache
    type. This covers the paths the 2-layer fixtures do not: Q8_0 everywhere with 9/3 heads (C1);
    Q4_0 with a Q4_1 ffn_down, a Q4_0 embedding, an untied Q6_K output and a GQA group of 8 (C3);
    llama3 rope factors and a tied Q6_K embedding/output (C4); qwen2 Q/K/V bias, the NeoX layout
    and a Q8_0 output (C5)."""
    import synth
    from dataclasses import replace
    spec = replace(synth.CONFIGS[cfg], name=f"pin-{cfg}-2l", n_layer=2, n_vocab=4096, seed=21)
    path = synth.cached_model(spec, tmp_path_factory.getbasetemp() / "pin-models")
    toks = np.random.default_rng(7).integers(0, spec.n_vocab, 20).astype(np.int32)
    om = OracleModel(path)
    rm = RefModel(path, max_seq=32, max_ctx=64, max_batch=4, n_threads=4, f16=f16)
    full = om.forward(toks)
    assert np.array_equal(full, rm.forward(toks))
    oc = om.new_cache(64, f16=f16)
    rc = rm.new_cache()
    assert np.array_equal(om.forward(toks[:12], oc), rm.forward_prefill(rc, toks[:12]))
    for i in range(12, 16):
        assert np.array_equal(om.forward(toks[i:i + 1], oc), rm.forward_prefill(rc, toks[i:i + 1])), i
    lens = (2, 7, 13)
    caches_o = [om.new_cache(64, f16=f16) for _ in lens]
    caches_r = [rm.new_cache() for _ in lens]
    for j, n in enumerate(lens):
        om.forward(toks[:n], caches_o[j])
        rm.forward_prefill(caches_r[j], toks[:n])
    nxt = np.array([toks[n] for n in lens], np.int32)
    assert np.array_equal(om.forward_batch(nxt, caches_o), rm.forward_batch(caches_r, nxt))

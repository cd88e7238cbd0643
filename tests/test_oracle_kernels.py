"""Pins the oracle's float kernels against the reference's NumPy float64 fixtures
(tests/golden/kernels) and closed forms, mirroring the reference's
test_kernels_{matmul,norm_act,rope,attention}.cpp."""
import numpy as np
import pytest

from helpers import golden
from tables import CTable


@pytest.fixture(scope="module")
def o():
    return CTable("oracle")


def f16_bits_to_f32(bits):
    return bits.view(np.float16).astype(np.float32)


@pytest.mark.parametrize("name", ["matmul_f32", "matmul_f32_odd", "matmul_f16", "matmul_bf16"])
def test_float_matmul_fixtures(o, name):
    w = golden(f"kernels/{name}.w.axt")
    x = golden(f"kernels/{name}.x.axt")
    want = golden(f"kernels/{name}.y.axt")
    kind = name.split("_")[1]
    n_out, n_in = w.shape
    y = o.matmul(kind, np.ascontiguousarray(w), x, n_out, n_in)
    assert np.max(np.abs(y - want)) < 1e-5
    if name != "matmul_f32_odd":
        xs = golden(f"kernels/{name}_rows.x.axt")
        ys = o.matmul(kind, np.ascontiguousarray(w), xs, n_out, n_in, n_rows=xs.shape[0])
        assert np.max(np.abs(ys - golden(f"kernels/{name}_rows.y.axt").ravel())) < 1e-5


def test_single_output_matmul_is_a_dot_product(o):
    w = np.array([1.0, 2.0, 3.0, 4.0, 5.0], np.float32)
    x = np.array([0.5, -1.0, 2.0, 0.0, 1.0], np.float32)
    assert o.matmul("f32", w, x, 1, 5)[0] == np.float32(0.5 - 2.0 + 6.0 + 5.0)


@pytest.mark.parametrize("n", [1, 64])
def test_rmsnorm_fixtures(o, n):
    x, w, want = (golden(f"kernels/rmsnorm_{n}.{s}.axt") for s in ("x", "w", "y"))
    assert np.max(np.abs(o.rmsnorm(x, w, 1e-5) - want)) < 1e-5


def test_rmsnorm_of_constant_is_weight(o):
    w = (np.arange(37) - 10).astype(np.float32)
    assert np.max(np.abs(o.rmsnorm(np.full(37, 4.5, np.float32), w, 0.0) - w)) < 1e-5


@pytest.mark.parametrize("n", [1, 5, 64])
def test_softmax_fixtures(o, n):
    x, want = golden(f"kernels/softmax_{n}.x.axt"), golden(f"kernels/softmax_{n}.y.axt")
    y = o.softmax(x)
    assert np.max(np.abs(y - want)) < 1e-5
    assert abs(float(np.sum(y.astype(np.float64))) - 1.0) < 1e-6


def test_silu_mul(o):
    g, u, want = (golden(f"kernels/silu_mul.{s}.axt") for s in ("gate", "up", "out"))
    assert np.max(np.abs(o.silu_mul(g, u) - want)) < 1e-5
    out = o.silu_mul(np.array([0.0, 40.0, -40.0], np.float32), np.array([7.0, 2.0, 2.0], np.float32))
    assert out[0] == 0.0 and abs(out[1] - 80.0) < 1e-4 and abs(out[2]) < 1e-6


@pytest.mark.parametrize("name,style,theta,factors", [
    ("rope_normal", 0, 10000.0, False), ("rope_neox", 1, 1000000.0, False), ("rope_llama3", 0, 500000.0, True),
])
def test_rope_fixtures(o, name, style, theta, factors):
    x = golden(f"kernels/{name}.x.axt")
    pos = golden(f"kernels/{name}.pos.axt")
    want = golden(f"kernels/{name}.y.axt")
    f = golden(f"kernels/{name}.factors.axt") if factors else None
    n_heads, hd = x.shape[1], x.shape[2]
    got = np.stack([o.rope(x[i], n_heads, int(pos[i]), hd, hd, theta, style, f) for i in range(len(pos))])
    assert np.max(np.abs(got - want)) < 1e-5


def test_rope_position_zero_is_identity_and_preserves_norms(o):
    x = golden("kernels/rope_normal.x.axt")[0]
    for style in (0, 1):
        assert np.array_equal(o.rope(x, x.shape[0], 0, x.shape[1], x.shape[1], 10000.0, style), x)
        y = o.rope(x, x.shape[0], 4095, x.shape[1], x.shape[1], 10000.0, style)
        assert np.allclose(np.linalg.norm(y, axis=1), np.linalg.norm(x, axis=1), rtol=1e-5)


SHAPES = [("attention_s1_h2_kv1_d8", 1, 2, 1, 8), ("attention_s5_h2_kv1_d8", 5, 2, 1, 8),
          ("attention_s8_h4_kv2_d16", 8, 4, 2, 16)]


@pytest.mark.parametrize("name,seq,nh,nkv,hd", SHAPES)
def test_attention_fixtures(o, name, seq, nh, nkv, hd):
    q, k, v, want = (golden(f"kernels/{name}.{s}.axt") for s in ("q", "k", "v", "out"))
    scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
    out = o.attention_kv_heads(q, k, v, seq, 0, nh, nkv, hd, scale, 0, nh)
    assert np.max(np.abs(out.ravel() - want.ravel())) < 1e-5


def test_attention_gqa_equals_mha_and_cache_growth(o):
    name, seq, nh, nkv, hd = SHAPES[2]
    q, k, v = (golden(f"kernels/{name}.{s}.axt") for s in ("q", "k", "v"))
    scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
    gqa = o.attention_kv_heads(q, k, v, seq, 0, nh, nkv, hd, scale, 0, nh)
    rep = lambda t: np.repeat(t.reshape(seq, nkv, hd), nh // nkv, axis=1)  # noqa: E731
    mha = o.attention_kv_heads(q, rep(k), rep(v), seq, 0, nh, nh, hd, scale, 0, nh)
    assert np.array_equal(gqa, mha)
    # One query row at a time over a growing cache gives the full pass bit for bit.
    qq = q.reshape(seq, nh, hd)
    for i in range(seq):
        step = o.attention_kv_heads(qq[i:i + 1], k, v, 1, i, nh, nkv, hd, scale, 0, nh)
        assert np.array_equal(step[0], gqa.reshape(seq, nh, hd)[i])


def test_attention_over_one_position_returns_its_value(o):
    rng = np.random.default_rng(3)
    nh, nkv, hd = 4, 2, 8
    q = rng.normal(size=(1, nh, hd)).astype(np.float32)
    k = rng.normal(size=(1, nkv, hd)).astype(np.float32)
    v = rng.normal(size=(1, nkv, hd)).astype(np.float32)
    out = o.attention_kv_heads(q, k, v, 1, 0, nh, nkv, hd, 0.35, 0, nh)
    for h in range(nh):
        assert np.array_equal(out[0, h], v[0, h // 2])

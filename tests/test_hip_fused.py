"""axon_hip_matvec_fused, the decode matvec with its neighbours folded in, against the separate
entries it replaces in the forward pass and against the oracle.

The fused launch must agree bit for bit with the unfused sequence (rmsnorm_rows or
quantize_rows_q8_0, then matmul_q8_fused, then rope_rows / silu_mul_rows / the residual add),
because a sequence decoded alone (fused) and inside a larger batch (unfused) has to produce the
same tokens. Against the oracle, the integer-exact parts are bit-exact; SiLU's exp is held to
2 ulp of the product. Shapes cover the models' widths (576, 896, 2048 inputs; 8192 for
the down projection), ragged output counts and 1..4 rows."""
import ctypes as C

import numpy as np
import pytest

from tables import CTable, HipTable, random_floats, random_weights

pytestmark = pytest.mark.gpu

TYPE_ID = {"q8_0": 8, "q4_0": 2, "q4_1": 3}
KINDS = tuple(TYPE_ID)


@pytest.fixture(scope="module")
def o():
    return CTable("oracle")


@pytest.fixture(scope="module")
def H():
    HipTable()
    import axon_hip
    return axon_hip


def ulp_diff(a, b):
    a = np.ascontiguousarray(a, np.float32).view(np.int32).astype(np.int64)
    b = np.ascontiguousarray(b, np.float32).view(np.int32).astype(np.int64)
    a = np.where(a < 0, -(a & 0x7fffffff), a)
    b = np.where(b < 0, -(b & 0x7fffffff), b)
    return int(np.max(np.abs(a - b))) if a.size else 0


def supported(H, kind, in_mode, n_rows, n_in, silu=False):
    return H.lib().axon_hip_matvec_fused_supported(C.c_int(TYPE_ID[kind]), C.c_int(in_mode), C.c_size_t(n_rows),
                                                   C.c_size_t(n_in), C.c_int(int(silu))) == 1


def fused(H, **kw):
    a = H.MatvecFusedArgs()
    for k, v in kw.items():
        if k in ("w", "y", "bias"):
            arr = getattr(a, k)
            for i, b in enumerate(v):
                arr[i] = H.ptr_of(b)
        elif k in ("n_out", "y_stride"):
            arr = getattr(a, k)
            for i, b in enumerate(v):
                arr[i] = b
        elif isinstance(v, H.DeviceBuffer):
            setattr(a, k, v.ptr)
        else:
            setattr(a, k, v)
    H.check(H.lib().axon_hip_matvec_fused(C.byref(a)), "matvec_fused")


def unfused_matmul(H, kind, xq, n_rows, n_in, ws, ys, n_out, y_stride, accumulate):
    n = len(ws)
    w_arr = (C.c_void_p * n)(*[b.ptr for b in ws])
    y_arr = (C.c_void_p * n)(*[b.ptr for b in ys])
    no = (C.c_size_t * n)(*n_out)
    st = (C.c_size_t * n)(*y_stride)
    H.check(H.lib().axon_hip_matmul_q8_fused(C.c_int(TYPE_ID[kind]), C.c_void_p(xq.ptr), C.c_size_t(n_rows),
                                             C.c_size_t(n_in), C.c_size_t(n), w_arr, y_arr, no, st,
                                             C.c_int(int(accumulate))), "matmul_q8_fused")


def oracle_rows(o, kind, w, x_rows, n_out, n_in):
    """Quantize each row with quantize_row_q8_0 and run the Q8_0-activation matmul row by row."""
    return np.stack([o.matmul(f"{kind}_q8", w, o.quantize_row_q8_0(r), n_out, n_in) for r in x_rows])


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("n_rows", [1, 2, 3, 4])
@pytest.mark.parametrize("n_in,n_out", [(576, 7), (896, 300), (2048, 2048), (2048, 1153)])
def test_norm_store_matches_unfused_and_oracle(H, o, kind, n_rows, n_in, n_out):
    """in_mode 2 / out_mode 0: RMSNorm, quantize and matvec (the output head, llama.cpp:630-634)."""
    if not supported(H, kind, 2, n_rows, n_in):
        pytest.skip("shape outside the fused kernel")
    eps = 1e-5
    x = random_floats(n_rows * n_in, n_in + n_rows, 3.0).reshape(n_rows, n_in)
    g = random_floats(n_in, n_in + 1, 1.0)
    w = random_weights(kind, n_out, n_in, n_out + n_rows)
    dx, dg, dw = H.DeviceBuffer.of(x), H.DeviceBuffer.of(g), H.DeviceBuffer.of(w)
    y = H.DeviceBuffer.of(np.full((n_rows, n_out + 5), -3.5, np.float32))
    fused(H, type=TYPE_ID[kind], n_seg=1, w=[dw], n_out=[n_out], n_rows=n_rows, n_in=n_in, in_mode=2, x=dx,
          x_stride=n_in, norm_w=dg, eps=eps, out_mode=0, y=[y], y_stride=[n_out + 5])
    got = y.download(np.float32).reshape(n_rows, n_out + 5)
    assert np.all(got[:, n_out:] == np.float32(-3.5))
    xq = H.DeviceBuffer(n_rows * n_in // 32 * 34)
    H.call("rmsnorm_rows", dx, dg, None, xq, n_in, n_rows, eps)
    y2 = H.DeviceBuffer.of(np.zeros((n_rows, n_out), np.float32))
    unfused_matmul(H, kind, xq, n_rows, n_in, [dw], [y2], [n_out], [n_out], False)
    assert np.array_equal(got[:, :n_out], y2.download(np.float32).reshape(n_rows, n_out))
    normed = np.stack([o.rmsnorm(r, g, eps) for r in x])
    assert np.array_equal(got[:, :n_out], oracle_rows(o, kind, w, normed, n_out, n_in))


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("n_rows", [1, 2, 4])
@pytest.mark.parametrize("n_in,n_out,x_stride", [(576, 576, 576), (2048, 2048, 2052), (8192, 2048, 8192),
                                                  (4864, 896, 4868), (64, 3, 64)])
def test_float_add_matches_unfused_and_oracle(H, o, kind, n_rows, n_in, n_out, x_stride):
    """in_mode 1 / out_mode 1: quantize float rows (strided), matvec, residual add (the wo and
    down projections, llama.cpp:594-595, 621-623)."""
    if not supported(H, kind, 1, n_rows, n_in):
        pytest.skip("shape outside the fused kernel")
    x = np.zeros((n_rows, x_stride), np.float32)
    x[:, :n_in] = random_floats(n_rows * n_in, n_in * 3 + n_rows, 2.0).reshape(n_rows, n_in)
    x[:, n_in:] = np.nan                   # padding between rows is never read
    res = random_floats(n_rows * n_out, n_out + 11, 1.0).reshape(n_rows, n_out)
    w = random_weights(kind, n_out, n_in, n_in + n_out + n_rows)
    dx, dw = H.DeviceBuffer.of(x), H.DeviceBuffer.of(w)
    y = H.DeviceBuffer.of(res)
    fused(H, type=TYPE_ID[kind], n_seg=1, w=[dw], n_out=[n_out], n_rows=n_rows, n_in=n_in, in_mode=1, x=dx,
          x_stride=x_stride, out_mode=1, y=[y], y_stride=[n_out])
    got = y.download(np.float32).reshape(n_rows, n_out)
    xq = H.DeviceBuffer(n_rows * n_in // 32 * 34)
    H.call("quantize_rows_q8_0", dx, xq, n_in, n_rows, x_stride)
    y2 = H.DeviceBuffer.of(res)
    unfused_matmul(H, kind, xq, n_rows, n_in, [dw], [y2], [n_out], [n_out], True)
    assert np.array_equal(got, y2.download(np.float32).reshape(n_rows, n_out))
    want = res + oracle_rows(o, kind, w, x[:, :n_in], n_out, n_in)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("n_rows", [1, 2, 4])
@pytest.mark.parametrize("n_in,ff", [(576, 1536), (2048, 8192), (896, 4864), (96, 5)])
def test_norm_silu_matches_unfused(H, o, kind, n_rows, n_in, ff):
    """in_mode 2 / out_mode 2: ffn_norm, quantize, gate and up in one workgroup, SiLU(gate) * up
    (llama.cpp:598-620)."""
    if not supported(H, kind, 2, n_rows, n_in, silu=True):
        pytest.skip("shape outside the fused kernel")
    eps = 1e-6
    x = random_floats(n_rows * n_in, ff + n_rows, 2.0).reshape(n_rows, n_in)
    g = random_floats(n_in, n_in + 5, 1.0)
    wg = random_weights(kind, ff, n_in, ff + 1)
    wu = random_weights(kind, ff, n_in, ff + 2)
    dx, dg, dwg, dwu = (H.DeviceBuffer.of(a) for a in (x, g, wg, wu))
    h = H.DeviceBuffer.of(np.full((n_rows, ff), -1.0, np.float32))
    fused(H, type=TYPE_ID[kind], n_seg=2, w=[dwg, dwu], n_out=[ff, ff], n_rows=n_rows, n_in=n_in, in_mode=2, x=dx,
          x_stride=n_in, norm_w=dg, eps=eps, out_mode=2, y=[h], y_stride=[ff])
    got = h.download(np.float32).reshape(n_rows, ff)
    xq = H.DeviceBuffer(n_rows * n_in // 32 * 34)
    H.call("rmsnorm_rows", dx, dg, None, xq, n_in, n_rows, eps)
    gate, up = (H.DeviceBuffer(n_rows * ff * 4) for _ in range(2))
    unfused_matmul(H, kind, xq, n_rows, n_in, [dwg, dwu], [gate, up], [ff, ff], [ff, ff], False)
    out = H.DeviceBuffer(n_rows * ff * 4)
    H.call("silu_mul_rows", gate, up, out, None, ff, n_rows)
    assert np.array_equal(got, out.download(np.float32).reshape(n_rows, ff))
    normed = np.stack([o.rmsnorm(r, g, eps) for r in x])
    og = oracle_rows(o, kind, wg, normed, ff, n_in)
    ou = oracle_rows(o, kind, wu, normed, ff, n_in)
    assert np.array_equal(gate.download(np.float32).reshape(n_rows, ff), og)
    want = np.stack([o.silu_mul(og[i], ou[i]) for i in range(n_rows)])
    assert np.array_equal(got, want)


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("n_rows", [1, 2, 4])
@pytest.mark.parametrize("n_in,ff", [(576, 1536), (2048, 8192), (896, 4864)])
def test_silu_q8_output_feeds_down(H, o, kind, n_rows, n_in, ff):
    """The SiLU epilogue's Q8_0 output (outq): byte-identical to quantize_rows_q8_0 of its own
    float output, with the float output unchanged; down over those blocks (in_mode 0) gives the
    bits of down over the floats (in_mode 1), the residual add included."""
    if not supported(H, kind, 2, n_rows, n_in, silu=True) or not supported(H, kind, 0, n_rows, ff):
        pytest.skip("shape outside the fused kernel")
    eps = 1e-6
    x = random_floats(n_rows * n_in, ff + 3 * n_rows, 2.0).reshape(n_rows, n_in)
    g = random_floats(n_in, n_in + 6, 1.0)
    wg = random_weights(kind, ff, n_in, ff + 3)
    wu = random_weights(kind, ff, n_in, ff + 4)
    dx, dg, dwg, dwu = (H.DeviceBuffer.of(a) for a in (x, g, wg, wu))
    args = dict(type=TYPE_ID[kind], n_seg=2, w=[dwg, dwu], n_out=[ff, ff], n_rows=n_rows, n_in=n_in, in_mode=2,
                x=dx, x_stride=n_in, norm_w=dg, eps=eps, out_mode=2, y_stride=[ff])
    h_plain = H.DeviceBuffer.of(np.full((n_rows, ff), -1.0, np.float32))
    fused(H, y=[h_plain], **args)
    h = H.DeviceBuffer.of(np.full((n_rows, ff), -1.0, np.float32))
    hq = H.DeviceBuffer.of(np.full(n_rows * ff // 32 * 34 + 34, 0x5A, np.uint8))
    try:
        fused(H, y=[h], outq=hq, **args)
    except H.HipError as e:
        # 32 rows of gate and up per workgroup: Q8_0 weights at several rows exceed LDS; the
        # model then hands h to down as floats.
        assert "exceed LDS" in str(e)
        pytest.skip("32-row gate|up tile does not fit LDS for this type and row count")
    hf = h.download(np.float32).reshape(n_rows, ff)
    assert np.array_equal(hf, h_plain.download(np.float32).reshape(n_rows, ff))
    ref_q = H.DeviceBuffer(n_rows * ff // 32 * 34)
    H.call("quantize_rows_q8_0", h, ref_q, ff, n_rows, ff)
    got_q = hq.download(np.uint8)
    assert got_q[:n_rows * ff // 32 * 34].tobytes() == ref_q.download(np.uint8).tobytes()
    assert np.all(got_q[n_rows * ff // 32 * 34:] == 0x5A)      # nothing past the blocks
    assert got_q[:ff // 32 * 34].tobytes() == o.quantize_row_q8_0(hf[0]).tobytes()
    # down: 2048 or the model width outputs, residual add, from the blocks and from the floats
    d = n_in
    wd = random_weights(kind, d, ff, d + ff)
    dwd = H.DeviceBuffer.of(wd)
    res = random_floats(n_rows * d, d + 9, 1.0).reshape(n_rows, d)
    y_q, y_f = H.DeviceBuffer.of(res), H.DeviceBuffer.of(res)
    fused(H, type=TYPE_ID[kind], n_seg=1, w=[dwd], n_out=[d], n_rows=n_rows, n_in=ff, in_mode=0, xq=hq,
          out_mode=1, y=[y_q], y_stride=[d])
    fused(H, type=TYPE_ID[kind], n_seg=1, w=[dwd], n_out=[d], n_rows=n_rows, n_in=ff, in_mode=1, x=h,
          x_stride=ff, out_mode=1, y=[y_f], y_stride=[d])
    assert np.array_equal(y_q.download(np.float32), y_f.download(np.float32))


def test_q8_output_needs_silu_and_whole_blocks(H):
    dw = H.DeviceBuffer(64 * 34)
    y, q = H.DeviceBuffer(256), H.DeviceBuffer(256)
    with pytest.raises(H.HipError):
        fused(H, type=TYPE_ID["q8_0"], n_seg=1, w=[dw], n_out=[64], n_rows=1, n_in=32, in_mode=0, xq=q,
              out_mode=0, y=[y], y_stride=[64], outq=q)
    with pytest.raises(H.HipError):
        fused(H, type=TYPE_ID["q8_0"], n_seg=2, w=[dw, dw], n_out=[40, 40], n_rows=1, n_in=32, in_mode=0, xq=q,
              out_mode=2, y=[y], y_stride=[40], outq=q)


def rope_table(max_pos, rotary_dim, theta):
    i = np.arange(rotary_dim // 2, dtype=np.float64)
    inv = np.power(np.float64(theta), -2.0 * i / rotary_dim)
    ang = np.arange(max_pos, dtype=np.float64)[:, None] * inv[None, :]
    t = np.stack([np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)], axis=-1)
    return np.ascontiguousarray(t)


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("n_rows", [1, 2, 3, 4])
@pytest.mark.parametrize("d,n_head,n_kv,hd,rot,bias", [(576, 9, 3, 64, 64, False), (2048, 32, 8, 64, 64, False),
                                                       (896, 14, 2, 64, 64, True), (256, 4, 2, 64, 32, True)])
def test_norm_qkv_rope_matches_unfused(H, o, kind, n_rows, d, n_head, n_kv, hd, rot, bias):
    """in_mode 2 / out_mode 3: attn_norm, quantize, q|k|v, bias, Normal-style RoPE, q out and
    k, v into each row's cache slot at its own position (llama.cpp:493-537), against rmsnorm_rows
    + matmul_q8_fused + rope_rows over the same pool."""
    if not supported(H, kind, 2, n_rows, d):
        pytest.skip("shape outside the fused kernel")
    eps = 1e-5
    dq, dkv = n_head * hd, n_kv * hd
    max_ctx = 40
    rng = np.random.default_rng(d + n_rows + rot)
    x = random_floats(n_rows * d, d + n_rows * 7, 2.0).reshape(n_rows, d)
    g = random_floats(d, d + 9, 1.0)
    ws = [random_weights(kind, n, d, n + d + s) for s, n in enumerate((dq, dkv, dkv))]
    bs = [random_floats(n, n + s, 0.5) for s, n in enumerate((dq, dkv, dkv))] if bias else [None] * 3
    pos = rng.integers(0, max_ctx, n_rows).astype(np.int32)
    slot = 2 * 3 * max_ctx * dkv                       # three layers of K and V rows per slot
    coff = (rng.permutation(n_rows + 1)[:n_rows] * slot).astype(np.int64)
    layer = 1
    k_layer, v_layer = 2 * layer * max_ctx * dkv, (2 * layer + 1) * max_ctx * dkv
    pool0 = rng.normal(0, 1, (n_rows + 1) * slot).astype(np.float32)
    table = rope_table(max_ctx, rot, 10000.0)
    dx, dg, dtab, dpos, dcoff = (H.DeviceBuffer.of(a) for a in (x, g, table, pos, coff))
    dws = [H.DeviceBuffer.of(w) for w in ws]
    dbs = [H.DeviceBuffer.of(b) if b is not None else None for b in bs]
    pool = H.DeviceBuffer.of(pool0)
    q = H.DeviceBuffer.of(np.zeros((n_rows, dq), np.float32))
    fused(H, type=TYPE_ID[kind], n_seg=3, w=dws, n_out=[dq, dkv, dkv], n_rows=n_rows, n_in=d, in_mode=2, x=dx,
          x_stride=d, norm_w=dg, eps=eps, out_mode=3, y=[q], y_stride=[dq], bias=dbs, rope_table=dtab,
          rot_half=rot // 2, head_dim=hd, pos=dpos, cache_off=dcoff, cache=pool, k_layer_off=k_layer,
          v_layer_off=v_layer)
    got_q = q.download(np.float32).reshape(n_rows, dq)
    got_pool = pool.download(np.float32)

    xq = H.DeviceBuffer(n_rows * d // 32 * 34)
    H.call("rmsnorm_rows", dx, dg, None, xq, d, n_rows, eps)
    q2, k2, v2 = (H.DeviceBuffer(n_rows * n * 4) for n in (dq, dkv, dkv))
    unfused_matmul(H, kind, xq, n_rows, d, dws, [q2, k2, v2], [dq, dkv, dkv], [dq, dkv, dkv], False)
    pool2 = H.DeviceBuffer.of(pool0)
    ra = H.RopeRowsArgs(q=q2.ptr, k=k2.ptr, v=v2.ptr, bq=H.ptr_of(dbs[0]), bk=H.ptr_of(dbs[1]), bv=H.ptr_of(dbs[2]),
                        pos=dpos.ptr, pos0=0, q_stride=dq, k_stride=dkv, n_head=n_head, n_kv=n_kv, head_dim=hd,
                        rotary_dim=rot, neox=0, theta=10000.0, freq_factors=0, table=dtab.ptr, cache=pool2.ptr,
                        cache_off=dcoff.ptr, k_layer_off=k_layer, v_layer_off=v_layer)
    H.check(H.lib().axon_hip_rope_rows(C.byref(ra), C.c_size_t(n_rows)), "rope_rows")
    assert np.array_equal(got_q, q2.download(np.float32).reshape(n_rows, dq))
    assert np.array_equal(got_pool, pool2.download(np.float32))
    # Only the rows' own K and V rows at their positions changed.
    changed = np.flatnonzero(got_pool != pool0)
    allowed = np.concatenate([c + lo + p * dkv + np.arange(dkv) for c, p in zip(coff, pos)
                              for lo in (k_layer, v_layer)])
    assert np.isin(changed, allowed).all()
    # q against the oracle: rmsnorm, quantize, matmul, bias, rope (src/kernels/ref/rope.cpp).
    normed = np.stack([o.rmsnorm(r, g, eps) for r in x])
    oq = oracle_rows(o, kind, ws[0], normed, dq, d)
    if bias:
        oq = oq + bs[0]
    for i in range(n_rows):
        want = o.rope(oq[i], n_head, int(pos[i]), hd, rot, 10000.0, 0)
        assert np.max(np.abs(got_q[i] - want)) <= 2e-6 * max(1.0, float(np.max(np.abs(want)))), i


def quantized_rows(o, x_rows):
    return np.concatenate([o.quantize_row_q8_0(r) for r in x_rows])


def qkv_rope(H, **kw):
    a = H.MatvecFusedArgs()
    for k, v in kw.items():
        if k in ("w", "y", "bias"):
            arr = getattr(a, k)
            for i, b in enumerate(v):
                arr[i] = H.ptr_of(b)
        elif k in ("n_out", "y_stride"):
            arr = getattr(a, k)
            for i, b in enumerate(v):
                arr[i] = b
        elif isinstance(v, H.DeviceBuffer):
            setattr(a, k, v.ptr)
        else:
            setattr(a, k, v)
    H.check(H.lib().axon_hip_matmul_q8_qkv_rope(C.byref(a)), "matmul_q8_qkv_rope")


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("n_rows", [1, 5, 16, 17, 33, 64])
@pytest.mark.parametrize("d,n_head,n_kv,hd,rot,bias", [(2048, 32, 8, 64, 64, False), (896, 14, 2, 64, 64, True),
                                                       (256, 4, 2, 64, 32, True)])
@pytest.mark.parametrize("f16", [0, 1])
def test_rows_qkv_rope_matches_unfused(H, o, kind, n_rows, d, n_head, n_kv, hd, rot, bias, f16):
    """axon_hip_matmul_q8_qkv_rope: q|k|v of 1..64 Q8_0 rows on the MFMA rows kernel with the
    bias, Normal-style RoPE and the KV write in its epilogue, against matmul_q8_fused + rope_rows
    over the same pool, bit for bit, with a float and an fp16 cache (workgroups of 8 and of 16
    weight rows both occur: the narrow form below 256 workgroups); q also against the oracle."""
    dq, dkv = n_head * hd, n_kv * hd
    max_ctx = 40
    rng = np.random.default_rng(d + n_rows + rot + 7 * f16)
    x = random_floats(n_rows * d, d + n_rows * 5, 2.0).reshape(n_rows, d)
    dxq = H.DeviceBuffer.of(quantized_rows(o, x))
    ws = [random_weights(kind, n, d, n + d + s + 1) for s, n in enumerate((dq, dkv, dkv))]
    bs = [random_floats(n, n + s + 2, 0.5) for s, n in enumerate((dq, dkv, dkv))] if bias else [None] * 3
    pos = rng.integers(0, max_ctx, n_rows).astype(np.int32)
    slot = 2 * 3 * max_ctx * dkv
    coff = (rng.permutation(n_rows + 1)[:n_rows] * slot).astype(np.int64)
    k_layer, v_layer = 2 * max_ctx * dkv, 3 * max_ctx * dkv
    if f16:
        pool0 = rng.integers(0, 0x7bff, (n_rows + 1) * slot).astype(np.uint16)
    else:
        pool0 = rng.normal(0, 1, (n_rows + 1) * slot).astype(np.float32)
    table = rope_table(max_ctx, rot, 10000.0)
    dtab, dpos, dcoff = (H.DeviceBuffer.of(a) for a in (table, pos, coff))
    dws = [H.DeviceBuffer.of(w) for w in ws]
    dbs = [H.DeviceBuffer.of(b) if b is not None else None for b in bs]
    pool, pool2 = H.DeviceBuffer.of(pool0), H.DeviceBuffer.of(pool0)
    q = H.DeviceBuffer.of(np.full((n_rows, dq + 3), -1.0, np.float32))
    qkv_rope(H, type=TYPE_ID[kind], n_seg=3, w=dws, n_out=[dq, dkv, dkv], n_rows=n_rows, n_in=d, in_mode=0, xq=dxq,
             out_mode=3, y=[q], y_stride=[dq + 3], bias=dbs, rope_table=dtab, rot_half=rot // 2, head_dim=hd,
             pos=dpos, cache_off=dcoff, cache=pool, cache_f16=f16, k_layer_off=k_layer, v_layer_off=v_layer)
    got_q = q.download(np.float32).reshape(n_rows, dq + 3)
    assert (got_q[:, dq:] == -1.0).all()  # the stride's padding is not written
    got_q = got_q[:, :dq]

    q2, k2, v2 = (H.DeviceBuffer(n_rows * n * 4) for n in (dq, dkv, dkv))
    unfused_matmul(H, kind, dxq, n_rows, d, dws, [q2, k2, v2], [dq, dkv, dkv], [dq, dkv, dkv], False)
    ra = H.RopeRowsArgs(q=q2.ptr, k=k2.ptr, v=v2.ptr, bq=H.ptr_of(dbs[0]), bk=H.ptr_of(dbs[1]), bv=H.ptr_of(dbs[2]),
                        pos=dpos.ptr, pos0=0, q_stride=dq, k_stride=dkv, n_head=n_head, n_kv=n_kv, head_dim=hd,
                        rotary_dim=rot, neox=0, theta=10000.0, freq_factors=0, table=dtab.ptr, cache=pool2.ptr,
                        cache_off=dcoff.ptr, k_layer_off=k_layer, v_layer_off=v_layer, cache_f16=f16)
    H.check(H.lib().axon_hip_rope_rows(C.byref(ra), C.c_size_t(n_rows)), "rope_rows")
    assert np.array_equal(got_q.view(np.uint32), q2.download(np.uint32).reshape(n_rows, dq))
    dt = np.uint16 if f16 else np.uint32
    got_pool, want_pool = pool.download(dt), pool2.download(dt)
    assert np.array_equal(got_pool, want_pool)
    changed = np.flatnonzero(got_pool != pool0.view(dt))
    allowed = np.concatenate([c + lo + p * dkv + np.arange(dkv) for c, p in zip(coff, pos) for lo in (k_layer, v_layer)])
    assert np.isin(changed, allowed).all()
    if n_rows <= 17:
        oq = oracle_rows(o, kind, ws[0], x, dq, d)
        if bias:
            oq = oq + bs[0]
        for i in range(n_rows):
            want = o.rope(oq[i], n_head, int(pos[i]), hd, rot, 10000.0, 0)
            assert np.max(np.abs(got_q[i] - want)) <= 2e-6 * max(1.0, float(np.max(np.abs(want)))), i


def test_rows_qkv_rope_refusals(H, o):
    """More than 64 rows, or blocks off a 4-byte boundary: E_UNSUPPORTED with nothing launched
    (the forward pass then runs matmul_q8_fused and rope_rows); malformed arguments: errors."""
    d, dq, dkv, hd = 256, 256, 128, 64
    dws = [H.DeviceBuffer.of(random_weights("q8_0", n, d, n + 1)) for n in (dq, dkv, dkv)]
    dxq = H.DeviceBuffer(65 * 8 * 34 + 16)
    q, pool = H.DeviceBuffer(65 * dq * 4), H.DeviceBuffer(4 * dkv * 4)
    table = H.DeviceBuffer.of(rope_table(4, hd, 10000.0))
    zeros = H.DeviceBuffer.of(np.zeros(65, np.int64))
    base = dict(type=TYPE_ID["q8_0"], n_seg=3, w=dws, n_out=[dq, dkv, dkv], n_rows=4, n_in=d, in_mode=0, xq=dxq,
                out_mode=3, y=[q], y_stride=[dq], rope_table=table, rot_half=hd // 2, head_dim=hd, pos=zeros,
                cache_off=zeros, cache=pool)
    for bad in (dict(n_rows=65), dict(xq=dxq.ptr + 2)):
        with pytest.raises(H.HipError, match="status -2"):
            qkv_rope(H, **{**base, **bad})
    for bad in (dict(n_seg=2), dict(in_mode=2), dict(out_mode=0), dict(n_in=48), dict(head_dim=63),
                dict(rot_half=33), dict(n_out=[dq, dkv, dkv - 2]), dict(pos=0), dict(y_stride=[dq - 1])):
        with pytest.raises(H.HipError, match="status -1"):
            qkv_rope(H, **{**base, **bad})


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("n_rows", [1, 2, 3, 4])
@pytest.mark.parametrize("n_in,n_out,out_mode", [(2048, 2048, 0), (2048, 1153, 1), (8192, 2048, 1), (576, 576, 1),
                                                  (896, 300, 0)])
@pytest.mark.parametrize("misalign", [0, 2])
def test_q8_input_matches_unfused(H, o, kind, n_rows, n_in, n_out, out_mode, misalign):
    """in_mode 0: Q8_0 activation blocks in, store or residual add out. Aligned blocks take the
    LDS-DMA kernel; blocks 2 bytes off a 4-byte boundary take the staged kernel."""
    if not supported(H, kind, 0, n_rows, n_in):
        pytest.skip("shape outside the fused kernel")
    x = random_floats(n_rows * n_in, n_in + 5 * n_rows, 2.0).reshape(n_rows, n_in)
    xq = quantized_rows(o, x)
    w = random_weights(kind, n_out, n_in, n_in + n_out)
    res = random_floats(n_rows * n_out, n_out + 3, 1.0).reshape(n_rows, n_out)
    raw = xq.tobytes()
    dxq = H.DeviceBuffer(len(raw) + 16)
    dxq.upload(np.frombuffer(raw, np.uint8), offset=misalign)
    dw = H.DeviceBuffer.of(w)
    y = H.DeviceBuffer.of(res)
    fused(H, type=TYPE_ID[kind], n_seg=1, w=[dw], n_out=[n_out], n_rows=n_rows, n_in=n_in, in_mode=0,
          xq=dxq.ptr + misalign, out_mode=out_mode, y=[y], y_stride=[n_out])
    got = y.download(np.float32).reshape(n_rows, n_out)
    want = oracle_rows(o, kind, w, x, n_out, n_in) + (res if out_mode == 1 else 0)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("n_rows", [1, 3, 4])
def test_q8_input_silu_and_rope_match_unfused(H, o, kind, n_rows):
    n_in, ff = 2048, 8192
    x = random_floats(n_rows * n_in, 17 + n_rows, 2.0).reshape(n_rows, n_in)
    dxq = H.DeviceBuffer.of(quantized_rows(o, x))
    wg, wu = random_weights(kind, ff, n_in, 5), random_weights(kind, ff, n_in, 6)
    dwg, dwu = H.DeviceBuffer.of(wg), H.DeviceBuffer.of(wu)
    h = H.DeviceBuffer(n_rows * ff * 4)
    fused(H, type=TYPE_ID[kind], n_seg=2, w=[dwg, dwu], n_out=[ff, ff], n_rows=n_rows, n_in=n_in, in_mode=0,
          xq=dxq, out_mode=2, y=[h], y_stride=[ff])
    gate, up = (H.DeviceBuffer(n_rows * ff * 4) for _ in range(2))
    unfused_matmul(H, kind, dxq, n_rows, n_in, [dwg, dwu], [gate, up], [ff, ff], [ff, ff], False)
    out = H.DeviceBuffer(n_rows * ff * 4)
    H.call("silu_mul_rows", gate, up, out, None, ff, n_rows)
    assert np.array_equal(h.download(np.float32), out.download(np.float32))

    n_head, n_kv, hd, max_ctx = 32, 8, 64, 16
    dq, dkv = n_head * hd, n_kv * hd
    ws = [random_weights(kind, nn, n_in, 30 + i) for i, nn in enumerate((dq, dkv, dkv))]
    dws = [H.DeviceBuffer.of(w) for w in ws]
    pos = (np.arange(n_rows) * 3 + 1).astype(np.int32)
    coff = (np.arange(n_rows) * 2 * max_ctx * dkv).astype(np.int64)
    table = rope_table(max_ctx, hd, 500000.0)
    dpos, dcoff, dtab = H.DeviceBuffer.of(pos), H.DeviceBuffer.of(coff), H.DeviceBuffer.of(table)
    pool0 = np.zeros(n_rows * 2 * max_ctx * dkv, np.float32)
    pool, pool2 = H.DeviceBuffer.of(pool0), H.DeviceBuffer.of(pool0)
    q = H.DeviceBuffer(n_rows * dq * 4)
    fused(H, type=TYPE_ID[kind], n_seg=3, w=dws, n_out=[dq, dkv, dkv], n_rows=n_rows, n_in=n_in, in_mode=0, xq=dxq,
          out_mode=3, y=[q], y_stride=[dq], rope_table=dtab, rot_half=hd // 2, head_dim=hd, pos=dpos,
          cache_off=dcoff, cache=pool, k_layer_off=0, v_layer_off=max_ctx * dkv)
    q2, k2, v2 = (H.DeviceBuffer(n_rows * nn * 4) for nn in (dq, dkv, dkv))
    unfused_matmul(H, kind, dxq, n_rows, n_in, dws, [q2, k2, v2], [dq, dkv, dkv], [dq, dkv, dkv], False)
    ra = H.RopeRowsArgs(q=q2.ptr, k=k2.ptr, v=v2.ptr, pos=dpos.ptr, q_stride=dq, k_stride=dkv, n_head=n_head,
                        n_kv=n_kv, head_dim=hd, rotary_dim=hd, neox=0, theta=500000.0, table=dtab.ptr,
                        cache=pool2.ptr, cache_off=dcoff.ptr, k_layer_off=0, v_layer_off=max_ctx * dkv)
    H.check(H.lib().axon_hip_rope_rows(C.byref(ra), C.c_size_t(n_rows)), "rope_rows")
    assert np.array_equal(q.download(np.float32), q2.download(np.float32))
    assert np.array_equal(pool.download(np.float32), pool2.download(np.float32))


def test_rejects_bad_arguments(H):
    """Shapes the kernel cannot hold come back as errors, never as launches."""
    w = H.DeviceBuffer(64 * 34)
    x = H.DeviceBuffer(4 * 64 * 4)
    y = H.DeviceBuffer(64 * 4)
    base = dict(type=TYPE_ID["q8_0"], n_seg=1, w=[w], n_out=[2], n_rows=1, n_in=64, in_mode=1, x=x, x_stride=64,
                out_mode=0, y=[y], y_stride=[2])
    for bad in (dict(n_rows=5), dict(n_in=48), dict(out_mode=7), dict(in_mode=9), dict(x_stride=65),
                dict(out_mode=3), dict(out_mode=2)):
        with pytest.raises(H.HipError):
            fused(H, **{**base, **bad})
    assert not supported(H, "q8_0", 2, 1, 4096)      # the norm prologue holds one chunk per thread
    assert supported(H, "q8_0", 1, 2, 8192)          # float rows are quantized one at a time
    assert not supported(H, "q8_0", 1, 1, 16384)     # a row of 16384 floats exceeds the registers
    assert supported(H, "q4_0", 1, 1, 8192)

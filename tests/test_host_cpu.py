"""CPU-side checks of the product libraries and the model writer: the C ABI libraries load and
export every function include/*.h declares; without a gfx950 device the table and the model refuse
to start (Unsupported, never a CPU fallback, as src/kernels/kernels.cpp:85-92 refuses NEON on a
CPU without it); the synthetic-model quantizers reproduce the reference's quantizer fixtures; the
GGUF writer's files load in the oracle and in the reference's own LlamaModel."""
import ctypes as C
import re
from dataclasses import replace
from pathlib import Path

import numpy as np
import pytest

from helpers import GOLDEN, GGUF, OracleModel, RefModel, golden, have_ref

ROOT = Path(__file__).resolve().parents[1]


def declared(header: str) -> list[str]:
    text = (ROOT / "include" / header).read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(axon_(?:hip|model)_\w+)\s*\(", text)))


@pytest.mark.parametrize("header,lib", [("axon_hip.h", "libaxon_hip.so"), ("axon_model.h", "libaxon_host.so")])
def test_library_exports_every_declared_symbol(header, lib):
    names = declared(header)
    assert len(names) > 10
    so = C.CDLL(str(ROOT / "axon-infer_amd" / lib))
    missing = [n for n in names if not hasattr(so, n)]
    assert not missing, missing


def test_hip_table_declares_all_thirty_entries():
    entries = ["matmul_f32", "matmul_f16", "matmul_bf16", "matmul_f32_rows", "matmul_f16_rows", "matmul_bf16_rows",
               "rmsnorm", "rope", "softmax", "silu_mul", "embedding_row", "attention", "attention_kv",
               "attention_kv_heads", "attention_kv_heads_f16", "matmul_q8_0", "matmul_q4_0", "matmul_q8_0_q8",
               "matmul_q4_0_q8", "matmul_q8_0_rows", "matmul_q4_0_rows", "matmul_q8_0_q8_rows",
               "matmul_q4_0_q8_rows", "quantize_row_q8_0", "matmul_q4_1", "matmul_q4_1_q8", "matmul_q4_1_rows",
               "matmul_q4_1_q8_rows", "matmul_q6_k", "matmul_q6_k_rows"]
    assert len(entries) == 30
    names = set(declared("axon_hip.h"))
    assert all(f"axon_hip_{e}" in names for e in entries)


def _no_gpu():
    import axon_hip as H
    return H.device_count() == 0


@pytest.mark.skipif("not _no_gpu()")
def test_without_a_device_the_table_refuses_to_start():
    import axon_hip as H
    with pytest.raises(H.HipError, match="no GPU|gfx950"):
        H.init(0)
    with pytest.raises(H.HipError, match="status -3"):
        H.DeviceBuffer(64)


@pytest.mark.skipif("not _no_gpu()")
def test_without_a_device_the_model_refuses_to_load():
    import axon_hip as H
    with pytest.raises(H.HipError, match="no usable gfx950 device"):
        H.Model(GOLDEN / "gguf" / "synthetic-2l-q4_0.gguf", max_seq=8, max_ctx=16)


@pytest.mark.parametrize("name", ["q8_0", "q4_0", "q4_1"])
def test_quantizers_reproduce_reference_fixture_bytes(name):
    import synth
    x = golden("quant/row.f32.axt").ravel()
    fn = {"q8_0": synth.quantize_q8_0, "q4_0": synth.quantize_q4_0, "q4_1": synth.quantize_q4_1}[name]
    assert fn(x).tobytes() == (GOLDEN / f"quant/row.{name}.bin").read_bytes()


def test_q8_0_quantizer_matches_oracle_on_random_rows():
    import synth
    from tables import CTable
    o = CTable("oracle")
    rng = np.random.default_rng(4)
    for scale in (1e-6, 0.02, 1.0, 300.0):
        x = (rng.standard_normal(4096) * scale).astype(np.float32)
        assert synth.quantize_q8_0(x).tobytes() == o.quantize_row_q8_0(x).tobytes()


def test_q6_k_quantizer_round_trips_within_one_step():
    import synth
    from tables import dequantize
    x = np.random.default_rng(2).normal(0, 0.02, 256 * 8).astype(np.float32)
    q = synth.quantize_q6_k(x)
    back = dequantize("q6_k", q, 1, x.size).ravel()
    blocks = x.reshape(-1, 16)
    step = np.repeat(np.max(np.abs(blocks), axis=1) / 31, 16)
    assert np.all(np.abs(back - x) <= 0.6 * step + 1e-4 * np.max(np.abs(x)))


def test_synthetic_model_loads_in_oracle_and_reference(tmp_path):
    import synth
    spec = replace(synth.QWEN25_05B, name="t-qwen-1l", n_layer=1, n_vocab=640, seed=3)
    path = synth.write_model(spec, tmp_path / "m.gguf")
    g = GGUF(path)
    assert g.meta["general.architecture"] == "qwen2"
    assert g.tensors["blk.0.attn_q.bias"][0] == [896]
    toks = np.array([1, 5, 600, 7], np.int32)
    lo = OracleModel(path).forward(toks)
    assert np.all(np.isfinite(lo))
    if have_ref():
        assert np.array_equal(lo, RefModel(path, max_seq=8, max_ctx=16).forward(toks))


@pytest.mark.parametrize("cname,pyname", [("axon_hip_rope_rows_args", "RopeRowsArgs"),
                                          ("axon_hip_attention_rows_args", "AttentionRowsArgs"),
                                          ("axon_hip_matvec_fused_args", "MatvecFusedArgs"),
                                          ("axon_model_options", "ModelOptions"),
                                          ("axon_model_info", "ModelInfo")])
def test_ctypes_structs_match_the_header_layout(tmp_path, cname, pyname):
    """The ctypes mirrors of the argument structs have the size and field offsets gcc gives the
    declarations in include/axon_hip.h and include/axon_model.h."""
    import subprocess
    import axon_hip as H
    py = getattr(H, pyname)
    fields = [f[0] for f in py._fields_]
    src = tmp_path / "layout.c"
    body = "".join(f'  printf("%zu\\n", offsetof({cname}, {f}));\n' for f in fields)
    src.write_text(f'#include <stddef.h>\n#include <stdio.h>\n#include "axon_hip.h"\n#include "axon_model.h"\n'
                   f'int main(void) {{\n  printf("%zu\\n", sizeof({cname}));\n{body}  return 0;\n}}\n')
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", str(ROOT / "include"), str(src), "-o", str(exe)], check=True)
    got = [int(v) for v in subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()]
    assert got[0] == C.sizeof(py)
    assert got[1:] == [getattr(py, f).offset for f in fields]


def _gguf_one_tensor(path, dims, type_id):
    """A GGUF v3 file holding general.architecture and one tensor info with the given extents,
    followed by 64 bytes of data."""
    import struct
    s = lambda t: struct.pack("<Q", len(t)) + t  # noqa: E731
    key, val = b"general.architecture", b"llama"
    head = struct.pack("<IIQQ", 0x46554747, 3, 1, 1) + s(key) + struct.pack("<I", 8) + s(val)
    info = s(b"blk.0.attn_q.weight") + struct.pack("<I", len(dims)) + struct.pack(f"<{len(dims)}Q", *dims)
    info += struct.pack("<IQ", type_id, 0)
    blob = head + info
    blob += b"\0" * ((-len(blob)) % 32) + b"\0" * 64
    Path(path).write_bytes(blob)


@pytest.mark.parametrize("dims,type_id,message", [
    ([32, 550 * 10 ** 15], 8, "byte size overflows"),    # 2^64 > elements, but 34-byte blocks wrap
    ([2 ** 40, 2 ** 30], 0, "element count overflows"),  # 2^70 elements
    ([32, 0], 8, "extent of zero"),
    ([2 ** 62, 1], 0, "row length overflows"),           # 4 * 2^62 bytes per row wraps to 0
])
def test_gguf_rejects_extents_whose_size_wraps(tmp_path, dims, type_id, message):
    """The GGUF reader refuses tensor extents whose byte size would wrap around and slip past
    the bounds check (the reference's checks, src/core/gguf.cpp:595-633): zero extents, element
    counts past 64 bits, rows times row bytes past size_t."""
    import axon_hip as H
    path = tmp_path / "wrapped.gguf"
    _gguf_one_tensor(path, dims, type_id)
    with pytest.raises(H.HipError, match=message):
        H.Model(path, max_seq=8, max_ctx=16)

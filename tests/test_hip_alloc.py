"""The reference's "forward performs no heap allocation" (tests/unit/test_model_forward.cpp:119-128,
counting with a replaced global operator new, tests/unit/alloc_counter.cpp:33-46), for the decode
passes of the device-resident model: after one warm-up call of each kind, 16 steps each of
forward_prefill (logits copied, and left in HBM followed by the device greedy choice),
forward_batch of 8 rows, forward_mixed and generate_greedy make no host allocation in either
library (each counts its own operator new calls: axon_model_host_allocations,
axon_hip_allocation_counts) and no device allocation. On the persistent step kernel and on the
per-layer launches."""
import ctypes as C
from dataclasses import replace

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def counts():
    import axon_hip as H
    host = H.host()
    host.axon_model_host_allocations.restype = C.c_size_t
    hn, dev = C.c_size_t(0), C.c_size_t(0)
    H.lib().axon_hip_allocation_counts(C.byref(hn), C.byref(dev))
    return {"host library operator new": host.axon_model_host_allocations(), "hip library operator new": hn.value,
            "device allocations": dev.value}


@pytest.mark.parametrize("persistent", [True, False])
def test_decode_passes_allocate_nothing(tmp_path_factory, persistent):
    import synth
    import axon_hip as H
    spec = replace(synth.CONFIGS["c4"], name="t-c4-alloc-2l", n_layer=2, n_vocab=4096, seed=43)
    path = synth.cached_model(spec, tmp_path_factory.mktemp("models"))
    m = H.Model(path, max_seq=64, max_ctx=256, max_batch=8, max_caches=10, persistent=persistent)
    assert m.persistent_decode() == persistent
    rng = np.random.default_rng(3)
    c = m.new_cache()
    batch = [m.new_cache() for _ in range(8)]
    chunk_cache = m.new_cache()
    prompt = rng.integers(0, 4096, 16).astype(np.int32)
    t = int(np.argmax(m.forward_prefill(c, prompt)[-1]))
    for b in batch:
        m.forward_prefill(b, rng.integers(0, 4096, 8).astype(np.int32), logits=False)
    toks = rng.integers(0, 4096, 8).astype(np.int32)

    def one_round(t, toks, chunk):
        t = int(np.argmax(m.forward_prefill(c, [t])[0]))
        m.forward_prefill(c, [t], logits=False)
        t = int(m.greedy(1)[0])
        toks = np.argmax(m.forward_batch(batch, toks), axis=1).astype(np.int32)
        m.forward_batch(batch, toks, logits=False)
        toks = m.greedy(8).astype(np.int32)
        m.forward_mixed(chunk_cache, chunk, batch[:4], toks[:4], logits=False)
        m.greedy(5)
        return t, toks

    chunk = rng.integers(0, 4096, 4).astype(np.int32)
    t, toks = one_round(t, toks, chunk)  # warm-up: every kind of call once
    t = int(m.generate_greedy(c, t, 2)[-1])
    before = counts()
    for _ in range(16):
        t, toks = one_round(t, toks, chunk)
    t = int(m.generate_greedy(c, t, 16)[-1])
    after = counts()
    assert after == before, f"allocations during decode: before {before}, after {after}"
    m.close()

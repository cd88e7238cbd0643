"""The persistent decode step's measurement hook (axon_hip_decode_layers_set_stamps): with a stamp
buffer the kernel records the device clock at four points of every phase of every layer in every
workgroup, and the extra barriers it takes for that change nothing in the results: 12 greedy
steps give logits bit-identical to a model running the unstamped kernel, and every workgroup's
points of a phase come in order (start <= inputs in <= second inputs in <= end), each phase
after the previous one ended in that workgroup."""
import ctypes as C
from dataclasses import replace

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def test_stamped_step_kernel_gives_the_same_logits(tmp_path_factory):
    import synth
    import axon_hip as H
    spec = replace(synth.CONFIGS["c4"], name="t-c4-stamps-2l", n_layer=2, n_vocab=2048, seed=45)
    path = synth.cached_model(spec, tmp_path_factory.mktemp("models"))
    a = H.Model(path, max_seq=32, max_ctx=128)
    b = H.Model(path, max_seq=32, max_ctx=128)
    assert a.persistent_decode() and b.persistent_decode()
    L = H.lib()
    shape = H.DecodeShape()
    shape.n_layer = a.info.n_layer
    tps = C.c_double(0.0)
    L.axon_hip_decode_layers_stamp_count.restype = C.c_size_t
    n = L.axon_hip_decode_layers_stamp_count(C.byref(shape), C.byref(tps))
    assert n > 0 and n % (a.info.n_layer * 20) == 0 and tps.value > 0
    wgs = n // (a.info.n_layer * 20)
    buf = H.DeviceBuffer(n * 8)
    prompt = np.random.default_rng(12).integers(0, 2048, 20).astype(np.int32)
    ca, cb = a.new_cache(), b.new_cache()
    la, lb = a.forward_prefill(ca, prompt)[-1], b.forward_prefill(cb, prompt)[-1]
    t = int(np.argmax(la))
    try:
        for step in range(12):
            buf.fill(0)
            H.check(L.axon_hip_decode_layers_set_stamps(C.c_void_p(H.ptr_of(buf))))
            la = a.forward_prefill(ca, [t])[0]
            H.check(L.axon_hip_decode_layers_set_stamps(None))
            lb = b.forward_prefill(cb, [t])[0]
            assert np.array_equal(la, lb), f"step {step}"
            st = buf.download(np.uint64).reshape(a.info.n_layer, 5, 4, wgs).astype(np.int64)
            assert (st > 0).all(), "a point was not stamped"
            assert (np.diff(st, axis=2) >= 0).all(), "points of a phase out of order"
            flat = st.reshape(a.info.n_layer * 5, 4, wgs)
            assert (flat[1:, 0] >= flat[:-1, 3]).all(), "a phase started before the previous one ended"
            t = int(np.argmax(la))
    finally:
        L.axon_hip_decode_layers_set_stamps(None)
    a.close()
    b.close()

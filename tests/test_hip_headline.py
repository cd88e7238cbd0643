"""The two headline workloads' own paths against the reference's LlamaModel (oracle/_ref, the
reference's scalar table compiled from its sources), at the load options and schedules bench.py
measures them with.

  decode-b1   C4 (Llama-3.2-1B shape) loaded as bench.py loads it (max_seq 512, max_ctx 2240,
              max_batch 32, 34 cache slots), bench.py's 512-token prompt, then 64 greedy steps:
              logits of the prompt and of every step (positions 512..575, past the step
              kernel's first 256-position V chunk) within 1e-4, and the ids that
              axon_model_generate_greedy (the bench's timed loop: each id kept on the device)
              produces equal to the reference's greedy ids step for step. Both cache types.
  ragged-32   bench.py's context draw for 32 sequences, caches filled with the same random
              rows on both sides, then a staggered schedule: eight cohorts of four joining one
              step apart and leaving after eight steps, so forward_batch sees every batch size
              4, 8, ..., 32 growing and 28, ..., 4 shrinking (each size takes its own matmul
              kernels); every step's logits within 1e-4 of the reference's forward_batch and the
              greedy ids identical. Both cache types.

Patterned on tests/unit/test_model_kernels.cpp:59-72 (a second table against the scalar table on
whole models) and tests/unit/test_model_batch.cpp:103-157 (batched rows over caches of different
lengths).
"""
import numpy as np
import pytest

from test_hip_configs import Reference, close, hip, model_path, random_rows

pytestmark = pytest.mark.gpu

# bench.py's load options for C4 (its decode-b1 and ragged-32 legs).
BENCH = dict(max_seq=512, max_ctx=2048 + 128 + 64, max_batch=32, max_caches=34)


@pytest.mark.parametrize("cache", ["f32", "f16"])
def test_c4_decode_b1_at_the_bench_options(cache):
    path = model_path("c4")
    hm = hip(path, **BENCH, cache=cache)
    assert hm.info.persistent_decode == 1
    rm = Reference(path, max_seq=512, max_ctx=BENCH["max_ctx"], max_batch=1, f16=cache == "f16")
    prompt = np.random.default_rng(0).integers(0, hm.n_vocab, 512).astype(np.int32)  # bench.py's draw (seed 0)
    steps = 64
    rc = rm.new_cache()
    rl = rm.prefill(rc, prompt)
    ref_ids = [int(np.argmax(rl[-1]))]
    ref_logits = []
    for _ in range(steps):
        row = rm.prefill(rc, [ref_ids[-1]])[0]
        ref_logits.append(row)
        ref_ids.append(int(np.argmax(row)))
    # The host-driven loop: forward_prefill of each id, logits to the host.
    hc = hm.new_cache()
    close(hm.forward_prefill(hc, prompt), rl, f"C4 bench options ({cache}): prompt logits")
    del rl
    for s in range(steps):
        row = hm.forward_prefill(hc, [ref_ids[s]])[0]
        close(row, ref_logits[s], f"C4 bench options ({cache}): step {s} (position {512 + s})")
        assert int(np.argmax(row)) == ref_ids[s + 1], f"C4 bench options ({cache}): greedy step {s}"
    # The bench's timed loop: the prompt's greedy id chosen on the device, then every step's id
    # kept on the device.
    gc = hm.new_cache()
    hm.forward_mixed(gc, prompt, [], [], logits=False)
    assert int(hm.greedy(1)[0]) == ref_ids[0]
    got = hm.generate_greedy(gc, ref_ids[0], steps)
    assert got.tolist() == ref_ids[1:], f"C4 bench options ({cache}): generate_greedy ids differ"
    assert hm.cache_pos(gc) == hm.cache_pos(hc) == 512 + steps
    hm.close()


@pytest.mark.parametrize("cache", ["f32", "f16"])
def test_c4_staggered_ragged_schedule(cache):
    path = model_path("c4")
    hm = hip(path, **BENCH, cache=cache)
    rm = Reference(path, max_seq=8, max_ctx=BENCH["max_ctx"], max_batch=32, f16=cache == "f16")
    n_seq, cohort, stay = 32, 4, 8
    lens = np.random.default_rng(7).integers(64, 2049, n_seq).tolist()  # bench.py's draw (seed 0 + 7)
    hcs, rcs = [], []
    for i, n in enumerate(lens):
        rows = random_rows(hm.info, n, 900 + i)
        hc, rc = hm.new_cache(), rm.new_cache()
        hm.cache_fill(hc, rows)
        rm.fill(rc, rows)
        hcs.append(hc)
        rcs.append(rc)
        del rows
    toks = np.random.default_rng(8).integers(0, hm.n_vocab, n_seq).astype(np.int32)
    done = [0] * n_seq
    sizes = []
    step = 0
    while any(d < stay for d in done):
        active = [i for i in range(n_seq) if i // cohort <= step and done[i] < stay]
        sizes.append(len(active))
        hl = hm.forward_batch([hcs[i] for i in active], toks[active])
        rl = rm.batch([rcs[i] for i in active], toks[active])
        close(hl, rl, f"C4 staggered ragged ({cache}): step {step}, {len(active)} rows")
        th, tr = np.argmax(hl, axis=1).astype(np.int32), np.argmax(rl, axis=1).astype(np.int32)
        assert np.array_equal(th, tr), f"C4 staggered ragged ({cache}): step {step} greedy ids differ"
        toks[active] = th
        for i in active:
            done[i] += 1
        step += 1
    assert sizes == [4, 8, 12, 16, 20, 24, 28, 32, 28, 24, 20, 16, 12, 8, 4]
    assert [hm.cache_pos(c) for c in hcs] == [n + stay for n in lens]
    hm.close()

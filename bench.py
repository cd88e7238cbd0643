#!/usr/bin/env python3
"""Decode throughput of the hip kernel table on one MI355X, on the Llama-3.2-1B-shaped Q4_0 model
(hidden 2048, 16 layers, 32/8 heads, FFN 8192, vocab 128256, tied Q6_K
embedding/output, llama3 rope scaling; seeded random-init GGUF written by synth.py).

Two workloads, both greedy:
  decode-b1    one sequence: a 512-token prompt is prefilled (untimed), W warm-up decode steps,
               then K timed decode steps, generated as the reference's Engine::generate does at
               temperature zero (src/engine/engine.cpp:50-58): each step is forward_one of the
               previous token + the greedy choice (Sampler::sample, src/sampling/sampler.cpp:67-102).
               Here the choice is made on the device next to the logits and stays there as the
               next step's input (axon_model_generate_greedy); the K ids reach the host at the
               end. value = K / seconds. Two host-driven variants of the same steps follow on the
               same sequence: decode_b1_host_ids (the id of each step copied to the host and
               passed back as the next forward's token) and decode_b1_host_argmax (the [n_vocab]
               logits copied to the host and argmax'd by numpy). All three give the same ids
               (tests/test_hip_configs.py, test_generate_greedy_equals_host_loop).
  ragged-32    continuous batching of 32 sequences with contexts drawn U[64, 2048] from the seed:
               eight cohorts of four join 16 steps apart, each sequence decodes 128 tokens. Joining
               sequences are prefilled in their join step (timed apart, as src/engine/batch.cpp:71-85
               runs the prefill chunk apart from forward_batch). tokens/s = decoded tokens over the
               forward_batch time (device greedy choice and the ids to the host included).

The line also carries:
  roofline     the dominant kernel: the persistent decode-step kernel (all layers of a one-row
               pass in one launch), or, where one-row passes run layer by layer, the Q4_0 decode
               matvec (matvec_dma_kernel<Q4_0> for q|k|v, wo and down, matvec_norm1_kernel<Q4_0>
               for gate|up), from a probe pass of the same decode-b1 steps in which each such
               launch is bracketed by HIP events on the library stream: achieved = algorithmic
               bytes (weights, norm vectors, the K and V rows read and written, activations) /
               summed kernel time. The Q6_K output matvec is probed the same way (roofline_q6_k).
  cpu_baseline the reference's own LlamaModel on its scalar table (oracle/_ref, compiled from the
               reference sources) on the same GGUF, threads = the host's cores, on a bounded sample.
               For ragged-32 the CPU sample is fixed 32-row forward_batch steps at the workload's
               contexts; vs_cpu_fixed_batch compares the GPU's same 32-row steps with it, and
               vs_cpu_schedule the staggered workload's rate.

  f16_cache    decode-b1 and ragged-32 again with the KV cache held as fp16 (LoadOptions::cache
               = F16): half the cache bytes per position (kv_bytes_per_position).

  c1, c3       configs 1 and 3 as decode-b1 on their own shapes (SmolLM2-135M Q8_0: 128-token
               prompt, 64 greedy steps; TinyLlama-1.1B Q4_0/Q4_1/Q6_K: 512-token prompt, 256 greedy
               steps): tokens/s, HBM fraction per step, the step kernel's roofline, and the
               reference's LlamaModel decoding the same model on the host cores.

  c5_mixed     config 5: the Qwen2.5-0.5B-shaped model, 64 sequences with prompts U[32, 1024]
               admitted together, each step one 512-token prompt chunk plus one token of every
               sequence in decode, seeded top-k 40 / top-p 0.9 / T 0.8 sampling (candidates on the
               device, the draw on the host), 128 tokens each. one_pass runs each step as one
               forward (axon_model_forward_mixed), two_pass as the reference's two; both must give
               the same token streams. tokens_per_s = sampled tokens over the whole run; its roofline
               = algorithmic HBM bytes (weights per pass, each row's visible K and V) over the run.
               mixed_step: one steady-state step (a 512-token chunk + 63 decode rows) on the GPU in
               one and in two passes, and on the reference's LlamaModel (cpu_baseline).

  traffic      HBM bytes per launch of that kernel, from two rocprofv3 counter passes over
               `bench.py --traffic-probe` (FETCH_SIZE, then WRITE_SIZE, KiB per dispatch), each
               scaled by what the same counter reads for a device-to-device copy of 256 MiB in the
               same process; `bench.py --traffic-summary FETCH_CSV WRITE_CSV` reduces the two
               counter files to profiles/traffic_decode_step.json, which this line reports.

Prints one JSON line. --gpus above 1 exits: this build measures one GPU.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "axon-infer_amd"))
sys.path.insert(0, str(ROOT / "tests"))

HBM_PEAK_GBS = 8000.0
TRAFFIC_FILE = ROOT / "profiles" / "traffic_decode_step.json"
COPY_BYTES = 256 << 20
# The Q4_0 decode matvec's two kernels (Q4_0 is ggml type 2): matvec_dma_kernel for q|k|v, wo
# and down, matvec_norm1_kernel (the row RMSNorm'd while the weights arrive) for gate|up.
MATVEC_KERNELS = ("matvec_dma_kernel<2>", "matvec_norm1_kernel<2>")
# The persistent decode-step kernel, the dominant kernel when one-row passes run as one launch.
STEP_KERNEL_NAME = "decode_step_kernel"
# The persistent decode-step kernel: every layer of a one-row pass in one launch.
STEP_KERNEL = ("decode_step_kernel: all 16 layers of one decode step (norms, q|k|v+rope+cache, attention, "
               "wo+add, gate|up+silu, down+add) in one persistent launch")
METRIC = "decode tokens/s + HBM GB/s (% peak), Q4_0 1B model, batch 1 and 32 ragged"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def prefill_greedy(model, cache, tokens):
    """Prefill with the logits left in HBM; the last row's greedy id, chosen on the device. The
    pass computes logits for the last row only, the one the reference's Sequence observes
    (src/engine/sequence.cpp:118)."""
    model.forward_mixed(cache, tokens, [], [], logits=False)
    return int(model.greedy(1)[0])


def greedy_decode(model, cache, tok, steps):
    for _ in range(steps):
        model.forward_prefill(cache, [tok], logits=False)
        tok = int(model.greedy(1)[0])
    return tok


def device_loop_decode(model, cache, tok, steps):
    """The same greedy steps with the chosen id kept on the device between steps
    (axon_model_generate_greedy): no host round trip per token."""
    return int(model.generate_greedy(cache, tok, steps)[-1])


def host_argmax_decode(model, cache, tok, steps):
    for _ in range(steps):
        logits = model.forward_prefill(cache, [tok])
        tok = int(np.argmax(logits[-1]))
    return tok


def bench_decode_b1(H, model, n_vocab, steps, warmup, prompt_len, seed):
    rng = np.random.default_rng(seed)
    prompt = rng.integers(0, n_vocab, prompt_len).astype(np.int32)
    # A warm-up prefill of another prompt first: the timed one then excludes one-time costs
    # (first launches, LDS grants).
    warm = model.new_cache()
    prefill_greedy(model, warm, rng.integers(0, n_vocab, prompt_len).astype(np.int32))
    model.free_cache(warm)
    H.synchronize()
    cache = model.new_cache()
    t0 = time.perf_counter()
    tok = prefill_greedy(model, cache, prompt)
    prefill_s = time.perf_counter() - t0
    tok = device_loop_decode(model, cache, tok, warmup)
    H.synchronize()
    t0 = time.perf_counter()
    tok = device_loop_decode(model, cache, tok, steps)
    H.synchronize()
    elapsed = time.perf_counter() - t0
    ctx_end = model.cache_pos(cache)
    # The same steps driven from the host, each id copied to the host and passed back as the
    # next forward's token, over the next steps of the same sequence (its warm-up first).
    tok = greedy_decode(model, cache, tok, warmup)
    H.synchronize()
    t0 = time.perf_counter()
    tok = greedy_decode(model, cache, tok, steps)
    H.synchronize()
    ids_s = time.perf_counter() - t0
    # The same step with the logits row copied to the host and argmax'd there (the reference's
    # placement of the sampler), over the next steps of the same sequence.
    host_steps = min(steps, 64)
    t0 = time.perf_counter()
    host_argmax_decode(model, cache, tok, host_steps)
    H.synchronize()
    host_s = time.perf_counter() - t0
    model.free_cache(cache)
    return {"tokens_per_s": steps / elapsed, "ms_per_step": 1e3 * elapsed / steps, "prefill_tokens_per_s":
            prompt_len / prefill_s, "context": [prompt_len + warmup, ctx_end],
            "host_argmax": {"tokens_per_s": round(host_steps / host_s, 2),
                            "ms_per_step": round(1e3 * host_s / host_steps, 4), "steps": host_steps},
            "host_ids": {"tokens_per_s": round(steps / ids_s, 2), "ms_per_step": round(1e3 * ids_s / steps, 4),
                         "steps": steps, "context": [ctx_end + warmup, ctx_end + warmup + steps]}}


def probe_pass(H, model, n_vocab, steps, prompt_len, seed, weight_type):
    rng = np.random.default_rng(seed + 1)
    prompt = rng.integers(0, n_vocab, prompt_len).astype(np.int32)
    cache = model.new_cache()
    tok = prefill_greedy(model, cache, prompt)
    model.probe(weight_type, True)
    model.probe_read()
    greedy_decode(model, cache, tok, steps)
    ms, launches, nbytes = model.probe_read()
    model.probe(weight_type, False)
    model.free_cache(cache)
    return ms, launches, nbytes


PHASES = ("A: norm, q|k|v, RoPE, KV row", "B: attention", "C: wo + residual", "D: norm, gate|up, SiLU",
          "E: down + residual")


def phase_probe(H, model, n_vocab, steps, prompt_len, seed):
    """The persistent decode step's phases, from the device clock stamps the kernel records when
    given a stamp buffer (axon_hip_decode_layers_set_stamps): decode-b1 steps after a
    prompt_len-token prompt, one forward_prefill + device greedy choice per step, the stamps of
    each step read back after it. Per phase of a layer, the maximum over workgroups of
      wait  = inputs in - phase start      (polls for the previous phase's outputs)
      mid   = second inputs in - first     (attention: scoring and the scores exchange)
      tail  = phase end - last inputs in   (compute after the last poll)
    and the phase's span on the critical path: the latest end of this phase minus the latest end
    of the one before. Averaged over layers and steps."""
    import ctypes as C
    L = H.lib()
    info = model.info
    shape = H.DecodeShape()
    shape.n_layer = info.n_layer
    tps = C.c_double(0.0)
    L.axon_hip_decode_layers_stamp_count.restype = C.c_size_t
    n = L.axon_hip_decode_layers_stamp_count(C.byref(shape), C.byref(tps))
    if n == 0 or tps.value <= 0:
        raise SystemExit("bench.py: no stamp buffer size or clock rate for the decode step")
    wgs = n // (info.n_layer * 20)
    buf = H.DeviceBuffer(n * 8)
    rng = np.random.default_rng(seed + 3)
    cache = model.new_cache()
    tok = prefill_greedy(model, cache, rng.integers(0, n_vocab, prompt_len).astype(np.int32))
    tok = greedy_decode(model, cache, tok, 8)
    H.synchronize()
    t0 = time.perf_counter()
    tok = greedy_decode(model, cache, tok, steps)
    plain_ms = 1e3 * (time.perf_counter() - t0) / steps
    wait, mid, tail, span, total = [], [], [], [], []
    L.axon_hip_decode_layers_set_stamps(C.c_void_p(H.ptr_of(buf)))
    try:
        for _ in range(steps):
            buf.fill(0)
            model.forward_prefill(cache, [tok], logits=False)
            tok = int(model.greedy(1)[0])
            t = buf.download(np.uint64).reshape(info.n_layer, 5, 4, wgs)
            t = t[..., (t != 0).any(axis=(0, 1, 2))]  # the grid's workgroups (a small model's is smaller)
            t = t.astype(np.float64) * (1e6 / tps.value)
            t -= t[0, 0, 0].min()
            wait.append((t[:, :, 1] - t[:, :, 0]).max(axis=2))
            mid.append((t[:, :, 2] - t[:, :, 1]).max(axis=2))
            tail.append((t[:, :, 3] - t[:, :, 2]).max(axis=2))
            ends = t[:, :, 3].max(axis=2).reshape(-1)
            span.append(np.diff(np.concatenate([[0.0], ends])).reshape(info.n_layer, 5))
            total.append(ends[-1])
    finally:
        L.axon_hip_decode_layers_set_stamps(None)
    model.free_cache(cache)
    mean = lambda a: np.mean(np.stack(a), axis=(0, 1))  # over steps and layers
    w, m, tl, sp = mean(wait), mean(mid), mean(tail), mean(span)
    return {"kernel": STEP_KERNEL_NAME, "steps": steps, "context": [prompt_len + 8 + steps, prompt_len + 8 + 2 * steps],
            "workgroups": int(t.shape[-1]), "clock_hz": tps.value, "us_per_step_stamped": round(float(np.mean(total)), 2),
            "ms_per_step_plain": round(plain_ms, 4), "us_per_layer_stamped": round(float(np.mean(total)) / info.n_layer, 2),
            "phases": [{"phase": PHASES[p], "span_us": round(float(sp[p]), 3), "wait_us": round(float(w[p]), 3),
                        "mid_us": round(float(m[p]), 3), "tail_us": round(float(tl[p]), 3)} for p in range(5)]}


def ragged_schedule(n_seq, cohort, gap, decode_steps):
    return [(i // cohort) * gap for i in range(n_seq)], decode_steps


def bench_ragged(H, model, n_vocab, seed, n_seq=32, decode_steps=128, cohort=4, gap=16):
    rng = np.random.default_rng(seed + 7)
    ctx = rng.integers(64, 2049, n_seq)
    prompts = [rng.integers(0, n_vocab, int(c)).astype(np.int32) for c in ctx]
    joins, _ = ragged_schedule(n_seq, cohort, gap, decode_steps)
    caches = [None] * n_seq
    next_tok = [0] * n_seq
    done = [0] * n_seq
    max_seq = model.info.max_seq
    decode_s = prefill_s = 0.0
    decoded = 0
    step = 0
    batch_sizes = []
    # Algorithmic HBM bytes of the decode steps: the weights once per step, and each row's K and
    # V rows over its visible positions.
    info = model.info
    kv_bytes = 0.0
    while any(d < decode_steps for d in done):
        t0 = time.perf_counter()
        for i in range(n_seq):
            if joins[i] == step:
                c = model.new_cache()
                p = prompts[i]
                for s in range(0, len(p), max_seq):
                    tok = prefill_greedy(model, c, p[s:s + max_seq])
                caches[i] = c
                next_tok[i] = tok
        H.synchronize()
        prefill_s += time.perf_counter() - t0
        active = [i for i in range(n_seq) if caches[i] is not None and done[i] < decode_steps]
        if active:
            kv_bytes += sum(int(ctx[i]) + done[i] + 1 for i in active) * info.kv_bytes_per_position
            t0 = time.perf_counter()
            model.forward_batch([caches[i] for i in active], [next_tok[i] for i in active], logits=False)
            toks = model.greedy(len(active))
            decode_s += time.perf_counter() - t0
            for j, i in enumerate(active):
                next_tok[i] = int(toks[j])
                done[i] += 1
                if done[i] == decode_steps:
                    model.free_cache(caches[i])
            decoded += len(active)
            batch_sizes.append(len(active))
        step += 1
    step_bytes = len(batch_sizes) * info.weight_bytes_per_token + kv_bytes
    return {"tokens_per_s": decoded / decode_s, "decoded_tokens": decoded, "steps": step,
            "hbm_gbs": step_bytes / decode_s / 1e9, "hbm_frac": step_bytes / decode_s / 1e9 / HBM_PEAK_GBS,
            "mean_batch": float(np.mean(batch_sizes)), "max_batch": int(max(batch_sizes)),
            "prefill_tokens": int(ctx.sum()), "prefill_s": prefill_s, "decode_s": decode_s,
            "contexts": {"min": int(ctx.min()), "mean": float(ctx.mean()), "max": int(ctx.max())}}


def probe_attention_ragged(H, model, n_vocab, seed, n_seq=32, steps=8):
    """The batched decode attention alone: 32 caches prefilled to the ragged workload's contexts,
    then `steps` forward_batch steps of all 32 rows with each layer's attention launches
    bracketed by events (AXON_MODEL_PROBE_ATTENTION): achieved = the rows' K and V bytes over
    their visible positions (+ q and the output) / the attention time."""
    rng = np.random.default_rng(seed + 7)
    ctx = rng.integers(64, 2049, n_seq)
    max_seq = model.info.max_seq
    caches, toks = [], []
    for i in range(n_seq):
        c = model.new_cache()
        p = rng.integers(0, n_vocab, int(ctx[i])).astype(np.int32)
        for s0 in range(0, len(p), max_seq):
            tok = prefill_greedy(model, c, p[s0:s0 + max_seq])
        caches.append(c)
        toks.append(tok)
    model.forward_batch(caches, toks, logits=False)  # untimed first batch
    toks = [int(t) for t in model.greedy(n_seq)]
    # The same 32-row steps as the CPU baseline's forward_batch sample, timed plainly (the
    # like-for-like figure beside it): forward_batch, the device greedy choice, the ids.
    H.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        model.forward_batch(caches, toks, logits=False)
        toks = [int(t) for t in model.greedy(n_seq)]
    fixed_tps = n_seq * steps / (time.perf_counter() - t0)
    H.synchronize()
    model.probe(H.PROBE_ATTENTION, True)
    model.probe_read()
    for _ in range(steps):
        model.forward_batch(caches, toks, logits=False)
        toks = [int(t) for t in model.greedy(n_seq)]
    ms, launches, nbytes = model.probe_read()
    model.probe(H.PROBE_ATTENTION, False)
    for c in caches:
        model.free_cache(c)
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"kernel": "attn_scores64_kernel + attn_mixd_kernel (one attention_rows call per layer)",
            "rows": n_seq, "contexts_mean": float(ctx.mean()), "layer_calls": launches,
            "fixed_batch_tokens_per_s": round(fixed_tps, 1),
            "us_per_layer": round(1e3 * ms / max(launches, 1), 2), "bytes_per_layer": round(nbytes / max(launches, 1)),
            "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4)}


C5_SAMPLER = dict(temperature=0.8, top_k=40, top_p=0.9, min_p=0.05, repeat_penalty=1.1, repeat_last_n=64)


def run_engine(H, model, prompts, decode_tokens, seed, one_pass):
    """BatchEngine::step (src/engine/batch.cpp:69-156) over sequences admitted together: each step
    feeds the next max_seq-token chunk of the oldest sequence still in prefill and one token of
    every sequence in decode, then samples (Sampler::sample with config 5's settings, each
    sequence with its own seeded generator; SamplerConfig's min_p 0.05 and repeat penalty 1.1
    over the last 64 ids are kept). The chunk that completes a prompt draws the sequence's first
    token from its last row (sequence.cpp:101-123); an earlier chunk draws nothing. one_pass:
    the chunk and the decode rows in one pass (axon_model_forward_mixed); else as the reference,
    the chunk's pass (its last row's logits only) then forward_batch. Logits stay in HBM."""
    n = len(prompts)
    max_seq = model.info.max_seq
    caches = [model.new_cache() for _ in range(n)]
    cfg = H.SamplerConfig(**C5_SAMPLER)
    quiet = H.SamplerConfig(temperature=0.0, repeat_penalty=1.0)  # an unfinished chunk: no draw
    gens = [H.Rng(seed * 1000 + i + 1) for i in range(n)]
    fed = [0] * n
    out = [[] for _ in range(n)]
    steps = 0
    # Algorithmic HBM bytes: per pass the weights once (a two-pass step reads them twice), and
    # each row's visible K and V rows (the chunk's span once for the chunk).
    info = model.info
    hbm_bytes = 0.0
    H.synchronize()
    t0 = time.perf_counter()
    while True:
        pre = [i for i in range(n) if fed[i] < len(prompts[i])]
        # Sequence::accept_pending (sequence.cpp:129-142): a sequence feeds its pending token until
        # it has generated decode_tokens, so the last pass samples one token that is dropped.
        dec = [i for i in range(n) if fed[i] == len(prompts[i]) and 0 < len(out[i]) <= decode_tokens]
        if not pre and not dec:
            break
        pi = pre[0] if pre else None
        chunk = prompts[pi][fed[pi]:fed[pi] + max_seq] if pi is not None else []
        done_prompt = pi is not None and fed[pi] + len(chunk) == len(prompts[pi])
        # The penalty reads the last repeat_last_n ids of each history (sampler.cpp:75-76).
        last_n = C5_SAMPLER["repeat_last_n"]

        def tail(i, upto):
            t = out[i][-last_n:]
            if len(t) < last_n:
                t = [int(v) for v in prompts[i][max(0, upto - (last_n - len(t))):upto]] + t
            return t

        hist = {i: tail(i, fed[i]) for i in dec}
        toks = [out[i][-1] for i in dec]
        dcfg, dgen, drec = [cfg] * len(dec), [gens[i] for i in dec], [hist[i] for i in dec]
        if pi is not None:
            pcfg = cfg if done_prompt else quiet
            prec = tail(pi, fed[pi] + len(chunk))
        if one_pass:
            model.forward_mixed(caches[pi] if pi is not None else None, chunk, [caches[i] for i in dec], toks,
                                logits=False)
            if pi is not None:
                ids = model.sample([pcfg] + dcfg, [gens[pi]] + dgen, [prec] + drec)
            else:
                ids = model.sample(dcfg, dgen, drec)
        else:
            ids = []
            if pi is not None:
                model.forward_mixed(caches[pi], chunk, [], [], logits=False)
                ids += list(model.sample([pcfg], [gens[pi]], [prec]))
            if dec:
                model.forward_batch([caches[i] for i in dec], toks, logits=False)
                ids += list(model.sample(dcfg, dgen, drec))
        passes = 1 if one_pass else int(pi is not None) + int(bool(dec))
        kv_rows = sum(fed[i] + 1 for i in dec) + (fed[pi] + len(chunk) if pi is not None else 0)
        hbm_bytes += passes * info.weight_bytes_per_token + kv_rows * info.kv_bytes_per_position
        r = 0
        if pi is not None:
            fed[pi] += len(chunk)
            if done_prompt:
                out[pi].append(int(ids[0]))
            r = 1
        for j, i in enumerate(dec):
            out[i].append(int(ids[r + j]))
        steps += 1
    H.synchronize()
    elapsed = time.perf_counter() - t0
    for c in caches:
        model.free_cache(c)
    return [o[:decode_tokens] for o in out], steps, elapsed, hbm_bytes


def bench_c5(H, seed, n_seq=64, decode_tokens=128):
    """Config 5 at full size: the Qwen2.5-0.5B-shaped model (Q4_0, q/k/v bias, NeoX RoPE, Q8_0
    output), 64 sequences with prompts drawn U[32, 1024] from the seed, 128 sampled tokens each,
    prompt chunks mixed with decode in the same steps. Both engines run the same schedule and
    must produce the same token streams."""
    import synth
    spec = synth.CONFIGS["c5"]
    path = synth.cached_model(spec)
    model = H.Model(path, max_seq=512, max_ctx=1024 + decode_tokens + 64, max_batch=n_seq, max_caches=n_seq)
    rng = np.random.default_rng(seed + 11)
    lens = rng.integers(32, 1025, n_seq)
    prompts = [rng.integers(0, spec.n_vocab, int(k)).astype(np.int32) for k in lens]
    # Warm-up: a short schedule of four sequences.
    run_engine(H, model, [p[:40] for p in prompts[:4]], 4, seed, True)
    res = {}
    streams = []
    for name, one in (("one_pass", True), ("two_pass", False)):
        out, steps, elapsed, nbytes = run_engine(H, model, prompts, decode_tokens, seed, one)
        gen = sum(len(o) for o in out)
        gbs = nbytes / elapsed / 1e9
        res[name] = {"tokens_per_s": round(gen / elapsed, 1),
                     "total_tokens_per_s": round((gen + int(lens.sum())) / elapsed, 1),
                     "seconds": round(elapsed, 3), "steps": steps,
                     "hbm_gbs": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}
        streams.append(out)
        log(f"c5 {name}: {gen} tokens in {elapsed:.2f}s over {steps} steps ({gen / elapsed:.0f} tok/s)")
    res["roofline"] = {"bound": "hbm", "kernel": "whole run (one_pass): every pass's weights plus each row's visible "
                                                "K and V rows, over the run's wall time",
                       "achieved": res["one_pass"]["hbm_gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                       "frac": res["one_pass"]["hbm_frac"]}
    res["mixed_step"] = c5_mixed_step(H, model, lens, seed)
    model.close()
    res["streams_identical"] = streams[0] == streams[1]
    res["generated_tokens"] = n_seq * decode_tokens
    res["prompt_tokens"] = int(lens.sum())
    res["speedup_one_pass"] = round(res["two_pass"]["seconds"] / res["one_pass"]["seconds"], 3)
    res["workload"] = ("config 5: Qwen2.5-0.5B-shaped (24 layers, hidden 896, 14/2 heads, FFN 4864, vocab 151936, "
                       "Q4_0 + q/k/v bias, NeoX, Q8_0 output), 64 sequences, prompts U[32, 1024], chunks of 512 "
                       "mixed with decode, top-k 40 / top-p 0.9 / T 0.8 / min-p 0.05 / penalty 1.1, 128 tokens each")
    return res


def c5_step_inputs(info, lens, seed, n_dec=63, chunk_len=512):
    """One continuous-batching step of config 5 in its steady state: a 512-token prompt chunk into a
    fresh cache and 63 sequences in decode at the prompt contexts lens[:63], their caches holding
    the same seeded random K and V rows on the GPU and on the CPU."""
    rng = np.random.default_rng(seed + 13)
    chunk = rng.integers(0, info.n_vocab, chunk_len).astype(np.int32)
    toks = rng.integers(0, info.n_vocab, n_dec).astype(np.int32)
    row = info.n_head_kv * info.head_dim

    def rows(i):
        return np.random.default_rng(seed + 100 + i).standard_normal((info.n_layer, 2, int(lens[i]), row), dtype=np.float32)
    return chunk, toks, rows


def c5_mixed_step(H, model, lens, seed, reps=5):
    """That step on the GPU, as one pass (forward_mixed: the chunk's last row and the 63 decode
    rows get logits) and as the reference's two (forward_prefill of the chunk, then
    forward_batch); tokens/s = the 64 tokens the step samples over the step's time."""
    info = model.info
    chunk, toks, rows = c5_step_inputs(info, lens, seed)
    dec = []
    for i in range(len(toks)):
        c = model.new_cache()
        model.cache_fill(c, rows(i))
        dec.append(c)
    res = {}
    for name in ("one_pass", "two_pass"):
        times = []
        for _ in range(reps + 1):
            pc = model.new_cache()
            H.synchronize()
            t0 = time.perf_counter()
            if name == "one_pass":
                model.forward_mixed(pc, chunk, dec, toks, logits=False)
            else:
                model.forward_mixed(pc, chunk, [], [], logits=False)
                model.forward_batch(dec, toks, logits=False)
            H.synchronize()
            times.append(time.perf_counter() - t0)
            model.free_cache(pc)
            for i, c in enumerate(dec):
                model.truncate(c, int(lens[i]))
        t = float(np.median(times[1:]))
        res[name] = {"ms": round(1e3 * t, 3), "tokens_per_s": round((len(toks) + 1) / t, 1)}
    for c in dec:
        model.free_cache(c)
    res["step"] = (f"one {len(chunk)}-token prompt chunk into a fresh cache + {len(toks)} decode rows at contexts "
                   f"U[32, 1024] (mean {float(np.mean(lens[:len(toks)])):.0f}); {len(toks) + 1} sampled tokens")
    return res


def traffic_probe(H, model, n_vocab, steps, prompt_len, seed):
    """The workload of the counter passes: one device-to-device copy of COPY_BYTES (the
    calibration), then a prefill and `steps` greedy decode steps of decode-b1."""
    src, dst = H.DeviceBuffer(COPY_BYTES), H.DeviceBuffer(COPY_BYTES)
    src.fill(1)
    H.call("memcpy_d2d", dst, src, COPY_BYTES)
    H.synchronize()
    src.free()
    dst.free()
    rng = np.random.default_rng(seed + 3)
    cache = model.new_cache()
    tok = prefill_greedy(model, cache, rng.integers(0, n_vocab, prompt_len).astype(np.int32))
    greedy_decode(model, cache, tok, steps)
    H.synchronize()
    model.free_cache(cache)


def attention_traffic_probe(H, model, n_vocab, seed):
    """The workload of the attention counter passes: the calibration copy of traffic_probe, then
    the ragged-32 attention probe (every attn_scores64_kernel / attn_mixd_kernel launch of the
    run is one layer of a 32-row batch at the ragged contexts); prints the probe's figures."""
    src, dst = H.DeviceBuffer(COPY_BYTES), H.DeviceBuffer(COPY_BYTES)
    src.fill(1)
    H.call("memcpy_d2d", dst, src, COPY_BYTES)
    H.synchronize()
    src.free()
    dst.free()
    print(json.dumps(probe_attention_ragged(H, model, n_vocab, seed)), flush=True)


def prefill_probe(H, model, n_vocab, seed, passes=4, prompt_len=512):
    """The workload of the prefill profiles: `passes` 512-token prefill passes (logits of the
    last row only), each on a new cache."""
    rng = np.random.default_rng(seed + 5)
    for i in range(passes):
        c = model.new_cache()
        t0 = time.perf_counter()
        model.forward_mixed(c, rng.integers(0, n_vocab, prompt_len).astype(np.int32), [], [], logits=False)
        H.synchronize()
        log(f"prefill {i}: {prompt_len / (time.perf_counter() - t0):.0f} tok/s")
        model.free_cache(c)


def _counter_rows(path):
    """(kernel name, counter name, value) of every dispatch in a rocprofv3 counter CSV."""
    import csv
    with open(path, newline="") as f:
        for row in csv.DictReader(f):
            keys = {k.lower(): k for k in row}
            yield (row[keys["kernel_name"]], row[keys["counter_name"]], float(row[keys["counter_value"]]))


def traffic_summary(fetch_csv, write_csv):
    """Per-dispatch FETCH_SIZE and WRITE_SIZE (KiB) of the dominant decode kernel (the
    persistent decode-step kernel, or the Q4_0 decode matvec where one-row passes run layer by
    layer), each scaled by the counter's reading for the calibration copy (COPY_BYTES read and
    written)."""
    def per_kernel(path, counter):
        copy, step, mv, q6 = [], [], [], []
        for name, cname, value in _counter_rows(path):
            if cname != counter:
                continue
            n = name.replace(" ", "")
            if "copyBuffer" in name:
                copy.append(value)
            elif STEP_KERNEL_NAME in n:
                step.append(value)
            elif any(k in n for k in MATVEC_KERNELS):
                mv.append(value)
            elif "q6k_planar_kernel<1>" in n or "q6k_planar_kernel<1,256>" in n:
                q6.append(value)
        main = step or mv
        if not copy or not main:
            raise SystemExit(f"{path}: no {counter} rows for the copy ({len(copy)}) or the decode kernel ({len(main)})")
        return max(copy), main, q6, bool(step)
    fcopy, fmv, fq6, is_step = per_kernel(fetch_csv, "FETCH_SIZE")
    wcopy, wmv, wq6, _ = per_kernel(write_csv, "WRITE_SIZE")
    f_scale = COPY_BYTES / (fcopy * 1024.0)
    w_scale = COPY_BYTES / (wcopy * 1024.0)
    fetch = float(np.mean(fmv)) * 1024.0 * f_scale
    write = float(np.mean(wmv)) * 1024.0 * w_scale
    out = {"kernel": STEP_KERNEL_NAME if is_step else " + ".join(MATVEC_KERNELS), "dispatches": len(fmv),
           "fetch_bytes_per_launch": round(fetch), "write_bytes_per_launch": round(write),
           "traffic_bytes_per_launch": round(fetch + write),
           "copy_bytes": COPY_BYTES, "copy_fetch_kib": fcopy, "copy_write_kib": wcopy,
           "fetch_scale": round(f_scale, 4), "write_scale": round(w_scale, 4),
           "passes": ["rocprofv3 --pmc FETCH_SIZE -f csv -- python3 bench.py --traffic-probe --steps 8",
                      "rocprofv3 --pmc WRITE_SIZE -f csv -- python3 bench.py --traffic-probe --steps 8",
                      "python3 bench.py --traffic-summary <FETCH_SIZE counter csv> <WRITE_SIZE counter csv>"]}
    if fq6 and wq6:  # the Q6_K output matvec over the planar copy, for comparison
        out["q6k_planar_kernel<1>"] = {"dispatches": len(fq6),
                                       "traffic_bytes_per_launch": round(float(np.mean(fq6)) * 1024.0 * f_scale +
                                                                         float(np.mean(wq6)) * 1024.0 * w_scale)}
    TRAFFIC_FILE.write_text(json.dumps(out, indent=1) + "\n")
    print(json.dumps(out))
    return 0


SWEEP_SHAPES = [(2048, 2048), (8192, 2048), (2048, 8192), (128256, 2048)]
SWEEP_ROWS = [1, 16, 64, 512]
# Beside the sweep: the Q6_K table entry over the GGUF blocks themselves (matmul_q6_k /
# matmul_q6_k_rows, what a caller binding the kernel table gets) on the output shape.
SWEEP_NATIVE = ("q6_k_native", 128256, 2048, [1, 4, 16, 32])
SWEEP_TYPES = {"q4_0": (2, 18 / 32), "q4_1": (3, 20 / 32), "q8_0": (8, 34 / 32), "q6_k": (14, 210 / 256)}
INT8_PEAK_TOPS = 5000.0
FP32_PEAK_TFLOPS = 157.3


def bench_sweep(H, seed, reps=20, rounds=3):
    """BASELINE configuration 2 through the table entries (the reference's bench_kernels.cpp:379-402
    sweep): every (N, K) x type x M. Integer types run matmul_*_q8 (one row) or matmul_*_q8_rows
    on Q8_0 activations; Q6_K runs matmul_q6_k_planar on float activations (the repacked copy the
    model streams), and beside the sweep ("q6_k_native") matmul_q6_k_rows over the GGUF blocks on
    the output shape. Each call is captured `reps` times into one graph, each capture on the next of
    enough weight copies that the copies exceed the 256 MB Infinity Cache, and the graph's
    replays are timed with events on the library stream: per-call time, dispatch included.
    Bytes are algorithmic: N*K weight bytes + the activations (Q8_0 blocks, or floats for Q6_K)
    + M*N float outputs; ops are 2*M*N*K."""
    import ctypes as C
    from tables import random_weights
    lib = H.lib()
    lib.axon_hip_q6k_planar_bytes.restype = C.c_size_t
    rows = []
    jobs = [(kind, n, k, SWEEP_ROWS) for kind in SWEEP_TYPES for n, k in SWEEP_SHAPES]
    jobs.append((SWEEP_NATIVE[0], SWEEP_NATIVE[1], SWEEP_NATIVE[2], SWEEP_NATIVE[3]))
    for kind, n, k, ms in jobs:
        tid, bpe = SWEEP_TYPES["q6_k" if kind == "q6_k_native" else kind]
        w = random_weights("q6_k" if kind == "q6_k_native" else kind, n, k, seed + n + k)
        wbytes = w.nbytes
        copies = int(max(2, min(64, -(-640_000_000 // wbytes))))
        bufs = []
        for _ in range(copies):
            b = H.DeviceBuffer.of(w)
            if kind == "q6_k":
                pl = H.DeviceBuffer(lib.axon_hip_q6k_planar_bytes(C.c_size_t(n), C.c_size_t(k)))
                H.call("q6k_repack", b, n, k, pl)
                b.free()
                b = pl
            bufs.append(b)
        del w
        for m in ms:
            x = np.random.default_rng(seed + m).standard_normal(m * k).astype(np.float32)
            dx = H.DeviceBuffer.of(x)
            dxq = H.DeviceBuffer(m * k // 32 * 34)
            H.call("quantize_rows_q8_0", dx, dxq, k, m, k)
            y = H.DeviceBuffer(m * n * 4)

            def one(i):
                wb = bufs[i % copies]
                if kind == "q6_k":
                    H.call("matmul_q6_k_planar", wb, dx, y, m, n, k, n)
                elif kind == "q6_k_native":
                    H.call("matmul_q6_k_rows", wb, dx, y, m, n, k, n)
                elif m == 1:
                    H.call(f"matmul_{kind}_q8", wb, dxq, y, n, k)
                else:
                    H.call(f"matmul_{kind}_q8_rows", wb, dxq, y, m, n, k, n)

            for i in range(copies):  # untimed: first launches, LDS grants
                one(i)
            H.synchronize()
            H.check(lib.axon_hip_graph_begin(), "graph_begin")
            for i in range(reps):
                one(i)
            g = C.c_void_p(0)
            H.check(lib.axon_hip_graph_end(C.byref(g)), "graph_end")
            H.check(lib.axon_hip_graph_launch(g), "graph_launch")
            H.synchronize()
            e0, e1 = H.Event(), H.Event()
            e0.record()
            for _ in range(rounds):
                H.check(lib.axon_hip_graph_launch(g), "graph_launch")
            e1.record()
            H.synchronize()
            lib.axon_hip_graph_destroy(g)
            us = 1e3 * e0.elapsed_ms(e1) / (rounds * reps)
            act = m * k * 4 if kind.startswith("q6_k") else m * k // 32 * 34
            nbytes = n * k * bpe + act + m * n * 4
            gbs = nbytes / (us * 1e-6) / 1e9
            tops = 2.0 * m * n * k / (us * 1e-6) / 1e12
            rows.append([kind, n, k, m, round(us, 2), round(gbs, 1), round(tops, 2)])
            log(f"sweep {kind} {n}x{k} M={m}: {us:.1f} us, {gbs:.0f} GB/s, {tops:.1f} TOPS")
            dx.free(); dxq.free(); y.free()
        for b in bufs:
            b.free()
    best_m1 = {f"{n}x{k}": max(r[5] for r in rows if r[1] == n and r[2] == k and r[3] == 1 and r[0] in SWEEP_TYPES)
               for n, k in SWEEP_SHAPES}
    return {"columns": ["type", "N", "K", "M", "us_per_call", "GB_per_s", "TOPS"], "rows": rows,
            "hbm_peak_GB_per_s": HBM_PEAK_GBS, "int8_peak_TOPS": INT8_PEAK_TOPS, "fp32_peak_TFLOPS": FP32_PEAK_TFLOPS,
            "best_M1_GB_per_s": best_m1,
            "method": "table entry captured 20x into a graph over rotating weight copies (> 256 MB), event-timed "
                      "replays on the library stream; algorithmic bytes; random weight blocks (tables.random_weights)"}


def host_cores() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


# Configs 1 and 3 (decode-b1 on their own shapes): (config, prompt, greedy steps, weight type of
# q|k|v, whose launches the kernel-time probe brackets).
B1_CONFIGS = {"c1": (128, 64, 8), "c3": (512, 256, 2)}


def bench_config_b1(H, name, warmup, seed):
    """BASELINE configs 1 and 3 as decode-b1: the config's prompt, then its greedy steps generated
    as the bench's C4 leg does (axon_model_generate_greedy); HBM bytes per step = the weights
    (llama.cpp:151-167) + the K and V rows of the visible positions; the dominant kernel's
    roofline from a probed pass of the same steps."""
    import synth
    prompt_len, steps, wtype = B1_CONFIGS[name]
    spec = synth.CONFIGS[name]
    path = synth.cached_model(spec)
    model = H.Model(path, max_seq=prompt_len, max_ctx=prompt_len + warmup + steps + 8)
    info = model.info
    prompt = np.random.default_rng(seed + 21).integers(0, info.n_vocab, prompt_len).astype(np.int32)
    warm = model.new_cache()
    prefill_greedy(model, warm, prompt)
    model.free_cache(warm)
    cache = model.new_cache()
    tok = prefill_greedy(model, cache, prompt)
    tok = device_loop_decode(model, cache, tok, warmup)
    H.synchronize()
    t0 = time.perf_counter()
    ids = model.generate_greedy(cache, tok, steps)
    H.synchronize()
    dt = time.perf_counter() - t0
    model.free_cache(cache)
    ctx = [prompt_len + warmup + 1, prompt_len + warmup + steps]
    step_bytes = info.weight_bytes_per_token + info.kv_bytes_per_position * 0.5 * (ctx[0] + ctx[1])
    ms, launches, nbytes = probe_pass(H, model, info.n_vocab, min(steps, 32), prompt_len, seed,
                                      H.PROBE_STEP if info.persistent_decode else wtype)
    achieved = nbytes / (ms * 1e-3) / 1e9 if launches else 0.0
    res = {"workload": f"{spec.name}-shaped random-init GGUF, {prompt_len}-token prompt, {steps} greedy steps, batch 1",
           "tokens_per_s": round(steps / dt, 2), "ms_per_step": round(1e3 * dt / steps, 4), "context": ctx,
           "weight_bytes_per_token": info.weight_bytes_per_token, "kv_bytes_per_position": info.kv_bytes_per_position,
           "hbm_gbs_per_step": round(step_bytes / (dt / steps) / 1e9, 1),
           "hbm_frac_per_step": round(step_bytes / (dt / steps) / 1e9 / HBM_PEAK_GBS, 4),
           "decode_path": "one persistent kernel per step" if info.persistent_decode else "per-layer launches",
           "roofline": {"bound": "hbm", "kernel": STEP_KERNEL_NAME if info.persistent_decode else "decode matvecs",
                        "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": round(achieved / HBM_PEAK_GBS, 4), "launches": launches,
                        "bytes_per_launch": round(nbytes / max(launches, 1)),
                        "avg_us": round(1e3 * ms / max(launches, 1), 3), "traffic": None},
           "first_ids": [int(v) for v in ids[:8]]}
    model.close()
    log(f"{name} decode-b1: {res['tokens_per_s']:.1f} tok/s, {res['hbm_frac_per_step'] * 100:.1f}% of HBM per step, "
        f"kernel {res['roofline']['frac'] * 100:.1f}%")
    return res, path, prompt


def cpu_decode_b1(path, n_vocab, seed, budget_s, ctx0, prompt=None, max_ctx=2176):
    """The reference's LlamaModel decoding greedily at batch 1 on the host cores: after a real
    prefill of `prompt`, or over a cache filled with ctx0 seeded random positions."""
    from helpers import GGUF, ModelConfig, RefModel, ref
    import ctypes as C
    cores = host_cores()
    rng = np.random.default_rng(seed)
    r = RefModel(path, max_seq=max(32, len(prompt) if prompt is not None else 0), max_ctx=max_ctx, max_batch=1,
                 n_threads=cores)
    c = r.new_cache()
    if prompt is not None:
        logits = r.forward_prefill(c, prompt)
        tok = int(np.argmax(logits[-1]))
        ctx0 = len(prompt)
        how = f"after a real prefill of the same {ctx0}-token prompt"
    else:
        cfg = ModelConfig(GGUF(path))
        row = cfg.n_head_kv * cfg.head_dim
        kv = (0.5 * rng.standard_normal(cfg.n_layer * 2 * ctx0 * row)).astype(np.float32)
        ref().ref_cache_fill(C.c_void_p(r.h), c, C.c_void_p(kv.ctypes.data), C.c_size_t(ctx0))
        del kv
        tok = int(rng.integers(0, n_vocab))
        how = f"over a cache filled with {ctx0} seeded random positions"
    steps, t0 = 0, time.perf_counter()
    while steps < 3 or (time.perf_counter() - t0 < budget_s and steps < 64):
        logits = r.forward_prefill(c, [tok])
        tok = int(np.argmax(logits[-1]))
        steps += 1
    dt = time.perf_counter() - t0
    return {"value": steps / dt, "unit": "tokens/s", "cores": cores, "kind": "reference",
            "sample": f"{steps} greedy decode steps at contexts {ctx0 + 1}..{ctx0 + steps}, {how}; reference "
                      f"LlamaModel on its scalar table, {cores} threads"}


def cpu_c5_step(path, lens, seed):
    """Config 5's steady-state step (c5_step_inputs) on the reference's LlamaModel, as its
    BatchEngine runs it: forward_prefill of the chunk, then forward_batch of the decode rows."""
    from helpers import GGUF, ModelConfig, RefModel, ref
    import ctypes as C
    cores = host_cores()
    cfg = ModelConfig(GGUF(path))

    class Info:
        n_vocab, n_head_kv, head_dim, n_layer = cfg.n_vocab, cfg.n_head_kv, cfg.head_dim, cfg.n_layer
    chunk, toks, rows = c5_step_inputs(Info, lens, seed)
    r = RefModel(path, max_seq=512, max_ctx=1024 + 128 + 64, max_batch=64, n_threads=cores)
    dec = []
    for i in range(len(toks)):
        c = r.new_cache()
        rr = np.ascontiguousarray(rows(i))
        ref().ref_cache_fill(C.c_void_p(r.h), c, C.c_void_p(rr.ctypes.data), C.c_size_t(int(lens[i])))
        dec.append(c)
    pc = r.new_cache()
    t0 = time.perf_counter()
    r.forward_prefill(pc, chunk)
    t1 = time.perf_counter()
    r.forward_batch(dec, toks)
    t2 = time.perf_counter()
    return {"value": (len(toks) + 1) / (t2 - t0), "unit": "tokens/s", "cores": cores, "kind": "reference",
            "sample": f"one step: forward_prefill of a {len(chunk)}-token chunk ({t1 - t0:.2f} s, logits of every row "
                      f"as the reference computes them) then forward_batch of {len(toks)} decode rows ({t2 - t1:.2f} s); "
                      f"reference LlamaModel on its scalar table, {cores} threads"}


def cpu_baseline(path, n_vocab, seed, budget_s, ctx0):
    """The reference's LlamaModel (scalar table) on the host cores: batch-1 decode and one
    32-sequence batched step over caches filled to the ragged contexts."""
    from helpers import have_ref
    if not have_ref():
        return None, None
    from helpers import RefModel, ref
    cores = host_cores()
    rng = np.random.default_rng(seed)
    log(f"cpu baseline: reference scalar table, {cores} threads, loading")
    r = RefModel(path, max_seq=32, max_ctx=2176, max_batch=32, n_threads=cores)
    from helpers import GGUF, ModelConfig
    import ctypes as C
    cfg = ModelConfig(GGUF(path))
    lib = ref()
    # decode-b1 at the GPU leg's context: the cache filled with ctx0 positions of seeded random
    # K/V rows (the GPU leg's prompt plus its warm-up steps), then greedy steps from there.
    c = r.new_cache()
    row = cfg.n_head_kv * cfg.head_dim
    kv = (0.5 * rng.standard_normal(cfg.n_layer * 2 * ctx0 * row)).astype(np.float32)
    lib.ref_cache_fill(C.c_void_p(r.h), c, C.c_void_p(kv.ctypes.data), C.c_size_t(ctx0))
    del kv
    tok = int(rng.integers(0, n_vocab))
    steps, t0 = 0, time.perf_counter()
    while steps < 3 or (time.perf_counter() - t0 < budget_s and steps < 64):
        logits = r.forward_prefill(c, [tok])
        tok = int(np.argmax(logits[-1]))
        steps += 1
    dt = time.perf_counter() - t0
    b1 = {"value": steps / dt, "unit": "tokens/s", "cores": cores, "kind": "reference",
          "sample": f"{steps} greedy decode steps at contexts {ctx0 + 1}..{ctx0 + steps} (the GPU leg's), over a "
                    f"cache filled with {ctx0} seeded random positions; reference LlamaModel on its scalar "
                    f"table, {cores} threads"}
    log(f"cpu baseline b1: {b1['value']:.3f} tok/s")
    # Ragged: 32 caches filled (zeros) to the ragged contexts, then batched decode steps.
    ctx = np.random.default_rng(seed + 7).integers(64, 2049, 32)
    zeros = np.zeros(cfg.n_layer * 2 * int(ctx.max()) * cfg.n_head_kv * cfg.head_dim, np.float32)
    ids = []
    for n in ctx:
        cid = r.new_cache()
        lib.ref_cache_fill(C.c_void_p(r.h), cid, C.c_void_p(zeros.ctypes.data), C.c_size_t(int(n)))
        ids.append(cid)
    toks = rng.integers(0, n_vocab, 32).astype(np.int32)
    steps, t0 = 0, time.perf_counter()
    while steps < 1 or (time.perf_counter() - t0 < budget_s and steps < 8):
        r.forward_batch(ids, toks)
        steps += 1
    dt = time.perf_counter() - t0
    rg = {"value": 32 * steps / dt, "unit": "tokens/s", "cores": cores, "kind": "reference",
          "sample": f"{steps} forward_batch steps of 32 sequences at contexts U[64, 2048] "
                    f"(mean {float(ctx.mean()):.0f}; caches zero-filled), {cores} threads"}
    log(f"cpu baseline ragged: {rg['value']:.3f} tok/s")
    return b1, rg


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--prompt", type=int, default=512)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-ragged", action="store_true", help="skip the 32-sequence workload")
    ap.add_argument("--no-f16", action="store_true", help="skip the fp16-cache runs")
    ap.add_argument("--no-c5", action="store_true", help="skip the config-5 mixed prefill/decode workload")
    ap.add_argument("--no-sweep", action="store_true", help="skip the config-2 matvec/matmul sweep")
    ap.add_argument("--no-configs", action="store_true", help="skip the config-1 and config-3 decode-b1 legs")
    ap.add_argument("--config-only", choices=sorted(B1_CONFIGS),
                    help="only run that config's decode-b1 leg and print its figures (the workload of its profile)")
    ap.add_argument("--sweep-only", action="store_true",
                    help="only run the config-2 sweep and print its figures (the workload of its profile)")
    ap.add_argument("--c5-only", action="store_true",
                    help="only run the config-5 workload and print its figures (the workload of its profile)")
    ap.add_argument("--attention-probe", action="store_true",
                    help="only the calibration copy and the ragged-32 attention probe (counter passes)")
    ap.add_argument("--phase-probe", action="store_true",
                    help="only the persistent decode step's per-phase clock stamps (decode-b1 steps)")
    ap.add_argument("--prefill-probe", action="store_true",
                    help="only run four 512-token prefill passes (the workload of the prefill profiles)")
    ap.add_argument("--cpu-budget", type=float, default=12.0, help="seconds per CPU baseline sample")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="run the workload of the FETCH_SIZE / WRITE_SIZE counter passes and exit")
    ap.add_argument("--traffic-summary", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help=f"reduce the two counter passes to {TRAFFIC_FILE.relative_to(ROOT)} and exit")
    args = ap.parse_args()
    if args.traffic_summary:
        return traffic_summary(*args.traffic_summary)
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(on several GPUs the path would shard by sequence, one process per GPU)", file=sys.stderr)
        return 2

    import axon_hip as H
    import synth

    if args.c5_only:
        H.init(0)
        print(json.dumps(bench_c5(H, args.seed)), flush=True)
        return 0
    if args.sweep_only:
        H.init(0)
        print(json.dumps(bench_sweep(H, args.seed)), flush=True)
        return 0
    if args.config_only:
        H.init(0)
        print(json.dumps(bench_config_b1(H, args.config_only, args.warmup, args.seed)[0]), flush=True)
        return 0
    spec = synth.LLAMA32_1B
    log(f"model: {spec.name} (writing the seeded GGUF on first use)")
    t0 = time.perf_counter()
    path = synth.cached_model(spec)
    log(f"model file {path} ready in {time.perf_counter() - t0:.1f}s")
    H.init(0)
    model = H.Model(path, max_seq=512, max_ctx=2048 + 128 + 64, max_batch=32, max_caches=34)
    info = model.info
    log(f"loaded on the {model.table_name} table: {info.device_bytes / 1e9:.2f} GB in HBM, "
        f"{info.weight_bytes_per_token / 1e6:.2f} MB of weights per token; one-row passes as "
        f"{'one persistent kernel' if info.persistent_decode else 'per-layer launches'}")
    if args.traffic_probe:
        traffic_probe(H, model, info.n_vocab, min(args.steps, 16), args.prompt, args.seed)
        model.close()
        log("traffic probe done")
        return 0
    if args.attention_probe:
        attention_traffic_probe(H, model, info.n_vocab, args.seed)
        model.close()
        log("attention probe done")
        return 0
    if args.phase_probe:
        print(json.dumps(phase_probe(H, model, info.n_vocab, min(args.steps, 64), args.prompt, args.seed)), flush=True)
        model.close()
        return 0
    if args.prefill_probe:
        prefill_probe(H, model, info.n_vocab, args.seed)
        model.close()
        log("prefill probe done")
        return 0

    b1 = bench_decode_b1(H, model, info.n_vocab, args.steps, args.warmup, args.prompt, args.seed)
    log(f"decode-b1: {b1['tokens_per_s']:.1f} tok/s ({b1['ms_per_step']:.3f} ms/step)")

    ms, launches, nbytes = probe_pass(H, model, info.n_vocab, min(args.steps, 32), args.prompt, args.seed,
                                      H.PROBE_STEP if info.persistent_decode else synth.Q4_0)
    if launches == 0:
        raise SystemExit("bench.py: the Q4_0 probe recorded no launch")
    achieved = nbytes / (ms * 1e-3) / 1e9
    q6_ms, q6_n, q6_b = probe_pass(H, model, info.n_vocab, min(args.steps, 32), args.prompt, args.seed, synth.Q6_K)
    q6_gbs = q6_b / (q6_ms * 1e-3) / 1e9
    log(f"step kernel: {launches} launches, {achieved:.0f} GB/s; Q6_K: {q6_n} launches, {q6_gbs:.0f} GB/s")

    kv_pos_bytes = info.kv_bytes_per_position
    mean_ctx = 0.5 * (b1["context"][0] + b1["context"][1])
    step_bytes = info.weight_bytes_per_token + kv_pos_bytes * mean_ctx
    result = {
        "metric": METRIC,
        "value": round(b1["tokens_per_s"], 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(b1["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": "decode-b1: Llama-3.2-1B-shaped Q4_0 (tied Q6_K output), 512-token prompt, "
                               "greedy, batch 1",
                   "model": spec.name, "global_batch": 1, "seq_len": args.prompt, "parallelism": "none"},
        "hbm_gbs_per_step": round(step_bytes / (b1["ms_per_step"] * 1e-3) / 1e9, 1),
        "hbm_frac_per_step": round(step_bytes / (b1["ms_per_step"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "roofline": {"bound": "hbm", "kernel": STEP_KERNEL if info.persistent_decode else
                     "decode matvec <Q4_0>: matvec_dma_kernel (q|k|v+rope, wo+add, down+add) "
                     "and matvec_norm1_kernel (gate|up+silu)",
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "launches": launches, "bytes_per_launch": round(nbytes / max(launches, 1)),
                     "avg_us": round(1e3 * ms / max(launches, 1), 3)},
        "roofline_q6_k": {"kernel": "q6k_planar_kernel<1, 256> (tied output, 128256 x 2048, repacked at upload)",
                          "achieved": round(q6_gbs, 1), "frac": round(q6_gbs / HBM_PEAK_GBS, 4),
                          "avg_us": round(1e3 * q6_ms / max(q6_n, 1), 3)},
        "decode_path": ("one persistent kernel per step" if info.persistent_decode else
                        "per-layer launches"),
        "prefill_tokens_per_s": round(b1["prefill_tokens_per_s"], 1),
        "decode_b1_host_argmax": b1["host_argmax"],
        "decode_b1_host_ids": b1["host_ids"],
        "cpu_baseline": None,
    }
    if TRAFFIC_FILE.exists():
        t = json.loads(TRAFFIC_FILE.read_text())
        result["roofline"]["traffic"] = t["traffic_bytes_per_launch"]
        result["roofline"]["traffic_over_algorithmic"] = round(
            t["traffic_bytes_per_launch"] / max(result["roofline"]["bytes_per_launch"], 1), 3)
        result["roofline"]["traffic_source"] = str(TRAFFIC_FILE.relative_to(ROOT))
    if not args.no_ragged:
        rg = bench_ragged(H, model, info.n_vocab, args.seed)
        log(f"ragged-32: {rg['tokens_per_s']:.1f} tok/s over {rg['steps']} steps (mean batch {rg['mean_batch']:.1f})")
        result["ragged32"] = {k: (round(v, 4) if isinstance(v, float) else v) for k, v in rg.items()}
        result["ragged32"]["attention_roofline"] = probe_attention_ragged(H, model, info.n_vocab, args.seed)
        log(f"ragged-32 attention: {result['ragged32']['attention_roofline']}")
    model.close()
    if not args.no_f16:
        # The same workloads over an fp16 KV cache (LoadOptions::cache = F16): half the cache
        # bytes per position, keys and values rounded once on the way in.
        m16 = H.Model(path, max_seq=512, max_ctx=2048 + 128 + 64, max_batch=32, max_caches=34, cache="f16")
        b16 = bench_decode_b1(H, m16, info.n_vocab, args.steps, args.warmup, args.prompt, args.seed)
        log(f"decode-b1 (f16 cache): {b16['tokens_per_s']:.1f} tok/s")
        f16 = {"kv_bytes_per_position": m16.info.kv_bytes_per_position,
               "decode_b1": {"tokens_per_s": round(b16["tokens_per_s"], 2), "ms_per_step": round(b16["ms_per_step"], 4)}}
        if not args.no_ragged:
            rg16 = bench_ragged(H, m16, info.n_vocab, args.seed)
            log(f"ragged-32 (f16 cache): {rg16['tokens_per_s']:.1f} tok/s")
            f16["ragged32"] = {"tokens_per_s": round(rg16["tokens_per_s"], 3), "decode_s": round(rg16["decode_s"], 3),
                               "prefill_s": round(rg16["prefill_s"], 3)}
        m16.close()
        result["f16_cache"] = f16
    b1_paths = {}
    if not args.no_configs:
        for name in sorted(B1_CONFIGS):
            result[name], p, pr = bench_config_b1(H, name, args.warmup, args.seed)
            b1_paths[name] = (p, pr)
    if not args.no_c5:
        result["c5_mixed"] = bench_c5(H, args.seed)
    if not args.no_sweep:
        result["c2_sweep"] = bench_sweep(H, args.seed)
    if not args.no_cpu:
        b1c, rgc = cpu_baseline(path, info.n_vocab, args.seed, args.cpu_budget, args.prompt + args.warmup)
        result["cpu_baseline"] = b1c
        if b1c is not None:
            result["vs_cpu"] = round(result["value"] / b1c["value"], 1)
        if rgc is not None and "ragged32" in result:
            result["ragged32"]["cpu_baseline"] = rgc
            # Like for like: the CPU's fixed 32-row steps against the GPU's same steps.
            fixed = result["ragged32"]["attention_roofline"]["fixed_batch_tokens_per_s"]
            result["ragged32"]["vs_cpu_fixed_batch"] = round(fixed / rgc["value"], 1)
            result["ragged32"]["vs_cpu_schedule"] = round(result["ragged32"]["tokens_per_s"] / rgc["value"], 1)
        if b1c is not None:
            import synth
            for name, (p, pr) in b1_paths.items():
                prompt_len = B1_CONFIGS[name][0]
                vocab = synth.CONFIGS[name].n_vocab
                if name == "c1":  # small enough for the reference to prefill the real prompt
                    cb = cpu_decode_b1(p, vocab, args.seed, args.cpu_budget, prompt_len, prompt=pr,
                                       max_ctx=prompt_len + 96)
                else:
                    cb = cpu_decode_b1(p, vocab, args.seed, args.cpu_budget, prompt_len + args.warmup,
                                       max_ctx=prompt_len + args.warmup + 96)
                result[name]["cpu_baseline"] = cb
                result[name]["vs_cpu"] = round(result[name]["tokens_per_s"] / cb["value"], 1)
                log(f"cpu baseline {name}: {cb['value']:.3f} tok/s")
            if "c5_mixed" in result:
                lens = np.random.default_rng(args.seed + 11).integers(32, 1025, 64)
                cs = cpu_c5_step(synth.cached_model(synth.CONFIGS["c5"]), lens, args.seed)
                step = result["c5_mixed"]["mixed_step"]
                step["cpu_baseline"] = cs
                step["vs_cpu_one_pass"] = round(step["one_pass"]["tokens_per_s"] / cs["value"], 1)
                step["vs_cpu_two_pass"] = round(step["two_pass"]["tokens_per_s"] / cs["value"], 1)
                result["c5_mixed"]["cpu_baseline"] = cs
                log(f"cpu baseline c5 step: {cs['value']:.3f} tok/s")
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

"""Benchmark: per-frame CFG decode on one MI355X.

Workload (full synthetic utterance, Qwen3-0.6B shape, FP32): random-init
weights N(0, 0.02); cond prefix = 96 text ids + BOS frame + 144 prompt frames
(241 positions), uncond prefix = [bos] + BOS frame + prompt frames (146);
240 decoded frames with CFG 1.5, temperature 0.9, top-k 50, top-p 0.95 and
seeded uniform draws; one hipGraph replay per frame.  A step is one frame.

Timed region: W warm-up replays, then K replays back to back on the engine's
stream bracketed by HIP events (inputs already resident in HBM; per-frame
uniforms uploaded before the timed region).  EOS is masked on every frame
so all K frames run (the work per frame does not depend on it).

Prints one JSON line.  ``--gpus N`` with N > 1 exits: this build runs on one
GPU (utterances shard across GPUs with no per-frame exchange).

``--model q17b`` runs the larger-backbone workload instead: Qwen3-1.7B shape
(hidden 2048, SwiGLU 6144) with BF16 weights (FP32 KV and accumulation), 95
text ids + BOS frame + 144 prompt frames (240 positions), 480 decoded frames,
same sampling.

``--greedy-192`` runs the CPU-sized workload instead: Qwen3-0.6B shape, FP32,
cond prefix = 192 random text ids + BOS frame (193 positions), uncond = [bos] +
BOS frame, 32 greedy frames (4 warm-up + 28 timed by default), seed 0.

The CPU baseline (``cpu_baseline``) is the oracle in NumPy FP32 on the host
cores, on the same weights and prefixes: prefill untimed, then 4 warm-up and
16 timed frames, each frame timed alone (median and p90).  It runs the
reference's native order, cond and uncond as two B=1 branches
(soraku_inference/model.py:573-578,611-612), and beside it the same frames
with both rows batched (M = 2), so the gain from batching alone is visible.

``--kernels`` times the isolated fused kernels at decode shape M = 2 instead
(RMSNorm over 1024, SwiGLU gate/up GEMV 1024 -> 2 x 3072, down GEMV
3072 -> 1024 + residual, one classifier head 1024 -> 2051 + bias, and the
16-head classifier 1024 -> 16 x 2051 + bias as one launch; FP32 and BF16
weights): each is captured as a chain of launches over distinct weight copies
totalling more than the 256 MB last-level cache (so every launch reads HBM),
replayed, and reported per launch with its bytes and HBM fraction.

``--utterances N`` (N > 1) runs the throughput batch instead: N synthetic
utterances with CFG decoded together (decode batch 2N) at Qwen3-0.6B shape
with BF16 weights and a BF16 KV cache (FP32 accumulation; the reference's
cache takes the weights' dtype, graph_frame.py:45-52); each prefix is 120-240
tokens drawn uniformly (text ids + BOS frame + prompt frames, the prompt ~60%
of it; the uncond row is [bos] + BOS frame + the same prompt); KV capacity
512.  A step is one frame of every utterance; ``value`` is utterance-frames/s.
With ``--requests R`` (R > N) it decodes R such requests through N slots with
``FastGenerator.generate_batch`` instead: a slot whose request retires is
prefilled with the next one between frames (continuous batching), and
``value`` is decoded frames per second of wall clock, prefills, refills and
the per-frame host synchronisation included.
"""

from __future__ import annotations

import argparse
import json
import re
import os
import platform
import subprocess
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "soraku-tts_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "codec frames/sec and µs/frame (CFG batch 2) + % HBM roofline, 1 MI355X"
HBM_PEAK_GBS = 8000.0
N_TEXT, N_PROMPT, N_FRAMES = 96, 144, 240
CFG, TEMP, TOP_K, TOP_P = 1.5, 0.9, 50, 0.95
TEXT_BOS = 151643


def workload_inputs(shape, seed=0, n_text=N_TEXT, n_prompt=N_PROMPT, n_frames=N_FRAMES):
    from soraku_amd.synthetic import utterance

    text, prompt = utterance(shape, seed + 100, n_text=n_text, n_prompt=n_prompt)
    text[0] = TEXT_BOS
    uncond = np.array([TEXT_BOS], np.int64)
    u = np.random.default_rng(seed + 1).random((n_frames, shape.n_codebooks))
    return text, prompt, uncond, u


def algorithmic_bytes(shape, kv_lens, w_bytes=4, kv_bytes=4):
    """Bytes one frame must move at minimum: every weight tensor read once
    (depth MLP counted once although applied Q times), K/V of every cached
    token of every row read once, the new token's K/V written, Q table rows
    gathered.  ``kv_lens``: cached tokens per row at the frame's start.
    ``w_bytes``: bytes per matrix element (norm gains and biases stay FP32)."""
    s = shape
    per_layer = (2 * s.n_q_heads * s.head_dim * s.d_model + 2 * s.n_kv_heads * s.head_dim * s.d_model
                 + 3 * s.trunk_inter * s.d_model)
    vectors = s.n_layers * (2 * s.d_model + 2 * s.head_dim) + s.d_model + 2 * s.d_model
    trunk = s.n_layers * per_layer
    depth = 3 * s.depth_inner * s.d_model
    table = s.n_codebooks * s.audio_vocab * s.d_model
    bias = s.n_codebooks * s.audio_vocab
    weights = (trunk + depth + table) * w_bytes + (vectors + bias) * 4
    kv_token = s.n_layers * 2 * s.n_kv_heads * s.head_dim * kv_bytes
    kv = sum(kv_lens) * kv_token + len(kv_lens) * kv_token
    gather = s.n_codebooks * s.d_model * 4
    return weights + kv + gather


def cpu_info():
    """(lscpu model name, logical CPUs, CPUs this process may run on)."""
    model = ""
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                model = line.split(":", 1)[1].strip()
                break
    except (OSError, subprocess.SubprocessError):
        pass
    if not model:
        try:
            for line in open("/proc/cpuinfo"):
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
        except OSError:
            model = platform.processor() or ""
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:
        usable = os.cpu_count() or 1
    return model, os.cpu_count() or 1, usable


def cpu_baseline(shape, weights, items, u, *, temperature, n_frames=16, n_warm=4, unit="frames/s", kv_bf16=False):
    """The oracle (NumPy FP32) on the host cores over a bounded sample of the
    workload: for each (text, prompt, uncond) in ``items`` (one utterance, or a
    few of a batch), prefill untimed, then ``n_warm`` + ``n_frames`` frames,
    each timed alone, first in the reference's order (cond and uncond as two
    B=1 branches, model.py:573-578,611-612), then again from the same prefilled
    state with both rows batched (M = 2)."""
    import copy

    from threadpoolctl import threadpool_info, threadpool_limits

    from oracle.generate import generate, start_states
    from oracle.model import OracleModel, Shape

    model, nproc, usable = cpu_info()
    with threadpool_limits(limits=usable):
        threads = max([i.get("num_threads", 1) for i in threadpool_info()] or [1])
        os_shape = Shape(**{k: getattr(shape, k) for k in Shape.__dataclass_fields__})
        m = OracleModel(os_shape, weights, np.float32, kv_bf16=kv_bf16)
        kw = dict(min_new_frames=10**6, temperature=temperature, top_k=TOP_K, top_p=TOP_P, cfg_scale=CFG)
        times = {False: [], True: []}
        for i, (text, prompt, uncond) in enumerate(items):
            max_ctx = text.size + 1 + prompt.shape[0] + n_frames + n_warm + 2
            st0 = start_states(m, text, prompt, uncond, CFG, max_ctx)
            for batched in (False, True):
                st = copy.deepcopy(st0)
                for f in range(n_warm + n_frames):
                    t0 = time.perf_counter()
                    generate(m, max_new_frames=1, uniforms=u[i][f:f + 1], states=st, input_ids=text,
                             batched=batched, **kw)
                    if f >= n_warm:
                        times[batched].append(time.perf_counter() - t0)
    two, bat = np.array(times[False]) * 1e3, np.array(times[True]) * 1e3
    text, prompt, uncond = items[0]
    return {"value": 1e3 / float(np.median(two)), "unit": unit, "cores": int(threads), "kind": "port",
            "ms_per_frame_median": float(np.median(two)), "ms_per_frame_p90": float(np.percentile(two, 90)),
            "frames_timed": int(two.size), "warmup_frames": n_warm * len(items),
            "nproc": nproc, "cpus_usable": usable, "lscpu_model": model, "threads": int(threads),
            "batched_m2": {"value": 1e3 / float(np.median(bat)), "unit": unit,
                           "ms_per_frame_median": float(np.median(bat)),
                           "ms_per_frame_p90": float(np.percentile(bat, 90))},
            "sample": (f"oracle/ (NumPy FP32) on {threads} BLAS threads: {len(items)} utterance(s), prefill "
                       f"untimed, {n_warm} warm-up + {n_frames} timed frames each, every frame timed alone; "
                       f"value = 1 / median frame time with cond and uncond as separate B=1 branches "
                       f"(the reference's order); batched_m2 = both rows in one pass; prefixes "
                       f"{text.size + 1 + prompt.shape[0]}/{uncond.size + 1 + prompt.shape[0]}"
                       + ("" if len(items) == 1 else " (first utterance)"))}


PROFILES = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles")
TRAFFIC_PROFILES = {
    "q06b_f32": "hbm_traffic_decode_frame_q06b_f32.md",
    "q17b_bf16": "hbm_traffic_decode_frame_q17b_bf16.md",
    "16utt_q06b_bf16": "hbm_traffic_decode_step_16utt_q06b_bf16.md",
}


def measured_traffic(key):
    """HBM bytes per graph launch from the committed counter summary
    (FETCH_SIZE + WRITE_SIZE passes, copy-calibrated) and the rows' KV
    lengths it was measured at; (None, None) when the summary is absent."""
    try:
        text = open(os.path.join(PROFILES, TRAFFIC_PROFILES[key])).read()
    except (OSError, KeyError):
        return None, None
    m = re.search(r"```json\s*(\{.*?\})\s*```", text, re.S)
    if not m:
        return None, None
    d = json.loads(m.group(1))
    return float(d["read_bytes_per_frame"]) + float(d["write_bytes_per_frame"]), d["kv_lens"]


def roofline(shape, us, kv_mid, w_bytes, traffic_key, unit_of_work, kv_bytes=4):
    """Roofline object: algorithmic bytes at the timed frames' average KV
    lengths over the measured frame time; measured traffic with the KV state
    it was taken at and the algorithmic bytes of that same state."""
    alg = algorithmic_bytes(shape, kv_mid, w_bytes=w_bytes, kv_bytes=kv_bytes)
    achieved = alg / (us * 1e-6) / 1e9
    traffic, tkv = measured_traffic(traffic_key)
    out = {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
           "frac": achieved / HBM_PEAK_GBS, "traffic": traffic, "unit_of_work": unit_of_work,
           "algorithmic_bytes_per_launch": alg, "algorithmic_kv_lens_avg": [float(k) for k in kv_mid]}
    if traffic is not None:
        alg_t = algorithmic_bytes(shape, tkv, w_bytes=w_bytes, kv_bytes=kv_bytes)
        out.update({"traffic_source": f"profiles/{TRAFFIC_PROFILES[traffic_key]} (rocprofv3 FETCH_SIZE + "
                                      "WRITE_SIZE, copy-calibrated, bytes per launch)",
                    "traffic_kv_lens": tkv, "algorithmic_bytes_at_traffic_kv": alg_t,
                    "traffic_over_algorithmic": traffic / alg_t})
    return out


def copy_probe(mib):
    """A plain device-to-device copy of known size: reading FETCH_SIZE / WRITE_SIZE
    for it gives the factor that turns those counters into HBM bytes."""
    import torch
    n = mib * (1 << 20) // 4
    src = torch.ones(n, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(4):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_bytes_each_way": n * 4, "copies": 4}))


def many_utterances(args):
    """The throughput batch (see the module docstring); prints one JSON line."""
    import torch

    from soraku_amd import GraphFrameEngine
    from soraku_amd.config import QWEN3_06B
    from soraku_amd.synthetic import synthetic_weights

    shape, n = QWEN3_06B, args.utterances
    t_setup = time.perf_counter()
    weights = synthetic_weights(shape, args.seed)
    rng = np.random.default_rng(args.seed + 7)
    items, kv0 = [], []
    for _ in range(n):
        p_len = int(rng.integers(120, 241))
        n_prompt = int(round(0.6 * p_len))
        text = rng.integers(0, shape.text_vocab, p_len - 1 - n_prompt)
        text[0] = TEXT_BOS
        prompt = rng.integers(0, shape.codebook_size, (n_prompt, shape.n_codebooks))
        items.append((text, np.array([TEXT_BOS], np.int64), prompt))
        kv0 += [p_len, n_prompt + 2]
    u = rng.random((N_FRAMES, n * shape.n_codebooks))
    dev = torch.device("cuda:0")
    # BF16 KV cache: the reference's StaticCache takes the weights' dtype
    # (soraku_inference/acceleration/graph_frame.py:45-52)
    e = GraphFrameEngine(device=dev, max_cache_len=512, cfg_scale=CFG, batch=2, state_dict=weights, shape=shape,
                         n_utts=n, bf16=True, kv_bf16=True, max_frames=N_FRAMES)
    del weights
    e.set_temperature(TEMP)
    e.set_sampling(sampled=True, top_k=TOP_K, top_p=TOP_P)
    t0 = time.perf_counter()
    e.prefill_utterances(items)
    t_prefill = time.perf_counter() - t0
    e.capture()
    total = args.warmup + args.steps
    e.queue_frames(u[:total], np.ones(total, np.int32))
    print(f"# setup {time.perf_counter() - t_setup:.1f}s, prefill of {n} utterances {t_prefill * 1e3:.1f} ms",
          file=sys.stderr, flush=True)
    stream = torch.cuda.ExternalStream(e.stream_handle, device=dev)
    e.replay(args.warmup)
    e.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    e.replay(args.steps)
    b.record(stream)
    e.synchronize()
    torch.cuda.synchronize(dev)
    us = a.elapsed_time(b) * 1e3 / args.steps
    codes = e.read_codes(args.steps)
    assert codes.min() >= 0 and codes.max() < shape.codebook_size, "decoded a special id"
    e.close()
    kv_mid = [k + args.warmup + (args.steps - 1) / 2 for k in kv0]
    out = {
        "metric": f"codec frames/sec summed over {n} utterances (CFG, decode batch {2 * n}) + % HBM roofline, "
                  "1 MI355X",
        "value": n * 1e6 / us, "unit": "utterance-frames/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": us / 1e3, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": (f"throughput batch: {n} synthetic utterances x CFG, Qwen3-0.6B shape, BF16 "
                                "weights, BF16 KV (the reference's cache takes the weights' dtype), FP32 "
                                "accumulation, ragged prefixes 120-240, KV capacity 512, CFG 1.5, T 0.9, "
                                "top-k 50, top-p 0.95, seeded uniforms, one hipGraph per frame"),
                   "global_batch": 2 * n, "seq_len": 512, "parallelism": "none",
                   "prefill_ms": t_prefill * 1e3},
        "roofline": roofline(shape, us, kv_mid, 2, f"{n}utt_q06b_bf16",
                             "one frame of every utterance = one hipGraph launch", kv_bytes=2),
    }
    if not args.no_cpu_baseline:
        # two of the utterances (prefill is the CPU's longest part), BF16-rounded weights as on the GPU
        from oracle.model import round_bf16
        from soraku_amd.synthetic import is_matrix

        w32 = {k: (round_bf16(v) if is_matrix(k) else v) for k, v in synthetic_weights(shape, args.seed).items()}
        q = shape.n_codebooks
        cb = cpu_baseline(shape, w32, [(t, p, un) for t, un, p in items[:2]],   # items hold (text, uncond, prompt)
                          [u[:, i * q:(i + 1) * q] for i in range(2)], temperature=TEMP, unit="utterance-frames/s",
                          kv_bf16=True)
        cb["speedup"] = out["value"] / cb["value"]
        out["cpu_baseline"] = cb
    print(json.dumps(out))


def continuous_batch(args):
    """R requests through N utterance slots with refills; one JSON line."""
    import torch

    from soraku_amd import FastGenerator
    from soraku_amd.config import QWEN3_06B
    from soraku_amd.synthetic import synthetic_weights

    shape, n, R = QWEN3_06B, args.utterances, args.requests
    weights = synthetic_weights(shape, args.seed)
    rng = np.random.default_rng(args.seed + 7)
    reqs = []
    for _ in range(R):
        p_len = int(rng.integers(120, 241))
        n_prompt = int(round(0.6 * p_len))
        text = rng.integers(0, shape.text_vocab, p_len - 1 - n_prompt)
        text[0] = TEXT_BOS
        reqs.append(dict(input_ids=torch.tensor(text[None]),
                         prompt_codes=torch.tensor(rng.integers(0, shape.codebook_size, (n_prompt, shape.n_codebooks))),
                         uncond_input_ids=torch.tensor([[TEXT_BOS]])))
    g = FastGenerator(device=torch.device("cuda:0"), state_dict=weights, shape=shape, bf16=True, kv_bf16=True)
    del weights
    kw = dict(max_new_frames=N_FRAMES, min_new_frames=4, temperature=TEMP, top_k=TOP_K, top_p=TOP_P,
              cfg_scale=CFG, max_batch=n)
    g.generate_batch(reqs[:n], seeds=list(range(n)), **dict(kw, max_new_frames=8))   # engine + capture
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    out = g.generate_batch(reqs, seeds=list(range(R)), **kw)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    frames = sum(o[1]["num_frames"] for o in out)
    stops = sum(o[1]["stop_reason"] == "eos" for o in out)
    print(json.dumps({
        "metric": f"codec frames/sec over {R} requests through {n} CFG slots (continuous batching), 1 MI355X",
        "value": frames / dt, "unit": "utterance-frames/s", "n_gpus": 1, "higher_is_better": True,
        "dtype": "bf16", "data": "synthetic",
        "config": {"workload": (f"{R} synthetic requests x CFG, Qwen3-0.6B shape, BF16 weights, BF16 KV, ragged "
                                f"prefixes 120-240, up to {N_FRAMES} frames each, CFG 1.5, T 0.9, top-k 50, "
                                "top-p 0.95; a retired slot is refilled between frames"),
                   "slots": n, "requests": R, "frames_decoded": frames, "stopped_at_eos": stops,
                   "wall_s": dt, "timing": "wall clock of generate_batch (prefills, refills, host sync per frame)"},
    }))


def isolated_kernels(args):
    """The isolated-kernel measurement (see the module docstring); one JSON line."""
    import torch

    from soraku_amd import ops

    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)
    B, D, I, V, Q = 2, 1024, 3072, 2051, 16
    mall = 256 << 20

    def rnd(*shape, std=1.0, dtype=torch.float32):
        return (torch.randn(*shape, generator=gen, device=dev) * std).to(dtype)

    def timed(name, wname, calls, nbytes, reps=20):
        ref = [c().clone() for c in calls[:2]]           # eager results (and warm-up)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        outs = []
        with torch.cuda.graph(graph):
            for c in calls:
                outs.append(c())
        for _ in range(3):                                # every replay equals eager
            graph.replay()
            torch.cuda.synchronize()
            for r, o in zip(ref, outs[:2]):
                assert torch.equal(r, o), f"{name}: graph replay differs from the eager launch"
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(reps):
            graph.replay()
        b.record()
        torch.cuda.synchronize()
        us = a.elapsed_time(b) * 1e3 / (reps * len(calls))
        gbs = nbytes / us / 1e3
        return {"kernel": name, "weights": wname, "us_per_launch": us, "bytes_per_launch": nbytes,
                "achieved_gbs": gbs, "frac_of_hbm_peak": gbs / HBM_PEAK_GBS, "launches_captured": len(calls)}

    out = []
    x, g = rnd(B, D), 1.0 + 0.1 * rnd(D)
    k = ops.rmsnorm(B, D, 1e-6)
    out.append(timed("rmsnorm hidden 1024", "f32 gain", [lambda: k(x, g)] * 64, 2 * B * D * 4 + D * 4))
    for wname, dt, wb in (("f32", torch.float32, 4), ("bf16", torch.bfloat16, 2)):
        gu_bytes = 2 * I * D * wb
        n = mall // gu_bytes + 2
        wg = [rnd(I, D, std=0.02, dtype=dt) for _ in range(n)]
        wu = [rnd(I, D, std=0.02, dtype=dt) for _ in range(n)]
        k = ops.swiglu_gemv(B, I, D)
        calls = [lambda i=i: k(x, wg[i], wu[i]) for i in range(n)]
        out.append(timed("swiglu gate/up GEMV 1024 -> 2x3072", wname, calls, gu_bytes + B * D * 4 + B * I * 4))
        del wg, wu
        act = rnd(B, I)
        n = mall // (D * I * wb) + 2
        wd = [rnd(D, I, std=0.02, dtype=dt) for _ in range(n)]
        k = ops.down_residual_gemv(B, D, I)
        calls = [lambda i=i: k(act, wd[i], x) for i in range(n)]
        out.append(timed("down GEMV 3072 -> 1024 + residual", wname, calls, D * I * wb + B * I * 4 + 2 * B * D * 4))
        del wd
        n = max(2, mall // (Q * V * D * wb) + 1)
        tables = [rnd(Q, V, D, std=0.02, dtype=dt) for _ in range(n)]
        bias = rnd(Q, V, std=0.02)
        k = ops.classifier_gemv(B, V, D)
        calls = [lambda i=i, q=q: k(x, tables[i][q], bias[q]) for i in range(n) for q in range(Q)]
        out.append(timed("classifier GEMV 1024 -> 2051 + bias (one of 16 heads)", wname, calls,
                         V * D * wb + V * 4 + B * D * 4 + B * V * 4))
        # the 16 heads as one unit: [16 x 2051, 1024] in one launch
        k16 = ops.classifier_gemv(B, Q * V, D)
        flat = [t.view(Q * V, D) for t in tables]
        bias16 = bias.view(Q * V)
        calls = [lambda i=i: k16(x, flat[i], bias16) for i in range(n)]
        out.append(timed("16-head classifier GEMV 1024 -> 16 x 2051 + bias (one launch)", wname, calls,
                         Q * V * D * wb + Q * V * 4 + B * D * 4 + B * Q * V * 4))
        del tables, flat
    print(json.dumps({"metric": "isolated decode kernels at M=2: us per launch and HBM fraction, 1 MI355X",
                      "n_gpus": 1, "data": "synthetic", "unit": "us/launch",
                      "note": "per launch inside a captured chain (includes the ~1.6 us per-kernel graph floor)",
                      "kernels": out}))


def single_utterance(args, mode):
    """One utterance with CFG (see the module docstring); one JSON line."""
    import torch

    from soraku_amd import GraphFrameEngine
    from soraku_amd.config import QWEN3_06B, QWEN3_17B
    from soraku_amd.synthetic import synthetic_weights

    big = mode == "q17b"
    greedy = mode == "greedy192"
    shape = QWEN3_17B if big else QWEN3_06B
    n_text, n_prompt, n_frames = {"q17b": (95, 144, 480), "greedy192": (192, 0, 32)}.get(
        mode, (N_TEXT, N_PROMPT, N_FRAMES))
    temp = 0.0 if greedy else TEMP
    t_setup = time.perf_counter()
    weights = synthetic_weights(shape, args.seed)
    text, prompt, uncond, u = workload_inputs(shape, args.seed, n_text, n_prompt, n_frames)
    if greedy:   # 192 random ids, uncond = [bos]: both followed by the BOS frame
        text = np.random.default_rng(args.seed).integers(0, shape.text_vocab, n_text)
    dev = torch.device("cuda:0")
    max_ctx = text.size + 1 + prompt.shape[0] + n_frames + 8
    e = GraphFrameEngine(device=dev, max_cache_len=max_ctx, cfg_scale=CFG, batch=2,
                         state_dict=weights, shape=shape, max_frames=n_frames, bf16=big)
    e.set_temperature(temp)
    e.set_sampling(sampled=not greedy, top_k=TOP_K, top_p=TOP_P)
    t0 = time.perf_counter()
    e.prefill(text, uncond, prompt)
    t_prefill = time.perf_counter() - t0
    e.capture()
    total = args.warmup + args.steps
    e.queue_frames(u[:total], np.ones(total, np.int32))
    kv0 = [text.size + 1 + prompt.shape[0], uncond.size + 1 + prompt.shape[0]]
    print(f"# {mode}: setup {time.perf_counter() - t_setup:.1f}s, prefill {t_prefill * 1e3:.1f} ms",
          file=sys.stderr, flush=True)

    stream = torch.cuda.ExternalStream(e.stream_handle, device=dev)
    e.replay(args.warmup)
    e.synchronize()
    torch.cuda.synchronize(dev)
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
    evs[0].record(stream)
    for i in range(args.steps):
        e.replay(1)
        evs[i + 1].record(stream)
    e.synchronize()
    torch.cuda.synchronize(dev)
    per = np.array([evs[i].elapsed_time(evs[i + 1]) for i in range(args.steps)]) * 1e3  # us
    total_ms = evs[0].elapsed_time(evs[-1])
    codes = e.read_codes(args.steps)
    assert codes.min() >= 0 and codes.max() < shape.codebook_size, "decoded a special id"
    e.close()

    us = total_ms * 1e3 / args.steps
    kv_mid = [k + args.warmup + (args.steps - 1) / 2 for k in kv0]
    workload = {
        "q17b": ("larger backbone, Qwen3-1.7B shape, BF16 weights (FP32 KV and accumulation): 95 text ids + "
                 "144 prompt frames (240 positions), 480 frames, CFG 1.5, T 0.9, top-k 50, top-p 0.95, "
                 "seeded uniforms, one hipGraph per frame"),
        "greedy192": ("CPU-sized greedy utterance, Qwen3-0.6B shape FP32: 192 random text ids + BOS frame "
                      "(uncond [bos] + BOS frame), 32 greedy frames, CFG 1.5, seed 0, one hipGraph per frame"),
    }.get(mode, "full synthetic utterance, Qwen3-0.6B shape FP32: 96 text ids + 144 prompt frames, CFG 1.5, "
                "T 0.9, top-k 50, top-p 0.95, seeded uniforms, one hipGraph per frame")
    out = {
        "metric": METRIC, "value": 1e6 / us, "unit": "frames/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": us / 1e3, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16" if big else "f32", "data": "synthetic",
        "config": {"workload": workload,
                   "global_batch": 2, "seq_len": int(kv0[0] + n_frames), "parallelism": "none",
                   "us_per_frame_median": float(np.median(per)),
                   "us_per_frame_p90": float(np.percentile(per, 90)),
                   "prefill_ms": t_prefill * 1e3},
        "roofline": roofline(shape, us, kv_mid, 2 if big else 4,
                             "q17b_bf16" if big else ("q06b_f32" if mode == "full" else None),
                             "one frame = one hipGraph launch"),
    }
    if not args.no_cpu_baseline:
        if big:
            from oracle.model import round_bf16
            from soraku_amd.synthetic import is_matrix

            weights = {k: (round_bf16(v) if is_matrix(k) else v) for k, v in weights.items()}
        cb = cpu_baseline(shape, weights, [(text, prompt, uncond)], [u], temperature=temp,
                          n_frames=16, n_warm=4)
        cb["speedup"] = out["value"] / cb["value"]
        out["cpu_baseline"] = cb
    print(json.dumps(out))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None, help="timed frames (default 200; 28 with --greedy-192)")
    ap.add_argument("--warmup", type=int, default=None, help="untimed frames first (default 8; 4 with --greedy-192)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--model", choices=("q06b", "q17b"), default="q06b",
                    help="q17b: Qwen3-1.7B shape with BF16 weights, 240-position prefix, 480 frames")
    ap.add_argument("--greedy-192", action="store_true",
                    help="the CPU-sized workload: 0.6B FP32, 192 random text ids, 32 greedy frames")
    ap.add_argument("--kernels", action="store_true",
                    help="time the isolated fused kernels at M=2 (FP32 and BF16 weights) instead")
    ap.add_argument("--utterances", type=int, default=1,
                    help="N > 1: the throughput batch of N utterances x CFG (BF16 weights) instead")
    ap.add_argument("--requests", type=int, default=0,
                    help="with --utterances N: decode this many requests through the N slots (refills)")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="only run 4 device copies of MIB MiB each (HBM counter calibration) and exit")
    args = ap.parse_args()
    if args.copy_probe:
        copy_probe(args.copy_probe)
        return
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for {args.gpus}): utterances shard across GPUs "
              "with no per-frame exchange, so the per-GPU figure is the N=1 line.", file=sys.stderr)
        sys.exit(2)
    mode = "q17b" if args.model == "q17b" else ("greedy192" if args.greedy_192 else "full")
    if args.steps is None:
        args.steps = 28 if mode == "greedy192" else 200
    if args.warmup is None:
        args.warmup = 4 if mode == "greedy192" else 8
    n_frames = {"q17b": 480, "greedy192": 32}.get(mode, N_FRAMES)
    if args.steps + args.warmup > n_frames:
        sys.exit(f"steps + warmup must be <= {n_frames} (the workload's decoded frames)")
    if args.kernels:
        isolated_kernels(args)
        return
    if args.utterances > 1 and args.requests > args.utterances:
        continuous_batch(args)
        return
    if args.utterances > 1:
        many_utterances(args)
        return
    single_utterance(args, mode)


if __name__ == "__main__":
    main()

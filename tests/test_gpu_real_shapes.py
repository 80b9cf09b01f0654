"""Sampled decoding at the benchmark shapes and prefix lengths, against the
reference's vectors and the oracle.

* Qwen3-0.6B, FP32, the full-utterance prefix (96 text ids + BOS frame + 144
  prompt frames = 241 positions for the cond row, text BOS + BOS frame + the
  prompt = 146 for the uncond row), CFG 1.5, T 0.9, top-k 50, top-p 0.95:
  teacher-forced logits and V = 2051 distributions against the reference
  (``q06b_sampled`` fixture), then free-running decode against the float64
  oracle under identical uniforms.
* Qwen3-0.6B with 543 / 448 cached positions: decode attention crosses a
  32-token chunk edge and merges more than 16 chunks (contexts above 512).
* Qwen3-1.7B, BF16 weights, 240-position prefix, sampled.
* The XCD-resident trunk layers (the path these two-row engines take)
  against the per-op layer kernels, at both shapes, and with more chunk slots
  than an XCD has workgroups.
* Two engines with XCD-resident layers taking turns on one GPU (queued
  replays on two streams, no host sync; one engine's prefill beside the
  other's queued frames): codes equal each engine's alone.
* The XCD-resident layers after a frame with the utterance retired, then a
  new prefill or a continuous-batching refill: equal to a fresh engine.
* An untied classifier head bound through ``GraphFrameEngine(model=...)``.

Tolerance: logits within 1e-3 of the reference / oracle, relative to the
row's largest |logit|.  Codes: equal under identical uniforms; a difference is
accepted only where the oracle's uniform lies within 1e-5 of a CDF boundary
of its own distribution (or its top-p mass within 1e-5 of the threshold),
i.e. where a sub-tolerance logit difference can move the draw, and the
comparison stops there.
"""

import dataclasses

import numpy as np
import pytest

from conftest import load_golden
from oracle.generate import Record, generate, start_states
from oracle.model import QWEN3_06B, QWEN3_17B, OracleModel, synthetic_weights
from oracle.sampler import apply_masks, candidates, filtered_probs, topp_weights

pytestmark = pytest.mark.gpu

LOGIT_TOL = 1e-3
MARGIN = 1e-5
C3 = dict(cfg_scale=1.5, temperature=0.9, top_k=50, top_p=0.95, min_new_frames=8)


def _shape(s):
    from soraku_amd.config import DecodeShape

    return DecodeShape(**{k: getattr(s, k) for k in DecodeShape.__dataclass_fields__})


def _rowwise_rel(got, ref):
    got, ref = np.atleast_2d(got), np.atleast_2d(ref)
    fin = np.isfinite(ref)
    assert (np.isfinite(got) == fin).all()
    num = np.abs(np.where(fin, got, 0) - np.where(fin, ref, 0)).max(axis=-1)
    den = np.abs(np.where(fin, ref, 0)).max(axis=-1)
    return float((num / den).max())


def _engine(s, w, hip_device, text, uncond, prompt, max_ctx, bf16=False, **gen):
    from soraku_amd import GraphFrameEngine

    e = GraphFrameEngine(device=hip_device, max_cache_len=max_ctx, cfg_scale=gen["cfg_scale"], batch=2,
                         state_dict=w, shape=_shape(s), bf16=bf16)
    e.set_temperature(gen["temperature"])
    e.set_sampling(sampled=gen["temperature"] > 0, top_k=gen["top_k"], top_p=gen["top_p"])
    e.set_debug(True)
    e.prefill(text, uncond, prompt)
    e.capture()
    return e


def _draw_margin(masked, gen, u):
    """Distance of u from the nearest CDF boundary of the oracle's filtered
    distribution, and of the top-p mass from its threshold."""
    x = (np.asarray(masked, np.float32) / np.float32(gen["temperature"])).astype(np.float32)
    order = candidates(x, gen["top_k"])
    _, W, n_keep = topp_weights(x[order], gen["top_p"])
    F = W[:n_keep] / W[n_keep - 1]
    m_u = float(np.min(np.abs(F - u)))
    m_p = float(np.min(np.abs(W / W[-1] - float(np.float32(gen["top_p"])))))
    return min(m_u, m_p)


def _free_running_vs_oracle(e, m, states, s, u, gen, text, prompt, uncond):
    """Decode len(u) frames on the engine and the oracle with the same
    uniforms; compare every step's masked logits and code.  Returns
    (frames compared in full, largest logit error)."""
    n = u.shape[0]
    rec = Record()
    ref, _ = generate(m, input_ids=text, prompt_codes=prompt, uncond_input_ids=uncond, uniforms=u,
                      max_new_frames=n, batched=True, record=rec, states=states, **gen)
    worst = 0.0
    for fi in range(n):
        codes, lg = e.step_frame(mask_eos_q0=fi < gen["min_new_frames"], uniforms=u[fi], return_logits=True)
        codes = codes.numpy().reshape(-1)
        oracle_eos = fi >= ref.shape[0]          # the oracle drew EOS at q0 of this frame
        for q in range(len(rec.merged[fi])):
            want = apply_masks(rec.merged[fi][q], q=q, frame_index=fi, min_new_frames=gen["min_new_frames"],
                               bos_id=s.bos_id, eos_id=s.eos_id, pad_id=s.pad_id)
            rel = _rowwise_rel(lg[0][q], want)
            worst = max(worst, rel)
            assert rel < LOGIT_TOL, (fi, q, rel)
            want_code = s.eos_id if oracle_eos else ref[fi][q]
            if codes[q] != want_code:
                margin = _draw_margin(want, gen, float(u[fi][q]))
                print(f"codes differ at frame {fi} codebook {q}: engine {codes[q]}, oracle {want_code}, "
                      f"margin {margin:.2e}")
                assert margin < MARGIN
                return fi, worst
        if oracle_eos:
            return fi, worst
    return n, worst


def _c3_inputs(f):
    return f["text_ids"], f["uncond_ids"], f["prompt_codes"]


def test_c3_prefix_teacher_forced_matches_reference(hip_device):
    """Teacher-forced on the reference's own codes: masked CFG logits of every
    depth step and the top-k / top-p distribution handed to torch.multinomial
    (V = 2051), from GPU logits, equal the reference's."""
    f, s, gen = load_golden("q06b_sampled")
    assert f["text_ids"].size + 1 + f["prompt_codes"].shape[0] == 241
    w = synthetic_weights(s, int(f["seed"]), norm_gain_std=float(f["norm_gain_std"]),
                          bias_std=float(f["bias_std"]))
    text, uncond, prompt = _c3_inputs(f)
    g = {k: gen[k] for k in ("cfg_scale", "temperature", "top_k", "top_p")}
    e = _engine(s, w, hip_device, text, uncond, prompt, 260, **g)
    assert e.xcd_layers   # two decode rows at the 0.6B shape: the XCD-resident trunk layers
    hid = e.hidden()
    assert np.abs(hid - f["hidden"][0]).max() / np.abs(f["hidden"][0]).max() < 1e-4
    got = []
    for fi in range(f["codes"].shape[0]):
        _, lg = e.step_frame(mask_eos_q0=True, uniforms=np.zeros(s.n_codebooks), forced_codes=f["codes"][fi],
                             return_logits=True)
        got.extend(lg[0])
        hid = e.hidden()
        assert np.abs(hid - f["hidden"][fi + 1]).max() / np.abs(f["hidden"][fi + 1]).max() < 1e-4
    e.close()
    got = np.stack(got)
    rel = _rowwise_rel(got, f["sample_logits"])
    print(f"C3 prefix, 0.6B FP32: max row-relative logit error vs reference {rel:.3e}")
    assert rel < LOGIT_TOL
    worst = 0.0
    for i, lg in enumerate(got):
        pr = filtered_probs((lg / np.float32(gen["temperature"])).astype(np.float32), gen["top_k"], gen["top_p"])
        np.testing.assert_array_equal(pr > 0, f["probs"][i] > 0)
        worst = max(worst, float(np.abs(pr - f["probs"][i]).max()))
    print(f"C3 prefix: max |p_gpu - p_reference| {worst:.2e}")
    assert worst < 1e-4


def test_c3_prefix_sampled_codes_match_oracle(hip_device):
    """Free-running sampled decode at the C3 settings: 10 frames of 16
    codebooks, codes and logits against the float64 oracle under identical
    uniforms."""
    f, s, _ = load_golden("q06b_sampled")
    w = synthetic_weights(s, int(f["seed"]), norm_gain_std=float(f["norm_gain_std"]),
                          bias_std=float(f["bias_std"]))
    text, uncond, prompt = _c3_inputs(f)
    n = 10
    u = np.random.default_rng(240).random((n, s.n_codebooks))
    m = OracleModel(s, w, np.float64)
    states = start_states(m, text, prompt, uncond, C3["cfg_scale"], 260)
    e = _engine(s, w, hip_device, text, uncond, prompt, 260, **C3)
    done, worst = _free_running_vs_oracle(e, m, states, s, u, C3, text, prompt, uncond)
    e.close()
    print(f"C3 sampled: {done} frames equal, max logit error {worst:.3e}")
    assert done >= 6


def test_q06b_context_past_512_tokens(hip_device):
    """Cond row 543 cached positions, uncond 448, KV capacity 600: decode
    attention merges 17-18 chunks of 32 (past the merge kernel's first
    block of 16) and the frames cross the chunk edge at 544 (cond) and start
    a chunk at 448 (uncond); teacher-forced logits against the float64
    oracle, then sampled codes."""
    s = dataclasses.replace(QWEN3_06B, text_vocab=4096)
    w = synthetic_weights(s, 12, norm_gain_std=0.1, bias_std=0.02)
    rng = np.random.default_rng(12)
    text = rng.integers(0, s.text_vocab, 96)
    prompt = rng.integers(0, s.codebook_size, (446, s.n_codebooks))
    uncond = np.array([7])
    assert text.size + 1 + prompt.shape[0] == 543 and uncond.size + 1 + prompt.shape[0] == 448
    m = OracleModel(s, w, np.float64)
    states = start_states(m, text, prompt, uncond, C3["cfg_scale"], 600)
    e = _engine(s, w, hip_device, text, uncond, prompt, 600, **C3)
    u = np.random.default_rng(13).random((4, s.n_codebooks))
    done, worst = _free_running_vs_oracle(e, m, states, s, u, C3, text, prompt, uncond)
    e.close()
    print(f"0.6B at 543/448 positions: {done} frames equal, max logit error {worst:.3e}")
    assert done >= 3


def test_q17b_c5_prefix_sampled(hip_device):
    """Qwen3-1.7B shape, BF16 weights (FP32 accumulation, FP32 KV), 240-position
    prefix (95 text ids + BOS frame + 144 prompt frames; uncond 146), sampled
    at T 0.9, top-k 50, top-p 0.95, CFG 1.5: logits and codes against the
    float64 oracle on the same BF16-rounded weights."""
    from test_gpu_engine import _device_weights

    s = dataclasses.replace(QWEN3_17B, text_vocab=4096)
    w = _device_weights(s, 240, hip_device)
    rng = np.random.default_rng(240)
    text = rng.integers(0, s.text_vocab, 95)
    prompt = rng.integers(0, s.codebook_size, (144, s.n_codebooks))
    uncond = np.array([11])
    m = OracleModel(s, w, np.float64)
    states = start_states(m, text, prompt, uncond, C3["cfg_scale"], 260)
    e = _engine(s, w, hip_device, text, uncond, prompt, 260, bf16=True, **C3)
    assert e.xcd_layers   # two decode rows at the 1.7B shape, BF16: the XCD-resident trunk layers
    u = np.random.default_rng(241).random((4, s.n_codebooks))
    done, worst = _free_running_vs_oracle(e, m, states, s, u, C3, text, prompt, uncond)
    e.close()
    print(f"1.7B BF16 at 240/146 positions: {done} frames equal, max logit error {worst:.3e}")
    assert done >= 3


@pytest.mark.parametrize("model", ["q06b", "q17b", "q17b_f32"])
def test_xcd_layers_match_per_op_layers(hip_device, monkeypatch, model):
    """The XCD-resident trunk layers (two launches per layer, projections
    summed as 8 per-XCD partials) against the per-op layer kernels
    (SORAKU_XCD_LAYERS=0) on the same weights and prefix: teacher-forced
    masked logits of every depth step within 1e-4 row-relative (two FP32
    summation orders of the same projections; measured 7e-7 at 0.6B, 3e-6 at
    1.7B), 4 frames, at the C3 (0.6B FP32) and C5 (1.7B BF16, and the same
    BF16-valued weights held as FP32) prefixes."""
    if model == "q06b":
        f, s, _ = load_golden("q06b_sampled")
        w = synthetic_weights(s, int(f["seed"]), norm_gain_std=float(f["norm_gain_std"]),
                              bias_std=float(f["bias_std"]))
        text, uncond, prompt = _c3_inputs(f)
        bf16 = False
    else:
        from test_gpu_engine import _device_weights

        s = dataclasses.replace(QWEN3_17B, text_vocab=4096)
        w = _device_weights(s, 240, hip_device)
        rng = np.random.default_rng(240)
        text = rng.integers(0, s.text_vocab, 95)
        prompt = rng.integers(0, s.codebook_size, (144, s.n_codebooks))
        uncond = np.array([11])
        bf16 = model == "q17b"
    g = {k: C3[k] for k in ("cfg_scale", "temperature", "top_k", "top_p")}
    e = _engine(s, w, hip_device, text, uncond, prompt, 260, bf16=bf16, **g)
    monkeypatch.setenv("SORAKU_XCD_LAYERS", "0")
    r = _engine(s, w, hip_device, text, uncond, prompt, 260, bf16=bf16, **g)
    monkeypatch.delenv("SORAKU_XCD_LAYERS")
    assert e.xcd_layers and not r.xcd_layers
    codes = np.random.default_rng(7).integers(0, s.codebook_size, (4, s.n_codebooks))
    worst = 0.0
    for fi in range(codes.shape[0]):
        step = dict(mask_eos_q0=True, uniforms=np.zeros(s.n_codebooks), forced_codes=codes[fi], return_logits=True)
        _, a = e.step_frame(**step)
        _, b = r.step_frame(**step)
        rel = _rowwise_rel(np.asarray(a[0]), np.asarray(b[0]))
        worst = max(worst, rel)
        assert rel < 1e-4, (fi, rel)
    e.close()
    r.close()
    print(f"{model}: XCD-resident vs per-op layers, max row-relative logit difference {worst:.3e}")


def test_xcd_layers_two_slots_per_workgroup(hip_device, monkeypatch):
    """Cond row 657 cached positions, uncond 562: 21 + 18 = 39 chunk slots, more
    than the 32 workgroups of an XCD, so some take a second slot (the
    attention half's slot loop, which the C5 frames past ~512 positions use).
    Teacher-forced masked logits of the XCD-resident layers against the per-op
    layer kernels within 1e-4 row-relative, 3 frames."""
    s = dataclasses.replace(QWEN3_06B, text_vocab=4096)
    w = synthetic_weights(s, 21, norm_gain_std=0.1, bias_std=0.02)
    rng = np.random.default_rng(21)
    text = rng.integers(0, s.text_vocab, 96)
    prompt = rng.integers(0, s.codebook_size, (560, s.n_codebooks))
    uncond = np.array([5])
    assert text.size + 1 + prompt.shape[0] == 657 and uncond.size + 1 + prompt.shape[0] == 562
    g = {k: C3[k] for k in ("cfg_scale", "temperature", "top_k", "top_p")}
    e = _engine(s, w, hip_device, text, uncond, prompt, 700, **g)
    monkeypatch.setenv("SORAKU_XCD_LAYERS", "0")
    r = _engine(s, w, hip_device, text, uncond, prompt, 700, **g)
    monkeypatch.delenv("SORAKU_XCD_LAYERS")
    assert e.xcd_layers and not r.xcd_layers
    codes = np.random.default_rng(22).integers(0, s.codebook_size, (3, s.n_codebooks))
    worst = 0.0
    for fi in range(codes.shape[0]):
        step = dict(mask_eos_q0=True, uniforms=np.zeros(s.n_codebooks), forced_codes=codes[fi], return_logits=True)
        _, a = e.step_frame(**step)
        _, b = r.step_frame(**step)
        rel = _rowwise_rel(np.asarray(a[0]), np.asarray(b[0]))
        worst = max(worst, rel)
        assert rel < 1e-4, (fi, rel)
    e.close()
    r.close()
    print(f"two slots per workgroup (657/562 positions): max row-relative logit difference {worst:.3e}")


def _teacher_forced_vs_oracle(e, m, states, s, text, prompt, uncond, codes, cfg):
    """Masked merged logits of every depth step, teacher-forced on `codes`,
    engine against the oracle from its prefilled `states`; the largest
    row-relative error."""
    from test_gpu_engine import _engine_forced_logits, _oracle_forced_logits

    ref = _oracle_forced_logits(m, s, text, prompt, uncond, codes, cfg, states=states)
    got = _engine_forced_logits(e, s, codes)
    return _rowwise_rel(got, ref)


def _long_prefix_vs_oracle(s, w, hip_device, text, uncond, prompt, max_ctx, bf16, seed):
    """Teacher-forced logits over 3 frames, then sampled codes over 4 frames
    (each on its own engine) against the float64 oracle at a long prefix."""
    import copy

    m = OracleModel(s, w, np.float64)
    states = start_states(m, text, prompt, uncond, C3["cfg_scale"], max_ctx)
    g = {k: C3[k] for k in ("cfg_scale", "temperature", "top_k", "top_p")}
    e = _engine(s, w, hip_device, text, uncond, prompt, max_ctx, bf16=bf16, **g)
    assert e.xcd_layers
    codes = np.random.default_rng(seed).integers(0, s.codebook_size, (3, s.n_codebooks))
    rel = _teacher_forced_vs_oracle(e, m, copy.deepcopy(states), s, text, prompt, uncond, codes, C3["cfg_scale"])
    e.close()
    print(f"teacher-forced, 3 frames: max row-relative logit error {rel:.3e}", flush=True)
    assert rel < LOGIT_TOL
    e = _engine(s, w, hip_device, text, uncond, prompt, max_ctx, bf16=bf16, **C3)
    u = np.random.default_rng(seed + 1).random((4, s.n_codebooks))
    done, worst = _free_running_vs_oracle(e, m, states, s, u, C3, text, prompt, uncond)
    e.close()
    print(f"sampled: {done} frames equal, max logit error {worst:.3e}")
    assert done >= 3
    return rel, worst


def test_q06b_two_slots_per_workgroup_vs_oracle(hip_device):
    """Qwen3-0.6B FP32 with 657 / 562 cached positions: 21 + 18 = 39 chunk
    slots of the XCD-resident attention half, more than the 32 workgroups
    of an XCD, so workgroups 0-6 take a second slot (K/V loads after the
    first slot's barrier, the merge over more than 16 chunks); teacher-forced
    logits and sampled codes against the float64 oracle."""
    s = dataclasses.replace(QWEN3_06B, text_vocab=4096)
    w = synthetic_weights(s, 21, norm_gain_std=0.1, bias_std=0.02)
    rng = np.random.default_rng(21)
    text = rng.integers(0, s.text_vocab, 96)
    prompt = rng.integers(0, s.codebook_size, (560, s.n_codebooks))
    uncond = np.array([5])
    assert text.size + 1 + prompt.shape[0] == 657 and uncond.size + 1 + prompt.shape[0] == 562
    _long_prefix_vs_oracle(s, w, hip_device, text, uncond, prompt, 680, False, 23)


def test_q17b_late_frame_contexts_vs_oracle(hip_device):
    """Qwen3-1.7B shape, BF16 weights, FP32 KV, at the contexts the last of
    C5's 480 frames reach: cond 720 positions (95 text ids + BOS frame + 624
    prompt frames, through the batched prefill), uncond 626.  That is 23 + 20
    = 43 chunk slots at d = 2048, so every XCD's workgroups 0-10 take a
    second slot; teacher-forced logits (3 frames) and sampled codes (4
    frames) against the float64 oracle on the same BF16-rounded weights
    (model.py:567-612, graph_frame.py:247-270)."""
    from test_gpu_engine import _device_weights

    s = dataclasses.replace(QWEN3_17B, text_vocab=4096)
    w = _device_weights(s, 720, hip_device)
    rng = np.random.default_rng(720)
    text = rng.integers(0, s.text_vocab, 95)
    prompt = rng.integers(0, s.codebook_size, (624, s.n_codebooks))
    uncond = np.array([13])
    assert text.size + 1 + prompt.shape[0] == 720 and uncond.size + 1 + prompt.shape[0] == 626
    _long_prefix_vs_oracle(s, w, hip_device, text, uncond, prompt, 740, True, 721)


def test_barrier_timeout_reports_error_and_fresh_engine_decodes(hip_device):
    """The XCD-resident layers' bounded waits, forced to give up from the
    host (sk_debug_set_spin_ticks(e, 0): every barrier or exchange wait that
    does not find its data at the first look ends): every kernel still
    exits, sk_step_frame returns SK_EHIP with its message soon after, and a
    freshly created engine on the same weights then decodes the C3 prefix's
    first teacher-forced frame as the reference did."""
    import time

    from soraku_amd._lib import SK_EHIP, SK_ESTATE, SkError, check, lib

    f, s, gen = load_golden("q06b_sampled")
    w = synthetic_weights(s, int(f["seed"]), norm_gain_std=float(f["norm_gain_std"]),
                          bias_std=float(f["bias_std"]))
    text, uncond, prompt = _c3_inputs(f)
    g = {k: gen[k] for k in ("cfg_scale", "temperature", "top_k", "top_p")}
    from soraku_amd import GraphFrameEngine

    e = GraphFrameEngine(device=hip_device, max_cache_len=260, cfg_scale=g["cfg_scale"], batch=2, state_dict=w,
                         shape=_shape(s))
    e.set_temperature(g["temperature"])
    e.set_sampling(sampled=True, top_k=g["top_k"], top_p=g["top_p"])
    e.prefill(text, uncond, prompt)
    check(lib().sk_debug_set_spin_ticks(e._h, 0))
    e.capture()
    assert e.xcd_layers
    with pytest.raises(SkError) as ei:
        check(lib().sk_debug_set_spin_ticks(e._h, 0))
    assert ei.value.code == SK_ESTATE   # only before capture
    t0 = time.time()
    with pytest.raises(SkError) as ei:
        e.step_frame(mask_eos_q0=True, uniforms=np.zeros(s.n_codebooks), forced_codes=f["codes"][0])
    dt = time.time() - t0
    print(f"forced timeout: {ei.value} after {dt:.3f} s", flush=True)
    assert ei.value.code == SK_EHIP and "barrier timed out" in str(ei.value)
    assert dt < 5.0
    e.close()
    e = _engine(s, w, hip_device, text, uncond, prompt, 260, **g)
    _, lg = e.step_frame(mask_eos_q0=True, uniforms=np.zeros(s.n_codebooks), forced_codes=f["codes"][0],
                         return_logits=True)
    e.synchronize()
    e.close()
    rel = _rowwise_rel(lg[0], f["sample_logits"][: s.n_codebooks])
    print(f"fresh engine after the timeout: row-relative logit error vs reference {rel:.3e}")
    assert rel < LOGIT_TOL


def test_two_engines_take_turns_on_one_gpu(hip_device):
    """Two engines with XCD-resident layers on one GPU, each on its own
    stream, replaying queued frames in turns with no host sync between them.
    Each launch's barriers need all of its workgroups resident; the device's
    frame order makes each engine's frames wait for the other's, so no
    barrier times out, and each engine's codes equal those it decodes alone
    (replays are bitwise deterministic)."""
    f, s, gen = load_golden("q06b_sampled")
    w = synthetic_weights(s, int(f["seed"]), norm_gain_std=float(f["norm_gain_std"]),
                          bias_std=float(f["bias_std"]))
    text, uncond, prompt = _c3_inputs(f)
    g = {k: gen[k] for k in ("cfg_scale", "temperature", "top_k", "top_p")}
    n = 8
    u = [np.random.default_rng(11 + i).random((n, s.n_codebooks)) for i in range(2)]
    mask = np.ones(n, np.int32)
    prompts = [prompt, prompt[:100]]   # 241 / 197 cond positions

    def make(i):
        e = _engine(s, w, hip_device, text, uncond, prompts[i], 260, **g)
        assert e.xcd_layers
        e.queue_frames(u[i], mask)
        return e

    alone = []
    for i in range(2):
        e = make(i)
        e.replay(n)
        alone.append(e.read_codes(n))
        e.close()
    engines = [make(0), make(1)]
    for _ in range(0, n, 2):
        for e in engines:
            e.replay(2)
    got = [e.read_codes(n) for e in engines]
    for e in engines:
        e.close()
    print("codes alone:", [a[:2, 0, :4].tolist() for a in alone], flush=True)
    for i in range(2):
        np.testing.assert_array_equal(got[i], alone[i])
    assert not np.array_equal(alone[0], alone[1])


def test_prefill_beside_another_engines_queued_frames(hip_device):
    """One engine's queued frames (no host sync) and a second engine's prefill,
    capture and frames enqueued meanwhile: in the device order of engines the
    prefill waits for the queued frames, and both engines' codes equal those
    they decode alone."""
    f, s, gen = load_golden("q06b_sampled")
    w = synthetic_weights(s, int(f["seed"]), norm_gain_std=float(f["norm_gain_std"]),
                          bias_std=float(f["bias_std"]))
    text, uncond, prompt = _c3_inputs(f)
    g = {k: gen[k] for k in ("cfg_scale", "temperature", "top_k", "top_p")}
    n = 8
    u = np.random.default_rng(13).random((n, s.n_codebooks))
    mask = np.ones(n, np.int32)

    def first():
        e = _engine(s, w, hip_device, text, uncond, prompt, 260, **g)
        e.queue_frames(u, mask)
        return e

    def second_codes(e):
        return np.stack([e.step_frame(mask_eos_q0=True, uniforms=u[i]).numpy() for i in range(3)])

    e = first()
    e.replay(n)
    alone_a = e.read_codes(n)
    e.close()
    e = _engine(s, w, hip_device, text, uncond, prompt[:100], 260, **g)
    alone_b = second_codes(e)
    e.close()
    a = first()
    a.replay(n)                                   # queued, not waited for
    b = _engine(s, w, hip_device, text, uncond, prompt[:100], 260, **g)
    got_b = second_codes(b)
    got_a = a.read_codes(n)
    a.close()
    b.close()
    np.testing.assert_array_equal(got_a, alone_a)
    np.testing.assert_array_equal(got_b, alone_b)


def test_xcd_layers_frame_with_retired_rows_then_prefill(hip_device):
    """The XCD-resident layers' residual accumulators across a retired
    utterance: an engine decodes one frame, retires its utterance, runs one
    frame with both rows retired (the next frame's first-layer accumulator
    must still be cleared for them), then prefills the C3 prefix again; its
    teacher-forced frames then equal a fresh engine's (same codes, logits
    within 1e-6 of the fresh engine's and within 1e-3 of the reference)."""
    f, s, gen = load_golden("q06b_sampled")
    w = synthetic_weights(s, int(f["seed"]), norm_gain_std=float(f["norm_gain_std"]),
                          bias_std=float(f["bias_std"]))
    text, uncond, prompt = _c3_inputs(f)
    g = {k: gen[k] for k in ("cfg_scale", "temperature", "top_k", "top_p")}
    z = np.zeros(s.n_codebooks)

    def frames(e, n):
        out = [e.step_frame(mask_eos_q0=True, uniforms=z, forced_codes=f["codes"][i], return_logits=True)
               for i in range(n)]
        return np.stack([c.numpy() for c, _ in out]), np.stack([lg[0] for _, lg in out])

    e = _engine(s, w, hip_device, text, uncond, prompt[:100], 270, **g)
    assert e.xcd_layers
    frames(e, 1)
    e.retire(0)
    e.step_frame(mask_eos_q0=True, uniforms=z)
    e.prefill(text, uncond, prompt)
    got = frames(e, 2)
    e.close()
    e = _engine(s, w, hip_device, text, uncond, prompt, 270, **g)
    want = frames(e, 2)
    e.close()
    np.testing.assert_array_equal(got[0], want[0])
    rel = _rowwise_rel(got[1].reshape(-1, got[1].shape[-1]), want[1].reshape(-1, want[1].shape[-1]))
    ref = _rowwise_rel(got[1].reshape(-1, got[1].shape[-1]), f["sample_logits"][: 2 * s.n_codebooks])
    print(f"after a frame with retired rows and a new prefill: vs fresh engine {rel:.3e}, vs reference {ref:.3e}")
    assert rel < 1e-6 and ref < LOGIT_TOL


def test_xcd_layers_refill_after_retired_frame(hip_device):
    """Continuous batching on the XCD-resident layers (one utterance slot):
    decode one frame, retire the utterance, run one frame with the slot
    retired, then refill the slot with the C3 prefix (the frame counter keeps
    running).  Its teacher-forced frames equal a fresh engine's (same codes,
    logits within 1e-6 of the fresh engine's and within 1e-3 of the
    reference)."""
    f, s, gen = load_golden("q06b_sampled")
    w = synthetic_weights(s, int(f["seed"]), norm_gain_std=float(f["norm_gain_std"]),
                          bias_std=float(f["bias_std"]))
    text, uncond, prompt = _c3_inputs(f)
    g = {k: gen[k] for k in ("cfg_scale", "temperature", "top_k", "top_p")}
    z = np.zeros(s.n_codebooks)

    def frames(e, n):
        out = [e.step_frame(mask_eos_q0=True, uniforms=z, forced_codes=f["codes"][i], return_logits=True)
               for i in range(n)]
        return np.stack([c.numpy() for c, _ in out]), np.stack([lg[0] for _, lg in out])

    e = _engine(s, w, hip_device, text, uncond, prompt[:60], 270, **g)
    assert e.xcd_layers
    frames(e, 1)
    e.retire(0)
    e.step_frame(mask_eos_q0=True, uniforms=z)
    e.refill({0: (text, uncond, prompt)})
    got = frames(e, 2)
    assert e.frames_done == 4
    e.close()
    e = _engine(s, w, hip_device, text, uncond, prompt, 270, **g)
    want = frames(e, 2)
    e.close()
    np.testing.assert_array_equal(got[0], want[0])
    V = got[1].shape[-1]
    rel = _rowwise_rel(got[1].reshape(-1, V), want[1].reshape(-1, V))
    ref = _rowwise_rel(got[1].reshape(-1, V), f["sample_logits"][: 2 * s.n_codebooks])
    print(f"refill after a retired frame: vs fresh engine {rel:.3e}, vs reference {ref:.3e}")
    assert rel < 1e-6 and ref < LOGIT_TOL


def test_untied_head_through_model_binding(hip_device):
    """GraphFrameEngine(model) with a SorakuTTSv2-like module whose config has
    tie_audio_head=False binds depth_head.out_proj as the classifier
    (model.py:141-145,171-174): teacher-forced logits equal the reference's
    ``tiny_untied`` vectors."""
    from types import SimpleNamespace

    import torch
    from soraku_amd import GraphFrameEngine

    f, s, gen = load_golden("tiny_untied")
    assert not s.tie_audio_head
    w = synthetic_weights(s, int(f["seed"]), norm_gain_std=float(f["norm_gain_std"]),
                          bias_std=float(f["bias_std"]))
    lang = tuple(int(v) for v in f["language_ids"])
    trunk = SimpleNamespace(config=SimpleNamespace(
        hidden_size=s.d_model, num_hidden_layers=s.n_layers, num_attention_heads=s.n_q_heads,
        num_key_value_heads=s.n_kv_heads, head_dim=s.head_dim, intermediate_size=s.trunk_inter,
        vocab_size=s.text_vocab, rms_norm_eps=s.trunk_eps, rope_parameters={"rope_theta": s.rope_theta}))
    cfg = SimpleNamespace(depth_ffn_mult=s.depth_mult, num_codebooks=s.n_codebooks, codebook_size=s.codebook_size,
                          language_token_ids=lang, tie_audio_head=False)
    model = SimpleNamespace(config=cfg, trunk=trunk,
                            state_dict=lambda: {k: torch.from_numpy(v) for k, v in w.items()})
    n = f["text_ids"].size + 1 + f["prompt_codes"].shape[0] + gen["max_new_frames"] + 2
    e = GraphFrameEngine(model, device=hip_device, max_cache_len=n, cfg_scale=gen["cfg_scale"], batch=2)
    e.set_temperature(gen["temperature"])
    e.set_sampling(sampled=True, top_k=gen["top_k"], top_p=gen["top_p"])
    e.set_debug(True)
    e.prefill(f["text_ids"], f["uncond_ids"], f["prompt_codes"])
    e.capture()
    got = []
    for fi in range(f["codes"].shape[0]):
        _, lg = e.step_frame(mask_eos_q0=fi < gen["min_new_frames"], uniforms=np.zeros(s.n_codebooks),
                             forced_codes=f["codes"][fi], return_logits=True)
        got.extend(lg[0])
    e.close()
    rel = _rowwise_rel(np.stack(got)[: f["sample_logits"].shape[0]], f["sample_logits"])
    print(f"untied head via model=: max row-relative logit error {rel:.3e}")
    assert rel < LOGIT_TOL

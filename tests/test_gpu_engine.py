"""Whole-frame engine parity on the GPU against the reference's golden
vectors and the oracle.

Tolerance: logits within 1e-3 relative (normalised by
the row's max |logit|) of the FP32 reference path; tokens bit-exact when both
sides get the same logits and the same uniform draw."""

import numpy as np
import pytest

from conftest import load_golden
from oracle.generate import Record, generate
from oracle.model import OracleModel, synthetic_weights
from oracle.sampler import apply_masks

pytestmark = pytest.mark.gpu

LOGIT_TOL = 1e-3


def _shape(s):
    from soraku_amd.config import DecodeShape

    return DecodeShape(**{k: getattr(s, k) for k in DecodeShape.__dataclass_fields__})


def _weights(f, s):
    return synthetic_weights(s, int(f["seed"]), norm_gain_std=float(f["norm_gain_std"]),
                             bias_std=float(f["bias_std"]))


def _engine(f, s, gen, w, hip_device, max_ctx=None):
    from soraku_amd import GraphFrameEngine

    cfg = gen.get("cfg_scale", 1.0)
    batch = 2 if cfg != 1.0 else 1
    n = f["text_ids"].size + 1 + f["prompt_codes"].shape[0] + gen["max_new_frames"] + 2
    e = GraphFrameEngine(device=hip_device, max_cache_len=max_ctx or n, cfg_scale=cfg, batch=batch,
                         state_dict=w, shape=_shape(s),
                         language_token_ids=tuple(int(v) for v in f["language_ids"]))
    sampled = gen["temperature"] > 0 or (gen.get("temperature_q0") or 0) > 0
    e.set_temperature(gen["temperature"], q0=gen.get("temperature_q0"))
    e.set_sampling(sampled=sampled, top_k=gen.get("top_k"), top_p=gen.get("top_p"),
                   top_k_q0=gen.get("top_k_q0"), top_p_q0=gen.get("top_p_q0"))
    e.set_debug(True)
    e.prefill(f["text_ids"], f["uncond_ids"] if batch == 2 else None, f["prompt_codes"])
    e.capture()
    return e


def _rowwise_rel(got, ref):
    fin = np.isfinite(ref)
    assert (np.isfinite(got) == fin).all()
    num = np.where(fin, np.abs(got - ref), 0).max(axis=-1)
    den = np.where(fin, np.abs(ref), 0).max(axis=-1)
    return float((num / den).max())


def _teacher_forced(e, f, s, gen):
    codes = f["codes"]
    n_calls = f["sample_logits"].shape[0]
    out = []
    for fi in range(gen["max_new_frames"]):
        if len(out) >= n_calls:
            break
        forced = codes[fi] if fi < codes.shape[0] else np.full(s.n_codebooks, s.eos_id)
        _, lg = e.step_frame(mask_eos_q0=fi < gen["min_new_frames"], uniforms=np.zeros(s.n_codebooks),
                             forced_codes=forced, return_logits=True)
        out.extend(lg[0])
    return np.stack(out[:n_calls])


@pytest.mark.parametrize("name", ["tiny_greedy", "tiny_sampled", "tiny_nocfg_topp", "q06b_greedy"])
def test_teacher_forced_logits_match_reference(hip_device, name):
    f, s, gen = load_golden(name)
    e = _engine(f, s, gen, _weights(f, s), hip_device)
    hid = e.hidden()
    ref_h = f["hidden"][0]
    assert np.abs(hid - ref_h).max() / np.abs(ref_h).max() < 1e-4
    got = _teacher_forced(e, f, s, gen)
    rel = _rowwise_rel(got, f["sample_logits"])
    print(f"{name}: max row-relative logit error {rel:.3e}")
    assert rel < LOGIT_TOL
    e.close()


@pytest.mark.parametrize("name", ["tiny_greedy", "q06b_greedy"])
def test_greedy_codes_match_reference(hip_device, name):
    import torch
    from soraku_amd import FastGenerator

    f, s, gen = load_golden(name)
    g = FastGenerator(device=hip_device, state_dict=_weights(f, s), shape=_shape(s),
                      language_token_ids=tuple(int(v) for v in f["language_ids"]))
    kw = {k: v for k, v in gen.items() if k != "seed"}
    codes, info = g.generate(input_ids=torch.tensor(f["text_ids"][None]),
                             prompt_codes=torch.tensor(f["prompt_codes"]),
                             uncond_input_ids=torch.tensor(f["uncond_ids"][None]), **kw)
    np.testing.assert_array_equal(codes.numpy(), f["codes"])
    assert info["stop_reason"] == ("eos" if int(f["stop_eos"]) else "max_frames")


def test_sampled_codes_match_oracle_under_identical_uniforms(hip_device):
    """Free-running sampled decode (top-k, top-p, q0 overrides, CFG) with the
    same uniforms on both sides; the oracle runs in float64."""
    f, s, gen = load_golden("tiny_sampled")
    w = _weights(f, s)
    n_frames = 12
    gen = dict(gen, max_new_frames=n_frames)
    u = np.random.default_rng(11).random((n_frames, s.n_codebooks))
    m = OracleModel(s, w, np.float64, language_token_ids=tuple(int(v) for v in f["language_ids"]))
    kw = {k: v for k, v in gen.items() if k != "seed"}
    ref, _ = generate(m, input_ids=f["text_ids"], prompt_codes=f["prompt_codes"],
                      uncond_input_ids=f["uncond_ids"], uniforms=u, batched=True, **kw)
    e = _engine(f, s, gen, w, hip_device)
    got = []
    for fi in range(ref.shape[0]):
        got.append(e.step_frame(mask_eos_q0=fi < gen["min_new_frames"], uniforms=u[fi]).numpy())
    np.testing.assert_array_equal(np.stack(got), ref)
    e.close()


def test_replays_are_deterministic(hip_device):
    f, s, gen = load_golden("tiny_sampled")
    w = _weights(f, s)
    u = np.random.default_rng(3).random((6, s.n_codebooks))
    runs = []
    for _ in range(2):
        e = _engine(f, s, dict(gen, max_new_frames=6), w, hip_device)
        frames = [e.step_frame(mask_eos_q0=False, uniforms=u[i], return_logits=True) for i in range(6)]
        runs.append((np.stack([c.numpy() for c, _ in frames]), np.stack([lg for _, lg in frames])))
        e.close()
    np.testing.assert_array_equal(runs[0][0], runs[1][0])
    np.testing.assert_array_equal(runs[0][1], runs[1][1])


def test_queued_replay_equals_stepwise(hip_device):
    """sk_queue_frames + sk_replay (no host sync per frame) = sk_step_frame."""
    f, s, gen = load_golden("tiny_sampled")
    w = _weights(f, s)
    n = 8
    u = np.random.default_rng(5).random((n, s.n_codebooks))
    mask = (np.arange(n) < gen["min_new_frames"]).astype(np.int32)
    e = _engine(f, s, dict(gen, max_new_frames=n), w, hip_device)
    step = np.stack([e.step_frame(mask_eos_q0=bool(mask[i]), uniforms=u[i]).numpy() for i in range(n)])
    e.close()
    e = _engine(f, s, dict(gen, max_new_frames=n), w, hip_device)
    e.queue_frames(u, mask)
    e.replay(n)
    got = e.read_codes(n)[:, 0]
    np.testing.assert_array_equal(got, step)
    e.close()


def test_engine_error_paths(hip_device):
    from soraku_amd import GraphFrameEngine, SkError
    from soraku_amd._lib import SK_EKVFULL, SK_ENOCAPTURE

    f, s, gen = load_golden("tiny_greedy")
    w = _weights(f, s)
    n_prefix = f["text_ids"].size + 1 + f["prompt_codes"].shape[0]
    e = GraphFrameEngine(device=hip_device, max_cache_len=n_prefix + 2, cfg_scale=1.5, batch=2,
                         state_dict=w, shape=_shape(s),
                         language_token_ids=tuple(int(v) for v in f["language_ids"]))
    e.prefill(f["text_ids"], f["uncond_ids"], f["prompt_codes"])
    with pytest.raises(RuntimeError):
        e.step_frame(mask_eos_q0=True)
    e.graph = True  # bypass the Python guard: the C ABI must refuse too
    with pytest.raises(SkError) as ei:
        e.step_frame(mask_eos_q0=True)
    assert ei.value.code == SK_ENOCAPTURE
    e.capture()
    e.step_frame(mask_eos_q0=True)
    e.step_frame(mask_eos_q0=True)
    with pytest.raises(SkError) as ei:
        e.step_frame(mask_eos_q0=True)
    assert ei.value.code == SK_EKVFULL
    with pytest.raises(ValueError):
        e.prefill(np.arange(n_prefix + 5) % s.text_vocab, f["uncond_ids"], f["prompt_codes"])
    e.close()

"""Write golden vectors from the reference's native decode path.

Runs ONLY in the development container, where the reference sources are
mounted read-only at /root/reference; the vectors it writes (``*.npz`` beside
this script) are what the tests read.  Nothing else in the repository imports
the reference.

What the reference pins here that closed forms cannot (its composition):
``SorakuTTSv2.generate`` (soraku_inference/model.py:515-621) driving
``_start_state``/``_advance`` (model.py:623-676) over the transformers Qwen3
trunk, the depth-head chain (model.py:129-174), CFG/masks (model.py:579-584)
and the top-k/top-p filter of ``_sample_logits`` (model.py:686-708).

Recorded per fixture: the seed and shape (weights are regenerated from them by
``oracle.model.synthetic_weights``), the inputs, every ``logits`` argument of
``_sample_logits`` (masked CFG-merged FP32 logits), every probability vector
handed to ``torch.multinomial`` (sampled runs), the returned codes and the
depth-input hidden state of every frame for both branches.

Fixtures: ``tiny_greedy``, ``tiny_sampled`` (q0 overrides), ``tiny_nocfg_topp``,
``tiny_untied`` (untied classifier head ``depth_head.out_proj``, model.py:141-145,
171-174) and, with ``--large``, ``q06b_greedy`` (Qwen3-0.6B shape, prefix 65,
greedy) and ``q06b_sampled`` (Qwen3-0.6B shape with the full-utterance prefix
layout: 96 text ids + BOS frame + 144 prompt frames for the cond row, the text
BOS id + BOS frame + the prompt for the uncond row, CFG 1.5, T 0.9, top-k 50,
top-p 0.95: the V = 2051 probability vectors of ``torch.multinomial``).

Usage:  python tests/golden/make_golden.py [--large] [--only NAME ...]
"""

from __future__ import annotations

import argparse
import os
import sys

import numpy as np

sys.dont_write_bytecode = True
HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle.model import QWEN3_06B, TINY, Shape, synthetic_weights  # noqa: E402

REFERENCE = "/root/reference"


def build_reference(shape: Shape, weights, language_ids=()):
    import torch
    from transformers import Qwen3Config, Qwen3Model

    sys.path.insert(0, REFERENCE)
    from soraku_inference import model as refmod

    tcfg = Qwen3Config(
        vocab_size=shape.text_vocab, hidden_size=shape.d_model,
        intermediate_size=shape.trunk_inter, num_hidden_layers=shape.n_layers,
        num_attention_heads=shape.n_q_heads, num_key_value_heads=shape.n_kv_heads,
        head_dim=shape.head_dim, rms_norm_eps=shape.trunk_eps,
        rope_parameters={"rope_type": "default", "rope_theta": shape.rope_theta},
        max_position_embeddings=4096, tie_word_embeddings=False,
    )
    trunk = Qwen3Model._from_config(tcfg, dtype=torch.float32, attn_implementation="sdpa")
    cfg = refmod.SorakuV2Config(num_codebooks=shape.n_codebooks,
                                codebook_size=shape.codebook_size,
                                tie_audio_head=shape.tie_audio_head,
                                language_token_ids=tuple(language_ids))
    model = refmod.SorakuTTSv2(cfg, trunk=trunk)
    state = {k: torch.from_numpy(np.ascontiguousarray(v)) for k, v in weights.items()}
    model.load_state_dict(state, strict=True, assign=True)
    model.eval()
    return model, refmod


def run(shape: Shape, *, wseed, norm_gain_std, bias_std, text_ids, prompt_codes, uncond_ids,
        language_ids=(), **gen):
    import torch

    weights = synthetic_weights(shape, wseed, norm_gain_std=norm_gain_std, bias_std=bias_std)
    model, refmod = build_reference(shape, weights, language_ids)
    logits_rec, probs_rec, hidden_rec = [], [], []

    orig_sample = refmod._sample_logits
    orig_multinomial = torch.multinomial

    def sample_spy(logits, **kw):
        logits_rec.append(logits.detach().numpy().copy())

        def multinomial_spy(p, n, generator=None):
            probs_rec.append(p.detach().numpy().copy())
            return orig_multinomial(p, n, generator=generator)

        torch.multinomial = multinomial_spy
        try:
            return orig_sample(logits, **kw)
        finally:
            torch.multinomial = orig_multinomial

    orig_start, orig_advance = model._start_state, model._advance

    def start_spy(*a, **k):
        st = orig_start(*a, **k)
        hidden_rec.append(st["hidden"][0].detach().numpy().copy())
        return st

    def advance_spy(*a, **k):
        h = orig_advance(*a, **k)
        hidden_rec.append(h[0].detach().numpy().copy())
        return h

    refmod._sample_logits = sample_spy
    model._start_state, model._advance = start_spy, advance_spy
    try:
        codes, info = model.generate(
            input_ids=torch.tensor([text_ids]),
            prompt_codes=torch.tensor(prompt_codes).view(-1, shape.n_codebooks),
            uncond_input_ids=torch.tensor([uncond_ids]), **gen)
    finally:
        refmod._sample_logits = orig_sample
    rows = 2 if gen.get("cfg_scale", 1.0) != 1.0 else 1
    hid = np.stack(hidden_rec).reshape(-1, rows, shape.d_model)
    out = dict(
        shape=np.array([shape.d_model, shape.n_layers, shape.n_q_heads, shape.n_kv_heads,
                        shape.head_dim, shape.trunk_inter, shape.depth_mult, shape.n_codebooks,
                        shape.codebook_size, shape.text_vocab, len(language_ids)], np.int64),
        tie_audio_head=np.int64(shape.tie_audio_head),
        seed=np.int64(wseed), norm_gain_std=np.float64(norm_gain_std), bias_std=np.float64(bias_std),
        text_ids=np.asarray(text_ids, np.int64), uncond_ids=np.asarray(uncond_ids, np.int64),
        prompt_codes=np.asarray(prompt_codes, np.int64).reshape(-1, shape.n_codebooks),
        language_ids=np.asarray(language_ids, np.int64),
        codes=codes.numpy().astype(np.int64), stop_eos=np.int64(info["stop_reason"] == "eos"),
        sample_logits=np.stack(logits_rec).astype(np.float32),
        probs=(np.stack(probs_rec).astype(np.float32) if probs_rec
               else np.zeros((0, shape.audio_vocab), np.float32)),
        hidden=hid.astype(np.float32),
    )
    for k, v in gen.items():
        out["gen_" + k] = np.float64(-1 if v is None else v)
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--large", action="store_true", help="also write the Qwen3-0.6B-shaped fixtures")
    ap.add_argument("--only", nargs="*", default=None, help="write only these fixtures")
    args = ap.parse_args()

    def want(name):
        return args.only is None or name in args.only

    rng = np.random.default_rng(7)
    s = Shape(**{**TINY.__dict__, "n_language": 4})
    lang = (90, 91, 92, 93)
    text = [5, 91, 17, 33, 2, 90, 64, 12, 7]
    prompt = rng.integers(0, s.codebook_size, size=(3, s.n_codebooks))
    common = dict(wseed=0, norm_gain_std=0.1, bias_std=0.02, text_ids=text,
                  prompt_codes=prompt, uncond_ids=[5], language_ids=lang)
    if want("tiny_greedy"):
        fx = run(s, **common, max_new_frames=6, min_new_frames=2, temperature=0.0,
                 cfg_scale=1.5)
        np.savez_compressed(os.path.join(HERE, "tiny_greedy.npz"), **fx)
    if want("tiny_sampled"):
        fx = run(s, **common, max_new_frames=8, min_new_frames=2, temperature=0.9, top_k=8,
                 top_p=0.9, temperature_q0=0.7, top_k_q0=5, top_p_q0=0.8, cfg_scale=1.5, seed=123)
        np.savez_compressed(os.path.join(HERE, "tiny_sampled.npz"), **fx)
    if want("tiny_nocfg_topp"):
        fx = run(s, **common, max_new_frames=4, min_new_frames=0, temperature=1.0, top_k=None,
                 top_p=0.6, cfg_scale=1.0, seed=5)
        np.savez_compressed(os.path.join(HERE, "tiny_nocfg_topp.npz"), **fx)
    # the draws above advance rng; later fixtures take their own generators
    if want("tiny_untied"):
        su = Shape(**{**TINY.__dict__, "n_language": 4, "tie_audio_head": False})
        fx = run(su, **{**common, "wseed": 4}, max_new_frames=5, min_new_frames=1, temperature=0.9,
                 top_k=8, top_p=0.9, cfg_scale=1.5, seed=31)
        np.savez_compressed(os.path.join(HERE, "tiny_untied.npz"), **fx)
    if args.large and want("q06b_greedy"):
        s6 = QWEN3_06B
        text6 = rng.integers(0, s6.text_vocab, size=40).tolist()
        prompt6 = rng.integers(0, s6.codebook_size, size=(24, s6.n_codebooks))
        fx = run(s6, wseed=1, norm_gain_std=0.1, bias_std=0.02, text_ids=text6,
                 prompt_codes=prompt6, uncond_ids=[text6[0]], max_new_frames=3,
                 min_new_frames=8, temperature=0.0, cfg_scale=1.5)
        np.savez_compressed(os.path.join(HERE, "q06b_greedy.npz"), **fx)
    if args.large and want("q06b_sampled"):
        s6 = QWEN3_06B
        r6 = np.random.default_rng(2051)
        text6 = r6.integers(0, s6.text_vocab, size=96).tolist()
        prompt6 = r6.integers(0, s6.codebook_size, size=(144, s6.n_codebooks))
        fx = run(s6, wseed=2, norm_gain_std=0.1, bias_std=0.02, text_ids=text6,
                 prompt_codes=prompt6, uncond_ids=[151643], max_new_frames=2,
                 min_new_frames=8, temperature=0.9, top_k=50, top_p=0.95, cfg_scale=1.5, seed=0)
        np.savez_compressed(os.path.join(HERE, "q06b_sampled.npz"), **fx)


if __name__ == "__main__":
    main()

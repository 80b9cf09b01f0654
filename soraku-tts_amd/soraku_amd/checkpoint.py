"""Soraku release checkpoints for the MI355X engine (runtime.py:14-44).

A release directory holds ``config.json`` (``format_version`` 1,
``model_type`` ``soraku_tts_v2``, ``soraku_config`` = SorakuV2Config fields,
model.py:34-47), ``text_config.json`` (the Qwen3 trunk config) and
``model.safetensors`` (the full state dict, trunk included).  ``load_release``
checks the same gate as the reference, derives the decode shape, and returns
the decode-path tensors by state-dict key; tensors are read with the
safetensors loader (no pickle).  BF16 storage is the engine's choice
(``bf16=True``): the reference computes in FP32, so a checkpoint stored in
BF16 is widened here unless the engine keeps BF16 matrices.
"""

from __future__ import annotations

import json
from dataclasses import dataclass
from pathlib import Path
from typing import Any

from .config import DecodeShape
from .synthetic import is_matrix, weight_shapes


@dataclass
class Release:
    shape: DecodeShape
    state_dict: dict            # key -> torch.Tensor (CPU)
    language_token_ids: tuple
    metadata: dict[str, Any]


def shape_from_configs(soraku: dict, text: dict) -> DecodeShape:
    """DecodeShape from ``soraku_config`` and the Qwen3 text config
    (hidden_size, num_hidden_layers, num_attention_heads,
    num_key_value_heads, head_dim, intermediate_size, vocab_size,
    rms_norm_eps, rope_theta)."""
    heads = int(text["num_attention_heads"])
    d = int(text["hidden_size"])
    lang = tuple(soraku.get("language_token_ids", ()) or ())
    return DecodeShape(
        d_model=d,
        n_layers=int(text["num_hidden_layers"]),
        n_q_heads=heads,
        n_kv_heads=int(text.get("num_key_value_heads", heads)),
        head_dim=int(text.get("head_dim") or d // heads),
        trunk_inter=int(text["intermediate_size"]),
        depth_mult=int(soraku.get("depth_ffn_mult", 2)),
        n_codebooks=int(soraku.get("num_codebooks", 16)),
        codebook_size=int(soraku.get("codebook_size", 2048)),
        text_vocab=int(text["vocab_size"]),
        trunk_eps=float(text.get("rms_norm_eps", 1e-6)),
        rope_theta=float(text.get("rope_theta", 1e6)),
        n_language=len(lang),
        tie_audio_head=bool(soraku.get("tie_audio_head", True)),
    )


def load_release(model_dir, *, bf16: bool = False) -> Release:
    """Read a release directory.  Raises ValueError for directories the
    reference would reject (runtime.py:17-22), for speaker-conditioned models
    (their prefill needs the speaker modules, which the fast path does not
    run; fast_generate.py refuses them too), for a wrong language-token list
    (model.py:186-191), and for missing or mis-shaped decode tensors.
    ``bf16``: matrices are returned in BF16 (what the engine stores with
    ``bf16=True``), everything else in FP32."""
    import torch
    from safetensors.torch import load_file

    directory = Path(model_dir)
    metadata = json.loads((directory / "config.json").read_text())
    if metadata.get("format_version") != 1 or metadata.get("model_type") != "soraku_tts_v2":
        raise ValueError("not a supported Soraku release model directory")
    soraku = dict(metadata["soraku_config"])
    if soraku.get("speaker_conditioning", False):
        raise ValueError("speaker-conditioned checkpoints are not supported by the MI355X decode path")
    lang = tuple(int(v) for v in (soraku.get("language_token_ids", ()) or ()))
    if lang and (len(lang) != 4 or len(set(lang)) != 4):
        raise ValueError("exactly four unique language token IDs are required")
    text = json.loads((directory / "text_config.json").read_text())
    shape = shape_from_configs(soraku, text)
    raw = load_file(str(directory / "model.safetensors"), device="cpu")
    out = {}
    for key, shp in weight_shapes(shape).items():
        if key not in raw:
            raise ValueError(f"model.safetensors lacks {key}")
        t = raw[key]
        if tuple(t.shape) != tuple(shp):
            raise ValueError(f"{key}: shape {tuple(t.shape)}, expected {shp}")
        dt = torch.bfloat16 if (bf16 and is_matrix(key)) else torch.float32
        out[key] = t.to(dt).contiguous()
    return Release(shape=shape, state_dict=out, language_token_ids=lang, metadata=metadata)

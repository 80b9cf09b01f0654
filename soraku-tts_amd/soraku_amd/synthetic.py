"""Seeded synthetic weights and inputs (no checkpoints are available offline).

Weights are drawn in sorted state-dict-key order from
``numpy.random.default_rng(seed)``: matrices / embeddings / codebook tables
N(0, 0.02) (model.py:103, initializer_range), RMSNorm gains 1 (or
1 + N(0, norm_gain_std)), depth bias 0 (or N(0, bias_std), model.py:138-140).
The depth head's ``norm_in`` / ``norm_out`` gains are drawn like the matrices
(N(0, 0.02)); the committed golden vectors were made with that draw.
"""

from __future__ import annotations

import numpy as np

from .config import DecodeShape


def weight_shapes(s: DecodeShape) -> dict[str, tuple[int, ...]]:
    """State-dict keys and shapes of the decode path (model.py:100-145,194;
    transformers Qwen3Model parameter names)."""
    hq, hkv = s.n_q_heads * s.head_dim, s.n_kv_heads * s.head_dim
    out: dict[str, tuple[int, ...]] = {"trunk.embed_tokens.weight": (s.text_vocab, s.d_model)}
    for i in range(s.n_layers):
        p = f"trunk.layers.{i}."
        out[p + "input_layernorm.weight"] = (s.d_model,)
        out[p + "self_attn.q_proj.weight"] = (hq, s.d_model)
        out[p + "self_attn.k_proj.weight"] = (hkv, s.d_model)
        out[p + "self_attn.v_proj.weight"] = (hkv, s.d_model)
        out[p + "self_attn.o_proj.weight"] = (s.d_model, hq)
        out[p + "self_attn.q_norm.weight"] = (s.head_dim,)
        out[p + "self_attn.k_norm.weight"] = (s.head_dim,)
        out[p + "post_attention_layernorm.weight"] = (s.d_model,)
        out[p + "mlp.gate_proj.weight"] = (s.trunk_inter, s.d_model)
        out[p + "mlp.up_proj.weight"] = (s.trunk_inter, s.d_model)
        out[p + "mlp.down_proj.weight"] = (s.d_model, s.trunk_inter)
    out["trunk.norm.weight"] = (s.d_model,)
    out["audio_codebooks.table"] = (s.n_codebooks, s.audio_vocab, s.d_model)
    out["depth_head.norm_in.weight"] = (s.d_model,)
    out["depth_head.mlp.gate_proj.weight"] = (s.depth_inner, s.d_model)
    out["depth_head.mlp.up_proj.weight"] = (s.depth_inner, s.d_model)
    out["depth_head.mlp.down_proj.weight"] = (s.d_model, s.depth_inner)
    out["depth_head.norm_out.weight"] = (s.d_model,)
    out["depth_head.bias"] = (s.n_codebooks, s.audio_vocab)
    if not getattr(s, "tie_audio_head", True):   # model.py:141-145
        out["depth_head.out_proj"] = (s.n_codebooks, s.audio_vocab, s.d_model)
    if s.n_language:
        out["language_embeddings.weight"] = (s.n_language, s.d_model)
    return out


def is_matrix(key: str) -> bool:
    """Tensors stored in the engine's weight dtype (everything but gains,
    bias and language rows)."""
    parts = key.split(".")
    return not ((len(parts) >= 2 and "norm" in parts[-2])
                or key in ("depth_head.bias", "language_embeddings.weight"))


def synthetic_weights(s: DecodeShape, seed: int = 0, *, std: float = 0.02,
                      norm_gain_std: float = 0.0, bias_std: float = 0.0) -> dict[str, np.ndarray]:
    rng = np.random.default_rng(seed)
    out = {}
    for key, shp in sorted(weight_shapes(s).items()):
        if key.endswith("norm.weight") or key.endswith("layernorm.weight"):
            w = np.ones(shp, np.float32)
            if norm_gain_std:
                w += rng.standard_normal(shp, dtype=np.float32) * np.float32(norm_gain_std)
        elif key == "depth_head.bias":
            w = np.zeros(shp, np.float32)
            if bias_std:
                w = rng.standard_normal(shp, dtype=np.float32) * np.float32(bias_std)
        else:
            w = rng.standard_normal(shp, dtype=np.float32)
            w *= np.float32(std)
        out[key] = w
    return out


def round_bf16(x: np.ndarray) -> np.ndarray:
    """FP32 -> nearest BF16 (ties to even), kept as FP32 values."""
    b = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    b = (b + 0x7FFF + ((b >> 16) & 1)) & 0xFFFF0000
    return b.astype(np.uint32).view(np.float32).reshape(x.shape)


def utterance(s: DecodeShape, seed: int, *, n_text: int, n_prompt: int):
    """Random text ids and prompt frames (codes 0..codebook_size-1)."""
    rng = np.random.default_rng(seed)
    text = rng.integers(0, s.text_vocab, size=n_text, dtype=np.int64)
    prompt = rng.integers(0, s.codebook_size, size=(n_prompt, s.n_codebooks), dtype=np.int64)
    return text, prompt

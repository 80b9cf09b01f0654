"""Model dimensions of the decode path and their C-ABI form.

Mirrors ``SorakuV2Config`` (soraku_inference/model.py:34-63) plus the Qwen3
text config fields the trunk uses (hidden size, layers, heads, rms_norm_eps,
rope_theta, intermediate_size).
"""

from __future__ import annotations

from dataclasses import dataclass, replace

import numpy as np

from ._lib import SK_BF16, SK_F32, SkConfig

FLT_EPS = float(np.finfo(np.float32).eps)  # nn.RMSNorm(eps=None), model.py:135,137


@dataclass(frozen=True)
class DecodeShape:
    d_model: int = 1024
    n_layers: int = 28
    n_q_heads: int = 16
    n_kv_heads: int = 8
    head_dim: int = 128
    trunk_inter: int = 3072
    depth_mult: int = 2
    n_codebooks: int = 16
    codebook_size: int = 2048
    text_vocab: int = 151936
    trunk_eps: float = 1e-6
    rope_theta: float = 1e6
    n_language: int = 0
    tie_audio_head: bool = True

    @property
    def audio_vocab(self) -> int:  # model.py:61-63
        return self.codebook_size + 3

    @property
    def bos_id(self) -> int:  # model.py:49-51
        return self.codebook_size

    @property
    def eos_id(self) -> int:  # model.py:53-55
        return self.codebook_size + 1

    @property
    def pad_id(self) -> int:  # model.py:57-59
        return self.codebook_size + 2

    @property
    def depth_inner(self) -> int:  # model.py:82-87
        return self.d_model * self.depth_mult

    @property
    def frame_scale(self) -> float:  # model.py:99
        return self.n_codebooks ** -0.5

    def with_(self, **kw) -> "DecodeShape":
        return replace(self, **kw)


QWEN3_06B = DecodeShape()
QWEN3_17B = DecodeShape(d_model=2048, trunk_inter=6144)
TINY = DecodeShape(d_model=64, n_layers=2, n_q_heads=4, n_kv_heads=2, head_dim=16,
                   trunk_inter=96, n_codebooks=4, codebook_size=32, text_vocab=100)


def shape_from_model(model) -> DecodeShape:
    """Read the dimensions off a ``SorakuTTSv2``-like module (model.py:177-212)."""
    cfg = model.config
    t = model.trunk.config
    rope = getattr(t, "rope_parameters", None) or {}
    theta = rope.get("rope_theta", getattr(t, "rope_theta", 1e6))
    return DecodeShape(
        d_model=int(t.hidden_size), n_layers=int(t.num_hidden_layers),
        n_q_heads=int(t.num_attention_heads), n_kv_heads=int(t.num_key_value_heads),
        head_dim=int(getattr(t, "head_dim", None) or t.hidden_size // t.num_attention_heads),
        trunk_inter=int(t.intermediate_size), depth_mult=int(cfg.depth_ffn_mult),
        n_codebooks=int(cfg.num_codebooks), codebook_size=int(cfg.codebook_size),
        text_vocab=int(t.vocab_size), trunk_eps=float(t.rms_norm_eps), rope_theta=float(theta),
        n_language=4 if getattr(cfg, "language_token_ids", ()) else 0,
        tie_audio_head=bool(getattr(cfg, "tie_audio_head", True)),   # model.py:131,141-145,172
    )


def to_sk_config(s: DecodeShape, *, n_utts: int, cfg_rows: int, max_ctx: int, max_frames: int,
                 bf16: bool = False, language_ids=(), kv_bf16: bool = False) -> SkConfig:
    c = SkConfig()
    c.d_model, c.n_layers, c.n_q_heads, c.n_kv_heads = s.d_model, s.n_layers, s.n_q_heads, s.n_kv_heads
    c.head_dim, c.trunk_inter, c.depth_inner = s.head_dim, s.trunk_inter, s.depth_inner
    c.n_codebooks, c.audio_vocab, c.text_vocab = s.n_codebooks, s.audio_vocab, s.text_vocab
    c.bos_id, c.eos_id, c.pad_id = s.bos_id, s.eos_id, s.pad_id
    c.trunk_eps, c.depth_eps, c.rope_theta, c.frame_scale = s.trunk_eps, FLT_EPS, s.rope_theta, s.frame_scale
    c.weight_dtype = SK_BF16 if bf16 else SK_F32
    c.kv_dtype = SK_BF16 if kv_bf16 else SK_F32
    c.n_utts, c.cfg_rows, c.max_ctx, c.max_frames = n_utts, cfg_rows, max_ctx, max_frames
    ids = list(language_ids)
    c.n_language = 4 if ids else 0
    for i in range(4):
        c.language_ids[i] = ids[i] if ids else -1
    return c

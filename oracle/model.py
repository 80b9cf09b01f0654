"""NumPy restatement of the soraku-TTS decode path (oracle; test infrastructure).

Follows the reference's native semantics:

* model container / special ids ............ soraku_inference/model.py:34-63
* AudioCodebooks.frame_embedding ............ model.py:93-114
* DepthHead.body / step ..................... model.py:129-174 (eps: fast_generate.py:71-78)
* prefill layout (text, BOS frame, prompt) .. model.py:623-656
* trunk advance per branch .................. model.py:658-676
* Qwen3 trunk arithmetic .................... transformers/models/qwen3/modeling_qwen3.py
  RMSNorm :49-64, MLP :70-83, RoPE :116-170, repeat_kv :173-182,
  attention with per-head QK-norm :210-280, decoder layer :294-323, final norm :423

All arithmetic runs in ``dtype`` (float32 mirrors the reference's FP32 path,
float64 is the exact-math pin).  Weights are a dict keyed by the reference's
state-dict names (model.py:100-145, modeling_qwen3.py:225-238,290-292,352-356).
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

FLT_EPS = float(np.finfo(np.float32).eps)  # nn.RMSNorm(eps=None) default, model.py:135,137


@dataclass(frozen=True)
class Shape:
    """Model dimensions (SorakuV2Config model.py:34-63 + Qwen3 text config)."""

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


QWEN3_06B = Shape()
QWEN3_17B = Shape(d_model=2048, trunk_inter=6144)
TINY = Shape(d_model=64, n_layers=2, n_q_heads=4, n_kv_heads=2, head_dim=16,
             trunk_inter=96, n_codebooks=4, codebook_size=32, text_vocab=100)


def weight_shapes(s: Shape) -> dict[str, tuple[int, ...]]:
    """Every tensor of the decode path, keyed by its state-dict name."""
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
    if not s.tie_audio_head:                     # model.py:141-145
        out["depth_head.out_proj"] = (s.n_codebooks, s.audio_vocab, s.d_model)
    if s.n_language:
        out["language_embeddings.weight"] = (s.n_language, s.d_model)
    return out


def is_norm_gain(key: str) -> bool:
    """Keys the synthetic draw sets to 1 (+ optional noise): the trunk's
    RMSNorm and q/k-norm gains.  The depth head's ``norm_in`` / ``norm_out``
    gains are drawn like matrices; the golden vectors were made that way."""
    return key.endswith("norm.weight") or key.endswith("layernorm.weight")


def synthetic_weights(s: Shape, seed: int = 0, *, std: float = 0.02,
                      norm_gain_std: float = 0.0, bias_std: float = 0.0) -> dict[str, np.ndarray]:
    """Seeded FP32 weights drawn in sorted-key order from ``default_rng(seed)``.

    Linear / embedding / codebook tables: N(0, std) (model.py:103,
    initializer_range 0.02).  RMSNorm gains: 1 (modeling_qwen3.py:56) or
    1 + N(0, norm_gain_std).  Depth bias: 0 (model.py:138-140) or N(0, bias_std).
    """
    rng = np.random.default_rng(seed)
    out = {}
    for key, shp in sorted(weight_shapes(s).items()):
        if is_norm_gain(key):
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
    """Round FP32 to the nearest BF16 (ties to even), returned as FP32."""
    b = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    b = (b + 0x7FFF + ((b >> 16) & 1)) & 0xFFFF0000
    return b.astype(np.uint32).view(np.float32).reshape(x.shape)


# --------------------------------------------------------------------- math

def rms_norm(x, w, eps):
    """``w * (x * rsqrt(mean(x^2) + eps))`` (modeling_qwen3.py:58-64; nn.RMSNorm
    computes the same form, model.py:135,137)."""
    var = np.mean(x * x, axis=-1, keepdims=True)
    return w * (x * (1.0 / np.sqrt(var + eps)))


def silu(g):
    """``g * sigmoid(g)`` (F.silu, model.py:90; ACT2FN['silu'] modeling_qwen3.py:79)."""
    return g / (1.0 + np.exp(-g))


def rope_inv_freq(head_dim: int, theta: float) -> np.ndarray:
    """FP32 ``1 / theta ** (arange(0, dim, 2) / dim)`` (modeling_qwen3.py:116-122)."""
    ex = np.arange(0, head_dim, 2, dtype=np.float32) / np.float32(head_dim)
    return (np.float32(1.0) / (np.float32(theta) ** ex)).astype(np.float32)


def rope_cos_sin(positions, head_dim: int, theta: float):
    """cos/sin of the FP32 angle ``inv_freq * pos`` (modeling_qwen3.py:126-137),
    evaluated in float64 and rounded once to FP32.  Returns ``[n, head_dim/2]``."""
    inv = rope_inv_freq(head_dim, theta)
    ang = np.asarray(positions, np.float32).reshape(-1, 1) * inv.reshape(1, -1)
    ang = ang.astype(np.float32).astype(np.float64)
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def apply_rope(x, cos, sin):
    """rotate-half RoPE (modeling_qwen3.py:140-170). ``x [..., hd]``, cos/sin
    ``[..., hd/2]`` broadcast over heads; ``emb = cat(freqs, freqs)``."""
    h = x.shape[-1] // 2
    x1, x2 = x[..., :h], x[..., h:]
    c = cos.astype(x.dtype)
    s = sin.astype(x.dtype)
    return np.concatenate((x1 * c - x2 * s, x2 * c + x1 * s), axis=-1)


def softmax(x, axis=-1):
    m = np.max(x, axis=axis, keepdims=True)
    e = np.exp(x - m)
    return e / np.sum(e, axis=axis, keepdims=True)


def attend(q, k, v, scale):
    """Single-query GQA attention for one row: ``q [Hq, hd]``, ``k/v [Hkv, ctx, hd]``
    (repeat_kv modeling_qwen3.py:173-182: q head h reads kv head h // (Hq/Hkv))."""
    rep = q.shape[0] // k.shape[0]
    kk = np.repeat(k, rep, axis=0)
    vv = np.repeat(v, rep, axis=0)
    s = np.matmul(kk, q[:, :, None])[..., 0] * scale          # [Hq, ctx]
    p = softmax(s, -1)
    return np.matmul(p[:, None, :], vv)[:, 0, :]


# --------------------------------------------------------------------- model

class RowState:
    """KV cache and position of one CFG row (one reference branch)."""

    def __init__(self, s: Shape, max_ctx: int, dtype):
        self.k = np.zeros((s.n_layers, s.n_kv_heads, max_ctx, s.head_dim), dtype)
        self.v = np.zeros_like(self.k)
        self.kv_len = 0
        self.hidden = None


class OracleModel:
    """``kv_bf16``: keys (after QK-norm and RoPE) and values are rounded to
    BF16 when appended to the cache, and every attention reads the rounded
    values (the BF16-KV configuration; the reference itself keeps FP32)."""

    def __init__(self, shape: Shape, weights: dict[str, np.ndarray], dtype=np.float32,
                 language_token_ids: tuple[int, ...] = (), kv_bf16: bool = False):
        self.s = shape
        self.dtype = np.dtype(dtype)
        self.w = {k: np.asarray(v, self.dtype) for k, v in weights.items()}
        self.language_token_ids = tuple(language_token_ids)
        self.scale_attn = self.dtype.type(shape.head_dim ** -0.5)
        self.kv_bf16 = kv_bf16

    def _kv_store(self, x):
        return round_bf16(np.asarray(x, np.float32)).astype(self.dtype) if self.kv_bf16 else x

    # ---- embeddings -----------------------------------------------------
    def frame_embedding(self, codes) -> np.ndarray:
        """``scale * sum_q table[q, codes[..., q]]``, summed in q order
        (AudioCodebooks.frame_embedding model.py:105-114)."""
        codes = np.asarray(codes)
        t = self.w["audio_codebooks.table"]
        total = None
        for q in range(self.s.n_codebooks):
            piece = t[q][codes[..., q]]
            total = piece if total is None else total + piece
        return total * self.dtype.type(self.s.frame_scale)

    def embed_text(self, ids) -> np.ndarray:
        """Text rows, with language-token rows replaced (model.py:326-338)."""
        ids = np.asarray(ids)
        out = self.w["trunk.embed_tokens.weight"][np.where(np.isin(ids, self.language_token_ids), 0, ids)]
        for j, ident in enumerate(self.language_token_ids):
            out[ids == ident] = self.w["language_embeddings.weight"][j]
        return out

    def prefix_embeds(self, text_ids, prompt_codes) -> np.ndarray:
        """[text, BOS frame, prompt frames] (model.py:632-653)."""
        q = self.s.n_codebooks
        frames = np.full((1, q), self.s.bos_id, np.int64)
        if prompt_codes is not None and np.size(prompt_codes):
            frames = np.concatenate((frames, np.asarray(prompt_codes, np.int64).reshape(-1, q)), 0)
        return np.concatenate((self.embed_text(text_ids), self.frame_embedding(frames)), 0)

    # ---- trunk ------------------------------------------------------------
    def _lw(self, i, name):
        return self.w[f"trunk.layers.{i}.{name}"]

    def _qkv(self, i, h):
        s = self.s
        x = rms_norm(h, self._lw(i, "input_layernorm.weight"), s.trunk_eps)
        n = h.shape[0]
        q = (x @ self._lw(i, "self_attn.q_proj.weight").T).reshape(n, s.n_q_heads, s.head_dim)
        k = (x @ self._lw(i, "self_attn.k_proj.weight").T).reshape(n, s.n_kv_heads, s.head_dim)
        v = (x @ self._lw(i, "self_attn.v_proj.weight").T).reshape(n, s.n_kv_heads, s.head_dim)
        q = rms_norm(q, self._lw(i, "self_attn.q_norm.weight"), s.trunk_eps)
        k = rms_norm(k, self._lw(i, "self_attn.k_norm.weight"), s.trunk_eps)
        return q, k, v

    def _mlp(self, i, h):
        x = rms_norm(h, self._lw(i, "post_attention_layernorm.weight"), self.s.trunk_eps)
        a = silu(x @ self._lw(i, "mlp.gate_proj.weight").T) * (x @ self._lw(i, "mlp.up_proj.weight").T)
        return h + a @ self._lw(i, "mlp.down_proj.weight").T

    def prefill(self, st: RowState, embeds) -> np.ndarray:
        """Causal forward of ``embeds [L, d]`` at positions ``kv_len..`` into
        ``st`` (model.py:658-671 over Qwen3Model.forward modeling_qwen3.py:367-427).
        Returns the last position's final-normed hidden ``[d]``."""
        s = self.s
        h = np.asarray(embeds, self.dtype)
        n = h.shape[0]
        p0 = st.kv_len
        cos, sin = rope_cos_sin(np.arange(p0, p0 + n), s.head_dim, s.rope_theta)
        rep = s.n_q_heads // s.n_kv_heads
        ctx = p0 + n
        causal = np.triu(np.ones((n, ctx), bool), k=p0 + 1)
        for i in range(s.n_layers):
            q, k, v = self._qkv(i, h)
            q = apply_rope(q, cos[:, None, :], sin[:, None, :])
            k = apply_rope(k, cos[:, None, :], sin[:, None, :])
            st.k[i, :, p0:ctx] = self._kv_store(k.transpose(1, 0, 2))
            st.v[i, :, p0:ctx] = self._kv_store(v.transpose(1, 0, 2))
            kk = np.repeat(st.k[i, :, :ctx], rep, axis=0)
            vv = np.repeat(st.v[i, :, :ctx], rep, axis=0)
            sc = np.matmul(q.transpose(1, 0, 2), kk.transpose(0, 2, 1)) * self.scale_attn   # [Hq, n, ctx]
            sc = np.where(causal[None], -np.inf, sc)
            o = np.matmul(softmax(sc, -1), vv).transpose(1, 0, 2).reshape(n, -1)
            h = h + o @ self._lw(i, "self_attn.o_proj.weight").T
            h = self._mlp(i, h)
        st.kv_len = ctx
        st.hidden = rms_norm(h[-1], self.w["trunk.norm.weight"], s.trunk_eps)
        return st.hidden

    def trunk_step(self, states: list[RowState], x) -> np.ndarray:
        """One token per row; row r sits at position ``states[r].kv_len``
        (model.py:673-676; fast_generate.py:295-297 per-row positions).
        Returns final-normed hidden ``[rows, d]``."""
        s = self.s
        h = np.asarray(x, self.dtype).reshape(len(states), s.d_model)
        pos = np.array([st.kv_len for st in states])
        cos, sin = rope_cos_sin(pos, s.head_dim, s.rope_theta)
        for i in range(s.n_layers):
            q, k, v = self._qkv(i, h)
            q = apply_rope(q, cos[:, None, :], sin[:, None, :])
            k = apply_rope(k, cos[:, None, :], sin[:, None, :])
            outs = []
            for r, st in enumerate(states):
                t = st.kv_len
                st.k[i, :, t] = self._kv_store(k[r])
                st.v[i, :, t] = self._kv_store(v[r])
                outs.append(attend(q[r], st.k[i, :, : t + 1], st.v[i, :, : t + 1], self.scale_attn))
            o = np.stack(outs).reshape(len(states), -1)
            h = h + o @ self._lw(i, "self_attn.o_proj.weight").T
            h = self._mlp(i, h)
        for st in states:
            st.kv_len += 1
        hid = rms_norm(h, self.w["trunk.norm.weight"], s.trunk_eps)
        for r, st in enumerate(states):
            st.hidden = hid[r]
        return hid

    # ---- depth head -----------------------------------------------------
    def depth_logits(self, hidden, prefix, q: int) -> np.ndarray:
        """``DepthHead.step``: ``a = norm_in(h + prefix)``,
        ``body = norm_out(a + mlp(a))``, ``logits = body @ table[q].T + bias[q]``
        (model.py:147-149,163-174; eps = FLT_EPSILON, fast_generate.py:71-78);
        an untied head uses ``depth_head.out_proj[q]`` instead of the table
        (model.py:171-174)."""
        w = self.w
        a = rms_norm(hidden + prefix, w["depth_head.norm_in.weight"], FLT_EPS)
        g = a @ w["depth_head.mlp.gate_proj.weight"].T
        u = a @ w["depth_head.mlp.up_proj.weight"].T
        y = a + (silu(g) * u) @ w["depth_head.mlp.down_proj.weight"].T
        body = rms_norm(y, w["depth_head.norm_out.weight"], FLT_EPS)
        head = w["audio_codebooks.table"] if self.s.tie_audio_head else w["depth_head.out_proj"]
        return body @ head[q].T + w["depth_head.bias"][q]

    def prefix_step(self, q: int, code: int) -> np.ndarray:
        """``embedding(code, table[q]) * scale`` (model.py:600-603)."""
        return self.w["audio_codebooks.table"][q][code] * self.dtype.type(self.s.frame_scale)

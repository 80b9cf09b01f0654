"""Oracle for CFG mixing, masking, temperature and top-k / top-p sampling.

Semantics follow the reference's native path:

* CFG ``u + s * (c - u)`` ................. soraku_inference/model.py:579-581
  (not the ``torch.lerp`` of fast_generate.py:412 / graph_frame.py:215)
* BOS/PAD always blocked, EOS blocked unless q == 0 and
  frame >= min_new_frames .................. model.py:556-559,582-584
* greedy when temperature <= 0 (first max) . model.py:694-695
* ``logits / T`` (division) ............... model.py:696
* top-k keeps every value >= the k-th largest (ties kept) .. model.py:697-699
* top-p removes ``cum > p`` shifted right by one, first kept model.py:700-706

The reference draws with ``torch.multinomial`` (model.py:707-708), whose RNG
stream cannot take external uniforms.  This build defines the draw so two
implementations fed the same logits and the same uniform ``u`` in [0, 1)
pick the same code:

1. candidates = finite values that survive top-k, ordered by value
   descending, ties by lower index first;
2. ``w_i = exp(x_i - x_0)`` in float64, ``W_i`` = prefix sums in a fixed
   order (``scan_sums``: groups of 64 scanned as rows of 16 then across
   rows, plus a running carry);
3. top-p keeps the leading candidates up to and including the first i with
   ``W_i > p * W_{n-1}`` (all n if none; p taken as an FP32 value promoted to
   float64, the product rounded once), i.e. ``cum > p`` shifted right by one;
4. the code is the first kept candidate with ``W_j > u * W_{n_keep-1}``
   (the last kept one if rounding leaves none).

Temperature, CFG scale and top-p cross every interface as FP32 values,
as they do in the reference (a Python float against an FP32 tensor).
"""

from __future__ import annotations

import numpy as np


def cfg_merge(cond, uncond, scale):
    """FP32 ``uncond + s * (cond - uncond)`` (model.py:581)."""
    c = np.asarray(cond, np.float32)
    u = np.asarray(uncond, np.float32)
    return (u + np.float32(scale) * (c - u)).astype(np.float32)


def apply_masks(merged, *, q: int, frame_index: int, min_new_frames: int,
                bos_id: int, eos_id: int, pad_id: int):
    """-inf on BOS/PAD always, on EOS unless q == 0 and frame >= min_new_frames
    (model.py:556-559,582-584)."""
    out = np.array(merged, np.float32, copy=True)
    out[bos_id] = -np.inf
    out[pad_id] = -np.inf
    if q != 0 or frame_index < min_new_frames:
        out[eos_id] = -np.inf
    return out


def greedy(merged) -> int:
    """First index of the maximum (torch.argmax, model.py:694-695)."""
    return int(np.argmax(np.asarray(merged, np.float32)))


def candidates(x, top_k):
    """Indices surviving top-k (model.py:697-699), finite only, ordered by
    value descending then index ascending."""
    x = np.asarray(x, np.float32)
    V = x.size
    keep = np.isfinite(x)
    if top_k is not None and 0 < top_k < V:
        cutoff = np.sort(x)[::-1][top_k - 1]
        keep &= x >= cutoff
    idx = np.nonzero(keep)[0]
    return idx[np.lexsort((idx, -x[idx].astype(np.float64)))]


def _scan64(blk):
    """Inclusive float64 scan of 64 values in the fixed order: within each
    row of 16 lanes add the value 1, 2, 4, 8 lanes below (same row only),
    then rows 1 and 3 add the last value of the row before, then rows 2 and
    3 add value 31.  Every step adds pre-step values, one rounding each."""
    b = np.array(blk, np.float64)
    lane = np.arange(64)
    for off in (1, 2, 4, 8):
        src = b.copy()
        on = (lane % 16) >= off
        b[on] = src[on] + src[lane[on] - off]
    src = b.copy()
    for r in (1, 3):
        b[16 * r:16 * r + 16] = src[16 * r:16 * r + 16] + src[16 * r - 1]
    src = b.copy()
    b[32:] = src[32:] + src[31]
    return b


def scan_sums(w) -> np.ndarray:
    """Inclusive float64 prefix sums in the fixed order both sides use:
    groups of 64 candidates, each scanned by ``_scan64``, plus the running
    total of the earlier groups (carry + group scan, one rounding)."""
    w = np.asarray(w, np.float64)
    n = w.size
    out = np.empty(n, np.float64)
    carry = 0.0
    for g0 in range(0, n, 64):
        m = min(64, n - g0)
        blk = np.zeros(64, np.float64)
        blk[:m] = w[g0:g0 + m]
        blk = _scan64(blk)
        out[g0:g0 + m] = carry + blk[:m]
        carry = carry + blk[63]
    return out


def topp_weights(vals, top_p):
    """float64 weights, prefix sums and the kept count (model.py:700-706
    restated in float64)."""
    v = np.asarray(vals, np.float32).astype(np.float64)
    w = np.exp(v - v[0])
    W = scan_sums(w)
    n = v.size
    n_keep = n
    if top_p is not None and 0 < top_p < 1:
        p = float(np.float32(top_p))
        over = np.nonzero(W[:-1] > p * W[-1])[0]
        if over.size:
            n_keep = int(over[0]) + 1
    return w, W, n_keep


def filtered_probs(x, top_k, top_p) -> np.ndarray:
    """The distribution the reference passes to ``torch.multinomial``
    (model.py:707), in float64, over all V entries."""
    x = np.asarray(x, np.float32)
    order = candidates(x, top_k)
    w, W, n_keep = topp_weights(x[order], top_p)
    out = np.zeros(x.size, np.float64)
    out[order[:n_keep]] = w[:n_keep] / W[n_keep - 1]
    return out


def draw(x, top_k, top_p, u: float) -> int:
    """Inverse-CDF draw over the filtered candidates (definition above)."""
    x = np.asarray(x, np.float32)
    order = candidates(x, top_k)
    _, W, n_keep = topp_weights(x[order], top_p)
    target = float(u) * float(W[n_keep - 1])
    hit = np.nonzero(W[:n_keep] > target)[0]
    j = int(hit[0]) if hit.size else n_keep - 1
    return int(order[j])


def sample(merged, *, temperature, top_k, top_p, u) -> int:
    """``_sample_logits`` (model.py:686-708) with the explicit-uniform draw."""
    if temperature <= 0:
        return greedy(merged)
    x = (np.asarray(merged, np.float32) / np.float32(temperature)).astype(np.float32)
    return draw(x, top_k, top_p, u)

"""CPU model of the many-row decode attention's slot decomposition
(attention_stream_kernel in csrc/sk_kernels.h): which cached tokens each slot
holds, and the per-slot online softmax the kernel runs over them before the
slots are merged.  It shows that the GPU tests of the throughput batch at its
own prefixes (tests/test_gpu_engine.py, 120-240 and 440-505 positions) give
slots several tokens, so a slot loop that dropped the running-max rescale
would fail them, while the short-prefix tests (at most ~36 cached tokens)
give every slot one token and cannot see that mistake.

The mistake is planted here, in this CPU model, never in GPU code.  Exact
attention (model.py:658-676, sdpa over a branch's own history) is the float64
softmax over all tokens.
"""

import numpy as np
import pytest

HD = 128
LPT = HD // 16          # lanes per slot (16 head dims per lane)
NTH = 512               # threads per workgroup
TPP = NTH // LPT        # slots per split


def slot_tokens(ctx, S, s, slot):
    """Tokens of slot `slot` of split `s`: t = s*TPP + slot + j*S*TPP < ctx."""
    return list(range(s * TPP + slot, ctx, S * TPP))


def slot_attention(q, k, v, S, rescale=True):
    """One query head: per-slot online softmax in token order, then the
    merge of every slot's (max, sum, output) -- the kernel's arithmetic
    order, in float32.  rescale=False drops the rescale of the running sum
    and output when a later token raises the slot's maximum."""
    ctx = k.shape[0]
    scale = np.float32(HD ** -0.5)
    states = []
    for s in range(S):
        for slot in range(TPP):
            m, l, o = np.float32(-np.inf), np.float32(0), np.zeros(HD, np.float32)
            for t in slot_tokens(ctx, S, s, slot):
                x = np.float32(q @ k[t]) * scale
                mn = max(m, x)
                c = np.exp(np.float32(m - mn)) if rescale else np.float32(1)
                e = np.exp(np.float32(x - mn))
                l = l * c + e
                o = o * c + e * v[t]
                m = mn
            if l > 0:
                states.append((m, l, o))
    M = max(m for m, _, _ in states)
    L = sum(l * np.exp(np.float32(m - M)) for m, l, _ in states)
    O = sum(o * np.exp(np.float32(m - M)) for m, _, o in states)
    return O / L


def exact_attention(q, k, v):
    x = (k.astype(np.float64) @ q.astype(np.float64)) * HD ** -0.5
    p = np.exp(x - x.max())
    return (p / p.sum()) @ v.astype(np.float64)


def _case(ctx, seed):
    rng = np.random.default_rng(seed)
    # unit-RMS rows, as after Qwen3's per-head RMSNorm with unit gain
    q = rng.standard_normal(HD).astype(np.float32)
    k = rng.standard_normal((ctx, HD)).astype(np.float32)
    v = rng.standard_normal((ctx, HD)).astype(np.float32)
    return q, k, v


def _rel(got, ref):
    return float(np.abs(got - ref).max() / np.abs(ref).max())


@pytest.mark.parametrize("ctx", [1, 36, 64, 65, 121, 241, 508])
def test_slot_model_equals_exact_attention(ctx):
    q, k, v = _case(ctx, ctx)
    assert _rel(slot_attention(q, k, v, 1), exact_attention(q, k, v)) < 1e-5


def test_split_model_equals_exact_attention():
    """Four splits (the tiny shape's 16 utterances): slots 2,048 apart."""
    q, k, v = _case(300, 3)
    assert _rel(slot_attention(q, k, v, 4), exact_attention(q, k, v)) < 1e-5


@pytest.mark.parametrize("ctx", [121, 241, 441, 508])
def test_dropped_rescale_fails_at_throughput_prefixes(ctx):
    """At the throughput batch's contexts (one split per (row, kv head), 64
    slots: 2-8 tokens each) the planted mistake moves the output far past the
    GPU tests' 1e-3 tolerance."""
    q, k, v = _case(ctx, 100 + ctx)
    assert _rel(slot_attention(q, k, v, 1, rescale=False), exact_attention(q, k, v)) > 1e-2


@pytest.mark.parametrize("ctx", [5, 36, 64])
def test_dropped_rescale_is_invisible_with_one_token_per_slot(ctx):
    """With at most 64 cached tokens every slot holds one token, so the
    mistake changes nothing: short-prefix tests cannot catch it."""
    q, k, v = _case(ctx, 200 + ctx)
    assert _rel(slot_attention(q, k, v, 1, rescale=False), exact_attention(q, k, v)) < 1e-5

"""Pins for the oracle's sampler and BF16 rounding that do not come from the
reference's golden vectors: closed forms, brute force and a chi-square test.

The reference draws with ``torch.multinomial`` (soraku_inference/model.py:707-708),
which takes no external uniform, so ``oracle.sampler.draw`` is this build's
definition of the draw: the inverse CDF of the filtered distribution, with
the candidates in descending-value order (ties: lower index first).  What
pins it here:

* the set of uniforms that lands on each candidate is one interval, the
  intervals follow the candidate order, and each has width
  ``filtered_probs[i]`` -- the distribution the reference hands to
  ``torch.multinomial``, itself pinned by the reference's probability
  vectors in ``tests/golden`` (test_oracle_golden.py);
* a uniform exactly on a boundary belongs to the upper interval
  (``u`` in ``[F_{j-1}, F_j)`` draws candidate j);
* k = 1 gives the argmax, a tiny top-p the top candidate, T <= 0 the first
  maximum, whatever the uniform;
* brute force of the reference's top-k / top-p rule on tiny V;
* a chi-square test of 10^5 seeded draws against ``filtered_probs``.

Each check is also run against planted mistakes (the draw replaced by an
argmax, ``>`` replaced by ``>=``, the kept mass normalised by the total
instead of the kept total) and must reject every one of them.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

from oracle.model import round_bf16
from oracle.sampler import (candidates, draw, filtered_probs, greedy, sample,
                            topp_weights)

U_MAX = 1.0 - 2.0 ** -53   # largest double below 1


# ---------------------------------------------------------------- black-box helpers

def draw_intervals(draw_fn, x, top_k, top_p):
    """The intervals of u in [0, 1) that map to each code, found by bisection
    on the draw alone: ``[(code, lo, hi), ...]`` in increasing u."""
    out = []
    lo = 0.0
    code = draw_fn(x, top_k, top_p, lo)
    last = draw_fn(x, top_k, top_p, U_MAX)
    while True:
        if code == last:
            out.append((code, lo, 1.0))
            return out
        a, b = lo, U_MAX          # draw(a) == code, draw(b) != code
        while True:
            mid = 0.5 * (a + b)
            if mid <= a or mid >= b:
                break
            if draw_fn(x, top_k, top_p, mid) == code:
                a = mid
            else:
                b = mid
        out.append((code, lo, b))
        lo = b
        code = draw_fn(x, top_k, top_p, b)
        if len(out) > 4 * len(x):
            raise AssertionError("draw is not monotone in u")


def check_preimage_widths(draw_fn, x, top_k, top_p, tol=1e-12):
    """Each kept candidate owns one interval of width filtered_probs[i], in
    candidate order; nothing else is ever drawn."""
    probs = filtered_probs(x, top_k, top_p)
    order = [int(i) for i in candidates(x, top_k) if probs[i] > 0]
    iv = draw_intervals(draw_fn, x, top_k, top_p)
    codes = [c for c, _, _ in iv]
    # candidates whose width is below double resolution may be skipped
    want = [i for i in order if probs[i] > 1e-15]
    assert [c for c in codes if probs[c] > 1e-15] == want, (codes, want)
    assert all(probs[c] > 0 for c in codes), "drew a filtered-out code"
    for c, lo, hi in iv:
        assert abs((hi - lo) - probs[c]) <= tol, (c, hi - lo, probs[c])


def check_boundary_convention(draw_fn):
    """Four equal logits: candidates 0..3 own [0,.25), [.25,.5), [.5,.75),
    [.75,1); every boundary is exact in binary, and u on a boundary belongs
    to the upper interval."""
    x = np.array([3.0, 3.0, 3.0, 3.0], np.float32)
    for u, want in ((0.0, 0), (0.25, 1), (0.5, 2), (0.75, 3), (0.2499999, 0), (U_MAX, 3)):
        got = draw_fn(x, None, None, u)
        assert got == want, (u, got, want)


def check_top_candidate_cases(draw_fn):
    rng = np.random.default_rng(5)
    for _ in range(20):
        x = (rng.standard_normal(37) * 3).astype(np.float32)
        for u in (0.0, 0.3, 0.77, U_MAX):
            assert draw_fn(x, 1, None, u) == int(np.argmax(x))          # k = 1
            assert draw_fn(x, None, 1e-9, u) == int(np.argmax(x))       # p -> 0
            assert draw_fn(x, 50, 1e-6, u) == int(np.argmax(x))


# ---------------------------------------------------------------- planted mistakes

def _draw_argmax(x, top_k, top_p, u):
    return int(np.argmax(np.asarray(x, np.float32)))


def _draw_ge(x, top_k, top_p, u):
    x = np.asarray(x, np.float32)
    order = candidates(x, top_k)
    _, W, n_keep = topp_weights(x[order], top_p)
    hit = np.nonzero(W[:n_keep] >= float(u) * float(W[n_keep - 1]))[0]
    return int(order[int(hit[0]) if hit.size else n_keep - 1])


def _draw_total_norm(x, top_k, top_p, u):
    x = np.asarray(x, np.float32)
    order = candidates(x, top_k)
    _, W, n_keep = topp_weights(x[order], top_p)
    hit = np.nonzero(W[:n_keep] > float(u) * float(W[-1]))[0]
    return int(order[int(hit[0]) if hit.size else n_keep - 1])


def _cases():
    rng = np.random.default_rng(17)
    out = []
    for V, k, p in ((9, None, None), (40, 12, 0.9), (64, None, 0.6), (130, 50, 0.95),
                    (300, 80, None), (2051, 50, 0.95)):
        x = (rng.standard_normal(V) * 2.5).astype(np.float32)
        x[rng.integers(0, V, 2)] = -np.inf
        out.append((x, k, p))
    # ties at the top-k cutoff are kept (model.py:697-699)
    x = np.array([1.0, 4.0, 2.0, 4.0, 2.0, 2.0, -1.0, 0.5], np.float32)
    out.append((x, 3, None))
    out.append((x, 3, 0.7))
    return out


# ---------------------------------------------------------------- tests

@pytest.mark.parametrize("case", range(8))
def test_draw_preimage_of_each_candidate_is_its_probability(case):
    x, k, p = _cases()[case]
    check_preimage_widths(draw, x, k, p)


def test_draw_boundary_belongs_to_upper_candidate():
    check_boundary_convention(draw)


def test_draw_k1_and_tiny_p_give_the_top_candidate():
    check_top_candidate_cases(draw)


def test_greedy_is_first_max_for_any_uniform():
    x = np.array([1.0, 5.0, -2.0, 5.0, 5.0], np.float32)
    assert greedy(x) == 1
    for u in (0.0, 0.5, U_MAX):
        for t in (0.0, -1.0):
            assert sample(x, temperature=t, top_k=2, top_p=0.5, u=u) == 1


def _reference_rule_bruteforce(x, top_k, top_p):
    """The filter of model.py:697-707 written out over a Python list in float64:
    cutoff = k-th largest, drop values below it; sort descending, softmax,
    cumulative sum, drop where the sum before an entry already exceeds p
    (the shift by one), then renormalise."""
    vals = [float(v) for v in x]
    V = len(vals)
    if top_k is not None and 0 < top_k < V:
        cutoff = sorted(vals, reverse=True)[top_k - 1]
        vals = [v if v >= cutoff else -math.inf for v in vals]
    keep = [v > -math.inf for v in vals]
    if top_p is not None and 0 < top_p < 1:
        order = sorted(range(V), key=lambda i: (-vals[i], i))
        m = vals[order[0]]
        den = math.fsum(math.exp(vals[i] - m) for i in order if vals[i] > -math.inf)
        cum = 0.0
        for i in order:
            if vals[i] == -math.inf:
                continue
            if cum > float(np.float32(top_p)):
                keep[i] = False
            cum += math.exp(vals[i] - m) / den
    kept = [i for i in range(V) if keep[i]]
    m = max(vals[i] for i in kept)
    den = math.fsum(math.exp(vals[i] - m) for i in kept)
    return np.array([math.exp(vals[i] - m) / den if keep[i] else 0.0 for i in range(V)])


def test_filter_matches_bruteforce_on_tiny_vocab():
    rng = np.random.default_rng(23)
    n = 0
    for V in range(2, 9):
        for _ in range(30):
            x = rng.integers(-3, 4, V).astype(np.float32) * np.float32(0.7)   # many ties
            if rng.random() < 0.3:
                x[rng.integers(0, V)] = -np.inf
            if not np.isfinite(x).any():
                continue
            k = int(rng.integers(1, V + 1)) if rng.random() < 0.7 else None
            p = float(rng.choice([0.3, 0.5, 0.8, 0.95])) if rng.random() < 0.7 else None
            want = _reference_rule_bruteforce(x, k, p)
            got = filtered_probs(x, k, p)
            np.testing.assert_allclose(got, want, rtol=0, atol=1e-12, err_msg=f"{x} k={k} p={p}")
            check_preimage_widths(draw, x, k, p)
            n += 1
    assert n > 150


def test_draw_chi_square_against_filtered_probs():
    from scipy.stats import chisquare

    rng = np.random.default_rng(2026)
    x = (rng.standard_normal(60) * 1.5).astype(np.float32)
    k, p = 30, 0.9
    probs = filtered_probs(x, k, p)
    n = 100_000
    us = np.random.default_rng(99).random(n)
    counts = np.bincount([draw(x, k, p, float(u)) for u in us], minlength=x.size)
    kept = probs > 0
    assert counts[~kept].sum() == 0
    stat, pval = chisquare(counts[kept], probs[kept] * n)
    assert pval > 1e-4, (stat, pval)


@pytest.mark.parametrize("mutant", [_draw_argmax, _draw_ge, _draw_total_norm],
                         ids=["argmax", "ge", "total_norm"])
def test_planted_draw_mistakes_are_rejected(mutant):
    def rejected(check, *args):
        try:
            check(mutant, *args)
        except AssertionError:
            return True
        return False

    caught = rejected(check_boundary_convention) or rejected(check_top_candidate_cases)
    for x, k, p in _cases():
        caught = caught or rejected(check_preimage_widths, x, k, p)
    assert caught, f"{mutant.__name__} passed every draw check"


def test_round_bf16_matches_torch():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(4)
    parts = [
        rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-30, 30, 20000),
        # exact halfway cases: the 16 dropped bits are 0x8000 (ties to even, both parities)
        (rng.integers(0, 2 ** 31, 4000, dtype=np.uint32) & 0xFFFF0000 | 0x8000).view(np.float32),
        (rng.integers(0, 2 ** 31, 4000, dtype=np.uint32) | 0x7FFF).view(np.float32),
        np.array([0.0, -0.0, np.inf, -np.inf, 3.4028235e38, -3.4028235e38, 1e-45, 1.1754944e-38,
                  3.3961776e38, 65504.0], np.float32),
        rng.integers(1, 2 ** 23, 2000, dtype=np.uint32).view(np.float32),    # subnormals
    ]
    x = np.concatenate([p[np.isfinite(p) | np.isinf(p)] for p in parts]).astype(np.float32)
    want = torch.from_numpy(x).to(torch.bfloat16).to(torch.float32).numpy()
    got = round_bf16(x)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


# ---------------------------------------------------------------- trunk math closed forms

def test_rms_norm_closed_forms():
    from oracle.model import rms_norm

    rng = np.random.default_rng(1)
    x = rng.standard_normal((5, 64))
    y = rms_norm(x, np.ones(64), 0.0)
    np.testing.assert_allclose(np.sqrt(np.mean(y * y, -1)), 1.0, rtol=1e-12)
    np.testing.assert_allclose(rms_norm(7.5 * x, np.ones(64), 0.0), y, rtol=1e-12)
    w = rng.standard_normal(64)
    np.testing.assert_allclose(rms_norm(x, w, 1e-6), w * x / np.sqrt(np.mean(x * x, -1, keepdims=True) + 1e-6),
                               rtol=1e-13)


def test_silu_closed_form():
    from oracle.model import silu

    from scipy.special import expit

    g = np.linspace(-20, 20, 401)
    np.testing.assert_allclose(silu(g), g * expit(g), rtol=1e-13)
    assert silu(0.0) == 0.0


def test_rope_identities():
    from oracle.model import apply_rope, rope_cos_sin

    rng = np.random.default_rng(2)
    hd = 128
    q = rng.standard_normal(hd)
    k = rng.standard_normal(hd)
    c0, s0 = rope_cos_sin([0], hd, 1e6)
    np.testing.assert_array_equal(apply_rope(q[None], c0, s0)[0], q)          # position 0
    pos = np.array([3, 17, 250, 480, 720])
    c, s = rope_cos_sin(pos, hd, 1e6)
    rq = apply_rope(np.repeat(q[None], len(pos), 0), c, s)
    rk = apply_rope(np.repeat(k[None], len(pos), 0), c, s)
    np.testing.assert_allclose(np.linalg.norm(rq, axis=-1), np.linalg.norm(q), rtol=1e-6)
    # <R_m q, R_n k> depends only on m - n: (17, 3) and (720 - 14 ... ) pairs
    c2, s2 = rope_cos_sin([31, 17], hd, 1e6)
    a = apply_rope(q[None], c2[:1], s2[:1])[0] @ apply_rope(k[None], c2[1:], s2[1:])[0]
    b = rq[1] @ rk[0]                                                        # 17 vs 3: same m - n = 14
    np.testing.assert_allclose(a, b, rtol=2e-5)
    # the rotation is rotate-half: pair (i, i + hd/2) turns by pos * theta^(-2i/hd)
    i = 5
    ang = np.float32(250) * np.float32(1.0 / np.float32(1e6) ** np.float32(2 * i / hd))
    z = complex(q[i], q[i + hd // 2]) * complex(math.cos(ang), math.sin(ang))
    np.testing.assert_allclose([rq[2][i], rq[2][i + hd // 2]], [z.real, z.imag], rtol=1e-6)


def test_attention_closed_forms():
    from oracle.model import attend

    rng = np.random.default_rng(3)
    Hq, Hkv, hd = 4, 2, 16
    q = rng.standard_normal((Hq, hd))
    k1 = rng.standard_normal((Hkv, 1, hd))
    v1 = rng.standard_normal((Hkv, 1, hd))
    out = attend(q, k1, v1, 0.25)
    np.testing.assert_allclose(out, np.repeat(v1[:, 0], 2, 0), rtol=1e-14)   # one token -> v
    keq = np.repeat(rng.standard_normal((Hkv, 1, hd)), 9, axis=1)             # equal keys -> mean of V
    v = rng.standard_normal((Hkv, 9, hd))
    np.testing.assert_allclose(attend(q, keq, v, 0.25), np.repeat(v.mean(1), 2, 0), rtol=1e-12, atol=1e-15)
    k = rng.standard_normal((Hkv, 9, hd))
    # GQA: q head h reads kv head h // (Hq / Hkv); brute force per head
    for h in range(Hq):
        s = k[h // 2] @ q[h] * 0.25
        p = np.exp(s - s.max())
        p /= p.sum()
        np.testing.assert_allclose(attend(q, k, v, 0.25)[h], p @ v[h // 2], rtol=1e-12)

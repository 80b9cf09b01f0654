"""Operator-level parity on the GPU: each fused kernel of the decode step
against the oracle at the isolated-kernel decode shape (M=2 rows, hidden
1024, SwiGLU 1024->2x3072->1024 and 1024->2x2048->1024, 16-codebook
classifier 1024->2051), FP32 and BF16 weights with FP32 accumulation."""

import numpy as np
import pytest

import oracle.model as om
import oracle.sampler as osm

pytestmark = pytest.mark.gpu

FLT_EPS = om.FLT_EPS
# GEMV tolerance: relative to the output's max |value|; FP32 accumulation of
# up to 3072 terms in a different order than float64.
TOL = 2e-5


def _t(x, dev, dtype=None):
    import torch

    t = torch.from_numpy(np.ascontiguousarray(x)).to(dev)
    return t if dtype is None else t.to(dtype)


def _rel(got, ref):
    return float(np.abs(np.asarray(got, np.float64) - ref).max() / max(np.abs(ref).max(), 1e-30))


@pytest.fixture(scope="module")
def ops(hip_device):
    from soraku_amd import ops as O

    return O


@pytest.mark.parametrize("eps", [1e-6, FLT_EPS])
def test_rmsnorm_and_add_rmsnorm(ops, hip_device, eps):
    rng = np.random.default_rng(1)
    x = rng.standard_normal((2, 1024), dtype=np.float32)
    p = rng.standard_normal((2, 1024), dtype=np.float32)
    w = (1 + 0.1 * rng.standard_normal(1024)).astype(np.float32)
    got = ops.rmsnorm(2, 1024, eps)(_t(x, hip_device), _t(w, hip_device)).cpu().numpy()
    assert _rel(got, om.rms_norm(x.astype(np.float64), w.astype(np.float64), eps)) < 1e-6
    got = ops.add_rmsnorm(2, 1024, eps)(_t(x, hip_device), _t(p, hip_device), _t(w, hip_device)).cpu().numpy()
    ref = om.rms_norm((x + p).astype(np.float64), w.astype(np.float64), eps)
    assert _rel(got, ref) < 1e-6


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("I", [2048, 3072, 4096, 6144])
def test_swiglu_and_down_gemv(ops, hip_device, bf16, I):
    import torch

    rng = np.random.default_rng(2)
    D, B = 1024, 2
    x = rng.standard_normal((B, D), dtype=np.float32)
    wg = (rng.standard_normal((I, D), dtype=np.float32) * 0.02).astype(np.float32)
    wu = (rng.standard_normal((I, D), dtype=np.float32) * 0.02).astype(np.float32)
    wd = (rng.standard_normal((D, I), dtype=np.float32) * 0.02).astype(np.float32)
    res = rng.standard_normal((B, D), dtype=np.float32)
    if bf16:
        wg, wu, wd = om.round_bf16(wg), om.round_bf16(wu), om.round_bf16(wd)
    dt = torch.bfloat16 if bf16 else torch.float32
    act = ops.swiglu_gemv(B, I, D)(_t(x, hip_device), _t(wg, hip_device, dt), _t(wu, hip_device, dt))
    x64 = x.astype(np.float64)
    ref_act = om.silu(x64 @ wg.T.astype(np.float64)) * (x64 @ wu.T.astype(np.float64))
    assert _rel(act.cpu().numpy(), ref_act) < TOL
    y = ops.down_residual_gemv(B, D, I)(act, _t(wd, hip_device, dt), _t(res, hip_device))
    ref_y = act.cpu().numpy().astype(np.float64) @ wd.T.astype(np.float64) + res
    assert _rel(y.cpu().numpy(), ref_y) < TOL


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("I", [2048, 6144])
def test_down_gemv_ragged_rows(ops, hip_device, bf16, I):
    """Down projection + residual with an output count that is not a multiple
    of the 4 rows a K-sliced workgroup owns (the last workgroup's extra rows
    re-read row N-1 and are not stored)."""
    rng = np.random.default_rng(5)
    D, B = 1030, 2
    import torch

    act = rng.standard_normal((B, I), dtype=np.float32)
    wd = (rng.standard_normal((D, I), dtype=np.float32) * 0.02).astype(np.float32)
    res = rng.standard_normal((B, D), dtype=np.float32)
    if bf16:
        wd = om.round_bf16(wd)
    dt = torch.bfloat16 if bf16 else torch.float32
    y = ops.down_residual_gemv(B, D, I)(_t(act, hip_device), _t(wd, hip_device, dt), _t(res, hip_device))
    ref_y = act.astype(np.float64) @ wd.T.astype(np.float64) + res
    assert y.shape == (B, D)
    assert _rel(y.cpu().numpy(), ref_y) < TOL


@pytest.mark.parametrize("bf16", [False, True])
def test_classifier_gemv_all_codebooks(ops, hip_device, bf16):
    import torch

    rng = np.random.default_rng(3)
    D, B, V, Q = 1024, 2, 2051, 16
    table = (rng.standard_normal((Q, V, D), dtype=np.float32) * 0.02).astype(np.float32)
    if bf16:
        table = om.round_bf16(table)
    bias = (rng.standard_normal((Q, V)) * 0.02).astype(np.float32)
    body = rng.standard_normal((B, D), dtype=np.float32)
    dt = torch.bfloat16 if bf16 else torch.float32
    tt = _t(table, hip_device, dt)
    k = ops.classifier_gemv(B, V, D)
    for q in range(Q):
        got = k(_t(body, hip_device), tt[q], _t(bias[q], hip_device)).cpu().numpy()
        ref = body.astype(np.float64) @ table[q].T.astype(np.float64) + bias[q]
        assert _rel(got, ref) < TOL, q


def test_gemv_odd_batches(ops, hip_device):
    """B = 1, 3, 5 rows (chunks of at most four rows per launch)."""
    rng = np.random.default_rng(4)
    D, V = 256, 37
    w = (rng.standard_normal((V, D), dtype=np.float32) * 0.02).astype(np.float32)
    bias = rng.standard_normal(V).astype(np.float32)
    for B in (1, 3, 5):
        x = rng.standard_normal((B, D), dtype=np.float32)
        got = ops.classifier_gemv(B, V, D)(_t(x, hip_device), _t(w, hip_device), _t(bias, hip_device))
        ref = x.astype(np.float64) @ w.T.astype(np.float64) + bias
        assert _rel(got.cpu().numpy(), ref) < TOL


def test_frame_embed_and_prefix_add_bitexact(ops, hip_device):
    """Gather-sums: same FP32 additions in the same order as the oracle."""
    import torch

    rng = np.random.default_rng(5)
    Q, V, D = 16, 2051, 1024
    table = (rng.standard_normal((Q, V, D), dtype=np.float32) * 0.02).astype(np.float32)
    codes = rng.integers(0, V, size=(3, Q)).astype(np.int64)
    scale = Q ** -0.5
    got = ops.frame_embed(3, Q, V, D, scale)(_t(codes, hip_device), _t(table, hip_device)).cpu().numpy()
    m = om.OracleModel(om.Shape(d_model=D, n_codebooks=Q, codebook_size=V - 3),
                       {"audio_codebooks.table": table}, np.float32)
    ref = m.frame_embedding(codes)
    np.testing.assert_array_equal(got, ref)
    prefix = rng.standard_normal((2, D), dtype=np.float32)
    code = torch.tensor([int(codes[0, 3])], dtype=torch.int64, device=hip_device)
    got = ops.prefix_add(2, V, D, scale)(_t(prefix, hip_device), _t(table[3], hip_device), code).cpu().numpy()
    np.testing.assert_array_equal(got, prefix + table[3][codes[0, 3]] * np.float32(scale))


def test_sampling_prep_bitexact(ops, hip_device):
    import torch

    rng = np.random.default_rng(6)
    V = 2051
    x = rng.standard_normal(V, dtype=np.float32) * 3
    for T, me in ((0.9, 1), (1.3, 0)):
        got = ops.sampling_prep(V, 2048, 2050, 2049)(
            _t(x, hip_device), torch.tensor([T], dtype=torch.float32, device=hip_device),
            torch.tensor([me], dtype=torch.int32, device=hip_device)).cpu().numpy()
        ref = x / np.float32(T)
        ref[2048] = ref[2050] = -np.inf
        if me:
            ref[2049] = -np.inf
        np.testing.assert_array_equal(got, ref)


def _sample_cases():
    rng = np.random.default_rng(7)
    cases = []
    for i in range(120):
        V = 2051 if i % 4 else int(rng.integers(8, 300))
        cfg = [1.0, 1.5, 0.0, 3.0][i % 4]
        rows = 1 if cfg == 1.0 else 2
        T = [0.9, 0.0, 0.5, 1.7, -1.0][i % 5]
        k = [50, None, 1, 200, V - 1, 64, 65][i % 7]
        p = [0.95, None, 0.5, 1e-6, 0.999][i % 5]
        scale = [1.0, 4.0, 0.05][i % 3]
        logits = (rng.standard_normal((rows, V)) * scale).astype(np.float32)
        if i % 6 == 0:  # heavy ties
            logits = np.round(logits * 2) / 2
        q = i % 3
        me = i % 2
        u = float(rng.random())
        cases.append((V, rows, cfg, T, k, p, logits, q, me, u))
    return cases


def test_sampler_bitexact_against_oracle(ops, hip_device):
    """Identical logits + identical uniform => identical code, over greedy,
    top-k only, top-p only, both, ties, k beyond one wave, tiny p, CFG 0/1/1.5/3."""
    mism = []
    for V, rows, cfg, T, k, p, logits, q, me, u in _sample_cases():
        bos, eos, pad = V - 3, V - 2, V - 1
        kern = ops.sample(V, bos, eos, pad)
        got = int(kern(_t(logits, hip_device), cfg_scale=cfg, q=q, mask_eos_q0=me, temperature=T,
                       top_k=k, top_p=p, u=u).cpu()[0])
        merged = logits[0] if rows == 1 else osm.cfg_merge(logits[0], logits[1], cfg)
        masked = osm.apply_masks(merged, q=q, frame_index=0 if me else 10**6, min_new_frames=1,
                                 bos_id=bos, eos_id=eos, pad_id=pad)
        ref = osm.sample(masked, temperature=T, top_k=k, top_p=p, u=u)
        if got != ref:
            mism.append((V, rows, cfg, T, k, p, q, me, u, got, ref))
    assert not mism, mism[:5]

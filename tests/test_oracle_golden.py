"""The oracle against golden vectors written by the reference's native path
(tests/golden/make_golden.py: SorakuTTSv2.generate over the transformers
Qwen3 trunk, CPU, seeded weights)."""

import numpy as np
import pytest

from conftest import load_golden
from oracle.generate import Record, generate
from oracle.model import OracleModel, synthetic_weights
from oracle.sampler import apply_masks, filtered_probs

TINY_FIXTURES = ["tiny_greedy", "tiny_sampled", "tiny_nocfg_topp", "tiny_untied"]


def _model(f, s, dtype):
    w = synthetic_weights(s, int(f["seed"]), norm_gain_std=float(f["norm_gain_std"]),
                          bias_std=float(f["bias_std"]))
    return OracleModel(s, w, dtype, language_token_ids=tuple(int(v) for v in f["language_ids"]))


def _masked_calls(rec, s, gen, n):
    out = []
    for fi, fr in enumerate(rec.merged):
        for q, m in enumerate(fr):
            out.append(apply_masks(m, q=q, frame_index=fi, min_new_frames=gen["min_new_frames"],
                                   bos_id=s.bos_id, eos_id=s.eos_id, pad_id=s.pad_id))
    return np.stack(out[:n])


def _forced(f, s):
    codes = f["codes"]
    if int(f["stop_eos"]):
        codes = np.concatenate([codes, np.full((1, s.n_codebooks), s.eos_id)])
    return codes


def _run(f, s, gen, dtype, batched=False):
    m = _model(f, s, dtype)
    g = {k: v for k, v in gen.items() if k != "seed"}
    rec = Record()
    codes, info = generate(m, input_ids=f["text_ids"], prompt_codes=f["prompt_codes"],
                           uncond_input_ids=f["uncond_ids"], forced_codes=_forced(f, s),
                           record=rec, batched=batched, **g)
    return rec, codes, info


@pytest.mark.parametrize("name", TINY_FIXTURES)
@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_sample_logits_match_reference(name, dtype):
    f, s, gen = load_golden(name)
    rec, codes, _ = _run(f, s, gen, dtype)
    ref = f["sample_logits"]
    got = _masked_calls(rec, s, gen, ref.shape[0])
    fin = np.isfinite(ref)
    assert (np.isfinite(got) == fin).all()
    rel = np.abs(got[fin] - ref[fin]).max() / np.abs(ref[fin]).max()
    assert rel < 2e-6, rel
    np.testing.assert_array_equal(codes, f["codes"])


@pytest.mark.parametrize("name", TINY_FIXTURES)
def test_hidden_states_match_reference(name):
    f, s, gen = load_golden(name)
    rec, _, _ = _run(f, s, gen, np.float64)
    ref = f["hidden"]
    got = np.stack(rec.hidden)
    n = min(len(got), len(ref))
    assert n >= ref.shape[0] - 1
    rel = np.abs(got[:n] - ref[:n]).max() / np.abs(ref).max()
    assert rel < 2e-6, rel


def test_greedy_free_running_codes_match_reference():
    f, s, gen = load_golden("tiny_greedy")
    m = _model(f, s, np.float64)
    g = {k: v for k, v in gen.items() if k != "seed"}
    codes, info = generate(m, input_ids=f["text_ids"], prompt_codes=f["prompt_codes"],
                           uncond_input_ids=f["uncond_ids"], **g)
    np.testing.assert_array_equal(codes, f["codes"])
    assert info["stop_reason"] == ("eos" if int(f["stop_eos"]) else "max_frames")


def _check_filtered(rec, f, s, gen):
    ref = f["probs"]
    got = _masked_calls(rec, s, gen, ref.shape[0])
    i = 0
    for fi in range(len(rec.merged)):
        for q in range(s.n_codebooks):
            if i >= ref.shape[0]:
                break
            t = gen.get("temperature_q0") if q == 0 and gen.get("temperature_q0") is not None else gen["temperature"]
            k = gen.get("top_k_q0") if q == 0 and gen.get("top_k_q0") is not None else gen.get("top_k")
            p = gen.get("top_p_q0") if q == 0 and gen.get("top_p_q0") is not None else gen.get("top_p")
            x = (got[i] / np.float32(t)).astype(np.float32)
            pr = filtered_probs(x, k, p)
            np.testing.assert_array_equal(pr > 0, ref[i] > 0)
            assert np.abs(pr - ref[i]).max() < 1e-6
            i += 1
    assert i == ref.shape[0]


@pytest.mark.parametrize("name", ["tiny_sampled", "tiny_nocfg_topp", "tiny_untied"])
def test_filtered_distribution_matches_reference(name):
    """Top-k / top-p filter = what _sample_logits hands to torch.multinomial."""
    f, s, gen = load_golden(name)
    rec, _, _ = _run(f, s, gen, np.float32)
    _check_filtered(rec, f, s, gen)


def test_untied_fixture_uses_out_proj():
    """The untied fixture's logits come from depth_head.out_proj: the tied
    head on the same weights misses them by far (model.py:171-174)."""
    from dataclasses import replace

    f, s, gen = load_golden("tiny_untied")
    assert not s.tie_audio_head
    m = _model(f, replace(s, tie_audio_head=True), np.float64)
    g = {k: v for k, v in gen.items() if k != "seed"}
    rec = Record()
    generate(m, input_ids=f["text_ids"], prompt_codes=f["prompt_codes"], uncond_input_ids=f["uncond_ids"],
             forced_codes=_forced(f, s), record=rec, **g)
    ref = f["sample_logits"]
    got = _masked_calls(rec, s, gen, ref.shape[0])
    fin = np.isfinite(ref)
    assert np.abs(got[fin] - ref[fin]).max() / np.abs(ref[fin]).max() > 1e-2


def test_batched_rows_equal_native_rows_to_rounding():
    f, s, gen = load_golden("tiny_sampled")
    rec_a, _, _ = _run(f, s, gen, np.float64, batched=False)
    rec_b, _, _ = _run(f, s, gen, np.float64, batched=True)
    a = np.stack([np.stack(x) for x in rec_a.merged])
    b = np.stack([np.stack(x) for x in rec_b.merged])
    assert np.abs(a - b).max() < 1e-12


def test_q06b_fixture_prefix_and_first_frames():
    """Qwen3-0.6B shape (28 layers, d=1024, V=2051): the reference's first
    frames, teacher-forced, in float32."""
    f, s, gen = load_golden("q06b_greedy")
    rec, codes, _ = _run(f, s, gen, np.float32, batched=True)
    ref = f["sample_logits"]
    got = _masked_calls(rec, s, gen, ref.shape[0])
    fin = np.isfinite(ref)
    rel = np.abs(got[fin] - ref[fin]).max() / np.abs(ref[fin]).max()
    assert rel < 1e-4, rel
    np.testing.assert_array_equal(codes, f["codes"])


def test_q06b_sampled_fixture_full_prefix():
    """Qwen3-0.6B shape with the full-utterance prefix (96 text ids + BOS frame
    + 144 prompt frames; uncond = text BOS + BOS frame + prompt), CFG 1.5,
    T 0.9, top-k 50, top-p 0.95: teacher-forced logits, depth-input hidden
    states and the V = 2051 distributions handed to torch.multinomial."""
    f, s, gen = load_golden("q06b_sampled")
    assert f["text_ids"].size == 96 and f["prompt_codes"].shape == (144, 16) and s.audio_vocab == 2051
    rec, codes, _ = _run(f, s, gen, np.float32, batched=True)
    ref = f["sample_logits"]
    got = _masked_calls(rec, s, gen, ref.shape[0])
    fin = np.isfinite(ref)
    assert (np.isfinite(got) == fin).all()
    rel = np.abs(got[fin] - ref[fin]).max() / np.abs(ref[fin]).max()
    assert rel < 1e-4, rel
    h = np.stack(rec.hidden)[: f["hidden"].shape[0]]
    assert np.abs(h - f["hidden"][: h.shape[0]]).max() / np.abs(f["hidden"]).max() < 1e-4
    np.testing.assert_array_equal(codes, f["codes"])
    _check_filtered(rec, f, s, gen)


def test_planted_mistakes_are_caught():
    """A dropped residual in the depth head or a swapped CFG order in the
    oracle must break agreement with the reference vectors."""
    import oracle.model as om
    import oracle.sampler as osm

    f, s, gen = load_golden("tiny_greedy")
    ref = f["sample_logits"]
    fin = np.isfinite(ref)

    def err():
        rec, _, _ = _run(f, s, gen, np.float64)
        got = _masked_calls(rec, s, gen, ref.shape[0])
        return np.abs(got[fin] - ref[fin]).max() / np.abs(ref[fin]).max()

    assert err() < 2e-6
    orig = om.OracleModel.depth_logits

    def no_residual(self, hidden, prefix, q):
        w = self.w
        a = om.rms_norm(hidden + prefix, w["depth_head.norm_in.weight"], om.FLT_EPS)
        y = (om.silu(a @ w["depth_head.mlp.gate_proj.weight"].T) * (a @ w["depth_head.mlp.up_proj.weight"].T)) \
            @ w["depth_head.mlp.down_proj.weight"].T
        body = om.rms_norm(y, w["depth_head.norm_out.weight"], om.FLT_EPS)
        return body @ w["audio_codebooks.table"][q].T + w["depth_head.bias"][q]

    om.OracleModel.depth_logits = no_residual
    try:
        assert err() > 1e-3
    finally:
        om.OracleModel.depth_logits = orig
    orig_merge = osm.cfg_merge
    import oracle.generate as og
    og.cfg_merge = lambda c, u, sc: orig_merge(u, c, sc)
    try:
        assert err() > 1e-3
    finally:
        og.cfg_merge = orig_merge


def test_scan_sums_is_an_inclusive_prefix_sum():
    """The fixed-order float64 scan of the draw: equal to the running sum
    exactly for small integers (exact in float64 at any order), within a few
    ulps of np.cumsum for random weights, at group sizes around 16/64."""
    from oracle.sampler import scan_sums

    rng = np.random.default_rng(7)
    for n in (1, 2, 15, 16, 17, 31, 33, 63, 64, 65, 127, 128, 129, 200, 300):
        ints = rng.integers(0, 1000, n).astype(np.float64)
        np.testing.assert_array_equal(scan_sums(ints), np.cumsum(ints))
        w = np.exp(-rng.exponential(3.0, n))
        got, ref = scan_sums(w), np.cumsum(w)
        assert np.all(np.abs(got - ref) <= 8 * np.finfo(np.float64).eps * ref), n
        assert np.all(np.diff(got) >= 0)


def test_scan_sums_order_is_the_row_scheme():
    """The addition order shows in the last bits.  Lanes 0-15 = 1, lane 16 =
    2^53, lanes 17-31 = 1, lane 32 = 2^53 (spacing 2 above 2^53, 4 above
    2^54, ties to even).  Row-of-16 scheme by hand: row 0 gives 16 at lane 15;
    row 1 locally reaches 2^53 + 14 at lane 31 (the first 1 is absorbed,
    pairs survive), + 16 from row 0 = 2^53 + 30; lane 32 = 2^53 + (2^53 + 30)
    = 2^54 + 30 -> 2^54 + 32.  A left-to-right sum gives 2^54 + 16 there and
    a 64-wide Hillis-Steele scan 2^54 + 28."""
    from oracle.sampler import scan_sums

    w = np.zeros(64)
    w[0:16] = 1.0
    w[16] = 2.0 ** 53
    w[17:32] = 1.0
    w[32] = 2.0 ** 53
    got = scan_sums(w)
    assert got[15] == 16.0
    assert got[31] == 2.0 ** 53 + 30.0
    assert got[32] == 2.0 ** 54 + 32.0
    assert np.cumsum(w)[32] == 2.0 ** 54 + 16.0


def test_bf16_kv_option_rounds_only_the_cache():
    """kv_bf16 changes nothing but the stored K/V: with weights whose K and V
    projections are exactly representable after the norm (zero K/V weights)
    the two modes agree bitwise; with random weights every cached value is a
    BF16 value and the hidden state moves only by the rounding (< 1e-2
    relative on the tiny shape)."""
    from oracle.model import TINY, RowState, round_bf16

    w = synthetic_weights(TINY, 3)
    emb = np.random.default_rng(4).normal(0, 1, (6, TINY.d_model)).astype(np.float32)
    outs = []
    for kv_bf16 in (False, True):
        m = OracleModel(TINY, w, np.float32, kv_bf16=kv_bf16)
        st = RowState(TINY, 16, np.float32)
        outs.append((m.prefill(st, emb), st))
    (h32, s32), (h16, s16) = outs
    k = s16.k[:, :, :6]
    assert np.array_equal(k, round_bf16(k)) and not np.array_equal(s32.k[:, :, :6], round_bf16(s32.k[:, :, :6]))
    # layer 0 sees identical inputs in both modes: its cache is the rounded FP32 cache
    assert np.array_equal(round_bf16(s32.k[0, :, :6]), s16.k[0, :, :6])
    assert np.array_equal(round_bf16(s32.v[0, :, :6]), s16.v[0, :, :6])
    rel = np.abs(h16 - h32).max() / np.abs(h32).max()
    assert 0 < rel < 1e-2
    wz = dict(w)
    for i in range(TINY.n_layers):
        for n in ("k_proj", "v_proj"):
            wz[f"trunk.layers.{i}.self_attn.{n}.weight"] = np.zeros_like(w[f"trunk.layers.{i}.self_attn.{n}.weight"])
    hz = []
    for kv_bf16 in (False, True):
        m = OracleModel(TINY, wz, np.float32, kv_bf16=kv_bf16)
        st = RowState(TINY, 16, np.float32)
        hz.append(m.prefill(st, emb))
    assert np.array_equal(hz[0], hz[1])

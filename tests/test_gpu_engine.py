"""Whole-frame engine parity on the GPU against the reference's golden
vectors and the oracle.

Tolerance: logits within 1e-3 relative (normalised by
the row's max |logit|) of the FP32 reference path; tokens bit-exact when both
sides get the same logits and the same uniform draw."""

import numpy as np
import pytest

from conftest import load_golden
from oracle.generate import Record, generate
from oracle.model import OracleModel, synthetic_weights
from oracle.sampler import apply_masks

pytestmark = pytest.mark.gpu

LOGIT_TOL = 1e-3


def _shape(s):
    from soraku_amd.config import DecodeShape

    return DecodeShape(**{k: getattr(s, k) for k in DecodeShape.__dataclass_fields__})


def _weights(f, s):
    return synthetic_weights(s, int(f["seed"]), norm_gain_std=float(f["norm_gain_std"]),
                             bias_std=float(f["bias_std"]))


def _engine(f, s, gen, w, hip_device, max_ctx=None):
    from soraku_amd import GraphFrameEngine

    cfg = gen.get("cfg_scale", 1.0)
    batch = 2 if cfg != 1.0 else 1
    n = f["text_ids"].size + 1 + f["prompt_codes"].shape[0] + gen["max_new_frames"] + 2
    e = GraphFrameEngine(device=hip_device, max_cache_len=max_ctx or n, cfg_scale=cfg, batch=batch,
                         state_dict=w, shape=_shape(s),
                         language_token_ids=tuple(int(v) for v in f["language_ids"]))
    sampled = gen["temperature"] > 0 or (gen.get("temperature_q0") or 0) > 0
    e.set_temperature(gen["temperature"], q0=gen.get("temperature_q0"))
    e.set_sampling(sampled=sampled, top_k=gen.get("top_k"), top_p=gen.get("top_p"),
                   top_k_q0=gen.get("top_k_q0"), top_p_q0=gen.get("top_p_q0"))
    e.set_debug(True)
    e.prefill(f["text_ids"], f["uncond_ids"] if batch == 2 else None, f["prompt_codes"])
    e.capture()
    return e


def _rowwise_rel(got, ref):
    fin = np.isfinite(ref)
    assert (np.isfinite(got) == fin).all()
    num = np.abs(np.where(fin, got, 0) - np.where(fin, ref, 0)).max(axis=-1)
    den = np.abs(np.where(fin, ref, 0)).max(axis=-1)
    return float((num / den).max())


def _teacher_forced(e, f, s, gen):
    codes = f["codes"]
    n_calls = f["sample_logits"].shape[0]
    out = []
    for fi in range(gen["max_new_frames"]):
        if len(out) >= n_calls:
            break
        forced = codes[fi] if fi < codes.shape[0] else np.full(s.n_codebooks, s.eos_id)
        _, lg = e.step_frame(mask_eos_q0=fi < gen["min_new_frames"], uniforms=np.zeros(s.n_codebooks),
                             forced_codes=forced, return_logits=True)
        out.extend(lg[0])
    return np.stack(out[:n_calls])


@pytest.mark.parametrize("name", ["tiny_greedy", "tiny_sampled", "tiny_nocfg_topp", "tiny_untied", "q06b_greedy"])
def test_teacher_forced_logits_match_reference(hip_device, name):
    f, s, gen = load_golden(name)
    e = _engine(f, s, gen, _weights(f, s), hip_device)
    hid = e.hidden()
    ref_h = f["hidden"][0]
    assert np.abs(hid - ref_h).max() / np.abs(ref_h).max() < 1e-4
    got = _teacher_forced(e, f, s, gen)
    rel = _rowwise_rel(got, f["sample_logits"])
    print(f"{name}: max row-relative logit error {rel:.3e}")
    assert rel < LOGIT_TOL
    e.close()


@pytest.mark.parametrize("name", ["tiny_greedy", "q06b_greedy"])
def test_greedy_codes_match_reference(hip_device, name):
    import torch
    from soraku_amd import FastGenerator

    f, s, gen = load_golden(name)
    g = FastGenerator(device=hip_device, state_dict=_weights(f, s), shape=_shape(s),
                      language_token_ids=tuple(int(v) for v in f["language_ids"]))
    kw = {k: v for k, v in gen.items() if k != "seed"}
    codes, info = g.generate(input_ids=torch.tensor(f["text_ids"][None]),
                             prompt_codes=torch.tensor(f["prompt_codes"]),
                             uncond_input_ids=torch.tensor(f["uncond_ids"][None]), **kw)
    np.testing.assert_array_equal(codes.numpy(), f["codes"])
    assert info["stop_reason"] == ("eos" if int(f["stop_eos"]) else "max_frames")


def test_sampled_codes_match_oracle_under_identical_uniforms(hip_device):
    """Free-running sampled decode (top-k, top-p, q0 overrides, CFG) with the
    same uniforms on both sides; the oracle runs in float64."""
    f, s, gen = load_golden("tiny_sampled")
    w = _weights(f, s)
    n_frames = 12
    gen = dict(gen, max_new_frames=n_frames)
    u = np.random.default_rng(11).random((n_frames, s.n_codebooks))
    m = OracleModel(s, w, np.float64, language_token_ids=tuple(int(v) for v in f["language_ids"]))
    kw = {k: v for k, v in gen.items() if k != "seed"}
    ref, _ = generate(m, input_ids=f["text_ids"], prompt_codes=f["prompt_codes"],
                      uncond_input_ids=f["uncond_ids"], uniforms=u, batched=True, **kw)
    e = _engine(f, s, gen, w, hip_device)
    got = []
    for fi in range(ref.shape[0]):
        got.append(e.step_frame(mask_eos_q0=fi < gen["min_new_frames"], uniforms=u[fi]).numpy())
    np.testing.assert_array_equal(np.stack(got), ref)
    e.close()


def test_replays_are_deterministic(hip_device):
    f, s, gen = load_golden("tiny_sampled")
    w = _weights(f, s)
    u = np.random.default_rng(3).random((6, s.n_codebooks))
    runs = []
    for _ in range(2):
        e = _engine(f, s, dict(gen, max_new_frames=6), w, hip_device)
        frames = [e.step_frame(mask_eos_q0=False, uniforms=u[i], return_logits=True) for i in range(6)]
        runs.append((np.stack([c.numpy() for c, _ in frames]), np.stack([lg for _, lg in frames])))
        e.close()
    np.testing.assert_array_equal(runs[0][0], runs[1][0])
    np.testing.assert_array_equal(runs[0][1], runs[1][1])


def test_queued_replay_equals_stepwise(hip_device):
    """sk_queue_frames + sk_replay (no host sync per frame) = sk_step_frame."""
    f, s, gen = load_golden("tiny_sampled")
    w = _weights(f, s)
    n = 8
    u = np.random.default_rng(5).random((n, s.n_codebooks))
    mask = (np.arange(n) < gen["min_new_frames"]).astype(np.int32)
    e = _engine(f, s, dict(gen, max_new_frames=n), w, hip_device)
    step = np.stack([e.step_frame(mask_eos_q0=bool(mask[i]), uniforms=u[i]).numpy() for i in range(n)])
    e.close()
    e = _engine(f, s, dict(gen, max_new_frames=n), w, hip_device)
    e.queue_frames(u, mask)
    e.replay(n)
    got = e.read_codes(n)[:, 0]
    np.testing.assert_array_equal(got, step)
    e.close()


def test_queued_replay_across_chunk_boundary(hip_device):
    """Queued replays (no host sync between frames) whose rows cross a 32-token
    attention chunk boundary mid-queue (cond 28 -> 40 positions): the host
    widens the attention grid between launches; codes equal step-by-step
    decoding and the float64 oracle's."""
    from oracle.model import TINY
    from soraku_amd import GraphFrameEngine

    s = TINY
    w = synthetic_weights(s, 61, norm_gain_std=0.1, bias_std=0.02)
    rng = np.random.default_rng(61)
    text, uncond = rng.integers(0, s.text_vocab, 26), np.array([4])
    prompt = rng.integers(0, s.codebook_size, (1, s.n_codebooks))
    n = 12
    u = rng.random((n, s.n_codebooks))
    kw = dict(temperature=0.9, top_k=8, top_p=0.9, cfg_scale=1.5, min_new_frames=n)
    ref, _ = generate(OracleModel(s, w, np.float64), input_ids=text, prompt_codes=prompt,
                      uncond_input_ids=uncond, uniforms=u, max_new_frames=n, batched=True, **kw)

    def engine():
        e = GraphFrameEngine(device=hip_device, max_cache_len=96, cfg_scale=1.5, batch=2, state_dict=w,
                             shape=_shape(s))
        e.set_temperature(0.9)
        e.set_sampling(sampled=True, top_k=8, top_p=0.9)
        e.prefill(text, uncond, prompt)
        e.capture()
        return e

    e = engine()
    step = np.stack([e.step_frame(mask_eos_q0=True, uniforms=u[i]).numpy() for i in range(n)])
    e.close()
    e = engine()
    e.queue_frames(u, np.ones(n, np.int32))
    e.replay(n)
    got = e.read_codes(n)[:, 0]
    e.close()
    np.testing.assert_array_equal(step, ref)
    np.testing.assert_array_equal(got, ref)


def test_frame_ring_reset(hip_device):
    """sk_reset_frames: an engine whose frame ring holds 3 frames decodes 7
    (restarting the ring whenever it is full) with the same codes and logits
    as an engine whose ring holds them all; a full ring refuses the next frame."""
    from soraku_amd import GraphFrameEngine, SkError
    from soraku_amd._lib import SK_EKVFULL

    f, s, gen = load_golden("tiny_sampled")
    w = _weights(f, s)
    n = 7
    u = np.random.default_rng(9).random((n, s.n_codebooks))
    runs = []
    for ring in (n, 3):
        e = GraphFrameEngine(device=hip_device, max_cache_len=64, cfg_scale=1.5, batch=2, state_dict=w,
                             shape=_shape(s), language_token_ids=tuple(int(v) for v in f["language_ids"]),
                             max_frames=ring)
        e.set_temperature(gen["temperature"])
        e.set_sampling(sampled=True, top_k=gen.get("top_k"), top_p=gen.get("top_p"))
        e.set_debug(True)
        e.prefill(f["text_ids"], f["uncond_ids"], f["prompt_codes"])
        e.capture()
        got = []
        for i in range(n):
            if e.frames_done == ring:
                with pytest.raises(SkError) as ei:
                    e.step_frame(mask_eos_q0=i < 2, uniforms=u[i])
                assert ei.value.code == SK_EKVFULL
                e.reset_frames()
            c, lg = e.step_frame(mask_eos_q0=i < 2, uniforms=u[i], return_logits=True)
            got.append((c.numpy(), lg))
        e.close()
        runs.append(got)
    for (c0, l0), (c1, l1) in zip(*runs):
        np.testing.assert_array_equal(c0, c1)
        np.testing.assert_array_equal(l0, l1)


def test_engine_error_paths(hip_device):
    from soraku_amd import GraphFrameEngine, SkError
    from soraku_amd._lib import SK_EKVFULL, SK_ENOCAPTURE

    f, s, gen = load_golden("tiny_greedy")
    w = _weights(f, s)
    n_prefix = f["text_ids"].size + 1 + f["prompt_codes"].shape[0]
    e = GraphFrameEngine(device=hip_device, max_cache_len=n_prefix + 2, cfg_scale=1.5, batch=2,
                         state_dict=w, shape=_shape(s),
                         language_token_ids=tuple(int(v) for v in f["language_ids"]))
    e.prefill(f["text_ids"], f["uncond_ids"], f["prompt_codes"])
    with pytest.raises(RuntimeError):
        e.step_frame(mask_eos_q0=True)
    e.graph = True  # bypass the Python guard: the C ABI must refuse too
    with pytest.raises(SkError) as ei:
        e.step_frame(mask_eos_q0=True)
    assert ei.value.code == SK_ENOCAPTURE
    e.capture()
    e.step_frame(mask_eos_q0=True)
    e.step_frame(mask_eos_q0=True)
    with pytest.raises(SkError) as ei:
        e.step_frame(mask_eos_q0=True)
    assert ei.value.code == SK_EKVFULL
    with pytest.raises(ValueError):
        e.prefill(np.arange(n_prefix + 5) % s.text_vocab, f["uncond_ids"], f["prompt_codes"])
    e.close()


def _oracle_forced_logits(m, s, text, prompt, uncond, codes, cfg, states=None):
    """Masked merged logits [frames*Q, V] of the oracle under teacher forcing
    (from prefilled ``states`` when given)."""
    rec = Record()
    n = codes.shape[0]
    generate(m, input_ids=text, prompt_codes=prompt, uncond_input_ids=uncond, max_new_frames=n,
             min_new_frames=0, temperature=0.0, cfg_scale=cfg, forced_codes=codes, batched=True,
             record=rec, states=states)
    out = [apply_masks(mg, q=q, frame_index=fi, min_new_frames=0, bos_id=s.bos_id, eos_id=s.eos_id,
                       pad_id=s.pad_id)
           for fi, fr in enumerate(rec.merged) for q, mg in enumerate(fr)]
    return np.stack(out)


def _engine_forced_logits(e, s, codes):
    out = []
    for fi in range(codes.shape[0]):
        _, lg = e.step_frame(mask_eos_q0=False, uniforms=np.zeros(s.n_codebooks), forced_codes=codes[fi],
                             return_logits=True)
        out.extend(lg[0])
    return np.stack(out)


def _bf16_weights(w):
    from oracle.model import round_bf16
    from soraku_amd.synthetic import is_matrix

    return {k: (round_bf16(v) if is_matrix(k) else v) for k, v in w.items()}


@pytest.mark.parametrize("bf16_w,bf16_kv", [(False, True), (True, False), (True, True)])
def test_bf16_weights_and_kv_cache_match_oracle(hip_device, bf16_w, bf16_kv):
    """Tiny shape with BF16 matrices (FP32 accumulation) and / or a BF16 KV
    cache, teacher-forced against the oracle holding the same BF16-rounded
    weights and rounding K/V at append."""
    from oracle.model import TINY
    from soraku_amd import GraphFrameEngine

    s = TINY
    w = synthetic_weights(s, 21, norm_gain_std=0.1, bias_std=0.02)
    if bf16_w:
        w = _bf16_weights(w)
    rng = np.random.default_rng(5)
    text, uncond = rng.integers(0, s.text_vocab, 9), np.array([3])
    prompt = rng.integers(0, s.codebook_size, (5, s.n_codebooks))
    codes = rng.integers(0, s.codebook_size, (6, s.n_codebooks))
    cfg = 1.5
    ref = _oracle_forced_logits(OracleModel(s, w, np.float64, kv_bf16=bf16_kv), s, text, prompt, uncond,
                                codes, cfg)
    e = GraphFrameEngine(device=hip_device, max_cache_len=40, cfg_scale=cfg, batch=2, state_dict=w,
                         shape=_shape(s), bf16=bf16_w, kv_bf16=bf16_kv)
    e.set_temperature(0.0)
    e.set_debug(True)
    e.prefill(text, uncond, prompt)
    e.capture()
    got = _engine_forced_logits(e, s, codes)
    e.close()
    rel = _rowwise_rel(got, ref)
    print(f"bf16 weights {bf16_w} kv {bf16_kv}: max row-relative logit error {rel:.3e}")
    assert rel < LOGIT_TOL


def _device_weights(s, seed, hip_device):
    """Seeded N(0, 0.02) matrices drawn on the GPU and rounded to BF16 there
    (round to nearest even, as round_bf16), unit norm gains, zero bias;
    returned as FP32 NumPy arrays shared by oracle and engine."""
    import torch
    from soraku_amd.synthetic import is_matrix, weight_shapes

    g = torch.Generator(device=hip_device)
    g.manual_seed(seed)
    out = {}
    for key, shp in weight_shapes(s).items():
        if is_matrix(key):
            t = torch.randn(shp, generator=g, device=hip_device, dtype=torch.float32) * 0.02
            t = t.to(torch.bfloat16).to(torch.float32)
        elif key == "depth_head.bias":
            t = torch.zeros(shp, device=hip_device)
        else:
            t = 1.0 + 0.1 * torch.randn(shp, generator=g, device=hip_device, dtype=torch.float32)
        out[key] = t.cpu().numpy()
    return out


def _engine_kv_bits(e, layer, kv):
    """Layer ``layer``'s BF16 K (kv=0) or V (kv=1) cache as uint16 bits
    ``[rows, n_kv_heads, max_ctx, head_dim]``, copied through the HIP runtime
    the library is linked against (the address comes from sk_kv_ptr)."""
    import ctypes as C

    from soraku_amd._lib import check, lib

    p = C.c_void_p()
    check(lib().sk_kv_ptr(e._h, layer, kv, C.byref(p)))
    e.synchronize()
    hip = C.CDLL("libamdhip64.so.7")
    hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    s = e.shape
    out = np.empty((e.rows, s.n_kv_heads, e.max_len, s.head_dim), np.uint16)
    assert hip.hipMemcpy(out.ctypes.data, p, out.nbytes, 2) == 0  # hipMemcpyDeviceToHost
    return out


def test_qwen3_17b_shape_bf16_weights_and_kv(hip_device):
    """Larger backbone configuration: Qwen3-1.7B shape (d 2048, inter 6144,
    depth inner 4096, 28 layers, 16 Q / 8 KV heads), BF16 weights with FP32
    accumulation and a BF16 KV cache, CFG batch 2, 3 teacher-forced frames
    after a short prefix.  The text vocabulary is cut to 4096 rows: only
    prefix ids are ever embedded.

    Rounding K/V to BF16 is discontinuous, so FP32-level differences that
    land a value on the other side of a rounding boundary move it by one BF16
    ulp (2^-8 relative), and 28 layers carry that to the logits: the oracle's
    own FP32 run differs from its FP64 run by ~1.8e-3 on this case, against
    ~5e-6 with an FP32 cache.  So the checks are (1) layer 0, whose inputs
    are the same embeddings in both, holds the FP64 oracle's BF16 cache
    except at rare near-ties (< 0.5% of elements), and every cached value is
    the unrounded FP64 value to within half an ulp plus FP32 noise, and
    (2) the logits sit within max(1e-3, 2 x that FP32-vs-FP64 spread) of the
    FP64 oracle: no further from it than an FP32 restatement is.  The FP32-KV
    case of the same weights is held to 1e-3 (it measures ~2e-6)."""
    import dataclasses

    from oracle.generate import start_states
    from oracle.model import QWEN3_17B
    from soraku_amd import GraphFrameEngine

    s = dataclasses.replace(QWEN3_17B, text_vocab=4096)
    w = _device_weights(s, 8, hip_device)
    rng = np.random.default_rng(6)
    text, uncond = rng.integers(0, s.text_vocab, 12), np.array([7])
    prompt = rng.integers(0, s.codebook_size, (3, s.n_codebooks))
    codes = rng.integers(0, s.codebook_size, (3, s.n_codebooks))
    cfg, max_len = 1.5, 32

    def oracle(dtype, kv_bf16):
        m = OracleModel(s, w, dtype, kv_bf16=kv_bf16)
        st = start_states(m, text, prompt, uncond, cfg, max_len)
        return _oracle_forced_logits(m, s, text, prompt, uncond, codes, cfg, states=st), st

    def engine(kv_bf16):
        e = GraphFrameEngine(device=hip_device, max_cache_len=max_len, cfg_scale=cfg, batch=2,
                             state_dict=w, shape=_shape(s), bf16=True, kv_bf16=kv_bf16)
        e.set_temperature(0.0)
        e.set_debug(True)
        e.prefill(text, uncond, prompt)
        e.capture()
        got = _engine_forced_logits(e, s, codes)
        kv = [_engine_kv_bits(e, 0, j) for j in (0, 1)] if kv_bf16 else None
        e.close()
        return got, kv

    ref64, st_exact = oracle(np.float64, False)
    got, _ = engine(False)
    rel = _rowwise_rel(got, ref64)
    print(f"Qwen3-1.7B BF16 weights, FP32 KV: max row-relative logit error {rel:.3e}")
    assert rel < LOGIT_TOL

    ref64, st64 = oracle(np.float64, True)
    ref32, _ = oracle(np.float32, True)
    got, kv = engine(True)
    spread = _rowwise_rel(ref32, ref64)
    rel = _rowwise_rel(got, ref64)
    tol = max(LOGIT_TOL, 2 * spread)
    for j, name in enumerate(("k", "v")):
        mism, total = 0, 0
        for r, (st, sx) in enumerate(zip(st64, st_exact)):
            n = st.kv_len - 1  # the oracle appends the last frame's token before the engine does
            ref_bits = (getattr(st, name)[0, :, :n].astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
            mine = kv[j][r, :, :n]
            mism += int((mine != ref_bits).sum())
            total += mine.size
            # every value is the unrounded FP64 one to within half a BF16 ulp
            # plus FP32-level noise (1e-5 of the head vector's largest entry)
            exact = getattr(sx, name)[0, :, :n]
            val = (mine.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
            ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(exact), 1e-30))) - 7)
            amax = np.abs(exact).max(axis=-1, keepdims=True)
            assert (np.abs(val - exact) <= 0.5 * ulp + 1e-5 * amax).all(), (name, r)
        print(f"layer 0 {name}: {mism} of {total} BF16 values differ from the FP64 oracle's rounding")
        assert mism <= total // 200
    print(f"Qwen3-1.7B BF16 weights + BF16 KV: engine {rel:.3e}, oracle FP32 vs FP64 {spread:.3e}")
    assert rel < tol


def _engine_kv(e, layer, kv, bf16):
    """Layer ``layer``'s K (kv=0) or V (kv=1) cache as float32
    ``[rows, n_kv_heads, max_ctx, head_dim]`` (BF16 widened)."""
    import ctypes as C

    from soraku_amd._lib import check, lib

    p = C.c_void_p()
    check(lib().sk_kv_ptr(e._h, layer, kv, C.byref(p)))
    e.synchronize()
    hip = C.CDLL("libamdhip64.so.7")
    hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    s = e.shape
    out = np.empty((e.rows, s.n_kv_heads, e.max_len, s.head_dim), np.uint16 if bf16 else np.float32)
    assert hip.hipMemcpy(out.ctypes.data, p, out.nbytes, 2) == 0  # hipMemcpyDeviceToHost
    return (out.astype(np.uint32) << 16).view(np.float32) if bf16 else out


@pytest.mark.parametrize("kv_bf16", [False, True])
def test_batched_prefill_matches_oracle(hip_device, kv_bf16):
    """The batched prefill (MFMA GEMMs over all prefix tokens, causal
    attention per row) against the oracle's prefill at the Qwen3-0.6B shape
    with very unequal rows (300 and 11 positions): each row's final-normed
    hidden state, and the K/V cache of both rows in the first, middle and last
    layer (relative to the largest entry; FP32 GEMMs differ from the oracle's
    only in summation order).  With a BF16 cache, values that sit near a BF16
    rounding boundary can round the other way (one ulp, 2^-8), and later
    layers carry that on, hence the looser bounds there."""
    from oracle.generate import start_states
    from oracle.model import QWEN3_06B
    from soraku_amd import GraphFrameEngine

    s = QWEN3_06B
    w = synthetic_weights(s, 4, norm_gain_std=0.1, bias_std=0.02)
    rng = np.random.default_rng(12)
    text, uncond = rng.integers(0, s.text_vocab, 290), np.array([9])
    prompt = rng.integers(0, s.codebook_size, (9, s.n_codebooks))
    m = OracleModel(s, w, np.float32, kv_bf16=kv_bf16)
    st = start_states(m, text, prompt, uncond, 1.5, 320)
    e = GraphFrameEngine(device=hip_device, max_cache_len=320, cfg_scale=1.5, batch=2, state_dict=w,
                         shape=_shape(s), kv_bf16=kv_bf16)
    e.prefill(text, uncond, prompt)
    hid = e.hidden()
    ref = np.stack([x.hidden for x in st])
    rel = float((np.abs(hid - ref).max(axis=1) / np.abs(ref).max(axis=1)).max())
    worst = 0.0
    for layer in (0, s.n_layers // 2, s.n_layers - 1):
        for kv, name in ((0, "k"), (1, "v")):
            got = _engine_kv(e, layer, kv, kv_bf16)
            for r, x in enumerate(st):
                n = x.kv_len
                want = getattr(x, name)[layer, :, :n]
                err = np.abs(got[r, :, :n] - want).max() / np.abs(want).max()
                worst = max(worst, float(err))
    e.close()
    print(f"prefill 300/11 rows, kv_bf16 {kv_bf16}: hidden rel {rel:.2e}, cache rel {worst:.2e}")
    assert [x.kv_len for x in st] == [300, 11]
    assert rel < (5e-3 if kv_bf16 else 1e-3)
    assert worst < (1e-2 if kv_bf16 else 1e-3)


def _many_utterance_case(s, w, n_utts, seed, hip_device, bf16=False, frames=2, max_len=64, text_len=(5, 30),
                         kv_bf16=False, prefix=None):
    """n_utts utterances with ragged prefixes, teacher-forced for `frames`
    frames through one engine; per utterance, the engine's masked merged
    logits and the oracle's for the same prefix and codes.  With kv_bf16 the
    engine and the oracle keep BF16 caches, and the result is the pair
    (engine vs FP64 oracle, FP32 oracle vs FP64 oracle).

    ``prefix=(lo, hi)`` (or one such pair per utterance): the throughput
    batch's prefixes instead of short ones -- each utterance's cond prefix
    has P positions, P uniform in [lo, hi]: round(0.6 P) prompt frames after
    the BOS frame, the rest text ids; its uncond row is one text id + the BOS
    frame + the same prompt frames (runtime.py:143, model.py:632-653)."""
    from soraku_amd import GraphFrameEngine

    rng = np.random.default_rng(seed)
    items, codes = [], []
    for ui in range(n_utts):
        if prefix is None:
            nt, npr = int(rng.integers(*text_len)), int(rng.integers(0, 4))
        else:
            lo, hi = prefix[ui] if isinstance(prefix, list) else prefix
            plen = int(rng.integers(lo, hi + 1))
            npr = int(0.6 * plen + 0.5)
            nt = plen - 1 - npr
        items.append((rng.integers(0, s.text_vocab, nt), np.array([int(rng.integers(0, s.text_vocab))]),
                      rng.integers(0, s.codebook_size, (npr, s.n_codebooks))))
        codes.append(rng.integers(0, s.codebook_size, (frames, s.n_codebooks)))
    lens = [(t.size + 1 + p.shape[0], 2 + p.shape[0]) for t, _, p in items]
    print(f"{n_utts} utterances, cond/uncond positions {lens}", flush=True)
    codes = np.stack(codes)                       # [utts, frames, Q]
    cfg = 1.5
    e = GraphFrameEngine(device=hip_device, max_cache_len=max_len, cfg_scale=cfg, batch=2, state_dict=w,
                         shape=_shape(s), n_utts=n_utts, bf16=bf16, kv_bf16=kv_bf16)
    e.set_temperature(0.0)
    e.set_debug(True)
    e.prefill_utterances(items)
    e.capture()
    got = []
    for fi in range(frames):
        _, lg = e.step_frame(mask_eos_q0=False, uniforms=np.zeros(n_utts * s.n_codebooks),
                             forced_codes=codes[:, fi], return_logits=True)
        got.append(lg)
    e.close()
    got = np.stack(got, axis=1)                   # [utts, frames, Q, V]
    worst = spread = 0.0
    m = OracleModel(s, w, np.float64, kv_bf16=kv_bf16)
    m32 = OracleModel(s, w, np.float32, kv_bf16=True) if kv_bf16 else None
    for u, (text, uncond, prompt) in enumerate(items):
        print(f"oracle, utterance {u}", flush=True)
        ref = _oracle_forced_logits(m, s, text, prompt, uncond, codes[u], cfg)
        worst = max(worst, _rowwise_rel(got[u].reshape(-1, got.shape[-1]), ref))
        if kv_bf16:
            ref32 = _oracle_forced_logits(m32, s, text, prompt, uncond, codes[u], cfg)
            spread = max(spread, _rowwise_rel(ref32, ref))
    return (worst, spread) if kv_bf16 else worst


def test_many_utterances_tiny(hip_device):
    """Eight decode rows (4 utterances x CFG) take the skinny-GEMM path; each
    utterance, with its own ragged prefix, matches the oracle run alone."""
    from oracle.model import TINY

    w = synthetic_weights(TINY, 31, norm_gain_std=0.1, bias_std=0.02)
    rel = _many_utterance_case(TINY, w, 4, 3, hip_device, frames=3)
    print(f"tiny, 4 utterances: max row-relative logit error {rel:.3e}")
    assert rel < LOGIT_TOL


def test_many_utterances_tiny_bf16_ten_rows(hip_device):
    """Ten decode rows (5 utterances x CFG) with BF16 weights: GEMM inputs
    pass between kernels in split form (BF16 hi/lo pairs with the next norm's
    gain, written by each producer; rows 10..31 of those buffers are never
    written), non-unit norm gains; each utterance matches the oracle on the
    same BF16-rounded weights."""
    from oracle.model import TINY

    w = _device_weights(TINY, 41, hip_device)
    rel = _many_utterance_case(TINY, w, 5, 7, hip_device, bf16=True, frames=3)
    print(f"tiny BF16, 5 utterances: max row-relative logit error {rel:.3e}")
    assert rel < LOGIT_TOL


def test_many_utterances_tiny_bf16_kv(hip_device):
    """Ten decode rows with BF16 weights and a BF16 KV cache at the tiny
    shape (head_dim 16: the streaming attention's slots are single lanes and
    merge over every lane distance); held to max(1e-3, 2 x the oracle's
    FP32-vs-FP64 spread with the same BF16 cache)."""
    from oracle.model import TINY

    w = _device_weights(TINY, 43, hip_device)
    rel, spread = _many_utterance_case(TINY, w, 5, 9, hip_device, bf16=True, frames=3, kv_bf16=True)
    print(f"tiny BF16 weights + BF16 KV, 5 utterances: engine {rel:.3e}, oracle FP32 vs FP64 {spread:.3e}")
    assert rel < max(LOGIT_TOL, 2 * spread)


def test_sixteen_utterances_q06b_bf16(hip_device):
    """Batch-32 decode (16 utterances x CFG) at the Qwen3-0.6B shape with BF16
    weights (FP32 accumulation), ragged prefixes: every utterance against the
    oracle on the same BF16-rounded weights."""
    import dataclasses

    from oracle.model import QWEN3_06B

    s = dataclasses.replace(QWEN3_06B, text_vocab=4096)   # only prefix ids are embedded
    w = _device_weights(s, 17, hip_device)
    rel = _many_utterance_case(s, w, 16, 5, hip_device, bf16=True, frames=2)
    print(f"q06b BF16, 16 utterances: max row-relative logit error {rel:.3e}")
    assert rel < LOGIT_TOL


def test_split_k_wait_timeout_reports_error_and_fresh_engine_decodes(hip_device):
    """The split-K GEMMs' bounded wait (slice 0 reading the other slices'
    tagged partials), forced to give up from the host with
    sk_debug_set_spin_ticks(e, 0): a merge that does not find every partial
    at its first look ends at once and sets the error word, every kernel
    exits, and sk_step_frame returns SK_EHIP with its message (within a few
    frames: a merge that finds its partials ready does not wait).  A fresh
    engine on the same weights then decodes three utterances x CFG (the
    skinny-GEMM path with split-K, Qwen3-0.6B shape, BF16 weights) to the
    oracle's logits."""
    import dataclasses

    from oracle.model import QWEN3_06B
    from soraku_amd import GraphFrameEngine
    from soraku_amd._lib import SK_EHIP, SkError, check, lib

    s = dataclasses.replace(QWEN3_06B, text_vocab=4096)
    w = _device_weights(s, 23, hip_device)
    rng = np.random.default_rng(23)
    items = [(rng.integers(0, s.text_vocab, 12), np.array([7]), rng.integers(0, s.codebook_size, (2, s.n_codebooks)))
             for _ in range(3)]
    e = GraphFrameEngine(device=hip_device, max_cache_len=64, cfg_scale=1.5, batch=2, state_dict=w,
                         shape=_shape(s), n_utts=3, bf16=True)
    e.set_temperature(0.0)
    e.prefill_utterances(items)
    check(lib().sk_debug_set_spin_ticks(e._h, 0))
    e.capture()
    err = None
    for fi in range(5):
        try:
            e.step_frame(mask_eos_q0=False, uniforms=np.zeros(3 * s.n_codebooks))
        except SkError as ex:
            err = ex
            break
    e.close()
    print(f"forced split-K timeout: {err} (frame {fi})", flush=True)
    assert err is not None and err.code == SK_EHIP and "split-K merge wait timed out" in str(err)
    rel = _many_utterance_case(s, w, 3, 24, hip_device, bf16=True, frames=2)
    print(f"fresh engine after the timeout: max row-relative logit error {rel:.3e}")
    assert rel < LOGIT_TOL


def test_split_k_tags_after_frame_counter_restart(hip_device):
    """The split-K merge's tags repeat once the frame counter restarts at 0 (a
    new prefill).  An engine (three utterances x CFG, Qwen3-0.6B shape, BF16
    weights: the skinny GEMMs with split-K) decodes one frame, so the tagged
    words hold frame 0's tags, then prefills other utterances and decodes
    three frames: its codes and logits equal, bit for bit, those of a fresh
    engine that decodes the second set alone."""
    import dataclasses

    from oracle.model import QWEN3_06B
    from soraku_amd import GraphFrameEngine

    s = dataclasses.replace(QWEN3_06B, text_vocab=4096)
    w = _device_weights(s, 29, hip_device)
    rng = np.random.default_rng(29)

    def items():
        return [(rng.integers(0, s.text_vocab, 10 + 3 * i), np.array([7]),
                 rng.integers(0, s.codebook_size, (2 + i, s.n_codebooks))) for i in range(3)]

    first, second = items(), items()
    u = np.zeros(3 * s.n_codebooks)

    def make(its):
        e = GraphFrameEngine(device=hip_device, max_cache_len=64, cfg_scale=1.5, batch=2, state_dict=w,
                             shape=_shape(s), n_utts=3, bf16=True)
        e.set_temperature(0.0)
        e.set_debug(True)
        e.prefill_utterances(its)
        e.capture()
        return e

    def decode(e, n):
        out = [e.step_frame(mask_eos_q0=True, uniforms=u, return_logits=True) for _ in range(n)]
        return np.stack([c.numpy() for c, _ in out]), np.stack([lg for _, lg in out])

    e = make(first)
    decode(e, 1)
    e.prefill_utterances(second)
    got = decode(e, 3)
    e.close()
    e = make(second)
    want = decode(e, 3)
    e.close()
    np.testing.assert_array_equal(got[0], want[0])
    np.testing.assert_array_equal(got[1], want[1])


def test_split_k_frames_after_ring_reset(hip_device):
    """sk_reset_frames on the split-K path: the frame counter restarts at 0 while
    the caches keep growing, so the frames after the reset reuse frame 0's
    tags.  Three utterances x CFG (Qwen3-0.6B shape, BF16 weights): one frame,
    a ring reset, two frames equal, bit for bit, frames 1 and 2 of an
    uninterrupted run."""
    import dataclasses

    from oracle.model import QWEN3_06B
    from soraku_amd import GraphFrameEngine

    s = dataclasses.replace(QWEN3_06B, text_vocab=4096)
    w = _device_weights(s, 31, hip_device)
    rng = np.random.default_rng(31)
    its = [(rng.integers(0, s.text_vocab, 9 + 4 * i), np.array([7]),
            rng.integers(0, s.codebook_size, (1 + i, s.n_codebooks))) for i in range(3)]
    u = np.zeros(3 * s.n_codebooks)

    def run(reset):
        e = GraphFrameEngine(device=hip_device, max_cache_len=64, cfg_scale=1.5, batch=2, state_dict=w,
                             shape=_shape(s), n_utts=3, bf16=True)
        e.set_temperature(0.0)
        e.set_debug(True)
        e.prefill_utterances(its)
        e.capture()
        out = []
        for i in range(3):
            if reset and i == 1:
                e.reset_frames()
            c, lg = e.step_frame(mask_eos_q0=True, uniforms=u, return_logits=True)
            out.append((c.numpy(), lg))
        e.close()
        return out

    plain, reset = run(False), run(True)
    for i in (1, 2):
        np.testing.assert_array_equal(reset[i][0], plain[i][0])
        np.testing.assert_array_equal(reset[i][1], plain[i][1])


def test_sixteen_utterances_q06b_bf16_kv(hip_device):
    """The throughput batch's precision: 16 utterances x CFG at the
    Qwen3-0.6B shape with BF16 weights and a BF16 KV cache (the streaming
    attention reads BF16 K/V).  Rounding K/V to BF16 is discontinuous, so the
    logits are held, as for the 1.7B shape, to max(1e-3, 2 x the oracle's own
    FP32-vs-FP64 spread with the same BF16 cache)."""
    import dataclasses

    from oracle.model import QWEN3_06B

    s = dataclasses.replace(QWEN3_06B, text_vocab=4096)
    w = _device_weights(s, 17, hip_device)
    rel, spread = _many_utterance_case(s, w, 16, 5, hip_device, bf16=True, frames=2, kv_bf16=True)
    print(f"q06b BF16 weights + BF16 KV, 16 utterances: engine {rel:.3e}, oracle FP32 vs FP64 {spread:.3e}")
    assert rel < max(LOGIT_TOL, 2 * spread)


def test_sixteen_utterances_q06b_real_prefixes(hip_device):
    """The throughput batch at its own workload: 16 utterances x CFG at the
    Qwen3-0.6B shape, BF16 weights and BF16 KV cache, ragged cond prefixes of
    120-240 positions from the batched prefill, KV capacity 512, 3
    teacher-forced frames.  The streaming attention runs one split per (row,
    kv head) here, 64 single-token slots of 8 lanes, so every slot holds 2-4
    tokens of these contexts and runs its own online softmax over them
    (model.py:658-676 attends over each branch's own history;
    fast_generate.py:232-328 batches the rows).  Held to max(1e-3, 2 x the
    oracle's own FP32-vs-FP64 spread with the same BF16 cache)."""
    import dataclasses

    from oracle.model import QWEN3_06B

    s = dataclasses.replace(QWEN3_06B, text_vocab=4096)
    w = _device_weights(s, 18, hip_device)
    rel, spread = _many_utterance_case(s, w, 16, 6, hip_device, bf16=True, frames=3, kv_bf16=True,
                                       max_len=512, prefix=(120, 240))
    print(f"q06b BF16 + BF16 KV, 16 utterances, 120-240-position prefixes: engine {rel:.3e}, "
          f"oracle FP32 vs FP64 {spread:.3e}")
    assert rel < max(LOGIT_TOL, 2 * spread)


def test_sixteen_utterances_q06b_near_kv_capacity(hip_device):
    """16 utterances x CFG at the Qwen3-0.6B shape, BF16 weights, FP32 KV
    cache of 512 positions per row: six utterances with cond prefixes of
    440-505 positions (uncond 266-305; 7-8 tokens per attention slot, and the
    3 frames append up to position 508), ten of 120-240; FP64 oracle within
    1e-3."""
    import dataclasses

    from oracle.model import QWEN3_06B

    s = dataclasses.replace(QWEN3_06B, text_vocab=4096)
    w = _device_weights(s, 19, hip_device)
    prefix = [(440, 505)] * 6 + [(120, 240)] * 10
    rel = _many_utterance_case(s, w, 16, 8, hip_device, bf16=True, frames=3, max_len=512, prefix=prefix)
    print(f"q06b BF16, 16 utterances, six with 440-505-position prefixes: max row-relative logit error {rel:.3e}")
    assert rel < LOGIT_TOL


def test_sixteen_utterances_tiny_long_contexts(hip_device):
    """Tiny shape (head_dim 16: a slot is one lane, 512 slots per workgroup),
    16 utterances x CFG: 4 splits per (row, kv head), so a slot's tokens are
    2,048 apart.  Four utterances have cond prefixes of 2,600-3,000
    positions (uncond 1,560-1,800), so a quarter to a half of their cond
    rows' slots hold 2 tokens, the rest one; twelve have 20-60.  FP32
    weights and cache against the FP64 oracle within 1e-3."""
    from oracle.model import TINY

    w = synthetic_weights(TINY, 33, norm_gain_std=0.1, bias_std=0.02)
    prefix = [(2600, 3000)] * 4 + [(20, 60)] * 12
    rel = _many_utterance_case(TINY, w, 16, 10, hip_device, frames=2, max_len=3072, prefix=prefix)
    print(f"tiny, 16 utterances, four with 2,600-3,000-position prefixes: max row-relative logit error {rel:.3e}")
    assert rel < LOGIT_TOL


def test_generate_batch_per_utterance_equals_oracle(hip_device):
    """FastGenerator.generate_batch: three utterances with ragged prefixes,
    decoded together (six rows: the skinny-GEMM path), sampled with top-k /
    top-p / CFG from explicit per-utterance uniforms; each utterance's codes
    and stop reason equal the float64 oracle's run of that utterance alone
    (including retirement at its own EOS)."""
    import torch
    from soraku_amd import FastGenerator

    f, s, gen = load_golden("tiny_sampled")
    w = _weights(f, s)
    w["depth_head.bias"] = w["depth_head.bias"].copy()
    w["depth_head.bias"][0, s.eos_id] += 0.2      # the utterances retire at frames 4, 12 and never (oracle)
    lang = tuple(int(v) for v in f["language_ids"])
    n_frames = 14
    kw = {k: v for k, v in gen.items() if k not in ("seed", "max_new_frames")}
    rng = np.random.default_rng(23)
    reqs, us = [], []
    for i in range(3):
        nt = 4 + 5 * i
        reqs.append(dict(input_ids=torch.tensor(rng.integers(0, s.text_vocab, nt)[None]),
                         prompt_codes=torch.tensor(rng.integers(0, s.codebook_size, (i, s.n_codebooks))),
                         uncond_input_ids=torch.tensor(f["uncond_ids"][None])))
        us.append(rng.random((n_frames, s.n_codebooks)))
    g = FastGenerator(device=hip_device, state_dict=w, shape=_shape(s), language_token_ids=lang)
    out = g.generate_batch(reqs, max_new_frames=n_frames, uniforms=np.stack(us), **kw)
    m = OracleModel(s, w, np.float64, language_token_ids=lang)
    for r, u, (codes, info) in zip(reqs, us, out):
        ref, rinfo = generate(m, input_ids=r["input_ids"].numpy()[0], prompt_codes=r["prompt_codes"].numpy(),
                              uncond_input_ids=r["uncond_input_ids"].numpy()[0], uniforms=u, batched=True,
                              max_new_frames=n_frames, **kw)
        np.testing.assert_array_equal(codes.numpy(), ref)
        assert info["stop_reason"] == rinfo["stop_reason"]
    print("stop reasons", [o[1]["stop_reason"] for o in out], "frames", [o[1]["num_frames"] for o in out])
    assert sorted(o[1]["stop_reason"] for o in out) == ["eos", "eos", "max_frames"]


@pytest.mark.parametrize("max_batch", [2, 3])
def test_generate_batch_continuous_refill(hip_device, max_batch):
    """Continuous batching: seven requests through 2 or 3 utterance slots (4
    rows: GEMV path; 6 rows: skinny-GEMM path).  A slot whose request retires
    (EOS or max_new_frames) is prefilled with the next request between frames
    while the other slots keep decoding; a refilled request starts at its own
    frame 0, so EOS is masked for it alone during its first min_new_frames.
    Every request's codes and stop reason equal the float64 oracle's run of
    that request alone."""
    import torch
    from soraku_amd import FastGenerator

    f, s, gen = load_golden("tiny_sampled")
    w = _weights(f, s)
    w["depth_head.bias"] = w["depth_head.bias"].copy()
    w["depth_head.bias"][0, s.eos_id] += 0.2      # staggered retirement: EOS or max_new_frames
    lang = tuple(int(v) for v in f["language_ids"])
    n_frames = 5
    kw = {k: v for k, v in gen.items() if k not in ("seed", "max_new_frames")}
    rng = np.random.default_rng(41)
    reqs, us = [], []
    for i in range(7):
        nt = 3 + 3 * (i % 4)
        reqs.append(dict(input_ids=torch.tensor(rng.integers(0, s.text_vocab, nt)[None]),
                         prompt_codes=torch.tensor(rng.integers(0, s.codebook_size, (i % 3, s.n_codebooks))),
                         uncond_input_ids=torch.tensor(f["uncond_ids"][None])))
        us.append(rng.random((n_frames, s.n_codebooks)))
    g = FastGenerator(device=hip_device, state_dict=w, shape=_shape(s), language_token_ids=lang)
    out = g.generate_batch(reqs, max_new_frames=n_frames, uniforms=np.stack(us), max_batch=max_batch, **kw)
    m = OracleModel(s, w, np.float64, language_token_ids=lang)
    for r, u, (codes, info) in zip(reqs, us, out):
        ref, rinfo = generate(m, input_ids=r["input_ids"].numpy()[0], prompt_codes=r["prompt_codes"].numpy(),
                              uncond_input_ids=r["uncond_input_ids"].numpy()[0], uniforms=u, batched=True,
                              max_new_frames=n_frames, **kw)
        np.testing.assert_array_equal(codes.numpy(), ref)
        assert info["stop_reason"] == rinfo["stop_reason"]
    reasons = [o[1]["stop_reason"] for o in out]
    print(f"max_batch {max_batch}: stop reasons {reasons}, frames {[o[1]['num_frames'] for o in out]}")
    assert "eos" in reasons and "max_frames" in reasons


def test_from_pretrained_release_untied_head(hip_device, tmp_path):
    """A release directory (config gate, text config, model.safetensors) with
    an untied classifier head and four language tokens, loaded by
    FastGenerator.from_pretrained: greedy CFG codes equal the float64
    oracle's on the same tensors; the text includes language-token ids."""
    import dataclasses

    import torch
    from oracle.model import TINY
    from soraku_amd import FastGenerator
    from test_checkpoint import write_release

    s = dataclasses.replace(TINY, tie_audio_head=False, n_language=4)
    w = synthetic_weights(s, 7, norm_gain_std=0.1, bias_std=0.02)
    lang = (90, 91, 92, 93)
    write_release(tmp_path, s, w, soraku_extra=dict(language_token_ids=list(lang)))
    rng = np.random.default_rng(2)
    text = np.concatenate([[91], rng.integers(0, 80, 9)])
    prompt = rng.integers(0, s.codebook_size, (2, s.n_codebooks))
    kw = dict(max_new_frames=10, min_new_frames=2, temperature=0.0, cfg_scale=1.5)
    g = FastGenerator.from_pretrained(tmp_path, device=hip_device)
    codes, info = g.generate(input_ids=torch.tensor(text[None]), prompt_codes=torch.tensor(prompt),
                             uncond_input_ids=torch.tensor([[3]]), **kw)
    ref, rinfo = generate(OracleModel(s, w, np.float64, language_token_ids=lang), input_ids=text,
                          prompt_codes=prompt, uncond_input_ids=np.array([3]), batched=True, **kw)
    np.testing.assert_array_equal(codes.numpy(), ref)
    assert info["stop_reason"] == rinfo["stop_reason"]


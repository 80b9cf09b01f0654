"""sk_prefill_run_noalloc (the prefill with its activation buffers in the
library's static scratch instead of engine-allocated memory) against
sk_prefill_run, called through the C ABI on two engines with the same
weights: the rows' depth-input hidden states and K/V caches are equal bit for
bit, and so are the logits of a decoded frame.  Two calls in a row, the
second with a shorter prefix (the scratch keeps the first call's contents);
a prefix larger than the scratch is refused with SK_EINVAL."""

import dataclasses

import numpy as np
import pytest

from oracle.model import QWEN3_06B, synthetic_weights

pytestmark = pytest.mark.gpu


def _shape(s):
    from soraku_amd.config import DecodeShape

    return DecodeShape(**{k: getattr(s, k) for k in DecodeShape.__dataclass_fields__})


def _kv(e, layer, kv):
    import ctypes as C

    from soraku_amd._lib import check, lib

    p = C.c_void_p()
    check(lib().sk_kv_ptr(e._h, layer, kv, C.byref(p)))
    e.synchronize()
    hip = C.CDLL("libamdhip64.so.7")
    hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    s = e.shape
    out = np.empty((e.rows, s.n_kv_heads, e.max_len, s.head_dim), np.float32)
    assert hip.hipMemcpy(out.ctypes.data, p, out.nbytes, 2) == 0   # hipMemcpyDeviceToHost
    return out


def _prefill(e, noalloc, text, uncond, prompt):
    from soraku_amd._lib import check, lib

    e._stage(0, text, uncond, prompt)
    fn = lib().sk_prefill_run_noalloc if noalloc else lib().sk_prefill_run
    print(f"prefill {'noalloc' if noalloc else 'alloc'}: {text.size}+{uncond.size} text ids, "
          f"{prompt.shape[0]} prompt frames", flush=True)
    check(fn(e._h))


def test_noalloc_prefill_equals_prefill(hip_device):
    from soraku_amd import GraphFrameEngine
    from soraku_amd._lib import SK_EINVAL, SkError

    s = dataclasses.replace(QWEN3_06B, text_vocab=4096)
    w = synthetic_weights(s, 77, norm_gain_std=0.1, bias_std=0.02)
    rng = np.random.default_rng(77)
    engines = [GraphFrameEngine(device=hip_device, max_cache_len=420, cfg_scale=1.5, batch=2, state_dict=w,
                                shape=_shape(s)) for _ in range(2)]
    for e in engines:
        e.set_temperature(0.0)
        e.set_debug(True)
    # first call: 96 text ids + BOS + 144 prompt frames (241 / 146 positions);
    # second call: a shorter prefix (65 / 26)
    cases = [(rng.integers(0, s.text_vocab, 96), np.array([5]), rng.integers(0, 2048, (144, 16))),
             (rng.integers(0, s.text_vocab, 40), np.array([9]), rng.integers(0, 2048, (24, 16)))]
    for ci, (text, uncond, prompt) in enumerate(cases):
        for noalloc, e in zip((False, True), engines):
            _prefill(e, noalloc, text, uncond, prompt)
        h = [e.hidden() for e in engines]
        np.testing.assert_array_equal(h[0], h[1])
        n = text.size + 1 + prompt.shape[0]
        for layer in (0, 13, 27):
            for kv in (0, 1):
                a, b = (_kv(e, layer, kv) for e in engines)
                np.testing.assert_array_equal(a[0, :, :n], b[0, :, :n])
                np.testing.assert_array_equal(a[1, :, :n - text.size + 1], b[1, :, :n - text.size + 1])
        lg = []
        for e in engines:
            e.capture()
            lg.append(e.step_frame(mask_eos_q0=True, return_logits=True)[1])
        np.testing.assert_array_equal(lg[0], lg[1])
        print(f"call {ci}: hidden, K/V caches and one frame's logits equal", flush=True)
    # more packed tokens than the scratch holds: refused before any kernel runs
    text = rng.integers(0, s.text_vocab, 400)
    e = engines[1]
    e._stage(0, text, text[:300], np.zeros((0, 16), np.int64))
    from soraku_amd._lib import lib

    assert lib().sk_prefill_run_noalloc(e._h) == SK_EINVAL
    with pytest.raises(SkError):
        from soraku_amd._lib import check

        check(lib().sk_prefill_run_noalloc(e._h))
    for e in engines:
        e.close()

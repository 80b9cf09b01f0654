"""C-ABI checks that need no GPU: the library loads, exports every entry point
include/soraku_mi355x.h declares, and rejects bad arguments before any HIP
call (the host-side failure list of the reference: graph_frame.py:128-129,
155-156, 301-302; fast_generate.py:250-251; model.py:541-544)."""

import ctypes as C
import os
import re

import numpy as np
import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "soraku_mi355x.h")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+char\*|void\*|int32_t|int)\s+(sk_\w+)\s*\(", text, re.M)))


@pytest.fixture(scope="module")
def L():
    from soraku_amd import _lib

    return _lib.load()


def test_every_declared_symbol_is_exported(L):
    names = declared_symbols()
    assert len(names) >= 25
    for n in names:
        assert hasattr(L, n), n


def test_binding_covers_header():
    from soraku_amd._lib import PROTOTYPES

    assert sorted(PROTOTYPES) == declared_symbols()


def test_config_struct_layout_matches_header():
    """sk_config: 23 int32/float fields, int32[4], then kv_dtype = 112 bytes;
    the field names and order are those of include/soraku_mi355x.h."""
    import re

    from conftest import ROOT
    from soraku_amd._lib import SkConfig

    assert C.sizeof(SkConfig) == 23 * 4 + 16 + 4
    hdr = open(f"{ROOT}/include/soraku_mi355x.h").read()
    body = hdr[hdr.index("typedef struct sk_config {"):hdr.index("} sk_config;")]
    names = re.findall(r"(?:int32_t|float)\s+([^;]+);", body)
    fields = [n.strip() for group in names for n in group.split(",")]
    fields = [re.sub(r"\[.*\]", "", f).strip() for f in fields]
    assert fields == [f[0] for f in SkConfig._fields_]


def _good_config():
    from soraku_amd.config import TINY, to_sk_config

    return to_sk_config(TINY, n_utts=1, cfg_rows=2, max_ctx=64, max_frames=16)


@pytest.mark.parametrize("field,value", [
    ("d_model", 12), ("head_dim", 24), ("n_kv_heads", 3), ("cfg_rows", 3), ("n_utts", 0),
    ("audio_vocab", 5000), ("max_ctx", 1), ("bos_id", 35), ("weight_dtype", 7), ("n_language", 2),
    ("trunk_eps", 0.0), ("kv_dtype", 5),
])
def test_create_rejects_bad_config(L, field, value):
    from soraku_amd._lib import SK_EINVAL

    c = _good_config()
    setattr(c, field, value)
    h = C.c_void_p()
    assert L.sk_create(C.byref(c), None, C.byref(h)) == SK_EINVAL
    assert h.value is None
    assert L.sk_last_error().decode()


def test_null_handles_are_rejected(L):
    from soraku_amd._lib import SK_EINVAL

    assert L.sk_create(None, None, None) == SK_EINVAL
    assert L.sk_destroy(None) == 0
    assert L.sk_prefill_run(None) == SK_EINVAL
    assert L.sk_capture(None) == SK_EINVAL
    assert L.sk_step_frame(None, 0, None, None, None, None) == SK_EINVAL
    assert L.sk_bind_weight(None, b"trunk.norm.weight", None, 0, None, 0) == SK_EINVAL
    assert L.sk_frames_done(None) == -1
    assert L.sk_xcd_layers(None) == -1
    assert L.sk_debug_set_spin_ticks(None, 0) == SK_EINVAL
    assert L.sk_prefill_run_noalloc(None) == SK_EINVAL
    assert L.sk_prefill_refill(None) == SK_EINVAL
    assert L.sk_retire_row(None, 0) == SK_EINVAL
    assert L.sk_reset_frames(None) == SK_EINVAL


def test_ops_reject_bad_arguments(L):
    from soraku_amd._lib import SK_EINVAL

    p = C.c_void_p(4096)
    assert L.sk_op_swiglu_gemv(None, 2, 16, 12, 0, p, p, p, p) == SK_EINVAL   # D % 8
    assert L.sk_op_swiglu_gemv(None, 2, 16, 16, 9, p, p, p, p) == SK_EINVAL   # dtype
    assert L.sk_op_classifier_gemv(None, 2, 16, 16, 0, p, None, p, p) == SK_EINVAL
    assert L.sk_op_down_residual_gemv(None, 0, 16, 16, 0, p, p, p, p) == SK_EINVAL
    assert L.sk_op_sample(None, 3, 64, p, 1.5, 0, 0, 61, 62, 63, 0.9, 50, 0.9, 0.5, p) == SK_EINVAL
    assert L.sk_op_sample(None, 2, 64, p, 1.5, 0, 0, 61, 62, 63, 0.9, 50, 0.9, 1.0, p) == SK_EINVAL
    assert L.sk_op_sample(None, 2, 9000, p, 1.5, 0, 0, 61, 62, 63, 0.9, 50, 0.9, 0.5, p) == SK_EINVAL
    assert L.sk_op_rmsnorm(None, 0, 16, 1e-6, p, p, p) == SK_EINVAL


def test_generate_argument_errors_before_gpu():
    """FastGenerator.generate validates like fast_generate.py:351-354."""
    from soraku_amd import FastGenerator

    g = FastGenerator.__new__(FastGenerator)
    with pytest.raises(ValueError):
        FastGenerator.generate(g, input_ids=np.zeros((2, 3), np.int64))
    with pytest.raises(ValueError):
        FastGenerator.generate(g, input_ids=np.zeros((1, 3), np.int64), cfg_scale=1.5)


def test_eos_mask_bits():
    """The per-utterance EOS mask passed to sk_step_frame / sk_queue_frames:
    bit u is utterance u; a bool covers every utterance; 32 utterances use
    all 32 bits of the signed argument."""
    from soraku_amd import GraphFrameEngine

    e = GraphFrameEngine.__new__(GraphFrameEngine)
    e.n_utts = 3
    assert e.eos_mask_bits(True) == 0b111 and e.eos_mask_bits(False) == 0
    assert e.eos_mask_bits([True, False, True]) == 0b101
    assert e.eos_mask_bits(np.array([0, 1, 0])) == 0b010
    with pytest.raises(ValueError):
        e.eos_mask_bits([True, False])
    e.n_utts = 1
    assert e.eos_mask_bits(1) == 1
    e.n_utts = 32
    assert e.eos_mask_bits(True) == -1
    assert e.eos_mask_bits([False] * 31 + [True]) == -(1 << 31)
    assert e.eos_mask_bits([True] + [False] * 31) == 1


def test_generate_batch_argument_errors_before_gpu():
    """generate_batch checks its requests and max_batch before any engine."""
    from soraku_amd import FastGenerator

    g = FastGenerator.__new__(FastGenerator)
    g._shape = None
    ok = dict(input_ids=np.zeros((1, 3), np.int64), uncond_input_ids=np.zeros((1, 1), np.int64))
    with pytest.raises(ValueError):
        FastGenerator.generate_batch(g, [])
    with pytest.raises(ValueError):
        FastGenerator.generate_batch(g, [dict(input_ids=np.zeros((1, 3), np.int64))], cfg_scale=1.5)
    with pytest.raises(ValueError):
        FastGenerator.generate_batch(g, [ok] * 3, cfg_scale=1.5, max_batch=17)
    with pytest.raises(ValueError):
        FastGenerator.generate_batch(g, [ok] * 3, cfg_scale=1.5, max_batch=0)


def test_synthetic_weights_match_oracle():
    """The package's seeded weights are the oracle's, value for value."""
    from oracle.model import TINY as OT, synthetic_weights as ow
    from soraku_amd.config import TINY
    from soraku_amd.synthetic import synthetic_weights as pw

    a = ow(OT, 3, norm_gain_std=0.1, bias_std=0.02)
    b = pw(TINY, 3, norm_gain_std=0.1, bias_std=0.02)
    assert sorted(a) == sorted(b)
    for k in a:
        np.testing.assert_array_equal(a[k], b[k])


def test_shape_from_model_reads_the_untied_head():
    """shape_from_model follows SorakuV2Config.tie_audio_head (model.py:131,
    141-145,171-174): an untied model binds depth_head.out_proj."""
    from types import SimpleNamespace

    from soraku_amd.config import shape_from_model
    from soraku_amd.synthetic import weight_shapes

    trunk = SimpleNamespace(config=SimpleNamespace(
        hidden_size=64, num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2, head_dim=16,
        intermediate_size=96, vocab_size=100, rms_norm_eps=1e-6, rope_parameters={"rope_theta": 1e6}))
    for tie in (True, False):
        cfg = SimpleNamespace(depth_ffn_mult=2, num_codebooks=4, codebook_size=32, language_token_ids=(),
                              tie_audio_head=tie)
        s = shape_from_model(SimpleNamespace(config=cfg, trunk=trunk))
        assert s.tie_audio_head is tie
        keys = weight_shapes(s)
        assert ("depth_head.out_proj" in keys) is (not tie)
        if not tie:
            assert keys["depth_head.out_proj"] == (4, 35, 64)
    # a config without the field is a tied head (the reference default)
    cfg = SimpleNamespace(depth_ffn_mult=2, num_codebooks=4, codebook_size=32)
    assert shape_from_model(SimpleNamespace(config=cfg, trunk=trunk)).tie_audio_head is True

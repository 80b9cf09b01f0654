"""Release-directory loading (runtime.py:14-44 layout) on the CPU: config
gate, decode shape, tensor selection and checks.  No GPU needed."""

import dataclasses
import json

import numpy as np
import pytest

from oracle.model import TINY, synthetic_weights

torch = pytest.importorskip("torch")


def write_release(path, s, w, *, soraku_extra=None, text_extra=None, extra_tensors=None, drop=None,
                  fmt=1, model_type="soraku_tts_v2"):
    """A release directory for shape ``s`` holding ``w`` (+ extra tensors)."""
    soraku = dict(num_codebooks=s.n_codebooks, codebook_size=s.codebook_size, depth_ffn_mult=s.depth_mult,
                  tie_audio_head=s.tie_audio_head, speaker_conditioning=False, language_token_ids=[])
    soraku.update(soraku_extra or {})
    text = dict(hidden_size=s.d_model, num_hidden_layers=s.n_layers, num_attention_heads=s.n_q_heads,
                num_key_value_heads=s.n_kv_heads, head_dim=s.head_dim, intermediate_size=s.trunk_inter,
                vocab_size=s.text_vocab, rms_norm_eps=s.trunk_eps, rope_theta=s.rope_theta,
                model_type="qwen3")
    text.update(text_extra or {})
    (path / "config.json").write_text(json.dumps(dict(format_version=fmt, model_type=model_type,
                                                      soraku_config=soraku)))
    (path / "text_config.json").write_text(json.dumps(text))
    tensors = {k: torch.from_numpy(np.ascontiguousarray(v)) for k, v in w.items() if k != drop}
    tensors.update(extra_tensors or {})
    from safetensors.torch import save_file

    save_file(tensors, str(path / "model.safetensors"))
    return path


def test_load_release_roundtrip(tmp_path):
    from soraku_amd import load_release

    w = synthetic_weights(TINY, 5, norm_gain_std=0.1, bias_std=0.02)
    extra = {"speaker_slot_embedding": torch.zeros(TINY.d_model)}   # not on the decode path: ignored
    write_release(tmp_path, TINY, w, extra_tensors=extra)
    rel = load_release(tmp_path)
    for f in ("d_model", "n_layers", "n_q_heads", "n_kv_heads", "head_dim", "trunk_inter", "depth_mult",
              "n_codebooks", "codebook_size", "text_vocab", "trunk_eps", "rope_theta", "tie_audio_head"):
        assert getattr(rel.shape, f) == getattr(TINY, f), f
    assert set(rel.state_dict) == set(w)
    for k, v in w.items():
        assert rel.state_dict[k].dtype == torch.float32
        np.testing.assert_array_equal(rel.state_dict[k].numpy(), v)
    bf = load_release(tmp_path, bf16=True)
    assert bf.state_dict["trunk.layers.0.mlp.up_proj.weight"].dtype == torch.bfloat16
    assert bf.state_dict["trunk.norm.weight"].dtype == torch.float32
    assert bf.state_dict["depth_head.bias"].dtype == torch.float32


def test_load_release_untied_head_and_languages(tmp_path):
    from soraku_amd import load_release

    s = dataclasses.replace(TINY, tie_audio_head=False, n_language=4)
    w = synthetic_weights(s, 6)
    assert "depth_head.out_proj" in w and "language_embeddings.weight" in w
    write_release(tmp_path, s, w, soraku_extra=dict(language_token_ids=[90, 91, 92, 93]))
    rel = load_release(tmp_path)
    assert rel.shape.tie_audio_head is False and rel.shape.n_language == 4
    assert rel.language_token_ids == (90, 91, 92, 93)
    np.testing.assert_array_equal(rel.state_dict["depth_head.out_proj"].numpy(), w["depth_head.out_proj"])


@pytest.mark.parametrize("case, msg", [
    (dict(fmt=2), "not a supported"),
    (dict(model_type="other"), "not a supported"),
    (dict(soraku_extra=dict(speaker_conditioning=True)), "speaker-conditioned"),
    (dict(soraku_extra=dict(language_token_ids=[1, 2, 3])), "four unique"),
    (dict(drop="trunk.norm.weight"), "lacks trunk.norm.weight"),
    (dict(text_extra=dict(intermediate_size=128)), "expected"),
])
def test_load_release_rejects(tmp_path, case, msg):
    from soraku_amd import load_release

    w = synthetic_weights(TINY, 5)
    write_release(tmp_path, TINY, w, **case)
    with pytest.raises(ValueError, match=msg):
        load_release(tmp_path)

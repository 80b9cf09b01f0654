"""CPU oracle for the soraku-TTS per-frame CFG decode step.

TEST INFRASTRUCTURE ONLY.  Nothing in the product package imports this
package; only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline``
leg of ``bench.py`` may use it, and only as the checker (or as the timed CPU
baseline), never as the thing measured or shipped.

It restates, in NumPy, the reference's *native* FP32 semantics
(``soraku_inference/model.py``) and the third-party Qwen3 trunk it calls
(``transformers/models/qwen3/modeling_qwen3.py``, pinned at
transformers==4.57.3 by ``pyproject.toml:14``; read from the installed 5.15.0
source, whose decode arithmetic is the same).  Every function cites the
reference file:line it follows.

Pinning status of each function (how a plausible mistake would be caught):

* ``rms_norm``, ``silu``, ``swiglu``, ``rope_cos_sin``/``apply_rope``,
  ``attend``, ``frame_embedding``, ``cfg_merge``, ``apply_masks`` --
  closed forms and invariants in ``tests/test_oracle_math.py`` (float64
  brute force, RoPE relative-position identity, ctx=1 attention, CFG s=0/1).
* ``trunk_prefill``/``trunk_step``/``depth_logits``/``generate`` (the
  composition) -- golden vectors written by ``tests/golden/make_golden.py``
  from the reference ``SorakuTTSv2.generate`` on CPU at a tiny shape
  (merged logits of every depth step, greedy codes, hidden states).
* ``topk_topp_filter`` -- golden probability vectors captured at the
  reference ``_sample_logits`` (model.py:686-708) plus brute force on tiny V.
* ``draw`` (the explicit-uniform inverse-CDF draw) -- the reference has no
  such function (``torch.multinomial`` takes no external uniforms); it is this
  build's definition, pinned by brute force and a chi-square test against the
  filtered distribution.  Bit-exactness is GPU vs this definition.
"""

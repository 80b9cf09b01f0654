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

* ``trunk_prefill``/``trunk_step``/``depth_logits``/``generate`` (the
  composition, tied and untied classifier head) -- golden vectors written by
  ``tests/golden/make_golden.py`` from the reference ``SorakuTTSv2.generate``
  on CPU (merged logits of every depth step, codes, hidden states) at a tiny
  shape and at the Qwen3-0.6B shape (``tests/test_oracle_golden.py``);
  ``test_planted_mistakes_are_caught`` shows a dropped depth residual or
  swapped CFG rows break the match.
* ``cfg_merge``, ``apply_masks`` -- the same golden vectors (every recorded
  ``_sample_logits`` argument is the masked CFG merge).
* ``rms_norm``, ``silu``, ``rope_cos_sin``/``apply_rope``, ``attend`` -- the
  golden vectors through the composition, plus closed forms in
  ``tests/test_oracle_math.py`` (unit RMS, scale invariance, position 0 is the
  identity, RoPE keeps norms and makes scores depend on m - n only, one-token
  attention returns v, equal keys average V, GQA equals repeated heads).
* ``filtered_probs`` (the top-k / top-p filter) -- the probability vectors the
  reference handed to ``torch.multinomial`` (model.py:707), V = 35 and
  V = 2051, plus brute force of the reference's rule on tiny V
  (``tests/test_oracle_math.py``).
* ``draw`` (the explicit-uniform inverse-CDF draw) -- the reference has no
  such function (``torch.multinomial`` takes no external uniforms); it is this
  build's definition, pinned in ``tests/test_oracle_math.py``: each kept
  candidate's preimage in u is one interval of width ``filtered_probs[i]`` in
  candidate order, boundaries belong to the upper candidate, k = 1 / tiny p /
  T <= 0 give the top candidate, and a chi-square test of 10^5 seeded draws.
  The same file shows that an argmax draw, ``>=`` for ``>`` and normalising
  by the total instead of the kept mass all fail those checks.
* ``scan_sums`` -- an inclusive prefix sum (float64 closed form) in the fixed
  row order, checked on a case where other orders round differently
  (``tests/test_oracle_golden.py``).
* ``round_bf16`` -- equal bit for bit to ``torch.Tensor.to(torch.bfloat16)``
  on CPU over normal, halfway, subnormal and extreme values.
"""

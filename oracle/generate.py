"""Oracle frame loop: ``SorakuTTSv2.generate`` native semantics
(soraku_inference/model.py:515-621) with the explicit-uniform draw.

Cond and uncond run as separate branches with their own caches and positions
(model.py:551-553,561-563,611-612).  ``batched=True`` evaluates both rows in
one call per op (the same arithmetic with both rows stacked, as the GPU
engine does); ``batched=False`` is the reference's B=1-per-branch order.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from .model import OracleModel, RowState
from .sampler import apply_masks, cfg_merge, sample


@dataclass
class Record:
    merged: list = field(default_factory=list)   # [frames][Q] FP32 [V] (after CFG, before masks)
    logits: list = field(default_factory=list)   # [frames][Q] [rows, V] per-branch logits
    hidden: list = field(default_factory=list)   # [frames] [rows, d] depth input of each frame


def start_states(m: OracleModel, text_ids, prompt_codes, uncond_ids, cfg_scale, max_ctx):
    """Prefill each branch (model.py:561-563,623-656)."""
    branches = [np.asarray(text_ids, np.int64).reshape(-1)]
    if cfg_scale != 1.0:
        if uncond_ids is None:
            raise ValueError("classifier-free guidance requires uncond_input_ids")
        branches.append(np.asarray(uncond_ids, np.int64).reshape(-1))
    states = []
    for ids in branches:
        st = RowState(m.s, max_ctx, m.dtype)
        m.prefill(st, m.prefix_embeds(ids, prompt_codes))
        states.append(st)
    return states


def generate(m: OracleModel, *, input_ids, prompt_codes=None, max_new_frames=384,
             min_new_frames=4, temperature=0.9, top_k=50, top_p=0.95,
             temperature_q0=None, top_k_q0=None, top_p_q0=None, cfg_scale=1.0,
             uncond_input_ids=None, uniforms=None, forced_codes=None,
             batched=False, record: Record | None = None, max_ctx=None, states=None):
    """Returns ``(codes [T, Q] int64, info)`` like model.py:614-621.

    ``uniforms [max_new_frames, Q]`` feed the draw (ignored when greedy).
    ``forced_codes [frames, Q]`` teacher-forces the codes (logits are still
    computed and recorded), which keeps two implementations on one trajectory.
    """
    s = m.s
    Q = s.n_codebooks
    if states is None:
        if max_ctx is None:
            plen = 1 + (0 if prompt_codes is None else np.asarray(prompt_codes).reshape(-1, Q).shape[0])
            max_ctx = np.asarray(input_ids).size + plen + max_new_frames + 1
        states = start_states(m, input_ids, prompt_codes, uncond_input_ids, cfg_scale, max_ctx)
    frames = []
    stop_reason = "max_frames"
    for index in range(max_new_frames):
        hiddens = np.stack([st.hidden for st in states])
        if record is not None:
            record.hidden.append(hiddens.copy())
        prefix = np.zeros_like(hiddens)
        codes = []
        reached_eos = False
        rec_m, rec_l = [], []
        for q in range(Q):
            if batched:
                logits = m.depth_logits(hiddens, prefix, q)
            else:
                logits = np.stack([m.depth_logits(hiddens[r:r + 1], prefix[r:r + 1], q)[0]
                                   for r in range(len(states))])
            logits = logits.astype(np.float32)
            merged = logits[0] if len(states) == 1 else cfg_merge(logits[0], logits[1], cfg_scale)
            rec_m.append(merged)
            rec_l.append(logits)
            masked = apply_masks(merged, q=q, frame_index=index, min_new_frames=min_new_frames,
                                 bos_id=s.bos_id, eos_id=s.eos_id, pad_id=s.pad_id)
            t = temperature_q0 if q == 0 and temperature_q0 is not None else temperature
            k = top_k_q0 if q == 0 and top_k_q0 is not None else top_k
            p = top_p_q0 if q == 0 and top_p_q0 is not None else top_p
            u = 0.0 if uniforms is None else float(uniforms[index][q])
            code = sample(masked, temperature=t, top_k=k, top_p=p, u=u)
            if forced_codes is not None:
                code = int(forced_codes[index][q])
            if q == 0 and code == s.eos_id:
                reached_eos = True
                break
            codes.append(code)
            prefix = prefix + m.prefix_step(q, code)
        if record is not None:
            record.merged.append(rec_m)
            record.logits.append(rec_l)
        if reached_eos:
            stop_reason = "eos"
            break
        frames.append(codes)
        emb = m.frame_embedding(np.asarray(codes, np.int64))
        x = np.stack([emb] * len(states))
        if batched:
            m.trunk_step(states, x)
        else:
            for r, st in enumerate(states):
                m.trunk_step([st], x[r:r + 1])
    out = np.asarray(frames, np.int64).reshape(-1, Q)
    return out, {"stop_reason": stop_reason, "num_frames": int(out.shape[0]), "cfg_scale": cfg_scale}

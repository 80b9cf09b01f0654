"""``generate`` on the MI355X engine, with the keyword contract of
``FastGenerator.generate`` / ``SorakuTTSv2.generate``
(soraku_inference/acceleration/fast_generate.py:331-489,492-569;
soraku_inference/model.py:515-621).

Frame loop as ``_generate_graph`` (fast_generate.py:549-556): one replay per
frame, codes copied to the host, EOS at q0 ends the utterance once
``index >= min_new_frames``.  Sampling uses explicit uniforms: pass
``uniforms [max_new_frames, Q]`` to reproduce a run exactly, or a ``seed``
from which ``numpy.random.default_rng(seed).random((max_new_frames, Q))`` is
drawn.
"""

from __future__ import annotations

from typing import Any

import numpy as np

from .config import DecodeShape
from .engine import GraphFrameEngine


class FastGenerator:
    """Drop-in for ``FastGenerator`` (fast_generate.py:28-79): same
    constructor keywords; every backend choice runs the MI355X engine."""

    def __init__(self, model=None, *, device="cuda:0", use_tilelang: bool = True,
                 compile_trunk: bool = False, batch_branches: bool = True,
                 native_sampling: bool = True, use_graph: bool = True, bf16: bool = False,
                 kv_bf16: bool = False,
                 state_dict=None, shape: DecodeShape | None = None, language_token_ids=()):
        cfg = getattr(model, "config", None)
        if cfg is not None and getattr(cfg, "speaker_conditioning", False):
            raise ValueError("speaker-conditioned checkpoints currently require native generate; "
                             "fast prefill is not validated")
        self.model = model
        self.device = device
        self.bf16 = bf16
        self.kv_bf16 = kv_bf16
        self._state_dict = state_dict
        self._shape = shape
        self._language_token_ids = tuple(language_token_ids)
        self._engine: GraphFrameEngine | None = None
        self._engine_key = None

    @classmethod
    def from_pretrained(cls, model_dir, *, device="cuda:0", bf16: bool = False, kv_bf16: bool = False):
        """A generator over a release directory (runtime.py:14-44 layout):
        config gate, decode shape and tensors from ``load_release``."""
        from .checkpoint import load_release

        rel = load_release(model_dir, bf16=bf16)
        return cls(device=device, state_dict=rel.state_dict, shape=rel.shape,
                   language_token_ids=rel.language_token_ids, bf16=bf16, kv_bf16=kv_bf16)

    def _engine_for(self, max_len: int, batch: int, cfg_scale: float, n_utts: int = 1) -> GraphFrameEngine:
        key = (batch, n_utts)
        e = self._engine
        if e is None or e.max_len < max_len or self._engine_key != key:
            if e is not None:
                e.close()
            e = GraphFrameEngine(self.model, device=self.device, max_cache_len=max(max_len, 512),
                                 cfg_scale=cfg_scale, batch=batch, state_dict=self._state_dict,
                                 shape=self._shape, language_token_ids=self._language_token_ids,
                                 bf16=self.bf16, kv_bf16=self.kv_bf16, n_utts=n_utts)
            self._engine, self._engine_key = e, key
        return e

    def generate(self, *, input_ids, prompt_codes=None, max_new_frames: int = 384,
                 min_new_frames: int = 4, temperature: float = 0.9, top_k: int | None = 50,
                 top_p: float | None = 0.95, temperature_q0: float | None = None,
                 top_k_q0: int | None = None, top_p_q0: float | None = None,
                 cfg_scale: float = 1.0, uncond_input_ids=None, seed: int | None = None,
                 on_frame: Any = None, use_graph: bool | None = None, uniforms=None):
        import torch

        shape = input_ids.shape if hasattr(input_ids, "shape") else np.asarray(input_ids).shape
        if len(shape) != 2 or shape[0] != 1:
            raise ValueError("generate expects input_ids of shape [1,L]")
        if cfg_scale != 1.0 and uncond_input_ids is None:
            raise ValueError("classifier-free guidance requires uncond_input_ids")
        batch = 2 if cfg_scale != 1.0 else 1
        n_prompt = 0 if prompt_codes is None else int(np.prod(prompt_codes.shape)) // (
            self._shape.n_codebooks if self._shape else 16)
        required = int(shape[1]) + 1 + n_prompt + max_new_frames + 8
        engine = self._engine_for(required, batch, cfg_scale)
        Q = engine.Q
        engine.cfg.fill_(cfg_scale)
        sampled = temperature > 0 or (temperature_q0 is not None and temperature_q0 > 0)
        engine.set_temperature(temperature, q0=temperature_q0)
        engine.set_sampling(sampled=sampled, top_k=top_k, top_p=top_p, top_k_q0=top_k_q0,
                            top_p_q0=top_p_q0)
        if uniforms is None:
            uniforms = np.random.default_rng(seed).random((max_new_frames, Q))
        uniforms = np.asarray(uniforms, np.float64).reshape(-1, Q)
        if uniforms.shape[0] < max_new_frames:
            raise ValueError("uniforms must cover max_new_frames rows")
        engine.prefill(input_ids, uncond_input_ids if batch == 2 else None, prompt_codes)
        if engine.graph is None:
            engine.capture()
        eos = engine.shape.eos_id
        frames = []
        stop_reason = "max_frames"
        for index in range(max_new_frames):
            codes = engine.step_frame(mask_eos_q0=index < min_new_frames, uniforms=uniforms[index])
            if index >= min_new_frames and int(codes[0]) == eos:
                stop_reason = "eos"
                break
            frames.append(codes.view(1, 1, Q))
            if on_frame is not None:
                on_frame(frames[-1])
        codes_tensor = (torch.cat(frames, dim=1).view(-1, Q) if frames
                        else torch.empty(0, Q, dtype=torch.long))
        return codes_tensor, {
            "stop_reason": stop_reason,
            "num_frames": codes_tensor.shape[0],
            "cfg_scale": cfg_scale,
            "backend": "mi355x",
            "sampled": sampled,
            "temperature": temperature,
        }

    def generate_batch(self, requests, *, max_new_frames: int = 384, min_new_frames: int = 4,
                       temperature: float = 0.9, top_k: int | None = 50, top_p: float | None = 0.95,
                       temperature_q0: float | None = None, top_k_q0: int | None = None,
                       top_p_q0: float | None = None, cfg_scale: float = 1.0, seeds=None, uniforms=None,
                       on_frame: Any = None, max_batch: int | None = None):
        """Several utterances decoded together (one engine, up to 16 utterance
        slots with CFG, 32 without; no reference counterpart beyond one
        utterance's CFG pair, fast_generate.py:232-328).  ``requests``: dicts
        with ``input_ids`` ``[1, L]`` and optional ``prompt_codes`` /
        ``uncond_input_ids``; prefixes may differ in length.  Request i draws
        from ``uniforms[i]`` (``[max_new_frames, Q]``) or from
        ``default_rng(seeds[i])`` exactly as ``generate(seed=seeds[i])``
        would, is decoded with its own frame index (EOS masked at q0 for its
        first ``min_new_frames`` frames) and retires at its own EOS or at
        ``max_new_frames``.  ``max_batch`` caps the slots; with more requests
        than slots, a slot whose request retires takes the next request
        between frames (continuous batching: only that slot is prefilled).
        Returns a list of ``(codes [T_i, Q], info)`` in request order."""
        import torch

        U = len(requests)
        if U < 1:
            raise ValueError("generate_batch needs at least one request")
        if cfg_scale != 1.0 and any(r.get("uncond_input_ids") is None for r in requests):
            raise ValueError("classifier-free guidance requires uncond_input_ids")
        batch = 2 if cfg_scale != 1.0 else 1
        cap = 32 // batch
        if max_batch is not None and not 1 <= max_batch <= cap:
            raise ValueError(f"max_batch must be in [1, {cap}]")
        slots = min(U, max_batch if max_batch is not None else cap)
        Qn = self._shape.n_codebooks if self._shape else 16
        longest = 0
        for r in requests:
            ids = r["input_ids"]
            shape = ids.shape if hasattr(ids, "shape") else np.asarray(ids).shape
            if len(shape) != 2 or shape[0] != 1:
                raise ValueError("generate_batch expects input_ids of shape [1,L]")
            pc = r.get("prompt_codes")
            n_prompt = 0 if pc is None else int(np.prod(pc.shape)) // Qn
            longest = max(longest, int(shape[1]) + 1 + n_prompt)
        engine = self._engine_for(longest + max_new_frames + 8, batch, cfg_scale, n_utts=slots)
        Q = engine.Q
        engine.cfg.fill_(cfg_scale)
        sampled = temperature > 0 or (temperature_q0 is not None and temperature_q0 > 0)
        engine.set_temperature(temperature, q0=temperature_q0)
        engine.set_sampling(sampled=sampled, top_k=top_k, top_p=top_p, top_k_q0=top_k_q0,
                            top_p_q0=top_p_q0)
        if uniforms is None:
            seeds = list(seeds) if seeds is not None else [None] * U
            uniforms = np.stack([np.random.default_rng(sd).random((max_new_frames, Q)) for sd in seeds])
        uniforms = np.asarray(uniforms, np.float64).reshape(U, -1, Q)
        if uniforms.shape[1] < max_new_frames:
            raise ValueError("uniforms must cover max_new_frames rows per utterance")

        def item(i):
            r = requests[i]
            return (r["input_ids"], r.get("uncond_input_ids") if batch == 2 else None, r.get("prompt_codes"))

        engine.prefill_utterances([item(i) for i in range(slots)])
        if engine.graph is None:
            engine.capture()
        eos = engine.shape.eos_id
        slot_req = list(range(slots))          # request decoded in each slot (None: idle)
        slot_idx = [0] * slots                 # that request's frame index
        next_req = slots
        frames: list[list] = [[] for _ in range(U)]
        reason = ["max_frames"] * U
        while any(i is not None for i in slot_req):
            if engine.frames_done + 1 > engine.max_frames:
                engine.reset_frames()
            mask = [i is not None and slot_idx[s] < min_new_frames for s, i in enumerate(slot_req)]
            u = np.zeros((slots, Q))
            for s, i in enumerate(slot_req):
                if i is not None:
                    u[s] = uniforms[i, slot_idx[s]]
            codes = engine.step_frame(mask_eos_q0=mask, uniforms=u).view(slots, Q)
            refill = {}
            for s, i in enumerate(slot_req):
                if i is None:
                    continue
                if slot_idx[s] >= min_new_frames and int(codes[s, 0]) == eos:
                    reason[i] = "eos"
                    done = True
                else:
                    frames[i].append(codes[s].clone().view(1, Q))
                    if on_frame is not None:
                        on_frame(i, frames[i][-1])
                    slot_idx[s] += 1
                    done = slot_idx[s] >= max_new_frames
                if done:
                    if next_req < U:
                        refill[s] = item(next_req)
                        slot_req[s], slot_idx[s] = next_req, 0
                        next_req += 1
                    else:
                        slot_req[s] = None
                        engine.retire(s)
            engine.refill(refill)
        out = []
        for i in range(U):
            c = torch.cat(frames[i], dim=0) if frames[i] else torch.empty(0, Q, dtype=torch.long)
            out.append((c, {"stop_reason": reason[i], "num_frames": c.shape[0], "cfg_scale": cfg_scale,
                            "backend": "mi355x", "sampled": sampled, "temperature": temperature}))
        return out

"""Whole-frame decode engine on one MI355X: the counterpart of
``GraphFrameEngine`` (soraku_inference/acceleration/graph_frame.py:23-328).

Differences from the reference engine that a caller can see:

* cond and uncond rows keep separate KV caches with their own lengths and
  RoPE positions (the native semantics of model.py:561-563,611-612) instead
  of left padding one StaticCache (graph_frame.py:126-136);
* sampling draws from explicit uniforms (``step_frame(uniforms=...)``), so a
  run is reproducible from its uniforms alone; ``set_seed`` seeds the
  generator that supplies them when the caller gives none;
* top-k / top-p / temperature / CFG scale are device parameters read on every
  replay, so changing them never re-captures the graph (graph_frame.py:311-324
  re-captures);
* prefill embeds text with the language-token rows of ``embed_text``
  (model.py:326-338) as the native path does.
"""

from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib
from ._lib import check, lib
from .config import DecodeShape, shape_from_model, to_sk_config
from .synthetic import is_matrix, weight_shapes


def _i64(a: np.ndarray):
    return a.ctypes.data_as(C.POINTER(C.c_int64))


class _DeviceScalar:
    """Stand-in for the reference's ``engine.cfg`` device scalar
    (graph_frame.py:68; written with ``fill_`` at fast_generate.py:530)."""

    def __init__(self, engine: "GraphFrameEngine", value: float):
        self._engine = engine
        self.value = float(value)

    def fill_(self, value: float) -> "_DeviceScalar":
        self.value = float(value)
        self._engine._push_sampling()
        return self

    def __float__(self) -> float:
        return self.value


class GraphFrameEngine:
    def __init__(self, model=None, *, device="cuda:0", max_cache_len: int, cfg_scale: float = 1.5,
                 batch: int = 2, state_dict=None, shape: DecodeShape | None = None,
                 language_token_ids=(), bf16: bool = False, max_frames: int | None = None,
                 n_utts: int = 1, kv_bf16: bool = False):
        import torch

        if model is not None:
            shape = shape or shape_from_model(model)
            language_token_ids = tuple(getattr(model.config, "language_token_ids", ()) or ())
            state_dict = model.state_dict()
        if state_dict is None or shape is None:
            raise ValueError("pass a SorakuTTSv2-like model, or state_dict= and shape=")
        if batch not in (1, 2):
            raise ValueError("batch must be 1 (no CFG) or 2 (cond + uncond)")
        self.shape = shape
        self.config = shape
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise ValueError("the MI355X engine runs on a HIP device ('cuda:N')")
        self.batch = batch
        self.n_utts = n_utts
        self.rows = batch * n_utts
        self.max_len = int(max_cache_len)
        self.max_frames = int(max_frames or max_cache_len)
        self.d_model = shape.d_model
        self.Q = shape.n_codebooks
        self.V = shape.audio_vocab
        self.bf16 = bf16
        self.kv_bf16 = kv_bf16
        self.language_token_ids = tuple(language_token_ids)
        self._weights: dict[str, "torch.Tensor"] = {}
        wdt = torch.bfloat16 if bf16 else torch.float32
        keys = weight_shapes(shape)
        with torch.cuda.device(self.device):
            for key, shp in keys.items():
                if key not in state_dict:
                    if key == "trunk.embed_tokens.weight":
                        continue
                    raise KeyError(f"state dict lacks {key}")
                t = state_dict[key]
                if isinstance(t, np.ndarray):
                    t = torch.from_numpy(np.ascontiguousarray(t))
                dt = wdt if is_matrix(key) else torch.float32
                t = t.to(device=self.device, dtype=dt).contiguous()
                if tuple(t.shape) != tuple(shp):
                    raise ValueError(f"{key}: shape {tuple(t.shape)}, expected {shp}")
                self._weights[key] = t
            torch.cuda.synchronize(self.device)
            cfg = to_sk_config(shape, n_utts=n_utts, cfg_rows=batch, max_ctx=self.max_len,
                               max_frames=self.max_frames, bf16=bf16,
                               language_ids=self.language_token_ids, kv_bf16=kv_bf16)
            h = C.c_void_p()
            check(lib().sk_create(C.byref(cfg), None, C.byref(h)))
        self._h = h
        for key, t in self._weights.items():
            shp = (C.c_int64 * t.dim())(*t.shape)
            dt = _lib.SK_BF16 if t.dtype == torch.bfloat16 else _lib.SK_F32
            check(lib().sk_bind_weight(self._h, key.encode(), C.c_void_p(t.data_ptr()), dt, shp, t.dim()))
        self.cfg = _DeviceScalar(self, cfg_scale)
        self.temp = 1.0
        self.temp_q0 = None
        self.sampled = False
        self.top_k: int | None = None
        self.top_p: float | None = None
        self.top_k_q0: int | None = None
        self.top_p_q0: float | None = None
        self.rng = np.random.default_rng()
        self.graph = None
        self._record = False
        self._push_sampling()

    # ------------------------------------------------------------ lifecycle
    def close(self) -> None:
        if getattr(self, "_h", None):
            lib().sk_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ------------------------------------------------------------ params
    def _push_sampling(self) -> None:
        greedy = not self.sampled
        t = 0.0 if greedy else float(self.temp)
        k = int(self.top_k) if self.top_k is not None else 0
        p = float(self.top_p) if self.top_p is not None else 0.0
        has_q0 = any(v is not None for v in (self.temp_q0, self.top_k_q0, self.top_p_q0))
        t0 = t if (self.temp_q0 is None or greedy) else float(self.temp_q0)
        k0 = k if self.top_k_q0 is None else int(self.top_k_q0)
        p0 = p if self.top_p_q0 is None else float(self.top_p_q0)
        check(lib().sk_set_sampling(self._h, float(self.cfg.value) if hasattr(self, "cfg") else 1.0,
                                    t, k, p, int(has_q0), t0, k0, p0))

    def set_temperature(self, value: float, *, q0: float | None = None) -> None:
        """graph_frame.py:307-309."""
        self.temp = float(value)
        self.temp_q0 = None if q0 is None else float(q0)
        self._push_sampling()

    def set_sampling(self, *, sampled: bool, top_k: int | None, top_p: float | None,
                     top_k_q0: int | None = None, top_p_q0: float | None = None) -> None:
        """graph_frame.py:311-324 (no re-capture needed here)."""
        self.sampled = bool(sampled)
        self.top_k, self.top_p = top_k, top_p
        self.top_k_q0, self.top_p_q0 = top_k_q0, top_p_q0
        self._push_sampling()

    def set_seed(self, seed: int | None) -> None:
        """graph_frame.py:326-328: seeds the source of the per-step uniforms."""
        if seed is not None:
            self.rng = np.random.default_rng(int(seed))

    def set_debug(self, record_logits: bool) -> None:
        self._record = bool(record_logits)
        check(lib().sk_set_debug(self._h, int(self._record)))

    # ------------------------------------------------------------ prefill
    def _frames(self, prompt_codes) -> np.ndarray:
        bos = np.full((1, self.Q), self.shape.bos_id, np.int64)
        if prompt_codes is None:
            return bos
        p = np.asarray(prompt_codes.cpu() if hasattr(prompt_codes, "cpu") else prompt_codes, np.int64)
        if p.size == 0:
            return bos
        return np.concatenate((bos, p.reshape(-1, self.Q)), 0)

    def prefill(self, cond_ids, uncond_ids=None, prompt_codes=None):
        """[text, BOS frame, prompt frames] per row (model.py:623-656); returns
        the depth-input hidden ``[rows, d]`` like graph_frame.py:118-198.
        With several utterances, every utterance gets this prefix."""
        return self.prefill_utterances([(cond_ids, uncond_ids, prompt_codes)] * self.n_utts)

    def _stage(self, u, cond_ids, uncond_ids, prompt_codes):
        """Stage utterance slot ``u``'s rows (cond, and uncond with CFG)."""
        def ids_of(x):
            return np.asarray(x.cpu() if hasattr(x, "cpu") else x, np.int64).reshape(-1)

        cond = ids_of(cond_ids)
        rows = [cond]
        if self.batch == 2:
            uncond = ids_of(uncond_ids) if uncond_ids is not None else cond
            if uncond.size > cond.size:
                raise ValueError("uncond text is longer than cond")
            rows.append(uncond)
        frames = self._frames(prompt_codes)
        for b, ids in enumerate(rows):
            n = ids.size + frames.shape[0]
            if n > self.max_len:
                raise ValueError(f"prefill {n} exceeds max_cache_len={self.max_len}")
            check(lib().sk_prefill_row(self._h, u * self.batch + b, _i64(ids), ids.size,
                                       _i64(np.ascontiguousarray(frames)), frames.shape[0]))

    def prefill_utterances(self, items):
        """Several utterances, each with its own prefix: ``items`` holds
        ``(cond_ids, uncond_ids, prompt_codes)`` per utterance (ragged lengths
        are fine; each row keeps its own length and positions).  Returns the
        depth-input hidden ``[rows, d]``."""
        import torch

        if len(items) != self.n_utts:
            raise ValueError(f"{len(items)} prefixes for {self.n_utts} utterances")
        for u, (cond_ids, uncond_ids, prompt_codes) in enumerate(items):
            self._stage(u, cond_ids, uncond_ids, prompt_codes)
        check(lib().sk_prefill_run(self._h))
        return torch.from_numpy(self.hidden()).to(self.device)

    # ---- continuous batching (no reference counterpart beyond one CFG pair) ----
    def refill(self, items: dict) -> None:
        """Between frames, give utterance slots new utterances: ``items`` maps
        slot -> ``(cond_ids, uncond_ids, prompt_codes)``.  Only those slots'
        rows are prefilled; every other slot keeps decoding where it was."""
        if not items:
            return
        for u, (cond_ids, uncond_ids, prompt_codes) in items.items():
            if not 0 <= u < self.n_utts:
                raise ValueError(f"slot {u} outside [0, {self.n_utts})")
            self._stage(u, cond_ids, uncond_ids, prompt_codes)
        check(lib().sk_prefill_refill(self._h))

    def retire(self, u: int) -> None:
        """Stop decoding utterance slot ``u`` (its rows no longer advance)."""
        if not 0 <= u < self.n_utts:
            raise ValueError(f"slot {u} outside [0, {self.n_utts})")
        for b in range(self.batch):
            check(lib().sk_retire_row(self._h, u * self.batch + b))

    def reset_frames(self) -> None:
        """Restart the frame ring (codes of earlier frames become unreadable)."""
        check(lib().sk_reset_frames(self._h))

    def eos_mask_bits(self, mask) -> int:
        """EOS-at-q0 mask as the engine's per-utterance bits: a bool applies to
        every utterance, a sequence of n_utts bools gives one per utterance."""
        if np.ndim(mask) == 0:
            bits = (1 << self.n_utts) - 1 if bool(mask) else 0
        else:
            m = np.asarray(mask, bool).reshape(-1)
            if m.size != self.n_utts:
                raise ValueError(f"EOS mask of {m.size} utterances for {self.n_utts}")
            bits = sum(1 << i for i in range(self.n_utts) if m[i])
        return int(np.array(bits, np.uint32).view(np.int32))

    def hidden(self) -> np.ndarray:
        out = np.empty((self.rows, self.d_model), np.float32)
        check(lib().sk_get_hidden(self._h, out.ctypes.data_as(C.POINTER(C.c_float))))
        return out

    # ------------------------------------------------------------ capture / replay
    def capture(self, warmup: int = 3) -> None:
        """graph_frame.py:274-296.  Stream capture records without executing,
        so no warm-up frames and no state restore are needed."""
        check(lib().sk_capture(self._h))
        self.graph = True

    def step_frame(self, *, mask_eos_q0, uniforms=None, forced_codes=None,
                   return_logits: bool = False):
        """One replay; returns this frame's codes as a CPU LongTensor ``[Q]``
        (``[n_utts, Q]`` for several utterances), graph_frame.py:298-305.
        ``mask_eos_q0``: a bool (every utterance) or one bool per utterance."""
        import torch

        if self.graph is None:
            raise RuntimeError("call capture() first")
        nq = self.n_utts * self.Q
        if uniforms is None:
            uniforms = self.rng.random(nq) if self.sampled else np.zeros(nq)
        u = np.ascontiguousarray(np.asarray(uniforms, np.float64).reshape(nq))
        fc = None
        if forced_codes is not None:
            fc = np.ascontiguousarray(np.asarray(forced_codes, np.int64).reshape(nq))
        codes = np.empty(nq, np.int64)
        logits = np.empty((self.n_utts, self.Q, self.V), np.float32) if return_logits else None
        check(lib().sk_step_frame(
            self._h, self.eos_mask_bits(mask_eos_q0), u.ctypes.data_as(C.POINTER(C.c_double)),
            _i64(fc) if fc is not None else None, _i64(codes),
            logits.ctypes.data_as(C.POINTER(C.c_float)) if logits is not None else None))
        out = torch.from_numpy(codes.reshape(self.n_utts, self.Q))
        if self.n_utts == 1:
            out = out[0]
        return (out, logits) if return_logits else out

    # ---- throughput path: many frames without host synchronisation -------
    def queue_frames(self, uniforms: np.ndarray, mask_eos_q0: np.ndarray) -> None:
        """``mask_eos_q0``: ``[n]`` (one flag per frame, for every utterance)
        or ``[n, n_utts]`` (per utterance)."""
        mk = np.asarray(mask_eos_q0)
        if mk.ndim == 2:
            bits = [self.eos_mask_bits(row) for row in mk]
        else:
            bits = [self.eos_mask_bits(bool(x)) for x in mk.reshape(-1)]
        n = len(bits)
        u = np.ascontiguousarray(np.asarray(uniforms, np.float64).reshape(n, self.n_utts * self.Q))
        m = np.ascontiguousarray(np.array(bits, np.int32))
        check(lib().sk_queue_frames(self._h, n, u.ctypes.data_as(C.POINTER(C.c_double)),
                                    m.ctypes.data_as(C.POINTER(C.c_int32))))

    def replay(self, n: int) -> None:
        check(lib().sk_replay(self._h, int(n)))

    def read_codes(self, n: int) -> np.ndarray:
        out = np.empty((n, self.n_utts, self.Q), np.int64)
        check(lib().sk_read_codes(self._h, int(n), _i64(out)))
        return out

    def synchronize(self) -> None:
        check(lib().sk_synchronize(self._h))

    @property
    def stream_handle(self) -> int:
        return int(lib().sk_stream(self._h) or 0)

    @property
    def frames_done(self) -> int:
        return int(lib().sk_frames_done(self._h))

    @property
    def xcd_layers(self) -> bool:
        """True when the trunk runs as XCD-resident layers (two launches per layer)."""
        return int(lib().sk_xcd_layers(self._h)) == 1

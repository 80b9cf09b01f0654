"""Operator API with the factory shape of the reference's TileLang kernels
(soraku_inference/acceleration/tilelang_kernels.py:34-254): ``factory(*shape)``
returns ``kernel(*inputs) -> out`` with the output allocated
(``out_idx=[-1]``).  Inputs are contiguous torch tensors on the HIP device;
matrices may be float32 or bfloat16 (FP32 accumulation).  Masking writes -inf
as the native path does (model.py:582-584), not -1e30 (tilelang_kernels.py:31).
"""

from __future__ import annotations

import ctypes as C

from . import _lib
from ._lib import check, lib


def _ptr(t) -> C.c_void_p:
    if not t.is_cuda:
        raise ValueError("operands must live on the HIP device")
    if not t.is_contiguous():
        raise ValueError("operands must be contiguous (fast_generate.py:94-97)")
    return C.c_void_p(t.data_ptr())


def _stream(t) -> C.c_void_p:
    import torch

    return C.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _wdtype(t) -> int:
    import torch

    if t.dtype == torch.float32:
        return _lib.SK_F32
    if t.dtype == torch.bfloat16:
        return _lib.SK_BF16
    raise ValueError(f"matrix dtype {t.dtype} not supported (float32 or bfloat16)")


def _empty(ref, *shape):
    import torch

    return torch.empty(*shape, device=ref.device, dtype=torch.float32)


def add_rmsnorm(B: int, D: int, eps: float):
    """out = rmsnorm(hidden + prefix) * w (tilelang_kernels.py:34-55)."""
    def kernel(hidden, prefix, weight):
        out = _empty(hidden, B, D)
        check(lib().sk_op_add_rmsnorm(_stream(hidden), B, D, eps, _ptr(hidden), _ptr(prefix),
                                      _ptr(weight), _ptr(out)))
        return out
    return kernel


def rmsnorm(B: int, D: int, eps: float):
    """tilelang_kernels.py:58-78."""
    def kernel(x, weight):
        out = _empty(x, B, D)
        check(lib().sk_op_rmsnorm(_stream(x), B, D, eps, _ptr(x), _ptr(weight), _ptr(out)))
        return out
    return kernel


def swiglu_gemv(B: int, I: int, D: int):
    """act = silu(x Wg^T) * (x Wu^T) (tilelang_kernels.py:81-112)."""
    def kernel(x, wg, wu):
        if wg.dtype != wu.dtype:
            raise ValueError("gate and up must share a dtype")
        out = _empty(x, B, I)
        check(lib().sk_op_swiglu_gemv(_stream(x), B, I, D, _wdtype(wg), _ptr(x), _ptr(wg), _ptr(wu),
                                      _ptr(out)))
        return out
    return kernel


def down_residual_gemv(B: int, D: int, I: int):
    """y = act Wd^T + residual (tilelang_kernels.py:115-143)."""
    def kernel(act, wd, residual):
        out = _empty(act, B, D)
        check(lib().sk_op_down_residual_gemv(_stream(act), B, D, I, _wdtype(wd), _ptr(act), _ptr(wd),
                                             _ptr(residual), _ptr(out)))
        return out
    return kernel


def classifier_gemv(B: int, V: int, D: int):
    """logits = body Wq^T + bias (tilelang_kernels.py:146-173)."""
    def kernel(body, wq, bias):
        out = _empty(body, B, V)
        check(lib().sk_op_classifier_gemv(_stream(body), B, V, D, _wdtype(wq), _ptr(body), _ptr(wq),
                                          _ptr(bias), _ptr(out)))
        return out
    return kernel


def frame_embed(R: int, Q: int, V: int, D: int, scale: float):
    """out[r] = scale * sum_q table[q, codes[r, q]] (tilelang_kernels.py:176-196)."""
    def kernel(codes, table):
        out = _empty(table, R, D)
        check(lib().sk_op_frame_embed(_stream(table), R, Q, V, D, scale, _ptr(codes), _ptr(table),
                                      _ptr(out)))
        return out
    return kernel


def prefix_add(B: int, V: int, D: int, scale: float):
    """out = prefix + table_q[code] * scale (tilelang_kernels.py:199-216)."""
    def kernel(prefix, table_q, code):
        out = _empty(prefix, B, D)
        check(lib().sk_op_prefix_add(_stream(prefix), B, V, D, scale, _ptr(prefix), _ptr(table_q),
                                     _ptr(code), _ptr(out)))
        return out
    return kernel


def sampling_prep(V: int, bos_id: int, pad_id: int, eos_id: int):
    """out = logits / T with BOS/PAD (and EOS if flagged) masked
    (tilelang_kernels.py:219-254)."""
    def kernel(logits, temperature, mask_eos):
        out = _empty(logits, V)
        check(lib().sk_op_sampling_prep(_stream(logits), V, bos_id, pad_id, eos_id, _ptr(logits),
                                        _ptr(temperature), _ptr(mask_eos), _ptr(out)))
        return out
    return kernel


def sample(V: int, bos_id: int, eos_id: int, pad_id: int):
    """Fused CFG + masks + temperature + top-k/top-p + explicit-uniform draw
    (model.py:579-595,686-708); ``kernel(logits[rows, V], ...) -> int64[1]``."""
    def kernel(logits, *, cfg_scale: float, q: int, mask_eos_q0: bool, temperature: float,
               top_k, top_p, u: float):
        import torch

        rows = logits.shape[0]
        out = torch.empty(1, device=logits.device, dtype=torch.int64)
        check(lib().sk_op_sample(_stream(logits), rows, V, _ptr(logits), float(cfg_scale), int(q),
                                 int(bool(mask_eos_q0)), bos_id, eos_id, pad_id, float(temperature),
                                 int(top_k or 0), float(top_p or 0.0), float(u), _ptr(out)))
        return out
    return kernel

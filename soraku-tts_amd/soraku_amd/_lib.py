"""ctypes binding of libsoraku_mi355x.so (the C ABI in include/soraku_mi355x.h).

The library is loaded from this package directory.  There is no fallback: if
it is missing, importing fails with instructions to build it.
"""

from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libsoraku_mi355x.so")

SK_OK, SK_EINVAL, SK_ENOWEIGHT, SK_ENOCAPTURE, SK_EKVFULL, SK_EHIP, SK_ESTATE = 0, -1, -2, -3, -4, -5, -6
SK_F32, SK_BF16 = 0, 1

ERROR_NAMES = {
    SK_EINVAL: "SK_EINVAL", SK_ENOWEIGHT: "SK_ENOWEIGHT", SK_ENOCAPTURE: "SK_ENOCAPTURE",
    SK_EKVFULL: "SK_EKVFULL", SK_EHIP: "SK_EHIP", SK_ESTATE: "SK_ESTATE",
}


class SkConfig(C.Structure):
    _fields_ = [
        ("d_model", C.c_int32), ("n_layers", C.c_int32), ("n_q_heads", C.c_int32),
        ("n_kv_heads", C.c_int32), ("head_dim", C.c_int32), ("trunk_inter", C.c_int32),
        ("depth_inner", C.c_int32), ("n_codebooks", C.c_int32), ("audio_vocab", C.c_int32),
        ("text_vocab", C.c_int32), ("bos_id", C.c_int32), ("eos_id", C.c_int32),
        ("pad_id", C.c_int32), ("trunk_eps", C.c_float), ("depth_eps", C.c_float),
        ("rope_theta", C.c_float), ("frame_scale", C.c_float), ("weight_dtype", C.c_int32),
        ("n_utts", C.c_int32), ("cfg_rows", C.c_int32), ("max_ctx", C.c_int32),
        ("max_frames", C.c_int32), ("n_language", C.c_int32), ("language_ids", C.c_int32 * 4),
        ("kv_dtype", C.c_int32),
    ]


class SkError(RuntimeError):
    """A non-zero status from the C ABI."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"{ERROR_NAMES.get(code, code)}: {msg}")
        self.code = code


_P = C.c_void_p
_I = C.c_int32
_F = C.c_float
_D = C.c_double
_PI64 = C.POINTER(C.c_int64)
_PI32 = C.POINTER(C.c_int32)
_PF = C.POINTER(C.c_float)
_PD = C.POINTER(C.c_double)

# name -> (restype, argtypes); keep in the order of include/soraku_mi355x.h.
PROTOTYPES = {
    "sk_last_error": (C.c_char_p, []),
    "sk_create": (_I, [C.POINTER(SkConfig), _P, C.POINTER(_P)]),
    "sk_destroy": (_I, [_P]),
    "sk_bind_weight": (_I, [_P, C.c_char_p, _P, _I, _PI64, _I]),
    "sk_prefill_row": (_I, [_P, _I, _PI64, _I, _PI64, _I]),
    "sk_prefill_run": (_I, [_P]),
    "sk_prefill_run_noalloc": (_I, [_P]),
    "sk_prefill_refill": (_I, [_P]),
    "sk_retire_row": (_I, [_P, _I]),
    "sk_reset_frames": (_I, [_P]),
    "sk_set_row_state": (_I, [_P, _I, _I, _I]),
    "sk_kv_ptr": (_I, [_P, _I, _I, C.POINTER(_P)]),
    "sk_get_hidden": (_I, [_P, _PF]),
    "sk_set_sampling": (_I, [_P, _F, _F, _I, _F, _I, _F, _I, _F]),
    "sk_set_debug": (_I, [_P, _I]),
    "sk_capture": (_I, [_P]),
    "sk_step_frame": (_I, [_P, _I, _PD, _PI64, _PI64, _PF]),
    "sk_queue_frames": (_I, [_P, _I, _PD, _PI32]),
    "sk_replay": (_I, [_P, _I]),
    "sk_read_codes": (_I, [_P, _I, _PI64]),
    "sk_synchronize": (_I, [_P]),
    "sk_stream": (_P, [_P]),
    "sk_frames_done": (_I, [_P]),
    "sk_xcd_layers": (_I, [_P]),
    "sk_debug_set_spin_ticks": (_I, [_P, C.c_uint64]),
    "sk_op_add_rmsnorm": (_I, [_P, _I, _I, _F, _P, _P, _P, _P]),
    "sk_op_rmsnorm": (_I, [_P, _I, _I, _F, _P, _P, _P]),
    "sk_op_swiglu_gemv": (_I, [_P, _I, _I, _I, _I, _P, _P, _P, _P]),
    "sk_op_down_residual_gemv": (_I, [_P, _I, _I, _I, _I, _P, _P, _P, _P]),
    "sk_op_classifier_gemv": (_I, [_P, _I, _I, _I, _I, _P, _P, _P, _P]),
    "sk_op_frame_embed": (_I, [_P, _I, _I, _I, _I, _F, _P, _P, _P]),
    "sk_op_prefix_add": (_I, [_P, _I, _I, _I, _F, _P, _P, _P, _P]),
    "sk_op_sampling_prep": (_I, [_P, _I, _I, _I, _I, _P, _P, _P, _P]),
    "sk_op_sample": (_I, [_P, _I, _I, _P, _F, _I, _I, _I, _I, _I, _F, _I, _F, _D, _P]),
}


def load(path: str = LIB_PATH) -> C.CDLL:
    if not os.path.exists(path):
        raise ImportError(
            f"{path} is missing: build the HIP library first "
            "(python soraku-tts_amd/build.py, or __graft_entry__.build())")
    lib = C.CDLL(path)
    for name, (res, args) in PROTOTYPES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


_LIB: C.CDLL | None = None


def lib() -> C.CDLL:
    global _LIB
    if _LIB is None:
        _LIB = load()
    return _LIB


def check(rc: int) -> None:
    if rc != SK_OK:
        raise SkError(rc, lib().sk_last_error().decode(errors="replace"))

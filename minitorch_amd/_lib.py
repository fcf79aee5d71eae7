"""ctypes binding of libmtx_hip.so (the C ABI declared in include/mtx.h).

This module is the only place that touches the shared library.  It loads the
in-tree build (``minitorch_amd/libmtx_hip.so``), declares every exported
signature, turns non-zero status codes into Python exceptions and converts
device arrays into pointers, element strides and the current HIP stream.

There is no fallback: if the library is missing or a call fails, an exception
is raised.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

_PKG = Path(__file__).resolve().parent
LIB_PATH = _PKG / "libmtx_hip.so"

MTX_OK, MTX_ERR_ARG, MTX_ERR_SHAPE, MTX_ERR_DTYPE, MTX_ERR_HIP = range(5)
MTX_F32, MTX_BF16 = 0, 1
MTX_GEMM_FP32, MTX_GEMM_BF16X3 = 0, 1
ATTN_SCRATCH_BYTES = 8 << 20  # MTX_ATTN_SCRATCH_BYTES (include/mtx.h)
ATTN_BWD_DELTA, ATTN_BWD_DKDV, ATTN_BWD_DQ, ATTN_BWD_ALL = 1, 2, 4, 7
ATTN_BWD_TWOPASS, ATTN_BWD_ONEPASS = 0, 8  # mtx_attn_set_bwd_mode; ONEPASS is also a phase bit

_P = C.c_void_p
_I = C.c_int
_I64P = C.POINTER(C.c_int64)
_F = C.c_float
_SZ = C.c_size_t
_I64 = C.c_int64
_IP = C.POINTER(C.c_int)
_D = C.c_double

EW = dict(COPY=0, ADD=1, SUB=2, MUL=3, DIV=4, POW=5, AXPBY=6, SCALE_SHIFT=7, EXP=8, LOG=9, TANH=10,
          NEG=11, RECIP_CLAMP=12, TANH_GRAD=13, SQUARE=14, SQRT=15, FILL=16, MAXIMUM=17, EQ=18, GT=19,
          ABS=20, SIGN=21)
RED_SUM, RED_MAX = 0, 1



class DecodeLayer(C.Structure):
    """mtx_decode_layer (include/mtx.h): one block's weights and caches."""
    _fields_ = [(n, _P) for n in ("ln1_gamma", "ln1_beta", "w_qkv", "b_qkv", "w_out", "b_out", "ln2_gamma",
                                  "ln2_beta", "w_fc1", "b_fc1", "w_fc2", "b_fc2", "k_cache", "v_cache")] + [
        ("ln1_eps", _F), ("ln2_eps", _F)]


class DecodeModel(C.Structure):
    """mtx_decode_model (include/mtx.h): the model a persistent decode step runs."""
    _fields_ = [("n_layer", _I), ("B", _I), ("C", _I), ("n_head", _I), ("F", _I), ("V", _I), ("Tmax", _I),
                ("tok_emb", _P), ("n_tok", _I64), ("pos_emb", _P), ("n_pos", _I64),
                ("layers", C.POINTER(DecodeLayer)), ("lnf_gamma", _P), ("lnf_beta", _P), ("lnf_eps", _F),
                ("w_head", _P), ("b_head", _P)]


# name -> (restype, argtypes); mirrors include/mtx.h
SIGNATURES = {
    "mtx_last_error": (C.c_char_p, []),
    "mtx_version": (C.c_char_p, []),
    "mtx_attn_fwd": (_I, [_I, _I, _I, _I, _I, _I,
                          _P, _I64P, _P, _I64P, _P, _I64P, _P, _I64P,
                          _P, _F, _I, _P]),
    "mtx_attn_bwd_workspace_bytes": (_SZ, [_I, _I, _I]),
    "mtx_attn_bwd": (_I, [_I, _I, _I, _I, _I, _I,
                          _P, _I64P, _P, _I64P, _P, _I64P, _P, _I64P, _P, _I64P,
                          _P,
                          _P, _I64P, _P, _I64P, _P, _I64P,
                          _P, _SZ, _F, _I, _I, _P]),
    "mtx_attn_bwd_phase": (_I, [_I, _I, _I, _I, _I, _I, _I,
                                _P, _I64P, _P, _I64P, _P, _I64P, _P, _I64P, _P, _I64P,
                                _P,
                                _P, _I64P, _P, _I64P, _P, _I64P,
                                _P, _SZ, _F, _I, _I, _P]),
    "mtx_attn_bwd_noalloc": (_I, [_I, _I, _I, _I, _I, _I,
                                  _P, _I64P, _P, _I64P, _P, _I64P, _P, _I64P, _P, _I64P,
                                  _P,
                                  _P, _I64P, _P, _I64P, _P, _I64P,
                                  _F, _I, _I, _P]),
    "mtx_attn_fwd_dropout": (_I, [_I, _I, _I, _I, _I, _I,
                                  _P, _I64P, _P, _I64P, _P, _I64P, _P, _I64P,
                                  _P, _F, _I, _P, _I64, _F, _P]),
    "mtx_attn_bwd_dropout": (_I, [_I, _I, _I, _I, _I, _I,
                                  _P, _I64P, _P, _I64P, _P, _I64P, _P, _I64P, _P, _I64P,
                                  _P,
                                  _P, _I64P, _P, _I64P, _P, _I64P,
                                  _P, _SZ, _F, _I, _I, _P, _I64, _F, _P]),
    "mtx_dropout_keep_philox": (_I, [_P, _I64, _I, _I64, _F, C.c_uint64, C.c_uint64, _P]),
    "mtx_pack3_f32": (_I, [_P, _P, _P, _I64, _I64, _P, _P]),
    "mtx_unpack3_f32": (_I, [_P, _I64, _I64, _P, _P, _P, _I, _P]),
    "mtx_attn_decode": (_I, [_I, _I, _I, _I, _I,
                             _P, _I64P, _P, _I64P, _P, _I64P, _P, _I64P,
                             _P, _P, _F, _P]),
    "mtx_argmax_f32": (_I, [_I, _I, _P, _I64, _P, _I64, _P, _I64, _P]),
    "mtx_kv_append_f32": (_I, [_I, _I, _I, _P, _I64, _P, _I64, _I64, _P, _P]),
    "mtx_decode_advance": (_I, [_I, _P, _P, _P]),
    "mtx_decode_step_workspace_bytes": (_SZ, [_I, _I, _I, _I]),
    "mtx_decode_step_f32": (_I, [_P, _I, _P, _P, _P, _I, _I, _P, _P, _P, _SZ, _I64, _P]),
    "mtx_decode_step_status": (_I, [_P, _P]),
    "mtx_decode_step_reset": (_I, [_P, _P]),
    "mtx_greedy_pick_f32": (_I, [_I, _I, _P, _I64, _P, _P, _I, _P, _I, _I, _P, _P, _P]),
    "mtx_embedding2_ln_fwd_f32": (_I, [_P, _I64, _I64, _P, _P, _I64, _I64, _P, _I64, _P, _I64, _I64, _I,
                                       _P, _P, _F, _P, _I64, _P]),
    "mtx_head_pick_f32": (_I, [_I, _I, _I, _P, _I64, _P, _I, _P, _P, _P, _F, _P, _I64, _P, _P, _P, _I, _P, _I,
                               _I, _P, _P, _P]),
    "mtx_decode_qkv_attn_f32": (_I, [_I, _I, _I, _P, _I64, _P, _I, _P, _P, _I64, _P, _P, _F, _P, _I64, _P, _P,
                                     _P, _I64, _I64, _I, _P, _F, _P, _I64, _P]),
    "mtx_gemm_partials_f32": (_I, [_I, _I, _I, _P, _I64, _I64, _P, _I64, _I64, _P, _SZ, _P, _P]),
    "mtx_embedding2_fwd_f32": (_I, [_P, _I64, _I64, _P, _P, _I64, _I64, _P, _I64, _P, _I64, _I64, _I, _P]),
    "mtx_gemm_workspace_bytes": (_SZ, [_I, _I, _I, _I]),
    "mtx_gemm_set_mode": (_I, [_I]),
    "mtx_attn_set_mode": (_I, [_I]),
    "mtx_attn_get_mode": (_I, []),
    "mtx_attn_set_bwd_mode": (_I, [_I]),
    "mtx_attn_get_bwd_mode": (_I, []),
    "mtx_gemm_get_mode": (_I, []),
    "mtx_gemm_step_f32": (_I, [_I, _I, _I, _P, _I64, _P, _I64, _F, _P, _I64, _P, _I, _I,
                               _P, _P, _I64, _I64, _I, _P, _P]),
    "mtx_gemm_f32": (_I, [_I, _I, _I, _I,
                          _F, _P, _I64, _I64, _I64,
                          _P, _I64, _I64, _I64,
                          _F, _P, _I64, _I64, _I64,
                          _P, _P, _SZ, _P]),
    "mtx_gemm_wgrad_f32": (_I, [_I, _I, _I, _P, _I64, _I64, _P, _I64, _I64, _F, _P, _I64, _I64,
                                _P, _I, _P, _SZ, _P]),
    "mtx_gemm_ln_workspace_bytes": (_SZ, [_I, _I, _I]),
    "mtx_gemm_ln_f32": (_I, [_I, _I, _I, _F, _P, _I64, _I64, _P, _I64, _I64, _F, _P, _I64,
                             _P, _P, _P, _F, _P, _I64, _P, _SZ, _P]),
    "mtx_gemm_act_f32": (_I, [_I, _I, _I, _I,
                              _F, _P, _I64, _I64, _I64,
                              _P, _I64, _I64, _I64,
                              _F, _P, _I64, _I64, _I64,
                              _P, _I, _P, _I64, _I64, _I64, _P, _SZ, _P]),
    "mtx_ewise_f32": (_I, [_I, _I, _I64P, _P, _I64P, _P, _I64P, _P, _I64P, _F, _F, _I, _P]),
    "mtx_reduce_workspace_bytes": (_SZ, [_I, _I64P, _IP]),
    "mtx_reduce_f32": (_I, [_I, _I, _I64P, _P, _I64P, _IP, _P, _F, _I, _P, _SZ, _P]),
    "mtx_softmax_fwd_f32": (_I, [_P, _I64, _P, _I64, _I64, _I, _I, _I, _P]),
    "mtx_softmax_bwd_f32": (_I, [_P, _I64, _P, _I64, _P, _I64, _I64, _I, _I, _I, _P]),
    "mtx_layernorm_fwd_f32": (_I, [_P, _I64, _P, _P, _P, _I64, _P, _P, _I64, _I, _F, _P]),
    "mtx_layernorm_bwd_workspace_bytes": (_SZ, [_I64, _I]),
    "mtx_layernorm_bwd_f32": (_I, [_P, _I64, _P, _P, _P, _P, _I64, _P, _I64, _P, _I64, _P, _P, _I64, _I,
                                   _I, _P, _SZ, _P]),
    "mtx_gelu_fwd_f32": (_I, [_P, _P, _I64, _P]),
    "mtx_gelu_bwd_f32": (_I, [_P, _P, _P, _I64, _I, _P]),
    "mtx_xent_fwd_f32": (_I, [_P, _I64, _P, _P, _P, _I64, _I, _P]),
    "mtx_xent_bwd_f32": (_I, [_P, _I64, _P, _P, _P, _F, _P, _I64, _I64, _I, _I, _P]),
    "mtx_embedding_fwd_f32": (_I, [_P, _I64, _I64, _P, _I64, _P, _I64, _I, _P]),
    "mtx_embedding_bwd_f32": (_I, [_P, _I64, _P, _I64, _P, _I64, _I64, _I, _I, _P]),
    "mtx_adam_blocks": (_I, [_I64P, _I, _I64P, _I64P]),
    "mtx_onehot_f32": (_I, [_P, _I64, _I64, _P, _P]),
    "mtx_adam_f32": (_I, [_P, _I, _I64, _D, _D, _D, _D, _D, _I, _P]),
    "mtx_adam_bias_table": (_I, [_D, _D, _I, _I, _P]),
    "mtx_adam_dev_f32": (_I, [_P, _I, _I64, _D, _D, _D, _D, _D, _P, _P, _I, _P]),
    "mtx_zero_grads_f32": (_I, [_P, _I, _I64, _P]),
    # runtime
    "mtx_device_count": (_I, [_IP]),
    "mtx_device_init": (_I, [_I]),
    "mtx_device_sync": (_I, []),
    "mtx_malloc": (_I, [C.POINTER(_P), _SZ]),
    "mtx_free": (_I, [_P]),
    "mtx_empty_cache": (_I, []),
    "mtx_memory_stats": (_I, [C.POINTER(_SZ), C.POINTER(_SZ)]),
    "mtx_memcpy_h2d": (_I, [_P, _P, _SZ, _P]),
    "mtx_memcpy_d2h": (_I, [_P, _P, _SZ, _P]),
    "mtx_memcpy_d2d": (_I, [_P, _P, _SZ, _P]),
    "mtx_fill": (_I, [_P, _SZ, C.c_uint64, _I, _P]),
    "mtx_stream_create": (_I, [C.POINTER(_P)]),
    "mtx_stream_destroy": (_I, [_P]),
    "mtx_stream_sync": (_I, [_P]),
    "mtx_event_create": (_I, [C.POINTER(_P)]),
    "mtx_event_destroy": (_I, [_P]),
    "mtx_event_record": (_I, [_P, _P]),
    "mtx_event_elapsed_ms": (_I, [_P, _P, C.POINTER(_F)]),
    "mtx_stream_wait_event": (_I, [_P, _P]),
    "mtx_graph_begin": (_I, [_P]),
    "mtx_graph_end": (_I, [_P, C.POINTER(_P)]),
    "mtx_graph_launch": (_I, [_P, _P]),
    "mtx_graph_destroy": (_I, [_P]),
}


class MtxError(RuntimeError):
    """A libmtx_hip call returned a non-zero status."""

    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn} failed (status {code}): {msg}")
        self.code = code


_lib = None


def lib():
    """Load (once) and return the CDLL with all signatures declared."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ImportError(
                f"{LIB_PATH} is not built; run `python -m minitorch_amd.build` "
                "(minitorch_amd has no CPU fallback)")
        handle = C.CDLL(str(LIB_PATH), mode=os.RTLD_NOW | os.RTLD_LOCAL)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def exported_symbols():
    return list(SIGNATURES)


def check(fn_name: str, status: int) -> None:
    if status != MTX_OK:
        msg = lib().mtx_last_error().decode(errors="replace")
        if status in (MTX_ERR_ARG, MTX_ERR_SHAPE, MTX_ERR_DTYPE):
            raise ValueError(f"{fn_name}: {msg}")
        raise MtxError(fn_name, status, msg)


def call(fn_name: str, *args) -> None:
    check(fn_name, getattr(lib(), fn_name)(*args))


# ---------------------------------------------------------------------------
# argument helpers: device arrays (minitorch_amd.device.DevBuf, or any object
# with data_ptr() / stride() / dtype, e.g. a framework tensor a test passes
# in) -> pointers, element strides, dtype codes; the current stream
# ---------------------------------------------------------------------------

# The stream every launch goes to: None = the null stream (eager work);
# graphs.capture() points it at its capture stream while recording.
_STREAM = [None]


def strides(t) -> C.Array:
    s = t.stride()
    return (C.c_int64 * len(s))(*s)


def ptr(t):
    return C.c_void_p(t.data_ptr())


def stream_handle(device=None):
    return _STREAM[0]


def capturing() -> bool:
    """True while a graph capture is recording this process's launches."""
    return _STREAM[0] is not None


def dtype_code(t) -> int:
    from .device import dtype_name

    name = dtype_name(t)
    if name == "float32":
        return MTX_F32
    if name == "bfloat16":
        return MTX_BF16
    raise ValueError(f"unsupported dtype {name} (float32 or bfloat16)")

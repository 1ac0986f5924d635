"""ctypes bindings of liblaya_hip.so (include/laya_hip.h).

The product path has no fallback: if the library is missing or a call fails, an exception is raised.
Status codes map to the exception types the reference throws (ArgumentException → ValueError,
ArgumentOutOfRangeException → IndexError, InvalidDataException → KeyError).
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# The in-tree build; LAYA_HIP_LIBRARY names another build of the same library (e.g. to compare two).
LIB_PATH = os.environ.get("LAYA_HIP_LIBRARY") or os.path.join(HERE, "liblaya_hip.so")

OK, ERR_ARGUMENT, ERR_OUT_OF_RANGE, ERR_MEMORY, ERR_HIP, ERR_NOT_FINITE, ERR_STATE, ERR_MISSING = range(8)


class LayaError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"[{code}] {message}")
        self.code = code


class LayaArgumentError(LayaError, ValueError):
    pass


class LayaOutOfRangeError(LayaError, IndexError):
    pass


class LayaMemoryError(LayaError, MemoryError):
    pass


class LayaMissingError(LayaError, KeyError):
    pass


class LayaNotFiniteError(LayaError, ArithmeticError):
    pass


class LayaStateError(LayaError):
    pass


_ERRORS = {ERR_ARGUMENT: LayaArgumentError, ERR_OUT_OF_RANGE: LayaOutOfRangeError, ERR_MEMORY: LayaMemoryError,
           ERR_MISSING: LayaMissingError, ERR_NOT_FINITE: LayaNotFiniteError, ERR_STATE: LayaStateError}

c_int, c_float, c_double, c_size, c_u64 = ctypes.c_int, ctypes.c_float, ctypes.c_double, ctypes.c_size_t, ctypes.c_uint64
P = ctypes.c_void_p
PP = ctypes.POINTER(ctypes.c_void_p)


class ModelConfigC(ctypes.Structure):
    _fields_ = [("vocab", c_int), ("hidden", c_int), ("intermediate", c_int), ("layers", c_int), ("heads", c_int),
                ("local_attention", c_int), ("global_every", c_int), ("layer_kinds", ctypes.POINTER(c_int)),
                ("theta_global", c_double), ("theta_local", c_double), ("norm_eps", c_float),
                ("norm_bias", c_int), ("attention_bias", c_int), ("mlp_bias", c_int),
                ("head_layers", c_int), ("head_ff", c_int), ("n_act", c_int)]


class BatchC(ctypes.Structure):
    _fields_ = [("n_items", c_int), ("lengths", P), ("tokens", P), ("n_options", P), ("markers", P), ("qtypes", P)]


# name: (restype, argtypes); every int-returning function is a status.
SIGNATURES = {
    "laya_last_error": (ctypes.c_char_p, []),
    "laya_version": (ctypes.c_char_p, []),
    "laya_ctx_create": (c_int, [c_int, PP]),
    "laya_ctx_destroy": (c_int, [P]),
    "laya_ctx_set_memory_cap": (c_int, [P, c_size]),
    "laya_ctx_memory_in_use": (c_int, [P, ctypes.POINTER(c_size)]),
    "laya_ctx_set_matmul_precision": (c_int, [P, c_int]),
    "laya_alloc": (c_int, [P, c_size, PP]),
    "laya_free": (c_int, [P, P]),
    "laya_upload": (c_int, [P, P, P, c_size]),
    "laya_download": (c_int, [P, P, P, c_size]),
    "laya_fill": (c_int, [P, P, c_float, c_size]),
    "laya_sync": (c_int, [P]),
    "laya_timer_begin": (c_int, [P, c_int]),
    "laya_timer_end": (c_int, [P, c_int]),
    "laya_timer_elapsed": (c_int, [P, c_int, ctypes.POINTER(c_float)]),
    "laya_profile_begin": (c_int, [P]),
    "laya_profile_end": (c_int, [P]),
    "laya_profile_count": (c_int, [P, ctypes.POINTER(c_int)]),
    "laya_profile_get": (c_int, [P, c_int, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(c_int),
                                 ctypes.POINTER(c_double), ctypes.POINTER(c_double), ctypes.POINTER(c_double)]),
    "laya_linear_fwd": (c_int, [P, P, c_int, c_int, P, c_int, P, P, P]),
    "laya_linear_bwd": (c_int, [P, P, P, c_int, c_int, c_int, P, P, P, P]),
    "laya_layernorm_fwd": (c_int, [P, P, c_int, c_int, P, P, c_float, P, P, P]),
    "laya_layernorm_bwd": (c_int, [P, P, c_int, c_int, P, c_float, P, P, P, P, P, P]),
    "laya_layernorm_bwd_noalloc": (c_int, [P, P, c_int, c_int, P, c_float, P, P, P, P, P, P]),
    "laya_gelu_fwd": (c_int, [P, P, c_size, P]),
    "laya_gelu_bwd": (c_int, [P, P, P, c_size]),
    "laya_geglu_fwd": (c_int, [P, P, c_int, c_int, P]),
    "laya_geglu_bwd": (c_int, [P, P, P, c_int, c_int, P]),
    "laya_uniform": (c_float, [c_u64, c_u64]),
    "laya_mix": (c_u64, [c_u64, c_u64]),
    "laya_dropout": (c_int, [P, P, c_size, c_float, c_u64]),
    "laya_relu_dropout_fwd": (c_int, [P, P, c_size, c_float, c_u64, P]),
    "laya_relu_dropout_bwd": (c_int, [P, P, P, c_size, c_float, c_u64]),
    "laya_add": (c_int, [P, P, P, c_size]),
    "laya_rotary_create": (c_int, [P, c_int, c_double, c_int, PP]),
    "laya_rotary_destroy": (c_int, [P, P]),
    "laya_rotary_apply": (c_int, [P, P, P, c_int, P, c_int]),
    "laya_segments_create": (c_int, [P, P, P, c_int, PP]),
    "laya_segments_destroy": (c_int, [P, P]),
    "laya_attention_fwd": (c_int, [P, P, P, c_int, c_int, c_float, c_int, P, c_float, c_u64, P, P]),
    "laya_attention_bwd": (c_int, [P, P, P, c_int, c_int, c_float, c_int, P, c_float, c_u64, P, P, P, P]),
    "laya_embedding_fwd": (c_int, [P, P, c_int, P, c_int, c_int, P, P]),
    "laya_embedding_plan": (c_int, [P, c_int, c_int, P, P, P, ctypes.POINTER(c_int)]),
    "laya_embedding_bwd": (c_int, [P, P, P, P, c_int, P, c_int, P]),
    "laya_gather_rows": (c_int, [P, P, P, c_int, c_int, P]),
    "laya_type_embedding_fwd": (c_int, [P, P, P, c_int, c_int, P]),
    "laya_type_embedding_bwd": (c_int, [P, P, P, c_int, c_int, P]),
    "laya_scatter_add_rows": (c_int, [P, P, P, c_int, c_int, P]),
    "laya_softmax_ce_bwd": (c_int, [P, P, P, P, c_int, c_float, c_float, P, P]),
    "laya_rlcd_objective": (c_int, [P, P, P, P, P, c_int, c_int, c_int, c_int, P, c_double, c_double, c_double,
                                    c_double, c_double, P, P]),
    "laya_grad_norm": (c_int, [P, P, c_size, c_double, P, P]),
    "laya_grad_norm_status": (c_int, [P]),
    "laya_adamw": (c_int, [P, P, P, P, P, c_int, P, P, P, c_double, c_double, c_double, c_double, c_int, P, c_int]),
    "laya_amax": (c_int, [P, P, c_size, P]),
    "laya_linear_fwd_w": (c_int, [P, P, c_int, c_int, P, c_int, P, P, P, P, P, P]),
    "laya_linear_bwd_w": (c_int, [P, P, P, c_int, c_int, c_int, P, P, P, P, P, P, P, P]),
    "laya_layernorm_fwd_w": (c_int, [P, P, c_int, c_int, P, P, c_float, P, P, P, P]),
    "laya_layernorm_bwd_w": (c_int, [P, P, c_int, c_int, P, c_float, P, P, P, P, P, P, P]),
    "laya_geglu_fwd_w": (c_int, [P, P, c_int, c_int, P, P]),
    "laya_geglu_bwd_w": (c_int, [P, P, P, c_int, c_int, P, P]),
    "laya_attention_fwd_w": (c_int, [P, P, P, c_int, c_int, c_float, c_int, P, c_float, c_u64, P, P, P, P]),
    "laya_attention_bwd_w": (c_int, [P, P, P, c_int, c_int, c_float, c_int, P, c_float, c_u64, P, P, P, P, P, P,
                                     P]),
    "laya_model_create": (c_int, [P, ctypes.POINTER(ModelConfigC), PP]),
    "laya_model_destroy": (c_int, [P]),
    "laya_model_num_params": (c_int, [P, ctypes.POINTER(c_int)]),
    "laya_model_param_info": (c_int, [P, c_int, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(c_int),
                                      ctypes.POINTER(c_int), ctypes.POINTER(c_size), ctypes.POINTER(c_size),
                                      ctypes.POINTER(c_int)]),
    "laya_model_find_param": (c_int, [P, ctypes.c_char_p, ctypes.POINTER(c_int)]),
    "laya_model_set_param": (c_int, [P, c_int, P]),
    "laya_model_get_param": (c_int, [P, c_int, P]),
    "laya_model_get_grad": (c_int, [P, c_int, P]),
    "laya_model_has_grad": (c_int, [P, c_int, ctypes.POINTER(c_int)]),
    "laya_model_head_activation": (c_int, [P, c_int, c_int, PP, ctypes.POINTER(c_size)]),
    "laya_model_init_random": (c_int, [P, c_u64, c_float]),
    "laya_model_set_trainable_encoder_layers": (c_int, [P, c_int]),
    "laya_model_set_head_dropout": (c_int, [P, c_float]),
    "laya_model_set_layer_checkpointing": (c_int, [P, c_int]),
    "laya_model_layer_checkpointing": (c_int, [P, P, P]),
    "laya_model_set_bf16_copies": (c_int, [P, c_int]),
    "laya_model_set_bf16_weights": (c_int, [P, c_int]),
    "laya_model_get_param_bf16": (c_int, [P, c_int, P]),
    "laya_model_forward": (c_int, [P, ctypes.POINTER(BatchC), c_int, c_u64, P]),
    "laya_model_backward": (c_int, [P, P]),
    "laya_model_backward_fallback": (c_int, [P, ctypes.POINTER(c_int)]),
    "laya_model_readout": (c_int, [P, P, P, P]),
    "laya_model_objective_rlcd": (c_int, [P, P, P, c_int, c_double, c_double, c_double, c_double, c_double, P]),
    "laya_model_backward_from_objective": (c_int, [P]),
    "laya_model_clip_grad_norm": (c_int, [P, c_double, ctypes.POINTER(c_double)]),
    "laya_model_grad_norm_status": (c_int, [P]),
    "laya_model_adamw_step": (c_int, [P, c_double, c_double, c_double, c_double, c_double, c_double]),
    "laya_model_zero_grad": (c_int, [P]),
    "laya_model_train_step": (c_int, [P, ctypes.POINTER(BatchC), P, c_float, c_float, c_u64, c_double, c_double,
                                      c_double, c_double, c_double, c_double, c_double, ctypes.POINTER(c_float)]),
    "laya_model_steps": (c_int, [P, ctypes.POINTER(c_int)]),
    "laya_model_get_moments": (c_int, [P, c_int, P, P]),
    "laya_model_set_moments": (c_int, [P, c_int, P, P]),
    "laya_model_set_steps": (c_int, [P, c_int]),
    "laya_model_stage_batch": (c_int, [P, ctypes.POINTER(BatchC), P, ctypes.POINTER(c_int)]),
    "laya_model_train_step_staged": (c_int, [P, c_int, c_float, c_float, c_u64, c_double, c_double, c_double, c_double,
                                             c_double, c_double, c_double, ctypes.POINTER(c_float)]),
    "laya_model_release_batch": (c_int, [P, c_int]),
}

_lib: Optional[ctypes.CDLL] = None


def lib() -> ctypes.CDLL:
    """The loaded library; raises if it has not been built (there is no CPU fallback)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"liblaya_hip.so is not built ({LIB_PATH}); run `python -m laya_amd.build`")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(rc: int) -> None:
    if rc != OK:
        msg = lib().laya_last_error().decode("utf-8", "replace")
        raise _ERRORS.get(rc, LayaError)(rc, msg)


def ptr(a) -> Optional[int]:
    """Raw pointer of a host numpy array, a DeviceArray, or None."""
    if a is None:
        return None
    if isinstance(a, np.ndarray):
        assert a.flags["C_CONTIGUOUS"], "host arrays passed to the library must be contiguous"
        return a.ctypes.data
    return a.ptr

"""ctypes binding of libnativebit_amd.so (the C ABI in include/nativebit_amd.h).

torch is imported before the library is opened so that the library's
libamdhip64 dependency resolves to the HIP runtime torch already loaded (one
runtime per process: torch's streams and pointers are valid in our calls).

There is no fallback: if the library is missing, or a call returns a non-zero
status, a NativeBitError is raised with the library's own message.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (must be loaded first, see module docstring)

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libnativebit_amd.so")

NB_OK = 0
NB_EINVAL = -1
NB_EUNSUPPORTED = -2
NB_EALIGN = -3
NB_ELAUNCH = -4
NB_ENODEV = -5
STATUS_NAMES = {
    NB_EINVAL: "NB_EINVAL", NB_EUNSUPPORTED: "NB_EUNSUPPORTED",
    NB_EALIGN: "NB_EALIGN", NB_ELAUNCH: "NB_ELAUNCH", NB_ENODEV: "NB_ENODEV",
}

NB_F32 = 0
NB_BF16 = 1
NB_U8 = 2

# nb_x_mode / nb_y_mode of a batched GEMV item
NB_X_BF16 = 0
NB_X_RMSNORM = 1
NB_X_SILU_MUL = 2
NB_Y_STORE = 0
NB_Y_ADD = 1
NB_Y_SILU_PAIRS = 2

ABI_VERSION = 2

# Every symbol include/nativebit_amd.h declares: (name, restype, argtypes).
_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64
SIGNATURES = {
    "nb_abi_version": (_I, []),
    "nb_last_error": (ctypes.c_char_p, []),
    "nb_packed_nbytes": (_L, [_L, _I]),
    "nb_gemv": (_I, [_P, _I, _L, _P, _P, _P, _I, _L, _I, _I, _I, _I, _I, _I, _P]),
    "nb_unpack": (_I, [_P, _P, _L, _I, _P]),
    "nb_pack": (_I, [_P, _P, _L, _I, _P]),
    "nb_dequant": (_I, [_P, _P, _P, _I, _L, _L, _I, _I, _I, _P]),
    "nb_quantize_pack": (_I, [_P, _L, _P, _L, _I, _I, _I, _P, _P]),
    "nb_block_codebooks": (_I, [_P, _L, _I, _I, _P, _P]),
    "nb_linspace01": (_I, [_I, _P]),
    "nb_gemv_batch_table_bytes": (_L, [_I]),
    "nb_gemv_batch_plan": (_I, [_P, _I, _P, _L]),
    "nb_gemv_batched": (_I, [_P, _P, _I, _I, _P]),
    "nb_gemv_batched_sel": (_I, [_P, _P, _I, _I, _P]),
    "nb_stream_layout": (_I, [_P, _P, _I, _I, _P]),
    "nb_gemm_skinny_batched": (_I, [_P, _P, _I, _I, _I, _P]),
    "nb_quad_layout_bytes": (_L, [_I, _I]),
    "nb_quad_layout": (_I, [_P, _P, _I, _I, _P, _P, _P]),
    "nb_gemm_skinny_quad_batched": (_I, [_P, _P, _I, _I, _I, _P]),
    "nb_tile_layout_bytes": (_L, [_I, _I]),
    "nb_tile_layout": (_I, [_P, _P, _I, _I, _P, _P, _P]),
    "nb_gemm_skinny_tile_batched": (_I, [_P, _P, _I, _I, _I, _P]),
    "nb_gemm_prefill": (_I, [_P, _L, _P, _P, _P, _I, _L, _I, _I, _I, _P]),
    "nb_gemm_prefill_split_ws_bytes": (_L, [_I, _I, _I]),
    "nb_gemm_prefill_split": (_I, [_P, _L, _P, _P, _P, _I, _L, _I, _I, _I, _P, _L, _P]),
    "nb_gemm_prefill_f32_ws_bytes": (_L, [_I, _I, _I]),
    "nb_gemm_prefill_f32": (_I, [_P, _L, _P, _P, _P, _L, _I, _I, _I, _P, _L, _P]),
    "nb_add_rmsnorm": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, ctypes.c_float, _P]),
    "nb_attention_step": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P]),
    "nb_attention_work_floats": (_I, [_I]),
    "nb_attention_step_static": (_I, [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P]),
    "nb_attention_static_scratch_bytes": (_L, []),
    "nb_silu_mul": (_I, [_P, _P, _I, _I, _P]),
    "nb_rmsnorm_rows": (_I, [_P, _P, _P, _P, _I, _P, _P, _I, _I, _I, ctypes.c_float, _P]),
    "nb_silu_pairs_rows": (_I, [_P, _P, _I, _I, _I, _P]),
    "nb_rope_kv_rows": (_I, [_P, _P, _P, _P, _P, _I, _I, _P, _I, _I, _I, _P]),
    "nb_attention_rows": (_I, [_P, _P, _P, _I, _I, _P, _I, _I, _I, _I, _P]),
    "nb_lm_head_argmax": (_I, [_P, _P, _P, _P, _P, _I, _P, _I, _I, _I, _P]),
    "nb_rmsnorm_lm_head_argmax": (_I, [_P, _P, ctypes.c_float, _P, _P, _P, _P, _I, _P, _I, _I,
                                       _I, _P]),
    "nb_decode_workspace_bytes": (_L, [_P]),
    "nb_decode_persistent": (_I, [_P, _P, _L, _P, _P, _P, _I, _P, _I, _I, _I, _P]),
}

# Byte offset of the persistent decode's error word in its workspace.
NB_DECODE_ERR_OFFSET = 2304


class BatchItem(ctypes.Structure):
    """struct nb_batch_item (include/nativebit_amd.h)."""
    _fields_ = [("x", ctypes.c_void_p), ("packed", ctypes.c_void_p),
                ("codebook", ctypes.c_void_p), ("y", ctypes.c_void_p),
                ("N", ctypes.c_int32), ("K", ctypes.c_int32),
                ("x_mode", ctypes.c_int32), ("y_mode", ctypes.c_int32),
                ("norm_w", ctypes.c_void_p), ("eps", ctypes.c_float),
                ("reserved", ctypes.c_int32)]


class DecodeState(ctypes.Structure):
    """struct nb_decode_state (include/nativebit_amd.h)."""
    _fields_ = [("key", ctypes.c_uint64), ("pos", ctypes.c_int32), ("token", ctypes.c_int32),
                ("step", ctypes.c_int32), ("done", ctypes.c_uint32)]


class DecodeLayer(ctypes.Structure):
    """struct nb_decode_layer (include/nativebit_amd.h): device pointers."""
    _fields_ = [(n, ctypes.c_void_p) for n in (
        "qkv_packed", "qkv_codebook", "o_packed", "o_codebook", "gu_packed", "gu_codebook",
        "down_packed", "down_codebook", "ln1", "ln2", "k_cache", "v_cache")]


class DecodeModel(ctypes.Structure):
    """struct nb_decode_model (include/nativebit_amd.h)."""
    _fields_ = [("n_layers", ctypes.c_int32), ("n_embd", ctypes.c_int32),
                ("n_head", ctypes.c_int32), ("head_dim", ctypes.c_int32),
                ("ffn_hidden", ctypes.c_int32), ("vocab", ctypes.c_int32),
                ("ctx", ctypes.c_int32), ("eps", ctypes.c_float),
                ("layers", ctypes.c_void_p), ("ln_f", ctypes.c_void_p),
                ("emb_f32", ctypes.c_void_p), ("emb_bf16", ctypes.c_void_p),
                ("rope_cos", ctypes.c_void_p), ("rope_sin", ctypes.c_void_p)]


class NativeBitError(RuntimeError):
    """A non-zero status from libnativebit_amd.so."""

    def __init__(self, status: int, message: str):
        self.status = status
        super().__init__(f"{STATUS_NAMES.get(status, status)}: {message}")


_lock = threading.Lock()
_lib = None


def load():
    """Opens the library once and declares every exported signature."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} not found: build it with `python -m nativebit_amd.build` "
                "(the HIP path has no CPU fallback)")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if lib.nb_abi_version() != ABI_VERSION:
            raise ImportError(f"{LIB_PATH}: ABI {lib.nb_abi_version()} != {ABI_VERSION}")
        _lib = lib
    return _lib


def check(status: int) -> None:
    if status != NB_OK:
        msg = load().nb_last_error().decode(errors="replace")
        raise NativeBitError(status, msg)


def last_error() -> str:
    return load().nb_last_error().decode(errors="replace")

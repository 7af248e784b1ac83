"""ctypes binding of the C ABI in include/littlebit_amd.h.

The library is built in-tree by ``littlebit_amd.build``.  There is no
fallback: if the library is missing, every compute entry point raises.

torch is imported before the library is opened so that the library's
``libamdhip64.so.7`` dependency resolves to the HIP runtime torch already
loaded (same SONAME); torch's stream handles are then valid here.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch  # noqa: F401  (load order: torch's HIP runtime first)

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "liblittlebit_amd.so"

LBK_F32 = 0
LBK_BF16 = 1

LBK_OK = 0
LBK_ERR_ARG = -1
LBK_ERR_DTYPE = -2
LBK_ERR_WORKSPACE = -3
LBK_ERR_HIP = -4

ERROR_NAMES = {
    LBK_ERR_ARG: "invalid argument",
    LBK_ERR_DTYPE: "unsupported dtype",
    LBK_ERR_WORKSPACE: "workspace too small",
    LBK_ERR_HIP: "HIP error",
}


class LbkBranch(ctypes.Structure):
    """Mirror of ``lbk_branch``."""

    _fields_ = [
        ("v_sign", ctypes.c_void_p),
        ("u_sign", ctypes.c_void_p),
        ("v2", ctypes.c_void_p),
        ("mid", ctypes.c_void_p),
        ("u1", ctypes.c_void_p),
        ("rank", ctypes.c_int64),
        ("v_sign_tiled", ctypes.c_void_p),
    ]


class LbkProjection(ctypes.Structure):
    """Mirror of ``lbk_projection``."""

    _fields_ = [
        ("branches", ctypes.POINTER(LbkBranch)),
        ("n_branches", ctypes.c_int),
        ("out_features", ctypes.c_int64),
        ("bias", ctypes.c_void_p),
        ("y", ctypes.c_void_p),
        ("residual", ctypes.c_void_p),
    ]


class LbkInput(ctypes.Structure):
    """Mirror of ``lbk_input``."""

    _fields_ = [
        ("kind", ctypes.c_int),
        ("rms_weight", ctypes.c_void_p),
        ("rms_eps", ctypes.c_float),
        ("x1", ctypes.c_void_p),
        ("head_dim", ctypes.c_int),
        ("max_seq", ctypes.c_int),
        ("pos_device", ctypes.c_void_p),
        ("pos", ctypes.c_int64),
    ]


class LbkChainLink(ctypes.Structure):
    """Mirror of ``lbk_chain_link``."""

    _fields_ = [
        ("projs", ctypes.POINTER(LbkProjection)),
        ("n_proj", ctypes.c_int),
        ("in_features", ctypes.c_int64),
        ("input", ctypes.POINTER(LbkInput)),
    ]


LBK_INPUT_PLAIN = 0
LBK_INPUT_RMSNORM = 1
LBK_INPUT_SILU_MUL = 2
LBK_INPUT_ATTN_MERGE = 3
LBK_MAX_GROUP = 4
LBK_MAX_CHAIN = 8
LBK_NOALLOC_SCRATCH_BYTES = 8 << 20

# name -> (restype, argtypes); must list every function of include/littlebit_amd.h
_VP = ctypes.c_void_p
_I64 = ctypes.c_int64
SIGNATURES = {
    "lbk_abi_version": (ctypes.c_int, []),
    "lbk_last_error": (ctypes.c_char_p, []),
    "lbk_set_deterministic": (ctypes.c_int, [ctypes.c_int]),
    "lbk_linear_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(LbkBranch), ctypes.c_int, _I64, _I64, _I64]),
    "lbk_linear_forward": (
        ctypes.c_int,
        [ctypes.POINTER(LbkBranch), ctypes.c_int, _I64, _I64, _I64, _VP, ctypes.c_int, _VP, _VP,
         ctypes.c_int, _VP, ctypes.c_size_t, _VP],
    ),
    "lbk_group_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(LbkProjection), ctypes.c_int, _I64, _I64]),
    "lbk_group_forward": (
        ctypes.c_int,
        [ctypes.POINTER(LbkProjection), ctypes.c_int, _I64, _I64, _VP, ctypes.c_int, ctypes.c_int, _VP,
         ctypes.c_size_t, _VP],
    ),
    "lbk_group_forward_ex": (
        ctypes.c_int,
        [ctypes.POINTER(LbkProjection), ctypes.c_int, _I64, _I64, _VP, ctypes.c_int, ctypes.POINTER(LbkInput),
         ctypes.c_int, _VP, ctypes.c_size_t, _VP],
    ),
    "lbk_group_forward_noalloc": (
        ctypes.c_int,
        [ctypes.POINTER(LbkProjection), ctypes.c_int, _I64, _I64, _VP, ctypes.c_int, ctypes.POINTER(LbkInput),
         ctypes.c_int, _VP],
    ),
    "lbk_chain_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(LbkChainLink), ctypes.c_int]),
    "lbk_chain_forward": (
        ctypes.c_int,
        [ctypes.POINTER(LbkChainLink), ctypes.c_int, _VP, _VP, ctypes.c_size_t, _VP],
    ),
    "lbk_chain_fused": (ctypes.c_int, [ctypes.POINTER(LbkChainLink), ctypes.c_int, _VP]),
    "lbk_littlebit_linear": (
        ctypes.c_int,
        [_VP, _I64, _VP, _VP, _I64, _VP, _VP, _I64, _VP, _I64, _VP, _VP, ctypes.c_size_t, _VP],
    ),
    "lbk_attention_partial_bytes": (ctypes.c_size_t, [ctypes.c_int, ctypes.c_int, ctypes.c_int]),
    "lbk_q4_0_quantize": (ctypes.c_int, [_VP, _I64, _I64, _VP, _VP, _VP]),
    "lbk_lm_head_q4_workspace_bytes": (ctypes.c_size_t, [_I64, _I64]),
    "lbk_lm_head_q4_argmax": (ctypes.c_int, [_VP, _VP, _I64, _I64, _VP, _VP, ctypes.c_float, _VP, _VP, _VP,
                                             ctypes.c_size_t, _VP]),
    "lbk_attention_decode": (
        ctypes.c_int,
        [_VP, _VP, _VP, _VP, _VP, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, _VP, _I64,
         ctypes.c_float, _VP, ctypes.c_size_t, _VP, _VP],
    ),
    "lbk_attention_batch_partial_bytes": (ctypes.c_size_t, [ctypes.c_int, ctypes.c_int, _I64, ctypes.c_int]),
    "lbk_attention_batch": (
        ctypes.c_int,
        [_VP, _VP, _VP, _VP, _VP, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, _VP, _I64,
         _VP, ctypes.c_float, _VP, ctypes.c_size_t, _VP, _VP],
    ),
    "lbk_unpack_signs": (ctypes.c_int, [_VP, _I64, _I64, _VP, _VP]),
    "lbk_pack_signs": (ctypes.c_int, [_VP, _I64, _I64, _VP, _VP]),
    "lbk_repack_signs_to_i2": (ctypes.c_int, [_VP, _I64, _I64, _I64, _VP, _VP]),
    "lbk_tiled_v_words": (ctypes.c_int64, [_I64, _I64]),
    "lbk_tile_v_signs": (ctypes.c_int, [_VP, _I64, _I64, _VP, _VP]),
}

_lib = None
_lock = threading.Lock()


class LittleBitLibraryMissing(RuntimeError):
    pass


def load() -> ctypes.CDLL:
    """Open the library once; raise if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise LittleBitLibraryMissing(
                f"{LIB_PATH} not found: build it with `python -m littlebit_amd.build` "
                "(the HIP library is required; there is no CPU fallback)")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = lib
    return _lib


def last_error() -> str:
    msg = load().lbk_last_error()
    return msg.decode() if msg else ""


def check(rc: int, what: str) -> None:
    """Turn a negative return code into RuntimeError (like TORCH_CHECK)."""
    if rc != LBK_OK:
        kind = ERROR_NAMES.get(rc, f"error {rc}")
        raise RuntimeError(f"{what}: {kind}: {last_error()}")

"""ctypes binding of libbh_hex.so (the C ABI declared in include/bh_hex.h).

torch is imported first so that the library's HIP runtime dependency (libamdhip64.so.7)
resolves to the copy torch has already loaded: one HIP runtime per process, and torch's
streams and device pointers are valid in the library. The library is looked up next to this
file (an in-tree build) or at $BLACKHOLE_HEX_LIB. There is no fallback: without the library,
every entry point raises.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch  # noqa: F401  (must precede the dlopen below)

LIB_NAME = "libbh_hex.so"

# bh_hex_status
OK, ERR_VALUE, ERR_ASSERT, ERR_HIP, ERR_UNSUPPORTED = 0, 1, 2, 3, 4
# bh_hex_dtype
F32, BF16, F16, I32, I64 = 0, 1, 2, 3, 4
# bh_hex_order
ORDER_R, ORDER_D, ORDER_T = 0, 1, 2

_DTYPES = {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16, torch.int32: I32, torch.int64: I64}


class HexProj(ctypes.Structure):
    """struct bh_hex_proj."""
    _fields_ = [("idx", ctypes.c_void_p), ("block_scale", ctypes.c_void_p), ("expert_scale", ctypes.c_void_p),
                ("levels", ctypes.c_void_p), ("s_ie", ctypes.c_int64), ("s_in", ctypes.c_int64),
                ("s_be", ctypes.c_int64), ("s_bn", ctypes.c_int64), ("block", ctypes.c_int32)]


class HexTile(ctypes.Structure):
    """struct bh_hex_tile."""
    _fields_ = [("block_m", ctypes.c_int32), ("block_n", ctypes.c_int32), ("k_split", ctypes.c_int32)]


class Routing(ctypes.Structure):
    """struct bh_hex_routing."""
    _fields_ = [("scoring", ctypes.c_int32), ("renormalize", ctypes.c_int32), ("n_group", ctypes.c_int32),
                ("topk_group", ctypes.c_int32), ("routed_scaling_factor", ctypes.c_float),
                ("correction_bias", ctypes.c_void_p)]


# bh_hex_scoring
SCORE_SOFTMAX, SCORE_SIGMOID = 0, 1

_P, _I32, _I64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64
_PROJ = ctypes.POINTER(HexProj)
_TILE = ctypes.POINTER(HexTile)
_ROUTING = ctypes.POINTER(Routing)

# name -> (restype, argtypes): every symbol include/bh_hex.h declares
SIGNATURES = {
    "bh_hex_last_error": (ctypes.c_char_p, []),
    "bh_hex_abi_version": (ctypes.c_int, []),
    "bh_hex_dequant": (ctypes.c_int, [_PROJ, _I32, _I64, _I64, _I64, _P, _P, _I32, _I64, _I64, _I64, _I32, _P]),
    "bh_hex_route_topk": (ctypes.c_int, [_P, _I32, _I64, _I64, _I32, _I32, _I32, _P, _P, _I32, _P]),
    "bh_hex_route_select": (ctypes.c_int, [_P, _I32, _I64, _I64, _I32, _I32, _ROUTING, _P, _P, _I32, _P]),
    "bh_hex_route_gemm": (ctypes.c_int, [_P, _I32, _I64, _P, _I64, _I64, _I32, _I32, _I32, _ROUTING, _P, _I64, _P, _P,
                                         _I32, _P, _I64, _P]),
    "bh_hex_route_gemm_workspace": (ctypes.c_int64, [_I64]),
    "bh_hex_align_max_blocks": (ctypes.c_int64, [_I64, _I32, _I32]),
    "bh_hex_align": (ctypes.c_int, [_P, _I32, _I64, _I32, _I32, _P, _P, _P, _P]),
    "bh_hex_align_tier": (ctypes.c_int, [_P, _I32, _I64, _I32, _P, _I32, _P, _P, _P, _P]),
    "bh_hex_align_workspace": (ctypes.c_int64, [_I64, _I32]),
    "bh_hex_align_ws": (ctypes.c_int, [_P, _I32, _I64, _I32, _P, _I32, _P, _I64, _P, _P, _P, _P]),
    "bh_hex_direct": (ctypes.c_int, [_P, _I32, _I64, _I32, _P, _P, _P, _P]),
    "bh_hex_moe_glu": (ctypes.c_int, [_P, _I32, _I64, _P, _I64, _PROJ, _PROJ, _I32, _I64, _I64, _P, _P, _I64, _P,
                                      _P, _I32, _I64, _I32, _TILE, _P, _I64, _P, _I64, _P]),
    "bh_hex_moe_down": (ctypes.c_int, [_P, _I32, _I64, _P, _I32, _I64, _PROJ, _I32, _I64, _I64, _P, _P, _I64, _P, _P, _I32,
                                       _I64, _P, _TILE, _P, _I64, _P, _I64, _P]),
    "bh_hex_moe_glu_ids": (ctypes.c_int, [_P, _I32, _I64, _P, _I64, _PROJ, _PROJ, _I32, _I64, _I64, _P, _I32, _P, _I32,
                                          _I64, _I32, _TILE, _P, _I64, _P, _I64, _P]),
    "bh_hex_moe_glu_ids_noalloc": (ctypes.c_int, [_P, _I32, _I64, _P, _I64, _PROJ, _PROJ, _I32, _I64, _I64, _P, _I32, _P,
                                                  _I32, _I64, _I32, _TILE, _P]),
    "bh_hex_moe_down_ids": (ctypes.c_int, [_P, _I32, _I64, _P, _I32, _I64, _PROJ, _I32, _I64, _I64, _P, _I32, _P, _I32,
                                           _I64, _P, _TILE, _P, _I64, _P, _I64, _P]),
    "bh_hex_moe_workspace": (ctypes.c_int, [_I64, _I64, _I64, _I32, _I32, ctypes.POINTER(ctypes.c_int64),
                                            ctypes.POINTER(ctypes.c_int64)]),
    "bh_hex_moe_reduce": (ctypes.c_int, [_P, _I32, _I64, _P, _I32, _I32, _I64, _I32, _I64, _P, _I32, _I64, _P]),
    "bh_hex_block_header": (ctypes.c_int, [_P, _I64, _I64, _I64, _I32, _P, _P, _P, _P, _P, _P, _P]),
    "bh_hex_fit_levels": (ctypes.c_int, [_P, _P, _I64, _I64, _I32, _P, _P, _P, _I32, _P, _P]),
    "bh_hex_gptq_sweep": (ctypes.c_int, [_P, _P, _P, _I32, _P, _I32, _P, _I64, _I64, _I64, _I32, _P, _P, _P]),
    "bh_hex_moe_gemv": (ctypes.c_int, [_P, _I32, _I64, _P, _I64, _P, _I32, _I64, _PROJ, _PROJ, _PROJ, _I32, _I64, _I64,
                                       _P, _I32, _P, _P, _I32, _I64, _I32, _P]),
}

ABI_VERSION = 13

_lib = None


def lib_path() -> Path:
    env = os.environ.get("BLACKHOLE_HEX_LIB")
    return Path(env) if env else Path(__file__).with_name(LIB_NAME)


def load() -> ctypes.CDLL:
    """The loaded library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        p = lib_path()
        if not p.exists():
            raise RuntimeError(f"{p} is missing: build it with `make -C blackhole-harness_amd` "
                               "(or __graft_entry__.build()); the HEX kernels have no fallback")
        lib = ctypes.CDLL(str(p))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype, fn.argtypes = res, args
        if lib.bh_hex_abi_version() != ABI_VERSION:
            raise RuntimeError(f"{p} has ABI {lib.bh_hex_abi_version()}, this module expects {ABI_VERSION}")
        _lib = lib
    return _lib


def check(rc: int, what: str) -> None:
    """Map a bh_hex status to the exception class the reference raises for the same condition."""
    if rc == OK:
        return
    msg = (_lib.bh_hex_last_error() or b"").decode(errors="replace") or what
    if rc == ERR_VALUE:
        raise ValueError(msg)
    if rc == ERR_ASSERT:
        raise AssertionError(msg)
    if rc == ERR_UNSUPPORTED:
        raise NotImplementedError(msg)
    raise RuntimeError(msg)


def dtype_code(t: torch.dtype) -> int:
    try:
        return _DTYPES[t]
    except KeyError:
        raise TypeError(f"unsupported dtype {t}") from None


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(t: torch.Tensor) -> int:
    """The current HIP stream of the tensor's device (what the reference's Triton launches use)."""
    return torch.cuda.current_stream(t.device).cuda_stream


def require_gpu(*ts: torch.Tensor) -> None:
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("the HEX kernels run on the GPU: got a tensor on " + str(t.device))

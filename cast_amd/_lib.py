"""Bindings of the C ABI declared in ``include/rcsa.h``.

``load()`` is the ctypes binding of ``librcsa.so``; ``torch_ops()`` loads the
PyTorch-ROCm extension ``librcsa_torch.so`` (torch custom ops ``torch.ops.rcsa``
over the same C ABI, used for the layer call's entry points) and binds it to
the library ``load()`` opened.  Both are built in-tree by ``cast_amd.build``.
There is no fallback: every operator raises if a library is missing or a call
fails.
"""
from __future__ import annotations

import ctypes
from ctypes import c_float, c_int, c_int64, c_void_p
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "librcsa.so"
TORCH_OPS_PATH = Path(__file__).resolve().parent / "_lib" / "librcsa_torch.so"

RCSA_OK = 0
RCSA_BF16 = 0
RCSA_F32 = 1
RCSA_ORDER_INDEX = 0
RCSA_ORDER_RANK = 1

_P = c_void_p
_I = c_int64

# name -> argument types (return type is int status unless noted)
SIGNATURES: dict[str, list] = {
    "rcsa_pool_query": [_P, c_int, _I, _I, _I, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P],
    "rcsa_pool_key": [_P, c_int, _I, _I, _I, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P],
    "rcsa_pool_query_key": [_P, _P, c_int, _I, _I, _I, _I, _I, _I, _I, _I, _I, _I, _I, _I,
                            _P, _P, _P, _I, _P, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P],
    "rcsa_pool_query_key_value": [_P, _P, _P, c_int] + [_I] * 15 + [_P, _P, _P, _I, _P, _I]
                                 + [_P] * 9 + [_P],
    "rcsa_block_scores": [_P, _P, _I, _I, _I, _I, _P, _P],
    "rcsa_quantize_key_select": [_P, c_int, _I, _I, _I, _I, _I, _I, _I, _I, _P, _P, _I,
                                 _P, _P, _P, _P, _P, _P, _P, _P, _I, _P, _P, _I, _I, _P, _P,
                                 _I, _P, _I, _P, _P],
    "rcsa_row_budgets": [_P, _I, _I, _I, _I, _I, _I, _P, _I, _P],
    "rcsa_closed_loop_degrees": [_P, _P, _I, _I, _P, _I, _I, _I, _I, _I, _I, _I, _I,
                                 c_float, c_int, c_int, _P, _P, _P],
    "rcsa_select_topk": [_P, _I, _I, _I, _P, _I, _I, _P, _P, _I, _P, _I, _P, c_int, _P],
    "rcsa_quantize_key": [_P, c_int, _I, _I, _I, _I, _I, _I, _I, _I, _P, _P, _I, _P, _P, _P,
                          _P, _P, _P, _P],
    "rcsa_sparse_attn_bf16": [_P, _P, _P, _P, c_float, _P, _P, _P, _P] + [_I] * 18
                             + [_I] * 8 + [_P],
    "rcsa_sparse_attn_int8": [_P, _P, _I, _P, _P, _I, _P, _P, _P, c_float, _P, _P, _P, _P]
                             + [_I] * 18 + [_I] * 8 + [_P, _I, _P],
    "rcsa_sparse_attn_bf16_split": [_P, _P, _P, _P, _P, c_float, _P, _P, _P, _P] + [_I] * 18
                                   + [_I] * 8 + [_I, _P, _I, _P, _I, _P, _I, _P, _I, _P],
    "rcsa_sparse_attn_int8_split": [_P, _P, _I, _P, _P, _I, _P, _P, _P, c_float, _P, _P, _P, _P]
                                   + [_I] * 18 + [_I] * 8 + [_I, _P, _I, _P, _I, _P, _I, _P],
    "rcsa_sparse_attn_int8_noalloc": [_P, _P, _I, _P, _P, _I, _P, _P, _P, c_float, _P, _P, _P,
                                      _P] + [_I] * 18 + [_I] * 8 + [_I, _P, _I, _P, _I, _P],
    "rcsa_attn_noalloc_scratch_bytes": [],
    "rcsa_attn_workspace_bytes": [_I, _I, _I, _I, _I],
    "rcsa_attn_split_plan": [_I, _I, _I, _I, _I, ctypes.POINTER(c_int64)],
    "rcsa_route_proxy": [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, c_float, _P, _P,
                         _P, _P],
    "rcsa_route_best_swap": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I,
                             c_int, _P, _P, _P],
    "rcsa_route_apply_swap": [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I,
                              c_float, _P],
    "rcsa_route_check": [_P, _P, _P, _P, _I, _I, _I, _I, _P, _P],
    "rcsa_quantize_rows_int8": [_P, c_int, _I, _I, _I, _P, _P, _P],
    "rcsa_int8_linear": [_P, _P, _P, _P, _P, _I, _I, _I, _P, _I, _P],
    "rcsa_pack_tokens": [_P, c_int, _I, _I, _I, _I, _I, _I, _I, _P, _I, _P, _P],
    "rcsa_unpack_tokens": [_P, _I, _I, _I, _I, _P, _I, _P, _P],
    "rcsa_status_string": [c_int],
    "rcsa_abi_version": [],
}

_lib = None


def load() -> ctypes.CDLL:
    """Load ``librcsa.so`` once and declare every entry point's signature."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"RCSA HIP library not built: {LIB_PATH} is missing "
            "(run `python -m cast_amd.build`)"
        )
    # torch first: the library must bind to the HIP runtime torch already loaded
    # (loaded first, the library would bring in a second runtime whose kernels
    # cannot run on torch's streams)
    import torch  # noqa: F401
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, argtypes in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = (ctypes.c_char_p if name == "rcsa_status_string"
                      else c_int64 if name in ("rcsa_attn_workspace_bytes",
                                               "rcsa_attn_noalloc_scratch_bytes")
                      else c_int)
    _lib = lib
    return lib


_torch_ops = None


def torch_ops():
    """``torch.ops.rcsa``: the extension's custom ops, bound to ``LIB_PATH``."""
    global _torch_ops
    if _torch_ops is not None:
        return _torch_ops
    load()
    if not TORCH_OPS_PATH.exists():
        raise RuntimeError(
            f"RCSA torch extension not built: {TORCH_OPS_PATH} is missing "
            "(run `python -m cast_amd.build`)"
        )
    import torch
    torch.ops.load_library(str(TORCH_OPS_PATH))
    torch.ops.rcsa.bind_library(str(LIB_PATH))
    _torch_ops = torch.ops.rcsa
    return _torch_ops


def check(status: int, fn: str) -> None:
    """Raise ``RuntimeError("<fn>: <reason>")`` for a non-zero status."""
    if status != RCSA_OK:
        reason = load().rcsa_status_string(status).decode()
        raise RuntimeError(f"{fn}: {reason} (status {status})")

"""Shared int8 Q/K/V projection on the device.

Mirrors ``shared_int8_qkv`` and ``SharedInt8QKVForwardCoordinator``
(P/matrix_shared_int8_qkv.py:19-147): the three int8 projections of a
self-attention block quantise their common input once and reuse it.  The
modules are the upstream Matrix ``Int8Linear`` layers (``in_features``,
``out_features``, ``weight_int8`` [out, in], ``weight_scales`` [out],
``bias``); the quantiser and the GEMMs are ``rcsa_quantize_rows_int8`` and
``rcsa_int8_linear`` (int8 MFMA with the dequantising epilogue) instead of the
upstream Triton kernels.  Each projection returns bf16(acc * x_scale * w_scale),
plus the bias in bf16, cast to the input's dtype, as the reference does.
"""
from __future__ import annotations

from types import MethodType
from typing import Any

import torch

from . import ops

_REQUIRED = ("in_features", "out_features", "weight_int8", "weight_scales", "bias")


def _project(module: Any, x_i8: torch.Tensor, x_scale: torch.Tensor, x_shape: torch.Size,
             output_dtype: torch.dtype) -> torch.Tensor:
    out = ops.int8_linear(x_i8, x_scale, module.weight_int8, module.weight_scales,
                          bias=module.bias)
    return out.view(*x_shape[:-1], int(module.out_features)).to(output_dtype)


def shared_int8_qkv(q_module: Any, k_module: Any, v_module: Any, x: torch.Tensor):
    """(q, k, v) of the three int8 projections with one quantisation of ``x``."""
    modules = (q_module, k_module, v_module)
    if not x.is_cuda or not x.is_contiguous():
        raise RuntimeError("shared Matrix QKV requires contiguous CUDA input")
    if x.dtype not in {torch.float32, torch.bfloat16, torch.float16}:
        raise RuntimeError("shared Matrix QKV received an unsupported input dtype")
    if any(not all(hasattr(m, name) for name in _REQUIRED) for m in modules):
        raise RuntimeError("shared Matrix QKV requires upstream Int8Linear modules")
    in_features = int(q_module.in_features)
    if any(int(m.in_features) != in_features for m in modules):
        raise RuntimeError("shared Matrix QKV input dimensions disagree")
    if int(x.shape[-1]) != in_features or in_features < 16:
        raise RuntimeError("shared Matrix QKV activation shape is unsupported")
    if any(m.weight_int8.dtype != torch.int8 for m in modules):
        raise RuntimeError("shared Matrix QKV weights must be int8")
    x_i8, x_scale = ops.quantize_rows_int8(x)
    return tuple(_project(m, x_i8, x_scale, x.shape, x.dtype) for m in modules)


class SharedInt8QKVForwardCoordinator:
    """Route a self-attention block's q, k and v calls through one shared
    quantisation (install / uninstall / project, as the reference)."""

    def __init__(self, self_attention: Any) -> None:
        self.module = self_attention
        self.modules = (self_attention.q, self_attention.k, self_attention.v)
        self.native_forwards = tuple(m.forward for m in self.modules)
        self._input = None
        self._outputs = None
        self._next = 0

    def install(self) -> None:
        if self._next or self._outputs is not None:
            raise RuntimeError("cannot install an active shared QKV coordinator")
        coordinator = self
        for index, module in enumerate(self.modules):
            def wrapped(_module: Any, x: torch.Tensor, _index: int = index) -> torch.Tensor:
                return coordinator.project(_index, x)
            module.forward = MethodType(wrapped, module)

    def uninstall(self) -> None:
        for module, native in zip(self.modules, self.native_forwards):
            module.forward = native
        self._input = None
        self._outputs = None
        self._next = 0

    def project(self, projection_index: int, x: torch.Tensor) -> torch.Tensor:
        if projection_index == 0:
            if self._outputs is not None:
                raise RuntimeError("overlapping native self-attention QKV calls")
            self._input = x
            self._outputs = shared_int8_qkv(*self.modules, x.contiguous())
            self._next = 1
            return self._outputs[0]
        if self._outputs is None or self._input is not x or projection_index != self._next:
            raise RuntimeError("native Matrix self-attention did not call q/k/v in order")
        out = self._outputs[projection_index]
        self._next += 1
        if self._next == 3:
            self._input = None
            self._outputs = None
            self._next = 0
        return out

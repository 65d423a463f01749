"""Tensor-level wrappers over the RCSA C ABI.

Each function validates shapes/dtypes/devices on the host, allocates its
outputs from the torch caching allocator, and launches on the current torch
stream.  No function reads device memory back to the host.
"""
from __future__ import annotations

import ctypes
import math
from typing import Optional

import torch

from . import _lib
from ._lib import RCSA_BF16, RCSA_F32, RCSA_ORDER_INDEX, RCSA_ORDER_RANK, check

__all__ = [
    "pool_query", "pool_key", "block_scores", "select_topk", "quantize_key",
    "sparse_attn_bf16", "sparse_attn_int8", "pack_tokens", "unpack_tokens", "row_budgets",
    "quantize_key_select",
]


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _dtype_code(t: torch.Tensor, fn: str) -> int:
    if t.dtype == torch.bfloat16:
        return RCSA_BF16
    if t.dtype == torch.float32:
        return RCSA_F32
    raise TypeError(f"{fn}: expected bfloat16 or float32, got {t.dtype}")


def _require_cuda(fn: str, *tensors: Optional[torch.Tensor]) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError(f"{fn}: tensors must live on a HIP device, got {t.device}")


def _bytes_mask(m: torch.Tensor, device) -> torch.Tensor:
    """A one-byte-per-entry mask on ``device``: bool (stored as 0/1 bytes) and
    uint8 pass through without a conversion kernel."""
    if m.dtype not in (torch.bool, torch.uint8):
        m = m != 0
    if m.device != device:
        m = m.to(device)
    return m.contiguous()


def _valid_u8(valid: Optional[torch.Tensor], n: int, device, fn: str) -> Optional[torch.Tensor]:
    if valid is None:
        return None
    v = valid.reshape(-1)
    if v.numel() != n:
        raise ValueError(f"{fn}: valid mask has {v.numel()} entries, expected {n}")
    v = _bytes_mask(v, device)
    if v.data_ptr() % 16:  # an offset view; the kernels read 16-byte chunks
        v = v.clone()
    return v


def _bhld(x: torch.Tensor, block_size: int, fn: str) -> tuple[int, int, int, int, int]:
    if x.ndim != 4:
        raise ValueError(f"{fn}: expected [B, H, L, D], got {tuple(x.shape)}")
    B, H, L, D = x.shape
    if L % block_size:
        raise ValueError(f"{fn}: length {L} is not a multiple of block_size {block_size}")
    if x.stride(3) != 1:
        raise ValueError(f"{fn}: last dimension must be contiguous")
    return B, H, L, D, L // block_size


def pool_query(q: torch.Tensor, valid: Optional[torch.Tensor], block_size: int,
               quantize: bool = False):
    """Masked mean-pool + L2-normalise query blocks, optionally fusing int8 quantisation.

    Follows P/matrix_curvature_phase_frame_weave.py:5685-5700.  Returns
    ``(qhat [B*H, NB, D] fp32, q_i8 [B, H, L, D] int8 | None, q_scale [B*H, NB] | None)``.
    """
    fn = "pool_query"
    _require_cuda(fn, q)
    code = _dtype_code(q, fn)
    B, H, L, D, NB = _bhld(q, block_size, fn)
    v = _valid_u8(valid, L, q.device, fn)
    qhat = torch.empty(B * H, NB, D, device=q.device, dtype=torch.float32)
    q_i8 = torch.empty(B, H, L, D, device=q.device, dtype=torch.int8) if quantize else None
    q_scale = torch.empty(B * H, NB, device=q.device, dtype=torch.float32) if quantize else None
    st = _lib.load().rcsa_pool_query(
        q.data_ptr(), code, B, H, NB, block_size, D, q.stride(0), q.stride(1), q.stride(2),
        _ptr(v), qhat.data_ptr(), _ptr(q_i8), _ptr(q_scale), _stream())
    check(st, fn)
    return qhat, q_i8, q_scale


def pool_key(k: torch.Tensor, valid: Optional[torch.Tensor], block_size: int,
             stats: bool = False, block_mask: bool = False):
    """Masked mean-pool + L2-normalise key blocks (+ sum/min/max for the quantiser).

    Returns ``(khat, ksum, kmin, kmax)``; the last three are None unless ``stats``.
    With ``block_mask`` a fifth value follows: the key validity as bits, int32
    ``[n_blocks, block_size // 32]`` (bit i of word w of block n = token
    ``n * block_size + 32 w + i``), the form ``sparse_attn_int8`` takes.
    """
    fn = "pool_key"
    _require_cuda(fn, k)
    code = _dtype_code(k, fn)
    B, H, L, D, NB = _bhld(k, block_size, fn)
    v = _valid_u8(valid, L, k.device, fn)
    khat = torch.empty(B * H, NB, D, device=k.device, dtype=torch.float32)
    if stats:
        ksum, kmin, kmax = (torch.empty(B * H, NB, D, device=k.device, dtype=torch.float32)
                            for _ in range(3))
    else:
        ksum = kmin = kmax = None
    mask = (torch.empty(NB, block_size // 32, device=k.device, dtype=torch.int32)
            if block_mask else None)
    st = _lib.load().rcsa_pool_key(
        k.data_ptr(), code, B, H, NB, block_size, D, k.stride(0), k.stride(1), k.stride(2),
        _ptr(v), khat.data_ptr(), _ptr(ksum), _ptr(kmin), _ptr(kmax), _ptr(mask), _stream())
    check(st, fn)
    return (khat, ksum, kmin, kmax, mask) if block_mask else (khat, ksum, kmin, kmax)


def _slot_map(m: torch.Tensor, block_size: int, device, fn: str) -> torch.Tensor:
    """int32 slot -> token map on ``device`` (-1 = empty slot), a whole number of blocks."""
    if m.ndim != 1 or m.numel() == 0 or m.numel() % block_size:
        raise ValueError(f"{fn}: slot map must be a vector of whole {block_size}-slot blocks")
    if m.dtype not in (torch.int32, torch.int64):
        raise TypeError(f"{fn}: slot map must be int32 or int64")
    return m.to(device=device, dtype=torch.int32).contiguous()


def _tokens_bhld(x: torch.Tensor, slots: torch.Tensor, block_size: int, fn: str):
    """Shape of a gathered source ``[B, L, H, D]``: (B, H, n_slots, D, n_blocks, L, strides)."""
    if x.ndim != 4 or x.stride(3) != 1:
        raise ValueError(f"{fn}: a gathered source must be [B, L, H, D] with a contiguous last dim")
    B, L, H, D = x.shape
    n = slots.numel()
    return B, H, n, D, n // block_size, L, (x.stride(0), x.stride(2), x.stride(1))


def pool_query_key(q: torch.Tensor, q_valid: Optional[torch.Tensor], k: torch.Tensor,
                   k_valid: Optional[torch.Tensor], block_size: int, *,
                   q_slot_token: Optional[torch.Tensor] = None,
                   k_slot_token: Optional[torch.Tensor] = None, quantize: bool = True):
    """``pool_query(q, q_valid, quantize=True)`` and ``pool_key(k, k_valid, stats=True,
    block_mask=True)`` in one launch (no reference counterpart: the int8 layer call's
    pooling pass).  Returns ``(qhat, q_i8, q_scale, khat, ksum, kmin, kmax, block_mask)``,
    bit for bit the two calls' outputs.  ``quantize=False`` drops the query
    quantiser and the key statistics (those five outputs are None): the bf16
    path's pass.

    With ``q_slot_token`` / ``k_slot_token`` (both or neither) q and k are token-major
    ``[B, L, H, D]`` sources gathered on the fly: the outputs equal those of
    ``pool_query_key(pack_tokens(q, q_slot_token), ..., pack_tokens(k, k_slot_token), ...)``
    (the q[:, flat] / k[:, flat] gathers of
    P/matrix_curvature_phase_frame_weave.py:5677-5684 fused into the pass); the valid
    masks, when given, stay per packed slot.
    """
    fn = "pool_query_key"
    _require_cuda(fn, q, k)
    code = _dtype_code(q, fn)
    if _dtype_code(k, fn) != code:
        raise TypeError(f"{fn}: q and k must share a dtype")
    if (q_slot_token is None) != (k_slot_token is None):
        raise ValueError(f"{fn}: give both slot maps or neither")
    if q_slot_token is not None:
        qm = _slot_map(q_slot_token, block_size, q.device, fn)
        km = _slot_map(k_slot_token, block_size, k.device, fn)
        B, H, Lq, D, NQ, q_src, q_strides = _tokens_bhld(q, qm, block_size, fn)
        Bk, Hk, Lk, Dk, NK, k_src, k_strides = _tokens_bhld(k, km, block_size, fn)
    else:
        qm = km = None
        q_src = k_src = 0
        B, H, Lq, D, NQ = _bhld(q, block_size, fn)
        Bk, Hk, Lk, Dk, NK = _bhld(k, block_size, fn)
        q_strides = (q.stride(0), q.stride(1), q.stride(2))
        k_strides = (k.stride(0), k.stride(1), k.stride(2))
    if (Bk, Hk, Dk) != (B, H, D):
        raise ValueError(f"{fn}: q {tuple(q.shape)} and k {tuple(k.shape)} differ in B, H or D")
    qv = _valid_u8(q_valid, Lq, q.device, fn)
    kv = _valid_u8(k_valid, Lk, k.device, fn)
    f32 = dict(device=q.device, dtype=torch.float32)
    qhat = torch.empty(B * H, NQ, D, **f32)
    khat = torch.empty(B * H, NK, D, **f32)
    if quantize:
        q_i8 = torch.empty(B, H, Lq, D, device=q.device, dtype=torch.int8)
        q_scale = torch.empty(B * H, NQ, **f32)
        ksum, kmin, kmax = (torch.empty(B * H, NK, D, **f32) for _ in range(3))
    else:
        q_i8 = q_scale = ksum = kmin = kmax = None
    mask = torch.empty(NK, block_size // 32, device=k.device, dtype=torch.int32)
    # through the torch extension (rcsa::pool_query_key -> rcsa_pool_query_key)
    _lib.torch_ops().pool_query_key(
        q, k, code, [B, H, NQ, NK, block_size, D], list(q_strides), list(k_strides),
        qv, kv, qm, q_src, km, k_src, qhat, q_i8, q_scale, khat, ksum, kmin, kmax, mask)
    return qhat, q_i8, q_scale, khat, ksum, kmin, kmax, mask


def pool_query_key_value(q: torch.Tensor, q_valid: Optional[torch.Tensor], k: torch.Tensor,
                         k_valid: Optional[torch.Tensor], v: torch.Tensor, block_size: int, *,
                         q_slot_token: Optional[torch.Tensor] = None,
                         k_slot_token: Optional[torch.Tensor] = None, quantize: bool = True):
    """:func:`pool_query_key` plus the block means of ``v`` in the same launch
    (``rcsa_pool_query_key_value``): the pooled values ``v_content`` of
    P/matrix_curvature_phase_frame_weave.py:5696-5700 that the FC-PASM router
    consumes.  ``v`` has k's layout (packed ``[B, H, L, D]``, or token-major
    ``[B, L, H, D]`` read through ``k_slot_token``) and shares its validity.
    Returns pool_query_key's eight outputs and ``vmean`` fp32 ``[B*H, NK, D]``."""
    fn = "pool_query_key_value"
    _require_cuda(fn, q, k, v)
    code = _dtype_code(q, fn)
    if _dtype_code(k, fn) != code or _dtype_code(v, fn) != code:
        raise TypeError(f"{fn}: q, k and v must share a dtype")
    if v.shape != k.shape:
        raise ValueError(f"{fn}: v {tuple(v.shape)} must have k's shape {tuple(k.shape)}")
    if (q_slot_token is None) != (k_slot_token is None):
        raise ValueError(f"{fn}: give both slot maps or neither")
    if q_slot_token is not None:
        qm = _slot_map(q_slot_token, block_size, q.device, fn)
        km = _slot_map(k_slot_token, block_size, k.device, fn)
        B, H, Lq, D, NQ, q_src, q_strides = _tokens_bhld(q, qm, block_size, fn)
        Bk, Hk, Lk, Dk, NK, k_src, k_strides = _tokens_bhld(k, km, block_size, fn)
        _, _, _, _, _, _, v_strides = _tokens_bhld(v, km, block_size, fn)
    else:
        qm = km = None
        q_src = k_src = 0
        B, H, Lq, D, NQ = _bhld(q, block_size, fn)
        Bk, Hk, Lk, Dk, NK = _bhld(k, block_size, fn)
        _bhld(v, block_size, fn)
        q_strides = (q.stride(0), q.stride(1), q.stride(2))
        k_strides = (k.stride(0), k.stride(1), k.stride(2))
        v_strides = (v.stride(0), v.stride(1), v.stride(2))
    if (Bk, Hk, Dk) != (B, H, D):
        raise ValueError(f"{fn}: q {tuple(q.shape)} and k {tuple(k.shape)} differ in B, H or D")
    qv = _valid_u8(q_valid, Lq, q.device, fn)
    kv = _valid_u8(k_valid, Lk, k.device, fn)
    f32 = dict(device=q.device, dtype=torch.float32)
    qhat = torch.empty(B * H, NQ, D, **f32)
    khat = torch.empty(B * H, NK, D, **f32)
    vmean = torch.empty(B * H, NK, D, **f32)
    if quantize:
        q_i8 = torch.empty(B, H, Lq, D, device=q.device, dtype=torch.int8)
        q_scale = torch.empty(B * H, NQ, **f32)
        ksum, kmin, kmax = (torch.empty(B * H, NK, D, **f32) for _ in range(3))
    else:
        q_i8 = q_scale = ksum = kmin = kmax = None
    mask = torch.empty(NK, block_size // 32, device=k.device, dtype=torch.int32)
    check(_lib.load().rcsa_pool_query_key_value(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), code, B, H, NQ, NK, block_size, D,
        *q_strides, *k_strides, *v_strides, _ptr(qv), _ptr(kv), _ptr(qm), q_src, _ptr(km),
        k_src, qhat.data_ptr(), _ptr(q_i8), _ptr(q_scale), khat.data_ptr(), _ptr(ksum),
        _ptr(kmin), _ptr(kmax), mask.data_ptr(), vmean.data_ptr(), _stream()), fn)
    return qhat, q_i8, q_scale, khat, ksum, kmin, kmax, mask, vmean


def row_budgets(weights: torch.Tensor, total_per_section: int, *, cap: int = 0,
                target_total: Optional[int] = None) -> torch.Tensor:
    """Per-row budgets on the device: ``budget.apportion_section_matrix(weights, total)``
    and, with ``cap > 0``, ``budget.saturate(row, cap, target_total)`` on every section
    row (P/qk_uncertainty_tangent_attention.py:847-865, 1239-1264;
    P/matrix_curvature_phase_frame_weave.py:5807-5817).  ``weights`` is float32
    ``[sections, n]`` on the GPU; returns int32 ``[sections, n]`` without a host sync."""
    fn = "row_budgets"
    _require_cuda(fn, weights)
    if weights.ndim != 2 or weights.dtype != torch.float32 or weights.stride(1) != 1:
        raise ValueError(f"{fn}: weights must be float32 [sections, n] with contiguous rows")
    S, n = weights.shape
    out = torch.empty(S, n, device=weights.device, dtype=torch.int32)
    check(_lib.load().rcsa_row_budgets(weights.data_ptr(), S, n, weights.stride(0),
                                       int(total_per_section), int(cap),
                                       int(target_total) if target_total is not None else 0,
                                       out.data_ptr(), n, _stream()), fn)
    return out


_CL_FEEDBACK = {"additive": 0, "centered_multiplicative": 1, "centered_inverse": 2}
_CL_ERRORS = ((1, "compact Current frame lies outside CWCA frame capacity"),
              (4, "compact Closed-Loop Current set contains Memory frames"),
              (2, "compact Closed-Loop CWCA exhausted key capacity"))


def closed_loop_degrees(curvature: torch.Tensor, frames, *, current_temporal_offset: int,
                        source_group: int, compact_group: int, mean_degree: int,
                        base_degree: int, total_blocks: int, memory_blocks: int,
                        response: Optional[torch.Tensor] = None, response_weight: float = 0.0,
                        feedback_form: str = "additive", fixed_query_budget: bool = False,
                        check_status: bool = True):
    """Row degrees of a compact woven layer under the closed-loop allocator
    (``rcsa_closed_loop_degrees``): int32 ``[total_blocks]`` on the device.

    ``curvature`` / ``response``: float32 ``[T_src, S]``; ``frames``: the active
    current-local frames (int sequence or tensor).  With ``check_status`` the
    device status word is read back once and a breach raises ``RuntimeError``
    with the reference's message; otherwise ``(degrees, status)`` is returned
    and nothing is read back."""
    fn = "closed_loop_degrees"
    _require_cuda(fn, curvature)
    dev = curvature.device
    if curvature.dtype != torch.float32 or curvature.ndim != 2:
        raise TypeError(f"{fn}: curvature must be float32 [T_src, S]")
    curvature = curvature.contiguous()
    if response is not None:
        if response.shape != curvature.shape or response.dtype != torch.float32:
            raise ValueError(f"{fn}: response must be float32 {tuple(curvature.shape)}")
        response = response.to(dev).contiguous()
    if feedback_form not in _CL_FEEDBACK:
        raise ValueError(f"unknown control-response feedback {feedback_form!r}")
    fr = torch.as_tensor(frames)
    if fr.device.type == "cpu":  # pinned, so the copy waits for nothing on the stream
        fr = fr.to(torch.int32).reshape(-1).contiguous().pin_memory()
    fr = fr.to(device=dev, dtype=torch.int32, non_blocking=True).reshape(-1).contiguous()
    degrees = torch.empty(int(total_blocks), device=dev, dtype=torch.int32)
    status = torch.empty(1, device=dev, dtype=torch.int32)
    t_src, spatial = curvature.shape
    st = _lib.load().rcsa_closed_loop_degrees(
        curvature.data_ptr(), _ptr(response), t_src, spatial, fr.data_ptr(), fr.numel(),
        int(current_temporal_offset), int(source_group), int(compact_group), int(mean_degree),
        int(base_degree), int(total_blocks), int(memory_blocks), float(response_weight),
        _CL_FEEDBACK[feedback_form], int(bool(fixed_query_budget)), degrees.data_ptr(),
        status.data_ptr(), _stream())
    check(st, fn)
    if not check_status:
        return degrees, status
    code = int(status.item())
    for bit, msg in _CL_ERRORS:
        if code & bit:
            raise RuntimeError(msg)
    return degrees


def block_scores(qhat: torch.Tensor, khat: torch.Tensor) -> torch.Tensor:
    """``score[bh] = qhat[bh] @ khat[bh]^T`` (P/matrix_curvature_phase_frame_weave.py:5701)."""
    fn = "block_scores"
    _require_cuda(fn, qhat, khat)
    if qhat.dtype != torch.float32 or khat.dtype != torch.float32:
        raise TypeError(f"{fn}: pooled vectors must be float32")
    if qhat.ndim != 3 or khat.ndim != 3 or qhat.shape[0] != khat.shape[0] \
            or qhat.shape[2] != khat.shape[2]:
        raise ValueError(f"{fn}: shapes {tuple(qhat.shape)} / {tuple(khat.shape)}")
    qhat = qhat.contiguous()
    khat = khat.contiguous()
    nbh, nq, d = qhat.shape
    nk = khat.shape[1]
    score = torch.empty(nbh, nq, nk, device=qhat.device, dtype=torch.float32)
    check(_lib.load().rcsa_block_scores(qhat.data_ptr(), khat.data_ptr(), nbh, nq, nk, d,
                                        score.data_ptr(), _stream()), fn)
    return score


def _mask_u8(mask: Optional[torch.Tensor], nbh: int, nq: int, nk: int, device, fn: str):
    """Return (uint8 mask, head stride) for a [NQ, NK] or [NBH, NQ, NK] mask."""
    if mask is None:
        return None, 0
    m = _bytes_mask(mask, device)
    if m.shape == (nq, nk):
        return m.contiguous(), 0
    if m.shape == (nbh, nq, nk):
        return m.contiguous(), nq * nk
    raise ValueError(f"{fn}: mask shape {tuple(mask.shape)} is neither [{nq}, {nk}] "
                     f"nor [{nbh}, {nq}, {nk}]")


def select_topk(score: torch.Tensor, k, *, forced: Optional[torch.Tensor] = None,
                allowed: Optional[torch.Tensor] = None, max_k: Optional[int] = None,
                order: str = "index"):
    """Fixed-budget top-k over key blocks for every (bh, query block) row.

    Order of preference: forced, then score descending, then block index
    ascending (the stable-argsort tie rule of
    P/qk_uncertainty_tangent_attention.py:978-980).  ``k`` is an int, or an
    int tensor of shape [NQ] (shared by heads) or [NBH, NQ].  Returns
    ``(indices int32 [NBH, NQ, max_k], counts int32 [NBH, NQ])``; unused
    slots hold -1.
    """
    fn = "select_topk"
    _require_cuda(fn, score)
    if score.dtype != torch.float32 or score.ndim != 3:
        raise TypeError(f"{fn}: score must be float32 [NBH, NQ, NK]")
    score = score.contiguous()
    nbh, nq, nk = score.shape
    row_k, stride, k_fixed, max_k, fm, am, mstride = _selection_args(
        nbh, nq, nk, k, forced, allowed, max_k, order, score.device, fn)
    indices = torch.empty(nbh, nq, max_k, device=score.device, dtype=torch.int32)
    counts = torch.empty(nbh, nq, device=score.device, dtype=torch.int32)
    st = _lib.load().rcsa_select_topk(
        score.data_ptr(), nbh, nq, nk, _ptr(row_k), stride, k_fixed, _ptr(fm), _ptr(am),
        mstride, indices.data_ptr(), max_k, counts.data_ptr(),
        RCSA_ORDER_RANK if order == "rank" else RCSA_ORDER_INDEX, _stream())
    check(st, fn)
    return indices, counts


def _selection_args(nbh, nq, nk, k, forced, allowed, max_k, order, device, fn):
    """(row_k, row_k stride, k_fixed, max_k, forced u8, allowed u8, mask stride) for the
    selection ABI."""
    if isinstance(k, int):
        row_k, stride, k_fixed = None, 0, int(k)
        kmax = int(k)
    else:
        kt = torch.as_tensor(k)
        if kt.shape == (nq,):
            stride = 0
        elif kt.shape == (nbh, nq):
            stride = nq
        else:
            raise ValueError(f"{fn}: k tensor shape {tuple(kt.shape)}")
        if max_k is None:
            kmax = int(kt.max().item())  # host read of the budget; pass max_k to avoid it
        else:
            kmax = int(max_k)
        row_k = kt.to(device=device, dtype=torch.int32).contiguous()
        k_fixed = 0
    if max_k is None:
        max_k = max(1, min(kmax, nk))
    if order not in ("index", "rank"):
        raise ValueError(f"{fn}: order must be 'index' or 'rank'")
    fm, fstride = _mask_u8(forced, nbh, nq, nk, device, fn)
    am, astride = _mask_u8(allowed, nbh, nq, nk, device, fn)
    if fm is not None and am is not None and fstride != astride:
        # the ABI shares one head stride between the masks: broadcast both
        fm = fm.expand(nbh, nq, nk).contiguous() if fstride == 0 else fm
        am = am.expand(nbh, nq, nk).contiguous() if astride == 0 else am
        fstride = astride = nq * nk
    mstride = fstride if fm is not None else astride
    return row_k, stride, k_fixed, max_k, fm, am, mstride


def quantize_key_select(k, valid, block_size, ksum, kmin, kmax, qhat, khat, k_select, *,
                        forced=None, allowed=None, max_k=None, slot_token=None):
    """``quantize_key`` + ``block_scores`` + ``select_topk(order="index")`` with the key
    quantiser and the selection in one launch (no reference counterpart: the int8 layer
    call's form).  Returns ``(k_i8, k_scale, kmean, score, indices, counts)``, bit for bit
    those of the separate calls.  Raises ``NotImplementedError`` for shapes the fused
    launch does not cover (use the separate calls)."""
    fn = "quantize_key_select"
    _require_cuda(fn, k, ksum, kmin, kmax, qhat, khat)
    code = _dtype_code(k, fn)
    if slot_token is not None:
        sm = _slot_map(slot_token, block_size, k.device, fn)
        B, H, L, D, NB, src_len, strides = _tokens_bhld(k, sm, block_size, fn)
    else:
        sm, src_len = None, 0
        B, H, L, D, NB = _bhld(k, block_size, fn)
        strides = (k.stride(0), k.stride(1), k.stride(2))
    if not (k.dtype == torch.bfloat16 and D == 128 and block_size == 128 and NB <= 1024):
        raise NotImplementedError(f"{fn}: fused launch needs bf16 keys, D 128, 128-key "
                                  "blocks and at most 1024 blocks")
    for t in (ksum, kmin, kmax):
        if t.shape != (B * H, NB, D) or t.dtype != torch.float32 or not t.is_contiguous():
            raise ValueError(f"{fn}: statistics must be contiguous float32 [{B * H}, {NB}, {D}]")
    nbh, nq = B * H, qhat.shape[1]
    for name, t, rows in (("qhat", qhat, nq), ("khat", khat, NB)):
        if t.shape != (nbh, rows, D) or t.dtype != torch.float32 or not t.is_contiguous():
            raise ValueError(f"{fn}: {name} must be contiguous float32 [{nbh}, {rows}, {D}]")
    row_k, stride, k_fixed, max_k, fm, am, mstride = _selection_args(
        nbh, nq, NB, k_select, forced, allowed, max_k, "index", k.device, fn)
    v = _valid_u8(valid, L, k.device, fn)
    kmean = torch.empty(nbh, D, device=k.device, dtype=torch.float32)
    k_i8 = torch.empty(B, H, L, D, device=k.device, dtype=torch.int8)
    k_scale = torch.empty(nbh, NB, device=k.device, dtype=torch.float32)
    score = torch.empty(nbh, nq, NB, device=k.device, dtype=torch.float32)
    indices = torch.empty(nbh, nq, max_k, device=k.device, dtype=torch.int32)
    counts = torch.empty(nbh, nq, device=k.device, dtype=torch.int32)
    # through the torch extension (rcsa::quantize_key_select -> rcsa_quantize_key_select)
    _lib.torch_ops().quantize_key_select(
        k, code, [B, H, NB, block_size, D], list(strides), v, sm, src_len, ksum, kmin, kmax,
        kmean, k_i8, k_scale, qhat, khat, nq, score, row_k, stride, k_fixed, fm, am, mstride,
        indices, max_k, counts)
    return k_i8, k_scale, kmean, score, indices, counts


def quantize_key(k: torch.Tensor, valid: Optional[torch.Tensor], block_size: int,
                 ksum: torch.Tensor, kmin: torch.Tensor, kmax: torch.Tensor, *,
                 slot_token: Optional[torch.Tensor] = None):
    """Per-head mean-smoothed, per-block symmetric int8 keys.

    Returns ``(k_i8 [B, H, L, D], k_scale [B*H, NB], kmean [B*H, D])``.  With
    ``slot_token`` k is a token-major ``[B, L_tokens, H, D]`` source gathered on the
    fly (as in :func:`pool_query_key`); k_i8 stays packed ``[B, H, n_slots, D]``.
    """
    fn = "quantize_key"
    _require_cuda(fn, k, ksum, kmin, kmax)
    code = _dtype_code(k, fn)
    if slot_token is not None:
        sm = _slot_map(slot_token, block_size, k.device, fn)
        B, H, L, D, NB, src_len, strides = _tokens_bhld(k, sm, block_size, fn)
    else:
        sm, src_len = None, 0
        B, H, L, D, NB = _bhld(k, block_size, fn)
        strides = (k.stride(0), k.stride(1), k.stride(2))
    for t in (ksum, kmin, kmax):
        if t.shape != (B * H, NB, D) or t.dtype != torch.float32 or not t.is_contiguous():
            raise ValueError(f"{fn}: statistics must be contiguous float32 [{B * H}, {NB}, {D}]")
    v = _valid_u8(valid, L, k.device, fn)
    kmean = torch.empty(B * H, D, device=k.device, dtype=torch.float32)
    k_i8 = torch.empty(B, H, L, D, device=k.device, dtype=torch.int8)
    k_scale = torch.empty(B * H, NB, device=k.device, dtype=torch.float32)
    st = _lib.load().rcsa_quantize_key(
        k.data_ptr(), code, B, H, NB, block_size, D, *strides,
        _ptr(v), _ptr(sm), src_len, ksum.data_ptr(), kmin.data_ptr(), kmax.data_ptr(),
        kmean.data_ptr(),
        k_i8.data_ptr(), k_scale.data_ptr(), _stream())
    check(st, fn)
    return k_i8, k_scale, kmean


def _attn_common(q, k, v, indices, counts, fn):
    for name, t in (("q", q), ("k", k), ("v", v)):
        if t.ndim != 4 or t.stride(3) != 1:
            raise ValueError(f"{fn}: {name} must be [B, H, L, D] with contiguous last dim")
    if indices.ndim != 4 or counts.ndim != 3:
        raise ValueError(f"{fn}: indices must be [B, H, NQB, maxK], lens [B, H, NQB]")
    if indices.dtype != torch.int32 or counts.dtype != torch.int32:
        raise TypeError(f"{fn}: indices/lens must be int32")
    if indices.stride(3) != 1:
        raise ValueError(f"{fn}: indices last dim must be contiguous")


def _split_plan(B, H, Lq, D, block_m, max_k, n_split, device, fn):
    """(n_split, workspace tensor or None, workspace bytes) for a split launch.

    ``n_split=None`` asks the library for the count that fills the device's
    compute units best (rcsa_attn_split_plan); the workspace holds the
    partial results that the merge pass combines."""
    lib = _lib.load()
    if n_split is None:
        ns = ctypes.c_int64(1)
        check(lib.rcsa_attn_split_plan(B, H, Lq, block_m, max_k, ctypes.byref(ns)), fn)
        n_split = ns.value
    n_split = int(n_split)
    if n_split < 1:
        raise ValueError(f"{fn}: n_split must be >= 1")
    if n_split == 1:
        return 1, None, 0
    nbytes = int(lib.rcsa_attn_workspace_bytes(B, H, Lq, D, n_split))
    return n_split, torch.empty(nbytes, dtype=torch.uint8, device=device), nbytes


def _expand_lists(indices, counts, B, H):
    # the reference expands a [1, 1, N, K] layout over (B, H) (stride 0 views)
    return indices.expand(B, H, -1, -1), counts.expand(B, H, -1)


def _check_block_mask(block_mask, Lk, block_n, device, fn):
    """The key-validity bits as the kernels read them: int32 [ceil(Lk / block_n),
    block_n // 32], contiguous, on ``device``."""
    nkb = -(-Lk // block_n)
    if block_mask.dtype != torch.int32 or block_mask.device != device \
            or block_mask.numel() < nkb * (block_n // 32):
        raise ValueError(f"{fn}: block_mask must be int32 [{nkb}, {block_n // 32}] "
                         "on the same device")
    return block_mask.contiguous()


def valid_bits(valid: torch.Tensor, block_size: int) -> torch.Tensor:
    """Per-key validity flags ``[n_blocks * block_size]`` as the attention's
    ``block_mask``: int32 ``[n_blocks, block_size // 32]``, bit i of word w of
    block n = key n * block_size + 32 w + i (the form the key pooling pass writes)."""
    if block_size % 32 or valid.numel() % block_size:
        raise ValueError("valid_bits: block_size must be a multiple of 32 dividing the keys")
    words = (valid.reshape(-1, block_size // 32, 32) != 0).to(torch.int64)
    bits = (words << torch.arange(32, device=valid.device)).sum(-1)
    return torch.where(bits >= 2 ** 31, bits - 2 ** 32, bits).to(torch.int32)


def _bhld_strides(x: torch.Tensor, token_major: bool):
    """(stride_b, stride_h, stride_row) of [B, H, L, D] or token-major [B, L, H, D]."""
    return ((x.stride(0), x.stride(2), x.stride(1)) if token_major
            else (x.stride(0), x.stride(1), x.stride(2)))


def sparse_attn_bf16(q, k, v, indices, counts, valid=None, *, block_m=128, block_n=128,
                     sm_scale=None, return_lse=False, out=None, n_split=None,
                     block_mask=None, q_token=None, kv_token=None, out_token=None,
                     out_len=None):
    """bf16 block-sparse attention; the ``_attn_fwd_bsa_align`` contract.

    q/k/v [B, H, L, D] bf16, indices int32 [B|1, H|1, NQB, maxK], counts
    int32 [B|1, H|1, NQB], valid: per key token (K_LEN entries) or None.
    ``block_mask`` (the key validity as bits, as :func:`pool_key` writes it)
    replaces ``valid`` when given.
    ``n_split`` splits every block list over that many workgroups (merged
    afterwards); None picks it from the device's compute-unit count.

    ``q_token`` / ``kv_token`` (slot -> token maps of the packed query and key
    slots, both or neither; needs ``block_mask``, D 128, 128-token blocks):
    q is token-major ``[B, Lq_tokens, H, D]`` and k, v ``[B, Lk_tokens, H, D]``;
    the kernel reads their rows through the maps (the q[:, flat] / k[:, flat] /
    v[:, flat] packing of P/matrix_curvature_phase_frame_weave.py:5677-5684)
    and writes the output (and LSE) to the token rows, ``[B, Lq_tokens, H, D]``
    (P/matrix_curvature_phase_frame_weave.py:6095).  Empty slots read zeros.
    ``out_token`` / ``out_len`` (with the maps) write output row r to row
    ``out_token[r]`` of ``[B, out_len, H, D]`` instead, e.g. a relay layer's
    query-frame rows (P/matrix_curvature_phase_frame_weave.py:8990-8994).
    """
    fn = "sparse_attn_bf16"
    _require_cuda(fn, q, k, v, indices, counts)
    _attn_common(q, k, v, indices, counts, fn)
    if q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16:
        raise TypeError(f"{fn}: q/k/v must be bfloat16")
    if (q_token is None) != (kv_token is None):
        raise ValueError(f"{fn}: give both slot maps or neither")
    gathered = q_token is not None
    if gathered:
        if block_mask is None:
            raise ValueError(f"{fn}: gathered sources need block_mask")
        qm = _slot_map(q_token, block_m, q.device, fn)
        km = _slot_map(kv_token, block_n, q.device, fn)
        B, n_qtok, H, D = q.shape
        n_ktok = k.shape[1]
        Lq, Lk = qm.numel(), km.numel()
        if k.shape != (B, n_ktok, H, D) or v.shape != (B, n_ktok, H, D):
            raise ValueError(f"{fn}: k/v must be token-major [B, Lk_tokens, H, D] alike")
        if out_token is not None:
            om = _slot_map(out_token, block_m, q.device, fn)
            if om.numel() != Lq or out_len is None or int(out_len) <= 0:
                raise ValueError(f"{fn}: out_token needs {Lq} slots and a positive out_len")
            n_out = int(out_len)
        else:
            om, n_out = None, n_qtok
    else:
        if out_token is not None:
            raise ValueError(f"{fn}: out_token needs the gathered form")
        qm = km = om = None
        n_qtok = n_ktok = n_out = 0
        B, H, Lq, D = q.shape
        Lk = k.shape[2]
        if k.shape != (B, H, Lk, D) or v.shape != (B, H, Lk, D):
            raise ValueError(f"{fn}: k/v shape mismatch")
    indices, counts = _expand_lists(indices, counts, B, H)
    if block_mask is not None:
        block_mask = _check_block_mask(block_mask, Lk, block_n, q.device, fn)
        kv = None
    else:
        kv = _valid_u8(valid, Lk, q.device, fn)
    n_rows = n_out if gathered else Lq
    if out is None:
        out = (torch.empty(B, n_out, H, D, device=q.device, dtype=torch.bfloat16) if gathered
               else torch.empty_like(q, memory_format=torch.contiguous_format))
    elif gathered and (out.shape != (B, n_out, H, D) or out.dtype != torch.bfloat16):
        raise ValueError(f"{fn}: out must be bfloat16 [{B}, {n_out}, {H}, {D}]")
    lse = torch.empty(B, H, n_rows, device=q.device, dtype=torch.float32) if return_lse else None
    scale = 1.0 / math.sqrt(D) if sm_scale is None else float(sm_scale)
    ns, ws, nbytes = _split_plan(B, H, Lq, D, block_m, indices.shape[3], n_split, q.device, fn)
    # through the torch extension (rcsa::sparse_attn_bf16 -> rcsa_sparse_attn_bf16_split)
    _lib.torch_ops().sparse_attn_bf16(
        q, k, v, kv, block_mask, scale, lse, out, indices, counts,
        [B, H, Lq, Lk, D, block_m, block_n, indices.shape[3]],
        [*_bhld_strides(q, gathered), *_bhld_strides(k, gathered), *_bhld_strides(v, gathered),
         *_bhld_strides(out, gathered), *indices.stride()[:3], *counts.stride()[:3]],
        ns, ws, qm, n_qtok, km, n_ktok, om, n_out if om is not None else 0)
    return (out, lse) if return_lse else out


def sparse_attn_int8(q_i8, q_scale, k_i8, k_scale, v, indices, counts, valid=None, *,
                     block_m=128, block_n=128, sm_scale=None, return_lse=False, out=None,
                     n_split=None, block_mask=None, out_token=None, out_len=None,
                     v_token=None):
    """int8-QK / bf16-PV block-sparse attention over quantiser outputs.

    ``block_mask`` (int32 ``[ceil(Lk / block_n), block_n // 32]``, e.g. from
    ``pool_key(..., block_mask=True)``) gives the key validity as bits and
    replaces ``valid``.  ``out_token`` (a slot -> token map of the packed queries)
    scatters the output into a token-major ``[B, out_len, H, D]`` tensor (and the
    LSE into ``[B, H, out_len]``): ``unpack_tokens`` fused into the epilogue
    (P/matrix_curvature_phase_frame_weave.py:6095).  Every token must own a slot.
    ``v_token`` (a slot -> token map of the packed keys; needs ``block_mask``,
    D 128, 128-token blocks) reads V rows from a token-major ``[B, Lv_tokens, H, D]``
    v through the map inside the attention's copy ring (the v[:, flat] packing
    of P/matrix_curvature_phase_frame_weave.py:5677-5684); empty slots read zeros."""
    fn = "sparse_attn_int8"
    _require_cuda(fn, q_i8, q_scale, k_i8, k_scale, v, indices, counts)
    _attn_common(q_i8, k_i8, v, indices, counts, fn)
    if q_i8.dtype != torch.int8 or k_i8.dtype != torch.int8 or v.dtype != torch.bfloat16:
        raise TypeError(f"{fn}: q/k must be int8 and v bfloat16")
    B, H, Lq, D = q_i8.shape
    Lk = k_i8.shape[2]
    if v_token is not None:
        if block_mask is None:
            raise ValueError(f"{fn}: a gathered V needs block_mask")
        vm = _slot_map(v_token, block_n, q_i8.device, fn)
        if vm.numel() != Lk or v.ndim != 4 or v.shape[0] != B or v.shape[2:] != (H, D):
            raise ValueError(f"{fn}: v_token needs {Lk} slots and v [B, Lv_tokens, H, D]")
        v_rows = v.shape[1]
        v_strides = _bhld_strides(v, True)
    else:
        vm, v_rows = None, 0
        v_strides = _bhld_strides(v, False)
    if k_i8.shape != (B, H, Lk, D) or (vm is None and (
            v.shape[:2] != (B, H) or v.shape[3] != D or v.shape[2] < Lk)):
        raise ValueError(f"{fn}: k/v shape mismatch")
    nqb = -(-Lq // block_m)
    nkb = -(-Lk // block_n)
    if q_scale.dtype != torch.float32 or k_scale.dtype != torch.float32:
        raise TypeError(f"{fn}: scales must be float32")
    q_scale = q_scale.reshape(B * H, -1).contiguous()
    k_scale = k_scale.reshape(B * H, -1).contiguous()
    if q_scale.shape[1] < nqb or k_scale.shape[1] < nkb:
        raise ValueError(f"{fn}: need {nqb} query and {nkb} key scales per head")
    indices, counts = _expand_lists(indices, counts, B, H)
    if block_mask is not None:
        block_mask = _check_block_mask(block_mask, Lk, block_n, q_i8.device, fn)
        kv = None
    else:
        kv = _valid_u8(valid, Lk, q_i8.device, fn)
    if out_token is not None:
        om = _slot_map(out_token, block_m, q_i8.device, fn)
        if om.numel() < Lq or out_len is None or int(out_len) <= 0:
            raise ValueError(f"{fn}: out_token needs {Lq} slots and a positive out_len")
        n_out = int(out_len)
        if out is None:
            out = torch.empty(B, n_out, H, D, device=q_i8.device, dtype=torch.bfloat16)
        if out.shape != (B, n_out, H, D) or out.dtype != torch.bfloat16 or out.stride(3) != 1:
            raise ValueError(f"{fn}: out must be bfloat16 [{B}, {n_out}, {H}, {D}]")
        o_strides = (out.stride(0), out.stride(2), out.stride(1))
    else:
        om, n_out = None, 0
        if out is None:
            out = torch.empty(B, H, Lq, D, device=q_i8.device, dtype=torch.bfloat16)
        o_strides = (out.stride(0), out.stride(1), out.stride(2))
    lse = (torch.empty(B, H, n_out if om is not None else Lq, device=q_i8.device,
                       dtype=torch.float32) if return_lse else None)
    scale = 1.0 / math.sqrt(D) if sm_scale is None else float(sm_scale)
    ns, ws, nbytes = _split_plan(B, H, Lq, D, block_m, indices.shape[3], n_split, q_i8.device, fn)
    # through the torch extension (rcsa::sparse_attn_int8 -> rcsa_sparse_attn_int8_split)
    _lib.torch_ops().sparse_attn_int8(
        q_i8, q_scale, q_scale.shape[1], k_i8, k_scale, k_scale.shape[1], v, kv, block_mask,
        scale, lse, out, indices, counts,
        [B, H, Lq, Lk, D, block_m, block_n, indices.shape[3]],
        [*q_i8.stride()[:3], *k_i8.stride()[:3], *v_strides, *o_strides,
         *indices.stride()[:3], *counts.stride()[:3]],
        ns, ws, om, n_out, vm, v_rows)
    return (out, lse) if return_lse else out


def pack_tokens(x: torch.Tensor, slot_token: torch.Tensor) -> torch.Tensor:
    """Gather ``x [B, L, H, D]`` into packed ``[B, H, n_slots, D]`` (x's dtype); slot -1 -> zeros.

    Mirrors ``q[:, flat].transpose(1, 2).contiguous(); q_packed[:, :, ~mask] = 0``
    (P/matrix_curvature_phase_frame_weave.py:5671-5684).
    """
    fn = "pack_tokens"
    _require_cuda(fn, x)
    code = _dtype_code(x, fn)
    if x.ndim != 4 or x.stride(3) != 1:
        raise ValueError(f"{fn}: x must be [B, L, H, D] with contiguous last dim")
    B, L, H, D = x.shape
    st_ = slot_token.to(device=x.device, dtype=torch.int64).contiguous()
    n_slots = st_.numel()
    out = torch.empty(B, H, n_slots, D, device=x.device, dtype=x.dtype)
    check(_lib.load().rcsa_pack_tokens(x.data_ptr(), code, B, L, H, D, x.stride(0),
                                       x.stride(1), x.stride(2), st_.data_ptr(), n_slots,
                                       out.data_ptr(), _stream()), fn)
    return out


def unpack_tokens(packed: torch.Tensor, token_slot: torch.Tensor) -> torch.Tensor:
    """``out[b, t, h] = packed[b, h, token_slot[t]]`` (P/matrix_curvature_phase_frame_weave.py:6095)."""
    fn = "unpack_tokens"
    _require_cuda(fn, packed)
    if packed.dtype != torch.bfloat16 or packed.ndim != 4:
        raise TypeError(f"{fn}: packed must be bfloat16 [B, H, n_slots, D]")
    packed = packed.contiguous()
    B, H, n_slots, D = packed.shape
    ts = token_slot.to(device=packed.device, dtype=torch.int64).contiguous()
    L = ts.numel()
    out = torch.empty(B, L, H, D, device=packed.device, dtype=torch.bfloat16)
    check(_lib.load().rcsa_unpack_tokens(packed.data_ptr(), B, H, n_slots, D, ts.data_ptr(),
                                         L, out.data_ptr(), _stream()), fn)
    return out


def route_proxy(score: torch.Tensor, pooled_value: torch.Tensor, local: torch.Tensor,
                selected: torch.Tensor, counts: torch.Tensor, *, memory_blocks: int,
                n_cand: int, cand_mult: int, sketch_groups: int, eps: float = 1e-6):
    """Candidates, omission proxies and errors of the current rows (``rcsa_route_proxy``).

    score [B, H, N, N] fp32, pooled_value [B, H, N, D] fp32, local [N, N] bool,
    selected [B, H, N, K] and counts [B, H, N] (any integer dtype).  Returns
    (cand int32 [B*H, R, n_cand], proxy fp32 [B*H, R, n_cand, G], error fp32
    [B*H, R, G]) with R = N - memory_blocks (P/fc_pasm_swap_routing.py:64-106, 826-868).
    """
    fn = "route_proxy"
    _require_cuda(fn, score, pooled_value, selected, counts)
    B, H, N, N2 = score.shape
    if N2 != N or pooled_value.shape[:3] != (B, H, N) or selected.shape[:3] != (B, H, N) \
            or counts.shape != (B, H, N) or tuple(local.shape) != (N, N):
        raise ValueError(f"{fn}: score [B, H, N, N], values [B, H, N, D], selected "
                         "[B, H, N, K], counts [B, H, N] and local [N, N] must agree")
    D, K, G = pooled_value.shape[3], selected.shape[3], int(sketch_groups)
    R = N - int(memory_blocks)
    dev = score.device
    sc = score.float().contiguous()
    pv = pooled_value.float().contiguous()
    lo = _bytes_mask(local, dev)
    sel = selected.to(torch.int32).contiguous()
    cnt = counts.to(torch.int32).contiguous()
    cand = torch.empty(B * H, max(R, 0), n_cand, device=dev, dtype=torch.int32)
    proxy = torch.empty(B * H, max(R, 0), n_cand, G, device=dev, dtype=torch.float32)
    error = torch.empty(B * H, max(R, 0), G, device=dev, dtype=torch.float32)
    check(_lib.load().rcsa_route_proxy(
        sc.data_ptr(), pv.data_ptr(), lo.data_ptr(), sel.data_ptr(), cnt.data_ptr(), B * H, N,
        int(memory_blocks), D, K, int(n_cand), int(cand_mult), G, float(eps), cand.data_ptr(),
        proxy.data_ptr(), error.data_ptr(), _stream()), fn)
    return cand, proxy, error


def route_best_swap(proxy: torch.Tensor, cand: torch.Tensor, local: torch.Tensor,
                    selected: torch.Tensor, counts: torch.Tensor, coef: torch.Tensor,
                    linear: torch.Tensor, error: torch.Tensor, *, memory_blocks: int,
                    cand_mult: int, same_bank: bool, row_gate: Optional[torch.Tensor] = None):
    """Best single exchange of every current row (``rcsa_route_best_swap``):
    (best fp32 [B*H, R], flat int32 [B*H, R] = slot * n_cand + candidate, -1 if none)
    (P/fc_pasm_swap_routing.py:899-950)."""
    fn = "route_best_swap"
    _require_cuda(fn, proxy, cand, selected, counts, coef, linear, error)
    BH, R, L, G = proxy.shape
    B, H, N, K = selected.shape
    if B * H != BH or N - int(memory_blocks) != R or cand.shape != (BH, R, L) \
            or error.shape != (BH, R, G) or linear.reshape(-1).numel() != BH * R * G \
            or coef.reshape(-1).numel() != R:
        raise ValueError(f"{fn}: inconsistent proxy/candidate/selection shapes")
    dev = proxy.device
    sel = selected.to(torch.int32).contiguous()
    cnt = counts.to(torch.int32).contiguous()
    gate = _bytes_mask(row_gate, dev) if row_gate is not None else None
    best = torch.empty(BH, R, device=dev, dtype=torch.float32)
    flat = torch.empty(BH, R, device=dev, dtype=torch.int32)
    check(_lib.load().rcsa_route_best_swap(
        proxy.contiguous().data_ptr(), cand.contiguous().data_ptr(),
        _bytes_mask(local, dev).data_ptr(), sel.data_ptr(), cnt.data_ptr(),
        coef.float().contiguous().data_ptr(), linear.float().contiguous().data_ptr(),
        error.float().contiguous().data_ptr(), _ptr(gate), B * H, N, int(memory_blocks), K, L,
        int(cand_mult), G, int(bool(same_bank)), best.data_ptr(), flat.data_ptr(), _stream()), fn)
    return best, flat


def route_apply_swap(best: torch.Tensor, flat: torch.Tensor, cand: torch.Tensor,
                     proxy: torch.Tensor, selected: torch.Tensor, error: torch.Tensor,
                     state: torch.Tensor, *, memory_blocks: int, max_swaps: int, eps: float
                     ) -> None:
    """One swap round's decision and exchange on the device (``rcsa_route_apply_swap``,
    P/fc_pasm_swap_routing.py:935-977): the strongest row's exchange is written into
    ``selected`` (int32 [B, H, N, K], in place) and its error row ``error``
    (fp32 [B*H, R, G], in place) unless ``state`` (int32 [2 + 6 * rounds], zero
    before the first round) says the refinement stopped, ``max_swaps`` (> 0) swaps
    are done or the best value is not below ``-eps``.  Nothing is read back."""
    fn = "route_apply_swap"
    _require_cuda(fn, best, flat, cand, proxy, selected, error, state)
    BH, R, L, G = proxy.shape
    B, H, N, K = selected.shape
    if (best.shape != (BH, R) or flat.shape != (BH, R) or cand.shape != (BH, R, L)
            or error.shape != (BH, R, G) or B * H != BH or N - int(memory_blocks) != R):
        raise ValueError(f"{fn}: inconsistent best/candidate/selection shapes")
    for name, t, dt in (("best", best, torch.float32), ("flat", flat, torch.int32),
                        ("cand", cand, torch.int32), ("proxy", proxy, torch.float32),
                        ("selected", selected, torch.int32), ("error", error, torch.float32),
                        ("state", state, torch.int32)):
        if t.dtype != dt or not t.is_contiguous():
            raise ValueError(f"{fn}: {name} must be contiguous {dt}")
    records = (state.numel() - 2) // 6
    if records < 1 or state.numel() != 2 + 6 * records:
        raise ValueError(f"{fn}: state must hold 2 + 6 * rounds int32 entries")
    check(_lib.load().rcsa_route_apply_swap(
        best.data_ptr(), flat.data_ptr(), cand.data_ptr(), proxy.data_ptr(), selected.data_ptr(),
        error.data_ptr(), state.data_ptr(), BH, N, int(memory_blocks), K, L, G, int(max_swaps),
        records, float(eps), _stream()), fn)


def route_check(base: torch.Tensor, selected: torch.Tensor, counts: torch.Tensor,
                local: torch.Tensor, *, memory_blocks: int) -> torch.Tensor:
    """The checks at the end of a refine as device sums (``rcsa_route_check``,
    P/fc_pasm_swap_routing.py:983-1033): int32 [10] = (rows whose memory-bank count
    changed, rows with a repeated block, local edges kept, rows whose current-bank
    blocks changed, memory-bank entries before, after, max_k - smallest count,
    largest count, count sum, local edges of the stencil over all rows).  Nothing
    is read back."""
    fn = "route_check"
    _require_cuda(fn, base, selected, counts)
    B, H, N, K = selected.shape
    if base.shape != selected.shape or counts.shape != (B, H, N) or local.shape != (N, N):
        raise ValueError(f"{fn}: inconsistent route/count/stencil shapes")
    dev = selected.device
    b32 = base.to(torch.int32).contiguous()
    s32 = selected.to(torch.int32).contiguous()
    c32 = counts.to(torch.int32).contiguous()
    loc = _bytes_mask(local, dev)
    out = torch.zeros(10, device=dev, dtype=torch.int32)
    check(_lib.load().rcsa_route_check(b32.data_ptr(), s32.data_ptr(), c32.data_ptr(),
                                       loc.data_ptr(), B * H, N, int(memory_blocks), K,
                                       out.data_ptr(), _stream()), fn)
    return out


def quantize_rows_int8(x: torch.Tensor):
    """Per-token symmetric int8 quantisation of ``x [..., C]`` (``rcsa_quantize_rows_int8``):
    (q int8 [M, C], scale fp32 [M]) with M the product of the leading dims."""
    fn = "quantize_rows_int8"
    _require_cuda(fn, x)
    if x.dtype == torch.float16:
        x = x.float()
    code = _dtype_code(x, fn)
    x2 = x.reshape(-1, x.shape[-1])
    if x2.stride(1) != 1:
        x2 = x2.contiguous()
    M, C = x2.shape
    q = torch.empty(M, C, device=x.device, dtype=torch.int8)
    scale = torch.empty(M, device=x.device, dtype=torch.float32)
    _lib.torch_ops().quantize_rows_int8(x2, code, q, scale)
    return q, scale


def int8_linear(x_i8: torch.Tensor, x_scale: torch.Tensor, w_i8: torch.Tensor,
                w_scale: torch.Tensor, bias: Optional[torch.Tensor] = None,
                out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """bf16 ``(x_i8 @ w_i8^T) * x_scale[:, None] * w_scale[None, :] (+ bias)`` on int8
    MFMA (``rcsa_int8_linear``); x_i8 [M, K], w_i8 [N, K] int8."""
    fn = "int8_linear"
    _require_cuda(fn, x_i8, x_scale, w_i8, w_scale)
    if x_i8.dtype != torch.int8 or w_i8.dtype != torch.int8:
        raise TypeError(f"{fn}: x and w must be int8")
    x_i8, w_i8 = x_i8.contiguous(), w_i8.contiguous()
    M, K = x_i8.shape
    N, K2 = w_i8.shape
    if K2 != K:
        raise ValueError(f"{fn}: x [M, {K}] and w [N, {K2}] disagree")
    xs = x_scale.reshape(-1).float().contiguous()
    ws = w_scale.reshape(-1).float().contiguous()
    if xs.numel() != M or ws.numel() != N:
        raise ValueError(f"{fn}: need {M} token scales and {N} channel scales")
    b = bias.reshape(-1).to(torch.bfloat16).contiguous() if bias is not None else None
    if b is not None and b.numel() != N:
        raise ValueError(f"{fn}: bias must have {N} entries")
    if out is None:
        out = torch.empty(M, N, device=x_i8.device, dtype=torch.bfloat16)
    if out.dtype != torch.bfloat16 or out.shape != (M, N) or out.stride(1) != 1:
        raise ValueError(f"{fn}: out must be bfloat16 [{M}, {N}] with contiguous rows")
    _lib.torch_ops().int8_linear(x_i8, xs, w_i8, ws, b, out)
    return out

"""The RCSA layer call on one GPU: pool/score -> top-k -> quantise -> sparse attention.

This is the compute of ``_compact_cwca_attention``
(P/matrix_curvature_phase_frame_weave.py:5643-6095) between the packed
gather and the unpack, with the reference's torch eager pooling/top-k and
the external Triton kernel replaced by the HIP kernels of ``librcsa.so``.
Every launch is stream-ordered; nothing is read back to the host.

Once Q and K are pooled, the block scores and the top-k run on a side
stream of the same device, beside the key mean and the int8 K on the
caller's stream; the caller's stream waits for both before the attention.
The two small latency-bound kernels then overlap the HBM-bound key pass.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional

import torch

from . import ops

_SIDE_STREAMS: dict = {}


def _side_stream(device: torch.device) -> torch.cuda.Stream:
    """One side stream per device (default priority), created on first use."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    s = _SIDE_STREAMS.get(idx)
    if s is None:
        s = torch.cuda.Stream(device=idx)
        _SIDE_STREAMS[idx] = s
    return s


@dataclass
class RCSAResult:
    out: torch.Tensor                 # [B, H, Lq, D] bf16
    indices: torch.Tensor             # [B, H, NQB, max_k] int32
    counts: torch.Tensor              # [B, H, NQB] int32
    score: torch.Tensor               # [B*H, NQB, NKB] fp32
    qhat: torch.Tensor
    khat: torch.Tensor
    lse: Optional[torch.Tensor] = None
    q_i8: Optional[torch.Tensor] = None
    q_scale: Optional[torch.Tensor] = None
    k_i8: Optional[torch.Tensor] = None
    k_scale: Optional[torch.Tensor] = None
    kmean: Optional[torch.Tensor] = None
    k_mask: Optional[torch.Tensor] = None  # key validity bits (int8 path)


def rcsa_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                   q_valid: Optional[torch.Tensor], k_valid: Optional[torch.Tensor], *,
                   block_size: int, k_select, forced: Optional[torch.Tensor] = None,
                   allowed: Optional[torch.Tensor] = None, int8: bool = True,
                   max_k: Optional[int] = None, sm_scale: Optional[float] = None,
                   return_lse: bool = False, order: str = "index",
                   n_split: Optional[int] = None, overlap: bool = True,
                   q_slot_token: Optional[torch.Tensor] = None,
                   k_slot_token: Optional[torch.Tensor] = None,
                   fuse_select: bool = True) -> RCSAResult:
    """One RCSA layer call over packed Q/K/V ``[B, H, NB*BS, D]`` (bf16 or fp32).

    ``k_select`` is the per-row number of key blocks handed to attention
    (history budget + forced blocks such as the current chunk); ``forced``
    marks blocks that are always kept, ``allowed`` the causal permissions.
    With ``int8`` QK^T runs on int8 MFMA over smoothed per-block quantised
    Q/K; otherwise on bf16 MFMA.  ``n_split`` splits every block list over
    that many workgroups (None: chosen from the device's compute-unit count).
    ``fuse_select`` (int8, index order, bf16 keys of D 128 in 128-key blocks)
    scores and selects inside the key quantiser's launch; otherwise
    ``overlap`` runs the scores and the top-k on a side stream beside the
    int8 key pass.  Results are identical either way.

    ``q_slot_token`` / ``k_slot_token`` (both or neither; e.g. a
    ``CompactLayout.slot_token``): q, k and v are token-major ``[B, L, H, D]``
    and the packing happens inside the kernels.  The pooling pass (and the
    int8 key quantiser) gather Q/K rows through the maps, the attention's copy
    ring gathers V (bf16: also K, and Q rows) through them, and the attention
    writes its output (and LSE) straight to the token rows, so ``out`` is
    ``[B, Lq_tokens, H, D]``.  The results equal those of the packed call on
    ``pack_tokens`` inputs followed by ``unpack_tokens``.  (D 128 and 128-token
    blocks; other shapes pack V first.)
    """
    gathered = q_slot_token is not None or k_slot_token is not None
    v_token = None
    if gathered:
        if q_slot_token is None or k_slot_token is None:
            raise ValueError("rcsa_attention: give both slot maps or neither")
        B, _, H, D = q.shape
        dev = q.device
        q_slot_token = q_slot_token.to(device=dev, dtype=torch.int32).contiguous()
        k_slot_token = k_slot_token.to(device=dev, dtype=torch.int32).contiguous()
        Lq, Lk = q_slot_token.numel(), k_slot_token.numel()
        ring_gather = D == 128 and block_size == 128 and v.dtype == torch.bfloat16
        if not int8 and not ring_gather:
            raise ValueError("rcsa_attention: gathered bf16 inputs need D 128, "
                             "128-token blocks and bf16 sources")
        if ring_gather:
            v_token = k_slot_token  # V rows are read through the map by the attention
        else:
            v = ops.pack_tokens(v, k_slot_token)
    else:
        B, H, Lq, D = q.shape
        Lk = k.shape[2]
    bs = block_size
    main = torch.cuda.current_stream(q.device) if q.is_cuda else None
    # the bf16 path has no key pass left to overlap with
    side = _side_stream(q.device) if (overlap and int8 and q.is_cuda) else None

    def on_side(fn):
        if side is None:
            return fn()
        with torch.cuda.stream(side):
            return fn()

    if int8:  # one launch pools Q (+ int8) and K (+ stats and validity bits)
        qhat, q_i8, q_scale, khat, ksum, kmin, kmax, k_mask = ops.pool_query_key(
            q, q_valid, k, k_valid, bs, q_slot_token=q_slot_token, k_slot_token=k_slot_token)
    elif gathered:  # bf16: pooled blocks and validity bits, through the maps
        qhat, q_i8, q_scale, khat, ksum, kmin, kmax, k_mask = ops.pool_query_key(
            q, q_valid, k, k_valid, bs, q_slot_token=q_slot_token, k_slot_token=k_slot_token,
            quantize=False)
    else:  # the bf16 attention takes the key validity as bits from the key pooling pass
        qhat, q_i8, q_scale = ops.pool_query(q, q_valid, bs)
        khat, ksum, kmin, kmax, k_mask = ops.pool_key(k, k_valid, bs, block_mask=True)
    # int8 at the layer call's shape: the scores and the top-k run inside the
    # key quantiser's launch (one stream, no cross-stream waits)
    fused = (int8 and fuse_select and order == "index" and k.dtype == torch.bfloat16
             and D == 128 and bs == 128 and Lk // bs <= 1024)
    if fused:
        k_i8, k_scale, kmean, score, indices, counts = ops.quantize_key_select(
            k, k_valid, bs, ksum, kmin, kmax, qhat, khat, k_select, forced=forced,
            allowed=allowed, max_k=max_k, slot_token=k_slot_token)
    else:
        if side is not None:
            side.wait_stream(main)  # qhat and khat

        def score_and_select():
            sc = ops.block_scores(qhat, khat)
            return sc, ops.select_topk(sc, k_select, forced=forced, allowed=allowed,
                                       max_k=max_k, order=order)

        score, (indices, counts) = on_side(score_and_select)
        if int8:
            k_i8, k_scale, kmean = ops.quantize_key(k, k_valid, bs, ksum, kmin, kmax,
                                                    slot_token=k_slot_token)
        if side is not None:
            main.wait_stream(side)  # the selection
            # No record_stream: the side stream is private to this function and
            # every use of it starts after a wait on the caller's stream, so memory
            # freed on either stream is reused only after the other stream's use.
            # (Each recorded stream would add event packets between the kernels.)
    nqb = Lq // bs
    idx4 = indices.view(B, H, nqb, -1)
    cnt3 = counts.view(B, H, nqb)
    scale = 1.0 / math.sqrt(D) if sm_scale is None else sm_scale
    lse = None
    if int8:
        res = ops.sparse_attn_int8(q_i8, q_scale, k_i8, k_scale, v if v.dtype == torch.bfloat16
                                   else v.to(torch.bfloat16), idx4, cnt3, None,
                                   block_m=bs, block_n=bs, sm_scale=scale,
                                   return_lse=return_lse, n_split=n_split, block_mask=k_mask,
                                   out_token=q_slot_token if gathered else None,
                                   out_len=q.shape[1] if gathered else None, v_token=v_token)
    else:
        k_i8 = k_scale = kmean = None
        qb = q if q.dtype == torch.bfloat16 else q.to(torch.bfloat16)
        kb = k if k.dtype == torch.bfloat16 else k.to(torch.bfloat16)
        vb = v if v.dtype == torch.bfloat16 else v.to(torch.bfloat16)
        res = ops.sparse_attn_bf16(qb, kb, vb, idx4, cnt3, None, block_m=bs, block_n=bs,
                                   sm_scale=scale, return_lse=return_lse, n_split=n_split,
                                   block_mask=k_mask,
                                   q_token=q_slot_token if gathered else None,
                                   kv_token=k_slot_token if gathered else None)
    out, lse = res if return_lse else (res, None)
    return RCSAResult(out, idx4, cnt3, score, qhat, khat, lse, q_i8, q_scale, k_i8, k_scale,
                      kmean, k_mask)


def relay_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, layout, selected,
                    counts, *, int8: bool = True, sm_scale: Optional[float] = None,
                    return_lse: bool = False, n_split: Optional[int] = None):
    """The attention core of a causal frame-relay layer: the query-frame rows
    of a full-world layout attend to every key block the full-layout
    selection kept (MatrixCausalFrameLayerRelay._current_query_attention,
    P/matrix_curvature_phase_frame_weave.py:8966-8995, after its selector).

    q, k, v: token-major ``[B, S, H, D]`` over all ``S`` tokens of the frames;
    ``layout``: a :class:`cast_amd.layout.RelayLayout`; ``selected`` /
    ``counts``: the selection of every CWCA block ``[B, H, n_blocks, max_k]``
    / ``[B, H, n_blocks]`` (int32), of which the query blocks' rows are used.
    Returns the attention output of the query-frame tokens,
    ``[B, len(layout.query_indices), H, D]`` bf16 in ``query_indices`` order
    (and the LSE ``[B, H, n]`` with ``return_lse``).  No packed copy is made:
    the pooling/quantiser passes and the attention read Q, K and V through the
    layout's slot maps and write the output rows through its query map.
    D 128 and 128-token blocks.
    """
    B, S, H, D = q.shape
    bs = layout.block_size
    if D != 128 or bs != 128:
        raise ValueError("relay_attention: D 128 and 128-token blocks")
    if k.shape != q.shape or v.shape != q.shape:
        raise ValueError("relay_attention: q, k and v must be token-major [B, S, H, D] alike")
    rows = layout.query_block_ids.to(selected.device)
    idx = selected.index_select(2, rows).to(torch.int32).contiguous()
    cnt = counts.index_select(2, rows).to(torch.int32).contiguous()
    n_out = layout.query_indices.numel()
    scale = 1.0 / math.sqrt(D) if sm_scale is None else sm_scale
    if int8:
        # Q quantised over the query rows, K statistics and bits over the key rows
        _, q_i8, q_scale, _, ksum, kmin, kmax, k_mask = ops.pool_query_key(
            q, None, k, None, bs, q_slot_token=layout.query_slot_token,
            k_slot_token=layout.key_slot_token)
        k_i8, k_scale, _ = ops.quantize_key(k, None, bs, ksum, kmin, kmax,
                                            slot_token=layout.key_slot_token)
        v = v if v.dtype == torch.bfloat16 else v.to(torch.bfloat16)
        return ops.sparse_attn_int8(q_i8, q_scale, k_i8, k_scale, v, idx, cnt, None,
                                    block_m=bs, block_n=bs, sm_scale=scale,
                                    return_lse=return_lse, n_split=n_split,
                                    block_mask=k_mask, out_token=layout.query_out_row,
                                    out_len=n_out, v_token=layout.key_slot_token)
    qb, kb, vb = (x if x.dtype == torch.bfloat16 else x.to(torch.bfloat16) for x in (q, k, v))
    return ops.sparse_attn_bf16(qb, kb, vb, idx, cnt, None, block_m=bs, block_n=bs,
                                sm_scale=scale, return_lse=return_lse, n_split=n_split,
                                block_mask=layout.key_block_mask,
                                q_token=layout.query_slot_token,
                                kv_token=layout.key_slot_token,
                                out_token=layout.query_out_row, out_len=n_out)

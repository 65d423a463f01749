"""Packed block layout of the compact active frames, and the local stencil.

``compact_layout`` builds the slot map that the packed kernels consume
(``rcsa_pack_tokens`` / ``rcsa_unpack_tokens`` and every ``valid`` mask): the
same format as the compact CWCA layout of
P/matrix_curvature_phase_frame_weave.py:5223-5308: a block holds the
compact tokens whose (temporal cell, h tile, w tile) id is that block, in
increasing token order, then ``-1`` padding.  ``local_stencil`` is the
Manhattan <= 1 neighbourhood of P/matrix_curvature_phase_frame_weave.py:5703-5725
(native: P/qk_uncertainty_tangent_attention.py:1025-1039) that the selector
receives as its forced mask.  Both are computed once per shape with a few
vectorised torch ops on the target device and cached, as the reference
caches its layout.
"""
from __future__ import annotations

import functools
import math
from dataclasses import dataclass
from typing import Sequence

import torch


@dataclass(frozen=True)
class CompactLayout:
    block_shape: tuple[int, int, int]
    n_blocks: int
    block_size: int
    block_indices: torch.Tensor    # int64 [n_blocks, block_size], compact token or -1
    block_valid: torch.Tensor      # bool  [n_blocks, block_size]
    token_to_packed: torch.Tensor  # int64 [n_compact_tokens], packed slot of each token
    grid: tuple[int, int]          # (h tiles, w tiles)
    slot_token32: torch.Tensor     # int32 [n_blocks * block_size], the kernels' slot map

    @property
    def slot_token(self) -> torch.Tensor:
        """Flat slot -> source token map (-1 = invalid), the pack kernel's input."""
        return self.block_indices.reshape(-1)

    @property
    def slot_valid(self) -> torch.Tensor:
        """One validity byte per packed slot, the kernels' ``valid`` input."""
        return self.block_valid.reshape(-1)


def _block_ids(n_frames: int, n_memory: int, height: int, width: int,
               block_shape: tuple[int, int, int], device) -> tuple[torch.Tensor, int]:
    tt, th, tw = block_shape
    spatial = height * width
    nh, nw = math.ceil(height / th), math.ceil(width / tw)
    tok = torch.arange(n_frames * spatial, device=device)
    t, s = tok // spatial, tok % spatial
    if n_memory:
        # memory frames and current frames fill separate temporal cells
        mem_cells = math.ceil(n_memory / tt)
        cell = torch.where(t < n_memory, t // tt, mem_cells + (t - n_memory) // tt)
        n_cells = mem_cells + math.ceil((n_frames - n_memory) / tt)
    else:
        cell = t // tt
        n_cells = math.ceil(n_frames / tt)
    ids = cell * (nh * nw) + (s // width // th) * nw + (s % width) // tw
    return ids, n_cells * nh * nw


@functools.lru_cache(maxsize=64)
def _compact_layout_cached(frames: tuple[int, ...], memory_temporal: int, height: int,
                           width: int, block_shape: tuple[int, int, int],
                           device: str) -> CompactLayout:
    n_memory = sum(1 for f in frames if f < memory_temporal)
    ids, n_blocks = _block_ids(len(frames), n_memory, height, width, block_shape, device)
    bs = block_shape[0] * block_shape[1] * block_shape[2]
    n_tok = ids.numel()
    # counting sort by block id: the (id, token) keys are unique, so an
    # ordinary sort keeps tokens in increasing order inside each block
    order = torch.sort(ids * n_tok + torch.arange(n_tok, device=device)).indices
    sorted_ids = ids[order]
    per_block = torch.bincount(sorted_ids, minlength=n_blocks)
    if int(per_block.max()) > bs:
        raise RuntimeError("compact frame block exceeds its packed capacity")
    first = torch.cumsum(per_block, 0) - per_block
    rank = torch.arange(n_tok, device=device) - first[sorted_ids]
    slot = sorted_ids * bs + rank
    block_indices = torch.full((n_blocks * bs,), -1, dtype=torch.long, device=device)
    block_indices[slot] = order
    token_to_packed = torch.empty(n_tok, dtype=torch.long, device=device)
    token_to_packed[order] = slot
    block_indices = block_indices.reshape(n_blocks, bs)
    nh = math.ceil(height / block_shape[1])
    nw = math.ceil(width / block_shape[2])
    return CompactLayout(block_shape, n_blocks, bs, block_indices, block_indices >= 0,
                         token_to_packed, (nh, nw),
                         block_indices.reshape(-1).to(torch.int32).contiguous())


def compact_layout(active_frames: Sequence[int], memory_temporal: int, height: int,
                   width: int, block_shape: Sequence[int], device="cpu") -> CompactLayout:
    """Packed block map of the compact frames ``active_frames`` (frame ids of
    a ``height x width`` latent grid; frames below ``memory_temporal`` are
    memory frames and start their own temporal cells)."""
    frames = tuple(sorted(int(f) for f in active_frames))
    if not frames:
        raise ValueError("compact_layout: no active frames")
    shape = tuple(int(x) for x in block_shape)
    if len(shape) != 3 or min(shape) <= 0:
        raise ValueError(f"compact_layout: bad block shape {block_shape}")
    return _compact_layout_cached(frames, int(memory_temporal), int(height), int(width),
                                  shape, str(torch.device(device)))


@functools.lru_cache(maxsize=64)
def _stencil_cached(n_blocks: int, nh: int, nw: int, device: str) -> torch.Tensor:
    ids = torch.arange(n_blocks, device=device)
    spatial = nh * nw
    t, s = ids // spatial, ids % spatial
    h, w = s // nw, s % nw
    dist = ((t[:, None] - t[None, :]).abs() + (h[:, None] - h[None, :]).abs()
            + (w[:, None] - w[None, :]).abs())
    return dist <= 1


def local_stencil(n_blocks: int, nh: int, nw: int, device="cpu") -> torch.Tensor:
    """bool [n_blocks, n_blocks]: blocks at Manhattan distance <= 1 in
    (temporal cell, h tile, w tile) coordinates, block id = t*nh*nw + h*nw + w."""
    return _stencil_cached(int(n_blocks), int(nh), int(nw), str(torch.device(device)))


@dataclass(frozen=True)
class RelayLayout:
    """Full-world keys with a compact set of complete-frame queries: the
    asymmetric layout of a causal frame-relay layer
    (P/matrix_curvature_phase_frame_weave.py:72-86, 8734-8846).

    Keys are every token of ``total_temporal`` frames in the CWCA blocks
    (memory and current frames in separate temporal cells when the layout
    protects the current chunk); query block ``r`` is CWCA block
    ``query_block_ids[r]`` restricted to the tokens of the query frames.
    Slot maps hold token ids of the full sequence (-1 = empty slot).
    """
    block_size: int
    n_blocks: int
    key_slot_token: torch.Tensor    # int32 [n_blocks * block_size]
    key_valid: torch.Tensor         # bool  [n_blocks * block_size]
    key_block_mask: torch.Tensor    # int32 [n_blocks, block_size // 32], key_valid as bits
                                    # (empty unless block_size is a multiple of 32)
    query_block_ids: torch.Tensor   # int64 [n_query_blocks], sorted CWCA block ids
    query_slot_token: torch.Tensor  # int32 [n_query_blocks * block_size]
    query_valid: torch.Tensor       # bool  [n_query_blocks * block_size]
    query_indices: torch.Tensor     # int64 [n_query_tokens], tokens of the query frames
    query_out_row: torch.Tensor     # int32 [n_query_blocks * block_size], row in query_indices


def _bits32(valid: torch.Tensor, block_size: int) -> torch.Tensor:
    """bool [n * block_size] -> int32 [n, block_size // 32] (bit i of word w = slot 32 w + i)."""
    from .ops import valid_bits
    return valid_bits(valid, block_size)


def _slots_of(ids: torch.Tensor, members: torch.Tensor, n_rows: int, bs: int,
              row_of: torch.Tensor) -> torch.Tensor:
    """Slot of each member token: row_of[ids] * bs + rank among the row's
    members in increasing token order (members sorted by (row, token))."""
    n = members.numel()
    rows = row_of[ids]
    order = torch.sort(rows * (members.max() + 1 if n else 1) + members).indices
    sorted_rows = rows[order]
    per_row = torch.bincount(sorted_rows, minlength=n_rows)
    if n and int(per_row.max()) > bs:
        raise RuntimeError("CWCA block contains too many tokens")
    first = torch.cumsum(per_row, 0) - per_row
    slot = torch.empty_like(members)
    slot[order] = sorted_rows * bs + (torch.arange(n, device=members.device) - first[sorted_rows])
    return slot


@functools.lru_cache(maxsize=64)
def _relay_layout_cached(total_temporal: int, memory_temporal: int, height: int, width: int,
                         block_shape: tuple[int, int, int], query_frames: tuple[int, ...],
                         protected_current: bool, device: str) -> RelayLayout:
    tt, th, tw = block_shape
    spatial = height * width
    nh, nw = math.ceil(height / th), math.ceil(width / tw)
    tok = torch.arange(total_temporal * spatial, device=device)
    t, s = tok // spatial, tok % spatial
    tile = (s // width // th) * nw + (s % width) // tw
    mem = memory_temporal
    if protected_current:
        mem_blocks = math.ceil(mem / tt) * nh * nw if mem else 0
        cell_base = torch.where(t < mem, 0, mem_blocks)
        cell = torch.where(t < mem, t // tt, (t - mem) // tt)
        ids = cell_base + cell * nh * nw + tile
        n_blocks = mem_blocks + math.ceil((total_temporal - mem) / tt) * nh * nw
    else:
        ids = (t // tt) * nh * nw + tile
        n_blocks = math.ceil(total_temporal / tt) * nh * nw
    bs = tt * th * tw
    key_slot = _slots_of(ids, tok, n_blocks, bs, torch.arange(n_blocks, device=device))
    key_tok = torch.full((n_blocks * bs,), -1, dtype=torch.long, device=device)
    key_tok[key_slot] = tok
    is_query = torch.zeros(total_temporal, dtype=torch.bool, device=device)
    is_query[torch.tensor(query_frames, dtype=torch.long, device=device)] = True
    q_tok = tok[is_query[t]]
    q_ids = ids[q_tok]
    q_blocks = torch.unique(q_ids, sorted=True)
    row_of = torch.full((n_blocks,), -1, dtype=torch.long, device=device)
    row_of[q_blocks] = torch.arange(q_blocks.numel(), device=device)
    q_slot = _slots_of(q_ids, q_tok, q_blocks.numel(), bs, row_of)
    n_q = q_blocks.numel() * bs
    query_tok = torch.full((n_q,), -1, dtype=torch.long, device=device)
    query_tok[q_slot] = q_tok
    out_row = torch.full((n_q,), -1, dtype=torch.long, device=device)
    out_row[q_slot] = torch.arange(q_tok.numel(), device=device)
    key_valid = key_tok >= 0
    bits = (_bits32(key_valid, bs) if bs % 32 == 0
            else torch.empty(0, dtype=torch.int32, device=device))
    return RelayLayout(bs, n_blocks, key_tok.to(torch.int32), key_valid, bits,
                       q_blocks, query_tok.to(torch.int32), query_tok >= 0, q_tok,
                       out_row.to(torch.int32))


def relay_layout(total_temporal: int, memory_temporal: int, height: int, width: int,
                 block_shape: Sequence[int], query_frames: Sequence[int], *,
                 protected_current: bool = True, allow_memory_queries: bool = False,
                 device="cpu") -> RelayLayout:
    """The asymmetric layout of a causal frame-relay layer
    (``MatrixCausalFrameLayerRelay._asymmetric_layout``,
    P/matrix_curvature_phase_frame_weave.py:8734-8846): every token of the
    ``total_temporal`` frames as keys, the tokens of ``query_frames`` as
    queries in the blocks that hold them.  Query frames in memory raise
    unless ``allow_memory_queries`` (:8812-8813)."""
    frames = tuple(sorted({int(f) for f in query_frames}))
    shape = tuple(int(x) for x in block_shape)
    if len(shape) != 3 or min(shape) <= 0:
        raise ValueError(f"relay_layout: bad block shape {block_shape}")
    if not frames or frames[0] < 0 or frames[-1] >= total_temporal:
        raise ValueError("relay_layout: query frames must lie in [0, total_temporal)")
    if not allow_memory_queries and frames[0] < memory_temporal:
        raise RuntimeError("causal relay may not write Memory on a relay layer")
    return _relay_layout_cached(int(total_temporal), int(memory_temporal), int(height),
                                int(width), shape, frames, bool(protected_current),
                                str(torch.device(device)))

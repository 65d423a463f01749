"""Drop-ins for the reference's sparse-attention kernel wrappers.

``longcat_active`` keeps the argument meaning, casting and error behaviour of
``MatrixJiTSpatialAcceleration._longcat_active``
(P/matrix_jit_spatial_acceleration.py:663-729) and ``longcat_asymmetric``
those of ``MatrixCausalFrameLayerRelay._longcat_asymmetric``
(P/matrix_curvature_phase_frame_weave.py:8847-8917); both launch the gfx950
HIP kernel ``rcsa_sparse_attn_bf16`` instead of the external Triton
``_attn_fwd_bsa_align``.
"""
from __future__ import annotations

import torch

from . import ops


def longcat_active(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, indices: torch.Tensor,
                   counts: torch.Tensor, valid: torch.Tensor, block_size: int) -> torch.Tensor:
    """Block-sparse attention over packed ``[B, H, L, D]`` tensors.

    q/k/v are cast to bf16 and made contiguous; indices/counts to int32;
    ``valid`` (one flag per packed key token) to uint8.  The query grid is
    ceil(q_len / block_size) blocks of ``block_size`` rows, keys are read in
    ``block_size`` blocks.  Returns bf16 ``[B, H, Lq, D]``.
    """
    q = q.to(torch.bfloat16).contiguous()
    k = k.to(torch.bfloat16).contiguous()
    v = v.to(torch.bfloat16).contiguous()
    indices = indices.to(torch.int32).contiguous()
    counts = counts.to(torch.int32).contiguous()
    key_valid = valid.reshape(-1)
    if block_size % 32 == 0 and key_valid.numel() == k.shape[2] \
            and k.shape[2] % block_size == 0:
        # the validity as bits (32 keys a word): the attention then reads 8 bytes
        # per wavefront and block instead of staging the bytes (about 6% faster)
        return ops.sparse_attn_bf16(q, k, v, indices, counts, None, block_m=block_size,
                                    block_n=block_size,
                                    block_mask=ops.valid_bits(key_valid, block_size))
    return ops.sparse_attn_bf16(q, k, v, indices, counts, key_valid.to(torch.uint8).contiguous(),
                                block_m=block_size, block_n=block_size)


def longcat_asymmetric(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                       indices: torch.Tensor, counts: torch.Tensor, key_valid: torch.Tensor,
                       *, query_block_size: int, key_block_size: int) -> torch.Tensor:
    """Asymmetric query/key storage; both lengths must be block aligned."""
    q = q.to(torch.bfloat16).contiguous()
    k = k.to(torch.bfloat16).contiguous()
    v = v.to(torch.bfloat16).contiguous()
    indices = indices.to(torch.int32).contiguous()
    counts = counts.to(torch.int32).contiguous()
    valid = key_valid.reshape(-1).to(torch.uint8).contiguous()
    if q.shape[2] % query_block_size or k.shape[2] % key_block_size:
        raise RuntimeError("asymmetric sparse storage is not block aligned")
    return ops.sparse_attn_bf16(q, k, v, indices, counts, valid, block_m=query_block_size,
                                block_n=key_block_size)

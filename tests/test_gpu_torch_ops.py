"""The PyTorch-ROCm extension (torch.ops.rcsa) called directly, the way a
maintainer binds it in place of the reference's kernel launch: the same bits as
the Python wrappers, the caller's current stream, and host-side rejection of
bad arguments before any launch."""
import math

import pytest
import torch

from cast_amd import _lib, ops

pytestmark = pytest.mark.gpu


def _inputs(dev, seed=3, H=2, nqb=3, nkb=8, D=128, bs=128, max_k=4):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(1, H, nqb * bs, D, generator=g).bfloat16().to(dev)
    k = torch.randn(1, H, nkb * bs, D, generator=g).bfloat16().to(dev)
    v = torch.randn(1, H, nkb * bs, D, generator=g).bfloat16().to(dev)
    valid = torch.ones(nkb * bs, dtype=torch.uint8)
    valid[-37:] = 0  # a ragged last block
    idx = torch.stack([torch.randperm(nkb, generator=g)[:max_k] for _ in range(H * nqb)])
    idx = idx.reshape(1, H, nqb, max_k).int().to(dev)
    cnt = torch.randint(1, max_k + 1, (1, H, nqb), generator=g).int().to(dev)
    return q, k, v, valid.to(dev), idx, cnt


def _stub_call(q, k, v, key_valid, indices, counts, out, block_size, sm_scale=None):
    """The direct launch of the binding example: unsplit, no workspace, no maps."""
    B, H, Lq, D = q.shape
    torch.ops.rcsa.sparse_attn_bf16(
        q, k, v, key_valid, None, 1.0 / math.sqrt(D) if sm_scale is None else sm_scale, None,
        out, indices, counts,
        [B, H, Lq, k.shape[2], D, block_size, block_size, indices.shape[3]],
        [*q.stride()[:3], *k.stride()[:3], *v.stride()[:3], *out.stride()[:3],
         *indices.stride()[:3], *counts.stride()[:3]],
        1, None, None, 0, None, 0, None, 0)


def test_direct_op_matches_wrapper(dev):
    _lib.torch_ops()  # loads the extension and binds librcsa.so
    q, k, v, valid, idx, cnt = _inputs(dev)
    out = torch.empty_like(q)
    _stub_call(q, k, v, valid, idx, cnt, out, 128)
    want = ops.sparse_attn_bf16(q, k, v, idx, cnt, valid, n_split=1)
    torch.cuda.synchronize()
    assert torch.equal(out, want)


def test_direct_op_runs_on_the_current_stream(dev):
    _lib.torch_ops()
    q, k, v, valid, idx, cnt = _inputs(dev, seed=4)
    want = ops.sparse_attn_bf16(q, k, v, idx, cnt, valid, n_split=1)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    out = torch.full_like(q, float("nan"))
    with torch.cuda.stream(side):
        _stub_call(q, k, v, valid, idx, cnt, out, 128)
        done = torch.cuda.Event()
        done.record(side)
    done.synchronize()
    assert torch.equal(out, want)


def test_direct_op_rejects_bad_arguments(dev):
    rcsa = _lib.torch_ops()
    q, k, v, valid, idx, cnt = _inputs(dev, seed=5)
    out = torch.empty_like(q)
    with pytest.raises(RuntimeError, match=r"sparse_attn_bf16: q/k/v/out has dtype"):
        _stub_call(q.float(), k, v, valid, idx, cnt, out, 128)
    with pytest.raises(RuntimeError, match=r"sparse_attn_bf16: indices must be"):
        B, H, Lq, D = q.shape
        rcsa.sparse_attn_bf16(
            q, k, v, valid, None, 1.0 / math.sqrt(D), None, out, idx[0], cnt,
            [B, H, Lq, k.shape[2], D, 128, 128, idx.shape[3]],
            [*q.stride()[:3], *k.stride()[:3], *v.stride()[:3], *out.stride()[:3],
             *idx.stride()[:3], *cnt.stride()[:3]],
            1, None, None, 0, None, 0, None, 0)
    with pytest.raises(RuntimeError, match=r"int8_linear: x and w disagree on K"):
        x = torch.zeros(4, 192, dtype=torch.int8, device=dev)
        w = torch.zeros(256, 384, dtype=torch.int8, device=dev)
        rcsa.int8_linear(x, torch.ones(4, device=dev), w, torch.ones(256, device=dev), None,
                         torch.empty(4, 256, dtype=torch.bfloat16, device=dev))
    # dims that reach past a tensor are refused before any launch
    with pytest.raises(RuntimeError, match=r"sparse_attn_bf16: k spans \d+ elements, the call "
                                           r"reaches \d+"):
        B, H, Lq, D = q.shape
        ks = k[:, :, :512]
        rcsa.sparse_attn_bf16(
            q, ks, v, valid, None, 1.0 / math.sqrt(D), None, out, idx, cnt,
            [B, H, Lq, k.shape[2], D, 128, 128, idx.shape[3]],
            [*q.stride()[:3], *ks.stride()[:3], *v.stride()[:3], *out.stride()[:3],
             *idx.stride()[:3], *cnt.stride()[:3]],
            1, None, None, 0, None, 0, None, 0)
    with pytest.raises(RuntimeError, match=r"sparse_attn_bf16: k_valid spans"):
        _stub_call(q, k, v, valid[:100], idx, cnt, out, 128)
    with pytest.raises(RuntimeError, match=r"sparse_attn_bf16: indices spans"):
        B, H, Lq, D = q.shape
        rcsa.sparse_attn_bf16(
            q, k, v, valid, None, 1.0 / math.sqrt(D), None, out, idx, cnt,
            [B, H, Lq, k.shape[2], D, 128, 128, idx.shape[3]],
            [*q.stride()[:3], *k.stride()[:3], *v.stride()[:3], *out.stride()[:3],
             idx.stride(0), idx.stride(1), 2 * idx.stride(2), *cnt.stride()[:3]],
            1, None, None, 0, None, 0, None, 0)
    # a library status becomes the same RuntimeError form as the ctypes path
    with pytest.raises(RuntimeError, match=r"sparse_attn_bf16: .*\(status \d+\)"):
        _stub_call(q, k, v, valid, idx, cnt, out, 128, sm_scale=0.0)  # refused by the library

"""Shared int8 Q/K/V projection (GPU) against the oracle's restatement of
shared_int8_qkv (P/matrix_shared_int8_qkv.py:19-147): the per-token quantiser
and the int8 GEMM with its dequantising epilogue, bit for bit; the Matrix
projection shape (38,720 tokens x 3072 -> 3 x 3072) on sampled rows; the
forward coordinator's call order."""
from types import SimpleNamespace

import pytest
import torch

from oracle import rcsa_oracle as orc

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_quantize_rows_matches_oracle(dev, dtype):
    from cast_amd import ops
    g = torch.Generator().manual_seed(1)
    x = (torch.randn(1003, 3072, generator=g) * torch.rand(1003, 1, generator=g) * 4).to(dtype)
    x[5] = 0
    print(f"quantize rows {dtype}", flush=True)
    q, s = ops.quantize_rows_int8(x.to(dev))
    wq, ws = orc.quantize_rows_int8(x)
    torch.cuda.synchronize()
    assert torch.equal(q.cpu(), wq) and torch.equal(s.cpu(), ws)


@pytest.mark.parametrize("M", [77, 128, 1000])
@pytest.mark.parametrize("with_bias", [False, True])
def test_int8_linear_matches_oracle(dev, M, with_bias):
    from cast_amd import ops
    g = torch.Generator().manual_seed(M)
    N, K = 512, 384
    x = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8)
    w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    xs = torch.rand(M, generator=g) * 0.01 + 1e-4
    ws = torch.rand(N, generator=g) * 0.01 + 1e-4
    bias = torch.randn(N, generator=g).bfloat16() if with_bias else None
    print(f"int8 linear M {M} bias {with_bias}", flush=True)
    got = ops.int8_linear(x.to(dev), xs.to(dev), w.to(dev), ws.to(dev),
                          bias.to(dev) if bias is not None else None)
    torch.cuda.synchronize()
    assert torch.equal(got.cpu(), orc.int8_linear(x, xs, w, ws, bias))


def test_int8_linear_short_last_round(dev):
    """5800 x 3072 x 128: 23 row blocks x 12 channel blocks of 256 x 256 tiles
    leave a short last round on 256 compute units, so the last 424 rows run as
    128 x 128 tiles (the last one 40 rows); every output element against the
    oracle, bit for bit."""
    from cast_amd import ops
    g = torch.Generator().manual_seed(11)
    M, N, K = 5800, 3072, 128
    x = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8)
    w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    xs = torch.rand(M, generator=g) * 0.01 + 1e-4
    ws = torch.rand(N, generator=g) * 0.01 + 1e-4
    bias = torch.randn(N, generator=g).bfloat16()
    print("int8 linear 5800 x 3072 x 128", flush=True)
    got = ops.int8_linear(x.to(dev), xs.to(dev), w.to(dev), ws.to(dev), bias.to(dev))
    torch.cuda.synchronize()
    assert torch.equal(got.cpu(), orc.int8_linear(x, xs, w, ws, bias))


def _int8_module(g, c_out, c_in, dev):
    w = torch.randint(-127, 128, (c_out, c_in), generator=g, dtype=torch.int8)
    return SimpleNamespace(in_features=c_in, out_features=c_out, weight_int8=w.to(dev),
                           weight_scales=(torch.rand(c_out, generator=g) * 2e-3).to(dev),
                           bias=(torch.randn(c_out, generator=g) * 0.1).bfloat16().to(dev))


def test_shared_qkv_matrix_shape(dev):
    """38,720 tokens x 3072 channels into q, k, v of 3072: every output row of a
    sample against the oracle, bit for bit."""
    from cast_amd.qkv import shared_int8_qkv
    g = torch.Generator().manual_seed(3)
    C, L = 3072, 38720
    mods = [_int8_module(g, C, C, dev) for _ in range(3)]
    x = (torch.randn(1, L, C, generator=g) * 0.5).bfloat16()
    print("shared qkv 38720 x 3072", flush=True)
    outs = shared_int8_qkv(*mods, x.to(dev))
    torch.cuda.synchronize()
    rows = torch.randperm(L, generator=g)[:48].sort().values
    # and the rows at 128-row boundaries of the last 640 rows
    edge = [L - d for d in (640, 577, 576, 513, 512, 385, 384, 257, 256, 129, 128, 65, 64, 1)]
    rows = torch.unique(torch.cat([rows, torch.tensor([0] + edge)]))
    xq, xs = orc.quantize_rows_int8(x[0, rows])
    for m, o in zip(mods, outs):
        assert o.shape == (1, L, C) and o.dtype == torch.bfloat16
        want = orc.int8_linear(xq, xs, m.weight_int8.cpu(), m.weight_scales.cpu(), m.bias.cpu())
        assert torch.equal(o[0, rows].cpu(), want)


def test_forward_coordinator_order(dev):
    from cast_amd.qkv import SharedInt8QKVForwardCoordinator, shared_int8_qkv
    g = torch.Generator().manual_seed(4)
    C = 768  # channels a multiple of 256, the input width a multiple of 128
    mods = [_int8_module(g, C, C, dev) for _ in range(3)]
    for m in mods:
        m.forward = lambda x: None
    attn = SimpleNamespace(q=mods[0], k=mods[1], v=mods[2])
    coord = SharedInt8QKVForwardCoordinator(attn)
    coord.install()
    x = torch.randn(1, 300, C, generator=g).to(dev)
    got = (mods[0].forward(x), mods[1].forward(x), mods[2].forward(x))
    want = shared_int8_qkv(*mods, x)
    assert all(torch.equal(a, b) for a, b in zip(got, want))
    with pytest.raises(RuntimeError, match="in order"):
        mods[1].forward(x)
    coord.uninstall()
    assert mods[0].forward(x) is None

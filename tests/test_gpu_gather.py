"""Packing fused into the kernels: token-major Q/K/V through slot maps.

On the Matrix latent grid (22 x 40 tokens per frame, (4, 4, 8) tiles with
64-token bottom tiles; 4 query frames, 8 memory + 4 current key frames) the
gathered pooling pass, key quantiser and layer call must equal, bit for bit,
the same calls on ``pack_tokens`` inputs followed by ``unpack_tokens``
(P/matrix_curvature_phase_frame_weave.py:5677-5684 gathers, :6095 unpack).
"""
import pytest
import torch

pytestmark = pytest.mark.gpu

SHAPE = (4, 4, 8)
HW = (22, 40)


def _case(seed=5, H=4, D=128, dtype=torch.bfloat16):
    from cast_amd import layout
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(seed)
    lay_q = layout.compact_layout(range(4), 0, *HW, SHAPE, dev)
    lay_k = layout.compact_layout(range(12), 8, *HW, SHAPE, dev)
    lq, lk = 4 * HW[0] * HW[1], 12 * HW[0] * HW[1]
    q = (torch.randn(1, lq, H, D, generator=g) / D ** 0.5).to(dtype).to(dev)
    k = (torch.randn(1, lk, H, D, generator=g) / D ** 0.5)
    k[..., 3] *= 10.0  # an outlier channel, as in the int8 workloads
    k = k.to(dtype).to(dev)
    v = (torch.randn(1, lk, H, D, generator=g) / D ** 0.5).to(dtype).to(dev)
    return lay_q, lay_k, q, k, v


def _packed(x, lay):
    from cast_amd import ops
    return ops.pack_tokens(x, lay.slot_token)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_gathered_pooling_and_quantiser_match_packed(dtype):
    from cast_amd import ops
    lay_q, lay_k, q, k, v = _case(dtype=dtype)
    print(f"gather pooling {dtype} q {tuple(q.shape)} k {tuple(k.shape)}", flush=True)
    want = ops.pool_query_key(_packed(q, lay_q), lay_q.slot_valid, _packed(k, lay_k),
                              lay_k.slot_valid, 128)
    got = ops.pool_query_key(q, None, k, None, 128, q_slot_token=lay_q.slot_token,
                             k_slot_token=lay_k.slot_token)
    names = ("qhat", "q_i8", "q_scale", "khat", "ksum", "kmin", "kmax", "block_mask")
    for name, a, b in zip(names, want, got):
        assert a.shape == b.shape and torch.equal(a, b), name
    ks, kn, kx = want[4], want[5], want[6]
    qk_want = ops.quantize_key(_packed(k, lay_k), lay_k.slot_valid, 128, ks, kn, kx)
    qk_got = ops.quantize_key(k, None, 128, ks, kn, kx, slot_token=lay_k.slot_token)
    for name, a, b in zip(("k_i8", "k_scale", "kmean"), qk_want, qk_got):
        assert torch.equal(a, b), name
    # every empty slot is invalid and quantises to zero
    empty = lay_k.slot_token < 0
    assert int(empty.sum()) > 0
    assert int(qk_got[0][:, :, empty].abs().sum()) == 0


@pytest.mark.parametrize("n_split", [1, 3])
def test_gathered_layer_call_matches_pack_unpack(n_split):
    from cast_amd import ops
    from cast_amd.pipeline import rcsa_attention
    lay_q, lay_k, q, k, v = _case(seed=6)
    nq, nk = lay_q.n_blocks, lay_k.n_blocks
    forced = torch.zeros(nq, nk, dtype=torch.bool)
    forced[:, nk - 30:] = True  # the current frames' blocks are always kept
    k_select = 30 + 16
    print(f"gather layer call n_split {n_split} q blocks {nq} k blocks {nk}", flush=True)
    ref = rcsa_attention(_packed(q, lay_q), _packed(k, lay_k), _packed(v, lay_k),
                         lay_q.slot_valid, lay_k.slot_valid, block_size=128, k_select=k_select,
                         forced=forced, int8=True, max_k=k_select, return_lse=True,
                         n_split=n_split)
    got = rcsa_attention(q, k, v, None, None, block_size=128, k_select=k_select,
                         forced=forced, int8=True, max_k=k_select, return_lse=True,
                         n_split=n_split, q_slot_token=lay_q.slot_token,
                         k_slot_token=lay_k.slot_token)
    torch.cuda.synchronize()
    assert torch.equal(got.indices, ref.indices) and torch.equal(got.counts, ref.counts)
    want_out = ops.unpack_tokens(ref.out, lay_q.token_to_packed)
    assert got.out.shape == q.shape
    assert torch.equal(got.out, want_out)
    # LSE rows follow their tokens: got [B, H, L] against the packed rows
    tp = lay_q.token_to_packed
    assert torch.equal(got.lse, ref.lse[:, :, tp])


def test_gathered_inputs_rejected_without_both_maps():
    from cast_amd import ops
    lay_q, lay_k, q, k, v = _case(H=2)
    with pytest.raises(ValueError):
        ops.pool_query_key(q, None, k, None, 128, q_slot_token=lay_q.slot_token)
    with pytest.raises(ValueError):  # a map that is not a whole number of blocks
        ops.quantize_key(k, None, 128, *(torch.zeros(2, 90, 128, device=k.device)
                                         for _ in range(3)),
                         slot_token=lay_k.slot_token[:-1])

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


def test_gathered_pooling_without_quantiser_matches_packed():
    """The bf16 path's pass: pooled blocks and validity bits only."""
    from cast_amd import ops
    lay_q, lay_k, q, k, v = _case(seed=8)
    print("gather pooling, no quantiser", flush=True)
    qhat, _, _ = ops.pool_query(_packed(q, lay_q), lay_q.slot_valid, 128)
    khat, _, _, _, mask = ops.pool_key(_packed(k, lay_k), lay_k.slot_valid, 128,
                                       block_mask=True)
    got = ops.pool_query_key(q, None, k, None, 128, q_slot_token=lay_q.slot_token32,
                             k_slot_token=lay_k.slot_token32, quantize=False)
    assert all(got[i] is None for i in (1, 2, 4, 5, 6))
    assert torch.equal(got[0], qhat) and torch.equal(got[3], khat) and torch.equal(got[7], mask)


def _holey_map(n_tokens, n_slots, g, dev):
    """A slot -> token map over n_slots slots: a random permutation of the
    tokens with every fifth slot empty (-1) and one slot past the tokens."""
    m = torch.full((n_slots,), -1, dtype=torch.int32)
    keep = torch.arange(n_slots) % 5 != 4
    perm = torch.randperm(n_tokens, generator=g)[:int(keep.sum())]
    m[keep] = perm.int()
    m[7] = n_tokens + 3  # a row past the source: empty as well
    return m.to(dev)


@pytest.mark.parametrize("n_split", [1, 3])
def test_int8_attention_reads_v_through_map(n_split):
    """sparse_attn_int8 with v_token (V rows gathered in the copy ring) equals
    the call on the packed V, bit for bit."""
    from cast_amd import ops
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(21 + n_split)
    B, H, D, nqb, nkb, max_k, n_tok = 1, 6, 128, 20, 24, 10, 2600
    q8 = torch.randint(-127, 128, (B, H, nqb * 128, D), generator=g, dtype=torch.int8).to(dev)
    k8 = torch.randint(-127, 128, (B, H, nkb * 128, D), generator=g, dtype=torch.int8).to(dev)
    qs = (torch.rand(B * H, nqb, generator=g) * 1e-3 + 1e-4).to(dev)
    ks = (torch.rand(B * H, nkb, generator=g) * 1e-3 + 1e-4).to(dev)
    v_tok = (torch.randn(B, n_tok, H, D, generator=g)).bfloat16().to(dev)
    vmap = _holey_map(n_tok, nkb * 128, g, dev)
    v_packed = ops.pack_tokens(v_tok, vmap)
    valid = (vmap >= 0) & (vmap < n_tok)
    # the validity bits of the packed keys, as the pooling pass writes them
    mask = ops.pool_key(v_packed, valid, 128, block_mask=True)[4]
    idx = torch.stack([torch.randperm(nkb, generator=g)[:max_k].sort().values
                       for _ in range(B * H * nqb)]).reshape(B, H, nqb, max_k).int().to(dev)
    cnt = torch.randint(1, max_k + 1, (B, H, nqb), generator=g, dtype=torch.int32).to(dev)
    print(f"int8 v_token n_split {n_split}", flush=True)
    want, lse_w = ops.sparse_attn_int8(q8, qs, k8, ks, v_packed, idx, cnt, None, block_mask=mask,
                                       return_lse=True, n_split=n_split)
    got, lse_g = ops.sparse_attn_int8(q8, qs, k8, ks, v_tok, idx, cnt, None, block_mask=mask,
                                      return_lse=True, n_split=n_split, v_token=vmap)
    torch.cuda.synchronize()
    assert torch.equal(got, want) and torch.equal(lse_g, lse_w)
    with pytest.raises(ValueError):  # the gathered V rides with the validity bits only
        ops.sparse_attn_int8(q8, qs, k8, ks, v_tok, idx, cnt, None, v_token=vmap)


@pytest.mark.parametrize("n_split", [1, 3])
def test_bf16_attention_reads_rows_through_maps(n_split):
    """sparse_attn_bf16 with q_token / kv_token equals the call on packed
    inputs followed by the unpack of its output, bit for bit."""
    from cast_amd import ops
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(31 + n_split)
    B, H, D, nqb, nkb, max_k = 1, 4, 128, 12, 20, 9
    nq_tok, nk_tok = nqb * 128 - 100, 2400
    q_tok = (torch.randn(B, nq_tok, H, D, generator=g) / D ** 0.5).bfloat16().to(dev)
    k_tok = (torch.randn(B, nk_tok, H, D, generator=g) / D ** 0.5).bfloat16().to(dev)
    v_tok = torch.randn(B, nk_tok, H, D, generator=g).bfloat16().to(dev)
    # every query token owns exactly one slot (the output is written through the map)
    qmap = torch.full((nqb * 128,), -1, dtype=torch.int32)
    qslots = torch.randperm(nqb * 128, generator=g)[:nq_tok]
    qmap[qslots] = torch.arange(nq_tok, dtype=torch.int32)
    qmap = qmap.to(dev)
    kmap = _holey_map(nk_tok, nkb * 128, g, dev)
    kvalid = ((kmap >= 0) & (kmap < nk_tok))
    _, _, _, _, mask = ops.pool_key(ops.pack_tokens(k_tok, kmap), kvalid, 128, block_mask=True)
    idx = torch.stack([torch.randperm(nkb, generator=g)[:max_k].sort().values
                       for _ in range(B * H * nqb)]).reshape(B, H, nqb, max_k).int().to(dev)
    cnt = torch.randint(1, max_k + 1, (B, H, nqb), generator=g, dtype=torch.int32).to(dev)
    print(f"bf16 q_token/kv_token n_split {n_split}", flush=True)
    want, lse_w = ops.sparse_attn_bf16(ops.pack_tokens(q_tok, qmap), ops.pack_tokens(k_tok, kmap),
                                       ops.pack_tokens(v_tok, kmap), idx, cnt, None,
                                       block_mask=mask, return_lse=True, n_split=n_split)
    got, lse_g = ops.sparse_attn_bf16(q_tok, k_tok, v_tok, idx, cnt, None, block_mask=mask,
                                      return_lse=True, n_split=n_split, q_token=qmap,
                                      kv_token=kmap)
    torch.cuda.synchronize()
    t2p = torch.empty(nq_tok, dtype=torch.long, device=dev)
    t2p[qmap[qslots.to(dev)].long()] = qslots.to(dev)
    assert got.shape == (B, nq_tok, H, D)
    assert torch.equal(got, ops.unpack_tokens(want, t2p))
    assert torch.equal(lse_g, lse_w[:, :, t2p])


def test_bf16_split_leaves_empty_query_slots_unwritten():
    """A gathered bf16 call whose output map sends empty query slots (no token)
    to real rows: no launch form writes those rows, so the split launch equals
    the unsplit one bit for bit, and those rows keep their previous contents."""
    from cast_amd import ops
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(41)
    B, H, D, nqb, nkb, max_k = 1, 24, 128, 28, 40, 12
    nq_tok, nk_tok = nqb * 128 - 300, nkb * 128
    q_tok = (torch.randn(B, nq_tok, H, D, generator=g) / D ** 0.5).bfloat16().to(dev)
    k_tok = (torch.randn(B, nk_tok, H, D, generator=g) / D ** 0.5).bfloat16().to(dev)
    v_tok = torch.randn(B, nk_tok, H, D, generator=g).bfloat16().to(dev)
    qmap = torch.full((nqb * 128,), -1, dtype=torch.int32)
    qslots = torch.randperm(nqb * 128, generator=g)[:nq_tok]
    qmap[qslots] = torch.arange(nq_tok, dtype=torch.int32)
    n_out = nq_tok + 40
    # every slot has an output row; empty query slots write rows nq_tok.. of out
    omap = qmap.clone()
    empty = torch.nonzero(qmap < 0).flatten()
    omap[empty] = nq_tok + (torch.arange(empty.numel()) % 40).int()
    qmap, omap = qmap.to(dev), omap.to(dev)
    kmap = torch.arange(nk_tok, dtype=torch.int32, device=dev)
    mask = torch.full((nkb, 4), -1, dtype=torch.int32, device=dev)
    idx = torch.stack([torch.randperm(nkb, generator=g)[:max_k].sort().values
                       for _ in range(B * H * nqb)]).reshape(B, H, nqb, max_k).int().to(dev)
    cnt = torch.randint(1, max_k + 1, (B, H, nqb), generator=g, dtype=torch.int32).to(dev)
    outs = []
    for ns in (1, 3):
        out = torch.full((B, n_out, H, D), 7.0, dtype=torch.bfloat16, device=dev)
        print(f"bf16 empty query slots, n_split {ns}", flush=True)
        ops.sparse_attn_bf16(q_tok, k_tok, v_tok, idx, cnt, None, block_mask=mask,
                             n_split=ns, q_token=qmap, kv_token=kmap, out_token=omap,
                             out_len=n_out, out=out)
        outs.append(out)
    torch.cuda.synchronize()
    for out in outs:
        assert bool((out[:, nq_tok:] == 7.0).all())
    # the merge sums the shares' partials in another order than one pass does
    torch.testing.assert_close(outs[1][:, :nq_tok].float(), outs[0][:, :nq_tok].float(),
                               atol=2e-3, rtol=1e-2)


@pytest.mark.parametrize("int8", [True, False])
@pytest.mark.parametrize("n_split", [1, 3])
def test_gathered_layer_call_matches_pack_unpack(n_split, int8):
    from cast_amd import ops
    from cast_amd.pipeline import rcsa_attention
    lay_q, lay_k, q, k, v = _case(seed=6)
    nq, nk = lay_q.n_blocks, lay_k.n_blocks
    forced = torch.zeros(nq, nk, dtype=torch.bool)
    forced[:, nk - 30:] = True  # the current frames' blocks are always kept
    k_select = 30 + 16
    print(f"gather layer call int8 {int8} n_split {n_split} q blocks {nq} k blocks {nk}",
          flush=True)
    ref = rcsa_attention(_packed(q, lay_q), _packed(k, lay_k), _packed(v, lay_k),
                         lay_q.slot_valid, lay_k.slot_valid, block_size=128, k_select=k_select,
                         forced=forced, int8=int8, max_k=k_select, return_lse=True,
                         n_split=n_split)
    got = rcsa_attention(q, k, v, None, None, block_size=128, k_select=k_select,
                         forced=forced, int8=int8, max_k=k_select, return_lse=True,
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


@pytest.mark.parametrize("int8", [False, True])
def test_gathered_call_repeats_bit_exact_at_layer_size(int8):
    """24 heads, 4 query frames against 40 memory + 4 current frames (30 x 330
    blocks, 105 per row): twenty gathered calls in a row each equal pack ->
    packed call -> unpack.  Guards the ring's first wait, which leaves exactly
    one step's copies (and map reads) in flight and so depends on the
    prologue's issue order."""
    from cast_amd import layout, ops
    from cast_amd.pipeline import rcsa_attention
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(11)
    H, D = 24, 128
    lay_q = layout.compact_layout(range(4), 0, *HW, SHAPE, dev)
    lay_k = layout.compact_layout(range(44), 40, *HW, SHAPE, dev)
    q, k, v = (torch.randn(1, n * 880, H, D, device=dev, generator=g).div_(D ** 0.5)
               .to(torch.bfloat16) for n in (4, 44, 44))
    nq, nk = lay_q.n_blocks, lay_k.n_blocks
    forced = torch.zeros(nq, nk, dtype=torch.bool, device=dev)
    forced[:, nk - 30:] = True
    k_sel = round(0.25 * (nk - 30)) + 30
    kw = dict(block_size=128, k_select=k_sel, forced=forced, int8=int8, max_k=k_sel)
    ref = rcsa_attention(ops.pack_tokens(q, lay_q.slot_token), ops.pack_tokens(k, lay_k.slot_token),
                         ops.pack_tokens(v, lay_k.slot_token), lay_q.slot_valid, lay_k.slot_valid,
                         **kw)
    want = ops.unpack_tokens(ref.out, lay_q.token_to_packed)
    print(f"gathered layer call x20, int8 {int8}", flush=True)
    bad = []
    for it in range(20):
        got = rcsa_attention(q, k, v, None, None, q_slot_token=lay_q.slot_token32,
                             k_slot_token=lay_k.slot_token32, **kw).out
        torch.cuda.synchronize()
        if not torch.equal(got, want):
            bad.append(it)
    assert not bad, f"calls {bad} differ"

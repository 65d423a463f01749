"""GPU parity of each HIP kernel against the CPU oracle (small, seeded inputs).

Tolerances: bit-exact for indices, counts and int8 values; 1e-5 absolute for
pooled vectors and scores (fp32 summation order only); attention output
cosine >= 0.999 and max-abs <= 3e-2 against the fp32 oracle (the bf16/int8
tolerance stated for this path), plus a tighter relative-L2 bound.
"""
import math

import pytest
import torch

from oracle import rcsa_oracle as orc

pytestmark = pytest.mark.gpu


def _case(seed, B=1, H=2, nqb=3, nkb=9, D=128, bs=128, q_valid_tail=0, k_valid_tail=0,
          dtype=torch.bfloat16, shift=0.5):
    g = torch.Generator().manual_seed(seed)

    def blocks(nb):
        x = torch.randn(B, H, nb, bs, D, generator=g)
        x = x + torch.randn(B, H, nb, 1, D, generator=g) * shift
        return x.reshape(B, H, nb * bs, D)

    q, k, v = blocks(nqb), blocks(nkb), blocks(nkb)
    qv = torch.ones(nqb * bs, dtype=torch.bool)
    kv = torch.ones(nkb * bs, dtype=torch.bool)
    if q_valid_tail:
        qv[-q_valid_tail:] = False
    if k_valid_tail:
        kv[-k_valid_tail:] = False
    q = q * qv[None, None, :, None]
    k = k * kv[None, None, :, None]
    v = v * kv[None, None, :, None]
    return q.to(dtype), k.to(dtype), v.to(dtype), qv, kv


@pytest.mark.parametrize("D,bs,dtype", [(64, 64, torch.float32), (128, 128, torch.bfloat16),
                                        (128, 64, torch.bfloat16), (64, 128, torch.float32)])
def test_pool_query_and_int8(dev, D, bs, dtype):
    from cast_amd import ops
    q, _, _, qv, _ = _case(1, D=D, bs=bs, dtype=dtype, q_valid_tail=bs // 2)
    qhat, q8, qs = ops.pool_query(q.to(dev), qv.to(dev), bs, quantize=True)
    ref_hat, _, _ = orc.pool_blocks(q, qv, bs)
    B, H = q.shape[:2]
    torch.testing.assert_close(qhat.cpu(), ref_hat.reshape(B * H, -1, D), atol=1e-5, rtol=0)
    ref8, refs = orc.quantize_query_blocks(q, qv, bs)
    torch.testing.assert_close(qs.cpu(), refs, atol=0, rtol=0)
    assert torch.equal(q8.cpu(), ref8)


@pytest.mark.parametrize("D,bs", [(128, 128), (64, 64)])
def test_pool_key_stats_and_quantize(dev, D, bs):
    from cast_amd import ops
    _, k, _, _, kv = _case(2, D=D, bs=bs, k_valid_tail=bs + 17)
    khat, ksum, kmin, kmax = ops.pool_key(k.to(dev), kv.to(dev), bs, stats=True)
    ref_hat, ref_sum, _ = orc.pool_blocks(k, kv, bs)
    B, H = k.shape[:2]
    torch.testing.assert_close(khat.cpu(), ref_hat.reshape(B * H, -1, D), atol=1e-5, rtol=0)
    torch.testing.assert_close(ksum.cpu(), ref_sum.reshape(B * H, -1, D), atol=1e-4, rtol=1e-5)
    nb = k.shape[2] // bs
    xb = k.float().reshape(B * H, nb, bs, D)
    w = kv.reshape(nb, bs)[None, :, :, None]
    big = torch.tensor(float("inf"))
    ref_min = torch.where(w, xb, big).amin(2)
    ref_max = torch.where(w, xb, -big).amax(2)
    empty = ~kv.reshape(nb, bs).any(1)
    ref_min[:, empty] = 0
    ref_max[:, empty] = 0
    assert torch.equal(kmin.cpu(), ref_min) and torch.equal(kmax.cpu(), ref_max)
    k8, ks, km = ops.quantize_key(k.to(dev), kv.to(dev), bs, ksum, kmin, kmax)
    torch.testing.assert_close(km.cpu(), orc.key_mean(k, kv), atol=1e-6, rtol=1e-5)
    # bit-exact given the device's own mean
    ref8, refs = orc.quantize_key_blocks(k, kv, bs, km.cpu())
    torch.testing.assert_close(ks.cpu(), refs, atol=0, rtol=0)
    assert torch.equal(k8.cpu(), ref8)


@pytest.mark.parametrize("D,bs,dtype", [(128, 128, torch.bfloat16), (64, 64, torch.float32),
                                        (128, 64, torch.bfloat16)])
def test_pool_query_key_fused(dev, D, bs, dtype):
    """The fused pooling launch equals the two separate calls bit for bit."""
    from cast_amd import ops
    q, k, _, qv, kv = _case(4, D=D, bs=bs, dtype=dtype, q_valid_tail=bs // 2,
                            k_valid_tail=bs + 17)
    q, k, qv, kv = q.to(dev), k.to(dev), qv.to(dev), kv.to(dev)
    got = ops.pool_query_key(q, qv, k, kv, bs)
    ref = ops.pool_query(q, qv, bs, quantize=True) + ops.pool_key(k, kv, bs, stats=True,
                                                                    block_mask=True)
    torch.cuda.synchronize()
    names = ("qhat", "q_i8", "q_scale", "khat", "ksum", "kmin", "kmax", "block_mask")
    for name, a, b in zip(names, got, ref):
        assert torch.equal(a, b), name


def test_block_scores(dev):
    from cast_amd import ops
    g = torch.Generator().manual_seed(3)
    qh = torch.nn.functional.normalize(torch.randn(5, 37, 128, generator=g), dim=-1)
    kh = torch.nn.functional.normalize(torch.randn(5, 301, 128, generator=g), dim=-1)
    s = ops.block_scores(qh.to(dev), kh.to(dev))
    torch.testing.assert_close(s.cpu(), orc.block_scores(qh, kh), atol=2e-6, rtol=0)


@pytest.mark.parametrize("nk,order", [(9, "index"), (303, "index"), (853, "rank"),
                                      (853, "index"), (5000, "index")])
def test_select_topk_bit_exact(dev, nk, order):
    from cast_amd import ops
    g = torch.Generator().manual_seed(nk)
    nbh, nq = 6, 7
    s = torch.randn(nbh, nq, nk, generator=g)
    # exact ties and near ties in some rows
    s[0, :, : nk // 2] = 0.25
    s[1] = torch.round(s[1] * 8) / 8
    s[2, 0, :] = -0.0
    forced = torch.rand(nq, nk, generator=g) < 0.05
    allowed = torch.rand(nq, nk, generator=g) < 0.9
    kk = torch.randint(0, min(nk, 120) + 1, (nq,), generator=g).to(torch.int32)
    kk[0] = nk + 5  # more than exists: clamps to max_k / allowed
    max_k = min(nk, 130)
    for fm, am in ((None, None), (forced, None), (forced, allowed)):
        idx, cnt = ops.select_topk(s.to(dev), kk, forced=None if fm is None else fm.to(dev),
                                   allowed=None if am is None else am.to(dev), max_k=max_k,
                                   order=order)
        ridx, rcnt = orc.select_topk(s, kk, forced=fm, allowed=am, max_k=max_k, order=order)
        assert torch.equal(cnt.cpu(), rcnt)
        assert torch.equal(idx.cpu(), ridx)


def _lists(nbh_shape, nqb, nkb, kmax, seed, with_bad=False):
    g = torch.Generator().manual_seed(seed)
    B, H = nbh_shape
    idx = torch.full((B, H, nqb, kmax), -1, dtype=torch.int32)
    cnt = torch.zeros(B, H, nqb, dtype=torch.int32)
    for b in range(B):
        for h in range(H):
            for m in range(nqb):
                c = int(torch.randint(0, kmax + 1, (1,), generator=g))
                sel = torch.randperm(nkb, generator=g)[:c].sort().values
                idx[b, h, m, :c] = sel.to(torch.int32)
                cnt[b, h, m] = c
    if with_bad:
        idx[0, 0, 0, 0] = nkb + 3      # out of range -> skipped
        cnt[0, 0, 0] = max(int(cnt[0, 0, 0]), 1)
        cnt[0, -1, -1] = 0             # empty row -> zeros
    return idx, cnt


def _check_out(out, ref, qv, tag, cos_min=0.999, max_abs=3e-2, rel=1e-2):
    rows = qv.nonzero().flatten()
    o = out.float().cpu()[:, :, rows]
    r = ref[:, :, rows]
    st = orc.equivalence_stats(r, o)
    assert st["cosine"] >= cos_min and st["max_abs"] <= max_abs and st["relative_l2"] <= rel, \
        f"{tag}: {st}"


@pytest.mark.parametrize("D,bm,bn", [(128, 128, 128), (64, 64, 64), (128, 64, 128),
                                     (128, 128, 64), (64, 128, 128)])
def test_sparse_attn_bf16(dev, D, bm, bn):
    from cast_amd import ops
    B, H = 1, 3
    nqb_tokens, nkb_tokens = 3 * 128, 9 * 128
    g = torch.Generator().manual_seed(D + bm + bn)
    q = torch.randn(B, H, nqb_tokens - 40, D, generator=g).to(torch.bfloat16)  # partial q block
    k = torch.randn(B, H, nkb_tokens, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, H, nkb_tokens, D, generator=g).to(torch.bfloat16)
    kv = torch.rand(nkb_tokens, generator=g) < 0.85
    kv[bn:2 * bn] = False  # a fully masked block
    nqb = -(-q.shape[2] // bm)
    nkb = nkb_tokens // bn
    idx, cnt = _lists((B, H), nqb, nkb, min(nkb, 7), 11, with_bad=True)
    out, lse = ops.sparse_attn_bf16(q.to(dev), k.to(dev), v.to(dev), idx.to(dev), cnt.to(dev),
                                    kv.to(dev), block_m=bm, block_n=bn, return_lse=True)
    ref, rlse = orc.sparse_attention(q.float(), k.float(), v.float(), idx, cnt, kv,
                                     block_m=bm, block_n=bn)
    _check_out(out, ref, torch.ones(q.shape[2], dtype=torch.bool), f"bf16 D{D} {bm}x{bn}")
    fin = torch.isfinite(rlse)
    assert torch.equal(fin, torch.isfinite(lse.cpu()))
    torch.testing.assert_close(lse.cpu()[fin], rlse[fin], atol=2e-2, rtol=0)
    # rows with no admissible key are exactly zero
    assert torch.all(out.cpu()[~fin] == 0)


@pytest.mark.parametrize("D,bs", [(128, 128), (64, 64)])
def test_sparse_attn_int8(dev, D, bs):
    from cast_amd import ops
    q, k, v, qv, kv = _case(5, H=3, nqb=3, nkb=10, D=D, bs=bs, q_valid_tail=bs // 2,
                            k_valid_tail=bs // 2 + 3)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    _, q8, qs = ops.pool_query(qd, qv.to(dev), bs, quantize=True)
    _, ksum, kmin, kmax = ops.pool_key(kd, kv.to(dev), bs, stats=True)
    k8, ks, km = ops.quantize_key(kd, kv.to(dev), bs, ksum, kmin, kmax)
    idx, cnt = _lists((1, 3), 3, 10, 6, 12)
    out = ops.sparse_attn_int8(q8, qs, k8, ks, vd, idx.to(dev), cnt.to(dev), kv.to(dev),
                               block_m=bs, block_n=bs)
    ref_deq, _ = orc.sparse_attention_int8(q8.cpu(), qs.cpu(), k8.cpu(), ks.cpu(), v, idx, cnt,
                                           kv, block_m=bs, block_n=bs)
    _check_out(out, ref_deq, qv, "int8 vs dequantised oracle", cos_min=0.9999, rel=5e-3)
    ref32, _ = orc.sparse_attention(q.float(), k.float(), v.float(), idx, cnt, kv,
                                    block_m=bs, block_n=bs)
    _check_out(out, ref32, qv, "int8 vs fp32 oracle")


@pytest.mark.parametrize("lk", [9 * 128 + 37, 128, 100])
def test_sparse_attn_int8_ragged_keys(dev, lk):
    """int8 attention over a key length that is not a whole number of blocks
    (the last block is partial), exactly one block, and less than one block."""
    from cast_amd import ops
    g = torch.Generator().manual_seed(lk)
    B, H, D, bs, lq = 1, 2, 128, 128, 2 * 128
    nkb = -(-lk // bs)
    q8 = torch.randint(-127, 128, (B, H, lq, D), generator=g, dtype=torch.int8)
    k8 = torch.randint(-127, 128, (B, H, lk, D), generator=g, dtype=torch.int8)
    v = torch.randn(B, H, lk, D, generator=g).to(torch.bfloat16)
    qs = torch.rand(B * H, lq // bs, generator=g) * 0.02 + 0.005
    ks = torch.rand(B * H, nkb, generator=g) * 0.02 + 0.005
    kv = torch.rand(lk, generator=g) < 0.9
    idx, cnt = _lists((B, H), lq // bs, nkb, nkb, 13)
    idx[..., 0] = nkb - 1  # every row reads the partial last block
    cnt.clamp_(min=1)
    out, lse = ops.sparse_attn_int8(q8.to(dev), qs.to(dev), k8.to(dev), ks.to(dev), v.to(dev),
                                    idx.to(dev), cnt.to(dev), kv.to(dev), return_lse=True)
    qf = (q8.float().reshape(B, H, lq // bs, bs, D) * qs.reshape(B, H, -1, 1, 1)).reshape(q8.shape)
    kblk = torch.arange(lk) // bs
    kf = k8.float() * ks.reshape(B, H, nkb)[:, :, kblk, None]
    ref, rlse = orc.sparse_attention(qf, kf, v.float(), idx, cnt, kv, block_m=bs, block_n=bs)
    _check_out(out, ref, torch.ones(lq, dtype=torch.bool), f"int8 ragged lk={lk}",
               cos_min=0.9999, rel=5e-3)
    fin = torch.isfinite(rlse)
    assert torch.equal(fin, torch.isfinite(lse.cpu()))
    torch.testing.assert_close(lse.cpu()[fin], rlse[fin], atol=2e-2, rtol=0)


@pytest.mark.parametrize("D,bs,lk", [(128, 128, 10 * 128), (128, 128, 9 * 128 + 37),
                                     (64, 64, 10 * 64), (128, 64, 10 * 64)])
def test_sparse_attn_int8_block_mask(dev, D, bs, lk):
    """Key validity passed as bits (pool_key's block_mask) gives exactly the
    output of the per-key validity bytes, on the 3-slot kernel (D 128,
    128 x 128 blocks) and the generic shapes, with a partial last block."""
    from cast_amd import ops
    g = torch.Generator().manual_seed(lk + D)
    B, H, lq = 1, 3, 3 * bs
    nkb = -(-lk // bs)
    k = torch.randn(B, H, nkb * bs, D, generator=g).to(torch.bfloat16)
    kv = torch.rand(nkb * bs, generator=g) < 0.8
    kv[lk:] = False
    kv[2 * bs: 3 * bs] = True  # one fully valid block, one fully invalid
    kv[3 * bs: 4 * bs] = False
    kd, kvd = k.to(dev), kv.to(dev)
    _, ksum, kmin, kmax, mask = ops.pool_key(kd, kvd, bs, stats=True, block_mask=True)
    bits = torch.tensor([(int(mask.cpu().view(-1)[i // 32]) >> (i % 32)) & 1
                         for i in range(nkb * bs)], dtype=torch.bool)
    assert torch.equal(bits, kv), "pool_key block_mask"
    k8, ks, _ = ops.quantize_key(kd, kvd, bs, ksum, kmin, kmax)
    k8, ks = k8[:, :, :lk].contiguous(), ks
    q8 = torch.randint(-127, 128, (B, H, lq, D), generator=g, dtype=torch.int8).to(dev)
    qs = (torch.rand(B * H, lq // bs, generator=g) * 0.02 + 0.005).to(dev)
    v = torch.randn(B, H, lk, D, generator=g).to(torch.bfloat16).to(dev)
    idx, cnt = _lists((B, H), lq // bs, nkb, nkb, 17)
    idx[..., 0] = nkb - 1
    cnt.clamp_(min=1)
    idx_d, cnt_d = idx.to(dev), cnt.to(dev)
    by_bytes, lse_b = ops.sparse_attn_int8(q8, qs, k8, ks, v, idx_d, cnt_d, kvd[:lk],
                                           block_m=bs, block_n=bs, return_lse=True, n_split=1)
    by_bits, lse_m = ops.sparse_attn_int8(q8, qs, k8, ks, v, idx_d, cnt_d, None,
                                          block_m=bs, block_n=bs, return_lse=True, n_split=1,
                                          block_mask=mask)
    assert torch.equal(by_bytes.cpu(), by_bits.cpu())
    assert torch.equal(lse_b.cpu(), lse_m.cpu())


@pytest.mark.parametrize("D,bs,lk,n_split", [(128, 128, 1280, 1), (128, 128, 1189, 1),
                                              (128, 128, 1189, 3), (64, 64, 640, 1)])
def test_sparse_attn_bf16_block_mask(dev, D, bs, lk, n_split):
    """bf16: key validity as bits gives exactly the output of the validity
    bytes (the 3-slot 64-key-step ring at D 128 and a generic shape), and both
    agree with the fp32 oracle."""
    from cast_amd import ops
    g = torch.Generator().manual_seed(lk + D + n_split)
    B, H, lq = 1, 3, 3 * bs
    nkb = -(-lk // bs)
    k = torch.randn(B, H, nkb * bs, D, generator=g).to(torch.bfloat16)
    kv = torch.rand(nkb * bs, generator=g) < 0.8
    kv[lk:] = False
    kv[2 * bs: 3 * bs] = True
    kv[3 * bs: 4 * bs] = False
    kd, kvd = k.to(dev), kv.to(dev)
    _, _, _, _, mask = ops.pool_key(kd, kvd, bs, block_mask=True)
    q = torch.randn(B, H, lq, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, H, lk, D, generator=g).to(torch.bfloat16)
    kk = k[:, :, :lk].contiguous()
    idx, cnt = _lists((B, H), lq // bs, nkb, nkb, 19)
    idx[..., 0] = nkb - 1
    cnt.clamp_(min=1)
    idx_d, cnt_d = idx.to(dev), cnt.to(dev)
    args = (q.to(dev), kk.to(dev), v.to(dev), idx_d, cnt_d)
    by_bytes, lse_b = ops.sparse_attn_bf16(*args, kvd[:lk], block_m=bs, block_n=bs,
                                           return_lse=True, n_split=n_split)
    by_bits, lse_m = ops.sparse_attn_bf16(*args, None, block_m=bs, block_n=bs,
                                          return_lse=True, n_split=n_split, block_mask=mask)
    assert torch.equal(by_bytes.cpu(), by_bits.cpu())
    assert torch.equal(lse_b.cpu(), lse_m.cpu())
    ref, _ = orc.sparse_attention(q.float(), kk.float(), v.float(), idx, cnt, kv[:lk],
                                  block_m=bs, block_n=bs)
    _check_out(by_bits, ref, torch.ones(lq, dtype=torch.bool), "bf16 bits vs oracle")


def test_pack_unpack_roundtrip(dev):
    from cast_amd import ops
    g = torch.Generator().manual_seed(7)
    B, L, H, D = 1, 700, 3, 128
    x = torch.randn(B, L, H, D, generator=g)
    slots = torch.full((6 * 128,), -1, dtype=torch.int64)
    perm = torch.randperm(L, generator=g)
    slots[: L] = perm
    ref = torch.zeros(B, H, slots.numel(), D)
    ok = slots >= 0
    ref[:, :, ok] = x[:, slots[ok]].transpose(1, 2)
    packed32 = ops.pack_tokens(x.to(dev), slots.to(dev))      # keeps fp32, no rounding
    assert packed32.dtype == torch.float32 and torch.equal(packed32.cpu(), ref)
    packed = ops.pack_tokens(x.to(dev, torch.bfloat16), slots.to(dev))
    assert torch.equal(packed.cpu(), ref.to(torch.bfloat16))
    # a [B, H, L, D] tensor viewed as [B, L, H, D] packs without a copy
    xt = x.transpose(1, 2).contiguous().to(dev)
    assert torch.equal(ops.pack_tokens(xt.transpose(1, 2), slots.to(dev)).cpu(), ref)
    token_slot = torch.empty(L, dtype=torch.int64)
    token_slot[perm] = torch.arange(L)
    back = ops.unpack_tokens(packed, token_slot.to(dev))
    assert torch.equal(back.cpu(), x.to(torch.bfloat16))


@pytest.mark.parametrize("int8", [False, True])
def test_sparse_attn_split_lists(dev, int8):
    """Splitting every block list over 2..8 workgroups and merging gives the
    unsplit result (up to the bf16 rounding of the partials) and the oracle's;
    rows with an empty list (or fewer blocks than splits) stay exact."""
    from cast_amd import _lib, ops
    B, H, D, bs = 1, 3, 128, 128
    q, k, v, qv, kv = _case(9, H=H, nqb=3, nkb=10, D=D, bs=bs, k_valid_tail=bs // 2 + 5)
    idx, cnt = _lists((B, H), 3, 10, 10, 21)
    cnt[0, 0, 0] = 0   # empty list
    cnt[0, 1, 1] = 1   # fewer blocks than splits
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    if int8:
        _, q8, qs = ops.pool_query(qd, qv.to(dev), bs, quantize=True)
        _, ksum, kmin, kmax = ops.pool_key(kd, kv.to(dev), bs, stats=True)
        k8, ks, _ = ops.quantize_key(kd, kv.to(dev), bs, ksum, kmin, kmax)
        run = lambda s: ops.sparse_attn_int8(q8, qs, k8, ks, vd, idx.to(dev), cnt.to(dev),  # noqa
                                             kv.to(dev), return_lse=True, n_split=s)
    else:
        run = lambda s: ops.sparse_attn_bf16(qd, kd, vd, idx.to(dev), cnt.to(dev), kv.to(dev),  # noqa
                                             return_lse=True, n_split=s)
    base, base_lse = run(1)
    ref, rlse = orc.sparse_attention(q.float(), k.float(), v.float(), idx, cnt, kv,
                                     block_m=bs, block_n=bs)
    fin = torch.isfinite(rlse)
    for s in (2, 3, 4, 8):
        out, lse = run(s)
        _check_out(out, base.float().cpu(), torch.ones(q.shape[2], dtype=torch.bool),
                   f"split {s} vs unsplit", cos_min=0.99999, max_abs=1e-2, rel=5e-3)
        _check_out(out, ref, qv, f"split {s} vs oracle")
        assert torch.equal(torch.isfinite(lse.cpu()), fin)
        # P is rounded to bf16 at each share's own running max: the sums agree
        # to the bf16 rounding of P, not bit for bit
        torch.testing.assert_close(lse.cpu()[fin], base_lse.cpu()[fin], atol=2e-3, rtol=0)
        assert torch.all(out.cpu()[~fin] == 0)
    # the workspace is checked before any launch
    lib = _lib.load()
    need = lib.rcsa_attn_workspace_bytes(B, H, q.shape[2], D, 3)
    assert need > 0 and lib.rcsa_attn_workspace_bytes(B, H, q.shape[2], D, 1) == 0
    small = torch.empty(need - 256, dtype=torch.uint8, device=dev)
    out = torch.empty_like(qd)
    idx_d, cnt_d = idx.to(dev), cnt.to(dev)
    args = [qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), None, 1 / math.sqrt(D), None,
            out.data_ptr(), idx_d.data_ptr(), cnt_d.data_ptr(), *qd.stride()[:3],
            *kd.stride()[:3], *vd.stride()[:3], *out.stride()[:3], *idx_d.stride()[:3],
            *cnt_d.stride(), B, H, q.shape[2], k.shape[2], D, bs, bs, idx.shape[3]]
    stream = torch.cuda.current_stream().cuda_stream
    split_args = args[:4] + [None] + args[4:]  # K_block_mask after K_valid
    no_maps = (None, 0, None, 0, None, 0)  # q_token, kv_token, out_token and their lengths
    assert lib.rcsa_sparse_attn_bf16_split(*split_args, 3, small.data_ptr(), need - 256,
                                           *no_maps, stream) == 2
    assert lib.rcsa_sparse_attn_bf16_split(*split_args, 3, None, need, *no_maps, stream) == 1
    # a K row spanning 16 MiB or more is refused before any launch (the copy
    # addressing multiplies row numbers by the row stride in 24 bits)
    big = list(args)
    big[14] = 1 << 23  # stride_kn of bf16 K: 16 MiB rows
    assert lib.rcsa_sparse_attn_bf16(*big, stream) == 3
    big = list(args)
    big[17] = 1 << 23  # stride_vn
    assert lib.rcsa_sparse_attn_bf16(*big, stream) == 3
    torch.cuda.synchronize()

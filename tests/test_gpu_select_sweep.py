"""Seeded sweep of the selection chain's kernels against the oracle.

Every case draws batch 1-2, heads 1-3, head_dim 64 or 128, block size 64 or
128, bf16 or fp32 inputs, 1-4 query blocks and 1-40 key blocks, query and key
validity with holes, a masked tail and (with several key blocks) a fully
masked block.  Per case: query pooling with its int8 quantiser, key pooling
with the block statistics, the mean-smoothed key quantiser, the cosine block
scores, and the top-k with per-row budgets (some above the blocks that
exist), forced and allowed masks, in index or rank order.  Bars: 1e-5 for the
pooled directions (fp32 summation order), bit-exact block minima/maxima,
int8 values and scales (the key quantiser given the device's own mean, which
is within 1e-6 / 1e-5 of the fp64 mean), 2e-6 for the scores, and bit-exact
indices and counts for the top-k on the device's own scores.
"""
import pytest
import torch

from oracle import rcsa_oracle as orc

pytestmark = pytest.mark.gpu

N_CASES = 24


def _draw(seed: int) -> dict:
    g = torch.Generator().manual_seed(seed)

    def pick(xs):
        return xs[int(torch.randint(0, len(xs), (1,), generator=g))]

    return dict(g=g, B=pick([1, 2]), H=pick([1, 2, 3]), D=pick([64, 128]), bs=pick([64, 128]),
                dtype=pick([torch.bfloat16, torch.float32]), nqb=pick([1, 2, 3, 4]),
                nkb=pick([1, 5, 17, 40]), order=pick(["index", "rank"]),
                masks=pick(["none", "forced", "both"]))


def _valid(g, n_tokens, bs, hole_frac, whole_block):
    v = torch.rand(n_tokens, generator=g) >= hole_frac
    v[-int(torch.randint(0, bs, (1,), generator=g)) - 1:] = False   # a masked tail
    if whole_block and n_tokens > bs:
        v[bs:2 * bs] = False                                          # a fully masked block
    return v


@pytest.mark.parametrize("ci", range(N_CASES))
def test_selection_chain_sweep(dev, ci):
    from cast_amd import ops
    c = _draw(3000 + ci)
    g, B, H, D, bs, dt = c["g"], c["B"], c["H"], c["D"], c["bs"], c["dtype"]
    nqb, nkb = c["nqb"], c["nkb"]
    print(f"selection case {ci}: B{B} H{H} D{D} bs {bs} {dt} q blocks {nqb} k blocks {nkb} "
          f"order {c['order']} masks {c['masks']}", flush=True)
    lq, lk = nqb * bs, nkb * bs
    q = (torch.randn(B, H, lq, D, generator=g) + torch.randn(B, H, 1, D, generator=g)).to(dt)
    k = (torch.randn(B, H, lk, D, generator=g) * 2 + torch.randn(B, H, 1, D, generator=g)).to(dt)
    qv = _valid(g, lq, bs, 0.1, False)
    kv = _valid(g, lk, bs, 0.2, True)

    qhat, q8, qs = ops.pool_query(q.to(dev), qv.to(dev), bs, quantize=True)
    ref_qhat, _, _ = orc.pool_blocks(q, qv, bs)
    torch.testing.assert_close(qhat.cpu(), ref_qhat.reshape(B * H, nqb, D), atol=1e-5, rtol=0)
    ref_q8, ref_qs = orc.quantize_query_blocks(q, qv, bs)
    assert torch.equal(qs.cpu(), ref_qs) and torch.equal(q8.cpu(), ref_q8)

    khat, ksum, kmin, kmax = ops.pool_key(k.to(dev), kv.to(dev), bs, stats=True)
    ref_khat, ref_ksum, _ = orc.pool_blocks(k, kv, bs)
    torch.testing.assert_close(khat.cpu(), ref_khat.reshape(B * H, nkb, D), atol=1e-5, rtol=0)
    torch.testing.assert_close(ksum.cpu(), ref_ksum.reshape(B * H, nkb, D), atol=1e-4, rtol=1e-5)
    xb = k.float().reshape(B * H, nkb, bs, D)
    w = kv.reshape(nkb, bs)[None, :, :, None]
    inf = torch.tensor(float("inf"))
    ref_min, ref_max = torch.where(w, xb, inf).amin(2), torch.where(w, xb, -inf).amax(2)
    empty = ~kv.reshape(nkb, bs).any(1)
    ref_min[:, empty] = 0
    ref_max[:, empty] = 0
    assert torch.equal(kmin.cpu(), ref_min) and torch.equal(kmax.cpu(), ref_max)

    k8, ks, km = ops.quantize_key(k.to(dev), kv.to(dev), bs, ksum, kmin, kmax)
    torch.testing.assert_close(km.cpu(), orc.key_mean(k, kv), atol=1e-6, rtol=1e-5)
    ref_k8, ref_ks = orc.quantize_key_blocks(k, kv, bs, km.cpu())
    assert torch.equal(ks.cpu(), ref_ks) and torch.equal(k8.cpu(), ref_k8)

    score = ops.block_scores(qhat, khat)
    torch.testing.assert_close(score.cpu(), orc.block_scores(qhat.cpu(), khat.cpu()), atol=2e-6,
                               rtol=0)

    kk = torch.randint(0, nkb + 3, (nqb,), generator=g).to(torch.int32)
    forced = torch.rand(nqb, nkb, generator=g) < 0.1 if c["masks"] != "none" else None
    allowed = torch.rand(nqb, nkb, generator=g) < 0.8 if c["masks"] == "both" else None
    max_k = max(1, min(nkb, int(kk.max())))
    idx, cnt = ops.select_topk(score, kk, forced=None if forced is None else forced.to(dev),
                               allowed=None if allowed is None else allowed.to(dev),
                               max_k=max_k, order=c["order"])
    ridx, rcnt = orc.select_topk(score.cpu(), kk, forced=forced, allowed=allowed, max_k=max_k,
                                 order=c["order"])
    assert torch.equal(cnt.cpu(), rcnt) and torch.equal(idx.cpu(), ridx)

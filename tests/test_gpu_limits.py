"""The attention at sizes past the ones the configurations reach: a key plane
of 268,723 tokens per head (int8 K 34 MB, bf16 V 69 MB per head, so block
offsets inside one head's plane pass 2^24 bytes), ragged query and key ends,
lists that reach the first, middle and partial last key blocks, and a query
block with an empty list (output 0, LSE -inf), against the fp32 oracle.

Tolerances as in the launch-form tests: int8 within cosine 0.9999 / max-abs
3e-2 / relative L2 5e-3 of the dequantised oracle, bf16 within cosine 0.999 /
max-abs 3e-2 / relative L2 1e-2 of the fp32 oracle, LSE within 2e-2."""
import pytest
import torch

from oracle import rcsa_oracle as orc

pytestmark = pytest.mark.gpu

BS, D, H = 128, 128, 2
LQ, LK = 3 * BS - 13, 2100 * BS - 77
NQB, NKB = 3, 2100
KMAX = 8


def _lists(g):
    idx = torch.full((1, H, NQB, KMAX), -1, dtype=torch.int32)
    cnt = torch.full((1, H, NQB), KMAX, dtype=torch.int32)
    for h in range(H):
        for m in range(NQB):
            rest = torch.randperm(NKB - 2, generator=g)[:KMAX - 3] + 1
            blocks = torch.cat([torch.tensor([0, NKB // 2, NKB - 1]), rest]).unique()
            blocks = blocks[:KMAX]
            idx[0, h, m, :blocks.numel()] = blocks.sort().values.int()
            cnt[0, h, m] = blocks.numel()
    cnt[0, 1, 1] = 0  # an empty list
    return idx, cnt


@pytest.mark.parametrize("int8", [True, False])
def test_attention_long_key_plane(dev, int8):
    from cast_amd import ops
    g = torch.Generator().manual_seed(77 + int(int8))
    idx, cnt = _lists(g)
    v = torch.randn(1, H, LK, D, generator=g).to(torch.bfloat16)
    print(f"long key plane: {LK} keys, int8 {int8}", flush=True)
    if int8:
        q8 = torch.randint(-127, 128, (1, H, LQ, D), generator=g, dtype=torch.int8)
        k8 = torch.randint(-127, 128, (1, H, LK, D), generator=g, dtype=torch.int8)
        qs = torch.rand(H, NQB, generator=g) * 0.02 + 0.005
        ks = torch.rand(H, NKB, generator=g) * 0.02 + 0.005
        out, lse = ops.sparse_attn_int8(q8.to(dev), qs.to(dev), k8.to(dev), ks.to(dev),
                                        v.to(dev), idx.to(dev), cnt.to(dev), None,
                                        return_lse=True)
        qf = q8.float() * qs[:, torch.arange(LQ) // BS][None, :, :, None]
        # only the selected key blocks are dequantised (the rest are never read)
        kf = torch.zeros(1, H, LK, D)
        for h in range(H):
            for n in idx[0, h].unique().tolist():
                if n >= 0:
                    r0, r1 = n * BS, min((n + 1) * BS, LK)
                    kf[0, h, r0:r1] = k8[0, h, r0:r1].float() * ks[h, n]
        ref, rlse = orc.sparse_attention(qf, kf, v.float(), idx, cnt, None, block_m=BS,
                                         block_n=BS)
        cos_min, rel = 0.9999, 5e-3
    else:
        q = torch.randn(1, H, LQ, D, generator=g).to(torch.bfloat16)
        k = torch.randn(1, H, LK, D, generator=g).to(torch.bfloat16)
        out, lse = ops.sparse_attn_bf16(q.to(dev), k.to(dev), v.to(dev), idx.to(dev),
                                        cnt.to(dev), None, return_lse=True)
        ref, rlse = orc.sparse_attention(q.float(), k.float(), v.float(), idx, cnt, None,
                                         block_m=BS, block_n=BS)
        cos_min, rel = 0.999, 1e-2
    out, lse = out.float().cpu(), lse.cpu()
    # the empty list: zero output, LSE -inf
    r0, r1 = BS, 2 * BS
    assert torch.equal(out[0, 1, r0:r1], torch.zeros(BS, D))
    assert bool(torch.isneginf(lse[0, 1, r0:r1]).all())
    st = orc.equivalence_stats(ref, out)
    assert st["cosine"] >= cos_min and st["max_abs"] <= 3e-2 and st["relative_l2"] <= rel, st
    fin = torch.isfinite(rlse)
    assert torch.equal(fin, torch.isfinite(lse))
    torch.testing.assert_close(lse[fin], rlse[fin], atol=2e-2, rtol=0)

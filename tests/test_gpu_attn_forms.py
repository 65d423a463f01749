"""Both launch forms of the D-128 attention against the fp32 oracle: one
8-wavefront workgroup per compute unit, and three 4-wavefront workgroups per
compute unit once every XCD has two full rounds of query blocks.  The head
count puts the grid just at and just below that threshold on the device at
hand; ragged query and key lengths, validity bytes and bits, the LSE and the
split of short last rounds (the default plan) are all exercised.

Tolerances as elsewhere: int8 output within cosine 0.9999 / relative L2 5e-3 of
the dequantised oracle, bf16 within cosine 0.999 / max-abs 3e-2 / relative L2
1e-2 of the fp32 oracle; LSE finite on the same rows and within 2e-2."""
import numpy as np
import pytest
import torch

from oracle import rcsa_oracle as orc

pytestmark = pytest.mark.gpu

BS, D, NQB, NKB, KMAX = 128, 128, 32, 24, 10


def _heads_at_gate():
    """Heads that make B*H*NQB work items fill two rounds of every XCD's compute units."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    return -(-2 * cus // NQB)


def _bits(kv: torch.Tensor, nkb: int) -> torch.Tensor:
    """Validity bits as pool_key writes them: int32 [nkb, BS / 32], key i at bit i % 32."""
    b = np.zeros(nkb * BS, dtype=np.uint8)
    b[: kv.numel()] = kv.numpy().astype(np.uint8)
    words = np.packbits(b, bitorder="little").view("<u4").view(np.int32)
    return torch.from_numpy(words.copy()).reshape(nkb, BS // 32)


def _lists(H, g):
    idx = torch.full((1, H, NQB, KMAX), -1, dtype=torch.int32)
    cnt = torch.randint(1, KMAX + 1, (1, H, NQB), generator=g, dtype=torch.int32)
    for h in range(H):
        for m in range(NQB):
            c = int(cnt[0, h, m])
            idx[0, h, m, :c] = torch.randperm(NKB, generator=g)[:c].sort().values.int()
    idx[0, :, ::3, 0] = NKB - 1  # every third row reads the partial last key block
    return idx, cnt


@pytest.mark.parametrize("bits", [True, False])
@pytest.mark.parametrize("int8", [True, False])
@pytest.mark.parametrize("below", [False, True])
def test_attention_forms_match_oracle(dev, below, int8, bits):
    from cast_amd import ops
    H = _heads_at_gate() - (1 if below else 0)
    lq, lk = NQB * BS - 50, NKB * BS - 37
    g = torch.Generator().manual_seed(1000 * int(below) + 10 * int(int8) + int(bits))
    kv = torch.rand(lk, generator=g) < 0.9
    idx, cnt = _lists(H, g)
    v = torch.randn(1, H, lk, D, generator=g).to(torch.bfloat16)
    valid = dict(block_mask=_bits(kv, NKB).to(dev)) if bits else {}
    kv_arg = None if bits else kv.to(dev)
    print(f"attention forms: H {H} int8 {int8} bits {bits}", flush=True)
    if int8:
        q8 = torch.randint(-127, 128, (1, H, lq, D), generator=g, dtype=torch.int8)
        k8 = torch.randint(-127, 128, (1, H, lk, D), generator=g, dtype=torch.int8)
        qs = torch.rand(H, NQB, generator=g) * 0.02 + 0.005
        ks = torch.rand(H, NKB, generator=g) * 0.02 + 0.005
        out, lse = ops.sparse_attn_int8(q8.to(dev), qs.to(dev), k8.to(dev), ks.to(dev),
                                        v.to(dev), idx.to(dev), cnt.to(dev), kv_arg,
                                        return_lse=True, **valid)
        # the dequantised operands (the last blocks are partial, so scale per row)
        qf = q8.float() * qs[:, torch.arange(lq) // BS][None, :, :, None]
        kf = k8.float() * ks[:, torch.arange(lk) // BS][None, :, :, None]
        ref, rlse = orc.sparse_attention(qf, kf, v.float(), idx, cnt, kv, block_m=BS,
                                         block_n=BS)
        cos_min, max_abs, rel = 0.9999, 3e-2, 5e-3
    else:
        q = torch.randn(1, H, lq, D, generator=g).to(torch.bfloat16)
        k = torch.randn(1, H, lk, D, generator=g).to(torch.bfloat16)
        out, lse = ops.sparse_attn_bf16(q.to(dev), k.to(dev), v.to(dev), idx.to(dev),
                                        cnt.to(dev), kv_arg, return_lse=True, **valid)
        ref, rlse = orc.sparse_attention(q.float(), k.float(), v.float(), idx, cnt, kv,
                                         block_m=BS, block_n=BS)
        cos_min, max_abs, rel = 0.999, 3e-2, 1e-2
    st = orc.equivalence_stats(ref, out.float().cpu())
    assert st["cosine"] >= cos_min and st["max_abs"] <= max_abs and st["relative_l2"] <= rel, st
    fin = torch.isfinite(rlse)
    assert torch.equal(fin, torch.isfinite(lse.cpu()))
    torch.testing.assert_close(lse.cpu()[fin], rlse[fin], atol=2e-2, rtol=0)

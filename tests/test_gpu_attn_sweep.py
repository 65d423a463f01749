"""Seeded sweep of the block-sparse attention entry points against the oracle.

Every case draws its own shape: batch 1-2, heads 1-5, head_dim 64 or 128,
query and key block sizes 64 or 128 (all eight tile shapes), ragged query and
key lengths, key validity as bytes or as bits, block lists in rank order (not
sorted) with empty rows, rows longer than the key blocks that exist and an
out-of-range block id, and a split of 1-3 shares or the library's own plan.
bf16 cases compare with the fp32 oracle; int8 cases with the oracle on the
dequantised int8 operands (the int8 kernel's own inputs), both at cosine >=
0.9999 / max-abs <= 3e-2 / relative L2 <= 5e-3 over the valid query rows, with
the log-sum-exp within 2e-2 and exact zeros / -inf for rows with no admissible
key.
"""
import pytest
import torch

from oracle import rcsa_oracle as orc

pytestmark = pytest.mark.gpu

N_CASES = 40


def _draw(seed: int) -> dict:
    g = torch.Generator().manual_seed(seed)

    def pick(xs):
        return xs[int(torch.randint(0, len(xs), (1,), generator=g))]

    bm, bn = pick([64, 128]), pick([64, 128])
    nqb, nkb = pick([1, 2, 3, 5]), pick([1, 3, 7, 12])
    lq = nqb * bm - pick([0, 1, bm // 2, bm - 1])
    lk = nkb * bn - pick([0, 3, bn // 2, bn - 1])
    return dict(g=g, B=pick([1, 2]), H=pick([1, 2, 3, 5]), D=pick([64, 128]), bm=bm, bn=bn,
                lq=lq, lk=lk, nqb=nqb, nkb=nkb, bits=bool(pick([0, 1])),
                n_split=pick([None, 1, 2, 3]), kmax=pick([1, 4, nkb, nkb + 2]))


def _lists(c):
    """Rank-ordered lists: distinct blocks in random order, count 0..kmax (a count
    past the blocks that exist reads the -1 padding, which is skipped)."""
    g, B, H, nqb, nkb, kmax = c["g"], c["B"], c["H"], c["nqb"], c["nkb"], c["kmax"]
    idx = torch.full((B, H, nqb, kmax), -1, dtype=torch.int32)
    cnt = torch.zeros(B, H, nqb, dtype=torch.int32)
    for b in range(B):
        for h in range(H):
            for m in range(nqb):
                n = int(torch.randint(0, kmax + 1, (1,), generator=g))
                sel = torch.randperm(nkb, generator=g)[:n]
                idx[b, h, m, :sel.numel()] = sel.to(torch.int32)
                cnt[b, h, m] = n
    cnt[0, 0, 0] = 0                                  # an empty row
    if kmax >= 2 and nqb > 1:
        idx[-1, -1, -1, 0] = nkb + 3                  # out of range: skipped
        cnt[-1, -1, -1] = max(int(cnt[-1, -1, -1]), 2)
    return idx, cnt


def _bits(kv: torch.Tensor, nkb: int, bn: int) -> torch.Tensor:
    """Key validity as pool_key writes it: int32 [nkb, bn / 32], bit i of word w
    of block n = key n * bn + 32 w + i (keys past the end invalid)."""
    full = torch.zeros(nkb * bn, dtype=torch.int64)
    full[:kv.numel()] = kv.to(torch.int64)
    words = (full.view(nkb, bn // 32, 32) << torch.arange(32)).sum(-1)
    return torch.where(words >= 2 ** 31, words - 2 ** 32, words).to(torch.int32)


def _valid(c, valid_frac=0.85):
    g, lk, bn = c["g"], c["lk"], c["bn"]
    kv = torch.rand(lk, generator=g) < valid_frac
    if c["nkb"] > 1:
        kv[:min(bn, lk)] = False                      # a fully masked block
    return kv


def _check(out, lse, ref, rlse, lq, tag):
    o = out.float().cpu()[:, :, :lq]
    fin = torch.isfinite(rlse[:, :, :lq])
    assert torch.equal(fin, torch.isfinite(lse.cpu()[:, :, :lq])), tag
    assert torch.all(o[~fin] == 0), tag               # rows with no admissible key
    if bool(fin.any()):
        st = orc.equivalence_stats(ref[:, :, :lq][fin], o[fin])
        assert st["cosine"] >= 0.9999 and st["max_abs"] <= 3e-2 and \
            st["relative_l2"] <= 5e-3, f"{tag}: {st}"
        torch.testing.assert_close(lse.cpu()[:, :, :lq][fin], rlse[:, :, :lq][fin], atol=2e-2,
                                   rtol=0)


def _case_tag(c):
    return (f"B{c['B']} H{c['H']} D{c['D']} tile {c['bm']}x{c['bn']} lq {c['lq']} "
            f"lk {c['lk']} kmax {c['kmax']} bits {c['bits']} split {c['n_split']}")


@pytest.mark.parametrize("ci", range(N_CASES))
def test_bf16_attention_sweep(dev, ci):
    from cast_amd import ops
    c = _draw(1000 + ci)
    tag = f"bf16 case {ci}: {_case_tag(c)}"
    print(tag, flush=True)
    g, B, H, D = c["g"], c["B"], c["H"], c["D"]
    q = torch.randn(B, H, c["lq"], D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, H, c["lk"], D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, H, c["lk"], D, generator=g).to(torch.bfloat16)
    kv = _valid(c)
    idx, cnt = _lists(c)
    kw = dict(block_m=c["bm"], block_n=c["bn"], return_lse=True, n_split=c["n_split"])
    if c["bits"]:
        kw["block_mask"] = _bits(kv, c["nkb"], c["bn"]).to(dev)
        valid = None
    else:
        valid = kv.to(dev)
    out, lse = ops.sparse_attn_bf16(q.to(dev), k.to(dev), v.to(dev), idx.to(dev), cnt.to(dev),
                                    valid, **kw)
    ref, rlse = orc.sparse_attention(q.float(), k.float(), v.float(), idx, cnt, kv,
                                     block_m=c["bm"], block_n=c["bn"])
    _check(out, lse, ref, rlse, c["lq"], tag)


@pytest.mark.parametrize("ci", range(N_CASES))
def test_int8_attention_sweep(dev, ci):
    from cast_amd import ops
    c = _draw(2000 + ci)
    tag = f"int8 case {ci}: {_case_tag(c)}"
    print(tag, flush=True)
    g, B, H, D, bm, bn = c["g"], c["B"], c["H"], c["D"], c["bm"], c["bn"]
    lq, lk, nqb, nkb = c["lq"], c["lk"], c["nqb"], c["nkb"]
    q8 = torch.randint(-127, 128, (B, H, lq, D), generator=g, dtype=torch.int8)
    k8 = torch.randint(-127, 128, (B, H, lk, D), generator=g, dtype=torch.int8)
    v = torch.randn(B, H, lk, D, generator=g).to(torch.bfloat16)
    qs = torch.rand(B * H, nqb, generator=g) * 0.02 + 0.005
    ks = torch.rand(B * H, nkb, generator=g) * 0.02 + 0.005
    kv = _valid(c)
    idx, cnt = _lists(c)
    kw = dict(block_m=bm, block_n=bn, return_lse=True, n_split=c["n_split"])
    if c["bits"]:
        kw["block_mask"] = _bits(kv, nkb, bn).to(dev)
        valid = None
    else:
        valid = kv.to(dev)
    out, lse = ops.sparse_attn_int8(q8.to(dev), qs.to(dev), k8.to(dev), ks.to(dev), v.to(dev),
                                    idx.to(dev), cnt.to(dev), valid, **kw)
    qf = q8.float() * qs.reshape(B, H, nqb)[:, :, torch.arange(lq) // bm, None]
    kf = k8.float() * ks.reshape(B, H, nkb)[:, :, torch.arange(lk) // bn, None]
    ref, rlse = orc.sparse_attention(qf, kf, v.float(), idx, cnt, kv, block_m=bm, block_n=bn)
    _check(out, lse, ref, rlse, lq, tag)

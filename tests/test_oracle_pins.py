"""Pins for the CPU oracle (oracle/rcsa_oracle.py).

The reference ships no golden vectors or known-answer tests for this path,
so each oracle function is checked here against something the mathematics
fixes independently of the oracle's own formula: fp64 brute-force loops,
closed forms, invariants, and textbook library routines.  The
``test_planted_*`` cases plant a plausible mistake in a copy of an oracle
function and show that the pin catches it.
"""
import math
import random
from fractions import Fraction

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import rcsa_oracle as orc


def _rand(shape, seed, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g, dtype=dtype)


# ---------------------------------------------------------------- pooling

def _pool_brute(x, valid, bs):
    """fp64 triple loop: masked mean over valid tokens, then x / max(|x|, 1e-12)."""
    B, H, L, D = x.shape
    nb = L // bs
    out = np.zeros((B, H, nb, D))
    xn = x.double().numpy()
    vn = np.ones(L, bool) if valid is None else valid.numpy().astype(bool)
    for b in range(B):
        for h in range(H):
            for n in range(nb):
                acc = np.zeros(D)
                cnt = 0
                for t in range(n * bs, (n + 1) * bs):
                    if vn[t]:
                        acc += xn[b, h, t]
                        cnt += 1
                mean = acc / max(cnt, 1)
                out[b, h, n] = mean / max(math.sqrt(float((mean * mean).sum())), 1e-12)
    return out


@pytest.mark.parametrize("masked", [False, True])
def test_pool_blocks_brute_force(masked):
    x = _rand((1, 2, 6 * 16, 8), 1)
    valid = None
    if masked:
        valid = torch.rand(96, generator=torch.Generator().manual_seed(2)) > 0.3
        valid[16:32] = False  # one empty block
    hat, sums, nvalid = orc.pool_blocks(x, valid, 16)
    ref = _pool_brute(x, valid, 16)
    np.testing.assert_allclose(hat.numpy(), ref, rtol=1e-5, atol=1e-6)
    if masked:
        assert float(nvalid[1]) == 0
        assert torch.all(hat[:, :, 1] == 0)


def test_pool_blocks_closed_forms():
    # a block whose tokens are all equal to c pools to c/|c|; an all-zero block to 0
    D = 8
    c = torch.arange(1, D + 1, dtype=torch.float32)
    x = torch.zeros(1, 1, 32, D)
    x[0, 0, :16] = c
    hat, _, _ = orc.pool_blocks(x, None, 16)
    torch.testing.assert_close(hat[0, 0, 0], c / c.norm())
    assert torch.all(hat[0, 0, 1] == 0)
    # invalid tokens do not move the mean
    y = x.clone()
    y[0, 0, 8:16] = 1e6
    valid = torch.ones(32, dtype=torch.bool)
    valid[8:16] = False
    hat2, _, n = orc.pool_blocks(y, valid, 16)
    torch.testing.assert_close(hat2[0, 0, 0], c / c.norm())
    assert n.tolist() == [8.0, 16.0]


# ---------------------------------------------------------------- scores

def test_block_scores_brute_force_and_bounds():
    q = F.normalize(_rand((2, 5, 16), 3), dim=-1)
    k = F.normalize(_rand((2, 7, 16), 4), dim=-1)
    s = orc.block_scores(q, k)
    qn, kn = q.double().numpy(), k.double().numpy()
    ref = np.array([[[sum(qn[b, i, d] * kn[b, j, d] for d in range(16)) for j in range(7)]
                     for i in range(5)] for b in range(2)])
    np.testing.assert_allclose(s.numpy(), ref, rtol=1e-5, atol=1e-6)
    assert float(s.abs().max()) <= 1 + 1e-6  # Cauchy-Schwarz on unit vectors
    self_s = orc.block_scores(q, q)
    torch.testing.assert_close(torch.diagonal(self_s, dim1=-2, dim2=-1),
                               torch.ones(2, 5), atol=1e-6, rtol=0)


# ---------------------------------------------------------------- stencil

def test_local_stencil_loop():
    nt, nh, nw = 3, 2, 4
    n = nt * nh * nw
    m = orc.local_stencil(n, nh, nw)
    for a in range(n):
        ta, ha, wa = a // (nh * nw), (a // nw) % nh, a % nw
        for b in range(n):
            tb, hb, wb = b // (nh * nw), (b // nw) % nh, b % nw
            assert bool(m[a, b]) == (abs(ta - tb) + abs(ha - hb) + abs(wa - wb) <= 1)
    assert torch.equal(m, m.T)
    assert int(m.sum(1).max()) <= 7


# ---------------------------------------------------------------- top-k

def _select_brute(score, k, forced, allowed, order):
    """Python sort with tuple keys: allowed first, then forced, score desc (NaN as
    +inf, -0 as +0), index asc; keep min(k, n_allowed); index or rank order."""
    nbh, nq, nk = score.shape
    idx, cnt = [], []
    for r in range(nbh):
        ri, rc = [], []
        for i in range(nq):
            cols = []
            for j in range(nk):
                s = float(score[r, i, j])
                if math.isnan(s):
                    s = math.inf
                if s == 0:
                    s = 0.0
                a = True if allowed is None else bool(allowed[r, i, j])
                f = False if forced is None else bool(forced[r, i, j])
                cols.append((not a, not f, -s, j))
            cols.sort()
            kk = k if isinstance(k, int) else int(k[r, i])
            n_allowed = sum(1 for c in cols if not c[0])
            c = min(kk, n_allowed)
            sel = [t[3] for t in cols[:c]]
            if order == "index":
                sel.sort()
            ri.append(sel)
            rc.append(c)
        idx.append(ri)
        cnt.append(rc)
    return idx, cnt


def _tie_heavy_scores(nbh, nq, nk, seed):
    g = torch.Generator().manual_seed(seed)
    s = torch.randint(-4, 5, (nbh, nq, nk), generator=g).float() / 4  # many exact ties
    s[0, 0, :3] = torch.tensor([0.0, -0.0, float("nan")])
    return s


@pytest.mark.parametrize("order", ["index", "rank"])
@pytest.mark.parametrize("seed", [0, 1, 2])
def test_select_topk_brute_force(order, seed):
    nbh, nq, nk = 3, 5, 23
    s = _tie_heavy_scores(nbh, nq, nk, seed)
    g = torch.Generator().manual_seed(100 + seed)
    forced = torch.rand(nbh, nq, nk, generator=g) < 0.15
    allowed = torch.rand(nbh, nq, nk, generator=g) < 0.8
    allowed[1, 2] = False  # a row with nothing allowed
    allowed[2, 3, :] = False
    allowed[2, 3, :4] = True  # a row with fewer allowed than k
    k = torch.randint(0, 12, (nbh, nq), generator=g)
    idx, cnt = orc.select_topk(s, k, forced=forced, allowed=allowed, max_k=12, order=order)
    bi, bc = _select_brute(s, k, forced, allowed, order)
    for r in range(nbh):
        for i in range(nq):
            c = bc[r][i]
            assert int(cnt[r, i]) == c
            assert idx[r, i, :c].tolist() == bi[r][i]
            assert torch.all(idx[r, i, c:] == -1)


def test_select_topk_invariants():
    nbh, nq, nk = 2, 6, 40
    s = _rand((nbh, nq, nk), 7)
    forced = torch.zeros(nq, nk, dtype=torch.bool)
    forced[:, ::8] = True  # 5 forced per row, as an anchor interval of 8
    forced_scores = s.clone()
    forced_scores[:, :, ::8] = -10.0  # forced columns carry the lowest scores
    idx, cnt = orc.select_topk(forced_scores, 9, forced=forced)
    for r in range(nbh):
        for i in range(nq):
            sel = set(idx[r, i, :9].tolist())
            assert set(range(0, nk, 8)) <= sel          # every forced block kept
            rest = sorted(sel - set(range(0, nk, 8)))
            free = [j for j in range(nk) if j % 8]
            best = sorted(free, key=lambda j: (-float(s[r, i, j]), j))[:4]
            assert rest == sorted(best)                 # then the best 4 by score
    assert torch.all(cnt == 9)


def test_topk_margin_brute_force():
    s = _rand((2, 4, 15), 9)
    forced = torch.zeros(4, 15, dtype=torch.bool)
    forced[0, :3] = True
    m = orc.topk_margin(s, 5, forced=forced)
    for r in range(2):
        for i in range(4):
            f = [bool(forced[i, j]) for j in range(15)]
            cols = sorted(range(15), key=lambda j: (not f[j], -float(s[r, i, j]), j))
            a, b = cols[4], cols[5]
            want = math.inf if f[a] != f[b] else float(s[r, i, a] - s[r, i, b])
            assert float(m[r, i]) == pytest.approx(want, rel=1e-6)


def test_planted_tie_order_is_caught():
    """Ties broken towards the higher index (a plausible slip) disagree with the
    brute-force rule on tie-heavy scores."""
    s = _tie_heavy_scores(2, 4, 19, 5)
    flipped = torch.flip(s, dims=[-1])
    idx_f, cnt = orc.select_topk(flipped, 6, order="rank")
    wrong = (18 - idx_f).clamp(max=18)  # index map back: ties now prefer high index
    bi, _ = _select_brute(s, 6, None, None, "rank")
    mismatched = any(wrong[r, i, :6].tolist() != bi[r][i] for r in range(2) for i in range(4))
    assert mismatched


# ---------------------------------------------------------------- quantiser

def test_quantize_query_error_bound_and_range():
    q = _rand((1, 2, 64, 16), 11) * 3
    valid = torch.ones(64, dtype=torch.bool)
    valid[40:] = False
    q8, scale = orc.quantize_query_blocks(q, valid, 32)
    deq = orc.dequantize_blocks(q8, scale, 32)
    x = q.reshape(1, 2, 2, 32, 16)
    err = (deq.reshape(1, 2, 2, 32, 16) - x).abs()
    sc = scale.reshape(1, 2, 2, 1, 1)
    vm = valid.reshape(2, 32)[None, None, :, :, None]
    assert torch.all(torch.where(vm, err, torch.zeros_like(err)) <= sc / 2 * (1 + 1e-6))
    assert int(q8.abs().max()) == 127
    assert torch.all(q8.reshape(1, 2, 64, 16)[:, :, 40:] == 0)
    # the block's largest |q| lands exactly on +-127
    for h in range(2):
        for n in range(2):
            blk = x[0, h, n][vm[0, 0, n, :, 0]]
            amax = float(blk.abs().max())
            assert float(scale[h, n]) == pytest.approx(amax / 127, rel=1e-7)


def test_quantize_idempotent_and_zero_block():
    q = _rand((1, 1, 64, 16), 12)
    q[0, 0, 32:] = 0
    q8, scale = orc.quantize_query_blocks(q, None, 32)
    assert float(scale[0, 1]) == 1.0 and torch.all(q8[0, 0, 32:] == 0)
    deq = orc.dequantize_blocks(q8, scale, 32)
    q8b, scale_b = orc.quantize_query_blocks(deq, None, 32)
    assert torch.equal(q8, q8b)
    torch.testing.assert_close(scale, scale_b, rtol=1e-6, atol=0)


def test_key_mean_and_smoothing_invariance():
    k = _rand((1, 2, 48, 8), 13, torch.float64)
    valid = torch.ones(48, dtype=torch.bool)
    valid[5] = valid[30] = False
    m = orc.key_mean(k.float(), valid)
    want = k[0][:, valid].mean(dim=1)
    torch.testing.assert_close(m.double(), want.reshape(2, 8), rtol=1e-6, atol=1e-7)
    # softmax(q . (k - m)) == softmax(q . k): the per-head mean shifts every
    # logit of a query row by the same q . m
    q = _rand((2, 5, 8), 14, torch.float64)
    a = torch.softmax(q @ k[0].transpose(-1, -2), dim=-1)
    b = torch.softmax(q @ (k[0] - m.double()[:, None]).transpose(-1, -2), dim=-1)
    torch.testing.assert_close(a, b, rtol=1e-12, atol=1e-14)


def test_quantize_key_error_bound():
    k = _rand((1, 2, 64, 16), 15) + 5.0  # a large common offset
    valid = torch.ones(64, dtype=torch.bool)
    valid[60:] = False
    m = orc.key_mean(k, valid)
    k8, scale = orc.quantize_key_blocks(k, valid, 32, m)
    deq = orc.dequantize_blocks(k8, scale, 32) + m.reshape(1, 2, 1, 16)
    err = (deq - k).abs().reshape(1, 2, 2, 32, 16)
    vm = valid.reshape(2, 32)[None, None, :, :, None]
    sc = scale.reshape(1, 2, 2, 1, 1)
    assert torch.all(torch.where(vm, err, torch.zeros_like(err)) <= sc / 2 * (1 + 1e-5))
    # smoothing shrinks the scale well below the unsmoothed absmax/127
    assert float(scale.max()) < float(k.abs().max()) / 127 * 0.75


# ---------------------------------------------------------------- attention

def _attn_brute(q, k, v, blocks_per_qblock, kvalid, bm, bn, scale):
    """fp64 per-row loops: explicit max-shifted exp and sums."""
    B, H, Lq, D = q.shape
    Lk = k.shape[2]
    out = np.zeros((B, H, Lq, D))
    lse = np.full((B, H, Lq), -np.inf)
    qn, kn, vn = q.double().numpy(), k.double().numpy(), v.double().numpy()
    for b in range(B):
        for h in range(H):
            for r in range(Lq):
                keys = [t for n in blocks_per_qblock[b][h][r // bm]
                        for t in range(n * bn, min((n + 1) * bn, Lk)) if kvalid[t]]
                if not keys:
                    continue
                logits = [scale * float(np.dot(qn[b, h, r], kn[b, h, t])) for t in keys]
                mx = max(logits)
                w = [math.exp(x - mx) for x in logits]
                z = sum(w)
                out[b, h, r] = sum(wi * vn[b, h, t] for wi, t in zip(w, keys)) / z
                lse[b, h, r] = mx + math.log(z)
    return out, lse


def test_sparse_attention_brute_force():
    B, H, D, bm, bn = 1, 2, 16, 8, 8
    Lq, Lk = 20, 44  # ragged: the last query block holds 4 rows, the last key block 4 keys
    q, k, v = _rand((B, H, Lq, D), 21), _rand((B, H, Lk, D), 22), _rand((B, H, Lk, D), 23)
    kvalid = torch.rand(Lk, generator=torch.Generator().manual_seed(24)) > 0.2
    kvalid[8:16] = False  # a fully masked key block
    nqb = 3
    idx = torch.full((B, H, nqb, 4), -1, dtype=torch.int32)
    cnt = torch.zeros(B, H, nqb, dtype=torch.int32)
    lists = [[[[5, 0, 2], [1], [3, 4, 5, 0]], [[], [1, 2], [4]]]]
    for h in range(H):
        for m in range(nqb):
            L = lists[0][h][m]
            idx[0, h, m, :len(L)] = torch.tensor(L, dtype=torch.int32)
            cnt[0, h, m] = len(L)
    out, lse = orc.sparse_attention(q, k, v, idx, cnt, kvalid, block_m=bm, block_n=bn,
                                    dtype=torch.float64)
    ref_o, ref_l = _attn_brute(q, k, v, lists, kvalid.tolist(), bm, bn, 1 / math.sqrt(D))
    np.testing.assert_allclose(out.numpy(), ref_o, rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(lse.numpy(), ref_l, rtol=1e-10, atol=1e-12)
    # the empty list and the block of masked keys both give 0 output / lse -inf
    assert torch.all(out[0, 1, :8] == 0) and torch.all(torch.isinf(lse[0, 1, :8]))
    assert torch.all(out[0, 0, 8:16] == 0)


def test_sparse_attention_matches_dense_sdpa():
    """With every block selected and every key valid the op is textbook attention."""
    B, H, L, D, bs = 1, 3, 32, 16, 8
    q, k, v = (_rand((B, H, L, D), s, torch.float64) for s in (31, 32, 33))
    nb = L // bs
    idx = torch.arange(nb, dtype=torch.int32).expand(B, H, nb, nb).contiguous()
    cnt = torch.full((B, H, nb), nb, dtype=torch.int32)
    out, _ = orc.sparse_attention(q, k, v, idx, cnt, None, block_m=bs, block_n=bs,
                                  dtype=torch.float64)
    ref = F.scaled_dot_product_attention(q, k, v)
    torch.testing.assert_close(out, ref, rtol=1e-10, atol=1e-12)


def test_sparse_attention_closed_forms():
    D, bs = 8, 4
    q = _rand((1, 1, 4, D), 41)
    v = _rand((1, 1, 8, D), 42)
    idx = torch.tensor([[[[1]]]], dtype=torch.int32)
    cnt = torch.tensor([[[1]]], dtype=torch.int32)
    # one valid key -> its value row, lse = its logit
    kvalid = torch.tensor([0, 0, 0, 0, 0, 0, 1, 0], dtype=torch.bool)
    k = _rand((1, 1, 8, D), 43)
    out, lse = orc.sparse_attention(q, k, v, idx, cnt, kvalid, block_m=bs, block_n=bs)
    torch.testing.assert_close(out[0, 0], v[0, 0, 6].expand(4, D))
    torch.testing.assert_close(lse[0, 0], (q[0, 0] @ k[0, 0, 6]) / math.sqrt(D))
    # equal logits (zero query) -> the mean of the listed values
    out0, lse0 = orc.sparse_attention(torch.zeros_like(q), k, v, idx, cnt, None,
                                      block_m=bs, block_n=bs)
    torch.testing.assert_close(out0[0, 0], v[0, 0, 4:8].mean(0).expand(4, D))
    torch.testing.assert_close(lse0[0, 0], torch.full((4,), math.log(4.0)))
    # index order inside the list does not matter
    idx2 = torch.tensor([[[[1, 0]]]], dtype=torch.int32)
    idx3 = torch.tensor([[[[0, 1]]]], dtype=torch.int32)
    c2 = torch.tensor([[[2]]], dtype=torch.int32)
    a, _ = orc.sparse_attention(q, k, v, idx2, c2, None, block_m=bs, block_n=bs)
    b, _ = orc.sparse_attention(q, k, v, idx3, c2, None, block_m=bs, block_n=bs)
    torch.testing.assert_close(a, b)


def test_planted_scale_slip_is_caught():
    """Forgetting the 1/sqrt(D) factor (a plausible slip) fails the dense pin."""
    B, H, L, D, bs = 1, 1, 16, 16, 8
    q, k, v = (_rand((B, H, L, D), s, torch.float64) for s in (51, 52, 53))
    idx = torch.arange(2, dtype=torch.int32).expand(B, H, 2, 2).contiguous()
    cnt = torch.full((B, H, 2), 2, dtype=torch.int32)
    wrong, _ = orc.sparse_attention(q, k, v, idx, cnt, None, block_m=bs, block_n=bs,
                                    sm_scale=1.0, dtype=torch.float64)
    ref = F.scaled_dot_product_attention(q, k, v)
    assert float((wrong - ref).abs().max()) > 1e-3


def test_sparse_attention_int8_is_dequantised_attention():
    B, H, L, D, bs = 1, 1, 16, 8, 8
    q, k, v = _rand((B, H, L, D), 61), _rand((B, H, L, D), 62), _rand((B, H, L, D), 63)
    q8, qs = orc.quantize_query_blocks(q, None, bs)
    m = orc.key_mean(k, None)
    k8, ks = orc.quantize_key_blocks(k, None, bs, m)
    idx = torch.arange(2, dtype=torch.int32).expand(B, H, 2, 2).contiguous()
    cnt = torch.full((B, H, 2), 2, dtype=torch.int32)
    a, _ = orc.sparse_attention_int8(q8, qs, k8, ks, v, idx, cnt, None, block_m=bs, block_n=bs)
    b, _ = orc.sparse_attention(orc.dequantize_blocks(q8, qs, bs), orc.dequantize_blocks(k8, ks, bs),
                                v, idx, cnt, None, block_m=bs, block_n=bs)
    torch.testing.assert_close(a, b)
    # and, by smoothing invariance, close to the unquantised result
    c, _ = orc.sparse_attention(q, k, v, idx, cnt, None, block_m=bs, block_n=bs)
    assert orc.equivalence_stats(c, a)["cosine"] > 0.999


def test_equivalence_stats_closed_forms():
    r = torch.tensor([3.0, 4.0])
    s = orc.equivalence_stats(r, r)
    assert s["cosine"] == pytest.approx(1.0) and s["max_abs"] == 0 and s["relative_l2"] == 0
    s2 = orc.equivalence_stats(r, torch.tensor([3.0, 5.0]))
    assert s2["relative_l2"] == pytest.approx(1 / 5, rel=1e-5)
    assert s2["max_abs"] == 1.0 and s2["mae"] == 0.5
    assert s2["cosine"] == pytest.approx(29 / (5 * math.sqrt(34)), rel=1e-6)


# ---------------------------------------------------------------- layout

def _layout_argsort(active_frames, mem_t, H, W, shape):
    """Independent formulation: block id per compact token, then a stable argsort."""
    tt, th, tw = shape
    frames = sorted(active_frames)
    ct, spatial = len(frames), H * W
    nh, nw = -(-H // th), -(-W // tw)
    cm = sum(1 for f in frames if f < mem_t)
    tok = np.arange(ct * spatial)
    lt, ls = tok // spatial, tok % spatial
    if cm:
        cells = -(-cm // tt)
        cell = np.where(lt < cm, lt // tt, cells + (lt - cm) // tt)
        nb = (cells + -(-(ct - cm) // tt)) * nh * nw
    else:
        cell = lt // tt
        nb = -(-ct // tt) * nh * nw
    bid = cell * nh * nw + (ls // W // th) * nw + (ls % W) // tw
    order = np.argsort(bid, kind="stable")
    return bid, order, nb


@pytest.mark.parametrize("frames,mem_t,H,W,shape", [
    ([0, 1, 2, 3], 0, 8, 8, (2, 4, 4)),
    ([0, 2, 5, 6, 7], 3, 6, 10, (2, 4, 4)),   # ragged spatial tiles + memory split
    ([1, 4], 2, 4, 4, (4, 2, 2)),
])
def test_compact_layout_vs_argsort(frames, mem_t, H, W, shape):
    idx, valid, t2p = orc.compact_layout(frames, mem_t, H, W, shape)
    bid, order, nb = _layout_argsort(frames, mem_t, H, W, shape)
    assert idx.shape[0] == nb
    bs = shape[0] * shape[1] * shape[2]
    flat = idx.reshape(-1)
    members = flat[flat >= 0].numpy()
    # grouped by block id, stable inside a block
    np.testing.assert_array_equal(np.sort(members), np.arange(len(bid)))
    np.testing.assert_array_equal(bid[members], np.sort(bid[order]))
    np.testing.assert_array_equal(members, order)
    # round trip: packed slot of token t holds t
    np.testing.assert_array_equal(flat[t2p].numpy(), np.arange(len(bid)))
    assert int(valid.sum()) == len(bid) and valid.shape == (nb, bs)


def test_relay_layout_hand_example():
    """3 frames (1 memory) of 2 x 3 tokens in (2, 1, 2) blocks, enumerated by hand."""
    pc = orc.relay_layout(3, 1, 2, 3, (2, 1, 2), [2])
    P = -1
    assert pc["key"].tolist() == [[0, 1, P, P], [2, P, P, P], [3, 4, P, P], [5, P, P, P],
                                  [6, 7, 12, 13], [8, 14, P, P], [9, 10, 15, 16], [11, 17, P, P]]
    # frame 2 shares its cell with frame 1: the query rows keep frame 2's tokens only
    assert pc["query_block_ids"].tolist() == [4, 5, 6, 7]
    assert pc["query"].tolist() == [[12, 13, P, P], [14, P, P, P], [15, 16, P, P], [17, P, P, P]]
    assert pc["query_indices"].tolist() == list(range(12, 18))
    un = orc.relay_layout(3, 1, 2, 3, (2, 1, 2), [0, 2], protected_current=False)
    assert un["key"].tolist() == [[0, 1, 6, 7], [2, 8, P, P], [3, 4, 9, 10], [5, 11, P, P],
                                  [12, 13, P, P], [14, P, P, P], [15, 16, P, P], [17, P, P, P]]
    assert un["query_block_ids"].tolist() == list(range(8))
    assert un["query"][0].tolist() == [0, 1, P, P] and un["query"][4].tolist() == [12, 13, P, P]


@pytest.mark.parametrize("T,mem,qf,prot", [(12, 4, [5, 6, 9], True), (19, 5, list(range(5, 19)), True),
                                           (8, 0, [1, 2, 7], True), (10, 3, [0, 4, 8], False)])
def test_relay_layout_invariants(T, mem, qf, prot):
    H, W, shape = 22, 40, (4, 4, 8)
    r = orc.relay_layout(T, mem, H, W, shape, qf, protected_current=prot)
    key, q = r["key"], r["query"]
    flat = key.reshape(-1)
    members = flat[flat >= 0]
    assert torch.equal(members.sort().values, torch.arange(T * H * W))  # each token once
    # rows hold increasing tokens, padding at the end
    for row in list(key) + list(q):
        live = row[row >= 0]
        assert torch.equal(live, live.sort().values) and bool((row[len(live):] < 0).all())
    # each query row = its key row's members that lie in a query frame
    qset = set(qf)
    for b, row in zip(r["query_block_ids"].tolist(), q):
        want = [t for t in key[b].tolist() if t >= 0 and t // (H * W) in qset]
        assert row[row >= 0].tolist() == want and want
    assert r["query_indices"].tolist() == [t for t in range(T * H * W) if t // (H * W) in qset]


# ---------------------------------------------------------------- budgets

def test_apportion_textbook_and_invariants():
    assert orc.apportion([0.5, 0.3, 0.2], 10) == [5, 3, 2]
    assert orc.apportion([1, 1, 1], 10) == [4, 3, 3]       # ties to the lower index
    assert orc.apportion([0, 0, 0], 4) == [2, 1, 1]        # all-zero weights -> uniform
    assert orc.apportion([-1, 3], 5) == [0, 5]              # negatives clamp to 0
    # Hamilton's method on a classic example: quotas 1.32, 3.37, 5.31 of 10 seats
    assert orc.apportion([132, 337, 531], 10) == [1, 4, 5]
    rnd = random.Random(0)
    for _ in range(200):
        n = rnd.randint(1, 9)
        w = [rnd.random() for _ in range(n)]
        total = rnd.randint(0, 50)
        res = orc.apportion(w, total)
        assert sum(res) == total
        quota = [Fraction(total) * Fraction(x) / sum(map(Fraction, w)) for x in w]
        assert all(abs(r - qv) < 1 for r, qv in zip(res, quota))  # quota rule
    rows = orc.apportion_section_matrix([[1, 2], [3, 1]], 7)
    assert rows == [orc.apportion([1, 2], 7), orc.apportion([3, 1], 7)]
    assert all(sum(r) == 7 for r in rows)


def test_budget_blocks_round_half_even():
    assert orc.budget_blocks(0.25, 275) == 69    # 68.75
    assert orc.budget_blocks(0.125, 275) == 34   # 34.375
    assert orc.budget_blocks(0.5, 275) == 138    # 137.5 -> 138 (even)
    assert orc.budget_blocks(0.5, 273) == 136    # 136.5 -> 136 (even)


# ---------------------------------------------------------------- whole layer

def test_rcsa_layer_composes_the_pinned_parts():
    from cast_amd import workloads
    w = workloads.plumbing(0)
    res = orc.rcsa_layer(w.q, w.k, w.v, w.q_valid, w.k_valid, block_size=w.block_size,
                         k_select=w.k_total, forced=w.forced)
    qhat, _, _ = orc.pool_blocks(w.q, w.q_valid, w.block_size)
    khat, _, _ = orc.pool_blocks(w.k, w.k_valid, w.block_size)
    score = orc.block_scores(qhat, khat).reshape(res["score"].shape)
    torch.testing.assert_close(res["score"], score)
    # the current chunk's blocks are forced and so always selected
    nh = w.n_hist_blocks
    for r in range(res["indices"].shape[0]):
        for i in range(res["indices"].shape[1]):
            sel = set(res["indices"][r, i].tolist())
            assert set(range(nh, w.n_kblocks)) <= sel


def test_saturate_pins():
    """Oracle saturation against its closed forms on random rows: the result sums
    to min(target, n * cap), never exceeds cap, keeps every row that was at or
    below cap at least where it was, and fills the lowest-index rows first (a
    row only gains when every lower row with room gained at least as much)."""
    import random
    rnd = random.Random(7)
    for _ in range(300):
        n = rnd.randint(1, 30)
        cap = rnd.randint(1, 12)
        deg = [rnd.randint(0, 20) for _ in range(n)]
        target = rnd.randint(0, 25 * n)
        got = orc.saturate(deg, cap, target)
        clamped = [min(x, cap) for x in deg]
        assert sum(got) == max(sum(clamped), min(target, n * cap))
        assert all(g <= cap for g in got)
        assert all(g >= c for g, c in zip(got, clamped))
        gain = [g - c for g, c in zip(got, clamped)]
        for i in range(n):
            for j in range(i):
                if clamped[j] + gain[j] < cap:  # row j still had room at the end
                    assert gain[j] >= gain[i]
    # a hand case: 2 edges lost to the cap go to rows 1 and 2
    assert orc.saturate([12, 1, 1], 10, 14) == [10, 2, 2]


# --------------------------------------------------------------------------
# closed-loop allocator (P/control_response_cwca_attention.py:1123-1363 and
# P/matrix_curvature_phase_frame_weave.py:5727-5817)

def test_compact_time_cells_hand_example():
    vals = torch.tensor([[1.0, 10.0], [2.0, 20.0], [3.0, 30.0]])
    # offset 3, source tiles of 4 frames: frames 0-2 are unprofiled (0), 3-6
    # read tile 0, 7-10 tile 1, 11-14 tile 2; cells of 2 frames
    got = orc.compact_time_cells(vals, [1, 3, 7, 8, 14], 2, 4, 3)
    want = torch.tensor([[(0 + 1) / 2, (0 + 10) / 2], [(2 + 2) / 2, (20 + 20) / 2], [3.0, 30.0]])
    assert torch.allclose(got, want)
    with pytest.raises(RuntimeError, match="outside CWCA tiles"):
        orc.compact_time_cells(vals, [15], 2, 4, 3)


def test_redistribute_closed_forms():
    g = torch.Generator().manual_seed(4)
    for _ in range(50):
        cells, S, cap = 4, 6, int(torch.randint(5, 12, (1,), generator=g))
        d = torch.randint(0, 20, (cells, S), generator=g)
        target = int(torch.randint(0, cells * cap + 1, (1,), generator=g))
        out = orc.redistribute_compact_capacity(d.clone(), capacity=cap,
                                                target_per_worldline=target)
        assert int(out.max()) <= cap
        for s in range(S):
            col0 = d[:, s].clamp(max=cap)
            want = max(target, int(col0.sum()))  # edges are only added, never removed
            assert int(out[:, s].sum()) == want
            assert torch.all(out[:, s] >= col0)
    with pytest.raises(RuntimeError, match="exhausted key capacity"):
        orc.redistribute_compact_capacity(torch.zeros(2, 1, dtype=torch.long), capacity=3,
                                          target_per_worldline=7)


def _fraction_closed_loop(curv, frames, offset, src, grp, mean, base, blocks, mem):
    """The allocation re-derived with exact rationals on the oracle's fp32 weights."""
    from fractions import Fraction
    cur = curv.float()
    norm = cur / cur.mean(dim=0, keepdim=True).clamp_min(torch.finfo(torch.float32).eps)
    cells = orc.compact_time_cells(norm, frames, grp, src, offset)
    w = (1.0 + torch.log1p(cells)).tolist()
    tc, S = len(w), len(w[0])
    deg = [[0] * S for _ in range(tc)]
    for s in range(S):
        col = [max(Fraction(w[c][s]), Fraction(0)) for c in range(tc)]
        share = orc.apportion([float(x) for x in col], tc * (mean - base))
        for c in range(tc):
            deg[c][s] = share[c] + base
    full = [mean] * mem + [deg[c][s] for c in range(tc) for s in range(S)]
    assert len(full) == blocks
    return full


def test_closed_loop_conservation_and_rationals():
    g = torch.Generator().manual_seed(9)
    for trial in range(20):
        S, tsrc = 6, 3
        curv = torch.rand(tsrc, S, generator=g) * 2 + 0.05
        frames = sorted(torch.randperm(14, generator=g)[:8].tolist())
        cells = -(-len(frames) // 4)
        mem, mean, base = 2 * S, 7, 5
        blocks = mem + cells * S
        d = orc.closed_loop_degrees(curv, frames, current_temporal_offset=2, source_group=4,
                                    compact_group=4, mean_degree=mean, base_degree=base,
                                    total_blocks=blocks, memory_blocks=mem)
        assert int(d.sum()) == blocks * mean
        assert torch.all(d[:mem] == mean)
        cur = d[mem:].reshape(cells, S)
        assert torch.all(cur.sum(0) == cells * mean) and torch.all(cur >= base)
        exact = _fraction_closed_loop(curv, frames, 2, 4, 4, mean, base, blocks, mem)
        assert d.tolist() == exact, trial


def test_closed_loop_uniform_and_slips():
    # uniform curvature: every cell of a worldline gets the same bonus when it divides
    curv = torch.full((2, 5), 0.7)
    d = orc.closed_loop_degrees(curv, [0, 1, 2, 3, 4, 5, 6, 7], current_temporal_offset=0,
                                source_group=4, compact_group=4, mean_degree=9, base_degree=7,
                                total_blocks=10 + 10, memory_blocks=10)
    assert torch.all(d == 9)
    # a planted slip -- no per-worldline column normalisation -- changes the split
    g = torch.Generator().manual_seed(2)
    curv = torch.rand(3, 6, generator=g) * torch.tensor([1.0, 3.0, 9.0, 0.2, 5.0, 1.0])
    kw = dict(current_temporal_offset=0, source_group=4, compact_group=4, mean_degree=30,
              base_degree=24, total_blocks=18 + 18, memory_blocks=18)
    frames = list(range(12))
    good = orc.closed_loop_degrees(curv, frames, **kw)
    slip = orc.closed_loop_degrees(curv / curv.mean(dim=0, keepdim=True), frames, **kw)
    assert torch.equal(good, slip)  # the normalisation is idempotent ...
    raw_w = 1.0 + torch.log1p(orc.compact_time_cells(curv, frames, 4, 4, 0))
    raw = orc.apportion_section_matrix_f32(raw_w.transpose(0, 1), 3 * 6).transpose(0, 1) + 24
    assert not torch.equal(good[18:].reshape(3, 6), raw)  # ... and dropping it is caught
    # the fixed query budget ignores the curvature
    fixed = orc.closed_loop_degrees(curv, frames, fixed_query_budget=True, **kw)
    assert torch.all(fixed == 30)
    # response feedback moves edges towards responsive cells (additive form)
    resp = torch.zeros(3, 6)
    resp[1] = 5.0
    fb = orc.closed_loop_degrees(curv, frames, response=resp, response_weight=1.0, **kw)
    cur, base_cur = fb[18:].reshape(3, 6), good[18:].reshape(3, 6)
    assert torch.all(cur[1] >= base_cur[1]) and int(cur[1].sum()) > int(base_cur[1].sum())


# ---------------------------------------------------------------- a7 router

def _route_cfg(**kw):
    from types import SimpleNamespace
    base = dict(candidate_multiplier=2, num_swap_rounds=1, swap_eps=1e-6, lambda_anchor=1.0,
                lambda_reconstruction=1.0, sketch_groups=16, require_fc_transport=False,
                min_transport_affinity=0.0, min_pair_transport_affinity=0.0,
                max_swaps_per_call=0, active_layers=(), historical_only=False,
                same_bank_only=False)
    base.update(kw)
    return SimpleNamespace(**base)


def _route_case(seed, *, H=2, mem=6, hw=(2, 3), cells=2, D=32, K=7):
    g = torch.Generator().manual_seed(seed)
    S = hw[0] * hw[1]
    N = mem + cells * S
    qh = torch.nn.functional.normalize(torch.randn(1, H, N, D, generator=g), dim=-1)
    kh = torch.nn.functional.normalize(torch.randn(1, H, N, D, generator=g), dim=-1)
    score = qh @ kh.transpose(-1, -2) * 4.0
    pooled_v = torch.randn(1, H, N, D, generator=g)
    local = torch.eye(N, dtype=torch.bool)  # the block itself is its only protected edge
    # selection: the block itself, then the best others by score
    rank = score + local[None, None] * 1e6
    sel = torch.sort(rank, dim=-1, descending=True, stable=True).indices[..., :K]
    counts = torch.randint(3, K + 1, (1, H, N), generator=g)
    return score, pooled_v, sel, counts, local


def test_route_fallbacks_are_identity():
    """Without transport (or with it switched off) the route comes back unchanged,
    with the reference's fallback reason (P/fc_pasm_swap_routing.py:647-748)."""
    score, pv, sel, cnt, local = _route_case(0)
    kw = dict(memory_blocks=6, spatial_shape=(2, 3), exact_current_frames=(0, 6),
              temporal_group_size=4, current_boundary=8, layer_index=22)
    cast_cfg = _route_cfg(require_fc_transport=True, min_transport_affinity=0.5,
                          max_swaps_per_call=1, active_layers=(22, 26), same_bank_only=True,
                          swap_eps=0.1)
    cases = [
        (cast_cfg, None, kw, "missing_previous_layer_fc_transport"),
        (cast_cfg, {"pairs": {(0, 6): {"theta": torch.zeros(1, 1, 1), "mean_affinity": 0.2}}},
         kw, "weak_previous_layer_fc_transport"),
        (cast_cfg, None, dict(kw, layer_index=5), "layer_not_enabled"),
        (_route_cfg(), None, dict(kw, exact_current_frames=(3,)), "fewer_than_two_exact_anchors"),
        (_route_cfg(), None, dict(kw, exact_current_frames=(3, 4)), "no_skipped_frames"),
        (_route_cfg(num_swap_rounds=0), None, kw, "zero_swap_rounds"),
        (_route_cfg(), None, dict(kw, memory_blocks=5), "no_rectangular_current_rows"),
    ]
    for cfg, transport, kwargs, reason in cases:
        out, rec = orc.fc_pasm_refine(score, pv, sel, cnt, local, transport=transport,
                                      config=cfg, **kwargs)
        assert torch.equal(out, sel) and rec["fallback_reason"] == reason, reason
        assert rec["swap_count"] == 0 and rec["status"] == "independent_topk_fallback"


def test_refine_refuses_invalid_routes():
    """The checks on the final route (P/fc_pasm_swap_routing.py:980-1033): a
    route that does not hold a row's local stencil, or holds a key twice,
    raises the reference's error."""
    score, pv, sel, cnt, local = _route_case(1)
    kw = dict(memory_blocks=6, spatial_shape=(2, 3), exact_current_frames=(0, 6),
              temporal_group_size=4, current_boundary=8, layer_index=0, transport=None)
    cfg = _route_cfg()
    out, rec = orc.fc_pasm_refine(score, pv, sel, cnt, local, config=cfg, **kw)
    assert rec["status"] == "refined"
    dropped = cnt.clone()
    dropped[0, 1, 9] = 0                   # row 9 keeps nothing, not even itself
    with pytest.raises(RuntimeError, match="removed a protected local edge"):
        orc.fc_pasm_refine(score, pv, sel, dropped, local, config=cfg, **kw)
    twice = sel.clone()
    twice[0, 0, 2, 1] = twice[0, 0, 2, 0]  # memory row 2 lists its first key twice
    with pytest.raises(RuntimeError, match="duplicate keys"):
        orc.fc_pasm_refine(score, pv, twice, cnt, local, config=cfg, **kw)


def test_omission_proxy_fp64_loops():
    g = torch.Generator().manual_seed(3)
    B, H, Q, K, D, L, G = 1, 2, 5, 9, 32, 4, 16
    prob = torch.softmax(torch.randn(B, H, Q, K, generator=g) * 3, dim=-1)
    v = torch.randn(B, H, K, D, generator=g)
    cand = torch.stack([torch.randperm(K, generator=g)[:L] for _ in range(B * H * Q)]).reshape(B, H, Q, L)
    got = orc.omission_proxy(prob, v, cand, sketch_groups=G)
    P, V = prob.double(), v.double()
    for b in range(B):
        for h in range(H):
            for q in range(Q):
                o = [sum(float(P[b, h, q, k]) * float(V[b, h, k, d]) for k in range(K)) for d in range(D)]
                for li in range(L):
                    c = int(cand[b, h, q, li])
                    p = float(P[b, h, q, c])
                    w = p / (1.0 - p + 1e-6)
                    for gi in range(G):
                        ds = range(gi * (D // G), (gi + 1) * (D // G))
                        want = sum(w * (o[d] - float(V[b, h, c, d])) for d in ds) / len(ds)
                        assert abs(float(got[b, h, q, li, gi]) - want) < 1e-5


def _route_operator_random(seed, S):
    g = torch.Generator().manual_seed(seed)
    mats = {}

    def op(pair, exponent):
        if pair not in mats:
            mats[pair] = torch.randn(S, S, generator=g) * 0.2
        return torch.eye(S) + exponent * mats[pair]
    return op


@pytest.mark.parametrize("operator_seed", [None, 5])
@pytest.mark.parametrize("frames,boundary", [((0, 6), 8), ((0, 3, 7), 8), ((1, 3, 5, 7), 4)])
def test_route_objective_terms_match_value_changes(operator_seed, frames, boundary):
    """Changing one row's error by d changes the objective value by exactly the
    quadratic form the terms predict."""
    g = torch.Generator().manual_seed(11)
    S, cells, G = 6, 2, 4
    op = _route_operator_random(operator_seed, S) if operator_seed is not None else None
    kw = dict(temporal_cells=cells, spatial=S, exact_frames=frames, temporal_group_size=4,
              current_boundary=boundary, operator=op, lambda_anchor=0.7,
              lambda_reconstruction=1.3)
    e = torch.randn(1, 2, cells * S, G, generator=g).double().float()
    a, b, used = orc.route_objective_terms(e, **kw)
    assert used == (operator_seed is not None and any(r - l > 1 for l, r in zip(frames, frames[1:])
                                                      if (l < boundary) == (r < boundary)))
    base = orc.route_objective_value(e, **kw)
    for h in range(2):
        for r in range(cells * S):
            d = torch.randn(G, generator=g)
            e2 = e.clone()
            e2[0, h, r] += d
            want = float(orc.route_objective_value(e2, **kw) - base)
            pred = float((a[0, 0, r, 0] * (2 * e[0, h, r] * d + d * d) + 2 * b[0, h, r] * d).sum())
            assert abs(pred - want) <= 1e-3 * max(1.0, abs(want)), (h, r, pred, want)


@pytest.mark.parametrize("same_bank", [False, True])
@pytest.mark.parametrize("operator_seed", [None, 7])
def test_route_swap_is_the_best_single_swap(same_bank, operator_seed):
    """The refine's swap equals a brute-force search of every admissible
    (row, removed slot, added candidate) exchange by objective value."""
    score, pv, sel, cnt, local = _route_case(4)
    mem, S, cells = 6, 6, 2
    op = _route_operator_random(operator_seed, S) if operator_seed is not None else None
    cfg = _route_cfg(same_bank_only=same_bank, max_swaps_per_call=1)
    kw = dict(memory_blocks=mem, spatial_shape=(2, 3), exact_current_frames=(0, 6),
              temporal_group_size=4, current_boundary=8, layer_index=0, transport=None)
    out, rec = orc.fc_pasm_refine(score, pv, sel, cnt, local, config=cfg, operator=op, **kw)
    assert rec["status"] == "refined"
    # brute force, from the oracle's own proxy and candidates
    N = score.shape[-1]
    K = sel.shape[-1]
    L = min(N, 2 * int(cnt.max()))
    cand = torch.sort(score + local[None, None] * 1e6, dim=-1, descending=True, stable=True).indices[..., :L]
    proxy = orc.omission_proxy(torch.softmax(score, -1), pv, cand, sketch_groups=16)
    limit = torch.clamp(cnt * 2, max=N)
    okw = dict(temporal_cells=cells, spatial=S, exact_frames=(0, 6), temporal_group_size=4,
               current_boundary=8, operator=op)
    err = torch.zeros(1, 2, N, proxy.shape[-1])
    for h in range(2):
        for r in range(N):
            kept = set(sel[0, h, r, :cnt[0, h, r]].tolist())
            for li in range(int(limit[0, h, r])):
                if int(cand[0, h, r, li]) not in kept:
                    err[0, h, r] += proxy[0, h, r, li]
    cur = err[:, :, mem:]
    base = float(orc.route_objective_value(cur, **okw))
    best = (0.0, None)
    for h in range(2):
        for rr in range(cells * S):
            r = mem + rr
            n = int(cnt[0, h, r])
            kept = sel[0, h, r, :n].tolist()
            for s_ in range(n):
                rem = kept[s_]
                if bool(local[r, rem]):
                    continue
                rp = sum((proxy[0, h, r, li] for li in range(L) if int(cand[0, h, r, li]) == rem),
                         torch.zeros(proxy.shape[-1]))
                for li in range(int(limit[0, h, r])):
                    add = int(cand[0, h, r, li])
                    if add in kept or (same_bank and ((rem < mem) != (add < mem))):
                        continue
                    e2 = cur.clone()
                    e2[0, h, rr] += rp - proxy[0, h, r, li]
                    imp = float(orc.route_objective_value(e2, **okw)) - base
                    if imp < best[0] - 1e-9:
                        best = (imp, (h, r, s_, add))
    if best[1] is None or best[0] >= -cfg.swap_eps:
        assert rec["swap_count"] == 0
    else:
        h, r, s_, add = best[1]
        sw = rec["swaps"][0]
        assert (sw["h"], sw["row"], sw["slot"], sw["added"]) == (h, r, s_, add)
        assert abs(-sw["improvement"] - best[0]) <= 1e-3 * max(1.0, abs(best[0]))
        assert int(out[0, h, r, s_]) == add
        assert rec["objective_after"] <= rec["objective_before"]


def _transport(seed, zero_theta=False):
    g = torch.Generator().manual_seed(seed)
    theta = (torch.rand(18, 6, 3, generator=g) * 2 - 1) * math.pi
    if zero_theta:
        theta = torch.zeros_like(theta)
    return {"output_shape": (22, 40), "transport_shape": (6, 5), "window_shape": (11, 10),
            "stride": (8, 8), "padding": (4, 5), "tile_grid": (3, 6),
            "pairs": {(0, 6): {"theta": theta, "affinity": torch.rand(18, 6, 3, generator=g),
                               "mean_affinity": torch.tensor(0.8)}}}


def test_transport_maps_identities():
    """No phase (exponent 0, or theta 0) moves nothing; a phase moves something."""
    g = torch.Generator().manual_seed(2)
    maps = torch.randn(3, 2, 6, 5, generator=g)
    tr = _transport(1)
    assert float(orc.transport_maps(tr, (0, 6), maps, 0.0).abs().max()) == 0.0
    assert float(orc.transport_maps(_transport(1, True), (0, 6), maps, 0.7).abs().max()) == 0.0
    moved = orc.transport_maps(tr, (0, 6), maps, 0.5)
    assert moved.shape == maps.shape and float(moved.abs().max()) > 1e-3
    # linear in the maps
    both = orc.transport_maps(tr, (0, 6), maps[:1] + 2 * maps[1:2], 0.5)
    torch.testing.assert_close(both, moved[:1] + 2 * moved[1:2], atol=1e-5, rtol=1e-5)


# ---------------------------------------------------------------- f4 int8 QKV

def test_quantize_rows_int8_bounds():
    g = torch.Generator().manual_seed(5)
    x = torch.randn(40, 64, generator=g) * torch.rand(40, 1, generator=g) * 10
    x[3] = 0.0
    q, s = orc.quantize_rows_int8(x)
    assert q.dtype == torch.int8 and int(q.abs().max()) <= 127
    err = (q.float() * s[:, None] - x).abs()
    assert bool((err <= s[:, None] / 2 + 1e-6).all())
    live = torch.arange(40) != 3
    assert bool((q[live].abs().amax(dim=1) == 127).all())
    assert float(s[3]) == 1.0 and int(q[3].abs().max()) == 0
    q2, s2 = orc.quantize_rows_int8(q.float() * s[:, None])   # idempotent on its grid
    assert torch.equal(q2, q)


def test_int8_linear_integer_loops():
    g = torch.Generator().manual_seed(6)
    M, N, K = 5, 7, 33
    x = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8)
    w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    xs, ws = torch.rand(M, generator=g) * 0.02, torch.rand(N, generator=g) * 0.02
    bias = torch.randn(N, generator=g)
    got = orc.int8_linear(x, xs, w, ws, bias)
    for m in range(M):
        for n in range(N):
            acc = sum(int(x[m, k]) * int(w[n, k]) for k in range(K))
            y = torch.tensor(acc, dtype=torch.float32) * xs[m] * ws[n]
            want = y.to(torch.bfloat16) + bias[n].to(torch.bfloat16)
            assert got[m, n] == want
    # the largest product a 3072-wide projection can accumulate stays exact in int32
    assert 3072 * 127 * 127 < 2 ** 31

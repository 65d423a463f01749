"""The key quantiser with the block scores and top-k in its launch
(rcsa_quantize_key_select) against the separate calls, bit for bit: C2
(303 key blocks), C3 (853 key blocks, 8 forced anchors, near-tied rows) and a
per-row k; and the int8 layer call with and without the fused launch."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _workload(case):
    from cast_amd import workloads
    dev = torch.device("cuda:0")
    if case == "c2":
        return workloads.matrix_dit(0, int8=True).to(dev)
    return workloads.selection_stress(0).to(dev)


@pytest.mark.parametrize("case", ["c2", "c3"])
def test_quantize_key_select_matches_separate(case):
    from cast_amd import ops
    w = _workload(case)
    print(f"fused select {case} k {tuple(w.k.shape)} k_total {w.k_total}", flush=True)
    p = ops.pool_query_key(w.q, w.q_valid, w.k, w.k_valid, 128)
    qhat, khat, ks, kn, kx = p[0], p[3], p[4], p[5], p[6]
    nq = qhat.shape[1]
    row_k = torch.full((nq,), w.k_total, dtype=torch.int32)
    row_k[::3] -= 5  # a per-row budget too
    for k_sel in (w.k_total, row_k):
        sc = ops.block_scores(qhat, khat)
        idx, cnt = ops.select_topk(sc, k_sel, forced=w.forced, max_k=w.k_total)
        want = ops.quantize_key(w.k, w.k_valid, 128, ks, kn, kx) + (sc, idx, cnt)
        got = ops.quantize_key_select(w.k, w.k_valid, 128, ks, kn, kx, qhat, khat, k_sel,
                                      forced=w.forced, max_k=w.k_total)
        names = ("k_i8", "k_scale", "kmean", "score", "indices", "counts")
        for name, a, b in zip(names, want, got):
            assert a.shape == b.shape and torch.equal(a, b), (name, type(k_sel))


def test_layer_call_fused_select_matches_side_stream():
    from cast_amd.pipeline import rcsa_attention
    w = _workload("c2")
    kw = dict(block_size=128, k_select=w.k_total, forced=w.forced, int8=True,
              max_k=w.k_total, return_lse=True)
    a = rcsa_attention(w.q, w.k, w.v, w.q_valid, w.k_valid, fuse_select=True, **kw)
    b = rcsa_attention(w.q, w.k, w.v, w.q_valid, w.k_valid, fuse_select=False, **kw)
    torch.cuda.synchronize()
    for name in ("out", "indices", "counts", "score", "k_i8", "k_scale", "lse"):
        assert torch.equal(getattr(a, name), getattr(b, name)), name


def _allowed(kind, nbh, nq, nk, seed):
    """Causal-permission masks: every current block allowed, a seeded 80% of history."""
    g = torch.Generator().manual_seed(seed)
    shape = (nq, nk) if kind == "shared" else (nbh, nq, nk)
    m = torch.rand(*shape, generator=g) < 0.8
    m[..., nk - 28:] = True
    return m


@pytest.mark.parametrize("allowed_kind", [None, "shared", "per_head"])
@pytest.mark.parametrize("row_k_kind", ["int", "per_head"])
def test_fused_select_masks_and_row_k(allowed_kind, row_k_kind):
    """Allowed masks of either shape (the forced mask stays [NQ, NK], so the ABI
    broadcasts one of them), a per-head [NBH, NQ] row_k with rows at 0 and above
    max_k, against rcsa_select_topk."""
    from cast_amd import ops, workloads
    dev = torch.device("cuda:0")
    w = workloads.matrix_dit(3, heads=6, int8=True).to(dev)
    p = ops.pool_query_key(w.q, w.q_valid, w.k, w.k_valid, 128)
    qhat, khat, ks, kn, kx = p[0], p[3], p[4], p[5], p[6]
    nbh, nq, nk = qhat.shape[0], qhat.shape[1], khat.shape[1]
    allowed = None if allowed_kind is None else _allowed(allowed_kind, nbh, nq, nk, 4).to(dev)
    max_k = w.k_total
    if row_k_kind == "int":
        k_sel = w.k_total
    else:
        g = torch.Generator().manual_seed(5)
        k_sel = torch.randint(0, max_k + 8, (nbh, nq), generator=g, dtype=torch.int32)
        k_sel[0, :3] = 0
        k_sel[1, :3] = max_k + 7
        k_sel = k_sel.to(dev)
    print(f"fused select allowed={allowed_kind} row_k={row_k_kind}", flush=True)
    sc = ops.block_scores(qhat, khat)
    idx, cnt = ops.select_topk(sc, k_sel, forced=w.forced, allowed=allowed, max_k=max_k)
    want = ops.quantize_key(w.k, w.k_valid, 128, ks, kn, kx) + (sc, idx, cnt)
    got = ops.quantize_key_select(w.k, w.k_valid, 128, ks, kn, kx, qhat, khat, k_sel,
                                  forced=w.forced, allowed=allowed, max_k=max_k)
    names = ("k_i8", "k_scale", "kmean", "score", "indices", "counts")
    for name, a, b in zip(names, want, got):
        assert a.shape == b.shape and torch.equal(a, b), name
    if row_k_kind == "per_head":
        assert int(got[5][0, 0]) == 0 and int(got[5][1, 0]) <= max_k


def test_fused_select_slot_token():
    """The gathered (slot map) form of the fused launch against the separate calls."""
    from cast_amd import layout, ops
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(9)
    H, D = 4, 128
    lay_q = layout.compact_layout(range(4), 0, 22, 40, (4, 4, 8), dev)
    lay_k = layout.compact_layout(range(12), 8, 22, 40, (4, 4, 8), dev)
    q = (torch.randn(1, 4 * 880, H, D, generator=g) / D ** 0.5).bfloat16().to(dev)
    k = (torch.randn(1, 12 * 880, H, D, generator=g) / D ** 0.5).bfloat16().to(dev)
    p = ops.pool_query_key(q, None, k, None, 128, q_slot_token=lay_q.slot_token,
                           k_slot_token=lay_k.slot_token)
    qhat, khat, ks, kn, kx = p[0], p[3], p[4], p[5], p[6]
    nq, nk = lay_q.n_blocks, lay_k.n_blocks
    forced = torch.zeros(nq, nk, dtype=torch.bool)
    forced[:, nk - 30:] = True
    k_sel = 30 + 12
    sc = ops.block_scores(qhat, khat)
    idx, cnt = ops.select_topk(sc, k_sel, forced=forced, max_k=k_sel)
    want = ops.quantize_key(k, None, 128, ks, kn, kx, slot_token=lay_k.slot_token) + \
        (sc, idx, cnt)
    got = ops.quantize_key_select(k, None, 128, ks, kn, kx, qhat, khat, k_sel, forced=forced,
                                  max_k=k_sel, slot_token=lay_k.slot_token)
    names = ("k_i8", "k_scale", "kmean", "score", "indices", "counts")
    for name, a, b in zip(names, want, got):
        assert a.shape == b.shape and torch.equal(a, b), name

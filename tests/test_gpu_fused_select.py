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

"""CPU checks of the committed golden fixtures: the seeded generators still
produce the fixtures' inputs, and the oracle still reproduces their outputs."""
import numpy as np
import pytest
import torch

import _golden
from oracle import rcsa_oracle as orc


@pytest.mark.parametrize("name", ["c0_plumbing", "c1_dit_bf16", "c2_dit_int8", "c3_selection"])
def test_generator_fingerprint(name):
    fx = _golden.load(name)
    assert _golden.fingerprint(_golden.workload(name)) == str(fx["fingerprint"])


@pytest.mark.parametrize("name", [f"c{c}_seed{s}" for c in (1, 2) for s in (1, 2, 3, 4)])
def test_seed_fixture(name):
    """Seeds 1-4: the generator still makes the fixture's inputs, every row
    keeps the forced current blocks and the full budget, and the oracle
    reproduces the selection of one head."""
    fx = _golden.seed_fixture(name)
    w = _golden.workload(name)
    assert _golden.fingerprint(w) == str(fx["fingerprint"])
    idx, cnt = fx["indices"], fx["counts"]
    assert np.all(cnt == w.k_total)
    cur = set(range(w.n_hist_blocks, w.n_kblocks))
    assert all(cur <= set(idx[r, i, :cnt[r, i]].tolist())
               for r in range(idx.shape[0]) for i in range(idx.shape[1]))
    h = int(fx["head"])
    i0, _ = orc.select_topk(_scores(w, [h]), w.k_total, forced=w.forced)
    np.testing.assert_array_equal(i0.numpy(), idx[h:h + 1])


def test_c0_oracle_reproduces_fixture():
    fx = _golden.load("c0_plumbing")
    w = _golden.workload("c0_plumbing")
    for tag, int8 in (("bf16", False), ("int8", True)):
        res = orc.rcsa_layer(w.q, w.k, w.v, w.q_valid, w.k_valid, block_size=w.block_size,
                             k_select=w.k_total, forced=w.forced, int8=int8)
        np.testing.assert_allclose(res["score"].numpy(), fx["score"], atol=1e-6, rtol=0)
        np.testing.assert_array_equal(res["indices"].numpy(), fx["indices"])
        np.testing.assert_array_equal(res["counts"].numpy(), fx["counts"])
        np.testing.assert_allclose(res["out"].numpy(), fx[f"out_{tag}"].astype(np.float32),
                                   atol=2e-3, rtol=1e-3)
        np.testing.assert_allclose(res["lse"].numpy(), fx[f"lse_{tag}"], atol=1e-5, rtol=1e-6)
        if int8:
            np.testing.assert_array_equal(res["q_scale"].numpy(), fx["q_scale"])
            np.testing.assert_array_equal(res["k_scale"].numpy(), fx["k_scale"])


def _scores(w, heads):
    qhat, _, _ = orc.pool_blocks(w.q[:, heads], w.q_valid, w.block_size)
    khat, _, _ = orc.pool_blocks(w.k[:, heads], w.k_valid, w.block_size)
    return orc.block_scores(qhat, khat).reshape(len(heads), qhat.shape[2], khat.shape[2])


def test_c1_scores_and_selection():
    fx = _golden.load("c1_dit_bf16")
    w = _golden.workload("c1_dit_bf16")
    score = _scores(w, [0, 1])
    np.testing.assert_allclose(score.numpy(), fx["score_h01"], atol=1e-6, rtol=0)
    idx, cnt = orc.select_topk(score, w.k_total, forced=w.forced)
    np.testing.assert_array_equal(idx.numpy(), fx["indices"][:2])
    np.testing.assert_array_equal(cnt.numpy(), fx["counts"][:2])
    assert np.all(fx["counts"] == w.k_total)


def test_c1_attention_rows():
    fx = _golden.load("c1_dit_bf16")
    w = _golden.workload("c1_dit_bf16")
    nqb = w.n_qblocks
    idx = torch.from_numpy(fx["indices"].astype(np.int32)).reshape(1, 24, nqb, -1)
    cnt = torch.from_numpy(fx["counts"]).reshape(1, 24, nqb)
    out, lse = orc.sparse_attention(w.q, w.k, w.v, idx, cnt, w.k_valid, block_m=128,
                                    block_n=128, heads=[0], qblocks=[0])
    rows = fx["attn_rows"][:128]
    np.testing.assert_allclose(out[0, 0, rows].numpy(), fx["out_h0"][:128], atol=1e-5, rtol=0)
    np.testing.assert_allclose(lse[0, 0, rows].numpy(), fx["lse_h0"][:128], atol=1e-5, rtol=0)


def test_c2_quantiser_scales():
    fx = _golden.load("c2_dit_int8")
    w = _golden.workload("c2_dit_int8")
    np.testing.assert_array_equal(np.asarray(w.meta["outlier_channels"]), fx["outlier_channels"])
    _, qs = orc.quantize_query_blocks(w.q[:, :2], w.q_valid, 128)
    km = orc.key_mean(w.k[:, :2], w.k_valid)
    _, ks = orc.quantize_key_blocks(w.k[:, :2], w.k_valid, 128, km)
    np.testing.assert_array_equal(qs.numpy(), fx["q_scale"][:2])
    np.testing.assert_array_equal(km.numpy(), fx["kmean"][:2])
    np.testing.assert_array_equal(ks.numpy(), fx["k_scale"][:2])
    # the int8 result of the fixture is within the path's tolerance of fp32 attention
    st = orc.equivalence_stats(torch.from_numpy(fx["out_h0_unquantised"]),
                               torch.from_numpy(fx["out_h0"]))
    assert st["cosine"] >= 0.999 and st["max_abs"] <= 3e-2


def test_c3_selection_invariants():
    fx = _golden.load("c3_selection")
    w = _golden.workload("c3_selection")
    idx, cnt = fx["indices"], fx["counts"]
    assert np.all(cnt == w.k_total)
    forced = w.forced.numpy()
    for r in range(idx.shape[0]):
        for i in range(idx.shape[1]):
            sel = set(idx[r, i, :cnt[r, i]].tolist())
            assert set(np.nonzero(forced[i])[0].tolist()) <= sel
    # the tied rows really are near-tied: their margins sit at the tie spread or below
    tied = fx["tied_rows"]
    assert np.median(fx["margin"].reshape(-1)[tied]) < 1e-3
    score = _scores(w, [0])
    i0, _ = orc.select_topk(score, w.k_total, forced=w.forced)
    np.testing.assert_array_equal(i0.numpy(), idx[:1])

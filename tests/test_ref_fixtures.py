"""The oracle's router transport / objective / refine, closed-loop allocator,
native-layer selection (pooling, cosine scores, local stencil, top-k) and
largest-remainder apportionments against fixtures the CAST reference itself
produced (tests/golden/make_ref_golden.py: P/fc_pasm_swap_routing.py:116-1077,
P/control_response_cwca_attention.py:1123-1363,
P/qk_uncertainty_tangent_attention.py:847-870, 988-1082, 1239-1264), and the
product's host-side transport operator and budget splits against the same
fixtures.

The GPU router and allocator are compared with these fixtures in
tests/test_gpu_ref_fixtures.py.
"""
import numpy as np
import pytest
import torch

from tests._ref_fixtures import (SELECT_CASES, apportion_cases, closed_loop_case,
                                 closed_loop_count, fp32_near_tie, motion_cases, objective_case,
                                 oracle_operator, refine_case, refine_count, router_fixture,
                                 select_case, select_grid, transport_case)
from oracle import rcsa_oracle as orc


@pytest.mark.parametrize("ci", [0, 1])
def test_oracle_transport_maps_match_reference(ci):
    tr, block, maps, exps, outs, mats = transport_case(ci)
    S = block[0] * block[1]
    eye = torch.eye(S).reshape(S, 1, *block)
    for a, want, want_mat in zip(exps, outs, mats):
        got = maps + orc.transport_maps(tr, (0, 6), maps, float(a))
        torch.testing.assert_close(got, want, atol=2e-6, rtol=1e-5)
        # the operator [output, input]: transport of the unit maps, transposed
        op = (torch.eye(S) + orc.transport_maps(tr, (0, 6), eye, float(a)).reshape(S, S)).T
        torch.testing.assert_close(op, want_mat, atol=2e-6, rtol=1e-5)


@pytest.mark.parametrize("ci", [0, 1])
def test_product_transport_operator_matches_reference(ci):
    from cast_amd.transport import fc_transport_operator, transport_maps
    tr, block, maps, exps, outs, mats = transport_case(ci)
    for a, want, want_mat in zip(exps, outs, mats):
        op = fc_transport_operator(tr, (0, 6), block, float(a))
        torch.testing.assert_close(op, want_mat, atol=2e-6, rtol=1e-5)
        torch.testing.assert_close(maps + transport_maps(tr, (0, 6), maps, float(a)), want,
                                   atol=2e-6, rtol=1e-5)


def test_transport_fixture_is_not_trivial():
    """The fixture would catch a transposed operator or a conjugated phase: the
    reference's operators are far from symmetric and from the zero-phase identity,
    and exponents of opposite sign give different operators."""
    for ci in (0, 1):
        tr, block, maps, exps, outs, mats = transport_case(ci)
        S = block[0] * block[1]
        for m in mats:
            assert float((m - torch.eye(S)).abs().max()) > 1e-2
            assert float((m - m.T).abs().max()) > 1e-3
        assert float((mats[0] - mats[1]).abs().max()) > 1e-2


@pytest.mark.parametrize("tag", ["g0", "fc"])
def test_oracle_objective_matches_reference(tag):
    err, kw, op, want_value, want_a, want_b = objective_case(tag)
    value = orc.route_objective_value(err, operator=op, **kw)
    a, b, used = orc.route_objective_terms(err, operator=op, **kw)
    assert used == (tag == "fc")
    assert abs(float(value) - want_value) <= 1e-5 * abs(want_value)
    torch.testing.assert_close(a, want_a, atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(b, want_b, atol=1e-6, rtol=1e-4)


def test_objective_fixture_distinguishes_transport():
    _, _, _, v0, a0, b0 = objective_case("g0")
    _, _, _, v1, a1, b1 = objective_case("fc")
    assert abs(v0 - v1) > 1e-3 * abs(v0)
    assert float((a0 - a1).abs().max()) > 1e-3


@pytest.mark.parametrize("ci", range(refine_count()))
def test_oracle_refine_matches_reference(ci):
    c = refine_case(ci)
    want_out, _, _ = c["out"], c["swap_count"], c["objective"]
    got, rec = orc.fc_pasm_refine(c["score"], c["pooled_value"], c["selected"], c["counts"],
                                  c["local"], transport=c["transport"], config=c["config"],
                                  operator=oracle_operator(c["transport"], c["block"]),
                                  **c["kw"])
    assert rec["status"] == "refined"
    assert rec["swap_count"] == c["swap_count"]
    assert torch.equal(got, want_out)
    before, after = c["objective"]
    assert abs(rec["objective_before"] - before) <= 1e-5 * abs(before)
    assert abs(rec["objective_after"] - after) <= 1e-5 * abs(after)
    assert [rec["historical_budget_before"], rec["historical_budget_after"]] == \
        list(c["historical_budget"])


def test_refine_fixtures_change_the_route():
    for ci in range(refine_count()):
        c = refine_case(ci)
        assert not torch.equal(c["out"], c["selected"])
        assert c["objective"][1] < c["objective"][0]


@pytest.mark.parametrize("ci", range(closed_loop_count()))
def test_oracle_closed_loop_matches_reference(ci):
    c = closed_loop_case(ci)
    p = c["params"]
    got = orc.closed_loop_degrees(c["curvature"], c["frames"], **c["oracle_kw"])
    mem = p["memory"]
    assert torch.equal(got[:mem], torch.full((mem,), p["mean"], dtype=torch.long))
    assert torch.equal(got[mem:], c["degrees"].reshape(-1))
    cells = orc.compact_time_cells(c["normalized"], c["frames"], p["compact_group"], 4,
                                   p["offset"])
    torch.testing.assert_close(cells, c["time_cells"], atol=0, rtol=0)


def test_closed_loop_fixtures_cover_the_feedback_forms():
    """The three feedback forms give three different allocations of the same
    curvature and response, and the peaked case saturates a row at the layer's
    block count."""
    deg = [closed_loop_case(i)["degrees"] for i in range(3)]
    assert not torch.equal(deg[0], deg[1]) and not torch.equal(deg[1], deg[2]) \
        and not torch.equal(deg[0], deg[2])
    peaked = closed_loop_case(closed_loop_count() - 1)
    assert int(peaked["degrees"].max()) == peaked["params"]["total"]


def test_oracle_redistribution_matches_reference():
    fx = router_fixture("closed_loop")
    got = orc.redistribute_compact_capacity(torch.from_numpy(fx["redistribute_in"]).clone(),
                                            capacity=10, target_per_worldline=18)
    assert torch.equal(got, torch.from_numpy(fx["redistribute_out"]))


def test_planted_closed_loop_mistake_is_caught():
    """A slip in the oracle (the centred inverse form with the sign of the
    multiplicative one) no longer matches the reference's allocation."""
    c = closed_loop_case(2)
    kw = dict(c["oracle_kw"], feedback_form="centered_multiplicative")
    got = orc.closed_loop_degrees(c["curvature"], c["frames"], **kw)
    assert not torch.equal(got[c["params"]["memory"]:], c["degrees"].reshape(-1))
    np.testing.assert_array_equal(
        orc.closed_loop_degrees(c["curvature"], c["frames"], **c["oracle_kw"])
        [c["params"]["memory"]:].numpy(), c["degrees"].reshape(-1).numpy())


def _oracle_select(c, *, stencil_as_mask_only=False):
    """The oracle's composition of the native select: visual tiles as the
    compact layout of every frame, pool_blocks, block_scores, local_stencil,
    select_topk in rank order at each row's budget.  The reference ranks a
    local block by fl(score + 1e6) (a 0.0625 grid at 1e6), so the oracle is
    given those values for the local columns, as the product does."""
    case = c["case"]
    q, k = c["q"], c["k"]
    B, H = q.shape[:2]
    idx, valid, _ = orc.compact_layout(range(case["T"]), 0, case["height"], case["width"],
                                       case["block_shape"])
    nb, bs = idx.shape
    flat, vflat = idx.reshape(-1).clamp_min(0), valid.reshape(-1)

    def pack(x):
        return x[:, :, flat] * vflat[None, None, :, None]
    qh, _, _ = orc.pool_blocks(pack(q), vflat, bs)
    kh, _, _ = orc.pool_blocks(pack(k), vflat, bs)
    score = orc.block_scores(qh, kh).reshape(B * H, nb, nb)
    _, nh, nw = select_grid(case)
    local = orc.local_stencil(nb, nh, nw)
    ranking = score if stencil_as_mask_only else torch.where(local, (score + 1e6) - 1e6, score)
    rows = c["rows"]
    sel, cnt = orc.select_topk(ranking, torch.tensor(rows), forced=local, max_k=max(rows),
                               order="rank")
    return sel.reshape(B, H, nb, -1), cnt.reshape(B, H, nb), score


@pytest.mark.parametrize("ci", range(len(SELECT_CASES)))
def test_oracle_select_matches_reference(ci):
    """Every row's selected prefix (its budget's worth, in rank order) and
    count equal the reference's select()."""
    c = select_case(ci)
    sel, cnt, score = _oracle_select(c)
    want = c["selected"]
    assert torch.equal(cnt, c["counts"])
    B, H, nb, _ = want.shape
    for b in range(B):
        for h in range(H):
            for r in range(nb):
                n = int(c["rows"][r])
                assert torch.equal(sel[b, h, r, :n], want[b, h, r, :n].to(torch.int32)), \
                    (ci, b, h, r)
    rep = c["report"]
    assert abs(float(score.double().mean()) - rep[0]) < 1e-6
    assert [int(v) for v in rep[3:]] == [min(c["rows"]), max(c["rows"]), sum(c["rows"])]


def test_select_fixtures_order_local_blocks_by_the_rounded_bonus():
    """The reference orders the local blocks by fl(score + 1e6), not by the
    exact score: ranking them by the exact score (the stencil only as a mask)
    changes the rank order of some row, so the fixtures pin that detail."""
    changed = False
    for ci in range(len(SELECT_CASES)):
        c = select_case(ci)
        sel, _, _ = _oracle_select(c, stencil_as_mask_only=True)
        want = c["selected"].to(torch.int32)
        changed |= not torch.equal(sel[..., :want.shape[-1]], want)
    assert changed


# ---- largest-remainder apportionments ----

def test_fp32_apportion_matches_reference():
    """orc.apportion_section_matrix_f32 (the reference's fp32 arithmetic) equals
    the reference's _apportion and _apportion_section_matrix on every stored
    split, the fp32 near-tie cases included."""
    cases = apportion_cases()
    assert len(cases) >= 17
    for name, w, total, want in cases:
        mat = w if w.ndim == 2 else w[None]
        got = orc.apportion_section_matrix_f32(mat, total).reshape(want.shape)
        assert torch.equal(got, want), name
        assert bool((want.sum(dim=-1) == total).all()), name


def test_exact_apportion_differs_from_reference_only_at_fp32_ties():
    """The exact-rational restatement (orc.apportion) equals the reference
    except on rows whose fractional parts tie within 1e-5, where fp32 rounding
    decides; the fixtures hold such rows (decimal weights), so the difference
    is real and confined to them."""
    differing = 0
    for name, w, total, want in apportion_cases():
        rows = w if w.ndim == 2 else w[None]
        wants = want if want.ndim == 2 else want[None]
        for r in range(rows.shape[0]):
            got = orc.apportion(rows[r].tolist(), total)
            if got != wants[r].tolist():
                differing += 1
                assert fp32_near_tie(rows[r], total), (name, r)
                assert sum(got) == total
                assert max(abs(a - b) for a, b in zip(got, wants[r].tolist())) <= 1
    assert differing >= 4


def test_host_budget_splits_match_reference():
    """cast_amd.budget.apportion / apportion_section_matrix and the motion
    row budgets (1 + motion / (mean + eps), then _apportion of n * degree)
    equal the reference bit for bit."""
    from cast_amd import budget
    for name, w, total, want in apportion_cases():
        got = (budget.apportion_section_matrix(w, total) if w.ndim == 2
               else budget.apportion(w, total))
        assert torch.equal(got, want), name
    for motion, degree, w_ref, rows_ref in motion_cases():
        n = motion.numel()
        eps = torch.finfo(torch.float32).eps
        assert torch.equal(1.0 + motion / (motion.mean() + eps), w_ref)
        rows = budget.motion_row_degrees(motion, degree, torch.zeros(n, 1, dtype=torch.bool))
        assert torch.equal(rows, rows_ref)

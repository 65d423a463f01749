"""The device router (FCPASMSwapRouter.refine: route_proxy_kernel /
route_swap_kernel) and the device closed-loop allocator
(rcsa_closed_loop_degrees) against fixtures written by the CAST reference's
own FCPASMLocalCoordinateSwapRouter.refine (P/fc_pasm_swap_routing.py:616-1077)
and compact_closed_loop_degrees (P/control_response_cwca_attention.py:1188-1363),
and the device selection of the native layers (cast_amd.selector.taba_select:
pooling, scores and top-k kernels) against the reference's own
MatrixTrajectoryAdaptiveBudgetAttentionCompiler.select
(P/qk_uncertainty_tangent_attention.py:988-1082), and the device per-row
budgets (rcsa_row_budgets) against its _apportion and _apportion_section_matrix
(:847-865, 1239-1264) (tests/golden/make_ref_golden.py)."""
import pytest
import torch

from tests._ref_fixtures import (SELECT_CASES, apportion_cases, closed_loop_case,
                                 closed_loop_count, fp32_near_tie, refine_case, refine_count,
                                 select_case)

pytestmark = pytest.mark.gpu


def _to(tr, dev):
    pairs = {p: {k: (v.to(dev) if isinstance(v, torch.Tensor) and v.ndim else v)
                 for k, v in e.items()} for p, e in tr["pairs"].items()}
    return dict(tr, pairs=pairs)


@pytest.mark.parametrize("ci", range(refine_count()))
def test_gpu_refine_matches_reference(dev, ci):
    from cast_amd.router import FCPASMSwapRouter
    c = refine_case(ci)
    print(f"refine fixture {ci}: same_bank {c['config'].same_bank_only} rounds "
          f"{c['config'].num_swap_rounds}", flush=True)
    got, rec = FCPASMSwapRouter(c["config"]).refine(
        score=c["score"].to(dev), pooled_value=c["pooled_value"].to(dev),
        selected=c["selected"].to(dev), counts=c["counts"].to(dev), local=c["local"].to(dev),
        transport=_to(c["transport"], dev), **c["kw"])
    torch.cuda.synchronize()
    assert rec["status"] == "refined" and rec["fc_cache_used"]
    assert rec["swap_count"] == c["swap_count"]
    assert torch.equal(got.cpu().long(), c["out"].long())
    before, after = c["objective"]
    assert abs(float(rec["objective_before"]) - before) <= 1e-4 * abs(before)
    assert abs(float(rec["objective_after"]) - after) <= 1e-4 * abs(after)
    assert [rec["historical_budget_before"], rec["historical_budget_after"]] == \
        c["historical_budget"]


@pytest.mark.parametrize("ci", range(closed_loop_count()))
def test_gpu_closed_loop_matches_reference(dev, ci):
    from cast_amd import ops
    c = closed_loop_case(ci)
    p, kw = c["params"], c["oracle_kw"]
    print(f"closed-loop fixture {ci}: {kw['feedback_form']} layer {p['layer']}", flush=True)
    got = ops.closed_loop_degrees(
        c["curvature"].to(dev), c["frames"], current_temporal_offset=p["offset"],
        source_group=p["source_group"], compact_group=p["compact_group"],
        mean_degree=p["mean"], base_degree=p["base"], total_blocks=p["total"],
        memory_blocks=p["memory"],
        response=kw["response"].to(dev) if p["layer"] > 0 and kw["response_weight"] else None,
        response_weight=kw["response_weight"], feedback_form=kw["feedback_form"],
        fixed_query_budget=p["fixed"])
    got = got.cpu().long()
    mem = p["memory"]
    assert torch.equal(got[:mem], torch.full((mem,), p["mean"], dtype=torch.long))
    assert torch.equal(got[mem:], c["degrees"].reshape(-1).long())


@pytest.mark.parametrize("ci", range(len(SELECT_CASES)))
def test_gpu_select_matches_reference(dev, ci):
    """taba_select on a stand-in compiler holding the attributes the
    reference's select reads: every row's selected prefix (rank order) and
    count, and the report's budget fields, equal the reference's."""
    from types import SimpleNamespace
    from cast_amd.selector import taba_select
    c = select_case(ci)
    case = c["case"]
    B, H = c["q"].shape[:2]
    rows = torch.tensor(c["rows"], dtype=torch.long)
    nb = rows.numel()
    comp = SimpleNamespace(
        _block_shape=tuple(case["block_shape"]), _num_blocks=nb, _degree=case["degree"],
        _row_degrees=rows, _ray_motion=torch.linspace(0.1, 1.0, nb),
        _first_order_motion=torch.linspace(0.2, 0.8, nb),
        trajectory_complexity_kind="motion_magnitude")
    comp._runtime_degrees = lambda q_blocks: comp._row_degrees
    print(f"select fixture {ci}: B {B} H {H} blocks {nb} tile {case['block_shape']}", flush=True)
    counts_in = torch.full((B, H, nb), case["degree"], dtype=torch.int32, device=dev)
    sel, cnt, rep = taba_select(
        comp, c["q"].to(dev), c["k"].to(dev),
        geometry_indices=torch.zeros(B, H, nb, case["degree"], dtype=torch.int32, device=dev),
        geometry_counts=counts_in, latent_hw=(case["height"], case["width"]),
        block_shape=tuple(case["block_shape"]))
    sel, cnt = sel.cpu(), cnt.cpu()
    want = c["selected"].to(torch.int32)
    assert torch.equal(cnt, c["counts"])
    for b in range(B):
        for h in range(H):
            for r in range(nb):
                n = int(rows[r])
                assert torch.equal(sel[b, h, r, :n], want[b, h, r, :n]), (ci, b, h, r)
    assert (rep.budget_min, rep.budget_max, rep.budget_total) == \
        (int(rows.min()), int(rows.max()), int(rows.sum()))
    assert abs(rep.mean_selected_qk_cosine - c["report"][0]) < 1e-5
    assert rep.protected_local_edges == int(c["report"][1]) and rep.missing_local_edges == 0


def test_gpu_row_budgets_match_reference(dev):
    """Every stored split, one section per row: bit for bit, except that a row
    whose fractional parts tie within 1e-5 may move one edge (the device sums
    the weights in a fixed tree order, the reference in torch's; the quotients
    can then round to the other side of the tie)."""
    from cast_amd import ops
    exact = 0
    for name, w, total, want in apportion_cases():
        rows = (w if w.ndim == 2 else w[None]).contiguous()
        wants = want if want.ndim == 2 else want[None]
        print(f"row budgets fixture {name}: {tuple(rows.shape)} total {total}", flush=True)
        got = ops.row_budgets(rows.to(dev), total).cpu().long()
        for r in range(rows.shape[0]):
            assert int(got[r].sum()) == total, (name, r)
            if torch.equal(got[r], wants[r]):
                exact += 1
                continue
            assert fp32_near_tie(rows[r], total), (name, r)
            assert int((got[r] - wants[r]).abs().max()) <= 1, (name, r)
    assert exact >= 20

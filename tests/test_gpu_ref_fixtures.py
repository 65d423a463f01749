"""The device router (FCPASMSwapRouter.refine: route_proxy_kernel /
route_swap_kernel) and the device closed-loop allocator
(rcsa_closed_loop_degrees) against fixtures written by the CAST reference's
own FCPASMLocalCoordinateSwapRouter.refine (P/fc_pasm_swap_routing.py:616-1077)
and compact_closed_loop_degrees (P/control_response_cwca_attention.py:1188-1363)
(tests/golden/make_ref_golden.py)."""
import pytest
import torch

from tests._ref_fixtures import closed_loop_case, closed_loop_count, refine_case, refine_count

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

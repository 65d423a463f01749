"""Seeded sweep of the device FC-PASM swap router against the oracle's
restatement of FCPASMLocalCoordinateSwapRouter.refine
(P/fc_pasm_swap_routing.py:616-1077).

Every case draws its geometry (spatial tiles 3 x 7, 4 x 5 or 6 x 5; 2-4
current cells; 0, 17 or 63 memory blocks; heads 1-3; head_dim 64 or 128),
the route (top-k of the pooled scores + 1e6 local at K 8-24, with per-row
counts below K that still hold the row's local stencil), two or three exact anchors with skipped frames between
them, the configuration (1 or 2 rounds, candidate multiplier 1-3, sketch
groups 4-16, objective weights, same-bank on or off) and the transport (the
identity, or a random FC operator per anchor pair).  The routes must match
bit for bit, the swap counts and the historical budget exactly, and the
objectives within 1e-4 relative.
"""
import pytest
import torch

from oracle import rcsa_oracle as orc

pytestmark = pytest.mark.gpu

N_CASES = 24


def _draw(seed: int) -> dict:
    g = torch.Generator().manual_seed(seed)

    def pick(xs):
        return xs[int(torch.randint(0, len(xs), (1,), generator=g))]

    cells = pick([2, 3, 4])
    frames = 4 * cells
    a0 = int(torch.randint(0, 2, (1,), generator=g))
    a1 = a0 + 2 + int(torch.randint(0, frames - a0 - 2, (1,), generator=g))
    anchors = [a0, a1]
    if a1 + 2 < frames and bool(torch.rand(1, generator=g) < 0.5):
        anchors.append(a1 + 2 + int(torch.randint(0, frames - a1 - 2, (1,), generator=g)))
    return dict(g=g, hw=pick([(3, 7), (4, 5), (6, 5)]), cells=cells, mem=pick([0, 17, 63]),
                H=pick([1, 2, 3]), D=pick([64, 128]), K=pick([8, 16, 24]),
                anchors=tuple(anchors), rounds=pick([1, 2]), mult=pick([1, 2, 3]),
                groups=pick([4, 8, 16]), lam=pick([(1.0, 1.0), (0.5, 2.0), (2.0, 0.25)]),
                same_bank=bool(pick([0, 1])), op=bool(pick([0, 1])))


def _inputs(c):
    g, H, D, K = c["g"], c["H"], c["D"], c["K"]
    S = c["hw"][0] * c["hw"][1]
    N = c["mem"] + c["cells"] * S
    qh = torch.nn.functional.normalize(torch.randn(1, H, N, D, generator=g), dim=-1)
    kh = torch.nn.functional.normalize(torch.randn(1, H, N, D, generator=g) + qh * 0.3, dim=-1)
    score = qh @ kh.transpose(-1, -2)
    pooled_v = torch.randn(1, H, N, D, generator=g) * 0.5
    local = orc.local_stencil(N, c["hw"][0], c["hw"][1])
    rank = score + local[None, None] * 1e6
    sel = torch.sort(rank, dim=-1, descending=True, stable=True).indices[..., :K]
    # every row keeps at least its local stencil (which ranks first): the
    # reference refuses a route that drops a protected local edge
    counts = torch.maximum(torch.randint(max(1, K - 6), K + 1, (1, H, N), generator=g),
                           local.sum(-1)[None, None])
    return score, pooled_v, sel, counts, local


def _operator(g, S):
    mats = {}

    def op(pair, exponent):
        if pair not in mats:
            mats[pair] = torch.randn(S, S, generator=g) * 0.1
        return torch.eye(S) + exponent * mats[pair]
    return op


@pytest.mark.parametrize("ci", range(N_CASES))
def test_refine_sweep_matches_oracle(dev, ci):
    from cast_amd.router import FCPASMSwapRouter, FCPASMSwapRoutingConfig
    c = _draw(4000 + ci)
    print(f"router case {ci}: hw {c['hw']} cells {c['cells']} mem {c['mem']} H{c['H']} "
          f"D{c['D']} K{c['K']} anchors {c['anchors']} rounds {c['rounds']} mult {c['mult']} "
          f"groups {c['groups']} lambdas {c['lam']} same_bank {c['same_bank']} op {c['op']}",
          flush=True)
    score, pv, sel, cnt, local = _inputs(c)
    S = c["hw"][0] * c["hw"][1]
    op = _operator(c["g"], S) if c["op"] else None
    transport = None
    if op is not None:
        pairs = {(lft, rgt): {"theta": torch.zeros(1, 1, 1), "mean_affinity": 0.9}
                 for lft, rgt in zip(c["anchors"], c["anchors"][1:])}
        transport = {"pairs": pairs, "attention_spatial_h": c["hw"][0],
                     "attention_spatial_w": c["hw"][1]}
    cfg = FCPASMSwapRoutingConfig(num_swap_rounds=c["rounds"], candidate_multiplier=c["mult"],
                                  sketch_groups=c["groups"], lambda_anchor=c["lam"][0],
                                  lambda_reconstruction=c["lam"][1],
                                  same_bank_only=c["same_bank"], swap_eps=1e-6)
    kw = dict(memory_blocks=c["mem"], spatial_shape=c["hw"], exact_current_frames=c["anchors"],
              temporal_group_size=4, current_boundary=4 * c["cells"], layer_index=22)
    want, rec_w = orc.fc_pasm_refine(score, pv, sel, cnt, local, transport=transport, config=cfg,
                                     operator=op, **kw)
    router = FCPASMSwapRouter(cfg, operator=(lambda t, p, shape, e: op(p, e)) if op else None)
    got, rec = router.refine(score=score.to(dev), pooled_value=pv.to(dev), selected=sel.to(dev),
                             counts=cnt.to(dev), local=local.to(dev), transport=transport, **kw)
    torch.cuda.synchronize()
    assert rec["status"] == rec_w["status"], (rec, rec_w)
    assert torch.equal(got.cpu(), want)
    if rec_w["status"] == "refined":
        assert rec["swap_count"] == rec_w["swap_count"]
        assert rec["historical_budget_after"] == rec_w["historical_budget_after"]
        for key in ("objective_before", "objective_after"):
            assert abs(float(rec[key]) - rec_w[key]) <= 1e-4 * abs(rec_w[key]) + 1e-9, key

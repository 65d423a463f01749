"""FC-PASM swap router on the device against the oracle's restatement of
FCPASMLocalCoordinateSwapRouter.refine (P/fc_pasm_swap_routing.py:616-1077).

Cases: a Matrix-like compact layer (6 x 5 spatial tiles, 4 current cells of
30 blocks after 63 memory blocks, D 128, 16 sketch groups) with a route from
the pooled scores' top-k, anchors 0 and 6 (five skipped frames over two
cells), the identity operator and a random FC operator; same-bank on and off.
"""
import pytest
import torch

from oracle import rcsa_oracle as orc

pytestmark = pytest.mark.gpu

HW, CELLS, MEM, D = (6, 5), 4, 63, 128


def _case(seed, H=2, K=24):
    g = torch.Generator().manual_seed(seed)
    S = HW[0] * HW[1]
    N = MEM + CELLS * S
    qh = torch.nn.functional.normalize(torch.randn(1, H, N, D, generator=g), dim=-1)
    kh = torch.nn.functional.normalize(torch.randn(1, H, N, D, generator=g) + qh * 0.3, dim=-1)
    score = qh @ kh.transpose(-1, -2)
    pooled_v = torch.randn(1, H, N, D, generator=g) * 0.5
    local = orc.local_stencil(N, HW[0], HW[1])
    rank = score + local[None, None] * 1e6
    sel = torch.sort(rank, dim=-1, descending=True, stable=True).indices[..., :K]
    counts = torch.randint(K - 6, K + 1, (1, H, N), generator=g)
    return score, pooled_v, sel, counts, local


def _cfg(**kw):
    from cast_amd.router import FCPASMSwapRoutingConfig
    return FCPASMSwapRoutingConfig(**kw)


def _random_operator(seed, S):
    g = torch.Generator().manual_seed(seed)
    mats = {}

    def op(pair, exponent):
        if pair not in mats:
            mats[pair] = torch.randn(S, S, generator=g) * 0.1
        return torch.eye(S) + exponent * mats[pair]
    return op


def test_route_proxy_matches_oracle(dev):
    from cast_amd import ops
    score, pv, sel, cnt, local = _case(1)
    L = min(score.shape[-1], 2 * int(cnt.max()))
    print(f"route proxy N {score.shape[-1]} L {L}", flush=True)
    cand, proxy, err = ops.route_proxy(score.to(dev), pv.to(dev), local.to(dev), sel.to(dev),
                                       cnt.to(dev), memory_blocks=MEM, n_cand=L, cand_mult=2,
                                       sketch_groups=16)
    torch.cuda.synchronize()
    ranking = score + local[None, None] * 1e6
    want_cand = torch.sort(ranking, dim=-1, descending=True, stable=True).indices[..., :L]
    assert torch.equal(cand.cpu().long(), want_cand[0, :, MEM:])
    want_proxy = orc.omission_proxy(torch.softmax(score, -1), pv, want_cand, sketch_groups=16)
    torch.testing.assert_close(proxy.cpu(), want_proxy[0, :, MEM:], atol=2e-6, rtol=1e-4)
    limit = torch.clamp(cnt * 2, max=score.shape[-1])
    keep = torch.zeros_like(want_cand, dtype=torch.bool)
    for h in range(score.shape[1]):
        for r in range(score.shape[2]):
            kept = set(sel[0, h, r, :cnt[0, h, r]].tolist())
            for li in range(int(limit[0, h, r])):
                keep[0, h, r, li] = int(want_cand[0, h, r, li]) not in kept
    want_err = (want_proxy * keep[..., None]).sum(-2)
    torch.testing.assert_close(err.cpu(), want_err[0, :, MEM:], atol=1e-5, rtol=1e-4)


@pytest.mark.parametrize("same_bank", [True, False])
@pytest.mark.parametrize("op_seed", [None, 3])
@pytest.mark.parametrize("seed", [2, 5])
def test_refine_matches_oracle(dev, seed, op_seed, same_bank):
    from cast_amd.router import FCPASMSwapRouter
    score, pv, sel, cnt, local = _case(seed)
    S = HW[0] * HW[1]
    op = _random_operator(op_seed, S) if op_seed is not None else None
    transport = None
    if op is not None:
        transport = {"pairs": {(0, 6): {"theta": torch.zeros(1, 1, 1), "mean_affinity": 0.9}},
                     "attention_spatial_h": HW[0], "attention_spatial_w": HW[1]}
    cfg = _cfg(same_bank_only=same_bank, num_swap_rounds=2, swap_eps=1e-6)
    kw = dict(memory_blocks=MEM, spatial_shape=HW, exact_current_frames=(0, 6),
              temporal_group_size=4, current_boundary=8, layer_index=22)
    want, rec_w = orc.fc_pasm_refine(score, pv, sel, cnt, local, transport=transport, config=cfg,
                                     operator=op, **kw)
    router = FCPASMSwapRouter(cfg, operator=(lambda t, p, shape, e: op(p, e)) if op else None)
    print(f"refine seed {seed} operator {op_seed} same_bank {same_bank}", flush=True)
    got, rec = router.refine(score=score.to(dev), pooled_value=pv.to(dev), selected=sel.to(dev),
                             counts=cnt.to(dev), local=local.to(dev), transport=transport, **kw)
    torch.cuda.synchronize()
    assert rec["status"] == "refined" and rec_w["status"] == "refined"
    assert rec["swap_count"] == rec_w["swap_count"] >= 1
    assert torch.equal(got.cpu(), want)
    assert abs(float(rec["objective_before"]) - rec_w["objective_before"]) <= \
        1e-4 * abs(rec_w["objective_before"])
    assert abs(float(rec["objective_after"]) - rec_w["objective_after"]) <= \
        1e-4 * abs(rec_w["objective_after"])
    assert rec["historical_budget_after"] == rec_w["historical_budget_after"]
    assert rec["fc_cache_used"] == (op is not None)


def test_cast_configuration_is_identity_without_transport(dev):
    """The configuration CAST ships (P/../cast_matrix.py:92-104): the route is
    returned unchanged when the previous layer published no FC transport."""
    from cast_amd.router import FCPASMSwapRouter
    score, pv, sel, cnt, local = _case(7)
    cfg = _cfg(candidate_multiplier=2, num_swap_rounds=1, swap_eps=0.10, sketch_groups=16,
               require_fc_transport=True, min_transport_affinity=0.5, max_swaps_per_call=1,
               active_layers=(22, 26), same_bank_only=True)
    router = FCPASMSwapRouter(cfg)
    kw = dict(score=score.to(dev), pooled_value=pv.to(dev), selected=sel.to(dev),
              counts=cnt.to(dev), local=local.to(dev), memory_blocks=MEM, spatial_shape=HW,
              exact_current_frames=(0, 6), temporal_group_size=4, current_boundary=8)
    for layer, transport, reason in (
            (22, None, "missing_previous_layer_fc_transport"),
            (26, {"pairs": {(0, 6): {"theta": torch.zeros(1, 1, 1), "mean_affinity": 0.3}}},
             "weak_previous_layer_fc_transport"),
            (5, None, "layer_not_enabled")):
        out, rec = router.refine(transport=transport, layer_index=layer, **kw)
        assert torch.equal(out, kw["selected"]) and rec["fallback_reason"] == reason
    s = router.summary()
    assert len(s["records"]) == 3 and s["config"]["active_layers"] == [22, 26]
    router.reset()
    assert router.summary()["records"] == []


def test_refine_with_published_transport(dev):
    """A strong published transport (per-window phases and affinities, the
    corrector's window geometry): the router's default operator against the
    oracle's window-loop transport, two rounds."""
    import math
    from cast_amd.router import FCPASMSwapRouter
    score, pv, sel, cnt, local = _case(9)
    g = torch.Generator().manual_seed(9)
    theta = (torch.rand(18, 6, 3, generator=g) * 2 - 1) * math.pi
    gain = torch.rand(18, 6, 3, generator=g)
    geo = {"output_shape": (22, 40), "transport_shape": (6, 5), "window_shape": (11, 10),
           "stride": (8, 8), "padding": (4, 5), "tile_grid": (3, 6),
           "attention_spatial_h": HW[0], "attention_spatial_w": HW[1]}
    host_tr = dict(geo, pairs={(0, 6): {"theta": theta, "affinity": gain,
                                        "mean_affinity": torch.tensor(0.9)}})
    dev_tr = dict(geo, pairs={(0, 6): {"theta": theta.to(dev), "affinity": gain.to(dev),
                                       "mean_affinity": torch.tensor(0.9)}})
    S = HW[0] * HW[1]
    eye = torch.eye(S).reshape(S, 1, *HW)

    def oracle_op(pair, exponent):
        d = orc.transport_maps(host_tr, pair, eye, exponent).reshape(S, S)
        return (torch.eye(S) + d).T
    cfg = _cfg(num_swap_rounds=2, require_fc_transport=True, min_transport_affinity=0.5)
    kw = dict(memory_blocks=MEM, spatial_shape=HW, exact_current_frames=(0, 6),
              temporal_group_size=4, current_boundary=8, layer_index=22)
    want, rec_w = orc.fc_pasm_refine(score, pv, sel, cnt, local, transport=host_tr, config=cfg,
                                     operator=oracle_op, **kw)
    print("refine with published transport", flush=True)
    got, rec = FCPASMSwapRouter(cfg).refine(score=score.to(dev), pooled_value=pv.to(dev),
                                            selected=sel.to(dev), counts=cnt.to(dev),
                                            local=local.to(dev), transport=dev_tr, **kw)
    torch.cuda.synchronize()
    assert rec["status"] == "refined" and rec["fc_cache_used"] and not rec["g0_fallback"]
    assert rec["swap_count"] == rec_w["swap_count"] >= 1
    assert torch.equal(got.cpu(), want)
    assert abs(float(rec["objective_after"]) - rec_w["objective_after"]) <= \
        1e-4 * abs(rec_w["objective_after"])


def test_refine_refuses_invalid_routes(dev):
    """The device router raises the reference's errors on routes that fail its
    final checks (P/fc_pasm_swap_routing.py:980-1033), as the oracle does: a row
    that drops its local stencil, a row that lists a key twice."""
    from cast_amd.router import FCPASMSwapRouter
    score, pv, sel, cnt, local = _case(2)
    cfg = _cfg(num_swap_rounds=1)
    kw = dict(memory_blocks=MEM, spatial_shape=HW, exact_current_frames=(0, 6),
              temporal_group_size=4, current_boundary=8, layer_index=22, transport=None)
    dropped = cnt.clone()
    dropped[0, 1, MEM + 4] = 0                 # a current row keeps nothing
    twice = sel.clone()
    twice[0, 0, 3, 1] = twice[0, 0, 3, 0]      # a memory row lists its first key twice
    router = FCPASMSwapRouter(cfg)
    for s, c, msg in ((sel, dropped, "removed a protected local edge"),
                      (twice, cnt, "duplicate keys")):
        print(f"refine refuses: {msg}", flush=True)
        with pytest.raises(RuntimeError, match=msg):
            orc.fc_pasm_refine(score, pv, s, c, local, config=cfg, **kw)
        with pytest.raises(RuntimeError, match=msg):
            router.refine(score=score.to(dev), pooled_value=pv.to(dev), selected=s.to(dev),
                          counts=c.to(dev), local=local.to(dev), **kw)
        torch.cuda.synchronize()

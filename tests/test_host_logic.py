"""Host-side product logic against the pinned oracle (CPU only): the packed
block layout, the local stencil, the budget arithmetic and the selector's
argument checks."""
import random

import pytest
import torch

from cast_amd import budget, layout
from cast_amd.selector import BlockSelector
from oracle import rcsa_oracle as orc


@pytest.mark.parametrize("frames,mem_t,H,W,shape", [
    ([0, 1, 2, 3], 0, 8, 8, (2, 4, 4)),
    ([0, 2, 5, 6, 7], 3, 6, 10, (2, 4, 4)),
    ([1, 4], 2, 4, 4, (4, 2, 2)),
    (list(range(8)), 4, 22, 40, (4, 4, 8)),   # Matrix latent grid: 64-token bottom tiles
])
def test_compact_layout_matches_oracle(frames, mem_t, H, W, shape):
    lay = layout.compact_layout(frames, mem_t, H, W, shape)
    idx, valid, t2p = orc.compact_layout(frames, mem_t, H, W, shape)
    assert torch.equal(lay.block_indices, idx)
    assert torch.equal(lay.block_valid, valid)
    assert torch.equal(lay.token_to_packed, t2p)
    assert lay.n_blocks == idx.shape[0] and lay.block_size == idx.shape[1]
    assert torch.equal(lay.slot_token[lay.token_to_packed], torch.arange(t2p.numel()))


@pytest.mark.parametrize("T,mem,qf,prot", [
    (3, 1, [2], True), (12, 4, [5, 6, 9], True), (19, 5, list(range(5, 19)), True),
    (10, 3, [0, 4, 8], False)])
def test_relay_layout_matches_oracle(T, mem, qf, prot):
    H, W, shape = (2, 3, (2, 1, 2)) if T == 3 else (22, 40, (4, 4, 8))
    lay = layout.relay_layout(T, mem, H, W, shape, qf, protected_current=prot,
                              allow_memory_queries=True)
    ref = orc.relay_layout(T, mem, H, W, shape, qf, protected_current=prot)
    bs = lay.block_size
    assert torch.equal(lay.key_slot_token.long(), ref["key"].reshape(-1))
    assert torch.equal(lay.query_slot_token.long(), ref["query"].reshape(-1))
    assert torch.equal(lay.query_block_ids, ref["query_block_ids"])
    assert torch.equal(lay.query_indices, ref["query_indices"])
    assert torch.equal(lay.key_valid, ref["key"].reshape(-1) >= 0)
    # the output row of a query slot is its token's position among the query tokens
    live = lay.query_slot_token >= 0
    assert torch.equal(lay.query_indices[lay.query_out_row[live].long()],
                       lay.query_slot_token[live].long())
    assert bool((lay.query_out_row[~live] == -1).all())
    # validity bits: bit i of word w of block n = slot n * bs + 32 w + i
    if bs % 32 == 0:
        words = lay.key_block_mask.reshape(-1).long() & 0xFFFFFFFF
        bits = (words[:, None] >> torch.arange(32)) & 1
        assert torch.equal(bits.reshape(-1).bool(), lay.key_valid)


def test_relay_layout_rejects_memory_queries():
    with pytest.raises(RuntimeError, match="may not write Memory"):
        layout.relay_layout(12, 4, 22, 40, (4, 4, 8), [2, 5])
    with pytest.raises(ValueError):
        layout.relay_layout(12, 4, 22, 40, (4, 4, 8), [12])


def test_compact_layout_rejects_bad_input():
    with pytest.raises(ValueError):
        layout.compact_layout([], 0, 4, 4, (1, 2, 2))
    with pytest.raises(ValueError):
        layout.compact_layout([0], 0, 4, 4, (1, 2))


@pytest.mark.parametrize("n,nh,nw", [(24, 2, 4), (60, 6, 5), (7, 1, 7)])
def test_local_stencil_matches_oracle(n, nh, nw):
    assert torch.equal(layout.local_stencil(n, nh, nw), orc.local_stencil(n, nh, nw))


def test_apportion_matches_exact_arithmetic():
    rnd = random.Random(1)
    for _ in range(300):
        n = rnd.randint(1, 40)
        w = [rnd.random() * rnd.choice([1, 10, 1000]) for _ in range(n)]
        total = rnd.randint(1, 400)
        got = budget.apportion(torch.tensor(w), total).tolist()
        # the oracle works in exact rationals on the fp32-rounded weights
        w32 = torch.tensor(w, dtype=torch.float32).tolist()
        want = orc.apportion(w32, total)
        if got != want:
            # only a sub-ulp tie between fractional parts may differ
            raw = torch.tensor(w32) * total / sum(w32)
            fr = sorted((raw - raw.floor()).tolist(), reverse=True)
            assert any(abs(a - b) < 1e-5 for a, b in zip(fr, fr[1:]))
        assert sum(got) == total


def test_apportion_reference_errors_and_cases():
    assert budget.apportion(torch.tensor([1.0, 1.0, 1.0]), 10).tolist() == [4, 3, 3]
    assert budget.apportion(torch.tensor([0.0, 0.0]), 3).tolist() == [2, 1]
    with pytest.raises(ValueError):
        budget.apportion(torch.tensor([]), 3)
    with pytest.raises(ValueError):
        budget.apportion(torch.tensor([1.0]), 0)
    m = torch.tensor([[1.0, 2.0, 3.0], [0.0, 0.0, 0.0], [5.0, 1.0, 1.0]])
    got = budget.apportion_section_matrix(m, 8).tolist()
    assert got == orc.apportion_section_matrix(m.tolist(), 8)
    assert all(sum(r) == 8 for r in got)


def test_budgets_and_saturation():
    assert [budget.budget_blocks(f, 275) for f in (0.125, 0.25, 0.5)] == [34, 69, 138]
    local = orc.local_stencil(24, 2, 4)
    assert budget.mean_degree(local, 0.1, 24) == int(local.sum(1).max())
    assert budget.mean_degree(local, 0.5, 24) == 12
    d = budget.saturate(torch.tensor([30, 2, 2, 30]), 10, 40)
    assert d.tolist() == [10, 10, 10, 10]
    d = budget.saturate(torch.tensor([12, 1, 1]), 10, 14)
    assert d.tolist() == [10, 2, 2] and int(d.sum()) == 14  # one each, lowest index first
    motion = torch.rand(24, generator=torch.Generator().manual_seed(0))
    rows = budget.motion_row_degrees(motion, 16, local)
    assert int(rows.sum()) == 24 * 16 and int(rows.min()) >= int(local.sum(1).max())
    w = 1.0 + motion / (motion.mean() + torch.finfo(torch.float32).eps)
    assert rows.tolist() == budget.apportion(w, 24 * 16).tolist()
    with pytest.raises(RuntimeError):
        budget.motion_row_degrees(motion, 3, local)   # cannot hold the local stencil


def test_selector_argument_checks():
    sel = BlockSelector((4, 4, 8), degree=16, num_blocks=60)
    q = torch.zeros(1, 2, 8 * 22 * 40, 64)
    counts = torch.full((1, 2, 60), 16, dtype=torch.int32)
    kw = dict(geometry_indices=None, geometry_counts=counts, latent_hw=(22, 40),
              block_shape=(4, 4, 8))
    with pytest.raises(RuntimeError, match="not compiled"):
        sel.select(q, q, **kw)
    rows = sel.compile_budgets(token_h=22, token_w=40)
    assert rows.tolist() == [16] * 60
    with pytest.raises(ValueError):
        sel.select(q, q[:, :, :-1], **kw)
    with pytest.raises(RuntimeError, match="block shape"):
        sel.select(q, q, **{**kw, "block_shape": (2, 4, 8)})
    with pytest.raises(RuntimeError, match="too small"):
        sel.compile_budgets(token_h=22, token_w=40, row_degrees=torch.full((60,), 3))


def test_router_config_checks():
    """The reference's configuration errors (P/fc_pasm_swap_routing.py:39-61)."""
    from cast_amd.router import FCPASMSwapRoutingConfig as C
    bad = [dict(candidate_multiplier=0), dict(num_swap_rounds=3), dict(swap_eps=-1.0),
           dict(swap_eps=float("inf")), dict(lambda_anchor=-1.0),
           dict(lambda_anchor=0.0, lambda_reconstruction=0.0), dict(sketch_groups=3),
           dict(min_transport_affinity=1.5), dict(min_pair_transport_affinity=-0.1),
           dict(max_swaps_per_call=-1), dict(active_layers=(-1,)),
           dict(historical_only=True, same_bank_only=True)]
    for kw in bad:
        with pytest.raises(ValueError):
            C(**kw)
    C(candidate_multiplier=2, num_swap_rounds=1, swap_eps=0.10, require_fc_transport=True,
      min_transport_affinity=0.5, max_swaps_per_call=1, active_layers=(22, 26),
      same_bank_only=True)


def test_router_fallbacks_on_the_host():
    """Every identity case is decided before any device work, with the
    reference's fallback reasons, and matches the oracle's restatement."""
    from cast_amd.router import FCPASMSwapRouter, FCPASMSwapRoutingConfig as C
    g = torch.Generator().manual_seed(0)
    N, K = 18, 5
    score = torch.randn(1, 2, N, N, generator=g)
    pv = torch.randn(1, 2, N, 32, generator=g)
    sel = torch.sort(score, dim=-1, descending=True).indices[..., :K]
    cnt = torch.full((1, 2, N), K)
    local = torch.eye(N, dtype=torch.bool)
    kw = dict(memory_blocks=6, spatial_shape=(2, 3), exact_current_frames=(0, 6),
              temporal_group_size=4, current_boundary=8, layer_index=22)
    cast = C(require_fc_transport=True, min_transport_affinity=0.5, max_swaps_per_call=1,
             active_layers=(22, 26), same_bank_only=True, swap_eps=0.1)
    weak = {"pairs": {(0, 6): {"theta": torch.zeros(1, 1, 1), "mean_affinity": torch.tensor(0.2)}}}
    cases = [(cast, None, kw), (cast, weak, kw), (cast, None, dict(kw, layer_index=3)),
             (C(), None, dict(kw, exact_current_frames=(2,))),
             (C(), None, dict(kw, exact_current_frames=(2, 3))),
             (C(num_swap_rounds=0), None, kw), (C(), None, dict(kw, memory_blocks=5)),
             (C(min_pair_transport_affinity=0.9), weak, kw)]
    router = FCPASMSwapRouter(cast)
    for cfg, transport, k in cases:
        router.config = cfg
        out, rec = router.refine(score=score, pooled_value=pv, selected=sel, counts=cnt,
                                 local=local, transport=transport, **k)
        _, want = orc.fc_pasm_refine(score, pv, sel, cnt, local, transport=transport,
                                     config=cfg, **k)
        assert torch.equal(out, sel) and rec["status"] == "independent_topk_fallback"
        assert rec["fallback_reason"] == want["fallback_reason"], (rec, want)
    assert len(router.summary()["records"]) == len(cases)
    with pytest.raises(ValueError, match="chronological"):
        router.config = C()
        router.refine(score=score, pooled_value=pv, selected=sel, counts=cnt, local=local,
                      transport=None, **dict(kw, exact_current_frames=(6, 0)))


def test_transport_operator_matches_oracle():
    """The router's [S, S] operator (unit maps through unfold/fold) against the
    oracle's window loops, on random maps; cached per exponent; None without
    a usable entry."""
    import math
    from cast_amd.transport import fc_transport_operator, transport_maps
    g = torch.Generator().manual_seed(4)
    theta = (torch.rand(18, 6, 3, generator=g) * 2 - 1) * math.pi
    tr = {"output_shape": (22, 40), "transport_shape": (6, 5), "window_shape": (11, 10),
          "stride": (8, 8), "padding": (4, 5), "tile_grid": (3, 6),
          "pairs": {(0, 6): {"theta": theta, "affinity": torch.rand(18, 6, 3, generator=g),
                             "mean_affinity": torch.tensor(0.8)}}}
    maps = torch.randn(4, 1, 6, 5, generator=g)
    for a in (0.25, -0.6):
        op = fc_transport_operator(tr, (0, 6), (6, 5), a)
        want = maps + orc.transport_maps(tr, (0, 6), maps, a)
        got = (op @ maps.reshape(4, 30).T).T.reshape(4, 1, 6, 5)
        torch.testing.assert_close(got, want, atol=2e-5, rtol=1e-4)
        assert fc_transport_operator(tr, (0, 6), (6, 5), a) is op
    multi = torch.randn(2, 3, 6, 5, generator=g)
    torch.testing.assert_close(transport_maps(tr, (0, 6), multi, 0.4),
                               orc.transport_maps(tr, (0, 6), multi, 0.4), atol=2e-5, rtol=1e-4)
    assert torch.equal(fc_transport_operator(tr, (0, 6), (6, 5), 0.0), torch.eye(30))
    assert fc_transport_operator(tr, (1, 6), (6, 5), 0.5) is None
    assert fc_transport_operator(None, (0, 6), (6, 5), 0.5) is None


def test_valid_bits_layout():
    """Key validity flags as the attention's block_mask words: bit i of word w
    of block n is key n * block_size + 32 w + i (a pure-Python loop)."""
    from cast_amd.ops import valid_bits
    g = torch.Generator().manual_seed(3)
    for bs in (64, 128):
        valid = torch.rand(5 * bs, generator=g) > 0.3
        got = valid_bits(valid, bs)
        assert got.shape == (5, bs // 32) and got.dtype == torch.int32
        for n in range(5):
            for w in range(bs // 32):
                word = 0
                for i in range(32):
                    word |= int(valid[n * bs + 32 * w + i]) << i
                assert (int(got[n, w]) & 0xffffffff) == word
    with pytest.raises(ValueError):
        valid_bits(torch.ones(100, dtype=torch.bool), 64)

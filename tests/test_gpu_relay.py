"""The causal frame-relay layer's attention core (GPU).

A relay layer keeps the full-world K/V in the CWCA blocks and attends only
from the query frames' tokens (P/matrix_curvature_phase_frame_weave.py:
8734-8846 builds that asymmetric layout, :8966-8995 packs, attends and
scatters).  ``relay_attention`` reads everything through the layout's slot
maps; these tests compare it, bit for bit, with the packed kernels on
explicitly packed inputs, and, within the attention tolerance, with the
oracle's gather -> sparse attention -> scatter over the oracle's own layout.
Grid: 22 x 40 tokens per frame, (4, 4, 8) blocks with 64-token bottom tiles,
12 frames (4 memory), query frames that fill only part of their cells.
"""
import pytest
import torch

from oracle import rcsa_oracle as orc

pytestmark = pytest.mark.gpu

HW, SHAPE, T, MEM, H, D = (22, 40), (4, 4, 8), 12, 4, 4, 128


def _check_attn(ref, got, what):
    st = orc.equivalence_stats(torch.as_tensor(ref).float(), torch.as_tensor(got).float())
    assert st["cosine"] >= 0.999 and st["max_abs"] <= 3e-2, f"{what}: {st}"


def _case(seed, query_frames, dev):
    from cast_amd import layout
    g = torch.Generator().manual_seed(seed)
    S = T * HW[0] * HW[1]
    q = (torch.randn(1, S, H, D, generator=g) / D ** 0.5).bfloat16()
    k = torch.randn(1, S, H, D, generator=g) / D ** 0.5
    k[..., 9] *= 10.0  # an outlier channel
    k = k.bfloat16()
    v = (torch.randn(1, S, H, D, generator=g) / D ** 0.5).bfloat16()
    lay = layout.relay_layout(T, MEM, *HW, SHAPE, query_frames, device=dev,
                              allow_memory_queries=min(query_frames) < MEM)
    nb = lay.n_blocks
    max_k = 24
    # a selection of every CWCA block: the block itself, then random others
    sel = torch.full((1, H, nb, max_k), -1, dtype=torch.int32)
    cnt = torch.randint(6, max_k + 1, (1, H, nb), generator=g, dtype=torch.int32)
    for h in range(H):
        for b in range(nb):
            others = torch.randperm(nb, generator=g)
            row = [b] + [int(x) for x in others if int(x) != b][:max_k - 1]
            n = int(cnt[0, h, b])
            sel[0, h, b, :n] = torch.tensor(sorted(row[:n]), dtype=torch.int32)
    return lay, q, k, v, sel, cnt


def _packed_reference(lay, q, k, v, sel, cnt, int8):
    """Explicit packed copies, the packed kernels, and the scatter to query rows."""
    from cast_amd import ops
    rows = lay.query_block_ids
    idx = sel.index_select(2, rows).contiguous()
    c = cnt.index_select(2, rows).contiguous()
    qp = ops.pack_tokens(q, lay.query_slot_token)
    kp = ops.pack_tokens(k, lay.key_slot_token)
    vp = ops.pack_tokens(v, lay.key_slot_token)
    if int8:
        _, q_i8, qs, _, ksum, kmin, kmax, mask = ops.pool_query_key(
            qp, lay.query_valid, kp, lay.key_valid, 128)
        k_i8, ks, _ = ops.quantize_key(kp, lay.key_valid, 128, ksum, kmin, kmax)
        out, lse = ops.sparse_attn_int8(q_i8, qs, k_i8, ks, vp, idx, c, None, block_mask=mask,
                                        return_lse=True)
    else:
        out, lse = ops.sparse_attn_bf16(qp, kp, vp, idx, c, None, block_mask=lay.key_block_mask,
                                        return_lse=True)
    live = lay.query_out_row >= 0
    slots = torch.nonzero(live).flatten()
    n = lay.query_indices.numel()
    order = torch.empty(n, dtype=torch.long, device=q.device)
    order[lay.query_out_row[slots].long()] = slots
    return out[0].transpose(0, 1)[order][None], lse[:, :, order]


@pytest.mark.parametrize("int8", [True, False])
@pytest.mark.parametrize("query_frames", [[5, 6, 9], [4, 5, 6, 7, 8, 9, 10, 11], [2, 7]])
def test_relay_attention_matches_packed(int8, query_frames):
    from cast_amd.pipeline import relay_attention
    dev = torch.device("cuda:0")
    lay, q, k, v, sel, cnt = _case(3, query_frames, dev)
    q, k, v, sel, cnt = (x.to(dev) for x in (q, k, v, sel, cnt))
    print(f"relay int8 {int8} query frames {query_frames} query blocks "
          f"{lay.query_block_ids.numel()} of {lay.n_blocks}", flush=True)
    out, lse = relay_attention(q, k, v, lay, sel, cnt, int8=int8, return_lse=True)
    want, want_lse = _packed_reference(lay, q, k, v, sel, cnt, int8)
    torch.cuda.synchronize()
    assert out.shape == (1, lay.query_indices.numel(), H, D)
    assert torch.equal(out, want) and torch.equal(lse, want_lse)


@pytest.mark.parametrize("int8", [True, False])
def test_relay_attention_vs_oracle(int8):
    """Against the oracle's own layout (a pure-Python restatement of the
    reference's builder), zero-filled gathers, fp32 attention and scatter."""
    from cast_amd.pipeline import relay_attention
    dev = torch.device("cuda:0")
    qf = [5, 6, 9]
    lay, q, k, v, sel, cnt = _case(4, qf, dev)
    out = relay_attention(q.to(dev), k.to(dev), v.to(dev), lay, sel.to(dev), cnt.to(dev),
                          int8=int8)
    torch.cuda.synchronize()
    ref = orc.relay_layout(T, MEM, *HW, SHAPE, qf)
    kidx, qidx = ref["key"], ref["query"]

    def gather(x, idx):
        flat = idx.reshape(-1)
        g_ = x[:, flat.clamp_min(0)].transpose(1, 2).float()
        return g_ * (flat >= 0)[None, None, :, None]

    qp, kp, vp = gather(q, qidx), gather(k, kidx), gather(v, kidx)
    rows = ref["query_block_ids"]
    o, _ = orc.sparse_attention(qp, kp, vp, sel[:, :, rows], cnt[:, :, rows],
                                kidx.reshape(-1) >= 0, block_m=128, block_n=128)
    # scatter the packed query rows to their tokens, keep the query frames
    full = torch.zeros(1, q.shape[1], H, D)
    live = qidx.reshape(-1) >= 0
    full[:, qidx.reshape(-1)[live]] = o.transpose(1, 2)[:, live]
    want = full[:, ref["query_indices"]]
    got = out.float().cpu()
    for h in range(H):
        _check_attn(want[0, :, h], got[0, :, h], f"relay int8 {int8} head {h}")

"""Seeded synthetic RCSA workloads at the Matrix-Game DiT attention shapes.

Every generator builds its tensors on the CPU from a seeded
``torch.Generator`` (so a CPU check and the GPU see identical bits) and
returns a :class:`Workload` that ``.to(device)`` moves to HBM.

Layout: the packed block layout is the identity on the token order of each
segment (history frames, then the current chunk), each segment padded with
invalid slots to a whole number of blocks.  A frame is 880 tokens (22 x 40
latent grid); a block is 128 tokens.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field, replace
from typing import Optional

import torch

FRAME_TOKENS = 880  # 22 x 40 latent tokens per frame


def budget_blocks(fraction: float, n_history_blocks: int) -> int:
    """Per-row history budget k = int(round(fraction * blocks)), Python
    round-half-even as P/matrix_curvature_phase_frame_weave.py:5729."""
    return int(round(fraction * n_history_blocks))


@dataclass
class Workload:
    name: str
    q: torch.Tensor            # [B, H, NQB*BS, D] packed, zero in invalid slots
    k: torch.Tensor            # [B, H, NKB*BS, D]
    v: torch.Tensor
    q_valid: torch.Tensor      # bool [NQB*BS]
    k_valid: torch.Tensor      # bool [NKB*BS]
    block_size: int
    n_hist_blocks: int         # key blocks [0, n_hist_blocks) are history
    k_hist: int                # history blocks kept per query block
    forced: torch.Tensor       # bool [NQB, NKB]: current chunk + anchor blocks
    int8: bool = False
    meta: dict = field(default_factory=dict)

    @property
    def n_qblocks(self) -> int:
        return self.q.shape[2] // self.block_size

    @property
    def n_kblocks(self) -> int:
        return self.k.shape[2] // self.block_size

    @property
    def k_total(self) -> int:
        """Blocks per row handed to the selector: history budget + current chunk."""
        return self.k_hist + (self.n_kblocks - self.n_hist_blocks)

    def to(self, device) -> "Workload":
        return replace(self, q=self.q.to(device), k=self.k.to(device), v=self.v.to(device),
                       q_valid=self.q_valid.to(device), k_valid=self.k_valid.to(device),
                       forced=self.forced.to(device))

    def attention_ops(self, indices: torch.Tensor, counts: torch.Tensor) -> float:
        """Algorithmic ops of the sparse attention: sum over heads and valid
        query rows of 2*D*(valid selected keys), once for QK^T and once for PV."""
        D = self.q.shape[3]
        bs = self.block_size
        kv_blocks = self.k_valid.reshape(-1, bs).sum(-1).to(torch.float64).cpu()
        q_rows = self.q_valid.reshape(-1, bs).sum(-1).to(torch.float64).cpu()
        idx = indices.reshape(-1, self.n_qblocks, indices.shape[-1]).cpu().long()
        cnt = counts.reshape(-1, self.n_qblocks).cpu().long()
        slot = torch.arange(idx.shape[-1])[None, None, :] < cnt[..., None]
        keys = torch.where(slot, kv_blocks[idx.clamp_min(0)], torch.zeros(()))
        keys_per_row = keys.sum(-1)                     # [BH, NQB]
        return float((keys_per_row * q_rows[None, :]).sum() * 2 * D * 2)


def _segments(lengths: list[int], bs: int) -> tuple[torch.Tensor, list[int]]:
    """Valid mask of segments padded to blocks; returns (valid, block counts)."""
    masks, nblocks = [], []
    for n in lengths:
        nb = -(-n // bs)
        m = torch.zeros(nb * bs, dtype=torch.bool)
        m[:n] = True
        masks.append(m)
        nblocks.append(nb)
    return torch.cat(masks), nblocks


def _scatter_segments(tokens: torch.Tensor, lengths: list[int], bs: int) -> torch.Tensor:
    """[B, H, sum(lengths), D] -> packed [B, H, sum(padded), D] with zero padding."""
    parts, start = [], 0
    B, H, _, D = tokens.shape
    for n in lengths:
        nb = -(-n // bs)
        buf = torch.zeros(B, H, nb * bs, D, dtype=tokens.dtype)
        buf[:, :, :n] = tokens[:, :, start:start + n]
        parts.append(buf)
        start += n
    return torch.cat(parts, dim=2)


def _frame_shifted(g, B, H, n_tokens, D, frame_tokens, shift_std, noise_std):
    n_frames = -(-n_tokens // frame_tokens)
    x = torch.randn(B, H, n_tokens, D, generator=g) * noise_std
    shift = torch.randn(B, H, n_frames, D, generator=g) * shift_std
    frame_of = torch.arange(n_tokens) // frame_tokens
    return x + shift[:, :, frame_of]


def matrix_dit(seed: int = 0, *, heads: int = 24, head_dim: int = 128,
               query_frames: int = 4, history_frames: int = 40, fraction: float = 0.25,
               int8: bool = False, outlier_channels: int = 4, dtype=torch.bfloat16,
               current_kv_frames: Optional[int] = None) -> Workload:
    """bf16 block-sparse attention at the Matrix-like DiT shape.

    Q/K/V ~ N(0,1)/sqrt(D) plus an N(0, 0.3^2) per-frame, per-channel mean
    shift (independent for Q, K and V).  With ``int8`` the K channels at
    ``outlier_channels`` seeded positions are scaled x10.  Current-chunk KV is
    always kept (forced); the history budget is round(fraction * history blocks).
    """
    g = torch.Generator().manual_seed(seed)
    bs = 128
    B, H, D = 1, heads, head_dim
    lq = query_frames * FRAME_TOKENS
    lh = history_frames * FRAME_TOKENS
    cur_frames = query_frames if current_kv_frames is None else current_kv_frames
    lc = cur_frames * FRAME_TOKENS
    noise = 1.0 / math.sqrt(D)
    q_tok = _frame_shifted(g, B, H, lq, D, FRAME_TOKENS, 0.3, noise)
    k_tok = _frame_shifted(g, B, H, lh + lc, D, FRAME_TOKENS, 0.3, noise)
    v_tok = _frame_shifted(g, B, H, lh + lc, D, FRAME_TOKENS, 0.3, noise)
    outliers = None
    if int8 and outlier_channels:
        outliers = torch.randperm(D, generator=g)[:outlier_channels].sort().values
        k_tok[..., outliers] *= 10.0
    q_valid, (nqb,) = _segments([lq], bs)
    k_valid, (nhb, ncb) = _segments([lh, lc], bs)
    q = _scatter_segments(q_tok, [lq], bs).to(dtype)
    k = _scatter_segments(k_tok, [lh, lc], bs).to(dtype)
    v = _scatter_segments(v_tok, [lh, lc], bs).to(dtype)
    forced = torch.zeros(nqb, nhb + ncb, dtype=torch.bool)
    forced[:, nhb:] = True
    name = f"matrix_dit_q{lq}_hist{lh}_{'int8' if int8 else 'bf16'}_f{fraction}"
    return Workload(name, q, k, v, q_valid, k_valid, bs, nhb, budget_blocks(fraction, nhb),
                    forced, int8, {"seed": seed, "outlier_channels": outliers,
                                   "fraction": fraction, "query_frames": query_frames,
                                   "history_frames": history_frames})


def plumbing(seed: int = 0) -> Workload:
    """CPU plumbing case, fp32: B=1, H=4, D=64, 64-token blocks.

    Q = 256 tokens (4 blocks); K/V = 8 history blocks + 4 current blocks.
    Q/K/V ~ N(0,1) with an extra N(0, 0.5^2) per-block mean offset; top-4
    history blocks, current kept.
    """
    g = torch.Generator().manual_seed(seed)
    B, H, D, bs = 1, 4, 64, 64
    nq, nh, nc = 4, 8, 4

    def blocks(nb):
        x = torch.randn(B, H, nb, bs, D, generator=g)
        off = torch.randn(B, H, nb, 1, D, generator=g) * 0.5
        return (x + off).reshape(B, H, nb * bs, D)

    q = blocks(nq)
    k = blocks(nh + nc)
    v = blocks(nh + nc)
    forced = torch.zeros(nq, nh + nc, dtype=torch.bool)
    forced[:, nh:] = True
    return Workload("plumbing_h4_d64_bs64", q, k, v, torch.ones(nq * bs, dtype=torch.bool),
                    torch.ones((nh + nc) * bs, dtype=torch.bool), bs, nh, 4, forced, False,
                    {"seed": seed})


def selection_stress(seed: int = 0, *, heads: int = 24, head_dim: int = 128,
                     query_frames: int = 4, history_frames: int = 120, budget: int = 64,
                     n_forced: int = 8, tied_fraction: float = 0.10, tie_sigma: float = 1e-3,
                     dtype=torch.bfloat16) -> Workload:
    """Selection stress case: long history, fixed budget with forced anchors, near ties.

    * each query block gets an anchor interval of ``n_forced`` consecutive
      history blocks at a seeded uniform offset (forced, counted in the budget);
    * history K block means are A*u_h + rho*e_j (e_j unit, orthogonal to a
      per-head direction u_h) with exactly zero-mean token noise;
    * in ``tied_fraction`` of the (head, query block) rows the query block
      mean is alpha*u_h + eta*w (w unit, orthogonal to u_h), which makes that
      row's history scores near-tied with spread ``tie_sigma``;
    * the current chunk and V follow the DiT-shape generator.
    """
    g = torch.Generator().manual_seed(seed)
    bs = 128
    B, H, D = 1, heads, head_dim
    lq = query_frames * FRAME_TOKENS
    lh = history_frames * FRAME_TOKENS
    lc = lq
    noise = 1.0 / math.sqrt(D)
    q_valid, (nqb,) = _segments([lq], bs)
    k_valid, (nhb, ncb) = _segments([lh, lc], bs)
    assert lh % bs == 0, "history must be whole blocks"

    def unit(x):
        return x / x.norm(dim=-1, keepdim=True)

    def ortho(x, u):  # remove the u component (u unit) and renormalise
        return unit(x - (x * u).sum(-1, keepdim=True) * u)

    A = rho = 2.4
    u = unit(torch.randn(B, H, 1, D, generator=g))
    e = ortho(torch.randn(B, H, nhb, D, generator=g), u)
    hist_mean = A * u + rho * e                                   # [B,H,nhb,D]
    z = torch.randn(B, H, nhb, bs, D, generator=g) * noise
    z = z - z.mean(dim=3, keepdim=True)
    k_hist = (hist_mean[:, :, :, None, :] + z).reshape(B, H, lh, D)
    k_cur = _frame_shifted(g, B, H, lc, D, FRAME_TOKENS, 0.3, noise)
    v_tok = _frame_shifted(g, B, H, lh + lc, D, FRAME_TOKENS, 0.3, noise)

    q_tok = _frame_shifted(g, B, H, lq, D, FRAME_TOKENS, 0.3, noise)
    q = _scatter_segments(q_tok, [lq], bs)                        # fp32 packed
    n_rows = H * nqb
    n_tied = int(round(tied_fraction * n_rows))
    tied_rows = torch.randperm(n_rows, generator=g)[:n_tied].sort().values
    alpha = 3.4
    qv = q_valid.reshape(nqb, bs)
    for r in tied_rows.tolist():
        h, m = divmod(r, nqb)
        w = ortho(torch.randn(D, generator=g), u[0, h, 0])
        # spread of (eta*rho*<w, e_j>) / (|q||mu|) with <w, e_j> ~ 1/sqrt(D-1)
        eta = tie_sigma * math.sqrt(D - 1) * alpha * math.hypot(A, rho) / rho
        mean = alpha * u[0, h, 0] + eta * w
        zz = torch.randn(bs, D, generator=g) * noise
        nv = int(qv[m].sum())
        zz[:nv] -= zz[:nv].mean(dim=0, keepdim=True)
        zz[nv:] = 0
        blk = zz + mean
        blk[nv:] = 0
        q[0, h, m * bs:(m + 1) * bs] = blk
    k = _scatter_segments(torch.cat([k_hist, k_cur], dim=2), [lh, lc], bs)
    v = _scatter_segments(v_tok, [lh, lc], bs)
    forced = torch.zeros(nqb, nhb + ncb, dtype=torch.bool)
    forced[:, nhb:] = True
    starts = torch.randint(0, nhb - n_forced + 1, (nqb,), generator=g)
    for m in range(nqb):
        forced[m, int(starts[m]):int(starts[m]) + n_forced] = True
    return Workload(f"selection_stress_hist{lh}_k{budget}_forced{n_forced}",
                    q.to(dtype), k.to(dtype), v.to(dtype), q_valid, k_valid, bs, nhb,
                    budget, forced, False,
                    {"seed": seed, "tied_rows": tied_rows, "anchor_starts": starts,
                     "tie_sigma": tie_sigma})


def step_sweep_plan(seed: int = 0, layers: int = 30) -> list[dict]:
    """Per-layer plan of a denoising step: anchor query frames in {1..4} and a
    history budget fraction in {12.5, 25, 50}%, drawn from the seed."""
    g = torch.Generator().manual_seed(seed)
    frames = torch.randint(1, 5, (layers,), generator=g)
    fracs = torch.tensor([0.125, 0.25, 0.5])[torch.randint(0, 3, (layers,), generator=g)]
    return [{"layer": i, "query_frames": int(frames[i]), "fraction": float(fracs[i])}
            for i in range(layers)]


def step_layer_view(base: Workload, plan: dict) -> Workload:
    """Derive one sweep layer from a 4-frame DiT workload without regenerating:
    queries = the first ``query_frames`` frames, current KV = the same frames,
    history unchanged, budget = round(fraction * history blocks).  Works on
    whatever device ``base`` lives on."""
    bs = base.block_size
    nf = int(plan["query_frames"])
    lq = nf * FRAME_TOKENS
    nqb = -(-lq // bs)
    nhb = base.n_hist_blocks
    lh = nhb * bs
    dev = base.q.device
    q = base.q[:, :, : nqb * bs].clone()
    q[:, :, lq:] = 0
    cur = base.k.shape[2] - lh
    take = min(nqb * bs, cur)
    k = torch.zeros(*base.k.shape[:2], lh + nqb * bs, base.k.shape[3], dtype=base.k.dtype,
                    device=dev)
    v = torch.zeros_like(k)
    k[:, :, : lh + take] = base.k[:, :, : lh + take]
    v[:, :, : lh + take] = base.v[:, :, : lh + take]
    k[:, :, lh + lq:] = 0
    v[:, :, lh + lq:] = 0
    q_valid = torch.zeros(nqb * bs, dtype=torch.bool, device=dev)
    q_valid[:lq] = True
    k_valid = torch.zeros(lh + nqb * bs, dtype=torch.bool, device=dev)
    k_valid[: lh] = base.k_valid[: lh]
    k_valid[lh: lh + lq] = True
    forced = torch.zeros(nqb, nhb + nqb, dtype=torch.bool, device=dev)
    forced[:, nhb:] = True
    return Workload(f"step_layer{plan['layer']}_f{nf}_b{plan['fraction']}", q, k, v, q_valid,
                    k_valid, bs, nhb, budget_blocks(plan["fraction"], nhb), forced, True,
                    dict(plan))


def step_layer(plan: dict, seed: int = 0, *, heads: int = 24, head_dim: int = 128,
               history_frames: int = 40) -> Workload:
    """One layer of the per-step sweep: only the anchor frames' queries, current
    KV = the same anchor frames (compact semantics of
    P/matrix_curvature_phase_frame_weave.py:5671-5684), int8 Q/K, bf16 V."""
    return matrix_dit(seed * 1000 + plan["layer"], heads=heads, head_dim=head_dim,
                      query_frames=plan["query_frames"], history_frames=history_frames,
                      fraction=plan["fraction"], int8=True)

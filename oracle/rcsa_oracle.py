"""CPU oracle for the RCSA hot path -- TEST INFRASTRUCTURE ONLY.

This module is the checker.  Only ``tests/``, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py`` may import it; the product path in
``cast_amd`` never does.  It restates, in plain PyTorch eager on the CPU
(fp32, fp64 where noted), what the CAST reference computes on this path.
Paths are relative to the CAST repository, P/ =
src/interaction_accel/methods/proposed/.

How each function is pinned (beyond being a restatement) is listed in its
docstring; the pins live in tests/test_oracle_pins.py:
  pool_blocks         fp64 brute-force loops; constant-block and zero-block closed forms
  block_scores        fp64 loops; Cauchy-Schwarz bound |s| <= 1; s(x, x) = 1
  local_stencil       pure-Python Manhattan loop
  select_topk         brute-force Python sort with tuple keys; forced/allowed invariants
  topk_margin         brute-force sort
  quantize_*          dequantisation error <= scale / 2; range [-127, 127]; idempotence
  sparse_attention    fp64 per-row loops; single-key => v; equal logits => mean(v);
                      per-row shift invariance of softmax
  compact_layout      reference's loop branch restated with pure-Python lists
  relay_layout        hand-enumerated small grid (block ids from coordinates,
                      partial-cell query frames); every key token in exactly
                      one slot, query rows = the key rows' query-frame members
  apportion*          exact rational arithmetic (fractions.Fraction) + conserved sums
  saturate            closed forms: the result sums to min(target, n * cap), never
                      exceeds cap, and only rows below cap before a pass gain
  compact_time_cells  hand-computed cells (profiled / unprofiled frames, partial
                      last cell); out-of-tile frames raise
  redistribute_compact_capacity
                      closed forms: worldline sums reach the target, no row
                      above capacity, raises exactly when capacity runs out
  closed_loop_degrees conserved edge budgets (every worldline Tc * mean, the
                      whole layer blocks * mean); uniform curvature gives
                      uniform degrees; a pure-Python Fraction re-derivation
                      on small cases; equal to the reference's own
                      compact_closed_loop_degrees on fixtures it wrote (all
                      three feedback forms with a response, bootstrap, weight
                      0, fixed budget, prefix frames, partial cells, a row
                      over capacity: tests/golden/ref_closed_loop.npz)
  omission_proxy      fp64 loops over rows, candidates and sketch groups
  route_objective_terms / route_objective_value
                      the quadratic terms reproduce the brute-force change of
                      the objective value for every single-row change (with the
                      identity operator and with random operators); equal to the
                      reference's _objective_value / _objective_terms with no
                      transport and with a published one
                      (tests/golden/ref_router.npz)
  transport_maps      exponent 0 and theta 0 give no change; the windows are cut
                      and overlap-added with explicit index loops (a different
                      formulation from the product's unfold/fold); equal to the
                      reference's _apply_transport_maps and _transport_matrix
                      on pooled and unpooled transport grids, exponents of both
                      signs (tests/golden/ref_router.npz)
  quantize_rows_int8  error <= scale / 2, the absmax element maps to +-127, zero rows
  int8_linear         pure-Python integer dot products on small shapes; exact
                      int32 accumulation bound; scales factor out
  compact_cwca_layer  a composition of the functions above (each pinned on its
                      own); the weights of the pooled V are the pooled-K
                      weights (pool_blocks' sums over valid slots)
  fc_pasm_refine      the identity (with the reference's fallback reasons) for
                      every missing-transport / disabled case; the chosen swap
                      equals a brute-force search over every admissible
                      single swap of the objective value; the same routes,
                      swap counts and objectives as the reference's refine
                      with a published transport (same bank on and off, one
                      and two rounds: tests/golden/ref_router.npz)
"""
from __future__ import annotations

import math
from typing import Optional, Sequence

import torch
import torch.nn.functional as F

__all__ = [
    "pool_blocks", "block_scores", "local_stencil", "select_topk", "topk_margin",
    "quantize_query_blocks", "key_mean", "quantize_key_blocks", "dequantize_blocks",
    "sparse_attention", "sparse_attention_int8", "equivalence_stats", "compact_layout",
    "apportion", "apportion_section_matrix", "saturate", "budget_blocks", "rcsa_layer",
    "apportion_section_matrix_f32", "compact_time_cells", "redistribute_compact_capacity",
    "closed_loop_degrees", "relay_layout", "omission_proxy", "route_objective_terms",
    "route_objective_value", "fc_pasm_refine", "transport_maps", "quantize_rows_int8",
    "int8_linear", "compact_cwca_layer",
]


# --------------------------------------------------------------------------
# a2 / a3: pooling and cosine scores

def pool_blocks(x: torch.Tensor, valid: Optional[torch.Tensor], block_size: int):
    """Masked mean over each block's valid tokens, then F.normalize.

    Restates P/matrix_curvature_phase_frame_weave.py:5685-5700
    (weights = valid, denominator = weights.sum().clamp_min(1)).
    x: [B, H, NB*BS, D]; valid: [NB*BS] bool/uint8 or None.
    Returns (hat [B, H, NB, D] fp32, block sums [B, H, NB, D] fp32, n_valid [NB]).
    """
    B, H, L, D = x.shape
    nb = L // block_size
    xb = x.reshape(B, H, nb, block_size, D).float()
    if valid is None:
        w = torch.ones(nb, block_size)
    else:
        w = valid.reshape(nb, block_size).float()
    weights = w[None, None, :, :, None]
    sums = (xb * weights).sum(dim=3)
    denom = weights.sum(dim=3).clamp_min(1.0)
    hat = F.normalize(sums / denom, dim=-1)
    return hat, sums, w.sum(dim=1)


def block_scores(qhat: torch.Tensor, khat: torch.Tensor) -> torch.Tensor:
    """score = q_content @ k_content^T (P/matrix_curvature_phase_frame_weave.py:5701)."""
    return torch.matmul(qhat, khat.transpose(-2, -1))


def local_stencil(n_blocks: int, nh: int, nw: int) -> torch.Tensor:
    """Manhattan <= 1 neighbourhood in (t, h, w) block coordinates.

    Restates P/matrix_curvature_phase_frame_weave.py:5718-5725 and
    P/qk_uncertainty_tangent_attention.py:1025-1039 (block id = t*nh*nw + h*nw + w).
    """
    spatial = nh * nw
    ids = torch.arange(n_blocks)
    bt, rem = ids // spatial, ids % spatial
    bh, bw = rem // nw, rem % nw
    return ((bt[:, None] - bt[None, :]).abs() + (bh[:, None] - bh[None, :]).abs()
            + (bw[:, None] - bw[None, :]).abs()) <= 1


# --------------------------------------------------------------------------
# a4 / a6: forced set and top-k

def _broadcast_mask(mask, nbh, nq, nk, default):
    if mask is None:
        return torch.full((nbh, nq, nk), default, dtype=torch.bool)
    m = mask.bool()
    if m.shape == (nq, nk):
        m = m[None].expand(nbh, nq, nk)
    return m


def _row_k(k, nbh, nq):
    if isinstance(k, int):
        return torch.full((nbh, nq), k, dtype=torch.int64)
    kt = torch.as_tensor(k).to(torch.int64)
    if kt.shape == (nq,):
        kt = kt[None].expand(nbh, nq)
    return kt


def select_topk(score: torch.Tensor, k, *, forced=None, allowed=None,
                max_k: Optional[int] = None, order: str = "index"):
    """Top-k per (bh, query block) under the total order
    (allowed, forced, score desc, index asc).

    Restates ``torch.topk(score + 1e6 * local, k)`` at
    P/matrix_curvature_phase_frame_weave.py:5829-5831 with forced blocks as a
    mask instead of +1e6 (fp32 has a 0.0625 ulp at 1e6), and the stable
    descending argsort of P/qk_uncertainty_tangent_attention.py:978-980 for
    ties (lower index first).  Disallowed columns (the -inf topology mask of
    P/qk_uncertainty_tangent_attention.py:820) are never selected.
    score: [NBH, NQ, NK].  Returns (indices int32 [NBH, NQ, max_k] padded
    with -1, counts int32 [NBH, NQ]).
    """
    nbh, nq, nk = score.shape
    fm = _broadcast_mask(forced, nbh, nq, nk, False)
    am = _broadcast_mask(allowed, nbh, nq, nk, True)
    kk = _row_k(k, nbh, nq)
    if max_k is None:
        max_k = max(1, min(int(kk.max()), nk))
    kk = kk.clamp(0, max_k)
    s = score.float().clone()
    s[s == 0] = 0.0  # -0 == +0
    s = torch.where(torch.isnan(s), torch.full_like(s, float("inf")), s)
    # stable sorts from the least significant key to the most significant
    idx = torch.arange(nk).expand(nbh, nq, nk)
    order1 = torch.sort(s, dim=-1, descending=True, stable=True).indices
    f1 = torch.gather(fm, -1, order1)
    order2 = torch.gather(order1, -1, torch.sort(f1.to(torch.int8), dim=-1,
                                                 descending=True, stable=True).indices)
    a2 = torch.gather(am, -1, order2)
    order3 = torch.gather(order2, -1, torch.sort(a2.to(torch.int8), dim=-1,
                                                 descending=True, stable=True).indices)
    n_allowed = am.sum(-1)
    counts = torch.minimum(kk, n_allowed).to(torch.int32)
    out = torch.full((nbh, nq, max_k), -1, dtype=torch.int32)
    for r in range(nbh):
        for i in range(nq):
            c = int(counts[r, i])
            sel = order3[r, i, :c]
            if order == "index":
                sel = torch.sort(sel).values
            out[r, i, :c] = sel.to(torch.int32)
    del idx
    return out, counts


def topk_margin(score: torch.Tensor, k, *, forced=None, allowed=None) -> torch.Tensor:
    """Score gap between the last selected and the first rejected column.

    inf when the boundary separates a forced from a non-forced column or when
    every allowed column is selected.  [NBH, NQ] fp32.
    """
    nbh, nq, nk = score.shape
    fm = _broadcast_mask(forced, nbh, nq, nk, False)
    am = _broadcast_mask(allowed, nbh, nq, nk, True)
    kk = _row_k(k, nbh, nq)
    out = torch.full((nbh, nq), float("inf"))
    for r in range(nbh):
        for i in range(nq):
            cols = [(bool(fm[r, i, j]), float(score[r, i, j]), j)
                    for j in range(nk) if am[r, i, j]]
            cols.sort(key=lambda t: (not t[0], -t[1], t[2]))
            c = min(int(kk[r, i]), len(cols))
            if 0 < c < len(cols) and cols[c - 1][0] == cols[c][0]:
                out[r, i] = cols[c - 1][1] - cols[c][1]
    return out


# --------------------------------------------------------------------------
# a10: int8 Q/K quantiser (no reference counterpart)

def quantize_query_blocks(q: torch.Tensor, valid, block_size: int):
    """Per (head, block) symmetric int8: scale = absmax/127, q8 = rne(q * (127/absmax)).

    Returns (q_i8 [B,H,L,D] int8, scale [B*H, NB] fp32).  Invalid tokens -> 0.
    """
    B, H, L, D = q.shape
    nb = L // block_size
    x = q.float().reshape(B, H, nb, block_size, D)
    w = (torch.ones(nb, block_size, dtype=torch.bool) if valid is None
         else valid.reshape(nb, block_size).bool())
    wm = w[None, None, :, :, None]
    amax = torch.where(wm, x.abs(), torch.zeros_like(x)).amax(dim=(3, 4))
    live = amax > 0
    scale = torch.where(live, amax / 127.0, torch.ones_like(amax))
    inv = torch.where(live, torch.tensor(127.0) / amax, torch.ones_like(amax))
    q8 = torch.round(x * inv[..., None, None]).clamp(-127, 127)
    q8 = torch.where(wm, q8, torch.zeros_like(q8)).to(torch.int8)
    return q8.reshape(B, H, L, D), scale.reshape(B * H, nb)


def key_mean(k: torch.Tensor, valid) -> torch.Tensor:
    """Per-head, per-channel mean over all valid key tokens (fp64 accumulate). [B*H, D]."""
    B, H, L, D = k.shape
    w = torch.ones(L, dtype=torch.bool) if valid is None else valid.reshape(L).bool()
    x = k.double() * w[None, None, :, None]
    return (x.sum(dim=2) / max(int(w.sum()), 1)).float().reshape(B * H, D)


def quantize_key_blocks(k: torch.Tensor, valid, block_size: int, kmean: torch.Tensor):
    """Mean-smoothed per-block symmetric int8 keys given the per-head mean.

    scale = max |k - m| / 127 over the block's valid tokens; k8 = rne((k - m) * (127/amax)).
    Returns (k_i8 [B,H,L,D], scale [B*H, NB]).
    """
    B, H, L, D = k.shape
    nb = L // block_size
    m = kmean.reshape(B, H, 1, 1, D).float()
    x = k.float().reshape(B, H, nb, block_size, D) - m
    w = (torch.ones(nb, block_size, dtype=torch.bool) if valid is None
         else valid.reshape(nb, block_size).bool())
    wm = w[None, None, :, :, None]
    amax = torch.where(wm, x.abs(), torch.zeros_like(x)).amax(dim=(3, 4))
    live = (amax > 0) & w.any(dim=1)[None, None]
    scale = torch.where(live, amax / 127.0, torch.ones_like(amax))
    inv = torch.where(live, torch.tensor(127.0) / amax, torch.ones_like(amax))
    k8 = torch.round(x * inv[..., None, None]).clamp(-127, 127)
    k8 = torch.where(wm, k8, torch.zeros_like(k8)).to(torch.int8)
    return k8.reshape(B, H, L, D), scale.reshape(B * H, nb)


def dequantize_blocks(x_i8: torch.Tensor, scale: torch.Tensor, block_size: int):
    """x_i8 * scale broadcast per block -> fp32 [B, H, L, D]."""
    B, H, L, D = x_i8.shape
    nb = L // block_size
    s = scale.reshape(B, H, nb, 1, 1)
    return (x_i8.float().reshape(B, H, nb, block_size, D) * s).reshape(B, H, L, D)


# --------------------------------------------------------------------------
# a8: block-sparse attention

def sparse_attention(q, k, v, indices, counts, kvalid=None, *, block_m: int, block_n: int,
                     sm_scale: Optional[float] = None, dtype=torch.float32,
                     heads: Optional[Sequence[int]] = None,
                     qblocks: Optional[Sequence[int]] = None):
    """Explicit softmax over the allowed key tokens of each query block.

    Restates the reference's own oracle at
    P/matrix_jit_spatial_acceleration.py:836-858 (logits = q.k / sqrt(D),
    softmax over the listed blocks' valid keys, weights @ v) for every query
    row, which is the contract of _attn_fwd_bsa_align as launched at :663-729.
    Rows with no admissible key get 0 output and lse = -inf.
    q: [B,H,Lq,D], k/v: [B,H,Lk,D], indices [B|1,H|1,NQB,maxK], counts [B|1,H|1,NQB].
    Optional ``heads``/``qblocks`` restrict the work (other rows left 0).
    Returns (out [B,H,Lq,D] dtype, lse [B,H,Lq] dtype).
    """
    B, H, Lq, D = q.shape
    Lk = k.shape[2]
    scale = 1.0 / math.sqrt(D) if sm_scale is None else sm_scale
    nqb = -(-Lq // block_m)
    nkb = -(-Lk // block_n)
    indices = indices.expand(B, H, -1, -1)
    counts = counts.expand(B, H, -1)
    kv = (torch.ones(Lk, dtype=torch.bool) if kvalid is None
          else kvalid.reshape(-1).bool())
    out = torch.zeros(B, H, Lq, D, dtype=dtype)
    lse = torch.full((B, H, Lq), float("-inf"), dtype=dtype)
    hs = range(H) if heads is None else heads
    qbs = range(nqb) if qblocks is None else qblocks
    maxk = indices.shape[-1]
    for b in range(B):
        for h in hs:
            for m in qbs:
                c = max(0, min(int(counts[b, h, m]), maxk))
                blocks = [int(n) for n in indices[b, h, m, :c] if 0 <= int(n) < nkb]
                toks = [t for n in blocks for t in range(n * block_n, min((n + 1) * block_n, Lk))]
                toks = torch.tensor(toks, dtype=torch.long)
                if toks.numel():
                    toks = toks[kv[toks]]
                r0, r1 = m * block_m, min((m + 1) * block_m, Lq)
                if toks.numel() == 0:
                    continue
                qq = q[b, h, r0:r1].to(dtype)
                kk = k[b, h, toks].to(dtype)
                vv = v[b, h, toks].to(dtype)
                logits = (qq @ kk.T) * scale
                out[b, h, r0:r1] = torch.softmax(logits, dim=-1) @ vv
                lse[b, h, r0:r1] = torch.logsumexp(logits, dim=-1)
    return out, lse


def sparse_attention_int8(q_i8, q_scale, k_i8, k_scale, v, indices, counts, kvalid=None, *,
                          block_m: int, block_n: int, sm_scale: Optional[float] = None,
                          heads=None, qblocks=None):
    """fp32 attention over the dequantised int8 Q/K (what the int8 kernel computes
    before its bf16 rounding of P), same contract as :func:`sparse_attention`."""
    q = dequantize_blocks(q_i8, q_scale, block_m)
    k = dequantize_blocks(k_i8, k_scale, block_n)
    return sparse_attention(q, k, v.float(), indices, counts, kvalid, block_m=block_m,
                            block_n=block_n, sm_scale=sm_scale, heads=heads, qblocks=qblocks)


def equivalence_stats(reference: torch.Tensor, candidate: torch.Tensor) -> dict:
    """relative_l2 / cosine / mae / max_abs, as P/matrix_jit_spatial_acceleration.py:880-897."""
    r = reference.detach().float()
    c = candidate.detach().float()
    d = c - r
    return {
        "relative_l2": float(torch.linalg.vector_norm(d) / (torch.linalg.vector_norm(r) + 1e-12)),
        "cosine": float(F.cosine_similarity(r.reshape(-1), c.reshape(-1), dim=0)),
        "mae": float(d.abs().mean()),
        "max_abs": float(d.abs().max()),
    }


# --------------------------------------------------------------------------
# a1: compact packed-block layout

def compact_layout(active_frames: Sequence[int], memory_temporal: int, height: int,
                   width: int, block_shape: tuple[int, int, int]):
    """Packed 128-slot block map of the compact active frames.

    Restates P/matrix_curvature_phase_frame_weave.py:5223-5301 through its
    per-block loop branch (:5290-5293): block members are the compact tokens
    with that block id, in increasing token order.
    Returns (block_indices [NB, BS] int64 with -1 padding, valid [NB, BS] bool,
    token_to_packed [T*H*W] int64).
    """
    tt, th, tw = block_shape
    frames = sorted(int(f) for f in active_frames)
    compact_t = len(frames)
    spatial = height * width
    nh, nw = -(-height // th), -(-width // tw)
    compact_memory = sum(1 for f in frames if f < memory_temporal)
    if compact_memory:
        memory_cells = -(-compact_memory // tt)
        n_blocks = (memory_cells + -(-(compact_t - compact_memory) // tt)) * nh * nw
    else:
        memory_cells = 0
        n_blocks = -(-compact_t // tt) * nh * nw
    block_size = tt * th * tw
    members: list[list[int]] = [[] for _ in range(n_blocks)]
    for tok in range(compact_t * spatial):
        lt, ls = tok // spatial, tok % spatial
        lh, lw = ls // width, ls % width
        if compact_memory:
            cell = lt // tt if lt < compact_memory else memory_cells + (lt - compact_memory) // tt
        else:
            cell = lt // tt
        members[cell * nh * nw + (lh // th) * nw + lw // tw].append(tok)
    idx = torch.full((n_blocks, block_size), -1, dtype=torch.long)
    t2p = torch.empty(compact_t * spatial, dtype=torch.long)
    for b, mem in enumerate(members):
        if len(mem) > block_size:
            raise RuntimeError("compact frame block exceeds its packed capacity")
        for slot, tok in enumerate(mem):
            idx[b, slot] = tok
            t2p[tok] = b * block_size + slot
    return idx, idx >= 0, t2p


def relay_layout(total_temporal: int, memory_temporal: int, height: int, width: int,
                 block_shape: tuple[int, int, int], query_frames: Sequence[int], *,
                 protected_current: bool = True):
    """Asymmetric frame-relay layout: full-world keys, query-frame queries.

    Restates MatrixCausalFrameLayerRelay._asymmetric_layout
    (P/matrix_curvature_phase_frame_weave.py:8734-8846) with pure-Python
    lists: a token's block id comes from its (frame, row, column); with a
    protected current chunk the memory frames and the current frames fill
    separate temporal cells (:8768-8782).  Key block b holds every token with
    id b in increasing order (:8795-8801); the query blocks are the sorted
    ids of the query-frame tokens and hold only those tokens (:8810-8824).
    Returns dict(key [NB, BS] int64 -1 padded, query_block_ids [NQ] int64,
    query [NQ, BS] int64 -1 padded, query_indices [n] int64).
    """
    tt, th, tw = block_shape
    spatial = height * width
    nh, nw = -(-height // th), -(-width // tw)
    mem = memory_temporal
    if protected_current:
        mem_blocks = -(-mem // tt) * nh * nw if mem else 0
        n_blocks = mem_blocks + -(-(total_temporal - mem) // tt) * nh * nw
    else:
        mem_blocks = 0
        n_blocks = -(-total_temporal // tt) * nh * nw
    qset = {int(f) for f in query_frames}
    block_size = tt * th * tw
    key: list[list[int]] = [[] for _ in range(n_blocks)]
    qmembers: dict[int, list[int]] = {}
    query_indices = []
    for tok in range(total_temporal * spatial):
        t, r = tok // spatial, tok % spatial
        h, w = r // width, r % width
        if protected_current and t >= mem:
            cell, base = (t - mem) // tt, mem_blocks
        else:
            cell, base = t // tt, 0
        b = base + cell * nh * nw + (h // th) * nw + w // tw
        key[b].append(tok)
        if t in qset:
            qmembers.setdefault(b, []).append(tok)
            query_indices.append(tok)
    ids = sorted(qmembers)
    kidx = torch.full((n_blocks, block_size), -1, dtype=torch.long)
    for b, mem_ in enumerate(key):
        if len(mem_) > block_size:
            raise RuntimeError("CWCA block contains too many tokens")
        kidx[b, :len(mem_)] = torch.tensor(mem_, dtype=torch.long)
    qidx = torch.full((len(ids), block_size), -1, dtype=torch.long)
    for r, b in enumerate(ids):
        qidx[r, :len(qmembers[b])] = torch.tensor(qmembers[b], dtype=torch.long)
    return {"key": kidx, "query_block_ids": torch.tensor(ids, dtype=torch.long),
            "query": qidx, "query_indices": torch.tensor(query_indices, dtype=torch.long)}


# --------------------------------------------------------------------------
# a5: budgets

def apportion(weights: Sequence[float], total: int) -> list[int]:
    """Largest-remainder apportionment, ties to the lower index.

    Restates P/qk_uncertainty_tangent_attention.py:847-865 with exact
    rational arithmetic (the reference uses fp32; equal unless a fractional
    part differs by < 1 ulp).
    """
    from fractions import Fraction
    w = [max(Fraction(x), Fraction(0)) for x in weights]
    if sum(w) <= 0:
        w = [Fraction(1)] * len(w)
    tot = sum(w)
    raw = [Fraction(total) * x / tot for x in w]
    res = [math.floor(r) for r in raw]
    rem = total - sum(res)
    order = sorted(range(len(w)), key=lambda i: (-(raw[i] - res[i]), i))
    for i in order[:rem]:
        res[i] += 1
    return res


def apportion_section_matrix(weights: Sequence[Sequence[float]], total_per_section: int):
    """Row-wise largest remainder (P/qk_uncertainty_tangent_attention.py:1239-1264)."""
    return [apportion(row, total_per_section) for row in weights]


def saturate(degrees: Sequence[int], cap: int, target_total: int) -> list[int]:
    """Clamp every row to ``cap``, then give the lost edges one each to the
    lowest-index rows below ``cap``, pass after pass, until ``target_total`` or
    no room is left (P/matrix_curvature_phase_frame_weave.py:5807-5817),
    with Python ints one edge at a time.
    """
    d = [min(int(x), cap) for x in degrees]
    missing = int(target_total) - sum(d)
    while missing > 0:
        gave = 0
        for i in range(len(d)):
            if missing == 0:
                break
            if d[i] < cap:
                d[i] += 1
                missing -= 1
                gave += 1
        if gave == 0:
            break
    return d


def apportion_section_matrix_f32(weights: torch.Tensor, total_per_section: int) -> torch.Tensor:
    """Row-wise largest remainder in fp32 torch arithmetic, as
    P/qk_uncertainty_tangent_attention.py:1239-1264 computes it (clamp_min(0),
    a non-positive row weighs every entry 1, raw = total * w / sum, floor, one
    more edge to the largest fractional parts by a stable descending sort)."""
    normalized = weights.float().clamp_min(0.0)
    normalized = torch.where(normalized.sum(dim=-1, keepdim=True) > 0, normalized,
                             torch.ones_like(normalized))
    raw = float(total_per_section) * normalized / normalized.sum(dim=-1, keepdim=True)
    result = torch.floor(raw).to(torch.long)
    remainder = total_per_section - result.sum(dim=-1)
    fractions = raw - result
    order = torch.argsort(fractions, dim=-1, descending=True, stable=True)
    ranks = torch.empty_like(order)
    ranks.scatter_(-1, order, torch.arange(weights.shape[-1])[None].expand_as(order))
    return result + (ranks < remainder[:, None]).to(result.dtype)


def compact_time_cells(values: torch.Tensor, active_current_local: Sequence[int],
                       compact_group: int, source_group: int, offset: int) -> torch.Tensor:
    """Per-worldline signal of the compact current time cells.

    Restates P/control_response_cwca_attention.py:1123-1163: frame f (current
    local) reads source tile floor((f - offset) / source_group) of ``values``
    [T_src, S] when f >= offset, else 0; each run of ``compact_group`` frames
    is averaged into one cell.  Returns [T_cells, S]."""
    local = torch.as_tensor(list(active_current_local), dtype=torch.long)
    profiled = local >= int(offset)
    cells = torch.div((local - int(offset)).clamp_min(0), int(source_group),
                      rounding_mode="floor")
    if bool(torch.any(profiled & (cells >= int(values.shape[0])))):
        raise RuntimeError("compact Current frame lies outside CWCA tiles")
    selected = torch.zeros(int(local.numel()), int(values.shape[1]), dtype=values.dtype)
    if bool(profiled.any()):
        selected[profiled] = values.index_select(0, cells[profiled])
    rows = [selected[lo:lo + int(compact_group)].mean(dim=0)
            for lo in range(0, int(selected.shape[0]), int(compact_group))]
    if not rows:
        raise RuntimeError("compact Closed-Loop CWCA has no Current cells")
    return torch.stack(rows)


def redistribute_compact_capacity(degrees: torch.Tensor, *, capacity: int,
                                  target_per_worldline: int) -> torch.Tensor:
    """Clamp every cell to ``capacity``, then per worldline (column) give the
    lost edges one each to the lowest cells below capacity, pass after pass;
    raise when a worldline has no room left
    (P/control_response_cwca_attention.py:1165-1186)."""
    degrees = degrees.clamp(max=capacity)
    for s in range(int(degrees.shape[1])):
        missing = target_per_worldline - int(degrees[:, s].sum())
        while missing > 0:
            cand = torch.nonzero(degrees[:, s] < capacity).flatten()
            if not int(cand.numel()):
                raise RuntimeError("compact Closed-Loop CWCA exhausted key capacity")
            take = min(missing, int(cand.numel()))
            degrees[cand[:take], s] += 1
            missing -= take
    return degrees


def closed_loop_degrees(curvature: torch.Tensor, active_current_local: Sequence[int], *,
                        current_temporal_offset: int, source_group: int, compact_group: int,
                        mean_degree: int, base_degree: int, total_blocks: int,
                        memory_blocks: int, response: Optional[torch.Tensor] = None,
                        response_weight: float = 0.0, feedback_form: str = "additive",
                        fixed_query_budget: bool = False, layer_index: int = 1) -> torch.Tensor:
    """Row degrees of a compact woven layer under the closed-loop allocator.

    Restates compact_closed_loop_degrees (P/control_response_cwca_attention.py:
    1188-1363) and how the frame weave composes it
    (P/matrix_curvature_phase_frame_weave.py:5727-5817): memory rows keep
    ``mean_degree``; the current cells get base + the largest-remainder split of
    Tc * (mean - base) edges per spatial worldline by 1 + log1p(signal), where
    the signal is the column-normalised curvature of the compact cells (plus the
    previous layer's response with the closed-loop feedback form); each
    worldline is saturated at ``total_blocks`` and redistributed; then the whole
    layer is clamped and saturated to ``total_blocks * mean_degree``.
    ``curvature`` / ``response``: [T_src, S] fp32.  Returns int64 [total_blocks].
    """
    cur = curvature.float()
    spatial = int(cur.shape[1])
    eps = torch.finfo(cur.dtype).eps
    current_capacity = int(current_temporal_offset) + int(cur.shape[0]) * int(source_group)
    local = [int(f) for f in active_current_local]
    if not local:
        raise RuntimeError("compact Closed-Loop has no active Current frames")
    if any(f < 0 for f in local):
        raise RuntimeError("compact Closed-Loop Current set contains Memory frames")
    if any(f >= current_capacity for f in local):
        raise RuntimeError("compact Current frame lies outside CWCA frame capacity")
    normalized = cur / cur.mean(dim=0, keepdim=True).clamp_min(eps)
    compact = compact_time_cells(normalized, local, compact_group, source_group,
                                 current_temporal_offset)
    cells = int(compact.shape[0])
    if fixed_query_budget:
        current = torch.full((cells, spatial), int(mean_degree), dtype=torch.long)
    else:
        if layer_index == 0 or response_weight == 0.0 or response is None:
            signal = compact
        else:
            resp = compact_time_cells(response.float(), local, compact_group, source_group,
                                      current_temporal_offset)
            if feedback_form == "additive":
                signal = compact + response_weight * resp
            else:
                sign = -1.0 if feedback_form == "centered_inverse" else 1.0
                signal = compact * torch.exp(sign * response_weight * (resp - 1.0))
        weights = 1.0 + torch.log1p(signal)
        residual = cells * (int(mean_degree) - int(base_degree))
        bonus = apportion_section_matrix_f32(weights.transpose(0, 1), residual).transpose(0, 1)
        current = redistribute_compact_capacity(bonus + int(base_degree),
                                                capacity=int(total_blocks),
                                                target_per_worldline=cells * int(mean_degree))
    if int(current.numel()) != int(total_blocks) - int(memory_blocks):
        raise RuntimeError("compact Closed-Loop degree layout differs from packed rows")
    degrees = torch.full((int(total_blocks),), int(mean_degree), dtype=torch.long)
    degrees[int(memory_blocks):] = current.reshape(-1)
    return torch.tensor(saturate(degrees.tolist(), int(total_blocks),
                                 int(total_blocks) * int(mean_degree)), dtype=torch.long)


def budget_blocks(fraction: float, n_history_blocks: int) -> int:
    """k = int(round(fraction * blocks)) (Python round-half-even),
    as P/matrix_curvature_phase_frame_weave.py:5729."""
    return int(round(fraction * n_history_blocks))


# --------------------------------------------------------------------------
# whole layer call

def rcsa_layer(q, k, v, q_valid, k_valid, *, block_size: int, k_select, forced=None,
               allowed=None, int8: bool = False, heads=None, qblocks=None):
    """score -> select -> (quantise) -> sparse attention, all on the CPU.

    Returns dict(score, indices, counts, out, lse[, q_i8, q_scale, k_i8, k_scale, kmean]).
    """
    qhat, _, _ = pool_blocks(q, q_valid, block_size)
    khat, _, _ = pool_blocks(k, k_valid, block_size)
    B, H = q.shape[:2]
    score = block_scores(qhat, khat).reshape(B * H, qhat.shape[2], khat.shape[2])
    idx, cnt = select_topk(score, k_select, forced=forced, allowed=allowed)
    nq = qhat.shape[2]
    idx4 = idx.reshape(B, H, nq, -1)
    cnt3 = cnt.reshape(B, H, nq)
    res = {"score": score, "indices": idx, "counts": cnt}
    if int8:
        q8, qs = quantize_query_blocks(q, q_valid, block_size)
        km = key_mean(k, k_valid)
        k8, ks = quantize_key_blocks(k, k_valid, block_size, km)
        out, lse = sparse_attention_int8(q8, qs, k8, ks, v, idx4, cnt3, k_valid,
                                         block_m=block_size, block_n=block_size,
                                         heads=heads, qblocks=qblocks)
        res.update(q_i8=q8, q_scale=qs, k_i8=k8, k_scale=ks, kmean=km)
    else:
        out, lse = sparse_attention(q, k, v, idx4, cnt3, k_valid, block_m=block_size,
                                    block_n=block_size, heads=heads, qblocks=qblocks)
    res.update(out=out, lse=lse)
    return res


def compact_cwca_layer(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                       block_indices: torch.Tensor, *, block_shape, spatial_hw,
                       active_frame_values, memory_temporal: int, sparse_density: float,
                       closed_loop: dict, router: Optional[dict] = None,
                       layer_index: int = 1):
    """The compact woven layer's attention, composed from the oracle's parts.

    Restates _compact_cwca_attention (P/matrix_curvature_phase_frame_weave.py:
    5643-6124) with a closed-loop geometry provider: the q/k/v[:, flat] gathers
    with invalid slots zeroed (:5677-5684), the masked block means (q and k
    normalised, v not: :5685-5700), the scores (:5701), the local stencil and
    mean degree (:5703-5731), the layer's degrees (closed_loop_degrees, which
    includes the saturation of :5807-5817), the top-k of score + 1e6 local at
    each row's degree (:5829-5832; select_topk), the router's refine with the
    score it is handed back (score + 1e6 local - 1e6 local in fp32, :6037) when
    ``router`` is given, then the sparse attention over the packed blocks and
    the scatter to the token rows (:6086-6095).

    q, k, v: token-major [B, L, H, D]; block_indices: int64 [blocks, block_size]
    (token or -1).  ``closed_loop``: the keywords of closed_loop_degrees other
    than the layout's (curvature, current_temporal_offset, source_group,
    response, response_weight, feedback_form, fixed_query_budget).  ``router``:
    dict(config=..., transport=..., operator=..., current_boundary=...).
    Returns dict(out [B, L, H, D] fp32, degrees int64 [blocks], selected
    [B, H, blocks, max] int64, counts [B, H, blocks], score, vmean, record).
    """
    B, L, H, D = q.shape
    blocks, bs = block_indices.shape
    flat = block_indices.clamp_min(0).reshape(-1)
    mask = (block_indices >= 0).reshape(-1)

    def packed(x):
        xp = x[:, flat].transpose(1, 2).float().clone()
        xp[:, :, ~mask] = 0
        return xp
    qp, kp, vp = packed(q), packed(k), packed(v)
    qhat, _, _ = pool_blocks(qp, mask, bs)
    khat, _, _ = pool_blocks(kp, mask, bs)
    _, vsum, nv = pool_blocks(vp, mask, bs)
    vmean = vsum / nv.clamp_min(1.0)[None, None, :, None]
    score = block_scores(qhat, khat)                                 # [B, H, N, N]
    tt, th, tw = (int(x) for x in block_shape)
    nh, nw = math.ceil(spatial_hw[0] / th), math.ceil(spatial_hw[1] / tw)
    spatial = nh * nw
    frames = [int(f) for f in active_frame_values]
    memory_frames = sum(1 for f in frames if f < memory_temporal)
    local = local_stencil(blocks, nh, nw)
    widest = int(local.sum(dim=-1).max())
    mean_degree = min(max(widest, int(round(sparse_density * blocks))), blocks)
    memory_blocks = min(blocks, math.ceil(memory_frames / tt) * spatial)
    base = max(widest, math.ceil(4 * mean_degree / 5))
    current_local = [f - memory_temporal for f in frames if f >= memory_temporal]
    degrees = closed_loop_degrees(
        closed_loop["curvature"], current_local, compact_group=tt, mean_degree=mean_degree,
        base_degree=base, total_blocks=blocks, memory_blocks=memory_blocks,
        layer_index=layer_index,
        **{kk: vv for kk, vv in closed_loop.items() if kk != "curvature"})
    sel, cnt = select_topk(score.reshape(B * H, blocks, blocks), degrees, forced=local,
                           order="rank")
    selected = sel.reshape(B, H, blocks, -1).long()
    counts = cnt.reshape(B, H, blocks)
    record = None
    if router is not None:
        bonus = local.to(score.dtype) * 1e6
        selected, record = fc_pasm_refine(
            (score + bonus) - bonus, vmean, selected, counts, local,
            memory_blocks=memory_blocks, spatial_shape=(nh, nw),
            exact_current_frames=tuple(current_local), temporal_group_size=tt,
            current_boundary=router.get("current_boundary", 4),
            transport=router.get("transport"), layer_index=layer_index,
            config=router["config"], operator=router.get("operator"))
    out_p, _ = sparse_attention(qp, kp, vp, selected, counts, mask, block_m=bs, block_n=bs)
    token_to_packed = torch.empty(L, dtype=torch.long)
    token_to_packed[block_indices.reshape(-1)[mask]] = torch.nonzero(mask).flatten()
    out = out_p.transpose(1, 2)[:, token_to_packed]
    return {"out": out, "degrees": degrees, "selected": selected, "counts": counts,
            "score": score, "vmean": vmean, "record": record, "mean_degree": mean_degree,
            "memory_blocks": memory_blocks, "base": base}


# --------------------------------------------------------------------------
# a7: FC-PASM swap router

def omission_proxy(probability: torch.Tensor, pooled_value: torch.Tensor,
                   candidates: torch.Tensor, *, sketch_groups: int,
                   eps: float = 1e-6) -> torch.Tensor:
    """Single-block omission proxy of candidate key blocks, sketched over
    ``sketch_groups`` equal groups of the value channels.

    Restates estimate_block_omission_error (P/fc_pasm_swap_routing.py:64-106):
    with o = P v (the pooled attention output of the row) and p_c the
    candidate's probability, proxy[l] = p_c / (1 - p_c + eps) * (o - v_c),
    averaged within each channel group.  probability [B, H, Q, K],
    pooled_value [B, H, K, D], candidates [B, H, Q, L] -> [B, H, Q, L, G].
    """
    if probability.ndim != 4 or pooled_value.ndim != 4 or candidates.ndim != 4:
        raise ValueError("omission proxy expects BHQK, BHKD and BHQL tensors")
    D = pooled_value.shape[-1]
    if D % sketch_groups:
        raise ValueError("value width must be divisible by sketch groups")
    v = pooled_value.float()
    out = torch.matmul(probability.float(), v)                        # [B, H, Q, D]
    B, H, Q, L = candidates.shape
    cand_v = torch.gather(v[:, :, None].expand(B, H, Q, -1, D), 3,
                          candidates[..., None].expand(B, H, Q, L, D))
    p_c = torch.gather(probability.float(), -1, candidates)
    weight = p_c / (1.0 - p_c + eps)
    diff = weight[..., None] * (out[..., None, :] - cand_v)
    return diff.reshape(B, H, Q, L, sketch_groups, D // sketch_groups).mean(-1)


def _route_cells(exact_frames, temporal_group_size, temporal_cells):
    return {int(f): min(int(f) // int(temporal_group_size), temporal_cells - 1)
            for f in exact_frames}


def _route_pairs(exact_frames, current_boundary):
    """(left, right, skipped targets) of consecutive anchors on one side of the boundary."""
    out = []
    for left, right in zip(exact_frames, exact_frames[1:]):
        if (left < current_boundary) != (right < current_boundary):
            continue
        out.append((int(left), int(right), tuple(range(left + 1, right))))
    return out


def _route_operator(operator, pair, exponent, spatial, device):
    """The FC transport operator of ``pair`` at ``exponent`` ([S, S], output x
    input), or the identity when there is none (the g = 0 case of
    P/fc_pasm_swap_routing.py:136-141)."""
    m = operator(pair, exponent) if operator is not None else None
    if m is None:
        return torch.eye(spatial, device=device, dtype=torch.float32), False
    return m.to(device=device, dtype=torch.float32), True


def route_objective_value(error: torch.Tensor, *, temporal_cells: int, spatial: int,
                          exact_frames, temporal_group_size: int, current_boundary: int,
                          operator=None, lambda_anchor: float = 1.0,
                          lambda_reconstruction: float = 1.0) -> torch.Tensor:
    """Anchor + reconstruction omission objective of the current rows.

    Restates _objective_value (P/fc_pasm_swap_routing.py:550-614): the squared
    error of every anchor frame's cell, plus, for every frame skipped between
    two anchors on one side of the current boundary, the squared error
    propagated to it: (1 - a) T^a e_left + a T^-(1-a) e_right, a the frame's
    position between the anchors.  error [B, H, cells * S, G]."""
    view = error.reshape(*error.shape[:2], temporal_cells, spatial, error.shape[-1])
    cell = _route_cells(exact_frames, temporal_group_size, temporal_cells)
    count = error.new_zeros(temporal_cells)
    for f in exact_frames:
        count[cell[int(f)]] += 1.0
    value = lambda_anchor * (view.square() * count[None, None, :, None, None]).sum()
    for left, right, skipped in _route_pairs(exact_frames, current_boundary):
        el, er = view[:, :, cell[left]], view[:, :, cell[right]]
        for target in skipped:
            a = float(target - left) / float(right - left)
            lm, _ = _route_operator(operator, (left, right), a, spatial, error.device)
            rm, _ = _route_operator(operator, (left, right), -(1.0 - a), spatial, error.device)
            prop = (1.0 - a) * torch.einsum("st,bhtg->bhsg", lm, el) + \
                a * torch.einsum("st,bhtg->bhsg", rm, er)
            value = value + lambda_reconstruction * prop.square().sum()
    return value


def route_objective_terms(error: torch.Tensor, *, temporal_cells: int, spatial: int,
                          exact_frames, temporal_group_size: int, current_boundary: int,
                          operator=None, lambda_anchor: float = 1.0,
                          lambda_reconstruction: float = 1.0):
    """Per-row quadratic coefficients of the objective: changing row r's error
    by d changes the objective by sum_g a_r (2 e_rg d_g + d_g^2) + 2 b_rg d_g.

    Restates _objective_terms (P/fc_pasm_swap_routing.py:414-547): a_r = the
    anchor count of the row's cell times lambda_anchor plus the diagonal of
    each reconstruction Hessian; b_r = the Hessians' off-diagonal couplings
    applied to the current errors (within the cell, and across the two
    anchor cells).  Returns (a [1, 1, rows, 1], b [B, H, rows, G], used)."""
    B, H, rows, G = error.shape
    if rows != temporal_cells * spatial:
        raise RuntimeError("routing error rows do not match Current cells")
    view = error.reshape(B, H, temporal_cells, spatial, G)
    cell = _route_cells(exact_frames, temporal_group_size, temporal_cells)
    count = error.new_zeros(temporal_cells)
    for f in exact_frames:
        count[cell[int(f)]] += 1.0
    coef = count[:, None].expand(-1, spatial).clone() * lambda_anchor
    lin = torch.zeros_like(view)
    used = False
    for left, right, skipped in _route_pairs(exact_frames, current_boundary):
        lc, rc = cell[left], cell[right]
        el, er = view[:, :, lc], view[:, :, rc]
        for target in skipped:
            a = float(target - left) / float(right - left)
            lm, f1 = _route_operator(operator, (left, right), a, spatial, error.device)
            rm, f2 = _route_operator(operator, (left, right), -(1.0 - a), spatial, error.device)
            used = used or f1 or f2
            lo, ro = (1.0 - a) * lm, a * rm
            if lc == rc:
                comb = lo + ro
                hess = lambda_reconstruction * (comb.T @ comb)
                dg = torch.diagonal(hess)
                coef[lc] += dg
                lin[:, :, lc] += torch.einsum("st,bhtg->bhsg", hess, el) - dg[None, None, :, None] * el
            else:
                hl = lambda_reconstruction * (lo.T @ lo)
                hr = lambda_reconstruction * (ro.T @ ro)
                hx = lambda_reconstruction * (lo.T @ ro)
                dl, dr = torch.diagonal(hl), torch.diagonal(hr)
                coef[lc] += dl
                coef[rc] += dr
                lin[:, :, lc] += (torch.einsum("st,bhtg->bhsg", hl, el)
                                  - dl[None, None, :, None] * el
                                  + torch.einsum("st,bhtg->bhsg", hx, er))
                lin[:, :, rc] += (torch.einsum("st,bhtg->bhsg", hr, er)
                                  - dr[None, None, :, None] * er
                                  + torch.einsum("st,bhtg->bhsg", hx.T, el))
    return coef.reshape(1, 1, rows, 1), lin.reshape(B, H, rows, G), used


def _route_fallback(layer_index, reason, **extra):
    rec = {"layer_index": int(layer_index), "status": "independent_topk_fallback",
           "fallback_reason": reason, "swap_count": 0, "fixed_budget": True}
    rec.update(extra)
    return rec


def _route_affinity(entry) -> float:
    if not isinstance(entry, dict):
        return 0.0
    a = entry.get("mean_affinity", 0.0)
    return float(a.detach().float().item()) if isinstance(a, torch.Tensor) else float(a)


def fc_pasm_refine(score: torch.Tensor, pooled_value: torch.Tensor, selected: torch.Tensor,
                   counts: torch.Tensor, local: torch.Tensor, *, memory_blocks: int,
                   spatial_shape, exact_current_frames, temporal_group_size: int,
                   current_boundary: int, transport, layer_index: int, config,
                   operator=None):
    """Fixed-budget coordinate-swap refinement of a top-k route.

    Restates FCPASMLocalCoordinateSwapRouter.refine (P/fc_pasm_swap_routing.py:
    616-1077) for the historical_only = False configurations: the fallbacks
    that return the route unchanged (:647-748, 783-819), the 2k candidates of
    the ranking score + 1e6 local (stable descending order: ties to the lower
    index), the omission proxy of each candidate, and up to num_swap_rounds
    rounds that each apply the single best (remove, add) exchange over all
    current rows when it lowers the objective by more than swap_eps
    (:843-977), with the same-bank rule when configured, and the checks on the
    final route that raise (:980-1033: same-bank memory counts, duplicate keys, a
    dropped local-stencil edge, a higher objective).  ``config`` carries the
    FCPASMSwapRoutingConfig fields; ``operator(pair, exponent)`` gives the FC
    transport operator of a pair (None: identity).  Returns (selected, record).
    """
    cfg = config
    score = score.detach().float()
    pooled_value = pooled_value.detach()
    baseline = selected.clone()
    sel = selected.clone().long()
    if cfg.active_layers and layer_index not in cfg.active_layers:
        return baseline, _route_fallback(layer_index, "layer_not_enabled")
    N = score.shape[-1]
    rows_cur = score.shape[-2] - int(memory_blocks)
    S = int(spatial_shape[0] * spatial_shape[1])
    if rows_cur <= 0 or rows_cur % S:
        return baseline, _route_fallback(layer_index, "no_rectangular_current_rows",
                                         fc_cache_used=False)
    cells = rows_cur // S
    frames = tuple(int(f) for f in exact_current_frames)
    if tuple(sorted(set(frames))) != frames:
        raise ValueError("routing Exact Current frames must be unique and chronological")
    pairs = [(l, r) for l, r in zip(frames, frames[1:])
             if r - l > 1 and (l < current_boundary) == (r < current_boundary)]
    if cfg.num_swap_rounds == 0 or len(frames) < 2 or not pairs:
        reason = ("zero_swap_rounds" if cfg.num_swap_rounds == 0 else
                  "fewer_than_two_exact_anchors" if len(frames) < 2 else "no_skipped_frames")
        return baseline, _route_fallback(layer_index, reason, fc_cache_used=False)
    tpairs = transport.get("pairs", {}) if isinstance(transport, dict) else {}
    matching = [tpairs[p] for p in pairs
                if isinstance(tpairs.get(p), dict) and isinstance(tpairs[p].get("theta"), torch.Tensor)]
    affinity = max((_route_affinity(e) for e in matching), default=0.0)
    strong = bool(matching) and affinity >= cfg.min_transport_affinity
    if cfg.require_fc_transport and not strong:
        return baseline, _route_fallback(
            layer_index, "weak_previous_layer_fc_transport" if matching
            else "missing_previous_layer_fc_transport",
            matching_transport_affinity=affinity, fc_cache_used=False, g0_fallback=True)
    gate = torch.ones(cells, dtype=torch.bool)
    if cfg.min_pair_transport_affinity > 0.0:
        gate.zero_()
        for l, r in pairs:
            if _route_affinity(tpairs.get((l, r))) < cfg.min_pair_transport_affinity:
                continue
            for t in range(l + 1, r):
                gate[min(t // temporal_group_size, cells - 1)] = True
        if not bool(gate.any()):
            return baseline, _route_fallback(layer_index, "no_strong_transport_pair_cells",
                                             fc_cache_used=bool(matching))
    row_gate = gate.repeat_interleave(S)
    K = sel.shape[-1]
    slot = torch.arange(K)
    valid = slot[None, None, None] < counts[..., None]
    hist = valid & (sel < memory_blocks)
    hist_counts = hist.sum(-1)
    swap_counts = valid.sum(-1)
    if int(swap_counts.max()) == 0:
        return baseline, _route_fallback(layer_index, "no_swappable_kv_selected")
    L = min(N, cfg.candidate_multiplier * int(swap_counts.max()))
    ranking = score + local[None, None].to(score.dtype) * 1e6
    cand = torch.sort(ranking, dim=-1, descending=True, stable=True).indices[..., :L]
    prob = torch.softmax(score, dim=-1)
    proxy = omission_proxy(prob, pooled_value, cand, sketch_groups=cfg.sketch_groups)
    limit = torch.minimum(swap_counts.long() * cfg.candidate_multiplier,
                          torch.full_like(swap_counts.long(), N))
    cand_valid = torch.arange(L)[None, None, None] < limit[..., None]

    def member(cur):
        v = slot[None, None, None] < counts[..., None]
        return ((cand[..., None] == cur[..., None, :]) & v[..., None, :]).any(-1)

    retained = member(sel)
    err = (proxy * (cand_valid & ~retained)[..., None]).sum(-2)
    cur_err = err[..., memory_blocks:, :]
    okw = dict(temporal_cells=cells, spatial=S, exact_frames=frames,
               temporal_group_size=temporal_group_size, current_boundary=current_boundary,
               operator=operator, lambda_anchor=cfg.lambda_anchor,
               lambda_reconstruction=cfg.lambda_reconstruction)
    obj_before = route_objective_value(cur_err, **okw)
    swaps = 0
    chosen = []
    m0 = int(memory_blocks)
    for _ in range(cfg.num_swap_rounds):
        a, b, _ = route_objective_terms(cur_err, **okw)
        retained = member(sel)
        v = slot[None, None, None] < counts[..., None]
        sel_local = torch.gather(local[None, None].expand(*sel.shape[:2], -1, -1), -1, sel.clamp_min(0))
        removable = v & ~sel_local
        addable = cand_valid & ~retained
        match = (cand[..., None] == sel[..., None, :]).float()        # [B, H, Q, L, K]
        rem_proxy = torch.einsum("bhqlg,bhqlk->bhqkg", proxy, match)[..., m0:, :, :]
        add_proxy = proxy[..., m0:, :, :]
        delta = rem_proxy[..., :, None, :] - add_proxy[..., None, :, :]   # [B, H, R, K, L, G]
        imp = (a[..., None, None] * (2.0 * cur_err[..., None, None, :] * delta + delta.square())
               + 2.0 * b[..., None, None, :] * delta).sum(-1)
        pair_ok = removable[..., m0:, :, None] & addable[..., m0:, None, :]
        if cfg.min_pair_transport_affinity > 0.0:
            pair_ok = pair_ok & row_gate[None, None, :, None, None]
        if cfg.same_bank_only:
            pair_ok = pair_ok & ((sel[..., m0:, :, None] < m0) == (cand[..., m0:, None, :] < m0))
        imp = imp.masked_fill(~pair_ok, float("inf"))
        best, best_flat = imp.flatten(-2).min(dim=-1)
        flat_best = best.reshape(-1)
        strongest = int(torch.argmin(flat_best))
        if cfg.max_swaps_per_call and swaps >= cfg.max_swaps_per_call:
            break
        if not bool(flat_best[strongest] < -cfg.swap_eps):
            break
        bb, hh, rr = (int(x) for x in torch.unravel_index(torch.tensor(strongest), best.shape))
        fl = int(best_flat[bb, hh, rr])
        rs, al = fl // L, fl % L
        added = int(cand[bb, hh, m0 + rr, al])
        removed = int(sel[bb, hh, m0 + rr, rs])
        sel[bb, hh, m0 + rr, rs] = added
        cur_err = cur_err.clone()
        cur_err[bb, hh, rr] += rem_proxy[bb, hh, rr, rs] - add_proxy[bb, hh, rr, al]
        swaps += 1
        chosen.append({"b": bb, "h": hh, "row": m0 + rr, "slot": rs, "removed": removed,
                       "added": added, "improvement": float(-flat_best[strongest])})
    v = slot[None, None, None] < counts[..., None]
    final_hist = ((sel < m0) & v).sum(-1)
    if cfg.same_bank_only and not torch.equal(hist_counts, final_hist):
        raise RuntimeError("same-bank FC-PASM routing changed Memory KV counts")
    dup = (sel[..., :, None] == sel[..., None, :]) & v[..., :, None] & v[..., None, :] & \
        torch.triu(torch.ones(K, K, dtype=torch.bool), diagonal=1)
    if bool(dup.any()):
        raise RuntimeError("FC-PASM routing emitted duplicate keys")
    kept_local = torch.gather(local[None, None].expand(*sel.shape[:2], -1, -1), -1,
                              sel.clamp_min(0)) & v
    if int(kept_local.sum()) != int(local.sum()) * sel.shape[0] * sel.shape[1]:
        raise RuntimeError("FC-PASM routing removed a protected local edge")
    obj_after = route_objective_value(cur_err, **okw)
    if bool(obj_after > obj_before + 1e-5 * obj_before.abs().clamp_min(1.0)):
        raise RuntimeError("FC-PASM swap increased its refinement objective")
    rec = {"layer_index": int(layer_index), "status": "refined", "candidate_max": L,
           "swap_count": swaps, "objective_before": float(obj_before),
           "objective_after": float(obj_after), "swaps": chosen, "fixed_budget": True,
           "historical_budget_before": int(hist_counts.sum()),
           "historical_budget_after": int(final_hist.sum())}
    return sel.to(selected.dtype), rec


def transport_maps(transport: dict, pair, maps: torch.Tensor, exponent: float) -> torch.Tensor:
    """Change of ``maps`` [N, C, h, w] (the attention block grid) under an
    anchor pair's FC transport at ``exponent``.

    Restates _apply_transport_maps (P/fc_pasm_swap_routing.py:271-412) with
    explicit loops over the overlap windows: bilinear lift to the output grid,
    reflect padding, square-root Hann windows, 2x average pooling to the
    transport grid when it is smaller, spectrum times exp(i exponent g theta),
    back to pixels (and up to the window), weighted overlap-add normalised by
    the summed squared window, the transported minus the zero-phase result,
    averaged over ceil-sized blocks back onto the h x w grid."""
    e = transport["pairs"][pair]
    theta, gain = e["theta"].float(), e["affinity"].float()
    oh, ow = transport["output_shape"]
    th, tw = transport["transport_shape"]
    wh, ww = transport["window_shape"]
    sh, sw = transport["stride"]
    ph, pw = transport["padding"]
    n, c, h, w = maps.shape
    wy = torch.hann_window(wh, periodic=False, dtype=torch.float32)
    wx = torch.hann_window(ww, periodic=False, dtype=torch.float32)
    win = torch.sqrt(torch.clamp(wy[:, None] * wx[None, :], min=0.0))
    up = F.interpolate(maps.float(), size=(oh, ow), mode="bilinear", align_corners=False)
    pad = F.pad(up, (pw, pw, ph, ph), mode="reflect")
    H2, W2 = oh + 2 * ph, ow + 2 * pw
    acc_m = torch.zeros(n, c, H2, W2)
    acc_s = torch.zeros(n, c, H2, W2)
    norm = torch.zeros(H2, W2)
    t = 0
    for y in range(0, H2 - wh + 1, sh):
        for x in range(0, W2 - ww + 1, sw):
            tile = pad[:, :, y:y + wh, x:x + ww] * win
            if (th, tw) != (wh, ww):
                tile = F.avg_pool2d(tile, 2, 2, ceil_mode=True, count_include_pad=False)
            spec = torch.fft.rfft2(tile)
            rot = torch.polar(torch.ones_like(theta[t]), exponent * gain[t] * theta[t])
            mv = torch.fft.irfft2(spec * rot, s=(th, tw))
            st = torch.fft.irfft2(spec, s=(th, tw))
            if (th, tw) != (wh, ww):
                mv = F.interpolate(mv, size=(wh, ww), mode="bilinear", align_corners=False)
                st = F.interpolate(st, size=(wh, ww), mode="bilinear", align_corners=False)
            acc_m[:, :, y:y + wh, x:x + ww] += mv * win
            acc_s[:, :, y:y + wh, x:x + ww] += st * win
            norm[y:y + wh, x:x + ww] += win * win
            t += 1
    if t != theta.shape[0]:
        raise RuntimeError("FC transport tiles do not match the overlap grid")
    nrm = norm[ph:ph + oh, pw:pw + ow].clamp_min(1e-8)
    diff = (acc_m - acc_s)[:, :, ph:ph + oh, pw:pw + ow] / nrm
    bh, bw = -(-oh // h), -(-ow // w)
    return F.avg_pool2d(diff, (bh, bw), (bh, bw), ceil_mode=True, count_include_pad=False)


# --------------------------------------------------------------------------
# f4: shared int8 Q/K/V projection

def quantize_rows_int8(x: torch.Tensor):
    """Per-token symmetric int8 quantisation, the shared step of
    shared_int8_qkv (P/matrix_shared_int8_qkv.py:79-84; the upstream
    int8_quantize_triton is not vendored, so its arithmetic is restated as
    stated): scale = absmax / 127 (1 for an all-zero row), q = clamp(rne(x * 127
    / absmax), -127, 127).  x [..., C] -> (q int8 [M, C], scale fp32 [M])."""
    x2 = x.reshape(-1, x.shape[-1]).float()
    amax = x2.abs().amax(dim=1)
    # (a tensor numerator: python-scalar / tensor would multiply by a rounded reciprocal)
    inv = torch.where(amax > 0, torch.tensor(127.0) / amax, torch.ones_like(amax))
    scale = torch.where(amax > 0, amax / 127.0, torch.ones_like(amax))
    q = torch.clamp(torch.round(x2 * inv[:, None]), -127, 127).to(torch.int8)
    return q, scale


def int8_linear(x_i8: torch.Tensor, x_scale: torch.Tensor, w_i8: torch.Tensor,
                w_scale: torch.Tensor, bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """One projection of shared_int8_qkv (P/matrix_shared_int8_qkv.py:19-38):
    the exact integer product x_i8 @ w_i8^T, dequantised in fp32 as
    (acc * x_scale[m]) * w_scale[n], rounded to bf16, then + bias in bf16."""
    acc = x_i8.to(torch.int64) @ w_i8.to(torch.int64).T
    y = (acc.to(torch.float32) * x_scale.float()[:, None]) * w_scale.float()[None, :]
    y = y.to(torch.bfloat16)
    if bias is not None:
        y = y + bias.to(torch.bfloat16)
    return y

"""RCSA layer-call benchmark on one MI355X.

Workload (the headline configuration): B=1, 24 heads x d128, 3520 query
tokens (4 frames x 880), 35200 history tokens (40 frames) + the 3520-token
current chunk as KV, 128-token blocks, 25% history budget (69 of 275 blocks)
plus the always-kept current chunk, int8 Q/K (per-block symmetric scales, K
mean-smoothed, 4 K channels x10 outliers), bf16 V, seeded synthetic data.

A step is one layer call of the hot path: pooled Q (+ fused int8 Q
quantiser), pooled K (+ smoothing statistics), block scores, top-k
selection, int8 K quantiser, block-sparse attention.  Inputs are resident in
HBM before the timed region.  Every timed region follows 40-60 ms of the same
work (the device's clock ramp after idle), then --warmup steps, then exactly
--steps timed steps.  By default each timed step is one replay of a HIP graph
holding the layer call's launches (checked equal to the eager call); the
eager call's time is reported beside it.

    python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--launch graph|eager]

prints ONE JSON line.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

INT8_PEAK_TOPS = 5000.0     # MI355X dense int8 MFMA
BF16_PEAK_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
HBM_PEAK_GBS = 8000.0       # MI355X HBM3E
# QK^T on int8 and PV on bf16 take equal op counts (2 D per key and query row
# each), so the attention's ceiling is the harmonic mean of the two peaks
MIXED_CEILING_TOPS = 1.0 / (0.5 / INT8_PEAK_TOPS + 0.5 / BF16_PEAK_TFLOPS)
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "attn_int8_dit_traffic.txt")


def _prewarm(fn, min_ms: float = 60.0) -> int:
    """Run ``fn`` back to back for at least ``min_ms`` of wall time.

    After an idle second the device needs about 30 ms of sustained work to
    reach its steady clock (the attention kernel runs 800 us on the first
    launch and 543 us from the 50th on), so every timed region is preceded by
    this much work of its own kind."""
    import torch
    t0 = time.perf_counter()
    calls = 0
    while (time.perf_counter() - t0) * 1e3 < min_ms:
        for _ in range(4):
            fn()
        calls += 4
        torch.cuda.synchronize()
    return calls


def _events_time(fn, iters: int, warmup: int = 3) -> float:
    """Average milliseconds of ``fn`` on the current stream (HIP events),
    after ``warmup`` calls and a pre-warm to the device's steady clock."""
    import torch
    for _ in range(warmup):
        fn()
    _prewarm(fn, 40.0)
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(iters):
        fn()
    stop.record()
    stop.synchronize()
    return start.elapsed_time(stop) / iters


def _read_traffic():
    """HBM bytes per attention launch measured with rocprofv3 --pmc
    (FETCH_SIZE + WRITE_SIZE, copy-kernel calibrated), if recorded."""
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return float(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def _capture(fn):
    """(HIP graph of one ``fn()`` call, that call's result): three warm calls on a
    side stream, then the capture (torch's graph memory pool keeps the captured
    outputs; nothing in the layer call writes memory with a memset)."""
    import torch
    cur = torch.cuda.current_stream()
    side = torch.cuda.Stream()
    side.wait_stream(cur)
    with torch.cuda.stream(side):
        for _ in range(3):
            fn()
    cur.wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        res = fn()
    torch.cuda.synchronize()
    return graph, res


def cpu_baseline(seed: int, heads: int) -> dict:
    """The reference's PyTorch eager fp32 path (restated by the oracle) on the
    host cores, on a bounded sample: ``heads`` of the 24 heads of the same
    layer call; scaled to the full layer call."""
    import torch
    from cast_amd import workloads
    from oracle import rcsa_oracle as orc
    torch.set_num_threads(os.cpu_count() or 1)
    w = workloads.matrix_dit(seed, int8=True)
    q = w.q[:, :heads].float()
    k = w.k[:, :heads].float()
    v = w.v[:, :heads].float()

    def run():
        return orc.rcsa_layer(q, k, v, w.q_valid, w.k_valid, block_size=w.block_size,
                              k_select=w.k_total, forced=w.forced)

    run()  # warmup
    times = []
    res = None
    for _ in range(3):
        t0 = time.perf_counter()
        res = run()
        times.append(time.perf_counter() - t0)
    sample_s = statistics.median(times)
    full_s = sample_s * w.q.shape[1] / heads
    ops = w.attention_ops(res["indices"].reshape(1, heads, w.n_qblocks, -1),
                          res["counts"].reshape(1, heads, w.n_qblocks)) * w.q.shape[1] / heads
    return {"value": ops / full_s / 1e12, "unit": "TOPS", "cores": torch.get_num_threads(),
            "kind": "port", "ms_per_layer_call": full_s * 1e3,
            "sample": (f"the whole layer call, all {heads} heads" if heads == w.q.shape[1] else
                       f"{heads} of {w.q.shape[1]} heads of the layer call, scaled "
                       f"x{w.q.shape[1] / heads:g}") +
                      " (fp32 eager: pool, score, top-k, masked softmax attention), "
                      "median of 3 after 1 warmup"}


def _compact_calls(seed: int, int8: bool = True):
    """The layer call (int8, or bf16) on token-major Q/K/V of the Matrix latent grid (22 x 40
    tokens per frame, (4, 4, 8) tiles with 64-token bottom tiles; 4 query frames,
    40 memory + 4 current key frames; 24 heads, D 128; history budget 25% + the
    current blocks): (packing fused into the kernels through slot maps,
    pack_tokens -> packed layer call -> unpack_tokens, sizes)."""
    import torch
    from cast_amd import layout, ops
    from cast_amd.pipeline import rcsa_attention
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(seed)
    hw, shape, H, D = (22, 40), (4, 4, 8), 24, 128
    lay_q = layout.compact_layout(range(4), 0, *hw, shape, dev)
    lay_k = layout.compact_layout(range(44), 40, *hw, shape, dev)
    lq, lk = 4 * 880, 44 * 880
    q, k, v = (torch.randn(1, n, H, D, device=dev, generator=g).div_(D ** 0.5)
               .to(torch.bfloat16) for n in (lq, lk, lk))
    nq, nk = lay_q.n_blocks, lay_k.n_blocks
    forced = torch.zeros(nq, nk, dtype=torch.bool, device=dev)
    forced[:, nk - 30:] = True
    k_sel = round(0.25 * (nk - 30)) + 30

    def fused():
        return rcsa_attention(q, k, v, None, None, block_size=128, k_select=k_sel,
                              forced=forced, int8=int8, max_k=k_sel,
                              q_slot_token=lay_q.slot_token32,
                              k_slot_token=lay_k.slot_token32).out

    def unfused():
        r = rcsa_attention(ops.pack_tokens(q, lay_q.slot_token), ops.pack_tokens(k, lay_k.slot_token),
                           ops.pack_tokens(v, lay_k.slot_token), lay_q.slot_valid,
                           lay_k.slot_valid, block_size=128, k_select=k_sel, forced=forced,
                           int8=int8, max_k=k_sel)
        return ops.unpack_tokens(r.out, lay_q.token_to_packed)

    return fused, unfused, {"q_blocks": nq, "k_blocks": nk, "k_select": k_sel}


def compact_layout_call(seed: int, iters: int) -> dict:
    """The gathered layer call against pack -> packed call -> unpack (int8,
    then the bf16 drop-in)."""
    import torch
    res = {}
    for int8 in (True, False):
        fused, unfused, sizes = _compact_calls(seed, int8)
        same = bool(torch.equal(fused(), unfused()))
        _prewarm(fused, 40.0)
        f_ms = _events_time(fused, iters)
        u_ms = _events_time(unfused, iters)
        res["int8" if int8 else "bf16"] = {"fused_ms": f_ms, "pack_unpack_ms": u_ms,
                                           "outputs_equal": same}
    return {**res, **sizes}


def router_call(seed: int, iters: int) -> dict:
    """One FC-PASM swap-router refinement on a compact Matrix layer (24 heads,
    303 blocks = 183 memory + 4 cells of 6 x 5 current blocks, 99 kept blocks
    per row, D 128, anchors 0 and 6 with five skipped frames, a route from the
    pooled scores' top-k, g = 0 transport), timed by wall clock around the
    whole call (it reads back the strongest row once per round)."""
    import torch
    from cast_amd import layout
    from cast_amd.router import FCPASMSwapRouter, FCPASMSwapRoutingConfig
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(seed)
    H, N, M, D, K = 24, 303, 183, 128, 99
    qh = torch.nn.functional.normalize(torch.randn(1, H, N, D, device=dev, generator=g), dim=-1)
    kh = torch.nn.functional.normalize(torch.randn(1, H, N, D, device=dev, generator=g), dim=-1)
    score = qh @ kh.transpose(-1, -2)
    pooled_v = torch.randn(1, H, N, D, device=dev, generator=g)
    local = layout.local_stencil(N, 6, 5, dev)
    sel = torch.sort(score + local[None, None] * 1e6, dim=-1, descending=True,
                     stable=True).indices[..., :K].to(torch.int32)
    counts = torch.full((1, H, N), K, device=dev, dtype=torch.int32)
    router = FCPASMSwapRouter(FCPASMSwapRoutingConfig(max_swaps_per_call=1, same_bank_only=True))
    kw = dict(score=score, pooled_value=pooled_v, selected=sel, counts=counts, local=local,
              memory_blocks=M, spatial_shape=(6, 5), exact_current_frames=(0, 6),
              temporal_group_size=4, current_boundary=8, transport=None, layer_index=22)
    _, rec = router.refine(**kw)
    for _ in range(3):
        router.refine(**kw)
    torch.cuda.synchronize()
    # wall clock with the garbage collector paused, as timeit does: one full
    # collection over the process's objects takes tens of ms, longer than the
    # whole timed loop
    import gc
    gc.collect()
    gc.disable()
    try:
        t0 = time.perf_counter()
        for _ in range(iters):
            router.refine(**kw)
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) * 1e3 / iters
    finally:
        gc.enable()
    return {"ms_per_refine": ms, "swap_count": rec["swap_count"],
            "candidates": rec["candidate_max"], "blocks": N, "heads": H}


def qkv_call(seed: int, iters: int) -> dict:
    """The shared int8 Q/K/V projection of a Matrix self-attention block:
    38,720 tokens x 3072 channels (44 frames of 22 x 40) into q, k and v of
    3072 channels each, bf16 in and out, random int8 weights: one per-token
    quantisation, three int8 GEMMs with the dequantising epilogue."""
    import torch
    from types import SimpleNamespace
    from cast_amd import ops
    from cast_amd.qkv import shared_int8_qkv
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(seed)
    L, C = 38720, 3072
    mods = [SimpleNamespace(in_features=C, out_features=C,
                            weight_int8=torch.randint(-127, 128, (C, C), device=dev, generator=g,
                                                      dtype=torch.int8),
                            weight_scales=torch.rand(C, device=dev, generator=g) * 2e-3,
                            bias=torch.randn(C, device=dev, generator=g).bfloat16())
            for _ in range(3)]
    x = torch.randn(1, L, C, device=dev, generator=g).bfloat16()
    xq, xs = ops.quantize_rows_int8(x)
    gemm_ms = _events_time(lambda: ops.int8_linear(xq, xs, mods[0].weight_int8,
                                                   mods[0].weight_scales, mods[0].bias), iters)
    quant_ms = _events_time(lambda: ops.quantize_rows_int8(x), iters)
    call_ms = _events_time(lambda: shared_int8_qkv(*mods, x), iters)
    ops_gemm = 2.0 * L * C * C
    return {"ms_per_call": call_ms, "quantize_ms": quant_ms, "gemm_ms": gemm_ms,
            "gemm_TOPS": ops_gemm / gemm_ms / 1e9,
            "gemm_frac_int8_peak": ops_gemm / gemm_ms / 1e9 / INT8_PEAK_TOPS,
            "quantize_GBs": (L * C * 3 + L * 4) / quant_ms / 1e6,
            "tokens": L, "channels": C}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extras", action="store_true")
    ap.add_argument("--cpu-heads", type=int, default=24)
    ap.add_argument("--launch", choices=["graph", "eager"], default="graph",
                    help="issue each timed layer call as one HIP graph replay (default) "
                         "or as the eager Python call")
    ap.add_argument("--only", choices=["attn_int8", "attn_bf16", "copy", "layer", "compact",
                                       "compact_bf16", "router", "qkv", "sweep"],
                    default=None,
                    help="profiling mode: run only this kernel (or the whole int8 layer "
                         "call, or the gathered call on the Matrix latent grid) --steps "
                         "times after --warmup, and print its average time; 'sweep' runs "
                         "--steps int8 attention launches per layer of the 30-layer step "
                         "sweep, in layer order")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU (the RCSA path needs no collective; "
              f"heads shard with no exchange); --gpus {args.gpus} is not supported",
              file=sys.stderr)
        return 2

    import torch
    from cast_amd import _lib, ops, workloads
    from cast_amd.pipeline import rcsa_attention
    _lib.load()  # fail loudly if the HIP library is missing
    dev = torch.device("cuda:0")

    if args.only == "copy":
        # calibration for HBM byte counters: a plain 1 GiB device copy
        src = torch.empty(1 << 28, device=dev, dtype=torch.float32).fill_(1.0)
        dst = torch.empty_like(src)
        ms = _events_time(lambda: dst.copy_(src), args.steps, args.warmup)
        print(json.dumps({"only": "copy", "bytes_read": src.numel() * 4,
                          "bytes_written": dst.numel() * 4, "avg_ms": ms}))
        return 0

    if args.only == "qkv":
        print(json.dumps({"only": "qkv", **qkv_call(args.seed, args.steps)}))
        return 0

    if args.only == "router":
        print(json.dumps({"only": "router", **router_call(args.seed, args.steps)}))
        return 0

    if args.only in ("compact", "compact_bf16"):
        fused, _, sizes = _compact_calls(args.seed, args.only == "compact")
        ms = _events_time(fused, args.steps, args.warmup)
        print(json.dumps({"only": args.only, "avg_ms": ms, **sizes}))
        return 0

    w = workloads.matrix_dit(args.seed, int8=args.only != "attn_bf16").to(dev)
    bs = w.block_size
    max_k = w.k_total

    if args.only == "sweep":
        # the 30-layer step sweep's attention launches for per-layer counters:
        # every layer's selection first (one layer call each), then --steps int8
        # attention launches per layer in layer order, one JSON line per layer
        plan = workloads.step_sweep_plan(args.seed)
        layers = [workloads.step_layer_view(w, p) for p in plan]
        prepared = []
        for lw in layers:
            r = rcsa_attention(lw.q, lw.k, lw.v, lw.q_valid, lw.k_valid, block_size=bs,
                               k_select=lw.k_total, forced=lw.forced, int8=True,
                               max_k=lw.k_total)
            prepared.append((lw, r, torch.empty_like(lw.q)))
        torch.cuda.synchronize()
        for i, ((lw, r, o), p) in enumerate(zip(prepared, plan)):
            for _ in range(args.steps):
                ops.sparse_attn_int8(r.q_i8, r.q_scale, r.k_i8, r.k_scale, lw.v, r.indices,
                                     r.counts, None, out=o, block_mask=r.k_mask)
            torch.cuda.synchronize()
            print(json.dumps({"only": "sweep", "layer": i, "query_frames": p["query_frames"],
                              "fraction": p["fraction"], "launches": args.steps,
                              "ops": lw.attention_ops(r.indices, r.counts)}), flush=True)
        return 0

    if args.only == "layer":
        def layer():
            return rcsa_attention(w.q, w.k, w.v, w.q_valid, w.k_valid, block_size=bs,
                                  k_select=w.k_total, forced=w.forced, int8=True, max_k=max_k)
        ms = _events_time(layer, args.steps, args.warmup)
        print(json.dumps({"only": "layer", "avg_ms": ms}))
        return 0

    if args.only is not None:
        r = rcsa_attention(w.q, w.k, w.v, w.q_valid, w.k_valid, block_size=bs,
                           k_select=w.k_total, forced=w.forced, int8=w.int8, max_k=max_k)
        out = torch.empty_like(w.q)
        if w.int8:
            fn = lambda: ops.sparse_attn_int8(r.q_i8, r.q_scale, r.k_i8, r.k_scale, w.v,  # noqa
                                              r.indices, r.counts, None, block_m=bs,
                                              block_n=bs, out=out, block_mask=r.k_mask)
        else:
            fn = lambda: ops.sparse_attn_bf16(w.q, w.k, w.v, r.indices, r.counts,  # noqa
                                              None, block_m=bs, block_n=bs, out=out,
                                              block_mask=r.k_mask)
        torch.cuda.synchronize()
        ms = _events_time(fn, args.steps, args.warmup)
        ops_attn = w.attention_ops(r.indices, r.counts)
        print(json.dumps({"only": args.only, "avg_ms": ms, "ops": ops_attn,
                          "TOPS": ops_attn / ms / 1e9}))
        return 0

    def step():
        return rcsa_attention(w.q, w.k, w.v, w.q_valid, w.k_valid, block_size=bs,
                              k_select=w.k_total, forced=w.forced, int8=True, max_k=max_k)

    # one int8 attention dispatch per step: the timed ones are dispatches
    # [first_timed, first_timed + steps) of this process (a kernel trace's order)
    dispatched = _prewarm(step, 60.0) + args.warmup
    for _ in range(args.warmup):
        res = step()
    run = step
    if args.launch == "graph":
        # The layer call captured once in a HIP graph and replayed: the same
        # launches, arguments and buffers as the eager call, issued by one
        # graph launch per step, so that the host's speed (a fresh box's
        # Python thread can take 100-260 us per eager call) never leaves the
        # GPU waiting between steps.  Every replay must equal the eager call.
        graph, gres = _capture(step)
        dispatched += 3
        for _ in range(3):
            graph.replay()
            torch.cuda.synchronize()
            if not (torch.equal(gres.out, res.out) and torch.equal(gres.indices, res.indices)
                    and torch.equal(gres.counts, res.counts)):
                raise RuntimeError("bench.py: the graph replay differs from the eager layer call")
            step()  # eager work between the replays
        dispatched += 6
        run = graph.replay
        dispatched += _prewarm(run, 60.0) + args.warmup
        for _ in range(args.warmup):
            run()
        res = gres
    first_timed = dispatched
    # HIP events around the entry points of the layer call, on the stream they
    # launch on (torch's current stream): the attention's launch time for the
    # roofline, and the fused pooling and quantiser/selection launches as they
    # run inside the layer call (K no longer in the MALL from the step before).
    # No event sits in the timed steps (each recorded event adds GPU time
    # between the launches, about 24 us per step for one pair); the entry points
    # are timed this way in as many steps right after them.
    names = ("sparse_attn_int8", "pool_query_key", "quantize_key_select")
    events = {n: [] for n in names}
    entries = {n: getattr(ops, n) for n in names}

    def timed(name):
        entry_ = entries[name]

        def wrapper(*a, **kw):
            ev0 = torch.cuda.Event(enable_timing=True)
            ev1 = torch.cuda.Event(enable_timing=True)
            ev0.record()
            r_ = entry_(*a, **kw)
            ev1.record()
            events[name].append((ev0, ev1))
            return r_
        return wrapper

    def instrumented(which, n_steps):
        for n in which:
            setattr(ops, n, timed(n))
        try:
            for _ in range(n_steps):
                r_ = step()
        finally:
            for n in which:
                setattr(ops, n, entries[n])
        return r_

    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        run()
    t_enqueued = time.perf_counter()  # the host has issued every timed step
    torch.cuda.synchronize()
    ms_per_step = (time.perf_counter() - t0) * 1e3 / args.steps
    host_ms_per_step = (t_enqueued - t0) * 1e3 / args.steps
    instrumented(names, args.steps)
    torch.cuda.synchronize()
    # the same steps issued by the eager Python call, for comparison
    t1 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    eager_ms_per_step = (time.perf_counter() - t1) * 1e3 / args.steps
    call_ms = {n: statistics.fmean(a.elapsed_time(b) for a, b in ev) for n, ev in events.items()}
    attn_ms = call_ms["sparse_attn_int8"]
    ops_attn = w.attention_ops(res.indices, res.counts)
    value = ops_attn / (ms_per_step * 1e-3) / 1e12

    # ---- per-kernel timings with HIP events on the launch stream ----
    iters = max(10, args.steps)
    qhat, q8, qs = ops.pool_query(w.q, w.q_valid, bs, quantize=True)
    khat, ksum, kmin, kmax, kmask = ops.pool_key(w.k, w.k_valid, bs, stats=True,
                                                 block_mask=True)
    score = ops.block_scores(qhat, khat)
    idx, cnt = ops.select_topk(score, w.k_total, forced=w.forced, max_k=max_k)
    k8, ks, km = ops.quantize_key(w.k, w.k_valid, bs, ksum, kmin, kmax)
    B, H, Lq, D = w.q.shape
    idx4, cnt3 = idx.view(B, H, -1, max_k), cnt.view(B, H, -1)
    out = torch.empty_like(w.q)
    stage_ms = {
        "pool_query_quant": _events_time(lambda: ops.pool_query(w.q, w.q_valid, bs, True), iters),
        "pool_key_stats": _events_time(lambda: ops.pool_key(w.k, w.k_valid, bs, True, True),
                                       iters),
        "block_scores": _events_time(lambda: ops.block_scores(qhat, khat), iters),
        "select_topk": _events_time(lambda: ops.select_topk(score, w.k_total, forced=w.forced,
                                                            max_k=max_k), iters),
        "quantize_key": _events_time(lambda: ops.quantize_key(w.k, w.k_valid, bs, ksum, kmin,
                                                              kmax), iters),
        "sparse_attn_int8": _events_time(lambda: ops.sparse_attn_int8(
            q8, qs, k8, ks, w.v, idx4, cnt3, None, block_m=bs, block_n=bs, out=out,
            block_mask=kmask), iters),
    }
    achieved = ops_attn / (attn_ms * 1e-3) / 1e12
    qk_ops = pv_ops = ops_attn / 2
    mixed_floor_ms = (qk_ops / (INT8_PEAK_TOPS * 1e12) + pv_ops / (BF16_PEAK_TFLOPS * 1e12)) * 1e3
    el = w.q.element_size()
    nbh = B * H
    lk = w.k.shape[2]
    nqb, nkb = w.n_qblocks, w.n_kblocks
    # algorithmic bytes: every input read once, every output written once
    pool_q = nbh * Lq * D * (el + 1) + nbh * nqb * (D + 1) * 4
    pool_k = nbh * lk * D * el + 4 * nbh * nkb * D * 4 + nkb * bs // 8
    quant_k = nbh * lk * D * (el + 1) + 3 * nbh * nkb * D * 4 + nbh * (nkb + D) * 4
    select = nbh * (nqb + nkb) * D * 4 + nbh * nqb * (nkb + max_k + 1) * 4
    hbm_bytes = {"pool_query_key": (pool_q + pool_k, call_ms["pool_query_key"]),
                 "quantize_key_select": (quant_k + select, call_ms["quantize_key_select"])}
    hbm_frac = {k_: {"bytes": b, "ms": ms_, "GB/s": b / (ms_ * 1e-3) / 1e9,
                     "frac": b / (ms_ * 1e-3) / 1e9 / HBM_PEAK_GBS}
                for k_, (b, ms_) in hbm_bytes.items()}

    line = {
        "metric": "block-sparse attn ms/layer-call + effective TOPS, int8-QK, 3.5k q x 35k KV",
        "value": value,
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": "rcsa_layer_call_int8qk_bf16pv", "batch": 1, "heads": H,
                   "head_dim": D, "query_tokens": 3520, "history_tokens": 35200,
                   "current_kv_tokens": 3520, "block_size": bs,
                   "history_budget_blocks": w.k_hist, "history_blocks": w.n_hist_blocks,
                   "blocks_per_row": w.k_total, "outlier_k_channels": 4},
        "roofline": {"bound": "mfma", "achieved": achieved, "peak": INT8_PEAK_TOPS,
                     "unit": "TFLOP/s", "frac": achieved / INT8_PEAK_TOPS,
                     "traffic": _read_traffic(),
                     "kernel": "sparse_attn_kernel<int8>", "ops_per_launch": ops_attn,
                     "avg_launch_ms": attn_ms,
                     "mixed_ceiling_frac": mixed_floor_ms / attn_ms},
    }
    ns_plan = ctypes.c_int64(0)
    _lib.load().rcsa_attn_split_plan(B, H, Lq, bs, max_k, ctypes.byref(ns_plan))
    extras = {"stage_ms": stage_ms, "layer_call_ms": call_ms, "hbm": hbm_frac,
              "launch": args.launch, "host_enqueue_ms_per_step": host_ms_per_step,
              "eager_ms_per_step": eager_ms_per_step,
              "ms_per_layer_call": ms_per_step,
              "attn_split_plan": ns_plan.value,
              "attn_timed_dispatches": [first_timed, args.steps]}

    if not args.no_extras:
        # bf16-QK attention on the same shape (the drop-in kernel)
        wb = workloads.matrix_dit(args.seed, int8=False).to(dev)
        rb = rcsa_attention(wb.q, wb.k, wb.v, wb.q_valid, wb.k_valid, block_size=bs,
                            k_select=wb.k_total, forced=wb.forced, int8=False, max_k=max_k)
        outb = torch.empty_like(wb.q)
        bf_ms = _events_time(lambda: ops.sparse_attn_bf16(
            wb.q, wb.k, wb.v, rb.indices, rb.counts, None, block_m=bs, block_n=bs,
            out=outb, block_mask=rb.k_mask), iters)
        bf_bytes_ms = _events_time(lambda: ops.sparse_attn_bf16(
            wb.q, wb.k, wb.v, rb.indices, rb.counts, wb.k_valid, block_m=bs, block_n=bs,
            out=outb), iters)
        bf_ops = wb.attention_ops(rb.indices, rb.counts)
        extras["bf16_attn"] = {"ms": bf_ms, "TFLOP/s": bf_ops / bf_ms / 1e9,
                               "frac_bf16_peak": bf_ops / bf_ms / 1e9 / BF16_PEAK_TFLOPS,
                               "validity": "bits (key pooling pass)",
                               "ms_validity_bytes": bf_bytes_ms}
        del wb, rb, outb
        # per-denoising-step sweep: 30 layers, 1-4 anchor frames, 12.5-50% budget
        plan = workloads.step_sweep_plan(args.seed)
        layers = [workloads.step_layer_view(w, p) for p in plan]

        def layer_call(lw):
            return rcsa_attention(lw.q, lw.k, lw.v, lw.q_valid, lw.k_valid, block_size=bs,
                                  k_select=lw.k_total, forced=lw.forced, int8=True,
                                  max_k=lw.k_total)

        # warm pass (also counts the ops); the timed passes keep no results, so
        # every layer reuses the previous layer's buffers
        sweep_ops = 0.0
        _prewarm(lambda: layer_call(layers[0]), 40.0)
        for lw in layers:
            r = layer_call(lw)
            sweep_ops += lw.attention_ops(r.indices, r.counts)
            del r
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        n_sweep = 3
        for _ in range(n_sweep):
            for lw in layers:
                layer_call(lw)
        torch.cuda.synchronize()
        step_ms = (time.perf_counter() - t0) * 1e3 / n_sweep
        # per layer: the attention launch alone (HIP events), its ops and the
        # fraction of the dense int8 peak and of the int8-QK + bf16-PV ceiling
        per_layer = []
        for p, lw in zip(plan, layers):
            r = layer_call(lw)
            ops_l = lw.attention_ops(r.indices, r.counts)
            o = torch.empty_like(lw.q)
            ms_l = _events_time(lambda: ops.sparse_attn_int8(
                r.q_i8, r.q_scale, r.k_i8, r.k_scale, lw.v, r.indices, r.counts, None, out=o,
                block_mask=r.k_mask), 10, 2)
            tops = ops_l / ms_l / 1e9
            call_l = _events_time(lambda: layer_call(lw), 10, 2)
            per_layer.append({"query_frames": p["query_frames"], "fraction": p["fraction"],
                              "layer_call_ms": round(call_l, 4),
                              "attn_ms": round(ms_l, 4), "attn_TOPS": round(tops, 1),
                              "frac_int8_peak": round(tops / INT8_PEAK_TOPS, 4),
                              "frac_mixed_ceiling": round(tops / MIXED_CEILING_TOPS, 4)})
            del r, o
        extras["step_sweep_30_layers"] = {"ms_per_step": step_ms,
                                          "effective_TOPS": sweep_ops / step_ms / 1e9,
                                          "attention_per_layer": per_layer}
        del layers
        extras["compact_layout_call"] = compact_layout_call(args.seed, iters)
        # per-row budgets on the device: 30 layers x 28 query blocks, and one
        # 853-row section (the longest history), largest remainder + saturation
        gb = torch.Generator(device=dev).manual_seed(args.seed)
        w30 = torch.rand(30, 28, device=dev, generator=gb)
        w853 = torch.rand(1, 853, device=dev, generator=gb)
        extras["row_budgets_us"] = {
            "30x28": 1e3 * _events_time(lambda: ops.row_budgets(w30, 28 * 69, cap=303), iters),
            "1x853": 1e3 * _events_time(lambda: ops.row_budgets(w853, 853 * 64, cap=853),
                                        iters)}
        # closed-loop degrees of a compact woven layer: 30 worldlines (6 x 5
        # spatial tiles), 16 current frames in 4 cells after 183 memory rows,
        # with the previous layer's response fed back; status left on the device
        curv = torch.rand(4, 30, device=dev, generator=gb) + 0.05
        resp = torch.rand(4, 30, device=dev, generator=gb) * 2
        cl_kw = dict(current_temporal_offset=3, source_group=4, compact_group=4,
                     mean_degree=61, base_degree=49, total_blocks=303, memory_blocks=183,
                     response=resp, response_weight=0.5, check_status=False)
        frames_d = torch.arange(3, 19, device=dev, dtype=torch.int32)
        extras["row_budgets_us"]["closed_loop_303"] = 1e3 * _events_time(
            lambda: ops.closed_loop_degrees(curv, frames_d, **cl_kw), iters)
        extras["fc_pasm_router"] = router_call(args.seed, iters)
        extras["int8_qkv_projection"] = qkv_call(args.seed, iters)

    line["extras"] = extras
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(args.seed, args.cpu_heads)
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())

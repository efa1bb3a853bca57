"""Benchmark: one page-sparse attention call on one MI355X.

Headline workload: the full-window base tier, 12 heads x 4608 queries x d128
bf16 against a 432-page (27648-token) window with 64 exact pages per 64-query
block (24 anchors + own + 39 by risk) and every other page compensated from
its summary.  One step = route + rep values + fused attention over one call's
inputs, all resident in HBM, in the arithmetic a drop-in caller gets by
default: the reference's two-term bf16 P.V (--single-av: one bf16 product).

Also measured in the same run:
* the same call in the other P.V arithmetic, and the 216-page window (base
  tier, 32 exact pages) in both;
* the intersection tier: 24 anchors + A current + B history pages per head,
  (A, B) from a seeded per-(step, layer, head) quota table;
* the same with the Full_Pset swap correction on heads {3, 4, 9}, plus what a
  denoise step refreshes first: the summaries (4-iteration k-means) and the
  encodings of the 72 current pages x 12 heads;
* dense attention over the whole window: torch's scaled_dot_product_attention
  and this library's kernel with every page exact;
* a chunk of the 30-layer streaming workload (rolling window runtime).

Before the first measured line, untimed headline calls run for
--device-warmup-ms (300 ms): a GPU leaving its idle clocks would otherwise
slow whatever is measured first.  The headline is timed right after them;
every line does its own warm-up calls (the headline exactly --warmup) before
its timed calls.

Prints ONE JSON line; `value` is ms per call (lower is better).  The
roofline object covers the dominant kernel (fused exact + compensation +
merge): its average duration inside a call, from HIP events recorded around
each launch on the stream it runs on, over a second pass of the same calls
right after the timed region.  cpu_baseline times the CPU oracle on a
bounded sample of the headline call; extra.cpu_baseline_other_configs the
same for the 216-page call, the intersection call and the Full_Pset call.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

# HBM bytes per attn_kernel launch of the base-tier call, keyed by (pages, exact pages, single-term P.V),
# measured with rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE on this bench (profiles/attn_kernel_base432_traffic.md):
# 139.9 MB read + 20.0 MB written by attn_kernel<true, 1, 0> (the two-term headline; the figure leaves out
# merge_kernel's 6.5 MB read and 1.6 MB written).  The single-term kernel was not measured: traffic null.
MEASURED_TRAFFIC = {(432, 64, False): 159.9e6}
METRIC = "ms per sparse-attn call at 432-page window, 12 heads; MFMA util + HBM GB/s"
PEAK_BF16_TFLOPS = 2500.0
PEAK_HBM_GBS = 8000.0
PSET_HEADS = (3, 4, 9)
# untimed calls before a line whose inputs were just made on the host, or that
# follows calls of another kind (ms)
LINE_WARMUP_MS = 100.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # one call is ~0.25 ms: 100 warmup calls (~25 ms) bring the clocks to
    # their steady state under this load, 200 timed calls take ~50 ms
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--frames", type=int, default=18, help="window frames (18 -> 432 pages)")
    ap.add_argument("--single-av", action="store_true",
                    help="headline in single-term bf16 P.V (default: the reference's two-term product)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-dense", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="skip the intersection / Full_Pset lines")
    ap.add_argument("--no-chunk", action="store_true", help="skip the per-chunk 30-layer line")
    ap.add_argument("--cpu-sample-blocks", type=int, default=4)
    ap.add_argument("--device-warmup-ms", type=float, default=300.0,
                    help="untimed headline calls for at least this long before the first measured line")
    ap.add_argument("--headline-only", action="store_true",
                    help="only the headline call (for a profiler run whose kernel averages are the headline's)")
    ap.add_argument("--staged", action="store_true",
                    help="with --headline-only: the call's attention as two launches (exact pages, then the "
                         "compensation) and a merge, so a profiler shows the stages apart")
    ap.add_argument("--chunk-only", action="store_true",
                    help="only the streaming chunk line (for a profiler run of the 30-layer chunk)")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only run a device-to-device copy of MIB MiB (scales rocprof FETCH/WRITE_SIZE)")
    return ap.parse_args()


def calibrate_copy(mib):
    import torch
    src = torch.empty(mib * (1 << 20), dtype=torch.uint8, device="cuda")
    src.fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"calibration_copy_bytes": src.numel(), "copies": 3}), flush=True)


def log(msg):
    """Progress line on stderr (the JSON line is the only stdout output)."""
    print(f"# {time.strftime('%H:%M:%S')} {msg}", file=sys.stderr, flush=True)


def time_loop(fn, iters, stream):
    """Average ms of `fn` over `iters` back-to-back launches, HIP events on
    the stream the work is enqueued on."""
    import torch
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for _ in range(iters):
        fn()
    b.record(stream)
    b.synchronize()
    return a.elapsed_time(b) / iters


def call_step(g, P, single, stream, staged=False):
    """One base-tier call (route + attention) as a function of optional HIP
    event marks recorded before the route, between the launches and after
    the attention."""
    import torch
    from streaming_sparse_amd.attention import Workspace
    from streaming_sparse_amd.legacy_components import REP_OP_ELEMS, attention, rep_tiles
    from streaming_sparse_amd.route import route
    dev = g.q.device
    H = 12
    ws = Workspace()
    basis = g.basis.to(torch.bfloat16).contiguous()   # the caller keeps the basis bf16-rounded
    ops = ws.tensor('call_rep_ops', (H, rep_tiles(P), REP_OP_ELEMS), dev, torch.bfloat16)

    def step(marks=None):
        # own page of block t is P-72+t (the router's default when own is None); the router also writes
        # the call's detail operand tiles, which the attention kernel reads
        if marks:
            marks[0].record(stream)
        ids, _, _, _ = route(g.q, g.summary, g.theta, tier='base', workspace=ws, want_mask=False, rep_out=ops)
        if marks:
            marks[1].record(stream)
        o = attention(g.q, g.k, g.v, g.summary, basis, ids, ws, single_av=single, rep_ops=ops, staged=staged)
        if marks:
            marks[2].record(stream)
        return o

    return step


def call_timings(g, P, C, single, steps, warmup, stream, staged=False):
    """One base-tier call (route + attention) timed over `steps` calls after
    `warmup`, then the kernels' average durations inside a call from HIP events
    recorded around each launch on its stream (a second pass of the same
    calls, kept out of the timed region whose calls they would space out).
    Also returns the host's enqueue time per call over the timed calls."""
    import torch
    step = call_step(g, P, single, stream, staged)
    for _ in range(warmup):
        step()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    host_ms = (time.perf_counter() - t0) * 1e3 / steps
    end.record(stream)
    torch.cuda.synchronize()
    ms_call = start.elapsed_time(end) / steps
    marks = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
    for i in range(steps):
        step(marks[i])
    torch.cuda.synchronize()
    route_in = sum(m[0].elapsed_time(m[1]) for m in marks) / steps
    attn_in = sum(m[1].elapsed_time(m[2]) for m in marks) / steps
    return ms_call, route_in, attn_in, host_ms


def device_warmup(step, ms):
    """Untimed headline calls (`step`) for at least `ms` milliseconds of wall
    time, before anything is measured: the GPU leaves its idle clocks within
    a few hundred ms of load.  Measured first in a fresh process, 5 warm-up
    and 20 timed calls of the headline read ~0.29 ms against ~0.25 ms after
    such a warm-up (the host enqueues a call in ~0.05 ms, so the loop is not
    host-bound)."""
    import torch
    t0 = time.perf_counter()
    calls = 0
    while (time.perf_counter() - t0) * 1e3 < ms:
        for _ in range(20):
            step()
        calls += 20
        torch.cuda.synchronize()
    return calls


def attn_flop(N, H, D, C, P):
    """Algorithmic FLOP of the fused kernel: exact QK + PV over C pages, and the
    compensation (rep QK, mean PV, detail PV, rank-8 projection)."""
    exact = 4.0 * N * H * D * 64 * C
    comp = 2.0 * N * H * D * 4 * P + 2.0 * N * H * P * D + 6.0 * N * H * P * 8 + 2.0 * N * H * 8 * D
    return exact, comp


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "bench.py measures one GPU only; heads shard across GPUs without "
                                   "exchange, so run --gpus 1"}))
        sys.exit(2)
    if args.calibrate_copy:
        calibrate_copy(args.calibrate_copy)
        return
    if args.chunk_only:
        print(json.dumps({"metric": "ms per 3-frame chunk, 30 layers", "chunk": chunk_line(args)}), flush=True)
        return
    import torch
    from streaming_sparse_amd import _lib, workload
    from streaming_sparse_amd.attention import Workspace
    from streaming_sparse_amd.legacy_components import (REP_OP_ELEMS, attention, kv_strides, rep_operands, rep_tiles,
                                                        split_workspace)
    from streaming_sparse_amd.route import route

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    t0 = time.time()
    x = workload.make_call(cfg=1, frames=args.frames)
    gen_s = time.time() - t0
    g = x.to(dev)
    P = x.pages
    H, N, D = 12, 4608, 128
    C = P * 15 // 100
    stream = torch.cuda.current_stream(dev)
    single = bool(args.single_av)
    print(f"# headline: base tier P={P} C={C} single_av={single} staged={bool(args.staged)}", file=sys.stderr,
          flush=True)
    warm_calls = device_warmup(call_step(g, P, single, stream, args.staged and args.headline_only),
                               args.device_warmup_ms) if args.device_warmup_ms > 0 else 0
    log(f"device warm-up: {warm_calls} untimed calls")
    # the headline is timed right after its own warm-up, before the dense
    # calls below: a few SDPA and every-page calls (~1 ms each) ahead of only
    # `warmup` headline calls left their first timed calls ~4% slower
    ms_call, route_in_ms, attn_in_ms, host_ms = call_timings(g, P, C, single, args.steps, args.warmup, stream,
                                                             staged=args.staged and args.headline_only)
    if args.headline_only:
        log(f"headline call {ms_call:.4f} ms (attention kernel {attn_in_ms:.4f} ms)")
        print(json.dumps({"metric": METRIC, "value": round(ms_call, 4), "unit": "ms", "headline_only": True,
                          "attention_kernel_ms": round(attn_in_ms, 4), "route_ms": round(route_in_ms, 4),
                          "host_enqueue_ms_per_call": round(host_ms, 4), "single_av": single,
                          "device_warmup": {"ms": args.device_warmup_ms, "untimed_calls": warm_calls},
                          "staged": bool(args.staged)}), flush=True)
        return

    # per-kernel timings back to back (same stream, same inputs), straight through the C ABI
    ws = Workspace()
    basis = g.basis.to(torch.bfloat16).contiguous()
    ids, _, _, _ = route(g.q, g.summary, g.theta, tier='base', workspace=ws, want_mask=False)
    ops = ws.tensor('ssa_rep_ops', (H, rep_tiles(P), REP_OP_ELEMS), dev, torch.bfloat16)
    rep_operands(g.summary, P, ops)
    out = torch.empty_like(g.q)
    tok, head = kv_strides(g.k, g.v)
    L = _lib.lib()

    def attn_only(flags):
        split = split_workspace(ws, N, H, P, C, flags, dev)
        _lib.check(L.ssa_attention(_lib.ptr(g.q), _lib.ptr(g.k), _lib.ptr(g.v), _lib.ptr(g.summary.keys),
                                   _lib.ptr(g.summary.mean), _lib.ptr(basis), _lib.ptr(ops), _lib.ptr(ids),
                                   _lib.ptr(out), N, H, P, g.summary.head_pages, ops.shape[1], C, tok, head, flags,
                                   _lib.ptr(split), 0 if split is None else split.numel(), _lib.stream_handle(dev)),
                   "ssa_attention")

    iters = max(10, args.steps)
    attn_ms = {name: time_loop(lambda f=f: attn_only(f), iters, stream) for name, f in (("two_term", 1),
                                                                                       ("single_term", 0))}
    rids, _, rrisk, _ = route(g.q, g.summary, g.theta, tier='base', workspace=ws, want_mask=False)
    ops_call = torch.empty(H, rep_tiles(P), REP_OP_ELEMS, device=dev, dtype=torch.bfloat16)
    theta32 = g.theta.float().contiguous()

    def route_only():
        _lib.check(L.ssa_route(_lib.ptr(g.q), D, 64 * H * D, H * D, 0, _lib.ptr(g.summary.keys),
                               _lib.ptr(g.summary.stats), _lib.ptr(theta32), None, None, _lib.ptr(rrisk),
                               _lib.ptr(rids), None, None, H, N // 64, P, g.summary.head_pages, C, 0, 0,
                               _lib.ptr(g.summary.detail), _lib.ptr(ops_call), ops_call.shape[1], 0.0, None, None,
                               _lib.stream_handle(dev)), "ssa_route")

    route_ms = time_loop(route_only, iters, stream)
    log(f"kernels back to back: attention {attn_ms}, route {route_ms:.4f} ms")

    dense_ms = None
    dense_own = {}
    if not args.no_dense:
        qd = g.q[0].transpose(0, 1)[None]
        kd = g.k[0].transpose(0, 1)[None]
        vd = g.v[0].transpose(0, 1)[None]
        dense = lambda: torch.nn.functional.scaled_dot_product_attention(qd, kd, vd)
        device_warmup(dense, LINE_WARMUP_MS)
        dense_ms = time_loop(dense, max(5, iters // 5), stream)
        # this library's kernel with every page exact (the dense layers' call)
        own = torch.arange(N // 64, device=dev) + P - N // 64
        allp = torch.arange(P, device=dev)
        dids = torch.cat([own[:, None], allp[None].expand(N // 64, -1)], 1)
        keep = dids != own[:, None]
        keep[:, 0] = True
        dids = dids[keep].reshape(N // 64, P)[None].expand(H, -1, -1).to(torch.int32).contiguous()
        for name, sgl in (("two_term", False), ("single_term", True)):
            fn = lambda s=sgl: attention(g.q, g.k, g.v, g.summary, basis, dids, ws, single_av=s, all_pages=True)
            device_warmup(fn, LINE_WARMUP_MS)
            dense_own[name] = time_loop(fn, max(5, iters // 5), stream)

    log(f"dense: sdpa {dense_ms} ms, this kernel {dense_own}")
    log(f"headline call {ms_call:.4f} ms (attention kernel {attn_in_ms:.4f} ms, host enqueue {host_ms:.4f} ms)")

    # the same call in the other arithmetic, staged, and the 216-page window (config 0)
    other = not single
    # after the dense calls above: untimed calls first, as before the headline
    device_warmup(call_step(g, P, other, stream), LINE_WARMUP_MS)
    o_call, o_route_in, o_attn_in, _ = call_timings(g, P, C, other, args.steps, args.warmup // 2, stream)
    st_call, st_route_in, st_attn_in, _ = call_timings(g, P, C, single, args.steps, args.warmup // 2, stream,
                                                        staged=True)
    log(f"other arithmetic call {o_call:.4f} ms")
    x0 = workload.make_call(cfg=0, frames=9)
    g0 = x0.to(dev)
    P0, C0 = x0.pages, x0.pages * 15 // 100
    cfg0 = {}
    # the GPU idled while the inputs were made on the host: untimed calls
    # first, as before the headline
    device_warmup(call_step(g0, P0, single, stream), LINE_WARMUP_MS)
    for name, sgl in (("two_term", False), ("single_term", True)):
        c_ms, c_route, c_attn, _ = call_timings(g0, P0, C0, sgl, args.steps, args.warmup // 2, stream)
        e0, m0 = attn_flop(N, H, D, C0, P0)
        cfg0[name] = {"call_ms": round(c_ms, 4), "attention_kernel_ms": round(c_attn, 4),
                      "route_ms": round(c_route, 4),
                      "attention_frac_of_bf16_peak": round((e0 + m0) / (c_attn * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4)}
    del g0

    extra = {"other_arithmetic": {"single_av": other, "call_ms": round(o_call, 4),
                                  "attention_kernel_ms": round(o_attn_in, 4), "route_ms": round(o_route_in, 4)},
             "staged": {"call_ms": round(st_call, 4), "attention_launches_ms": round(st_attn_in, 4),
                        "note": "the headline call with its attention as exact-page launch + compensation "
                                "launch + merge (the reference's kernel split); per-stage durations in a "
                                "kernel trace"},
             "config0_p216_c32": cfg0}
    if not args.no_extra:
        extra.update(intersection_lines(args, dense_ms, iters))
        log("intersection lines done")
        if not args.no_chunk:
            extra["chunk"] = chunk_line(args)
            log(f"chunk line {extra['chunk']}")

    exact_flop, comp_flop = attn_flop(N, H, D, C, P)
    gather_bytes = H * (N // 64) * C * 64 * D * 2 * 2
    achieved_tflops = (exact_flop + comp_flop) / (attn_in_ms * 1e-3) / 1e12
    gather_gbs = gather_bytes / (attn_in_ms * 1e-3) / 1e9
    o_tflops = (exact_flop + comp_flop) / (o_attn_in * 1e-3) / 1e12
    extra["other_arithmetic"]["roofline_frac"] = round(o_tflops / PEAK_BF16_TFLOPS, 4)

    # HBM bytes per attn_kernel launch (rocprofv3 FETCH_SIZE x 2.0 + WRITE_SIZE x 1.0, factors from a copy
    # kernel), known for the default workload only
    traffic = MEASURED_TRAFFIC.get((P, C, single))

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(x, C, args.cpu_sample_blocks, cfg=1)
        log(f"cpu baseline config 1: {cpu['value']} ms")
        extra["cpu_baseline_other_configs"] = cpu_other_configs(args.cpu_sample_blocks)

    line = {
        "metric": METRIC,
        "value": round(ms_call, 4),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_call, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) Q/K/V with RoPE, k-means page summaries)",
        "config": {"workload": f"full-window base tier: P={P} pages ({64 * P} KV tokens), {C} exact pages "
                               f"per 64-query block, 12 heads x 4608 queries x d128, route + attention, "
                               f"{'single-term' if single else 'two-term (reference)'} bf16 P.V",
                   "tier": "base", "pages": P, "exact_pages": C, "heads": H, "queries": N, "head_dim": D,
                   "single_av": single},
        "host_enqueue_ms_per_call": round(host_ms, 4),
        "device_warmup": {"ms": args.device_warmup_ms, "untimed_calls": warm_calls},
        "breakdown_ms": {"route_and_rep_operands": round(route_in_ms, 4), "attention_kernel": round(attn_in_ms, 4),
                         "route_back_to_back": round(route_ms, 4),
                         "attention_back_to_back_two_term": round(attn_ms["two_term"], 4),
                         "attention_back_to_back_single_term": round(attn_ms["single_term"], 4)},
        "dense_sdpa_ms": None if dense_ms is None else round(dense_ms, 4),
        "ratio_vs_dense": None if dense_ms is None else round(ms_call / dense_ms, 4),
        "dense_this_kernel_ms": {k: round(v, 4) for k, v in dense_own.items()},
        "ratio_vs_dense_this_kernel": None if not dense_own else
        round(ms_call / dense_own["single_term" if single else "two_term"], 4),
        "roofline": {"bound": "mfma", "achieved": round(achieved_tflops, 2), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved_tflops / PEAK_BF16_TFLOPS, 4), "traffic": traffic,
                     "kernel": "attn_kernel (exact + compensation + merge)",
                     "algorithmic_gflop": round((exact_flop + comp_flop) / 1e9, 2),
                     "hbm_GBps": None if traffic is None else round(traffic / (attn_in_ms * 1e-3) / 1e9, 1),
                     "hbm_frac_of_peak": None if traffic is None else
                     round(traffic / (attn_in_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                     "page_gather_gb": round(gather_bytes / 1e9, 3),
                     "page_gather_GBps_from_l2": round(gather_gbs, 1)},
        "extra": extra,
        "cpu_baseline": cpu,
        "input_gen_s": round(gen_s, 2),
    }
    print(json.dumps(line), flush=True)


def intersection_lines(args, dense_ms, iters):
    """The intersection tier (per-head A/B quotas, layer 3 step 0 of a seeded
    table) and the same call with Full_Pset on heads {3,4,9} plus the
    current-page encodings."""
    import torch
    from streaming_sparse_amd import pset, summary, workload
    from streaming_sparse_amd.attention import Workspace
    from streaming_sparse_amd.legacy_components import REP_OP_ELEMS, attention, rep_tiles
    from streaming_sparse_amd.route import route

    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev)
    x = workload.make_call(cfg=2, frames=args.frames)
    g = x.to(dev)
    P = x.pages
    tab = workload.quota_table(2)
    a = tab[0, 3, :, 0]
    n = int(tab[0, 3, 0].sum())
    ac = a.to(dev)
    basis = g.basis.to(torch.bfloat16).contiguous()
    ws = Workspace()
    reader = pset.Reader(workload.reader_weights(), dev)
    enc = pset.encode(g.summary, basis, reader)
    init = workload.kmeans_init(12, 72, torch.Generator().manual_seed(workload.seed_for(2, 3, 0, 9))).to(
        device=dev, dtype=torch.int32)
    recompute = lambda: summary.build(g.k, g.v, basis, init, g.summary, P - 72, 72)

    ops = ws.tensor('call_rep_ops', (12, rep_tiles(P), REP_OP_ELEMS), dev, torch.bfloat16)

    def plain(single=None):
        ids, _, _, _ = route(g.q, g.summary, g.theta, tier='intersection', current_slots=ac, n=n, workspace=ws,
                             want_mask=False, rep_out=ops)
        return attention(g.q, g.k, g.v, g.summary, basis, ids, ws, rep_ops=ops, single_av=single)

    def corrected():
        recompute()
        pset.encode(g.summary, basis, reader, out=enc, first=P - 72, pages=72)
        ids, _, _, _ = route(g.q, g.summary, g.theta, tier='intersection', current_slots=ac, n=n, workspace=ws,
                             full_pset=PSET_HEADS, encoding=enc, reader=reader, rep_out=ops)
        return attention(g.q, g.k, g.v, g.summary, basis, ids, ws, rep_ops=ops)

    out = {}
    # the GPU idled while the inputs were made on the host: untimed calls
    # first, as before the headline
    device_warmup(plain, LINE_WARMUP_MS)
    for name, fn in (("intersection", plain), ("intersection_single_term", lambda: plain(True)),
                     ("intersection_full_pset", corrected)):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        out[name + "_ms"] = round(time_loop(fn, iters, stream), 4)
    out["intersection_exact_pages"] = 24 + n
    out["intersection_current_quota_A"] = a.tolist()
    out["ratio_intersection_vs_dense"] = None if dense_ms is None else round(out["intersection_ms"] / dense_ms, 4)
    out["ratio_full_pset_vs_dense"] = None if dense_ms is None else \
        round(out["intersection_full_pset_ms"] / dense_ms, 4)
    lse = torch.empty(12, 72, 16, device=dev)
    route_i = lambda: route(g.q, g.summary, g.theta, tier='intersection', current_slots=ac, n=n, workspace=ws,
                            want_mask=True, lse_out=lse)
    out["route_intersection_ms"] = round(time_loop(route_i, iters, stream), 4)
    ids, mask, risk, _ = route_i()
    out["pset_correction_ms"] = round(time_loop(
        lambda: pset.correct(g.q, g.summary, enc, reader, risk, lse, mask, ids, None, PSET_HEADS, ws), iters, stream), 4)
    out["summary_current_72x12_ms"] = round(time_loop(recompute, iters, stream), 4)
    out["encode_current_72x12_ms"] = round(time_loop(
        lambda: pset.encode(g.summary, basis, reader, out=enc, first=P - 72, pages=72), iters, stream), 4)
    out["full_pset_heads"] = list(PSET_HEADS)
    return out


def chunk_line(args):
    """Total attention-path time of one 3-frame chunk of a 30-layer stack on
    the rolling 432-page window: 4 denoise steps (layer 0 dense, layers 1-29
    current-page summaries + intersection route + attention, Full_Pset on
    layers {3,4,5,8,14,17,27} x heads {3,4,9} at step 0) and the clean step
    (every layer dense, then the commit of the chunk's 72 pages, summaries
    and encodings into the ring), plus the anchor rebase.  Chunks 0-5 fill
    the window untimed; chunk 6 is the first with a full window after the
    ring wrapped and the anchor was rebased, and is the one timed.  Beside it
    the same chunk's calls fully dense (this library's kernel with every page
    exact, and torch scaled_dot_product_attention)."""
    import torch
    from streaming_sparse_amd.runtime import StreamConfig, StreamRuntime
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev)
    t0 = time.time()
    rt = StreamRuntime(StreamConfig(history_pages=24 * args.frames - 72), dev)
    for c in range(6):
        rt.run_chunk(rt.chunk_inputs())
        torch.cuda.synchronize()
    setup_s = time.time() - t0
    inputs = rt.chunk_inputs()
    dense_kernel_ms = time_loop(lambda: rt.run_dense_chunk(inputs, False), 1, stream)
    dense_sdpa_ms = time_loop(lambda: rt.run_dense_chunk(inputs, True), 1, stream)
    calls = rt.calls_per_chunk()
    from streaming_sparse_amd import group
    grouping_ms = time_loop(lambda: group.order(inputs.clean_k, inputs.clean_v, rt.group_weights,
                                                page_dst=rt.page_dst, workspace=rt.ws), 3, stream)
    torch.cuda.synchronize()
    chunk_ms = time_loop(lambda: rt.run_chunk(inputs), 1, stream)
    return {"workload": f"30 layers x (4 denoise steps + clean commit), rolling {rt.cap}-page window, 12 heads; "
                        f"chunk 6 (window full, ring wrapped, anchor rebased)",
            "calls": calls, "chunk_ms": round(chunk_ms, 3),
            "dense_chunk_ms_this_kernel": round(dense_kernel_ms, 3),
            "dense_chunk_ms_sdpa": round(dense_sdpa_ms, 3),
            "ratio_vs_dense_sdpa": round(chunk_ms / dense_sdpa_ms, 4),
            "commit_grouping_30_layers_ms": round(grouping_ms, 3), "setup_s": round(setup_s, 2)}


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return ""


def cpu_baseline(x, count, blocks, cfg, tier='base', quota=None, pset_heads=None):
    """CPU oracle on a bounded sample of one call: the router over the whole
    call (all 72 blocks x 12 heads, it is cheap), the tier's selection, for
    config 3 the current pages' summaries and encodings and the Full_Pset
    correction of the scoped heads, and the attention over `blocks` query
    blocks scaled to the full 72; median of 3 after 1 warm-up."""
    import torch
    from oracle import reference as ref
    from oracle import pset as opset
    from oracle import summary as osum
    from streaming_sparse_amd import workload
    cores = os.cpu_count() or 1
    torch.set_num_threads(cores)
    tiles = list(range(0, 72, max(1, 72 // blocks)))[:blocks]
    P = x.pages
    if pset_heads:
        w = workload.reader_weights()
        s = x.summary
        enc = opset.encode(s.keys, s.mean, s.detail, s.stats, x.basis, w)
        kp = x.k[0].transpose(0, 1).reshape(12, P, 64, 128)[:, P - 72:]
        vp = x.v[0].transpose(0, 1).reshape(12, P, 64, 128)[:, P - 72:]
        init = workload.kmeans_init(12, 72, torch.Generator().manual_seed(workload.seed_for(cfg, 3, 0, 9)))

    def run():
        t0 = time.perf_counter()
        if pset_heads:
            cs = osum.summaries(kp, vp, x.basis, init)
            opset.encode(cs['keys'], cs['mean'], cs['detail'], cs['stats'], x.basis, w)
        pr = ref.probes(x.q)
        z = ref.route_logits(pr, x.summary.keys)
        r = ref.risk(pr, z, x.summary.stats, x.theta)
        if tier == 'base':
            ids = ref.select_base(r, x.own, count)
        else:
            a, n = quota
            mask = ref.quota_mask(r, x.own, a, n)
            if pset_heads:
                mask, _, _ = opset.correct(pr, z, r, mask, x.own, enc, w['wq'], list(pset_heads))
            ids = ref.lut(r, mask, x.own, 24 + n)
        t1 = time.perf_counter()
        ref.selected_attention(x.q, x.k, x.v, x.summary, x.basis, ids, tiles=tiles)
        t2 = time.perf_counter()
        return t1 - t0, t2 - t1

    run()
    times = sorted((run() for _ in range(3)), key=lambda a: a[0] + a[1])
    route_s, attn_s = times[1]
    total_ms = (route_s + attn_s * 72 / len(tiles)) * 1e3
    what = {'base': "base-tier route", 'intersection': "intersection route"}[tier]
    if pset_heads:
        what = f"current summaries + encodings, intersection route + Full_Pset on heads {list(pset_heads)}"
    return {"value": round(total_ms, 1), "unit": "ms", "cores": cores, "kind": "port",
            "sample": f"config {cfg}: oracle {what} over the full call + attention over {len(tiles)} of 72 "
                      f"query blocks (x12 heads), scaled to 72 blocks; median of 3 after 1 warm-up; "
                      f"cpu: {_cpu_model()}"}


def cpu_other_configs(blocks):
    """cpu_baseline of configs 0 (216 pages, base), 2 (432 pages,
    intersection) and 3 (config 2 plus Full_Pset on heads {3,4,9})."""
    from streaming_sparse_amd import workload
    out = {}
    x0 = workload.make_call(cfg=0, frames=9)
    out["config0"] = cpu_baseline(x0, x0.pages * 15 // 100, blocks, 0)
    log(f"cpu baseline config 0: {out['config0']['value']} ms")
    del x0
    x2 = workload.make_call(cfg=2, frames=18)
    tab = workload.quota_table(2)
    quota = (tab[0, 3, :, 0], int(tab[0, 3, 0].sum()))
    out["config2"] = cpu_baseline(x2, None, blocks, 2, tier='intersection', quota=quota)
    log(f"cpu baseline config 2: {out['config2']['value']} ms")
    out["config3"] = cpu_baseline(x2, None, blocks, 3, tier='intersection', quota=quota, pset_heads=PSET_HEADS)
    return out


if __name__ == "__main__":
    main()

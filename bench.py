"""Benchmark of the MTP verify MoE on one MI355X.

A step is one routed MXFP4 MoE layer forward (prep, gate_up, down, combine) at real dims
(H=4096, I=1024, 512 experts, top-10) over one batch of synthetic rows. The headline workload is
config 3's widest verify width, M = B*(k+1) = 48*4 = 192 rows with Zipf(1.1) expert popularity
and 5% zeroed routing weights; M=1 (config 2) and M=32 (config 3, B=8) are reported beside it.

Weights rotate over --layers distinct copies (3.4 GB each) so no step is served from the
256 MB last-level cache. `value` = algorithmic HBM bytes of the routed layer / measured time:
D_live * 6,684,672 + 2 * M * 4096 * 2, where D_live counts experts with a nonzero-weight
assignment (the reference's definition, bench_moe_bw.py:29, :76-77).

More legs are reported beside `value` in the same JSON line:
- "accept" (config 4): greedy acceptance (argmax over [48, 4, 248320] bf16 target logits, then
  the accept kernel with every rollback index) and sampling-mode acceptance at T = 0.7
  (rejection sampling with the target and draft logits, then the same index kernel), as us per
  call and GB/s over one read of the logits they take;
- "dense_moe": the real checkpoint's MTP-layer MoE, whose 512 experts are bf16 (12.9 GB), at the
  draft step's 48 rows with Zipf(1.1) and uniform routing, as us per call and GB/s over
  D_live * 25,165,824 + 2 * 48 * 4096 * 2 bytes;
- "mtp_round" (config 5): full speculative rounds on the reduced-depth real-dims model (3
  DeltaNet + 1 gated GQA layer, MXFP4 MoE on every layer, 1 MTP layer; B = 48, k = 3, 8192
  tokens of synthetic context per sequence), as ms per round and committed tok/s. The weights
  are random, so the draft rarely agrees with the target and a round commits about one token
  per lane.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--layers L] [--no-accept] [--no-mtp]
                       [--no-dense]
Prints one JSON line.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
PKG = ROOT / "qwen3.5-397b-mi300a-bespoke-vibesys-20260920_amd"
for _p in (str(ROOT), str(PKG)):
    if _p not in sys.path:
        sys.path.insert(0, _p)

H, I, E, TOP_K = 4096, 1024, 512, 10
EXPERT_BYTES = 4_194_304 + 262_144 + 2_097_152 + 131_072  # gate_up + scales + down + scales
GATE_UP_BYTES = 4_194_304 + 262_144
PEAK_GBS = 8000.0
METRIC = json.loads((ROOT / "BASELINE.json").read_text())["metric"]
WORKLOAD_TEXT = {
    "M192": "C3 routed MXFP4 MoE verify layer, M=192 (B=48, k=3), Zipf(1.1) top-10 of 512, "
            "H=4096 I=1024, 5% zero weights",
    "M32": "C3 routed MXFP4 MoE verify layer, M=32 (B=8, k=3), Zipf(1.1) top-10 of 512, "
           "H=4096 I=1024, 5% zero weights",
    "M1": "C2 routed MXFP4 MoE decode layer, M=1, router softmax top-10 of 512, H=4096 I=1024",
}


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def zipf_routing(tokens, seed, zero_frac=0.05, s=1.1):
    rng = np.random.default_rng(seed)
    logp = -s * np.log(np.arange(1, E + 1, dtype=np.float64))
    perm = rng.permutation(E)
    g = rng.gumbel(size=(tokens, E)) + logp[None, :]
    picks = perm[np.argsort(-g, axis=1)[:, :TOP_K]]
    z = rng.standard_normal((tokens, TOP_K))
    w = np.exp(z - z.max(-1, keepdims=True))
    w = (w / w.sum(-1, keepdims=True)).astype(np.float32)
    w[rng.random(w.shape) < zero_frac] = 0.0
    return picks.astype(np.int32).reshape(-1), w.reshape(-1)


def d_live(a_e, a_w):
    return int(np.unique(a_e[a_w != 0]).size)


def layer_bytes(m, dl):
    return dl * EXPERT_BYTES + 2 * m * H * 2


def gate_up_kernel(m: int) -> str:
    """The gate_up kernel the unit path launches at m rows (8-wave workgroups from 96 rows)."""
    return "k_moe_gate_up_lds<4, 8>" if m >= 96 else "k_moe_gate_up_lds<4, 4>"


def profiled_traffic(kernel: str) -> float | None:
    """HBM bytes per launch of `kernel` (fetched + written, calibrated) from the committed
    rocprofv3 PMC summary profiles/moe_kernels_mi355x.md, or None if it has no row for it."""
    path = ROOT / "profiles" / "moe_kernels_mi355x.md"
    if not path.exists():
        return None
    text = path.read_text()
    pmc = text.find("## HBM traffic per dispatch")
    if pmc < 0:
        return None
    # PMC rows: kernel | grid | dispatches | FETCH_SIZE KiB | WRITE_SIZE KiB | fetched GB | written GB
    for line in text[pmc:].splitlines():
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if len(cells) == 7 and cells[0] == f"`{kernel}`":
            try:
                return (float(cells[5]) + float(cells[6])) * 1e9
            except ValueError:
                return None
    return None


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=40)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--layers", type=int, default=4)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="also run a plain device copy of this many MiB (3 launches) so a PMC "
                         "profile can scale FETCH_SIZE/WRITE_SIZE by a known byte count")
    ap.add_argument("--no-accept", action="store_true", help="skip the acceptance leg")
    ap.add_argument("--no-mtp", action="store_true", help="skip the MTP-round leg")
    ap.add_argument("--no-dense", action="store_true",
                    help="skip the bf16-expert leg (the real checkpoint's MTP-layer MoE)")
    ap.add_argument("--no-full", action="store_true",
                    help="skip the whole-layer leg (router + routed + shared expert, fused against unfused)")
    ap.add_argument("--no-stream", action="store_true",
                    help="skip the streaming-read probe (the HBM read ceiling at the MoE byte counts)")
    ap.add_argument("--workloads", default="M1,M32,M192",
                    help="comma list of M1, M32, M192; `value` is measured on M192 when listed, "
                         "else on the last one listed")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); got --gpus {args.gpus}",
              file=sys.stderr)
        return 2

    import torch

    import __graft_entry__

    __graft_entry__._ensure_built()
    import mxfp4_gemv
    import router_fused

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    L = args.layers
    log(f"allocating {L} layer copies of MXFP4 experts ({L * E * EXPERT_BYTES / 1e9:.1f} GB)")
    layers = []
    for li in range(L):
        g = torch.Generator(dev).manual_seed(1000 + li)
        layers.append({
            "gate_up": torch.randint(0, 256, (E, 2 * I, H // 2), dtype=torch.uint8, device=dev, generator=g),
            "gate_up_scale": torch.randint(118, 131, (E, 2 * I, H // 32), dtype=torch.uint8, device=dev, generator=g),
            "down": torch.randint(0, 256, (E, H, I // 2), dtype=torch.uint8, device=dev, generator=g),
            "down_scale": torch.randint(118, 131, (E, H, I // 32), dtype=torch.uint8, device=dev, generator=g),
        })  # fmt: skip

    def make_inputs(m, li, kind):
        g = torch.Generator(dev).manual_seed(7 * m + li)
        x = torch.randn(m, H, device=dev, generator=g).to(torch.bfloat16)
        if kind == "router":  # config 2: N(0,1) bf16 router logits, softmax top-10 renormalised
            logits = torch.randn(m, E, device=dev, generator=g).to(torch.bfloat16)
            w, i = router_fused.route(logits, E, TOP_K, index_dtype=torch.int32)
            a_e, a_w = i.reshape(-1).contiguous(), w.reshape(-1).contiguous()
            ne, nw = a_e.cpu().numpy(), a_w.cpu().numpy()
        else:
            ne, nw = zipf_routing(m, seed=100 * m + li)
            a_e, a_w = torch.from_numpy(ne).to(dev), torch.from_numpy(nw).to(dev)
        return x, a_e, a_w, d_live(ne, nw)

    if args.calibrate_copy:
        n = args.calibrate_copy << 20
        src_c = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
        dst_c = torch.empty_like(src_c)
        for _ in range(3):
            dst_c.copy_(src_c)
        torch.cuda.synchronize()
        log(f"calibration copy: 3 x {args.calibrate_copy} MiB")
        del src_c, dst_c

    results = {}
    wanted = args.workloads.split(",")
    rows_of = {"M1": 1, "M32": 32, "M192": 192}
    if not wanted or any(w not in rows_of for w in wanted):
        print(f"--workloads takes a comma list of {sorted(rows_of)}", file=sys.stderr)
        return 2
    head = "M192" if "M192" in wanted else wanted[-1]
    head_m = rows_of[head]
    for name, m, kind in (("M1", 1, "router"), ("M32", 32, "zipf"), ("M192", 192, "zipf")):
        if name not in wanted:
            continue
        runner = mxfp4_gemv.MoeLayerRunner(m, TOP_K, E, I, H, dev)
        ins = [make_inputs(m, li, kind) for li in range(L)]
        outs = [torch.empty(m, H, dtype=torch.bfloat16, device=dev) for _ in range(L)]
        dls = [d for *_, d in ins]
        for w in range(args.warmup):
            li = w % L
            runner.run(ins[li][0], layers[li], ins[li][1], ins[li][2], (0, E), outs[li])
        torch.cuda.synchronize()
        # graph replay: one capture holds GRAPH_ROUNDS steps on every layer copy in turn (24
        # layer steps, as a round's graph holds all of its layers; a 4-step graph adds the
        # graph launch gap to every fourth step)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(GRAPH_ROUNDS):
                for li in range(L):
                    runner.run(ins[li][0], layers[li], ins[li][1], ins[li][2], (0, E), outs[li])
        for _ in range(3):
            graph.replay()
        torch.cuda.synchronize()
        reps = max(3, args.steps // (L * GRAPH_ROUNDS))
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            graph.replay()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / (reps * L * GRAPH_ROUNDS)
        byts = float(np.mean([layer_bytes(m, d) for d in dls]))
        results[name] = {"us_per_layer": us, "gbs": byts / us / 1e3, "d_live_mean": float(np.mean(dls)),
                         "graph": True}
        log(f"{name}: {us:.1f} us/layer (graph replay), {byts / us / 1e3:.0f} GB/s, D_live~{np.mean(dls):.0f}")
        results[name]["_state"] = (runner, ins, outs, dls)

    # timed region for `value`: K eager steps of the headline workload, with nothing between the
    # two events but the steps (the reference times its layer as a whole, `bench_moe_bw.py`)
    runner, ins, outs, dls = results[head].pop("_state")
    for k in results:
        results[k].pop("_state", None)
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    wall0 = time.perf_counter()
    t0.record()
    for s in range(args.steps):
        li = s % L
        runner.run(ins[li][0], layers[li], ins[li][1], ins[li][2], (0, E), outs[li])
    t1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    ms = t0.elapsed_time(t1) / args.steps
    # the same K steps again with HIP events around gate_up and down on the launch stream: the
    # roofline kernel's live duration. The event records add about 13 us to a step, which is
    # why they stay out of the region `value` is timed on.
    ev = {k: [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(args.steps)] for k in ("gate_up", "down")}
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for s in range(args.steps):
        li = s % L
        runner.run(ins[li][0], layers[li], ins[li][1], ins[li][2], (0, E), outs[li],
                   events={"gate_up": ev["gate_up"][s], "down": ev["down"][s]})
    e1.record()
    torch.cuda.synchronize()
    ms_events = e0.elapsed_time(e1) / args.steps
    gu_ms = float(np.mean([a.elapsed_time(b) for a, b in ev["gate_up"]]))
    dn_ms = float(np.mean([a.elapsed_time(b) for a, b in ev["down"]]))
    step_bytes = [layer_bytes(head_m, dls[s % L]) for s in range(args.steps)]
    value = float(np.mean(step_bytes)) / (ms * 1e-3) / 1e9
    gu_bytes = float(np.mean([dls[s % L] * GATE_UP_BYTES + head_m * H * 2 for s in range(args.steps)]))
    gu_gbs = gu_bytes / (gu_ms * 1e-3) / 1e9
    log(f"eager {head}: {ms * 1e3:.1f} us/step; with per-kernel events {ms_events * 1e3:.1f} us/step, "
        f"gate_up {gu_ms * 1e3:.1f} us ({gu_gbs:.0f} GB/s), down {dn_ms * 1e3:.1f} us, wall {wall:.2f}s")

    cpu = None
    if not args.no_cpu and head == "M192":
        cpu = cpu_baseline(layers[0], ins[0], dls[0], args.cpu_seconds)
    direct = runner.direct
    full_layer = None if args.no_full else full_layer_bench(dev, layers)
    stream = None if args.no_stream else stream_bench(dev)
    del runner, ins, outs, layers
    torch.cuda.empty_cache()
    accept = None if args.no_accept else accept_bench(dev)
    dense_moe = None if args.no_dense else dense_moe_bench(dev)
    mtp_round = None if args.no_mtp else mtp_round_bench(dev)

    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random MXFP4 bytes 0..255, e8m0 scales 118..130, bf16 N(0,1) x)",
        "config": {
            "workload": WORKLOAD_TEXT[head],
            "rows": head_m, "hidden": H, "intermediate": I, "experts": E, "top_k": TOP_K,
            "layer_copies": L,
            "timing": "eager stream, HIP events around the K steps; a second pass of the same K steps "
                      "with events around each kernel gives roofline.avg_us",
        },
        "frac_of_peak": round(value / PEAK_GBS, 4),
        "us_per_layer": {k: round(v["us_per_layer"], 2) for k, v in results.items()},
        "gbs_graph": {k: round(v["gbs"], 1) for k, v in results.items()},
        "d_live": {k: round(v["d_live_mean"], 1) for k, v in results.items()},
        "roofline": {
            "kernel": "k_moe_gate_up_single<1,2,true> (direct)" if direct else gate_up_kernel(head_m),
            "bound": "hbm",
            "achieved": round(gu_gbs, 1),
            "peak": PEAK_GBS,
            "unit": "GB/s",
            "frac": round(gu_gbs / PEAK_GBS, 4),
            "traffic": None if direct else profiled_traffic("mtpk::" + gate_up_kernel(head_m)),
            "traffic_source": "profiles/moe_kernels_mi355x.md (rocprofv3 --pmc FETCH_SIZE, WRITE_SIZE; "
                              "copy-calibrated)",
            "avg_us": round(gu_ms * 1e3, 2),
            "step_us_with_kernel_events": round(ms_events * 1e3, 2),
            "algorithmic_bytes": round(gu_bytes),
        },
        "cpu_baseline": cpu,
        "full_layer": full_layer,
        "stream": stream,
        "accept": accept,
        "dense_moe": dense_moe,
        "mtp_round": mtp_round,
    }
    print(json.dumps(line), flush=True)
    return 0


def full_layer_bench(dev, layers, rows=(1, 48, 192), shared_inter=1024):
    """The whole MoE layer of config 2 (router GEMM, softmax top-10, routed MXFP4 experts, shared
    expert, gated add) at M rows: `fused_moe_layer` (router and shared expert inside the routed
    layer's launches) against the same pieces launched one by one, graph replay over the layer
    copies. Router logits come from random bf16 router weights (N(0, 0.02)), so routing is near
    uniform, not Zipf."""
    import torch

    import dense
    import mxfp4_gemv
    import router_fused

    dense_w = []
    for li in range(len(layers)):
        g = torch.Generator(dev).manual_seed(2000 + li)
        dense_w.append({
            "router_gate": (torch.randn(E + 1, H, device=dev, generator=g) * 0.02).to(torch.bfloat16),
            "shared_gate_up": (torch.randn(2 * shared_inter, H, device=dev, generator=g) * 0.02).to(torch.bfloat16),
            "shared_down": (torch.randn(H, shared_inter, device=dev, generator=g) * 0.02).to(torch.bfloat16),
        })  # fmt: skip

    def unfused(h, ex, w, out):
        routing = dense.linear(h, w["router_gate"])
        top_w, top_i = router_fused.route(routing, E, TOP_K, index_dtype=torch.int32)
        shared = dense.linear(dense.silu_linear(h, w["shared_gate_up"]), w["shared_down"])
        mxfp4_gemv.fused_moe(h, ex, (top_i.reshape(-1), top_w.reshape(-1)), TOP_K, (0, E), out=out,
                             shared=shared, shared_gate=routing[:, E:])

    def fused(h, ex, w, out):
        mxfp4_gemv.fused_moe_layer(h, w["router_gate"], w["shared_gate_up"], w["shared_down"], ex,
                                   TOP_K, (0, E), out=out)

    res = {"workload": "whole MoE layer (router 513 x 4096, top-10 of 512 MXFP4 experts, shared "
                       "expert 1024, gated add), bf16, random router weights",
           "timing": f"HIP-graph replay over {len(layers)} layer copies"}
    for m in rows:
        hs = [torch.randn(m, H, device=dev, generator=torch.Generator(dev).manual_seed(li)).to(torch.bfloat16)
              for li in range(len(layers))]
        outs = [torch.empty(m, H, dtype=torch.bfloat16, device=dev) for _ in layers]
        r = {}
        for name, fn in (("unfused_us", unfused), ("fused_us", fused)):
            def call(c, fn=fn):
                fn(hs[c], layers[c], dense_w[c], outs[c])
            r[name] = round(_time_graph(call, len(layers), GRAPH_ROUNDS * len(layers)), 2)
        res[f"M{m}"] = r
        log(f"full layer M{m}: unfused {r['unfused_us']:.1f} us, fused {r['fused_us']:.1f} us")
    del dense_w
    return res


def _time_graph(fn, copies, calls, replays=5):
    """us per call of `fn(c)` captured `calls` times (c cycling over `copies`) in one HIP graph."""
    import torch

    for c in range(copies):
        fn(c)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(calls):
            fn(i % copies)
    graph.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(replays):
        graph.replay()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) * 1e3 / (replays * calls)  # us


def _time_calls(fn, reps):
    import torch

    for _ in range(3):
        fn()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        fn()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) * 1e3 / reps  # us


GRAPH_ROUNDS = 6  # passes over the layer copies per captured graph (per-layer timing)

STREAM_SIZES = {
    "M1_down": 10 * (2_097_152 + 131_072),
    "M1_gate_up": 10 * GATE_UP_BYTES,
    "M1_layer": 10 * EXPERT_BYTES,
    "M32_layer": 134 * EXPERT_BYTES,
    "M192_layer": 351 * EXPERT_BYTES,
}


def stream_bench(dev, calls=24, region_gib=6):
    """The HBM read ceiling at the MoE's byte counts: `mtpk_probe_stream` (16-byte loads, no
    stores) reads a window of each size per launch, successive launches taking successive
    windows of a 6 GiB buffer, so no launch is served by the last-level cache; graph replay,
    best over grids of 256..4096 workgroups and 8 or 16 loads in flight.
    `M1_pair_us` chains a gate_up-sized and a down-sized read as two dependent launches, the
    shape of the M = 1 layer."""
    import torch

    import _mtpk

    lib = _mtpk.lib()
    sink = torch.zeros(1024, dtype=torch.int32, device=dev)
    st = lambda: _mtpk.stream_of(dev)  # noqa: E731
    region = torch.zeros(region_gib << 30, dtype=torch.uint8, device=dev)
    span = [(region.data_ptr(), region.numel())]

    def windows(size):
        out = []
        for base, n in span:
            off = 0
            while off + size <= n:
                out.append(base + off)
                off += (size + 4095) // 4096 * 4096
        return out

    def launch(ptr, size, grid, u):
        _mtpk.check(lib.mtpk_probe_stream(ptr, size, grid, u, sink.data_ptr(), st()), "mtpk_probe_stream")

    res = {}
    for name, size in STREAM_SIZES.items():
        wins = windows(size)
        best = None
        for grid in (256, 512, 1024, 2048, 4096):
            for u in (8, 16):
                n = min(calls, len(wins))
                us = _time_graph(lambda i, g=grid, u=u: launch(wins[i], size, g, u), n, n)
                if best is None or us < best[0]:
                    best = (us, grid, u)
        us, grid, u = best
        res[name] = {"bytes": size, "us": round(us, 2), "gbs": round(size / us / 1e3, 1),
                     "grid": grid, "loads_in_flight": u}
        log(f"stream {name}: {size / 1e6:.1f} MB in {us:.2f} us = {size / us / 1e3:.0f} GB/s "
            f"(grid {grid}, {u} loads in flight)")
    gu, dn = STREAM_SIZES["M1_gate_up"], STREAM_SIZES["M1_down"]
    wg, wd = windows(gu), windows(dn)
    cg, cd = res["M1_gate_up"], res["M1_down"]

    def pair(i):
        launch(wg[i], gu, cg["grid"], cg["loads_in_flight"])
        launch(wd[-1 - i], dn, cd["grid"], cd["loads_in_flight"])

    res["M1_pair_us"] = round(_time_graph(pair, min(calls, len(wg)), min(calls, len(wg))), 2)
    log(f"stream: gate_up-sized then down-sized read, two dependent launches: {res['M1_pair_us']:.2f} us")
    res["probe"] = "mtpk_probe_stream (16-byte buffer loads, grid-stride, no stores)"
    del region
    torch.cuda.empty_cache()
    return res


def accept_bench(dev, b=48, k=3, vocab=248320, temperature=0.7):
    """Config 4: greedy and rejection-sampling acceptance with the round's rollback indices."""
    import torch

    import graph_mtp
    import mtp

    t = k + 1
    g = torch.Generator(dev).manual_seed(44)
    target = (torch.randn(b, t, vocab, device=dev, generator=g) * 3).to(torch.bfloat16)
    draft = (target[:, :k].float() + torch.randn(b, k, vocab, device=dev, generator=g)).to(torch.bfloat16)
    draft_tok = mtp.sample_rows(draft, temperature, torch.rand(b * k, device=dev, generator=g)).view(b, k)
    u_acc = torch.rand(b, k, device=dev, generator=g)
    u_smp = torch.rand(b, device=dev, generator=g)
    active = torch.ones(b, dtype=torch.bool, device=dev)
    pos = torch.full((b,), 8188, dtype=torch.long, device=dev)
    budget = torch.full((b,), 1 << 20, dtype=torch.long, device=dev)
    stops = torch.full((b, mtp.MAX_STOP_IDS), -1, dtype=torch.long, device=dev)
    ws = graph_mtp.rejection_workspace(b, k, vocab, dev)

    # Three copies of the logits (500 MB) rotate so the 256 MB last-level cache does not serve
    # repeats; draft tokens are the same for every copy.
    targets = [target] + [target.clone() for _ in range(2)]
    drafts = [draft] + [draft.clone() for _ in range(2)]

    def greedy(c=0):
        # two launches: the argmax chunk keys, then acceptance finishing the argmax
        sa = torch.empty(b, t, dtype=torch.long, device=dev)
        return graph_mtp.greedy_accept(sa, draft_tok, active, pos, budget, stops, 3,
                                       keys=mtp.argmax_keys(targets[c].view(b * t, vocab)))

    def greedy_3(c=0):
        sa = mtp.argmax_rows(targets[c])
        return graph_mtp.greedy_accept(sa, draft_tok, active, pos, budget, stops, 3)

    def rejection(c=0):
        # the sampler's launches also write every acceptance output (mtpk_rejection_accept)
        return graph_mtp.rejection_accept(targets[c], drafts[c], draft_tok, u_acc, u_smp,
                                          temperature, active, pos, budget, stops, 3,
                                          workspace=ws)[0]

    def rejection_2(c=0):
        _, _, em, _ = graph_mtp.rejection_sample(targets[c], drafts[c], draft_tok, u_acc, u_smp,
                                                 temperature, workspace=ws)
        return graph_mtp.greedy_accept(em, draft_tok, active, pos, budget, stops, 3)

    us_g = _time_graph(greedy, 3, 30)
    us_g3 = _time_graph(greedy_3, 3, 30)
    us_r = _time_graph(rejection, 3, 30)
    us_r2 = _time_graph(rejection_2, 3, 30)
    eager_g = _time_calls(lambda: greedy(0), 50)
    eager_r = _time_calls(lambda: rejection(0), 50)
    acc_g = float(greedy().accept_len.float().mean())
    if not torch.equal(greedy().accept_len, greedy_3().accept_len):
        raise RuntimeError("greedy acceptance: the two-launch and three-launch paths differ")
    acc_r = float(rejection().accept_len.float().mean())
    if not torch.equal(rejection().bonus, rejection_2().bonus):
        raise RuntimeError("rejection acceptance: the fused and the two-call paths differ")
    logit_bytes = b * t * vocab * 2
    log(f"accept: greedy {us_g:.1f} us (argmax finished in a third launch {us_g3:.1f}), rejection {us_r:.1f} us (sample then accept as two calls {us_r2:.1f}; T={temperature}; graph replay, "
        f"eager calls {eager_g:.1f} / {eager_r:.1f} us), mean accept {acc_g:.2f} / {acc_r:.2f}")
    return {
        "workload": f"C4 acceptance, target/draft bf16 [{b}, {t}, {vocab}], T={temperature}",
        "timing": "HIP-graph replay of 30 calls over 3 rotating logit copies",
        "greedy_us": round(us_g, 2),
        "greedy_gbs": round(logit_bytes / us_g / 1e3, 1),
        "greedy_us_three_launches": round(us_g3, 2),
        "rejection_us": round(us_r, 2),
        "rejection_us_sample_then_accept": round(us_r2, 2),
        "rejection_gbs": round((logit_bytes + b * k * vocab * 2) / us_r / 1e3, 1),
        "greedy_us_eager": round(eager_g, 2),
        "rejection_us_eager": round(eager_r, 2),
        "mean_accept_greedy": round(acc_g, 3),
        "mean_accept_rejection": round(acc_r, 3),
    }


DENSE_EXPERT_BYTES = (2 * I * H + H * I) * 2  # bf16 gate_up + down of one expert


def uniform_routing(tokens, seed):
    """Top-10 of 512 uniformly without replacement, softmax weights of N(0,1) logits."""
    rng = np.random.default_rng(seed)
    picks = np.stack([rng.permutation(E)[:TOP_K] for _ in range(tokens)])
    z = rng.standard_normal((tokens, TOP_K))
    w = np.exp(z - z.max(-1, keepdims=True))
    return picks.astype(np.int32).reshape(-1), (w / w.sum(-1, keepdims=True)).astype(np.float32).reshape(-1)


def dense_moe_bench(dev, b=48, copies=2, calls=20):
    """The real checkpoint's MTP-layer MoE: 512 bf16 experts (12.9 GB a copy) at the draft
    step's B = 48 rows, top-10, Zipf(1.1) and uniform routing, timed by graph replay over
    rotating copies so repeats are not served from the last-level cache."""
    import torch

    import mtp_dense_moe as dm

    g = torch.Generator(device=dev).manual_seed(17)
    layers = []
    for _ in range(copies):
        ex = {"gate_up": torch.empty(E, 2 * I, H, dtype=torch.bfloat16, device=dev),
              "down": torch.empty(E, H, I, dtype=torch.bfloat16, device=dev)}
        for ten in ex.values():
            for e0 in range(0, E, 64):
                ten[e0 : e0 + 64] = torch.randn(ten[e0 : e0 + 64].shape, generator=g, device=dev) * 0.02
        layers.append(ex)
    x = (torch.randn(b, H, generator=g, device=dev)).to(torch.bfloat16)
    res = {"workload": f"MTP-layer routed bf16 experts, B={b}, top-{TOP_K} of {E}, H={H} I={I}",
           "timing": f"HIP-graph replay of {calls} calls over {copies} rotating expert copies"}
    for name, (a_e, a_w) in (("zipf", zipf_routing(b, seed=71)), ("uniform", uniform_routing(b, seed=72))):
        route = (torch.from_numpy(a_e).view(b, TOP_K).to(dev), torch.from_numpy(a_w).view(b, TOP_K).to(dev))
        scratch = dm.grouped_scratch(b, TOP_K, E, H, dev, intermediate=I)
        inter = torch.empty(b * TOP_K, I, dtype=torch.bfloat16, device=dev)
        out = torch.empty(b, H, dtype=torch.bfloat16, device=dev)

        def call(c):
            dm.grouped_moe(x, layers[c], route, TOP_K, (0, E), inter, out, scratch)

        us = _time_graph(call, copies, calls)
        dl = d_live(a_e, a_w)
        byts = dl * DENSE_EXPERT_BYTES + 2 * b * H * 2
        res[name] = {"us": round(us, 1), "d_live": dl, "gbs": round(byts / us / 1e3, 1),
                     "frac_of_peak": round(byts / us / 1e3 / PEAK_GBS, 4)}
        log(f"dense MoE ({name}): {us:.1f} us, D_live {dl}, {byts / us / 1e3:.0f} GB/s")
    del layers
    torch.cuda.empty_cache()
    return res


def mtp_round_bench(dev, b=48, k=3, ctx=8192, rounds=8):
    """Config 5: speculative rounds (draft k steps, verify B*(k+1) rows, accept, commit)."""
    import torch

    import blas_tune
    import graph_mtp
    import mtp
    import verify_model as vm

    t0 = time.perf_counter()
    model = vm.Model(vm.verify_cfg(), dev, torch.bfloat16, lanes=b, max_seq=ctx + 64, seed=0,
                     expert_mode="bytes", moe_rows=b * (k + 1))
    mtp.attach(model, k=k, seed=1, expert_mode="bytes")
    # boot: capture the B-row bucket and validate the replay against the eager round
    # boot also tunes the round's library GEMMs before the capture (blas_tune)
    runner = graph_mtp.GraphMTPRunner(model, buckets=[b], tune_blas=True)
    t_boot = time.perf_counter()
    validated = runner.prepare()
    tuned = sorted(blas_tune.tuned_shapes())
    log(f"mtp round: captured bucket {b} in {time.perf_counter() - t_boot:.1f}s, validation "
        f"{'passed' if validated else 'FAILED (eager rounds)'}, tuned library GEMMs (m, n, k) {tuned}")
    start = ctx - 32
    for lane in range(b):
        model.blocks.grow(lane, start)
    g = torch.Generator(device=dev).manual_seed(3)
    for ty, pool in zip(model.cfg.layer_types, model.pool):
        if ty == vm.ATTN:
            pool["k"].normal_(generator=g)
            pool["v"].normal_(generator=g)
        else:
            pool["conv"].normal_(generator=g)
            pool["rec"].normal_(0, 0.05, generator=g)
    model.mtp.pool["k"].normal_(generator=g)
    model.mtp.pool["v"].normal_(generator=g)
    model.hidden_cache.normal_(generator=g)
    toks = torch.randint(0, model.cfg.vocab, (b,), generator=torch.Generator().manual_seed(4)).tolist()
    pos = [start] * b
    torch.cuda.synchronize()
    log(f"mtp round: model ready in {time.perf_counter() - t0:.1f}s, "
        f"{torch.cuda.memory_allocated() / 1e9:.1f} GB allocated")

    def one_round():
        got = runner.speculative_decode(list(range(b)), toks, pos)
        n = 0
        for j, c in enumerate(got):
            pos[j] += len(c)
            toks[j] = c[-1]
            n += len(c)
        return n

    for _ in range(2):
        one_round()
    torch.cuda.synchronize()
    w0 = time.perf_counter()
    committed = sum(one_round() for _ in range(rounds))
    torch.cuda.synchronize()
    wall = time.perf_counter() - w0
    ms = wall * 1e3 / rounds
    log(f"mtp round: {ms:.2f} ms/round, {committed / rounds:.1f} committed/round, "
        f"{committed / wall:.0f} tok/s")

    # Forced full acceptance: every lane feeds k forced drafts and commits k + 1 tokens per
    # round (the reference's forced-draft leg), through the same captured graph.
    gen = torch.Generator().manual_seed(6)
    forced = [torch.randint(0, model.cfg.vocab, (k,), generator=gen).tolist() for _ in range(b)]

    def forced_round():
        got = runner.speculative_decode(list(range(b)), toks, pos, forced=forced)
        n = 0
        for j, c in enumerate(got):
            pos[j] += len(c)
            toks[j] = c[-1]
            n += len(c)
        return n

    forced_round()
    torch.cuda.synchronize()
    f0 = time.perf_counter()
    f_committed = sum(forced_round() for _ in range(rounds))
    torch.cuda.synchronize()
    f_wall = time.perf_counter() - f0
    log(f"mtp round, forced full acceptance: {f_wall * 1e3 / rounds:.2f} ms/round, "
        f"{f_committed / rounds:.1f} committed/round, {f_committed / f_wall:.0f} tok/s")
    res = {
        "workload": f"C5 reduced-depth verify: 3 DeltaNet + 1 gated GQA (32q/2kv, hd 256) + MTP layer, "
                    f"MXFP4 MoE 512 x top-10 per layer, B={b}, k={k}, {ctx}-token paged context",
        "ms_per_round": round(ms, 3),
        "committed_per_round": round(committed / rounds, 2),
        "accepted_tok_s": round(committed / wall, 1),
        "rounds": rounds,
        "weights": "random init (draft acceptance near zero)",
        "runner": "GraphMTPRunner (draft + verify + accept + commit replayed as one HIP graph)",
        "capture_validated": bool(validated),
        "blas_tuned": [list(x) for x in tuned],
        "forced_full_accept": {
            "ms_per_round": round(f_wall * 1e3 / rounds, 3),
            "committed_per_round": round(f_committed / rounds, 2),
            "accepted_tok_s": round(f_committed / f_wall, 1),
        },
    }
    del runner, model
    torch.cuda.empty_cache()
    return res


def cpu_threads() -> int:
    """Host threads for the CPU legs: the process's own OpenMP allotment (`OMP_NUM_THREADS`, 16
    per GPU on the GPU boxes, whose `os.cpu_count()` counts every core of the node), else every
    core the OS reports."""
    cores = os.cpu_count() or 1
    try:
        return max(1, min(int(os.environ.get("OMP_NUM_THREADS", cores)), cores))
    except ValueError:
        return cores


def _per_call(fn, budget_s: float, min_reps: int = 3) -> tuple[float, int]:
    """Mean seconds per call of `fn` over at least `min_reps` calls and about `budget_s`."""
    fn()
    reps, t0 = 0, time.perf_counter()
    while reps < min_reps or time.perf_counter() - t0 < budget_s:
        fn()
        reps += 1
    return (time.perf_counter() - t0) / reps, reps


def cpu_legs(threads: int) -> dict:
    """The rest of the reference's CPU path, timed on the host beside the GPU legs: the torch
    router chain at M = 192 (`model.py:2840-2843`), config 4's greedy acceptance (the argmax of
    the bf16 [48, 4, 248320] logits, then the host `greedy_accept_length` / `commit_limit` per
    lane, `mtp.py:691-726`, and the batched tensor forms, `graph_mtp.py:440-474`), config 4's
    rejection sampling (the float64 restatement of the method), and config 1's CPU plumbing
    (the tiny model's greedy MTP decode on the CPU engine, accepted tokens per second)."""
    import torch

    import graph_mtp
    import mtp
    import verify_model as vm
    from oracle import cpu_path, rejection_ref

    torch.set_num_threads(threads)
    out = {}
    g = torch.Generator().manual_seed(11)
    routing = torch.randn(192, E + 1, generator=g)
    sec, reps = _per_call(lambda: cpu_path.route(routing, E, TOP_K), 1.0)
    out["router_chain"] = {"rows": 192, "us_per_call": round(sec * 1e6, 1), "reps": reps}

    b, k, vocab = 48, 3, 248320
    t = k + 1
    target = (torch.randn(b, t, vocab, generator=g) * 3).to(torch.bfloat16)
    draft_logits = (target.float() + torch.randn(b, t, vocab, generator=g)).to(torch.bfloat16)
    drafts = draft_logits[:, :k].float().argmax(-1)
    rng = np.random.default_rng(44)
    budget = torch.from_numpy(rng.integers(1, 8, b))
    stops = torch.full((b, mtp.MAX_STOP_IDS), -1, dtype=torch.long)
    stops[:, 0] = torch.from_numpy(rng.integers(0, vocab, b))

    def greedy_host():
        sa = target.float().argmax(-1)
        rows, dr = sa.tolist(), drafts.tolist()
        for j in range(b):
            a = mtp.greedy_accept_length(dr[j], rows[j][:k])
            mtp.commit_limit(a, rows[j], int(budget[j]), [int(x) for x in stops[j] if x >= 0])

    def greedy_tensor():
        sa = target.float().argmax(-1)
        graph_mtp._commit_limit(graph_mtp._accept_len(drafts, sa), sa, budget, stops)

    sec_h, reps_h = _per_call(greedy_host, 2.0)
    sec_t, reps_t = _per_call(greedy_tensor, 2.0)
    sa0 = target.float().argmax(-1)
    sec_a, _ = _per_call(lambda: graph_mtp._commit_limit(graph_mtp._accept_len(drafts, sa0), sa0,
                                                         budget, stops), 0.5)
    out["c4_greedy"] = {"shape": [b, t, vocab], "us_host_forms": round(sec_h * 1e6, 1),
                        "us_tensor_forms": round(sec_t * 1e6, 1),
                        "us_accept_tail_only": round(sec_a * 1e6, 1), "reps": [reps_h, reps_t]}

    tnp, dnp = target.float().numpy(), draft_logits[:, :k].float().numpy()
    ua = rng.random((b, k)).astype(np.float32)
    us = rng.random(b).astype(np.float32)
    dtok = dnp.argmax(-1)

    def rejection():
        rejection_ref.rejection_accept(tnp, dnp, dtok, ua, us, 0.7)

    t0 = time.perf_counter()
    rejection()
    out["c4_rejection"] = {"us_per_call": round((time.perf_counter() - t0) * 1e6, 1), "reps": 1,
                           "form": "float64 restatement of Leviathan et al. Alg. 1"}

    cfg = vm.tiny_cfg()
    model = vm.Model(cfg, "cpu", torch.float32, lanes=2, max_seq=96, seed=0)
    mtp.attach(model, k=1, seed=1)
    gp = torch.Generator().manual_seed(5)
    prompts = [torch.randint(0, cfg.vocab, (16,), generator=gp).tolist() for _ in range(2)]
    toks, pos = [], []
    for lane, p in enumerate(prompts):
        toks.append(int(model.argmax(model.prefill(lane, p)[None])[0]))
        pos.append(len(p))
    made, rounds = [1, 1], 0
    t0 = time.perf_counter()
    while min(made) < 32 + 1:
        got = mtp.speculative_decode(model, [0, 1], toks, pos)
        rounds += 1
        for j, c in enumerate(got):
            made[j] += len(c)
            pos[j] += len(c)
            toks[j] = c[-1]
    wall = time.perf_counter() - t0
    committed = sum(made) - 2
    out["c1_plumbing"] = {"accepted_tok_s": round(committed / wall, 1), "rounds": rounds,
                          "committed": committed, "tokens_per_lane_round": round(committed / rounds / 2, 3),
                          "wall_s": round(wall, 3),
                          "workload": "tiny Qwen3.5-MoE (hidden 64, 4 layers, 8 experts top-2, MXFP4), "
                                      "2 prompts of 16 ids, greedy MTP decode k=1 for 32 tokens"}
    return out


def cpu_baseline(layer, inp, dl_full, budget_s):
    """The reference's CPU path (oracle.cpu_path, torch fp32) on a bounded sample of the M=192
    workload: consecutive groups of 8 rows until ~budget_s of CPU work; scaled per expert. The
    other CPU legs (router chain, acceptance, config 1) ride in `legs`."""
    import torch

    from oracle import cpu_path

    threads = cpu_threads()
    torch.set_num_threads(threads)
    x, a_e, a_w, _ = inp
    ne, nw = a_e.cpu().numpy(), a_w.cpu().numpy()
    xs = x.float().cpu()
    total_t, total_d, total_bytes, rows = 0.0, 0, 0.0, 0
    for t0 in range(0, 192, 8):
        sel = slice(t0 * TOP_K, (t0 + 8) * TOP_K)
        e_sel, w_sel = ne[sel], nw[sel]
        used = np.unique(e_sel[w_sel != 0])
        if used.size == 0:
            continue
        idx = torch.from_numpy(used).to(layer["gate_up"].device).long()
        sub = {k: v[idx].cpu() for k, v in layer.items()}
        remap = {int(e): i for i, e in enumerate(used)}
        ti = torch.tensor([remap.get(int(e), 0) for e in e_sel]).view(8, TOP_K)
        tw = torch.from_numpy(np.where(np.isin(e_sel, used), w_sel, 0)).view(8, TOP_K)
        start = time.perf_counter()
        cpu_path.routed_grouped(xs[t0 : t0 + 8], sub, ti, tw, (0, used.size))
        total_t += time.perf_counter() - start
        total_d += used.size
        total_bytes += layer_bytes(8, used.size)
        rows += 8
        if total_t >= budget_s:
            break
    us_layer = total_t / total_d * dl_full * 1e6
    log(f"cpu baseline: {rows} rows, {total_d} expert dequants in {total_t:.1f}s on {threads} threads")
    model = "unknown"
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {
        "value": round(total_bytes / total_t / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "threads": threads,
        "cpu_count": os.cpu_count(),
        "cpu_model": model,
        "kind": "port",
        "sample": f"first {rows} of 192 rows in groups of 8 ({total_d} expert dequants, "
                  f"{total_t:.1f} s); torch fp32 restatement of Model._routed_grouped",
        "us_per_layer_est": round(us_layer, 1),
        "threads_rule": "OMP_NUM_THREADS (the process's CPU share; 16 per GPU on the GPU box), "
                        "capped by os.cpu_count()",
        "legs": cpu_legs(threads),
    }


if __name__ == "__main__":
    sys.exit(main())

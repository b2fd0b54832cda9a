"""Benchmark: one PLM round of dense linears on one MI355X.

A step is one full 1.3B-shape round at k=7 (M = 56 rows): 24 GPT-style blocks (QKV 2048->6144,
attention-out 2048->2048, MLP up 2048->8192, MLP down 8192->2048) plus the LM head 2048->50257,
97 linears chained output-to-input as in the model, with random-init bf16 weights
(~N(0, 0.02^2)) resident in HBM. The round is recorded once as a HIP graph and replayed (the
reference replays its round as a CUDA graph, plm/decoder.py:414-447), two ways, both over
weights packed once into the MFMA fragment layout (as a served model keeps them):
  * all 97 linears in one chained launch (plm_gemm_chain_packed), checked bit for bit against
  * the per-GEMM drop-in path: 97 fast_gemm launches (plm_gemm_packed, tuned tile per shape).

Prints one JSON line: ``value`` is microseconds per round (lower is better) of the faster of the
two (both are reported), plus the round's HBM GB/s and fraction of the 8 TB/s peak, the dominant
kernel's roofline from HIP-event timing, the partial-round M sweep, the fused LM-head verify step,
and the torch-CPU baseline of the same linears timed on this host.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "plm-anon_amd"))

METRIC = "µs/round of linears + HBM GB/s (% of peak) at M=56, 1.3B-shape bf16"
HBM_PEAK_GBPS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--hidden", type=int, default=2048)
    ap.add_argument("--mlp", type=int, default=8192)
    ap.add_argument("--layers", type=int, default=24)
    ap.add_argument("--M", type=int, default=56)
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="CPU baseline budget (0 disables it)")
    ap.add_argument("--no-sweep", action="store_true", help="skip the partial-round M sweep")
    ap.add_argument("--no-verify", action="store_true", help="skip the fused LM-head verify timing")
    ap.add_argument("--no-llama", action="store_true", help="skip the reference's Llama-style linear sets")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the per-config lines (single GEMM, one block, the 32 x H2560 round)")
    ap.add_argument("--only-round", action="store_true", help="time the round only (for profiling runs)")
    ap.add_argument("--no-voronoi", action="store_true", help="skip the verify rows' auxiliary decode timing")
    ap.add_argument("--no-prefill", action="store_true", help="skip the prefill-width timing")
    ap.add_argument("--no-fp16", action="store_true", help="skip the fp16 round timing")
    ap.add_argument("--profile", choices=("eager", "copy", "verify", "voronoi", "lora", "act"),
                    help="no JSON: 'eager' launches the round and the fused verify step --steps times without a "
                         "graph (for rocprofv3 counter runs); 'copy' runs a 1 GiB device copy, the reference "
                         "kernel that scales the HBM byte counters; 'verify' runs the fused verify step and the "
                         "LM-head GEMM --steps times each over six LM-head copies (for kernel traces); "
                         "'voronoi' runs the verify rows' auxiliary decode --steps times")
    return ap.parse_args()


class Round:
    """The round's weights, activation chain and captured graph at one width M. ``act``: the
    Llama-style gate/up projections carry their SiLU-and-multiply (output ``[M, I]``, read whole by
    down: the MLP's real dataflow); otherwise each linear reads the leading columns of the one
    before it."""

    def __init__(self, M, hidden, mlp, layers, weights, tables, device, gemms=None, act=False, dtype=None):
        import torch

        dtype = dtype or torch.bfloat16
        from plm_amd import gemm_tables
        from plm_amd.workloads import GPT2_VOCAB, gpt_block

        self.M = M
        if gemms is None:
            gemms = [g for _ in range(layers) for g in gpt_block(hidden, mlp)]
            gemms.append(type(gemms[0])("lm_head", GPT2_VOCAB, hidden))
        self.gemms = list(gemms)
        self.weights = weights
        self.cfgs = [tables[(M, g.N, g.K)] for g in self.gemms]
        self.act = [act and gm.name == "gate_up" for gm in self.gemms]
        act_tables = gemm_tables.read_act_table(hidden) if act else {}
        for i, a in enumerate(self.act):
            if a:   # the fastest tile whose gate and up fragments pair up
                self.cfgs[i] = act_tables.get((M, self.gemms[i].N, self.gemms[i].K), self.cfgs[i])
                if self.cfgs[i]["wave_frags"] % 2:
                    self.cfgs[i] = dict(self.cfgs[i], wave_frags=2)
        g = torch.Generator(device=device).manual_seed(3000 + M)
        self.x0 = torch.randn(M, hidden, generator=g, device=device).to(dtype)
        self.outs = [torch.empty(M, gm.N // 2 if a else gm.N, device=device, dtype=dtype)
                     for gm, a in zip(self.gemms, self.act)]
        self.inputs = []
        x = self.x0
        for gm, out in zip(self.gemms, self.outs):
            self.inputs.append(x if x.shape[1] == gm.K else x[:, :gm.K])
            x = out
        self.graph = None

    def launch(self, indices=None):
        from plm_amd.fast_gemm import gate_up_silu, hip_linear

        for i in (range(len(self.gemms)) if indices is None else indices):
            fn = gate_up_silu if self.act[i] else hip_linear
            fn(self.inputs[i], self.weights[i], self.cfgs[i], self.outs[i])

    def capture(self, indices=None):
        import torch

        self.launch(indices)                          # eager pass: sizes the split-K workspace
        torch.cuda.synchronize()
        stream = torch.cuda.Stream()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            self.launch(indices)
        return graph

    @property
    def bytes(self):
        return sum(g.bytes(self.M) for g in self.gemms)


def time_graph(graph, steps, warmup):
    """Milliseconds per replay: warm-up replays, then `steps` replays bracketed by HIP events."""
    import torch

    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def kernel_class(M, K, cfg):
    """The compiled kernel a GEMM launches: (MT, wave_frags, unroll, k_waves)."""
    return (math.ceil(M / 16), cfg["wave_frags"], cfg["unroll"], cfg["k_waves"])


def kernel_name(cls):
    mt, nf, d, kw = cls
    return f"packed_gemm_kernel<bf16, MT={mt}, NF={nf}, D={d}, KW={kw}>"


def dominant_kernel_roofline(rnd, steps):
    """Per kernel class: graph of that class's launches only (in round order), HIP-event timed."""
    classes = {}
    for i, (g, cfg) in enumerate(zip(rnd.gemms, rnd.cfgs)):
        classes.setdefault(kernel_class(rnd.M, g.K, cfg), []).append(i)
    rows = []
    for cls, idx in classes.items():
        graph = rnd.capture(idx)
        ms = time_graph(graph, max(5, steps // 2), 2)
        per_launch_us = ms * 1000.0 / len(idx)
        nbytes = sum(rnd.gemms[i].bytes(rnd.M) for i in idx) / len(idx)
        flops = sum(rnd.gemms[i].flops(rnd.M) for i in idx) / len(idx)
        rows.append({"kernel": kernel_name(cls), "launches": len(idx), "us_per_launch": per_launch_us,
                     "bytes_per_launch": nbytes, "flops_per_launch": flops, "total_us": per_launch_us * len(idx)})
        del graph
    rows.sort(key=lambda r: -r["total_us"])
    return rows


def traffic_for(kernel: str):
    """HBM bytes per launch measured with rocprofv3 counters, if a committed summary holds them."""
    path = REPO / "profiles" / "traffic.json"
    if not path.exists():
        return None
    try:
        return json.loads(path.read_text()).get(kernel)
    except (OSError, ValueError):
        return None


def mfma_for(kernel: str):
    """MFMA busy % and bf16 MFMA flops per dispatch from the committed rocprofv3 counter summary."""
    path = REPO / "profiles" / "mfma.json"
    if not path.exists():
        return None
    try:
        return json.loads(path.read_text()).get(kernel)
    except (OSError, ValueError):
        return None


def cpu_baseline(hidden, mlp, M, budget_s):
    """torch-CPU F.linear (the reference's --mode default op) over one block and the LM head, timed
    on this host; the full round is 24 blocks + LM head, scaled from the per-GEMM medians."""
    import torch

    import oracle
    from plm_amd.workloads import GPT2_VOCAB, gpt_block, normal

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    gemms = gpt_block(hidden, mlp) + [type(gpt_block(hidden, mlp)[0])("lm_head", GPT2_VOCAB, hidden)]
    xs = {g.K: normal((M, g.K), 7000 + g.K) for g in gemms}
    ws = [normal((g.N, g.K), 7100 + i, 0.02) for i, g in enumerate(gemms)]
    medians = []
    deadline = time.perf_counter() + budget_s
    for g, w in zip(gemms, ws):
        oracle.linear(xs[g.K], w)                     # warm-up
        times = []
        while len(times) < 5 or (time.perf_counter() < deadline and len(times) < 50):
            t0 = time.perf_counter()
            oracle.linear(xs[g.K], w)
            times.append(time.perf_counter() - t0)
            if len(times) >= 5 and time.perf_counter() > deadline:
                break
        medians.append(sorted(times)[len(times) // 2])
    block_s = sum(medians[:4])
    round_s = 24 * block_s + medians[4]
    cpu_model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": round_s * 1e6, "unit": "us/round", "cores": threads, "kind": "port",
            "sample": f"torch CPU F.linear bf16, median of >=5 reps per GEMM of one {hidden}/{mlp} block and the "
                      f"LM head at M={M}; round = 24 x block + LM head; CPU {cpu_model}"}


def capture_graph(fn):
    """A HIP graph of ``fn()`` recorded on a side stream after one eager call."""
    import torch

    fn()
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        fn()
    return graph




class ChainedRound:
    """The round as two launches: its 96 block linears chained output-to-input in one persistent
    launch over packed weights (plm_gemm_chain_packed, on the chain tile measured fastest for the
    round's hidden size and width, each linear's K split chosen for the resident grid), then the LM head (read by no later linear) as its own launch with its tuned tile, which
    streams a 206 MB weight faster than the chain's tile does."""

    def __init__(self, rnd):
        from plm_amd import _lib, gemm_tables
        from plm_amd.chain import Link, LinearChain
        from plm_amd.fast_gemm import _tile
        from plm_amd.tiles import packed_chain_split

        cfg = gemm_tables.round_chain_tile(rnd.x0.shape[1], rnd.M, act=any(rnd.act))
        G = _lib.lib().plm_gemm_packed_resident_workgroups(_lib.DTYPE_CODES[rnd.x0.dtype], rnd.M, _tile(cfg))
        _lib.check(min(G, 0), "plm_gemm_packed_resident_workgroups")
        n = len(rnd.gemms) - 1
        links = [Link(x, w, y, i - 1, packed_chain_split(g.N, g.K, cfg, G), a)
                 for i, (g, x, w, y, a) in enumerate(zip(rnd.gemms[:n], rnd.inputs[:n], rnd.weights[:n], rnd.outs[:n],
                                                         rnd.act[:n]))]
        self.chain = LinearChain(links, cfg, packed=True)
        self.head = (rnd.inputs[n], rnd.weights[n], rnd.cfgs[n], rnd.outs[n])
        self.chain_bytes = sum(g.bytes(rnd.M) for g in rnd.gemms[:n])

    def run(self):
        from plm_amd.fast_gemm import hip_linear

        self.chain.run()
        hip_linear(*self.head)


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build runs the round's linears on a single MI355X); "
              f"got --gpus {args.gpus}", file=sys.stderr)
        sys.exit(2)
    import torch

    from plm_amd import gemm_tables
    from plm_amd.fast_gemm import hip_linear  # noqa: F401  (fails loudly if the library is missing)
    from plm_amd.workloads import GPT2_VOCAB, gpt_block

    torch.cuda.set_device(0)
    device = torch.device("cuda", 0)
    if args.profile == "copy":
        src = torch.empty(1 << 30, dtype=torch.uint8, device=device).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(max(1, args.steps)):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(f"[bench] copied 1 GiB x {max(1, args.steps)}", file=sys.stderr)
        return
    if args.profile == "verify":
        profile_verify(args, device)
        return
    if args.profile == "voronoi":
        profile_voronoi(args, device)
        return
    if args.profile == "lora":
        profile_lora(args, device)
        return
    if args.profile == "act":
        profile_act(args, device)
        return
    tables = gemm_tables.read_table(args.hidden)
    gemms = [g for _ in range(args.layers) for g in gpt_block(args.hidden, args.mlp)]
    gemms.append(type(gemms[0])("lm_head", GPT2_VOCAB, args.hidden))
    gen = torch.Generator(device=device)
    weights = []
    for i, g in enumerate(gemms):
        gen.manual_seed(1 + 1000 * 3 + i)
        weights.append((0.02 * torch.randn(g.N, g.K, generator=gen, device=device)).bfloat16())
    print(f"[bench] weights resident: {sum(w.numel() * 2 for w in weights) / 1e9:.2f} GB", file=sys.stderr,
          flush=True)

    rnd = Round(args.M, args.hidden, args.mlp, args.layers, weights, tables, device)
    chained = ChainedRound(rnd)
    chain = chained.chain
    if args.profile == "eager":
        from plm_amd.verify import lm_head_verify
        from plm_amd.workloads import TOP_P, proposals

        pending = proposals(args.M).to(device)
        for _ in range(max(1, args.steps)):
            chained.run()
            rnd.launch()
            lm_head_verify(rnd.inputs[-1], weights[-1], pending, TOP_P)
        torch.cuda.synchronize()
        print(f"[bench] eager chained round + per-GEMM round + verify x {max(1, args.steps)}", file=sys.stderr)
        return

    # Headline: the round as the chained launch of its block linears + the LM-head launch, replayed
    # as a HIP graph; the chained launch alone is timed too (its own roofline).
    graph = capture_graph(chained.run)
    ms = time_graph(graph, args.steps, args.warmup)
    if chain.error_flag():
        print("[bench] chained launch reported a timed-out wait: results invalid", file=sys.stderr)
        sys.exit(1)
    chain_outs = [o.clone() for o in rnd.outs]
    del graph
    graph = capture_graph(chain.run)
    us_chain = time_graph(graph, args.steps, args.warmup) * 1000.0
    del graph
    # The chained launch computes what the single-linear kernel does with the same tiles, bit for
    # bit, through all 96 block linears; the LM head is the per-GEMM path's own launch.
    for i, ln in enumerate(chain.links):
        hip_linear(ln.x, ln.w, dict(chain.cfg, split_k=ln.split_k), rnd.outs[i])
    hip_linear(*chained.head)
    torch.cuda.synchronize()
    mismatched = [i for i, (a, b) in enumerate(zip(chain_outs, rnd.outs)) if not torch.equal(a, b)]
    if mismatched:
        print(f"[bench] chained round differs from per-linear launches at linears {mismatched[:8]}", file=sys.stderr)
        sys.exit(1)
    us_round = ms * 1000.0
    gbps = rnd.bytes / (us_round * 1e-6) / 1e9
    print(f"[bench] chained round: {us_round:.1f} us, {gbps:.0f} GB/s (chained launch alone {us_chain:.1f} us)",
          file=sys.stderr, flush=True)

    # The per-GEMM drop-in path (fast_gemm's kernel, 97 launches) replayed as a HIP graph.
    graph = rnd.capture()
    ms_graph = time_graph(graph, args.steps, args.warmup)
    del graph
    us_graph = ms_graph * 1000.0
    print(f"[bench] per-GEMM graph round: {us_graph:.1f} us, {rnd.bytes / (us_graph * 1e-6) / 1e9:.0f} GB/s",
          file=sys.stderr, flush=True)

    # For comparison only (not a path of this build): the same 97 linears through the vendor
    # library (torch F.linear -> hipBLASLt) on the row-major weights, one graph.
    us_blas = None
    if not args.only_round:
        graph = capture_graph(lambda: [torch.nn.functional.linear(x, w)
                                       for x, w in zip(rnd.inputs, rnd.weights)])
        us_blas = time_graph(graph, args.steps, args.warmup) * 1000.0
        del graph
        print(f"[bench] the same round through hipBLASLt (F.linear, row-major weights): {us_blas:.1f} us",
              file=sys.stderr, flush=True)

    # value: the faster of the two complete implementations of the round (both verified above:
    # the chain bit for bit against the per-linear launches, those against the oracle in the tests).
    chain_wins = us_round <= us_graph
    us_value = us_round if chain_wins else us_graph
    gbps_value = rnd.bytes / (us_value * 1e-6) / 1e9
    n_lin = len(rnd.gemms)
    timing = (f"HIP graph replay, HIP events; value = the round as one chained launch of its {n_lin - 1} block "
              "linears over packed weights (plm_gemm_chain_packed) + the LM-head launch (plm_gemm_packed)"
              if chain_wins else
              f"HIP graph replay, HIP events; value = the round as {n_lin} fast_gemm launches (plm_gemm_packed, "
              "tuned tile per shape) in one graph")
    result = {
        "metric": METRIC, "value": round(us_value, 2), "unit": "us/round", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(us_value / 1000.0, 4), "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (random-init weights ~N(0,0.02^2), seeded)",
        "config": {"workload": f"{'1.3B' if args.hidden == 2048 else str(args.hidden)}-shape round of linears: "
                               f"{args.layers} GPT-style blocks + LM head, M={args.M} (k=7)",
                   "M": args.M, "hidden": args.hidden, "mlp": args.mlp, "layers": args.layers,
                   "vocab": GPT2_VOCAB, "gemm_launches": len(gemms), "bytes_per_round": rnd.bytes,
                   "timing": timing, "chain_tile": chain.cfg},
        "gbps": round(gbps_value, 1), "pct_of_hbm_peak": round(100.0 * gbps_value / HBM_PEAK_GBPS, 2),
        "chained_round": {"us": round(us_round, 2), "gbps": round(gbps, 1), "launches": 2,
                          "chain_launch_us": round(us_chain, 2)},
        "per_gemm_graph": {"us": round(us_graph, 2), "gbps": round(rnd.bytes / (us_graph * 1e-6) / 1e9, 1),
                           "launches": len(gemms)},
    }
    if us_blas is not None:
        result["hipblaslt_round"] = {"us": round(us_blas, 2), "gbps": round(rnd.bytes / (us_blas * 1e-6) / 1e9, 1),
                                     "note": "comparison only: the 97 linears as torch F.linear (hipBLASLt) on "
                                             "row-major weights, one graph; not a path of this build"}
    if not args.only_round:
        rows = dominant_kernel_roofline(rnd, args.steps)
        result["per_gemm_kernels"] = [{k: (round(v, 3) if isinstance(v, float) else v) for k, v in r.items()}
                                      for r in rows]
        if chain_wins:
            # The chained launch is the round's dominant kernel: its HIP-event time per replay (a graph
            # of that launch alone) is its duration.
            kernel = "packed_gemm_kernel<bf16, MT=%d, NF=%d, D=%d, KW=%d> (chained block linears)" % (
                math.ceil(args.M / 16), chain.cfg["wave_frags"], chain.cfg["unroll"], chain.cfg["k_waves"])
            achieved = chained.chain_bytes / (us_chain * 1e-6) / 1e9
            result["roofline"] = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                                  "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
                                  "traffic": traffic_for("chain_round"), "kernel": kernel, "launches_per_round": 1,
                                  "us_per_launch": round(us_chain, 2), "bytes_per_launch": chained.chain_bytes}
        else:
            # The kernel class with the most time in the round; its launches timed alone as a graph.
            top = rows[0]
            achieved = top["bytes_per_launch"] / (top["us_per_launch"] * 1e-6) / 1e9
            result["roofline"] = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                                  "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
                                  "traffic": traffic_for(top["kernel"]), "kernel": top["kernel"],
                                  "launches_per_round": top["launches"],
                                  "us_per_launch": round(top["us_per_launch"], 3),
                                  "bytes_per_launch": round(top["bytes_per_launch"], 1)}
        if not args.no_sweep:
            sweep = {}
            for M in (7, 14, 28, 42, 56):
                r = Round(M, args.hidden, args.mlp, args.layers, weights, tables, device)
                g = capture_graph(ChainedRound(r).run) if chain_wins else r.capture()
                us = time_graph(g, max(10, args.steps // 2), 3) * 1000.0
                sweep[str(M)] = {"us": round(us, 1), "gbps": round(r.bytes / (us * 1e-6) / 1e9, 1)}
                del g, r
            result["m_sweep"] = sweep
            print(f"[bench] M sweep: {sweep}", file=sys.stderr, flush=True)
        if not args.no_verify:
            result["verify"] = time_verify(weights[-1], args.hidden, device, args.steps)
            if args.cpu_seconds > 0:
                result["verify"]["cpu_baseline"] = cpu_verify_baseline(args.hidden, args.cpu_seconds)
        if not args.no_fp16:
            result["fp16_round"] = time_fp16_round(args, device, tables)
        if not args.no_voronoi:
            result["voronoi"] = time_voronoi(args, device, weights[-1])
        if not args.no_configs:
            result["configs"] = time_configs(args, device, rnd, chained, us_round, us_graph)
        if not args.no_llama:
            result["llama_rounds"] = time_llama_rounds(args, device)
            result["gated_lora"] = time_gated_lora(args, device)
            result["gate_up_silu"] = time_gate_up_silu(args, device)
        if not args.no_prefill:
            result["prefill"] = time_prefill(args, device, weights[:-1])
    if args.cpu_seconds > 0:
        result["cpu_baseline"] = cpu_baseline(args.hidden, args.mlp, args.M, args.cpu_seconds)
    print(json.dumps(result), flush=True)


def cpu_verify_baseline(hidden, budget_s):
    """The verify step of config 5 on this host's CPU, the reference's composition: torch-CPU
    F.linear logits in bf16 (plm/fast_gemm.py:111), then nucleus acceptance and the argmax
    (plm/decoder.py:71-75, 362) over them; median of >= 5 reps after one warm-up."""
    import torch

    import oracle
    from plm_amd.workloads import GPT2_VOCAB, TOP_P, normal, proposals

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    x = normal((56, hidden), 5000)
    w = normal((GPT2_VOCAB, hidden), 5001, 0.02)
    pending = proposals(56)
    oracle.verify(oracle.linear(x, w).float(), pending, TOP_P)  # warm-up
    times = []
    deadline = time.perf_counter() + budget_s / 3
    while len(times) < 5 or (time.perf_counter() < deadline and len(times) < 30):
        t0 = time.perf_counter()
        oracle.verify(oracle.linear(x, w).float(), pending, TOP_P)
        times.append(time.perf_counter() - t0)
    return {"us": round(sorted(times)[len(times) // 2] * 1e6, 1), "cores": threads, "kind": "port",
            "sample": "torch CPU F.linear bf16 logits [56, 50257], then the oracle's nucleus acceptance "
                      "(top-p 0.94) and argmax; median over the reps"}


def time_fp16_round(args, device, tables):
    """The 1.3B round in fp16, the reference's default round dtype (plm/rounds.py:50): the chained
    launch of the block linears + the LM head, and the per-GEMM graph, on fp16 weights drawn from the
    same seeds; the chain is checked bit for bit against per-linear launches with its tile."""
    import torch

    from plm_amd.fast_gemm import hip_linear
    from plm_amd.workloads import GPT2_VOCAB, gpt_block

    gemms = [g for _ in range(args.layers) for g in gpt_block(args.hidden, args.mlp)]
    gemms.append(type(gemms[0])("lm_head", GPT2_VOCAB, args.hidden))
    gen = torch.Generator(device=device)
    weights = []
    for i, g in enumerate(gemms):
        gen.manual_seed(1 + 1000 * 3 + i)
        weights.append((0.02 * torch.randn(g.N, g.K, generator=gen, device=device)).half())
    rnd = Round(args.M, args.hidden, args.mlp, args.layers, weights, tables, device, dtype=torch.float16)
    chained = ChainedRound(rnd)
    graph = capture_graph(chained.run)
    us_chain = time_graph(graph, args.steps, args.warmup) * 1000.0
    del graph
    if chained.chain.error_flag():
        raise RuntimeError("fp16 chained launch reported a timed-out wait")
    chain_outs = [o.clone() for o in rnd.outs]
    for i, ln in enumerate(chained.chain.links):
        hip_linear(ln.x, ln.w, dict(chained.chain.cfg, split_k=ln.split_k), rnd.outs[i])
    hip_linear(*chained.head)
    torch.cuda.synchronize()
    bit_exact = all(torch.equal(a, b) for a, b in zip(chain_outs, rnd.outs))
    graph = rnd.capture()
    us_graph = time_graph(graph, args.steps, args.warmup) * 1000.0
    del graph, rnd, chained, weights
    print(f"[bench] fp16 round: chained {us_chain:.1f} us, per-GEMM {us_graph:.1f} us", file=sys.stderr, flush=True)
    return {"chained_us": round(us_chain, 2), "per_gemm_us": round(us_graph, 2),
            "gbps": round(gemm_bytes(gemms, args.M) / (min(us_chain, us_graph) * 1e-6) / 1e9, 1),
            "chain_bit_exact_vs_per_linear": bit_exact,
            "note": "fp16 weights and activations (the reference's default round dtype); tiles as tuned for bf16"}


def gemm_bytes(gemms, M):
    return sum(g.bytes(M) for g in gemms)


def cpu_linear_us(shapes, M, budget_s):
    """Median microseconds of torch-CPU F.linear (the reference's --mode default op, via the oracle)
    for each (N, K) at width M on this host's cores: one warm-up, then at least 5 repetitions within
    the budget."""
    import torch

    import oracle
    from plm_amd.workloads import normal

    torch.set_num_threads(len(os.sched_getaffinity(0)))
    out = []
    deadline = time.perf_counter() + budget_s
    for i, (N, K) in enumerate(shapes):
        x, w = normal((M, K), 7200 + K), normal((N, K), 7300 + i, 0.02)
        oracle.linear(x, w)
        times = []
        while len(times) < 5 or (time.perf_counter() < deadline and len(times) < 30):
            t0 = time.perf_counter()
            oracle.linear(x, w)
            times.append(time.perf_counter() - t0)
        out.append(sorted(times)[len(times) // 2] * 1e6)
    return out


def _line(us, nbytes, cpu_us=None, **extra):
    gbps = nbytes / (us * 1e-6) / 1e9
    d = {"us": round(us, 2), "gbps": round(gbps, 1), "pct_of_hbm_peak": round(100.0 * gbps / HBM_PEAK_GBPS, 2),
         "bytes": nbytes}
    if cpu_us is not None:
        d["cpu_us"] = round(cpu_us, 1)
        d["speedup_vs_cpu"] = round(cpu_us / us, 1)
    d.update(extra)
    return d


def time_configs(args, device, rnd, chained, us_round, us_graph):
    """The BASELINE configs other than the headline round, each with its algorithmic bytes, GB/s,
    % of the 8 TB/s peak and the torch-CPU time of the same linears on this host:
      1  the single GEMM X[42,1024] x W[4096,1024]^T: a graph of 128 launches over 128 distinct
         weight copies (1 GiB, four times the 256 MB Infinity Cache), per launch;
      2  one 1.3B-shape block at M = 56 (QKV, attn-out, MLP up, down): the headline round's 96 block
         linears (24 blocks of distinct weights) timed as the chained launch and as the per-GEMM
         graph, per block;
      4  the 32-block hidden-2560 round (QKV 2560->7680, attn-out, MLP up 2560->10240, down) + LM head
         2560->50257 at M = 56, both implementations, with the chained launch's own roofline.
    Config 3 is the headline; config 5 is `verify`."""
    import torch

    from plm_amd import gemm_tables
    from plm_amd.fast_gemm import hip_linear
    from plm_amd.workloads import GPT2_VOCAB, gpt_block

    out = {}
    budget = max(1.0, args.cpu_seconds / 4) if args.cpu_seconds > 0 else 0
    # Config 1.
    M, N, K = 42, 4096, 1024
    cfg = gemm_tables.read_table(1024)[(M, N, K)]
    gen = torch.Generator(device=device).manual_seed(1 + 1000)
    x = torch.randn(M, K, generator=gen, device=device).bfloat16()
    copies = [(0.02 * torch.randn(N, K, generator=gen, device=device)).bfloat16() for _ in range(128)]
    y = torch.empty(M, N, device=device, dtype=torch.bfloat16)
    graph = capture_graph(lambda: [hip_linear(x, w, cfg, y) for w in copies])
    us = time_graph(graph, max(5, args.steps // 4), 2) * 1000.0 / len(copies)
    del graph, copies
    cpu = cpu_linear_us([(N, K)], M, budget)[0] if budget else None
    out["1_single_gemm"] = _line(us, 2 * (N * K + M * K + M * N), cpu, shape="X[42,1024] x W[4096,1024]^T",
                                 tile=cfg, timing="graph of 128 launches over 128 weight copies (1 GiB)")
    print(f"[bench] config 1: {us:.2f} us", file=sys.stderr, flush=True)
    # Config 2 from the headline round's 96 block linears.
    block = gpt_block(args.hidden, args.mlp)
    block_bytes = sum(g.bytes(rnd.M) for g in block)
    n_blocks = len(rnd.gemms[:-1]) // len(block)
    graph = capture_graph(lambda: rnd.launch(range(len(rnd.gemms) - 1)))
    us_blocks = time_graph(graph, max(5, args.steps // 2), 2) * 1000.0
    del graph
    graph = capture_graph(chained.chain.run)
    us_chain = time_graph(graph, max(5, args.steps // 2), 2) * 1000.0
    del graph
    cpu = sum(cpu_linear_us([(g.N, g.K) for g in block], rnd.M, budget)) if budget else None
    out["2_block"] = {"chained": _line(us_chain / n_blocks, block_bytes, cpu),
                      "per_gemm": _line(us_blocks / n_blocks, block_bytes, cpu),
                      "shape": f"one {args.hidden}/{args.mlp} block at M={rnd.M}",
                      "timing": f"the round's {n_blocks} blocks (distinct weights), per block"}
    print(f"[bench] config 2: chained {us_chain / n_blocks:.2f} us, per-GEMM {us_blocks / n_blocks:.2f} us per block",
          file=sys.stderr, flush=True)
    # Config 4.
    hidden, mlp, layers = 2560, 10240, 32
    tables = gemm_tables.read_table(hidden)
    gemms = [g for _ in range(layers) for g in gpt_block(hidden, mlp)]
    gemms.append(type(gemms[0])("lm_head", GPT2_VOCAB, hidden))
    gen = torch.Generator(device=device)
    weights = []
    for i, g in enumerate(gemms):
        gen.manual_seed(1 + 1000 * 4 + i)
        weights.append((0.02 * torch.randn(g.N, g.K, generator=gen, device=device)).bfloat16())
    r4 = Round(rnd.M, hidden, mlp, layers, weights, tables, device)
    c4 = ChainedRound(r4)
    c4.run()
    torch.cuda.synchronize()
    chain_outs = [o.clone() for o in r4.outs]
    for i, ln in enumerate(c4.chain.links):
        hip_linear(ln.x, ln.w, dict(c4.chain.cfg, split_k=ln.split_k), r4.outs[i])
    hip_linear(*c4.head)
    torch.cuda.synchronize()
    same = all(torch.equal(a, b) for a, b in zip(chain_outs, r4.outs))
    c4.chain.check()
    graph = capture_graph(c4.run)
    us_c4 = time_graph(graph, max(5, args.steps // 2), 2) * 1000.0
    del graph
    graph = capture_graph(c4.chain.run)
    us_c4_chain = time_graph(graph, max(5, args.steps // 2), 2) * 1000.0
    del graph
    graph = r4.capture()
    us_g4 = time_graph(graph, max(5, args.steps // 2), 2) * 1000.0
    del graph
    cpu = None
    if budget:
        per = cpu_linear_us([(g.N, g.K) for g in gpt_block(hidden, mlp)] + [(GPT2_VOCAB, hidden)], rnd.M, budget)
        cpu = layers * sum(per[:4]) + per[4]
    achieved = c4.chain_bytes / (us_c4_chain * 1e-6) / 1e9
    out["4_round_h2560"] = {
        "chained": _line(us_c4, r4.bytes, cpu, launches=2, chain_matches_per_linear=bool(same)),
        "per_gemm": _line(us_g4, r4.bytes, cpu, launches=len(gemms)),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBPS, 4), "kernel": "chained launch of the 128 block linears",
                     "us_per_launch": round(us_c4_chain, 2), "bytes_per_launch": c4.chain_bytes},
        "shape": f"{layers} GPT-style blocks of hidden {hidden} (QKV {3 * hidden}, MLP {mlp}) + LM head "
                 f"{hidden}->{GPT2_VOCAB}, M={rnd.M}",
        "cpu_note": "torch CPU F.linear: one block + LM head timed, round = 32 x block + LM head" if cpu else None}
    print(f"[bench] config 4: chained {us_c4:.1f} us, per-GEMM {us_g4:.1f} us", file=sys.stderr, flush=True)
    del r4, c4, weights, chain_outs
    torch.cuda.empty_cache()
    out["3_round_1p3b"] = {"chained": _line(us_round, rnd.bytes), "per_gemm": _line(us_graph, rnd.bytes),
                           "note": "the headline; cpu_baseline holds its CPU figure"}
    out["round_w110"] = time_wide_round(args, device, rnd)
    return out


def time_wide_round(args, device, rnd):
    """The headline round's linears (the same 24 blocks + LM head) at the relaxed setting's width
    W = k + k^2 = 110 (k = 10, plm/rounds.py:26-29), both implementations; the chain is first checked
    bit for bit against per-linear launches with its tile."""
    import torch

    from plm_amd import gemm_tables
    from plm_amd.fast_gemm import hip_linear

    tables = gemm_tables.read_table(args.hidden)
    wide = Round(110, args.hidden, args.mlp, args.layers, rnd.weights, tables, device, gemms=rnd.gemms)
    cw = ChainedRound(wide)
    cw.run()
    torch.cuda.synchronize()
    chain_outs = [o.clone() for o in wide.outs]
    for i, ln in enumerate(cw.chain.links):
        hip_linear(ln.x, ln.w, dict(cw.chain.cfg, split_k=ln.split_k), wide.outs[i])
    hip_linear(*cw.head)
    torch.cuda.synchronize()
    same = all(torch.equal(a, b) for a, b in zip(chain_outs, wide.outs))
    cw.chain.check()
    graph = capture_graph(cw.run)
    us_chain = time_graph(graph, max(5, args.steps // 2), 2) * 1000.0
    del graph
    graph = wide.capture()
    us_graph = time_graph(graph, max(5, args.steps // 2), 2) * 1000.0
    del graph
    line = {"chained": _line(us_chain, wide.bytes, launches=2, chain_matches_per_linear=bool(same)),
            "per_gemm": _line(us_graph, wide.bytes, launches=len(wide.gemms)),
            "shape": f"the headline round's {len(wide.gemms)} linears at M=110 (k=10)"}
    print(f"[bench] W=110 round: chained {us_chain:.1f} us, per-GEMM {us_graph:.1f} us", file=sys.stderr, flush=True)
    del cw, wide, chain_outs
    torch.cuda.empty_cache()
    return line


def profile_verify(args, device):
    """The fused verify step and the LM-head GEMM (its tuned tile), eager, rotating over six
    LM-head copies (1.2 GB: no call finds its weight in the Infinity Cache)."""
    import torch

    from plm_amd import gemm_tables
    from plm_amd.fast_gemm import hip_linear
    from plm_amd.verify import lm_head_verify
    from plm_amd.workloads import GPT2_VOCAB, TOP_P, proposals

    gen = torch.Generator(device=device).manual_seed(5000)
    x = torch.randn(args.M, args.hidden, generator=gen, device=device).bfloat16()
    copies = [(0.02 * torch.randn(GPT2_VOCAB, args.hidden, generator=gen, device=device)).bfloat16() for _ in range(6)]
    pending = proposals(args.M).to(device)
    cfg = gemm_tables.read_table(args.hidden)[(args.M, GPT2_VOCAB, args.hidden)]
    for i in range(max(1, args.steps)):
        lm_head_verify(x, copies[i % 6], pending, TOP_P)
    for i in range(max(1, args.steps)):
        hip_linear(x, copies[i % 6], cfg)
    torch.cuda.synchronize()
    print(f"[bench] verify x {max(1, args.steps)}, LM-head GEMM {cfg} x {max(1, args.steps)}", file=sys.stderr)


def profile_lora(args, device):
    """The gated-LoRA linear on the Llama-style 1.3B fused QKV (one launch: h and the corrected base
    GEMM) and the base GEMM alone, eager, rotating over 20 weight sets (252 MB)."""
    import torch

    from plm_amd import gemm_tables
    from plm_amd.fast_gemm import hip_linear
    from plm_amd.gated_lora import gated_linear, stack_b

    M, K, shards, rank, gate = args.M, 2048, (2048, 512, 512), 16, 7
    N = sum(shards)
    cfg = gemm_tables.read_table(K)[(M, N, K)]
    gen = torch.Generator(device=device).manual_seed(77)
    x = torch.randn(M, K, generator=gen, device=device).bfloat16()
    sets = []
    for _ in range(20):
        w = (0.02 * torch.randn(N, K, generator=gen, device=device)).bfloat16()
        a = (0.05 * torch.randn(len(shards) * rank, K, generator=gen, device=device)).bfloat16()
        bs = [(0.5 * torch.randn(n, rank, generator=gen, device=device)).bfloat16() for n in shards]
        sets.append((w, a, bs, stack_b(bs)))
    for i in range(max(1, args.steps)):
        w, a, bs, b = sets[i % len(sets)]
        gated_linear(x, w, a, bs, gate, cfg=cfg, lora_b=b)
    for i in range(max(1, args.steps)):
        hip_linear(x, sets[i % len(sets)][0], cfg)
    torch.cuda.synchronize()
    print(f"[bench] gated LoRA x {max(1, args.steps)}, base GEMM {cfg} x {max(1, args.steps)}", file=sys.stderr)


def profile_act(args, device):
    """The Llama-style 1.3B MLP (gate_up 2048 -> 2 x 5632, down 5632 -> 2048) at width M, eager,
    rotating over 8 weight sets (552 MB): the fused gate/up + SiLU-and-multiply launch, the gate/up
    projection alone, and the MLP as one chained launch (gate/up with its activation, then down)."""
    import torch

    from plm_amd import _lib, gemm_tables
    from plm_amd.chain import Link, LinearChain
    from plm_amd.fast_gemm import gate_up_silu, hip_linear
    from plm_amd.tiles import packed_chain_split, packed_chain_tile

    M, K, I = args.M, 2048, 5632
    cfg = gemm_tables.read_table(K)[(M, 2 * I, K)]
    act_cfg = gemm_tables.read_act_table(K).get((M, 2 * I, K), cfg)
    gen = torch.Generator(device=device).manual_seed(78)
    x = torch.randn(M, K, generator=gen, device=device).bfloat16()
    sets = [((0.02 * torch.randn(2 * I, K, generator=gen, device=device)).bfloat16(),
             (0.02 * torch.randn(K, I, generator=gen, device=device)).bfloat16()) for _ in range(8)]
    ccfg = packed_chain_tile(M)
    G = _lib.lib().plm_gemm_packed_resident_workgroups(_lib.PLM_BF16, M, _lib.Tile.from_config(ccfg))
    _lib.check(min(G, 0), "plm_gemm_packed_resident_workgroups")
    act = torch.empty(M, I, device=device, dtype=torch.bfloat16)
    out = torch.empty(M, K, device=device, dtype=torch.bfloat16)
    chains = [LinearChain([Link(x, wg, act, -1, packed_chain_split(2 * I, K, ccfg, G), True),
                           Link(act, wd, out, 0, packed_chain_split(K, I, ccfg, G))], ccfg) for wg, wd in sets]
    n = max(1, args.steps)
    for i in range(n):
        gate_up_silu(x, sets[i % 8][0], act_cfg)
    for i in range(n):
        hip_linear(x, sets[i % 8][0], cfg)
    for i in range(n):
        chains[i % 8].run()
    torch.cuda.synchronize()
    chains[0].check()
    print(f"[bench] gate_up_silu {act_cfg} x {n}, gate_up GEMM {cfg} x {n}, MLP chain {ccfg} x {n}", file=sys.stderr)


def time_llama_rounds(args, device):
    """The reference's Llama-style linear sets (hidden 2048 and 3072: GQA QKV, fused gate/up, vocabulary
    50304) as rounds at width M, both ways: the chained launch of the block linears + LM-head launch
    (checked bit for bit against per-linear launches first) and the per-GEMM graph with the tuned
    table's tile per shape; each once as bare linears (each reading the leading columns of the one
    before) and once with the gate/up projections carrying their SiLU-and-multiply, read whole by
    down (``act``: the MLP's dataflow)."""
    import torch

    from plm_amd import gemm_tables
    from plm_amd.fast_gemm import gate_up_silu, hip_linear
    from plm_amd.workloads import LLAMA_SETS, llama_round

    out = {}
    for name, spec in LLAMA_SETS.items():
        gemms = llama_round(name)
        tables = gemm_tables.read_table(spec["hidden"])
        gen = torch.Generator(device=device)
        weights = []
        for i, g in enumerate(gemms):
            # std 1/sqrt(K): every linear keeps its input's scale, so 28 layers of products (and of
            # silu(g) * u) neither overflow nor vanish without the norms a real layer has
            gen.manual_seed(7 + 1000 * 6 + i)
            weights.append((torch.randn(g.N, g.K, generator=gen, device=device) / g.K ** 0.5).bfloat16())
        res = {"layers": spec["layers"], "hidden": spec["hidden"]}
        for act in (False, True):
            rnd = Round(args.M, spec["hidden"], None, spec["layers"], weights, tables, device, gemms=gemms, act=act)
            chained = ChainedRound(rnd)
            chained.run()
            torch.cuda.synchronize()
            chain_outs = [o.clone() for o in rnd.outs]
            for i, ln in enumerate(chained.chain.links):
                fn = gate_up_silu if ln.act else hip_linear
                fn(ln.x, ln.w, dict(chained.chain.cfg, split_k=ln.split_k), rnd.outs[i])
            hip_linear(*chained.head)
            torch.cuda.synchronize()
            same = all(torch.equal(a.view(torch.int16), b.view(torch.int16)) for a, b in zip(chain_outs, rnd.outs))
            same = same and not chained.chain.error_flag()
            graph = capture_graph(chained.run)
            us_chain = time_graph(graph, max(10, args.steps // 2), 3) * 1000.0
            del graph
            graph = rnd.capture()
            us_graph = time_graph(graph, max(10, args.steps // 2), 3) * 1000.0
            del graph
            nbytes = rnd.bytes
            key = "mlp_act" if act else "linears"
            res[key] = {"bytes": nbytes, "chained_us": round(us_chain, 1),
                        "chained_gbps": round(nbytes / (us_chain * 1e-6) / 1e9, 1), "per_gemm_us": round(us_graph, 1),
                        "per_gemm_gbps": round(nbytes / (us_graph * 1e-6) / 1e9, 1),
                        "chain_matches_per_linear": bool(same)}
            print(f"[bench] Llama-style {name} round ({key}): chained {us_chain:.1f} us, per-GEMM {us_graph:.1f} us, "
                  f"chain matches {same}", file=sys.stderr, flush=True)
            del rnd, chained, chain_outs
            torch.cuda.empty_cache()
        out[name] = res
        del weights
        torch.cuda.empty_cache()
    return out


def time_gated_lora(args, device):
    """Gated LoRA on the Llama-style 1.3B fused QKV (2048 -> 2048+512+512, rank 16, gate at k = 7):
    the fused one-launch form (plm_gemm_packed_lora) against the same GEMMs as the reference composes
    them (base GEMM, hidden GEMM, one addmm per shard; the GEMMs on this build's kernel), graphs
    rotating enough weight copies that each call streams its weight from HBM."""
    import torch

    from plm_amd import gemm_tables
    from plm_amd.fast_gemm import hip_linear
    from plm_amd.gated_lora import gated_linear, stack_b

    M, K, shards, rank, gate = args.M, 2048, (2048, 512, 512), 16, 7
    N = sum(shards)
    cfg = gemm_tables.read_table(K)[(M, N, K)]
    gen = torch.Generator(device=device).manual_seed(77)
    x = torch.randn(M, K, generator=gen, device=device).bfloat16()
    sets = []
    for _ in range(20):   # 20 x 12.6 MB > 256 MB
        w = (0.02 * torch.randn(N, K, generator=gen, device=device)).bfloat16()
        a = (0.05 * torch.randn(len(shards) * rank, K, generator=gen, device=device)).bfloat16()
        bs = [(0.5 * torch.randn(n, rank, generator=gen, device=device)).bfloat16() for n in shards]
        sets.append((w, a, bs, stack_b(bs)))   # B stacked once, as GatedLoraMethod does at install
    down_cfg = {"wave_frags": 1, "k_waves": 4, "split_k": 1, "unroll": 2}

    def composed(w, a, bs, _b):
        out = hip_linear(x, w, cfg)
        hidden = hip_linear(x[gate:], a, down_cfg)
        col = 0
        for s_, b in enumerate(bs):
            out[gate:, col:col + b.shape[0]].addmm_(hidden[:, s_ * rank:(s_ + 1) * rank], b.t().contiguous())
            col += b.shape[0]
        return out

    res = {}
    for name, fn in (("fused_us", lambda w, a, bs, b: gated_linear(x, w, a, bs, gate, cfg=cfg, lora_b=b)),
                     ("composed_us", composed), ("base_gemm_us", lambda w, a, bs, b: hip_linear(x, w, cfg))):
        for st in sets:
            fn(*st)
        torch.cuda.synchronize()
        stream = torch.cuda.Stream()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for st in sets:
                fn(*st)
        res[name] = round(time_graph(graph, max(5, args.steps // 4), 2) * 1000.0 / len(sets), 2)
        del graph
    print(f"[bench] gated LoRA qkv: {res}", file=sys.stderr, flush=True)
    return dict(res, shape=f"M={M} N={N} K={K} rank={rank} shards={list(shards)} gate={gate}")


def time_gate_up_silu(args, device):
    """The Llama-style 1.3B MLP's gate_up_proj (2048 -> 2 x 5632) and its SiLU-and-multiply: the
    fused launch (gate_up_silu) against the projection alone and the projection followed by the
    activation as separate launches (torch's silu and mul), graphs rotating enough weight copies
    that each call streams its weight from HBM."""
    import torch
    import torch.nn.functional as F

    from plm_amd import gemm_tables
    from plm_amd.fast_gemm import gate_up_silu, hip_linear

    M, K, I = args.M, 2048, 5632
    N = 2 * I
    cfg = gemm_tables.read_table(K)[(M, N, K)]
    act_cfg = gemm_tables.read_act_table(K).get((M, N, K), cfg)
    gen = torch.Generator(device=device).manual_seed(78)
    x = torch.randn(M, K, generator=gen, device=device).bfloat16()
    ws = [(0.02 * torch.randn(N, K, generator=gen, device=device)).bfloat16() for _ in range(8)]  # 8 x 46 MB

    def separate(w):
        y = hip_linear(x, w, cfg)
        return F.silu(y[:, :I]) * y[:, I:]

    res = {}
    for name, fn in (("fused_us", lambda w: gate_up_silu(x, w, act_cfg)), ("gemm_then_act_us", separate),
                     ("gemm_alone_us", lambda w: hip_linear(x, w, cfg))):
        for w in ws:
            fn(w)
        torch.cuda.synchronize()
        stream = torch.cuda.Stream()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for w in ws:
                fn(w)
        res[name] = round(time_graph(graph, max(5, args.steps // 4), 2) * 1000.0 / len(ws), 2)
        del graph
    print(f"[bench] gate_up + SiLU-and-multiply: {res}", file=sys.stderr, flush=True)
    return dict(res, shape=f"M={M} N={N} K={K}", fused_tile=act_cfg, gemm_tile=cfg)


def time_prefill(args, device, block_weights):
    """Prefill widths (M = 64 ... 640, plm/rounds.py:16; the reference hands them to F.linear) over
    the round's 96 block linears: the packed kernel on the packed copies (fast_gemm's path for a
    released weight: the tuned tile or default_config, 128-row slices above 128 rows) against
    F.linear (hipBLASLt) on the row-major weights, each a graph of the 96 launches; per block."""
    import torch
    import torch.nn.functional as F

    from plm_amd.fast_gemm import CONFIGS, default_config, hip_linear, packed_weight, unpack_weight

    out = {}
    for M in (64, 128, 256, 640):
        gen = torch.Generator(device=device).manual_seed(900 + M)
        xs = {K: torch.randn(M, K, generator=gen, device=device).bfloat16()
              for K in sorted({w.shape[1] for w in block_weights})}
        cfgs = [CONFIGS.get((M, w.shape[0], w.shape[1])) or default_config(M, w.shape[0], w.shape[1])
                for w in block_weights]
        flops = sum(2 * M * w.shape[0] * w.shape[1] for w in block_weights)
        line = {}
        packs = [packed_weight(w) for w in block_weights]
        unpack = {id(w): p for w, p in zip(block_weights, packs)}
        for name, fn in (("packed", lambda w, c: hip_linear(xs[w.shape[1]], w, c)),
                         ("unpacked_f_linear", lambda w, c: F.linear(
                             xs[w.shape[1]], unpack_weight(unpack[id(w)], w.shape[0], w.shape[1], w.dtype))),
                         ("f_linear", lambda w, c: F.linear(xs[w.shape[1]], w))):
            for w, c in zip(block_weights, cfgs):
                fn(w, c)
            torch.cuda.synchronize()
            stream = torch.cuda.Stream()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=stream):
                for w, c in zip(block_weights, cfgs):
                    fn(w, c)
            us = time_graph(graph, max(5, args.steps // 5), 2) * 1000.0
            del graph
            line[name] = {"us_per_block": round(us / (len(block_weights) / 4), 2),
                          "tflops": round(flops / (us * 1e-6) / 1e12, 1)}
        out[str(M)] = line
        print(f"[bench] prefill M={M}: {line}", file=sys.stderr, flush=True)
    return dict(out, note="96 block linears of the headline round per graph; packed = plm_gemm_packed "
                          "(its wide kernel above 128 rows), unpacked_f_linear = plm_unpack_weight into a "
                          "transient buffer + F.linear (a released weight's path above 128 rows), f_linear = "
                          "torch F.linear on a kept row-major weight")


# The auxiliary decode's workload: the k = 7 verify rows of a width-56 round, the GPT-2 vocabulary,
# the reference's engine defaults, and an auxiliary vocabulary of 1024 cells. The released
# checkpoints' size is not in the reference's sources; its fit holds a k x A tile in one 32-warp
# program, which keeps A near 1024 on the GPU it ran on. 4096 is timed beside it.
VORONOI = {"rows": 7, "n_items": 1024, "n_targets": 128, "k": 8, "rounds": 2, "iterations": 12}
VORONOI_LARGE_ITEMS = 4096


def voronoi_inputs(device, vocab, seed=7000, n_items=None):
    import torch

    n_items = n_items or VORONOI["n_items"]
    gen = torch.Generator(device=device).manual_seed(seed)
    table = torch.randn(vocab, n_items, generator=gen, device=device).bfloat16()
    logits = (2.5 * torch.randn(VORONOI["rows"], vocab, generator=gen, device=device)).bfloat16()
    values = torch.randint(0, n_items, (VORONOI["rows"],), generator=gen, device=device)
    return table, logits, values


def profile_voronoi(args, device):
    """The auxiliary decode of the verify rows, eager, --steps times (for kernel traces)."""
    import torch

    from plm_amd.voronoi import Voronoi
    from plm_amd.workloads import GPT2_VOCAB

    table, logits, values = voronoi_inputs(device, GPT2_VOCAB)
    eng = Voronoi.from_table(table)
    out = torch.empty(VORONOI["rows"], dtype=torch.int64, device=device)
    for _ in range(max(1, args.steps)):
        eng.decode(logits, values, out)
    torch.cuda.synchronize()
    print(f"[bench] voronoi decode x {max(1, args.steps)}", file=sys.stderr)


def time_voronoi(args, device, w_lm):
    """The verify rows' auxiliary decode (LogitVoronoiAuxiliary.decode_unmasked: shortlist, two
    rounds of condense + fit, the decode) for the 7 verify rows of a width-56 round, as a graph; the
    round's whole LM-head end with it (verify + the verify rows' logits, the decode, the epilogue);
    and the oracle's time for the same decode on the host."""
    import torch

    from plm_amd.verify import AuxRoundVerify
    from plm_amd.voronoi import LogitVoronoiAuxiliary, Voronoi
    from plm_amd.workloads import GPT2_VOCAB, TOP_P, proposals

    n = VORONOI["rows"]
    table, logits, values = voronoi_inputs(device, GPT2_VOCAB)
    eng = Voronoi.from_table(table)
    out = torch.empty(n, dtype=torch.int64, device=device)
    graph = capture_graph(lambda: eng.decode(logits, values, out))
    us = time_graph(graph, max(20, args.steps), 5) * 1000.0
    del graph
    line = {"us": round(us, 2), "us_per_verify_row": round(us / n, 2), **VORONOI, "vocab": GPT2_VOCAB}
    big_table, big_logits, big_values = voronoi_inputs(device, GPT2_VOCAB, 7002, VORONOI_LARGE_ITEMS)
    big = Voronoi.from_table(big_table)
    graph = capture_graph(lambda: big.decode(big_logits, big_values, out))
    us_big = time_graph(graph, max(20, args.steps), 5) * 1000.0
    del graph, big, big_table
    line[f"us_n_items_{VORONOI_LARGE_ITEMS}"] = round(us_big, 2)
    # The steady round's LM-head end with the decode in it (k = 7, width 56): one fused verify that
    # also writes the 7 verify rows' logits, the decode, the epilogue.
    gen = torch.Generator().manual_seed(7001)
    scheme = LogitVoronoiAuxiliary(VORONOI["n_items"], w_lm.shape[1], GPT2_VOCAB, dtype=torch.bfloat16).to(device)
    scheme.auxiliary_vocabulary.copy_((0.02 * torch.randn(VORONOI["n_items"], w_lm.shape[1], generator=gen))
                                      .to(torch.bfloat16))
    x = torch.randn(56, w_lm.shape[1], generator=gen).to(torch.bfloat16).to(device)
    rv = AuxRoundVerify(n, scheme, GPT2_VOCAB, "nucleus", TOP_P, device=device)
    state = [proposals(n)[: n - 1].clone().to(device), torch.zeros(1, dtype=torch.int64, device=device),
             torch.full((1 << 17,), -1, dtype=torch.int64, device=device),
             torch.zeros((), dtype=torch.int64, device=device), torch.zeros((), dtype=torch.int64, device=device)]
    graph = capture_graph(lambda: rv(x, w_lm, values, *state))
    line["aux_round_us"] = round(time_graph(graph, max(10, args.steps // 2), 3) * 1000.0, 2)
    del graph
    if args.cpu_seconds > 0:
        import numpy as np

        from oracle import voronoi_oracle as vo

        tab, lg = table.float().cpu().numpy(), logits.float().cpu().numpy()
        t0 = time.perf_counter()
        vo.decode_unmasked(tab, lg, values.cpu().numpy(), "bf16")
        line["oracle_cpu_us"] = round((time.perf_counter() - t0) * 1e6, 1)
        line["oracle_cpu_note"] = "numpy oracle, one decode of the same 7 rows, host cores"
        del np
    print(f"[bench] voronoi decode: {line}", file=sys.stderr, flush=True)
    return line


def time_verify(w_lm, hidden, device, steps):
    """Fused LM-head verify (X[56,hidden] x W[50257,hidden]^T, softmax/argmax/top-p) as a graph,
    rotating over enough LM-head copies that each replay streams its weight from HBM."""
    import torch

    from plm_amd.verify import lm_head_verify
    from plm_amd.workloads import TOP_P, proposals

    copies = [w_lm] + [w_lm.clone() for _ in range(4)]          # 5 x 206 MB > 256 MB MALL
    gen = torch.Generator(device=device).manual_seed(5000)
    x = torch.randn(56, hidden, generator=gen, device=device).bfloat16()
    pending = proposals(56).to(device)
    acc = torch.empty(56, dtype=torch.bool, device=device)
    am = torch.empty(56, dtype=torch.int64, device=device)
    for w in copies:
        lm_head_verify(x, w, pending, TOP_P, accept=acc, argmax=am)
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for w in copies:
            lm_head_verify(x, w, pending, TOP_P, accept=acc, argmax=am)
    ms = time_graph(graph, max(5, steps // 2), 2) / len(copies)
    nbytes = 2 * (w_lm.shape[0] * hidden + 56 * hidden) + 56 * (8 + 8 + 1)
    del graph
    # The round's whole LM-head end (k = 7): proposals into the verify rows, the fused verify, and the
    # epilogue's state update (plm/decoder.py:351-365), as one graph per round.
    from plm_amd.verify import RoundVerify

    k = 7
    rv = RoundVerify(k, "nucleus", TOP_P, "bf16", device)
    verify_tokens = proposals(k).to(device)
    state = [pending[: k - 1].clone(), torch.zeros(1, dtype=torch.int64, device=device),
             torch.full((1 << 17,), -1, dtype=torch.int64, device=device),
             torch.zeros((), dtype=torch.int64, device=device), torch.zeros((), dtype=torch.int64, device=device)]
    for w in copies:
        rv(x, w, verify_tokens, *state)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for w in copies:
            rv(x, w, verify_tokens, *state)
    ms_round = time_graph(graph, max(5, steps // 2), 2) / len(copies)
    del graph, copies
    from plm_amd.verify import VERIFY_CONFIG

    mfma = mfma_for("verify_packed_main_kernel<bf16, MT=4, NF=%d, D=%d>" % (
        VERIFY_CONFIG["wave_frags"], VERIFY_CONFIG["unroll"])) or {}
    from plm_amd import gemm_tables
    from plm_amd.workloads import GPT2_VOCAB

    head_cfg = gemm_tables.read_table(hidden)[(56, GPT2_VOCAB, hidden)]
    head = mfma_for(kernel_name(kernel_class(56, hidden, head_cfg))) or {}
    return {"us": round(ms * 1000.0, 2), "gbps": round(nbytes / (ms * 1e-3) / 1e9, 1),
            "pct_of_hbm_peak": round(100.0 * nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 2),
            "bytes": nbytes, "accepted": int(acc.sum().item()), "round_us": round(ms_round * 1000.0, 2),
            "mfma_busy_pct": mfma.get("mfma_busy_pct"), "lm_head_gemm_mfma_busy_pct": head.get("mfma_busy_pct"),
            "mfma_source": "profiles/mfma.json (rocprofv3 --pmc MfmaUtil MfmaFlopsBF16)"}


if __name__ == "__main__":
    main()

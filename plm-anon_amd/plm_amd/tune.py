"""Per-shape tile tuner for MI355X and the tile-table key sets.

``python -m plm_amd.tune --heuristic`` writes every table from ``tiles.heuristic_tile`` (no GPU).
``python -m plm_amd.tune [--hidden 2048 ...]`` times every candidate tile of every key on the GPU
and writes the fastest into ``gpu_tuning/tiles_hidden<H>.json``. ``--chain`` instead times every
compiled tile as the tile of a chained round (``chain.LinearChain``) of GPT-style blocks and writes
the fastest per round width into ``gpu_tuning/chain_tiles_hidden<H>.json``.

Timing: each candidate runs as a HIP graph of back-to-back launches that rotate over enough
distinct weight copies (>= 1 GiB in total) that no launch finds its weight in the 256 MB
Infinity Cache; the figure is graph time / launches, so it includes the inter-kernel gap a round
sees. Only correct candidates count: each is checked against the fp32 product first.
"""

from __future__ import annotations

import argparse
import json
import math
import sys

from . import tiles
from .gemm_tables import TABLES
from .workloads import GPT2_VOCAB, M_SWEEP

# The reference's tuned keys (plm/gpu_tuning/tiles_hidden<H>.json): Llama shapes from
# model_shapes() at the widths the reference tunes.
REFERENCE_KEYS: dict[int, list[tuple[int, int, int]]] = {
    512: [(42, 768, 512), (42, 512, 512), (42, 2816, 512), (42, 512, 1408), (42, 50304, 512)],
    768: [(42, 1152, 768), (42, 768, 768), (42, 4096, 768), (42, 768, 2048), (42, 50304, 768)],
    1024: [(42, 1536, 1024), (42, 1024, 1024), (42, 5120, 1024), (42, 1024, 2560), (42, 50304, 1024)],
    2048: [(w, n, k) for w in (42, 56, 110)
           for n, k in ((3072, 2048), (2048, 2048), (11264, 2048), (2048, 5632), (50304, 2048))],
    3072: [(w, n, k) for w in (42, 56, 110)
           for n, k in ((4608, 3072), (3072, 3072), (16384, 3072), (3072, 8192), (50304, 3072))],
}


def _gpt_keys(M: int, hidden: int, mlp: int) -> list[tuple[int, int, int]]:
    return [(M, 3 * hidden, hidden), (M, hidden, hidden), (M, mlp, hidden), (M, hidden, mlp), (M, GPT2_VOCAB, hidden)]


# The GPT-style shapes the benchmark measures: the 350M MLP up at k=6, the 1.3B round at every
# partial-round width and at the relaxed setting's width 110 (k = 10), and the 3B round at k=7.
BENCH_KEYS: dict[int, list[tuple[int, int, int]]] = {
    1024: [(42, 4096, 1024)],
    2048: [key for M in (*M_SWEEP, 110) for key in _gpt_keys(M, 2048, 8192)],
    2560: _gpt_keys(56, 2560, 10240),
}


def table_keys(hidden: int) -> list[tuple[int, int, int]]:
    keys = REFERENCE_KEYS.get(hidden, []) + BENCH_KEYS.get(hidden, [])
    return sorted(set(keys), key=lambda k: (k[0], k[1], k[2]))


def all_hidden() -> list[int]:
    return sorted(set(REFERENCE_KEYS) | set(BENCH_KEYS))


def write_act_table(hidden: int, table: dict[tuple[int, int, int], dict]) -> None:
    """The fastest tile with an even wave_frags per key (``act_tiles_hidden<H>.json``): the tile a
    fused gate/up projection with its SiLU-and-multiply runs (``fast_gemm.gate_up_silu``), whose
    gate and up fragments pair up inside a wavefront's or a tile's fragments."""
    text = json.dumps({f"{M},{N},{K}": cfg for (M, N, K), cfg in sorted(table.items())}, indent=1)
    (TABLES / f"act_tiles_hidden{hidden}.json").write_text(text + "\n")


def write_table(hidden: int, table: dict[tuple[int, int, int], dict]) -> None:
    TABLES.mkdir(exist_ok=True)
    text = json.dumps({f"{M},{N},{K}": cfg for (M, N, K), cfg in sorted(table.items())}, indent=1)
    (TABLES / f"tiles_hidden{hidden}.json").write_text(text + "\n")


def heuristic_tables() -> None:
    from .fast_gemm import tile_supported

    for hidden in all_hidden():
        write_table(hidden, {key: tiles.heuristic_tile(*key, supported=lambda c, k=key: tile_supported(k[0], k[2], c))
                             for key in table_keys(hidden)})


# --------------------------------------------------------------------------- GPU tuning


def time_tile(M: int, N: int, K: int, cfg: dict, weights, x, out, reps: int = 3) -> float:
    """Microseconds per launch of ``cfg`` over the rotating weight copies, from graph replays."""
    import torch

    from .fast_gemm import hip_linear

    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        for w in weights:                       # eager warm-up (also sizes the workspace)
            hip_linear(x, w, cfg, out)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for w in weights:
                hip_linear(x, w, cfg, out)
        graph.replay()
        torch.cuda.synchronize()
        best = math.inf
        for _ in range(reps):
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record(stream)
            graph.replay()
            end.record(stream)
            end.synchronize()
            best = min(best, start.elapsed_time(end) * 1000.0 / len(weights))
    return best


# Candidates within this fraction of the fastest are ties (timing noise between runs is about
# that); a tie goes to an even wave_frags, the tiles the gated-LoRA launch and the gate/up
# activation also run well on.
TIE = 0.01


def pick(results: list[tuple[float, dict]]) -> tuple[dict, float]:
    """The table's tile from a key's ``(us, tile)`` results sorted fastest first."""
    best_us = results[0][0]
    for us, cfg in results:
        if us > best_us * (1 + TIE):
            break
        if cfg["wave_frags"] % 2 == 0:
            return cfg, us
    return results[0][1], best_us


def tune_key(M: int, N: int, K: int, verbose: bool = True) -> tuple[dict, float, list]:
    import torch

    from .fast_gemm import hip_linear, tile_supported

    dev = torch.device("cuda")
    w_bytes = 2 * N * K
    copies = max(2, min(64, math.ceil((1 << 30) / w_bytes)))
    gen = torch.Generator(device=dev).manual_seed(N * 7 + K)
    weights = [(0.02 * torch.randn(N, K, generator=gen, device=dev)).bfloat16() for _ in range(copies)]
    x = torch.randn(M, K, generator=gen, device=dev).bfloat16()
    out = torch.empty(M, N, device=dev, dtype=torch.bfloat16)
    ref = (x.float() @ weights[0].float().T)
    results = []
    for cfg in tiles.candidates(M, N, K, lambda c: tile_supported(M, K, c)):
        y = hip_linear(x, weights[0], cfg).float()
        if not torch.allclose(y, ref, rtol=1e-2, atol=2e-2):
            raise RuntimeError(f"tile {cfg} is wrong at {(M, N, K)}: max err {(y - ref).abs().max().item()}")
        results.append((time_tile(M, N, K, cfg, weights, x, out), cfg))
    results.sort(key=lambda r: r[0])
    best, best_us = pick(results)
    if verbose:
        gbps = (2 * (N * K + M * K + M * N)) / (best_us * 1e-6) / 1e9
        print(f"{M},{N},{K}: {best} {best_us:.2f} us {gbps:.0f} GB/s ({len(results)} candidates)", flush=True)
    del weights
    torch.cuda.empty_cache()
    return best, best_us, results


# --------------------------------------------------------------------------- chain tiles

# The chained rounds the benchmark runs, per hidden size: the block's linears (each reading the
# output before it: GPT-style QKV 3H, attn-out, MLP up, down; at 3072 the Llama 3B set's GQA QKV,
# o, fused gate/up and down) and the round widths.
def chain_rounds() -> dict[int, tuple[list, tuple[int, ...]]]:
    from .workloads import LLAMA_SETS, gpt_block, llama_block

    s = LLAMA_SETS["3B"]
    return {2048: (gpt_block(2048, 8192), (*M_SWEEP, 110)), 2560: (gpt_block(2560, 10240), (56,)),
            3072: (llama_block(s["hidden"], s["qkv"], s["intermediate"]), (42, 56, 110))}


def chain_candidates() -> list[dict]:
    return [{"wave_frags": nf, "k_waves": kw, "split_k": 1, "unroll": d}
            for nf in (1, 2, 4) for kw in (1, 4, 8, 16) for d in (2, 4, 6, 8)]


def tune_chain(hidden: int, block: list, M: int, verbose: bool = True) -> tuple[dict, float, list]:
    """The fastest tile for a chained round at width M: a chain of ``block``'s linears with distinct
    weights (at least 1 GiB of them, so that the Infinity Cache holds none across replays), timed
    as graph replays per linear. Each candidate's outputs must equal per-linear launches of the
    same tile and K splits bit for bit; a tile that is not compiled for M, or whose chain does not
    fit the counter area, is skipped."""
    import torch

    from . import _lib
    from .chain import Link, LinearChain
    from .fast_gemm import _tile, hip_linear

    dev = torch.device("cuda")
    block_bytes = sum(2 * g.N * g.K for g in block)
    blocks = max(4, math.ceil((1 << 30) / block_bytes))
    gemms = [g for _ in range(blocks) for g in block]
    gen = torch.Generator(device=dev).manual_seed(hidden * 31 + M)
    weights = [((g.K ** -0.5) * torch.randn(g.N, g.K, generator=gen, device=dev)).bfloat16() for g in gemms]
    x0 = torch.randn(M, hidden, generator=gen, device=dev).bfloat16()
    outs = [torch.empty(M, -(-g.N // 64) * 64, device=dev, dtype=torch.bfloat16)[:, :g.N] for g in gemms]
    inputs, x = [], x0
    for g, y in zip(gemms, outs):
        inputs.append(x[:, :g.K])
        x = y
    results = []
    for cfg in chain_candidates():
        G = int(_lib.lib().plm_gemm_packed_resident_workgroups(_lib.PLM_BF16, M, _tile(cfg)))
        if G <= 0:
            continue
        links = [Link(xi, w, y, i - 1, tiles.packed_chain_split(g.N, g.K, cfg, G))
                 for i, (g, xi, w, y) in enumerate(zip(gemms, inputs, weights, outs))]
        try:
            chain = LinearChain(links, cfg, packed=True)
        except RuntimeError:
            continue
        chain.run()
        chain.check()
        got = [y.clone() for y in outs]
        for ln in links:
            hip_linear(ln.x, ln.w, dict(cfg, split_k=ln.split_k), ln.y)
        if not all(torch.equal(a, b) for a, b in zip(got, outs)):
            raise RuntimeError(f"chain tile {cfg} differs from its per-linear launches at hidden {hidden}, M={M}")
        stream = torch.cuda.Stream()
        with torch.cuda.stream(stream):
            chain.run()
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=stream):
                chain.run()
            graph.replay()
            torch.cuda.synchronize()
            best = math.inf
            for _ in range(3):
                start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                start.record(stream)
                graph.replay()
                end.record(stream)
                end.synchronize()
                best = min(best, start.elapsed_time(end) * 1000.0 / len(links))
        chain.check()
        del graph, chain
        results.append((best, cfg))
        if verbose:
            print(f"  chain h{hidden} M{M} {cfg}: {best:.2f} us per linear", flush=True)
    results.sort(key=lambda r: r[0])
    best_cfg, best_us = _pick_chain(results, tiles.packed_chain_tile(M))
    if verbose:
        print(f"chain h{hidden} M{M}: {best_cfg} {best_us:.2f} us per linear ({len(results)} candidates)", flush=True)
    del weights, outs
    torch.cuda.empty_cache()
    return best_cfg, best_us, results


def _pick_chain(results: list[tuple[float, dict]], default: dict) -> tuple[dict, float]:
    """The fastest chain tile, or the width's default tile (``tiles.packed_chain_tile``) when it is
    within TIE of the fastest."""
    best_us = results[0][0]
    for us, cfg in results:
        if cfg == default and us <= best_us * (1 + TIE):
            return cfg, us
    return results[0][1], best_us


def write_chain_table(hidden: int, table: dict[int, dict]) -> None:
    text = json.dumps({str(M): cfg for M, cfg in sorted(table.items())}, indent=1)
    (TABLES / f"chain_tiles_hidden{hidden}.json").write_text(text + "\n")


def tune_chains(hiddens: list[int] | None, log: dict, only_widths: list[int] | None = None) -> None:
    from .gemm_tables import read_chain_table

    rounds = chain_rounds()
    for hidden in hiddens or sorted(rounds):
        block, widths = rounds[hidden]
        table = read_chain_table(hidden)
        for M in widths:
            if only_widths and M not in only_widths:
                continue
            best, _, results = tune_chain(hidden, block, M)
            table[M] = best
            log[f"chain,{hidden},{M}"] = [(us, cfg) for us, cfg in results]
            write_chain_table(hidden, table)


def main(argv: list[str] | None = None) -> None:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--heuristic", action="store_true", help="write heuristic tables without a GPU")
    ap.add_argument("--hidden", type=int, nargs="*", help="hidden sizes to tune (default: all)")
    ap.add_argument("--keys", nargs="*", help="only these M,N,K keys")
    ap.add_argument("--log", help="write every candidate's timing to this JSON file")
    ap.add_argument("--chain", action="store_true", help="tune the chained rounds' tiles instead")
    ap.add_argument("--widths", type=int, nargs="*", help="with --chain: only these round widths")
    args = ap.parse_args(argv)
    if args.heuristic:
        heuristic_tables()
        return
    log = {}
    if args.chain:
        tune_chains(args.hidden, log, args.widths)
        if args.log:
            with open(args.log, "w") as fh:
                json.dump(log, fh)
        print("chain tuning done", file=sys.stderr)
        return
    for hidden in args.hidden or all_hidden():
        path = TABLES / f"tiles_hidden{hidden}.json"
        table = {tuple(int(v) for v in k.split(",")): c for k, c in json.loads(path.read_text()).items()} \
            if path.exists() else {}
        act_path = TABLES / f"act_tiles_hidden{hidden}.json"
        act_table = {tuple(int(v) for v in k.split(",")): c for k, c in json.loads(act_path.read_text()).items()} \
            if act_path.exists() else {}
        for key in table_keys(hidden):
            if args.keys and f"{key[0]},{key[1]},{key[2]}" not in args.keys:
                continue
            best, best_us, results = tune_key(*key)
            table[key] = best
            even = [cfg for _, cfg in results if cfg["wave_frags"] % 2 == 0]
            if even:
                act_table[key] = even[0]
            log[f"{key[0]},{key[1]},{key[2]}"] = [(us, cfg) for us, cfg in results]
            write_table(hidden, table)
            write_act_table(hidden, act_table)
    if args.log:
        with open(args.log, "w") as fh:
            json.dump(log, fh)
    print("tuning done", file=sys.stderr)


if __name__ == "__main__":
    main()

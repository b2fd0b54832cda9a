"""Per-link phase timestamps of the chained round: a measuring tool, not part of the library.

``python -m plm_amd.chain_probe build [DIR]`` copies ``csrc/`` into DIR (default ``_probe/`` at the
repository root) with ``s_memrealtime`` stamps written by thread 0 of every workgroup at the
chained path's phase points, and builds ``DIR/libplm_probe.so`` with the library's own flags.
``python -m plm_amd.chain_probe run [DIR]`` (on an MI355X, from the repository root) loads that
library in place of ``libplm_amd.so``, runs the 1.3B round's chained launch of the 96 block linears
at M = 56 and M = 7 (bench.py's ``ChainedRound``, five warm-up launches, then one stamped launch)
and prints, per linear class, the medians over its 24 linears (the first left out) of the
per-workgroup phase times, first item of each linear, in microseconds.

Stamps (slot k of ``stamps[linear][workgroup]``): 0 link start, 1 producer flags seen, 2 first
pipeline stage done, 3 last K step done, 4 item end; inside the item end 5 accumulators in LDS
(barrier), 6 sums read (barrier), 7 Y stored (split 1) or partials written through (split > 1),
8 stores complete before the tile flag, 9 split counter returned."""
import argparse
import ctypes
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

from ._build import CSRC, HIPCC_FLAGS, INCLUDE, hipcc

REPO = Path(__file__).resolve().parents[2]
SLOTS, LINEARS, GROUPS = 10, 128, 512


def _patch(text: str, old: str, new: str) -> str:
    if text.count(old) != 1:
        raise SystemExit(f"chain_probe: the kernel source changed; no single match for {old[:60]!r}")
    return text.replace(old, new)


def instrument(out: Path) -> None:
    if out.exists():
        shutil.rmtree(out)
    shutil.copytree(CSRC, out / "csrc")
    p = out / "csrc" / "packed_gemm.h"
    s = p.read_text()
    s = _patch(s, "namespace plm {\n", f"""namespace plm {{
static __device__ uint64_t probe_stamps[{LINEARS} * {GROUPS} * {SLOTS}];
static __shared__ int probe_linear, probe_first;
__device__ __forceinline__ void probe_stamp(int gi, int k) {{
  if (threadIdx.x == 0 && gi < {LINEARS} && blockIdx.x < {GROUPS})
    probe_stamps[(gi * {GROUPS} + blockIdx.x) * {SLOTS} + k] = __builtin_amdgcn_s_memrealtime();
}}
__device__ __forceinline__ void probe_stamp_end(int k) {{
  if (threadIdx.x == 0 && probe_first == 1 && probe_linear >= 0 && probe_linear < {LINEARS} && blockIdx.x < {GROUPS})
    probe_stamps[(probe_linear * {GROUPS} + blockIdx.x) * {SLOTS} + k] = __builtin_amdgcn_s_memrealtime();
}}
""")
    s = _patch(s, """    const PLinear L = load_linear<NF, KW, EPI>(a, gi, epoch);
    POffsets<MT, NF, XN> o;""", """    probe_stamp(gi, 0);
    int probe_item = 0;
    const PLinear L = load_linear<NF, KW, EPI>(a, gi, epoch);
    POffsets<MT, NF, XN> o;""")
    s = _patch(s, """        wait_producer_tiles<NF, KW>(a, L, load_linear<NF, KW>(a, gi - 1, epoch), wave, lane);""",
               """        wait_producer_tiles<NF, KW>(a, L, load_linear<NF, KW>(a, gi - 1, epoch), wave, lane);
        probe_stamp(gi, 1);""")
    s = _patch(s, """#pragma unroll
        for (int j = 0; j < D; ++j) stage(j);
        for (int i = D; i < steps; i += D) {
#pragma unroll
          for (int j = 0; j < D; ++j) stage(j);
        }""", """        stage(0);
        if (probe_item == 0) probe_stamp(gi, 2);
#pragma unroll
        for (int j = 1; j < D; ++j) stage(j);
        for (int i = D; i < steps; i += D) {
#pragma unroll
          for (int j = 0; j < D; ++j) stage(j);
        }
        if (probe_item == 0) probe_stamp(gi, 3);
        if (threadIdx.x == 0) {
          probe_linear = gi;
          probe_first = probe_item == 0;
        }""")
    s = _patch(s, """        cp.item += a.G;
        if (cp.item >= L.items) break;
        pc_enter<NF, D, KW>(L, wave, cp);""", """        if (probe_item == 0) probe_stamp(gi, 4);
        ++probe_item;
        cp.item += a.G;
        if (cp.item >= L.items) break;
        pc_enter<NF, D, KW>(L, wave, cp);""")
    s = _patch(s, """    for (int t = 0; t < MT; ++t) red[(wave * Q + f * MT + t) * 64 + lane] = acc[f][t];
  lds_sync();
  int tile, s;""", """    for (int t = 0; t < MT; ++t) red[(wave * Q + f * MT + t) * 64 + lane] = acc[f][t];
  lds_sync();
  probe_stamp_end(5);
  int tile, s;""")
    s = _patch(s, """  lds_sync();  // every wavefront has read the tiles; LDS is free for the next item
  if (L.split == 1) {
    if constexpr (EPI == kEpiLora) {
      if (L.role == 2) lora_wait_h(a, lane, probe);
    }
#pragma unroll
    for (int i = 0; i * KW < Q; ++i) {
      const int q = wave + KW * i;
      if (q < Q) packed_store_frag<DT, MT, EPI>(a, L, M, n0, q, lane, sum[i]);
    }""", """  lds_sync();  // every wavefront has read the tiles; LDS is free for the next item
  probe_stamp_end(6);
  if (L.split == 1) {
    if constexpr (EPI == kEpiLora) {
      if (L.role == 2) lora_wait_h(a, lane, probe);
    }
#pragma unroll
    for (int i = 0; i * KW < Q; ++i) {
      const int q = wave + KW * i;
      if (q < Q) packed_store_frag<DT, MT, EPI>(a, L, M, n0, q, lane, sum[i]);
    }
    probe_stamp_end(7);""")
    s = _patch(s, """(s * Q + q) * kFragBytes + lane * 16), 0, kCoherent);
  }
  __builtin_amdgcn_s_waitcnt(0);  // this wavefront's partial is written through""",
               """(s * Q + q) * kFragBytes + lane * 16), 0, kCoherent);
  }
  __builtin_amdgcn_s_waitcnt(0);  // this wavefront's partial is written through
  probe_stamp_end(7);""")
    s = _patch(s, """  lds_sync();
  if (*last_flag == 0) return;
  if constexpr (EPI == kEpiLora) {
    if (L.role == 2) lora_wait_h(a, lane, probe);
  }
#pragma unroll
  for (int i = 0; i * KW < Q; ++i) {""", """  lds_sync();
  probe_stamp_end(9);
  if (*last_flag == 0) return;
  if constexpr (EPI == kEpiLora) {
    if (L.role == 2) lora_wait_h(a, lane, probe);
  }
#pragma unroll
  for (int i = 0; i * KW < Q; ++i) {""")
    s = _patch(s, """  if (L.flag == nullptr) return;
  __builtin_amdgcn_s_waitcnt(0);
  asm volatile("s_barrier" ::: "memory");""", """  if (L.flag == nullptr) return;
  __builtin_amdgcn_s_waitcnt(0);
  probe_stamp_end(8);
  asm volatile("s_barrier" ::: "memory");""")
    p.write_text(s)
    k8 = out / "csrc" / "packed_bf16_k8.hip"
    k8.write_text(k8.read_text() + f"""
extern "C" int plm_probe_read(void* host, size_t bytes) {{
  return hipMemcpyFromSymbol(host, HIP_SYMBOL(plm::probe_stamps), bytes, 0, hipMemcpyDeviceToHost) == hipSuccess ? 0 : -1;
}}
extern "C" int plm_probe_clear() {{
  static uint64_t zero[{LINEARS} * {GROUPS} * {SLOTS}];
  return hipMemcpyToSymbol(HIP_SYMBOL(plm::probe_stamps), zero, sizeof(zero), 0, hipMemcpyHostToDevice) == hipSuccess ? 0 : -1;
}}
""")


def build(out: Path) -> Path:
    instrument(out)
    src = out / "csrc"
    obj = out / "obj"
    obj.mkdir(exist_ok=True)

    def cc(f: Path) -> Path:
        o = obj / (f.stem + ".o")
        r = subprocess.run([hipcc(), *HIPCC_FLAGS, f"-I{INCLUDE}", f"-I{src}", "-c", str(f), "-o", str(o)],
                           capture_output=True, text=True)
        if r.returncode:
            raise SystemExit(r.stderr[-3000:])
        return o

    with ThreadPoolExecutor(8) as ex:
        objs = list(ex.map(cc, sorted(src.glob("*.hip"))))
    lib = out / "libplm_probe.so"
    r = subprocess.run([hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", *map(str, objs), "-o", str(lib)],
                       capture_output=True, text=True)
    if r.returncode:
        raise SystemExit(r.stderr[-3000:])
    return lib


def run(out: Path) -> None:
    import numpy as np
    import torch

    from . import _lib

    _lib.LIBRARY = out / "libplm_probe.so"
    lib = _lib.lib()
    lib.plm_probe_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    sys.path.insert(0, str(REPO))
    import bench
    from . import gemm_tables
    from .workloads import GPT2_VOCAB, gpt_block

    dev = torch.device("cuda:0")
    gemms = [g for _ in range(24) for g in gpt_block(2048, 8192)]
    gemms.append(type(gemms[0])("lm_head", GPT2_VOCAB, 2048))
    gen = torch.Generator(device=dev)
    weights = []
    for i, g in enumerate(gemms):
        gen.manual_seed(1 + 3000 + i)
        weights.append((0.02 * torch.randn(g.N, g.K, generator=gen, device=dev)).bfloat16())
    names = ["qkv", "attn-out", "mlp-up", "mlp-down"]
    for M in (56, 7):
        ch = bench.ChainedRound(bench.Round(M, 2048, 8192, 24, weights, gemm_tables.read_table(2048), dev))
        for _ in range(5):
            ch.chain.run()
        torch.cuda.synchronize()
        if lib.plm_probe_clear() != 0:
            raise SystemExit("chain_probe: could not clear the stamps")
        ch.chain.run()
        torch.cuda.synchronize()
        ch.chain.check()
        buf = np.zeros(LINEARS * GROUPS * SLOTS, dtype=np.uint64)
        if lib.plm_probe_read(buf.ctypes.data, buf.nbytes) != 0:
            raise SystemExit("chain_probe: could not read the stamps")
        d = buf.reshape(LINEARS, GROUPS, SLOTS).astype(np.int64)[:96]
        t0 = d[0, :, 0][d[0, :, 0] > 0].min()
        print(f"M={M}: stamped chained launch {(d[:, :, 4][d[:, :, 4] > 0].max() - t0) * 0.01:.1f} us", flush=True)
        rows = {n: [] for n in names}
        ends = []
        for gi in range(96):
            v = d[gi]
            ok = (v[:, 4] > 0) & (v[:, 3] > 0) & (v[:, 2] > 0) & ((v[:, 1] > 0) if gi > 0 else True)
            e = v[ok]
            last_end = v[:, 4][v[:, 4] > 0].max()
            ends.append(last_end)

            def med(a, b):
                m = (v[:, a] > 0) & (v[:, b] > 0)
                return float(np.median(v[m, b] - v[m, a]) * 0.01) if m.any() else float("nan")

            r = {"flag_after_producer_last": np.median(e[:, 1] - ends[gi - 1]) * 0.01 if gi else 0.0,
                 "wait": np.median(e[:, 1] - e[:, 0]) * 0.01 if gi else 0.0,
                 "first_stage": np.median(e[:, 2] - (e[:, 1] if gi else e[:, 0])) * 0.01,
                 "k_steps": np.median(e[:, 3] - e[:, 2]) * 0.01,
                 "item_end": np.median(e[:, 4] - e[:, 3]) * 0.01,
                 "tail": (last_end - np.median(v[:, 4][v[:, 4] > 0])) * 0.01,
                 "link": (last_end - ends[gi - 1]) * 0.01 if gi else 0.0,
                 "acc_in_lds": med(3, 5), "sums": med(5, 6), "stored": med(6, 7),
                 "counter": med(7, 9), "last_split": med(9, 8), "stores_complete": med(7, 8), "flag": med(8, 4)}
            rows[names[gi % 4]].append(r)
        for n in names:
            keys = list(rows[n][1])
            agg = {k: float(np.nanmedian([r[k] for r in rows[n][1:]])) for k in keys}
            print(f"  {n:8s} " + "  ".join(f"{k} {agg[k]:.2f}" for k in keys), flush=True)
        # Item ends by XCD (workgroup b on XCD b mod 8 under the default round-robin dispatch):
        # per linear, each workgroup's item end less the linear's median item end; medians per XCD.
        late = [[] for _ in range(8)]
        for gi in range(1, 96):
            v = d[gi, :, 4]
            have = np.nonzero(v > 0)[0]
            if len(have) == 0:
                continue
            med = np.median(v[have])
            for b in have:
                late[b % 8].append((v[b] - med) * 0.01)
        print("  item end vs the linear's median, by XCD (median, p90 us): " +
              "  ".join(f"{x}: {np.median(l):+.2f}/{np.percentile(l, 90):+.2f}" for x, l in enumerate(late) if l), flush=True)
        print(f"  last tile to last tile per linear: {(ends[-1] - ends[0]) * 0.01 / 95:.2f} us", flush=True)


def main(argv: list[str] | None = None) -> None:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("action", choices=("build", "run"))
    ap.add_argument("dir", nargs="?", default=str(REPO / "_probe"))
    args = ap.parse_args(argv)
    out = Path(args.dir).resolve()
    if args.action == "build":
        print(f"built {build(out)}")
    else:
        run(out)


if __name__ == "__main__":
    main()

"""AI.IF throughput on one MI355X: rows/s and prefill tokens/s.

Workload (one step): a full AI.IF filter over 4096 synthetic rows on a
random-init Qwen3-4B-architecture fp8 model (36 layers, hidden 2560,
32 Q / 8 KV heads, head_dim 128, FFN 9728, vocab 151936). Every row is a
shared 64-token instruction + a document of lognormal length (median 180,
mean ~230, capped at 1024, uniform random ids) + a 24-token question tail;
one TRUE/FALSE logit readout per row. The KV arena is sized by the
reference's budget formula for MI355X (288 GB HBM).

The JSON line reports value = rows/s over the timed steps (inputs already
resident in HBM; the packer's H2D staging is inside the step, as in the
reference's loop), prefill tokens/s, and a roofline for the dominant kernel
(the fp8 block-scaled GEMM) measured live with HIP events on the launch
stream, plus the attention kernel's MFMA fraction. cpu_baseline times the
CPU oracle (this repo's torch restatement of the path) on a bounded row
sample on the host cores.
"""

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

FP8_PEAK_TFLOPS = 5033.2     # MI355X dense fp8 MFMA (AMD published)
BF16_PEAK_TFLOPS = 2516.6    # MI355X dense bf16 MFMA
HBM_PEAK_GBPS = 8000.0
PEAK_CLOCK_GHZ = 2.4         # the clock the published MFMA peaks assume


def host_cpu():
    """(threads, model name) of the CPU baseline: every core of this process's
    affinity set, and the host CPU's model name as lscpu prints it."""
    import subprocess
    threads = len(os.sched_getaffinity(0))
    name = "unknown"
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                name = line.split(":", 1)[1].strip()
                break
    except (OSError, subprocess.SubprocessError):
        pass
    return threads, name


class KernelClock:
    """HIP-event timing of every GEMM and attention launch in a window."""

    def __init__(self, torch):
        self.torch = torch
        self.active = False
        self.gemm = []        # (flops, start, end, shape name)
        self.attn = []        # (flops, bytes, start, end, kind)
        self.n_q = self.d = self.n_kv = 0

    def gemm_hook(self, name, M, N, K, launch):
        if not self.active:
            return launch()
        e0 = self.torch.cuda.Event(enable_timing=True)
        e1 = self.torch.cuda.Event(enable_timing=True)
        e0.record()
        out = launch()
        e1.record()
        # algorithmic HBM bytes: A, B and their scales once, the output once
        # (bf16, or e4m3 + scales for the fused gate_up)
        out_bytes = (M * (N // 2) + M * (N // 256) * 4) if name == "gate_up" else 2 * M * N
        nbytes = M * K + N * K + M * (K // 128) * 4 + (N // 128) * (K // 128) * 4 + out_bytes
        self.gemm.append((2.0 * M * N * K, e0, e1, name, nbytes))
        return out

    def attention_hook(self, kind, pairs, kv_rows, n_queries, launch):
        if not self.active:
            return launch()
        e0 = self.torch.cuda.Event(enable_timing=True)
        e1 = self.torch.cuda.Event(enable_timing=True)
        e0.record()
        out = launch()
        e1.record()
        flops = 4.0 * self.n_q * self.d * pairs
        # unified gather: each sequence reads its own K and V rows (the node is
        # re-read per sequence), plus Q in (bf16) and O out (e4m3 for the
        # unified call, which quantizes in its epilogue; bf16 otherwise)
        out_bytes = 1 if kind == "unified" else 2
        nbytes = (kv_rows * self.n_kv * self.d * 2 * 2
                  + n_queries * self.n_q * self.d * (2 + out_bytes))
        self.attn.append((flops, nbytes, e0, e1, kind))
        return out

    def summary(self):
        self.torch.cuda.synchronize()
        g_flops = sum(x[0] for x in self.gemm)
        g_bytes = sum(x[4] for x in self.gemm)
        g_ms = sum(x[1].elapsed_time(x[2]) for x in self.gemm)
        per_shape = {}
        for flops, e0, e1, name, _ in self.gemm:
            f, t, n = per_shape.get(name, (0.0, 0.0, 0))
            per_shape[name] = (f + flops, t + e0.elapsed_time(e1), n + 1)
        a_flops = sum(x[0] for x in self.attn)
        a_bytes = sum(x[1] for x in self.attn)
        a_ms = sum(x[2].elapsed_time(x[3]) for x in self.attn)
        kinds = {}
        for flops, nbytes, e0, e1, kind in self.attn:
            f, t, n = kinds.get(kind, (0.0, 0.0, 0))
            kinds[kind] = (f + flops, t + e0.elapsed_time(e1), n + 1)
        return dict(
            attn_kinds={k: dict(launches=n, ms=round(t, 3),
                                tflops=round(f / t / 1e9, 1) if t else 0.0)
                        for k, (f, t, n) in kinds.items()},
            gemm_launches=len(self.gemm), gemm_ms=g_ms, gemm_flops=g_flops, gemm_bytes=g_bytes,
            gemm_tflops=g_flops / g_ms / 1e9 if g_ms else 0.0,
            gemm_shapes={k: dict(launches=n, ms=round(t, 3),
                                 tflops=round(f / t / 1e9, 1) if t else 0.0)
                         for k, (f, t, n) in per_shape.items()},
            attn_launches=len(self.attn), attn_ms=a_ms, attn_flops=a_flops,
            attn_tflops=a_flops / a_ms / 1e9 if a_ms else 0.0,
            attn_gbps=a_bytes / a_ms / 1e6 if a_ms else 0.0)


def cpu_baseline(model, spec, instruction, documents, tail, rows, threads, ue8m0=False):
    """The CPU oracle forward over a bounded sample of rows (the first `rows`)."""
    import numpy as np
    import torch

    from oracle import forward as oforward
    from oracle import ops as oops
    from quail_amd import loop
    from quail_amd.arena import KVArena
    from quail_amd.model import SYNTHETIC_FALSE_IDS, SYNTHETIC_TRUE_IDS

    torch.set_num_threads(threads)
    w = oforward.cpu_weights(model)
    gemm = oforward.DequantGemm()
    for L in w["layers"]:            # dequantize once, outside the timing
        for name in ("qkv", "o", "gate_up", "down"):
            q, s = L[name]
            gemm.cache[q.data_ptr()] = oops.dequant_weight(q, s).T.contiguous()
    docs = [np.concatenate([instruction, d]) for d in documents[:rows]]
    pages = sum(-(-(len(doc) + len(tail)) // 16) for doc in docs) + 4
    arena = KVArena(1, pages, 16, 1, 1, device="cpu", allocate=False)
    groups = []
    for i, doc in enumerate(docs):
        arena.activate(i, len(doc), capacity_tokens=len(doc) + len(tail))
        groups.append(dict(key=i, prefix=doc, f=len(doc), suffixes=[list(tail)]))
    chunk = loop.pack_chunk(torch, arena, groups, attention_mode="unified")
    oarena = oforward.OracleArena(spec.layers, pages, spec.n_kv, spec.d_head)
    t0 = time.perf_counter()
    normed = oforward.forward_chunk(w, chunk.host, "unified", oarena, gemm=gemm, ue8m0=ue8m0)
    bits, margins = oforward.readout(w, normed, SYNTHETIC_TRUE_IDS, SYNTHETIC_FALSE_IDS)
    wall = time.perf_counter() - t0
    return dict(rows_per_s=rows / wall, tok_per_s=chunk.tokens / wall, wall_s=wall,
                tokens=chunk.tokens, bits=bits.tolist(), margins=margins.tolist())


def cpu_baseline_join(model, spec, anchor, frame, partners, threads):
    """The CPU oracle forward of one anchor (prefix + frame written once) and
    its first len(partners) partners, unified attention, one chunk."""
    import numpy as np
    import torch

    from oracle import forward as oforward
    from oracle import ops as oops
    from quail_amd import loop
    from quail_amd.arena import KVArena
    from quail_amd.model import SYNTHETIC_FALSE_IDS, SYNTHETIC_TRUE_IDS

    torch.set_num_threads(threads)
    w = oforward.cpu_weights(model)
    gemm = oforward.DequantGemm()
    for L in w["layers"]:
        for name in ("qkv", "o", "gate_up", "down"):
            q, s = L[name]
            gemm.cache[q.data_ptr()] = oops.dequant_weight(q, s).T.contiguous()
    kept = np.concatenate([anchor, frame])
    rows = sum(-(-(len(kept) % 16 + len(p)) // 16) for p in partners)
    pages = -(-len(kept) // 16) + rows + 4
    arena = KVArena(1, pages, 16, 1, 1, device="cpu", allocate=False)
    arena.activate(0, len(kept), capacity_tokens=len(kept))
    group = dict(key=0, prefix=list(anchor), f=len(anchor), suffixes=[list(frame)],
                 write_suffix_tokens=len(frame))
    pairs = dict(key=0, prefix=None, f=len(kept), suffixes=[list(p) for p in partners])
    chunk = loop.pack_chunk(torch, arena, [group, pairs], attention_mode="unified")
    oarena = oforward.OracleArena(spec.layers, pages, spec.n_kv, spec.d_head)
    t0 = time.perf_counter()
    normed = oforward.forward_chunk(w, chunk.host, "unified", oarena, gemm=gemm)
    bits, margins = oforward.readout(w, normed, SYNTHETIC_TRUE_IDS, SYNTHETIC_FALSE_IDS)
    wall = time.perf_counter() - t0
    for key in chunk.temporary_keys:
        arena.free_key(key)
    return dict(rows_per_s=len(partners) / wall, tok_per_s=chunk.tokens / wall, wall_s=wall,
                tokens=chunk.tokens, bits=bits.tolist()[1:], margins=margins.tolist()[1:])


def copy_calibration(nbytes):
    """A plain elementwise copy kernel that reads and writes `nbytes` each."""
    import torch
    src = torch.ones(nbytes // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(3):
        torch.mul(src, 1.0, out=dst)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": src.numel() * 4, "dispatches": 3}), flush=True)


# HBM bytes per GEMM launch measured with rocprofv3 counters on this same
# workload (FETCH_SIZE and WRITE_SIZE passes, scaled by a copy kernel of
# known size); the profile summary records the commands and the factors.
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "gemm_fp8_aiif_qwen3_4b_hbm_traffic.md")


CLOCK_PROFILE = os.path.join(ROOT, "profiles", "gpu_clock_aiif_qwen3_4b_1024rows.md")


def profiled_clocks():
    """The shader clocks (GHz) the fp8 GEMMs and the paged attention kernel held
    on the AI.IF filter, from the committed GRBM clock-counter profile of this
    workload: GEMM = dispatch-time-weighted mean over the fp8_gemm_kernel rows.
    Returns (gemm, attention, source) or (None, None, reason); the clock is
    not measured by this run."""
    import re
    try:
        with open(CLOCK_PROFILE) as f:
            text = f.read()
    except OSError:
        return None, None, "no clock profile"
    gemm_w = gemm_t = 0.0
    attn = None
    for line in text.splitlines():
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if len(cells) < 4:
            continue
        try:
            n, us, mhz = int(cells[1]), float(cells[2]), float(cells[3])
        except ValueError:
            continue
        if "fp8_gemm_kernel" in cells[0]:
            gemm_w += n * us * mhz
            gemm_t += n * us
        elif re.search(r"attn_paged_kernel<true, true>", cells[0]):
            attn = mhz / 1e3
    if not gemm_t:
        return None, None, "clock profile has no fp8_gemm_kernel rows"
    return gemm_w / gemm_t / 1e3, attn, os.path.relpath(CLOCK_PROFILE, ROOT)


def measured_gemm_traffic():
    """(bytes per launch, source) from the committed counter profile, or (None, reason)."""
    import re
    try:
        with open(TRAFFIC_PROFILE) as f:
            text = f.read()
    except OSError:
        return None, "no counter profile"
    m = re.search(r"gemm_hbm_bytes_per_launch\s*=\s*([0-9.eE+]+)", text)
    if not m:
        return None, "counter profile has no gemm_hbm_bytes_per_launch line"
    return float(m.group(1)), os.path.relpath(TRAFFIC_PROFILE, ROOT)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--workload", default="aiif-4b",
                    choices=["aiif-4b", "aiif-32b", "join-4b", "attn-c1", "gemm-c2"],
                    help="aiif-4b: Qwen3-4B, 64-token instruction, lognormal docs (median "
                         "180, cap 1024); aiif-32b: Qwen3-32B, 128-token instruction, docs "
                         "uniform in [1024, 4096]; join-4b: Qwen3-4B AI join, anchors = "
                         "48-token root + left doc (lognormal median 120), partners = right "
                         "docs (lognormal median 120, cap 512), tree attention; attn-c1: "
                         "one attention layer, 64 rows sharing a 256-token prefix of a "
                         "paged arena, suffixes U[32, 256], 32/8 heads; gemm-c2: the fp8 "
                         "block-scaled GEMM at the four Qwen3-4B shapes, M = 16384")
    ap.add_argument("--anchors", type=int, default=32,
                    help="join-4b: left rows (anchors); 256 is the full 256 x 256 join")
    ap.add_argument("--partners", type=int, default=256, help="join-4b: right rows")
    ap.add_argument("--cpu-pairs", type=int, default=4)
    ap.add_argument("--rows", type=int, default=None,
                    help="rows (default 4096 for aiif-4b, 256 for aiif-32b)")
    ap.add_argument("--layers", type=int, default=None)
    ap.add_argument("--documents", default="token-store", choices=["token-store", "memory"],
                    help="aiif workloads: rows read from a memory-mapped Arrow token store "
                         "file (the reference's scan input) or from in-memory arrays")
    ap.add_argument("--attention", default=None, choices=["unified", "tree"],
                    help="default: unified for filters, tree for the join")
    ap.add_argument("--tree-kernel", default="fused", choices=["fused", "resident", "two_pass"],
                    help="the tree path's attention kernel (aiif and join workloads): node "
                         "pages streamed per q-tile, a node's K/V held in LDS, or the "
                         "three-launch form")
    ap.add_argument("--arena-pages", type=int, default=None)
    ap.add_argument("--cpu-rows", type=int, default=8)
    ap.add_argument("--ue8m0", action="store_true",
                    help="power-of-two (UE8M0) activation and weight scales, applied by the "
                         "MFMA: the reference's DeepGEMM UE8M0 mode (aiif-4b, gemm-c2)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--progress", action="store_true",
                    help="aiif workloads: a line on stderr after each chunk's answers")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--gemm-m", type=int, default=16384,
                    help="gemm-c2: tokens M (16384 is the C2 sweep; a C3 chunk is ~102,700)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="BYTES",
                    help="only run a plain device copy of BYTES (fp32 x * 1) three times: "
                         "the known-size kernel that scales rocprofv3 FETCH_SIZE/WRITE_SIZE")
    args = ap.parse_args()
    if args.copy_calibration:
        copy_calibration(args.copy_calibration)
        return
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for {args.gpus}): quail_amd has no "
              f"multi-GPU path; rows shard per GPU with no device communication.",
              file=sys.stderr)
        sys.exit(2)

    if args.workload == "join-4b":
        join_bench(args)
        return
    if args.workload == "attn-c1":
        attention_bench(args)
        return
    if args.workload == "gemm-c2":
        gemm_bench(args)
        return
    if args.attention is None:
        args.attention = "unified"

    import torch

    from quail_amd import budgets
    from quail_amd.aiif import FilterRunner, synthetic_filter_workload
    from quail_amd.model import build_random_qwen3
    from quail_amd.specs import MI355X, QWEN3_32B_FP8, QWEN3_4B_FP8
    from dataclasses import replace

    big = args.workload == "aiif-32b"
    if args.rows is None:
        args.rows = 256 if big else 4096
    base = QWEN3_32B_FP8 if big else QWEN3_4B_FP8
    spec = base if args.layers is None else replace(base, layers=args.layers)
    t_build = time.perf_counter()
    model = build_random_qwen3(spec, seed=args.seed, device="cuda",
                               max_pos=8192 if big else 2048, ue8m0=args.ue8m0)
    if big:
        instruction, documents, tail = synthetic_filter_workload(
            args.rows, prefix_tokens=128, uniform_lengths=(1024, 4096), seed=args.seed,
            vocab=spec.vocab)
    else:
        instruction, documents, tail = synthetic_filter_workload(args.rows, seed=args.seed,
                                                                 vocab=spec.vocab)
    store_dir = None
    if args.documents == "token-store":
        import tempfile
        from quail_amd.tokens import TokenStore
        store_dir = tempfile.mkdtemp(prefix="quail_amd_rows_")
        import atexit
        import shutil
        atexit.register(shutil.rmtree, store_dir, True)
        documents = TokenStore.from_documents(os.path.join(store_dir, "documents.arrow"),
                                              documents)
    clock = KernelClock(torch)
    clock.n_q, clock.d, clock.n_kv = spec.n_q, spec.d_head, spec.n_kv
    runner = FilterRunner(model, spec, device_spec=MI355X, n_pages=args.arena_pages,
                          attention_mode=args.attention, gemm_hook=clock.gemm_hook,
                          attention_hook=clock.attention_hook, ue8m0=args.ue8m0,
                          tree_kernel=args.tree_kernel)
    torch.cuda.synchronize()
    build_s = time.perf_counter() - t_build

    done = None
    if args.progress:
        # a line on stderr per chunk report: rows answered so far in this pass
        count = [0]

        def done(finished):
            count[0] += len(finished)
            print(f"[{time.perf_counter() - t_build:8.1f}s] {count[0] % args.rows or args.rows}"
                  f"/{args.rows} rows answered", file=sys.stderr, flush=True)

    for _ in range(args.warmup):
        runner.run(instruction, documents, tail, document_done=done)
    clock.active = True
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    results = []
    host = {}   # host-side phases of the loop (admission, allocation, packing, ...)
    for _ in range(args.steps):
        answers, stats = runner.run(instruction, documents, tail, timing=host,
                                    document_done=done)
        results.append((answers, stats))
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    clock.active = False
    k = clock.summary()

    stats = results[-1][1]
    answers = results[-1][0]
    ms_per_step = wall / args.steps * 1e3
    rows_per_s = args.rows * args.steps / wall
    fresh_tok_s = stats["fresh_tokens"] * args.steps / wall
    input_tok_s = stats["input_tokens"] * args.steps / wall
    steady = all(r[0] == answers for r in results)

    cpu = None
    if big and not args.no_cpu_baseline:
        # one 32B row of 1-4 k tokens is ~0.2 PFLOP: minutes on the host cores
        cpu = {"value": None, "unit": "rows/s", "cores": 0, "kind": "port",
               "sample": "not run for the Qwen3-32B workload (one row is minutes of CPU)"}
    elif not args.no_cpu_baseline and args.cpu_rows > 0:
        threads, cpu_model = host_cpu()
        try:
            base = cpu_baseline(model, spec, instruction, documents, tail, args.cpu_rows,
                                threads, ue8m0=args.ue8m0)
            agree = sum(int(b == a) for b, a in zip(base["bits"], answers[:args.cpu_rows]))
            cpu = {"value": round(base["rows_per_s"], 4), "unit": "rows/s",
                   "cores": threads, "cpu_model": cpu_model, "kind": "port",
                   "sample": (f"oracle forward (torch fp32, fp8 dequantized) of rows "
                              f"0..{args.cpu_rows - 1}: {base['tokens']} tokens, "
                              f"{base['wall_s']:.1f} s, {base['tok_per_s']:.1f} tok/s; "
                              f"decisions agree with the GPU on {agree}/{args.cpu_rows} "
                              f"(margins {[round(m, 3) for m in base['margins']]})")}
        except Exception as exc:   # report, never hide: the GPU line still prints
            cpu = {"value": None, "unit": "rows/s", "cores": 0, "kind": "port",
                   "sample": f"failed: {exc!r}"}

    if big:   # the counter profile covers the Qwen3-4B workload only
        traffic, traffic_src = None, "not measured for this workload"
    else:
        traffic, traffic_src = measured_gemm_traffic()
    gemm_clk, attn_clk, clk_src = ((None, None, "not profiled for this workload") if big
                                   else profiled_clocks())
    line = {
        "metric": (f"rows/s + prefill tok/s, {'Qwen3-32B' if big else 'Qwen3-4B'} fp8 AI.IF "
                   f"on 1 GPU; attn/GEMM % of MFMA peak"),
        "value": round(rows_per_s, 2), "unit": "rows/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_per_step, 1),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp8",
        "data": "synthetic",
        "config": {"workload": (
                       f"AI.IF filter, {'Qwen3-32B' if big else 'Qwen3-4B'}-arch fp8 random "
                       f"init, {spec.layers} layers, {args.rows} rows, "
                       + ("128-token shared instruction, docs uniform in [1024, 4096]"
                          if big else "64-token shared instruction, lognormal docs "
                                      "(median 180, cap 1024)")
                       + f", 24-token tail, {args.attention} attention, "
                       + ("rows read from a memory-mapped Arrow token store"
                          if args.documents == "token-store" else "rows in memory")
                       + (", UE8M0 scales applied by the MFMA" if args.ue8m0
                          else ", fp32 block scales")),
                   "rows": args.rows, "layers": spec.layers,
                   "tree_kernel": args.tree_kernel if args.attention == "tree" else None,
                   "fresh_tokens": stats["fresh_tokens"],
                   "input_tokens": stats["input_tokens"], "chunks": stats.get("chunks"),
                   "chunk_budget": runner.budget, "arena_pages": runner.arena.n_pages},
        "prefill_tok_per_s": round(fresh_tok_s, 1),
        "input_tok_per_s": round(input_tok_s, 1),
        "roofline": {"bound": "mfma", "achieved": round(k["gemm_tflops"], 1),
                     "peak": FP8_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(k["gemm_tflops"] / FP8_PEAK_TFLOPS, 4),
                     "traffic": traffic,
                     "traffic_unit": "HBM bytes per GEMM launch (rocprofv3 counters)",
                     "traffic_source": traffic_src,
                     "algorithmic_bytes_per_launch": round(k["gemm_bytes"] / max(1, k["gemm_launches"])),
                     "kernel": ("qh fp8_gemm_kernel: qkv, o, down (bf16 out) and gate_up "
                                "(fused SiLU gate + fp8 quant epilogue)"),
                     # the published peak assumes 2.4 GHz; the GEMMs' clock on this workload
                     # comes from the committed GRBM clock-counter profile (not this run)
                     "at_profiled_clock": None if gemm_clk is None else {
                         "clock_ghz": round(gemm_clk, 3),
                         "peak": round(FP8_PEAK_TFLOPS * gemm_clk / PEAK_CLOCK_GHZ, 1),
                         "frac": round(k["gemm_tflops"] / (FP8_PEAK_TFLOPS * gemm_clk
                                                           / PEAK_CLOCK_GHZ), 4),
                         "source": clk_src}},
        "gemm": {"share_of_step": round(k["gemm_ms"] / (ms_per_step * args.steps), 3),
                 "shapes": k["gemm_shapes"]},
        "attention": {"tflops": round(k["attn_tflops"], 1),
                      "frac_bf16_peak": round(k["attn_tflops"] / BF16_PEAK_TFLOPS, 4),
                      "frac_bf16_peak_at_profiled_clock": None if attn_clk is None else round(
                          k["attn_tflops"] / (BF16_PEAK_TFLOPS * attn_clk / PEAK_CLOCK_GHZ), 4),
                      "profiled_clock_ghz": None if attn_clk is None else round(attn_clk, 3),
                      "gather_gbps": round(k["attn_gbps"], 1),
                      "gather_frac_hbm": round(k["attn_gbps"] / HBM_PEAK_GBPS, 4),
                      "share_of_step": round(k["attn_ms"] / (ms_per_step * args.steps), 3),
                      "calls": k["attn_kinds"]},
        "host_ms_per_step": {k: round(1e3 * v / args.steps, 1) for k, v in host.items()
                             if k != "n_chunks"},
        "answers_true": int(sum(answers)), "deterministic_across_steps": steady,
        "build_s": round(build_s, 1),
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


GEMM_SHAPES = (("qkv", 6144, 2560), ("o", 2560, 4096), ("gate_up", 19456, 2560),
               ("down", 2560, 9728))


def gemm_bench(args):
    """The fp8 block-scaled GEMM at the Qwen3-4B projection shapes, M = 16384.

    W ~ N(0, 0.02) quantized to e4m3 with fp32 128x128 block scales
    (amax/448); X ~ N(0, 1) quantized with 1x128 per-token scales; bf16
    out (the gate_up shape also runs the fused SiLU-gate + fp8 quant
    epilogue the model uses). Each launch is timed with HIP events on the
    launch stream.
    """
    import torch

    from oracle import ops as oops
    from quail_amd import kernels as K

    M = args.gemm_m
    g = torch.Generator().manual_seed(args.seed)
    stream = torch.cuda.current_stream()
    iters = max(args.steps, 1) * 10
    shapes, total_f, total_ms, cpu = {}, 0.0, 0.0, None
    x = torch.randn(M, 9728, generator=g)
    for name, N, Kd in GEMM_SHAPES:
        w = torch.randn(N, Kd, generator=g) * 0.02
        wq, ws = oops.quantize_weight_blocks(w, ue8m0=args.ue8m0)
        xq, xs = oops.group_quant(x[:, :Kd], ue8m0=args.ue8m0)
        a = xq.to("cuda")
        sa = K.col_major_scales(M, Kd, "cuda")
        sa.copy_(xs.to("cuda"))
        wq, ws = wq.to("cuda"), ws.to("cuda")
        hw = bool(args.ue8m0)
        variants = [("bf16 out", lambda: K.fp8_gemm_nt(a, sa, wq, ws, ue8m0_scales=hw))]
        if name == "gate_up":
            variants.append(("silu+fp8 out", lambda: K.fp8_gemm_silu_quant(
                a, sa, wq, ws, ue8m0=hw, ue8m0_scales=hw)))
        flops = 2.0 * M * N * Kd
        rec = {}
        for label, fn in variants:
            for _ in range(max(args.warmup, 1) * 3):
                fn()
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            e0.record(stream)
            for _ in range(iters):
                fn()
            e1.record(stream)
            torch.cuda.synchronize()
            ms = e0.elapsed_time(e1) / iters
            rec[label] = dict(ms=round(ms, 4), tflops=round(flops / ms / 1e9, 1),
                              frac=round(flops / ms / 1e9 / FP8_PEAK_TFLOPS, 4))
        rec["library_scaled_mm"] = library_gemm(a, wq, M, N, Kd, iters, max(args.warmup, 1) * 3)
        total_f += flops
        total_ms += rec["bf16 out"]["ms"]
        # parity on a row sample: the oracle's exact block sums
        rows = torch.arange(0, M, M // 64)
        got = K.fp8_gemm_nt(a, sa, wq, ws, ue8m0_scales=hw)[rows.to("cuda")].float().cpu()
        want = oops.fp8_gemm(xq[rows], xs[rows].contiguous(), wq.cpu(), ws.cpu()).float()
        rec["rel_l2_vs_oracle_64_rows"] = round(((got - want).norm() / want.norm()).item(), 6)
        shapes[name] = dict(N=N, K=Kd, gflop=round(flops / 1e9, 1), **rec)
    if not args.no_cpu_baseline:
        threads, cpu_model = host_cpu()
        torch.set_num_threads(threads)
        name, N, Kd = GEMM_SHAPES[0]
        rows = 1024
        w = torch.randn(N, Kd, generator=g) * 0.02
        wq, ws = oops.quantize_weight_blocks(w)
        xq, xs = oops.group_quant(x[:rows, :Kd])
        t0 = time.perf_counter()
        ref = oops.dequant_rows(xq, xs) @ oops.dequant_weight(wq, ws).T
        cpu_s = time.perf_counter() - t0
        cpu = {"value": round(2.0 * rows * N * Kd / cpu_s / 1e12, 4), "unit": "TFLOP/s",
               "cores": threads, "cpu_model": cpu_model, "kind": "port",
               "sample": f"oracle fp8 GEMM (dequantize with block scales, fp32 matmul), "
                         f"qkv shape with M = {rows}: {cpu_s:.2f} s"}
        del ref
    achieved = total_f / total_ms / 1e9
    line = {
        "metric": f"fp8 block-scaled GEMM TFLOP/s at the Qwen3-4B shapes (M = {M}) on 1 GPU; "
                  "% of fp8 MFMA peak",
        "value": round(achieved, 1), "unit": "TFLOP/s", "n_gpus": 1, "steps": iters,
        "warmup": max(args.warmup, 1) * 3, "ms_per_step": round(total_ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp8",
        "data": "synthetic",
        "config": {"workload": f"fp8 block-scaled GEMM sweep, M = {M}, (N, K) in "
                               "{(6144, 2560), (2560, 4096), (19456, 2560), (2560, 9728)}, "
                               + ("UE8M0 (power-of-two) 128x128 weight / 1x128 activation "
                                  "scales applied by the MFMA, bf16 out" if args.ue8m0 else
                                  "fp32 128x128 weight / 1x128 activation scales, bf16 out")},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 1), "peak": FP8_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / FP8_PEAK_TFLOPS, 4),
                     "traffic": None, "kernel": "qh fp8_gemm_kernel"},
        "shapes": shapes,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def library_gemm(a, wq, M, N, Kd, iters, warmup):
    """For context, not the product path: ROCm's tuned library fp8 GEMM
    (torch._scaled_mm, hipBLASLt) on the same e4m3 operands with the scalings
    it supports, one fp32 scale per row of A and per row of B ("rowwise") or
    one per tensor, bf16 out. Its 128x128 / 1x128 block-scale modes are
    marked "not supported yet" in this ROCm's hipblaslt.h, so no library GEMM
    computes the block-scaled product itself; these figures bound what the
    library reaches at the same shapes without per-block promotion."""
    import torch

    out = {}
    flops = 2.0 * M * N * Kd
    scalings = {
        "rowwise": (torch.full((M, 1), 1.0 / 448, device="cuda"),
                    torch.full((1, N), 1.0 / 448, device="cuda")),
        "tensor": (torch.tensor(1.0 / 448, device="cuda"), torch.tensor(1.0 / 448, device="cuda")),
    }
    for mode, (sa, sb) in scalings.items():
        try:
            def fn():
                return torch._scaled_mm(a, wq.t(), scale_a=sa, scale_b=sb,
                                        out_dtype=torch.bfloat16)
            for _ in range(warmup):
                fn()
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            e0.record()
            for _ in range(iters):
                fn()
            e1.record()
            torch.cuda.synchronize()
            ms = e0.elapsed_time(e1) / iters
            out[mode] = dict(ms=round(ms, 4), tflops=round(flops / ms / 1e9, 1),
                             frac=round(flops / ms / 1e9 / FP8_PEAK_TFLOPS, 4))
        except Exception as err:  # a torch build without fp8 _scaled_mm on this device
            out[mode] = {"error": repr(err)[:160]}
    return out


def attention_bench(args):
    """One prefix-shared attention layer (64 rows x 256-token prefix).

    Inputs: Q, K, V ~ N(0, 1)/sqrt(128) bf16; the prefix's 16 pages and the
    rows' own pages are a seeded random permutation of the arena's pages.
    Timed per layer with HIP events on the launch stream:
      unified   KV scatter of the rows into their pages + the paged causal
                call (fp8 out) over prefix + own pages;
      tree      the fused kernel: node (prefix pages) + own rows, one softmax;
      two_pass  call A (own rows) + call B (node, stacked) + merge_attn_quant.
    """
    import numpy as np
    import torch

    from oracle import ops as oops
    from quail_amd import kernels as K
    from quail_amd import layout

    rng = np.random.default_rng(args.seed)
    n_q, n_kv, d, page, prefix, rows = 32, 8, 128, 16, 256, 64
    suf = rng.integers(32, 257, size=rows)
    T = int(suf.sum())
    own_pages = [-(-int(n) // page) for n in suf]
    n_pages = prefix // page + sum(own_pages) + 8
    perm = rng.permutation(n_pages).astype(np.int32)
    node_pages = perm[:prefix // page]
    at = prefix // page
    table_u = np.zeros((rows, (prefix + 256) // page), dtype=np.int32)
    dst = []
    for r, n in enumerate(suf):
        mine = perm[at:at + own_pages[r]]
        at += own_pages[r]
        table_u[r, :prefix // page] = node_pages
        table_u[r, prefix // page:prefix // page + own_pages[r]] = mine
        j = np.arange(int(n))
        dst.append(mine[j // page].astype(np.int64) * page + j % page)
    dst = np.concatenate(dst)
    cu = np.concatenate([[0], np.cumsum(suf)]).astype(np.int32)
    g = torch.Generator().manual_seed(args.seed)
    sd = 1 / np.sqrt(d)
    q = (torch.randn(T, n_q, d, generator=g) * sd).to(torch.bfloat16)
    k3 = (torch.randn(T, n_kv, d, generator=g) * sd).to(torch.bfloat16)
    v3 = (torch.randn(T, n_kv, d, generator=g) * sd).to(torch.bfloat16)
    k_rows = torch.zeros(n_pages * page, n_kv, d, dtype=torch.bfloat16)
    v_rows = torch.zeros(n_pages * page, n_kv, d, dtype=torch.bfloat16)
    node_rows = torch.from_numpy(node_pages[np.arange(prefix) // page].astype(np.int64) * page
                                 + np.arange(prefix) % page)
    k_rows[node_rows] = (torch.randn(prefix, n_kv, d, generator=g) * sd).to(torch.bfloat16)
    v_rows[node_rows] = (torch.randn(prefix, n_kv, d, generator=g) * sd).to(torch.bfloat16)
    dev = "cuda"
    kp = layout.k_pool_from_rows(k_rows).to(dev)
    vp = layout.v_pool_from_rows(v_rows).to(dev)
    qd, kd, vd = q.to(dev), k3.to(dev), v3.to(dev)
    cu_d = torch.from_numpy(cu).to(dev)
    used_u = torch.from_numpy((prefix + suf).astype(np.int32)).to(dev)
    tab_u = torch.from_numpy(table_u).to(dev)
    src_d = torch.arange(T, dtype=torch.int64, device=dev)
    dst_d = torch.from_numpy(dst).to(dev)
    seg_read = torch.zeros(rows, dtype=torch.int32, device=dev)
    node_tab = torch.from_numpy(node_pages[None, :].copy()).to(dev)
    node_used = torch.tensor([prefix], dtype=torch.int32, device=dev)
    scale = 1 / np.sqrt(d)
    a_len = (cu_d[1:] - cu_d[:-1]).to(torch.int32)
    all_rows = torch.arange(T, dtype=torch.int64, device=dev)
    source = torch.arange(T, dtype=torch.int32, device=dev)
    cu_b = torch.tensor([0, T], dtype=torch.int32, device=dev)

    def unified():
        K.kv_row_scatter(kd, vd, kp, vp, src_d, dst_d)
        return K.attention_fp8(qd, cu_d, used_u, n_queries=T, max_q=int(suf.max()),
                               softmax_scale=scale, causal=True, k_pool=kp, v_pool=vp,
                               table=tab_u, n_kv=n_kv)

    def tree():
        return K.tree_attention(qd, kd, vd, cu_d, seg_read, softmax_scale=scale, k_pool=kp,
                                v_pool=vp, table=node_tab, used=node_used)

    def tree_resident():
        return K.tree_attention(qd, kd, vd, cu_d, seg_read, softmax_scale=scale, k_pool=kp,
                                v_pool=vp, table=node_tab, used=node_used, resident=True)

    def two_pass():
        out_a, lse_a = K.attention(qd, cu_d, a_len, n_queries=T, max_q=int(suf.max()),
                                   softmax_scale=scale, causal=True, k_rows=kd, v_rows=vd,
                                   cu_k=cu_d, n_kv=n_kv, want_lse=True)
        out_b, lse_b = K.attention(qd, cu_b, node_used, n_queries=T, max_q=T,
                                   softmax_scale=scale, causal=False, k_pool=kp, v_pool=vp,
                                   table=node_tab, q_rows=all_rows, n_kv=n_kv, want_lse=True)
        return K.merge_attn_quant(out_a, lse_a, out_b, lse_b, source)

    pairs = int((suf * prefix + suf * (suf + 1) // 2).sum())
    flops = 4.0 * n_q * d * pairs
    # unique HBM bytes: Q in (bf16), O out (e4m3 + scales), node K/V once,
    # the rows' own K/V once
    unique = T * n_q * d * 2 + T * n_q * (d + 4) + (prefix + T) * n_kv * d * 4
    stream = torch.cuda.current_stream()
    results = {}
    iters = max(args.steps, 1) * 10
    for name, fn in (("unified", unified), ("tree", tree), ("tree_resident", tree_resident),
                     ("two_pass", two_pass)):
        for _ in range(max(args.warmup, 1) * 3):
            fn()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record(stream)
        for _ in range(iters):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / iters
        results[name] = dict(us_per_layer=round(us, 2),
                             tflops=round(flops / us / 1e6, 1),
                             frac_bf16_peak=round(flops / us / 1e6 / BF16_PEAK_TFLOPS, 4),
                             unique_gbps=round(unique / us / 1e3, 1))
    # the node-resident kernel gives the streaming kernel's bits
    (q1, s1), (q2, s2) = tree(), tree_resident()
    same_bits = bool(torch.equal(q1.view(torch.uint8), q2.view(torch.uint8))
                     and torch.equal(s1, s2))
    # parity: the fused kernel (bf16 out) against the fp32 oracle, all rows
    got = K.tree_attention(qd, kd, vd, cu_d, seg_read, softmax_scale=scale, k_pool=kp,
                           v_pool=vp, table=node_tab, used=node_used, fp8=False).float().cpu()
    cpu = None
    threads, cpu_model = host_cpu()
    torch.set_num_threads(threads)
    t0 = time.perf_counter()
    want = oops.tree_attention(q, k3, v3, cu, torch.zeros(rows, dtype=torch.int32), k_rows,
                               v_rows, torch.from_numpy(node_pages[None, :].copy()),
                               torch.tensor([prefix], dtype=torch.int32), scale)
    cpu_s = time.perf_counter() - t0
    err = (got - want).abs().max().item()
    # the unified path computes the same function (prefix pages + own pages,
    # bottom-right causal): its bf16 output against the same oracle
    K.kv_row_scatter(kd, vd, kp, vp, src_d, dst_d)
    got_u = K.attention(qd, cu_d, used_u, n_queries=T, max_q=int(suf.max()),
                        softmax_scale=scale, causal=True, k_pool=kp, v_pool=vp, table=tab_u,
                        n_kv=n_kv)[0].float().cpu()
    err_u = (got_u - want).abs().max().item()
    if not args.no_cpu_baseline:
        cpu = {"value": round(flops / cpu_s / 1e12, 4), "unit": "TFLOP/s", "cores": threads,
               "cpu_model": cpu_model, "kind": "port",
               "sample": (f"oracle tree attention (torch fp32) over the whole layer: "
                          f"{cpu_s * 1e6:.0f} us per layer")}
    best = results["tree"]
    line = {
        "metric": "prefix-shared attention TFLOP/s per layer (64 rows x 256-token prefix, "
                  "32/8 heads, d 128) on 1 GPU; % of bf16 MFMA peak",
        "value": best["tflops"], "unit": "TFLOP/s", "n_gpus": 1, "steps": iters,
        "warmup": max(args.warmup, 1) * 3, "ms_per_step": round(best["us_per_layer"] / 1e3, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "one attention layer over a paged KV arena: 64 rows sharing a "
                               "256-token prefix, suffixes U[32, 256], 32 q / 8 kv heads, "
                               "head_dim 128, page 16, pages randomly permuted",
                   "rows": rows, "query_rows": T, "pairs": pairs, "gflop": round(flops / 1e9, 2),
                   "unique_bytes": unique},
        "roofline": {"bound": "mfma", "achieved": best["tflops"], "peak": BF16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": best["frac_bf16_peak"], "traffic": None,
                     "kernel": "qh attn_tree_kernel (fused node + own rows, fp8 out)"},
        "paths": results,
        "parity_max_abs_vs_oracle": round(err, 6),
        "unified_parity_max_abs_vs_oracle": round(err_u, 6),
        "tree_resident_bit_identical": same_bits,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def join_bench(args):
    """The AI join workload: anchors x partners pairs, one TRUE/FALSE per pair."""
    import torch

    from quail_amd.aiif import JoinRunner, synthetic_join_workload
    from quail_amd.model import build_random_qwen3
    from quail_amd.specs import MI355X, QWEN3_4B_FP8
    from dataclasses import replace

    attention = args.attention or "tree"
    spec = QWEN3_4B_FP8 if args.layers is None else replace(QWEN3_4B_FP8, layers=args.layers)
    t_build = time.perf_counter()
    model = build_random_qwen3(spec, seed=args.seed, device="cuda", max_pos=2048)
    anchors, frame, partners = synthetic_join_workload(args.anchors, args.partners,
                                                       seed=args.seed, vocab=spec.vocab)
    clock = KernelClock(torch)
    clock.n_q, clock.d, clock.n_kv = spec.n_q, spec.d_head, spec.n_kv
    runner = JoinRunner(model, spec, device_spec=MI355X, n_pages=args.arena_pages,
                        attention_mode=attention, gemm_hook=clock.gemm_hook,
                        attention_hook=clock.attention_hook, tree_kernel=args.tree_kernel)
    torch.cuda.synchronize()
    build_s = time.perf_counter() - t_build
    for _ in range(args.warmup):
        runner.run_join(anchors, frame, partners)
    clock.active = True
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    results = [runner.run_join(anchors, frame, partners) for _ in range(args.steps)]
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    clock.active = False
    k = clock.summary()
    answers, stats = results[-1]
    steady = all(r[0] == answers for r in results)
    pairs = stats["rows"]
    ms_per_step = wall / args.steps * 1e3
    cpu = None
    if not args.no_cpu_baseline and args.cpu_pairs > 0:
        threads, cpu_model = host_cpu()
        try:
            base = cpu_baseline_join(model, spec, anchors[0], frame,
                                     partners[:args.cpu_pairs], threads)
            gpu_bits = answers[0][0][:args.cpu_pairs]
            agree = sum(int(b == a) for b, a in zip(base["bits"], gpu_bits))
            cpu = {"value": round(base["rows_per_s"], 4), "unit": "rows/s",
                   "cores": threads, "cpu_model": cpu_model, "kind": "port",
                   "sample": (f"oracle forward (torch fp32, fp8 dequantized) of anchor 0 "
                              f"(prefix + frame, once) and its first {args.cpu_pairs} "
                              f"partners, unified attention: {base['tokens']} tokens, "
                              f"{base['wall_s']:.1f} s; decisions agree with the GPU on "
                              f"{agree}/{args.cpu_pairs} (margins "
                              f"{[round(m, 3) for m in base['margins']]})")}
        except Exception as exc:
            cpu = {"value": None, "unit": "rows/s", "cores": 0, "kind": "port",
                   "sample": f"failed: {exc!r}"}
    line = {
        "metric": "rows/s + prefill tok/s, Qwen3-4B fp8 AI join on 1 GPU (row = pair); "
                  "attn/GEMM % of MFMA peak",
        "value": round(pairs * args.steps / wall, 2), "unit": "rows/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_per_step, 1),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp8",
        "data": "synthetic",
        "config": {"workload": (f"AI join, Qwen3-4B-arch fp8 random init, {spec.layers} "
                                f"layers, {args.anchors} x {args.partners} pairs, 48-token "
                                f"root + left doc (lognormal median 120) anchors, 8-token "
                                f"frame, partners = 4-token label + right doc (lognormal "
                                f"median 120, cap 512) + 16-token tail, {attention} "
                                f"attention"),
                   "pairs": pairs, "anchors": args.anchors, "partners": args.partners,
                   "tree_kernel": args.tree_kernel if attention == "tree" else None,
                   "layers": spec.layers, "fresh_tokens": stats["fresh_tokens"],
                   "input_tokens": stats["input_tokens"], "chunks": stats.get("chunks"),
                   "borrowed_tokens": stats.get("borrowed_tokens"),
                   "chunk_budget": runner.budget, "arena_pages": runner.arena.n_pages},
        "prefill_tok_per_s": round(stats["fresh_tokens"] * args.steps / wall, 1),
        "input_tok_per_s": round(stats["input_tokens"] * args.steps / wall, 1),
        "roofline": {"bound": "mfma", "achieved": round(k["gemm_tflops"], 1),
                     "peak": FP8_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(k["gemm_tflops"] / FP8_PEAK_TFLOPS, 4),
                     "traffic": None, "traffic_source": "not measured for this workload",
                     "algorithmic_bytes_per_launch": round(k["gemm_bytes"] / max(1, k["gemm_launches"])),
                     "kernel": "qh fp8_gemm_kernel (all four projections)"},
        "gemm": {"share_of_step": round(k["gemm_ms"] / (ms_per_step * args.steps), 3),
                 "shapes": k["gemm_shapes"]},
        "attention": {"tflops": round(k["attn_tflops"], 1),
                      "frac_bf16_peak": round(k["attn_tflops"] / BF16_PEAK_TFLOPS, 4),
                      "gather_gbps": round(k["attn_gbps"], 1),
                      "share_of_step": round(k["attn_ms"] / (ms_per_step * args.steps), 3),
                      "calls": k["attn_kinds"]},
        "answers_true": int(sum(sum(row) for row in answers[0].values())),
        "deterministic_across_steps": steady, "build_s": round(build_s, 1),
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()

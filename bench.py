"""Benchmark of the MI355X DiT-block hot path.

One step = one forward pass of the LTX-2-like video DiT block (benchmark config 3: 9216 video
tokens with 3D RoPE + 256 text tokens by cross-attention, D = 4096, 32 heads x 128, GELU MLP x4)
over synthetic seeded inputs already resident in HBM. Prints ONE JSON line:

  value        block throughput, algorithmic TFLOP/s (GEMM 2MNK + attention 4 H Tq Tk Dh)
  ms_per_step  milliseconds per block, from a timed loop with no per-launch instrumentation
  roofline     the dominant kernel's achieved TFLOP/s (its algorithmic FLOPs per launch over its
               average launch time, measured with HIP events on the launch stream in a second
               timed loop over the same block) against the 2.5 PFLOP/s dense bf16 MFMA peak
  cpu_baseline the FP32 numpy restatement of the config-1 block timed on this host's cores

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 3|4|5] [--no-cpu-baseline]

With --denoise-step the step is instead one whole LTX-2 video denoising step (patchify, the
timestep / AdaLN producers, the RoPE tables, --blocks blocks, the output head, the X0
conversion, the Euler update and the finite check) at the config's shape, or at --grid T,H,W
latent tokens; value is then milliseconds per denoising step.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from collections import defaultdict

PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA (AMD published)
PEAK_HBM_GBS = 8000.0


def _kernel_flops(name: str, args: tuple) -> float:
    """Algorithmic FLOPs of one launch from its C arguments (0 for memory-bound kernels)."""
    if name in ("kx_gemm_bf16", "kx_gemm_splitk_bf16"):
        m, n, k = args[7], args[8], args[9]
        return 2.0 * m * n * k
    if name == "kx_qgemm_affine_bf16":
        m, n, k = args[8], args[9], args[10]
        return 2.0 * m * n * k
    if name == "kx_qgemm_affine_tiled_bf16":
        m, n, k = args[7], args[8], args[9]
        return 2.0 * m * n * k
    if name == "kx_attention_fwd_bf16":
        batch, tq, tk, heads, dh = args[8], args[9], args[10], args[11], args[12]
        return 4.0 * batch * heads * tq * tk * dh
    return 0.0


def _kernel_bytes(name: str, args: tuple) -> float:
    """Algorithmic HBM bytes of one launch of a memory-bound kernel (each operand read or written
    once; 0 for the MFMA-bound kernels)."""
    if name == "kx_adaln_norm_bf16":
        rows, dim, kind = args[4], args[5], args[11]
        return rows * dim * ((4 if kind & 16 else 2) + 2) + 2 * dim * 4
    if name == "kx_qk_rmsnorm_rope_bf16":
        rows, dim = args[8], args[9]
        return 2 * rows * dim * (2 + 2) + 2 * rows * (dim // 2) * 4
    if name == "kx_rmsnorm_rope_bf16":
        rows, dim, rope = args[4], args[5], args[11]
        return rows * dim * (2 + 2) + (2 * rows * (dim // 2) * 4 if rope else 0)
    if name == "kx_modulate_bf16":
        return args[4] * args[5] * (2 + 2)
    if name == "kx_table_add_f32":
        count = args[8] * args[9] * args[10] * args[11]
        return count * 4 + (count * (2 if args[3] else 4) if args[2] else 0) + args[10] * args[11] * (2 if args[1] else 4)
    if name == "kx_gemm_bf16" and args[8] <= 64:
        m, n, k = args[7], args[8], args[9]
        return (m * k + n * k + m * n) * 2
    return 0.0


def _kernel_label(name: str, args: tuple) -> str:
    if name == "kx_gemm_bf16":
        return f"gemm m{args[7]} n{args[8]} k{args[9]}"
    if name == "kx_gemm_splitk_bf16":
        return f"gemm splitk{args[18]} m{args[7]} n{args[8]} k{args[9]}"
    if name == "kx_qgemm_affine_bf16":
        return f"qgemm{args[12]} m{args[8]} n{args[9]} k{args[10]}"
    if name == "kx_qgemm_affine_tiled_bf16":
        return f"qgemm{args[10]} tiled m{args[7]} n{args[8]} k{args[9]}"
    if name == "kx_attention_fwd_bf16":
        return f"attention tq{args[9]} tk{args[10]} h{args[11]} d{args[12]}"
    return name.replace("kx_", "").replace("_bf16", "")


def cpu_baseline(budget_s: float = 12.0) -> dict:
    """Config-1 block (1024 + 128 tokens, D = 1024) through the FP32 torch-CPU restatement
    (``oracle/torch_cpu.py``, pinned to the numpy oracle) on the host cores, with
    ``torch.set_num_threads`` at the cores this process may use: median of repeated runs within
    ``budget_s`` seconds."""
    import torch

    from kinomlx_amd import workloads
    from oracle import torch_cpu

    spec = workloads.CONFIGS[1]
    p = workloads.flux_params(spec, 0)
    inputs = workloads.flux_inputs(spec, 0)
    tp = torch_cpu.to_torch({k: v.float().numpy() for k, v in p.items()})
    image = inputs["image"][0].float().contiguous()
    text = inputs["text"][0].float().contiguous()
    rope = tuple(t.float().contiguous() for t in workloads.flux_rope(spec))
    flops = workloads.flop_count(spec)["total"]
    cores = len(os.sched_getaffinity(0))
    threads_before = torch.get_num_threads()
    torch.set_num_threads(cores)
    times = []
    try:
        with torch.no_grad():
            start = time.perf_counter()
            while len(times) < 3 or (time.perf_counter() - start < budget_s and len(times) < 50):
                t0 = time.perf_counter()
                torch_cpu.config1_double_block(tp, image, text, tp["image_mod"], tp["text_mod"], rope,
                                               heads=spec.heads)
                times.append(time.perf_counter() - t0)
    finally:
        torch.set_num_threads(threads_before)
    med = statistics.median(times)
    return {
        "value": round(flops / med / 1e12, 4),
        "unit": "TFLOP/s",
        "cores": cores,
        "kind": "port",
        "sample": f"config-1 block (1024 image + 128 text tokens, D=1024, 16x64, GELU MLP), FP32 torch-CPU "
                  f"restatement, torch.set_num_threads({cores}), median of {len(times)} runs "
                  f"({med * 1e3:.1f} ms/block); CPU restatement (fp32), not reference code",
        "ms_per_block": round(med * 1e3, 2),
    }


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=20)
    parser.add_argument("--warmup", type=int, default=20,
                        help="untimed steps first (the first ~10 blocks after launch run up to 25 %% slower while "
                             "the clock settles)")
    parser.add_argument("--config", type=int, default=3, choices=(3, 4, 5))
    parser.add_argument("--dtype", default="bf16", choices=("bf16", "fp16"),
                        help="activation and weight type of the block (fp16: the reference's default LTX-2 "
                             "transformer dtype); the headline is bf16")
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--breakdown", action="store_true", help="print the per-kernel table to stderr")
    parser.add_argument("--denoise-step", action="store_true",
                        help="time one whole denoising step of the video transformer instead of one block")
    parser.add_argument("--blocks", type=int, default=48, help="blocks of the --denoise-step transformer")
    parser.add_argument("--grid", type=str, default="", help="T,H,W latent grid for --denoise-step")
    parser.add_argument("--audio-tokens", type=int, default=0,
                        help="with --denoise-step: add the audio stream (this many latents, 25 per second) and "
                             "the A/V cross-attention to every block")
    parser.add_argument("--load-checkpoint", action="store_true",
                        help="time loading a --blocks-block checkpoint into HBM, plain and quantized on load")
    parser.add_argument("--launch-log", type=str, default="",
                        help="write one block's launch sequence (labels, FLOPs, bytes) as JSON to this path")
    parser.add_argument("--profile-summary", type=str, default="", metavar="DIR",
                        help="only summarize the rocprofv3 runs under DIR (see profiles/) as a markdown table")
    parser.add_argument("--kernel-table", type=str, default="", metavar="DIR",
                        help="only print, from the rocprofv3 --kernel-trace run under DIR of a --denoise-step run "
                             "with --warmup W and --steps S (W warm-up steps, then S timed steps twice: without and "
                             "with per-launch events), this library's kernels per instantiation as a markdown table")
    parser.add_argument("--compare-rope-fold", action="store_true",
                        help="only time LTX's Q/K norm + RoPE folded into the QKV GEMM epilogue against the "
                             "separate pass, and exit")
    parser.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                        help="only run 5 device-to-device copies of MIB MiB (the known-size kernel that "
                             "scales the FETCH_SIZE / WRITE_SIZE counters) and exit")
    args = parser.parse_args()
    if args.profile_summary:
        return profile_summary(args.profile_summary, args.warmup)
    if args.kernel_table:
        return kernel_table(args.kernel_table, args.warmup + 2 * args.steps)
    if args.calibrate_copy:
        import torch

        src = torch.ones(args.calibrate_copy << 19, dtype=torch.bfloat16, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibrate_copy_bytes": src.numel() * 2}))
        return 0
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (run with --gpus 1)", file=sys.stderr)
        return 2
    if args.compare_rope_fold:
        return rope_fold_main(args)
    if args.denoise_step:
        return denoise_main(args)
    if args.load_checkpoint:
        return load_main(args)

    import torch

    from kinomlx_amd import _lib, workloads
    from kinomlx_amd.ltx2.rope import precompute_freqs_cis
    from kinomlx_amd.ltx2.transformer import TransformerArgs

    device = torch.device("cuda:0")
    spec = workloads.CONFIGS[args.config]
    act = torch.float16 if args.dtype == "fp16" else torch.bfloat16
    if spec.bits and act != torch.bfloat16:
        print("--dtype fp16 runs the dense configs only (the quantized layers carry bf16 scales)", file=sys.stderr)
        return 2
    p = workloads.ltx_params(spec, 0, act)
    if spec.bits:
        p = workloads.quantize_ltx_params(p, spec.bits, spec.group_size)
    inputs = workloads.ltx_inputs(spec, 0, act)
    block = workloads.build_ltx_block(spec, p, device)
    pe = precompute_freqs_cis(inputs["positions"].to(device), dim=spec.dim, theta=10000.0,
                              max_pos=(20, 2048, 2048), use_middle_indices_grid=True,
                              num_attention_heads=spec.heads)
    video = TransformerArgs(x=inputs["x"].to(device), context=inputs["context"].to(device),
                            timesteps=p["timesteps"].to(device), positional_embeddings=pe)
    del p

    def step():
        return block(video)[0].x

    for _ in range(args.warmup):
        out = step()
    torch.cuda.synchronize()
    if not torch.isfinite(out).all():
        print("non-finite block output", file=sys.stderr)
        return 1

    # headline: the block alone, no per-launch events
    begin, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    begin.record()
    for _ in range(args.steps):
        out = step()
    end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    ms_per_step = begin.elapsed_time(end) / args.steps

    # breakdown: a second timed loop with HIP events around every launch (on its stream)
    timer = _lib.LaunchTimer()
    _lib.set_timer(timer)
    b2, e2 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    b2.record()
    for _ in range(args.steps):
        out = step()
    e2.record()
    torch.cuda.synchronize()
    _lib.set_timer(None)
    instrumented_ms = b2.elapsed_time(e2) / args.steps

    per_kernel: dict[str, list[float]] = defaultdict(list)
    flops_of: dict[str, float] = {}
    name_of: dict[str, str] = {}
    # an fp16 entry point takes its bf16 twin's arguments: label and count it as that one
    records = [(n[:-4] + "_bf16" if n.endswith("_f16") else n, a, ms) for n, a, ms in timer.durations_ms()]
    for name, cargs, ms in records:
        label = _kernel_label(name, cargs)
        per_kernel[label].append(ms)
        flops_of[label] = _kernel_flops(name, cargs)
        name_of[label] = name
    kernel_ms_per_step = {k: sum(v) / args.steps for k, v in per_kernel.items()}
    if args.launch_log:
        per_block = len(records) // args.steps
        with open(args.launch_log, "w") as fh:
            json.dump([{"label": _kernel_label(n, a), "entry": n, "flops": _kernel_flops(n, a),
                        "bytes": _kernel_bytes(n, a)} for n, a, _ in records[:per_block]], fh, indent=1)
    dominant = max(kernel_ms_per_step, key=kernel_ms_per_step.get)
    dom_avg_ms = statistics.mean(per_kernel[dominant])
    dom_tflops = flops_of[dominant] / (dom_avg_ms * 1e-3) / 1e12

    # HBM bytes per launch of the dominant kernel, from the committed rocprofv3 FETCH_SIZE /
    # WRITE_SIZE summary of the same workload (None when no summary covers the kernel)
    traffic = None
    traffic_file = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "roofline_traffic.json")
    if os.path.exists(traffic_file):
        with open(traffic_file) as fh:
            entry = json.load(fh).get(dominant)
        if entry:
            traffic = entry["fetch_bytes"] + entry["write_bytes"]

    flops = workloads.flop_count(spec)
    attn_ms = sum(v for k, v in kernel_ms_per_step.items() if name_of[k] == "kx_attention_fwd_bf16")
    gemm_ms = sum(v for k, v in kernel_ms_per_step.items()
                  if name_of[k] in ("kx_gemm_bf16", "kx_gemm_splitk_bf16", "kx_qgemm_affine_bf16",
                                    "kx_qgemm_affine_tiled_bf16"))
    other_ms = sum(kernel_ms_per_step.values()) - attn_ms - gemm_ms
    attn_tflops = flops["attention"] / (attn_ms * 1e-3) / 1e12
    gemm_tflops = flops["gemm"] / (gemm_ms * 1e-3) / 1e12
    value = flops["total"] / (ms_per_step * 1e-3) / 1e12

    if args.breakdown:
        for label, ms in sorted(kernel_ms_per_step.items(), key=lambda kv: -kv[1]):
            f = flops_of[label]
            extra = f"  {f / (statistics.mean(per_kernel[label]) * 1e-3) / 1e12:7.1f} TFLOP/s" if f else ""
            print(f"{ms:8.3f} ms/step  x{len(per_kernel[label]) // args.steps}  {label}{extra}", file=sys.stderr)

    result = {
        "metric": "DiT block ms + attention/GEMM TFLOP/s (% bf16 MFMA peak), 9216-token block",
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": args.dtype,
        "data": "synthetic (seeded N(0,0.02) weights, N(0,1) activations; no checkpoint)",
        "config": {
            "workload": f"LTX2-like video DiT block, BASELINE config {args.config}",
            "video_tokens": spec.tokens,
            "latent_grid_thw": list(spec.grid),
            "text_tokens": spec.text_tokens,
            "dim": spec.dim,
            "heads": spec.heads,
            "head_dim": spec.head_dim,
            "ff_mult": spec.ff_mult,
            "weights": f"int{spec.bits} affine g{spec.group_size}" if spec.bits else "bf16",
            "batch": 1,
        },
        "block_ms": round(ms_per_step, 4),
        "attention": {"ms": round(attn_ms, 4), "tflops": round(attn_tflops, 1),
                      "frac_of_peak": round(attn_tflops / PEAK_BF16_TFLOPS, 4)},
        "gemm": {"ms": round(gemm_ms, 4), "tflops": round(gemm_tflops, 1),
                 "frac_of_peak": round(gemm_tflops / PEAK_BF16_TFLOPS, 4)},
        "memory_bound_ms": round(other_ms, 4),
        "instrumented_ms_per_step": round(instrumented_ms, 4),
        "wall_s": round(wall, 3),
        "roofline": {
            "kernel": dominant,
            "bound": "mfma",
            "achieved": round(dom_tflops, 1),
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(dom_tflops / PEAK_BF16_TFLOPS, 4),
            "traffic": traffic,
            "avg_launch_ms": round(dom_avg_ms, 4),
        },
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline()
    print(json.dumps(result))
    return 0


_DISPATCHES = {"kx_gemm_splitk_bf16": 2, "kx_gemm_splitk_noalloc_bf16": 2, "kx_attention_split_fwd_bf16": 2,
               "kx_all_finite": 2}


def profile_summary(root: str, warmup: int = 0) -> int:
    """Markdown table of one block's kernels from rocprofv3 runs of this script: ``root/trace``
    (``--kernel-trace``), ``root/mfma`` (``--pmc SQ_VALU_MFMA_BUSY_CYCLES GRBM_GUI_ACTIVE``),
    ``root/fetch`` / ``root/write`` (``FETCH_SIZE`` / ``WRITE_SIZE``), ``root/copy_fetch`` /
    ``root/copy_write`` (the same counters over ``--calibrate-copy 1024``) and ``root/launches.json``
    (``--launch-log``). Dispatches of the kx kernels are matched to the block's launch sequence by
    position (every block launches the same sequence), so launches of one kernel with different
    shapes (self- and cross-attention) get their own rows. The first ``warmup`` blocks of each run
    (its untimed warm-up) are left out of the means."""
    import csv
    import glob

    with open(os.path.join(root, "launches.json")) as fh:
        launches = json.load(fh)
    # kernel dispatches per launch: the split forms add their reduction / merge pass, the finite
    # check its flag initialisation
    groups, period = [], 0
    for entry in launches:
        count = _DISPATCHES.get(entry.get("entry", ""), 1)
        groups.append(range(period, period + count))
        period += count

    def kx_rows(sub, pattern):
        files = glob.glob(os.path.join(root, sub, "**", pattern), recursive=True)
        if not files:
            return None
        with open(files[0]) as fh:
            return [r for r in csv.DictReader(fh)]

    def per_position(values):
        # values: per kx dispatch in order -> list per launch position (blocks aligned at the end)
        usable = len(values) - len(values) % period
        vals = values[len(values) - usable:]
        out = [[] for _ in range(period)]
        for i, v in enumerate(vals):
            out[i % period].append(v)
        return [lst[warmup:] if len(lst) > warmup else lst for lst in out]

    trace = sorted(kx_rows("trace", "*kernel_trace.csv"), key=lambda r: int(r["Dispatch_Id"]))
    durations, names = [], []
    for r in trace:
        if "kx::" in r["Kernel_Name"]:
            durations.append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
            names.append(r["Kernel_Name"])
    dur = per_position(durations)
    kname = per_position(names)

    def counters(sub, names_wanted):
        rows = kx_rows(sub, "*counter_collection.csv")
        if rows is None:
            return {}
        per = defaultdict(lambda: defaultdict(float))
        order = []
        for r in rows:
            if "kx::" not in r["Kernel_Name"] and "copy" not in sub:
                continue
            d = int(r["Dispatch_Id"])
            if d not in per:
                order.append(d)
            per[d][r["Counter_Name"]] += float(r["Counter_Value"])
        return {c: [per[d].get(c, 0.0) for d in sorted(order)] for c in names_wanted}

    mfma = counters("mfma", ["SQ_VALU_MFMA_BUSY_CYCLES", "GRBM_GUI_ACTIVE"])
    fetch = counters("fetch", ["FETCH_SIZE"]).get("FETCH_SIZE")
    write = counters("write", ["WRITE_SIZE"]).get("WRITE_SIZE")
    copy_f = counters("copy_fetch", ["FETCH_SIZE"]).get("FETCH_SIZE")
    copy_w = counters("copy_write", ["WRITE_SIZE"]).get("WRITE_SIZE")
    # FETCH_SIZE / WRITE_SIZE are KiB per dispatch; scale by what they read for a 1 GiB copy
    fscale = (1 << 30) / (max(copy_f) * 1024) if copy_f else None
    wscale = (1 << 30) / (max(copy_w) * 1024) if copy_w else None
    busy = per_position(mfma["SQ_VALU_MFMA_BUSY_CYCLES"]) if mfma else None
    gui = per_position(mfma["GRBM_GUI_ACTIVE"]) if mfma else None
    fpos = per_position(fetch) if fetch else None
    wpos = per_position(write) if write else None

    print(f"Counter scale from a 1 GiB device copy: FETCH_SIZE x{fscale:.3f}, WRITE_SIZE x{wscale:.3f}." if fscale
          else "No copy calibration.")
    print()
    print("| # | launch | kernel | avg us | TFLOP/s | of 2.5 PF | MFMA busy | algorithmic GB/s | of 8 TB/s "
          "| HBM fetch MB | HBM write MB |")
    print("|---|---|---|---|---|---|---|---|---|---|---|")
    total_us = 0.0
    for i, entry in enumerate(launches):
        g = groups[i]
        avg = sum(statistics.mean(dur[j]) for j in g)
        total_us += avg
        kernel = " + ".join(kname[j][0].replace("kx::(anonymous namespace)::", "").split("(")[0] for j in g)
        tf = entry["flops"] / (avg * 1e-6) / 1e12 if entry["flops"] else None
        gbs = entry["bytes"] / (avg * 1e-6) / 1e9 if entry["bytes"] else None
        b = None
        if busy:
            # SQ_VALU_MFMA_BUSY_CYCLES sums the 1024 SIMDs; GRBM_GUI_ACTIVE sums the 8 XCDs' cycles
            cyc = sum(statistics.mean(gui[j]) for j in g) / 8
            b = sum(statistics.mean(busy[j]) for j in g) / (1024 * cyc) if cyc else None
        fm = sum(statistics.mean(fpos[j]) for j in g) * 1024 * fscale / 1e6 if fpos and fscale else None
        wm = sum(statistics.mean(wpos[j]) for j in g) * 1024 * wscale / 1e6 if wpos and wscale else None

        def f(x, fmt):
            return fmt.format(x) if x is not None else "-"

        print(f"| {i} | {entry['label']} | `{kernel}` | {avg:.1f} | {f(tf, '{:.0f}')} | "
              f"{f(tf / PEAK_BF16_TFLOPS if tf else None, '{:.3f}')} | {f(b if tf else None, '{:.2f}')} | "
              f"{f(gbs, '{:.0f}')} | {f(gbs / PEAK_HBM_GBS if gbs else None, '{:.2f}')} | "
              f"{f(fm, '{:.1f}')} | {f(wm, '{:.1f}')} |")
    print(f"\nSum of the block's kernels: {total_us / 1e3:.3f} ms (means over the {len(dur[0])} timed blocks, "
          f"after {warmup} warm-up blocks).")

    # further counter passes (root/ctr_<name>, each a --pmc run of the same command): the mean per
    # launch of each counter, for the launches that carry FLOPs (GEMMs and attention); busy and
    # stall counters that sum the CUs' cycles are also given per CU-cycle (GRBM_GUI_ACTIVE / 8 XCDs
    # x 256 CUs), SQ_VALU_MFMA_BUSY_CYCLES per SIMD-cycle, and TCP_TCC_READ_REQ_LATENCY per request
    per_cu = {"TA_TA_BUSY", "TD_TD_BUSY", "TD_TC_STALL", "TA_ADDR_STALLED_BY_TC_CYCLES", "TCP_PENDING_STALL_CYCLES",
              "TCP_UTCL1_STALL_INFLIGHT_MAX", "SQ_LDS_BANK_CONFLICT"}
    for sub in sorted(d for d in os.listdir(root) if d.startswith("ctr_")):
        names: list[str] = []
        rows = kx_rows(sub, "*counter_collection.csv") or []
        for r in rows:
            if r["Counter_Name"] not in names:
                names.append(r["Counter_Name"])
        vals = counters(sub, names)
        if not vals or not vals.get(names[0]):
            continue
        pos = {c: per_position(v) for c, v in vals.items()}
        shown = [c for c in names if c != "GRBM_GUI_ACTIVE"]
        print(f"\nCounter pass `{sub[4:]}` (mean per launch):\n")
        print("| # | launch | " + " | ".join(shown) + " |")
        print("|---|---|" + "---|" * len(shown))
        for i, entry in enumerate(launches):
            if not entry["flops"]:
                continue
            g = groups[i]
            gui = sum(statistics.mean(pos["GRBM_GUI_ACTIVE"][j]) for j in g) / 8 if "GRBM_GUI_ACTIVE" in pos else 0
            cells = []
            for c in shown:
                v = sum(statistics.mean(pos[c][j]) for j in g)
                if c in per_cu and gui:
                    cells.append(f"{v / (256 * gui):.3f}/CU-cyc")
                elif c == "SQ_VALU_MFMA_BUSY_CYCLES" and gui:
                    cells.append(f"{v / (1024 * gui):.3f}/SIMD-cyc")
                elif c == "TCP_TCC_READ_REQ_LATENCY" and "TCP_TCC_READ_REQ" in pos:
                    req = sum(statistics.mean(pos["TCP_TCC_READ_REQ"][j]) for j in g)
                    cells.append(f"{v / req:.0f} cyc/req" if req else "-")
                else:
                    cells.append(f"{v:.4g}")
            print(f"| {i} | {entry['label']} | " + " | ".join(cells) + " |")
    return 0


def kernel_table(root: str, steps: int) -> int:
    """Per kernel instantiation (name with template arguments, workgroups over both grid axes):
    calls, calls per step, mean / min / max duration and ms per step over the ``steps`` steps of a
    rocprofv3 kernel trace; this library's kernels only."""
    import csv
    import glob
    import re

    files = glob.glob(os.path.join(root, "**", "*kernel_trace.csv"), recursive=True)
    if not files:
        print(f"no kernel trace under {root}", file=sys.stderr)
        return 1
    agg: dict[tuple[str, int], list[float]] = defaultdict(list)
    with open(files[0]) as fh:
        for r in csv.DictReader(fh):
            name = r["Kernel_Name"]
            if "kx::" not in name:
                continue
            name = name.replace("kx::(anonymous namespace)::", "")
            m = re.match(r"void ([\w:]+(<[^()]*>)?)\(", name)
            short = m.group(1) if m else name[:70]
            wg = (int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"])) // (int(r["Workgroup_Size_X"]) * int(r["Workgroup_Size_Y"]))
            agg[(short, wg)].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    total = sum(sum(v) for v in agg.values())
    print("| kernel | workgroups | calls | calls/step | avg us | min us | max us | ms/step | share |")
    print("|---|---|---|---|---|---|---|---|---|")
    for (k, wg), v in sorted(agg.items(), key=lambda kv: -sum(kv[1])):
        print(f"| `{k}` | {wg} | {len(v)} | {len(v) // steps} | {sum(v) / len(v):.1f} | {min(v):.1f} | {max(v):.1f} | "
              f"{sum(v) / steps / 1e3:.3f} | {100 * sum(v) / total:.1f}% |")
    print(f"\nSum of this library's kernels: {total / steps / 1e3:.1f} ms per step.")
    return 0


def load_main(args) -> int:
    """Checkpoint -> HBM: the staged safetensors loader and quantize-on-load, on a synthetic
    reference-named checkpoint written to a temporary directory (so read from the page cache:
    this times the host-memory -> HBM path, not a disk)."""
    import tempfile
    from pathlib import Path

    import torch
    from safetensors.torch import save_file

    from kinomlx_amd import _lib, workloads
    from kinomlx_amd.io import inspect_safetensors, load_to_device
    from kinomlx_amd.ltx2.weights import load_transformer

    device = torch.device("cuda:0")
    spec = workloads.CONFIGS[3]
    model = workloads.random_ltx_model(spec, args.blocks, device, seed=3)
    tensors = {}
    for i, block in enumerate(model.transformer_blocks):
        pre = f"model.diffusion_model.transformer_blocks.{i}"
        for a in ("attn1", "attn2"):
            attn = getattr(block, a)
            for n in ("to_q", "to_k", "to_v", "to_out", "to_gate_logits"):
                layer = getattr(attn, n)
                src = f"{pre}.{a}.{n}" + (".0" if n == "to_out" else "")
                tensors[f"{src}.weight"] = layer.weight.cpu().contiguous()
                tensors[f"{src}.bias"] = layer.bias.cpu()
            tensors[f"{pre}.{a}.q_norm.weight"] = attn.q_norm.weight.cpu()
            tensors[f"{pre}.{a}.k_norm.weight"] = attn.k_norm.weight.cpu()
        for src, layer in ((f"{pre}.ff.net.0.proj", block.ff.project_in.proj), (f"{pre}.ff.net.2", block.ff.project_out)):
            tensors[f"{src}.weight"] = layer.weight.cpu().contiguous()
            tensors[f"{src}.bias"] = layer.bias.cpu()
        tensors[f"{pre}.scale_shift_table"] = block.scale_shift_table.cpu()
        tensors[f"{pre}.prompt_scale_shift_table"] = block.prompt_scale_shift_table.cpu()
    top = {"patchify_proj": model.patchify_proj, "proj_out": model.proj_out,
           "adaln_single.linear": model.adaln_single.linear,
           "prompt_adaln_single.linear": model.prompt_adaln_single.linear}
    for prefix in ("adaln_single", "prompt_adaln_single"):
        emb = getattr(model, prefix).emb.timestep_embedder
        top[f"{prefix}.emb.timestep_embedder.linear_1"] = emb.linear_1
        top[f"{prefix}.emb.timestep_embedder.linear_2"] = emb.linear_2
    for name, layer in top.items():
        tensors[f"model.diffusion_model.{name}.weight"] = layer.weight.cpu().contiguous()
        tensors[f"model.diffusion_model.{name}.bias"] = layer.bias.cpu()
    tensors["model.diffusion_model.scale_shift_table"] = model.scale_shift_table.cpu()
    del model
    torch.cuda.empty_cache()
    with tempfile.TemporaryDirectory(dir="/tmp") as tmp:
        path = Path(tmp) / "ltx.safetensors"
        save_file(tensors, str(path))
        del tensors
        payload = inspect_safetensors(path).payload_bytes
        load_to_device(path, device)  # warm the page cache and the allocator
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        loaded = load_to_device(path, device)
        torch.cuda.synchronize()
        raw_s = time.perf_counter() - t0
        del loaded
        torch.cuda.empty_cache()
        t0 = time.perf_counter()
        plain = load_transformer(path, device)
        torch.cuda.synchronize()
        plain_s = time.perf_counter() - t0
        del plain
        torch.cuda.empty_cache()
        timer = _lib.LaunchTimer()
        _lib.set_timer(timer)
        t0 = time.perf_counter()
        quant = load_transformer(path, device, quantize_bits=4)
        torch.cuda.synchronize()
        quant_s = time.perf_counter() - t0
        _lib.set_timer(None)
        del quant
    q = [(cargs, ms) for name, cargs, ms in timer.durations_ms() if name == "kx_quantize_affine_bf16"]
    q_bytes = sum(c[5] * c[6] * 2 + c[5] * c[6] * 4 // 8 + 4 * c[5] * c[6] // 64 for c, _ in q)
    q_ms = sum(ms for _, ms in q)
    result = {
        "metric": "LTX-2 checkpoint -> HBM load GB/s (safetensors, page-cached) and quantize-on-load GB/s",
        "value": round(payload / raw_s / 1e9, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "higher_is_better": True,
        "dtype": "bf16 -> int4 g64",
        "data": "synthetic reference-named checkpoint (N(0,0.02) weights), written to /tmp then read back",
        "config": {"workload": f"LTX2-like video transformer, {args.blocks} blocks, config-3 block shape",
                   "payload_bytes": payload},
        "load_to_device_s": round(raw_s, 3),
        "load_transformer_bf16_s": round(plain_s, 3),
        "load_transformer_int4_s": round(quant_s, 3),
        "quantize_kernel": {"launches": len(q), "ms": round(q_ms, 3),
                            "hbm_gbs": round(q_bytes / (q_ms * 1e-3) / 1e9, 1) if q_ms else None},
    }
    print(json.dumps(result))
    return 0


def rope_fold_main(args) -> int:
    """The config-3 self-attention Q/K/V projection (9216 x 12288 x 4096, bias) three ways: plain;
    with the per-head RMSNorm + RoPE epilogue of the fused QKV GEMM (``kx_gemm_qknorm_rope_bf16``,
    cos/sin tables of LTX's size: 64 fp32 per head and token); and the separate
    ``kx_qk_rmsnorm_rope_bf16`` pass over its Q and K columns that LTX runs. LTX's Q/K norms span
    the whole 4096-wide row, so a folded LTX epilogue would cost at least the per-head epilogue plus
    a cross-tile reduction: the fold pays only if ``epilogue_extra_us`` stays below
    ``separate_pass_us``. Timing only (the inputs are random)."""
    import torch

    from kinomlx_amd import _lib, workloads
    from kinomlx_amd.kernels import mpp_linear

    _lib.load()
    device = torch.device("cuda:0")
    spec = workloads.CONFIGS[3]
    m, d, half = spec.tokens, spec.dim, spec.head_dim // 2
    g = torch.Generator(device=device).manual_seed(0)
    a = torch.randn(m, d, device=device, generator=g).to(torch.bfloat16)
    w = (torch.randn(3 * d, d, device=device, generator=g) * 0.02).to(torch.bfloat16)
    b = (torch.randn(3 * d, device=device, generator=g) * 0.02).to(torch.bfloat16)
    norm_w = torch.ones(d, device=device, dtype=torch.bfloat16)
    qkv = torch.empty(m, 3 * d, dtype=torch.bfloat16, device=device)
    # the epilogue reads 128 table entries per head from head * table_hs: 64 more per row than LTX's
    # (tokens, heads * 64) tables hold, so the fold's table is padded by one half head
    fold_ld = spec.heads * half + half
    cos_f, sin_f = (torch.rand(m, fold_ld, device=device, generator=g) for _ in range(2))
    cos, sin = (t[:, : spec.heads * half].contiguous() for t in (cos_f, sin_f))
    q_out, k_out = torch.empty(m, d, dtype=torch.bfloat16, device=device), torch.empty(m, d, dtype=torch.bfloat16,
                                                                                       device=device)

    def timed(fn, iters=max(args.steps, 10)):
        for _ in range(max(args.warmup, 2)):
            fn()
        begin, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        begin.record()
        for _ in range(iters):
            fn()
        end.record()
        torch.cuda.synchronize()
        return begin.elapsed_time(end) / iters * 1e3

    plain = timed(lambda: mpp_linear.fused_linear(a, w, b, out=qkv))
    folded = timed(lambda: _lib.launch_gemm_qknorm_rope(
        a, w, qkv, bias=b, q_end=d, k_end=2 * d, norm_q=norm_w[:128], norm_k=norm_w[:128], eps=1e-6,
        weight_offset=0.0, cos=cos_f, sin=sin_f, table_ld=fold_ld, table_hs=half, table_rows=m, table_bs=0))

    def separate():
        if not _lib.launch_qk_rmsnorm_rope(qkv[:, :d], qkv[:, d:2 * d], q_out, k_out, norm_w, norm_w, 1e-6, cos=cos,
                                           sin=sin, table_ld=spec.heads * half, table_hs=half, tokens=m,
                                           table_batched=False):
            raise RuntimeError("kx_qk_rmsnorm_rope_bf16 refused the config-3 shape")

    pass_us = timed(separate)
    extra = folded - plain
    print(json.dumps({
        "compare": "LTX Q/K norm + RoPE: folded into the QKV GEMM epilogue vs the separate pass",
        "workload": f"config 3: {m} tokens, QKV {m}x{3 * d}x{d} bf16 + bias, {spec.heads} heads x {spec.head_dim}",
        "qkv_plain_us": round(plain, 1),
        "qkv_per_head_norm_rope_epilogue_us": round(folded, 1),
        "epilogue_extra_us": round(extra, 1),
        "separate_pass_us": round(pass_us, 1),
        "fold_saves_at_most_us": round(pass_us - extra, 1),
        "note": "a full-row (4096-wide) norm adds a cross-tile reduction to the per-head epilogue's cost",
    }))
    return 0


def denoise_main(args) -> int:
    """One LTX-2 video denoising step: ``denoise_step`` over ``X0Model(LTXAVModel)``."""
    import dataclasses

    import torch

    from kinomlx_amd import _lib, workloads
    from kinomlx_amd.ltx2.denoise import denoise_step
    from kinomlx_amd.ltx2.state import LatentState
    from kinomlx_amd.ltx2.wrappers import X0Model

    device = torch.device("cuda:0")
    spec = workloads.CONFIGS[args.config]
    if args.grid:
        spec = dataclasses.replace(spec, grid=tuple(int(v) for v in args.grid.split(",")))
    audio = workloads.LTXAudioSpec(tokens=args.audio_tokens, text_tokens=spec.text_tokens) if args.audio_tokens else None
    build0 = time.perf_counter()
    if audio is None:
        model = X0Model(workloads.random_ltx_model(spec, args.blocks, device))
    else:
        model = X0Model(workloads.random_ltx_av_model(spec, audio, args.blocks, device))
    torch.cuda.synchronize()
    build_s = time.perf_counter() - build0
    gen = torch.Generator(device=device).manual_seed(1)
    latent = torch.randn((1, spec.tokens, 128), generator=gen, device=device).to(torch.bfloat16)
    context = torch.randn((1, spec.text_tokens, spec.dim), generator=gen, device=device).to(torch.bfloat16)
    positions = workloads.ltx_positions(spec.grid).to(device)
    state = LatentState(latent=latent, denoise_mask=torch.ones((1, spec.tokens, 1), device=device),
                        positions=positions, clean_latent=latent)
    audio_state = audio_context = None
    if audio is not None:
        a_latent = torch.randn((1, audio.tokens, 128), generator=gen, device=device).to(torch.bfloat16)
        audio_context = torch.randn((1, audio.text_tokens, audio.dim), generator=gen, device=device).to(torch.bfloat16)
        start = torch.arange(audio.tokens, dtype=torch.float32, device=device)
        audio_state = LatentState(latent=a_latent, denoise_mask=torch.ones((1, audio.tokens, 1), device=device),
                                  positions=torch.stack([start, start + 1.0], dim=-1)[None, None],
                                  clean_latent=a_latent)
    sigmas = (0.909375, 0.725, 0.421875)

    def step(s):
        return denoise_step(s, audio_state, sigma=sigmas[0], sigma_next=sigmas[1], transformer=model,
                            video_context=context, audio_context=audio_context)[0]

    for _ in range(args.warmup):
        step(state)
    # headline: the steps alone, no per-launch events
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    for _ in range(args.steps):
        out = step(state)
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    ms_per_step = wall * 1e3 / args.steps
    # breakdown: the same steps again with HIP events around every launch (on its stream)
    timer = _lib.LaunchTimer()
    _lib.set_timer(timer)
    wall1 = time.perf_counter()
    for _ in range(args.steps):
        out = step(state)
    torch.cuda.synchronize()
    instrumented_ms = (time.perf_counter() - wall1) * 1e3 / args.steps
    _lib.set_timer(None)

    per_kernel: dict[str, list[float]] = defaultdict(list)
    name_of: dict[str, str] = {}
    for name, cargs, ms in timer.durations_ms():
        label = _kernel_label(name, cargs)
        per_kernel[label].append(ms)
        name_of[label] = name
    kernel_ms = {k: sum(v) / args.steps for k, v in per_kernel.items()}
    block_flops = workloads.flop_count(spec)["total"] * args.blocks
    attn_ms = sum(v for k, v in kernel_ms.items() if name_of[k] == "kx_attention_fwd_bf16")
    gemm_ms = sum(v for k, v in kernel_ms.items() if name_of[k].startswith(("kx_gemm", "kx_qgemm")))
    outside = ("kx_timestep_embedding", "kx_ltx_rope_tables", "kx_to_denoised", "kx_euler_step", "kx_all_finite",
               "kx_mask_composite", "kx_silu_bf16")
    if args.breakdown:
        for label, ms in sorted(kernel_ms.items(), key=lambda kv: -kv[1]):
            print(f"{ms:9.3f} ms/step  x{len(per_kernel[label]) // args.steps}  {label}", file=sys.stderr)
    same_work = (spec.tokens == 5376 and audio is not None and args.blocks == 48 and not spec.bits)
    result = {
        "metric": "LTX-2 video denoising step ms (X0 transformer + Euler update + finite check)",
        "value": round(ms_per_step, 2),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 2),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": round(ms_per_step / 18000.0, 5) if same_work else None,
        "dtype": "bf16",
        "data": "synthetic (N(0,0.02) weights drawn on the device, N(0,1) latent and context; no checkpoint)",
        "config": {
            "workload": (f"LTX2-like {'joint audio/video' if audio else 'video'} transformer, {args.blocks} blocks, "
                         f"BASELINE config {args.config} block shape"),
            "audio_tokens": audio.tokens if audio else 0,
            "video_tokens": spec.tokens,
            "latent_grid_thw": list(spec.grid),
            "text_tokens": spec.text_tokens,
            "dim": spec.dim,
            "latent_channels": 128,
            "weights": f"int{spec.bits} affine g{spec.group_size}" if spec.bits else "bf16",
            "batch": 1,
        },
        "block_tflops": round(block_flops / (ms_per_step * 1e-3) / 1e12, 1),
        "published_reference": {"s_per_step": 18.0, "workload": "stage-2 768x448x121: 5376 video tokens, 48 joint "
                                "A/V blocks, FP16, Apple silicon", "source": "docs/ltx2/performance.md:17-28"},
        "attention_ms": round(attn_ms, 2),
        "gemm_ms": round(gemm_ms, 2),
        "outside_block_kernels_ms": round(sum(v for k, v in kernel_ms.items() if name_of[k] in outside), 3),
        "kernel_sum_ms": round(sum(kernel_ms.values()), 2),
        "instrumented_ms_per_step": round(instrumented_ms, 2),
        "build_s": round(build_s, 1),
        "finite": bool(torch.isfinite(out.latent.float()).all()),
    }
    print(json.dumps(result))
    return 0


if __name__ == "__main__":
    sys.exit(main())

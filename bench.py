#!/usr/bin/env python3
"""MoE block forward throughput on one MI355X.

Workload (the headline): N = 16384 tokens (B=64,
T=256), C = 1024, E = 16 experts, top-k = 2, SwiGLU hidden H = 2816, bf16
activations and weights with fp32 accumulation, router bias ~ N(0,1)
(skewed expert load).  A step is one MoELayer forward over the N tokens,
inputs already resident in HBM.  Synthetic seeded data (mgpt_amd.workload).

Prints one JSON line: tokens/s (value), ms/step, the roofline of the
dominant kernel (the gate/up grouped GEMM, MFMA-bound) measured with HIP
events inside the timed region, and the reference CPU path timed on a
bounded sample of the same workload on this host.

--pass train measures a training step instead, in the reference Trainer's
per-step order (pipeline/Trainer.cpp:303-305, then forward and backward):
zero_grad, the training forward (which also keeps the backward's caches),
then the backward with dy ~ N(0,1).  It reports tokens/s of the step, the
forward and backward stage times, the roofline of the backward's dominant
GEMM, and the reference's CPU zero_grad + forward + backward on a sample.

--pass block measures the fused MoE half of a transformer block,
out = x + MoE(RMSNorm(x) * gamma) (mgpt_moe_forward_block), beside the same
computation unfused (torch RMSNorm, the layer forward, torch add) on the
same inputs, and the reference's CPU RMSNormLayer + MoELayer + add.

--pass decode (default config cfg5) measures the layer inside the engine's
sampling loop (pipeline/Generator.cpp:13-36: B = 1, no KV cache, the whole
context re-run every step, cropped to max_seq_len S = cfg.N): the growing
phase N = 1 .. S enqueued without any host synchronisation, then
steady-state steps at N = S, eager and replayed from one captured HIP
graph.  value = steady-state steps/s of the faster of the two (named in
steady_mode; both are reported).  The driver's headline line is the
default forward.
"""
from __future__ import annotations

import argparse
import json
import os
import re
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_F32_TFLOPS = 157.3      # MI355X dense fp32 matrix
PEAK_BF16_TFLOPS = 2500.0     # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0         # MI355X HBM3E
METRIC = "MoE layer tokens/s + expert-GEMM % MFMA peak (N=16384,C=1024,E=16,k=2)"
METRIC_TRAIN = ("MoE layer training tokens/s, zero_grad + forward + backward "
                "(N=16384,C=1024,E=16,k=2)")
METRIC_DECODE = ("MoE decode steps/s in the sampling loop (Generator B=1, no KV cache, "
                 "context S=64, C=2048, E=64, k=8, H=1408, fp8 weights)")
METRIC_BLOCK = ("MoE block tokens/s, out = x + MoE(RMSNorm(x) * gamma) "
                "(N=16384,C=1024,E=16,k=2)")
METRIC_BLOCK_TRAIN = ("MoE block training tokens/s, zero_grad + forward + backward of "
                      "out = x + MoE(RMSNorm(x) * gamma) (N=16384,C=1024,E=16,k=2)")
CALIB_MIB = 512               # known-size elementwise copy for counter calibration
NUM_XCD = 8                   # MI355X: 8 XCDs; GRBM_GUI_ACTIVE is counted per XCD
SIMD_NUM = 256 * 4            # MI355X: 256 CUs x 4 SIMDs (rocprof's MfmaUtil denominator)
MFMA_COUNTERS = ("SQ_VALU_MFMA_BUSY_CYCLES", "GRBM_GUI_ACTIVE", "SQ_INSTS_VALU_MFMA_MOPS_BF16",
                 "SQ_BUSY_CU_CYCLES")


def stage_of(kernel_name: str):
    """Stage of a kernel in a rocprofv3 trace (None: not a forward or
    backward kernel).  The down GEMM kernel also runs the backward's dX
    product in a training pass; the per-stage HIP-event times separate them."""
    short = kernel_name.replace("(anonymous namespace)", "").split("(")[0]
    if "scatter_bwd_kernel" in short:
        return "scatter_bwd"
    if re.search(r"token_d[lx](?:_wide)?_kernel", short):
        return "token_bwd"
    if "router_wgrad" in short:
        return "router_wgrad"
    if "rmsnorm_bwd" in short or "rmsnorm_dgamma" in short:
        return "ln2_bwd"
    m = re.search(r"wgrad(?:_tr)?_kernel<(?:[^,>]*, )?(\d)>", short)
    if m:
        return ("wgrad_down", "wgrad_gateup")[int(m.group(1))]
    if re.search(r"router_(?:topk|logits|softmax|decode)", short):
        return "router_topk"
    if "permute_kernel" in short:
        return "permute"
    if re.search(r"combine\d?_kernel", short):
        return "combine"
    m = re.search(r"gemm_(?:dma|ring5|decode|split_reduce)_kernel<(\d)[,>]", short)
    if m:
        return ("gemm_gateup", "gemm_down", "gemm_dact_swiglu_bwd")[int(m.group(1))]
    m = re.search(r"grouped_gemm_kernel<([^>]*)>", short)
    if m:
        epi = int(m.group(1).split(",")[6])
        return ("gemm_gateup", "gemm_down", "gemm_dact_swiglu_bwd")[epi]
    if "MulFunctor" in kernel_name:
        return "calib_copy"
    return None


def _counter_means(d: str, counter: str):
    """Counter value per forward, by stage, from a rocprofv3 --pmc csv: the
    mean per dispatch of each kernel, summed over the kernels of a stage (the
    down GEMM stage, for one, is the GEMM plus its split-K reduction)."""
    import csv
    vals = {}
    with open(os.path.join(d, "run_counter_collection.csv")) as f:
        for r in csv.DictReader(f):
            if r["Counter_Name"] != counter:
                continue
            st = stage_of(r["Kernel_Name"])
            if st:
                vals.setdefault(st, {}).setdefault(r["Kernel_Name"], []).append(
                    float(r["Counter_Value"]))
    out = {}
    for st, kerns in vals.items():
        if st == "calib_copy":    # the 512 MiB copies only, not torch's small multiplies
            allv = [v for vs in kerns.values() for v in vs]
            big = max(allv)
            allv = [v for v in allv if v > 0.5 * big]
            out[st] = sum(allv) / len(allv)
        else:
            out[st] = sum(sum(vs) / len(vs) for vs in kerns.values())
    return out


def summarize_traffic(fetch_dir: str, write_dir: str, workload: str, commands) -> dict:
    """HBM bytes per launch of each forward kernel from two rocprofv3 --pmc
    runs (FETCH_SIZE, WRITE_SIZE; KiB per dispatch), each scaled by the factor
    that makes the same counter read exactly the known size of the
    calibration copy (CALIB_MIB read and CALIB_MIB written)."""
    fetch = _counter_means(fetch_dir, "FETCH_SIZE")
    write = _counter_means(write_dir, "WRITE_SIZE")
    known = CALIB_MIB * 1024.0
    ff = known / fetch["calib_copy"]
    fw = known / write["calib_copy"]
    kern = {st: {"fetch_bytes": round(fetch[st] * 1024 * ff), "write_bytes": round(write[st] * 1024 * fw)}
            for st in fetch if st != "calib_copy" and st in write}
    for v in kern.values():
        v["hbm_bytes"] = v["fetch_bytes"] + v["write_bytes"]
    return {"workload": workload, "calib_copy_mib": CALIB_MIB,
            "calib_fetch_kib_read": round(fetch["calib_copy"], 1),
            "calib_write_kib_read": round(write["calib_copy"], 1),
            "fetch_factor": round(ff, 4), "write_factor": round(fw, 4),
            "kernels": kern, "commands": commands}


def summarize_mfma(pmc_dir: str, cfg, command: str) -> dict:
    """MFMA utilisation of the expert GEMMs from one rocprofv3 --pmc run with
    MFMA_COUNTERS.  Per dispatch: rocprof's MfmaUtil,
    sum(SQ_VALU_MFMA_BUSY_CYCLES) / (GRBM_GUI_ACTIVE per XCD x SIMD_NUM) (the
    csv sums GRBM_GUI_ACTIVE over the XCDs); the shader clock during the
    kernel, GRBM_GUI_ACTIVE per XCD / duration; the MFMA flops the hardware
    counted (SQ_INSTS_VALU_MFMA_MOPS_BF16 x 512, padding rows included)
    against the algorithmic 4ACH (gate/up) and 2ACH (down).  Means over the
    dispatches of each stage."""
    import csv
    per = {}
    with open(os.path.join(pmc_dir, "run_counter_collection.csv")) as f:
        for r in csv.DictReader(f):
            st = stage_of(r["Kernel_Name"])
            if st not in ("gemm_gateup", "gemm_down") or "split_reduce" in r["Kernel_Name"]:
                continue
            d = per.setdefault(st, {}).setdefault(r["Dispatch_Id"], {})
            d[r["Counter_Name"]] = float(r["Counter_Value"])
            d["dur_ns"] = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
    A = cfg.N * cfg.k
    alg = {"gemm_gateup": 4.0 * A * cfg.C * cfg.H, "gemm_down": 2.0 * A * cfg.H * cfg.C}
    out = {"workload": workload_name(cfg), "command": command, "simd_num": SIMD_NUM,
           "xcds": NUM_XCD, "kernels": {}}
    for st, ds in per.items():
        ds = [d for d in ds.values() if all(c in d for c in MFMA_COUNTERS)]
        if not ds:
            continue
        mean = lambda f: sum(f(d) for d in ds) / len(ds)   # noqa: E731
        grbm = mean(lambda d: d["GRBM_GUI_ACTIVE"] / NUM_XCD)
        busy = mean(lambda d: d["SQ_VALU_MFMA_BUSY_CYCLES"])
        dur = mean(lambda d: d["dur_ns"])
        mops = mean(lambda d: d["SQ_INSTS_VALU_MFMA_MOPS_BF16"] * 512)
        out["kernels"][st] = {
            "dispatches": len(ds),
            "mean_duration_us": round(dur / 1e3, 2),
            "mfma_busy_cycles": round(busy),
            "grbm_gui_active_per_xcd": round(grbm),
            "mfma_util": round(busy / (grbm * SIMD_NUM), 4),
            "shader_clock_ghz": round(grbm / dur, 3),
            "counted_mfma_flops": round(mops),
            "algorithmic_flops": alg[st],
            "algorithmic_tflops": round(alg[st] / dur / 1e3, 2),
            "frac_of_peak_at_measured_clock": round(
                alg[st] / dur / 1e3 / (PEAK_BF16_TFLOPS * (grbm / dur) / 2.4), 4),
        }
    return out


def cpu_sample_tokens(cfg) -> int:
    """A CPU-baseline sample of about the work of 4096 cfg3 tokens (the
    reference runs one core at roughly 1000 cfg3 tokens/s): 4096 tokens
    scaled by cfg3's per-token flops over this config's, in multiples of 64."""
    per_token = 6.0 * cfg.k * cfg.C * cfg.H + 2.0 * cfg.C * cfg.E
    cfg3_per_token = 6.0 * 2 * 1024 * 2816 + 2.0 * 1024 * 16
    n = int(4096 * cfg3_per_token / per_token) // 64 * 64
    return max(64, min(n, cfg.N))


def cpu_baseline(cfg, sample_tokens: int, reps: int, mode: str = "forward"):
    """The reference's own CPU MoE forward (train: zero_grad + forward +
    backward; block: ln2 RMSNormLayer + forward + residual add; block_train:
    zero_grad, the block forward and its backward)
    (oracle/_ref/ref_driver, built from the unmodified reference sources),
    single-threaded as the reference is, on `sample_tokens` tokens of the
    workload's shape."""
    drv = os.path.join(ROOT, "oracle", "_ref", "ref_driver")
    if not os.path.exists(drv):
        return None
    # the x86-64-v4 (AVX-512) build where this host has every v4 feature
    build = "x86-64-v3 (AVX2) build"
    try:
        flags = set()
        for l in open("/proc/cpuinfo"):
            if l.startswith("flags"):
                flags = set(l.split(":", 1)[1].split())
                break
        v4 = os.path.join(ROOT, "oracle", "_ref", "ref_driver_v4")
        if {"avx512f", "avx512bw", "avx512cd", "avx512dq", "avx512vl"} <= flags and os.path.exists(v4):
            drv, build = v4, "x86-64-v4 (AVX-512) build"
    except OSError:
        pass
    sub = {"forward": "bench", "train": "bench_train", "block": "bench_block",
           "block_train": "bench_block_train"}[mode]
    what = {"forward": "MoELayer::forward_into",
            "train": "Tensor::zero_grad + MoELayer::forward_into + backward_into",
            "block": "RMSNormLayer::forward_into + MoELayer::forward_into + Tensor::add_into",
            "block_train": "Tensor::zero_grad, then RMSNormLayer + MoELayer forward_into and "
                           "Tensor::add_into, then MoELayer + RMSNormLayer backward_into and "
                           "Tensor::add_into"}[mode]
    cmd = [drv, sub, str(sample_tokens), str(cfg.C), str(cfg.H),
           str(cfg.E), str(cfg.k), str(reps)]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    if r.returncode != 0:
        return {"error": r.stderr[-500:]}
    res = json.loads(r.stdout.strip().splitlines()[-1])
    try:
        model = [l.split(":", 1)[1].strip() for l in open("/proc/cpuinfo")
                 if l.startswith("model name")][0]
    except Exception:
        model = "unknown"
    return {
        "value": round(res["tokens_per_s"], 3), "unit": "tokens/s", "cores": 1,
        "kind": "reference",
        "sample": (f"{sample_tokens} of {cfg.N} tokens at the workload's shape "
                   f"(C={cfg.C}, E={cfg.E}, k={cfg.k}, H={cfg.H}), fp32 reference CPU path "
                   f"({what}), {build}, "
                   f"1 warmup + median of {reps}; "
                   f"1 thread of {os.cpu_count()} visible cores, {model}"),
        "median_s": res["median_s"],
    }


def summarize_stats(stats_csv: str, bench_json: str, config: str) -> str:
    """Markdown table of a rocprofv3 kernel-statistics csv next to the HIP-event
    stage means that bench.py measured in the same run."""
    import csv
    with open(bench_json) as f:
        b = json.loads(f.read().strip().splitlines()[-1])
    rows = list(csv.DictReader(open(stats_csv)))
    mode = str(b.get("pass", "forward")).split(" ")[0]
    train = mode in ("train", "block_train")
    extra = "" if mode == "forward" else f" --pass {mode}"
    cfg_arg = "" if mode == "decode" else f"--config {config} "
    cmd = (f"rocprofv3 --kernel-trace --stats --output-format csv -d <dir> -o run -- python bench.py "
           f"{cfg_arg}{extra.strip()} --steps {b['steps']} --warmup {b['warmup']} "
           "--no-cpu-baseline").replace("  ", " ")
    what = {"train": "training step (zero_grad + forward + backward)",
            "block_train": "fused block training step (zero_grad + RMSNorm + MoE + residual, "
                           "forward and backward)",
            "block": "fused block (RMSNorm + MoE + residual)",
            "decode": "decode steps in the sampling loop"}.get(mode, "forward")
    w, k = b["warmup"], b["steps"]
    runs = {"train": f"{w + 2 * k} training steps ({w} warmup, {k} timed, {k} profiled); "
                     "outside the profiled steps the d(act) product (on 5/8 of the CUs) and the "
                     "down weight gradient run concurrently on two streams, so their averages "
                     "mix those launches with the serial ones of the profiled steps",
            "block": f"{w + 2 * k} fused block forwards ({w} warmup, {k} timed, {k} profiled) "
                     f"and {w + k} unfused ({w} warmup, {k} timed)",
            "block_train": f"{w + 2 * k} fused block training steps ({w} warmup, {k} timed, "
                           f"{k} profiled); outside the profiled steps the backward's weight "
                           "gradients run on a second stream beside its d(act) and dX products",
            "decode": f"{w + 1} growing loops of {b.get('growing_phase_steps')} steps "
                      f"(N = 1 .. {b['config']['N']}), then {k} eager, {k} "
                      f"profiled, 1 + {max(w, 30) + k} graph-replayed steady-state "
                      "steps (kernel averages mix every N)"}.get(
        mode, f"{w + 2 * k} forwards ({w} warmup, {k} timed, {k} profiled)")
    out = [f"# {b['config']['workload'].split(':')[0]} MoE {what}: rocprofv3 kernel statistics "
           "(MI355X)", "",
           "Command (repository root, on the GPU box), then "
           "`python bench.py --summarize-stats <dir>/run_kernel_stats.csv <json line>`:", "",
           "```", cmd, "```", "",
           f"Workload: {b['config']['workload']}.  {runs}; pack/pad/quantise/copy/transpose "
           "kernels are the one-time parameter load and backward weight layouts.", "",
           "| Kernel | Stage | Calls | Average (us) | Share of GPU time |", "|---|---|---|---|---|"]
    for r in rows:
        name = r["Name"].replace("unsigned short", "bf16").replace("mgpt::(anonymous namespace)::", "")
        if len(name) > 110:
            name = name[:107] + "..."
        st = stage_of(r["Name"]) or "-"
        if mode == "block" and r["Name"].startswith(("void at::native", "at::native")):
            st = "unfused (torch)"   # the unfused comparison's torch kernels
        out.append(f"| `{name}` | {st} | {r['Calls']} | "
                   f"{float(r['AverageNs']) / 1e3:.1f} | {float(r['Percentage']):.2f}% |")
    out += ["", "HIP-event stage means measured by bench.py in the same run (ms):", "",
            "| Stage | ms |", "|---|---|"]
    out += [f"| {k} | {v} |" for k, v in b["stage_ms"].items()]
    rf = b["roofline"]
    if train:
        out += [f"| {k} (backward) | {v} |" for k, v in b["backward_stage_ms"].items()]
        out += ["", f"bench.py: {b['value']:.0f} training tokens/s, {b['ms_per_step']} ms/step "
                f"(backward {b['backward_ms']} ms); backward products (TFLOP/s): "
                + ", ".join(f"{k} {v}" for k, v in b["backward_gemm_tflops"].items())
                + f"; dominant: {rf['kernel']} = {100 * rf['frac']:.1f}% of {rf['peak']} TFLOP/s."]
    elif mode == "decode":
        out += ["", f"bench.py: {b['value']:.0f} steady-state steps/s ({b['ms_per_step']} ms/step, "
                f"{b['steady_graph_ms_per_step']} ms replayed from a HIP graph, "
                f"{b['steady_eager_ms_per_step']} ms eager); growing "
                f"loop of {b['growing_phase_steps']} steps {b['growing_phase_ms']} ms on the "
                f"device, enqueued by the host in {b['growing_phase_host_enqueue_ms']} ms; "
                f"{rf['kernel']}: {rf['achieved']} GB/s = {100 * rf['frac']:.1f}% of "
                f"{rf['peak']} GB/s."]
    elif rf["unit"] == "GB/s":
        # weight-streaming decode shapes: an HBM roofline
        out += ["", f"bench.py: {b['value']:.0f} tokens/s, {b['ms_per_step']} ms/step; "
                f"{rf['kernel']}: {rf['achieved']} GB/s of weights = {100 * rf['frac']:.1f}% of "
                f"{rf['peak']} GB/s HBM; both expert GEMMs {b['expert_gemm_tflops']} TFLOP/s."]
    else:
        out += ["", f"bench.py: {b['value']:.0f} tokens/s, {b['ms_per_step']} ms/step; gate/up GEMM "
                f"{rf['achieved']} TFLOP/s = {100 * rf['frac']:.1f}% of {rf['peak']} TFLOP/s dense "
                f"{'fp32' if rf['peak'] == PEAK_F32_TFLOPS else 'bf16'}; both expert GEMMs "
                f"{b['expert_gemm_tflops']} TFLOP/s."]
        if mode == "block":
            out += [f"Unfused (torch RMSNorm, the layer forward, torch add) on the same inputs: "
                    f"{b['unfused_ms_per_step']} ms/step."]
    return "\n".join(out)


def workload_name(cfg) -> str:
    return (f"{cfg.name}: MoE block forward N={cfg.N} (B={cfg.B},T={cfg.T}) C={cfg.C} E={cfg.E} "
            f"k={cfg.k} H={cfg.H} act={cfg.act} weights={cfg.weights} "
            f"router_bias={cfg.router_bias}")


def traffic_path(cfg) -> str:
    return os.path.join(ROOT, "profiles", f"{cfg.name}_hbm_traffic.json")


def load_traffic(cfg):
    """Committed per-kernel HBM traffic of this workload (summarize_traffic's
    output), if it was measured for exactly this workload."""
    try:
        with open(traffic_path(cfg)) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None
    return t if t.get("workload") == workload_name(cfg) else None


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="cfg3")
    ap.add_argument("--cpu-tokens", type=int, default=None,
                    help="tokens of the CPU baseline's sample (default: about 10 s of the "
                         "reference's work per run, 4096 tokens at cfg3's per-token cost)")
    ap.add_argument("--cpu-reps", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--pass", dest="mode",
                    choices=["forward", "train", "block", "block_train", "decode"],
                    default="forward",
                    help="forward (default, the headline), train (zero_grad + forward + backward), "
                         "block (RMSNorm + MoE + residual, fused), block_train (zero_grad + the "
                         "fused block's forward and backward) or decode (the sampling loop at "
                         "cfg5's shape)")
    ap.add_argument("--calib-copy", action="store_true",
                    help=f"after the timed run, copy {CALIB_MIB} MiB with an elementwise kernel 3 "
                         "times (known-size traffic for calibrating FETCH_SIZE/WRITE_SIZE)")
    ap.add_argument("--summarize-traffic", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="no GPU run: turn two rocprofv3 --pmc outputs (FETCH_SIZE, WRITE_SIZE) "
                         "of 'bench.py --calib-copy' into the per-kernel HBM traffic JSON")
    ap.add_argument("--summarize-stats", nargs=2, metavar=("STATS_CSV", "BENCH_JSON"),
                    help="no GPU run: markdown summary of a rocprofv3 --kernel-trace --stats run "
                         "of this script and of the JSON line that run printed")
    ap.add_argument("--summarize-mfma", metavar="PMC_DIR",
                    help="no GPU run: MFMA utilisation of the expert GEMMs from a rocprofv3 "
                         "--pmc " + " ".join(MFMA_COUNTERS) + " run of this script")
    args = ap.parse_args()
    if args.summarize_mfma:
        from mgpt_amd import workload as wl
        cfg = wl.CONFIGS[args.config]
        cmd = ("rocprofv3 --pmc " + " ".join(MFMA_COUNTERS) + " --output-format csv -d <dir> "
               f"-o run -- python bench.py --config {args.config} --steps 3 --warmup 1 "
               "--no-cpu-baseline")
        print(json.dumps(summarize_mfma(args.summarize_mfma, cfg, cmd), indent=1))
        return 0
    if args.summarize_stats:
        print(summarize_stats(*args.summarize_stats, args.config))
        return 0
    if args.summarize_traffic:
        from mgpt_amd import workload as wl
        cfg = wl.CONFIGS[args.config]
        cmd = ("rocprofv3 --pmc {c} --output-format csv -d {d} -o run -- python bench.py "
               f"--config {args.config} --steps 3 --warmup 1 --no-cpu-baseline --calib-copy")
        out = summarize_traffic(*args.summarize_traffic, workload_name(cfg),
                                [cmd.format(c="FETCH_SIZE", d=args.summarize_traffic[0]),
                                 cmd.format(c="WRITE_SIZE", d=args.summarize_traffic[1])])
        print(json.dumps(out, indent=1))
        return 0
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); the "
              "expert-parallel multi-GPU path is a design note, not implemented", file=sys.stderr)
        return 2

    import numpy as np
    import torch

    from mgpt_amd import workload as wl
    from mgpt_amd.moe import MoELayer

    if args.mode == "decode":
        return decode_main(args)
    cfg = wl.CONFIGS[args.config]
    dev = torch.device("cuda", 0)
    t0 = time.time()
    inp = wl.make_inputs(cfg, seed=20261201)
    layer = MoELayer(cfg.C, cfg.H, cfg.E, cfg.k, act=cfg.act, weights=cfg.weights)
    layer.load_parameters(inp.params(raw=True))
    dt = torch.float32 if cfg.act == "f32" else torch.bfloat16
    x = torch.from_numpy(inp.x).to(dev).to(dt)
    y = torch.empty_like(x)
    del inp
    block_train = args.mode == "block_train"
    train = args.mode in ("train", "block_train")
    block = args.mode in ("block", "block_train")
    if train:
        g = torch.Generator(device="cpu").manual_seed(7)
        dy = torch.randn(x.shape, generator=g).to(dev).to(dt)
        dx = torch.empty_like(x)
    if block:
        # x1: the workload's rows scaled per token by 0.25 .. 4; gamma ~ 1 + 0.2 N(0,1)
        g = torch.Generator(device="cpu").manual_seed(13)
        scale = torch.exp2(torch.randint(-2, 3, (x.shape[0], 1), generator=g).float())
        x = (x.float() * scale.to(dev)).to(dt)
        gamma = (1.0 + 0.2 * torch.randn(cfg.C, generator=g)).to(dev)
        eps = 1e-5
        dgamma = torch.zeros(cfg.C, dtype=torch.float32, device=dev)
    print(f"setup {time.time() - t0:.1f}s", file=sys.stderr, flush=True)

    def step():
        if block_train:
            layer.zero_grad()
            dgamma.zero_()
            layer.forward_block_into(x, gamma, eps, y, train=True)
            layer.backward_block_into(dy, dx, dgamma)
            return
        if block:
            layer.forward_block_into(x, gamma, eps, y)
            return
        if train:
            layer.zero_grad()
        layer.forward_into(x, y, train)
        if train:
            layer.backward_into(dy, dx)

    def unfused_step():
        # the same block unfused: torch RMSNorm in fp32, the layer, torch add
        xf = x.float()
        xn = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps) * gamma).to(dt)
        layer.forward_into(xn, y)
        y.add_(x)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    counts = layer.get_expert_counts()

    # The timed steps record HIP events on the launch stream around the
    # gate/up GEMM only: an event at every stage boundary adds a gap of a few
    # microseconds between launches (about 2.5% of the cfg3 forward, 3.5% of
    # its training step).  The other stage times, the backward's included,
    # come from a separate, fully profiled pass of as many steps.
    layer.set_profiling(True, gemm_only=True)
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    w0 = time.perf_counter()
    start.record()
    for _ in range(args.steps):
        step()
    stop.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - w0
    ms_per_step = start.elapsed_time(stop) / args.steps
    stages = layer.stage_times()
    n_prof = stages.pop("forwards")
    gemm_gateup_timed = stages["gemm_gateup"]
    layer.set_profiling(True)
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    stages = layer.stage_times()
    stages.pop("forwards")
    stages["gemm_gateup"] = gemm_gateup_timed
    bstages = layer.backward_stage_times() if train else None
    if bstages:
        bstages.pop("backwards")
    layer.set_profiling(False)

    N, C, H, E, k = cfg.N, cfg.C, cfg.H, cfg.E, cfg.k
    A = N * k
    a = 2 if cfg.act == "bf16" else 4
    w = {"bf16": 2, "fp8": 1, "f32": 4}[cfg.weights]
    gateup_flops = 4.0 * A * C * H
    down_flops = 2.0 * A * H * C
    t_gu = stages["gemm_gateup"] * 1e-3
    t_dn = stages["gemm_down"] * 1e-3
    gu_tflops = gateup_flops / t_gu / 1e12
    gemm_tflops = (gateup_flops + down_flops) / (t_gu + t_dn) / 1e12
    # the hot path's algorithmic byte counts per launch; the permute's counts x
    # once per assignment (the kernel reads each row once: see the counter bytes)
    permute_bytes = 2.0 * A * C * a + 8 * A
    combine_bytes = A * C * a + N * C * a + 8 * A
    router_bytes = N * C * a + C * E * 4 + 8 * A
    hbm = {
        "router_topk_GBs": router_bytes / (stages["router_topk"] * 1e-3) / 1e9,
        "permute_GBs": permute_bytes / (stages["permute"] * 1e-3) / 1e9,
        "combine_GBs": combine_bytes / (stages["combine"] * 1e-3) / 1e9,
    }
    # the bytes each kernel must move: the permute reads each row once and
    # writes it k times (plus perm and slot_of)
    moved = {"router_topk": router_bytes, "permute": N * C * a + A * C * a + 8.0 * A,
             "combine": combine_bytes}
    total_flops = 2.0 * N * C * E + 6.0 * A * C * H
    # fp32 runs on the fp32 matrix cores (v_mfma_f32_32x32x2f32), whose peak differs
    peak_mm = PEAK_F32_TFLOPS if cfg.weights == "f32" else PEAK_BF16_TFLOPS
    used = sum(1 for c_ in counts if c_ > 0)
    # decode shape with fp8 weights: the gate/up launch streams 2*H*C weight
    # bytes (plus fp32 scales) for every expert that received a token
    weight_stream = cfg.weights == "fp8" and A < 64 * E
    gu_weight_bytes = used * (2.0 * H * C * w + 2 * H * 4)
    result = {
        "metric": METRIC,
        "value": round(N / (ms_per_step * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if cfg.act == "bf16" else "f32",
        "data": "synthetic (seeded; mgpt_amd.workload)",
        "config": {"workload": workload_name(cfg),
                   "N": N, "C": C, "E": E, "k": k, "H": H, "global_batch": cfg.B,
                   "seq_len": cfg.T, "parallelism": "single GPU"},
        "layer_tflops": round(total_flops / (ms_per_step * 1e-3) / 1e12, 2),
        "expert_gemm_tflops": round(gemm_tflops, 2),
        "expert_gemm_mfma_frac": round(gemm_tflops / peak_mm, 4),
        "stage_ms": {kk: round(v, 4) for kk, v in stages.items()},
        "stage_ms_forwards_averaged": n_prof,
        # achieved HBM bandwidth over peak, by the bytes each kernel must move
        "hbm_frac": {kk: round(v / (stages[kk] * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)
                     for kk, v in moved.items()},
        # the per-unit byte formulas of the scope table (router N*C*a + C*E*4 + 8A,
        # permute 2*A*C*a + 8A, combine A*C*a + N*C*a + 8A) over the stage time and
        # HBM peak: the permute's formula counts k reads of each row, which the
        # kernel does not make, so this is a ratio, not a bandwidth
        "formula_bytes_ratio": {kk.replace("_GBs", ""): round(v / PEAK_HBM_GBS, 4)
                                for kk, v in hbm.items()},
        "expert_counts_max_over_mean": round(max(counts) / (sum(counts) / len(counts)), 3),
        "roofline": ({
            "kernel": "gate/up fp8 weight-streaming GEMM + SwiGLU epilogue",
            "bound": "hbm", "achieved": round(gu_weight_bytes / t_gu / 1e9, 1),
            "peak": PEAK_HBM_GBS, "unit": "GB/s",
            "frac": round(gu_weight_bytes / t_gu / 1e9 / PEAK_HBM_GBS, 4), "traffic": None,
        } if weight_stream else {
            "kernel": "grouped_gemm gate/up + SwiGLU epilogue",
            "bound": "mfma", "achieved": round(gu_tflops, 2), "peak": peak_mm,
            "unit": "TFLOP/s", "frac": round(gu_tflops / peak_mm, 4),
            "traffic": None,
        }),
        "wall_s_timed": round(wall, 3),
    }
    if train:
        # backward products: d(act) 2ACH, dX 4ACH, dW_down 2ACH, dW_gate/up 4ACH
        bw = {"gemm_dact_swiglu_bwd": 2.0 * A * C * H, "gemm_dx": 4.0 * A * C * H,
              "wgrad_down": 2.0 * A * C * H, "wgrad_gateup": 4.0 * A * C * H}
        rates = {kk: f / (bstages[kk] * 1e-3) / 1e12 for kk, f in bw.items()}
        dom = max(bw, key=lambda kk: bstages[kk])
        train_flops = total_flops + sum(bw.values()) + 4.0 * N * C * E
        bwd_ms = sum(bstages.values())
        result.update({
            "metric": METRIC_TRAIN,
            "pass": "train (zero_grad + forward_train + backward)",
            "layer_tflops": round(train_flops / (ms_per_step * 1e-3) / 1e12, 2),
            "backward_stage_ms": {kk: round(v, 4) for kk, v in bstages.items()},
            "backward_ms": round(bwd_ms, 4),
            "backward_gemm_tflops": {kk: round(v, 2) for kk, v in rates.items()},
            "roofline": {
                "kernel": f"backward {dom}", "bound": "mfma", "achieved": round(rates[dom], 2),
                "peak": peak_mm, "unit": "TFLOP/s", "frac": round(rates[dom] / peak_mm, 4),
                "traffic": None},
        })
    if block_train:
        result.update({
            "metric": METRIC_BLOCK_TRAIN,
            "pass": "block_train (zero_grad + mgpt_moe_forward_block_train + "
                    "mgpt_moe_backward_block: ln2 RMSNorm backward and residual in one kernel)",
        })
    if block and not block_train:
        for _ in range(args.warmup):
            unfused_step()
        torch.cuda.synchronize()
        start.record()
        for _ in range(args.steps):
            unfused_step()
        stop.record()
        torch.cuda.synchronize()
        ms_unfused = start.elapsed_time(stop) / args.steps
        result.update({
            "metric": METRIC_BLOCK,
            "pass": "block (mgpt_moe_forward_block: RMSNorm in the router, residual in combine)",
            "value": round(N / (ms_per_step * 1e-3), 1),
            "unfused_ms_per_step": round(ms_unfused, 4),
            "unfused": "torch fp32 RMSNorm -> bf16, mgpt_moe_forward, torch add (same inputs)",
        })
    traffic = None if (train or block) else load_traffic(cfg)
    if traffic:
        gu = traffic["kernels"].get("gemm_gateup")
        result["roofline"]["traffic"] = gu["hbm_bytes"] if gu else None
        result["roofline"]["traffic_source"] = (
            "rocprofv3 --pmc FETCH_SIZE + WRITE_SIZE bytes per launch, calibrated on a "
            f"{CALIB_MIB} MiB copy (factors {traffic['fetch_factor']}, {traffic['write_factor']}); "
            "profiles/" + os.path.basename(traffic_path(cfg)))
        result["hbm_bytes_per_launch"] = {st: v["hbm_bytes"] for st, v in traffic["kernels"].items()}
        # achieved bandwidth by the counters' bytes (what the kernel moved)
        result["hbm_frac_counters"] = {
            st: round(traffic["kernels"][st]["hbm_bytes"] / (stages[st] * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)
            for st in ("router_topk", "permute", "combine")
            if st in traffic["kernels"] and stages.get(st)}
    if args.calib_copy:
        n = CALIB_MIB * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):                  # an elementwise kernel, not a DMA-engine copy
            torch.mul(src, 1.0, out=dst)
        torch.cuda.synchronize()
        result["calib_copy_mib"] = CALIB_MIB
    if not args.no_cpu_baseline:
        print("cpu baseline ...", file=sys.stderr, flush=True)
        tokens = args.cpu_tokens or cpu_sample_tokens(cfg)
        tokens = min(tokens // 4 if train else tokens, N)
        result["cpu_baseline"] = cpu_baseline(cfg, tokens, args.cpu_reps, args.mode)
    print(json.dumps(result))
    return 0


def decode_main(args) -> int:
    """The sampling-loop measurement (--pass decode)."""
    import torch

    from mgpt_amd import workload as wl
    from mgpt_amd.moe import MoELayer

    cfg = wl.CONFIGS["cfg5" if args.config == "cfg3" else args.config]
    S, C, H, E, k = cfg.N, cfg.C, cfg.H, cfg.E, cfg.k
    dev = torch.device("cuda", 0)
    inp = wl.make_inputs(cfg, seed=20261201)
    layer = MoELayer(C, H, E, k, act=cfg.act, weights=cfg.weights)
    layer.load_parameters(inp.params(raw=True))
    dt = torch.float32 if cfg.act == "f32" else torch.bfloat16
    x = torch.from_numpy(inp.x).to(dev).to(dt)
    y = torch.empty_like(x)
    layer.reserve(S)
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def grow():
        for n in range(1, S + 1):
            layer.forward_into(x[:n], y[:n])

    for _ in range(max(1, args.warmup)):
        grow()
    torch.cuda.synchronize()
    # growing context: N = 1 .. S, the host never waits
    t0 = time.perf_counter()
    start.record()
    grow()
    stop.record()
    host_enqueue_s = time.perf_counter() - t0
    torch.cuda.synchronize()
    grow_ms = start.elapsed_time(stop)

    # steady state, eager (also the per-stage timing)
    K = args.steps
    start.record()
    for _ in range(K):
        layer.forward_into(x, y)
    stop.record()
    torch.cuda.synchronize()
    eager_ms = start.elapsed_time(stop) / K
    layer.set_profiling(True)
    for _ in range(K):
        layer.forward_into(x, y)
    torch.cuda.synchronize()
    stages = layer.stage_times()
    stages.pop("forwards")
    layer.set_profiling(False)
    counts = layer.get_expert_counts()

    # steady state, one captured HIP graph replayed
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        layer.forward_into(x, y)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        layer.forward_into(x, y)
    # the first replays of a new graph carry one-time costs (about 0.6 ms over
    # the first few dozen on MI355X), so the graph warms up longer
    for _ in range(max(args.warmup, 30)):
        g.replay()
    torch.cuda.synchronize()
    w0 = time.perf_counter()
    start.record()
    for _ in range(K):
        g.replay()
    stop.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - w0
    graph_ms = start.elapsed_time(stop) / K

    used = sum(1 for c_ in counts if c_ > 0)
    w = {"bf16": 2, "fp8": 1, "f32": 4}[cfg.weights]
    gu_bytes = used * (2.0 * H * C * w + 2 * H * 4)
    dn_bytes = used * (1.0 * H * C * w + C * 4)
    t_gu = stages["gemm_gateup"] * 1e-3
    best_ms = min(eager_ms, graph_ms)
    result = {
        "metric": METRIC_DECODE,
        "value": round(1e3 / best_ms, 1),
        "unit": "steps/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": round(best_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if cfg.act == "bf16" else "f32",
        "data": "synthetic (seeded; mgpt_amd.workload)",
        "pass": "decode (sampling loop: growing context, then steady state)",
        "config": {"workload": workload_name(cfg) + f"; sampling loop, max_seq_len S={S}, B=1",
                   "N": S, "C": C, "E": E, "k": k, "H": H, "parallelism": "single GPU"},
        "steady_mode": "graph" if graph_ms <= eager_ms else "eager",
        "steady_eager_ms_per_step": round(eager_ms, 4),
        "steady_graph_ms_per_step": round(graph_ms, 4),
        "growing_phase_ms": round(grow_ms, 4),
        "growing_phase_steps": S,
        "growing_phase_host_enqueue_ms": round(host_enqueue_s * 1e3, 3),
        "stage_ms": {kk: round(v, 4) for kk, v in stages.items()},
        "experts_used": used,
        "weight_bytes_per_step": gu_bytes + dn_bytes,
        "weight_stream_GBs": round((gu_bytes + dn_bytes) / (best_ms * 1e-3) / 1e9, 1),
        "roofline": {
            "kernel": "gate/up fp8 weight-streaming GEMM + SwiGLU epilogue (steady-state step)",
            "bound": "hbm", "achieved": round(gu_bytes / t_gu / 1e9, 1), "peak": PEAK_HBM_GBS,
            "unit": "GB/s", "frac": round(gu_bytes / t_gu / 1e9 / PEAK_HBM_GBS, 4),
            "traffic": None},
        "wall_s_timed": round(wall, 3),
    }
    if not args.no_cpu_baseline:
        print("cpu baseline ...", file=sys.stderr, flush=True)
        cb = cpu_baseline(cfg, S, args.cpu_reps, "forward")
        if cb and "value" in cb:
            cb = dict(cb, value=round(cb["value"] / S, 4), unit="steps/s",
                      sample=cb["sample"] + f"; one steady-state step = {S} tokens")
        result["cpu_baseline"] = cb
    print(json.dumps(result))
    return 0


if __name__ == "__main__":
    sys.exit(main())

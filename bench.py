#!/usr/bin/env python
"""Benchmark of the pair-representation hot path on one MI355X.

Workload (one "step"): B=1, N=512, c_z=128, bf16, synthetic seeded inputs
(z ~ N(0,1), mask all ones) and random weights (W ~ N(0, 1/fan_in), tri-mul
gate biases 1.0, other biases 0; tri-attn H=4, d=32, c_h=128):
    triangle multiplication outgoing + incoming, triangle attention starting
    + ending node, and LayerNorm over the pair tensor,
each through the genie_tk modules' HIP kernel path (forward).

Prints one JSON line.  value = algorithmic TFLOP/s of the step (dense
2*M*N*K of every projection and contraction; LayerNorm and softmax count 0),
with per-operator ms / TFLOP/s / fraction of the 2516.6 TFLOP/s bf16 MFMA
peak (each the mean over 5 back-to-back calls between two events; 10 warmup
calls, then the median of 50 repetitions), LayerNorm GB/s against 8 TB/s HBM, the roofline of the
dominant kernel (per-kernel durations from HIP events recorded on the launch
stream) and the CPU baseline (the modules' PyTorch path in fp32 on the host
cores).
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

# the kernels or an error, never the modules' PyTorch path
os.environ["GENIE_TK_STRICT"] = "1"

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "genie-tk_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

PEAK_BF16_FLOPS = 2516.6e12
PEAK_HBM_BYTES = 8.0e12
METRIC = "fwd ms + % bf16 MFMA peak, tri-mul & tri-attn at N=512 c_z=128; LN GB/s"
C_Z, C_HID, HEADS, HEAD_DIM = 128, 128, 4, 32
# per-operator timings: calls back to back between two events (the step runs
# its operators the same way), OP_WARM untimed calls, the median of OP_REPS
OP_INNER = 5
OP_WARM = 10
OP_REPS = 50


def trimul_flops(N: int, B: int = 1) -> dict:
    return {
        "trimul_prologue": 2.0 * B * N * N * C_Z * 4 * C_HID,
        "trimul_contract": 2.0 * B * N ** 3 * C_HID,
        "trimul_epilogue": 2.0 * B * N * N * (C_Z * C_Z + C_HID * C_Z),
    }


def triattn_flops(N: int, B: int = 1, heads: int = HEADS, head_dim: int = HEAD_DIM) -> dict:
    ch = heads * head_dim
    core = 4.0 * B * heads * head_dim * N ** 3  # Q K^T and P V
    w_o = 2.0 * B * N * N * ch * C_Z           # output projection
    out = {"triattn_prologue": 2.0 * B * N * N * C_Z * (4 * ch + heads)}
    if -(-N // 128) * 128 <= 1024:
        # (row, head) flash kernel; the output projection runs in its own kernel
        out.update({"triattn_flash": core, "triattn_out": w_o})
    else:
        out["triattn_flash"] = core + w_o
    return out


def step_flops_of(fm: dict, fa: dict) -> float:
    """Tri-mul outgoing + incoming and tri-attn starting + ending."""
    return 2 * sum(fm.values()) + 2 * sum(fa.values())


def ln_bytes(N: int, B: int = 1, elem: int = 2) -> float:
    return 2.0 * B * N * N * C_Z * elem


def build_modules(torch, N: int, dev: str):
    import numpy as np

    from genie_tk import (TriangleAttentionEndingNode, TriangleAttentionStartingNode,
                          TriangleMultiplicationIncoming, TriangleMultiplicationOutgoing)

    def init_(mod, seed, gate_names=()):
        g = torch.Generator().manual_seed(seed)
        sd = {}
        for name, p in sorted(mod.state_dict().items()):
            if name.endswith("weight") and p.dim() == 2:
                v = torch.randn(p.shape, generator=g) / np.sqrt(p.shape[1])
            elif "layer_norm" in name:
                v = torch.ones(p.shape) if name.endswith("weight") else torch.zeros(p.shape)
            else:
                v = torch.full(p.shape, 1.0) if name.rsplit(".", 1)[0] in gate_names else torch.zeros(p.shape)
            sd[name] = v
        mod.load_state_dict(sd)
        return mod.to(dev, torch.bfloat16).eval()

    gates = ("linear_a_g", "linear_b_g", "linear_g")
    mods = {
        "tri_mul_out": init_(TriangleMultiplicationOutgoing(C_Z, C_HID), 1, gates),
        "tri_mul_in": init_(TriangleMultiplicationIncoming(C_Z, C_HID), 2, gates),
        "tri_att_start": init_(TriangleAttentionStartingNode(C_Z, HEADS * HEAD_DIM, HEADS), 3),
        "tri_att_end": init_(TriangleAttentionEndingNode(C_Z, HEADS * HEAD_DIM, HEADS), 4),
    }
    for m in mods.values():
        assert m.use_fused_kernel, "HIP kernel path not enabled"
    return mods


def build_pair_layer(torch, dev: str, c_att: int = HEADS * HEAD_DIM):
    """One PairTransformLayer (c_p = c = 128, attention c_hidden c_att over 4
    heads), random weights, eval mode."""
    import numpy as np

    from genie_tk import PairTransformLayer

    layer = PairTransformLayer(c_p=C_Z, c_hidden_mul=C_HID, c_hidden_tri_att=c_att,
                               n_head_tri=HEADS, tri_dropout=0.25)
    g = torch.Generator().manual_seed(7)
    sd = {}
    for name, p in sorted(layer.state_dict().items()):
        if name.endswith("weight") and p.dim() == 2:
            sd[name] = torch.randn(p.shape, generator=g) / np.sqrt(p.shape[1])
        elif "layer_norm" in name:
            sd[name] = torch.ones(p.shape) if name.endswith("weight") else torch.zeros(p.shape)
        else:
            sd[name] = torch.zeros(p.shape)
    layer.load_state_dict(sd)
    return layer.to(dev, torch.bfloat16).eval()


def transition_flops(N: int, B: int = 1) -> float:
    return 2.0 * 2 * B * N * N * C_Z * 4 * C_Z


def event_time_ms(torch, fn, reps: int, warm: int = OP_WARM, flush=None, inner: int = 1) -> list:
    """Per-call durations from events on the current stream: each repetition
    times `inner` back-to-back calls between two events (a pipeline of calls,
    as in the step; inner = 1 also counts the host's launch latency of the
    call) and reports their mean."""
    for _ in range(warm):
        fn()
    out = []
    for _ in range(reps):
        if flush is not None:
            flush()
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(inner):
            fn()
        b.record()
        b.synchronize()
        out.append(a.elapsed_time(b) / inner)
    return out


def ln_cold_ms(torch, C, n: int, ln_w, ln_b, reps: int, dev) -> float:
    """Per-launch LayerNorm time over [1, n, n, 128] bf16 with inputs and
    outputs outside every cache: K launches, launch k reading its own input
    (K inputs in rotation, together at least 768 MiB, three times the
    256 MiB MALL, so an input was last touched K - 1 launches earlier) and
    writing its own output.  The K launches are captured in a HIP graph and
    replayed between two events, so the figure is device time (no host
    dispatch between launches); a 1 GiB read ahead of the first event keeps
    the queue busy.  Median over reps of (elapsed / K)."""
    per = n * n * C_Z * 2
    k = max(4, -(-(768 << 20) // per))
    xs = [torch.randn(1, n, n, C_Z, device=dev).to(torch.bfloat16) for _ in range(k)]
    flush = torch.zeros(1 << 30, dtype=torch.uint8, device=dev)
    run = lambda: [C.layernorm(x, ln_w, ln_b, 1e-5) for x in xs]  # noqa: E731
    run()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        ys = run()
    out = []
    for rep in range(reps + 2):
        flush.sum()
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        graph.replay()
        b.record()
        b.synchronize()
        if rep >= 2:
            out.append(a.elapsed_time(b) / k)
    del ys, graph, xs, flush
    return statistics.median(out)


def calibration_copy(torch, dev, mib: int) -> None:
    """Three copies of a mib-MiB fp32 tensor (HIP's own copy kernel, mib MiB
    read and mib MiB written): the known traffic that scales the HBM byte
    counters."""
    src = torch.ones((mib << 20) // 4, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    del src, dst


LN_ROTATIONS = {1024: 3, 512: 12}  # inputs in rotation per N (>= 768 MiB each)


def ln_counter_run(torch, C, dev, calibrate_mib: int) -> int:
    """LayerNorm launches only, for HBM byte counters (rocprofv3 --pmc
    FETCH_SIZE, then WRITE_SIZE) and a kernel trace of the same launches.
    For each N in LN_ROTATIONS: K bf16 inputs [1, N, N, 128] (K x N^2 x 256 B
    >= 768 MiB, three times the 256 MiB MALL), launched in rotation for two
    passes, each launch writing its own output; so the input a launch reads
    was last touched K - 1 launches earlier and cannot be cached.  Then the
    calibration copy.  Prints per-launch kernel times (HIP events around each
    launch, second pass) as one JSON line."""
    w, b = torch.ones(C_Z, device=dev), torch.zeros(C_Z, device=dev)
    times = {}
    with torch.no_grad():
        for n, k in LN_ROTATIONS.items():
            print(f"[bench] LayerNorm counter run: N={n}, {k} inputs x 2 passes", file=sys.stderr,
                  flush=True)
            xs = [torch.randn(1, n, n, C_Z, device=dev).to(torch.bfloat16) for _ in range(k)]
            ys = [C.layernorm(x, w, b, 1e-5) for x in xs]
            torch.cuda.synchronize()
            C.timing_enable(True)
            ys = [C.layernorm(x, w, b, 1e-5) for x in xs]
            rep = C.timing_report()
            C.timing_enable(False)
            torch.cuda.synchronize()
            cnt, total, mn, mx = rep["layernorm"]
            avg = total / cnt
            times[f"n{n}"] = {"launches": cnt, "avg_ms": round(avg, 4), "min_ms": round(mn, 4),
                              "gbps": round(ln_bytes(n) / (avg * 1e-3) / 1e9, 1),
                              "frac_hbm": round(ln_bytes(n) / (avg * 1e-3) / PEAK_HBM_BYTES, 4)}
            del xs, ys
            torch.cuda.empty_cache()
        if calibrate_mib > 0:
            calibration_copy(torch, dev, calibrate_mib)
    torch.cuda.synchronize()
    print(json.dumps({"layernorm_rotation": times}))
    return 0


def summarize_ln(fetch_csv: str, write_csv: str, trace_csv: str, copy_mib: int) -> int:
    """Markdown table of HBM bytes and rate per LayerNorm launch from
    `bench.py --only-ln` run three times: under rocprofv3 --pmc FETCH_SIZE,
    --pmc WRITE_SIZE (both with --calibrate-copy copy_mib) and --kernel-trace.
    Launches are grouped by N (grid = 8 N^2 threads); each group's second
    rotation pass is summarised (median bytes, calibrated by the copy kernel;
    mean duration from the kernel trace)."""
    import csv

    fetch = _pmc_per_dispatch(fetch_csv, "FETCH_SIZE")
    write = _pmc_per_dispatch(write_csv, "WRITE_SIZE")
    copy_bytes = copy_mib * 2.0 ** 20
    f_fac = copy_bytes / (max(v for (n, g, v) in fetch.values() if "copyBuffer" in n) * 1024.0)
    w_fac = copy_bytes / (max(v for (n, g, v) in write.values() if "copyBuffer" in n) * 1024.0)

    def second_pass(d, grid):
        ids = sorted((int(i) for i, (n, g, _) in d.items() if "ln_rows_kernel" in n and g == grid))
        return ids[len(ids) // 2:]

    durs = {}
    for r in csv.DictReader(open(trace_csv)):
        if "ln_rows_kernel" not in r["Kernel_Name"]:
            continue
        grid = int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"])
        durs.setdefault(grid, []).append(
            (int(r["Dispatch_Id"]), (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) * 1e-9))
    mib = 2.0 ** 20
    print("| N | launches | read MiB | written MiB | HBM MiB | algorithmic MiB | HBM / algorithmic | "
          "avg us (kernel trace) | GB/s (algorithmic bytes) | GB/s (counter bytes) | % of 8 TB/s |")
    print("|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|")
    for n in sorted(LN_ROTATIONS):
        grid = 8 * n * n
        fi, wi = second_pass(fetch, grid), second_pass(write, grid)
        if not fi or not wi or grid not in durs:
            continue
        fb = statistics.median(fetch[str(i)][2] * 1024.0 * f_fac for i in fi)
        wb = statistics.median(write[str(i)][2] * 1024.0 * w_fac for i in wi)
        d = sorted(durs[grid])
        t = statistics.mean(x for _, x in d[len(d) // 2:])
        alg = ln_bytes(n)
        print(f"| {n} | {len(fi)} | {fb / mib:.1f} | {wb / mib:.1f} | {(fb + wb) / mib:.1f} | "
              f"{alg / mib:.1f} | {(fb + wb) / alg:.3f} | {t * 1e6:.1f} | {alg / t / 1e9:.0f} | "
              f"{(fb + wb) / t / 1e9:.0f} | {100 * (fb + wb) / t / PEAK_HBM_BYTES:.1f} |")
    print(f"\ncalibration ({copy_mib} MiB copy): fetch bytes = FETCH_SIZE x {f_fac:.4f} KiB, "
          f"write bytes = WRITE_SIZE x {w_fac:.4f} KiB")
    return 0


def host_cpu() -> dict:
    """CPU model and physical core count of this host (from /proc/cpuinfo)."""
    model, cores = None, set()
    phys = core = None
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                k, _, v = line.partition(":")
                k, v = k.strip(), v.strip()
                if k == "model name" and model is None:
                    model = v
                elif k == "physical id":
                    phys = v
                elif k == "core id":
                    core = v
                elif not k and phys is not None:
                    cores.add((phys, core))
                    phys = core = None
    except OSError:  # pragma: no cover
        pass
    return {"model": model, "physical_cores": len(cores) or None}


def cpu_threads() -> int:
    """torch threads for the CPU baseline: the CPUs this process may run on,
    at most 16 (the host share of a one-GPU box)."""
    return max(1, min(len(os.sched_getaffinity(0)), 16))


def cpu_modules(torch, mods: dict) -> dict:
    """fp32 host copies of the GPU modules (same weights), PyTorch path only."""
    import copy

    out = {}
    for k, m in mods.items():
        c = copy.deepcopy(m).to("cpu", torch.float32).eval()
        c._fused_requested = False
        out[k] = c
    return out


def cpu_time_ops(torch, cmods: dict, N: int, tail: int = 0, reps: int = 3,
                 chunk: int = 64) -> dict:
    """Median seconds (after one warmup) of each operator's PyTorch path in
    fp32 on the host: tri-mul outgoing / incoming, tri-attn starting / ending
    (attention rows chunked by `chunk`, result-identical), LayerNorm.  The
    inputs are seeded; tail > 0 masks pairs past `tail`."""
    import torch.nn.functional as F

    g = torch.Generator().manual_seed(0)
    z = torch.randn(1, N, N, C_Z, generator=g)
    m = torch.ones(1, N, N)
    if tail:
        m[:, tail:, :] = 0
        m[:, :, tail:] = 0
    w, b = torch.ones(C_Z), torch.zeros(C_Z)
    fns = {
        "tri_mul_out": lambda: cmods["tri_mul_out"](z, m),
        "tri_mul_in": lambda: cmods["tri_mul_in"](z, m),
        "tri_att_start": lambda: cmods["tri_att_start"](z, m, chunk_size=chunk),
        "tri_att_end": lambda: cmods["tri_att_end"](z, m, chunk_size=chunk),
        "layernorm": lambda: F.layer_norm(z, (C_Z,), w, b, 1e-5),
    }
    out = {}
    with torch.no_grad():
        for k, f in fns.items():
            f()
            ts = []
            for _ in range(reps):
                t0 = time.perf_counter()
                f()
                ts.append(time.perf_counter() - t0)
            out[k] = statistics.median(ts)
    return out


def cpu_baseline(torch, mods: dict, N: int) -> dict:
    """The reference's PyTorch fallback (the modules' _forward_pytorch, fp32)
    on the host cores, for the same step: 1 warmup, median of 3 per operator."""
    threads = cpu_threads()
    torch.set_num_threads(threads)
    cmods = cpu_modules(torch, mods)
    t = cpu_time_ops(torch, cmods, N)
    step_s = sum(t.values())
    flops = step_flops_of(trimul_flops(N), triattn_flops(N))
    cpu = host_cpu()
    return {
        "value": round(flops / step_s / 1e12, 4),
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"the modules' PyTorch path (the reference fallback) in fp32 on the host, the "
                   f"whole step at N={N}: each operator 1 warmup + median of 3 "
                   f"(tri-attn rows in chunks of 64, result-identical); "
                   + ", ".join(f"{k} {v:.3f} s" for k, v in t.items())
                   + f"; {threads} torch threads (sched_getaffinity, at most 16) on "
                   f"{cpu['model']} ({cpu['physical_cores']} physical cores)"),
        "ms_per_step": round(step_s * 1e3, 1),
        "op_ms": {k: round(v * 1e3, 1) for k, v in t.items()},
        "cpu_model": cpu["model"],
        "physical_cores": cpu["physical_cores"],
    }


# rocprofv3 kernel names -> the per-kernel names used above (first match wins)
KERNEL_KEYS = [
    ("trimul_prologue_bf16_kernel", "trimul_prologue"),
    ("trimul_contract_bf16_kernel", "trimul_contract"),
    ("trimul_epilogue_bf16_kernel", "trimul_epilogue"),
    ("triattn_prologue_bf16_kernel", "triattn_prologue"),
    ("triattn_flash_rh_kernel", "triattn_flash"),
    ("triattn_flash_kernel", "triattn_flash"),
    ("triattn_out_kernel", "triattn_out"),
    ("ln_rows_kernel", "layernorm"),
    ("pair_transition_bf16_kernel", "pair_transition"),
]


def algorithmic_bytes(N: int, B: int = 1) -> dict:
    """Compulsory HBM bytes per launch of each forward kernel (bf16 pair
    tensors, fp32 mask; the bench's modules run without residual)."""
    pair = 2.0 * B * N * N * C_Z
    mask = 4.0 * B * N * N
    plane = 2.0 * B * N * N * C_HID
    bias16 = 2.0 * B * HEADS * N * N  # the triangle bias, bf16
    return {
        "trimul_prologue": pair + mask + 2 * plane,
        "trimul_contract": 3 * plane,
        "trimul_epilogue": plane + 2 * pair,
        "triattn_prologue": pair + 4 * pair + bias16 + mask + mask / 16,
        "triattn_flash": 4 * pair + bias16 + mask / 16 + pair,
        "triattn_out": 2 * pair,
        "layernorm": 2 * pair,
        "pair_transition": 2 * pair + mask,
    }


def _kernel_key(name: str):
    for frag, key in KERNEL_KEYS:
        if frag in name:
            return key
    return None


def _pmc_per_dispatch(path: str, counter: str) -> dict:
    """{dispatch id: (kernel name, grid size, summed counter value)} of a
    rocprofv3 counter_collection.csv."""
    import csv

    out = {}
    with open(path) as fh:
        for r in csv.DictReader(fh):
            if r["Counter_Name"] != counter:
                continue
            d = r["Dispatch_Id"]
            name, grid, val = out.get(d, (r["Kernel_Name"], int(r["Grid_Size"]), 0.0))
            out[d] = (name, grid, val + float(r["Counter_Value"]))
    return out


def summarize_traffic(fetch_csv: str, write_csv: str, N: int, copy_mib: int) -> int:
    """FETCH_SIZE / WRITE_SIZE (KiB per dispatch) of a bench run under
    rocprofv3 --pmc, scaled by what the counters read for the calibration copy
    (--calibrate-copy: copy_mib MiB read and written), as bytes per launch;
    medians over each kernel's launches at this N.  Writes
    profiles/traffic.json and prints a markdown table."""
    fetch = _pmc_per_dispatch(fetch_csv, "FETCH_SIZE")
    write = _pmc_per_dispatch(write_csv, "WRITE_SIZE")
    copy_bytes = copy_mib * 2.0 ** 20
    # the calibration copy: --calibrate-copy's copy_() runs as HIP's own
    # buffer-copy kernel (the largest launch of it)
    def calib(d):
        return max(v for (n, g, v) in d.values() if "copyBuffer" in n)
    f_fac = copy_bytes / (calib(fetch) * 1024.0)
    w_fac = copy_bytes / (calib(write) * 1024.0)
    alg = algorithmic_bytes(N)
    # meant for a run of `--only-step`, where every launch is at this N; a
    # full bench run also launches every kernel at N = 256 and 2N, and of
    # those only LayerNorm's are told apart here (grid 8 N^2 threads)
    ln_grid = 8 * N * N
    by = {}
    for src, fac, kind in ((fetch, f_fac, "fetch"), (write, w_fac, "write")):
        for name, grid, val in src.values():
            key = _kernel_key(name)
            if key is None:
                continue
            if key == "layernorm" and grid != ln_grid:
                continue
            by.setdefault(key, {}).setdefault(kind, []).append((grid, val * 1024.0 * fac))
    out = {"_calibration": {"copy_bytes": int(copy_bytes), "fetch_factor": round(f_fac, 4),
                            "write_factor": round(w_fac, 4)}}
    print("| kernel | read MiB | written MiB | HBM MiB | algorithmic MiB | HBM / algorithmic |")
    print("|---|---:|---:|---:|---:|---:|")
    for key in alg:
        if key not in by:
            continue
        kinds = by[key]
        if key == "layernorm":
            kinds = {k: [x for x in v if x[0] == ln_grid] for k, v in kinds.items()}
        fb = statistics.median(v for _, v in kinds["fetch"])
        wb = statistics.median(v for _, v in kinds["write"])
        out[f"{key}@N={N}"] = {"fetch_bytes": int(fb), "write_bytes": int(wb), "hbm_bytes": int(fb + wb),
                               "algorithmic_bytes": int(alg[key]), "ratio": round((fb + wb) / alg[key], 3)}
        mib = 2.0 ** 20
        print(f"| {key} | {fb / mib:.1f} | {wb / mib:.1f} | {(fb + wb) / mib:.1f} | {alg[key] / mib:.1f} | "
              f"{(fb + wb) / alg[key]:.2f} |")
    print(f"\ncalibration: fetch bytes = FETCH_SIZE x {f_fac:.4f} KiB, write bytes = WRITE_SIZE x {w_fac:.4f} KiB")
    with open(os.path.join(ROOT, "profiles", "traffic.json"), "w") as fh:
        json.dump(out, fh, indent=1)
        fh.write("\n")
    return 0


def _short_name(name: str) -> str:
    """Readable kernel name: demangled by c++filt when it is on PATH, template
    arguments kept, parameter list dropped."""
    if name.startswith("_Z"):
        import shutil
        import subprocess

        if shutil.which("c++filt"):
            name = subprocess.run(["c++filt", name], capture_output=True, text=True).stdout.strip() or name
    if name.startswith("_ZN"):
        # left mangled (a demangler without the bf16 type): the kernel's own
        # name and its integer template arguments
        import re

        m = re.match(r"_ZN(?:3gtk)?(\d+)", name)
        if m:
            base = name[m.end():m.end() + int(m.group(1))]
            rest = name[m.end() + int(m.group(1)):]
            tmpl = rest[:rest.find("Ev")] if "Ev" in rest else ""
            args = ["bf16" if t == "DF16b" else t for t in re.findall(r"Li(\d+)E|(DF16b)", tmpl) for t in t if t]
            return f"{base}<{', '.join(args)}>" if args else base
    return name.split("(")[0].replace("void ", "").replace("gtk::", "")


def _pmc_by_kernel(path: str) -> dict:
    """{short kernel name: {counter: [per-dispatch values]}} of a rocprofv3
    counter_collection.csv (values summed over a dispatch's rows)."""
    import csv

    per = {}
    with open(path) as fh:
        for r in csv.DictReader(fh):
            key = (r["Dispatch_Id"], r["Counter_Name"])
            per.setdefault(key, [r["Kernel_Name"], 0.0])[1] += float(r["Counter_Value"])
    out, names = {}, {}
    for (_, ctr), (raw, v) in per.items():
        name = names.setdefault(raw, _short_name(raw))
        out.setdefault(name, {}).setdefault(ctr, []).append(v)
    return out


def summarize_pmc(mfma_csv: str, issue_csv: str, stats_csv: str, N: int) -> int:
    """Markdown table of the matrix-core and VALU counters per product kernel
    from two rocprofv3 --pmc passes over `bench.py --only-step` (pass 1:
    MfmaUtil MfmaFlopsBF16 VALUBusy; pass 2: SQ_INSTS_VALU_TRANS_F32
    SQ_INSTS_VALU SQ_INSTS_MFMA SQ_VALU_MFMA_BUSY_CYCLES
    SQ_VALU_MFMA_COEXEC_CYCLES SQ_WAIT_INST_ANY SQ_WAVE_CYCLES SQ_BUSY_CYCLES)
    and the kernel-trace stats of the same command (durations)."""
    import csv

    a, b = _pmc_by_kernel(mfma_csv), _pmc_by_kernel(issue_csv)
    dur = {}
    for r in csv.DictReader(open(stats_csv)):
        dur[_short_name(r["Name"])] = float(r["AverageNs"]) * 1e-9
    work = dict(trimul_flops(N))
    work.update(triattn_flops(N))
    med = statistics.median
    print("| kernel | avg us | MFMA GFLOP (counter) | algorithmic GFLOP | counter TFLOP/s | "
          "% bf16 peak | MfmaUtil % | VALUBusy % | v_exp etc. (M lanes) | VALU instr (M) | "
          "MFMA instr (M) | MFMA-VALU co-exec % of MFMA busy | wait % of wave cycles |")
    print("|---|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|")
    for name in sorted(a, key=lambda n: -dur.get(n, 0.0)):
        key = _kernel_key(name)
        ca, cb = a[name], b.get(name, {})
        if "MfmaFlopsBF16" not in ca or name not in dur:
            continue
        fl = med(ca["MfmaFlopsBF16"])
        t = dur[name]
        alg = work.get(key)
        busy = med(cb["SQ_VALU_MFMA_BUSY_CYCLES"]) if "SQ_VALU_MFMA_BUSY_CYCLES" in cb else 0.0
        coex = med(cb["SQ_VALU_MFMA_COEXEC_CYCLES"]) if "SQ_VALU_MFMA_COEXEC_CYCLES" in cb else 0.0
        wait = (med(cb["SQ_WAIT_INST_ANY"]) / med(cb["SQ_WAVE_CYCLES"])
                if cb.get("SQ_WAVE_CYCLES") and med(cb["SQ_WAVE_CYCLES"]) > 0 else float("nan"))
        cell = lambda c, f=1e-6: f"{med(cb[c]) * f:.1f}" if c in cb else "—"  # noqa: E731
        print(f"| {name} | {t * 1e6:.1f} | {fl / 1e9:.2f} | {alg / 1e9 if alg else float('nan'):.2f} | "
              f"{fl / t / 1e12:.0f} | {100 * fl / t / PEAK_BF16_FLOPS:.1f} | {med(ca['MfmaUtil']):.1f} | "
              f"{med(ca['VALUBusy']):.1f} | {med(cb['SQ_INSTS_VALU_TRANS_F32']) * 64e-6 if 'SQ_INSTS_VALU_TRANS_F32' in cb else float('nan'):.0f} | "
              f"{cell('SQ_INSTS_VALU')} | {cell('SQ_INSTS_MFMA')} | "
              f"{100 * coex / busy if busy else float('nan'):.1f} | {100 * wait:.1f} |")
    return 0


def summarize_stats(stats_csv: str) -> int:
    """Markdown table of a rocprofv3 --kernel-trace --stats kernel_stats.csv
    (durations in microseconds per launch)."""
    import csv

    rows = list(csv.DictReader(open(stats_csv)))
    total = sum(float(r["TotalDurationNs"]) for r in rows)
    print("| kernel | calls | avg us | min us | max us | % of GPU time |")
    print("|---|---:|---:|---:|---:|---:|")
    for r in sorted(rows, key=lambda r: -float(r["TotalDurationNs"])):
        short = _short_name(r["Name"])
        print(f"| {short} | {r['Calls']} | {float(r['AverageNs']) / 1e3:.1f} | {float(r['MinNs']) / 1e3:.1f} | "
              f"{float(r['MaxNs']) / 1e3:.1f} | {100 * float(r['TotalDurationNs']) / total:.2f} |")
    return 0


def op_targets(N: int) -> dict:
    """ms of each operator at the targets: 50 % of bf16 MFMA peak for the
    triangle operators, 70 % of HBM for LayerNorm."""
    fm, fa = sum(trimul_flops(N).values()), sum(triattn_flops(N).values())
    return {"tri_mul": fm / (0.5 * PEAK_BF16_FLOPS) * 1e3, "tri_att": fa / (0.5 * PEAK_BF16_FLOPS) * 1e3,
            "layernorm": ln_bytes(N) / (0.7 * PEAK_HBM_BYTES) * 1e3}


def call_split(torch, C, call, reps: int) -> dict:
    """Where one operator call's time goes: device_ms, the sum of its kernels'
    durations (HIP events around each launch on its stream), and host_us,
    the host time to issue one call (Python, binding, allocations and
    launches; calls issued back to back, the GPU synchronised only at the
    end).  A call time (ms) near device_ms means the operator is bound by
    the GPU, not by the host."""
    C.timing_enable(True)
    for _ in range(reps):
        call()
    rep = C.timing_report()
    C.timing_enable(False)
    dev_ms = sum(v[1] for v in rep.values()) / reps
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        call()
    host_us = (time.perf_counter() - t0) / reps * 1e6
    torch.cuda.synchronize()
    return {"device_ms": round(dev_ms, 4), "host_us": round(host_us, 1),
            "kernels_ms": {k: round(v[1] / reps, 4) for k, v in rep.items()}}


def gpu_ops_at(torch, C, dev: str, N: int, tail: int, reps: int) -> dict:
    """Median event time of each operator (bf16, module kernel path) at size N,
    with the pair mask zero past `tail` (0: all ones); TFLOP/s or GB/s, and the
    fraction of the target time."""
    mods = build_modules(torch, N, dev)
    g = torch.Generator(device=dev).manual_seed(N)
    z = torch.randn(1, N, N, C_Z, device=dev, generator=g).to(torch.bfloat16)
    m = torch.ones(1, N, N, device=dev)
    if tail:
        m[:, tail:, :] = 0
        m[:, :, tail:] = 0
    w, b = torch.ones(C_Z, device=dev), torch.zeros(C_Z, device=dev)
    tg = op_targets(N)
    out = {"N": N, "mask": f"pairs with i, j < {tail}" if tail else "ones"}
    with torch.no_grad():
        for k in ("tri_mul_out", "tri_mul_in", "tri_att_start", "tri_att_end"):
            call = lambda: mods[k](z, m)  # noqa: E731
            ms = statistics.median(event_time_ms(torch, call, reps, inner=OP_INNER))
            fl = sum((trimul_flops if k.startswith("tri_mul") else triattn_flops)(N).values())
            t = tg["tri_mul" if k.startswith("tri_mul") else "tri_att"]
            out[k] = {"ms": round(ms, 4), "tflops": round(fl / (ms * 1e-3) / 1e12, 1),
                      "frac_bf16_peak": round(fl / (ms * 1e-3) / PEAK_BF16_FLOPS, 4),
                      "target_ms": round(t, 4), "time_over_target": round(ms / t, 2)}
            if N <= 256:
                out[k].update(call_split(torch, C, call, reps))
        ms = statistics.median(event_time_ms(torch, lambda: C.layernorm(z, w, b, 1e-5), reps,
                                             inner=OP_INNER))
        out["layernorm"] = {"ms": round(ms, 4), "gbps": round(ln_bytes(N) / (ms * 1e-3) / 1e9, 1),
                            "frac_hbm": round(ln_bytes(N) / (ms * 1e-3) / PEAK_HBM_BYTES, 4),
                            "target_ms": round(tg["layernorm"], 4)}
    del mods, z
    torch.cuda.synchronize()
    return out


def config_table(torch, C, dev: str) -> int:
    """GPU (bf16 kernels, fp32 for the N=64 tri-mul) and host-CPU (the PyTorch
    fallback in fp32) times of the operators at the five benchmark workloads,
    numbered in the table's first column:
    1: tri-mul outgoing, fp32, N=64; 2: tri-mul outgoing / incoming, N=256,
    mask i, j < 224; 3: tri-attn starting / ending, same; 4: the pair-stack
    block (LN-free PairTransformLayer order: tri-mul out, in, tri-attn start,
    end, transition, each with residual, then the mask), B=2, N=512, lengths
    384 and 512; 5: tri-mul outgoing, tri-attn starting and LayerNorm,
    N=1024."""
    import torch.nn.functional as F

    threads = cpu_threads()
    torch.set_num_threads(threads)
    cpu = host_cpu()
    rows = []

    def gpu_ms(fn, reps=OP_REPS):
        with torch.no_grad():
            return statistics.median(event_time_ms(torch, fn, reps, inner=OP_INNER))

    def cpu_ms(fn, reps=3):
        with torch.no_grad():
            fn()
            ts = []
            for _ in range(reps):
                t0 = time.perf_counter()
                fn()
                ts.append(time.perf_counter() - t0)
        return statistics.median(ts) * 1e3

    def mask(B, N, lengths):
        m = torch.zeros(B, N, N)
        for i, L in enumerate(lengths):
            m[i, :L, :L] = 1
        return m

    def add(cfg, op, N, gms, cms, gflop=None, mb=None):
        perf = (f"{gflop / gms:.0f} TFLOP/s ({100 * gflop * 1e9 / (gms * 1e-3) / PEAK_BF16_FLOPS:.1f} %)"
                if gflop else f"{mb * 1e6 / (gms * 1e-3) / 1e9:.0f} GB/s "
                              f"({100 * mb * 1e6 / (gms * 1e-3) / PEAK_HBM_BYTES:.1f} % HBM)")
        rows.append(f"| {cfg} | {op} | {N} | {cms:.1f} | {gms:.4f} | {cms / gms:.0f}x | {perf} |")
        print(f"[config-table] {cfg} {op}: GPU {gms:.4f} ms, CPU {cms:.1f} ms", file=sys.stderr, flush=True)

    for n_cfg, N, lengths, ops in ((1, 64, None, ("tri_mul_out",)),
                                   (2, 256, [224], ("tri_mul_out", "tri_mul_in")),
                                   (3, 256, [224], ("tri_att_start", "tri_att_end")),
                                   (5, 1024, None, ("tri_mul_out", "tri_att_start"))):
        mods = build_modules(torch, N, dev)
        dt = torch.float32 if n_cfg == 1 else torch.bfloat16
        if n_cfg == 1:
            mods = {k: v.float() for k, v in mods.items()}
        cm = cpu_modules(torch, mods)
        g = torch.Generator().manual_seed(n_cfg)
        zc = torch.randn(1, N, N, C_Z, generator=g)
        mc = mask(1, N, lengths) if lengths else torch.ones(1, N, N)
        zg, mg = zc.to(dev, dt), mc.to(dev)
        for op in ops:
            chunk = {"chunk_size": 64} if op.startswith("tri_att") else {}
            gms = gpu_ms(lambda: mods[op](zg, mg))
            cms = cpu_ms(lambda: cm[op](zc, mc, **chunk))
            fl = sum((trimul_flops if op.startswith("tri_mul") else triattn_flops)(N).values())
            add(n_cfg, op, N, gms, cms, gflop=fl / 1e9)
        if n_cfg == 5:
            w, b = torch.ones(C_Z), torch.zeros(C_Z)
            gms = gpu_ms(lambda: C.layernorm(zg, w.to(dev), b.to(dev), 1e-5))
            cms = cpu_ms(lambda: F.layer_norm(zc, (C_Z,), w, b, 1e-5))
            add(5, "layernorm", N, gms, cms, mb=ln_bytes(N) / 1e6)
        del mods, cm, zg
        torch.cuda.synchronize()
    # workload 4: the pair-stack block, B = 2, N = 512, lengths 384 and 512
    layer = build_pair_layer(torch, dev)
    cl = copy_layer = cpu_modules(torch, {"l": layer})["l"]
    for mod in cl.modules():
        if hasattr(mod, "_fused_requested"):
            mod._fused_requested = False
    g = torch.Generator().manual_seed(4)
    zc = torch.randn(2, 512, 512, C_Z, generator=g)
    mc = mask(2, 512, [384, 512])
    zg, mg = zc.to(dev, torch.bfloat16), mc.to(dev)

    def cpu_block():
        p = zc
        p = p + cl.tri_mul_out(p, mc)
        p = p + cl.tri_mul_in(p, mc)
        p = p + cl.tri_att_start(p, mc, chunk_size=64)
        p = p + cl.tri_att_end(p, mc, chunk_size=64)
        p = p + cl.pair_transition(p, mc)
        return p * mc.unsqueeze(-1)

    gms = gpu_ms(lambda: layer((zg, mg)))
    cms = cpu_ms(cpu_block, reps=1)
    fl = 2 * (step_flops_of(trimul_flops(512), triattn_flops(512)) + transition_flops(512))
    add(4, "pair-stack block (B=2)", 512, gms, cms, gflop=fl / 1e9)
    del layer, copy_layer
    print(f"Host CPU: {cpu['model']}, {cpu['physical_cores']} physical cores; {threads} torch "
          f"threads. CPU: the modules' PyTorch path in fp32 (tri-attn rows in chunks of 64), "
          f"1 warmup + median of 3 (the pair-stack block: 1 warmup + 1). GPU: bf16 kernels (the N=64 tri-mul: "
          f"fp32), median of {OP_REPS} repetitions after {OP_WARM} warmup calls, each {OP_INNER} back-to-back calls between two "
          f"events.\n")
    print("| config | operator | N | CPU fp32 ms | GPU ms | speed-up | GPU throughput |")
    print("|---|---|---:|---:|---:|---:|---|")
    print("\n".join(rows))
    return 0


def fwd_bwd_run(torch, mods, z, mask, steps: int, warmup: int) -> int:
    """Forward + backward (the input's and every parameter's gradient) of
    tri-mul outgoing and tri-attn starting node, `steps` times each after
    `warmup`; prints their median times as one JSON line."""
    maskb = mask.to(torch.bfloat16)
    out = {}
    for name in ("tri_mul_out", "tri_att_start"):
        mod = mods[name]
        zg = z.detach().clone().requires_grad_(True)
        dy = torch.randn_like(z)

        def run():
            zg.grad = None
            for p in mod.parameters():
                p.grad = None
            mod(zg, maskb).backward(dy)
        for _ in range(warmup):
            run()
        out[name] = round(statistics.median(event_time_ms(torch, run, steps)), 4)
        print(f"[bench] {name} forward+backward {out[name]:.3f} ms", file=sys.stderr, flush=True)
    print(json.dumps({"fwd_bwd_ms": out}))
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--n", type=int, default=512, help="pair length N")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="after the measurements, copy a MIB-MiB fp32 tensor 3 times (a plain "
                         "copy kernel of known traffic, for scaling HBM byte counters)")
    ap.add_argument("--summarize-traffic", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="no run: summarize the counter_collection.csv files of FETCH_SIZE and "
                         "WRITE_SIZE passes over a bench run with --calibrate-copy (its MiB in "
                         "--calibrate-copy) into profiles/traffic.json")
    ap.add_argument("--summarize-stats", metavar="STATS_CSV",
                    help="no run: markdown table of a rocprofv3 kernel_stats.csv")
    ap.add_argument("--summarize-pmc", nargs=3, metavar=("MFMA_CSV", "ISSUE_CSV", "STATS_CSV"),
                    help="no run: matrix-core / VALU counter table of two --pmc passes and the "
                         "kernel-trace stats of `bench.py --only-step`")
    ap.add_argument("--only-step", action="store_true",
                    help="time the step and its kernels only (for counter collection)")
    ap.add_argument("--only-fwd-bwd", action="store_true",
                    help="no bench line: forward + backward of tri-mul outgoing and tri-attn "
                         "starting at N (for a kernel trace of the backward kernels)")
    ap.add_argument("--only-ln", action="store_true",
                    help="no bench line: LayerNorm launches over rotating inputs at N=1024 and "
                         "N=512 (for HBM byte counters and a kernel trace), then --calibrate-copy")
    ap.add_argument("--summarize-ln", nargs=3, metavar=("FETCH_CSV", "WRITE_CSV", "TRACE_CSV"),
                    help="no run: LayerNorm HBM bytes and rate per launch from FETCH_SIZE / "
                         "WRITE_SIZE passes and a kernel trace of `bench.py --only-ln` (its MiB "
                         "in --calibrate-copy)")
    ap.add_argument("--config-table", action="store_true",
                    help="no bench line: GPU and host-CPU times of the operators at the "
                         "benchmark configurations 1-5, as a markdown table")
    args = ap.parse_args()
    if args.summarize_traffic:
        return summarize_traffic(*args.summarize_traffic, N=args.n, copy_mib=args.calibrate_copy)
    if args.summarize_stats:
        return summarize_stats(args.summarize_stats)
    if args.summarize_pmc:
        return summarize_pmc(*args.summarize_pmc, N=args.n)
    if args.summarize_ln:
        return summarize_ln(*args.summarize_ln, copy_mib=args.calibrate_copy)
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(the path has no multi-GPU implementation)", file=sys.stderr)
        return 2

    import torch

    from genie_tk import _ext

    C = _ext.require()
    dev = "cuda:0"
    torch.cuda.set_device(0)
    if args.config_table:
        return config_table(torch, C, dev)
    if args.only_ln:
        return ln_counter_run(torch, C, dev, args.calibrate_copy)
    N = args.n
    torch.manual_seed(0)
    z = torch.randn(1, N, N, C_Z, device=dev).to(torch.bfloat16)
    mask = torch.ones(1, N, N, device=dev)
    ln_w = torch.ones(C_Z, device=dev)
    ln_b = torch.zeros(C_Z, device=dev)
    mods = build_modules(torch, N, dev)
    if args.only_fwd_bwd:
        return fwd_bwd_run(torch, mods, z, mask, args.steps, args.warmup)

    ops = {
        "tri_mul_out": lambda: mods["tri_mul_out"](z, mask),
        "tri_mul_in": lambda: mods["tri_mul_in"](z, mask),
        "tri_att_start": lambda: mods["tri_att_start"](z, mask),
        "tri_att_end": lambda: mods["tri_att_end"](z, mask),
        "layernorm": lambda: C.layernorm(z, ln_w, ln_b, 1e-5),
    }

    def step():
        for f in ops.values():
            f()

    with torch.no_grad():
        print(f"[bench] N={N} warmup {args.warmup}", file=sys.stderr, flush=True)
        for _ in range(args.warmup):
            step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            step()
        torch.cuda.synchronize()
        step_ms = (time.perf_counter() - t0) * 1e3 / args.steps
        print(f"[bench] timed {args.steps} steps: {step_ms:.3f} ms/step", file=sys.stderr, flush=True)

        # per-operator event timing
        reps = max(OP_REPS, args.steps)
        op_ms = {k: statistics.median(event_time_ms(torch, f, reps, inner=OP_INNER))
                 for k, f in ops.items()}

        # per-kernel durations from events around each launch
        C.timing_enable(True)
        for _ in range(args.steps):
            step()
        rep = C.timing_report()
        C.timing_enable(False)
        if args.only_step:
            if args.calibrate_copy > 0:
                calibration_copy(torch, dev, args.calibrate_copy)
            torch.cuda.synchronize()
            print(json.dumps({"ms_per_step": round(step_ms, 4),
                              "op_ms": {k: round(v, 4) for k, v in op_ms.items()},
                              "kernels": {k: round(v[1] / v[0], 4) for k, v in rep.items()}}))
            return 0
        # the operators at the other benchmark sizes: N = 256 (tail mask at
        # 224) and N = 1024 (mask ones)
        print("[bench] operators at N=256 and N=1024", file=sys.stderr, flush=True)
        sizes = {f"n{n}": gpu_ops_at(torch, C, dev, n, tail, reps)
                 for n, tail in ((256, 224), (2 * N, 0))}

        # LayerNorm bandwidth with cold caches: launches over rotating inputs
        # larger than the 256 MiB MALL (ln_cold_ms); and, for comparison, one
        # launch after a 1 GiB read that evicts the MALL with clean lines,
        # timed between two events (that figure also holds the launch's
        # dispatch latency after the first event)
        flush_buf = torch.zeros(1 << 30, dtype=torch.uint8, device=dev)
        ln_ms_cold = ln_cold_ms(torch, C, N, ln_w, ln_b, reps, dev)
        ln_ms_cold_single = statistics.median(event_time_ms(torch, ops["layernorm"], reps,
                                                            flush=lambda: flush_buf.sum()))
        # the fp8 a/b storage experiment (outside the bf16 contract): the
        # tri-mul outgoing forward with a and b in fp8 E4M3, against the bf16
        # kernels' output (informational)
        tmo = mods["tri_mul_out"]
        pk8 = tmo._packed_params(False)
        fp8_fwd = lambda: C.tri_mul_forward_fp8ab(z, mask, pk8, C_Z, tmo.c_hidden, True)  # noqa: E731
        fp8_ms = statistics.median(event_time_ms(torch, fp8_fwd, reps))
        y8, y16 = fp8_fwd().float(), tmo(z, mask).float()
        fp8_rel = ((y8 - y16).norm() / y16.norm()).item()
        fp8_max = (y8 - y16).abs().max().item()
        del y8, y16
        # the rest of the pair-stack block on the kernels (informational)
        layer = build_pair_layer(torch, dev)
        trans_ms = statistics.median(event_time_ms(
            torch, lambda: layer.pair_transition.forward_residual_masked(z, mask), reps))
        layer_ms = statistics.median(event_time_ms(torch, lambda: layer((z, mask)), reps))
        del layer
        # the reference layer's default attention shape, c_hidden_tri_att = 32
        # over 4 heads (head dim 8; pair_transform.py:116-117), which the
        # packed weights pad to heads of 32 channels
        layer8 = build_pair_layer(torch, dev, c_att=32)
        att8 = layer8.tri_att_start
        assert att8._kernel_supported(z)
        att8_ms = statistics.median(event_time_ms(torch, lambda: att8(z, mask), reps, inner=OP_INNER))
        layer8_ms = statistics.median(event_time_ms(torch, lambda: layer8((z, mask)), reps))
        del layer8, att8
        # LayerNorm + Linear (nn.Linear-layout weight) over the pair tensor, c -> c
        lw = (torch.randn(C_Z, C_Z, device=dev) / C_Z ** 0.5).to(torch.bfloat16)
        lb = torch.randn(C_Z, device=dev)
        lnlin_ms = statistics.median(event_time_ms(
            torch, lambda: C.layernorm_linear(z, ln_w, ln_b, lw, lb, 1e-5), reps))
        C.timing_enable(True)
        for _ in range(reps):
            C.layernorm_linear(z, ln_w, ln_b, lw, lb, 1e-5)
        lnlin_rep = C.timing_report()
        C.timing_enable(False)
        lnlin_kernel_ms = (lnlin_rep["ln_linear"][1] / lnlin_rep["ln_linear"][0]
                           if "ln_linear" in lnlin_rep else None)
        z2 = torch.randn(1, 2 * N, 2 * N, C_Z, device=dev).to(torch.bfloat16)
        ln2 = lambda: C.layernorm(z2, ln_w, ln_b, 1e-5)  # noqa: E731
        ln2_ms = statistics.median(event_time_ms(torch, ln2, reps))
        del z2, flush_buf
        ln2_ms_cold = ln_cold_ms(torch, C, 2 * N, ln_w, ln_b, reps, dev)
        if args.calibrate_copy > 0:
            calibration_copy(torch, dev, args.calibrate_copy)
    torch.cuda.synchronize()

    # one training step of tri-mul outgoing (forward + backward, gradients of z
    # and every parameter): on the kernels, and through the PyTorch path's
    # autograd for comparison (informational)
    tm = mods["tri_mul_out"]
    zg = z.detach().clone().requires_grad_(True)
    dyg = torch.randn_like(z)
    maskb = mask.to(torch.bfloat16)  # the PyTorch path keeps the mask's dtype

    def fb(fwd):
        def run():
            zg.grad = None
            for p in tm.parameters():
                p.grad = None
            fwd(zg, maskb).backward(dyg)
        return run
    print("[bench] tri-mul forward+backward", file=sys.stderr, flush=True)
    fb_ms = statistics.median(event_time_ms(torch, fb(tm), reps))
    fb_torch_ms = statistics.median(event_time_ms(torch, fb(tm._forward_pytorch), max(3, reps // 4)))
    C.timing_enable(True)
    for _ in range(3):
        fb(tm)()
    fb_rep = C.timing_report()
    C.timing_enable(False)
    del zg, dyg
    # the same for tri-attn starting node
    ta = mods["tri_att_start"]
    xg = z.detach().clone().requires_grad_(True)
    dya = torch.randn_like(z)

    def fba(fwd):
        def run():
            xg.grad = None
            for p in ta.parameters():
                p.grad = None
            fwd(xg, maskb).backward(dya)
        return run
    print("[bench] tri-attn forward+backward", file=sys.stderr, flush=True)
    fba_ms = statistics.median(event_time_ms(torch, fba(ta), reps))
    fba_torch_ms = statistics.median(event_time_ms(torch, fba(ta._forward_pytorch), 3, warm=1))
    C.timing_enable(True)
    for _ in range(3):
        fba(ta)()
    fba_rep = C.timing_report()
    C.timing_enable(False)
    del xg, dya
    torch.cuda.synchronize()

    fm, fa = trimul_flops(N), triattn_flops(N)
    op_flops = {"tri_mul_out": sum(fm.values()), "tri_mul_in": sum(fm.values()),
                "tri_att_start": sum(fa.values()), "tri_att_end": sum(fa.values())}
    per_op = {}
    for k, fl in op_flops.items():
        tf = fl / (op_ms[k] * 1e-3) / 1e12
        per_op[k] = {"ms": round(op_ms[k], 4), "gflop": round(fl / 1e9, 2),
                     "tflops": round(tf, 2), "frac_bf16_peak": round(tf * 1e12 / PEAK_BF16_FLOPS, 4)}
    lnb = ln_bytes(N)
    per_op["layernorm"] = {
        "ms": round(op_ms["layernorm"], 4), "mb": round(lnb / 1e6, 1),
        "gbps_warm": round(lnb / (op_ms["layernorm"] * 1e-3) / 1e9, 1),
        "ms_cold": round(ln_ms_cold, 4),
        "gbps_cold": round(lnb / (ln_ms_cold * 1e-3) / 1e9, 1),
        "frac_hbm_cold": round(lnb / (ln_ms_cold * 1e-3) / PEAK_HBM_BYTES, 4),
        "ms_cold_single_launch": round(ln_ms_cold_single, 4),
        "note": ("cold = launches replayed back to back from a HIP graph, each over its own input, "
                 "the inputs in rotation (at least 768 MiB, 3x the 256 MiB MALL); "
                 "ms_cold_single_launch = one launch after a 1 GiB read, between two events "
                 "(includes the launch's dispatch latency)"),
    }
    ln2b = ln_bytes(2 * N)
    per_op[f"layernorm_n{2 * N}"] = {
        "ms": round(ln2_ms, 4), "mb": round(ln2b / 1e6, 1),
        "gbps": round(ln2b / (ln2_ms * 1e-3) / 1e9, 1),
        "frac_hbm": round(ln2b / (ln2_ms * 1e-3) / PEAK_HBM_BYTES, 4),
        "ms_cold": round(ln2_ms_cold, 4),
        "gbps_cold": round(ln2b / (ln2_ms_cold * 1e-3) / 1e9, 1),
        "frac_hbm_cold": round(ln2b / (ln2_ms_cold * 1e-3) / PEAK_HBM_BYTES, 4),
    }

    per_op["tri_mul_out_fp8ab"] = {
        "ms": round(fp8_ms, 4), "bf16_ms": round(op_ms["tri_mul_out"], 4),
        "speedup_vs_bf16": round(op_ms["tri_mul_out"] / fp8_ms, 3),
        "rel_diff_vs_bf16": round(fp8_rel, 5), "max_abs_diff_vs_bf16": round(fp8_max, 5),
        "workspace_mib": round(C_HID * (N + 255) // 256 * 256 * ((N + 255) // 256 * 256) * 4 / 2 ** 20, 1),
        "note": "experiment: a and b stored as fp8 E4M3 and contracted on the fp8 matrix cores "
                "(x and the epilogue bf16); outside the bf16 tolerance, reported beside it",
    }
    tf = transition_flops(N)
    per_op["pair_transition"] = {
        "ms": round(trans_ms, 4), "gflop": round(tf / 1e9, 2),
        "tflops": round(tf / (trans_ms * 1e-3) / 1e12, 2),
        "frac_bf16_peak": round(tf / (trans_ms * 1e-3) / PEAK_BF16_FLOPS, 4),
        "note": "fused LN -> c->4c -> ReLU -> 4c->c, residual and mask (informational)",
    }
    llf, llb = 2.0 * N * N * C_Z * C_Z, 2 * N * N * C_Z * 2
    per_op["layernorm_linear"] = {
        "ms": round(lnlin_ms, 4), "gflop": round(llf / 1e9, 2), "mb": round(llb / 1e6, 1),
        "kernel_ms": round(lnlin_kernel_ms, 4) if lnlin_kernel_ms else None,
        "kernel_gbps": round(llb / (lnlin_kernel_ms * 1e-3) / 1e9, 1) if lnlin_kernel_ms else None,
        "kernel_frac_hbm": (round(llb / (lnlin_kernel_ms * 1e-3) / PEAK_HBM_BYTES, 4)
                            if lnlin_kernel_ms else None),
        "note": "LN + Linear c->c, nn.Linear-layout weight, bf16; ms includes the per-call weight "
                "packing, kernel_ms is the LN+Linear kernel alone (informational; HBM-bound)",
    }
    lf = step_flops_of(fm, fa) + tf
    per_op["pair_layer"] = {
        "ms": round(layer_ms, 4), "gflop": round(lf / 1e9, 2),
        "tflops": round(lf / (layer_ms * 1e-3) / 1e12, 2),
        "note": "one PairTransformLayer forward on the kernels, residuals fused (informational)",
    }
    fa8 = sum(triattn_flops(N, head_dim=8).values())
    per_op["tri_att_start_d8"] = {
        "ms": round(att8_ms, 4), "gflop": round(fa8 / 1e9, 2),
        "tflops": round(fa8 / (att8_ms * 1e-3) / 1e12, 2),
        "frac_bf16_peak": round(fa8 / (att8_ms * 1e-3) / PEAK_BF16_FLOPS, 4),
        "gflop_as_run": round(sum(fa.values()) / 1e9, 2),
        "ms_head_dim_32": round(op_ms["tri_att_start"], 4),
        "note": "tri-attn starting node of the reference layer's default shape (4 heads of 8 "
                "channels, c_hidden 32); gflop counts head dim 8, the kernels run the heads "
                "padded to 32 (gflop_as_run)",
    }
    lf8 = 2 * sum(fm.values()) + 2 * fa8 + tf
    per_op["pair_layer_default"] = {
        "ms": round(layer8_ms, 4), "gflop": round(lf8 / 1e9, 2),
        "tflops": round(lf8 / (layer8_ms * 1e-3) / 1e12, 2),
        "note": "one PairTransformLayer forward with the reference's default c_hidden_tri_att "
                "= 32 over 4 heads, on the kernels (gflop at head dim 8)",
    }
    fbf = 3 * sum(fm.values())
    per_op["tri_mul_out_fwd_bwd"] = {
        "ms": round(fb_ms, 4), "gflop": round(fbf / 1e9, 2),
        "tflops": round(fbf / (fb_ms * 1e-3) / 1e12, 2),
        "pytorch_autograd_ms": round(fb_torch_ms, 4),
        "speedup_vs_pytorch_autograd": round(fb_torch_ms / fb_ms, 2),
        "stage_ms_per_step": {k: round(v[1] / 3, 4) for k, v in fb_rep.items()},
        "note": "forward + backward (dz and all parameter gradients) of tri-mul outgoing; gflop "
                "counts 3x the forward's products (the backward recomputes the forward on top)",
    }
    fbaf = 3 * sum(fa.values())
    per_op["tri_att_start_fwd_bwd"] = {
        "ms": round(fba_ms, 4), "gflop": round(fbaf / 1e9, 2),
        "tflops": round(fbaf / (fba_ms * 1e-3) / 1e12, 2),
        "pytorch_autograd_ms": round(fba_torch_ms, 4),
        "speedup_vs_pytorch_autograd": round(fba_torch_ms / fba_ms, 2),
        "stage_ms_per_step": {k: round(v[1] / 3, 4) for k, v in fba_rep.items()},
        "note": "forward + backward (dx and all parameter gradients) of tri-attn starting node; "
                "gflop counts 3x the forward's products",
    }
    work = dict(fm)
    work.update(fa)
    kernels = {}
    for name, (cnt, total, mn, mx) in rep.items():
        avg = total / cnt
        entry = {"launches": cnt, "avg_ms": round(avg, 4), "total_ms": round(total, 3)}
        if name in work:
            a = work[name] / (avg * 1e-3)
            entry.update({"bound": "mfma", "achieved_tflops": round(a / 1e12, 2),
                          "frac": round(a / PEAK_BF16_FLOPS, 4)})
        elif name == "layernorm":
            a = lnb / (avg * 1e-3)
            entry.update({"bound": "hbm", "achieved_gbps": round(a / 1e9, 1),
                          "frac": round(a / PEAK_HBM_BYTES, 4)})
        kernels[name] = entry
    dom = max((k for k in kernels if k in work), key=lambda k: kernels[k]["total_ms"])
    traffic = None
    tfile = os.path.join(ROOT, "profiles", "traffic.json")
    if os.path.exists(tfile):
        with open(tfile) as fh:
            traffic = json.load(fh).get(f"{dom}@N={N}")
    dom_avg_s = kernels[dom]["avg_ms"] * 1e-3
    roofline = {"kernel": dom, "bound": "mfma",
                "achieved": round(work[dom] / dom_avg_s / 1e12, 2),
                "peak": PEAK_BF16_FLOPS / 1e12, "unit": "TFLOP/s",
                "frac": round(work[dom] / dom_avg_s / PEAK_BF16_FLOPS, 4),
                "traffic": traffic,
                "algorithmic_gflop_per_launch": round(work[dom] / 1e9, 3)}

    step_flops = sum(op_flops.values())
    cpu = None
    if not args.no_cpu:
        print("[bench] CPU baseline (PyTorch fallback, fp32, host cores)", file=sys.stderr, flush=True)
        cpu = cpu_baseline(torch, mods, N)
    out = {
        "metric": METRIC,
        "value": round(step_flops / (step_ms * 1e-3) / 1e12, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded z ~ N(0,1), mask ones, random weights)",
        "config": {"workload": "pair-stack forward step: tri-mul out+in, tri-attn start+end, LayerNorm",
                   "B": 1, "N": N, "c_z": C_Z, "c_hidden_mul": C_HID, "heads": HEADS,
                   "head_dim": HEAD_DIM, "parallelism": "single GPU"},
        "ops": per_op,
        "ops_other_sizes": sizes,
        "kernels": kernels,
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out))
    return 0


if __name__ == "__main__":
    sys.exit(main())

"""Benchmark of the convolution hot path on one MI355X (BASELINE metric: conv fwd+dgrad+wgrad fp32 TFLOP/s and % of
fp32-MFMA peak; ResNet-18 b32 train ms/step).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload c5|c1] [--no-cpu] [--no-models] [--no-nhwc]

One step = forward + grad-input + grad-weight of every conv layer of the workload, over one synthetic batch already
resident in HBM:
  c5 (default): BASELINE config 5, the ResNet-50 body at batch 256, 224x224 input: 3x3 s1 p1 convs at
                (C=K=64, 56x56), (128, 28x28), (256, 14x14), (512, 7x7) and the 1x1 C->4C / 4C->C convs at the
                same sizes; x, w, gy ~ N(0,1) / sqrt(C*R*S). 1341.6 GFLOP per step.
  c1:           BASELINE config 1, AlexNet conv1 (16x3x224x224, 64x11x11, stride 4, pad 2). 6.747 GFLOP per step.
FLOPs per direction = 2*N*K*OH*OW*C*R*S (never the padded or stride-phase-expanded work).

The one JSON line also carries, as sub-objects, the same C5 sweep in channels-last layout (c5_nhwc: NHWC activations
through the channels-last kernels), config 1's sweep (alexnet_conv1_b16) and the training steps of
configs 2, 3 and 4 (plaincnn_b128, resnet18_b32, mobilenetv3_b32): device ms/step eager and replayed as a HIP graph,
the same steps on PyTorch CPU fp32 from the same weights and data, the speed-up and the 5-step loss agreement.

The roofline object reports the dominant kernel, the implicit-GEMM gather (conv_gather_kernel, its direct-to-LDS
form conv_gather_dl_kernel, or the persistent 1x1 kernels conv1x1_stream_kernel and conv1x1_wst_kernel, whichever
the tuned plan of each layer runs), from its forward launches: algorithmic FLOPs per launch over the launch's HIP-event duration, measured on the
launch stream inside the timed steps. cpu_baseline is the reference's CPU path, PyTorch CPU fp32 convolutions (the
reference runs and checks these ops on PyTorch's CPU kernels), timed on a bounded sample of the same workload with
every host core and, as the reference's README states its CPU numbers, with 4 threads; oracle_cpu_baseline times
this repository's float64 CPU oracle (oracle/) on a smaller sample. Both are baselines, not targets.
miopen_same_sweep times the same sweep through torch's own convolutions on the same GPU (MIOpen), the convolution a
PyTorch-ROCm user gets without this library (--no-miopen skips it).
"""

import argparse
import contextlib
import json
import os
import pathlib
import platform
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
for _p in (str(ROOT), str(ROOT / "omarchy-mac-torch_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

PEAK_FP32_MFMA = 157.3e12  # MI355X dense fp32 matrix peak, FLOP/s
PEAK_HBM = 8.0e12          # bytes/s

C5_LAYERS = [
    # name, n, c, k, h, ks, stride, pad
    ("3x3_56", 256, 64, 64, 56, 3, 1, 1), ("3x3_28", 256, 128, 128, 28, 3, 1, 1),
    ("3x3_14", 256, 256, 256, 14, 3, 1, 1), ("3x3_7", 256, 512, 512, 7, 3, 1, 1),
    ("1x1_exp_56", 256, 64, 256, 56, 1, 1, 0), ("1x1_red_56", 256, 256, 64, 56, 1, 1, 0),
    ("1x1_exp_28", 256, 128, 512, 28, 1, 1, 0), ("1x1_red_28", 256, 512, 128, 28, 1, 1, 0),
    ("1x1_exp_14", 256, 256, 1024, 14, 1, 1, 0), ("1x1_red_14", 256, 1024, 256, 14, 1, 1, 0),
    ("1x1_exp_7", 256, 512, 2048, 7, 1, 1, 0), ("1x1_red_7", 256, 2048, 512, 7, 1, 1, 0),
]
C1_LAYERS = [("alexnet_conv1", 16, 3, 64, 224, 11, 4, 2)]
# ResNet-18 at batch 32 on 64x64 inputs (config 3): name, n, c, k, h, ks, stride, pad, uses per training step
RESNET18_LAYERS = [
    ("stem_7x7s2", 32, 3, 64, 64, 7, 2, 3, 1), ("l1_3x3", 32, 64, 64, 16, 3, 1, 1, 4),
    ("l2_3x3s2", 32, 64, 128, 16, 3, 2, 1, 1), ("l2_1x1s2", 32, 64, 128, 16, 1, 2, 0, 1),
    ("l2_3x3", 32, 128, 128, 8, 3, 1, 1, 3), ("l3_3x3s2", 32, 128, 256, 8, 3, 2, 1, 1),
    ("l3_1x1s2", 32, 128, 256, 8, 1, 2, 0, 1), ("l3_3x3", 32, 256, 256, 4, 3, 1, 1, 3),
    ("l4_3x3s2", 32, 256, 512, 4, 3, 2, 1, 1), ("l4_1x1s2", 32, 256, 512, 4, 1, 2, 0, 1),
    ("l4_3x3", 32, 512, 512, 2, 3, 1, 1, 3),
]


def out_size(h, ks, s, p):
    return (h + 2 * p - ks) // s + 1


def flops_dir(n, c, k, h, ks, s, p):
    o = out_size(h, ks, s, p)
    return 2.0 * n * k * o * o * c * ks * ks


def cpu_info():
    model = platform.processor() or ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return model


def oracle_baseline(layers, budget_s=8.0):
    """The CPU oracle on a bounded sample: each layer at batch 1, fwd+dgrad+wgrad, repeated until ~budget_s."""
    import numpy as np

    from oracle import oracle as orc

    rng = np.random.default_rng(0)
    flops = secs = 0.0
    t_start = time.time()
    done = 0
    while time.time() - t_start < budget_s:
        for (name, n, c, k, h, ks, s, p) in layers:
            scale = (c * ks * ks) ** -0.5
            x = rng.standard_normal((1, c, h, h)).astype(np.float32)
            w = (rng.standard_normal((k, c, ks, ks)) * scale).astype(np.float32)
            t0 = time.time()
            y = orc.conv_fwd(x, w, None, s, p)
            gy = (rng.standard_normal(y.shape) * scale).astype(np.float32)
            orc.conv_dgrad(gy, w, x.shape, s, p)
            orc.conv_wgrad(x, gy, ks, s, p)
            secs += time.time() - t0
            flops += 3 * flops_dir(1, c, k, h, ks, s, p)
            done += 1
            if time.time() - t_start > budget_s:
                break
    threads = int(os.environ.get("OMP_NUM_THREADS", str(len(os.sched_getaffinity(0)))))
    return {"value": flops / secs / 1e12, "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": f"{done} layer passes (fwd+dgrad+wgrad) of the workload's layers at batch 1, "
                      f"{flops / 1e9:.1f} GFLOP in {secs:.1f} s, float64 OpenMP oracle, {cpu_info()}"}


def torch_cpu_sweep(layers, batch, threads, secs_per_layer):
    """PyTorch CPU fp32 conv2d + convolution_backward (grad input and grad weight) over the layers at `batch`, each
    layer repeated for about secs_per_layer after one untimed pass. Returns (TFLOP/s, GFLOP timed, seconds)."""
    import torch

    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(0)
    flops = secs = 0.0
    try:
        for (name, n, c, k, h, ks, s, p) in layers:
            b = min(batch, n)
            scale = (c * ks * ks) ** -0.5
            x = torch.randn((b, c, h, h), generator=g)
            w = torch.randn((k, c, ks, ks), generator=g) * scale
            o = out_size(h, ks, s, p)
            gy = torch.randn((b, k, o, o), generator=g) * scale

            def step():
                torch.nn.functional.conv2d(x, w, None, s, p)
                torch.ops.aten.convolution_backward(gy, x, w, None, [s, s], [p, p], [1, 1], False, [0, 0], 1,
                                                    [True, True, False])

            step()
            reps = 0
            t0 = time.perf_counter()
            while reps < 2 or time.perf_counter() - t0 < secs_per_layer:
                step()
                reps += 1
            secs += time.perf_counter() - t0
            flops += reps * 3 * flops_dir(b, c, k, h, ks, s, p)
    finally:
        torch.set_num_threads(prev)
    return flops / secs / 1e12, flops / 1e9, secs


def torch_cpu_baseline(layers, batch, secs_per_layer=0.8):
    """cpu_baseline: the reference's CPU path (PyTorch CPU fp32 convolutions) on a bounded sample of the workload, with
    every host core (len(sched_getaffinity)) and with 4 threads (the reference's README convention)."""
    import torch

    threads = len(os.sched_getaffinity(0))
    value, gf, secs = torch_cpu_sweep(layers, batch, threads, secs_per_layer)
    v4, gf4, secs4 = torch_cpu_sweep(layers, batch, 4, secs_per_layer)
    return {"value": round(value, 4), "unit": "TFLOP/s", "cores": threads, "kind": "reference",
            "sample": f"PyTorch {torch.__version__} CPU fp32 conv2d + convolution_backward (grad input, grad weight), "
                      f"every layer of the workload at batch {batch}, {gf:.0f} GFLOP in {secs:.1f} s; {cpu_info()}",
            "at_4_threads": {"value": round(v4, 4), "unit": "TFLOP/s", "cores": 4,
                             "sample": f"the same at 4 threads, {gf4:.0f} GFLOP in {secs4:.1f} s"}}


GATHER_KERNELS = ("conv_gather_kernel", "conv_gather_dl_kernel", "conv1x1_stream_kernel", "conv1x1_wst_kernel")


def _is_gather(kernel_name):
    """The implicit-GEMM gather kernels: staged conv_gather_kernel, direct-to-LDS conv_gather_dl_kernel and the
    persistent 1x1 conv1x1_stream_kernel and conv1x1_wst_kernel."""
    return any(k in kernel_name for k in GATHER_KERNELS)


def trace_summary(trace_csv, steps, n_layers):
    """Reads the kernel_trace.csv of a `rocprofv3 --kernel-trace` run of this bench (sweep only) and prints the
    timed region's per-kernel table as markdown. Warm-up and timed steps launch the same dispatch sequence, so the
    timed region is the latest stretch of `steps` x D dispatches that repeats with period D (the step length).
    Each layer launches its forward, then its grad input through a gather kernel (the grad weight through the wgrad
    kernel), so the even-numbered gather dispatches of the region are the forward launches: their mean duration is
    the figure the bench's roofline.avg_launch_ms measures with HIP events."""
    import csv

    rows = sorted((int(r["Dispatch_Id"]), r["Kernel_Name"], int(r["Start_Timestamp"]), int(r["End_Timestamp"]))
                  for r in csv.DictReader(open(trace_csv)))
    names = [r[1] for r in rows]
    # the latest stretch that repeats one period `steps` times (the parity check after the timed steps launches
    # other dispatches, so the timed region need not be the trace's tail)
    n, gat = len(names), [0]
    for nm in names:
        gat.append(gat[-1] + _is_gather(nm))
    found = None  # (end, period) with the latest end, then the shortest period
    for d in range(2 * n_layers, min(n // steps, 40 * n_layers) + 1):
        run = 0  # consecutive positions i with names[i] == names[i - d], ending at i
        for i in range(n):
            run = run + 1 if i >= d and names[i] == names[i - d] else 0
            end = i + 1
            if run >= (steps - 1) * d and gat[end] - gat[end - d] == 2 * n_layers and \
                    (found is None or end > found[0]):
                found = (end, d)
    if found is None:
        raise SystemExit(f"no {steps}-fold periodic stretch with {2 * n_layers} gather dispatches per step")
    end, period = found
    region = rows[end - steps * period:end]
    busy = sum(e - s for (_, _, s, e) in region) / 1e6
    span = (region[-1][3] - region[0][2]) / 1e6
    per = {}
    for (_, n, s, e) in region:
        per.setdefault(n, []).append((e - s) / 1e6)

    def short(n):
        n = n.split("(")[0].strip()
        return n[5:] if n.startswith("void ") else n

    print(f"timed region: {len(region)} dispatches ({period} per step), {busy:.3f} ms of kernel time, "
          f"span {span:.3f} ms\n")
    print("| Kernel (timed region) | Calls | Average ms | % of kernel time |\n|---|---|---|---|")
    for n, v in sorted(per.items(), key=lambda kv: -sum(kv[1])):
        print(f"| `{short(n)}` | {len(v)} | {sum(v) / len(v):.4f} | {100 * sum(v) / busy:.1f} |")
    gathers = [r for r in region if _is_gather(r[1])]
    fwd = [(e - s) / 1e6 for (_, _, s, e) in gathers[0::2]]
    kinds = {}
    for (_, n, _, _) in gathers[0::2]:
        kinds[short(n).split("<")[0]] = kinds.get(short(n).split("<")[0], 0) + 1
    print(f"\nforward launches: {len(fwd)} ({', '.join(f'{k} x{v}' for k, v in sorted(kinds.items()))}), "
          f"average {sum(fwd) / len(fwd):.4f} ms")


def kernel_table(trace_csv, prefix="omt::"):
    """Per-kernel launch count, mean and median duration (us) of the kernels whose names contain `prefix`, from the
    kernel_trace.csv of a rocprofv3 --kernel-trace run, as markdown (largest total time first)."""
    import csv

    per = {}
    for r in csv.DictReader(open(trace_csv)):
        if prefix not in r["Kernel_Name"]:
            continue
        n = r["Kernel_Name"].split("(")[0].strip()
        n = n[5:] if n.startswith("void ") else n
        per.setdefault(n, []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    print("| Kernel | Launches | Mean us | Median us |\n|---|---|---|---|")
    for n, v in sorted(per.items(), key=lambda kv: -sum(kv[1])):
        m = sorted(v)[len(v) // 2]
        print(f"| `{n}` | {len(v)} | {sum(v) / len(v):.2f} | {m:.2f} |")


RESNET_FAMILIES = [
    # (family, substrings of the kernel name), first match wins
    ("omt conv_bwd_dual_kernel (grad input + grad weight, one launch)", ("conv_bwd_dual_kernel",)),
    ("omt gather (forward; grad input alone)", GATHER_KERNELS),
    ("omt conv_wgrad_kernel (grad weight alone)", ("conv_wgrad_kernel", "conv_wgrad_nhwc_kernel")),
    ("omt split-K sums (gather_reduce, split_reduce, dual_reduce)", ("gather_reduce", "split_reduce", "dual_reduce")),
    ("omt filter re-pack", ("pack_tapmajor", "pack_dgrad")),
    ("omt BatchNorm", ("omt::bn_",)),
    ("omt depthwise convolution", ("omt::dw_",)),
    ("omt squeeze-excite MLP, gate and plane sums", ("omt::se_", "plane_dot", "channel_scale")),
    ("omt pools", ("maxpool", "avgpool", "adapool", "gap_")),
    ("omt fused Adam / SGD (multi-tensor)", ("fused_adam_kernel", "fused_sgd_kernel")),
    ("omt log-softmax / NLL loss", ("log_softmax_", "nll_fwd_kernel", "nll_bwd_kernel")),
    ("omt pointwise, plane sums, bias gradient, step counts and batch counters",
     ("pointwise_kernel", "plane_s", "foreach_add_kernel", "zero_fill_kernel", "bias_grad_kernel", "bias_grad_cols")),
    ("torch fused Adam", ("FusedAdam",)),
    ("torch foreach / elementwise (counters, ReLU, add)", ("BinaryOpScalarFunctor", "foreach", "elementwise")),
    ("hipBLASLt / rocBLAS GEMM (linear layer)", ("Cijk", "hipblaslt", "rocblas")),
    ("torch softmax / nll / reductions", ("softmax", "nll", "reduce_kernel")),
    ("runtime copies / fills", ("fill", "copy", "Copy")),
]


def resnet_trace_summary(trace_csv, replays=22, channels_last=True):
    """Reads the kernel_trace.csv of a `rocprofv3 --kernel-trace` run of `bench.py --workload resnet` (or, with
    channels_last False, `--workload mobilenet`, which has no channels-last run) and prints, for the channels-last
    compiled graphed replays (ResNet-18's last run), the compiled graphed replays (the last run of `replays`
    identical steps before it), the eager-model graphed replays (the run before that) and the compiled model with
    the backend's own graph replay (the run before that: its 20 timed steps), kernel time per step by family as
    markdown. Replays of one graph launch the same dispatch sequence, so a
    run is the latest stretch of the trace that repeats with some period D `replays` times (20 for the third); any D
    consecutive dispatches of it are one step's launches."""
    import csv

    rows = sorted((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r["Kernel_Name"])
                  for r in csv.DictReader(open(trace_csv)))
    names = [r[2] for r in rows]

    def periodic_run(end_max, end_min, replays):
        for end in range(end_max, end_min, -1):
            for d in range(50, 1000):
                st = end - replays * d
                if st < 0:
                    break
                if names[end - 1] != names[end - 1 - d]:
                    continue
                if all(names[i] == names[i - d] for i in range(st + d, end)):
                    return st, d
        return None

    runs = []
    hi = len(names)
    for reps in ((replays,) if channels_last else ()) + (replays, replays, 20):
        found = periodic_run(hi, max(0, hi - 20000), reps)
        if not found:
            break
        st, d = found
        runs.append((reps, rows[st:st + reps * d]))
        hi = st
    titles = (("channels_last compiled model, whole step captured by the caller and replayed",) if channels_last
              else ()) + ("compiled model, whole step captured by the caller (graphs.Graph) and replayed",
              "eager model, whole step captured by the caller and replayed",
              "compiled model alone: the backend replays its forward and backward graphs, the rest runs eagerly")
    for title, (replays, run) in zip(titles, runs):
        d = len(run) // replays
        per, cnt = {}, {}
        for (t0, t1, name) in run:
            fam = next((f for f, keys in RESNET_FAMILIES if any(k in name for k in keys)), "other")
            per[fam] = per.get(fam, 0) + (t1 - t0) / 1e3
            cnt[fam] = cnt.get(fam, 0) + 1
        busy = sum(per.values()) / replays
        print(f"## {title}: {replays} steps, {d} dispatches/step, kernel time {busy:.0f} us/step")
        print("| Family | Launches / step | us / step | share |\n|---|---|---|---|")
        for fam, us in sorted(per.items(), key=lambda kv: -kv[1]):
            print(f"| {fam} | {cnt[fam] // replays} | {us / replays:.0f} | {100 * us / replays / busy:.1f}% |")
        print()


def resnet_layer_trace(trace_csv, reps=100):
    """Reads the kernel_trace.csv of a rocprofv3 --kernel-trace run of `bench.py --workload resnet-layers --no-tune`
    (plans from the tuning file of an earlier run, so the trace holds the timed calls alone) and prints ResNet-18's
    convolution launches layer by layer as markdown: for each layer and direction, every kernel of one call with its
    workgroups and median duration, the call's total and its TFLOP/s. Each op of the table runs its kernel sequence
    121 times in a row (one eager call, then 121 replayed calls of a 20-call graph: 1 warm + 5 timed replays), so the
    trace is 22 periodic runs in the table's order; durations are medians over the last `reps` calls."""
    import csv
    import statistics

    rows = []
    for r in csv.DictReader(open(trace_csv)):
        wg = 1
        for d in "XYZ":
            wg *= max(1, int(r[f"Grid_Size_{d}"]) // max(1, int(r[f"Workgroup_Size_{d}"])))
        rows.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r["Kernel_Name"], wg))
    rows.sort()
    names = [r[2] for r in rows]
    ops, i = [], 0
    while i < len(rows) and len(ops) < 2 * len(RESNET18_LAYERS):
        found = None
        for d in range(1, 9):
            end = i + d * reps
            if end <= len(names) and all(names[j] == names[j - d] for j in range(i + d, end)):
                found = d
                break
        if found is None:
            i += 1
            continue
        d, end = found, i + found * reps
        while end + d <= len(names) and names[end:end + d] == names[end - d:end]:
            end += d
        ops.append(rows[end - reps * d:end])
        i = end
    print("| Layer | Direction | Kernel | Workgroups | us (median) |\n|---|---|---|---|---|")
    total = {"fwd": 0.0, "bwd": 0.0}
    for k, run in enumerate(ops):
        name, n, c, kk, h, ks, s, p, uses = RESNET18_LAYERS[k // 2]
        direction = "fwd" if k % 2 == 0 else ("wgrad" if name.startswith("stem") else "bwd (dgrad + wgrad)")
        d = len(run) // reps
        call_us = 0.0
        for pos in range(d):
            us = statistics.median((run[j * d + pos][1] - run[j * d + pos][0]) / 1e3 for j in range(reps))
            call_us += us
            kname = run[pos][2].split("(")[0].replace("void ", "")
            print(f"| {name if pos == 0 else ''} | {direction if pos == 0 else ''} | `{kname}` | {run[pos][3]} | "
                  f"{us:.1f} |")
        f = flops_dir(n, c, kk, h, ks, s, p) * (1 if k % 2 == 0 or name.startswith("stem") else 2)
        total["fwd" if k % 2 == 0 else "bwd"] += uses * call_us
        print(f"| | | **call: {call_us:.1f} us, {f / call_us / 1e6:.1f} TFLOP/s, used {uses}x per step** | | |")
    print(f"\nper step (each layer times its uses): forward {total['fwd']:.0f} us, backward {total['bwd']:.0f} us")


def pmc_summary(fetch_csv, write_csv, layers, workload):
    """Reads the FETCH_SIZE and WRITE_SIZE counter dumps of two `--pmc-probe` runs: the 1 GiB device copy calibrates
    each counter (bytes it must move / what the counter reports), then the forward gather-kernel dispatches after
    it are the workload's layers in order. Writes profiles/conv_gather_<workload>_traffic.json and prints a markdown
    table."""
    import csv

    def rows(path, counter):
        out = []
        for r in csv.DictReader(open(path)):
            if r["Counter_Name"] == counter:
                out.append((int(r["Dispatch_Id"]), r["Kernel_Name"], float(r["Counter_Value"]) * 1024.0))
        return sorted(out)

    res = {}
    for counter, path in (("FETCH_SIZE", fetch_csv), ("WRITE_SIZE", write_csv)):
        rs = rows(path, counter)
        ci = max((i for i, r in enumerate(rs) if "copy" in r[1].lower()), key=lambda i: rs[i][2])
        factor = (1 << 30) / rs[ci][2]
        gathers = [r for r in rs[ci + 1:] if _is_gather(r[1])]
        if len(gathers) != len(layers):
            raise SystemExit(f"{counter}: {len(gathers)} gather dispatches after the copy, {len(layers)} layers")
        res[counter] = (factor, [g[2] * factor for g in gathers])
    out = {"workload": workload, "fetch_factor": round(res["FETCH_SIZE"][0], 4),
           "write_factor": round(res["WRITE_SIZE"][0], 4), "layers": {}}
    lines = ["| Layer | algorithmic bytes | FETCH (scaled) | WRITE (scaled) | traffic / algorithmic |", "|---|---|---|---|---|"]
    for i, (name, n, c, k, h, ks, st, pd) in enumerate(layers):
        o = out_size(h, ks, st, pd)
        alg = 4 * (n * c * h * h + k * c * ks * ks + n * k * o * o)
        f, w = res["FETCH_SIZE"][1][i], res["WRITE_SIZE"][1][i]
        out["layers"][name] = {"algorithmic_bytes": alg, "fetch_bytes": round(f), "write_bytes": round(w)}
        lines.append(f"| {name} | {alg / 1e6:.1f} MB | {f / 1e6:.1f} MB | {w / 1e6:.1f} MB | {(f + w) / alg:.2f} |")
    (ROOT / "profiles" / f"conv_gather_{workload}_traffic.json").write_text(json.dumps(out, indent=1) + "\n")
    print(f"FETCH_SIZE factor {out['fetch_factor']}, WRITE_SIZE factor {out['write_factor']}")
    print("\n".join(lines))


def traffic_per_launch(workload):
    """HBM bytes per forward launch (mean over the workload's layers) from the committed FETCH_SIZE / WRITE_SIZE
    counter passes (profiles/conv_gather_<workload>_traffic.json, written from `bench.py --pmc-probe` runs and
    scaled by the copy-kernel calibration), or None when no such measurement exists."""
    path = ROOT / "profiles" / f"conv_gather_{workload}_traffic.json"
    try:
        data = json.loads(path.read_text())
        per = [v["fetch_bytes"] + v["write_bytes"] for v in data["layers"].values()]
        return {"bytes": round(sum(per) / len(per)), "algorithmic_bytes": round(
            sum(v["algorithmic_bytes"] for v in data["layers"].values()) / len(per)), "source": str(path.name)}
    except (OSError, ValueError, KeyError, ZeroDivisionError):
        return None


def miopen_sweep(layers, dev, reps):
    """The same sweep through stock PyTorch-ROCm convolutions (MIOpen, its default find mode; fp32): the convolution
    a user of this GPU gets without this library. TFLOP/s per direction and over the sweep, each direction's time the
    mean of `reps` calls after one untimed call (which includes MIOpen's own kernel search)."""
    import torch

    gen = torch.Generator(device=dev).manual_seed(1)
    tot, fl_tot, layer = {"fwd": 0.0, "dgrad": 0.0, "wgrad": 0.0}, 0, {}

    def timed(fn):
        fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps

    for (name, n, c, k, h, ks, s, p) in layers:
        o = out_size(h, ks, s, p)
        x = torch.randn((n, c, h, h), device=dev, generator=gen)
        w = torch.randn((k, c, ks, ks), device=dev, generator=gen) * (c * ks * ks) ** -0.5
        gy = torch.randn((n, k, o, o), device=dev, generator=gen)
        fl = flops_dir(n, c, k, h, ks, s, p)

        def bwd(mask):
            return lambda: torch.ops.aten.convolution_backward(gy, x, w, None, [s, s], [p, p], [1, 1], False, [0, 0],
                                                              1, mask)
        ms = {"fwd": timed(lambda: torch.nn.functional.conv2d(x, w, None, s, p)),
              "dgrad": timed(bwd([True, False, False])), "wgrad": timed(bwd([False, True, False]))}
        for d in ms:
            tot[d] += ms[d]
        fl_tot += fl
        layer[name] = {d: round(fl / ms[d] / 1e9, 1) for d in ms}
        print(f"miopen {name}: {layer[name]}", file=sys.stderr, flush=True)
    return {"value": round(3 * fl_tot / sum(tot.values()) / 1e9, 3), "unit": "TFLOP/s",
            "per_direction": {d: round(fl_tot / tot[d] / 1e9, 2) for d in tot}, "per_layer_tflops": layer,
            "library": f"torch {torch.__version__} conv2d / convolution_backward (MIOpen, default find mode)"}


def bandwidth_cases(dev):
    """(name, fn, algorithmic bytes) of the HBM-bound ops measured by bandwidth_kernels and bw_pmc_probe: shapes from
    the BASELINE configs; bytes are compulsory traffic -- each input read once, each output written once, fp32, int64
    pool indices."""
    import torch

    from omarchy_mac_torch import hip_ops as H

    gen = torch.Generator(device=dev).manual_seed(0)

    def rnd(*shape):
        return torch.randn(shape, device=dev, generator=gen)

    def nbytes(*ts):
        return sum(t.numel() * t.element_size() for t in ts)

    cases = []
    # depthwise (config 4, MobileNetV3-Small-style, b32): 3x3 at 72 x 56^2 and 5x5 at 96 x 28^2, stride 1 "same"
    for (n, c, h, ks) in ((32, 72, 56, 3), (32, 96, 28, 5)):
        x, w = rnd(n, c, h, h), rnd(c, 1, ks, ks)
        y = H.depthwise_conv2d(x, w, None, 1, ks // 2)
        gy = rnd(*y.shape)
        gx = H.depthwise_dgrad(gy, w, x.shape, 1, ks // 2)
        gw = H.depthwise_wgrad(x, gy, ks, 1, ks // 2)
        tag = f"dw{ks}x{ks} [{n},{c},{h},{h}]"
        cases += [(f"{tag} fwd", lambda x=x, w=w, ks=ks: H.depthwise_conv2d(x, w, None, 1, ks // 2), nbytes(x, w, y)),
                  (f"{tag} dgrad", lambda gy=gy, w=w, x=x, ks=ks: H.depthwise_dgrad(gy, w, x.shape, 1, ks // 2),
                   nbytes(gy, w, gx)),
                  (f"{tag} wgrad", lambda x=x, gy=gy, ks=ks: H.depthwise_wgrad(x, gy, ks, 1, ks // 2),
                   nbytes(x, gy, gw))]
    # BatchNorm(+ReLU) train forward / backward: config 2's largest [128,32,32^2] and ResNet-50's [256,64,56^2]
    for (n, c, h) in ((128, 32, 32), (256, 64, 56)):
        x, gam, bet, rm, rv = rnd(n, c, h, h), rnd(c), rnd(c), rnd(c), rnd(c).abs() + 0.5
        y, sm, si = H.batch_norm_train(x, gam, bet, rm, rv, relu=True)
        g = rnd(n, c, h, h)
        tag = f"bn+relu [{n},{c},{h},{h}]"
        cases += [(f"{tag} train fwd", lambda x=x, gam=gam, bet=bet, rm=rm, rv=rv: H.batch_norm_train(
                       x, gam, bet, rm, rv, relu=True), 2 * nbytes(x)),
                  (f"{tag} bwd", lambda g=g, x=x, sm=sm, si=si, gam=gam, y=y: H.batch_norm_backward(
                       g, x, sm, si, gam, relu_y=y), 4 * nbytes(x))]
    # the same BatchNorm(+ReLU) train forward over a convolution's output with the statistics from that convolution's
    # epilogue (omt_conv_fwd_stats -> omt_bn_train_fwd_stats, as the compile backend's conv -> BN op runs it for
    # channels past 8192 elements): the finalize, then one read of the input
    for (n, c, h) in ((128, 32, 32), (256, 64, 56)):
        xc, wc = rnd(n, c, h, h), rnd(c, c, 3, 3) * (9 * c) ** -0.5
        y, st, groups = H.conv2d_stats(xc, wc, 1, 1)
        del xc
        gam, bet, rm, rv = rnd(c), rnd(c), rnd(c), rnd(c).abs() + 0.5
        cases.append((f"bn+relu [{n},{c},{h},{h}] train fwd, conv-epilogue statistics",
                      lambda y=y, st=st, groups=groups, gam=gam, bet=bet, rm=rm, rv=rv: H.batch_norm_train_stats(
                          y, st, groups, gam, bet, rm, rv, relu=True), 2 * nbytes(y)))
    # max pools: config 2's 2x2 on [128,32,32^2], config 3's stem 3x3 s2 p1 on [32,64,32^2]
    for (n, c, h, k, st, pd) in ((128, 32, 32, 2, 2, 0), (32, 64, 32, 3, 2, 1)):
        x = rnd(n, c, h, h)
        y, idx = H.max_pool2d(x, k, st, pd)
        g = rnd(*y.shape)
        tag = f"maxpool{k}x{k}s{st} [{n},{c},{h},{h}]"
        cases += [(f"{tag} fwd", lambda x=x, k=k, st=st, pd=pd: H.max_pool2d(x, k, st, pd), nbytes(x, y, idx)),
                  (f"{tag} bwd", lambda g=g, x=x, idx=idx, k=k, st=st, pd=pd: H.max_pool2d_backward(
                       g, x.shape, idx, k, st, pd), nbytes(g, idx, x))]
    # global average pool (ResNet-50 head, b256)
    x = rnd(256, 2048, 7, 7)
    cases.append(("gap [256,2048,7,7] fwd", lambda x=x: H.adaptive_avg_pool2d(x, 1), nbytes(x) + 256 * 2048 * 4))
    # fused Adam over ResNet-18's parameters (62 tensors, 11.7 M elements): p, g, m, v read, p, m, v written
    import omarchy_mac_torch  # noqa: F401  (registers the device and its fused optimizer ops)
    from omarchy_mac_torch import models

    params = [p.detach().to(dev) for p in models.resnet18(1000).parameters()]
    grads, ms = ([torch.randn_like(p) * 1e-2 for p in params] for _ in range(2))
    vs = [torch.rand_like(p) * 1e-4 for p in params]
    steps = [torch.ones((), device=dev) for _ in params]
    numel = sum(p.numel() for p in params)
    cases.append((f"fused adam [{len(params)} tensors, {numel / 1e6:.1f}M]",
                  lambda: H.fused_adam(params, grads, ms, vs, steps), 7 * 4 * numel))
    # the floor of the method: a one-element fill kernel timed the same way (kernel boundary, ramp and drain)
    one = torch.empty(1, device=dev)
    cases.append(("launch floor (one-element fill)", lambda: H.fill_(one, 1.0), 4))
    return cases


def bandwidth_kernels(dev, reps=20):
    """The HBM-bound kernels of the path (bandwidth_cases): achieved GB/s from algorithmic bytes over the op's GPU time
    (all of its launches: BN's statistics, finalize and apply passes). The calls are captured into a HIP graph and
    timed with HIP events around its replays, so host dispatch (which exceeds the smallest kernels' run time) is not
    counted."""
    import torch

    cases = bandwidth_cases(dev)
    stream = torch.cuda.current_stream(dev)
    out = []
    for name, fn, b in cases:
        side = torch.cuda.Stream(dev)
        side.wait_stream(stream)
        with torch.cuda.stream(side):
            fn()
        stream.wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(reps):
                fn()
        graph.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(3):
            graph.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) / (3 * reps) * 1e3
        del graph
        out.append({"op": name, "bytes": b, "us": round(us, 2), "GB/s": round(b / us / 1e3, 1),
                    "frac_of_hbm_peak": round(b / (us * 1e-6) / PEAK_HBM, 3)})
    return out


def bw_pmc_probe(dev):
    """For rocprofv3 --pmc passes over the HBM-bound ops: a 1 GiB device-to-device copy (the FETCH_SIZE / WRITE_SIZE
    calibration), then each op of bandwidth_cases once, each preceded by a one-element fill (torch's fill kernel: the
    marker that separates the ops' dispatches in the counter dump)."""
    import torch

    cases = bandwidth_cases(dev)
    src = torch.ones(256 * 1024 * 1024, device=dev)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    mark = torch.empty(1, device=dev)
    for name, fn, _ in cases:
        mark.fill_(1.0)
        fn()
        torch.cuda.synchronize()
    print("bw pmc probe done:", len(cases), "ops", flush=True)


def bw_pmc_summary(fetch_csv, write_csv):
    """Reads the FETCH_SIZE and WRITE_SIZE dumps of two `--workload bw --pmc-probe` runs: the copy calibrates each
    counter; the dispatches between consecutive fill markers are one op's (all of its kernels). Writes
    profiles/hbm_kernels_traffic.json and prints a markdown table of HBM bytes against the algorithmic bytes."""
    import csv

    import torch

    names = [(c[0], c[2]) for c in bandwidth_cases(torch.device("cuda:0"))] if torch.cuda.is_available() else None
    res = {}
    for counter, path in (("FETCH_SIZE", fetch_csv), ("WRITE_SIZE", write_csv)):
        rs = sorted((int(r["Dispatch_Id"]), r["Kernel_Name"], float(r["Counter_Value"]) * 1024.0)
                    for r in csv.DictReader(open(path)) if r["Counter_Name"] == counter)
        ci = max((i for i, r in enumerate(rs) if "copy" in r[1].lower()), key=lambda i: rs[i][2])
        factor = (1 << 30) / rs[ci][2]
        ops, cur = [], None
        for _, kname, v in rs[ci + 1:]:
            if "FillFunctor" in kname:
                cur = {"bytes": 0.0, "kernels": []}
                ops.append(cur)
            elif cur is not None:
                cur["bytes"] += v * factor
                short = kname.split("(")[0].replace("void ", "")
                if short not in cur["kernels"]:
                    cur["kernels"].append(short)
        res[counter] = (factor, ops)
    n_ops = len(res["FETCH_SIZE"][1])
    if names is None or len(names) != n_ops or len(res["WRITE_SIZE"][1]) != n_ops:
        raise SystemExit(f"{n_ops} ops in the dump; expected {len(names) if names else '?'} (run on the GPU box)")
    out = {"fetch_factor": round(res["FETCH_SIZE"][0], 4), "write_factor": round(res["WRITE_SIZE"][0], 4), "ops": {}}
    lines = ["| Op | kernels | algorithmic | FETCH (scaled) | WRITE (scaled) | traffic / algorithmic |",
             "|---|---|---|---|---|---|"]
    for i, (name, alg) in enumerate(names):
        f, w = res["FETCH_SIZE"][1][i], res["WRITE_SIZE"][1][i]
        out["ops"][name] = {"algorithmic_bytes": alg, "fetch_bytes": round(f["bytes"]), "write_bytes": round(w["bytes"]),
                            "kernels": f["kernels"]}
        lines.append(f"| {name} | {', '.join('`' + k + '`' for k in f['kernels'])} | {alg / 1e6:.1f} MB | "
                     f"{f['bytes'] / 1e6:.1f} MB | {w['bytes'] / 1e6:.1f} MB | {(f['bytes'] + w['bytes']) / alg:.2f} |")
    (ROOT / "profiles" / "hbm_kernels_traffic.json").write_text(json.dumps(out, indent=1) + "\n")
    print(f"FETCH_SIZE factor {out['fetch_factor']}, WRITE_SIZE factor {out['write_factor']}")
    print("\n".join(lines))


def pmc_probe(layers, dev, plans_log=None):
    """For the rocprofv3 --pmc passes: the forward plans are tuned first (as in the bench; those dispatches come
    before the copy) or, with plans_log, set to the forward plans of the bench run whose JSON line that file holds
    (so that the traffic is measured on the plans that run timed), then a 1 GiB device-to-device copy (1 GiB read +
    1 GiB written: the FETCH_SIZE / WRITE_SIZE calibration launch), then one forward conv per layer, each on its own
    freshly written input."""
    import torch

    from omarchy_mac_torch import hip_ops

    fixed = None
    if plans_log:
        line = [ln for ln in open(plans_log) if ln.startswith('{"metric"')][-1]
        fixed = json.loads(line)["plans"]["tile_slices"]
    for (name, n, c, k, h, ks, s, p) in layers:
        if fixed:
            hip_ops.set_conv_plan("fwd", (n, c, h, h), (k, c, ks, ks), s, p, *fixed[name]["fwd"])
        else:
            hip_ops.autotune_conv("fwd", (n, c, h, h), (k, c, ks, ks), s, p)
        print(name, "fwd plan", hip_ops.conv_plan("fwd", (n, c, h, h), (k, c, ks, ks), s, p)[:2], flush=True)
    torch.cuda.synchronize()
    src = torch.ones(256 * 1024 * 1024, device=dev)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    for (name, n, c, k, h, ks, s, p) in layers:
        x = torch.randn((n, c, h, h), device=dev)
        w = torch.randn((k, c, ks, ks), device=dev) * (c * ks * ks) ** -0.5
        hip_ops.conv2d(x, w, None, s, p)
        torch.cuda.synchronize()
    print("pmc probe done", flush=True)


def train_configs():
    """(key, description, model factory, batch, input shape, classes, optimizer factory). The
    optimizer factory takes capturable=... (a graph-replayed step needs the device-side step counts of Adam / AdamW;
    SGD keeps no step count)."""
    import torch

    from omarchy_mac_torch import models

    def sgd(p, capturable=False):
        return torch.optim.SGD(p, lr=0.01, momentum=0.9)

    def adam(p, capturable=False):
        return torch.optim.Adam(p, lr=1e-3, capturable=capturable)

    def adamw(p, capturable=False):
        return torch.optim.AdamW(p, lr=1e-3, weight_decay=0.01, capturable=capturable)

    return [
        ("plaincnn_b128", "PlainCNN b128 3x32x32: 4 x (conv3x3 + BN + ReLU + maxpool2x2) at 32-64-128-256, GAP, "
                          "linear 256->10, SGD lr 0.01 momentum 0.9 (BASELINE config 2)",
         lambda: models.plain_cnn(10), 128, (3, 32, 32), 10, sgd),
        ("resnet18_b32", "ResNet-18 b32 3x64x64, 1000 classes, BN train, Adam lr 1e-3 (BASELINE config 3)",
         lambda: models.resnet18(1000), 32, (3, 64, 64), 1000, adam),
        ("mobilenetv3_b32", "MobileNetV3-Small-style b32 3x224x224: stride-1 depthwise 3x3/5x5, 1x1 expand/project, "
                            "hardswish, BN, squeeze-excite; 1000 classes, AdamW lr 1e-3 wd 0.01 (BASELINE config 4)",
         lambda: models.mobilenet_v3_small(1000), 32, (3, 224, 224), 1000, adamw),
    ]


def train_step_bench(cfg, dev_name, steps, warmup, cpu_steps, cpu, compiled=False, fp64=False):
    """One training configuration on the omarchy_mac_torch device and, from the same weights and data, on the host
    CPU: ms/step eager (enqueue time too: small steps are host-bound), replayed as a HIP graph (and, with `compiled`,
    under torch.compile(backend="omarchy_mac_torch") and replayed), PyTorch CPU fp32 with every host core (1 warm-up
    step, then the mean of `cpu_steps`, as the reference's acceptance tool times it), the speed-ups and the relative
    loss differences over the common steps (the north-star criterion: 1e-3 over 5 steps). fp64 adds a float64 CPU
    run of the same steps, the rounding-free trajectory both fp32 runs are compared with."""
    import copy

    import torch
    import torch.nn.functional as F

    key, title, make_model, batch, shape, classes, make_opt = cfg
    torch.manual_seed(0)
    base = make_model()
    g = torch.Generator().manual_seed(1)
    n_batches = max(warmup + steps, cpu_steps + 1)
    data = [(torch.randn(batch, *shape, generator=g), torch.randint(0, classes, (batch,), generator=g))
            for _ in range(n_batches)]

    def run(model, device, batches, timed_from, dtype=torch.float32, compile_it=False):
        opt = make_opt(model.parameters())
        fwd = torch.compile(model, backend=dev_name) if compile_it else model
        losses, t0 = [], None
        for i, (x, t) in enumerate(batches):
            if i == timed_from:
                if device != "cpu":
                    torch.cuda.synchronize()
                t0 = time.perf_counter()
            opt.zero_grad(set_to_none=True)
            loss = F.cross_entropy(fwd(x.to(dtype)), t)
            loss.backward()
            opt.step()
            losses.append(loss.detach())
        host_ms = (time.perf_counter() - t0) / (len(batches) - timed_from) * 1e3  # enqueue time, before the sync
        if device != "cpu":
            torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) / (len(batches) - timed_from) * 1e3
        run.host_ms = host_ms
        return ms, [float(l) for l in losses]

    def run_graphed(model, batches, timed_from, compile_it=False):
        """The same step captured once as a HIP graph (omarchy_mac_torch.graphs) after `timed_from` eager warm-up
        steps, then replayed per batch; each batch is copied into the captured input tensors first (timed). The
        compiled model's own graph replay is off here (the whole step is the graph)."""
        from omarchy_mac_torch import graphs, replay

        prev = replay.set_enabled(False)
        try:
            return _run_graphed(model, batches, timed_from, compile_it, graphs)
        finally:
            replay.set_enabled(prev)

    def _run_graphed(model, batches, timed_from, compile_it, graphs):
        opt = make_opt(model.parameters(), capturable=True)
        sx, st = torch.empty_like(batches[0][0]), torch.empty_like(batches[0][1])
        fwd = torch.compile(model, backend=dev_name) if compile_it else model

        def step():
            opt.zero_grad(set_to_none=True)
            loss = F.cross_entropy(fwd(sx), st)
            loss.backward()
            opt.step()
            return loss.detach()

        losses = []
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for x, t in batches[:timed_from]:
                sx.copy_(x)
                st.copy_(t)
                losses.append(step().clone())
        torch.cuda.current_stream().wait_stream(side)
        gr = graphs.Graph()
        with gr.capture():
            static_loss = step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for x, t in batches[timed_from:]:
            sx.copy_(x)
            st.copy_(t)
            gr.replay()
            losses.append(static_loss.clone())
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) / (len(batches) - timed_from) * 1e3
        out = [float(l) for l in losses]
        gr.release()
        return ms, out

    def rel_diff(a, b):
        return max(abs(u - v) / abs(v) for u, v in zip(a, b))

    dev_batches = [(x.to(dev_name), t.to(dev_name)) for (x, t) in data[:warmup + steps]]
    torch.cuda.synchronize()
    dev_ms, dev_losses = run(copy.deepcopy(base).to(dev_name), dev_name, dev_batches, warmup)
    out = {"config": title, "ms_per_step": round(dev_ms, 3), "host_enqueue_ms_per_step": round(run.host_ms, 3),
           "steps": steps, "warmup": warmup}
    n_ops = aten_ops_per_step(copy.deepcopy(base).to(dev_name), make_opt, dev_batches[0])
    out.update({"aten_ops_per_step": n_ops, "host_us_per_aten_op": round(run.host_ms * 1e3 / n_ops, 2)})
    variants = {}
    if compiled:
        from omarchy_mac_torch import replay

        replay.reset_stats()
        c_ms, variants["compiled"] = run(copy.deepcopy(base).to(dev_name), dev_name, dev_batches, warmup,
                                         compile_it=True)
        out["compiled"] = {
            "ms_per_step": round(c_ms, 3), "host_enqueue_ms_per_step": round(run.host_ms, 3), "steps": steps,
            "warmup": warmup, "graph_replay": {k: replay.STATS[k] for k in ("captures", "replays", "eager")},
            "how": "torch.compile(model, backend=\"omarchy_mac_torch\") and nothing else: the backend's rewrites, its "
                   "forward and backward graphs replayed as HIP graphs from the third step on; loss, log-softmax, "
                   "the optimizer and zero_grad run eagerly around them"}
    g_ms, variants["graphed"] = run_graphed(copy.deepcopy(base).to(dev_name), dev_batches, 3)
    out["graphed"] = {"ms_per_step": round(g_ms, 3), "steps": len(dev_batches) - 3, "eager_warmup": 3,
                      "how": "omarchy_mac_torch.graphs.Graph: forward + backward + fused optimizer captured once, "
                             "replayed per batch after an in-place copy of the batch"}
    if compiled:
        c_ms, variants["compiled_graphed"] = run_graphed(copy.deepcopy(base).to(dev_name), dev_batches, 3, True)
        out["compiled_graphed"] = {
            "ms_per_step": round(c_ms, 3), "steps": len(dev_batches) - 3, "eager_warmup": 3,
            "how": "the graphed step with the model under torch.compile(backend=\"omarchy_mac_torch\"): BatchNorm "
                   "running statistics updated in place, BatchNorm + ReLU and BatchNorm + residual add + ReLU fused, "
                   "batch counters in one launch"}
    if compiled and key == "resnet18_b32":
        cl = torch.channels_last
        cl_batches = [(x.contiguous(memory_format=cl), t) for x, t in dev_batches]
        cl_model = copy.deepcopy(base).to(memory_format=cl).to(dev_name)
        c_ms, variants["channels_last_compiled_graphed"] = run_graphed(cl_model, cl_batches, 3, True)
        out["channels_last_compiled_graphed"] = {
            "ms_per_step": round(c_ms, 3), "steps": len(dev_batches) - 3, "eager_warmup": 3,
            "how": "the compiled + graphed step with the model and its batches in torch.channels_last memory order: "
                   "the NHWC convolution, BatchNorm and pooling kernels, no layout conversion"}
    if not cpu:
        return out
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    cpu_ms, cpu_losses = run(copy.deepcopy(base), "cpu", data[:cpu_steps + 1], 1)
    k = min(len(cpu_losses), len(dev_losses))
    f64 = None
    if fp64:
        _, f64 = run(copy.deepcopy(base).double(), "cpu", data[:k], 0, torch.float64)
    for name, ls in variants.items():
        out[name].update({"speedup_vs_cpu": round(cpu_ms / out[name]["ms_per_step"], 2),
                          "max_rel_loss_diff": rel_diff(ls[:k], cpu_losses[:k]),
                          "max_rel_loss_diff_5_steps": rel_diff(ls[:5], cpu_losses[:5]),
                          "losses": [round(v, 6) for v in ls[:k]]})
        if f64:
            out[name]["max_rel_loss_diff_vs_fp64"] = rel_diff(ls[:k], f64)
    out.update({"cpu_ms_per_step": round(cpu_ms, 2), "cpu_cores": threads, "cpu_steps": cpu_steps,
                "speedup_vs_cpu": round(cpu_ms / dev_ms, 2), "max_rel_loss_diff": rel_diff(dev_losses[:k], cpu_losses[:k]),
                "loss_steps_compared": k, "max_rel_loss_diff_5_steps": rel_diff(dev_losses[:5], cpu_losses[:5]),
                "losses": {"device": [round(v, 6) for v in dev_losses[:k]],
                           "cpu": [round(v, 6) for v in cpu_losses[:k]]},
                "cpu": f"PyTorch {torch.__version__} CPU fp32, {cpu_info()}"})
    if f64:
        out["losses"]["cpu_fp64"] = [round(v, 6) for v in f64]
        out["max_rel_loss_diff_vs_fp64"] = {"device": rel_diff(dev_losses[:k], f64),
                                            "cpu_fp32": rel_diff(cpu_losses[:k], f64)}
    return out


def aten_ops_per_step(model, make_opt, batch):
    """The aten operators one eager training step dispatches (forward, loss, backward, optimizer; views included):
    the host-side work per step that graph replay removes."""
    import torch
    import torch.nn.functional as F
    from torch.utils._python_dispatch import TorchDispatchMode

    class Count(TorchDispatchMode):
        n = 0

        def __torch_dispatch__(self, func, types, args=(), kwargs=None):
            Count.n += 1
            return func(*args, **(kwargs or {}))

    opt = make_opt(model.parameters())
    x, t = batch
    for counting in (False, True):  # the first step creates the optimizer state
        with Count() if counting else contextlib.nullcontext():
            opt.zero_grad(set_to_none=True)
            F.cross_entropy(model(x), t).backward()
            opt.step()
    torch.cuda.synchronize()
    return Count.n


def resnet_layer_table(dev, tune=True, calls=20, reps=5):
    """ResNet-18's convolutions (config 3) one by one with the plans the device tunes for them: forward (omt_conv_fwd,
    with its slice sum) and backward (omt_conv_bwd: grad input and grad weight; the stem, whose input needs no
    gradient, grad weight alone), each timed as replays of a captured HIP graph of `calls` calls (GPU time per call,
    as in a replayed training step). tune=False keeps the plans the cache holds (a tuning file of an earlier run:
    a profiled run then traces the timed calls alone). Prints a markdown table and returns it as a dict."""
    import torch

    from omarchy_mac_torch import hip_ops

    gen = torch.Generator(device=dev).manual_seed(0)
    rows, total = {}, {"fwd": 0.0, "bwd": 0.0}

    def per_call_us(fn):
        fn()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for _ in range(calls):
                fn()
        g.replay()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(reps):
            g.replay()
        b.record()
        torch.cuda.synchronize()
        us = a.elapsed_time(b) * 1e3 / (reps * calls)
        g.reset()
        return us

    print("| Layer | n x c x h^2 -> k, ks/s | uses | fwd us | fwd TFLOP/s | fwd plan | bwd us | bwd TFLOP/s | "
          "bwd plans (dgrad, wgrad) |\n|---|---|---|---|---|---|---|---|---|")
    for (name, n, c, k, h, ks, s, p, uses) in RESNET18_LAYERS:
        o = out_size(h, ks, s, p)
        x = torch.randn((n, c, h, h), device=dev, generator=gen)
        w = torch.randn((k, c, ks, ks), device=dev, generator=gen) * (c * ks * ks) ** -0.5
        gy = torch.randn((n, k, o, o), device=dev, generator=gen)
        f = flops_dir(n, c, k, h, ks, s, p)
        if tune:
            hip_ops.autotune_conv("fwd", x.shape, w.shape, s, p)
        stem = name.startswith("stem")
        if stem:
            if tune:
                hip_ops.autotune_conv("wgrad", x.shape, w.shape, s, p)
            bwd = lambda: hip_ops.conv2d_wgrad(x, gy, ks, s, p)  # noqa: E731
            bf = f
        else:
            if tune:
                hip_ops.autotune_conv_bwd(x.shape, w.shape, s, p)
            bwd = lambda: hip_ops.conv2d_bwd(x, gy, w, s, p)  # noqa: E731
            bf = 2 * f
        tf = per_call_us(lambda: hip_ops.conv2d(x, w, None, s, p))
        tb = per_call_us(bwd)
        plans = {d: hip_ops.conv_plan(d, x.shape, w.shape, s, p)[:2] for d in ("fwd", "dgrad", "wgrad")}
        rows[name] = {"uses": uses, "fwd_us": round(tf, 2), "fwd_tflops": round(f / tf / 1e6, 1), "bwd_us": round(tb, 2),
                      "bwd_tflops": round(bf / tb / 1e6, 1), "plans": plans}
        total["fwd"] += uses * tf
        total["bwd"] += uses * tb
        print(f"| {name} | {n}x{c}x{h}^2 -> {k}, {ks}/{s} | {uses} | {tf:.1f} | {f / tf / 1e6:.1f} | {plans['fwd']} | "
              f"{tb:.1f} | {bf / tb / 1e6:.1f} | {'-' if stem else plans['dgrad']}, {plans['wgrad']} |", flush=True)
    flops = sum(u * flops_dir(n, c, k, h, ks, s, p) * (2 if name.startswith("stem") else 3)
                for (name, n, c, k, h, ks, s, p, u) in RESNET18_LAYERS)
    us = total["fwd"] + total["bwd"]
    print(f"\nper training step: forward {total['fwd']:.0f} us, backward {total['bwd']:.0f} us, "
          f"{us:.0f} us for {flops / 1e9:.2f} GFLOP = {flops / us / 1e6:.1f} TFLOP/s", flush=True)
    return {"layers": rows, "step_us": {k: round(v, 1) for k, v in total.items()}, "step_gflop": round(flops / 1e9, 3)}


def conv_sweep(layers, dev, steps, warmup, tune, nhwc=False):
    """The sweep of `layers` (fwd + dgrad + wgrad each) on synthetic inputs resident in HBM: plans tuned first (as the
    reference tunes every new shape on first use, csrc/conv.cpp:56), `warmup` untimed steps, then `steps` timed ones
    with HIP events around every launch on the launch stream. nhwc: every tensor channels_last, through the
    channels-last kernels. Returns the figures the bench line reports."""
    import torch

    from omarchy_mac_torch import hip_ops

    gen = torch.Generator(device=dev).manual_seed(0)
    fmt = torch.channels_last if nhwc else torch.contiguous_format
    data = []
    for (name, n, c, k, h, ks, s, p) in layers:
        scale = (c * ks * ks) ** -0.5
        o = out_size(h, ks, s, p)
        x = (torch.randn((n, c, h, h), device=dev, generator=gen) * scale).contiguous(memory_format=fmt)
        w = (torch.randn((k, c, ks, ks), device=dev, generator=gen) * scale).contiguous(memory_format=fmt)
        gy = (torch.randn((n, k, o, o), device=dev, generator=gen) * scale).contiguous(memory_format=fmt)
        data.append((name, n, c, k, h, ks, s, p, x, w, gy))
    sfx = "_nhwc" if nhwc else ""
    fwd_op = hip_ops.conv2d_nhwc if nhwc else hip_ops.conv2d
    dgrad_op = hip_ops.conv2d_dgrad_nhwc if nhwc else hip_ops.conv2d_dgrad
    wgrad_op = hip_ops.conv2d_wgrad_nhwc if nhwc else hip_ops.conv2d_wgrad

    plans = {}
    for (name, n, c, k, h, ks, s, p, x, w, gy) in data:
        for d in ("fwd", "dgrad", "wgrad"):
            if tune:
                hip_ops.autotune_conv(d + sfx, x.shape, w.shape, s, p)
            plans.setdefault(name, {})[d] = list(hip_ops.conv_plan(d + sfx, x.shape, w.shape, s, p)[:2])
    torch.cuda.synchronize()

    stream = torch.cuda.current_stream(dev)
    fwd_events = []  # (flops, start, end) per forward launch in the timed steps
    dir_events = {"fwd": [], "dgrad": [], "wgrad": []}

    def step(timed):
        for (name, n, c, k, h, ks, s, p, x, w, gy) in data:
            f = flops_dir(n, c, k, h, ks, s, p)
            evs = [torch.cuda.Event(enable_timing=True) for _ in range(4)] if timed else None
            if timed:
                evs[0].record(stream)
            fwd_op(x, w, None, s, p)
            if timed:
                evs[1].record(stream)
            dgrad_op(gy, w, x.shape, s, p)
            if timed:
                evs[2].record(stream)
            wgrad_op(x, gy, ks, s, p)
            if timed:
                evs[3].record(stream)
                fwd_events.append((f, evs[0], evs[1]))
                dir_events["fwd"].append((name, f, evs[0], evs[1]))
                dir_events["dgrad"].append((name, f, evs[1], evs[2]))
                dir_events["wgrad"].append((name, f, evs[2], evs[3]))

    for _ in range(warmup):
        step(False)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step(True)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0

    check = verify_sweep(data, fwd_op, dgrad_op, wgrad_op)
    step_flops = sum(3 * flops_dir(n, c, k, h, ks, s, p) for (_, n, c, k, h, ks, s, p, *_r) in data)
    fwd_ms = [a.elapsed_time(b) for (_, a, b) in fwd_events]
    fwd_flops = [f for (f, _, _) in fwd_events]
    per_dir, per_layer = {}, {}
    for d, evs in dir_events.items():
        tot_f = sum(f for (_, f, _, _) in evs)
        tot_ms = sum(a.elapsed_time(b) for (_, _, a, b) in evs)
        per_dir[d] = {"tflops": round(tot_f / (tot_ms / 1e3) / 1e12, 2),
                      "frac_peak": round(tot_f / (tot_ms / 1e3) / PEAK_FP32_MFMA, 4),
                      "ms_per_step": round(tot_ms / steps, 4)}
        for (name, f, a, b) in evs:
            per_layer.setdefault(name, {}).setdefault(d, []).append(a.elapsed_time(b))
    layer_flops = {l[0]: flops_dir(*l[1:8]) for l in data}
    return {
        "value": step_flops * steps / elapsed / 1e12,
        "ms_per_step": elapsed / steps * 1e3,
        "step_flops": step_flops,
        "avg_launch_ms": sum(fwd_ms) / len(fwd_ms),
        "achieved": sum(fwd_flops) / (sum(fwd_ms) / 1e3) / 1e12,  # TFLOP/s over all forward launches
        "flop_per_launch_avg": sum(fwd_flops) / len(fwd_flops),
        "per_direction": per_dir,
        "per_layer_tflops": {name: {d: round(layer_flops[name] / (sum(v) / len(v) / 1e3) / 1e12, 1)
                                    for d, v in dd.items()} for name, dd in per_layer.items()},
        "plans": plans,
        "rel_l2_vs_torch_cpu": check,
    }


def verify_sweep(data, fwd_op, dgrad_op, wgrad_op, images=(0, -1), samples=24):
    """The outputs of the timed launches (same inputs, same plans) against PyTorch CPU in float64, per layer: y and gx
    on two images of the batch (each image's output depends on that image alone), and `samples` random entries of gw
    (each a float64 sum over the whole batch of gy[:, co] times the shifted x[:, ci]). Returns {layer: {"y", "gx", "gw":
    rel-L2}}; the bench line carries it."""
    import torch
    import torch.nn.functional as F

    out = {}
    gen = torch.Generator().manual_seed(1)
    for (name, n, c, k, h, ks, s, p, x, w, gy) in data:
        y = fwd_op(x, w, None, s, p)
        gx = dgrad_op(gy, w, x.shape, s, p)
        gw = wgrad_op(x, gy, ks, s, p)
        wc = w.double().cpu().contiguous()
        r = {}
        idx = [i % n for i in images]
        xi, gyi = x[idx].double().cpu().contiguous(), gy[idx].double().cpu().contiguous()
        ry = F.conv2d(xi, wc, None, s, p)
        r["y"] = float((y[idx].double().cpu() - ry).norm() / ry.norm())
        rgx = torch.ops.aten.convolution_backward(gyi, xi, wc, None, [s, s], [p, p], [1, 1], False, [0, 0], 1,
                                                  [True, False, False])[0]
        r["gx"] = float((gx[idx].double().cpu() - rgx).norm() / rgx.norm())
        pick = [tuple(int(torch.randint(0, m, (1,), generator=gen)) for m in (k, c, ks, ks)) for _ in range(samples)]
        got, ref = [], []
        for (co, ci, ky, kx) in pick:
            g = gy[:, co].double().cpu()
            xs = F.pad(x[:, ci].double().cpu(), (p, p, p, p))
            o = g.shape[-1]
            xs = xs[:, ky:ky + s * (o - 1) + 1:s, kx:kx + s * (o - 1) + 1:s]
            ref.append(float((g * xs).sum()))
            got.append(float(gw[co, ci, ky, kx]))
        got, ref = torch.tensor(got, dtype=torch.float64), torch.tensor(ref, dtype=torch.float64)
        r["gw"] = float((got - ref).norm() / ref.norm())
        out[name] = {key: float(f"{v:.2e}") for key, v in r.items()}
    return out


def c1_sub_object(dev, steps, warmup, cpu):
    """Config 1 (AlexNet conv1 b16, fwd + dgrad + wgrad) as a sub-object of the bench line: its sweep with tuned plans,
    parity of y, gx and gw with PyTorch CPU fp32 on the same full-size inputs (rel-L2), and PyTorch CPU at every host
    core on the same full-size layer."""
    import torch

    from omarchy_mac_torch import hip_ops

    sw = conv_sweep(C1_LAYERS, dev, steps, warmup, True)
    out = {"config": "C1 AlexNet conv1 b16 3x224x224 -> 64x55x55, 11x11 s4 p2, fwd+dgrad+wgrad (BASELINE config 1)",
           "value": round(sw["value"], 3), "unit": "TFLOP/s", "frac_of_peak": round(sw["value"] * 1e12 / PEAK_FP32_MFMA, 4),
           "ms_per_step": round(sw["ms_per_step"], 4), "per_direction": sw["per_direction"], "plans": sw["plans"]}
    g = torch.Generator().manual_seed(0)
    x = torch.randn(16, 3, 224, 224, generator=g)
    w = torch.nn.init.kaiming_normal_(torch.empty(64, 3, 11, 11), generator=g)
    b = torch.rand(64, generator=g) * 0.2 - 0.1
    gy = torch.randn(16, 64, 55, 55, generator=g)
    dx, dw_, db, dgy = (t.to(dev) for t in (x, w, b, gy))
    y = hip_ops.conv2d(dx, dw_, db, 4, 2)
    gx = hip_ops.conv2d_dgrad(dgy, dw_, x.shape, 4, 2)
    gw = hip_ops.conv2d_wgrad(dx, dgy, 11, 4, 2)
    ry = torch.nn.functional.conv2d(x, w, b, 4, 2)
    rgx, rgw, _ = torch.ops.aten.convolution_backward(gy, x, w, None, [4, 4], [2, 2], [1, 1], False, [0, 0], 1,
                                                      [True, True, False])

    def rel(a, r):
        return float((a.cpu().double() - r.double()).norm() / r.double().norm())

    out["rel_l2_vs_torch_cpu"] = {"y": rel(y, ry), "gx": rel(gx, rgx), "gw": rel(gw, rgw)}
    if cpu:
        v, gf, secs = torch_cpu_sweep(C1_LAYERS, 16, len(os.sched_getaffinity(0)), 2.0)
        out["cpu"] = {"value": round(v, 4), "unit": "TFLOP/s", "cores": len(os.sched_getaffinity(0)),
                      "sample": f"PyTorch {torch.__version__} CPU fp32, the full layer at batch 16, {gf:.0f} GFLOP in "
                                f"{secs:.1f} s; {cpu_info()}"}
        out["speedup_vs_cpu"] = round(sw["value"] / v, 1)
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--workload", choices=["c5", "c1", "resnet", "mobilenet", "resnet-layers", "models", "bw"],
                    default="c5",
                    help="resnet / mobilenet: only the ResNet-18 / MobileNetV3 training-step measurement; "
                         "resnet-layers: ResNet-18's "
                         "convolutions one by one (tuned plans, per-call GPU time); models: only the training steps "
                         "of configs 2-4; bw: only the HBM-bound kernels (all three for profiling)")
    ap.add_argument("--no-bw", action="store_true", help="skip the HBM-bound kernel measurements")
    ap.add_argument("--no-miopen", action="store_true",
                    help="skip timing the same sweep through torch's own convolutions (MIOpen)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    ap.add_argument("--no-nhwc", action="store_true", help="skip the channels-last C5 sweep")
    ap.add_argument("--no-models", "--no-resnet", dest="no_models", action="store_true",
                    help="skip config 1's sub-object and the training steps of configs 2-4")
    ap.add_argument("--model-steps", "--resnet-steps", dest="model_steps", type=int, default=20)
    ap.add_argument("--no-tune", action="store_true",
                    help="skip plan tuning (tile / K split per layer and direction) before the warmup")
    ap.add_argument("--pmc-summary", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="summarize two --pmc-probe counter dumps into profiles/conv_gather_<workload>_traffic.json")
    ap.add_argument("--trace-summary", metavar="KERNEL_TRACE_CSV",
                    help="per-kernel table of the timed steps of a rocprofv3 --kernel-trace run of the sweep "
                         "(--no-bw --no-models --no-cpu, same --steps)")
    ap.add_argument("--resnet-trace-summary", metavar="KERNEL_TRACE_CSV",
                    help="kernel time per step by family of a rocprofv3 --kernel-trace run of --workload resnet")
    ap.add_argument("--mobilenet-trace-summary", metavar="KERNEL_TRACE_CSV",
                    help="the same for a run of --workload mobilenet (no channels-last run)")
    ap.add_argument("--resnet-layer-trace", metavar="KERNEL_TRACE_CSV",
                    help="ResNet-18's convolution launches per layer (workgroups, us) from a rocprofv3 --kernel-trace "
                         "run of --workload resnet-layers --no-tune")
    ap.add_argument("--kernel-table", metavar="KERNEL_TRACE_CSV",
                    help="per-kernel launches and mean / median duration of this library's kernels in a kernel trace")
    ap.add_argument("--pmc-probe", action="store_true",
                    help="for rocprofv3 --pmc passes: one 1 GiB device copy (counter calibration), then one forward "
                         "launch per layer (with --workload bw: each HBM-bound op once, after a fill marker)")
    ap.add_argument("--pmc-plans", metavar="BENCH_LOG",
                    help="with --pmc-probe: the forward plans of the bench run whose JSON line BENCH_LOG holds, "
                         "instead of tuning them again")
    args = ap.parse_args()
    if args.pmc_summary:
        if args.workload == "bw":
            bw_pmc_summary(*args.pmc_summary)
        else:
            pmc_summary(*args.pmc_summary, C5_LAYERS if args.workload == "c5" else C1_LAYERS, args.workload)
        return
    if args.kernel_table:
        kernel_table(args.kernel_table)
        return
    if args.resnet_layer_trace:
        resnet_layer_trace(args.resnet_layer_trace)
        return
    if args.resnet_trace_summary:
        resnet_trace_summary(args.resnet_trace_summary)
        return
    if args.mobilenet_trace_summary:
        resnet_trace_summary(args.mobilenet_trace_summary, channels_last=False)
        return
    if args.trace_summary:
        trace_summary(args.trace_summary, args.steps, len(C5_LAYERS if args.workload == "c5" else C1_LAYERS))
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (each MI355X runs the same kernels on "
              "its batch share, the weight gradients summed over the GPUs afterwards). Run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)

    import torch

    dev = torch.device("cuda:0")
    if args.workload == "resnet-layers":
        print(json.dumps({"resnet18_conv_layers": resnet_layer_table(dev, not args.no_tune)}), flush=True)
        return
    if args.workload in ("resnet", "mobilenet", "models"):
        import omarchy_mac_torch

        cfgs = train_configs()
        if args.workload != "models":
            cfgs = [c for c in cfgs if c[0] == {"resnet": "resnet18_b32", "mobilenet": "mobilenetv3_b32"}[args.workload]]
        print(json.dumps({c[0]: train_step_bench(c, omarchy_mac_torch.DEVICE, args.model_steps, 5, 5, not args.no_cpu,
                                                 compiled=c[0] in ("resnet18_b32", "mobilenetv3_b32"),
                                                 fp64=c[0] == "resnet18_b32")
                          for c in cfgs}), flush=True)
        return
    if args.workload == "bw":
        if args.pmc_probe:
            bw_pmc_probe(dev)
        else:
            print(json.dumps({"bandwidth_kernels": bandwidth_kernels(dev)}), flush=True)
        return
    layers = C5_LAYERS if args.workload == "c5" else C1_LAYERS
    if args.pmc_probe:
        pmc_probe(layers, dev, args.pmc_plans)
        return
    sw = conv_sweep(layers, dev, args.steps, args.warmup, not args.no_tune)
    value = sw["value"]
    traffic = traffic_per_launch(args.workload)
    out = {
        "metric": "conv fwd+dgrad+wgrad fp32 TFLOP/s (% of fp32-MFMA peak); ResNet-18 b32 train ms/step",
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(sw["ms_per_step"], 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": ("C5 ResNet-50 body b256 224^2: 3x3 s1 convs at (64,56^2),(128,28^2),(256,14^2),"
                                "(512,7^2) + 1x1 C->4C and 4C->C at the same sizes, fwd+dgrad+wgrad"
                                if args.workload == "c5" else
                                "C1 AlexNet conv1 b16 3x224x224 -> 64x55x55, 11x11 s4 p2, fwd+dgrad+wgrad"),
                   "gflop_per_step": round(sw["step_flops"] / 1e9, 2), "layout": "NCHW"},
        "frac_of_peak": round(value * 1e12 / PEAK_FP32_MFMA, 4),
        "roofline": {"kernel": "conv_gather_kernel / conv_gather_dl_kernel / conv1x1_stream_kernel / conv1x1_wst_kernel "
                               "(forward launches)",
                     "bound": "mfma", "achieved": round(sw["achieved"], 3), "peak": PEAK_FP32_MFMA / 1e12,
                     "unit": "TFLOP/s", "frac": round(sw["achieved"] * 1e12 / PEAK_FP32_MFMA, 4),
                     "traffic": traffic["bytes"] if traffic else None,
                     "traffic_algorithmic_bytes": traffic["algorithmic_bytes"] if traffic else None,
                     "traffic_source": traffic["source"] if traffic else None,
                     "avg_launch_ms": round(sw["avg_launch_ms"], 4),
                     "flop_per_launch_avg": round(sw["flop_per_launch_avg"])},
        "per_direction": sw["per_direction"],
        "per_layer_tflops": sw["per_layer_tflops"],
        "plans": {"tuned": not args.no_tune, "tile_slices": sw["plans"]},
        "parity": {"what": "outputs of the timed plans on the same inputs against PyTorch CPU float64: y and gx on "
                           "images 0 and N-1, 24 random entries of gw (whole-batch sums); rel-L2, bound 1e-4",
                   "max_rel_l2": max(v for d in sw["rel_l2_vs_torch_cpu"].values() for v in d.values()),
                   "per_layer": sw["rel_l2_vs_torch_cpu"]},
        "device": torch.cuda.get_device_name(dev),
    }
    if args.workload == "c5" and not args.no_nhwc:
        print("channels-last sweep ...", file=sys.stderr, flush=True)
        nw = conv_sweep(layers, dev, args.steps, args.warmup, not args.no_tune, nhwc=True)
        out["c5_nhwc"] = {
            "config": "the same C5 sweep with every tensor channels_last (NHWC activations, [co][ky][kx][ci] filters) "
                      "through the channels-last kernels",
            "value": round(nw["value"], 3), "unit": "TFLOP/s", "frac_of_peak": round(nw["value"] * 1e12 / PEAK_FP32_MFMA, 4),
            "ms_per_step": round(nw["ms_per_step"], 3), "per_direction": nw["per_direction"],
            "per_layer_tflops": nw["per_layer_tflops"], "plans": nw["plans"],
            "parity_max_rel_l2": max(v for d in nw["rel_l2_vs_torch_cpu"].values() for v in d.values())}
    if not args.no_cpu:
        print("cpu baselines ...", file=sys.stderr, flush=True)
        out["cpu_baseline"] = torch_cpu_baseline(layers, batch=16)
        out["oracle_cpu_baseline"] = oracle_baseline(layers)
    if not args.no_miopen:
        out["miopen_same_sweep"] = miopen_sweep(layers, dev, args.steps)
    if not args.no_bw:
        out["bandwidth_kernels"] = bandwidth_kernels(dev)
    if not args.no_models:
        import omarchy_mac_torch

        if args.workload == "c5":
            print("config 1 ...", file=sys.stderr, flush=True)
            out["alexnet_conv1_b16"] = c1_sub_object(dev, args.steps, args.warmup, not args.no_cpu)
        for cfg in train_configs():
            print(f"{cfg[0]} ...", file=sys.stderr, flush=True)
            out[cfg[0]] = train_step_bench(cfg, omarchy_mac_torch.DEVICE, args.model_steps, 5, 5, not args.no_cpu,
                                           compiled=cfg[0] in ("resnet18_b32", "mobilenetv3_b32"),
                                           fp64=cfg[0] == "resnet18_b32")
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()

"""Benchmark of the PECO per-layer attention hot path on one MI355X.

One step = one PecoAttention.attention call (sparse path) on the HunyuanVideo 480x720x17f
layer: 24 heads, 6750 video + 256 text tokens, D=128, bf16, k-means with 64 Q / 256 K
clusters and 10 Lloyd iterations from explicit initial centroids, 25% of key clusters
kept, Base-Offset off (``--workload hunyuan_480p_bo4`` turns it on). Inputs are
synthetic (Gaussian mixtures) and resident in HBM before timing starts.

value = effective TFLOP/s = 4*D*sum(kept |Q_i||K_j|) / layer time, the reference's metric.
The roofline object reports the attention kernel (the dominant MFMA kernel): its
algorithmic FLOPs over its average duration in the timed steps, measured with events
recorded on the launch stream around each of its launches.
cpu_baseline times the oracle's restatement of the reference CPU torch path on a bounded
sample of heads of the same workload.

The default run then times the other benchmark configurations under the same clock and
reports them under "other_workloads": the 480p layer with Base-Offset 4-bit, the 720p layer
(118800 + 256 tokens, 256/1024 clusters, 8 iterations, 15% kept, Base-Offset 4-bit) and the
544p Zipf denoising sequence (10 layer calls on drifting Q/K, warm-started k-means).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import subprocess
import sys
import time
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "PECO attn-layer ms + effective TFLOP/s at 24h x 7k tok bf16; % MFMA/HBM peak"
PEAK_BF16_TFLOPS = 2516.6
PEAK_HBM_GBS = 8000.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="hunyuan_480p")
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="budget of the CPU baseline sample")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--stage-reps", type=int, default=10)
    ap.add_argument("--profile-target", choices=("attention", "kmeans", "pack", "copy", "integer"), default=None,
                    help="replay only the attention launch, the Q+K k-means fit, the pack launch (fake-quant and "
                         "gather; Base-Offset workloads) or a plain device copy of --copy-mib MiB, --reps times "
                         "(for rocprofv3 counter runs)")
    ap.add_argument("--reps", type=int, default=10)
    ap.add_argument("--copy-mib", type=int, default=1024)
    ap.add_argument("--sequence", action="store_true",
                    help="time the workload's denoising sequence: its `steps` layer calls on drifting Q/K, the "
                         "first from the seeded centroids, the rest warm-started from the previous call's centroids")
    ap.add_argument("--headline-only", action="store_true",
                    help="skip the other configurations (Base-Offset 480p, 720p, the 544p Zipf sequence)")
    ap.add_argument("--summarize", metavar="CSV", default=None,
                    help="print per-kernel averages of a rocprofv3 counter_collection.csv or kernel_stats.csv")
    return ap.parse_args()


def make_layer(wl):
    from peco_amd import processor

    s = wl.shape
    cfg = processor.PecoConfig(num_q_centroids=s.num_q_centroids, num_k_centroids=s.num_k_centroids, top_p=wl.top_p,
                               min_kc_ratio=wl.min_kc_ratio, kmeans_iter_init=s.iterations,
                               kmeans_iter_step=s.iterations, warmup_steps=0, base_offset_bits=s.bits)
    ctx = processor.InferenceContext(step=0, text_length=s.text, valid_text_length=s.text)
    return processor.PecoAttention(0, cfg, ctx)


def run_step(layer, wl, q, k, v, q_init, k_init):
    # Every step fits from the same explicit initial centroids (the workload's k-means spec).
    layer.q_centroids, layer.k_centroids = q_init, k_init
    return layer.attention(q, k, v)


def stage_breakdown(layer, wl, q, k, v, q_init, k_init, reps):
    """Per-stage device time (ms) with events on the current stream, and the realised FLOPs.

    The stages follow ``PecoAttention.attention``: the selection launch also writes the
    attention's work list (kept-segment lists and ordered items). The attention reads Q/K/V
    through the sort permutations; with Base-Offset on, the fit ends with a launch that writes
    Q and K fake-quantized in original order, counted in the k-means stage. The repetitions are queued back to back, as the layer steps are,
    so the host's launch work overlaps the device's; the first repetition, which starts on
    an idle device, is not counted.
    """
    from peco_amd import _native, clustering_cuda, workloads

    s = wl.shape
    n, dim, heads = s.video, s.dims, s.heads
    names = ("kmeans", "select", "attention")
    minimum = math.ceil(wl.min_kc_ratio * s.num_k_centroids)
    length = q.shape[2]
    events = []
    for _ in range(reps + 1):
        ev = [_native.FencelessEvent() for _ in range(len(names) + 1)]
        ev[0].record()
        layer.q_centroids, layer.k_centroids = q_init, k_init
        fit = layer._fit_clusters(q[:, :, :n], k[:, :, :n], pack_keys=(s.bits, k, None) if s.bits else None,
                                  pack_order="original", query_full=q if s.bits else None)
        qs, ks, q_idx, k_idx = fit.q_sizes, fit.k_sizes, fit.q_idx, fit.k_idx
        ev[1].record()
        work = clustering_cuda.select_work(
            layer.q_centroids.reshape(1, heads, -1, dim), layer.k_centroids.reshape(1, heads, -1, dim), qs, ks,
            wl.top_p, minimum, (s.text, s.text), length, length)
        ev[2].record()
        if s.bits == 0:
            attn_args = (q, k, v, work, q_idx, k_idx, n, None, 0)
        else:
            attn_args = (fit.q_hat, fit.pack[0], v, work, q_idx, k_idx, n, None, 0)
        run_attention(attn_args)
        ev[3].record()
        events.append(ev)
    torch.cuda.synchronize()
    acc = {k_: 0.0 for k_ in names}
    for ev in events[1:]:
        for i, nm in enumerate(names):
            acc[nm] += ev[i].elapsed_time(ev[i + 1])
    # Realised F4 from the same selection as a map (outside the timed region).
    emap, eqs, eks = clustering_cuda.select_connections(
        layer.q_centroids.reshape(1, heads, -1, dim), layer.k_centroids.reshape(1, heads, -1, dim), qs, ks,
        wl.top_p, minimum, text=(s.text, s.text))
    flops = workloads.attention_flops(emap, eqs, eks, dim)
    return {k_: v_ / reps for k_, v_ in acc.items()}, flops, attn_args


def run_attention(args_):
    """The layer's attention launch over the selection's work list: indexed inputs when
    k_index is given, else packed ones."""
    from peco_amd import attention_cuda

    q, k, v, work, q_idx, k_idx, rows, q_centroids, bits = args_
    return attention_cuda.sparse_attention_work(q, k, v, work, out_index=q_idx, out_index_rows=rows, k_index=k_idx,
                                                q_centroids=q_centroids, bits=bits)


def attention_kernel_time(args_, reps=20):
    """Average duration of the sparse-attention launch on its stream."""
    from peco_amd import _native

    for _ in range(3):
        run_attention(args_)
    torch.cuda.synchronize()
    start, end = _native.FencelessEvent(), _native.FencelessEvent()
    start.record()
    for _ in range(reps):
        run_attention(args_)
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / reps


def measured_traffic(workload):
    """HBM bytes per attention launch from the committed rocprofv3 counter summary, if any."""
    import re

    path = ROOT / "profiles" / f"sparse_attention_{workload}_traffic.txt"
    if not path.exists():
        return None
    m = re.search(r"^traffic_bytes_per_launch:\s*([0-9.eE+]+)", path.read_text(), re.M)
    return float(m.group(1)) if m else None


def cpu_model():
    """The host CPU's model name, as lscpu reports it, with family/model/stepping and clock
    (a virtual machine may report only a generic name such as "AMD EPYC")."""
    fields = {}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            key, _, value = line.partition(":")
            fields[key.strip()] = value.strip()
    except (OSError, subprocess.SubprocessError):
        pass
    if "Model name" not in fields:
        try:
            for line in open("/proc/cpuinfo"):
                key, _, value = line.partition(":")
                fields.setdefault({"model name": "Model name", "cpu family": "CPU family", "model": "Model",
                                   "stepping": "Stepping", "cpu MHz": "CPU MHz"}.get(key.strip(), "_"), value.strip())
        except OSError:
            pass
    name = fields.get("Model name", "unknown")
    detail = [f"{k.lower()} {fields[k]}" for k in ("CPU family", "Model", "Stepping") if fields.get(k)]
    mhz = fields.get("CPU max MHz") or fields.get("CPU MHz")
    if mhz:
        detail.append(f"{float(mhz):.0f} MHz")
    if fields.get("Socket(s)"):
        detail.append(f"{fields['Socket(s)']} socket(s)")
    return f"{name} ({', '.join(detail)})" if detail else name


def cpu_baseline(wl, budget_s):
    """Oracle (reference CPU torch path) on whole heads of the workload until the budget is spent."""
    from oracle import reference_path
    from peco_amd import workloads

    s = wl.shape
    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    n = s.video
    done, flops, elapsed = 0, 0.0, 0.0
    while done < s.heads and (elapsed < budget_s or done == 0):
        h = slice(done, done + 1)
        q, k, v = (t[:, h].cpu().contiguous() for t in (wl.query, wl.key, wl.value))
        stages = {}
        t0 = time.perf_counter()
        reference_path.peco_layer(q, k, v, num_q_centroids=s.num_q_centroids, num_k_centroids=s.num_k_centroids,
                                  iterations=s.iterations, q_init=wl.q_init[h].cpu(), k_init=wl.k_init[h].cpu(),
                                  top_p=wl.top_p, min_kc_ratio=wl.min_kc_ratio, bits=s.bits, text_length=s.text,
                                  valid_text=s.text, stages=stages)
        elapsed += time.perf_counter() - t0
        flops += workloads.attention_flops(stages["ext_map"], stages["ext_q_sizes"], stages["ext_k_sizes"], s.dims)
        done += 1
    return {"value": flops / elapsed / 1e12, "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "cpu_model": cpu_model(),
            "sample": f"{done} of {s.heads} heads of {s.name}, full sequence, oracle reference_path "
                      f"(torch CPU, {threads} threads); {elapsed:.2f} s; "
                      f"layer {1e3 * elapsed / done * s.heads:.1f} ms extrapolated to {s.heads} heads"}


def summarize(path):
    """Per-kernel averages from a rocprofv3 CSV (counter collection or kernel stats)."""
    import csv
    from collections import defaultdict

    rows = list(csv.DictReader(open(path)))
    if rows and "Counter_Name" in rows[0]:
        acc = defaultdict(lambda: defaultdict(float))
        disp = defaultdict(set)
        for r in rows:
            name = r["Kernel_Name"].replace("(anonymous namespace)::", "").split("(")[0]
            acc[name][r["Counter_Name"]] += float(r["Counter_Value"])
            disp[name].add(r["Dispatch_Id"])
        for name, counters in acc.items():
            n = len(disp[name])
            vals = ", ".join(f"{k}={v / n:.6g}" for k, v in sorted(counters.items()))
            print(f"{name}: dispatches={n} per-dispatch {vals}")
    else:
        for r in rows[:20]:
            print(",".join(r.values()))


def profile_target(args):
    dev = torch.device("cuda:0")
    if args.profile_target == "copy":
        n = args.copy_mib * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(args.reps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(f"copy {args.copy_mib} MiB x {args.reps}: reads {args.copy_mib * 1024} KiB and writes "
              f"{args.copy_mib * 1024} KiB per dispatch", flush=True)
        return
    if args.profile_target == "integer":
        # The integer-score attention and the launch over rounded rows on the same selection
        # (Base-Offset workloads), each args.reps times after two untimed calls.
        print(json.dumps(measure_integer_scores(args.workload, 1, 1, args.reps)), flush=True)
        return
    from peco_amd import _native, clustering_cuda, workloads

    wl = workloads.make_workload(args.workload, device=dev)
    s = wl.shape
    layer = make_layer(wl)
    n = s.video
    with torch.no_grad():
        if args.profile_target == "kmeans":
            # The layer's fused Q+K fit from the seeded centroids (stage 1).
            problems = [clustering_cuda.KMeansProblem(wl.query[0, :, :n], wl.q_init),
                        clustering_cuda.KMeansProblem(wl.key[0, :, :n], wl.k_init)]
            clustering_cuda.kmeans_fit(problems, s.iterations)
            torch.cuda.synchronize()
            start, end = _native.FencelessEvent(), _native.FencelessEvent()
            start.record()
            for _ in range(args.reps):
                clustering_cuda.kmeans_fit(problems, s.iterations)
            end.record()
            torch.cuda.synchronize()
            t = start.elapsed_time(end) / args.reps
            f1 = 2.0 * s.dims * n * (s.num_q_centroids + s.num_k_centroids) * s.heads * s.iterations
            print(f"kmeans fit {t * 1e3:.1f} us, F1 {f1:.6g} FLOPs ({f1 / (t * 1e-3) / 1e12:.1f} TFLOP/s); "
                  f"per iteration and launch: assign, sort, update", flush=True)
            return
        if args.profile_target == "pack":
            # Stages 2+3: fake-quant Q/K against their centroids and gather Q/K/V into cluster order.
            layer.q_centroids, layer.k_centroids = wl.q_init, wl.k_init
            fit = layer._fit_clusters(wl.query[:, :, :n], wl.key[:, :, :n])
            ql, kl, q_idx, k_idx = fit.q_labels, fit.k_labels, fit.q_idx, fit.k_idx
            pack_args = ([wl.query, wl.key, wl.value], [q_idx, k_idx, k_idx], [ql, kl, None],
                         [layer.q_centroids, layer.k_centroids, None], [s.bits, s.bits, 0], n)
            clustering_cuda.pack_clustered(*pack_args)
            torch.cuda.synchronize()
            start, end = _native.FencelessEvent(), _native.FencelessEvent()
            start.record()
            for _ in range(args.reps):
                clustering_cuda.pack_clustered(*pack_args)
            end.record()
            torch.cuda.synchronize()
            t = start.elapsed_time(end) / args.reps
            # B2 + B3 of the pack: read x and write x-hat for Q, K (2D bytes each way per row, plus
            # label and index) and V (gather only), text rows copied.
            rows = s.heads * s.length
            b = 3 * rows * 2 * s.dims * 2 + s.heads * n * (4 + 4) * 2 + s.heads * n * 4
            print(f"pack launch {t * 1e3:.1f} us, algorithmic {b:.6g} bytes ({b / (t * 1e-3) / 1e9:.0f} GB/s)",
                  flush=True)
            return
        _, flops, attn_args = stage_breakdown(layer, wl, wl.query, wl.key, wl.value, wl.q_init, wl.k_init, 1)
        t = attention_kernel_time(attn_args, args.reps)
    print(f"attention launch {t * 1e3:.1f} us, {flops / (t * 1e-3) / 1e12:.1f} TFLOP/s, flops {flops:.6g}",
          flush=True)


def run_sequence(workload, steps, warmup):
    """Multi-step scenario: one repetition = the workload's `steps` calls of one layer on Q/K
    drifting by N(0, drift^2) per step (V fixed), k-means warm-started between calls.

    Call 0 fits from the seeded centroids with `iterations` Lloyd iterations; calls 1.. start
    from the layer's cached centroids with `warm_iterations` (PecoAttention's kmeans_iter_step),
    as PecoAttention.attention does across denoising steps (peco/processor.py:98-113). All
    inputs are generated before timing. value = sum of the calls' F4 / sequence time. The
    roofline covers one more pass of the sequence with HIP events around each attention launch:
    the calls' summed F4 over the launches' summed durations.
    """
    from peco_amd import _native, attention_cuda, clustering_cuda, processor, workloads

    dev = torch.device("cuda:0")
    wl = workloads.make_workload(workload, device=dev)
    s = wl.shape
    calls = max(1, s.steps)
    inputs = [wl]
    for step in range(1, calls):
        inputs.append(workloads.drift(inputs[-1], step))
    layer = make_layer(wl)
    first_cfg = layer.config
    warm_cfg = processor.PecoConfig(**{**first_cfg.__dict__, "kmeans_iter_step": s.warm_iterations or s.iterations})

    def sequence(times=None):
        outs = []
        for i, cur in enumerate(inputs):
            if times is not None:
                ev = _native.FencelessEvent()
                ev.record()
                times.append(ev)
            if i == 0:
                layer.config = first_cfg
                layer.q_centroids, layer.k_centroids = wl.q_init, wl.k_init
            else:
                layer.config = warm_cfg
            outs.append(layer.attention(cur.query, cur.key, cur.value))
        if times is not None:
            ev = _native.FencelessEvent()
            ev.record()
            times.append(ev)
        return outs

    with torch.no_grad():
        for _ in range(warmup):
            sequence()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            sequence()
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) * 1e3 / steps
        evs = []
        timer = attention_cuda.launch_timer = _native.LaunchTimer()
        try:
            sequence(evs)
            torch.cuda.synchronize()
        finally:
            attention_cuda.launch_timer = None
        call_ms = [evs[i].elapsed_time(evs[i + 1]) for i in range(calls)]
        launches = timer.elapsed_ms()
        if len(launches) != calls:
            raise RuntimeError(f"expected one attention launch per call, timed {len(launches)} for {calls} calls")
        # Realised F4 of every call: the same fits (bit-exact) rerun with the selection.
        flops = []
        n, dim = s.video, s.dims
        minimum = math.ceil(wl.min_kc_ratio * s.num_k_centroids)
        for i, cur in enumerate(inputs):
            layer.config = first_cfg if i == 0 else warm_cfg
            if i == 0:
                layer.q_centroids, layer.k_centroids = wl.q_init, wl.k_init
            _, _, qs, ks = layer._update_cluster_state(cur.query[:, :, :n], cur.key[:, :, :n])
            emap, eqs, eks = clustering_cuda.select_connections(
                layer.q_centroids.reshape(1, s.heads, -1, dim), layer.k_centroids.reshape(1, s.heads, -1, dim), qs,
                ks, wl.top_p, minimum, text=(s.text, s.text))
            flops.append(workloads.attention_flops(emap, eqs, eks, dim))
    total = sum(flops)
    value = total / (ms * 1e-3) / 1e12
    attn_ms = sum(launches)
    achieved = total / (attn_ms * 1e-3) / 1e12
    line = {
        "metric": METRIC, "value": round(value, 3), "unit": "TFLOP/s", "n_gpus": 1, "steps": steps,
        "warmup": warmup, "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": s.name, "heads": s.heads, "video_tokens": s.video, "text_tokens": s.text,
                   "head_dim": s.dims, "q_clusters": s.num_q_centroids, "k_clusters": s.num_k_centroids,
                   "kmeans_iterations": s.iterations, "warm_iterations": s.warm_iterations, "drift": s.drift,
                   "keep_ratio": s.keep_ratio, "base_offset_bits": s.bits, "layer_calls_per_step": calls},
        "sequence": {"call_ms": [round(t, 4) for t in call_ms], "call_flops": flops,
                     "first_call_ms": round(call_ms[0], 4),
                     "warm_call_ms": round(sum(call_ms[1:]) / max(1, calls - 1), 4),
                     "attention_ms": [round(t, 4) for t in launches]},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_BF16_TFLOPS, 4), "traffic": measured_traffic(s.name),
                     "kernel": "sparse_attention_kernel, indexed inputs, work list from the selection launch; "
                               "the calls' F4 over their launches' summed durations",
                     "kernel_ms": round(attn_ms / calls, 4), "flops": total / calls},
        "layer_frac_of_peak": round(value / PEAK_BF16_TFLOPS, 4),
    }
    return line


def measure(name, steps, warmup, stage_reps):
    """One workload's layer: ms per step, stage times, realised F4 and the attention roofline
    (the attention launch's average duration over the timed steps, from HIP timing events recorded
    on its stream immediately around each launch, created without the system-scope fence)."""
    from peco_amd import _native, attention_cuda, workloads

    dev = torch.device("cuda:0")
    wl = workloads.make_workload(name, device=dev)
    s = wl.shape
    layer = make_layer(wl)
    q, k, v = wl.query, wl.key, wl.value
    q_init, k_init = wl.q_init, wl.k_init
    with torch.no_grad():
        for _ in range(warmup):
            run_step(layer, wl, q, k, v, q_init, k_init)
        torch.cuda.synchronize()
        timer = attention_cuda.launch_timer = _native.LaunchTimer()
        try:
            t0 = time.perf_counter()
            for _ in range(steps):
                run_step(layer, wl, q, k, v, q_init, k_init)
            torch.cuda.synchronize()
            ms = (time.perf_counter() - t0) * 1e3 / steps
        finally:
            attention_cuda.launch_timer = None
        if not len(timer):
            raise RuntimeError("the layer step ran no work-list attention launch to time")
        launches = timer.elapsed_ms()
        t_attn = sum(launches) / len(launches)
        stages, flops, attn_args = stage_breakdown(layer, wl, q, k, v, q_init, k_init, stage_reps)
    value = flops / (ms * 1e-3) / 1e12
    achieved = flops / (t_attn * 1e-3) / 1e12
    out = {
        "value": round(value, 3), "ms_per_step": round(ms, 4), "steps": steps, "warmup": warmup,
        "config": {"workload": s.name, "heads": s.heads, "video_tokens": s.video, "text_tokens": s.text,
                   "head_dim": s.dims, "q_clusters": s.num_q_centroids, "k_clusters": s.num_k_centroids,
                   "kmeans_iterations": s.iterations, "keep_ratio": s.keep_ratio, "base_offset_bits": s.bits},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_BF16_TFLOPS, 4), "traffic": measured_traffic(s.name),
                     "kernel": "sparse_attention_kernel, " + ("indexed" if attn_args[5] is not None else
                                                              "K/V packed by the fit, Q quantized at load")
                     + " inputs, work list from the selection launch", "kernel_ms": round(t_attn, 4),
                     "flops": flops},
        "stages_ms": {k_: round(v_, 4) for k_, v_ in stages.items()},
        "layer_frac_of_peak": round(value / PEAK_BF16_TFLOPS, 4),
    }
    # Stage 1 on its own: F1 = 2*D*N*(KQ+KK)*BH*iterations useful FLOPs over the fit's stage time.
    f1 = 2.0 * s.dims * s.video * (s.num_q_centroids + s.num_k_centroids) * s.heads * s.iterations
    if stages.get("kmeans"):
        t1 = f1 / (stages["kmeans"] * 1e-3) / 1e12
        out["kmeans_fit"] = {"flops": f1, "tflops": round(t1, 2), "frac_of_peak": round(t1 / PEAK_BF16_TFLOPS, 4)}
    return out, wl


def measure_integer_scores(name, steps, warmup, reps):
    """The Base-Offset layer with integer scores (PecoAttention.integer_scores, an extension
    with no counterpart in the reference): ms per layer step, and the integer-score attention
    launch against the launch over rounded reconstructions on the same selection."""
    from peco_amd import _native, attention_cuda, clustering_cuda, workloads

    wl = workloads.make_workload(name, device=torch.device("cuda:0"))
    s = wl.shape
    n, heads, dim = s.video, s.heads, s.dims
    layer = make_layer(wl)
    layer.integer_scores = True
    q, k, v = wl.query, wl.key, wl.value
    with torch.no_grad():
        for _ in range(warmup):
            run_step(layer, wl, q, k, v, wl.q_init, wl.k_init)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            run_step(layer, wl, q, k, v, wl.q_init, wl.k_init)
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) * 1e3 / steps
        layer.q_centroids, layer.k_centroids = wl.q_init, wl.k_init
        fit = layer._fit_clusters(q[:, :, :n], k[:, :, :n], pack_keys=(s.bits, k, v, True))
        qs, ks, q_idx = fit.q_sizes, fit.k_sizes, fit.q_idx
        kp, vp, codes, low, scale = fit.pack
        minimum = math.ceil(wl.min_kc_ratio * s.num_k_centroids)
        qc4 = layer.q_centroids.reshape(1, heads, -1, dim)
        kc4 = layer.k_centroids.reshape(1, heads, -1, dim)
        emap, eqs, eks = clustering_cuda.select_connections(qc4, kc4, qs, ks, wl.top_p, minimum,
                                                            text=(s.text, s.text))
        work = clustering_cuda.select_work(qc4, kc4, qs, ks, wl.top_p, minimum, (s.text, s.text), q.shape[2],
                                           q.shape[2])
        flops = workloads.attention_flops(emap, eqs, eks, dim)

        def integer():
            return attention_cuda.base_offset_attention(
                q, kp, vp, emap, eqs, eks, out_index=q_idx, q_centroids=layer.q_centroids,
                k_centroids=layer.k_centroids, k_codes=codes, k_low=low, k_scale=scale, bits=s.bits)

        def rounded():
            return attention_cuda.sparse_attention_work(q, kp, vp, work, out_index=q_idx, out_index_rows=n,
                                                        q_centroids=layer.q_centroids, bits=s.bits)

        times = {}
        for label, fn in (("integer", integer), ("rounded", rounded)):
            for _ in range(2):
                fn()
            torch.cuda.synchronize()
            start, end = _native.FencelessEvent(), _native.FencelessEvent()
            start.record()
            for _ in range(reps):
                fn()
            end.record()
            torch.cuda.synchronize()
            times[label] = start.elapsed_time(end) / reps
    return {
        "ms_per_step": round(ms, 4), "value": round(flops / (ms * 1e-3) / 1e12, 3), "steps": steps,
        "attention_ms": round(times["integer"], 4),
        "attention_tflops": round(flops / (times["integer"] * 1e-3) / 1e12, 2),
        "rounded_attention_ms": round(times["rounded"], 4),
        "note": "video x video scores from the Base-Offset codes on v_mfma_i32_32x32x32_i8 (extension); "
                "attention_ms includes the centroid-plane preparation launches",
    }


# The other benchmark configurations, timed in the default run after the headline one:
# (workload, steps, warmup, stage reps, attention reps); the denoising sequence separately.
OTHER_WORKLOADS = (("hunyuan_480p_bo4", 20, 3, 5), ("hunyuan_720p", 3, 1, 2))
SEQUENCE_WORKLOAD = ("hunyuan_544p_zipf", 2, 1)


def main():
    args = parse()
    if args.summarize:
        summarize(args.summarize)
        return
    if args.profile_target:
        profile_target(args)
        return
    if args.gpus != 1:
        print(json.dumps({"error": "bench.py measures one GPU; runs on more than one are not supported",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    if args.sequence:
        print(json.dumps(run_sequence(args.workload, args.steps, args.warmup)), flush=True)
        return
    head, wl = measure(args.workload, args.steps, args.warmup, args.stage_reps)
    line = {
        "metric": METRIC, "value": head["value"], "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": head["ms_per_step"], "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
    }
    line.update({k_: v_ for k_, v_ in head.items() if k_ not in ("value", "ms_per_step", "steps", "warmup")})
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(wl, args.cpu_seconds)
    del wl
    if not args.headline_only and args.workload == "hunyuan_480p":
        others = {}
        for name, steps, warmup, stage_reps in OTHER_WORKLOADS:
            others[name], _ = measure(name, steps, warmup, stage_reps)
            torch.cuda.empty_cache()
        others["hunyuan_480p_bo4_integer_scores"] = measure_integer_scores("hunyuan_480p_bo4", 10, 2, 10)
        torch.cuda.empty_cache()
        name, steps, warmup = SEQUENCE_WORKLOAD
        seq = run_sequence(name, steps, warmup)
        keep = ("value", "steps", "warmup", "ms_per_step", "config", "roofline", "layer_frac_of_peak")
        others[name + "_sequence"] = {k_: v_ for k_, v_ in seq.items() if k_ not in line or k_ in keep}
        line["other_workloads"] = others
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()

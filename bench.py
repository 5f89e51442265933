"""Throughput benchmark: speaker embeddings on one MI355X.

Default workload (the headline line): WeSpeaker ResNet34, batch 64 x 3 s 16 kHz
synthetic clips (FBank 64x80x298), random-init f16 weights with folded BN, the
full path PCM -> FBank -> ResNet34 -> TSTP -> FC -> L2 on the GPU.  `--model`
selects one of the other encoder workloads (ECAPA-TDNN B=64 x 4 s, CAM++
B=32 x 10 s q8_0, ERes2Net B=16 x 20 s q8_0) for the same measurement, or
one of the wav2vec2 analyze workloads (emotion: wav2vec2-base + weighted-sum
classifier; age/gender: wav2vec2-large-robust + two heads; B=64 x 3 s raw
waveform, clips/s).

A step is one batch; inputs are resident in HBM before the timed region.
Prints one JSON line (rank 0, N=1).  Without --model the line's `value`,
`roofline` and `cpu_baseline` are the headline workload's and `configs` carries
every workload of the benchmark's config list, measured the same way in the
same process: the batch-1 ResNet34 latency (median ms per clip, device-resident
and host-buffer paths, beside the reference's published per-clip figures) and
the ECAPA-TDNN, CAM++ and ERes2Net batches (throughput, dominant kernel's
roofline fraction, a bounded CPU-baseline sample).

`roofline` covers the dominant kernel: the conv class with the most time in a
pass with HIP events around every launch (on the library's stream).  A second
timed pass of the same steps records events around that class's launches only
(a few events per step), and its average launch duration gives
achieved = algorithmic FLOPs (direct conv) or bytes per launch / duration,
against the MFMA f16 or HBM peak depending on which side of the ridge the
kernel's arithmetic intensity lies.  `traffic` is that kernel's HBM bytes per
launch, measured in the same run: before the bench touches the GPU, two
child processes run the run's workloads under `rocprofv3 --pmc FETCH_SIZE`
and `--pmc WRITE_SIZE`, each counter scaled by its reading for a device copy
of known size; `traffic_source` names the kernel and launch grid it was read
from (null with the reason where rocprofv3 is absent or --no-traffic is
given).  The CPU baseline times the oracle
(this repository's C restatement of the reference CPU path) on a bounded
sample of the same clips, clip-parallel on min(cores, 8) threads like the
reference's default.
"""
import argparse
import json
import os
import sys
import tempfile
import time
from concurrent.futures import ThreadPoolExecutor

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "voice-detect.cpp_amd"))

from vdamd import lib, synth  # noqa: E402

PEAK_F16_TFLOPS = 2500.0     # MI355X dense f16 MFMA
PEAK_HBM_GBS = 8000.0        # MI355X HBM3E
RIDGE_FLOP_PER_BYTE = PEAK_F16_TFLOPS * 1e12 / (PEAK_HBM_GBS * 1e9)
CLIP_SEED = 1234

# HBM traffic of the dominant kernels, measured in the same bench run: before
# this process touches the GPU, two child processes run every workload of the
# run under `rocprofv3 --pmc FETCH_SIZE` and `--pmc WRITE_SIZE` (one counter
# per pass), with a device copy of known size after each workload that both
# separates the workloads in the dispatch list and calibrates the counters
# (bytes moved / counter reading).  A workload's dominant class is then the
# (kernel, grid) group of its dispatches whose count matches the class's
# launches per step and which takes the most time.
TRAFFIC_STEPS = 3
TRAFFIC_COPY_MIB = 96        # above any workload's PCM upload, so the copies are told apart
TRAFFIC_TIMEOUT_S = 150

# The reference's own published figures for these workloads (per clip, batch 1;
# it publishes nothing batched): reported beside ours, not divided into them.
REFERENCE_PUBLISHED = {
    "resnet34_cpu_encoder_8t_emb_s": {
        "value": 115.0, "unit": "embeddings/s",
        "note": "WeSpeaker ResNet34 encoder only (FBank excluded), 3 s clip, ~8.7 ms at 8 threads on a Ryzen 9 "
                "9950X3D, f32 blocked direct conv (docs/cpu-optimization.md:142-146)"},
    "resnet34_b1_ms": [
        {"value": 8.46, "unit": "ms per clip", "note": "ggml GPU backend (cuDNN conv), NVIDIA GB10, batch 1 "
                                                       "(benchmarks/RESULTS.md:183-190)"},
        {"value": 15.01, "unit": "ms per clip", "note": "wav -> embedding end to end, 8 threads, Ryzen 9 9950X3D "
                                                        "(benchmarks/demo/spec.json:2-3)"}],
    "per_clip_8t_ms": {"ecapa": 54.1, "resnet34": 56.1, "eres2net": 82.9, "campplus": 30.5,
                       "note": "per-clip end to end at 8 threads, older build, Ryzen 9 9950X3D "
                               "(benchmarks/RESULTS.md:163-170)"},
    "gb10_b1_ms": {"ecapa": 8.92, "resnet34": 8.46, "eres2net": 10.06, "campplus": 15.74,
                   "note": "ggml GPU backend, NVIDIA GB10, batch 1 (benchmarks/RESULTS.md:183-190)"},
}

# The workloads of the benchmark's config list beside the headline (ResNet34 B=64).
CONFIG_SET = ("ecapa", "campplus", "eres2net")

MODELS = {
    "resnet34": {
        "metric": "embeddings/s, ResNet34 B=64 3 s clips; conv MFMA util vs f16 peak",
        "write": synth.write_resnet34, "seed": 2024, "batch": 64, "n": 48000, "oracle": "OracleResNet",
        "dtype": "f16",
        "config": {"workload": "WeSpeaker ResNet34 embed, batch 64 x 3 s 16 kHz clips (FBank 64x80x298), "
                               "random-init f16 weights with folded BN, PCM->FBank->ResNet34->TSTP->FC->L2 on GPU",
                   "batch": 64, "clip_seconds": 3.0, "frames": 298, "channels": [32, 64, 128, 256],
                   "blocks": [3, 4, 6, 3]},
    },
    "ecapa": {
        "metric": "embeddings/s, ECAPA-TDNN B=64 4 s clips; conv MFMA util vs f16 peak",
        "write": synth.write_ecapa, "seed": 7, "batch": 64, "n": 64000, "oracle": "OracleEcapa", "dtype": "f16",
        "config": {"workload": "ECAPA-TDNN embed, batch 64 x 4 s clips (398 frames), C=1024 k=5, 3 SE-Res2 "
                               "blocks (dil 2/3/4, scale 8, SE 128), MFA 1536, ASP, 192-d, random-init f16 weights",
                   "batch": 64, "clip_seconds": 4.0, "frames": 398},
    },
    "campplus": {
        "metric": "embeddings/s, CAM++ B=32 10 s clips q8_0; conv MFMA util vs f16 peak",
        "write": synth.write_campplus, "seed": 5, "batch": 32, "n": 160000, "oracle": "OracleCampplus",
        "dtype": "f16",
        "config": {"workload": "CAM++ embed, batch 32 x 10 s clips (998 frames), FCM 32ch, D-TDNN 12/24/16 "
                               "growth 32 bottleneck 128 with context masks, stats, 192-d, q8_0 1x1 weights",
                   "batch": 32, "clip_seconds": 10.0, "frames": 998},
    },
    "w2v2_emotion": {
        "metric": "analyzed clips/s, wav2vec2-base emotion B=64 3 s clips; GEMM MFMA util vs f16 peak",
        "write": lambda path, seed: synth.write_w2v2(path, seed, "emotion"), "seed": 7, "batch": 64, "n": 48000,
        "oracle": "w2v2", "dtype": "f16", "kind": "analyze",
        "config": {"workload": "wav2vec2-base emotion analyze, batch 64 x 3 s 16 kHz clips (149 frames): 7 conv "
                               "feature layers (512), 12 post-norm layers 768/12 heads/3072, pos conv 128x16 groups, "
                               "weighted layer sum, projector 256, 4 labels; random-init f16 weights",
                   "batch": 64, "clip_seconds": 3.0, "frames": 149},
    },
    "w2v2_age_gender": {
        "metric": "analyzed clips/s, wav2vec2-large-robust age/gender B=64 3 s clips; GEMM MFMA util vs f16 peak",
        "write": lambda path, seed: synth.write_w2v2(path, seed, "age_gender"), "seed": 7, "batch": 64, "n": 48000,
        "oracle": "w2v2", "dtype": "f16", "kind": "analyze",
        "config": {"workload": "wav2vec2-large-robust age/gender analyze, batch 64 x 3 s 16 kHz clips (149 frames): "
                               "waveform normalisation, 7 LayerNorm conv layers (512, bias), 24 pre-norm layers "
                               "1024/16 heads/4096, age + gender tanh heads; random-init f16 weights",
                   "batch": 64, "clip_seconds": 3.0, "frames": 149},
    },
    "eres2net": {
        "metric": "embeddings/s, ERes2Net B=16 20 s clips q8_0; conv MFMA util vs f16 peak",
        "write": synth.write_eres2net, "seed": 9, "batch": 16, "n": 320000, "oracle": "OracleEres2net",
        "dtype": "split-f16",
        "config": {"workload": "ERes2Net base embed, batch 16 x 20 s clips (1998 frames), m_channels 32, "
                               "blocks 3/4/6/3, Res2 scale 2, AFF, TSTP, 512-d, q8_0 1x1 weights, split-f16 convs",
                   "batch": 16, "clip_seconds": 20.0, "frames": 1998},
    },
}


def profile_pass(ctx, run, steps):
    ctx.set_profiling(True)
    ctx.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        run()
    ctx.synchronize()
    wall = (time.perf_counter() - t0) / steps
    recs = ctx.profile()
    ctx.set_profiling(False)
    per = {}
    for name, ms, fl, by in recs:
        p = per.setdefault(name, {"launches": 0, "ms": 0.0, "flops": 0.0, "bytes": 0.0})
        p["launches"] += 1
        p["ms"] += ms
        p["flops"] += fl
        p["bytes"] += by
    return per, wall * 1e3


def dominant_pass(ctx, run, steps, name):
    """Timed steps with events around the launches named `name` only."""
    ctx.set_profiling(True, name)
    ctx.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        run()
    ctx.synchronize()
    wall = (time.perf_counter() - t0) / steps
    recs = [r for r in ctx.profile() if r[0] == name]
    ctx.set_profiling(False)
    return recs, wall * 1e3


def registry_bench(L, d_emb, batch, dim, rows, k, steps):
    """Identify: the batch's embeddings against `rows` random unit rows, top k
    (vdk_registry_topk; f64 sums of exact f32 products)."""
    rng = np.random.default_rng(99)
    reg = rng.standard_normal((rows, dim)).astype(np.float32)
    reg /= np.linalg.norm(reg, axis=1, keepdims=True)
    d_reg = lib.DeviceBuffer.from_array(reg)
    ws = L.vdk_registry_topk_workspace_size(batch, rows, k)
    d_ws, d_idx, d_sc = lib.DeviceBuffer(ws), lib.DeviceBuffer(batch * k * 4), lib.DeviceBuffer(batch * k * 4)
    call = lambda: lib.check(L.vdk_registry_topk(d_emb.ptr, batch, d_reg.ptr, rows, dim, k, d_ws.ptr, ws,
                                                 d_idx.ptr, d_sc.ptr, None))
    for _ in range(3):
        call()
    lib.check(L.vdk_synchronize())
    t0 = time.perf_counter()
    for _ in range(steps):
        call()
    lib.check(L.vdk_synchronize())
    dt = (time.perf_counter() - t0) / steps
    flops = 2.0 * batch * rows * dim
    return {"queries": batch, "rows": rows, "dim": dim, "k": k, "ms_per_call": round(dt * 1e3, 4),
            "queries_per_s": round(batch / dt, 1), "f64_tflops": round(flops / dt / 1e12, 3),
            "f64_peak_tflops": 78.6, "registry_gbs": round(rows * dim * 4 / dt / 1e9, 1)}


def cpu_baseline(model, gguf_path, pcm, n_seconds, min_seconds=10.0):
    """The oracle on the host: rounds of `threads` clips (cycling through the
    batch's clips) until at least min_seconds of wall time have passed."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import pyoracle
    from vdamd import gguf

    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = os.cpu_count() or 1
    threads = max(1, min(8, avail))            # the reference's default min(hw, 8) threads
    if model["oracle"] == "w2v2":
        return cpu_baseline_w2v2(gguf_path, pcm, n_seconds, threads, avail, min_seconds)
    net = getattr(pyoracle, model["oracle"])(gguf.GGUFFile(gguf_path))
    done = 0
    t0 = time.perf_counter()
    with ThreadPoolExecutor(threads) as ex:
        while True:
            idx = [(done + i) % len(pcm) for i in range(threads)]
            if model["oracle"] == "OracleResNet":
                net.embed_batch(pcm[idx], n_threads=threads)
            else:
                # the oracle releases the GIL inside its C calls: one clip per thread
                list(ex.map(lambda k: net.forward(pyoracle.fbank(pcm[k])), idx))
            done += threads
            if time.perf_counter() - t0 >= min_seconds:
                break
    dt = time.perf_counter() - t0
    cpu_name = _cpu_name()
    return {"value": round(done / dt, 3), "unit": "embeddings/s", "cores": threads, "kind": "port",
            "sample": f"{done} clips (the batch's {len(pcm)} synthetic {n_seconds:g} s clips, cycled) through the "
                      f"oracle's FBank + encoder (f32), clip-parallel on {threads} threads, {dt:.1f} s wall; "
                      f"host {cpu_name}, {avail} cores available",
            "note": "the port is this repository's plain scalar C restatement of the reference's CPU path (the "
                    "parity oracle), not the reference's AVX-512 blocked build, which the reference publishes at "
                    "about 7x this rate for ResNet34 (see reference_published)"}


def _cpu_name():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return ""


def cpu_baseline_w2v2(gguf_path, pcm, n_seconds, threads, avail, min_seconds):
    """The wav2vec2 oracle (numpy f64, its GEMMs on `threads` BLAS threads),
    one clip after another until min_seconds have passed."""
    import oracle_w2v2
    from threadpoolctl import threadpool_limits

    net = oracle_w2v2.OracleW2V2(gguf_path)
    done = 0
    with threadpool_limits(limits=threads):
        t0 = time.perf_counter()
        while True:
            net.raw_outputs(pcm[done % len(pcm)])
            done += 1
            if time.perf_counter() - t0 >= min_seconds:
                break
        dt = time.perf_counter() - t0
    return {"value": round(done / dt, 3), "unit": "clips/s", "cores": threads, "kind": "port",
            "sample": f"{done} clips (the batch's synthetic {n_seconds:g} s clips, cycled) through the oracle's "
                      f"wav2vec2 forward (numpy f64, BLAS on {threads} threads), {dt:.1f} s wall; "
                      f"host {_cpu_name()}, {avail} cores available"}


def traffic_child(keys):
    """Child of a traffic pass (run under rocprofv3 --pmc): each workload for
    TRAFFIC_STEPS batches after one warmup batch, then TRAFFIC_COPY_MIB device
    copies (3x) that close its segment of the dispatch list."""
    L = lib.lib()
    nb = TRAFFIC_COPY_MIB << 20
    src, dst = lib.DeviceBuffer(nb), lib.DeviceBuffer(nb)
    lib.check(L.vdk_memset(src.ptr, 1, nb))
    for key in keys:
        model = MODELS[key]
        batch, n = model["batch"], model["n"]
        path = os.path.join(tempfile.mkdtemp(), f"{key}.gguf")
        model["write"](path, seed=model["seed"])
        ctx = lib.Context(path)
        d_pcm = lib.DeviceBuffer.from_array(synth.clips(CLIP_SEED, batch, n))
        width = ctx.analyze_outputs() if model.get("kind") == "analyze" else ctx.dim
        d_out = lib.DeviceBuffer(batch * width * 4)
        run = (lambda: ctx.analyze_device_async(d_pcm.ptr, batch, n, d_out.ptr)) if model.get("kind") == "analyze" \
            else (lambda: ctx.embed_device_async(d_pcm.ptr, batch, n, d_out.ptr))
        run()                                    # warmup, unmarked
        ctx.synchronize()
        # the measured batches with every labelled launch bracketed by marker
        # dispatches, so the parent can attribute each dispatch to its label
        ctx.set_profiling(True)
        ctx.set_profiling_markers(True)
        for _ in range(TRAFFIC_STEPS):
            run()
        ctx.synchronize()
        labels = [r[0] for r in ctx.profile()]
        ctx.set_profiling_markers(False)
        ctx.set_profiling(False)
        ctx.close()
        with open(os.environ["VDK_TRAFFIC_LABELS"] + "." + key, "w") as fh:
            json.dump(labels, fh)
        for _ in range(3):
            lib.check(L.vdk_memcpy_d2d(dst.ptr, src.ptr, nb))
        lib.check(L.vdk_synchronize())


def traffic_passes(keys):
    """Run the two counter passes; returns {key: [dispatch groups]} where a
    group is {kernel, grid, count, us, fetch_b, write_b} (bytes per dispatch,
    calibrated), or {"error": why}."""
    import csv
    import shutil
    import subprocess
    if shutil.which("rocprofv3") is None:
        return {"error": "rocprofv3 not on PATH"}
    out = {}
    env = dict(os.environ, TMPDIR=os.environ.get("TMPDIR", "/tmp"))
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        d = tempfile.mkdtemp()
        env["VDK_TRAFFIC_LABELS"] = os.path.join(d, "labels")
        cmd = ["rocprofv3", "--pmc", counter, "--output-format", "csv", "-d", d, "-o", "run", "--",
               sys.executable, os.path.abspath(__file__), "--traffic-child", ",".join(keys)]
        try:
            r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, timeout=TRAFFIC_TIMEOUT_S,
                               env=env)
        except subprocess.TimeoutExpired:
            return {"error": f"rocprofv3 --pmc {counter} pass timed out"}
        files = [os.path.join(dp, f) for dp, _, fs in os.walk(d) for f in fs if f.endswith("counter_collection.csv")]
        if not files:
            return {"error": f"rocprofv3 --pmc {counter} wrote no counters (rc {r.returncode})"}
        rows = sorted(csv.DictReader(open(files[0])), key=lambda row: int(row["Dispatch_Id"]))
        # segments: the dispatches of workload i end at its 3 calibration copies
        seg, segs, cal = [], [], []
        for row in rows:
            if "copyBuffer" in row["Kernel_Name"]:
                if float(row["Counter_Value"]) > (TRAFFIC_COPY_MIB << 10) / 4:   # KiB: a calibration copy
                    cal.append(float(row["Counter_Value"]) * 1024.0)
                    if seg:
                        segs.append(seg)
                        seg = []
                continue
            seg.append(row)
        if len(segs) != len(keys) or not cal:
            return {"error": f"{counter}: {len(segs)} dispatch segments for {len(keys)} workloads"}
        factor = (TRAFFIC_COPY_MIB << 20) / float(np.median(cal))
        for key, sg in zip(keys, segs):
            groups = out.setdefault(key, {})
            marker = lambda row: "profile_marker_kernel" in row["Kernel_Name"]
            for row in sg:
                if marker(row):
                    continue
                g = groups.setdefault((row["Kernel_Name"], int(row["Grid_Size"])),
                                      {"count": 0, "us": 0.0, "FETCH_SIZE": 0.0, "WRITE_SIZE": 0.0})
                if counter == "FETCH_SIZE":
                    g["count"] += 1
                    g["us"] += (int(row["End_Timestamp"]) - int(row["Start_Timestamp"])) / 1e3
                g[counter] += float(row["Counter_Value"]) * 1024.0 * factor
            # per label: the dispatches between each pair of markers (begin,
            # end alternate: labelled launches do not nest), in launch order
            try:
                labels = json.load(open(env["VDK_TRAFFIC_LABELS"] + "." + key))
            except (OSError, ValueError):
                labels = None
            per_label, i, inside, cur = {}, 0, False, 0.0
            ok = labels is not None
            for row in sg:
                if not ok:
                    break
                if marker(row):
                    if inside:
                        if i >= len(labels):
                            ok = False
                            break
                        p = per_label.setdefault(labels[i], {"launches": 0, "bytes": 0.0})
                        p["launches"] += 1
                        p["bytes"] += cur
                        i += 1
                    inside, cur = not inside, 0.0
                elif inside:
                    cur += float(row["Counter_Value"]) * 1024.0 * factor
            if ok and i == len(labels) and not inside:
                lab = out.setdefault(key + "/labels", {})
                for name, p in per_label.items():
                    q = lab.setdefault(name, {"launches": p["launches"]})
                    q[counter] = p["bytes"]
            out.setdefault("_factors", {})[counter] = round(factor, 4)
    return out


def short_kernel_name(name):
    """A kernel trace name without its namespace and argument list (names the
    profiler left mangled: the identifier and its integer template arguments)."""
    import re
    if name.startswith("_ZN"):
        i, ident = 3, name
        while i < len(name) and name[i].isdigit():   # <length><identifier> parts of the nested name
            j = i
            while name[j].isdigit():
                j += 1
            n = int(name[i:j])
            ident, i = name[j:j + n], j + n
        rest = name[i:]
        targs = re.findall(r"L[ib](\d+)E", rest.split("EEv")[0]) if rest.startswith("I") else []
        return ident + ("<" + ", ".join(targs) + ">" if targs else "")
    name = re.sub(r"^void ", "", name)
    name = re.sub(r"\bvdk::|\(anonymous namespace\)::", "", name)
    depth, cut = 0, len(name)
    for i, ch in enumerate(name):       # the argument list: the first '(' outside template brackets
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == "(" and depth == 0:
            cut = i
            break
    return name[:cut].replace("_Float16", "half")


def traffic_table(tr, keys, path):
    """Markdown table of every (kernel, grid) group's HBM bytes per launch from
    the two counter passes, one section per workload."""
    lines = ["# HBM traffic per launch (rocprofv3 FETCH_SIZE / WRITE_SIZE)", "",
             "Made by `python bench.py " + " ".join(sys.argv[1:]) + "` on one MI355X.  Each workload ran "
             f"{1 + TRAFFIC_STEPS} batches (the first a warmup) under `rocprofv3 --pmc FETCH_SIZE` and again under "
             "`--pmc WRITE_SIZE` in a child process; each counter's KiB per dispatch is scaled by its reading for a "
             f"{TRAFFIC_COPY_MIB} MiB device-to-device copy run right after the workload "
             f"(bytes per counted byte: {tr.get('_factors')}).  Durations are from the counter runs "
             "(slower than the bench's own passes).", ""]
    for key in keys:
        groups = tr.get(key) or {}
        steps = 1 + TRAFFIC_STEPS
        lines += [f"## {key}: {MODELS[key]['config']['workload']}", "",
                  "| kernel | grid (threads) | launches / batch | us / launch | FETCH MB | WRITE MB | HBM MB / launch |",
                  "|---|---:|---:|---:|---:|---:|---:|"]
        for (name, grid), g in sorted(groups.items(), key=lambda kv: -(kv[1]["FETCH_SIZE"] + kv[1]["WRITE_SIZE"])):
            n = g["count"]
            if n == 0:
                continue
            f, w = g["FETCH_SIZE"] / n / 1e6, g["WRITE_SIZE"] / n / 1e6
            if (f + w) * n / steps < 1.0:      # under 1 MB per batch: left out
                continue
            lines.append(f"| `{short_kernel_name(name)}` | {grid} | {n / steps:g} | {g['us'] / n:.1f} | "
                         f"{f:.2f} | {w:.2f} | {f + w:.2f} |")
        lines.append("")
        lab = tr.get(key + "/labels") or {}
        if lab:
            lines += ["Per launch class (the dispatches between the marker dispatches around each labelled "
                      f"launch of the {TRAFFIC_STEPS} measured batches):", "",
                      "| class | launches / batch | FETCH MB | WRITE MB | HBM MB / launch |", "|---|---:|---:|---:|---:|"]
            for name, q in sorted(lab.items(), key=lambda kv: -(kv[1].get("FETCH_SIZE", 0) +
                                                                kv[1].get("WRITE_SIZE", 0))):
                n = q["launches"]
                f, w = q.get("FETCH_SIZE", 0.0) / n / 1e6, q.get("WRITE_SIZE", 0.0) / n / 1e6
                if (f + w) * n / TRAFFIC_STEPS < 1.0:
                    continue
                lines.append(f"| `{name}` | {n / TRAFFIC_STEPS:g} | {f:.2f} | {w:.2f} | {f + w:.2f} |")
            lines.append("")
    with open(path, "w") as fh:
        fh.write("\n".join(lines))


def traffic_of(tr, key, launches_per_step, label):
    """Measured HBM bytes per launch of `key`'s dominant class, or (None, why):
    the dispatches between the markers around that label's launches (every
    kernel and grid the class uses), else the (kernel, grid) group with that
    many launches per step (a conv kernel for a conv class) that takes the
    most time."""
    if not tr or "error" in tr:
        return None, (tr or {}).get("error", "traffic not measured")
    lab = (tr.get(key + "/labels") or {}).get(label)
    if lab and lab.get("launches") and "FETCH_SIZE" in lab and "WRITE_SIZE" in lab:
        n = lab["launches"]
        return {"kernel": f"every dispatch between the markers around the {label} launches", "grid": None,
                "fetch_bytes": lab["FETCH_SIZE"] / n, "write_bytes": lab["WRITE_SIZE"] / n,
                "factors": tr.get("_factors")}, None
    groups = tr.get(key)
    if not groups:
        return None, f"no dispatches recorded for {key}"
    want = launches_per_step * TRAFFIC_STEPS
    conv_kernel = lambda name: "conv" in name or "gemm" in name   # the kernels behind vdk_conv2d_ex
    cands = [(g["us"], name, grid, g) for (name, grid), g in groups.items()
             if g["count"] in (want, want + launches_per_step) and (not label.startswith("conv") or conv_kernel(name))]
    if not cands:
        return None, (f"no single kernel launch group with the class's {launches_per_step} launches per step "
                      "(its launches use several kernels or grids)")
    _, name, grid, g = max(cands, key=lambda c: c[0])
    n = g["count"]
    return {"kernel": name, "grid": grid, "fetch_bytes": g["FETCH_SIZE"] / n, "write_bytes": g["WRITE_SIZE"] / n,
            "factors": tr.get("_factors")}, None


def measure(L, key, steps, warmup, cpu_seconds, registry=0, copy_mib=0, b1_reps=0, traffic=None):
    """One workload: throughput over `steps` batches, a per-kernel events pass,
    the dominant kernel's roofline from an events pass over its launches only,
    the host-buffer rate, optionally the batch-1 latency and the CPU baseline."""
    model = MODELS[key]
    batch, n = model["batch"], model["n"]
    tmp = tempfile.mkdtemp()
    path = os.path.join(tmp, f"{key}.gguf")
    model["write"](path, seed=model["seed"])
    ctx = lib.Context(path)
    pcm = synth.clips(CLIP_SEED, batch, n)
    d_pcm = lib.DeviceBuffer.from_array(pcm)
    analyze = model.get("kind") == "analyze"
    width = ctx.analyze_outputs() if analyze else ctx.dim
    unit = "clips/s" if analyze else "embeddings/s"
    d_out = lib.DeviceBuffer(batch * width * 4)
    if analyze:
        run = lambda: ctx.analyze_device_async(d_pcm.ptr, batch, n, d_out.ptr)
    else:
        run = lambda: ctx.embed_device_async(d_pcm.ptr, batch, n, d_out.ptr)

    for _ in range(warmup):
        run()
    ctx.synchronize()
    lib.check(L.vdk_synchronize())
    t0 = time.perf_counter()
    for _ in range(steps):
        run()
    ctx.synchronize()
    lib.check(L.vdk_synchronize())
    elapsed = time.perf_counter() - t0
    ms_per_step = elapsed * 1e3 / steps
    value = batch * steps / elapsed
    res = d_out.to_array(np.float32, (batch, width))
    assert np.all(np.isfinite(res))
    if not analyze:
        assert np.allclose(np.linalg.norm(res, axis=1), 1.0, atol=1e-4)

    per, prof_ms = profile_pass(ctx, run, steps)
    conv = {"ms": 0.0, "flops": 0.0, "bytes": 0.0, "launches": 0}
    for name, p in per.items():
        if name.startswith("conv"):
            for k in conv:
                conv[k] += p[k]
    conv_tflops = conv["flops"] / (conv["ms"] * 1e-3) / 1e12 if conv["ms"] > 0 else 0.0
    kernels = []
    for name, p in sorted(per.items(), key=lambda kv: -kv[1]["ms"]):
        t = p["ms"] * 1e-3
        kernels.append({
            "name": name, "launches_per_step": p["launches"] // steps,
            "ms_per_step": round(p["ms"] / steps, 5),
            "tflops": round(p["flops"] / t / 1e12, 2) if p["flops"] and t > 0 else None,
            "gbs": round(p["bytes"] / t / 1e9, 1) if t > 0 else None,
        })

    # the dominant kernel, timed again with events around its launches only
    dom = max((k for k in per if k.startswith("conv")), key=lambda k: per[k]["ms"])
    recs, dom_wall_ms = dominant_pass(ctx, run, steps, dom)
    nl = len(recs)
    avg_s = sum(r[1] for r in recs) / nl * 1e-3
    fl = sum(r[2] for r in recs) / nl
    by = sum(r[3] for r in recs) / nl
    if by > 0 and fl / by >= RIDGE_FLOP_PER_BYTE:
        bound, achieved, peak, r_unit = "mfma", fl / avg_s / 1e12, PEAK_F16_TFLOPS, "TFLOP/s"
    else:
        bound, achieved, peak, r_unit = "hbm", by / avg_s / 1e9, PEAK_HBM_GBS, "GB/s"
    tinfo, twhy = traffic_of(traffic, key, nl // steps, dom)
    traffic = round(tinfo["fetch_bytes"] + tinfo["write_bytes"]) if tinfo else None
    tsrc = ({"how": "rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE passes of this run, scaled by a "
                    f"{TRAFFIC_COPY_MIB} MiB device copy", "kernel": tinfo["kernel"], "grid": tinfo["grid"],
             "fetch_bytes": round(tinfo["fetch_bytes"]), "write_bytes": round(tinfo["write_bytes"]),
             "counter_factors": tinfo["factors"]} if tinfo else {"how": "not measured", "why": twhy})
    roofline = {
        "kernel": dom, "bound": bound, "achieved": round(achieved, 2), "peak": peak, "unit": r_unit,
        "frac": round(achieved / peak, 4), "traffic": traffic, "traffic_source": tsrc,
        "launches_per_step": nl // steps, "avg_launch_us": round(avg_s * 1e6, 2),
        "flops_per_launch": fl, "algorithmic_bytes_per_launch": by,
        "traffic_over_algorithmic": round(traffic / by, 3) if traffic else None,
        "events_pass_ms_per_step": round(dom_wall_ms, 4),
        "all_conv": {"launches_per_step": conv["launches"] // steps, "ms_per_step": round(conv["ms"] / steps, 4),
                     "flops_per_step": conv["flops"] / steps, "achieved_tflops": round(conv_tflops, 2),
                     "frac": round(conv_tflops / PEAK_F16_TFLOPS, 4)},
        "all_events_pass_ms_per_step": round(prof_ms, 4),
        "kernels": kernels,
    }
    out = {"value": round(value, 2), "unit": unit, "ms_per_step": round(ms_per_step, 4), "roofline": roofline}
    # the drop-in boundary hands over host PCM: the same batch through the
    # host-buffer entry point (H2D copy of the PCM and D2H of the embeddings
    # included), reported beside `value`, never as it
    host = (lambda: ctx.analyze_pcm(pcm)) if analyze else (lambda: ctx.embed_batch(pcm))
    host()
    times = []
    for _ in range(max(5, min(steps, 15))):
        t0 = time.perf_counter()
        host()
        times.append(time.perf_counter() - t0)
    dt = float(np.median(times))   # the median call: one slow host-side call does not move it
    out["host_buffers"] = {"value": round(batch / dt, 2), "unit": unit, "ms_per_step": round(dt * 1e3, 4),
                           "calls": len(times), "min_ms": round(min(times) * 1e3, 4),
                           "note": ("voicedetect_gpu_analyze_pcm" if analyze else "voicedetect_capi_embed_pcm_batch") +
                                   ": host PCM in, host results out (PCIe included), median of the calls"}
    if b1_reps > 0 and not analyze:
        out["batch1"] = batch1_latency(ctx, pcm[0], n, b1_reps)
    if registry > 0 and not analyze:
        out["registry"] = registry_bench(L, d_out, batch, ctx.dim, registry, 10, steps)
    if cpu_seconds > 0:
        out["cpu_baseline"] = cpu_baseline(model, path, pcm, n / 16000.0, min_seconds=cpu_seconds)
    ctx.close()
    if copy_mib > 0:
        nb = copy_mib << 20
        src, dst = lib.DeviceBuffer(nb), lib.DeviceBuffer(nb)
        lib.check(L.vdk_memset(src.ptr, 1, nb))
        for _ in range(3):
            lib.check(L.vdk_memcpy_d2d(dst.ptr, src.ptr, nb))
        lib.check(L.vdk_synchronize())
        print(f"copy calibration: 3 device copies of {nb} bytes", file=sys.stderr)
    for k in kernels:
        print(f"  [{key}] {k['name']:28s} x{k['launches_per_step']:3d} {k['ms_per_step']*1e3:9.1f} us/step "
              f"{k['tflops'] or 0:8.1f} TFLOP/s {k['gbs'] or 0:8.1f} GB/s", file=sys.stderr, flush=True)
    return out


def batch1_latency(ctx, clip, n, reps):
    """One clip per call: the device-resident path (PCM already in HBM, the
    embedding left there; the call returns once the stream has finished) and
    the host-buffer path voicedetect_capi_embed_pcm (PCM in and embedding out
    through host memory); median and 90th percentile over `reps` calls."""
    d_pcm = lib.DeviceBuffer.from_array(clip[None])
    d_out = lib.DeviceBuffer(ctx.dim * 4)
    dev, hst = [], []
    for i in range(reps + 5):
        t0 = time.perf_counter()
        ctx.embed_device_async(d_pcm.ptr, 1, n, d_out.ptr)
        ctx.synchronize()
        t1 = time.perf_counter()
        ctx.embed_pcm(clip)
        t2 = time.perf_counter()
        if i >= 5:
            dev.append((t1 - t0) * 1e3)
            hst.append((t2 - t1) * 1e3)
    med = float(np.median(dev))
    return {"device_ms_median": round(med, 4), "device_ms_p90": round(float(np.percentile(dev, 90)), 4),
            "host_ms_median": round(float(np.median(hst)), 4), "host_ms_p90": round(float(np.percentile(hst, 90)), 4),
            "clips_per_s": round(1e3 / med, 1), "calls": reps,
            "reference_published": REFERENCE_PUBLISHED["resnet34_b1_ms"]}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--model", choices=sorted(MODELS), default=None,
                    help="one workload only (default: the ResNet34 B=64 headline plus the config set)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="wall time of the headline's CPU-baseline sample (the config set's get half)")
    ap.add_argument("--registry", type=int, default=0,
                    help="also time identify: the batch's embeddings scored against this many enrolled rows, top 10")
    ap.add_argument("--copy-calibration-mib", type=int, default=0,
                    help="after the bench, run 3 device-to-device copies of this many MiB (PMC traffic calibration)")
    ap.add_argument("--no-traffic", action="store_true",
                    help="skip the two rocprofv3 counter passes that measure the dominant kernels' HBM traffic")
    ap.add_argument("--traffic-table", default=None, metavar="PATH",
                    help="also write every kernel's measured HBM bytes per launch as a markdown table to PATH")
    ap.add_argument("--traffic-child", default=None, help=argparse.SUPPRESS)
    args = ap.parse_args()
    if args.traffic_child:
        traffic_child(args.traffic_child.split(","))
        return
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE {world}); "
              "clips are independent, so N GPUs would each run this same per-GPU batch.", file=sys.stderr)
        sys.exit(2)
    key = args.model or "resnet34"
    keys = [key] + ([] if args.model else list(CONFIG_SET))
    # the counter passes run first, before this process initialises the GPU
    traffic = None if args.no_traffic else traffic_passes(keys)
    if traffic and "error" in traffic:
        print(f"bench.py: traffic not measured: {traffic['error']}", file=sys.stderr)
    elif traffic and args.traffic_table:
        traffic_table(traffic, keys, args.traffic_table)
    L = lib.lib()
    if L.vdk_device_count() < 1:
        print("bench.py: no HIP device visible", file=sys.stderr)
        sys.exit(1)
    cpu_s = 0.0 if args.no_cpu_baseline else args.cpu_seconds
    head = measure(L, key, args.steps, args.warmup, cpu_s, registry=args.registry,
                   copy_mib=args.copy_calibration_mib, b1_reps=50 if key == "resnet34" else 0, traffic=traffic)
    model = MODELS[key]
    out = {
        "metric": model["metric"], "value": head["value"], "unit": head["unit"], "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": head["ms_per_step"],
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": model["dtype"],
        "data": "synthetic", "config": model["config"], "roofline": head["roofline"],
        "host_buffers": head["host_buffers"],
    }
    for k in ("registry", "cpu_baseline"):
        if k in head:
            out[k] = head[k]
    if "cpu_baseline" in out and key == "resnet34":
        out["cpu_baseline"]["reference_published"] = REFERENCE_PUBLISHED["resnet34_cpu_encoder_8t_emb_s"]
    if args.model is None:
        # every workload of the config list, measured the same way
        cfgs = [{"config": "ResNet34 batch 1 x 3 s (latency)", "model": "resnet34", "batch": 1, **head["batch1"]},
                {"config": "ResNet34 batch 64 x 3 s (the headline above)", "model": "resnet34", "batch": 64,
                 "value": head["value"], "unit": head["unit"], "ms_per_step": head["ms_per_step"],
                 "dominant_kernel": head["roofline"]["kernel"], "roofline_frac": head["roofline"]["frac"]}]
        for ck in CONFIG_SET:
            r = measure(L, ck, max(10, args.steps // 2), args.warmup, cpu_s / 2, traffic=traffic)
            m = MODELS[ck]
            e = {"config": m["config"]["workload"], "model": ck, "batch": m["batch"], "dtype": m["dtype"],
                 "value": r["value"], "unit": r["unit"], "ms_per_step": r["ms_per_step"],
                 "dominant_kernel": r["roofline"]["kernel"], "roofline": {
                     k: r["roofline"][k] for k in ("bound", "achieved", "peak", "unit", "frac", "avg_launch_us",
                                                   "traffic", "traffic_over_algorithmic", "traffic_source")},
                 "all_conv_frac": r["roofline"]["all_conv"]["frac"], "host_buffers": r["host_buffers"]["value"],
                 "reference_published_ms_per_clip": {"cpu_8t": REFERENCE_PUBLISHED["per_clip_8t_ms"][ck],
                                                     "gb10_b1": REFERENCE_PUBLISHED["gb10_b1_ms"][ck]}}
            if "cpu_baseline" in r:
                e["cpu_baseline"] = r["cpu_baseline"]
            cfgs.append(e)
        out["configs"] = cfgs
        out["reference_published_sources"] = {k: v for k, v in REFERENCE_PUBLISHED.items()
                                              if k in ("per_clip_8t_ms", "gb10_b1_ms")}
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()

"""Benchmark of the ocrs whole-page pipeline on one MI355X.

Workload (one step): 12 synthetic 300-dpi US Letter RGB pages (2550 x 3300, ~36 text lines each,
Gaussian noise sigma 4) through the whole pipeline, starting from the pages in (pageable) host
memory as the reference's run receives them: upload (pinned staging, a copy stream of its own,
overlapped with the GPU work of earlier pages), GPU grey conversion, pad and resize to 800 x 600,
the detection U-Net, the page-size mask; host words, lines and line padding; GPU line images
(64 high); the CNN + 2 x BiGRU recogniser; host CTC. Models are random-init (Kaiming, seed 0) with
the ocrs architecture; data are synthetic.

Prints one JSON line: value = pages/s over K timed steps (PCIe included), plus the same with the
pages already resident in HBM and with the pages in page-locked host memory, recognition lines/s,
the dominant kernel's roofline (HIP events on the kernel's own stream over the timed region), the
per-configuration figures (36-line recognition, the 800 x 600 detector, PP-OCR recognition), and
a CPU baseline on a bounded sample: the same page loop with the graphs on torch-CPU (the stand-in
for the reference's rten path), and the oracle's C restatement beside it.
"""
import argparse
import json
import os
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [ROOT, os.path.join(ROOT, "wgpu-ocr_amd")]

import numpy as np  # noqa: E402

METRIC = "pages/sec + ms/page (ocrs det+rec) on 1 MI355X; rec lines/sec; % roofline"
HBM_PEAK_GBS = 8000.0
F16_PEAK_TFLOPS = 2500.0


# The kernel family with the most GPU time in this workload (the per-family breakdown each run
# reports says whether it still is).
DOMINANT = "conv3x3_dma"


def roofline(kernels, traffic=True):
    """The kernel family with the most time in the timed region, against its bound. `traffic`:
    attach the rocprofv3-measured bytes a launch, which are measured on the page pipeline only."""
    fam, k = max(kernels.items(), key=lambda kv: kv[1]["ms"])
    secs = k["ms"] / 1e3
    intensity = k["flops"] / max(k["bytes"], 1.0)
    ridge = F16_PEAK_TFLOPS * 1e12 / (HBM_PEAK_GBS * 1e9)
    if k["flops"] > 0 and intensity >= ridge:
        achieved = k["flops"] / secs / 1e12
        out = {"bound": "mfma", "achieved": achieved, "peak": F16_PEAK_TFLOPS, "unit": "TFLOP/s",
               "frac": achieved / F16_PEAK_TFLOPS}
    else:
        achieved = k["bytes"] / secs / 1e9
        out = {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
               "frac": achieved / HBM_PEAK_GBS}
    calls = max(k["calls"], 1)
    out.update({"kernel": fam, "calls": k["calls"], "avg_us": 1e3 * k["ms"] / calls,
                "traffic": measured_traffic(fam) if traffic else None,
                "algorithmic_bytes_per_launch": k["bytes"] / calls, "algorithmic_flops_per_launch": k["flops"] / calls,
                # both views of the same launches: algorithmic bytes over HBM peak, algorithmic FLOPs
                # over the dense f16 matrix-core peak
                "frac_hbm": k["bytes"] / secs / (HBM_PEAK_GBS * 1e9),
                "frac_mfma_f16": k["flops"] / secs / (F16_PEAK_TFLOPS * 1e12)})
    return out


def measured_traffic(fam):
    """HBM bytes per launch of kernel family `fam` in this workload, as measured by rocprofv3
    (FETCH_SIZE + WRITE_SIZE per dispatch, scaled by the same counters on a copy of known size)
    and recorded in profiles/traffic_<family>.md as a `bytes_per_launch:` line; None if absent."""
    path = os.path.join(ROOT, "profiles", f"traffic_{fam}.md")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("bytes_per_launch:"):
                    return float(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def copy_calibration():
    """A device-to-device copy of 1 GiB, three times: the reference point for the HBM traffic
    counters (run under rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE)."""
    import torch
    n = 1 << 28
    x = torch.ones(n, dtype=torch.float32, device="cuda")
    y = torch.empty_like(x)
    for _ in range(3):
        y.copy_(x)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes": 4 * n, "copies": 3}))


def conv_layer(spec, reps=5):
    """One 3x3 convolution (+ ReLU, optional max pool) as a one-node graph: CIN,COUT,N,H,W[,PHxPW].
    Random float16-exact weights, random input; one warm-up launch, then `reps` launches with
    every kernel family probed. Prints the launch time per family (the single-layer figures and
    the single-layer counter profiles run this)."""
    import ocrhip
    from ocrhip import onnx_write as ow
    f = spec.split(",")
    cin, cout, n, h, w = (int(v) for v in f[:5])
    pool = tuple(int(v) for v in f[5].split("x")) if len(f) > 5 else None
    rng = np.random.default_rng(0)
    g = ow.Graph("layer")
    wt = g.init("w", (rng.standard_normal((cout, cin, 3, 3)) * np.sqrt(2 / (cin * 9))).astype(np.float16)
                .astype(np.float32))
    b = g.init("b", (rng.standard_normal(cout) * 0.01).astype(np.float16).astype(np.float32))
    y = g.add("Relu", [g.add("Conv", ["x", wt, b], kernel_shape=[3, 3], pads=[1, 1, 1, 1])])
    oh, ow_ = h, w
    if pool:
        y = g.add("MaxPool", [y], kernel_shape=list(pool), strides=list(pool))
        oh, ow_ = h // pool[0], w // pool[1]
    path = os.path.join(tempfile.gettempdir(), f"ocrhip_layer_{os.getpid()}.onnx")
    with open(path, "wb") as fh:
        fh.write(g.model("x", [n, cin, h, w], y, [n, cout, oh, ow_]))
    ctx = ocrhip.Context()
    graph = ocrhip.Graph(ctx, path)
    os.unlink(path)
    x = rng.standard_normal((n, cin, h, w)).astype(np.float32)
    graph.run(x)
    kern = _probed(ocrhip.FAMILIES, lambda: [graph.run(x) for _ in range(reps)])
    out = {"layer": spec, "flops": 2.0 * n * h * w * cin * cout * 9}
    for fam, k in kern.items():
        if k["calls"]:
            us = 1e3 * k["ms"] / k["calls"]
            out[fam] = {"us_per_launch": us, "launches_per_run": k["calls"] / reps,
                        "tflops": k["flops"] / k["ms"] / 1e9 if k["flops"] else None,
                        "gbps": k["bytes"] / k["ms"] / 1e6 if k["bytes"] else None}
    print(json.dumps(out))


def gru_lines(nlines, reps=5):
    """The recogniser on `nlines` synthetic lines (widths in [200, 800]) resident in device
    memory: one warm-up pass, then `reps` passes; prints the GRU's time per launch and per step."""
    import ocrhip
    from ocrhip import synth
    ctx = ocrhip.Context()
    rec = ocrhip.Recognizer(ctx, synth.model_path("rec"))
    batches, _, _ = synth.batch_lines(synth.rec_lines(nlines, seed=0, wmin=200, wmax=800))
    dev = []
    for data, n, w in batches:
        buf = ctx.alloc(data.nbytes)
        buf.upload(np.ascontiguousarray(data))
        dev.append((buf, n, w))
    tmax, ntot, _ = rec.dims(dev)
    d_best = ctx.alloc(tmax * ntot * 4)
    rec.recognize_device(dev, d_best=d_best)
    ctx.synchronize()
    kern = _probed(["gru"], lambda: [rec.recognize_device(dev, d_best=d_best) for _ in range(reps)])
    k = kern["gru"]
    us = 1e3 * k["ms"] / k["calls"]
    print(json.dumps({"lines": nlines, "steps": tmax, "gru_us_per_launch": us, "gru_us_per_step": us / tmax}))


def bandwidth(npages=16, nlines=540, reps=5):
    """The bandwidth-bound families at multi-page launch sizes (a single page's tensors are launch-
    dominated): detection of `npages` resident pages as one pass (grey_resize, the U-Net, mask_up)
    and recognition of `nlines` resident lines as one pass (conv_direct, argmax and the rest);
    prints each family's launches, average time, algorithmic bytes a launch and GB/s."""
    import ocrhip
    from ocrhip import synth
    ctx = ocrhip.Context()
    det = ocrhip.Detector(ctx, synth.model_path("det"))
    rec = ocrhip.Recognizer(ctx, synth.model_path("rec"))
    pages = [synth.page(i % 12) for i in range(npages)]
    d_pages, d_bits = [], []
    for p in pages:
        b = ctx.alloc(p.nbytes)
        b.upload(p)
        d_pages.append(b)
        d_bits.append(ctx.alloc(p.shape[0] * ((p.shape[1] + 31) // 32) * 4))
    ws, hs = [p.shape[1] for p in pages], [p.shape[0] for p in pages]
    batches, _, _ = synth.batch_lines(synth.rec_lines(nlines, seed=0, wmin=200, wmax=800))
    dev = []
    for data, n, w in batches:
        buf = ctx.alloc(data.nbytes)
        buf.upload(np.ascontiguousarray(data))
        dev.append((buf, n, w))
    tmax, ntot, _ = rec.dims(dev)
    d_best = ctx.alloc(tmax * ntot * 4)

    def step():
        det.detect_pages_device(d_pages, ws, hs, 0.5, d_bits)
        rec.recognize_device(dev, d_best=d_best)
    step()
    ctx.synchronize()
    kern = _probed(ocrhip.FAMILIES, lambda: ([step() for _ in range(reps)], ctx.synchronize()))
    out = {"workload": f"detection of {npages} resident 2550x3300 pages as one pass and recognition of {nlines} "
                       f"resident lines as one pass, {reps} times", "families": {}}
    for f, k in sorted(kern.items(), key=lambda kv: -kv[1]["ms"]):
        calls = max(k["calls"], 1)
        secs = k["ms"] / 1e3
        out["families"][f] = {"calls": k["calls"], "avg_us": 1e3 * k["ms"] / calls,
                              "algorithmic_mb_per_launch": k["bytes"] / calls / 1e6,
                              "gbps": k["bytes"] / max(secs, 1e-12) / 1e9,
                              "frac_hbm": k["bytes"] / max(secs, 1e-12) / (HBM_PEAK_GBS * 1e9),
                              "tflops": k["flops"] / max(secs, 1e-12) / 1e12}
    print(json.dumps(out))


def host_cpu():
    """The host CPU the baseline runs on: model name from /proc/cpuinfo, the cores this process
    may run on (its affinity mask) and the logical CPUs the system shows."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    affinity = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    return {"model": model, "affinity_cores": affinity, "logical_cpus": os.cpu_count()}


def baseline_threads():
    """Threads for a CPU baseline: OMP_NUM_THREADS when set (the GPU box sets it to its CPU
    share), else every core of the affinity mask, never more than the mask holds."""
    cpu = host_cpu()
    want = int(os.environ.get("OMP_NUM_THREADS", cpu["affinity_cores"]))
    return max(1, min(want, cpu["affinity_cores"])), cpu


def cpu_baseline(det_path, rec_path, pages, min_secs=10.0):
    """The oracle (C restatement, OpenMP on all host cores) page by page, as the reference's CPU
    baseline loop runs (src/bin/ocr-bench.rs:431-444): oracle detection, the oracle's layout,
    oracle line images and recognition, greedy CTC. One untimed warm-up page, then
    pages of the same workload until at least `min_secs` have passed (a bounded sample)."""
    from oracle import graph as og
    from oracle import layout as ol
    from oracle import onnx_read

    cores, cpu = baseline_threads()
    os.environ["OMP_NUM_THREADS"] = str(cores)
    det, rec = onnx_read.load(det_path), onnx_read.load(rec_path)
    og.lib()
    layout = ol.Layout
    og.page_pipeline(det, rec, pages[0], 0.5, layout)
    n, t = 0, time.perf_counter()
    while time.perf_counter() - t < min_secs and n < 4 * len(pages):
        og.page_pipeline(det, rec, pages[n % len(pages)], 0.5, layout)
        n += 1
    secs = time.perf_counter() - t
    return {"value": n / secs, "unit": "pages/s", "cores": cores, "kind": "port", "cpu": cpu,
            "sample": f"{n} of the synthetic 2550x3300 pages, whole pipeline page by page, {secs:.1f} s "
                      f"on {cores} threads of {cpu['model']} (oracle: C restatement with OpenMP, float32)"}


def cpu_baseline_torch(det_path, rec_path, pages, min_secs=10.0):
    """The same page loop with the detection and recognition graphs on torch-CPU (one library
    call per ONNX node, float32, torch's threads on all host cores): the stand-in for the
    reference's rten CPU path, which cannot run here. Grey resize, mask, layout, line crops and
    CTC are the oracle's. One untimed warm-up page, then pages until min_secs have passed."""
    import torch
    from oracle import layout as ol
    from oracle import onnx_read
    from oracle import torch_cpu

    cores, cpu = baseline_threads()
    torch.set_num_threads(cores)
    cores = torch.get_num_threads()
    det = torch_cpu.TorchGraph(onnx_read.load(det_path))
    rec = torch_cpu.TorchGraph(onnx_read.load(rec_path))
    torch_cpu.page_pipeline(det, rec, pages[0], 0.5, ol.Layout)
    n, t = 0, time.perf_counter()
    while time.perf_counter() - t < min_secs and n < 4 * len(pages):
        torch_cpu.page_pipeline(det, rec, pages[n % len(pages)], 0.5, ol.Layout)
        n += 1
    secs = time.perf_counter() - t
    return {"value": n / secs, "unit": "pages/s", "cores": cores, "kind": "port", "cpu": cpu,
            "sample": f"{n} of the synthetic 2550x3300 pages, whole pipeline page by page, {secs:.1f} s "
                      f"on {cores} threads of {cpu['model']} "
                      f"(torch {torch.__version__} CPU for the detection and recognition graphs, float32; "
                      f"the stand-in for rten)"}


def pp_pipeline(ctx, d_pages, ws, hs, merge, steps=2, host_pages=None):
    """The PP-OCR whole-page pipeline (DB detector at long side 960, threshold 0.3, host boxes,
    SVTR recogniser with the 18 708-class head) on the same pages, resident in device memory and,
    when given, from host memory (each detection pass's pages uploaded right before it, as the
    reference uploads a page in its detection path): a supplementary figure, not the headline
    value."""
    import ocrhip
    from ocrhip import synth_pp

    det = ocrhip.NdGraph(ctx, synth_pp.model_path("det"))
    rec = ocrhip.NdGraph(ctx, synth_pp.model_path("rec"), stop_before_softmax=True)
    pipe = ocrhip.PpPipeline(det, rec, merge=merge)
    pipe.run_device(d_pages, ws, hs)
    ctx.synchronize()
    lines = 0
    t = time.perf_counter()
    for _ in range(steps):
        pipe.run_device(d_pages, ws, hs)
        lines += pipe.stats()["lines"]
    ctx.synchronize()
    secs = time.perf_counter() - t
    n = steps * len(d_pages)
    out = {"workload": f"PP-OCRv6-architecture DB det + SVTR rec, {len(d_pages)} synthetic 2550x3300 pages per step",
           "pages_per_sec": n / secs, "ms_per_page": 1e3 * secs / n, "lines_per_page": lines / n,
           "rec_lines_per_sec": lines / secs, "steps": steps}
    if host_pages is not None:
        pipe.run(host_pages)
        ctx.synchronize()
        t = time.perf_counter()
        for _ in range(steps):
            pipe.run(host_pages)
        ctx.synchronize()
        hsecs = time.perf_counter() - t
        out["host_pages_per_sec"] = steps * len(host_pages) / hsecs
        out["resident_pages_per_sec"] = out["pages_per_sec"]
    return out


def _probed(families, fn):
    """Runs fn once with every family probed; returns {family: probe} for those that ran."""
    import ocrhip
    for f in families:
        ocrhip.probe_start(f)
    fn()
    out = {f: ocrhip.probe_stop(f) for f in families}
    return {f: k for f, k in out.items() if k["calls"]}


def _timed(ctx, fn, reps, warmup=3):
    for _ in range(warmup):
        fn()
    ctx.synchronize()
    t = time.perf_counter()
    for _ in range(reps):
        fn()
    ctx.synchronize()
    return (time.perf_counter() - t) / reps


# The recurrence's floor a time step: a SIMD issues the 96 v_mfma_f32_16x16x32_f16 of its four
# wavefronts (16 cycles each) at 2.4 GHz; the gate arithmetic and the step's barrier come on top.
GRU_FLOOR_US = 96 * 16 / 2400.0


def _gru_latency(k, steps):
    """The recurrence as what bounds it, the latency of a time step's dependent chain, against
    the matrix-core floor of a step (a bytes- or FLOP-rate fraction says nothing for it)."""
    us = 1e3 * k["ms"] / max(k["calls"] * steps, 1)
    secs = k["ms"] / 1e3
    return {"bound": "latency", "achieved": us, "peak": GRU_FLOOR_US, "unit": "us/step", "frac": GRU_FLOOR_US / us,
            "kernel": "gru", "calls": k["calls"], "avg_us": 1e3 * k["ms"] / max(k["calls"], 1), "steps_per_launch": steps,
            "traffic": None, "frac_hbm": k["bytes"] / secs / (HBM_PEAK_GBS * 1e9),
            "frac_mfma_f16": k["flops"] / secs / (F16_PEAK_TFLOPS * 1e12)}


def _kernel_summary(kernels, units, gru_steps=0):
    """Per-family ms per unit, the dominant family, and its roofline (algorithmic work over its
    summed launch time; for the recurrence, time a step against its floor)."""
    top = max(kernels, key=lambda f: kernels[f]["ms"])
    dom = _gru_latency(kernels[top], gru_steps) if top == "gru" and gru_steps else roofline({top: kernels[top]}, traffic=False)
    return {"kernels_ms": {f: round(k["ms"] / units, 4) for f, k in sorted(kernels.items(), key=lambda kv: -kv[1]["ms"])},
            "dominant": dom}


def config_figures(ctx, det, rec, reps=20):
    """The per-configuration figures (the reference reports them per stage: src/bin/stages.rs,
    ppocr-bench.rs): inputs resident in device memory where the entry point takes them."""
    import ocrhip
    from ocrhip import synth, synth_pp
    out = {}
    # 36 grey line images, height 64, widths uniform in [200, 800] (ocrs batching: width rounded
    # up to 50, at most 20 a batch): the CNN trunk, 2 x BiGRU(256), projection, arg-max.
    lines = synth.rec_lines(36, seed=0, wmin=200, wmax=800)
    batches, _, _ = synth.batch_lines(lines)
    dev = []
    for data, n, w in batches:
        b = ctx.alloc(data.nbytes)
        b.upload(np.ascontiguousarray(data))
        dev.append((b, n, w))
    tmax, ntot, _ = rec.dims(dev)
    d_best = ctx.alloc(tmax * ntot * 4)
    secs = _timed(ctx, lambda: rec.recognize_device(dev, d_best=d_best), reps)
    kern = _probed(ocrhip.FAMILIES, lambda: (rec.recognize_device(dev, d_best=d_best), ctx.synchronize()))
    gru = kern.get("gru", {"ms": 0.0, "calls": 0})
    out["rec_36_lines"] = {
        "workload": "36 grey lines 64 x [200, 800], ocrs batching, CNN trunk + 2 x BiGRU(256) + 97-class head",
        "ms_per_batch": 1e3 * secs, "lines_per_sec": 36 / secs, "gru_steps": 2 * tmax,
        "us_per_gru_step": 1e3 * gru["ms"] / max(gru["calls"] * tmax, 1),
        "gflop_per_batch": sum(k["flops"] for k in kern.values()) / 1e9, **_kernel_summary(kern, 1, tmax)}
    # The detection U-Net on one [1, 1, 800, 600] grey image (host in, probabilities out).
    img = synth.det_input(0)
    secs = _timed(ctx, lambda: det.detect(img), reps)
    kern = _probed(ocrhip.FAMILIES, lambda: det.detect(img))
    out["det_800x600"] = {"workload": "ocrs-architecture U-Net 16-256 on [1, 1, 800, 600] (host in and out)",
                          "ms_per_page": 1e3 * secs, "gflop_per_page": sum(k["flops"] for k in kern.values()) / 1e9,
                          **_kernel_summary(kern, 1)}
    out["pp_rec_36_lines"] = pp_rec_figure(ctx, reps)
    return out


def pp_rec_figure(ctx, reps=20):
    """PP-OCRv6-architecture recognition: 36 RGB lines 3 x 48 x [160, 960], 16 a batch, SVTR
    neck, 18 708-class CTC head (arg-max fused: the logits are never written), inputs resident."""
    import ocrhip
    from ocrhip import synth_pp
    prec = ocrhip.NdGraph(ctx, synth_pp.model_path("rec"), stop_before_softmax=True)
    pb, _ = synth_pp.batch_lines(synth_pp.rec_lines(36, seed=0))
    pdev = []
    for data, n, w in pb:
        b = ctx.alloc(data.nbytes)
        b.upload(np.ascontiguousarray(data))
        bb = ctx.alloc(int(np.prod(prec.dims(data.shape)[:-1])) * 4)
        pdev.append((b, data.shape, bb))

    def pp_rec():
        for b, shape, bb in pdev:
            prec.argmax_device(b, shape, bb)
    secs = _timed(ctx, pp_rec, reps)
    kern = _probed(ocrhip.ND_FAMILIES, lambda: (pp_rec(), ctx.synchronize()))
    return {"workload": "PP-OCRv6-architecture rec, 36 RGB lines 3 x 48 x [160, 960], 16 a batch",
            "ms_per_batch": 1e3 * secs, "lines_per_sec": 36 / secs,
            "gflop_per_batch": sum(k["flops"] for k in kern.values()) / 1e9, **_kernel_summary(kern, 1)}


def pp_only(npages, merge):
    """Only the PP-OCR figures: the whole-page pipeline on `npages` synthetic pages (resident and
    from host memory) and the 36-line recogniser batch (for kernel and counter profiles)."""
    import ocrhip
    from ocrhip import synth
    ctx = ocrhip.Context()
    pages = [synth.page(i) for i in range(npages)]
    d_pages = []
    for p in pages:
        b = ctx.alloc(p.nbytes)
        b.upload(p)
        d_pages.append(b)
    ws, hs = [p.shape[1] for p in pages], [p.shape[0] for p in pages]
    out = {"pp_pipeline": pp_pipeline(ctx, d_pages, ws, hs, merge, host_pages=pages),
           "pp_rec_36_lines": pp_rec_figure(ctx, reps=5)}
    print(json.dumps(out))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=160, help="timed steps (160 host-page steps take about 2 s)")
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--pages", type=int, default=12)
    ap.add_argument("--merge", type=int, default=6)
    ap.add_argument("--det-batch", type=int, default=3, help="pages per detection pass")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-pp", action="store_true", help="skip the PP-OCR pipeline measurement")
    ap.add_argument("--no-configs", action="store_true", help="skip the per-configuration figures")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only copy 1 GiB device to device (the reference for traffic counters)")
    ap.add_argument("--conv-layer", metavar="CIN,COUT,N,H,W[,PHxPW]",
                    help="only time one 3x3 convolution layer (+ ReLU, optional max pool)")
    ap.add_argument("--gru-lines", type=int, metavar="N", help="only time the GRU on N recognised lines")
    ap.add_argument("--bandwidth", action="store_true",
                    help="only the bandwidth-bound families at multi-page sizes: detection of 16 pages and "
                         "recognition of 540 lines, each as one pass")
    ap.add_argument("--pp-only", action="store_true",
                    help="only the PP-OCR figures: page pipeline (resident and host pages) and the 36-line "
                         "recogniser batch")
    ap.add_argument("--trace", action="store_true",
                    help="after the warm-up, run one step from host memory with the pipeline's trace "
                         "(OCR_PIPE_TRACE: upload, detection and recognition spans on the GPU, host "
                         "steps) printed to stderr, and stop")
    args = ap.parse_args()
    if args.copy_calibration:
        copy_calibration()
        return
    if args.conv_layer:
        conv_layer(args.conv_layer)
        return
    if args.gru_lines:
        gru_lines(args.gru_lines)
        return
    if args.pp_only:
        pp_only(args.pages, args.merge)
        return
    if args.bandwidth:
        bandwidth()
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: the pipeline shards by page with no exchange, so N GPUs run N "
              "independent copies with no collective; run it with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import ocrhip
    from ocrhip import synth

    det_path, rec_path = synth.model_path("det"), synth.model_path("rec")
    pages = [synth.page(i) for i in range(args.pages)]
    ctx = ocrhip.Context()
    det = ocrhip.Detector(ctx, det_path)
    rec = ocrhip.Recognizer(ctx, rec_path)
    pipe = ocrhip.Pipeline(det, rec, merge=args.merge, det_batch=args.det_batch)
    h, w = pages[0].shape[:2]
    page_bytes = sum(p.nbytes for p in pages)
    for _ in range(args.warmup):
        pipe.run(pages)
    ctx.synchronize()
    if args.trace:
        os.environ["OCR_PIPE_TRACE"] = "1"
        pipe.run(pages)
        del os.environ["OCR_PIPE_TRACE"]
        return

    # The timed region probes only the dominant kernel family (two events around each of its
    # launches, for the roofline); the per-family breakdown comes from one more step outside the
    # timed region with every family probed, so the events do not slow the timed steps.
    ocrhip.probe_start(DOMINANT)
    lines = 0
    rec_steps = 0
    cpu_busy = 0.0
    ctx.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        pipe.run(pages)
        st = pipe.stats()
        lines += st["lines"]
        rec_steps += st["rec_steps"]
        cpu_busy += st["cpu_busy_ms"]
    ctx.synchronize()
    secs = time.perf_counter() - t0
    dominant = ocrhip.probe_stop(DOMINANT)

    # The same workload for at least 2 s (a longer sample of the headline rate).
    n_sus, t_sus = 0, time.perf_counter()
    while time.perf_counter() - t_sus < 2.0:
        pipe.run(pages)
        n_sus += 1
    sus_secs = time.perf_counter() - t_sus

    # The pages already resident in HBM (no PCIe), and in page-locked host memory (no staging copy).
    d_pages = []
    for p in pages:
        b = ctx.alloc(p.nbytes)
        b.upload(p)
        d_pages.append(b)
    ws, hs = [w] * len(pages), [h] * len(pages)
    for _ in range(2):
        pipe.run_device(d_pages, ws, hs)
    ctx.synchronize()
    t1 = time.perf_counter()
    for _ in range(args.steps):
        pipe.run_device(d_pages, ws, hs)
    ctx.synchronize()
    dev_secs = time.perf_counter() - t1
    pinned = []
    for p in pages:
        a = ctx.host_array(p.shape)
        a.array[...] = p
        pinned.append(a)
    pinned_arrays = [a.array for a in pinned]
    pipe.run(pinned_arrays)
    t2 = time.perf_counter()
    for _ in range(args.steps):
        pipe.run(pinned_arrays)
    pin_secs = time.perf_counter() - t2

    for fam in ocrhip.FAMILIES:
        ocrhip.probe_start(fam)
    pipe.run(pages)
    ctx.synchronize()
    kernels = {f: ocrhip.probe_stop(f) for f in ocrhip.FAMILIES}
    kernels = {f: k for f, k in kernels.items() if k["calls"]}
    top = max(kernels, key=lambda f: kernels[f]["ms"])

    n_pages = args.steps * len(pages)
    out = {
        "metric": METRIC,
        "value": n_pages / secs,
        "unit": "pages/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": 1e3 * secs / args.steps,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": f"ocrs whole-page pipeline from host memory (PCIe included), {len(pages)} synthetic "
                               f"300-dpi US Letter RGB pages (2550x3300) per step: det U-Net 16-256 + CNN/2xBiGRU(256) "
                               f"rec, merge {args.merge}, det batch {args.det_batch}",
                   "pages_per_step": len(pages), "page": [h, w], "models": "random-init ocrs architecture"},
        "ms_per_page": 1e3 * secs / n_pages,
        "h2d_GBps": page_bytes * args.steps / secs / 1e9,
        "sustained_pages_per_sec": n_sus * len(pages) / sus_secs,
        "sustained_secs": sus_secs,
        "resident_pages_per_sec": n_pages / dev_secs,
        "pinned_host_pages_per_sec": n_pages / pin_secs,
        "rec_lines_per_sec": lines / secs,
        "lines_per_page": lines / n_pages,
        "gru_steps_per_page": rec_steps / n_pages,
        "host_busy_ms_per_page": cpu_busy / n_pages,
        "roofline": roofline({DOMINANT: dominant}),
        "dominant_in_breakdown": top,
        "kernels_ms_per_page": {f: round(k["ms"] / len(pages), 4) for f, k in
                                sorted(kernels.items(), key=lambda kv: -kv[1]["ms"])},
    }
    if not args.no_pp:
        out["pp_pipeline"] = pp_pipeline(ctx, d_pages, ws, hs, args.merge, host_pages=pages)
    if not args.no_configs:
        out["configs"] = config_figures(ctx, det, rec)
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline_torch(det_path, rec_path, pages)
        out["cpu_oracle"] = cpu_baseline(det_path, rec_path, pages)
    print(json.dumps(out))


if __name__ == "__main__":
    main()

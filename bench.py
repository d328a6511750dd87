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
the dominant kernel's roofline (HIP events on the kernel's own stream over the timed region), and
a CPU baseline (the oracle: a C / numpy restatement of the same path, on a bounded sample).
"""
import argparse
import json
import os
import sys
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


def roofline(kernels):
    """The kernel family with the most time in the timed region, against its bound."""
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
    out.update({"kernel": fam, "calls": k["calls"], "avg_us": 1e3 * k["ms"] / max(k["calls"], 1),
                "traffic": measured_traffic(fam)})
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


def cpu_baseline(det_path, rec_path, pages, min_secs=10.0):
    """The oracle (C restatement, OpenMP on all host cores) page by page, as the reference's CPU
    baseline loop runs (src/bin/ocr-bench.rs:431-444): oracle detection, the oracle's layout,
    oracle line images and recognition, greedy CTC. One untimed warm-up page, then
    pages of the same workload until at least `min_secs` have passed (a bounded sample)."""
    from oracle import graph as og
    from oracle import layout as ol
    from oracle import onnx_read

    det, rec = onnx_read.load(det_path), onnx_read.load(rec_path)
    og.lib()
    layout = ol.Layout
    og.page_pipeline(det, rec, pages[0], 0.5, layout)
    n, t = 0, time.perf_counter()
    while time.perf_counter() - t < min_secs and n < 4 * len(pages):
        og.page_pipeline(det, rec, pages[n % len(pages)], 0.5, layout)
        n += 1
    secs = time.perf_counter() - t
    cores = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    return {"value": n / secs, "unit": "pages/s", "cores": cores, "kind": "port",
            "sample": f"{n} of the synthetic 2550x3300 pages, whole pipeline page by page, {secs:.1f} s "
                      f"(oracle: C restatement with OpenMP, float32)"}


def pp_pipeline(ctx, d_pages, ws, hs, merge, steps=2):
    """The PP-OCR whole-page pipeline on the same resident pages (DB detector at long side 960,
    threshold 0.3, host boxes, SVTR recogniser with the 18 708-class head): a supplementary
    figure, not the headline value."""
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
    return {"workload": f"PP-OCRv6-architecture DB det + SVTR rec, {len(d_pages)} synthetic 2550x3300 pages per step",
            "pages_per_sec": n / secs, "ms_per_page": 1e3 * secs / n, "lines_per_page": lines / n,
            "rec_lines_per_sec": lines / secs, "steps": steps}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--pages", type=int, default=12)
    ap.add_argument("--merge", type=int, default=6)
    ap.add_argument("--det-batch", type=int, default=2, help="pages per detection pass")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-pp", action="store_true", help="skip the PP-OCR pipeline measurement")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only copy 1 GiB device to device (the reference for traffic counters)")
    args = ap.parse_args()
    if args.copy_calibration:
        copy_calibration()
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
        out["pp_pipeline"] = pp_pipeline(ctx, d_pages, ws, hs, args.merge)
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(det_path, rec_path, pages)
    print(json.dumps(out))


if __name__ == "__main__":
    main()

#!/usr/bin/env python3
"""Throughput of the GPU path on one MI355X, as one JSON line.

value: detector images/s on 1x3x960x960 (the synthetic PP-OCR mobile DB
detector plan, weights N(0, 0.05)), inputs resident in HBM, `--steps`
forward passes timed with HIP events on the model's stream after
`--warmup` untimed ones. Beside it: recogniser lines/s on batches of 16
lines of 3x48x320 (weights N(0, 0.02), 18385 classes, CTC argmax), the
fused depthwise block on 1x96x160x160, the layer microkernels, the
roofline of the dominant launch of the detector, and the CPU oracle timed
on this host on a bounded sample.
"""
from __future__ import annotations

import argparse
import importlib.util
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
# The page pipeline runs four streams at once (the detector's and three
# recogniser handles'); with HIP's default of four hardware queues a
# process puts five streams (the null stream too) on four queues, and the
# two that share one run their work in turn: a page took 1.75 ms there and
# 1.50 ms with eight queues (the detector and recogniser, one stream each,
# are the same either way). HIP reads this once, when it starts.
if int(os.environ.get("GPU_MAX_HW_QUEUES", "4")) < 8:
    os.environ["GPU_MAX_HW_QUEUES"] = "8"
PEAK_HBM_GBS = 8000.0
PEAK_FP32_MFMA_TFLOPS = 157.3
GEMM_LAUNCHES = {"pointwise_gemm", "conv_gemm", "conv_patch", "convt_gemm", "ctc_gemm"}
# Launches whose products run as FP32 fused multiply-adds on the vector ALUs
# (in the CPU engine's order), scored against the unpacked FP32 vector rate:
# 256 CUs x 4 SIMDs x 16 lanes x 2 flops x 2.4 GHz (packed FP32 is not used).
PEAK_FP32_VALU_TFLOPS = 78.6
VALU_LAUNCHES = {"stem_block"}
# HBM bytes per launch measured with rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE,
# scaled by a plain copy kernel's counters (x2.0 / x1.0), for the launches
# the bench reports a roofline of: (kernel, plan operations) -> (read, write)
# KiB and the profile summary the numbers come from.
MEASURED_TRAFFIC = {("conv_patch", (65, 71, 77, 83)): (32559, 9209, "profiles/hbm_counters_detector_recognizer.md"),
                    ("conv_patch", (94,)): (9102, 5400, "profiles/hbm_counters_detector_recognizer.md")}


def package():
    d = ROOT / "ppocr-native_amd"
    spec = importlib.util.spec_from_file_location("ppocr_native_amd", d / "__init__.py",
                                                  submodule_search_locations=[str(d)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["ppocr_native_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def roofline(name: str, flops: float, nbytes: float, ms: float) -> dict:
    """A launch's achieved rate against MI355X's peak for its class. A GEMM
    is also scored against its attainable roof, min(FP32-MFMA peak,
    arithmetic intensity x HBM peak): a thin 1x1 layer cannot reach the MFMA
    peak whatever the kernel does."""
    if name in GEMM_LAUNCHES and flops > 0:
        ach = flops / (ms * 1e-3) / 1e12
        roof = min(PEAK_FP32_MFMA_TFLOPS, flops / max(nbytes, 1.0) * PEAK_HBM_GBS / 1e3)
        return {"bound": "mfma", "achieved": round(ach, 3), "peak": PEAK_FP32_MFMA_TFLOPS,
                "unit": "TFLOP/s", "frac": round(ach / PEAK_FP32_MFMA_TFLOPS, 4),
                "attainable": round(roof, 3), "frac_attainable": round(ach / roof, 4)}
    if name in VALU_LAUNCHES and flops > 0:
        ach = flops / (ms * 1e-3) / 1e12
        return {"bound": "valu", "achieved": round(ach, 3), "peak": PEAK_FP32_VALU_TFLOPS,
                "unit": "TFLOP/s", "frac": round(ach / PEAK_FP32_VALU_TFLOPS, 4)}
    ach = nbytes / (ms * 1e-3) / 1e9
    return {"bound": "hbm", "achieved": round(ach, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
            "frac": round(ach / PEAK_HBM_GBS, 4)}


def profile(model, repeats: int) -> list[dict]:
    names = model.launches()
    ops = model.launch_ops()
    work = model.launch_work()
    times = model.profile_launches(repeats)
    rows = []
    for (name, op), members, (fl, by), ms in zip(names, ops, work, times):
        r = {"name": name, "op": op, "ops": members, "ms": ms, "flops": fl, "bytes": by}
        r.update(roofline(name, fl, by, ms))
        rows.append(r)
    return rows


def launch_label(r: dict) -> str:
    """A launch's kernel and plan operations (a grouped launch runs several)."""
    ops = r.get("ops") or [r["op"]]
    if len(ops) == 1:
        return f"{r['name']} (op {ops[0]})"
    return f"{r['name']} x{len(ops)} (ops {', '.join(str(o) for o in ops)})"


def by_kernel(rows: list[dict]) -> dict:
    agg: dict = {}
    for r in rows:
        a = agg.setdefault(r["name"], {"launches": 0, "ms": 0.0, "flops": 0.0, "bytes": 0.0})
        a["launches"] += 1
        a["ms"] += r["ms"]
        a["flops"] += r["flops"]
        a["bytes"] += r["bytes"]
    out = {}
    for k, a in sorted(agg.items(), key=lambda kv: -kv[1]["ms"]):
        rl = roofline(k, a["flops"], a["bytes"], a["ms"])
        out[k] = {"launches": a["launches"], "ms": round(a["ms"], 4), "achieved": rl["achieved"],
                  "unit": rl["unit"], "frac": rl["frac"]}
        if "frac_attainable" in rl:
            out[k]["frac_attainable"] = rl["frac_attainable"]
    return out


def time_model(model, steps: int, warmup: int) -> tuple[float, float]:
    """(device ms per step, wall ms per step) of resident runs."""
    model.run_resident(warmup)
    t0 = time.perf_counter()
    ms = model.run_resident(steps)
    wall = (time.perf_counter() - t0) * 1e3
    return ms / steps, wall / steps


def bench_detector(P, nets, steps, warmup):
    plan = nets.detector_plan(h=960, w=960, init="baseline")
    g = P.GpuModel.load(plan)
    g.input_mut()[:] = nets.page_image(960, 960).reshape(-1)
    g.upload()
    ms, wall = time_model(g, steps, warmup)
    g.set_graphs(False)
    eager_ms, _ = time_model(g, steps, warmup)
    g.set_graphs(True)
    # With the host copies of run() (pinned memory, PCIe), for reference.
    g.run()
    t0 = time.perf_counter()
    n = max(5, steps // 4)
    for _ in range(n):
        g.run()
    pcie_ms = (time.perf_counter() - t0) * 1e3 / n
    rows = profile(g, 20)
    g.close()
    return plan, ms, wall, pcie_ms, rows, eager_ms


def bench_recognizer(P, nets, steps, warmup):
    plan = nets.recognizer_plan(init="baseline")
    g = P.GpuModel.load(plan)
    lines = nets.line_images(16)
    g.set_sizes([(48, 320)] * 16)
    for i in range(16):
        g.lane_input_mut(i)[:] = lines[i].reshape(-1)
    g.upload()
    ms, wall = time_model(g, steps, warmup)
    g.set_graphs(False)
    eager_ms, _ = time_model(g, steps, warmup)
    rows = profile(g, 20)
    g.close()
    return plan, ms, wall, rows, eager_ms


def bench_block(P, nets, steps, warmup):
    plan = nets.fused_block_plan()
    g = P.GpuModel.load(plan)
    g.input_mut()[:] = np.random.default_rng(5).uniform(-1, 1, 160 * 160 * 96).astype(np.float32)
    g.upload()
    ms, _ = time_model(g, steps, warmup)
    # The same runs launched eagerly, for reference: three short launches,
    # where a graph replay's fixed cost weighs most.
    g.set_graphs(False)
    eager_ms, _ = time_model(g, steps, warmup)
    g.set_graphs(True)
    rows = profile(g, 20)
    g.close()
    flops = sum(r["flops"] for r in rows)
    # Compulsory bytes: the block's input read once and its output written
    # once (weights are a few hundred KB and stay in cache).
    compulsory = 2 * 160 * 160 * 96 * 4
    rate = compulsory / (ms * 1e-3) / 1e9
    return {"workload": "fused dw3x3+SE+pw block 1x96x160x160", "ms": round(ms, 4),
            "eager_ms": round(eager_ms, 4),
            "gflops_per_s": round(flops / (ms * 1e-3) / 1e9, 1),
            "compulsory_bytes": compulsory,
            "compulsory_gb_per_s": round(rate, 1),
            "compulsory_frac": round(rate / PEAK_HBM_GBS, 4),
            "compulsory_floor_ms": round(compulsory / (PEAK_HBM_GBS * 1e9) * 1e3, 4),
            "launches": by_kernel(rows)}


def bench_micro(P, repeats: int = 20) -> dict:
    """The layer microkernels at the benchmark's sizes. `warm`: one set of
    buffers, called back to back (small ones stay in the 256 MB last-level
    cache). `cold`: the calls rotate over enough sets of buffers (over 256 MB
    in all) that each call reads its inputs from HBM."""
    from ppocr_native_amd.devmem import DeviceArray, Timer
    rng = np.random.default_rng(0)
    out = {}
    MALL = 256 << 20

    def timeit(fns):
        for fn in fns[:2]:
            fn()
        t = Timer()
        t.start()
        for k in range(repeats):
            fns[k % len(fns)]()
        return t.stop() / repeats

    def sets(nbytes):
        return max(1, -(-(MALL + (64 << 20)) // nbytes))

    def both(name, make, nbytes, per_set_bytes, frac=True):
        warm = timeit([make(0)])
        cold = timeit([make(k) for k in range(sets(per_set_bytes))])
        r = {"ms": round(warm, 4), "gb_per_s": round(nbytes / warm / 1e6, 1),
             "cold_ms": round(cold, 4), "cold_gb_per_s": round(nbytes / cold / 1e6, 1)}
        if frac:
            r["frac_hbm"] = round(nbytes / warm / 1e6 / PEAK_HBM_GBS, 3)
            r["cold_frac_hbm"] = round(nbytes / cold / 1e6 / PEAK_HBM_GBS, 3)
        out[name] = r

    n = 240 * 240 * 256
    # Two sets of inputs and outputs: 354 MB, past the last-level cache.
    A = [DeviceArray.of(rng.uniform(-1, 1, n).astype(np.float32)) for _ in range(2)]
    B = [DeviceArray.of(rng.uniform(-1, 1, n).astype(np.float32)) for _ in range(2)]
    Y = [DeviceArray(4 * n) for _ in range(2)]
    for name, call, nbytes in [
        # A plain copy (activation code 0): the reference for HBM counters.
        ("copy 1x256x240x240", lambda k: lambda: P.hip_activation(A[k % 2].addr, Y[k % 2].addr, n, 0), 8 * n),
        ("add 1x256x240x240", lambda k: lambda: P.hip_add(A[k % 2].addr, B[k % 2].addr, Y[k % 2].addr, n), 12 * n),
        ("mul 1x256x240x240", lambda k: lambda: P.hip_mul(A[k % 2].addr, B[k % 2].addr, Y[k % 2].addr, n), 12 * n),
        ("hardswish 1x256x240x240", lambda k: lambda: P.hip_activation(A[k % 2].addr, Y[k % 2].addr, n, 7), 8 * n),
    ]:
        both(name, call, nbytes, nbytes)
    del A, B, Y
    px, c = 3600, 480
    ns = sets(8 * px * c)
    X = [DeviceArray.of(rng.uniform(-1, 1, px * c).astype(np.float32)) for _ in range(ns)]
    YY = [DeviceArray(4 * px * c) for _ in range(ns)]
    g = DeviceArray.of(rng.uniform(-1, 1, c).astype(np.float32))
    both("mean 1x480x60x60", lambda k: lambda: P.hip_channel_mean(X[k].addr, YY[k].addr, px, c),
         4 * px * c + 4 * c, 8 * px * c)
    both("channel_mul 1x480x60x60", lambda k: lambda: P.hip_channel_mul(X[k].addr, g.addr, YY[k].addr, px, c),
         8 * px * c, 8 * px * c)
    del X, YY
    rows, cc = 1280, 120
    ns = sets(8 * rows * cc)
    XL = [DeviceArray.of(rng.uniform(-1, 1, rows * cc).astype(np.float32)) for _ in range(ns)]
    YL = [DeviceArray(4 * rows * cc) for _ in range(ns)]
    wl = DeviceArray.of(np.concatenate([np.ones(cc), np.zeros(cc), [1e-6]]).astype(np.float32))
    both("layernorm 1280x120", lambda k: lambda: P.hip_layer_norm(XL[k].addr, wl.addr, YL[k].addr, rows, cc),
         8 * rows * cc, 8 * rows * cc)
    del XL, YL
    cols = 18385
    nb = 4 * rows * cols
    ns = sets(nb)
    XA = [DeviceArray.of(rng.normal(0, 3, rows * cols).astype(np.float32)) for _ in range(ns)]
    ya = DeviceArray(8 * rows)
    both("row_argmax 1280x18385", lambda k: lambda: P.hip_row_argmax(XA[k].addr, ya.addr, rows, cols),
         nb + 8 * rows, nb)
    del XA
    return out


def bench_stages(P, nets, repeats: int = 20) -> dict:
    """The stages either side of the networks: GPU image kernels on a
    2550x3300 page (letter at 300 dpi) resident in HBM, and the host DB and
    CTC steps on this host's CPU."""
    import ctypes as C
    from ppocr_native_amd import images, post
    from ppocr_native_amd.devmem import DeviceArray, Timer, synchronize
    L = images._sig()
    rng = np.random.default_rng(3)
    out = {}

    def timeit(fn):
        fn()
        synchronize()
        t = Timer()
        t.start()
        for _ in range(repeats):
            fn()
        return t.stop() / repeats

    ph, pw = 3300, 2550
    page = rng.integers(0, 256, (ph, pw, 3), dtype=np.uint8)
    dpage = DeviceArray.of(page.reshape(-1))
    oh, ow = 960, 736
    dinp = DeviceArray(4 * oh * ow * 3)
    m, sd = (C.c_double * 3)(*images.MEAN), (C.c_double * 3)(*images.STD)
    ms = timeit(lambda: L.ppocr_hip_det_input(dpage.addr, pw, ph, dinp.addr, ow, oh, m, sd, None))
    # Bytes the kernel must move: the f32 tensor written and, at most, the
    # page rows and columns its taps touch (2 source rows x 2 columns per
    # output pixel, less where neighbours share them).
    nb = 4 * oh * ow * 3 + min(ph, 2 * oh) * min(pw, 2 * ow) * 3
    out["det_input 2550x3300 -> 736x960"] = {"ms": round(ms, 4), "gb_per_s": round(nb / ms / 1e6, 1),
                                             "frac_hbm": round(nb / ms / 1e6 / PEAK_HBM_GBS, 3),
                                             "bytes": nb}
    # 16 tilted line crops of about 600 x 40 pixels, then their recogniser inputs.
    quads = []
    for i in range(16):
        x, y, w, h, t = 100 + 7 * i, 200 + 180 * i, 600 + 10 * i, 40, 0.02 * (i - 8)
        c, s = np.cos(t), np.sin(t)
        quads.append(np.asarray([[x, y], [x + w * c, y + w * s], [x + w * c - h * s, y + w * s + h * c],
                                 [x - h * s, y + h * c]], np.float32))
    sizes = [images.crop_size(q) for q in quads]
    dcrop = [DeviceArray(cw * ch * 3) for cw, ch in sizes]
    widths = [images.rec_width(cw, ch)[0] for cw, ch in sizes]
    dins = [DeviceArray(4 * 48 * wd * 3) for wd in widths]
    ow_, oh_ = C.c_size_t(), C.c_size_t()
    qps = [q.ctypes.data_as(C.POINTER(C.c_float)) for q in quads]

    def crops():
        for q, d, (cw, ch) in zip(qps, dcrop, sizes):
            L.ppocr_hip_crop_text(dpage.addr, pw, ph, q, d.addr, cw * ch * 3, C.byref(ow_), C.byref(oh_), None)

    ms = timeit(crops)
    px = sum(cw * ch for cw, ch in sizes)
    out["crop_text 16 lines"] = {"ms": round(ms, 4), "pixels": px,
                                 "gb_per_s": round(px * 3 * 2 / ms / 1e6, 1)}
    wd_ = C.c_size_t()

    def rec_inputs():
        for d, di, (cw, ch), wd in zip(dcrop, dins, sizes, widths):
            L.ppocr_hip_rec_input(d.addr, cw, ch, di.addr, 48 * wd * 3, C.byref(wd_), None)

    ms = timeit(rec_inputs)
    out["rec_input 16 lines"] = {"ms": round(ms, 4), "floats": sum(48 * w * 3 for w in widths)}
    # Host: DB boxes of the 320x320 reference map and of a 960x960 map, and
    # CTC decode of 16 lines of 80 steps.
    gold = ROOT / "tests" / "golden"
    prob = np.load(gold / "prob.npy", allow_pickle=False)
    t0 = time.perf_counter()
    for _ in range(repeats):
        boxes = post.boxes_from_prob(prob, 320, 320, 325, 323)
    out["db_boxes 320x320 (host)"] = {"ms": round((time.perf_counter() - t0) * 1e3 / repeats, 4),
                                      "boxes": int(boxes.shape[0])}
    big = np.kron(prob, np.ones((3, 3), np.float32))
    t0 = time.perf_counter()
    for _ in range(5):
        boxes = post.boxes_from_prob(big, 960, 960, 2550, 3300)
    out["db_boxes 960x960 (host)"] = {"ms": round((time.perf_counter() - t0) * 1e3 / 5, 4),
                                      "boxes": int(boxes.shape[0])}
    # The same from the threshold as row bitmasks (what the detector's run
    # hands the host with its DB mask set): the host's border following
    # starts from the pixels where a row's bits change.
    bits = post.pack_rows(big > np.float32(0.3))
    t0 = time.perf_counter()
    for _ in range(5):
        boxes = post.boxes_from_bits(big, bits, 960, 960, 2550, 3300)
    out["db_boxes_bits 960x960 (host)"] = {"ms": round((time.perf_counter() - t0) * 1e3 / 5, 4),
                                           "boxes": int(boxes.shape[0])}
    d = post.Dictionary.from_metadata((gold / "characters.txt").read_text(encoding="utf-8"))
    pairs = [np.stack([rng.integers(0, 18710, 80).astype(np.float32),
                       rng.uniform(0.5, 1, 80).astype(np.float32)], 1) for _ in range(16)]
    t0 = time.perf_counter()
    for _ in range(repeats):
        for q in pairs:
            post.ctc_decode_pairs(q, d)
    out["ctc_decode 16 lines x 80 steps (host)"] = {
        "ms": round((time.perf_counter() - t0) * 1e3 / repeats, 4)}
    return out


def page_plans(nets):
    """The page pipeline's networks: the detector graph at 736 x 960 with
    its ink path set (the boxes land on the page's lines) and the
    recogniser with scaled seeded weights (non-trivial text)."""
    return nets.detector_plan(h=960, w=736, init="ink"), nets.recognizer_plan(init="scaled")


def bench_page(P, nets, repeats: int = 10) -> dict:
    """The page pipeline on a 2550 x 3300 letter page with 44 text lines:
    detector input, detector, DB boxes (host), crops, recogniser inputs,
    recogniser in batches of 16 and CTC text (host)."""
    from ppocr_native_amd import post
    from ppocr_native_amd.devmem import DeviceArray
    from ppocr_native_amd.pipeline import PagePipeline
    gold = ROOT / "tests" / "golden"
    d = post.Dictionary.from_metadata((gold / "characters.txt").read_text(encoding="utf-8"))
    page = nets.letter_page()
    H, W = page.shape[:2]
    det_plan, rec_plan = page_plans(nets)
    pipe = PagePipeline(det_plan, rec_plan, d)
    dpage = DeviceArray.of(page.reshape(-1))
    for _ in range(3):
        lines = pipe.read_device(dpage.addr, W, H)
    # One page at a time (its detector, then boxes, then its batches on three
    # recogniser handles at once), then `repeats` pages in one call, each
    # page's detector queued while the page before is read.
    stages = {"detect": 0.0, "boxes": 0.0, "read": 0.0, "decode": 0.0}
    t0 = time.perf_counter()
    for _ in range(repeats):
        lines = pipe.read_device(dpage.addr, W, H)
        for k in stages:
            stages[k] += getattr(pipe.times, k) / repeats
    single_ms = (time.perf_counter() - t0) * 1e3 / repeats
    pipe.read_pages([(dpage.addr, W, H)] * 2)
    t0 = time.perf_counter()
    lines = pipe.read_pages([(dpage.addr, W, H)] * repeats)[-1]
    ms = (time.perf_counter() - t0) * 1e3 / repeats
    t0 = time.perf_counter()
    for _ in range(3):
        pipe.read(page)
    up_ms = (time.perf_counter() - t0) * 1e3 / 3
    out = {"metric": "pages/s and lines/s, 2550x3300 letter page, 44 lines, detector at 736x960, "
                     "recogniser 48x320 in batches of 16",
           "pages_per_s": round(1e3 / ms, 2), "lines_per_s": round(len(lines) * 1e3 / ms, 1),
           "ms_per_page": round(ms, 3), "lines": len(lines), "batches": pipe.times.batches[:3],
           "one_page_at_a_time_pages_per_s": round(1e3 / single_ms, 2),
           "stages_ms": {k: round(v, 3) for k, v in stages.items()},
           "with_page_upload_pages_per_s": round(1e3 / up_ms, 2),
           "text_chars": sum(len(x.text) for x in lines)}
    pipe.close()
    return out


def cpu_page(nets, threads: int) -> dict:
    """The same page on the CPU path: the oracle's stages, host boxes and
    decode; one page."""
    sys.path.insert(0, str(ROOT))
    import oracle
    from ppocr_native_amd import post
    gold = ROOT / "tests" / "golden"
    d = post.Dictionary.from_metadata((gold / "characters.txt").read_text(encoding="utf-8"))
    page = nets.letter_page()
    H, W = page.shape[:2]
    det_plan, rec_plan = page_plans(nets)
    det, rec = oracle.OracleModel(det_plan), oracle.OracleModel(rec_plan)
    det.set_size(960, 736)
    rec.set_size(48, 320)
    mean, std = (0.485, 0.456, 0.406), (0.229, 0.224, 0.225)
    t0 = time.perf_counter()
    prob = det.run(oracle.det_input(page, 736, 960, mean, std), threads)[0]
    quads = post.boxes_from_prob(prob, 736, 960, W, H)
    for q in quads:
        post.ctc_decode_pairs(rec.run(oracle.rec_input(oracle.crop_text(page, q), 320), threads)[0], d)
    s = time.perf_counter() - t0
    return {"value": round(1 / s, 4), "unit": "pages/s", "lines_per_s": round(len(quads) / s, 2),
            "cores": threads, "kind": "port",
            "sample": f"one page of {len(quads)} lines through the C oracle's stages, {threads} threads"}


def cpu_threads() -> tuple[int, int]:
    """(threads for the all-cores run, nproc): the cores this process may
    run on, at most OMP_NUM_THREADS (the CPU share a one-GPU box gives)."""
    nproc = len(os.sched_getaffinity(0))
    cap = int(os.environ.get("OMP_NUM_THREADS", nproc) or nproc)
    return max(1, min(nproc, cap)), nproc


def cpu_runs(fn, budget_s: float, want: int = 20, least: int = 3) -> tuple[float, float, int]:
    """Median wall seconds and median process CPU seconds of calls of fn:
    `want` calls, fewer (at least `least`) when they would overrun budget_s."""
    fn()
    walls, cpus = [], []
    t_start = time.perf_counter()
    while len(walls) < want and (len(walls) < least or time.perf_counter() - t_start < budget_s):
        t0, c0 = time.perf_counter(), time.process_time()
        fn()
        walls.append(time.perf_counter() - t0)
        cpus.append(time.process_time() - c0)
    return float(np.median(walls)), float(np.median(cpus)), len(walls)


def cpu_baseline(nets, det_plan, rec_plan, budget_s: float) -> tuple[dict, dict]:
    """The C oracle (the engine's CPU path at the AVX2+FMA tier's summation
    orders, vectorised across outputs) on this host: one thread pinned to
    one core, and all the cores this process may use, as the reference's
    benches time its CPU path (tools/bench_ocr_abba.py:32-43,
    examples/plan.rs:57-90): medians of repeated runs, wall and process CPU
    time."""
    sys.path.insert(0, str(ROOT))
    import oracle
    threads, nproc = cpu_threads()
    m = oracle.OracleModel(det_plan)
    img = nets.page_image(960, 960)
    r = oracle.OracleModel(rec_plan)
    lines = nets.line_images(16)
    k = [0]

    def line(th):
        r.run(lines[k[0] % 16], th)
        k[0] += 1

    res = {}
    affinity = os.sched_getaffinity(0)
    one = min(affinity)
    os.sched_setaffinity(0, {one})
    try:
        res["det1"] = cpu_runs(lambda: m.run(img, 1), budget_s * 0.5)
        res["rec1"] = cpu_runs(lambda: line(1), budget_s * 0.1)
    finally:
        os.sched_setaffinity(0, affinity)
    res["detN"] = cpu_runs(lambda: m.run(img, threads), budget_s * 0.3)
    res["recN"] = cpu_runs(lambda: line(threads), budget_s * 0.1)

    def entry(key1, keyN, unit, per, what):
        w1, c1, n1 = res[key1]
        wN, cN, nN = res[keyN]
        return {"value": round(per / wN, 3), "unit": unit, "cores": threads, "kind": "port",
                "nproc": nproc, "one_thread_value": round(per / w1, 3),
                "cpu_s_per_unit": round(cN / per, 4), "one_thread_cpu_s_per_unit": round(c1 / per, 4),
                "sample": f"{what}: median of {nN} runs on {threads} OpenMP threads (nproc {nproc}) and of "
                          f"{n1} runs on one thread pinned to core {one}; C oracle, tier-3 FMA order"}

    return (entry("det1", "detN", "img/s", 1.0, "detector forwards at 1x3x960x960"),
            entry("rec1", "recN", "lines/s", 1.0, "recogniser lines of 3x48x320, one line a run"))


def trace_runs(P, nets, which: str, runs: int) -> None:
    """For rocprofv3 counter and kernel-trace runs: `runs` eager passes of
    one workload, inputs resident, then its launch list (kernel, plan
    operations, layer FLOPs and algorithmic bytes), one JSON line each, in
    dispatch order. `copy` is the plain copy kernel (activation code 0) over
    1x256x240x240 floats that HBM counters are scaled by; `copy_lds` the same
    copy through LDS by direct loads, the scale for kernels that load so."""
    if which in ("copy", "copy_lds"):
        from ppocr_native_amd.devmem import DeviceArray, synchronize
        n = 240 * 240 * 256
        a = DeviceArray.of(np.random.default_rng(0).uniform(-1, 1, n).astype(np.float32))
        y = DeviceArray(4 * n)
        for _ in range(runs):
            if which == "copy":
                P.hip_activation(a.addr, y.addr, n, 0)
            else:
                P.hip_copy_lds(a.addr, y.addr, n)
        synchronize()
        print(json.dumps({"name": which, "ops": [], "flops": 0, "bytes": 8 * n}), flush=True)
        return
    if which == "det":
        g = P.GpuModel.load(nets.detector_plan(h=960, w=960, init="baseline"))
        g.input_mut()[:] = nets.page_image(960, 960).reshape(-1)
    elif which == "rec":
        g = P.GpuModel.load(nets.recognizer_plan(init="baseline"))
        lines = nets.line_images(16)
        g.set_sizes([(48, 320)] * 16)
        for i in range(16):
            g.lane_input_mut(i)[:] = lines[i].reshape(-1)
    else:
        g = P.GpuModel.load(nets.fused_block_plan())
        g.input_mut()[:] = np.random.default_rng(5).uniform(-1, 1, 160 * 160 * 96).astype(np.float32)
    g.set_graphs(False)
    g.upload()
    g.run_resident(runs)
    for (name, _), ops, (fl, by) in zip(g.launches(), g.launch_ops(), g.launch_work()):
        print(json.dumps({"name": name, "ops": ops, "flops": fl, "bytes": by}), flush=True)
    g.close()


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--cpu-seconds", type=float, default=30.0)
    ap.add_argument("--only", choices=["det", "rec", "all"], default="all")
    ap.add_argument("--trace", choices=["det", "rec", "block", "copy", "copy_lds"],
                    help="only run --trace-runs eager passes of one workload (for rocprofv3) "
                         "and print its launch list")
    ap.add_argument("--trace-runs", type=int, default=3)
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: the GPU path shards by page and by line batch with "
              f"no exchange, and no multi-GPU figure is asked for (got --gpus {args.gpus})",
              file=sys.stderr)
        return 2
    P = package()
    from ppocr_native_amd import nets
    if args.trace:
        trace_runs(P, nets, args.trace, args.trace_runs)
        return 0

    log("bench: detector 1x3x960x960")
    det_plan, det_ms, det_wall, pcie_ms, det_rows, det_eager = bench_detector(P, nets, args.steps,
                                                                              args.warmup)
    dom = max(det_rows, key=lambda r: r["ms"])
    result = {
        "metric": "det img/s @960², rec lines/s @16×3×48×320; % of HBM / FP32-MFMA roofline",
        "value": round(1e3 / det_ms, 2),
        "unit": "img/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(det_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "PP-OCR mobile-style DB detector forward, 1x3x960x960 synthetic "
                               "page, seeded N(0,0.05) weights (synthetic PPOCRPL1 plan)",
                   "batch": 1, "height": 960, "width": 960},
        "roofline": {k: dom[k] for k in ("bound", "achieved", "peak", "unit", "frac") if k in dom}
                    | {k: dom[k] for k in ("attainable", "frac_attainable") if k in dom},
        "wall_ms_per_step": round(det_wall, 4),
        "eager_ms_per_step": round(det_eager, 4),
        "with_host_copies_img_per_s": round(1e3 / pcie_ms, 2),
    }
    measured = MEASURED_TRAFFIC.get((dom["name"], tuple(dom["ops"])))
    result["roofline"]["traffic"] = (measured[0] + measured[1]) * 1024 if measured else None
    if measured:
        result["roofline"]["traffic_source"] = measured[2]
        result["roofline"]["algorithmic_bytes"] = round(dom["bytes"])
    result["roofline"]["kernel"] = launch_label(dom)
    result["roofline"]["launch_ms"] = round(dom["ms"], 5)
    result["det_kernels"] = by_kernel(det_rows)
    result["det_launches"] = [[r["name"], r["ops"], round(r["ms"] * 1e3, 1), r["frac"], r.get("frac_attainable")]
                              for r in det_rows]
    if args.only in ("rec", "all"):
        log("bench: recogniser 16x3x48x320")
        rec_plan, rec_ms, rec_wall, rec_rows, rec_eager = bench_recognizer(P, nets, args.steps,
                                                                           args.warmup)
        rdom = max(rec_rows, key=lambda r: r["ms"])
        result["rec"] = {"metric": "rec lines/s @16x3x48x320", "value": round(16e3 / rec_ms, 1),
                         "unit": "lines/s", "ms_per_batch": round(rec_ms, 4),
                         "eager_ms_per_batch": round(rec_eager, 4),
                         "roofline": {k: rdom[k] for k in ("bound", "achieved", "peak", "unit", "frac",
                                                           "attainable", "frac_attainable") if k in rdom}
                         | {"kernel": launch_label(rdom)},
                         "kernels": by_kernel(rec_rows),
                         "launches": [[r["name"], r["ops"], round(r["ms"] * 1e3, 1), r["frac"],
                                       r.get("frac_attainable")] for r in rec_rows]}
        log("bench: fused block, microkernels")
        result["block"] = bench_block(P, nets, args.steps, args.warmup)
        result["micro"] = bench_micro(P)
        log("bench: stages either side of the networks")
        result["stages"] = bench_stages(P, nets)
        log("bench: page pipeline 2550x3300")
        result["page"] = bench_page(P, nets)
    else:
        rec_plan = nets.recognizer_plan(init="baseline")
    if not args.no_cpu:
        log("bench: CPU oracle baseline")
        det_cpu, rec_cpu = cpu_baseline(nets, det_plan, rec_plan, args.cpu_seconds)
        result["cpu_baseline"] = det_cpu
        if "rec" in result:
            result["rec"]["cpu_baseline"] = rec_cpu
        if "page" in result:
            log("bench: CPU page")
            result["page"]["cpu_baseline"] = cpu_page(nets, det_cpu["cores"])
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

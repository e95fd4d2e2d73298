"""Benchmark of the quantized-weight products on one MI355X.

Headline (BASELINE.json metric): int4 GEMM HBM GB/s at M=1 on the 27B-scale decode layer set:
(K, N) = (5120, 17408) x 2, (17408, 5120), (5120, 6144), (6144, 5120) symmetric int4 group 128, plus the int4
output head K=5120, N=248320 (argmax epilogue). A step is one pass over FOUR distinct device copies of the layer set
(680 MB, beyond the 256 MB MALL) and the head, captured once in a HIP graph and replayed; value = algorithmic bytes
of the step / step time. Extra lines: the same at M=5, the prefill GEMM at M=2048 in TFLOP/s, W8A16 at M=1.

Algorithmic bytes per product: int4 K N / 2 + (K / 128) N 2 [+ (K / 128) N / 2 zero points] + M K 2 + M N 2;
int8 K N + 2 N + 2 M K + 2 M N. Flops 2 M N K.
"""

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK = 8000.0  # GB/s, MI355X
BF16_PEAK = 2500.0  # TFLOP/s dense, MI355X

SET_27B = [(5120, 17408), (5120, 17408), (17408, 5120), (5120, 6144), (6144, 5120)]
HEAD_27B = (5120, 248320)
PREFILL_27B = [(5120, 17408), (17408, 5120), (5120, 6144)]


def int4_bytes(k, n, m, zp=False):
    return k * n // 2 + (k // 128) * n * 2 + ((k // 128) * n // 2 if zp else 0) + m * k * 2 + m * n * 2


def int8_bytes(k, n, m):
    return k * n + 2 * n + 2 * m * k + 2 * m * n


def quant(seed, kind, k, n):
    """A synthetic stored matrix [n][k] in the checkpoint's form: 'i4' symmetric int4, 'i4z' int4 with packed zero
    points, 'i8' per-channel int8, 'i8g' int8 with a scale per row and 128 columns (qwenny_amd.synth)."""
    from qwenny_amd import synth
    from qwenny_amd.checkpoint import quant_from_packed

    name = f"{kind}_{n}_{k}"
    if kind in ("i8", "i8g"):
        g = 128 if kind == "i8g" else 0
        t = synth.int8_quant(seed, name, n, k, group=g)
        return quant_from_packed(t["weight_packed"], synth.bf16_to_f32(t["weight_scale"]), 8, g, None,
                                 t["weight_shape"])
    t = synth.int4_quant(seed, name, n, k, zp=kind == "i4z")
    return quant_from_packed(t["weight_packed"], synth.bf16_to_f32(t["weight_scale"]), 4, 128,
                             t.get("weight_zero_point"), t["weight_shape"])


def upload_copies(gemm, q, copies):
    """`copies` distinct device matrices of the same packed data."""
    from qwenny_amd._lib import check, lib
    from qwenny_amd.core import Mat, P, Wt, pack_quant
    import ctypes

    z = q.zero_points()
    wt = Wt.I8 if q.bits == 8 else (Wt.I4 if (z == 8).all() else Wt.I4Z)
    order = np.arange(q.rows)
    codes, scales, zs = pack_quant(q, order, wt, None if wt != Wt.I4Z else z)
    mats = []
    for _ in range(copies):
        h = P()
        check(lib().qh_mat_upload(gemm._ctx, int(wt), q.rows, q.cols, codes.ctypes.data, scales.ctypes.data,
                                  None if zs is None else zs.ctypes.data, q.rows, ctypes.byref(h)))
        mats.append(Mat(gemm, h))
    return mats


class Step:
    """A list of product launches (mat, m, epi, bytes, flops) with their buffers, replayable as a HIP graph."""

    def __init__(self, gemm, m, kmax):
        import torch

        self.gemm, self.m = gemm, m
        self.launches = []
        self.x = torch.randn(max(m, 1), kmax, device="cuda").to(torch.bfloat16)
        self.keys = torch.zeros(max(m, 64), dtype=torch.int64, device="cuda")
        # the logit rows of an argmax product, gathered as the engine passes them (Step::out_rows)
        self.out_rows = torch.arange(max(m, 1), dtype=torch.int32, device="cuda")
        self.ys = {}

    def add(self, mat, epi, nbytes, flops):
        import torch

        from qwenny_amd import Epi

        rows = mat.rows
        split = mat.split(self.m) if epi == Epi.Plain else 1
        key = (rows, split, epi)
        if key not in self.ys:
            self.ys[key] = torch.empty(split * self.m * rows, dtype=torch.float32, device="cuda")
        self.launches.append((mat, epi, self.ys[key], nbytes, flops))

    def run(self, stream=None):
        from qwenny_amd import Epi

        for mat, epi, y, _, _ in self.launches:
            if epi == Epi.Argmax:
                self.gemm.run(stream, self.m, mat, self.x, y, epi, out_rows=self.out_rows, n_out=self.m, keys=self.keys)
            else:
                self.gemm.run(stream, self.m, mat, self.x, y, epi)

    def bytes(self):
        return sum(b for *_, b, _ in self.launches)

    def flops(self):
        return sum(f for *_, f in self.launches)


def time_step(step, steps, warmup, graph=True, per_graph=10, min_reps=100, stats=None):
    """ms per step: the MEDIAN over at least `min_reps` timed repetitions (whatever `steps` is), each repetition timed
    with its own pair of HIP events on the launching stream, after `warmup` untimed steps. With `graph`, the step's
    launches are captured `per_graph` times into one HIP graph (so that a replay's own start-up, about 20 us, is
    spread over that many steps) and one repetition is one replay; else one repetition is one eager step. `stats`
    (a dict) receives the mean and the spread of the repetitions and the steps timed."""
    import torch

    stream = torch.cuda.current_stream()
    if graph:
        per_graph = max(1, min(per_graph, steps))
        step.run()  # the kernels' first launches outside the capture
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        with torch.cuda.stream(s):
            with torch.cuda.graph(g, stream=s):
                for _ in range(per_graph):
                    step.run(s)
        torch.cuda.synchronize()
        go = g.replay
        warm = max(1, warmup // per_graph)
    else:
        go, warm, per_graph = step.run, warmup, 1
    reps = max(min_reps, -(-steps // per_graph))
    for _ in range(warm):
        go()
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
    ev[0].record(stream)
    for i in range(reps):
        go()
        ev[i + 1].record(stream)
    torch.cuda.synchronize()
    per = np.array([ev[i].elapsed_time(ev[i + 1]) for i in range(reps)]) / per_graph
    if stats is not None:
        stats.update({"reps": reps, "steps_timed": reps * per_graph, "mean_ms": float(per.mean()),
                      "p10_ms": float(np.percentile(per, 10)), "p90_ms": float(np.percentile(per, 90))})
    return float(np.median(per))


def cpu_baseline(budget_s=12.0):
    """The reference's CPU form (Quant::row_into to f32 then an f32 dot, threaded over rows) on the host cores, on a
    bounded sample of the headline workload: whole passes over the 27B layer set at M=1 until `budget_s` is spent."""
    import oracle
    from qwenny_amd.synth import activations

    threads = min(os.cpu_count() or 1, 16)
    qs = [quant(100 + i, "i4", k, n) for i, (k, n) in enumerate(SET_27B)]
    xs = {k: activations(9, "x", 1, k) for k, _ in SET_27B}
    done_bytes, t0, passes = 0, time.perf_counter(), 0
    while True:
        for q, (k, n) in zip(qs, SET_27B):
            oracle.gemm_f32(4, 128, q.q, q.scales, q.offsets, xs[k], threads=threads)
            done_bytes += int4_bytes(k, n, 1)
        passes += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    return {"value": round(done_bytes / el / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "host_cpus": os.cpu_count(), "host_cpus_usable": len(os.sched_getaffinity(0)),
            "sample": f"{passes} pass(es) over the 27B decode layer set (5 matrices, 170.5 MB) at M=1, "
                      f"scalar C restatement of Quant::row_into + f32 dot, {threads} threads, {el:.1f} s"}


TRAFFIC_NAME = "skinny_i4_m1_27b_set"
COPY_BYTES = 512 << 20  # the calibration copy: reads and writes this many bytes


def load_traffic(name):
    """HBM bytes per launch from the committed rocprofv3 --pmc summary, if there is one for this workload."""
    p = os.path.join(ROOT, "profiles", f"{name}_traffic.json")
    if os.path.exists(p):
        with open(p) as f:
            return json.load(f).get("traffic_bytes_per_launch")
    return None


def traffic_run(gemm, set_mats, steps=5):
    """The workload of the rocprofv3 --pmc passes: the roofline kernel's launches (27B set at M=1, plain, no graph)
    and two calibrations of the counters over COPY_BYTES: a plain torch copy (reads and writes COPY_BYTES) and
    qh_diag_read's contiguous pass (reads COPY_BYTES with the decode kernel's own non-temporal 16-byte loads)."""
    import torch

    from qwenny_amd import Epi

    from qwenny_amd.core import diag_read

    src = torch.empty(COPY_BYTES, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    # the read-only kernel with the decode kernel's own 16-byte non-temporal loads over the same known bytes
    sink = torch.zeros(1, dtype=torch.int32, device="cuda")
    for _ in range(3):
        diag_read(None, src, COPY_BYTES >> 10, 1, 0, sink)
    st = Step(gemm, 1, 17408)
    for c in range(4):
        for mats, (k, n) in zip(set_mats, SET_27B):
            st.add(mats[c], Epi.Plain, int4_bytes(k, n, 1), 2 * k * n)
    for _ in range(steps):
        st.run()
    torch.cuda.synchronize()
    print(json.dumps({"traffic_run": "done", "launches": steps * len(st.launches), "algorithmic_bytes_per_launch":
                      st.bytes() / len(st.launches)}))


def summarize_traffic(fetch_dir, write_dir, out_name=TRAFFIC_NAME):
    """From the two rocprofv3 --pmc CSVs (FETCH_SIZE, then WRITE_SIZE, KiB per dispatch): the copy kernel's readings
    give the scale factors (known bytes / reading), the skinny kernel's mean readings scaled by them give its HBM bytes
    per launch. Writes profiles/<out_name>_traffic.json."""
    import csv
    import glob

    def readings(d, counter):
        out = {}
        for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            for r in csv.DictReader(open(f)):
                if r["Counter_Name"] != counter:
                    continue
                name = r["Kernel_Name"]
                kind = "diag" if "diag_read_kernel" in name else (
                    "copy" if ("copy" in name.lower() and "skinny" not in name) else (
                        "skinny" if ("skinny_kernel" in name or "skinny_m1_kernel" in name) else None))
                if kind:
                    out.setdefault(kind, []).append(float(r["Counter_Value"]))
        return out

    fetch, write = readings(fetch_dir, "FETCH_SIZE"), readings(write_dir, "WRITE_SIZE")
    mean = lambda v: sum(v) / len(v)
    # the copy: the largest readings are the full copies (torch may launch small copies too)
    fcopy, wcopy = max(fetch["copy"]), max(write["copy"])
    cfac, wfac = COPY_BYTES / (fcopy * 1024), COPY_BYTES / (wcopy * 1024)
    # the fetch scale from the read with the skinny kernel's own loads (the torch copy's, beside it, cross-checks it)
    fdiag = max(fetch["diag"]) if fetch.get("diag") else None
    ffac = COPY_BYTES / (fdiag * 1024) if fdiag else cfac
    fk, wk = mean(fetch["skinny"]) * 1024 * ffac, mean(write["skinny"]) * 1024 * wfac
    res = {"kernel": "skinny_m1_kernel (int4 plain M=1), 27B layer set (5 shapes x 4 copies)",
           "fetch_kib_per_dispatch": mean(fetch["skinny"]), "write_kib_per_dispatch": mean(write["skinny"]),
           "copy_fetch_kib": fcopy, "copy_write_kib": wcopy, "copy_bytes": COPY_BYTES,
           "diag_read_fetch_kib": fdiag, "copy_fetch_scale": cfac,
           "fetch_scale": ffac, "write_scale": wfac, "traffic_bytes_per_launch": round(fk + wk),
           "fetch_bytes_per_launch": round(fk), "write_bytes_per_launch": round(wk)}
    os.makedirs(os.path.join(ROOT, "profiles"), exist_ok=True)
    with open(os.path.join(ROOT, "profiles", f"{out_name}_traffic.json"), "w") as f:
        json.dump(res, f, indent=1)
    print(json.dumps(res))


class ReadStep:
    """The read floor of the roofline launches: qh_diag_read's tile-layout pass (pattern 1: the one-token plain
    product's loads, partition and block walk) over buffers the size of each matrix's codes, replayable like Step."""

    def __init__(self, shapes, copies):
        import torch

        self.bufs = [(torch.empty(k * n // 2, dtype=torch.uint8, device="cuda"), n // 16, k // 128)
                     for _ in range(copies) for k, n in shapes]
        self.sink = torch.zeros(1, dtype=torch.int32, device="cuda")
        self.launches = self.bufs

    def run(self, stream=None):
        from qwenny_amd.core import diag_read

        for buf, tiles, groups in self.bufs:
            diag_read(stream, buf, tiles, groups, 1, self.sink)


def read_floor(set_mats, args):
    """Per launch, the time a read-only pass with the plain M=1 product's own loads and partition takes over the same
    code bytes (no activations, scales, arithmetic or stores): the floor a product launch cannot go under on this part
    (its launch and ramp included)."""
    st = ReadStep(SET_27B, 4)
    ms = time_step(st, args.steps, args.warmup, not args.no_graph)
    per = ms * 1e-3 / len(st.launches)
    code = sum(k * n // 2 for k, n in SET_27B) / len(SET_27B)
    shapes = {}
    for k, n in SET_27B[1:]:
        one = ReadStep([(k, n)], 4)
        shapes[f"{k}x{n}"] = round(time_step(one, args.steps, args.warmup, not args.no_graph) * 1e3 / 4, 3)
    algo = sum(int4_bytes(k, n, 1) for k, n in SET_27B) / len(SET_27B)
    out = {"us_per_launch": round(per * 1e6, 3), "code_GBps": round(code / per / 1e9, 1),
           "frac_at_algorithmic_bytes": round(algo / per / 1e9 / HBM_PEAK, 4), "us_per_shape": shapes}
    print(f"# read floor (diag read, the M=1 product's loads over its code bytes): {per * 1e6:.2f} us per launch, "
          f"{code / per / 1e9:.1f} GB/s of codes; per shape {shapes} us", file=sys.stderr, flush=True)
    return out


CLOCK_NAME = "prefill_i4_m2048_27b_clock_mfma_busy"


def load_clock(name=CLOCK_NAME):
    """The committed rocprofv3 clock / MFMA-busy summary of the prefill kernels, if there is one."""
    p = os.path.join(ROOT, "profiles", f"{name}.json")
    if os.path.exists(p):
        with open(p) as f:
            return json.load(f)
    return None


def roofline_prefill(extra):
    """The MFMA half of the metric: the int4 prefill kernel at M=2048 on (5120, 17408), plain, symmetric; achieved
    TFLOP/s from this run's HIP-event timing, MFMA busy and clock from the committed profile of the same launch."""
    tf = extra["prefill_m2048_TFLOPs"]["5120x17408"]
    flops = 2 * 2048 * 5120 * 17408
    out = {"bound": "mfma", "achieved": tf, "peak": BF16_PEAK, "unit": "TFLOP/s", "frac": round(tf / BF16_PEAK, 4),
           "kernel": "prefill_kernel<int4, plain> 256 x 256 items (ping-pong), M=2048, (K, N) = (5120, 17408)",
           "flops_per_launch": flops, "us_per_launch": round(flops / (tf * 1e12) * 1e6, 2)}
    clk = load_clock()
    if clk:
        row = clk.get("5120x17408")
        if row:
            out.update({"profile_us_per_launch": row["us"], "profile_clock_GHz": row["clock_GHz"],
                        "mfma_busy": row["mfma_busy"]})
    return out


def dense_weights(seed, n, k):
    """Synthetic dense bf16 weights [n][k] ~ N(0, 0.05^2)."""
    from qwenny_amd.synth import f32_to_bf16

    rng = np.random.default_rng(seed)
    return f32_to_bf16((rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.05)))


def dense_lines(gemm, args):
    """The dense 16-bit products (Wt::F16 rows, kept bf16): M = 1 over (5120, 17408) and (17408, 5120) in 4 device
    copies (HBM GB/s), and M = 2048 on (5120, 17408) (TFLOP/s) beside torch's bf16 product of the same shape."""
    import torch

    from qwenny_amd import Epi, Mat

    shapes = [(5120, 17408), (17408, 5120)]
    mats = []
    for i, (k, n) in enumerate(shapes):
        w = dense_weights(400 + i, n, k)
        mats.append([Mat.new(gemm, w, k, int8=False) for _ in range(4)])
        del w
    st = Step(gemm, 1, 17408)
    for c in range(4):
        for m, (k, n) in zip(mats, shapes):
            st.add(m[c], Epi.Plain, k * n * 2 + 2 * k + 2 * n, 2 * k * n)
    ms = time_step(st, args.steps, args.warmup, not args.no_graph)
    out = {"bf16_dense_m1_GBps": round(st.bytes() / (ms * 1e-3) / 1e9, 1)}
    k, n = shapes[0]
    pst = Step(gemm, 2048, k)
    pst.add(mats[0][0], Epi.Plain, k * n * 2 + 2048 * (k + n) * 2, 2 * 2048 * k * n)
    msp = time_step(pst, max(10, args.steps // 10), 3, not args.no_graph)
    out["bf16_dense_prefill_m2048_TFLOPs"] = round(pst.flops() / (msp * 1e-3) / 1e12, 1)
    a = torch.randn(2048, k, device="cuda").to(torch.bfloat16)
    b = torch.randn(n, k, device="cuda").to(torch.bfloat16)
    for _ in range(3):
        a @ b.t()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    reps = max(10, args.steps // 10)
    t0.record()
    for _ in range(reps):
        a @ b.t()
    t1.record()
    torch.cuda.synchronize()
    out["torch_bf16_prefill_m2048_TFLOPs"] = round(2 * 2048 * k * n / (t0.elapsed_time(t1) / reps * 1e-3) / 1e12, 1)
    print(f"# dense bf16 M=1: {ms:.4f} ms/step, {out['bf16_dense_m1_GBps']} GB/s; M=2048 (5120x17408): "
          f"{out['bf16_dense_prefill_m2048_TFLOPs']} TFLOP/s (torch {out['torch_bf16_prefill_m2048_TFLOPs']})",
          file=sys.stderr, flush=True)
    return out


def dequant_line(args):
    """The trainer's dequant of a whole (5120, 17408) int4 group-128 matrix in the checkpoint layout to bf16 rows,
    rotating 4 device copies of the input: HBM GB/s over words + f32 scales + u8 zeros read and bf16 written."""
    import torch

    from qwenny_amd import dequant

    k, n = 5120, 17408
    q = quant(500, "i4", k, n)
    z = q.zero_points()
    ins = [(torch.from_numpy(q.q).cuda(), torch.from_numpy(q.scales).cuda(), torch.from_numpy(z).cuda())
           for _ in range(4)]
    out = torch.empty((n, k), dtype=torch.int16, device="cuda")
    words = q.q.shape[1]
    run = lambda i: dequant(None, ins[i][0], ins[i][1], ins[i][2], n, words, k, 128, 4, 0, n, out)
    for i in range(4):
        run(i)
    torch.cuda.synchronize()
    reps = max(20, args.steps // 5)
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for i in range(reps):
        run(i % 4)
    t1.record()
    torch.cuda.synchronize()
    s = t0.elapsed_time(t1) / reps * 1e-3
    nbytes = n * words * 4 + q.scales.size * 4 + z.size + n * k * 2
    gbs = round(nbytes / s / 1e9, 1)
    print(f"# dequant (5120, 17408) int4 -> bf16: {s * 1e6:.1f} us, {gbs} GB/s", file=sys.stderr, flush=True)
    return {"dequant_i4_to_bf16_GBps": gbs}


SET_4B = [(2560, 4096), (4096, 2560), (2560, 1024), (2560, 9728), (2560, 9728), (9728, 2560)]


def set4b_line(gemm, args):
    """the 4B-scale layer set, int4 with packed zero points, at M = 1, 2, 4, 5 and 8, 12 distinct
    device copies (590 MB per pass, beyond the 256 MB MALL), HIP graphs: HBM GB/s over the algorithmic bytes."""
    from qwenny_amd import Epi

    mats = [upload_copies(gemm, quant(600 + i, "i4z", k, n), 12) for i, (k, n) in enumerate(SET_4B)]
    out = {}
    for m in (1, 2, 4, 5, 8):
        st = Step(gemm, m, 9728)
        for c in range(12):
            for ms_, (k, n) in zip(mats, SET_4B):
                st.add(ms_[c], Epi.Plain, int4_bytes(k, n, m, zp=True), 2 * m * k * n)
        ms = time_step(st, args.steps, args.warmup, not args.no_graph)
        out[f"m{m}_GBps"] = round(st.bytes() / (ms * 1e-3) / 1e9, 1)
        print(f"# 4B set with zero points M={m}: {ms * 1e3 / len(st.launches):.2f} us per launch, "
              f"{out[f'm{m}_GBps']} GB/s", file=sys.stderr, flush=True)
    return {"set4b_i4z": out}


def consumers_line(args):
    """The partials consumers and the LoRA epilogue at 27B sizes, after the down projection (K 17408 -> 5120 rows) and
    on [gate; up] (34816 rows, rank 16): M = 1 (34 split-K partials) and M = 2048 (one). HBM GB/s over the bytes each
    reads and writes once; microseconds per launch (these launches are short: the launch and its ramp dominate)."""
    import torch

    from qwenny_amd import add_rmsnorm, lora_add, lora_silu, sum_parts

    out = {}
    hid, gu, rank, mcols = 5120, 34816, 16, 64
    g = torch.Generator(device="cuda").manual_seed(7)
    b = (torch.randn(gu, rank, device="cuda", generator=g) * 0.05).half().view(torch.int16)
    tab_add = torch.tensor([2**31 - 1] * 4 + [0, -1, -1, -1], dtype=torch.int32, device="cuda")
    tab_silu = torch.tensor([2**31 - 1] * 4 + [0, rank, -1, -1], dtype=torch.int32, device="cuda")
    scale = torch.tensor([1.0], dtype=torch.float32, device="cuda")
    for m, split in ((1, 34), (1, 1), (2048, 1)):
        x = torch.randn(split, m, hid, device="cuda", generator=g)
        h = torch.randn(m, hid, device="cuda", generator=g)
        w = torch.ones(hid, device="cuda")
        yb = torch.empty(m, hid, dtype=torch.bfloat16, device="cuda")
        ys = torch.empty(m, hid, device="cuda")
        xa = torch.randn(1, m, mcols, device="cuda", generator=g)
        slot = torch.zeros(m, dtype=torch.int32, device="cuda")
        ygu = torch.randn(m, gu, device="cuda", generator=g)
        mid = torch.empty(m, gu // 2, dtype=torch.bfloat16, device="cuda")
        cases = {
            "sum_parts": (lambda: sum_parts(None, x, split, m, hid, ys), (split + 1) * m * hid * 4),
            "add_rmsnorm": (lambda: add_rmsnorm(None, h, x, split, m, hid, w, yb),
                            (split + 2) * m * hid * 4 + hid * 4 + m * hid * 2),
            "lora_add": (lambda: lora_add(None, xa, 1, mcols, b, rank, hid, tab_add, slot, scale, m, ys),
                         m * mcols * 4 + hid * rank * 2 * -(-m // 16) + 2 * m * hid * 4),
            "lora_silu": (lambda: lora_silu(None, xa, 1, mcols, b, rank, gu, tab_silu, slot, scale, m, ygu, mid),
                          m * mcols * 4 + gu * rank * 2 * -(-m // 16) + m * gu * 4 + m * gu),
        }
        for name, (fn, nbytes) in cases.items():
            if split == 1 and m == 1 and name not in ("add_rmsnorm", "sum_parts"):
                continue  # one partial at M = 1: the residual step's cost without the split-K partials
            for _ in range(3):
                fn()
            torch.cuda.synchronize()
            # 20 launches per HIP graph, replayed: the kernels' own time plus the graph's per-launch cost
            graph, st = torch.cuda.CUDAGraph(), torch.cuda.Stream()
            with torch.cuda.stream(st):
                with torch.cuda.graph(graph, stream=st):
                    for _ in range(20):
                        fn()
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            reps = 10
            t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            t0.record()
            for _ in range(reps):
                graph.replay()
            t1.record()
            torch.cuda.synchronize()
            s = t0.elapsed_time(t1) / (reps * 20) * 1e-3
            key = f"{name}_m{m}" + ("_split1" if m == 1 and split == 1 else "")
            out[key] = {"us": round(s * 1e6, 2), "GBps": round(nbytes / s / 1e9, 1)}
            print(f"# {key}: {s * 1e6:.2f} us, {nbytes / s / 1e9:.1f} GB/s", file=sys.stderr, flush=True)
    return {"consumers": out}


class LayerStep:
    """One 27B decode layer's quantized products at M = 1 as the engine runs them, each with the consumer of its
    output (4 device copies): the attention in-projection (5120 -> 6144) as whole rows (one partial, for attn_prep;
    measured faster than its split product followed by the sum of the partials); the out-projection (6144 -> 5120)
    and the down projection (17408 -> 5120), plain, each then the residual step (add_rmsnorm over its partials, which
    reads many partials for little more than one: faster than a whole-row product there); [gate; up] (5120 -> 2 x
    17408) with the SwiGLU epilogue (whole sums, no partials)."""

    def __init__(self, gemm, set_mats, gate_up):
        import torch

        self.gemm = gemm
        self.x = torch.randn(1, 17408, device="cuda").to(torch.bfloat16)
        self.h = torch.randn(1, 5120, device="cuda")
        self.w = torch.ones(5120, device="cuda")
        self.yb = torch.empty(1, 5120, dtype=torch.bfloat16, device="cuda")
        self.mid = torch.empty(1, 17408, dtype=torch.bfloat16, device="cuda")
        self.parts = {}
        self.launches = []
        for c in range(4):
            for mat, kind in ((set_mats[3][c], "in"), (set_mats[4][c], "res"), (gate_up[c], "silu"),
                              (set_mats[2][c], "res")):
                split = mat.split(1) if kind == "res" else 1
                if (mat.rows, split) not in self.parts:
                    self.parts[(mat.rows, split)] = torch.empty(split, 1, mat.rows, device="cuda")
                self.launches.append((mat, kind, self.parts[(mat.rows, split)]))

    def run(self, stream=None):
        from qwenny_amd import Epi, add_rmsnorm

        for mat, kind, y in self.launches:
            if kind == "silu":
                self.gemm.run(stream, 1, mat, self.x, self.mid, Epi.Silu)
                continue
            if kind == "in":
                self.gemm.run_split(stream, 1, mat, self.x, y, Epi.Plain, True)
                continue
            split = self.gemm.run(stream, 1, mat, self.x, y, Epi.Plain)
            add_rmsnorm(stream, self.h, y, split, 1, 5120, self.w, self.yb)

    def bytes(self):
        k, n = 5120, 2 * 17408  # [gate; up]: int4 codes and scales, x once, bf16 output of n / 2 rows
        gate_up = k * n // 2 + (k // 128) * n * 2 + 2 * k + (n // 2) * 2
        return 4 * (int4_bytes(5120, 6144, 1) + int4_bytes(6144, 5120, 1) + gate_up + int4_bytes(17408, 5120, 1))


def layer_line(gemm, set_mats, args):
    """The decode layer as the engine runs it (LayerStep): HBM GB/s over the products' algorithmic bytes, beside the
    products alone (the same products, no consumers)."""
    from qwenny_amd import Mat

    gate, up = quant(100, "i4", 5120, 17408), quant(101, "i4", 5120, 17408)
    gate_up = [Mat.stack(gemm, [gate, up], silu=True) for _ in range(4)]
    st = LayerStep(gemm, set_mats, gate_up)
    ms = time_step(st, args.steps, args.warmup, not args.no_graph)
    out = {"ms_per_step": round(ms, 5), "GBps": round(st.bytes() / (ms * 1e-3) / 1e9, 1)}
    print(f"# decode layer x4 as the engine runs it (products + consumers): {ms:.4f} ms, {out['GBps']} GB/s",
          file=sys.stderr, flush=True)
    return {"m1_layer_with_consumers": out}


class SummedStep(Step):
    """A Step of one plain product followed, when it returns several partials, by their sum (`sum_parts`): a product
    of split 1 is already the sum and has no consumer launch."""

    def __init__(self, gemm, m, kmax, mat):
        import torch

        super().__init__(gemm, m, kmax)
        self.split = mat.split(m)
        self.sum = torch.empty(m * mat.rows, dtype=torch.float32, device="cuda")

    def run(self, stream=None):
        from qwenny_amd import sum_parts

        super().run(stream)
        if self.split > 1:
            mat, _, y, _, _ = self.launches[0]
            sum_parts(stream, y, self.split, self.m, mat.rows, self.sum)


def short_prefill_line(gemm, set_mats, args):
    """Plain int4 products of 40, 64, 256 and 512 tokens on the 27B prefill shapes (K slices or stream-K, whichever the
    launcher picks; at 40 tokens (5120, 17408) and (17408, 5120) take the prefill kernel, (5120, 6144) the skinny
    kernel), in HIP graphs: TFLOP/s of the product alone, and of the product followed by the sum of its
    partials (sum_parts, only when the split is above 1), with the split used."""
    from qwenny_amd import Epi

    out = {}
    for m in (40, 64, 256, 512):
        for i, (k, n) in enumerate(PREFILL_27B):
            mat = set_mats[[0, 2, 3][i]][0]
            alone = Step(gemm, m, k)
            alone.add(mat, Epi.Plain, int4_bytes(k, n, m), 2 * m * k * n)
            ms_a = time_step(alone, max(50, args.steps), 5, not args.no_graph)
            st = SummedStep(gemm, m, k, mat)
            st.add(mat, Epi.Plain, int4_bytes(k, n, m), 2 * m * k * n)
            ms = time_step(st, max(50, args.steps), 5, not args.no_graph)
            tf_a = alone.flops() / (ms_a * 1e-3) / 1e12
            tf = st.flops() / (ms * 1e-3) / 1e12
            out[f"m{m}_{k}x{n}"] = {"TFLOPs": round(tf_a, 1), "TFLOPs_with_sum": round(tf, 1), "split": st.split}
            print(f"# prefill M={m} K={k} N={n}: {ms_a * 1e3:.1f} us alone ({tf_a:.1f} TFLOP/s), "
                  f"{ms * 1e3:.1f} us with the sum ({tf:.1f}), split {st.split}", file=sys.stderr, flush=True)
    return {"prefill_short_TFLOPs": out}


def lora_line(gemm, args):
    """An unmerged rank-16 LoRA adapter on the 27B [gate; up] (34816 x 5120, SwiGLU) and down (5120 x 17408, plain)
    products at M = 1 and 2048, HIP graphs: the adapter fused into the product's epilogue (qh_gemm_lora) against the
    reference's sequence (the plain product, then lora_silu over its f32 [gate; up] output, or lora_add on its split
    0), with the product without adapter beside them; microseconds per product."""
    import torch

    from qwenny_amd import Epi, lora_add, lora_silu

    rank = 16
    gu = upload_copies(gemm, quant(690, "i4", 5120, 34816), 4)
    dn = upload_copies(gemm, quant(691, "i4", 17408, 5120), 4)
    g = torch.Generator(device="cuda").manual_seed(11)
    out = {}
    for m, copies in ((1, 4), (2048, 1)):
        xg = torch.randn(m, 17408, device="cuda").to(torch.bfloat16)
        res = {}
        for name, mats, rows, k in (("gate_up_silu", gu, 34816, 5120), ("down_plain", dn, 5120, 17408)):
            silu = name.startswith("gate")
            cols = 2 * rank
            xa = torch.randn(1, m, cols, device="cuda", generator=g)
            b = (torch.randn(rows, rank, device="cuda", generator=g) * 0.05).half().view(torch.int16)
            tab = torch.tensor([2**31 - 1] * 4 + [0, rank if silu else -1, -1, -1], dtype=torch.int32, device="cuda")
            slot = torch.zeros(m, dtype=torch.int32, device="cuda")
            scale = torch.tensor([1.0], dtype=torch.float32, device="cuda")
            lora = (xa, 1, cols, b, rank, tab, slot, scale)
            split = mats[0].split(m)
            yf = torch.empty(split * m * rows, dtype=torch.float32, device="cuda")
            mid = torch.empty(m * rows // 2, dtype=torch.bfloat16, device="cuda")
            use = mats[:copies]

            class Fused(Step):
                def run(self, stream=None):
                    for mt in use:
                        gemm.run_lora(stream, m, mt, xg, mid if silu else yf, Epi.Silu if silu else Epi.Plain, lora,
                                      ldx=17408)

            class Unfused(Step):
                def run(self, stream=None):
                    for mt in use:
                        if silu:
                            gemm.run_split(stream, m, mt, xg, yf, Epi.Plain, True, ldx=17408)
                            lora_silu(stream, xa, 1, cols, b, rank, rows, tab, slot, scale, m, yf, mid)
                        else:
                            gemm.run(stream, m, mt, xg, yf, Epi.Plain, ldx=17408)
                            lora_add(stream, xa, 1, cols, b, rank, rows, tab, slot, scale, m, yf)

            class Bare(Step):
                def run(self, stream=None):
                    for mt in use:
                        gemm.run(stream, m, mt, xg, mid if silu else yf, Epi.Silu if silu else Epi.Plain, ldx=17408)

            r = {}
            for tag, cls in (("fused", Fused), ("unfused", Unfused), ("no_adapter", Bare)):
                st = cls(gemm, m, 8)
                ms = time_step(st, args.steps if m == 1 else 20, 3, not args.no_graph, per_graph=2 if m == 1 else 1,
                               min_reps=100 if m == 1 else 20)
                r[tag + "_us"] = round(ms * 1e3 / len(use), 2)
            res[name] = r
        out[f"m{m}"] = res
        print(f"# LoRA rank {rank} M={m}: {res} (us per product)", file=sys.stderr, flush=True)
    return {"lora_27b": out}


def config0_line(gemm, args):
    """BASELINE.json configs[0] on the GPU: the single int4 GEMV M=1, K=2560, N=9728, symmetric, over 48 distinct
    device copies (617 MB per pass, beyond the 256 MB MALL) in HIP graphs: HBM GB/s over the algorithmic bytes."""
    from qwenny_amd import Epi

    k, n = 2560, 9728
    mats = upload_copies(gemm, quant(650, "i4", k, n), 48)
    st = Step(gemm, 1, k)
    for m in mats:
        st.add(m, Epi.Plain, int4_bytes(k, n, 1), 2 * k * n)
    ms = time_step(st, args.steps, args.warmup, not args.no_graph, per_graph=2)
    gbs = round(st.bytes() / (ms * 1e-3) / 1e9, 1)
    print(f"# configs[0] M=1 (2560, 9728): {ms * 1e3 / len(st.launches):.2f} us per launch, {gbs} GB/s",
          file=sys.stderr, flush=True)
    return {"config0_m1_GBps": gbs}


def grouped_int8_line(gemm, args):
    """int8 with a scale per row and 128 columns (the reference's default load mode: bf16 weights requantized at
    load), on the configs[4] shapes: M = 1 over 4 device copies of (5120, 17408) and (17408, 5120) (GB/s over
    K N + (K / 128) N 4 + 2 M K + 2 M N), and M = 2048 per shape (TFLOP/s)."""
    from qwenny_amd import Epi

    shapes = [(5120, 17408), (17408, 5120)]
    mats = [upload_copies(gemm, quant(660 + i, "i8g", k, n), 4) for i, (k, n) in enumerate(shapes)]
    gbytes = lambda k, n, m: k * n + (k // 128) * n * 4 + 2 * m * k + 2 * m * n
    st = Step(gemm, 1, 17408)
    for c in range(4):
        for ms_, (k, n) in zip(mats, shapes):
            st.add(ms_[c], Epi.Plain, gbytes(k, n, 1), 2 * k * n)
    ms1 = time_step(st, args.steps, args.warmup, not args.no_graph)
    out = {"m1_GBps": round(st.bytes() / (ms1 * 1e-3) / 1e9, 1)}
    for ms_, (k, n) in zip(mats, shapes):
        stp = Step(gemm, 2048, k)
        stp.add(ms_[0], Epi.Plain, gbytes(k, n, 2048), 2 * 2048 * k * n)
        msp = time_step(stp, max(10, args.steps // 10), 3, not args.no_graph)
        out[f"m2048_{k}x{n}_TFLOPs"] = round(stp.flops() / (msp * 1e-3) / 1e12, 1)
    print(f"# grouped int8: {out}", file=sys.stderr, flush=True)
    return {"int8_grouped": out}


def prefill_zp_line(gemm, args):
    """BASELINE.json configs[3] with zero points: int4 with packed zero points, M = 2048, the three 27B prefill
    shapes, activations with 1% outlier columns x20 (TFLOP/s)."""
    import torch

    from qwenny_amd import Epi
    from qwenny_amd.synth import activations

    out = {}
    for i, (k, n) in enumerate(PREFILL_27B):
        mat = upload_copies(gemm, quant(670 + i, "i4z", k, n), 1)[0]
        st = Step(gemm, 2048, k)
        st.x = torch.from_numpy(activations(671, "x", 2048, k, outliers=0.01).view(np.int16)).cuda().view(
            torch.bfloat16)
        st.add(mat, Epi.Plain, int4_bytes(k, n, 2048, zp=True), 2 * 2048 * k * n)
        msp = time_step(st, max(10, args.steps // 10), 3, not args.no_graph)
        out[f"{k}x{n}"] = round(st.flops() / (msp * 1e-3) / 1e12, 1)
    print(f"# prefill M=2048 with zero points: {out} TFLOP/s", file=sys.stderr, flush=True)
    return {"prefill_zp_m2048_TFLOPs": out}


def summarize_clock(pmc_dir, min_ns=50000):
    """Per kernel (name, grid) of a rocprofv3 --pmc GRBM_GUI_ACTIVE SQ_VALU_MFMA_BUSY_CYCLES run: mean duration, the
    clock it ran at (GRBM_GUI_ACTIVE sums the 8 XCDs' cycles) and the fraction of cycles each SIMD's MFMA unit was busy
    (the counter sums the 1024 SIMDs). Dispatches shorter than min_ns are left out."""
    import collections
    import glob
    import sqlite3

    per = collections.defaultdict(lambda: collections.defaultdict(float))
    meta = {}
    for db in glob.glob(os.path.join(pmc_dir, "**", "*_results.db"), recursive=True):
        c = sqlite3.connect(db)
        for disp, name, cn, v, du, grid in c.execute(
                "select dispatch_id, kernel_name, counter_name, value, duration, grid_size from counters_collection"):
            per[(db, disp)][cn] += v
            meta[(db, disp)] = (name, grid, du)
    rows = collections.defaultdict(list)
    for key, cnt in per.items():
        name, grid, du = meta[key]
        if du >= min_ns and cnt.get("GRBM_GUI_ACTIVE"):
            cyc = cnt["GRBM_GUI_ACTIVE"] / 8
            rows[(name.split("(")[0][:70], grid)].append((du, cyc / du, cnt.get("SQ_VALU_MFMA_BUSY_CYCLES", 0) / 1024 / cyc))
    print("| Kernel | Grid (threads) | Dispatches | Mean duration (us) | Clock (GHz) | MFMA busy per SIMD |")
    print("|---|---|---|---|---|---|")
    for (name, grid), v in sorted(rows.items()):
        n = len(v)
        print(f"| `{name}` | {grid} | {n} | {sum(x[0] for x in v) / n / 1e3:.1f} | {sum(x[1] for x in v) / n:.2f} | "
              f"{sum(x[2] for x in v) / n:.3f} |")
    # the --prefill-run workload launches the int4 prefill kernel 5 times per PREFILL_27B shape, in that order: the
    # per-shape figures the bench's roofline_prefill reads (profiles/<CLOCK_NAME>.json)
    pf = sorted((key[1], key) for key, (name, _, du) in meta.items() if "prefill_kernel" in name and du >= min_ns)
    if len(pf) == 5 * len(PREFILL_27B):
        out = {}
        for i, (k, n) in enumerate(PREFILL_27B):
            v = []
            for _, key in pf[5 * i:5 * i + 5]:
                cnt, du = per[key], meta[key][2]
                cyc = cnt["GRBM_GUI_ACTIVE"] / 8
                v.append((du, cyc / du, cnt.get("SQ_VALU_MFMA_BUSY_CYCLES", 0) / 1024 / cyc))
            out[f"{k}x{n}"] = {"us": round(sum(x[0] for x in v) / 5 / 1e3, 2),
                               "clock_GHz": round(sum(x[1] for x in v) / 5, 3),
                               "mfma_busy": round(sum(x[2] for x in v) / 5, 4),
                               "TFLOPs": round(2 * 2048 * k * n / (sum(x[0] for x in v) / 5 * 1e-9) / 1e12, 1)}
        with open(os.path.join(ROOT, "profiles", f"{CLOCK_NAME}.json"), "w") as f:
            json.dump(out, f, indent=1)
        print(json.dumps(out))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", default="",
                    help="comma list of lines: m1,m1sum,m5,prefill,pfzp,pfshort,int8,i8g,dense,dequant,set4b,c0,consumers,"
                         "lora,layer")
    ap.add_argument("--traffic-run", action="store_true", help="the rocprofv3 --pmc workload (see traffic_run)")
    ap.add_argument("--with-torch", action="store_true",
                    help="--prefill-run: also run each shape as a dense bf16 torch product (hipBLASLt)")
    ap.add_argument("--set4b-run", action="store_true",
                    help="the profiling workload of configs[1]: the 4B layer set at M=1, with zero points and "
                         "symmetric, 5 eager launches per matrix each")
    ap.add_argument("--prefill-run", action="store_true",
                    help="the prefill profiling workload: 5 launches of each M=2048 prefill shape, no graph")
    ap.add_argument("--summarize-traffic", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="write profiles/*_traffic.json from the two --pmc runs' output directories")
    ap.add_argument("--summarize-clock", metavar="PMC_DIR",
                    help="print per-kernel clock and MFMA busy from a --kernel-trace --pmc GRBM_GUI_ACTIVE "
                         "SQ_VALU_MFMA_BUSY_CYCLES run's output directory (markdown)")
    args = ap.parse_args()
    if args.summarize_clock:
        summarize_clock(args.summarize_clock)
        return
    if args.summarize_traffic:
        summarize_traffic(*args.summarize_traffic)
        return
    if args.gpus != 1:
        print(json.dumps({"error": "single-GPU build: the products run on one MI355X; --gpus must be 1 "
                                   "(across GPUs a product would shard by output rows, or by K with its split-K "
                                   "partials summed by an all-reduce)"}))
        sys.exit(2)

    import torch

    from qwenny_amd import Epi, Gemm

    torch.cuda.init()
    gemm = Gemm.load(0)
    if args.set4b_run:
        for kind in ("i4z", "i4"):
            for i, (k, n) in enumerate(SET_4B):
                st = Step(gemm, 1, k)
                st.add(upload_copies(gemm, quant(600 + i, kind, k, n), 1)[0], Epi.Plain, 0, 0)
                for _ in range(5):
                    st.run()
        torch.cuda.synchronize()
        print(json.dumps({"set4b_run": "done"}))
        return
    only = set(args.only.split(",")) if args.only else {"m1", "m1sum", "m5", "prefill", "pfzp", "pfshort", "int8", "i8g", "dense",
                                                         "dequant", "set4b", "c0", "consumers", "lora", "layer"}
    print("# generating the 27B-scale layer set and head", file=sys.stderr, flush=True)
    set_mats = [upload_copies(gemm, quant(100 + i, "i4", k, n), 4) for i, (k, n) in enumerate(SET_27B)]
    if args.traffic_run:
        traffic_run(gemm, set_mats)
        return
    if args.prefill_run:
        for i, (k, n) in enumerate(PREFILL_27B):
            st = Step(gemm, 2048, k)
            st.add(set_mats[[0, 2, 3][i]][0], Epi.Plain, int4_bytes(k, n, 2048), 2 * 2048 * k * n)
            for _ in range(5):
                st.run()
            if args.with_torch:  # the same shape as a dense bf16 product through torch (hipBLASLt), for comparison
                a = torch.randn(2048, k, device="cuda").to(torch.bfloat16)
                b = torch.randn(n, k, device="cuda").to(torch.bfloat16)
                for _ in range(5):
                    a @ b.t()
        torch.cuda.synchronize()
        print(json.dumps({"prefill_run": "done"}))
        return
    head = upload_copies(gemm, quant(200, "i4", *HEAD_27B), 1)[0]

    def decode_step(m):
        st = Step(gemm, m, 17408)
        for c in range(4):
            for mats, (k, n) in zip(set_mats, SET_27B):
                st.add(mats[c], Epi.Plain, int4_bytes(k, n, m), 2 * m * k * n)
        st.add(head, Epi.Argmax, int4_bytes(*HEAD_27B, m), 2 * m * HEAD_27B[0] * HEAD_27B[1])
        return st

    out = {}
    step = decode_step(1)
    head_stats = {}
    ms = time_step(step, args.steps, args.warmup, not args.no_graph, stats=head_stats)
    gbs = step.bytes() / (ms * 1e-3) / 1e9
    launches = len(step.launches)
    out["m1"] = {"ms_per_step": ms, "GB/s": gbs, "launches": launches, "bytes": step.bytes()}
    print(f"# M=1 27B set x4 + head: {ms:.4f} ms/step, {gbs:.1f} GB/s ({gbs / HBM_PEAK:.1%} of 8 TB/s)",
          file=sys.stderr, flush=True)

    # the roofline kernel alone: the set's plain skinny launches (one kernel: rocprof's average duration for it is
    # the same quantity)
    rst = Step(gemm, 1, 17408)
    for c in range(4):
        for mats, (k, n) in zip(set_mats, SET_27B):
            rst.add(mats[c], Epi.Plain, int4_bytes(k, n, 1), 2 * k * n)
    rms = time_step(rst, args.steps, args.warmup, not args.no_graph)
    per_launch_bytes = rst.bytes() / len(rst.launches)
    per_launch_s = rms * 1e-3 / len(rst.launches)
    print(f"# roofline kernel (plain M=1 set): {per_launch_s * 1e6:.2f} us per launch, "
          f"{per_launch_bytes / per_launch_s / 1e9:.1f} GB/s", file=sys.stderr, flush=True)

    def whole_rows_step(m):
        """The decode step with each plain product asked for whole rows (one partial, as the reference's int4 products
        return): the workgroup-per-tile-pair kernels, their sums met in LDS."""
        wst = decode_step(m)
        wys = {}

        def run_whole(stream=None):
            for mat, epi, y, _, _ in wst.launches:
                if epi == Epi.Argmax:
                    gemm.run(stream, m, mat, wst.x, y, epi, out_rows=wst.out_rows, n_out=m, keys=wst.keys)
                    continue
                if mat.rows not in wys:
                    wys[mat.rows] = torch.empty(m * mat.rows, dtype=torch.float32, device="cuda")
                gemm.run_split(stream, m, mat, wst.x, wys[mat.rows], epi, True)

        wst.run = run_whole
        wms = time_step(wst, args.steps, args.warmup, not args.no_graph)
        print(f"# M={m} 27B set x4 + head, each plain product as whole rows: {wms:.4f} ms/step, "
              f"{wst.bytes() / (wms * 1e-3) / 1e9:.1f} GB/s", file=sys.stderr, flush=True)
        return {"GBps": round(wst.bytes() / (wms * 1e-3) / 1e9, 1), "ms_per_step": round(wms, 5)}

    extra = {}
    floor = read_floor(set_mats, args)
    extra["read_floor"] = floor
    if "m1sum" in only:
        # the same step with each plain product's split-K partials summed (sum_parts, one launch after each): what a
        # caller that needs whole rows pays on top of the products, over the same algorithmic bytes
        sst = decode_step(1)
        sums = {}

        def run_with_sums(stream=None):
            from qwenny_amd import sum_parts

            for mat, epi, y, _, _ in sst.launches:
                if epi == Epi.Argmax:
                    gemm.run(stream, 1, mat, sst.x, y, epi, out_rows=sst.out_rows, n_out=1, keys=sst.keys)
                    continue
                split = gemm.run(stream, 1, mat, sst.x, y, epi)
                key = mat.rows
                if key not in sums:
                    sums[key] = torch.empty(mat.rows, dtype=torch.float32, device="cuda")
                sum_parts(stream, y, split, 1, mat.rows, sums[key])

        sst.run = run_with_sums
        sms = time_step(sst, args.steps, args.warmup, not args.no_graph)
        extra["m1_with_sums"] = {"GBps": round(sst.bytes() / (sms * 1e-3) / 1e9, 1), "ms_per_step": round(sms, 5)}
        print(f"# M=1 27B set x4 + head, each plain product's partials summed: {sms:.4f} ms/step, "
              f"{sst.bytes() / (sms * 1e-3) / 1e9:.1f} GB/s", file=sys.stderr, flush=True)
        extra["m1_whole_rows"] = whole_rows_step(1)
    if "m5" in only:
        st5 = decode_step(5)
        ms5 = time_step(st5, args.steps, args.warmup, not args.no_graph)
        extra["m5_GBps"] = round(st5.bytes() / (ms5 * 1e-3) / 1e9, 1)
        print(f"# M=5: {ms5:.4f} ms/step, {extra['m5_GBps']} GB/s", file=sys.stderr, flush=True)
        if "m1sum" in only:
            extra["m5_whole_rows"] = whole_rows_step(5)
    if "prefill" in only:
        pf = {}
        for i, (k, n) in enumerate(PREFILL_27B):
            mat = set_mats[[0, 2, 3][i]][0]
            st = Step(gemm, 2048, k)
            st.add(mat, Epi.Plain, int4_bytes(k, n, 2048), 2 * 2048 * k * n)
            msp = time_step(st, max(10, args.steps // 10), 3, not args.no_graph)
            tf = st.flops() / (msp * 1e-3) / 1e12
            pf[f"{k}x{n}"] = round(tf, 1)
            print(f"# prefill M=2048 K={k} N={n}: {msp:.3f} ms, {tf:.1f} TFLOP/s ({tf / BF16_PEAK:.1%})",
                  file=sys.stderr, flush=True)
        extra["prefill_m2048_TFLOPs"] = pf
    if "pfshort" in only:
        extra.update(short_prefill_line(gemm, set_mats, args))
    if "int8" in only:
        i8 = [upload_copies(gemm, quant(300 + i, "i8", k, n), 4) for i, (k, n) in
              enumerate([(5120, 17408), (17408, 5120)])]
        st = Step(gemm, 1, 17408)
        for c in range(4):
            for mats, (k, n) in zip(i8, [(5120, 17408), (17408, 5120)]):
                st.add(mats[c], Epi.Plain, int8_bytes(k, n, 1), 2 * k * n)
        ms8 = time_step(st, args.steps, args.warmup, not args.no_graph)
        extra["int8_m1_GBps"] = round(st.bytes() / (ms8 * 1e-3) / 1e9, 1)
        print(f"# int8 M=1: {ms8:.4f} ms/step, {extra['int8_m1_GBps']} GB/s", file=sys.stderr, flush=True)
        st5 = Step(gemm, 5, 17408)  # configs[4] at M = 5 and 2048 as well
        for c in range(4):
            for mats, (k, n) in zip(i8, [(5120, 17408), (17408, 5120)]):
                st5.add(mats[c], Epi.Plain, int8_bytes(k, n, 5), 2 * 5 * k * n)
        ms85 = time_step(st5, args.steps, args.warmup, not args.no_graph)
        extra["int8_m5_GBps"] = round(st5.bytes() / (ms85 * 1e-3) / 1e9, 1)
        pf8 = {}
        for mats, (k, n) in zip(i8, [(5120, 17408), (17408, 5120)]):
            stp = Step(gemm, 2048, k)
            stp.add(mats[0], Epi.Plain, int8_bytes(k, n, 2048), 2 * 2048 * k * n)
            msp = time_step(stp, max(10, args.steps // 10), 3, not args.no_graph)
            pf8[f"{k}x{n}"] = round(stp.flops() / (msp * 1e-3) / 1e12, 1)
        extra["int8_prefill_m2048_TFLOPs"] = pf8
        print(f"# int8 M=5: {ms85:.4f} ms/step, {extra['int8_m5_GBps']} GB/s; M=2048: {pf8} TFLOP/s",
              file=sys.stderr, flush=True)
    if "dense" in only:
        extra.update(dense_lines(gemm, args))
    if "dequant" in only:
        extra.update(dequant_line(args))
    if "set4b" in only:
        extra.update(set4b_line(gemm, args))
    if "consumers" in only:
        extra.update(consumers_line(args))
    if "c0" in only:
        extra.update(config0_line(gemm, args))
    if "lora" in only:
        extra.update(lora_line(gemm, args))
    if "i8g" in only:
        extra.update(grouped_int8_line(gemm, args))
    if "pfzp" in only:
        extra.update(prefill_zp_line(gemm, args))
    if "layer" in only:
        extra.update(layer_line(gemm, set_mats, args))

    line = {
        "metric": "int4 GEMM HBM GB/s (% of 8 TB/s) at M=1/5; TFLOP/s (% bf16 MFMA peak) at M=2048",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "timing": dict(head_stats, statistic="median of per-replay HIP-event times (10 steps per graph replay)"),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded int4 codes, bf16 scales U(0.002,0.02), bf16 x N(0,1))",
        "config": {"workload": "27B-scale int4 sym g128 decode M=1: (5120,17408)x2,(17408,5120),(5120,6144),"
                               "(6144,5120) x4 device copies + head (5120,248320) argmax",
                   "m": 1, "copies": 4, "graph": not args.no_graph},
        "roofline": {"bound": "hbm", "achieved": round(per_launch_bytes / per_launch_s / 1e9, 1), "peak": HBM_PEAK,
                     "unit": "GB/s", "frac": round(per_launch_bytes / per_launch_s / 1e9 / HBM_PEAK, 4),
                     "traffic": load_traffic(TRAFFIC_NAME),
                     "kernel": "skinny_m1_kernel<int4 symmetric, 4 groups per wave> (plain M=1) over the 27B set (20 launches)",
                     "bytes_per_launch": round(per_launch_bytes), "us_per_launch": round(per_launch_s * 1e6, 3)},
        "extra": extra,
    }
    line["roofline"]["read_floor_us_per_launch"] = floor["us_per_launch"]
    line["roofline"]["frac_of_read_floor"] = round(floor["us_per_launch"] / (per_launch_s * 1e6), 4)
    if "prefill" in only:
        line["roofline_prefill"] = roofline_prefill(extra)
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()

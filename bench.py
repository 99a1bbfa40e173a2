"""Benchmark of the quantized linear-layer path on one MI355X.

Headline (BASELINE.json metric, config 3): the 27B-class decode sweep at M = 1. One step = the ternary products of
one decode token through all 64 layers, in the engine's launch order per layer: q/k/v in one launch, o, gate/up in
one launch, down (256 launches, k_tc_mv3 / k_tc_mv as spec.py:619-673 issues them), over int8 activations that are
resident and quantized before the timed region. The 448 weight matrices (5.62 GB packed) are resident in HBM and
streamed once per step. value = algorithmic bytes per step / time per step (GB/s).

Also reported (under "configs"): config 0 (one product), config 1 (2B layer, M = 1 / 4 / 8), config 2 (prefill
int8 TOPS, M = 512 / 2048), config 3 at M = 16, config 4 (q8_0 MoE step, M = 1 / 256).

The CPU baseline (cpu_baseline) is the reference's own kcpu.c fp32 pair-table GEMV (oracle/_ref, compiled from
the reference source) on one 27B layer, or the repo's restatement of it when _ref is absent.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick]
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

def log(*a):
    print("[bench %.0fs]" % (time.time() - T0), *a, file=sys.stderr, flush=True)


T0 = time.time()
HBM_PEAK = 8000.0            # GB/s, MI355X published
INT8_PEAK = 5000.0           # TOPS dense, MI355X published


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--quick", action="store_true", help="headline only")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-graph", action="store_true", help="eager launches instead of a HIP graph")
    ap.add_argument("--unpooled", action="store_true", help="one allocation per weight matrix instead of one pool")
    ap.add_argument("--plan", action="store_true",
                    help="also time the step as launch records replayed with hipModuleLaunchKernel from the host "
                         "(linear.Plan: Kindi's HIP plan replay), beside the graph-captured launches")
    ap.add_argument("--only", choices=("c0", "c1", "c2", "c3m16", "c4", "producers"),
                    help="run one secondary config alone and print its figures (for profiler runs)")
    ap.add_argument("--cpu-child", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--cpu-runs", type=int, default=5, help=argparse.SUPPRESS)
    ap.add_argument("--cpu-run-s", type=float, default=2.0, help=argparse.SUPPRESS)
    ap.add_argument("--calib", action="store_true",
                    help="only a plain 1 GiB device copy (the known-size kernel that scales FETCH_SIZE/WRITE_SIZE)")
    return ap.parse_args()


def tern_bytes(R, C, M, shared_input=True):
    """algorithmic HBM bytes of one product: codes 2 b/w + fp16 scale per 128, int8 input + XS/XA per group,
    fp32 output"""
    return R * C // 4 + R * (C // 128) * 2 + (M * C + M * (C // 128) * 8 if shared_input else 0) + M * R * 4


class Timer(object):
    """HIP events on torch's current stream (the stream every kt_* launch here goes to)"""

    def __init__(self, torch):
        self.t = torch

    def run(self, fn, steps, warmup):
        t = self.t
        for _ in range(warmup):
            fn()
        t.cuda.synchronize()
        e0, e1 = t.cuda.Event(enable_timing=True), t.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            fn()
        e1.record()
        t.cuda.synchronize()
        return e0.elapsed_time(e1) / steps           # ms per step


def graphed(torch, fn, use_graph):
    """capture fn's launches in a HIP graph (no memsets inside: every buffer is prepared before capture)"""
    if not use_graph:
        return fn
    fn()
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g.replay


# ----------------------------------------------------------------------------------------------- config 3
def build_27b(torch, linear, synth, M_list, pooled=True):
    """the 64 layers' 448 matrices, packed into one device pool (or one allocation each)"""
    cfg = synth.CFG["c3"]
    lib = linear.gpudrv.load()
    sizes = [(lib.kt_tern_weight_bytes(R, C) + 255) // 256 * 256 for n, R, C in cfg["mats"]]
    pool = torch.empty(sum(sizes) * cfg["layers"], dtype=torch.uint8, device="cuda") if pooled else None
    off = 0
    layers = []
    for l in range(cfg["layers"]):
        mats = {}
        for i, (n, R, C) in enumerate(cfg["mats"]):
            bc, dpm = synth.tern_pack(R, C, 100 + l * 8 + i, device="cuda")
            W = pool[off:off + sizes[i]] if pooled else None
            off += sizes[i]
            mats[n] = linear.TernaryMatrix(bc, dpm, R, C, W=W)
            del bc, dpm
        layers.append(mats)
    torch.cuda.synchronize()
    return layers


def sweep_step(torch, linear, layers, M, seed=7):
    """the per-layer launches of one decode step over resident int8 activations; returns (fn, bytes, launches)"""
    Lin = linear.Linear({})
    acts, outs = [], []
    nbytes, launches = 0, []
    for l, mats in enumerate(layers):
        for n, m in mats.items():
            Lin.add("%d.%s" % (l, n), m)
        x = [torch.randn((M, C), device="cuda", generator=torch.Generator(device="cuda").manual_seed(seed + 4 * l + i))
             for i, C in enumerate((5120, 5120, 5120, 17408))]
        a = [linear.quantize(xi) for xi in x]
        o = {n: torch.empty((M, m.R), dtype=torch.float32, device="cuda") for n, m in mats.items()}
        acts.append(a)
        outs.append(o)
        nbytes += sum(tern_bytes(mats[n].R, mats[n].C, M, i == 0) for grp in (("q", "k", "v"), ("o",), ("gate", "up"), ("down",))
                      for i, n in enumerate(grp))
        launches += [("%d.q/k/v" % l, tern_bytes(mats["q"].R + mats["k"].R + mats["v"].R, 5120, M)),
                     ("%d.o" % l, tern_bytes(5120, 5120, M)),
                     ("%d.gate/up" % l, tern_bytes(2 * 17408, 5120, M)),
                     ("%d.down" % l, tern_bytes(5120, 17408, M))]

    calls = []
    for l in range(len(layers)):
        a, o = acts[l], outs[l]
        p = "%d." % l
        calls.append((Lin.gemv_q, [p + "q", p + "k", p + "v"], a[0], [o["q"], o["k"], o["v"]]))
        calls.append((Lin.gemv_q, [p + "o"], a[1], [o["o"]]))
        calls.append((Lin.gemv_q, [p + "gate", p + "up"], a[2], [o["gate"], o["up"]]))
        calls.append((Lin.gemv_q, [p + "down"], a[3], [o["down"]]))

    def step():
        for f, names, act, o in calls:
            f(names, act, o)

    stages = [([Lin.w[n] for n in names], act, o) for _, names, act, o in calls]
    return step, nbytes, calls, launches, stages


def config3_kinds(torch, linear, layers, M, timer, steps, use_graph):
    """config 3's step at M tokens and its four launch kinds, each timed alone: the kind's launches of every layer back
    to back in one graph (so a launch's weights are not in cache from the one before)"""
    step, nbytes, calls, launches, _ = sweep_step(torch, linear, layers, M)
    ms = timer.run(graphed(torch, step, use_graph), steps, 2)
    out = {"ms_per_step": round(ms, 4), "GB/s": round(nbytes / ms / 1e6, 1),
           "frac_hbm": round(nbytes / ms / 1e6 / HBM_PEAK, 4), "us_per_launch": {}}
    for k, kind in enumerate(("q/k/v", "o", "gate/up", "down")):
        sel = calls[k::4]

        def fn(sel=sel):
            for f, names, act, o in sel:
                f(names, act, o)
        us = timer.run(graphed(torch, fn, use_graph), steps, 2) * 1e3 / len(sel)
        out["us_per_launch"][kind] = round(us, 2)
    return out


def step_with_producers(torch, linear, layers, M=1):
    """config 3's decode step with each product's input made by its fused producer, as Kindi's decode runs them: per
    layer rmsfold (one residual part) -> q/k/v, fold -> o, rmsfold (one part) -> gate/up, smfold (17408 columns) ->
    down: 512 dependent launches a step. One set of fp32 input buffers serves every layer (the timing does not depend
    on their values); each product reads the int8 row its producer just wrote."""
    H, F = 5120, 17408
    Lin = linear.Linear({})
    g = torch.Generator(device="cuda").manual_seed(70)
    x, r = (torch.randn((M, H), device="cuda", generator=g) for _ in range(2))
    a, b2 = (torch.randn((M, F), device="cuda", generator=g) for _ in range(2))
    w = torch.ones(H, device="cuda")
    sgH = torch.where(torch.rand(H, device="cuda", generator=g) < 0.5, -1.0, 1.0).float()
    sgF = torch.where(torch.rand(F, device="cuda", generator=g) < 0.5, -1.0, 1.0).float()
    xw = torch.empty_like(x)
    aH, aO, aG = (linear._act_out(M, H, "cuda") for _ in range(3))
    aF = linear._act_out(M, F, "cuda")
    outs = []
    for l, mats in enumerate(layers):
        for n, m in mats.items():
            Lin.add("%d.%s" % (l, n), m)
        outs.append({n: torch.empty((M, m.R), dtype=torch.float32, device="cuda") for n, m in mats.items()})

    def step():
        for l in range(len(layers)):
            p, o = "%d." % l, outs[l]
            linear.rmsfold(x, w, sgH, 1024, r=r, nparts=1, xw=xw, out=aH)
            Lin.gemv_q([p + "q", p + "k", p + "v"], aH, [o["q"], o["k"], o["v"]])
            linear.fold(x, sgH, 1024, out=aO)
            Lin.gemv_q([p + "o"], aO, [o["o"]])
            linear.rmsfold(x, w, sgH, 1024, r=r, nparts=1, xw=xw, out=aG)
            Lin.gemv_q([p + "gate", p + "up"], aG, [o["gate"], o["up"]])
            linear.smfold(a, b2, sgF, 1024, out=aF)
            Lin.gemv_q([p + "down"], aF, [o["down"]])

    return step


# ----------------------------------------------------------------------------------------------- other configs
def config0(torch, linear, synth, timer, steps, use_graph):
    R, C = synth.CFG["c0"]["R"], synth.CFG["c0"]["C"]
    bc, dpm = synth.tern_pack(R, C, 0, device="cuda")
    L = linear.Linear({"w": linear.TernaryMatrix(bc, dpm, R, C)})
    act = linear.quantize(synth.activations(1, C, 1, device="cuda"), per_row=True)
    Y = torch.empty((1, R), dtype=torch.float32, device="cuda")
    reps = 50

    def fn():
        for _ in range(reps):
            L.gemv_q(["w"], act, [Y])

    ms = timer.run(graphed(torch, fn, use_graph), steps, 2) / reps
    b = tern_bytes(R, C, 1)
    return {"shape": [R, C], "M": 1, "us": round(ms * 1e3, 3), "GB/s": round(b / ms / 1e6, 1),
            "bytes": b, "note": "%d back-to-back launches per timed step" % reps}


def config1(torch, linear, synth, timer, steps, use_graph):
    cfg = synth.CFG["c1"]
    mats = {}
    for i, (n, R, C) in enumerate(cfg["mats"]):
        bc, dpm = synth.tern_pack(R, C, 10 + i, device="cuda")
        mats[n] = linear.TernaryMatrix(bc, dpm, R, C)
    L = linear.Linear(mats)
    res = {}
    for M in (1, 4, 8):
        x = [synth.activations(M, C, 30 + i, device="cuda") for i, C in enumerate((2048, 2048, 2048, 6144))]
        a = [linear.quantize(xi, per_row=True) for xi in x]
        o = {n: torch.empty((M, m.R), dtype=torch.float32, device="cuda") for n, m in mats.items()}
        reps = 20

        def fn():
            for _ in range(reps):
                L.gemv_q(["q", "k", "v"], a[0], [o["q"], o["k"], o["v"]])
                L.gemv_q(["o"], a[1], [o["o"]])
                L.gemv_q(["gate", "up"], a[2], [o["gate"], o["up"]])
                L.gemv_q(["down"], a[3], [o["down"]])

        ms = timer.run(graphed(torch, fn, use_graph), steps, 2) / reps
        b = (tern_bytes(3072, 2048, M) + tern_bytes(2048, 2048, M) + tern_bytes(12288, 2048, M)
             + tern_bytes(2048, 6144, M))
        res["M=%d" % M] = {"us_per_layer": round(ms * 1e3, 2), "GB/s": round(b / ms / 1e6, 1), "bytes": b}
    return res


def config2(torch, linear, synth, timer, steps):
    res = {}
    for i, (n, R, C) in enumerate(synth.CFG["c2"]["mats"]):
        bc, dpm = synth.tern_pack(R, C, 20 + i, device="cuda")
        W = linear.TernaryMatrix(bc, dpm, R, C)
        L = linear.Linear({"w": W})
        W8 = W.expand()
        ms_x = timer.run(lambda: W.expand(out=W8), max(steps // 2, 3), 2)
        for M in (512, 2048):
            act = linear.quantize(synth.activations(M, C, 22 + i, device="cuda"), per_row=True)
            Y16 = torch.empty((M, R), dtype=torch.float16, device="cuda")
            ms = timer.run(lambda: L.gemm("w", act, Y16=Y16), max(steps // 2, 3), 2)
            tops = 2.0 * M * R * C / ms / 1e9
            # every MFMA the kernels issue is useful work (2 M R C operations exactly, counted by
            # SQ_INSTS_VALU_MFMA_MOPS_I8), so the achieved rate over the int8 peak is the fraction of peak; the
            # counters put the clock under this load at 2.08-2.17 GHz
            # the same product over the int8 trit copy (kt_tern_expand once, kept with the weights: 4.25 times their
            # bytes; kt_tern_gemm8, the same bits); expand_us is the copy's cost per matrix
            ms8 = timer.run(lambda: L.gemm8("w", act, W8, Y16=Y16), max(steps // 2, 3), 2)
            tops8 = 2.0 * M * R * C / ms8 / 1e9
            res["%s M=%d" % (n, M)] = {"shape": [R, C], "us": round(ms * 1e3, 1), "TOPS": round(tops, 1),
                                       "frac_int8_peak": round(tops / INT8_PEAK, 4),
                                       "int8_copy_us": round(ms8 * 1e3, 1), "int8_copy_TOPS": round(tops8, 1),
                                       "int8_copy_frac_int8_peak": round(tops8 / INT8_PEAK, 4),
                                       "expand_us": round(ms_x * 1e3, 1),
                                       # the faster of the two product paths (both give the same bits)
                                       "best_TOPS": round(max(tops, tops8), 1),
                                       "best_frac_int8_peak": round(max(tops, tops8) / INT8_PEAK, 4),
                                       "best_path": "int8 trit copy (kt_tern_gemm8)" if tops8 > tops
                                                    else "packed trits (kt_tern_gemm)"}
            # the vendor's plain int8 GEMM (hipBLASLt through torch._int_mm: int32 out, no scales, no trit unpack)
            # on the same shapes and box, as the practical ceiling of an int8 product here
            try:
                qa = act.XQ[:, :C].contiguous()
                qb = torch.randint(-1, 2, (C, R), dtype=torch.int8, device="cuda")
                vms = timer.run(lambda: torch._int_mm(qa, qb), max(steps // 2, 3), 2)
                vt = 2.0 * M * R * C / vms / 1e9
                res["%s M=%d" % (n, M)].update({"vendor_int8_TOPS": round(vt, 1), "vs_vendor": round(tops / vt, 3)})
                del qb
            except Exception as e:                                   # not every build routes int8 mm
                res["%s M=%d" % (n, M)]["vendor_int8"] = repr(e)[:80]
        del W8
    return res


def config4(torch, moe, synth, timer, steps, use_graph):
    c = synth.CFG["c4"]
    E, k, H, F = c["E"], c["k"], c["H"], c["F"]
    up = moe.Q8Experts([synth.q8_rows(F, H, 40_000 + e, device="cuda") for e in range(E)], F, H)
    down = moe.Q8Experts([synth.q8_rows(H, F, 50_000 + e, device="cuda") for e in range(E)], H, F)
    layer = moe.MoE(up, down, k)
    res = {}
    for M in (1, 256):
        x0 = synth.activations(M, H, 42, device="cuda")
        lg = synth.logits(M, E, 41, device="cuda")
        x = x0.clone()
        bufs = layer.buffers(M)
        out, st = layer.forward(x, lg, bufs)
        torch.cuda.synchronize()
        touched = int((st["lists"][0] > 0).sum().item())
        per_expert = 2 * up.bytes_per_expert
        b = touched * per_expert + M * H * (4 + 1 + 4 / 32) + M * k * (F * (4 + 1 + 4 / 32) + H * 4) + M * H * 4
        reps = 20 if M == 1 else 1           # back-to-back layers in one graph, as config 1

        def rep(fn):
            def f():
                for _ in range(reps):
                    fn()
            return f
        if M * k <= 64:
            # kt_moe_decode (one token: two launches); the six separate launches beside it
            work = layer.workspace(M)
            ms = timer.run(graphed(torch, rep(lambda: layer.decode(x, lg, work)), use_graph), steps, 2) / reps
            ms_sep = timer.run(graphed(torch, rep(lambda: layer.forward(x, lg, bufs)), use_graph), steps, 2) / reps
            extra = {"launches": 2 if M == 1 else 4, "us_separate_launches": round(ms_sep * 1e3, 1)}
        else:
            ms = timer.run(graphed(torch, rep(lambda: layer.forward(x, lg, bufs)), use_graph), steps, 2) / reps
            extra = {"launches": 6}
        extra["note"] = "%d back-to-back layers per timed graph" % reps
        res["M=%d" % M] = {"experts_touched": touched, "us": round(ms * 1e3, 1), "GB/s": round(b / ms / 1e6, 1),
                           "bytes": int(b), "frac_hbm": round(b / ms / 1e6 / HBM_PEAK, 4)}
        res["M=%d" % M].update(extra)
    return res


def producers(torch, linear, synth, timer, steps, use_graph):
    """the fused input producers (kt_rmsfold_q8 / kt_fold_q8 / kt_smfold_q8): a 27B-class decode layer's four
    (attention rmsfold with one residual part, o-input fold, FFN rmsfold with one part, down-input smfold over
    17408 columns) at M = 1 / 16, and a 9B-class prefill pair (rmsfold 4096, smfold 12288, HB 4096) at M = 2048.
    Bytes: fp32 inputs and parts read once, weights/signs once, x + parts and the int8 row with XS/XA written."""
    def sgn(C, seed):
        return torch.where(torch.rand(C, device="cuda", generator=torch.Generator("cuda").manual_seed(seed)) < 0.5,
                           -1.0, 1.0).float()

    def qbytes(M, C):
        return M * C + M * (C // 128) * 8

    res = {}
    mats = synth.CFG["c3"]["mats"]
    H, F = mats[0][2], mats[4][1]                       # hidden 5120, FFN 17408
    for M in (1, 16):
        x = synth.activations(M, H, 60, device="cuda")
        r = synth.activations(M, H, 61, device="cuda")
        a = synth.activations(M, F, 62, device="cuda")
        b2 = synth.activations(M, F, 63, device="cuda")
        w, sgH, sgF = torch.ones(H, device="cuda"), sgn(H, 1), sgn(F, 2)
        xw = torch.empty_like(x)
        oH = linear._act_out(M, H, "cuda")
        oF = linear._act_out(M, F, "cuda")
        reps = 20

        def fn():
            for _ in range(reps):
                linear.rmsfold(x, w, sgH, 1024, r=r, nparts=1, xw=xw, out=oH)
                linear.fold(x, sgH, 1024, out=oH)
                linear.rmsfold(x, w, sgH, 1024, r=r, nparts=1, xw=xw, out=oH)
                linear.smfold(a, b2, sgF, 1024, out=oF)

        ms = timer.run(graphed(torch, fn, use_graph), steps, 2) / reps
        nb = 2 * (3 * M * H * 4 + 2 * H * 4 + qbytes(M, H)) + (M * H * 4 + H * 4 + qbytes(M, H)) \
            + (2 * M * F * 4 + F * 4 + qbytes(M, F))
        res["27B layer M=%d" % M] = {"us_per_layer": round(ms * 1e3, 2), "launches": 4, "bytes": nb,
                                     "GB/s": round(nb / ms / 1e6, 1)}
    M, H9, F9 = 2048, 4096, 12288
    x = synth.activations(M, H9, 64, device="cuda")
    r = synth.activations(M, H9, 65, device="cuda")
    a = synth.activations(M, F9, 66, device="cuda")
    b2 = synth.activations(M, F9, 67, device="cuda")
    w, sgH, sgF = torch.ones(H9, device="cuda"), sgn(H9, 3), sgn(F9, 4)
    xw = torch.empty_like(x)
    oH, oF = linear._act_out(M, H9, "cuda"), linear._act_out(M, F9, "cuda")
    ms_r = timer.run(lambda: linear.rmsfold(x, w, sgH, 4096, r=r, nparts=1, xw=xw, out=oH), max(steps // 2, 3), 2)
    ms_s = timer.run(lambda: linear.smfold(a, b2, sgF, 4096, out=oF), max(steps // 2, 3), 2)
    nr = 3 * M * H9 * 4 + 2 * H9 * 4 + qbytes(M, H9)
    ns = 2 * M * F9 * 4 + F9 * 4 + qbytes(M, F9)
    res["9B prefill M=2048 rmsfold"] = {"us": round(ms_r * 1e3, 1), "GB/s": round(nr / ms_r / 1e6, 1),
                                        "frac_hbm": round(nr / ms_r / 1e6 / HBM_PEAK, 4)}
    res["9B prefill M=2048 smfold"] = {"us": round(ms_s * 1e3, 1), "GB/s": round(ns / ms_s / 1e6, 1),
                                       "frac_hbm": round(ns / ms_s / 1e6 / HBM_PEAK, 4)}
    return res


# ----------------------------------------------------------------------------------------------- CPU baseline
def physical_cores():
    """the physical cores (package, core id) among the CPUs this process may run on, and the first CPU of each"""
    cores = {}
    for cpu in sorted(os.sched_getaffinity(0)):
        base = "/sys/devices/system/cpu/cpu%d/topology/" % cpu
        try:
            key = (open(base + "physical_package_id").read().strip(), open(base + "core_id").read().strip())
        except OSError:
            key = ("?", str(cpu))
        cores.setdefault(key, cpu)
    return cores


def cpu_baseline(synth, runs=5, run_s=2.0):
    """kcpu.c's pair-table GEMV over 27B layers, timed in a child process that owns its OpenMP setup: one thread per
    physical core this process may use, OMP_PROC_BIND=close, OMP_PLACES=cores; a warm-up pass, then `runs` timed
    runs of about run_s seconds; the median run is the value"""
    import subprocess
    cores = physical_cores()
    env = dict(os.environ, OMP_NUM_THREADS=str(len(cores)), OMP_PROC_BIND="close", OMP_PLACES="cores")
    r = subprocess.run([sys.executable, os.path.abspath(__file__), "--cpu-child", "--cpu-runs", str(runs),
                        "--cpu-run-s", str(run_s)], env=env, capture_output=True, text=True, timeout=600)
    if r.returncode != 0:
        raise RuntimeError("cpu baseline child failed:\n" + r.stderr[-2000:])
    out = json.loads(r.stdout.strip().splitlines()[-1])
    out["allowed_cpus"] = len(os.sched_getaffinity(0))         # before the child's OpenMP binding narrows its mask
    return out


def cpu_child_moe(orc, runs, run_s, nsets=16):
    """config 4 at one token on the host with the reference's q8_0 kernel (dsv41_cpu.c k_q8g, oracle/_ref): per token
    its 6 experts' up products, relu^2 and the reference's quantizer (quant_q8), their down products. nsets sets of 6
    experts rotate (1 GB of q8_0 weights: copies of one generated set at distinct addresses, beyond the host's
    caches) so the sample streams from DRAM."""
    import numpy as np
    from kindi_amd import synth
    c = synth.CFG["c4"]
    k, H, F = c["k"], c["H"], c["F"]
    up0 = [orc.q8_0_group4(synth.q8_rows(F, H, 40_000 + e).numpy(), F, H) for e in range(k)]
    down0 = [orc.q8_0_group4(synth.q8_rows(H, F, 50_000 + e).numpy(), H, F) for e in range(k)]
    ups = [up0[e % k].copy() for e in range(k * nsets)]
    downs = [down0[e % k].copy() for e in range(k * nsets)]
    x = np.random.default_rng(42).normal(0, 1, H).astype(np.float32)
    u = np.empty(F, np.float32)
    yd = np.empty(H, np.float32)
    nbytes = k * (F * H + H * F) * 34 // 32

    def token(i):
        q, d = orc.ref_quant_q8(x)
        for e in range(k * (i % nsets), k * (i % nsets) + k):
            orc.ref_q8_matvec(ups[e], F, H, q, d, u)
            r = np.maximum(u, np.float32(0))
            q2, d2 = orc.ref_quant_q8(r * r)
            orc.ref_q8_matvec(downs[e], H, F, q2, d2, yd)

    for i in range(nsets):
        token(i)
    rates = []
    for _ in range(runs):
        n, t0 = 0, time.perf_counter()
        while n < nsets or time.perf_counter() - t0 < run_s:
            token(n)
            n += 1
        rates.append(n / (time.perf_counter() - t0))
    rates.sort()
    med = rates[len(rates) // 2]
    return {"value": round(nbytes * med / 1e9, 2), "unit": "GB/s", "us_per_token": round(1e6 / med, 1),
            "runs_GBs": [round(nbytes * r / 1e9, 2) for r in rates],
            "sample": "config 4 at M=1 (6 experts: up [1856x2688] q8_0 product, relu^2 + quant_q8, down [2688x1856]; "
                      "%.1f MB of q8_0 weights a token, %d expert sets rotating): dsv41_cpu.c k_q8g over OpenMP "
                      "threads, median of %d runs" % (nbytes / 1e6, nsets, runs)}


def cpu_child(runs, run_s, nlayers=4):
    """the measurement cpu_baseline starts: nlayers distinct layers (352 MB of codes) rotate so the sample streams
    from DRAM rather than the host's caches"""
    import numpy as np
    from kindi_amd import synth
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as orc
    ref = orc.ref_kcpu() is not None
    layers = []
    nbytes = kbytes = 0
    for l in range(nlayers):
        mats = []
        for i, (n, R, C) in enumerate(synth.CFG["c3"]["mats"]):
            bc, dpm = synth.tern_pack(R, C, 100 + l * 8 + i, device="cpu")
            bc = bc.numpy()
            dpm = dpm.numpy().view(np.uint16)
            mats.append((orc.paircodes_fast(bc, R, C), orc.pair_scales(dpm, R, C), R, C))
            if l == 0:
                nbytes += tern_bytes(R, C, 1)
                # what kcpu.c streams: 4-bit pair codes (2 bits a weight), fp32 scales per (row, 128 columns), fp32
                # x in and y out
                kbytes += R * C // 4 + R * (C // 128) * 4 + C * 4 + R * 4
        layers.append(mats)
    xs = {C: np.random.default_rng(C).normal(0, 1, C).astype(np.float32) for C in (5120, 17408)}
    gemv = orc.ref_gemv if ref else orc.pair_gemv

    def layer(mats):
        for Pc, S, R, C in mats:
            gemv(Pc, S, R, C, xs[C])

    for mats in layers:                                          # warm-up: every layer once
        layer(mats)
    rates, passes, total = [], 0, 0.0
    for _ in range(runs):
        reps = 0
        t0 = time.perf_counter()
        while reps < nlayers or time.perf_counter() - t0 < run_s:
            layer(layers[reps % nlayers])
            reps += 1
        el = time.perf_counter() - t0
        rates.append(reps / el)                                  # layer passes a second
        passes += reps
        total += el
    rates.sort()
    moe = cpu_child_moe(orc, runs, run_s / 2) if orc.ref_dsv41() is not None else None
    threads = int(os.environ.get("OMP_NUM_THREADS", "0"))
    model = ""
    try:
        for ln in open("/proc/cpuinfo"):
            if ln.startswith("model name"):
                model = ln.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    med = rates[len(rates) // 2]
    print(json.dumps({
        "value": round(nbytes * med / 1e9, 2), "unit": "GB/s", "cores": threads, "cpu": model,
        "kcpu_stream_GBs": round(kbytes * med / 1e9, 2),
        "host_cpus": os.cpu_count(),
        "kind": "reference" if ref else "port", "runs_GBs": [round(nbytes * x / 1e9, 2) for x in rates],
        "omp": "OMP_NUM_THREADS=%d (physical cores allowed) OMP_PROC_BIND=%s OMP_PLACES=%s" % (
            threads, os.environ.get("OMP_PROC_BIND"), os.environ.get("OMP_PLACES")),
        "moe_c4": moe,
        "sample": "median of %d runs (%d layer passes in %.1f s after a warm-up) of the 27B-class decode (q,k,v,o,gate,"
                  "up,down; %.1f MB of ternary weights per layer, %d distinct layers rotating): fp32 pair-table GEMV "
                  "(kcpu.c gemv), %d OpenMP threads. value counts the GPU line's algorithmic bytes per layer (the same "
                  "work unit); kcpu_stream_GBs the %.1f MB a layer kcpu.c itself streams (2-bit pair codes, fp32 "
                  "scales and vectors)" % (runs, passes, total, nbytes / 1e6, nlayers, threads, kbytes / 1e6)}))


# ----------------------------------------------------------------------------------------------- HBM traffic
def calib_copy(torch, nbytes=1 << 30):
    """a plain device copy of nbytes (reads nbytes, writes nbytes): the kernel whose FETCH_SIZE / WRITE_SIZE
    counters give the scale from counter KiB to HBM bytes"""
    src = torch.randint(0, 255, (nbytes,), dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"calib_copy_bytes": nbytes}))


def pmc_traffic():
    """HBM bytes per launch of the decode kernel from the committed rocprofv3 --pmc summary (FETCH_SIZE +
    WRITE_SIZE per dispatch, scaled by the copy kernel's counters); None when the summary is absent"""
    path = os.path.join(ROOT, "profiles", "tern_gemv_27b_decode_pmc.md")
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch:"):
            return {"bytes_per_launch": int(float(line.split(":")[1])),
                    "source": "profiles/tern_gemv_27b_decode_pmc.md"}
    return None


# ----------------------------------------------------------------------------------------------- main
def main():
    a = parse()
    if a.cpu_child:                                              # the CPU baseline's own process (no GPU)
        cpu_child(a.cpu_runs, a.cpu_run_s)
        return
    if a.gpus != 1:
        print("bench.py: this build measures one GPU; the product shards per GPU (see DESIGN.md) but multi-GPU "
              "runs are not part of it. Use --gpus 1.", file=sys.stderr)
        sys.exit(2)
    import torch
    from kindi_amd import linear, moe, synth
    torch.cuda.set_device(0)
    if a.calib:
        calib_copy(torch)
        return
    timer = Timer(torch)
    use_graph = not a.no_graph
    if a.only:
        fn = {"c0": lambda: config0(torch, linear, synth, timer, a.steps, use_graph),
              "c3m16": lambda: config3_kinds(torch, linear, build_27b(torch, linear, synth, (16,)), 16, timer,
                                             a.steps, use_graph),
              "c1": lambda: config1(torch, linear, synth, timer, a.steps, use_graph),
              "c2": lambda: config2(torch, linear, synth, timer, a.steps),
              "c4": lambda: config4(torch, moe, synth, timer, a.steps, use_graph),
              "producers": lambda: producers(torch, linear, synth, timer, a.steps, use_graph)}[a.only]
        print(json.dumps({"only": a.only, "result": fn()}))
        return

    t0 = time.time()
    log("building the 27B-class weights")
    layers = build_27b(torch, linear, synth, (1, 16), pooled=not a.unpooled)
    log("config 3, M=1")
    step, nbytes, calls, launches, stages = sweep_step(torch, linear, layers, 1)
    ms_l = timer.run(graphed(torch, step, use_graph), a.steps, a.warmup)
    ms, nlaunch, kernel = ms_l, len(calls), "k_gemv_step<1> (q/k/v, o, gate/up) + k_gemv_flat1 (down)"
    replay = None
    if a.plan:
        # the same launches as records replayed from the host (no graph): Kindi's HIP plan replay
        plan = linear.Plan(step)
        ms_r = timer.run(plan.launch, a.steps, a.warmup)
        replay = {"ms_per_step": round(ms_r, 4), "GB/s": round(nbytes / ms_r / 1e6, 1), "launches": plan.n,
                  "note": "launch records (kt_record_begin/end) replayed with hipModuleLaunchKernel, no graph"}
        del plan
    gbs = nbytes / ms / 1e6
    # the dominant kernel is every launch of the step (back to back in the graph): its average duration is the timed region over the launch count (an upper bound: it includes the gaps)
    launch_ms = ms / nlaunch
    achieved = nbytes / nlaunch / launch_ms / 1e6
    traffic = pmc_traffic()
    out = {
        "metric": "decode GEMV HBM GB/s (% of 8 TB/s) + prefill int8 TOPS, ternary 27B shapes",
        "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8 x ternary (int32 accumulate, fp32 scale)", "data": "synthetic (seeded; BASELINE config 3)",
        "config": {"workload": "config 3: 27B-class decode sweep, 64 layers x {q,k,v,o,gate,up,down}, M=1",
                   "tokens": 1, "bytes_per_step": nbytes, "launches_per_step": nlaunch,
                   "products_per_step": len(calls), "executor": "launches",
                   "graph": use_graph, "frac_hbm": round(gbs / HBM_PEAK, 4)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK, 4),
                     "traffic": traffic["bytes_per_launch"] if traffic else None,
                     "traffic_source": traffic["source"] if traffic else None,
                     "algorithmic_bytes_per_launch": nbytes // nlaunch,
                     "kernel": kernel, "launches": nlaunch,
                     "avg_launch_us": round(launch_ms * 1e3, 3)},
    }
    if not a.quick:
        cfgs = {"c3 M=1 launches": {"ms_per_step": round(ms_l, 4), "GB/s": round(nbytes / ms_l / 1e6, 1),
                                    "frac_hbm": round(nbytes / ms_l / 1e6 / HBM_PEAK, 4),
                                    "note": "%d graph-captured launches (kt_tern_gemv / gemv3) per step" % len(calls)}}
        log("config 3, M=1 with producers")
        stepP = step_with_producers(torch, linear, layers, 1)
        msP = timer.run(graphed(torch, stepP, use_graph), a.steps, a.warmup)
        cfgs["c3 M=1 step with producers"] = {
            "ms_per_step": round(msP, 4), "launches_per_step": 8 * len(layers),
            "products_GB/s": round(nbytes / msP / 1e6, 1),
            "note": "the headline's 256 products, each input made by its fused producer (rmsfold / fold / rmsfold / "
                    "smfold) in the launch before it; products_GB/s counts only the products' bytes"}
        del stepP
        log("config 3, M=16")
        cfgs["c3 M=16"] = config3_kinds(torch, linear, layers, 16, timer, max(a.steps // 2, 3), use_graph)
        if replay:
            cfgs["c3 M=1 record replay"] = replay
        del layers, step, calls, stages
        torch.cuda.empty_cache()
        log("configs 0, 1, 2, 4")
        cfgs["c0"] = config0(torch, linear, synth, timer, a.steps, use_graph)
        cfgs["c1"] = config1(torch, linear, synth, timer, a.steps, use_graph)
        cfgs["c2"] = config2(torch, linear, synth, timer, a.steps)
        cfgs["c4"] = config4(torch, moe, synth, timer, a.steps, use_graph)
        log("input producers")
        cfgs["producers"] = producers(torch, linear, synth, timer, a.steps, use_graph)
        out["configs"] = cfgs
    if not a.no_cpu:
        log("cpu baseline")
        out["cpu_baseline"] = cpu_baseline(synth)
    out["wall_s"] = round(time.time() - t0, 1)
    print(json.dumps(out))


if __name__ == "__main__":
    main()

"""Launch records (kt_record_begin / kt_record_end) replayed with hipModuleLaunchKernel from ctypes, as Kindi's HIP
plan replay launches its (fn, grid, block, args) tuples (Replay.launch, /root/reference/kindi/spec.py:303-320; the
tuples are built by Plan.add, tp.py:282-302). Every replay gives the bits of the direct calls: the decode product at
1 and 16 tokens, the prefill product at 512 tokens, the quantizer, and a chained decode step whose products read what
earlier records wrote."""
import ctypes

import numpy as np
import pytest
import torch

import oracle as orc
from kt_cases import say, tern_case, dev, host, rng

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def kt():
    assert torch.cuda.is_available(), "GPU tests need the MI355X"
    from kindi_amd import gpudrv, linear
    return gpudrv, linear


def mat(linear, R, C, seed):
    dig, bc, dpm = tern_case(R, C, seed)
    return linear.TernaryMatrix(bc, dpm, R, C), bc, dpm


def replay_raw(gpudrv, recs, n):
    """the replay loop of Kindi's Replay.launch, with the record's dynamic LDS bytes, on torch's stream"""
    L = gpudrv.hip().hipModuleLaunchKernel
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for r in recs[:n]:
        rc = L(r.fn, r.grid[0], r.grid[1], r.grid[2], r.block[0], r.block[1], r.block[2], r.shmem, s,
               ctypes.cast(r.args, ctypes.c_void_p), None)
        assert rc == 0, "hipModuleLaunchKernel %d" % rc


def record(gpudrv, fn, cap=16):
    lib = gpudrv.load()
    recs = (gpudrv.KtLaunch * cap)()
    assert lib.kt_record_begin(recs, cap) == 0
    try:
        fn()
    finally:
        n = ctypes.c_int(0)
        rc = lib.kt_record_end(ctypes.byref(n))
    assert rc == 0
    return recs, n.value


@pytest.mark.parametrize("R,C,M", [(5120, 5120, 1), (17408, 5120, 1), (5120, 17408, 1), (6144, 2048, 16),
                                   (5120, 17408, 16), (1000, 384, 3)])
def test_gemv_records(kt, R, C, M):
    gpudrv, linear = kt
    say("records gemv", R, C, M)
    W, bc, dpm = mat(linear, R, C, R + C + M)
    L = linear.Linear({"w": W})
    act = linear.quantize(dev(rng(M + C).normal(0, 1, (M, C)).astype(np.float32)))
    Y = torch.empty((M, R), dtype=torch.float32, device="cuda")
    dbg = torch.empty((M, R, C // 128), dtype=torch.int32, device="cuda")
    L.gemv_q(["w"], act, [Y], dbg=dbg)
    want, wdbg = host(Y).copy(), host(dbg).copy()
    recs, n = record(gpudrv, lambda: L.gemv_q(["w"], act, [Y], dbg=dbg))
    assert n == 1
    assert recs[0].fn and recs[0].nargs > 0
    torch.cuda.synchronize()
    # the recording launched nothing: the outputs still hold the direct call's values after a fill
    Y.fill_(np.nan)
    dbg.fill_(-1)
    torch.cuda.synchronize()
    replay_raw(gpudrv, recs, n)
    assert np.array_equal(host(Y), want) and np.array_equal(host(dbg), wdbg)
    # and against the oracle's int32 group values (the records run the product, not a copy of its result)
    acc = orc.tern_acc(bc, R, C, host(act.XQ)[:, :C])
    assert np.array_equal(host(dbg), acc)


@pytest.mark.parametrize("R,C,M,per_row", [(12288, 4096, 512, True), (4096, 12288, 512, True), (2048, 2048, 512, False),
                                           (12288, 4096, 2048, True)])
def test_gemm_records(kt, R, C, M, per_row):
    gpudrv, linear = kt
    say("records gemm", R, C, M, per_row)
    W, bc, dpm = mat(linear, R, C, R * 3 + M)
    L = linear.Linear({"w": W})
    act = linear.quantize(dev(rng(M).normal(0, 1, (M, C)).astype(np.float32)), per_row=per_row)
    Y = torch.empty((M, R), dtype=torch.float32, device="cuda")
    Y16 = torch.empty((M, R), dtype=torch.float16, device="cuda")
    L.gemm("w", act, Y=Y, Y16=Y16)
    want, want16 = host(Y).copy(), host(Y16).copy()
    recs, n = record(gpudrv, lambda: L.gemm("w", act, Y=Y, Y16=Y16))
    assert n == 1
    Y.fill_(np.nan)
    Y16.fill_(np.nan)
    replay_raw(gpudrv, recs, n)
    assert np.array_equal(host(Y), want) and np.array_equal(host(Y16), want16)
    if per_row:
        # the int8-copy product (145 KB of dynamic LDS: the record carries it): the expansion and the product
        W8 = torch.empty(gpudrv.load().kt_tern_expand_bytes(R, C), dtype=torch.int8, device="cuda")
        recs, n = record(gpudrv, lambda: (W.expand(out=W8), L.gemm8("w", act, W8, Y=Y, Y16=Y16)))
        assert n == 2
        Y.fill_(np.nan)
        Y16.fill_(np.nan)
        replay_raw(gpudrv, recs, n)
        assert np.array_equal(host(Y), want) and np.array_equal(host(Y16), want16)


def test_step_plan_chained(kt):
    """a 2B-class decode layer as a plan (linear.Plan: recorded once, replayed): quantize -> q/k/v, and a chain in
    which each product's int8 input is quantized from the previous product's output inside the plan, so a record
    reads what an earlier record wrote. Replayed three times with new inputs in between; each replay equals the
    direct calls on the same inputs."""
    gpudrv, linear = kt
    say("records plan chain")
    H, F = 2048, 6144
    mats = {"q": mat(linear, 2048, H, 1)[0], "k": mat(linear, 512, H, 2)[0], "v": mat(linear, 512, H, 3)[0],
            "o": mat(linear, 2048, H, 4)[0], "gate": mat(linear, F, H, 5)[0], "up": mat(linear, F, H, 6)[0],
            "down": mat(linear, H, F, 7)[0]}
    L = linear.Linear(mats)
    x = torch.empty((1, H), dtype=torch.float32, device="cuda")
    a0, a1, a2 = linear._act_out(1, H, "cuda"), linear._act_out(1, H, "cuda"), linear._act_out(1, F, "cuda")
    y = {n: torch.empty((1, m.R), dtype=torch.float32, device="cuda") for n, m in mats.items()}

    def step():
        linear.quantize(x, out=a0)
        L.gemv_q(["q", "k", "v"], a0, [y["q"], y["k"], y["v"]])
        linear.quantize(y["q"], out=a1)
        L.gemv_q(["o"], a1, [y["o"]])
        L.gemv_q(["gate", "up"], a1, [y["gate"], y["up"]])
        linear.quantize(y["up"], out=a2)
        L.gemv_q(["down"], a2, [y["down"]])

    plan = linear.Plan(step)
    assert plan.n == 7
    for it in range(3):
        x.copy_(dev(rng(50 + it).normal(0, 1, (1, H)).astype(np.float32)))
        step()
        want = {n: host(t).copy() for n, t in y.items()}
        for t in y.values():
            t.fill_(np.nan)
        plan.launch()                                       # kt_replay: the records in one C loop
        for n, t in y.items():
            assert np.array_equal(host(t), want[n]), (it, n)
        for t in y.values():
            t.fill_(np.nan)
        plan.launch_nodes()                                 # Kindi's Replay loop over the node tuples
        for n, t in y.items():
            assert np.array_equal(host(t), want[n]), (it, n)


@pytest.mark.parametrize("M", [1, 4])
def test_moe_and_producer_records(kt, M):
    """the MoE decode chain (two launches at one token, four above; Kindi's sigmoid router) and a fused producer
    (rmsfold) recorded and replayed: the same x and int8 rows as the direct calls"""
    gpudrv, linear = kt
    from kindi_amd import moe
    from kt_cases import q8_case
    say("records moe + rmsfold", M)
    E, H, F, k = 16, 2688, 1856, 6
    ups = moe.Q8Experts([q8_case(F, H, 100 + e)[0] for e in range(E)], F, H)
    downs = moe.Q8Experts([q8_case(H, F, 200 + e)[0] for e in range(E)], H, F)
    bias = dev(rng(3).normal(0, 0.3, E).astype(np.float32))
    layer = moe.MoE(ups, downs, k, score="sigmoid", bias=bias, scale=2.0)
    x0 = dev(rng(M).normal(0, 1, (M, H)).astype(np.float32))
    lg = dev(rng(M + 1).normal(0, 1, (M, E)).astype(np.float32))
    work = layer.workspace(M)
    x = x0.clone()
    layer.decode(x, lg, work)
    want = host(x).copy()
    x.copy_(x0)
    torch.cuda.synchronize()
    recs, n = record(gpudrv, lambda: layer.decode(x, lg, work))
    assert n == (2 if M == 1 else 4)
    assert np.array_equal(host(x), host(x0))                       # recording launched nothing
    replay_raw(gpudrv, recs, n)
    assert np.array_equal(host(x).view(np.uint32), want.view(np.uint32))
    # rmsfold: x + one residual part -> norm -> fold -> int8 row
    C = 5120
    xs = dev(rng(7 + M).normal(0, 1, (M, C)).astype(np.float32))
    r = dev(rng(8 + M).normal(0, 1, (M, C)).astype(np.float32))
    w = dev(rng(9).normal(1, 0.1, C).astype(np.float32))
    sg = dev(np.where(rng(10).random(C) < 0.5, -1.0, 1.0).astype(np.float32))
    out = linear._act_out(M, C, "cuda")
    a1 = linear.rmsfold(xs, w, sg, 1024, r=r, nparts=1, out=out)
    q1, s1, x1 = host(a1.XQ).copy(), host(a1.XS).copy(), host(a1.XA).copy()
    for t in (out.XQ, out.XS, out.XA):
        t.zero_()
    recs, n = record(gpudrv, lambda: linear.rmsfold(xs, w, sg, 1024, r=r, nparts=1, out=out))
    assert n == 1
    replay_raw(gpudrv, recs, n)
    assert np.array_equal(host(out.XQ), q1) and np.array_equal(host(out.XS), s1) and np.array_equal(host(out.XA), x1)

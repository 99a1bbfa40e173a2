"""GPU parity of the ternary path (kt_tern_pack, kt_quant_q8, kt_tern_gemv / gemv3, kt_tern_gemm) against the CPU
oracle. Bars: quantized activations and the int32 group values bit-exact; fp32 outputs bit-exact against the oracle
evaluated in the kernel's documented summation tree, and within 1e-3 relative of the oracle's sequential
(reference-order) value."""
import numpy as np
import pytest
import torch

import oracle as orc
from kt_cases import say, tern_case, dev, host, max_rel, rng

pytestmark = pytest.mark.gpu
TOL = 1e-3                                   # north_star: scaled outputs within 1e-3 relative


@pytest.fixture(scope="module")
def kt():
    assert torch.cuda.is_available(), "GPU tests need the MI355X"
    from kindi_amd import gpudrv, linear
    lib = gpudrv.load()
    return lib, linear


def upload(linear, R, C, seed):
    dig, bc, dpm = tern_case(R, C, seed)
    return linear.TernaryMatrix(bc, dpm, R, C), dig, bc, dpm


@pytest.mark.parametrize("per_row", [False, True])
@pytest.mark.parametrize("M,C", [(1, 128), (3, 2048), (17, 5120), (64, 17408)])
def test_quantizer_bit_exact(kt, M, C, per_row):
    lib, linear = kt
    say("quant", M, C, per_row)
    X = rng(M * 7 + C).normal(0, 1, (M, C)).astype(np.float32)
    X[0, :128] = 0.0                                        # a zero group
    if C > 256:
        X[-1, 256:384] = np.float32(127.0)                  # a group of exact maxima
        X[-1, 300] = np.float32(-63.5)                      # a tie: 63.5 -> 64 (even)
    act = linear.quantize(dev(X), per_row=per_row)
    Q, XS, XA = orc.quant_q8(X, per_row)
    assert np.array_equal(host(act.XQ), Q)
    assert np.array_equal(host(act.XS), XS)
    assert np.array_equal(host(act.XA), XA)


# one token: k_gemv_step (up to 8 steps: C <= 8192; two row groups a block on large grids), k_gemv_flat1 (wider),
# k_gemv_pair (wider rows on grids beyond the wave slots: 10240 x 12288)
SHAPES = [(64, 128), (100, 256), (6144, 2048), (1024, 5120), (2048, 6144), (5120, 17408), (34816, 5120),
          (10240, 12288)]


@pytest.mark.parametrize("R,C", SHAPES)
def test_gemv_m1(kt, R, C):
    lib, linear = kt
    say("gemv M=1", R, C)
    W, dig, bc, dpm = upload(linear, R, C, R + C)
    X = rng(R * 3 + C).normal(0, 1, (1, C)).astype(np.float32)
    L = linear.Linear({"w": W})
    act = linear.quantize(dev(X))
    Y = torch.empty((1, R), dtype=torch.float32, device="cuda")
    dbg = torch.empty((1, R, C // 128), dtype=torch.int32, device="cuda")
    L.gemv_q(["w"], act, [Y], dbg=dbg)
    Q, XS, XA = orc.quant_q8(X)
    acc = orc.tern_acc(bc, R, C, Q)
    assert np.array_equal(host(dbg), acc), "int32 group values"
    dq = dpm.view(np.float16).astype(np.float32)
    tree = orc.out_lanes(acc, XS, dq, 8, 0, lib.kt_decode_kslices(C, 0))
    y = host(Y)
    assert np.array_equal(y, tree), "fp32 in the kernel's summation order"
    seq = orc.tern_out(acc, XS, dpm, R, C)
    assert max_rel(y, seq) < TOL
    # without dbg the output is the same
    Y2 = torch.empty_like(Y)
    L.gemv_q(["w"], act, [Y2])
    assert np.array_equal(host(Y2), y)


@pytest.mark.parametrize("M,C", [(1, 128), (5, 2048), (33, 17408)])
def test_quantizer_hp_bit_exact(kt, M, C):
    """the two-row (hp) quantizer (k_tc_q8 with hp, tc.cu:195-209): both rows, scales and sums bit-exact"""
    lib, linear = kt
    say("quant hp", M, C)
    X = (rng(M + C).normal(0, 1, (M, C)) * np.exp(rng(M).normal(0, 2, (M, 1)))).astype(np.float32)
    X[0, :128] = 0.0
    act = linear.quantize(dev(X), hp=True)
    Q, XS, XA = orc.quant_q8(X, 2)
    assert act.hp and act.M == M and act.XQ.shape[0] == 2 * M
    assert np.array_equal(host(act.XQ), Q) and np.array_equal(host(act.XS), XS) and np.array_equal(host(act.XA), XA)


@pytest.mark.parametrize("R,C", [(640, 1024), (1024, 5120), (5120, 17408), (256, 24576)])
def test_gemv_hp_pairs(kt, R, C):
    """hp decode (tc.cu:405-407): token t's output is the fp32 sum of its two rows' results, row 2t first. Every row's
    result does not depend on M, so the hp product must equal, bit for bit, the one-row product of the same 2M rows
    with each pair added; checked at 1 .. 16 tokens (2 .. 32 rows: the v_dot4 chunks and both matrix-core kernels)
    and against the oracle's tree"""
    lib, linear = kt
    say("gemv hp", R, C)
    W, dig, bc, dpm = upload(linear, R, C, 7 * R + C)
    L = linear.Linear({"w": W})
    X = rng(R + C).normal(0, 1, (16, C)).astype(np.float32)
    Q, XS, XA = orc.quant_q8(X, 2)
    acc = orc.tern_acc(bc, R, C, Q)
    dq = dpm.view(np.float16).astype(np.float32)
    tree = orc.out_lanes(acc, XS, dq, 8, 0, lib.kt_decode_kslices(C, 0))
    want = (tree[0::2] + tree[1::2]).astype(np.float32)
    xd = dev(X)
    for M in (1, 2, 3, 4, 5, 8, 16):
        say("  M", M)
        act = linear.quantize(xd[:M], hp=True)
        Y = torch.full((M, R), float("nan"), dtype=torch.float32, device="cuda")
        dbg = torch.empty((2 * M, R, C // 128), dtype=torch.int32, device="cuda")
        L.gemv_q(["w"], act, [Y], dbg=dbg)
        assert np.array_equal(host(dbg), acc[:2 * M]), M
        assert np.array_equal(host(Y), want[:M]), M
        rows = linear.Act(act.XQ, act.XS, act.XA, 2 * M, C, False)          # the same rows without hp
        Y2 = torch.empty((2 * M, R), dtype=torch.float32, device="cuda")
        L.gemv_q(["w"], rows, [Y2])
        y2 = host(Y2)
        assert np.array_equal(host(Y), (y2[0::2] + y2[1::2]).astype(np.float32)), M


@pytest.mark.parametrize("R,C", [(640, 1024), (2048, 6144), (4096, 4096)])
def test_gemv_token_invariance(kt, R, C):
    """a token's output does not depend on how many tokens share the pass (tc_hip.cu:14-15), for M = 1 .. 32: the
    bandwidth kernels (1 - 2 tokens) and the matrix-core kernels (from 3 tokens; 16x16x64 tiles up to 10 K slices,
    their k-lanes split over 4 waves) give the same bits"""
    lib, linear = kt
    say("gemv T-invariance", R, C)
    W, dig, bc, dpm = upload(linear, R, C, 5 + R)
    L = linear.Linear({"w": W})
    X = rng(9).normal(0, 1, (32, C)).astype(np.float32)
    Xd = dev(X)
    Q, XS, XA = orc.quant_q8(X)
    acc = orc.tern_acc(bc, R, C, Q)
    dq = dpm.view(np.float16).astype(np.float32)
    tree = orc.out_lanes(acc, XS, dq, 8, 0, lib.kt_decode_kslices(C, 0))
    for M in (1, 2, 3, 4, 5, 6, 7, 8, 9, 12, 13, 16, 17, 20, 24, 32):
        act = linear.quantize(Xd[:M])
        Y = torch.empty((M, R), dtype=torch.float32, device="cuda")
        dbg = torch.empty((M, R, C // 128), dtype=torch.int32, device="cuda")
        L.gemv_q(["w"], act, [Y], dbg=dbg)
        assert np.array_equal(host(dbg), acc[:M]), M
        assert np.array_equal(host(Y), tree[:M]), M


@pytest.mark.parametrize("R,C", [(5120, 5120), (1024, 5120), (17408, 5120), (5120, 17408), (256, 24576), (17403, 5120),
                                 (256, 20480), (256, 22528)])
def test_gemv_27b_tokens(kt, R, C):
    """the config 3 shapes at M = 1, 2, 3, 4, 5, 6, 8, 13, 16, 32, against the oracle: every launch kind that serves
    them. The v_dot4 kernels at 1 token, and at 2 below 2^26 weights; from 3 tokens (2 on the 2^26-weight launches)
    the 16x16x64 matrix-core kernel up to 10 K slices, its k-lanes split over 4 waves up to 4 slices (C = 5120), a
    wave taking its k-lane pair of several slices above 4 at up to 8 tokens (C = 17408, 20480) and its k-lane quad
    above 8 tokens; the 32x32x32 kernel above 10 slices (C = 22528, 24576). Edges: a ragged row count (17403:
    a partial last tile and row group), exactly 10 K slices (C = 20480, the 16x16x64 kernel's limit) and 11
    (C = 22528). int32 group values and fp32 outputs bit-exact against the oracle's decode tree, with and without
    the dbg output"""
    lib, linear = kt
    say("gemv 27B tokens", R, C)
    W, dig, bc, dpm = upload(linear, R, C, 3 * R + C)
    L = linear.Linear({"w": W})
    X = rng(R + 11).normal(0, 1, (32, C)).astype(np.float32)
    Xd = dev(X)
    Q, XS, XA = orc.quant_q8(X)
    acc = orc.tern_acc(bc, R, C, Q)
    dq = dpm.view(np.float16).astype(np.float32)
    tree = orc.out_lanes(acc, XS, dq, 8, 0, lib.kt_decode_kslices(C, 0))
    assert max_rel(tree, orc.tern_out(acc, XS, dpm, R, C)) < TOL
    for M in (1, 2, 3, 4, 5, 6, 8, 13, 16, 32):
        say("  M", M)
        act = linear.quantize(Xd[:M])
        Y = torch.empty((M, R), dtype=torch.float32, device="cuda")
        dbg = torch.empty((M, R, C // 128), dtype=torch.int32, device="cuda")
        L.gemv_q(["w"], act, [Y], dbg=dbg)
        assert np.array_equal(host(dbg), acc[:M]), M
        assert np.array_equal(host(Y), tree[:M]), M
        Y2 = torch.full((M, R), float("nan"), dtype=torch.float32, device="cuda")
        L.gemv_q(["w"], act, [Y2])
        assert np.array_equal(host(Y2), tree[:M]), M


@pytest.mark.parametrize("M", [1, 4, 16])
def test_gemv3_gate_up_27b(kt, M):
    """gate and up [17408 x 5120] in one launch at 1, 4 and 16 tokens (one token: two row groups a block): each
    matrix's rows equal its own launch's bits (the multi-matrix offsets of every kernel), and 64 sampled rows of each
    equal the oracle's tree"""
    lib, linear = kt
    say("gemv3 gate/up", M)
    R, C = 17408, 5120
    mats = {n: upload(linear, R, C, s) for n, s in (("gate", 71), ("up", 72))}
    L = linear.Linear({n: m[0] for n, m in mats.items()})
    X = rng(M).normal(0, 1, (M, C)).astype(np.float32)
    act = linear.quantize(dev(X))
    outs = [torch.empty((M, R), dtype=torch.float32, device="cuda") for _ in range(2)]
    L.gemv_q(["gate", "up"], act, outs)
    Q, XS, XA = orc.quant_q8(X)
    rows = np.sort(rng(5).choice(R, 64, replace=False))
    for n, o in zip(("gate", "up"), outs):
        one = torch.empty((M, R), dtype=torch.float32, device="cuda")
        L.gemv_q([n], act, [one])
        assert torch.equal(one, o), n
        W, dig, bc, dpm = mats[n]
        acc = orc.tern_acc(np.ascontiguousarray(bc[:, rows]), 64, C, Q)
        dq = np.ascontiguousarray(dpm[:, rows]).view(np.float16).astype(np.float32)
        assert np.array_equal(host(o)[:, rows], orc.out_lanes(acc, XS, dq, 8, 0, lib.kt_decode_kslices(C, 0))), n


@pytest.mark.parametrize("R,M,sp", [(100, 1, 1), (5120, 1, 3), (5120, 5, 9), (333, 4, 17), (6144, 2, 16)])
def test_tern_sum(kt, R, M, sp):
    """kt_tern_sum (k_tc_sum, tc_hip.cu:271-279): the parts added in part order, bit-exact against the oracle; a
    case where another order gives other bits is included (large and small parts of both signs)"""
    lib, linear = kt
    say("tern_sum", R, M, sp)
    r = rng(R + sp)
    P = (r.normal(0, 1, (M, sp, R)) * np.exp(r.normal(0, 6, (M, sp, R)))).astype(np.float32)
    want = orc.tern_sum(P.reshape(-1), R, M, sp)
    Pd = dev(P)
    y = torch.full((M, R), float("nan"), dtype=torch.float32, device="cuda")
    from kindi_amd import gpudrv
    gpudrv.check(lib.kt_tern_sum(Pd.data_ptr(), y.data_ptr(), R, M, sp, None), "kt_tern_sum")
    assert np.array_equal(host(y), want)
    if sp >= 3:
        rev = P[:, ::-1, :].astype(np.float32)
        other = np.zeros((M, R), np.float32)
        for p in range(sp):
            other = (other + rev[:, p, :]).astype(np.float32)
        assert not np.array_equal(other, want)          # the order is observable on these inputs


@pytest.mark.parametrize("per_row", [False, True])
@pytest.mark.parametrize("R,C", [(6144, 2048), (2048, 2048), (512, 2048), (2048, 6144)])
def test_gemv_vs_kcpu(kt, R, C, per_row):
    """the kcpu.c half of the parity bar (kcpu.c:72-135): the CPU engine's fp32 pair-table GEMV (the oracle's
    restatement, pinned bit-exact to kcpu.c's own gemv; the reference build itself where it travelled) run on the
    dequantized activations x^ = q XS equals the GPU product of the quantized row within 1e-3 relative (configs 0
    and 1: per-row and per-group scales)"""
    lib, linear = kt
    say("gemv vs kcpu", R, C, per_row)
    W, dig, bc, dpm = upload(linear, R, C, R + 3 * C)
    L = linear.Linear({"w": W})
    X = rng(C + R).normal(0, 1, (1, C)).astype(np.float32)
    act = linear.quantize(dev(X), per_row=per_row)
    Y = torch.empty((1, R), dtype=torch.float32, device="cuda")
    L.gemv_q(["w"], act, [Y])
    Q, XS, XA = orc.quant_q8(X, per_row)
    xhat = (Q[0].astype(np.float32).reshape(-1, 128) * XS[0][:, None]).reshape(-1).astype(np.float32)
    Pc = orc.paircodes_fast(bc, R, C)
    S = orc.pair_scales(dpm, R, C)
    y_cpu = orc.pair_gemv(Pc, S, R, C, xhat)
    y = host(Y)[0]
    assert max_rel(y, y_cpu) < TOL
    assert max_rel(y, y_cpu) < 1e-5                     # in practice: only fp32 summation-order differences
    if orc.ref_kcpu() is not None:
        assert np.array_equal(orc.ref_gemv(Pc, S, R, C, xhat), y_cpu)


def test_gemv3_qkv(kt):
    """q / k / v of the 2B layer in one launch (k_tc_mv3, spec.py:659-673), M = 4"""
    lib, linear = kt
    say("gemv3 qkv")
    C, M = 2048, 4
    mats = {n: upload(linear, R, C, s) for n, R, s in (("q", 2048, 1), ("k", 512, 2), ("v", 512, 3))}
    L = linear.Linear({n: m[0] for n, m in mats.items()})
    X = rng(4).normal(0, 1, (M, C)).astype(np.float32)
    outs = [torch.empty((M, mats[n][0].R), dtype=torch.float32, device="cuda") for n in "qkv"]
    assert L.gemv(["q", "k", "v"], dev(X), outs) == 1
    for n, o in zip("qkv", outs):
        W, dig, bc, dpm = mats[n]
        ref, acc, (Q, XS, XA) = orc.tern_linear(bc, dpm, W.R, C, X)
        assert max_rel(host(o), ref) < TOL, n
        assert np.array_equal(host(o), orc.out_lanes(acc, XS, dpm.view(np.float16).astype(np.float32), 8, 0, lib.kt_decode_kslices(C, 0))), n
        # a separate launch of the same tensor gives the same bits
        Y1 = torch.empty_like(o)
        L.gemv_q([n], linear.quantize(dev(X)), [Y1])
        assert np.array_equal(host(Y1), host(o)), n


@pytest.mark.parametrize("R,C,M", [(128, 256, 128), (100, 256, 5), (256, 512, 300), (384, 1024, 200)])
def test_gemm_small(kt, R, C, M):
    lib, linear = kt
    say("gemm", R, C, M)
    W, dig, bc, dpm = upload(linear, R, C, R * 11 + M)
    L = linear.Linear({"w": W})
    X = rng(M + 1).normal(0, 1, (M, C)).astype(np.float32)
    act = linear.quantize(dev(X))
    Y = torch.empty((M, R), dtype=torch.float32, device="cuda")
    Y16 = torch.empty((M, R), dtype=torch.float16, device="cuda")
    dbg = torch.empty((M, R, C // 128), dtype=torch.int32, device="cuda")
    L.gemm("w", act, Y=Y, Y16=Y16, dbg=dbg)
    Q, XS, XA = orc.quant_q8(X)
    acc = orc.tern_acc(bc, R, C, Q)
    assert np.array_equal(host(dbg), acc), "int32 group values"
    seq = orc.tern_out(acc, XS, dpm, R, C)
    y = host(Y)
    assert np.array_equal(y, seq), "fp32: groups in order, the reference expression"
    assert np.array_equal(host(Y16), seq.astype(np.float16))


@pytest.mark.parametrize("R,C,M", [(128, 256, 128), (100, 384, 5), (256, 512, 300), (384, 1024, 200),
                                   (8192, 128, 1024), (8100, 256, 1000), (8200, 256, 130)])
def test_gemm_per_row(kt, R, C, M):
    """per-row activation scales (the per-row order on both block shapes: small blocks below 8192 rows, 128 x 128
    from 8192; ragged rows and tokens): int32 group values exact, fp32 bit-exact in the documented order, fp16 its
    rounding, and within the tolerance of the reference's sequential order"""
    lib, linear = kt
    say("gemm per-row", R, C, M)
    W, dig, bc, dpm = upload(linear, R, C, R * 7 + M)
    L = linear.Linear({"w": W})
    X = rng(M + 2).normal(0, 1, (M, C)).astype(np.float32)
    act = linear.quantize(dev(X), per_row=True)
    Y = torch.empty((M, R), dtype=torch.float32, device="cuda")
    Y16 = torch.empty((M, R), dtype=torch.float16, device="cuda")
    dbg = torch.empty((M, R, C // 128), dtype=torch.int32, device="cuda")
    L.gemm("w", act, Y=Y, Y16=Y16, dbg=dbg)
    Q, XS, XA = orc.quant_q8(X, per_row=True)
    acc = orc.tern_acc(bc, R, C, Q)
    assert np.array_equal(host(dbg), acc), "int32 group values"
    seq = orc.tern_out(acc, XS, dpm, R, C)
    want = orc.tern_out_rs(acc, XS, dpm, R, C)                             # the per-row order at every R
    y = host(Y)
    assert np.array_equal(y, want), "fp32 in the documented order"
    assert np.array_equal(host(Y16), want.astype(np.float16))
    assert max_rel(y, seq) < TOL
    # without the debug output (the other instantiation) the same bits
    Y2 = L.gemm("w", act)
    assert np.array_equal(host(Y2), y)


@pytest.mark.parametrize("R,C,M", [(12288, 4096, 512), (4096, 12288, 512), (12288, 4096, 2048), (4096, 12288, 2048)])
def test_gemm_config2_sampled(kt, R, C, M):
    """config 2 shapes at M = 512 and 2048: int32 group values and outputs of 96 sampled rows against the oracle, all rows
    against the decode kernel's fp32 output for 16 tokens (the same int32 values, another summation tree)"""
    lib, linear = kt
    say("gemm config2", R, C, M)
    import kindi_amd.synth as syn
    bc_t, dpm_t = syn.tern_pack(R, C, 20, device="cuda")
    W = linear.TernaryMatrix(bc_t, dpm_t, R, C)
    L = linear.Linear({"w": W})
    Xd = syn.activations(M, C, 22, device="cuda")
    act = linear.quantize(Xd, per_row=True)
    rows = np.sort(rng(1).choice(R, 96, replace=False))
    dbg = torch.empty((M, R, C // 128), dtype=torch.int32, device="cuda")
    Y = torch.empty((M, R), dtype=torch.float32, device="cuda")
    L.gemm("w", act, Y=Y, dbg=dbg)
    Y2 = L.gemm("w", act)                                                   # the instantiation without dbg
    assert torch.equal(Y, Y2)
    bc = host(bc_t)[:, rows]
    dpm = host(dpm_t).view(np.uint16)[:, rows]
    X = host(Xd)
    Q, XS, XA = orc.quant_q8(X, per_row=True)
    assert np.array_equal(host(act.XQ), Q)
    acc = orc.tern_acc(np.ascontiguousarray(bc), len(rows), C, Q)
    assert np.array_equal(host(dbg[:, torch.from_numpy(rows).cuda()]), acc), "int32 group values"
    del dbg
    seq = orc.tern_out(acc, XS, np.ascontiguousarray(dpm), len(rows), C)
    want = orc.tern_out_rs(acc, XS, np.ascontiguousarray(dpm), len(rows), C)
    y = host(Y)
    assert np.array_equal(y[:, rows], want), "documented order"
    assert max_rel(y[:, rows], seq) < TOL
    Yd = torch.empty((16, R), dtype=torch.float32, device="cuda")
    sub = linear.quantize(Xd[:16], per_row=True)
    L.gemv_q(["w"], sub, [Yd])
    assert max_rel(host(Yd), y[:16]) < 1e-5


@pytest.mark.parametrize("R,C", [(8, 128), (24, 384), (200, 1152), (64, 896), (100, 2944), (1000, 1408)])
def test_gemv_ragged_units(kt, R, C):
    """widths whose group count is not a multiple of 8 (a partial last step), row counts of one row group and rows
    that end inside a 32-row tile, at every decode kernel's token counts (v_dot4 chunks 1 .. 5, the 32x32x32
    matrix-core kernel at 6 .. 8, the 16x16x64 one above 8) and in the two-row (hp) form"""
    lib, linear = kt
    say("gemv ragged", R, C)
    W, dig, bc, dpm = upload(linear, R, C, 7 * R + C)
    L = linear.Linear({"w": W})
    X = rng(R).normal(0, 1, (32, C)).astype(np.float32)
    Q, XS, XA = orc.quant_q8(X)
    acc = orc.tern_acc(bc, R, C, Q)
    dq = dpm.view(np.float16).astype(np.float32)
    tree = orc.out_lanes(acc, XS, dq, 8, 0, lib.kt_decode_kslices(C, 0))
    xd = dev(X)
    for M in (1, 3, 6, 8, 9, 13, 16, 32):
        act = linear.quantize(xd[:M])
        Y = torch.full((M, R), float("nan"), dtype=torch.float32, device="cuda")
        dbg = torch.empty((M, R, C // 128), dtype=torch.int32, device="cuda")
        L.gemv_q(["w"], act, [Y], dbg=dbg)
        assert np.array_equal(host(dbg), acc[:M]), M
        assert np.array_equal(host(Y), tree[:M]), M
    act = linear.quantize(xd[:3])
    Yp = L.gemm("w", act)
    assert np.array_equal(host(Yp), orc.tern_out(acc[:3], XS[:3], dpm, R, C))
    Qh, XSh, XAh = orc.quant_q8(X[:16], 2)
    th = orc.out_lanes(orc.tern_acc(bc, R, C, Qh), XSh, dq, 8, 0, lib.kt_decode_kslices(C, 0))
    for M in (1, 3, 5, 16):                                     # hp: 2 .. 32 rows
        act = linear.quantize(xd[:M], hp=True)
        Y = torch.full((M, R), float("nan"), dtype=torch.float32, device="cuda")
        L.gemv_q(["w"], act, [Y])
        assert np.array_equal(host(Y), (th[0:2 * M:2] + th[1:2 * M:2]).astype(np.float32)), M


def test_gemv_full_size_linearity(kt):
    """config 3 gate shape [17408 x 5120]: the exact group values are linear in the int8 input (v(q1 + q2) =
    v(q1) + v(q2)), checked over every row; 64 sampled rows against the oracle"""
    lib, linear = kt
    say("gemv 27B gate linearity")
    import kindi_amd.synth as syn
    R, C = 17408, 5120
    bc_t, dpm_t = syn.tern_pack(R, C, 104, device="cuda")
    W = linear.TernaryMatrix(bc_t, dpm_t, R, C)
    L = linear.Linear({"w": W})
    r = rng(3)
    q1 = r.integers(-63, 64, (2, C)).astype(np.int8)
    q2 = r.integers(-63, 64, (2, C)).astype(np.int8)
    outs = []
    for q in (q1, q2, (q1.astype(np.int16) + q2).astype(np.int8)):
        XS = np.ones((2, C // 128), np.float32)
        XA = q.astype(np.int32).reshape(2, -1, 128).sum(2).astype(np.int32)
        act = linear.Act(dev(q), dev(XS), dev(XA), 2, C, False)
        dbg = torch.empty((2, R, C // 128), dtype=torch.int32, device="cuda")
        Y = torch.empty((2, R), dtype=torch.float32, device="cuda")
        L.gemv_q(["w"], act, [Y], dbg=dbg)
        outs.append(host(dbg))
    assert np.array_equal(outs[0] + outs[1], outs[2])
    rows = np.sort(r.choice(R, 64, replace=False))
    acc = orc.tern_acc(np.ascontiguousarray(host(bc_t)[:, rows]), 64, C, q1)
    assert np.array_equal(outs[0][:, rows], acc)


def test_repeated_launches_same_bits(kt):
    """back-to-back launches alternating shapes reproduce the same bits every time"""
    lib, linear = kt
    say("repeated launches x300")
    shapes = [(1024, 5120), (5120, 5120), (640, 2048)]
    acts, refs, outs = {}, {}, {}
    L = linear.Linear({})
    for i, (R, C) in enumerate(shapes):
        L.add(str(i), upload(linear, R, C, 50 + i)[0])
        acts[i] = linear.quantize(dev(rng(i).normal(0, 1, (1, C)).astype(np.float32)))
        outs[i] = torch.empty((1, R), dtype=torch.float32, device="cuda")
        L.gemv_q([str(i)], acts[i], [outs[i]])
        refs[i] = host(outs[i]).copy()
    bad = 0
    for k in range(300):
        i = k % 3
        outs[i].fill_(float("nan"))
        L.gemv_q([str(i)], acts[i], [outs[i]])
        if k % 10 == 9 or k > 290:
            bad += int(not np.array_equal(host(outs[i]), refs[i]))
    assert bad == 0


@pytest.mark.parametrize("R,C", [(8, 128), (100, 256), (6144, 2048), (1024, 17408)])
def test_pack_from_ptq1(kt, R, C, tmp_path):
    """the GGUF PTQ1_0 tensor decoded on the device gives the same kt2 bytes as the reference pack of the same
    digits (through kt_tern_pack), whole and streamed from a file in row chunks (ragged last chunk)"""
    lib, linear = kt
    say("ptq1", R, C)
    dig, bc, dpm = tern_case(R, C, R + C)
    NG = C // 128
    raw = orc.ptq1_from_digits(dig.reshape(R * NG, 128), np.ascontiguousarray(dpm.T).reshape(R * NG))
    assert np.array_equal(orc.trits_from_ptq1(raw).reshape(R, C), dig)
    want = host(linear.TernaryMatrix(bc, dpm, R, C).W)
    got = linear.TernaryMatrix.from_ptq1(raw, R, C)
    assert np.array_equal(host(got.W), want)
    f = tmp_path / "t.gguf"
    pad = 96
    with open(f, "wb") as fh:
        fh.write(b"\0" * pad)
        fh.write(raw.tobytes())
    m = linear.load_ptq1(str(f), pad, R, C, chunk_rows=40)
    assert np.array_equal(host(m.W), want)


@pytest.mark.parametrize("R,C", [(16, 512), (6144, 2048), (1024, 17408)])
def test_pack_from_layout(kt, R, C):
    """a tensor in Kindi's load-time GEMV layout (the oracle's restatement of layout.repack) gives the same kt2 bytes
    as the reference pack it came from (so every product over it has the same bits)"""
    lib, linear = kt
    say("layout", R, C)
    dig, bc, dpm = tern_case(R, C, 3 * R + C)
    wg, sg = orc.layout_g4(bc, dpm, R, C)
    want = linear.TernaryMatrix(bc, dpm, R, C)
    got = linear.TernaryMatrix.from_layout(wg, sg, R, C)
    assert np.array_equal(host(got.W), host(want.W))
    assert want.W.numel() == lib.kt_tern_weight_bytes(R, C)


def _gguf_bytes(tensors, kv):
    """a small GGUF v3 file: kv {key: (type, value)}, tensors [(name, dims, type, data bytes)]"""
    import struct
    s = lambda x: struct.pack("<Q", len(x.encode())) + x.encode()
    out = b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(kv))
    for k, (ty, v) in kv.items():
        out += s(k) + struct.pack("<I", ty)
        if ty == 8:
            out += s(v)
        elif ty == 9:
            out += struct.pack("<IQ", 4, len(v)) + b"".join(struct.pack("<I", x) for x in v)
        else:
            out += struct.pack("<I", v)
    off, datas = 0, []
    for name, dims, ty, data in tensors:
        out += s(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        out += struct.pack("<IQ", ty, off)
        datas.append((off, data))
        off = (off + len(data) + 31) // 32 * 32
    out += b"\0" * ((len(out) + 31) // 32 * 32 - len(out))
    body = bytearray(off)
    for o, d in datas:
        body[o:o + len(d)] = d
    return out + bytes(body)


def test_gguf_ptq1_by_name(kt, tmp_path):
    lib, linear = kt
    from kindi_amd import gguf
    say("gguf")
    tens, wants = [], {}
    for i, (R, C) in enumerate([(24, 256), (16, 128)]):
        dig, bc, dpm = tern_case(R, C, 50 + i)
        NG = C // 128
        raw = orc.ptq1_from_digits(dig.reshape(R * NG, 128), np.ascontiguousarray(dpm.T).reshape(R * NG))
        tens.append(("blk.%d.ffn_up.weight" % i, [C, R], gguf.PTQ1_0, raw.tobytes()))
        wants[tens[-1][0]] = host(linear.TernaryMatrix(bc, dpm, R, C).W)
    f = tmp_path / "m.gguf"
    f.write_bytes(_gguf_bytes(tens, {"general.architecture": (8, "test"), "general.alignment": (4, 32),
                                     "x.list": (9, [1, 2, 3])}))
    g = gguf.GGUF(str(f))
    assert g.kv["general.architecture"] == "test" and g.kv["x.list"] == [1, 2, 3]
    for name, want in wants.items():
        m = gguf.load_ternary(str(f), name, chunk_rows=8, g=g)
        assert np.array_equal(host(m.W), want), name


@pytest.mark.parametrize("R,C,M", [(64, 128, 1), (100, 256, 7), (300, 384, 130), (2048, 2048, 512),
                                   (8200, 128, 1000), (8200, 256, 1000), (8200, 384, 1000), (8200, 640, 1000),
                                   (12288, 4096, 700), (4096, 12288, 2048), (12288, 1024, 512),
                                   (12288, 128, 1500), (12288, 256, 2048), (12288, 384, 2048)])
def test_gemm8(kt, R, C, M):
    """the int8-trit prefill product (kt_tern_expand + kt_tern_gemm8): the expanded trits equal the pack's digits - 1,
    the int32 group values equal the oracle's, and Y / Y16 carry the bits of kt_tern_gemm with per-row activations.
    Grids of at least 0.7 of a 128 x 256 tile a CU run the DMA kernel (ragged rows and tokens; 1, 2, 3 and 5 groups:
    every turn of its two-group loop and both tails; 192 tiles on fewer blocks than CUs; 2 and 3 tiles a block, so
    the DMAs run ahead across tile ends and the token-scale slots rotate); smaller ones the packed-trit kernel"""
    lib, linear = kt
    say("gemm8", R, C, M)
    W, dig, bc, dpm = upload(linear, R, C, R * 5 + M)
    W8 = W.expand()
    w8 = host(W8).reshape(-1, C)
    assert w8.shape[0] == (R + 7) // 8 * 8
    assert np.array_equal(w8[:R], dig.astype(np.int16) - 1)
    L = linear.Linear({"w": W})
    X = rng(M + 9).normal(0, 1, (M, C)).astype(np.float32)
    act = linear.quantize(dev(X), per_row=True)
    Y = torch.empty((M, R), dtype=torch.float32, device="cuda")
    Y16 = torch.empty((M, R), dtype=torch.float16, device="cuda")
    L.gemm("w", act, Y=Y, Y16=Y16)
    Y8 = torch.full((M, R), np.nan, dtype=torch.float32, device="cuda")
    Y8h = torch.empty((M, R), dtype=torch.float16, device="cuda")
    L.gemm8("w", act, W8, Y=Y8, Y16=Y8h)
    assert np.array_equal(host(Y8).view(np.uint32), host(Y).view(np.uint32))
    assert np.array_equal(host(Y8h).view(np.uint16), host(Y16).view(np.uint16))
    if R * M * (C // 128) <= (1 << 24):
        dbg = torch.empty((M, R, C // 128), dtype=torch.int32, device="cuda")
        Y2 = L.gemm8("w", act, W8, dbg=dbg)
        Q, XS, XA = orc.quant_q8(X, per_row=True)
        assert np.array_equal(host(dbg), orc.tern_acc(bc, R, C, Q))
        assert np.array_equal(host(Y2).view(np.uint32), host(Y).view(np.uint32))


@pytest.mark.parametrize("pad", [8, 4])
def test_gemm8_strided_rows(kt, pad):
    """the int8-trit prefill product into rows of a wider buffer (ldy = R + pad): a pad that keeps the 16-byte row
    stores aligned (8 fp16 / fp32 elements) runs the DMA kernel, one that does not the packed-trit kernel; both write
    exactly the R columns of each row, with kt_tern_gemm's bits, and leave the pad untouched; and kt_tern_gemm itself
    into the same rows"""
    lib, linear = kt
    R, C, M = 12288, 1024, 512
    say("gemm8 strided", R, C, M, pad)
    W, dig, bc, dpm = upload(linear, R, C, 77 + pad)
    W8 = W.expand()
    L = linear.Linear({"w": W})
    X = rng(pad).normal(0, 1, (M, C)).astype(np.float32)
    act = linear.quantize(dev(X), per_row=True)
    Y = torch.empty((M, R), dtype=torch.float32, device="cuda")
    Y16 = torch.empty((M, R), dtype=torch.float16, device="cuda")
    L.gemm("w", act, Y=Y, Y16=Y16)
    B = torch.full((M, R + pad), 7.0, dtype=torch.float32, device="cuda")
    B16 = torch.full((M, R + pad), 7.0, dtype=torch.float16, device="cuda")
    L.gemm8("w", act, W8, Y=B[:, :R], Y16=B16[:, :R])
    assert np.array_equal(host(B[:, :R]).view(np.uint32), host(Y).view(np.uint32))
    assert np.array_equal(host(B16[:, :R]).view(np.uint16), host(Y16).view(np.uint16))
    assert bool((B[:, R:] == 7.0).all()) and bool((B16[:, R:] == 7.0).all())
    # the packed-trit product itself into the same wider rows (its 16-byte fp16 row stores need the aligned pad)
    B.fill_(7.0)
    B16.fill_(7.0)
    L.gemm("w", act, Y=B[:, :R], Y16=B16[:, :R])
    assert np.array_equal(host(B[:, :R]).view(np.uint32), host(Y).view(np.uint32))
    assert np.array_equal(host(B16[:, :R]).view(np.uint16), host(Y16).view(np.uint16))
    assert bool((B[:, R:] == 7.0).all()) and bool((B16[:, R:] == 7.0).all())

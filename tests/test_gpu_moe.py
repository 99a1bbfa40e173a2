"""GPU parity of the q8_0 path (kt_q8_pack, kt_q8_quant, kt_q8_gemv) and the MoE dispatch (kt_moe_topk(_r),
kt_moe_sort, kt_q8_grouped, kt_moe_combine, kt_moe_decode(_r)) against the CPU oracle, with BASELINE's softmax router
and Kindi's sigmoid + bias router (lightning.cu:373-468)."""
import numpy as np
import pytest
import torch

import oracle as orc
from kt_cases import say, q8_case, dev, host, max_rel, rng

pytestmark = pytest.mark.gpu
TOL = 1e-3


@pytest.fixture(scope="module")
def kt():
    assert torch.cuda.is_available(), "GPU tests need the MI355X"
    from kindi_amd import gpudrv, moe
    return gpudrv.load(), moe


@pytest.mark.parametrize("act", [0, 1])
@pytest.mark.parametrize("M,C", [(1, 32), (5, 1856), (256, 2688)])
def test_q8_quant_bit_exact(kt, M, C, act):
    lib, moe = kt
    say("q8 quant", M, C, act)
    X = rng(M + C).normal(0, 1, (M, C)).astype(np.float32)
    X[0, :32] = 0.0
    Q, D = moe.q8_quantize(dev(X), act)
    Xr = np.maximum(X, np.float32(0)) * np.maximum(X, np.float32(0)) if act else X
    q, d = orc.q8_quant(Xr.astype(np.float32))
    assert np.array_equal(host(Q), q)
    assert np.array_equal(host(D), d)


@pytest.mark.parametrize("R,C,M", [(64, 32, 1), (100, 96, 3), (1856, 2688, 1), (2688, 1856, 6), (1856, 2688, 16),
                                   (100, 96, 13), (2688, 1856, 40)])
def test_q8_gemv(kt, R, C, M):
    lib, moe = kt
    say("q8 gemv", R, C, M)
    rows, codes, sc = q8_case(R, C, R + C + M)
    W = moe.Q8Matrix(rows, R, C)
    X = rng(M).normal(0, 1, (M, C)).astype(np.float32)
    Q, D = moe.q8_quantize(dev(X))
    dbg = torch.empty((M, R, C // 32), dtype=torch.int32, device="cuda")
    Y = W.gemv(Q, D, dbg=dbg)
    q, d = orc.q8_quant(X)
    acc = orc.q8_acc(rows, R, C, q)
    assert np.array_equal(host(dbg), acc)
    dq = np.ascontiguousarray(sc.view(np.float16).astype(np.float32).T)
    tree = orc.out_lanes(acc, d, dq, 8, 1, lib.kt_decode_kslices(C, 1))
    y = host(Y)
    assert np.array_equal(y, tree)
    assert max_rel(y, orc.q8_out(acc, rows, R, C, d)) < TOL


@pytest.mark.parametrize("R", [96, 100])
@pytest.mark.parametrize("C", [512, 1024, 1536, 1856, 2688, 3584, 4096])
def test_grouped_mma_widths(kt, C, R):
    """the grouped matrix-core q8_0 product (16 entries an expert on average) at widths of 1 to 8 K slices: one slice
    a wave (up to 2 slices) and two waves taking the slices in turn (3 to 8, odd counts included). int32 unit values
    exact against the oracle, and every expert's rows bit-identical to the dense product of the same tokens"""
    lib, moe = kt
    E, k, M = 16, 4, 64
    say("grouped mma", R, C, "KS", lib.kt_decode_kslices(C, 1))
    rows = [q8_case(R, C, 300 + e)[0] for e in range(E)]
    ups = moe.Q8Experts(rows, R, C)
    # the token lists depend on the ids and E only: a layer of small placeholder experts makes them
    layer = moe.MoE(moe.Q8Experts([q8_case(32, 32, e)[0] for e in range(E)], 32, 32),
                    moe.Q8Experts([q8_case(32, 32, 50 + e)[0] for e in range(E)], 32, 32), k)
    r = rng(C)
    ids = np.stack([r.permutation(E)[:k] for _ in range(M)]).astype(np.int32)
    lists = layer.lists(dev(ids))
    X = r.normal(0, 1, (M, C)).astype(np.float32)
    Q, D = moe.q8_quantize(dev(X))
    q, d = orc.q8_quant(X)
    n = M * k
    Y = torch.empty((n, R), dtype=torch.float32, device="cuda")
    dbg = torch.empty((n, R, C // 32), dtype=torch.int32, device="cuda")
    ups.grouped(lists, M, Q, D, Y, xrow=True, dbg=dbg)
    Y2 = torch.full((n, R), float("nan"), dtype=torch.float32, device="cuda")
    ups.grouped(lists, M, Q, D, Y2, xrow=True)
    assert np.array_equal(host(Y).view(np.uint32), host(Y2).view(np.uint32))
    cnt, off, xrow, where = orc.moe_sort(ids, E)
    y, g = host(Y), host(dbg)
    for e in range(E):
        p = np.arange(off[e], off[e] + cnt[e])
        assert np.array_equal(g[p], orc.q8_acc(rows[e], R, C, q[xrow[p]])), e
        idx = torch.from_numpy(xrow[p]).cuda().long()
        dense = moe.Q8Matrix(rows[e], R, C).gemv(Q[idx], D[idx])
        assert np.array_equal(host(dense).view(np.uint32), y[p].view(np.uint32)), e


def test_grouped_mma_odd_experts(kt):
    """the grouped matrix-core product with an expert count that is not a multiple of 8 (13 experts, 3 picks, 64
    tokens: about 15 entries an expert, the matrix-core path): every expert's rows bit-identical to the dense
    product"""
    lib, moe = kt
    E, k, M, R, C = 13, 3, 64, 100, 2688
    say("grouped mma odd E", E, R, C)
    rows = [q8_case(R, C, 700 + e)[0] for e in range(E)]
    ups = moe.Q8Experts(rows, R, C)
    layer = moe.MoE(moe.Q8Experts([q8_case(32, 32, e)[0] for e in range(E)], 32, 32),
                    moe.Q8Experts([q8_case(32, 32, 90 + e)[0] for e in range(E)], 32, 32), k)
    r = rng(C + E)
    ids = np.stack([r.permutation(E)[:k] for _ in range(M)]).astype(np.int32)
    lists = layer.lists(dev(ids))
    X = r.normal(0, 1, (M, C)).astype(np.float32)
    Q, D = moe.q8_quantize(dev(X))
    n = M * k
    Y = torch.full((n, R), float("nan"), dtype=torch.float32, device="cuda")
    ups.grouped(lists, M, Q, D, Y, xrow=True)
    cnt, off, xrow, where = orc.moe_sort(ids, E)
    y = host(Y)
    for e in range(E):
        p = np.arange(off[e], off[e] + cnt[e])
        idx = torch.from_numpy(xrow[p]).cuda().long()
        dense = moe.Q8Matrix(rows[e], R, C).gemv(Q[idx], D[idx])
        assert np.array_equal(host(dense).view(np.uint32), y[p].view(np.uint32)), e


@pytest.mark.parametrize("E,M", [(60, 1), (60, 300), (1024, 200), (1000, 700)])
def test_sort_wide(kt, E, M):
    """kt_moe_sort at other expert counts (not a power of two, the 1024 maximum), one expert taking half the
    entries, several 1024-entry chunks: the lists equal the oracle's (stable order)"""
    lib, moe = kt
    say("sort wide", E, M)
    from kindi_amd.linear import ptr, stream
    k = 6
    ids = rng(E + M).integers(0, E, (M, k)).astype(np.int32)
    ids[: (M + 1) // 2, 0] = E - 1
    d = dev(ids)
    cnt, off, xrow, where, act = [torch.empty(n, dtype=torch.int32, device="cuda") for n in (E, E, M * k, M * k, E)]
    nact = torch.empty(1, dtype=torch.int32, device="cuda")
    assert lib.kt_moe_sort(ptr(d), M, k, E, ptr(cnt), ptr(off), ptr(xrow), ptr(where), ptr(act), ptr(nact),
                           stream()) == 0
    rc, ro, rx, rw = orc.moe_sort(ids, E)
    assert np.array_equal(host(cnt), rc) and np.array_equal(host(off), ro)
    assert np.array_equal(host(xrow), rx) and np.array_equal(host(where), rw)
    active = np.nonzero(rc)[0]
    assert host(nact)[0] == len(active) and np.array_equal(host(act)[:len(active)], active)


def test_topk_and_sort(kt):
    lib, moe = kt
    say("topk + sort")
    E, k = 128, 6
    ups = moe.Q8Experts([q8_case(64, 32, e)[0] for e in range(E)], 64, 32)
    downs = moe.Q8Experts([q8_case(32, 64, 500 + e)[0] for e in range(E)], 32, 64)
    layer = moe.MoE(ups, downs, k)
    for M in (1, 2, 10, 37, 256, 700):
        lg = rng(M).normal(0, 1, (M, E)).astype(np.float32)
        if M == 37:
            lg[3, [10, 11, 12, 13, 14, 15, 16]] = 5.0                # a tie across the k-th place
        ids, gw = layer.route(dev(lg))
        rid, rgw = orc.router_topk(lg, k)
        assert np.array_equal(host(ids), rid), M
        assert np.allclose(host(gw), rgw, rtol=2e-6, atol=1e-7), M
        lists = layer.lists(ids)
        cnt, off, xrow, where = orc.moe_sort(rid, E)
        got = [host(t) for t in lists]
        assert np.array_equal(got[0], cnt) and np.array_equal(got[1], off)
        assert np.array_equal(got[2], xrow) and np.array_equal(got[3], where)
        active = np.nonzero(cnt)[0]
        assert got[5][0] == len(active) and np.array_equal(got[4][:len(active)], active)
        if M * k <= 64:                                             # the one-launch router + lists
            xr = rng(M + 5).normal(0, 1, (M, 96)).astype(np.float32)
            xr[0, 32:64] = 0.0                                      # a zero block
            Qr = torch.empty((M, 96), dtype=torch.int8, device="cuda")
            Dr = torch.empty((M, 3), dtype=torch.float32, device="cuda")
            ids2, gw2, lists2 = layer.route_lists(dev(lg), dev(xr), Qr, Dr)
            Q1, D1 = moe.q8_quantize(dev(xr))
            assert np.array_equal(host(Qr), host(Q1)) and np.array_equal(host(Dr), host(D1)), M
            assert np.array_equal(host(ids2), rid) and np.array_equal(host(gw2), host(gw)), M
            for a_, b_ in zip(lists2[:4], lists[:4]):
                assert np.array_equal(host(a_), host(b_)), M
            n2 = int(host(lists2[5])[0])                           # act: only its first nact entries are defined
            assert n2 == len(active) and np.array_equal(host(lists2[4])[:n2], active), M


def test_topk_wide(kt):
    """E = 1000 logits (16 a lane), k = 16, with ties and -inf entries"""
    lib, moe = kt
    say("topk wide")
    E, k, M = 1000, 16, 5
    lg = rng(9).normal(0, 1, (M, E)).astype(np.float32)
    lg[1, 500:520] = 3.0
    lg[2, :] = -np.inf
    lg[2, [7, 900]] = 1.0
    ids = torch.empty((M, k), dtype=torch.int32, device="cuda")
    gw = torch.empty((M, k), dtype=torch.float32, device="cuda")
    from kindi_amd.linear import ptr, stream
    assert lib.kt_moe_topk(ptr(dev(lg)), M, E, k, ptr(ids), ptr(gw), stream()) == 0
    rid, rgw = orc.router_topk(lg, k)
    assert np.array_equal(host(ids), rid)
    assert np.allclose(host(gw), rgw, rtol=2e-6, atol=1e-7, equal_nan=True)


def oracle_moe(x, lg, up_rows, down_rows, H, F, k):
    """the whole MoE step on the oracle: quantize, route, sort, per entry up (canonical), relu^2, quantize, down,
    combine; returns (x_out, yd, ids, gw)"""
    M = x.shape[0]
    ids, gw = orc.router_topk(lg, k)
    cnt, off, xrow, where = orc.moe_sort(ids, len(up_rows))
    q, d = orc.q8_quant(x)
    n = M * k
    u = np.empty((n, F), np.float32)
    for e in np.nonzero(cnt)[0]:
        p = np.arange(off[e], off[e] + cnt[e])
        acc = orc.q8_acc(up_rows[e], F, H, q[xrow[p]])
        u[p] = orc.q8_out(acc, up_rows[e], F, H, d[xrow[p]])
    r = np.maximum(u, np.float32(0))
    uq, ud = orc.q8_quant((r * r).astype(np.float32))
    yd = np.empty((n, H), np.float32)
    for e in np.nonzero(cnt)[0]:
        p = np.arange(off[e], off[e] + cnt[e])
        acc = orc.q8_acc(down_rows[e], H, F, uq[p])
        yd[p] = orc.q8_out(acc, down_rows[e], H, F, ud[p])
    return orc.moe_combine(yd, None, where, gw, x), yd, u, ids, gw


@pytest.mark.parametrize("M", [1, 64, 256])
def test_moe_forward_config4(kt, M):
    """config 4 shapes: 128 experts, up [1856 x 2688], down [2688 x 1856], top-6. Stage by stage, each oracle stage
    fed the GPU's previous stage: routing and lists exact, up / down within 1e-3 (their unit values exact), the
    intermediate's requantization and the combine bit-exact. End to end against the all-oracle chain the int8
    requantization of the intermediate amplifies last-bit differences, so that bound is looser (1e-2)."""
    lib, moe = kt
    say("moe forward", M)
    E, k, H, F = 128, 6, 2688, 1856
    import kindi_amd.synth as syn
    up_rows = [host(syn.q8_rows(F, H, 1000 + e, device="cuda")) for e in range(E)]
    down_rows = [host(syn.q8_rows(H, F, 2000 + e, device="cuda")) for e in range(E)]
    layer = moe.MoE(moe.Q8Experts(up_rows, F, H), moe.Q8Experts(down_rows, H, F), k)
    x = rng(M + 40).normal(0, 1, (M, H)).astype(np.float32)
    lg = rng(M + 41).normal(0, 1, (M, E)).astype(np.float32)
    xd = dev(x)
    out, st = layer.forward(xd, dev(lg))
    ids, gw = orc.router_topk(lg, k)
    assert np.array_equal(host(st["ids"]), ids)
    cnt, off, xrow, where = orc.moe_sort(ids, E)
    q, d = orc.q8_quant(x)
    assert np.array_equal(host(st["xq"]), q) and np.array_equal(host(st["xd"]), d)
    u_g, uq_g, ud_g, yd_g = host(st["u"]), host(st["uq"]), host(st["ud"]), host(st["yd"])
    n = M * k
    u = np.empty((n, F), np.float32)
    yd = np.empty((n, H), np.float32)
    for e in np.nonzero(cnt)[0]:
        p = np.arange(off[e], off[e] + cnt[e])
        u[p] = orc.q8_out(orc.q8_acc(up_rows[e], F, H, q[xrow[p]]), up_rows[e], F, H, d[xrow[p]])
    assert max_rel(u_g, u) < TOL
    r = np.maximum(u_g, np.float32(0))
    uq, ud = orc.q8_quant((r * r).astype(np.float32))
    assert np.array_equal(uq_g, uq) and np.array_equal(ud_g, ud)
    for e in np.nonzero(cnt)[0]:
        p = np.arange(off[e], off[e] + cnt[e])
        yd[p] = orc.q8_out(orc.q8_acc(down_rows[e], H, F, uq[p]), down_rows[e], H, F, ud[p])
    assert max_rel(yd_g, yd) < TOL
    assert np.array_equal(host(out), orc.moe_combine(yd_g, None, where, host(st["gw"]), x))
    ref = oracle_moe(x, lg, up_rows, down_rows, H, F, k)[0]
    e2e = max_rel(host(out) - x, ref - x)
    say("moe end-to-end max rel vs the all-oracle chain: %.2e" % e2e)
    assert e2e < 1e-2
    # the grouped up product of one expert: unit values exact, outputs exact in the kernel's summation tree
    dbg = torch.empty((n, F, H // 32), dtype=torch.int32, device="cuda")
    Y = torch.empty((n, F), dtype=torch.float32, device="cuda")
    layer.up.grouped(st["lists"], M, st["xq"], st["xd"], Y, xrow=True, dbg=dbg)
    e = int(ids[0, 0])
    p = np.arange(off[e], off[e] + cnt[e])
    acc = orc.q8_acc(up_rows[e], F, H, q[xrow[p]])
    assert np.array_equal(host(dbg)[p], acc)
    dq = np.ascontiguousarray(up_rows[e].reshape(F, H // 32, 34)[:, :, :2].copy().view(np.float16)[..., 0]
                              .astype(np.float32).T)
    KS = lib.kt_decode_kslices(H, 1)
    assert np.array_equal(host(Y)[p], orc.out_lanes(acc, d[xrow[p]], dq, 8, 1, KS))   # the q8_0 decode tree
    # and every expert's rows equal the dense q8_0 product of the same tokens (one kernel, one tree)
    for e in np.nonzero(cnt)[0][:8]:
        p = np.arange(off[e], off[e] + cnt[e])
        dense = moe.Q8Matrix(up_rows[e], F, H).gemv(st["xq"][torch.from_numpy(xrow[p]).cuda().long()],
                                                    st["xd"][torch.from_numpy(xrow[p]).cuda().long()])
        assert np.array_equal(host(dense).view(np.uint32), host(Y)[p].view(np.uint32)), e


def test_combine_bit_exact(kt):
    lib, moe = kt
    say("combine")
    M, k, H = 9, 6, 2688
    r = rng(77)
    yd = r.normal(0, 1, (M * k, H)).astype(np.float32)
    where = r.permutation(M * k).astype(np.int32)
    gw = r.random((M, k)).astype(np.float32)
    x = r.normal(0, 1, (M, H)).astype(np.float32)
    ups = moe.Q8Experts([q8_case(64, 32, e)[0] for e in range(8)], 64, 32)
    downs = moe.Q8Experts([q8_case(32, 64, e)[0] for e in range(8)], 32, 64)
    layer = moe.MoE(ups, downs, k)
    xd = dev(x)
    layer.combine(dev(yd), dev(where), dev(gw), xd)
    assert np.array_equal(host(xd), orc.moe_combine(yd, None, where, gw, x))


@pytest.mark.parametrize("E,H,F,M,k", [(128, 2688, 1856, 1, 6), (128, 2688, 1856, 4, 6), (128, 2688, 1856, 10, 6),
                                       (8, 96, 64, 10, 6), (16, 160, 96, 64, 1), (4, 64, 32, 3, 4), (8, 128, 64, 1, 3),
                                       (16, 96, 4096, 1, 8), (16, 96, 8192, 1, 2), (4, 64, 32, 1, 4), (64, 2688, 1856, 1, 1),
                                       (256, 96, 64, 1, 6), (1024, 64, 32, 1, 4), (1024, 64, 32, 3, 8)])
def test_moe_decode_chain(kt, E, H, F, M, k):
    """kt_moe_decode (one token: two launches, the up product routing for itself and the down product combining a row
    group of every pick; more tokens: route, up and down with the quantization in their staging, combine) gives x bit
    for bit as the separate launches (forward: route + quant + grouped up + quant + grouped down + combine), with and
    without the shared-expert rows, on a workspace full of garbage (it needs no initialisation), twice in a row;
    ragged row groups (H = 96, 128: a last row group of a 32-row block), one pick a token, every expert active, k not a
    register-set size (3), the widest down input the one-token chain takes (F = 4096) and one past it (F = 8192: the
    four-launch chain); more than 128 experts (E = 256, 1024: the up launch reads the chosen expert's pointer from the
    table, and the top-k scans 4 / 16 logits a lane)"""
    lib, moe = kt
    say("moe decode chain", E, H, F, M, k)
    ups = moe.Q8Experts([q8_case(F, H, 3000 + e)[0] for e in range(E)], F, H)
    downs = moe.Q8Experts([q8_case(H, F, 4000 + e)[0] for e in range(E)], H, F)
    layer = moe.MoE(ups, downs, k)
    x = rng(M + H).normal(0, 1, (M, H)).astype(np.float32)
    lg = rng(M + E).normal(0, 1, (M, E)).astype(np.float32)
    ysh = rng(7).normal(0, 1, (M, H)).astype(np.float32)
    lgd = dev(lg)
    want, st = layer.forward(dev(x), lgd)
    want = host(want)
    work = layer.workspace(M)
    assert work.numel() == lib.kt_moe_decode_workspace(M, k, E, H, F) > 0
    work.fill_(0xFF)
    for rep in range(2):
        xd = dev(x)
        layer.decode(xd, lgd, work)
        assert np.array_equal(host(xd).view(np.uint32), want.view(np.uint32)), rep
    # the shared expert's rows: x += s + ysh, as kt_moe_combine with ysh
    xs = dev(x)
    layer.decode(xs, lgd, work, ysh=dev(ysh))
    ref = dev(x)
    layer.combine(st["yd"], st["lists"][3], st["gw"], ref, ysh=dev(ysh))
    assert np.array_equal(host(xs).view(np.uint32), host(ref).view(np.uint32))
    # the intermediates it stands for, against the oracle at the small shapes
    if H <= 160:
        ids, gw = orc.router_topk(lg, k)
        assert np.array_equal(host(st["ids"]), ids)



def sig_layer(moe, E, H, F, k, seed, scale=2.5):
    ups = moe.Q8Experts([q8_case(F, H, seed + e)[0] for e in range(E)], F, H)
    downs = moe.Q8Experts([q8_case(H, F, seed + 1000 + e)[0] for e in range(E)], H, F)
    bias = rng(seed).normal(0, 0.3, E).astype(np.float32)
    return moe.MoE(ups, downs, k, score="sigmoid", bias=dev(bias), scale=scale), bias


@pytest.mark.parametrize("E,k", [(128, 6), (1000, 16), (256, 8)])
def test_topk_sigmoid(kt, E, k):
    """Kindi's router (sigmoid, bias for the choice, weights = chosen scores / their sum * scale) at config 4's token
    counts: ids bit-exact against the oracle (pinned in tests/test_oracle.py by a float64 restatement and brute-force
    top-k), weights within 2e-6 relative (the device expf and the host's differ in the last bit on some inputs: 58
    of 60 weights bit-equal at 10 tokens); the one-launch route + lists gives the same ids, weights and lists"""
    lib, moe = kt
    say("topk sigmoid", E, k)
    layer, bias = sig_layer(moe, E, 64, 32, k, 7000 + E)
    for M in (1, 4, 10, 256):
        lg = rng(M + E).normal(0, 1, (M, E)).astype(np.float32)
        if M == 10:
            lg[2, 5:5 + k + 3] = 0.5                                  # equal logits: the bias alone orders them
        ids, gw = layer.route(dev(lg))
        rid, rgw = orc.router_sig(lg, bias, 2.5, k)
        assert np.array_equal(host(ids), rid), M
        g = host(gw)
        assert np.allclose(g, rgw, rtol=2e-6, atol=0), M
        say("sigmoid weights bit-exact: %d of %d" % (int((g.view(np.uint32) == rgw.view(np.uint32)).sum()), g.size))
        if M * k <= 64:
            ids2, gw2, lists2 = layer.route_lists(dev(lg))
            assert np.array_equal(host(ids2), rid) and np.array_equal(host(gw2), g), M
            lists = layer.lists(ids)
            for a_, b_ in zip(lists2[:4], lists[:4]):
                assert np.array_equal(host(a_), host(b_)), M


def test_topk_nan_distinct(kt):
    """a token with fewer numbers than k: the numbers first (by value), then NaN entries from the lowest index, every
    pick distinct, as the oracle ranks them (both scorings)"""
    lib, moe = kt
    say("topk NaN")
    E, k, M = 128, 6, 3
    lg = np.full((M, E), np.nan, np.float32)
    lg[0, [9, 40, 100]] = [-3.0, 1.0, 0.5]
    lg[1, :] = rng(3).normal(0, 1, E)
    lg[1, ::2] = np.nan
    lg[2, 127] = 2.0
    layer, bias = sig_layer(moe, E, 64, 32, k, 7500)
    soft = moe.MoE(layer.up, layer.down, k)
    ids, gw = soft.route(dev(lg))
    rid, _ = orc.router_topk(lg, k)
    assert np.array_equal(host(ids), rid)
    assert all(len(set(r)) == k for r in host(ids).tolist())
    zb = moe.MoE(layer.up, layer.down, k, score="sigmoid", bias=torch.zeros(E, device="cuda"), scale=1.0)
    ids, gw = zb.route(dev(lg))
    rid, _ = orc.router_sig(lg, np.zeros(E, np.float32), 1.0, k)
    assert np.array_equal(host(ids), rid)
    assert all(len(set(r)) == k for r in host(ids).tolist())


@pytest.mark.parametrize("E,H,F,M,k", [(128, 2688, 1856, 1, 6), (128, 2688, 1856, 8, 6), (256, 96, 64, 1, 6),
                                       (32, 96, 64, 40, 4), (1024, 64, 32, 1, 8), (1024, 64, 32, 3, 8)])
def test_moe_sigmoid_chain(kt, E, H, F, M, k):
    """the MoE layer with Kindi's router: kt_moe_decode_r gives x bit for bit as forward() (route_r / topk_r, sort,
    grouped up, relu^2 quantize, grouped down, combine), whose picks and weights are the oracle's"""
    lib, moe = kt
    say("moe sigmoid chain", E, H, F, M, k)
    layer, bias = sig_layer(moe, E, H, F, k, 8000)
    x = rng(M + H + 1).normal(0, 1, (M, H)).astype(np.float32)
    lg = rng(M + E + 1).normal(0, 1, (M, E)).astype(np.float32)
    lgd = dev(lg)
    want, st = layer.forward(dev(x), lgd)
    rid, rgw = orc.router_sig(lg, bias, 2.5, k)
    assert np.array_equal(host(st["ids"]), rid)
    assert np.allclose(host(st["gw"]), rgw, rtol=2e-6, atol=0)
    if M * k <= 64:
        xd = dev(x)
        layer.decode(xd, lgd)
        assert np.array_equal(host(xd).view(np.uint32), host(want).view(np.uint32))


def test_moe_decode_row_at_allocation_end(kt):
    """the one-token chain with an odd slice count (H = 96: the up launch's second task of its last wave is off) reads
    only inside x: x and the logits sit at the very end of allocations of exactly 2 MiB"""
    lib, moe = kt
    say("moe decode x at allocation end")
    E, H, F, k = 8, 96, 64, 6
    ups = moe.Q8Experts([q8_case(F, H, 9000 + e)[0] for e in range(E)], F, H)
    downs = moe.Q8Experts([q8_case(H, F, 9100 + e)[0] for e in range(E)], H, F)
    layer = moe.MoE(ups, downs, k)
    x = rng(11).normal(0, 1, (1, H)).astype(np.float32)
    lg = rng(12).normal(0, 1, (1, E)).astype(np.float32)
    n = (2 << 20) // 4
    xb = torch.empty(n, dtype=torch.float32, device="cuda")
    lb = torch.empty(n, dtype=torch.float32, device="cuda")
    xe = xb[n - H:].view(1, H)
    le = lb[n - E:].view(1, E)
    xe.copy_(dev(x))
    le.copy_(dev(lg))
    want, _ = layer.forward(dev(x), dev(lg))
    layer.decode(xe, le)
    assert np.array_equal(host(xe).view(np.uint32), host(want).view(np.uint32))

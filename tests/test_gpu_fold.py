"""GPU parity of the fused input producers (kt_rmsfold_q8, kt_fold_q8, kt_smfold_q8) against the CPU oracle's
restatement of k_rmsfold_qT / k_fold_fwht_qT / k_smfold_qT. Bar: every output (x + parts, the normed row, the folded
row, the int8 row and its XS / XA) bit-exact for rmsfold and fold; smfold goes through the exponential, whose last
bit the GPU's and the host's libraries may round differently, so its fp32 outputs are held to 1e-6 relative of the
row's largest value and its int8 values to +-1 on at most 0.1% of the columns."""
import numpy as np
import pytest
import torch

import oracle as orc
from kt_cases import say, dev, host, rng

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lin():
    assert torch.cuda.is_available(), "GPU tests need the MI355X"
    from kindi_amd import linear
    return linear


def signs(C, seed):
    return np.where(rng(seed).random(C) < 0.5, -1.0, 1.0).astype(np.float32)


def same(a, b):
    return np.array_equal(np.asarray(a).view(np.uint8), np.asarray(b).view(np.uint8))


@pytest.mark.parametrize("M,C,HB,nparts", [(1, 512, 512, 0), (1, 2048, 512, 0), (1, 2560, 512, 2),
                                           (1, 5120, 1024, 0), (3, 5120, 1024, 3), (2, 4096, 4096, 1),
                                           (16, 5120, 1024, 1), (1, 8192, 4096, 8), (5, 1536, 512, 0),
                                           (256, 5120, 1024, 2)])
def test_rmsfold_bit_exact(lin, M, C, HB, nparts):
    say("rmsfold", M, C, HB, nparts)
    r = rng(M * 31 + C + nparts)
    x = r.standard_normal((M, C)).astype(np.float32)
    parts = (r.standard_normal((M, max(nparts, 1) * C)) * 0.5).astype(np.float32)
    w = (1.0 + 0.2 * r.standard_normal(C)).astype(np.float32)
    sg = signs(C, C)
    if M > 2:
        x[1] = 0.0                                              # a zero row (with its parts, if any, zero too)
        parts[1] = 0.0
        x[2, :128] *= 1e-30                                     # a tiny group
    want = orc.rmsfold_q8(x, parts if nparts else None, nparts, w, sg, HB)
    X, Pt = dev(x), dev(parts)
    xw = torch.empty_like(X)
    xn = torch.empty_like(X)
    xo = torch.empty_like(X)
    act = lin.rmsfold(X, dev(w), dev(sg), HB, r=Pt if nparts else None, nparts=nparts, xw=xw, xn=xn, xo=xo)
    torch.cuda.synchronize()
    if nparts:
        assert same(host(xw), want["xw"])
    assert same(host(xn), want["xn"])
    assert same(host(xo), want["xo"])
    assert np.array_equal(host(act.XQ), want["Q"])
    assert same(host(act.XS), want["XS"])
    assert np.array_equal(host(act.XA), want["XA"])


def test_rmsfold_in_place_and_outputs_optional(lin):
    say("rmsfold in place")
    M, C, HB = 4, 5120, 1024
    r = rng(3)
    x = r.standard_normal((M, C)).astype(np.float32)
    parts = r.standard_normal((M, 2 * C)).astype(np.float32)
    w = np.ones(C, np.float32)
    sg = signs(C, 4)
    want = orc.rmsfold_q8(x, parts, 2, w, sg, HB)
    X = dev(x)
    act = lin.rmsfold(X, dev(w), dev(sg), HB, r=dev(parts), nparts=2, xw=X)   # x + parts written over x
    torch.cuda.synchronize()
    assert same(host(X), want["xw"])
    assert np.array_equal(host(act.XQ), want["Q"]) and same(host(act.XS), want["XS"])


@pytest.mark.parametrize("M,C,HB", [(1, 2048, 512), (1, 5120, 1024), (7, 4096, 4096), (64, 8192, 1024), (3, 12288, 4096),
                                    (2, 17408, 1024)])
def test_fold_bit_exact(lin, M, C, HB):
    say("fold", M, C, HB)
    x = rng(C + M).standard_normal((M, C)).astype(np.float32)
    sg = signs(C, 9)
    want = orc.fold_q8(x, sg, HB)
    xo = torch.empty((M, C), dtype=torch.float32, device="cuda")
    act = lin.fold(dev(x), dev(sg), HB, xo=xo)
    torch.cuda.synchronize()
    assert same(host(xo), want["xo"])
    assert np.array_equal(host(act.XQ), want["Q"])
    assert same(host(act.XS), want["XS"]) and np.array_equal(host(act.XA), want["XA"])


@pytest.mark.parametrize("M,C,HB,perm", [(1, 6144, 512, (1, 1, 1)), (3, 6144, 1024, (1, 1, 1)),
                                         (2, 4096, 4096, (128, 4, 8)), (16, 5120, 1024, (128, 8, 5)),
                                         (2, 17408, 1024, (1, 1, 1)), (4, 12288, 4096, (128, 16, 6))])
def test_smfold(lin, M, C, HB, perm):
    say("smfold", M, C, HB, perm)
    r = rng(C * 3 + M)
    a = (r.standard_normal((M, C)) * 3).astype(np.float32)
    b = r.standard_normal((M, C)).astype(np.float32)
    sg = signs(C, 5)
    want = orc.smfold_q8(a, b, sg, HB, perm)
    xo = torch.empty((M, C), dtype=torch.float32, device="cuda")
    act = lin.smfold(dev(a), dev(b), dev(sg), HB, perm=perm, xo=xo)
    torch.cuda.synchronize()
    got = host(xo)
    assert np.abs(got - want["xo"]).max() <= 1e-6 * np.abs(want["xo"]).max()
    dq = np.abs(host(act.XQ).astype(np.int32) - want["Q"].astype(np.int32))
    assert dq.max() <= 1 and (dq > 0).mean() <= 1e-3
    assert np.allclose(host(act.XS), want["XS"], rtol=1e-6, atol=0)


@pytest.mark.parametrize("M,C,HB", [(1, 5120, 1024), (3, 4096, 4096), (40, 5120, 1024), (2, 17408, 1024)])
def test_producers_hp_bit_exact(lin, M, C, HB):
    """the producers' two-row (hp) output (ff_q8 tcf.cu:150-205): rmsfold and fold bit-exact in every row, scale and
    sum; smfold's rows follow its folded row (the exponential's last bit aside), so its two rows are checked against
    the oracle's quantizer of the GPU's own folded row"""
    say("producers hp", M, C, HB)
    r = rng(C + 3 * M)
    x = r.standard_normal((M, C)).astype(np.float32)
    w = (1.0 + 0.1 * r.standard_normal(C)).astype(np.float32)
    sg = signs(C, 11)
    if C <= 8192:
        want = orc.rmsfold_q8(x, None, 0, w, sg, HB, hp=True)
        xo = torch.empty((M, C), dtype=torch.float32, device="cuda")
        act = lin.rmsfold(dev(x), dev(w), dev(sg), HB, xo=xo, hp=True)
        torch.cuda.synchronize()
        assert act.hp and act.XQ.shape[0] == 2 * M and same(host(xo), want["xo"])
        assert np.array_equal(host(act.XQ), want["Q"])
        assert same(host(act.XS), want["XS"]) and np.array_equal(host(act.XA), want["XA"])
    want = orc.fold_q8(x, sg, HB, hp=True)
    act = lin.fold(dev(x), dev(sg), HB, hp=True)
    assert np.array_equal(host(act.XQ), want["Q"])
    assert same(host(act.XS), want["XS"]) and np.array_equal(host(act.XA), want["XA"])
    b = r.standard_normal((M, C)).astype(np.float32)
    xo = torch.empty((M, C), dtype=torch.float32, device="cuda")
    act = lin.smfold(dev(x), dev(b), dev(sg), HB, xo=xo, hp=True)
    Q, XS, XA = orc.quant_q8(host(xo), 3)
    assert np.array_equal(host(act.XQ), Q) and same(host(act.XS), XS) and np.array_equal(host(act.XA), XA)

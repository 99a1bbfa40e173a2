"""The launchers under HIP graph capture (torch.cuda.graph): a captured sequence is replayed several times, with new
inputs written and other GPU work run eagerly between the replays, and every replay's outputs must equal, bit for
bit, the same launches run eagerly on the same inputs. Covers a decode layer's launches (quantizer, three-matrix
product, fused producer, the matrix-core decode kernels, the two-row form), the MoE decode chain (caller workspace
and the library's own array) and the many-token MoE layer (routing, token lists, grouped products, combine)."""
import numpy as np
import pytest
import torch

from kt_cases import say, tern_case, q8_case, host, rng

pytestmark = pytest.mark.gpu
REPLAYS = 4


@pytest.fixture(scope="module")
def mods():
    assert torch.cuda.is_available(), "GPU tests need the MI355X"
    from kindi_amd import gpudrv, linear, moe
    return gpudrv.load(), linear, moe


def capture(fn):
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()                                                    # warm-up outside the graph
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


def eager_noise():
    """unrelated eager GPU work between replays"""
    a = torch.randn((512, 512), device="cuda")
    (a @ a).sum().item()


def same(a, b):
    return np.array_equal(host(a).view(np.uint8), host(b).view(np.uint8))


def test_graph_decode_layer(mods):
    lib, linear, _ = mods
    say("graph decode layer")
    C, F = 1024, 2560
    mats = {}
    for i, (n, R, Cn) in enumerate((("q", 640, C), ("k", 128, C), ("v", 128, C), ("o", C, 640), ("down", C, F))):
        dig, bc, dpm = tern_case(R, Cn, 900 + i)
        mats[n] = linear.TernaryMatrix(bc, dpm, R, Cn)
    L = linear.Linear(mats)
    r = rng(5)
    x1 = torch.empty((1, C), device="cuda")
    x16 = torch.empty((16, F), device="cuda")
    xo = torch.empty((3, 640), device="cuda")
    res = torch.empty((1, C), device="cuda")
    w = torch.from_numpy((1 + 0.1 * r.standard_normal(C)).astype(np.float32)).cuda()
    sg = torch.from_numpy(np.where(r.random(C) < 0.5, -1.0, 1.0).astype(np.float32)).cuda()

    def bufs():
        return dict(a1=linear._act_out(1, C, "cuda"), ah=linear._act_out(1, C, "cuda"),
                    a16=linear._act_out(16, F, "cuda"), ao=linear._act_out(3, 640, "cuda", hp=True),
                    xw=torch.empty((1, C), device="cuda"),
                    y={n: torch.empty((16 if n == "down" else 3 if n == "o" else 1, m.R), device="cuda")
                       for n, m in mats.items()},
                    y2=torch.empty((1, 640), device="cuda"))

    def run(b):
        a1 = linear.quantize(x1, out=b["a1"])
        L.gemv_q(["q", "k", "v"], a1, [b["y"]["q"], b["y"]["k"], b["y"]["v"]])
        ah = linear.rmsfold(x1, w, sg, 512, r=res, nparts=1, xw=b["xw"], out=b["ah"])
        L.gemv_q(["q"], ah, [b["y2"]])
        a16 = linear.quantize(x16, out=b["a16"])                  # 16 tokens: the 16x16x64 matrix-core kernel
        L.gemv_q(["down"], a16, [b["y"]["down"]])
        ao = linear.quantize(xo, out=b["ao"], hp=True)             # the two-row form, 3 tokens (6 rows)
        L.gemv_q(["o"], ao, [b["y"]["o"]])

    gb = bufs()
    g = capture(lambda: run(gb))
    for it in range(REPLAYS):
        for t in (x1, x16, xo, res):
            t.copy_(torch.from_numpy(r.standard_normal(tuple(t.shape)).astype(np.float32)))
        eager_noise()
        g.replay()
        torch.cuda.synchronize()
        eb = bufs()
        run(eb)
        torch.cuda.synchronize()
        for n in mats:
            assert same(gb["y"][n], eb["y"][n]), (it, n)
        assert same(gb["y2"], eb["y2"]) and same(gb["xw"], eb["xw"]), it
        assert same(gb["ao"].XQ, eb["ao"].XQ) and same(gb["ao"].XS, eb["ao"].XS), it


def _layer(moe, E, H, F, k, seed):
    ups = moe.Q8Experts([q8_case(F, H, seed + e)[0] for e in range(E)], F, H)
    downs = moe.Q8Experts([q8_case(H, F, seed + 500 + e)[0] for e in range(E)], H, F)
    return moe.MoE(ups, downs, k)


@pytest.mark.parametrize("M", [1, 8])
def test_graph_moe_decode(mods, M):
    """kt_moe_decode (two launches at one token, four at more) and kt_moe_decode_noalloc under capture; x is updated
    in place, so each replay starts from a fresh x written eagerly"""
    lib, linear, moe = mods
    say("graph moe decode", M)
    E, H, F, k = 32, 512, 384, 4
    layer = _layer(moe, E, H, F, k, 7000)
    from kindi_amd.linear import ptr, stream
    r = rng(M)
    x = torch.empty((M, H), device="cuda")
    xn = torch.empty((M, H), device="cuda")
    lg = torch.empty((M, E), device="cuda")
    work = layer.workspace(M)
    assert lib.kt_init(0) == 0                                  # the no-alloc array's address, before capture

    def run_ws():
        layer.decode(x, lg, work)

    def run_na():
        rc = lib.kt_moe_decode_noalloc(ptr(layer.up.table), ptr(layer.down.table), E, H, F, k, ptr(lg), M, ptr(xn),
                                       xn.stride(0), None, stream())
        assert rc == 0, rc

    g1, g2 = capture(run_ws), capture(run_na)
    for it in range(REPLAYS):
        x0 = torch.from_numpy(r.standard_normal((M, H)).astype(np.float32)).cuda()
        lg.copy_(torch.from_numpy(r.standard_normal((M, E)).astype(np.float32)))
        x.copy_(x0)
        xn.copy_(x0)
        eager_noise()
        g1.replay()
        g2.replay()
        torch.cuda.synchronize()
        want = x0.clone()
        layer.decode(want, lg, layer.workspace(M))
        torch.cuda.synchronize()
        assert same(x, want) and same(xn, want), it


def test_graph_moe_forward(mods):
    """the many-token layer (quantize, top-k, token lists, grouped up / down, relu^2 quantize, combine) at 24 tokens"""
    lib, linear, moe = mods
    say("graph moe forward")
    E, H, F, k, M = 32, 512, 384, 4, 24
    layer = _layer(moe, E, H, F, k, 7500)
    r = rng(77)
    x = torch.empty((M, H), device="cuda")
    lg = torch.empty((M, E), device="cuda")
    gbufs = layer.buffers(M)
    g = capture(lambda: layer.forward(x, lg, gbufs))
    for it in range(REPLAYS):
        x0 = torch.from_numpy(r.standard_normal((M, H)).astype(np.float32)).cuda()
        lg.copy_(torch.from_numpy(r.standard_normal((M, E)).astype(np.float32)))
        x.copy_(x0)
        eager_noise()
        g.replay()
        torch.cuda.synchronize()
        want = x0.clone()
        layer.forward(want, lg, layer.buffers(M))
        torch.cuda.synchronize()
        assert same(x, want), it

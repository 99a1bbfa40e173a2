"""The decode plan executor (kt_plan_*) against the single launches it replaces: every output bit equal, stage order
and visibility as separate stream-ordered launches give them, no barrier timeouts."""
import numpy as np
import pytest
import torch

from kt_cases import dev, host, say

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def linear():
    from kindi_amd import linear as lin
    return lin


@pytest.fixture(scope="module")
def synth():
    from kindi_amd import synth as sy
    return sy


def _mats(linear, synth, shapes, seed):
    out = {}
    for i, (n, R, C) in enumerate(shapes):
        bc, dpm = synth.tern_pack(R, C, seed + i, device="cuda")
        out[n] = linear.TernaryMatrix(bc, dpm, R, C)
    return out


GROUPS = (("q", "k", "v"), ("o",), ("gate", "up"), ("down",))


def _layer_stages(linear, synth, shapes, layers, M, seed):
    """the per-layer stages of a decode step over resident quantized inputs; returns (stages, launch outputs)"""
    stages, ref = [], []
    L = linear.Linear({})
    for l in range(layers):
        mats = _mats(linear, synth, shapes, seed + 10 * l)
        for g, names in enumerate(GROUPS):
            C = mats[names[0]].C
            act = linear.quantize(synth.activations(M, C, seed + 100 * l + g, device="cuda"))
            outs = [torch.full((M, mats[n].R), float("nan"), device="cuda") for n in names]
            refs = [torch.empty((M, mats[n].R), device="cuda") for n in names]
            for n in names:
                L.add("%d.%s" % (l, n), mats[n])
            L.gemv_q(["%d.%s" % (l, n) for n in names], act, refs)
            stages.append(([mats[n] for n in names], act, outs))
            ref.append(refs)
    return stages, ref


@pytest.mark.parametrize("M", [1, 2, 4])
def test_plan_matches_launches_2b(linear, synth, M):
    shapes = synth.CFG["c1"]["mats"]
    stages, ref = _layer_stages(linear, synth, shapes, 2, M, 300)
    plan = linear.Plan(stages)
    say("plan 2B x2 layers M=%d: %d stages, grid %d, %d data waves" % (M, len(stages), plan.info.grid,
                                                                        plan.info.waves))
    for rep in range(3):
        plan.run()
        torch.cuda.synchronize()
        assert plan.status() == 0
        for k, ((_, _, outs), refs) in enumerate(zip(stages, ref)):
            for o, r in zip(outs, refs):
                assert np.array_equal(host(o).view(np.uint32), host(r).view(np.uint32)), (rep, k)


def test_plan_matches_launches_27b_layer(linear, synth):
    shapes = synth.CFG["c3"]["mats"]
    stages, ref = _layer_stages(linear, synth, shapes, 1, 1, 700)
    plan = linear.Plan(stages)
    say("plan 27B layer: grid %d, %d data waves, executor %d" % (plan.info.grid, plan.info.waves, plan.info.exec))
    plan.run()
    torch.cuda.synchronize()
    assert plan.status() == 0
    for k, ((_, _, outs), refs) in enumerate(zip(stages, ref)):
        for o, r in zip(outs, refs):
            assert np.array_equal(host(o).view(np.uint32), host(r).view(np.uint32)), k


@pytest.mark.parametrize("M", [1, 2, 4])
def test_plan_stage_reads_earlier_output(linear, synth, M):
    """stage k + 1's group scales XS are stage k's output rows: the plan must give what launches in order give (one
    token: the streamed executor; two and four: the register-ring executor)"""
    C = 2048
    NG = C // 128
    mats = [_mats(linear, synth, [("m%d" % i, NG, C)], 900 + i)["m%d" % i] for i in range(4)]
    big = _mats(linear, synth, [("big", 8192, C)], 990)["big"]      # keeps the other blocks busy between
    x = synth.activations(M, C, 77, device="cuda")
    a0 = linear.quantize(x)

    def chain(XS0, outs):
        acts = [a0._replace(XS=XS0)]
        for i in range(1, 4):
            acts.append(a0._replace(XS=outs[i - 1]))
        return acts

    # in order, one launch each
    L = linear.Linear({"m%d" % i: m for i, m in enumerate(mats)})
    ref = [torch.empty((M, NG), device="cuda") for _ in range(4)]
    acts = chain(a0.XS, ref)
    for i in range(4):
        L.gemv_q(["m%d" % i], acts[i], [ref[i]])
    # the plan: the same chain, a large unrelated product between each pair
    outs = [torch.full((M, NG), float("nan"), device="cuda") for _ in range(4)]
    ybig = [torch.empty((M, 8192), device="cuda") for _ in range(4)]
    acts = chain(a0.XS, outs)
    stages = []
    for i in range(4):
        stages.append(([mats[i]], acts[i], [outs[i]]))
        stages.append(([big], a0, [ybig[i]]))
    plan = linear.Plan(stages)
    say("plan chain M=%d: executor %d" % (M, plan.info.exec))
    for rep in range(3):
        for o in outs:
            o.fill_(float("nan"))
        plan.run()
        torch.cuda.synchronize()
        assert plan.status() == 0
        for i in range(4):
            assert np.array_equal(host(outs[i]).view(np.uint32), host(ref[i]).view(np.uint32)), (rep, i)


@pytest.mark.parametrize("M", [1, 2])
def test_plan_graph_replays(linear, synth, M):
    """the plan run (its reset kernel and the plan kernel) captured in a HIP graph and replayed with new activations
    quantized eagerly between replays: every replay equals the single launches on the same inputs"""
    say("plan graph M=%d" % M)
    shapes = [("q", 256, 1024), ("k", 64, 1024), ("v", 64, 1024), ("o", 1024, 256), ("gate", 512, 1024),
              ("up", 512, 1024), ("down", 1024, 512)]
    stages, _ = _layer_stages(linear, synth, shapes, 2, M, 900)
    plan = linear.Plan(stages)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        plan.run()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        plan.run()
    torch.cuda.synchronize()
    L = linear.Linear({})
    for it in range(4):
        for k, (mats, act, outs) in enumerate(stages):         # new inputs, quantized into the stages' buffers
            x = synth.activations(M, act.C, 5000 + 10 * it + k, device="cuda")
            linear.quantize(x, out=act)
        a = torch.randn((256, 256), device="cuda")
        (a @ a).sum().item()
        g.replay()
        torch.cuda.synchronize()
        assert plan.status() == 0, it
        for k, (mats, act, outs) in enumerate(stages):
            for i, m in enumerate(mats):
                L.add("m", m)
                ref = torch.empty_like(outs[i])
                L.gemv_q(["m"], act, [ref])
                torch.cuda.synchronize()
                assert np.array_equal(host(outs[i]).view(np.uint32), host(ref).view(np.uint32)), (it, k, i)

"""kt_moe_decode_noalloc (the MoE decode chain with its workspace in the library's own device array) against
kt_moe_decode with a caller workspace, through the C ABI: bit for bit, on two calls in a row, the second with fewer
tokens than the first (the array keeps the first call's contents), on one token (two launches) and several (four);
a shape whose workspace exceeds the array is refused before any launch."""
import ctypes

import numpy as np
import pytest
import torch

from kt_cases import say, q8_case, dev, host, rng

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def kt():
    assert torch.cuda.is_available(), "GPU tests need the MI355X"
    from kindi_amd import gpudrv, moe
    return gpudrv.load(), moe


def _layer(moe, E, H, F, k, seed):
    ups = moe.Q8Experts([q8_case(F, H, seed + e)[0] for e in range(E)], F, H)
    downs = moe.Q8Experts([q8_case(H, F, seed + 500 + e)[0] for e in range(E)], H, F)
    return moe.MoE(ups, downs, k)


@pytest.mark.parametrize("E,H,F,k,Ms", [(128, 2688, 1856, 6, (10, 1)), (128, 2688, 1856, 6, (1, 1)),
                                        (16, 96, 64, 3, (20, 7))])
def test_noalloc_equals_workspace(kt, E, H, F, k, Ms):
    lib, moe = kt
    say("moe decode noalloc", E, H, F, k, Ms)
    layer = _layer(moe, E, H, F, k, 6000)
    from kindi_amd.linear import ptr, stream
    for M in Ms:
        x = rng(M + 3).normal(0, 1, (M, H)).astype(np.float32)
        lg = rng(M + 4).normal(0, 1, (M, E)).astype(np.float32)
        ysh = rng(M + 5).normal(0, 1, (M, H)).astype(np.float32)
        lgd, yshd = dev(lg), dev(ysh)
        want = dev(x)
        layer.decode(want, lgd, layer.workspace(M), ysh=yshd)
        got = dev(x)
        rc = lib.kt_moe_decode_noalloc(ptr(layer.up.table), ptr(layer.down.table), E, H, F, k, ptr(lgd), M, ptr(got),
                                       got.stride(0), ptr(yshd), stream())
        assert rc == 0, rc
        assert np.array_equal(host(got).view(np.uint32), host(want).view(np.uint32)), M


def test_noalloc_limit(kt):
    lib, moe = kt
    say("moe decode noalloc limit")
    cap = lib.kt_moe_decode_noalloc_max()
    assert cap == 4 << 20
    # 64 entries of 8192 + 8192 fp32 columns need 4 MiB and more: refused before any launch
    assert lib.kt_moe_decode_workspace(64, 1, 128, 8192, 8192) > cap
    f = ctypes.c_void_p(1 << 20)
    assert lib.kt_moe_decode_noalloc(f, f, 128, 8192, 8192, 1, f, 64, f, 8192, None, None) == 1

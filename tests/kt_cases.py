"""Shared builders for the GPU parity tests: the same seeded inputs go to the HIP library (through kindi_amd) and to
the CPU oracle (oracle/). Every GPU step prints the case it runs first, so a failing run names its case."""
import sys

import numpy as np
import torch

import oracle as orc


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


def rng(seed):
    return np.random.default_rng(seed)


def tern_case(R, C, seed):
    """(digits [R, C], bcodes [C/4, R], dpm uint16 [C/128, R]) with the BASELINE distribution"""
    u = rng(seed).random((R, C))
    dig = (u >= 0.3).astype(np.uint8) + (u >= 0.7).astype(np.uint8)
    dpm = np.exp(rng(seed + 1).normal(-3.0, 0.3, (C // 128, R))).astype(np.float16).view(np.uint16)
    return dig, orc.pack_from_digits(dig), dpm


def q8_case(R, C, seed):
    r = rng(seed)
    codes = r.integers(-127, 128, (R, C)).astype(np.int8)
    sc = np.exp(r.normal(-6, 0.5, (R, C // 32))).astype(np.float16).view(np.uint16)
    return orc.q8_0_rows(codes, sc), codes, sc


def dev(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).cuda()
    return t if dtype is None else t.to(dtype)


def host(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def max_rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))

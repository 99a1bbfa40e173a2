"""The decode plan's work deal, checked on the CPU from the image kt_plan_layout builds (the same image kt_plan_build
uploads): every step of every stage is in exactly one data wave's record list, each record's code and scale addresses
are the kt2 layout's for its row group and step (so every lane's loads stay inside its matrix), slices are whole,
in order and on one wave, slice-sum slots match the control wave's reduction order, and every list is padded as far
as the kernel reads ahead. The matrices are fake device addresses: nothing is dereferenced."""
import ctypes
import struct

import numpy as np
import pytest

from kt_cases import rng

W_PER_BLOCK = 8
KT_PLAN_MAXG = 1024
SIZEOF_STAGE = 184                      # KtPStage: 3 x KtMat (40) + 3 pointers + 10 ints
SIZEOF_CTL = 64


def r256(n):
    return (n + 255) // 256 * 256


def offsets(n):
    ctl = r256(64 + n * SIZEOF_STAGE)
    idx = ctl + r256(n * SIZEOF_CTL)
    ctr = idx + r256(KT_PLAN_MAXG * W_PER_BLOCK * 4)
    rec = ctr + r256(33 * 32 * 4)
    return ctl, idx, rec


@pytest.fixture(scope="module")
def lib():
    from kindi_amd import gpudrv
    return gpudrv.load()


def code_bytes(R, NU):
    return (R + 7) // 8 * NU * 256


def make_stages(gpudrv, groups, M=1):
    """groups: [(C, [R...])]; fake, non-overlapping 4 KB-aligned weight and output addresses"""
    arr = (gpudrv.KtStage * len(groups))()
    base = 1 << 40
    mats = []
    for k, (C, Rs) in enumerate(groups):
        st = arr[k]
        NU = C // 128
        for i, R in enumerate(Rs):
            st.W[i] = base
            st.R[i] = R
            st.Y[i] = base + (1 << 36)
            mats.append((k, i, base, R, NU))
            base += (code_bytes(R, NU) + (R + 7) // 8 * NU * 16 + 4095) // 4096 * 4096 + 4096
        st.C = C
        st.XQ = base; st.ldq = (C + 15) // 16 * 16; st.XS = base + (1 << 20); st.XA = base + (2 << 20); st.M = M
        base += 4 << 20
    return arr, mats


def layout(lib, arr, n, G):
    used = ctypes.c_size_t(0)
    assert lib.kt_plan_layout(arr, n, G, None, 0, ctypes.byref(used)) == 0
    buf = (ctypes.c_uint8 * used.value)()
    assert lib.kt_plan_layout(arr, n, G, buf, used.value, ctypes.byref(used)) == 0
    return np.frombuffer(buf, dtype=np.uint8)


def kslices(NU):
    S = (NU + 7) // 8
    return min((S + 1) // 2, 16)


def pad(L):
    return ((L + 1 + 7) // 8 + 4) * 8


def check(lib, groups, G, M=1):
    from kindi_amd import gpudrv
    arr, mats = make_stages(gpudrv, groups, M)
    n = len(groups)
    img = layout(lib, arr, n, G)
    hdr = struct.unpack_from("16i", img, 0)
    assert hdr[0] == n and hdr[1] == G and hdr[2] == W_PER_BLOCK and hdr[7] == M
    red = hdr[6]
    _, idx_off, rec_off = offsets(n)
    idx = np.frombuffer(img, dtype=np.uint32, count=G * W_PER_BLOCK, offset=idx_off)
    recs = np.frombuffer(img, dtype=np.uint32, offset=rec_off).reshape(-1, 4)
    # expected work
    want = set()
    stage_info = []
    off = 0
    for s, (C, Rs) in enumerate(groups):
        NU = C // 128
        S = (NU + 7) // 8
        KS = kslices(NU)
        rg0 = np.cumsum([0] + [(R + 7) // 8 for R in Rs])
        stage_info.append((NU, S, KS, rg0, off))
        for i, R in enumerate(Rs):
            for lrg in range((R + 7) // 8):
                for sp in range(S):
                    want.add((s, i, lrg, sp))
        off = (off + int(rg0[-1])) % G
    mat_of = {}
    for (s, i, base, R, NU) in mats:
        mat_of.setdefault(s, []).append((base, R, NU))
    got = set()
    for b in range(G):
        for w in range(W_PER_BLOCK):
            v = b * W_PER_BLOCK + w
            start = int(idx[v])
            end = int(idx[v + 1]) if v + 1 < G * W_PER_BLOCK else len(recs)
            L = 0
            while int(recs[start + L][3]) >> 20 < n:
                L += 1
            assert end - start == pad(L), (b, w, L, end - start)
            assert all(int(x) >> 20 == n for x in recs[start + L:end, 3])     # padding records
            last_stage, open_slice = -1, None
            for q in recs[start:start + L]:
                code = int(q[0]) | int(q[1]) << 32
                soff = int(np.int32(q[2]))
                bits = int(q[3])
                s, sp, nc = bits >> 20, bits & 31, ((bits >> 5) & 7) + 1
                first, last, slot = bool(bits & 0x100), bool(bits & 0x200), (bits >> 10) & 1023
                assert s >= last_stage
                last_stage = s
                NU, S, KS, rg0, soff_stage = stage_info[s]
                hits = [(i, base, R) for i, (base, R, NUm) in enumerate(mat_of[s])
                        if base <= code < base + code_bytes(R, NU)]
                assert len(hits) == 1
                i, base, R = hits[0]
                o = code - base
                lrg, rem = divmod(o, NU * 256)
                assert rem == sp * 128 * 16
                assert nc == min(8, NU - 8 * sp)
                # every lane's loads inside the matrix's codes / scales
                for c in range(nc):
                    for r in range(8):
                        lo = (c * 8 + r) * 16
                        assert base <= code + lo and code + nc * 128 + lo + 16 <= base + code_bytes(R, NU)
                        h = code + soff + (c * 8 + r) * 2
                        scales = base + code_bytes(R, NU)
                        assert h == scales + ((lrg * NU + sp * 8 + c) * 8 + r) * 2
                key = (s, i, lrg, sp)
                assert key not in got
                got.add(key)
                # the slot: task t = rgk KS + ks of this block's deal, rg = p + rgk G
                rgk, ks = divmod(slot, KS)
                p = (b - soff_stage) % G
                assert p + rgk * G == int(rg0[i]) + lrg
                slo, shi = ks * S // KS, (ks + 1) * S // KS
                assert slo <= sp < shi and first == (sp == slo) and last == (sp == shi - 1)
                assert slot < red
                if first:
                    assert open_slice is None
                    open_slice = (s, slot, sp)
                else:
                    assert open_slice is not None and open_slice[:2] == (s, slot) and sp == open_slice[2] + 1
                    open_slice = (s, slot, sp)
                if last:
                    open_slice = None
            assert open_slice is None
    assert got == want


@pytest.mark.parametrize("G", [256, 80, 40])
def test_plan_layout_27b_layer(lib, G):
    groups = [(5120, [5120, 1024, 1024]), (5120, [5120]), (5120, [17408, 17408]), (17408, [5120])]
    check(lib, groups, G)


@pytest.mark.parametrize("G", [256, 13])
def test_plan_layout_ragged(lib, G):
    """ragged rows and units (C not a multiple of 1024), many stages, small and large matrices"""
    r = rng(5)
    groups = []
    for _ in range(12):
        C = int(r.integers(1, 60)) * 128
        k = int(r.integers(1, 4))
        groups.append((C, [int(x) for x in r.integers(1, 700, size=k)]))
    check(lib, groups, G, M=2)


def test_plan_layout_rejects(lib):
    from kindi_amd import gpudrv
    arr, _ = make_stages(gpudrv, [(5120, [64])])
    used = ctypes.c_size_t(0)
    assert lib.kt_plan_layout(arr, 1, 0, None, 0, ctypes.byref(used)) != 0
    assert lib.kt_plan_layout(arr, 1, KT_PLAN_MAXG + 1, None, 0, ctypes.byref(used)) != 0
    arr[0].C = 100
    assert lib.kt_plan_layout(arr, 1, 256, None, 0, ctypes.byref(used)) != 0

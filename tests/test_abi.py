"""The C ABI without a GPU: the library loads, exports exactly what include/kt.h declares, and its host-side
validation rejects shapes the kernels do not take (those paths return before any launch)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HDR = os.path.join(ROOT, "include", "kt.h")
INVALID = 1                                              # hipErrorInvalidValue


def declared():
    src = open(HDR).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(kt_\w+)\s*\(", src, flags=re.M)))


@pytest.fixture(scope="module")
def lib():
    from kindi_amd import gpudrv
    if not os.path.exists(gpudrv.LIB):
        pytest.fail("libkt_gfx950.so not built: run __graft_entry__.build()")
    return gpudrv.load()


def test_exports_every_declared_symbol(lib):
    names = declared()
    assert len(names) == 38
    for n in names:
        assert hasattr(lib, n), n
    from kindi_amd import gpudrv
    assert sorted(n for n, _, _ in gpudrv.SIGNATURES) == names      # the ctypes table covers the header exactly


def test_version_and_sizes(lib):
    assert lib.kt_version() == 1
    # kt2: 32 bytes of codes + one fp16 per row and 128-column group (2.125 b/w), rows padded to 8
    assert lib.kt_tern_weight_bytes(6144, 2048) == 6144 * 2048 // 4 + 6144 * 16 * 2
    assert lib.kt_tern_weight_bytes(100, 256) == 104 * 2 * 34
    assert lib.kt_tern_weight_bytes(64, 100) == 0
    # kq8: 34 bytes per 32 columns, no padding along K (1856 rows = 232 row groups)
    assert lib.kt_q8_weight_bytes(1856, 2688) == 1856 * 2688 // 32 * 34
    assert lib.kt_q8_weight_bytes(2688, 1856) == 2688 * 1856 // 32 * 34
    assert lib.kt_q8_weight_bytes(64, 48) == 0


def test_decode_kslices(lib):
    """the K-slice count of the decode order depends on the width only"""
    assert [lib.kt_decode_kslices(C, 0) for C in (128, 2048, 4096, 5120, 12288, 17408)] == [1, 1, 2, 3, 6, 9]
    assert [lib.kt_decode_kslices(C, 1) for C in (1856, 2688)] == [4, 6]
    assert lib.kt_decode_kslices(100, 0) == 0


def test_validation_rejects_bad_shapes(lib):
    fake = ctypes.c_void_p(0x1000)
    # C not a multiple of 128
    assert lib.kt_tern_pack(fake, fake, 64, 100, fake, None) == INVALID
    assert lib.kt_quant_q8(fake, 100, 1, 100, 0, fake, 112, fake, fake, None) == INVALID
    assert lib.kt_quant_q8(fake, 128, 1, 128, 3, fake, 128, fake, fake, None) == INVALID   # modes 0, 1, 2 (hp)
    assert lib.kt_tern_gemv(fake, 64, 256, fake, 256, fake, fake, (1 << 30) | (1 << 29) + 1, fake, 64, None,
                            None) == INVALID                                               # hp token count
    # ldq not a multiple of 16
    assert lib.kt_tern_gemv(fake, 64, 256, fake, 260, fake, fake, 1, fake, 64, None, None) == INVALID
    # ldy < R
    assert lib.kt_tern_gemv(fake, 64, 256, fake, 256, fake, fake, 1, fake, 63, None, None) == INVALID
    # null output
    assert lib.kt_tern_gemm(fake, 64, 256, fake, 256, fake, fake, 0, 4, None, None, 64, None, None) == INVALID
    assert lib.kt_tern_gemm(fake, 64, 256, fake, 256, fake, fake, 2, 4, fake, None, 256, None, None) == INVALID
    # the 128 x 128 kernel's 32-bit buffer offsets: M ldq at 2^31 bytes and more is refused (per-group scales, and
    # per-row scales from 8192 rows, take that kernel)
    assert lib.kt_tern_gemm(fake, 64, 256, fake, 1 << 16, fake, fake, 0, 1 << 15, fake, None, 256, None, None) == INVALID
    assert lib.kt_tern_gemm(fake, 8192, 256, fake, 1 << 16, fake, fake, 1, 1 << 15, fake, None, 8192, None,
                            None) == INVALID
    # q8: C % 32
    assert lib.kt_q8_gemv(fake, 64, 48, fake, 48, fake, 1, 1, fake, 64, None, None) == INVALID
    assert lib.kt_q8_quant(fake, 66, 2, 64, 0, fake, 64, fake, 2, None) == INVALID      # ldx % 4 (vector loads)
    assert lib.kt_q8_quant(fake, 64, 2, 64, 0, fake, 66, fake, 2, None) == INVALID      # ldq % 4 (word stores)
    # moe: k > 16, E > 1024
    assert lib.kt_moe_topk(fake, 1, 128, 17, fake, fake, None) == INVALID
    assert lib.kt_moe_sort(fake, 1, 6, 2048, fake, fake, fake, fake, fake, fake, None) == INVALID
    assert lib.kt_moe_sort(fake, 1, 17, 128, fake, fake, fake, fake, fake, fake, None) == INVALID      # k > 16
    assert lib.kt_moe_sort(fake, 1 << 27, 16, 128, fake, fake, fake, fake, fake, fake, None) == INVALID  # M k > 2^30
    # the one-wave route: M k <= 64, checked without int overflow (M k = 2^32 + 6 wraps to 6 in 32 bits)
    route = [fake, 1, 128, 6] + [fake] * 8 + [None, 0, 0, None, 0, None, 0, None]
    assert lib.kt_moe_route(*(route[:1] + [11] + route[2:])) == INVALID                  # 66 entries
    assert lib.kt_moe_route(*(route[:1] + [(1 << 31) // 3 + 1] + route[2:])) == INVALID
    assert lib.kt_moe_route(*(route[:1] + [715827883] + route[2:])) == INVALID          # 6 M wraps to 2 in int32
    # tern_sum: a token count past the grid's y range
    assert lib.kt_tern_sum(fake, fake, 64, 70000, 2, None) == INVALID
    # M = 0: a no-op
    assert lib.kt_tern_gemv(fake, 64, 256, fake, 256, fake, fake, 0, fake, 64, None, None) == 0
    # dbg with several matrices in one launch


def test_record_protocol(lib):
    """kt_record_begin / kt_record_end (launch records): no nesting, no end without a begin, a launcher's own
    validation error still returned while recording and nothing recorded for it, M = 0 records no launch"""
    from kindi_amd import gpudrv
    recs = (gpudrv.KtLaunch * 4)()
    n = ctypes.c_int(-1)
    assert ctypes.sizeof(gpudrv.KtLaunch) == 8 + 4 * 7 + 4 + 8 * 24 + 4 * 24 + 512
    assert lib.kt_record_end(ctypes.byref(n)) == INVALID
    assert lib.kt_record_begin(None, 4) == INVALID
    assert lib.kt_record_begin(recs, -1) == INVALID
    assert lib.kt_record_begin(recs, 4) == 0
    assert lib.kt_record_begin(recs, 4) == INVALID                   # no nesting
    fake = ctypes.c_void_p(0x1000)
    assert lib.kt_tern_gemv(fake, 64, 256, fake, 260, fake, fake, 1, fake, 64, None, None) == INVALID
    assert lib.kt_tern_gemv(fake, 64, 256, fake, 256, fake, fake, 0, fake, 64, None, None) == 0
    assert lib.kt_moe_topk_r(fake, 1, 128, 6, 1, None, 1.0, fake, fake, None) == INVALID   # sigmoid needs a bias
    assert lib.kt_moe_topk_r(fake, 1, 128, 6, 2, fake, 1.0, fake, fake, None) == INVALID   # unknown scoring
    assert lib.kt_record_end(ctypes.byref(n)) == 0 and n.value == 0
    assert lib.kt_record_begin(None, 0) == 0                         # counting only
    assert lib.kt_record_end(None) == 0
    ss = (ctypes.c_void_p * 1)(None)
    assert lib.kt_replay(recs, -1, ss, 1) == INVALID                 # kt_replay checks before launching
    assert lib.kt_replay(None, 1, ss, 1) == INVALID
    assert lib.kt_replay(recs, 1, ss, 0) == INVALID
    assert lib.kt_replay(recs, 0, ss, 1) == 0


def test_fold_validation(lib):
    f = ctypes.c_void_p(0x1000)
    ok = (f, 5120, None, 0, 0, f, f, 1, 5120, 1024, None, 0, None, 0, None, 0, f, 5120, f, f, None)

    def call(**kw):
        a = list(ok)
        names = ["x", "ldx", "r", "ldr", "nparts", "w", "sg", "M", "C", "HB", "xw", "ldxw", "xn", "ldxn", "xo", "ldxo",
                 "XQ", "ldq", "XS", "XA", "stream"]
        for k, v in kw.items():
            a[names.index(k)] = v
        return lib.kt_rmsfold_q8(*a)
    assert call(M=0) == 0                                       # nothing to do: no launch
    assert call(HB=2048) == INVALID                             # fold sizes 512 / 1024 / 4096 only
    assert call(HB=4096) == INVALID                             # 5120 % 4096
    assert call(C=8704, ldx=8704, ldq=8704) == INVALID          # wider than one block's row
    assert call(nparts=9, r=f, ldr=9 * 5120) == INVALID
    assert call(nparts=2, r=None) == INVALID
    assert call(nparts=2, r=f, ldr=5120) == INVALID             # ldr < nparts C
    assert call(sg=None) == INVALID
    assert call(w=None) == INVALID
    assert call(ldq=5000) == INVALID
    assert lib.kt_fold_q8(f, 4000, f, 1, 4096, 4096, None, 0, f, 4096, f, f, None) == INVALID
    assert lib.kt_smfold_q8(f, 4096, f, 4096, f, 128, 4, 7, 1, 4096, 4096, None, 0, f, 4096, f, f, None) == INVALID
    assert lib.kt_smfold_q8(f, 4096, f, 4096, f, 128, 4, 0, 1, 4096, 4096, None, 0, f, 4096, f, f, None) == INVALID


def test_layout_validation(lib):
    f = ctypes.c_void_p(16)
    assert lib.kt_tern_pack_layout(f, f, 100, 512, f, None) == INVALID      # R % 16 (layout.py:38)
    assert lib.kt_tern_pack_layout(f, f, 64, 384, f, None) == INVALID       # C % 512
    assert lib.kt_tern_pack_layout(None, f, 64, 512, f, None) == INVALID
    assert lib.kt_tern_pack_layout(f, f, 64, 512, ctypes.c_void_p(8), None) == INVALID   # W not 16-byte aligned


def test_ptq1_validation(lib):
    f = ctypes.c_void_p(0x1000)
    assert lib.kt_tern_pack_ptq1(f, 100, 200, 0, 100, f, None) == INVALID     # C % 128
    assert lib.kt_tern_pack_ptq1(f, 100, 256, 4, 96, f, None) == INVALID      # row0 % 8
    assert lib.kt_tern_pack_ptq1(f, 100, 256, 0, 20, f, None) == INVALID      # a middle chunk of 20 rows
    assert lib.kt_tern_pack_ptq1(f, 100, 256, 96, 8, f, None) == INVALID      # past R
    assert lib.kt_tern_pack_ptq1(f, 100, 256, 0, 0, f, None) == 0             # nothing to do


def test_moe_decode_validation(lib):
    f = ctypes.c_void_p(1 << 20)
    assert lib.kt_moe_decode_workspace(11, 6, 128, 2688, 1856) == 0           # M k > 64
    assert lib.kt_moe_decode_workspace(1, 6, 128, 2680, 1856) == 0           # H % 32
    n = lib.kt_moe_decode_workspace(1, 6, 128, 2688, 1856)
    assert n > 0
    assert lib.kt_moe_decode(f, f, 128, 2688, 1856, 6, f, 1, f, 2688, None, f, n - 1, None) == 1   # short workspace
    assert lib.kt_moe_decode(f, f, 128, 2688, 1856, 6, f, 1, f, 2686, None, f, n, None) == 1       # ldx % 4
    assert lib.kt_moe_decode(f, f, 128, 2688, 1856, 6, f, 0, f, 2688, None, f, n, None) == 0       # nothing to do


def test_validation_remaining_entries(lib):
    """the entry points the tests above leave out: each rejects a bad argument (or does nothing for an empty call)
    before any device call"""
    f = ctypes.c_void_p(0x1000)
    odd = ctypes.c_void_p(0x1008)                                  # not 16-byte aligned
    assert lib.kt_error_string(INVALID)                              # a message for every return code
    # q8_0 pack: C % 32, the output's alignment, null rows
    assert lib.kt_q8_pack(f, 64, 48, f, None) == INVALID
    assert lib.kt_q8_pack(f, 64, 64, odd, None) == INVALID
    assert lib.kt_q8_pack(None, 64, 64, f, None) == INVALID
    # the int8 trit copy and the product over it
    assert lib.kt_tern_expand_bytes(100, 256) == 104 * 256               # rows padded to the kt2 row groups
    assert lib.kt_tern_expand_bytes(64, 100) == 0
    assert lib.kt_tern_expand(f, 64, 100, f, None) == INVALID
    assert lib.kt_tern_expand(f, 64, 256, odd, None) == INVALID
    assert lib.kt_tern_gemm8(f, f, 64, 256, f, 256, f, 0, f, None, 64, None, None) == 0           # nothing to do
    assert lib.kt_tern_gemm8(f, f, 64, 256, f, 260, f, 1, f, None, 64, None, None) == INVALID     # ldq % 16
    assert lib.kt_tern_gemm8(f, f, 64, 256, f, 256, f, 1, None, None, 64, None, None) == INVALID  # no output
    assert lib.kt_tern_gemm8(f, f, 64, 256, f, 256, f, 1, f, None, 63, None, None) == INVALID     # ldy < R
    assert lib.kt_tern_gemm8(f, f, 64, 256, f, 1 << 16, f, 1 << 15, f, None, 64, None, None) == INVALID  # 2^31 bytes
    # three matrices in one launch: C % 128, a null output of a present matrix
    assert lib.kt_tern_gemv3(f, 64, f, f, 64, f, f, 64, f, 100, f, 112, f, f, 1, None) == INVALID
    assert lib.kt_tern_gemv3(f, 64, f, f, 64, None, f, 64, f, 256, f, 256, f, f, 1, None) == INVALID
    assert lib.kt_tern_gemv3(f, 64, f, f, 64, f, f, 64, f, 256, f, 256, f, f, 0, None) == 0
    # the grouped q8_0 product: C % 32, ldq % 16; no entries is a no-op
    grouped = [f, 64, 64, 8, f, f, f, f, None, 4, 4, f, 64, f, 2, f, 64, None, None]
    assert lib.kt_q8_grouped(*(grouped[:2] + [48] + grouped[3:12] + [48] + grouped[13:])) == INVALID
    assert lib.kt_q8_grouped(*(grouped[:12] + [72] + grouped[13:])) == INVALID
    assert lib.kt_q8_grouped(*(grouped[:9] + [0] + grouped[10:])) == 0
    # combine: k > 16, null inputs; M = 0 is a no-op
    assert lib.kt_moe_combine(f, None, f, f, 0, 6, 64, f, None) == 0
    assert lib.kt_moe_combine(f, None, f, f, 1, 17, 64, f, None) == INVALID
    assert lib.kt_moe_combine(None, None, f, f, 1, 6, 64, f, None) == INVALID
    # the scorings of the routed entry points: sigmoid needs its bias, unknown ones are refused
    route = [f, 1, 128, 6, 1, None, 1.0] + [f] * 8 + [None, 0, 0, None, 0, None, 0, None]
    assert lib.kt_moe_route_r(*route) == INVALID
    assert lib.kt_moe_route_r(*(route[:4] + [2, f] + route[6:])) == INVALID
    assert lib.kt_moe_decode_r(f, f, 128, 2688, 1856, 6, 1, None, 1.0, f, 1, f, 2688, None, f, 1 << 20, None) == INVALID
    assert lib.kt_moe_decode_r(f, f, 128, 2688, 1856, 6, 3, f, 1.0, f, 1, f, 2688, None, f, 1 << 20, None) == INVALID
    # the no-allocation chain: its array's size, shapes past the one-wave route or past the array refused first
    assert lib.kt_moe_decode_noalloc_max() == 4 << 20
    assert lib.kt_moe_decode_noalloc(f, f, 128, 2688, 1856, 6, f, 0, f, 2688, None, None) == 0
    assert lib.kt_moe_decode_noalloc(f, f, 128, 2688, 1856, 6, f, 11, f, 2688, None, None) == INVALID   # M k > 64
    assert lib.kt_moe_decode_workspace(10, 6, 128, 4096, 16384) > lib.kt_moe_decode_noalloc_max()
    assert lib.kt_moe_decode_noalloc(f, f, 128, 4096, 16384, 6, f, 10, f, 4096, None, None) == INVALID


def test_no_fallback_without_library(tmp_path):
    """with the library absent the product path raises KernelError (no CPU fallback): a child process with
    KINDI_KT_LIB pointing at a missing file builds a TernaryMatrix and calls quantize"""
    import subprocess
    import sys
    code = ("import numpy as np, torch\n"
            "from kindi_amd import gpudrv, linear\n"
            "for f in (lambda: linear.TernaryMatrix(np.zeros((32, 8), np.uint8), np.zeros((1, 8), np.uint16), 8, 128,"
            " device='cpu'), lambda: linear.quantize(torch.zeros((1, 128)))):\n"
            "    try:\n"
            "        f()\n"
            "    except gpudrv.KernelError as e:\n"
            "        print('raised', 'not built' in str(e))\n")
    env = dict(os.environ, KINDI_KT_LIB=str(tmp_path / "absent.so"))
    r = subprocess.run([sys.executable, "-c", code], cwd=ROOT, env=env, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    assert r.stdout.split("\n")[:2] == ["raised True", "raised True"], r.stdout

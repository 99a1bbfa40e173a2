"""The kernel module behind the linear-layer calls: libkt_gfx950.so through ctypes.

Kindi loads its kernels by compiling CUDA/HIP source at run time (cp.RawModule, spec.py:144-151; engine.py:88-92)
and launches them through gpudrv.driver() (gpudrv.py:97-101), libamdhip64 under the CUDA driver names. Here the
kernels are prebuilt for gfx950 and each launch is one C call with plain pointers, sizes and a stream
(include/kt.h). There is no fallback: if the library is missing, or the GPU is not a gfx950, loading fails.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.environ.get("KINDI_KT_LIB", os.path.join(HERE, "libkt_gfx950.so"))

P = ctypes.c_void_p
I = ctypes.c_int
S = ctypes.c_size_t

REC_MAXARGS = 24
REC_ARGBYTES = 512


class KtLaunch(ctypes.Structure):
    """kt_launch (include/kt.h): one launch record, the (function, grid, block, arguments) Kindi's plan holds"""
    _fields_ = [("fn", P), ("grid", ctypes.c_uint * 3), ("block", ctypes.c_uint * 3), ("shmem", ctypes.c_uint),
                ("nargs", I), ("args", P * REC_MAXARGS), ("off", ctypes.c_uint * REC_MAXARGS),
                ("argbuf", ctypes.c_uint64 * (REC_ARGBYTES // 8))]


# (name, restype, argtypes): the declarations of include/kt.h
SIGNATURES = [
    ("kt_version", I, []),
    ("kt_init", I, [I]),
    ("kt_error_string", ctypes.c_char_p, [I]),
    ("kt_tern_weight_bytes", S, [I, I]),
    ("kt_tern_pack", I, [P, P, I, I, P, P]),
    ("kt_tern_pack_ptq1", I, [P, I, I, I, I, P, P]),
    ("kt_tern_pack_layout", I, [P, P, I, I, P, P]),
    ("kt_quant_q8", I, [P, I, I, I, I, P, I, P, P, P]),
    ("kt_decode_kslices", I, [I, I]),
    ("kt_tern_gemv", I, [P, I, I, P, I, P, P, I, P, I, P, P]),
    ("kt_tern_gemv3", I, [P, I, P, P, I, P, P, I, P, I, P, I, P, P, I, P]),
    ("kt_tern_sum", I, [P, P, I, I, I, P]),
    ("kt_record_begin", I, [ctypes.POINTER(KtLaunch), I]),
    ("kt_record_end", I, [ctypes.POINTER(I)]),
    ("kt_replay", I, [ctypes.POINTER(KtLaunch), I, ctypes.POINTER(P), I]),
    ("kt_tern_gemm", I, [P, I, I, P, I, P, P, I, I, P, P, I, P, P]),
    ("kt_tern_expand_bytes", S, [I, I]),
    ("kt_tern_expand", I, [P, I, I, P, P]),
    ("kt_tern_gemm8", I, [P, P, I, I, P, I, P, I, P, P, I, P, P]),
    ("kt_q8_weight_bytes", S, [I, I]),
    ("kt_q8_pack", I, [P, I, I, P, P]),
    ("kt_q8_quant", I, [P, I, I, I, I, P, I, P, I, P]),
    ("kt_q8_gemv", I, [P, I, I, P, I, P, I, I, P, I, P, P]),
    ("kt_moe_topk", I, [P, I, I, I, P, P, P]),
    ("kt_moe_topk_r", I, [P, I, I, I, I, P, ctypes.c_float, P, P, P]),
    ("kt_moe_sort", I, [P, I, I, I, P, P, P, P, P, P, P]),
    ("kt_q8_grouped", I, [P, I, I, I, P, P, P, P, P, I, I, P, I, P, I, P, I, P, P]),
    ("kt_moe_combine", I, [P, P, P, P, I, I, I, P, P]),
    ("kt_moe_route", I, [P, I, I, I, P, P, P, P, P, P, P, P, P, I, I, P, I, P, I, P]),
    ("kt_moe_route_r", I, [P, I, I, I, I, P, ctypes.c_float, P, P, P, P, P, P, P, P, P, I, I, P, I, P, I, P]),
    ("kt_rmsfold_q8", I, [P, I, P, I, I, P, P, I, I, I, P, I, P, I, P, I, P, I, P, P, P]),
    ("kt_fold_q8", I, [P, I, P, I, I, I, P, I, P, I, P, P, P]),
    ("kt_smfold_q8", I, [P, I, P, I, P, I, I, I, I, I, I, P, I, P, I, P, P, P]),
    ("kt_moe_decode_workspace", S, [I, I, I, I, I]),
    ("kt_moe_decode", I, [P, P, I, I, I, I, P, I, P, I, P, P, S, P]),
    ("kt_moe_decode_r", I, [P, P, I, I, I, I, I, P, ctypes.c_float, P, I, P, I, P, P, S, P]),
    ("kt_moe_decode_noalloc_max", S, []),
    ("kt_moe_decode_noalloc", I, [P, P, I, I, I, I, P, I, P, I, P, P]),
]

_lib = [None]


class KernelError(RuntimeError):
    pass


def load():
    """the library with its argument types set; raises if it is not built"""
    if _lib[0] is None:
        if not os.path.exists(LIB):
            raise KernelError("libkt_gfx950.so is not built (%s): run `python -m kindi_amd.build`" % LIB)
        h = ctypes.CDLL(LIB)
        for name, res, args in SIGNATURES:
            f = getattr(h, name)
            f.restype = res
            f.argtypes = args
        _lib[0] = h
    return _lib[0]


def driver():
    """the loaded kernel library (the role of Kindi's gpudrv.driver())"""
    return load()


_hip = [None]


def hip():
    """the HIP runtime already in the process (the one the library and torch use), with hipModuleLaunchKernel's
    argument types: Kindi's HIP driver stand-in (gpudrv.py:24-101) binds the same call"""
    if _hip[0] is None:
        h = ctypes.CDLL("libamdhip64.so.7")
        h.hipModuleLaunchKernel.restype = I
        h.hipModuleLaunchKernel.argtypes = [P] + [ctypes.c_uint] * 7 + [P, P, P]
        _hip[0] = h
    return _hip[0]


def check(rc, what=""):
    """raise on a nonzero hipError_t, as Kindi raises on a failed launch (tp.py:944-945, chunk.py:517-518)"""
    if rc:
        msg = load().kt_error_string(rc)
        raise KernelError("%s failed: %s (%d)" % (what or "kernel launch", msg.decode() if msg else "?", rc))
    return rc

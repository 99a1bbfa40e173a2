"""Ternary linear layers on MI355X: the host side of Kindi's linear-call surface over libkt_gfx950.so.

Kindi's callers and what each maps to here:
  Engine.gemv(names, x, outs, parts_ok)       engine.py:254-274      Linear.gemv          (<= 3 tensors, one input)
  build_plan gemm / gemm3 (k_tc_q8 + k_tc_mv) spec.py:619-672        quantize + Linear.gemv_q / gemv3_q
  chunk gemm_tc (k_tc_q8 + k_tc_mm2)          chunk.py:273-296       quantize + Linear.gemm
  layout.repack / spec.repack                 layout.py:32-48, spec.py:327-383   TernaryMatrix (kt_tern_pack)
  a tensor already in layout.repack's layout  layout.py:32-48, kindi.cu:525-536  TernaryMatrix.from_layout

Torch provides device memory and the current stream only; every product runs in the HIP library. Tensors are
CUDA (HIP) tensors on one device; activations fp32 [M, C] row-major.
"""
import ctypes
from collections import namedtuple

import numpy as np
import torch

from . import gpudrv

VP = ctypes.c_void_p


def ptr(t):
    return VP(t.data_ptr()) if t is not None else None


def stream():
    return VP(torch.cuda.current_stream().cuda_stream)


def _dev_u8(a, device):
    if isinstance(a, torch.Tensor):
        return a.to(device=device, dtype=torch.uint8).contiguous()
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint8)).to(device)


def _dev_u16(a, device):
    """uint16 bits (numpy uint16 / torch int16 or uint16) -> a device int16 tensor with the same bits"""
    if isinstance(a, torch.Tensor):
        return a.to(device=device).view(torch.int16).contiguous()
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint16).view(np.int16)).to(device)


class TernaryMatrix(object):
    """One ternary tensor resident in HBM in the kt2 layout (2.125 bits per weight).

    bcodes: the reference pack's codes [C/4, R] (byte = d0 + 3 d1 + 9 d2 + 27 d3, convert.py:49-52);
    dpm: its fp16 scales [C/128, R] as uint16 bits. Numpy arrays are uploaded; device tensors are used as they are.
    W: an optional uint8 device buffer (a slice of a larger pool) to pack into."""

    def __init__(self, bcodes, dpm, R, C, device="cuda", W=None):
        lib = gpudrv.load()
        self.R, self.C = int(R), int(C)
        nbytes = lib.kt_tern_weight_bytes(self.R, self.C)
        if nbytes == 0:
            raise ValueError("ternary tensor %d x %d does not fit the kt2 layout (C %% 128 != 0)" % (R, C))
        bc = _dev_u8(bcodes, device).reshape(-1)
        dp = _dev_u16(dpm, device).reshape(-1)
        if bc.numel() != self.R * self.C // 4 or dp.numel() != self.R * (self.C // 128):
            raise ValueError("pack arrays do not match %d x %d" % (R, C))
        self.W = torch.empty(nbytes, dtype=torch.uint8, device=device) if W is None else W[:nbytes]
        if self.W.numel() < nbytes or self.W.data_ptr() % 16:
            raise ValueError("weight buffer too small or not 16-byte aligned")
        gpudrv.check(lib.kt_tern_pack(ptr(bc), ptr(dp), self.R, self.C, ptr(self.W), stream()), "kt_tern_pack")

    @property
    def nbytes(self):
        return self.W.numel()

    def expand(self, out=None):
        """the signed trits as int8 [8 ceil(R/8), C] (kt_tern_expand): the operand of kt_tern_gemm8. With out=None a
        new tensor; pass a buffer of kt_tern_expand_bytes to reuse one"""
        lib = gpudrv.load()
        n = lib.kt_tern_expand_bytes(self.R, self.C)
        if out is None:
            out = torch.empty(n, dtype=torch.int8, device=self.W.device)
        if out.numel() < n or out.dtype != torch.int8 or out.data_ptr() % 16:
            raise ValueError("int8 trit buffer: %d bytes, 16-byte aligned" % n)
        gpudrv.check(lib.kt_tern_expand(ptr(self.W), self.R, self.C, ptr(out), stream()), "kt_tern_expand")
        return out

    @classmethod
    def _empty(cls, R, C, device, W):
        lib = gpudrv.load()
        self = cls.__new__(cls)
        self.R, self.C = int(R), int(C)
        nbytes = lib.kt_tern_weight_bytes(self.R, self.C)
        if nbytes == 0:
            raise ValueError("ternary tensor %d x %d does not fit the kt2 layout (C %% 128 != 0)" % (R, C))
        self.W = torch.empty(nbytes, dtype=torch.uint8, device=device) if W is None else W[:nbytes]
        if self.W.numel() < nbytes or self.W.data_ptr() % 16:
            raise ValueError("weight buffer too small or not 16-byte aligned")
        return self

    @classmethod
    def from_ptq1(cls, raw, R, C, device="cuda", W=None):
        """the GGUF PTQ1_0 tensor data itself (R rows of C / 128 blocks of 28 bytes; convert.py:33-46), decoded on
        the device straight into the kt2 layout (the same W as the reference pack of it would give)"""
        self = cls._empty(R, C, device, W)
        rd = _dev_u8(raw, device).reshape(-1)
        if rd.numel() != self.R * (self.C // 128) * 28:
            raise ValueError("PTQ1_0 data does not match %d x %d" % (R, C))
        gpudrv.check(gpudrv.load().kt_tern_pack_ptq1(ptr(rd), self.R, self.C, 0, self.R, ptr(self.W), stream()),
                     "kt_tern_pack_ptq1")
        return self

    @classmethod
    def from_layout(cls, wg4, sg4, R, C, device="cuda", W=None):
        """a tensor already repacked by Kindi's layout.repack (layout.py:32-48: the weight bytes in the GEMV layout
        and the scales16 array, as the engine holds them for k_g4), rearranged on the device into the kt2 layout (the
        same W as the pack it came from). R % 16 == 0 and C % 512 == 0, as layout.repack requires"""
        if R % 16 or C % 512:
            raise ValueError("the GEMV layout takes R %% 16 == 0 and C %% 512 == 0 (got %d x %d)" % (R, C))
        self = cls._empty(R, C, device, W)
        wb = _dev_u8(wg4, device).reshape(-1)
        sb = _dev_u16(sg4, device).reshape(-1)
        if wb.numel() != self.R * self.C // 4 or sb.numel() != self.R * (self.C // 128):
            raise ValueError("GEMV-layout arrays do not match %d x %d" % (R, C))
        gpudrv.check(gpudrv.load().kt_tern_pack_layout(ptr(wb), ptr(sb), self.R, self.C, ptr(self.W), stream()),
                     "kt_tern_pack_layout")
        return self


def load_ptq1(path, offset, R, C, device="cuda", W=None, chunk_rows=8192):
    """stream one PTQ1_0 tensor from a GGUF file (its data at byte `offset`) to the device in row chunks: two pinned
    host buffers and two device buffers alternate, so reading chunk i + 1 from the file overlaps its copy and the
    decode of chunk i (the role of tp._stream_to_card, tp.py:236-254, for the packed layout)"""
    m = TernaryMatrix._empty(R, C, device, W)
    bpr = (C // 128) * 28
    chunk_rows = max(8, chunk_rows // 8 * 8)
    src = np.memmap(path, dtype=np.uint8, mode="r", offset=offset, shape=(R * bpr,))
    n = min(chunk_rows, R)
    host = [torch.empty(n * bpr, dtype=torch.uint8, pin_memory=True) for _ in range(2)]
    dev = [torch.empty(n * bpr, dtype=torch.uint8, device=device) for _ in range(2)]
    done = [None, None]
    lib = gpudrv.load()
    for k, r0 in enumerate(range(0, R, chunk_rows)):
        b = k & 1
        rows = min(chunk_rows, R - r0)
        if done[b] is not None:
            done[b].synchronize()                   # the buffers' previous chunk has been decoded
        host[b][:rows * bpr].numpy()[:] = src[r0 * bpr:(r0 + rows) * bpr]
        dev[b][:rows * bpr].copy_(host[b][:rows * bpr], non_blocking=True)
        gpudrv.check(lib.kt_tern_pack_ptq1(ptr(dev[b]), R, C, r0, rows, ptr(m.W), stream()), "kt_tern_pack_ptq1")
        done[b] = torch.cuda.Event()
        done[b].record()
    torch.cuda.current_stream().synchronize()
    return m


# hp (tc.cu tc_hp, KINDI_TC_HP spec.py:63-67): two int8 rows a token, row 2n its int8 row and 2n + 1 the residual's,
# for about 14 bits of activation precision at the same weight traffic; the decode products add each token's two
# row results. XQ / XS / XA then hold 2M rows.
Act = namedtuple("Act", "XQ XS XA M C per_row hp", defaults=(False,))
KT_HP = 1 << 30                                    # the flag carried in M (products) and HB (producers)


def quantize(X, per_row=False, out=None, hp=False):
    """fp32 [M, C] -> int8 rows per 128-column group (k_tc_q8, tc_hip.cu:43-74) or per row; hp: the two-row form
    (k_tc_q8 with hp, tc.cu:195-209, per group). Returns Act."""
    if X.dim() == 1:
        X = X.reshape(1, -1)
    M, C = X.shape
    if X.dtype != torch.float32 or X.stride(1) != 1:
        raise ValueError("quantize takes fp32 rows with unit column stride")
    if hp and per_row:
        raise ValueError("hp is per 128-column group")
    if out is None:
        out = _act_out(M, C, X.device, hp)
    lib = gpudrv.load()
    gpudrv.check(lib.kt_quant_q8(ptr(X), X.stride(0), M, C, 2 if hp else (1 if per_row else 0), ptr(out.XQ),
                                 out.XQ.stride(0), ptr(out.XS), ptr(out.XA), stream()), "kt_quant_q8")
    return Act(out.XQ, out.XS, out.XA, M, C, per_row, hp)


def _act_out(M, C, device, hp=False):
    Mq = 2 * M if hp else M
    return Act(torch.empty((Mq, C), dtype=torch.int8, device=device),
               torch.empty((Mq, C // 128), dtype=torch.float32, device=device),
               torch.empty((Mq, C // 128), dtype=torch.int32, device=device), M, C, False, hp)


def _f32_rows(t, what):
    if t is None:
        return None
    if t.dtype != torch.float32 or t.dim() != 2 or t.stride(1) != 1:
        raise ValueError("%s: fp32 rows with unit column stride" % what)
    return t


def rmsfold(x, w, sg, HB, r=None, nparts=0, xw=None, xn=None, xo=None, out=None, hp=False):
    """k_rmsfold_qT (tcf.cu:370-390; k_rmsfold kindi.cu:350-394) as one launch: x [M, C] fp32 (+ the nparts residual
    parts of r [M, >= nparts C], C apart, in part order) -> RMS norm (weights w) -> sign sg -> Hadamard fold of each
    HB block -> int8 row (hp: the two-row form, ff_q8 tcf.cu:150-205). Returns the Act; xw (x + parts), xn (normed)
    and xo (folded) are written when given."""
    x = _f32_rows(x.reshape(1, -1) if x.dim() == 1 else x, "x")
    M, C = x.shape
    _f32_rows(r, "r"), _f32_rows(xw, "xw"), _f32_rows(xn, "xn"), _f32_rows(xo, "xo")
    out = out or _act_out(M, C, x.device, hp)
    gpudrv.check(gpudrv.load().kt_rmsfold_q8(
        ptr(x), x.stride(0), ptr(r), r.stride(0) if r is not None else 0, nparts, ptr(w), ptr(sg), M, C,
        HB | (KT_HP if hp else 0),
        ptr(xw), xw.stride(0) if xw is not None else 0, ptr(xn), xn.stride(0) if xn is not None else 0,
        ptr(xo), xo.stride(0) if xo is not None else 0, ptr(out.XQ), out.XQ.stride(0), ptr(out.XS), ptr(out.XA),
        stream()), "kt_rmsfold_q8")
    return Act(out.XQ, out.XS, out.XA, M, C, False, hp)


def fold(x, sg, HB, xo=None, out=None, hp=False):
    """k_fold_fwht_qT (tcf.cu:410-426): sign, Hadamard fold of each HB block, int8 row (hp: two rows a token)"""
    x = _f32_rows(x.reshape(1, -1) if x.dim() == 1 else x, "x")
    M, C = x.shape
    _f32_rows(xo, "xo")
    out = out or _act_out(M, C, x.device, hp)
    gpudrv.check(gpudrv.load().kt_fold_q8(ptr(x), x.stride(0), ptr(sg), M, C, HB | (KT_HP if hp else 0), ptr(xo),
                                          xo.stride(0) if xo is not None else 0, ptr(out.XQ), out.XQ.stride(0),
                                          ptr(out.XS), ptr(out.XA), stream()), "kt_fold_q8")
    return Act(out.XQ, out.XS, out.XA, M, C, False, hp)


def smfold(a, b, sg, HB, perm=(1, 1, 1), xo=None, out=None, hp=False):
    """k_smfold_qT (tcf.cu:392-408): SiLU(a) * b in the grouped-head order perm = (hd, nk, rep), sign, fold, int8
    (hp: two rows a token)"""
    a = _f32_rows(a.reshape(1, -1) if a.dim() == 1 else a, "a")
    b = _f32_rows(b.reshape(1, -1) if b.dim() == 1 else b, "b")
    M, C = a.shape
    _f32_rows(xo, "xo")
    out = out or _act_out(M, C, a.device, hp)
    gpudrv.check(gpudrv.load().kt_smfold_q8(ptr(a), a.stride(0), ptr(b), b.stride(0), ptr(sg), perm[0], perm[1],
                                            perm[2], M, C, HB | (KT_HP if hp else 0), ptr(xo),
                                            xo.stride(0) if xo is not None else 0,
                                            ptr(out.XQ), out.XQ.stride(0), ptr(out.XS), ptr(out.XA), stream()),
                 "kt_smfold_q8")
    return Act(out.XQ, out.XS, out.XA, M, C, False, hp)


class Linear(object):
    """The ternary tensors of a model and the products over them (Kindi's linear-call surface).

    decode_max: up to this many tokens a product runs on the wave64 bandwidth kernel (kt_tern_gemv), above it on
    the matrix cores (kt_tern_gemm). Within one kernel a token's result does not depend on how many tokens share
    the pass (tc_hip.cu:14-15)."""

    def __init__(self, mats=None, device="cuda", decode_max=16, per_row=False, hp=False):
        self.w = dict(mats or {})
        self.device = device
        self.decode_max = decode_max
        self.per_row = per_row
        self.hp = hp                               # gemv quantizes x in the two-row form (KINDI_TC_HP)

    def add(self, name, mat):
        self.w[name] = mat

    # ------------------------------------------------------------------ decode
    def gemv_q(self, names, act, outs, dbg=None):
        """up to three tensors with the same (quantized) input in one launch: outs[i] fp32 [M, R_i]
        (k_tc_mv3_* / k_tc_mv*, spec.py:646-673)"""
        lib = gpudrv.load()
        ms = [self.w[n] for n in names]
        if not 1 <= len(ms) <= 3:
            raise ValueError("1 to 3 tensors per launch")
        C = ms[0].C
        if any(m.C != C for m in ms) or act.C != C:
            raise ValueError("tensors of one launch share the input width")
        for m, o in zip(ms, outs):
            if o.dtype != torch.float32 or o.shape[-1] != m.R or o.numel() < act.M * m.R or not o.is_contiguous():
                raise ValueError("output for %d rows x %d tokens" % (m.R, act.M))
        Mf = act.M | (KT_HP if act.hp else 0)          # hp: M tokens of two rows, each output row their sum
        if len(ms) == 1:
            rc = lib.kt_tern_gemv(ptr(ms[0].W), ms[0].R, C, ptr(act.XQ), act.XQ.stride(0), ptr(act.XS), ptr(act.XA),
                                  Mf, ptr(outs[0]), ms[0].R, ptr(dbg), stream())
            return gpudrv.check(rc, "kt_tern_gemv") or 1
        if dbg is not None:
            raise ValueError("dbg takes a single tensor")
        Rs = [m.R for m in ms] + [0] * (3 - len(ms))
        Ws = [ptr(m.W) for m in ms] + [None] * (3 - len(ms))
        Ys = [ptr(o) for o in outs] + [None] * (3 - len(ms))
        rc = lib.kt_tern_gemv3(Ws[0], Rs[0], Ys[0], Ws[1], Rs[1], Ys[1], Ws[2], Rs[2], Ys[2], C, ptr(act.XQ),
                               act.XQ.stride(0), ptr(act.XS), ptr(act.XA), Mf, stream())
        return gpudrv.check(rc, "kt_tern_gemv3") or 1

    def gemv(self, names, x, outs, parts_ok=False):
        """Engine.gemv (engine.py:254-274): up to three ternary tensors with the same fp32 input x ([C] or [M, C]).
        The input is quantized once (the int8 path); every row's sum is completed inside the launch, so the part
        count returned is always 1 (parts_ok is accepted for the reference's signature)."""
        act = quantize(x, self.per_row, hp=self.hp)
        outs = [o.reshape(act.M, -1) for o in outs]
        return self.gemv_q(names, act, outs)

    # ------------------------------------------------------------------ prefill
    def gemm(self, name, act, Y=None, Y16=None, dbg=None):
        """chunk.gemm_tc (chunk.py:273-296): Y fp32 and/or Y16 fp16 [M, R] on the matrix cores"""
        lib = gpudrv.load()
        m = self.w[name]
        if act.C != m.C:
            raise ValueError("input width %d != %d" % (act.C, m.C))
        if act.hp:
            raise ValueError("the prefill product takes one int8 row a token (hp is a decode form)")
        if Y is None and Y16 is None:
            Y = torch.empty((act.M, m.R), dtype=torch.float32, device=act.XQ.device)
        ldy = (Y if Y is not None else Y16).stride(0)
        y16 = Y16.view(torch.int16) if Y16 is not None else None
        rc = lib.kt_tern_gemm(ptr(m.W), m.R, m.C, ptr(act.XQ), act.XQ.stride(0), ptr(act.XS), ptr(act.XA),
                              1 if act.per_row else 0, act.M, ptr(Y), ptr(y16), ldy, ptr(dbg), stream())
        gpudrv.check(rc, "kt_tern_gemm")
        return Y if Y is not None else Y16

    def gemm8(self, name, act, W8, Y=None, Y16=None, dbg=None):
        """the prefill product over the int8 trits W8 (TernaryMatrix.expand) with per-token activation scales: the bits
        of gemm() with per_row activations"""
        lib = gpudrv.load()
        m = self.w[name]
        if act.C != m.C or not act.per_row or act.hp:
            raise ValueError("gemm8 takes per-token int8 activations of width %d" % m.C)
        if Y is None and Y16 is None:
            Y = torch.empty((act.M, m.R), dtype=torch.float32, device=act.XQ.device)
        ldy = (Y if Y is not None else Y16).stride(0)
        y16 = Y16.view(torch.int16) if Y16 is not None else None
        rc = lib.kt_tern_gemm8(ptr(W8), ptr(m.W), m.R, m.C, ptr(act.XQ), act.XQ.stride(0), ptr(act.XS), act.M,
                               ptr(Y), ptr(y16), ldy, ptr(dbg), stream())
        gpudrv.check(rc, "kt_tern_gemm8")
        return Y if Y is not None else Y16

    # ------------------------------------------------------------------ either
    def forward(self, name, X, per_row=None):
        """Y = W X for fp32 X [M, C]: decode kernel up to decode_max tokens, matrix cores above"""
        act = quantize(X, self.per_row if per_row is None else per_row)
        m = self.w[name]
        if act.M <= self.decode_max:
            Y = torch.empty((act.M, m.R), dtype=torch.float32, device=X.device)
            self.gemv_q([name], act, [Y])
            return Y
        return self.gemm(name, act)


class Plan(object):
    """A decode step as launch records: the launches fn() makes through the kt_* launchers, recorded once
    (kt_record_begin / kt_record_end) and replayed in order with hipModuleLaunchKernel, as Kindi's HIP path replays
    its plan (Plan.add tp.py:282-302, Replay.launch spec.py:303-320). The records hold fn's pointers and sizes: the
    buffers it used must live as long as the plan. A failed recording raises KernelError."""

    def __init__(self, fn, max_launches=4096):
        lib = gpudrv.load()
        recs = (gpudrv.KtLaunch * max_launches)()
        gpudrv.check(lib.kt_record_begin(recs, max_launches), "kt_record_begin")
        try:
            fn()
        finally:
            n = ctypes.c_int(0)
            rc = lib.kt_record_end(ctypes.byref(n))
        gpudrv.check(rc, "kt_record_end (%d launches, room for %d)" % (n.value, max_launches))
        self.recs = recs
        self.n = n.value
        # Kindi's node tuples: (fn, grid, block, kernelParams); shmem added, which Replay passes as 0
        self.nodes = [(r.fn, tuple(r.grid), tuple(r.block), r.shmem, r.args) for r in recs[:self.n]]

    def launch(self):
        """the records in order on the current stream, in one C loop (kt_replay)"""
        ss = (VP * 1)(torch.cuda.current_stream().cuda_stream)
        gpudrv.check(gpudrv.load().kt_replay(self.recs, self.n, ss, 1), "kt_replay")

    def launch_nodes(self):
        """the node tuples launched one by one from Python with hipModuleLaunchKernel, as Kindi's Replay does"""
        L = gpudrv.hip().hipModuleLaunchKernel
        s = stream()
        for fn, g, b, sh, args in self.nodes:
            rc = L(fn, g[0], g[1], g[2], b[0], b[1], b[2], sh, s, ctypes.cast(args, VP), None)
            if rc:
                raise gpudrv.KernelError("a plan launch failed (%d)" % rc)

    run = launch


def tern_sum(P, R, M, sp, y=None):
    """k_tc_sum (tc_hip.cu:271-279): parts [M, sp, R] -> [M, R] in part order"""
    if y is None:
        y = torch.empty((M, R), dtype=torch.float32, device=P.device)
    gpudrv.check(gpudrv.load().kt_tern_sum(ptr(P), ptr(y), R, M, sp, stream()), "kt_tern_sum")
    return y

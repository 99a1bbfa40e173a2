"""q8_0 expert products and the MoE dispatch on MI355X (the host side over libkt_gfx950.so).

Kindi's MoE layer (lightning.py:687-785) and what each step maps to here:
  lt_router_topk / lt_router + lt_topk   lightning.cu:348-468     MoE.route        (kt_moe_topk_r: softmax top-k, or
                                                                                    Kindi's sigmoid + bias scoring)
  lt_quant / lt_quant2 (int8 runs)       lightning.cu:70-88, 470   q8_quantize      (kt_q8_quant, act = relu^2)
  lt_moe_lists                           lightning.cu:1318-1349    MoE.lists        (kt_moe_sort)
  lt_mv_q2 slots / lt_mm_* groups        lightning.cu:154-195, 958 Q8Experts.grouped (kt_q8_grouped)
  lt_moe_combine                         lightning.cu:1352-1361    MoE.combine      (kt_moe_combine)
  lt_mv_q8 / dsv41 k_q8 (dense q8_0)     lightning.cu:258-284      Q8Matrix.gemv    (kt_q8_gemv)
"""
import ctypes

import numpy as np
import torch

from . import gpudrv
from .linear import ptr, stream, _dev_u8


def q8_quantize(X, act=0, Q=None, D=None):
    """fp32 [M, C] -> (Q int8 [M, C], D f32 [M, C/32]) per 32 columns; act = 1 applies relu^2 first"""
    M, C = X.shape
    if Q is None:
        Q = torch.empty((M, C), dtype=torch.int8, device=X.device)
    if D is None:
        D = torch.empty((M, C // 32), dtype=torch.float32, device=X.device)
    rc = gpudrv.load().kt_q8_quant(ptr(X), X.stride(0), M, C, act, ptr(Q), Q.stride(0), ptr(D), D.stride(0), stream())
    gpudrv.check(rc, "kt_q8_quant")
    return Q, D


class Q8Matrix(object):
    """One Q8_0 matrix in HBM in the kq8 layout. rows: GGUF Q8_0 rows [R, C/32 * 34] (uint8)."""

    def __init__(self, rows, R, C, device="cuda", W=None):
        lib = gpudrv.load()
        self.R, self.C = int(R), int(C)
        nbytes = lib.kt_q8_weight_bytes(self.R, self.C)
        if nbytes == 0:
            raise ValueError("q8_0 matrix %d x %d: C %% 32 != 0" % (R, C))
        src = _dev_u8(rows, device).reshape(-1)
        if src.numel() != self.R * (self.C // 32) * 34:
            raise ValueError("q8_0 rows do not match %d x %d" % (R, C))
        self.W = torch.empty(nbytes, dtype=torch.uint8, device=device) if W is None else W
        gpudrv.check(lib.kt_q8_pack(ptr(src), self.R, self.C, ptr(self.W), stream()), "kt_q8_pack")

    def gemv(self, Q, D, Y=None, dbg=None):
        """Y [M, R] = W x for the quantized rows (Q, D)"""
        lib = gpudrv.load()
        M = Q.shape[0]
        if Y is None:
            Y = torch.empty((M, self.R), dtype=torch.float32, device=Q.device)
        rc = lib.kt_q8_gemv(ptr(self.W), self.R, self.C, ptr(Q), Q.stride(0), ptr(D), D.stride(0), M, ptr(Y),
                            Y.stride(0), ptr(dbg), stream())
        gpudrv.check(rc, "kt_q8_gemv")
        return Y


class Q8Experts(object):
    """E Q8_0 matrices of one shape (a MoE layer's up or down experts) and their device pointer table.
    rows: uint8 [E, R, C/32 * 34] (numpy or torch) or a list of E such arrays."""

    def __init__(self, rows, R, C, device="cuda"):
        lib = gpudrv.load()
        self.R, self.C = int(R), int(C)
        self.E = len(rows)
        per = lib.kt_q8_weight_bytes(self.R, self.C)
        self.stride = (per + 255) // 256 * 256
        self.W = torch.empty(self.E * self.stride, dtype=torch.uint8, device=device)
        for e in range(self.E):
            Q8Matrix(rows[e], R, C, device, W=self.W[e * self.stride:(e + 1) * self.stride])
        base = self.W.data_ptr()
        self.table = torch.tensor([base + e * self.stride for e in range(self.E)], dtype=torch.int64, device=device)

    @property
    def bytes_per_expert(self):
        return gpudrv.load().kt_q8_weight_bytes(self.R, self.C)

    def grouped(self, lists, M, Q, D, Y, xrow=True, dbg=None):
        """Y[p] = W_e x[xrow[p]] (or x[p]) for every list entry p of every active expert e"""
        cnt, off, xr, where, act, nact = lists
        n = where.numel()
        rc = gpudrv.load().kt_q8_grouped(ptr(self.table), self.R, self.C, self.E, ptr(cnt), ptr(off), ptr(act),
                                         ptr(nact), ptr(xr) if xrow else None, n, M, ptr(Q), Q.stride(0), ptr(D),
                                         D.stride(0), ptr(Y), Y.stride(0), ptr(dbg), stream())
        gpudrv.check(rc, "kt_q8_grouped")
        return Y


SCORES = {"softmax": 0, "sigmoid": 1}          # KT_SCORE_SOFTMAX, KT_SCORE_SIGMOID (include/kt.h)


class MoE(object):
    """A q8_0 MoE feed-forward: x += sum_j gw_j * down_e(relu^2(up_e(x))) over the k routed experts e_j of each
    token (the Lightning expert shape: up [F, H], down [H, F]), token-sorted grouped dispatch.
    score: "softmax" or "sigmoid" (Kindi's Lightning router, lightning.cu:373-468: the k largest
    sigmoid(l) + bias, weights sigmoid(l_j) / sum * scale; bias fp32 [E] on the device)."""

    def __init__(self, up, down, k, device="cuda", score="softmax", bias=None, scale=1.0):
        assert up.E == down.E and up.R == down.C and down.R == up.C
        self.up, self.down, self.k, self.E, self.device = up, down, k, up.E, device
        self.score = SCORES[score]
        if self.score == 1 and (bias is None or bias.numel() != self.E or bias.dtype != torch.float32):
            raise ValueError("the sigmoid router takes an fp32 bias of E = %d entries" % self.E)
        self.bias, self.scale = bias, float(scale)

    def _rt(self):
        return self.score, ptr(self.bias), ctypes.c_float(self.scale)

    def route(self, logits):
        M, E = logits.shape
        ids = torch.empty((M, self.k), dtype=torch.int32, device=logits.device)
        gw = torch.empty((M, self.k), dtype=torch.float32, device=logits.device)
        gpudrv.check(gpudrv.load().kt_moe_topk_r(ptr(logits), M, E, self.k, *self._rt(), ptr(ids), ptr(gw), stream()),
                     "kt_moe_topk_r")
        return ids, gw

    def route_lists(self, logits, x=None, Q=None, D=None):
        """route + lists in one launch: the same ids, weights and lists (and, with x, its int8 rows into Q, D as
        q8_quantize(x) writes them)"""
        M, E = logits.shape
        dev = logits.device
        ids = torch.empty((M, self.k), dtype=torch.int32, device=dev)
        gw = torch.empty((M, self.k), dtype=torch.float32, device=dev)
        cnt = torch.empty(self.E, dtype=torch.int32, device=dev)
        off = torch.empty(self.E, dtype=torch.int32, device=dev)
        xrow = torch.empty(M * self.k, dtype=torch.int32, device=dev)
        where = torch.empty(M * self.k, dtype=torch.int32, device=dev)
        act = torch.empty(self.E, dtype=torch.int32, device=dev)
        nact = torch.empty(1, dtype=torch.int32, device=dev)
        H = x.shape[1] if x is not None else 0
        rc = gpudrv.load().kt_moe_route_r(ptr(logits), M, E, self.k, *self._rt(), ptr(ids), ptr(gw), ptr(cnt),
                                          ptr(off), ptr(xrow), ptr(where), ptr(act), ptr(nact), ptr(x),
                                          x.stride(0) if x is not None else 0, H, ptr(Q),
                                          Q.stride(0) if Q is not None else 0, ptr(D),
                                          D.stride(0) if D is not None else 0, stream())
        gpudrv.check(rc, "kt_moe_route_r")
        return ids, gw, (cnt, off, xrow, where, act, nact)

    def lists(self, ids):
        M, k = ids.shape
        dev = ids.device
        cnt = torch.empty(self.E, dtype=torch.int32, device=dev)
        off = torch.empty(self.E, dtype=torch.int32, device=dev)
        xrow = torch.empty(M * k, dtype=torch.int32, device=dev)
        where = torch.empty(M * k, dtype=torch.int32, device=dev)
        act = torch.empty(self.E, dtype=torch.int32, device=dev)
        nact = torch.empty(1, dtype=torch.int32, device=dev)
        rc = gpudrv.load().kt_moe_sort(ptr(ids), M, k, self.E, ptr(cnt), ptr(off), ptr(xrow), ptr(where), ptr(act),
                                       ptr(nact), stream())
        gpudrv.check(rc, "kt_moe_sort")
        return cnt, off, xrow, where, act, nact

    def combine(self, yd, where, gw, x, ysh=None):
        M, cols = x.shape
        rc = gpudrv.load().kt_moe_combine(ptr(yd), ptr(ysh), ptr(where), ptr(gw), M, self.k, cols, ptr(x), stream())
        gpudrv.check(rc, "kt_moe_combine")
        return x

    def forward(self, x, logits, bufs=None):
        """x fp32 [M, H] updated in place; returns (x, intermediates)"""
        M, H = x.shape
        F = self.up.R
        b = bufs or self.buffers(M)
        if M * self.k <= 64:                     # quantize, route and sort in one launch
            Q, D = b["xq"], b["xd"]
            ids, gw, lists = self.route_lists(logits, x, Q, D)
        else:
            Q, D = q8_quantize(x, 0, b["xq"], b["xd"])
            ids, gw = self.route(logits)
            lists = self.lists(ids)
        self.up.grouped(lists, M, Q, D, b["u"], xrow=True)
        q8_quantize(b["u"], 1, b["uq"], b["ud"])
        self.down.grouped(lists, M, b["uq"], b["ud"], b["yd"], xrow=False)
        self.combine(b["yd"], lists[3], gw, x)
        return x, dict(ids=ids, gw=gw, lists=lists, **b)

    def decode(self, x, logits, work=None, ysh=None):
        """the whole layer at few tokens (M k <= 64) in three launches (kt_moe_decode): x fp32 [M, H] updated in place,
        with the same bits as forward(); work: a uint8 device buffer of workspace(M) bytes (allocated when None)"""
        M, H = x.shape
        lib = gpudrv.load()
        if work is None:
            work = self.workspace(M)
        rc = lib.kt_moe_decode_r(ptr(self.up.table), ptr(self.down.table), self.E, H, self.up.R, self.k, *self._rt(),
                                 ptr(logits), M, ptr(x), x.stride(0), ptr(ysh), ptr(work), work.numel(), stream())
        gpudrv.check(rc, "kt_moe_decode_r")
        return x

    def workspace(self, M):
        n = gpudrv.load().kt_moe_decode_workspace(M, self.k, self.E, self.down.R, self.up.R)
        if n == 0:
            raise ValueError("kt_moe_decode takes M k <= 64 (M = %d, k = %d)" % (M, self.k))
        return torch.empty(n, dtype=torch.uint8, device=self.device)

    def buffers(self, M):
        dev, H, F, n = self.device, self.down.R, self.up.R, M * self.k
        return dict(xq=torch.empty((M, H), dtype=torch.int8, device=dev),
                    xd=torch.empty((M, H // 32), dtype=torch.float32, device=dev),
                    u=torch.empty((n, F), dtype=torch.float32, device=dev),
                    uq=torch.empty((n, F), dtype=torch.int8, device=dev),
                    ud=torch.empty((n, F // 32), dtype=torch.float32, device=dev),
                    yd=torch.empty((n, H), dtype=torch.float32, device=dev))

"""CPU oracle for the quantized linear-layer path. TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module, and only as the
checker (or as the timed CPU baseline). The product (kindi_amd/) never calls it.

Contents:
  - ctypes bindings of oracle/_build/libkt_oracle.so (kt_oracle.c: exact integer restatements and the canonical
    fp32 expressions; AVX2/OpenMP CPU baselines);
  - ctypes bindings of oracle/_ref/*.so when present: the reference's own CPU kernels (kcpu.c, dsv41_cpu.c)
    compiled from their sources by oracle/Makefile;
  - NumPy codecs for the reference's byte formats:
      pack_from_digits / digits_from_pack  - convert.py:49-52 (phase_bytes) and its inverse (convert.py:55-60)
      trits_from_ptq1 / ptq1_from_digits  - convert.py:33-46 (PTQ1_0 decode) and the matching encoder
      paircodes                           - cpu.py:69-88
      layout_g4                           - layout.repack / scales16 (layout.py:14-48), the GEMV layout Kindi's
                                            engine holds on the card for k_g4 / k_deq_emb3 (kindi.cu:525-536)
      q8_0_rows / q8_0_group4             - GGUF Q8_0 rows (dsv41_cpu.c:77-78) and k_q8g's 4-row groups
                                            (dsv41_cpu.c:781-790)
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "_build", "libkt_oracle.so")
REF_KCPU = os.path.join(HERE, "_ref", "libkcpu_ref.so")
REF_DSV41 = os.path.join(HERE, "_ref", "libdsv41_ref.so")

P = ctypes.c_void_p
I = ctypes.c_int
_lib = [None]


def build():
    """compile the oracle (and oracle/_ref where the reference sources exist)"""
    if os.system("make -s -C %s" % HERE):
        raise RuntimeError("oracle build failed")


def lib():
    if _lib[0] is None:
        if not os.path.exists(LIB):
            build()
        h = ctypes.CDLL(LIB)
        h.or_h2f.argtypes = [ctypes.c_uint16]
        h.or_h2f.restype = ctypes.c_float
        h.or_f2h.argtypes = [ctypes.c_float]
        h.or_f2h.restype = ctypes.c_uint16
        h.or_quant_q8.argtypes = [P, I, I, I, I, P, I, P, P]
        h.or_tern_acc.argtypes = [P, I, I, P, I, I, P]
        h.or_tern_out.argtypes = [P, P, P, I, I, I, P, I]
        h.or_tern_out_rs.argtypes = [P, P, P, I, I, I, P, I]
        h.or_tern_sum.argtypes = [P, P, I, I, I]
        h.or_out_tree.argtypes = [P, P, I, P, I, I, I, I, I, I, P, I]
        h.or_out_lanes.argtypes = [P, P, I, P, I, I, I, I, I, I, P, I]
        h.or_pair_gemv.argtypes = [P, P, I, I, P, P, P]
        h.or_paircodes.argtypes = [P, I, I, P]
        h.or_q8_quant.argtypes = [P, I, P, P]
        h.or_q8_acc.argtypes = [P, I, I, P, I, I, P]
        h.or_q8_out.argtypes = [P, P, I, I, P, I, I, P, I]
        h.or_q8_gemv_avx2.argtypes = [P, I, I, P, P, P]
        h.or_moe_sort.argtypes = [P, I, I, I, P, P, P, P]
        h.or_moe_combine.argtypes = [P, P, P, P, I, I, I, P]
        h.or_router_topk.argtypes = [P, I, I, I, P, P]
        h.or_router_sig.argtypes = [P, P, ctypes.c_float, I, I, I, P, P]
        h.or_sumsq.argtypes = [P, I]
        h.or_sumsq.restype = ctypes.c_double
        h.or_fwht_blocks.argtypes = [P, I, I]
        h.or_rmsfold_q8.argtypes = [P, I, P, I, I, P, P, I, I, I, P, I, P, I, P, I, P, I, P, P]
        h.or_fold_q8.argtypes = [P, I, P, I, I, I, P, I, P, I, P, P]
        h.or_perm_src.argtypes = [I, I, I, I]
        h.or_smfold_q8.argtypes = [P, I, P, I, P, I, I, I, I, I, I, P, I, P, I, P, P]
        _lib[0] = h
    return _lib[0]


def _p(a):
    return a.ctypes.data_as(P) if a is not None else None


def _c(a, dt):
    a = np.ascontiguousarray(a, dtype=dt)
    return a


# ----------------------------------------------------------------------------------------------- pack formats
POW3 = np.array([1, 3, 9, 27, 81, 243], dtype=np.uint32)


def pack_from_digits(dig):
    """digits [R, C] in {0,1,2} -> bcodes [C/4, R] (byte = d0 + 3 d1 + 9 d2 + 27 d3 of columns 4s..4s+3;
    convert.py:49-52, stored slot-major as convert.py:154)"""
    R, C = dig.shape
    g = dig.reshape(R, C // 4, 4).astype(np.int32)
    b = (g[:, :, 0] + 3 * g[:, :, 1] + 9 * g[:, :, 2] + 27 * g[:, :, 3]).astype(np.uint8)
    return np.ascontiguousarray(b.T)


def digits_from_pack(bcodes, R, C):
    """bcodes [C/4, R] -> digits [R, C] (the inverse, as convert.selftest convert.py:55-60)"""
    b = np.asarray(bcodes, dtype=np.int32).reshape(C // 4, R).T
    return np.stack([b % 3, (b // 3) % 3, (b // 9) % 3, (b // 27) % 3], axis=2).reshape(R, C).astype(np.uint8)


def trits_from_ptq1(raw):
    """GGUF PTQ1_0 blocks (nb, 28) -> (nb, 128) digits (convert.py:33-46: byte j of qs holds 5 digits, digit n =
    the top of (byte * 3^n mod 256) * 3 / 256)"""
    nb = raw.shape[0]
    out = np.empty((nb, 128), dtype=np.uint8)
    for n in range(5):
        q = (raw[:, 0:16].astype(np.uint32) * POW3[n]) & 0xFF
        out[:, n * 16:(n + 1) * 16] = (q * 3) >> 8
    for n in range(5):
        q = (raw[:, 16:24].astype(np.uint32) * POW3[n]) & 0xFF
        out[:, 80 + n * 8:88 + n * 8] = (q * 3) >> 8
    for n in range(4):
        q = (raw[:, 24:26].astype(np.uint32) * POW3[n]) & 0xFF
        out[:, 120 + n * 2:122 + n * 2] = (q * 3) >> 8
    return out


def ptq1_from_digits(dig, scales):
    """(nb, 128) digits + (nb,) fp16 bits -> (nb, 28) PTQ1_0 blocks: the TQ1 encoding ceil(v * 256 / 243) of
    v = sum of the 5 (or 4) digits weighted 81, 27, 9, 3, 1 (ggml's order: element n*16 + j in byte j), which
    trits_from_ptq1 inverts"""
    nb = dig.shape[0]
    raw = np.zeros((nb, 28), dtype=np.uint8)
    d = dig.astype(np.uint32)

    def enc(cols, nd):
        v = np.zeros(cols[0].shape, dtype=np.uint32)
        for n in range(nd):
            v = v * 3 + cols[n]
        for n in range(nd, 5):
            v = v * 3
        return ((v * 256 + 242) // 243).astype(np.uint8)

    raw[:, 0:16] = enc([d[:, n * 16:(n + 1) * 16] for n in range(5)], 5)
    raw[:, 16:24] = enc([d[:, 80 + n * 8:88 + n * 8] for n in range(5)], 5)
    raw[:, 24:26] = enc([d[:, 120 + n * 2:122 + n * 2] for n in range(4)], 4)
    raw[:, 26:28] = np.asarray(scales, dtype=np.uint16).reshape(nb, 1).view(np.uint8)
    return raw


def _g4_base_row(lane):
    """first of the two rows of a 16-row group that lane (0..7 within its group) holds: bit 0 of the lane selects
    8 rows, bit 1 four, bit 2 two (layout.py:14-15)"""
    return (lane & 1) * 8 + ((lane >> 1) & 1) * 4 + ((lane >> 2) & 1) * 2


def layout_g4(bcodes, dpm, R, C):
    """the reference pack (bcodes [C/4, R], dpm [C/128, R]) -> Kindi's load-time GEMV layout (layout.py:1-8,32-48):
    bytes in the order [16-row group][512-column phase][4-row chunk][lane 0..31][row in chunk][byte in word], lane l of
    a phase holding pack bytes 4 (32 ph + l) .. + 3 (columns 16 (32 ph + l) .. + 15); scales in the order
    [16-row group][phase][lane][2], lane l holding rows b(l), b(l) + 1 of its group for the 128-column group
    4 ph + l / 8 (scales16, layout.py:18-28). Written here as a gather over the output positions."""
    if R % 16 or C % 512:
        raise ValueError("the GEMV layout takes R % 16 == 0 and C % 512 == 0")
    bc = np.asarray(bcodes, dtype=np.uint8).reshape(C // 4, R)
    dp = np.asarray(dpm, dtype=np.uint16).reshape(C // 128, R)
    g16, ph, ch, ln, rl, sl = np.indices((R // 16, C // 512, 4, 32, 4, 4), sparse=True)
    w = bc[(ph * 32 + ln) * 4 + sl, (g16 * 4 + ch) * 4 + rl]
    g16, ph, ln, jj = np.indices((R // 16, C // 512, 32, 2), sparse=True)
    sc = dp[ph * 4 + (ln >> 3), g16 * 16 + _g4_base_row(ln & 7) + jj]
    return np.ascontiguousarray(w).reshape(-1), np.ascontiguousarray(sc).reshape(-1)


_CODE = np.array([0, 1, 2, 3, 8, 4, 5, 6, 7], dtype=np.uint32)     # d0 + 3 d1 -> pair code (both zero -> 8)


def paircodes(bcodes, R, C):
    """bcodes [C/4, R] -> uint32 [R/8, C/128, 64]: word p holds the 8 rows' 4-bit pair codes of columns 2p, 2p+1
    (cpu.py:69-88)"""
    G = C // 128
    dig = digits_from_pack(bcodes, R, C).reshape(R, G, 64, 2).astype(np.uint32)
    pc = _CODE[dig[..., 0] + 3 * dig[..., 1]].reshape(R // 8, 8, G, 64)
    word = np.zeros((R // 8, G, 64), dtype=np.uint32)
    for l in range(8):
        word |= pc[:, l] << np.uint32(4 * l)
    return word


def paircodes_fast(bcodes, R, C):
    """paircodes() in C (OpenMP), for full-size matrices"""
    out = np.empty((R // 8, C // 128, 64), np.uint32)
    lib().or_paircodes(_p(_c(bcodes, np.uint8)), R, C, _p(out))
    return out


def pair_scales(dpm, R, C):
    """dpm [C/128, R] fp16 bits -> fp32 [R/8, C/128, 8] (kcpu.c Mat.S)"""
    G = C // 128
    s = np.asarray(dpm, dtype=np.uint16).reshape(G, R).view(np.float16).astype(np.float32)
    return np.ascontiguousarray(s.T.reshape(R // 8, 8, G).transpose(0, 2, 1))


def q8_0_rows(codes, scales):
    """codes int8 [R, C], scales fp16 bits [R, C/32] -> GGUF Q8_0 rows uint8 [R, C/32 * 34]"""
    R, C = codes.shape
    nb = C // 32
    out = np.empty((R, nb, 34), dtype=np.uint8)
    out[:, :, :2] = np.asarray(scales, dtype=np.uint16).reshape(R, nb, 1).view(np.uint8)
    out[:, :, 2:] = np.asarray(codes, dtype=np.int8).reshape(R, nb, 32).view(np.uint8)
    return out.reshape(R, nb * 34)


def q8_0_group4(rows, R, C):
    """GGUF Q8_0 rows -> k_q8g's 4-row groups (dsv41_cpu.c:781-790): per group and block, 4 fp16 scales then
    4 x 32 codes"""
    nb = C // 32
    b = np.asarray(rows, dtype=np.uint8).reshape(R // 4, 4, nb, 34)
    out = np.empty((R // 4, nb, 136), dtype=np.uint8)
    out[:, :, :8] = b[:, :, :, :2].transpose(0, 2, 1, 3).reshape(R // 4, nb, 8)
    out[:, :, 8:] = b[:, :, :, 2:].transpose(0, 2, 1, 3).reshape(R // 4, nb, 128)
    return out


# ----------------------------------------------------------------------------------------------- wrappers
def h2f(h):
    return lib().or_h2f(int(h))


def f2h(f):
    return lib().or_f2h(float(f))


def quant_q8(X, per_row=False):
    """fp32 [M, C] -> (Q int8 [M', C], XS f32 [M', C/128], XA i32 [M', C/128]). per_row: 0 / False per 128-column
    group, 1 / True per row, 2 hp as k_tc_q8 (tc.cu:195-209), 3 hp as the producers' ff_q8 (tcf.cu:150-205); with hp
    M' = 2M (row 2n the int8 row, 2n + 1 its residual), else M' = M"""
    X = _c(X, np.float32)
    M, C = X.shape
    mode = int(per_row)
    Mo = 2 * M if mode >= 2 else M
    Q = np.empty((Mo, C), np.int8)
    XS = np.empty((Mo, C // 128), np.float32)
    XA = np.empty((Mo, C // 128), np.int32)
    lib().or_quant_q8(_p(X), C, M, C, mode, _p(Q), C, _p(XS), _p(XA))
    return Q, XS, XA


def tern_acc(bcodes, R, C, Q):
    """exact int32 group values [M, R, C/128]"""
    Q = _c(Q, np.int8)
    M = Q.shape[0]
    acc = np.empty((M, R, C // 128), np.int32)
    lib().or_tern_acc(_p(_c(bcodes, np.uint8)), R, C, _p(Q), Q.shape[1], M, _p(acc))
    return acc


def tern_out(acc, XS, dpm, R, C):
    M = acc.shape[0]
    Y = np.empty((M, R), np.float32)
    lib().or_tern_out(_p(_c(acc, np.int32)), _p(_c(XS, np.float32)), _p(_c(dpm, np.uint16)), R, C // 128, M, _p(Y), R)
    return Y


def tern_out_rs(acc, XS, dpm, R, C):
    """the prefill order for per-row activation scales: Y = XS[n][0] * (fma chain of v_g * d_g over the groups)"""
    M = acc.shape[0]
    Y = np.empty((M, R), np.float32)
    lib().or_tern_out_rs(_p(_c(acc, np.int32)), _p(_c(XS, np.float32)), _p(_c(dpm, np.uint16)), R, C // 128, M,
                         _p(Y), R)
    return Y


def out_tree(acc, XS, dq, nsplit, nwave, fmt):
    """Y [M, R] from exact unit values acc [M, R, NU] in the fixed split tree (fmt 0 ternary, 1 q8_0);
    XS [M, NU] activation scales; dq [NU, R] fp32 weight scales"""
    acc = _c(acc, np.int32)
    M, R, NU = acc.shape
    XS = _c(XS, np.float32)
    Y = np.empty((M, R), np.float32)
    lib().or_out_tree(_p(acc), _p(XS), XS.shape[1], _p(_c(dq, np.float32)), R, NU, M, nsplit, nwave, fmt, _p(Y), R)
    return Y


def out_lanes(acc, XS, dq, KL, fmt, KS=1):
    """Y [M, R] from exact unit values in the decode products' order: KS slices of steps of KL units; in a slice
    units dealt to KL lanes (strided fma chains), the lanes added by an xor butterfly, slices left to right.
    fmt 0 ternary, 1 q8_0; XS [M, NU]; dq [NU, R] fp32 weight scales"""
    acc = _c(acc, np.int32)
    M, R, NU = acc.shape
    XS = _c(XS, np.float32)
    Y = np.empty((M, R), np.float32)
    lib().or_out_lanes(_p(acc), _p(XS), XS.shape[1], _p(_c(dq, np.float32)), R, NU, M, KL, KS, fmt, _p(Y), R)
    return Y


def tern_sum(Pt, R, M, sp):
    y = np.empty((M, R), np.float32)
    lib().or_tern_sum(_p(_c(Pt, np.float32)), _p(y), R, M, sp)
    return y


def tern_linear(bcodes, dpm, R, C, X, per_row=False):
    """the whole oracle product: quantize, exact group values, canonical fp32 output"""
    Q, XS, XA = quant_q8(X, per_row)
    acc = tern_acc(bcodes, R, C, Q)
    return tern_out(acc, XS, dpm, R, C), acc, (Q, XS, XA)


def pair_gemv(Pc, S, R, C, x):
    y = np.empty(R, np.float32)
    T = np.empty(C * 4 + 8, np.float32)
    off = (-T.ctypes.data % 32) // 4
    Tv = T[off:off + C * 4]
    lib().or_pair_gemv(_p(_c(Pc, np.uint32)), _p(_c(S, np.float32)), R, C, _p(_c(x, np.float32)), _p(y), _p(Tv))
    return y


def q8_quant(x):
    """fp32 [..., n] -> (q int8, d f32 [..., n/32]) per row"""
    x = _c(x, np.float32)
    sh = x.shape
    x2 = x.reshape(-1, sh[-1])
    q = np.empty(x2.shape, np.int8)
    d = np.empty((x2.shape[0], sh[-1] // 32), np.float32)
    for i in range(x2.shape[0]):
        lib().or_q8_quant(_p(x2[i]), sh[-1], _p(q[i]), _p(d[i]))
    return q.reshape(sh), d.reshape(sh[:-1] + (sh[-1] // 32,))


def q8_acc(rows, R, C, Q):
    Q = _c(Q, np.int8)
    M = Q.shape[0]
    acc = np.empty((M, R, C // 32), np.int32)
    lib().or_q8_acc(_p(_c(rows, np.uint8)), R, C, _p(Q), Q.shape[1], M, _p(acc))
    return acc


def q8_out(acc, rows, R, C, D):
    D = _c(D, np.float32)
    M = acc.shape[0]
    Y = np.empty((M, R), np.float32)
    lib().or_q8_out(_p(_c(acc, np.int32)), _p(_c(rows, np.uint8)), R, C, _p(D), D.shape[1], M, _p(Y), R)
    return Y


def q8_gemv_avx2(rows, R, C, q, d):
    y = np.empty(R, np.float32)
    lib().or_q8_gemv_avx2(_p(_c(rows, np.uint8)), R, C, _p(_c(q, np.int8)), _p(_c(d, np.float32)), _p(y))
    return y


def moe_sort(ids, E):
    ids = _c(ids, np.int32)
    M, k = ids.shape
    cnt = np.empty(E, np.int32)
    off = np.empty(E, np.int32)
    xrow = np.empty(M * k, np.int32)
    where = np.empty(M * k, np.int32)
    lib().or_moe_sort(_p(ids), M, k, E, _p(cnt), _p(off), _p(xrow), _p(where))
    return cnt, off, xrow, where


def moe_combine(yd, ysh, where, gw, x):
    x = np.array(x, dtype=np.float32, copy=True)
    M, cols = x.shape
    k = gw.shape[1]
    lib().or_moe_combine(_p(_c(yd, np.float32)), _p(_c(ysh, np.float32)) if ysh is not None else None,
                         _p(_c(where, np.int32)), _p(_c(gw, np.float32)), M, k, cols, _p(x))
    return x


def router_topk(logits, k):
    logits = _c(logits, np.float32)
    M, E = logits.shape
    ids = np.empty((M, k), np.int32)
    gw = np.empty((M, k), np.float32)
    lib().or_router_topk(_p(logits), M, E, k, _p(ids), _p(gw))
    return ids, gw


def router_sig(logits, bias, scale, k):
    """Kindi's sigmoid + bias router (lt_topk, lightning.cu:373-412)"""
    logits = _c(logits, np.float32)
    bias = _c(bias, np.float32)
    M, E = logits.shape
    ids = np.empty((M, k), np.int32)
    gw = np.empty((M, k), np.float32)
    lib().or_router_sig(_p(logits), _p(bias), scale, M, E, k, _p(ids), _p(gw))
    return ids, gw


# ----------------------------------------------------------------------------------------------- the reference's own
_ref = {}


def ref_kcpu():
    """oracle/_ref/libkcpu_ref.so (kcpu.c's gemv), or None when it was not built"""
    if "kcpu" not in _ref:
        h = None
        if os.path.exists(REF_KCPU):
            h = ctypes.CDLL(REF_KCPU)
            h.ref_gemv.argtypes = [P, P, I, I, P, P, P]
            h.ref_pair_tables.argtypes = [P, P, I, I]
            h.ref_rows8.argtypes = [P, P, I, I, P, P, I, I]
        _ref["kcpu"] = h
    return _ref["kcpu"]


def ref_dsv41():
    """oracle/_ref/libdsv41_ref.so (dsv41_cpu.c's quant_q8 and k_q8g), or None"""
    if "dsv41" not in _ref:
        h = None
        if os.path.exists(REF_DSV41):
            h = ctypes.CDLL(REF_DSV41)
            h.ref_quant_q8.argtypes = [P, I, P, P]
            h.ref_k_q8g.argtypes = [P, I, I, P, P, I, P, I]
            h.ref_q8_matvec.argtypes = [P, I, I, I, P, P, P, I]
        _ref["dsv41"] = h
    return _ref["dsv41"]


def aligned_empty(n, dtype=np.float32, align=32):
    dt = np.dtype(dtype)
    raw = np.empty(n * dt.itemsize + align, np.uint8)
    off = (-raw.ctypes.data) % align
    return raw[off:off + n * dt.itemsize].view(dt)


def ref_gemv(Pc, S, R, C, x):
    h = ref_kcpu()
    y = np.empty(R, np.float32)
    T = aligned_empty(C * 4)
    h.ref_gemv(_p(_c(Pc, np.uint32)), _p(_c(S, np.float32)), R, C, _p(_c(x, np.float32)), _p(y), _p(T))
    return y


def ref_quant_q8(x):
    h = ref_dsv41()
    x = _c(x, np.float32)
    q = np.empty(x.shape, np.int8)
    d = np.empty(x.size // 32, np.float32)
    h.ref_quant_q8(_p(x), x.size, _p(q), _p(d))
    return q, d


def ref_q8_matvec(g4, R, C, q, d, y):
    """every 4-row group of one matrix through k_q8g (the reference's AVX2 q8_0 kernel), threads over groups; q, d one
    token's int8 row and block scales (quant_q8); y fp32 [R]"""
    ref_dsv41().ref_q8_matvec(_p(g4), R, C, 1, _p(q), _p(d), _p(y), 1)
    return y


def ref_k_q8g(g4, R, C, q, d):
    """one token through k_q8g over all 4-row groups"""
    h = ref_dsv41()
    nb = C // 32
    y = np.empty(R, np.float32)
    q = _c(q, np.int8)
    d = _c(d, np.float32)
    g4 = _c(g4, np.uint8)
    for g in range(R // 4):
        h.ref_k_q8g(g4[g].ctypes.data_as(P), nb, 1, _p(q), _p(d), C, y[4 * g:].ctypes.data_as(P), 1)
    return y


# ----------------------------------------------------------------------------------------------- fused producers
HP = 1 << 30                                   # HB | HP: the producers' two-row (hp) int8 output


def _prod_out(M, C, hp=False):
    Mq = 2 * M if hp else M
    return (np.empty((M, C), np.float32), np.empty((Mq, C), np.int8), np.empty((Mq, C // 128), np.float32),
            np.empty((Mq, C // 128), np.int32))


def sumsq(xf):
    """the reference's double sum of squares of one row (512 threads, 32-lane butterflies)"""
    xf = _c(xf, np.float32)
    return lib().or_sumsq(_p(xf), xf.size)


def fwht_blocks(v, HB):
    """per-HB-block unnormalised Walsh-Hadamard transform, then the 1/sqrt(HB) scale (returns a new array)"""
    v = np.array(v, dtype=np.float32, copy=True)
    lib().or_fwht_blocks(_p(v), v.size, HB)
    return v


def rmsfold_q8(x, r, nparts, w, sg, HB, hp=False):
    """k_rmsfold_qT: x [M, C]; r [M, nparts * C] (parts C apart) or None -> dict xw, xn, xo, Q, XS, XA (hp: Q, XS, XA
    with rows 2n / 2n + 1, ff_q8 tcf.cu:150-205)"""
    x = _c(x, np.float32)
    M, C = x.shape
    rr = _c(r, np.float32).reshape(M, -1) if nparts else None
    xw = np.empty((M, C), np.float32)
    xn = np.empty((M, C), np.float32)
    xo, Q, XS, XA = _prod_out(M, C, hp)
    lib().or_rmsfold_q8(_p(x), C, _p(rr), rr.shape[1] if nparts else 0, nparts, _p(_c(w, np.float32)),
                        _p(_c(sg, np.float32)), M, C, HB | (HP if hp else 0), _p(xw), C, _p(xn), C, _p(xo), C, _p(Q), C,
                        _p(XS), _p(XA))
    return dict(xw=xw if nparts else None, xn=xn, xo=xo, Q=Q, XS=XS, XA=XA)


def fold_q8(x, sg, HB, hp=False):
    """k_fold_fwht_qT: x [M, C] -> dict xo, Q, XS, XA"""
    x = _c(x, np.float32)
    M, C = x.shape
    xo, Q, XS, XA = _prod_out(M, C, hp)
    lib().or_fold_q8(_p(x), C, _p(_c(sg, np.float32)), M, C, HB | (HP if hp else 0), _p(xo), C, _p(Q), C, _p(XS),
                     _p(XA))
    return dict(xo=xo, Q=Q, XS=XS, XA=XA)


def smfold_q8(a, b, sg, HB, perm=(1, 1, 1), hp=False):
    """k_smfold_qT: SiLU(a) * b at the permuted columns (perm = (hd, nk, rep)) -> dict xo, Q, XS, XA"""
    a = _c(a, np.float32)
    b = _c(b, np.float32)
    M, C = a.shape
    xo, Q, XS, XA = _prod_out(M, C, hp)
    lib().or_smfold_q8(_p(a), C, _p(b), C, _p(_c(sg, np.float32)), perm[0], perm[1], perm[2], M, C,
                       HB | (HP if hp else 0), _p(xo), C,
                       _p(Q), C, _p(XS), _p(XA))
    return dict(xo=xo, Q=Q, XS=XS, XA=XA)

"""Pins of the CPU oracle (oracle/), each against something other than its own formula: the reference's compiled
CPU code (oracle/_ref), brute-force integer arithmetic in NumPy, float64 closed forms, format round trips and
hand-built known answers."""
import numpy as np
import pytest


def rng(seed):
    return np.random.default_rng(seed)


def rand_digits(R, C, seed):
    u = rng(seed).random((R, C))
    return ((u >= 0.3).astype(np.uint8) + (u >= 0.7).astype(np.uint8))


def rand_scales(shape, seed):
    return np.exp(rng(seed).normal(-3.0, 0.3, shape)).astype(np.float16).view(np.uint16)


# ------------------------------------------------------------------------------------------- formats
def test_pack_round_trip_selftest(orc):
    """convert.selftest (convert.py:55-60): 4096 x 128 random digits, seed 7, survive bytes -> digits"""
    tr = np.random.RandomState(7).randint(0, 3, size=(4096, 128)).astype(np.uint8)
    b = orc.pack_from_digits(tr)
    assert b.shape == (32, 4096) and b.max() <= 80
    assert np.array_equal(orc.digits_from_pack(b, 4096, 128), tr)


def test_pack_known_answers(orc):
    # byte = d0 + 3 d1 + 9 d2 + 27 d3 (convert.py:49-52): digits (2,0,1,2) -> 2 + 0 + 9 + 54 = 65; all zero-weights
    # (digit 1) -> 40 (the padding code layout.py:76 uses)
    d = np.array([[2, 0, 1, 2, 1, 1, 1, 1]], dtype=np.uint8)
    b = orc.pack_from_digits(d)
    assert b[:, 0].tolist() == [65, 40]


def _deq_emb3_index(row, e, C):
    """k_deq_emb3's reads of column e of a row in the GEMV layout (kindi.cu:525-536): (byte index, slot within the
    byte, scale index) - the consumer's statement of the layout, written out per element"""
    s, p, slot = e >> 2, e >> 7, e & 3
    r4, rl, g16, rr = row >> 2, row & 3, row >> 4, row & 15
    bi = ((((row >> 4) * (C >> 9) + (s >> 7)) * 4 + (r4 & 3)) * 32 + ((s >> 2) & 31)) * 16 + rl * 4 + (s & 3)
    lane_low = ((rr >> 3) & 1) | (((rr >> 2) & 1) << 1) | (((rr >> 1) & 1) << 2)
    lane = ((p & 3) << 3) | lane_low
    return bi, slot, ((g16 * (C >> 9) + (p >> 2)) * 32 + lane) * 2 + (rr & 1)


def test_layout_g4_against_deq_emb3(orc):
    """layout_g4 (restated from layout.py) read back element by element with kindi.cu's own decode of that layout:
    every weight digit and scale of a 32 x 1024 tensor comes back; hand-placed known answers"""
    R, C = 32, 1024
    dig = rand_digits(R, C, 11)
    bc = orc.pack_from_digits(dig)
    dpm = rand_scales((C // 128, R), 12)
    wg, sg = orc.layout_g4(bc, dpm, R, C)
    assert wg.size == bc.size and sg.size == dpm.size
    for row in range(R):
        for e in range(C):
            bi, slot, si = _deq_emb3_index(row, e, C)
            assert (int(wg[bi]) // 3 ** slot) % 3 == dig[row, e], (row, e)
            if e % 128 == 0:
                assert sg[si] == dpm[e // 128, row], (row, e)
    # row 5, column 100 of a 16 x 512 tensor: pack byte 25 -> phase 0, lane 6, byte 1 of chunk 1's row 1:
    # ((1 * 32 + 6) * 16) + 4 + 1 = 613; its group-2 scale: row 5 = base 4 (lane 2) + 1, lane 2 + 8 * 2 = 18 -> 37
    bc1 = np.zeros((128, 16), np.uint8)
    bc1[25, 5] = 77
    dp1 = np.zeros((4, 16), np.uint16)
    dp1[2, 5] = 0x3C00
    w1, s1 = orc.layout_g4(bc1, dp1, 16, 512)
    assert np.flatnonzero(w1).tolist() == [613] and w1[613] == 77
    assert np.flatnonzero(s1).tolist() == [37] and s1[37] == 0x3C00
    with pytest.raises(ValueError):
        orc.layout_g4(bc1[:, :8], dp1[:, :8], 8, 512)


def test_ptq1_round_trip_and_known_answer(orc):
    """PTQ1_0 decode (convert.py:33-46) inverts the TQ1 encoding ceil(v * 256 / 243)"""
    dig = rand_digits(300, 128, 3)
    sc = rand_scales(300, 4)
    raw = orc.ptq1_from_digits(dig, sc)
    assert np.array_equal(orc.trits_from_ptq1(raw), dig)
    assert np.array_equal(raw[:, 26:28].copy().view(np.uint16).ravel(), sc)
    # all digits 2: v = 242 -> byte ceil(242 * 256 / 243) = 255; all digits 0 -> 0
    d2 = np.full((1, 128), 2, np.uint8)
    r2 = orc.ptq1_from_digits(d2, [0])
    assert (r2[0, :24] == 255).all()
    assert np.array_equal(orc.trits_from_ptq1(r2), d2)


def test_paircodes_fast_matches_numpy(orc):
    R, C = 64, 512
    bc = orc.pack_from_digits(rand_digits(R, C, 6))
    assert np.array_equal(orc.paircodes_fast(bc, R, C), orc.paircodes(bc, R, C))


def test_paircodes_decode(orc):
    """cpu.paircodes (cpu.py:69-88): code k < 8 -> the k-th nonzero (w0, w1) pair, 8 -> both zero"""
    R, C = 16, 256
    dig = rand_digits(R, C, 5)
    words = orc.paircodes(orc.pack_from_digits(dig), R, C)
    pairs = [(-1, -1), (0, -1), (1, -1), (-1, 0), (1, 0), (-1, 1), (0, 1), (1, 1)]
    t = dig.astype(int) - 1
    for r in (0, 7, 9, 15):
        for c in (0, 2, 100, 254):
            g, p = c // 128, (c % 128) // 2
            code = (int(words[r // 8, g, p]) >> (4 * (r % 8))) & 15
            got = (0, 0) if code == 8 else pairs[code]
            assert got == (t[r, c], t[r, c + 1])


def test_fp16_conversions(orc):
    vals = np.array([0.0, -0.0, 1.0, 65504.0, 65519.0, 6.1e-5, 5.96e-8, 1e-9, 3.14159, -2.5e-3, 2 ** -24 * 1.5],
                    dtype=np.float32)
    vals = np.concatenate([vals, rng(2).normal(0, 3, 2000).astype(np.float32),
                           np.exp(rng(3).normal(-6, 3, 2000)).astype(np.float32)])
    for v in vals:
        assert orc.f2h(v) == int(np.float32(v).astype(np.float16).view(np.uint16))
    for h in rng(1).integers(0, 0x7C00, 2000):
        assert orc.h2f(h) == float(np.uint16(h).view(np.float16))


# ------------------------------------------------------------------------------------------- activations
def test_quant_special_cases(orc):
    C = 256
    X = np.zeros((3, C), np.float32)
    X[1, :128] = np.linspace(-1.0, 1.0, 128, dtype=np.float32)
    X[1, 128:] = 0.0                              # an all-zero group: q = 0, XS = 0, XA = 0
    X[2, 5] = -3.0                                # lone max: q = -127 exactly
    Q, XS, XA = orc.quant_q8(X)
    assert (Q[0] == 0).all() and (XS[0] == 0).all() and (XA[0] == 0).all()
    assert Q[1, 0] == -127 and Q[1, 127] == 127 and (Q[1, 128:] == 0).all() and XS[1, 1] == 0
    assert Q[2, 5] == -127 and XS[2, 0] == np.float32(3.0) / np.float32(127.0)
    assert np.array_equal(XA, Q.reshape(3, 2, 128).astype(np.int64).sum(2))
    assert np.abs(Q.astype(int)).max() <= 127


def test_quant_ties_round_to_even(orc):
    """q = rne(x * (127 / amax)): with amax = 127 the factor is exactly 1, so x = k + 0.5 rounds to even"""
    x = np.zeros((1, 128), np.float32)
    x[0, 0] = 127.0
    x[0, 1:9] = [0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5, 126.5]
    Q, XS, _ = orc.quant_q8(x)
    assert Q[0, :9].tolist() == [127, 0, 2, 2, 0, -2, -2, 4, 126]
    assert XS[0, 0] == 1.0


def test_quant_matches_reference_quant_q8(orc):
    """the reference's own rounding (dsv41_cpu.c quant_q8, compiled from its source): give every 32-block of a
    128-group the group's amax, so the 32-block and 128-group quantizers see the same amax and must agree"""
    if orc.ref_dsv41() is None:
        pytest.skip("oracle/_ref not built (reference sources absent)")
    r = rng(11)
    X = r.normal(0, 1, (8, 1024)).astype(np.float32)
    G = X.reshape(8, 8, 4, 32)
    amax = np.abs(X.reshape(8, 8, 128)).max(2)
    G[:, :, :, 7] = amax[:, :, None] * np.where(r.random((8, 8, 4)) < 0.5, -1, 1)
    X = G.reshape(8, 1024)
    Q, XS, XA = orc.quant_q8(X)
    for n in range(8):
        q, d = orc.ref_quant_q8(X[n])
        assert np.array_equal(q, Q[n])
    # per-row mode: every group's q follows the row amax
    Qr, XSr, XAr = orc.quant_q8(X, per_row=True)
    rmax = np.abs(X).max(1)
    assert np.all(XSr == (rmax / np.float32(127))[:, None])
    assert np.array_equal(XAr, Qr.reshape(8, 8, 128).astype(np.int64).sum(2))


def test_quant_per_row_matches_reference_on_uniform_groups(orc):
    """per-row = per-group whenever each group holds the row max"""
    X = rng(12).normal(0, 1, (4, 512)).astype(np.float32)
    m = np.abs(X).max(1, keepdims=True)
    X.reshape(4, 4, 128)[:, :, 0] = m
    assert all(np.array_equal(a, b) for a, b in zip(orc.quant_q8(X), orc.quant_q8(X, per_row=True)))


@pytest.mark.parametrize("mode", [2, 3])
def test_quant_hp_two_rows(orc, mode):
    """hp (tc.cu:195-209 mode 2; tcf.cu:150-205 mode 3): row 2n is the plain per-group row bit for bit; row 2n + 1
    stays within +-127, and together they rebuild x to within half a residual step (x - q XS - q2 XS2 is the
    residual's own rounding, about 14 bits of precision instead of 8); an all-zero group gives zeros; the two modes'
    residual scales agree to 2 ulp (amax / 254 / 127 against amax / 32258)"""
    r = rng(40 + mode)
    X = (r.standard_normal((5, 512)) * np.exp(r.normal(0, 2, (5, 1)))).astype(np.float32)
    X[3, 128:256] = 0.0
    X[4, 0] = 1e-30                                 # a tiny amax
    Q, XS, XA = orc.quant_q8(X, mode)
    Q0, XS0, XA0 = orc.quant_q8(X)
    assert Q.shape == (10, 512)
    assert np.array_equal(Q[0::2], Q0) and np.array_equal(XS[0::2], XS0) and np.array_equal(XA[0::2], XA0)
    q2 = Q[1::2].astype(np.int64)
    assert np.abs(q2).max() <= 127 and np.abs(q2).max() >= 120      # the residual row uses its range
    assert np.array_equal(XA[1::2], q2.reshape(5, 4, 128).sum(2))
    xs, xs2 = np.repeat(XS[0::2], 128, 1).astype(np.float64), np.repeat(XS[1::2], 128, 1).astype(np.float64)
    rec = Q[0::2].astype(np.float64) * xs + q2 * xs2
    err = np.abs(rec - X.astype(np.float64))
    amax = np.repeat(np.abs(X).reshape(5, 4, 128).max(2), 128, 1).astype(np.float64)
    assert (err <= 0.5 * xs2 * 1.01 + 1e-6 * amax).all()
    assert (err.max(1) < np.abs(X.astype(np.float64) - Q0.astype(np.float64) * xs).max(1) / 50).all()
    assert (Q[6, 128:256] == 0).all() and (Q[7, 128:256] == 0).all() and XS[7, 1] == 0 and XA[7, 1] == 0
    a = np.abs(X).reshape(5, 4, 128).max(2)
    other = (a / np.float32(254) / np.float32(127)) if mode == 3 else (a / np.float32(32258))
    assert np.all(np.abs(XS[1::2] - other) <= 2 * np.spacing(XS[1::2]))


def test_producers_hp(orc):
    """the producers' two-row output is their folded row xo through the mode-3 quantizer, and its even rows are the
    one-row producer's int8 row"""
    M, C, HB = 3, 4096, 1024
    r = rng(45)
    x = r.standard_normal((M, C)).astype(np.float32)
    w = (1.0 + 0.1 * r.standard_normal(C)).astype(np.float32)
    sg = np.where(r.random(C) < 0.5, -1.0, 1.0).astype(np.float32)
    for d, d1 in ((orc.rmsfold_q8(x, None, 0, w, sg, HB, hp=True), orc.rmsfold_q8(x, None, 0, w, sg, HB)),
                  (orc.fold_q8(x, sg, HB, hp=True), orc.fold_q8(x, sg, HB)),
                  (orc.smfold_q8(x, x[::-1].copy(), sg, HB, hp=True), orc.smfold_q8(x, x[::-1].copy(), sg, HB))):
        assert np.array_equal(d["xo"], d1["xo"])
        Q, XS, XA = orc.quant_q8(d["xo"], 3)
        assert np.array_equal(Q, d["Q"]) and np.array_equal(XS, d["XS"]) and np.array_equal(XA, d["XA"])
        assert np.array_equal(d["Q"][0::2], d1["Q"]) and np.array_equal(d["XS"][0::2], d1["XS"])


# ------------------------------------------------------------------------------------------- ternary products
def test_tern_acc_brute_force(orc):
    """the exact group values equal an int64 matmul of the decoded trits (sum (d - 1) q, tc_hip.cu:12-15)"""
    R, C, M = 40, 384, 3
    dig = rand_digits(R, C, 21)
    Q = rng(22).integers(-127, 128, (M, C)).astype(np.int8)
    acc = orc.tern_acc(orc.pack_from_digits(dig), R, C, Q)
    t = dig.astype(np.int64) - 1
    ref = np.einsum("rgc,mgc->mrg", t.reshape(R, 3, 128), Q.astype(np.int64).reshape(M, 3, 128))
    assert np.array_equal(acc, ref)
    # the digit form with the activation sum: sum d q - XA
    XA = Q.astype(np.int64).reshape(M, 3, 128).sum(2)
    dq = np.einsum("rgc,mgc->mrg", dig.astype(np.int64).reshape(R, 3, 128), Q.astype(np.int64).reshape(M, 3, 128))
    assert np.array_equal(acc, dq - XA[:, None, :])


def test_tern_extremes(orc):
    """|v| <= 128 * 127: all +1 against all 127 (and -1 against -127)"""
    R, C = 2, 128
    dig = np.full((R, C), 2, np.uint8)
    dig[1] = 0
    Q = np.full((1, C), 127, np.int8)
    acc = orc.tern_acc(orc.pack_from_digits(dig), R, C, Q)
    assert acc[0, :, 0].tolist() == [16256, -16256]


def test_tern_out_float64(orc):
    """the fp32 output agrees with the float64 value of sum_g v XS d"""
    R, C, M = 64, 1024, 2
    dig = rand_digits(R, C, 31)
    dpm = rand_scales((C // 128, R), 32)
    X = rng(33).normal(0, 1, (M, C)).astype(np.float32)
    Y, acc, (Q, XS, XA) = orc.tern_linear(orc.pack_from_digits(dig), dpm, R, C, X)
    d = dpm.view(np.float16).astype(np.float64)                     # [G, R]
    ref = np.einsum("mrg,mg,gr->mr", acc.astype(np.float64), XS.astype(np.float64), d)
    assert np.allclose(Y, ref, rtol=1e-5, atol=1e-6 * np.abs(ref).max())
    # and the dequantized-activation product it approximates
    W = (dig.astype(np.float64) - 1) * np.repeat(d.T, 128, axis=1)
    deq = Q.astype(np.float64) * np.repeat(XS, 128, axis=1)
    assert np.allclose(Y, deq @ W.T, rtol=1e-5, atol=1e-5 * np.abs(ref).max())


def test_tern_out_rs(orc):
    """the per-row prefill order: float64 value, agreement with the reference order on per-row inputs, and a
    hand-computed case where the chain order shows (fp32 rounding of each step)"""
    R, C, M = 48, 768, 3
    dig = rand_digits(R, C, 41)
    dpm = rand_scales((C // 128, R), 42)
    X = rng(43).normal(0, 1, (M, C)).astype(np.float32)
    bc = orc.pack_from_digits(dig)
    Q, XS, XA = orc.quant_q8(X, per_row=True)
    assert np.all(XS == XS[:, :1])                                   # per-row: one scale a token
    acc = orc.tern_acc(bc, R, C, Q)
    Y = orc.tern_out_rs(acc, XS, dpm, R, C)
    d = dpm.view(np.float16).astype(np.float64)
    ref = np.einsum("mrg,mg,gr->mr", acc.astype(np.float64), XS.astype(np.float64), d)
    assert np.allclose(Y, ref, rtol=2e-6, atol=1e-6 * np.abs(ref).max())
    Yseq = orc.tern_out(acc, XS, dpm, R, C)
    assert np.allclose(Y, Yseq, rtol=1e-5, atol=1e-6 * np.abs(ref).max())
    # hand case where the order shows: v = (2^24, 1, 1), d = 1, XS = 0.5. In group order the chain rounds 2^24 + 1
    # back to 2^24 twice (ties to even), so Y = 2^23; the float64 value (and the reverse order) is 2^23 + 1
    acc1 = np.array([[[2 ** 24, 1, 1]]], np.int32)
    XS1 = np.full((1, 3), 0.5, np.float32)
    one = orc.f2h(1.0)
    assert orc.tern_out_rs(acc1, XS1, np.full((3, 1), one, np.uint16), 1, 384)[0, 0] == 2.0 ** 23
    # and XS multiplies the sum, not each term: v = (3), d = 1, XS = 1/3 gives fp32(3 * fp32(1/3)) = 1
    third = np.float32(1.0) / np.float32(3.0)
    assert orc.tern_out_rs(np.array([[[3]]], np.int32), np.array([[third]], np.float32),
                           np.full((1, 1), one, np.uint16), 1, 128)[0, 0] == np.float32(3.0) * third


def test_out_tree_cases(orc):
    """the split tree with one split and one slice is the sequential chain; other trees differ only in rounding"""
    R, C, M = 64, 2048, 2
    dig = rand_digits(R, C, 41)
    dpm = rand_scales((C // 128, R), 42)
    X = rng(43).normal(0, 1, (M, C)).astype(np.float32)
    Y, acc, (Q, XS, XA) = orc.tern_linear(orc.pack_from_digits(dig), dpm, R, C, X)
    dq = dpm.view(np.float16).astype(np.float32)
    assert np.array_equal(orc.out_tree(acc, XS, dq, 1, 1, 0), Y)
    for sp, nw in ((2, 4), (3, 4), (1, 4), (5, 1)):
        T = orc.out_tree(acc, XS, dq, sp, nw, 0)
        assert np.allclose(T, Y, rtol=1e-5, atol=1e-6 * np.abs(Y).max())
    # a hand-summed tree: 16 groups, 2 ranges x 4 slices of 2 groups
    v = acc[0, 3].astype(np.float64)
    s = (XS[0] * dq[:, 3]).astype(np.float32).astype(np.float64)

    def fma32(a, b, c):        # a * b + c rounded once: the float64 sum is exact here (|v| < 2^15, 24-bit s)
        return np.float32(a * b + np.float64(c))

    ch = [fma32(v[2 * i + 1], s[2 * i + 1], fma32(v[2 * i], s[2 * i], 0.0)) for i in range(8)]
    q0 = np.float32(np.float32(np.float32(ch[0] + ch[1]) + ch[2]) + ch[3])
    q1 = np.float32(np.float32(np.float32(ch[4] + ch[5]) + ch[6]) + ch[7])
    assert orc.out_tree(acc, XS, dq, 2, 4, 0)[0, 3] == np.float32(q0 + q1)


def test_out_lanes_tree(orc):
    """the decode order: with one lane it is the sequential chain; with 8 lanes a hand-built butterfly"""
    R, C, M = 16, 2048, 2
    dig = rand_digits(R, C, 44)
    dpm = rand_scales((C // 128, R), 45)
    X = rng(46).normal(0, 1, (M, C)).astype(np.float32)
    Y, acc, (Q, XS, XA) = orc.tern_linear(orc.pack_from_digits(dig), dpm, R, C, X)
    dq = dpm.view(np.float16).astype(np.float32)
    assert np.array_equal(orc.out_lanes(acc, XS, dq, 1, 0), Y)
    T = orc.out_lanes(acc, XS, dq, 8, 0)
    assert np.allclose(T, Y, rtol=1e-5, atol=1e-6 * np.abs(Y).max())
    v = acc[1, 5].astype(np.float64)
    s = (XS[1] * dq[:, 5]).astype(np.float32).astype(np.float64)
    lane = []
    for c in range(8):                     # 16 groups: lane c takes c and c + 8
        a = np.float32(v[c] * s[c])
        lane.append(np.float32(v[c + 8] * s[c + 8] + np.float64(a)))
    f = np.float32
    ref = f(f(f(lane[0] + lane[1]) + f(lane[2] + lane[3])) + f(f(lane[4] + lane[5]) + f(lane[6] + lane[7])))
    assert T[1, 5] == ref


def test_tern_sum_order(orc):
    P = rng(5).normal(0, 1, (2, 3, 7)).astype(np.float32)
    y = orc.tern_sum(P, 7, 2, 3)
    ref = np.float32(np.float32(P[:, 0] + P[:, 1]) + P[:, 2])
    assert np.array_equal(y, ref)


# ------------------------------------------------------------------------------------------- kcpu pair GEMV
def test_pair_gemv_matches_reference_kcpu(orc):
    """the restatement of kcpu.c's pair-table GEMV equals the reference's own gemv() (kcpu.c:116-135, compiled
    from its source) bit for bit, and both match the float64 product"""
    R, C = 256, 1024
    dig = rand_digits(R, C, 51)
    dpm = rand_scales((C // 128, R), 52)
    bc = orc.pack_from_digits(dig)
    Pc, S = orc.paircodes(bc, R, C), orc.pair_scales(dpm, R, C)
    x = rng(53).normal(0, 1, C).astype(np.float32)
    y = orc.pair_gemv(Pc, S, R, C, x)
    W = (dig.astype(np.float64) - 1) * np.repeat(dpm.view(np.float16).astype(np.float64).T, 128, axis=1)
    ref = W @ x.astype(np.float64)
    assert np.allclose(y, ref, rtol=1e-4, atol=1e-5 * np.abs(ref).max())
    if orc.ref_kcpu() is None:
        pytest.skip("oracle/_ref not built")
    assert np.array_equal(orc.ref_gemv(Pc, S, R, C, x), y)


def test_pair_gemv_equals_int_path_on_dequantized_input(orc):
    """fed the dequantized int8 activations, the fp32 table path and the int8 path agree to ~1e-6"""
    R, C = 128, 2048
    dig = rand_digits(R, C, 61)
    dpm = rand_scales((C // 128, R), 62)
    bc = orc.pack_from_digits(dig)
    X = rng(63).normal(0, 1, (1, C)).astype(np.float32)
    Y, acc, (Q, XS, XA) = orc.tern_linear(bc, dpm, R, C, X)
    xhat = (Q[0].astype(np.float32) * np.repeat(XS[0], 128)).astype(np.float32)
    y = orc.pair_gemv(orc.paircodes(bc, R, C), orc.pair_scales(dpm, R, C), R, C, xhat)
    assert np.allclose(y, Y[0], rtol=1e-4, atol=2e-6 * np.abs(Y).max())


# ------------------------------------------------------------------------------------------- q8_0
def q8_case(R, C, seed):
    r = rng(seed)
    codes = r.integers(-127, 128, (R, C)).astype(np.int8)
    sc = np.exp(r.normal(-6, 0.5, (R, C // 32))).astype(np.float16).view(np.uint16)
    return codes, sc


def test_q8_quant_matches_reference(orc):
    """llama.cpp's CPU q8_0 rounding as the reference's dsv41_cpu.c quant_q8 implements it, bit for bit"""
    x = rng(71).normal(0, 1, (6, 2688)).astype(np.float32)
    x[2, :32] = 0.0
    x[3, 64:96] = 0.5                                   # amax = 0.5 throughout a block
    q, d = orc.q8_quant(x)
    assert (q[2, :32] == 0).all() and d[2, 0] == 0
    if orc.ref_dsv41() is None:
        pytest.skip("oracle/_ref not built")
    for n in range(6):
        rq, rd = orc.ref_quant_q8(x[n])
        assert np.array_equal(rq, q[n]) and np.array_equal(rd, d[n])


def test_q8_acc_and_out(orc):
    R, C, M = 48, 640, 3
    codes, sc = q8_case(R, C, 72)
    rows = orc.q8_0_rows(codes, sc)
    x = rng(73).normal(0, 1, (M, C)).astype(np.float32)
    q, d = orc.q8_quant(x)
    acc = orc.q8_acc(rows, R, C, q)
    ref = np.einsum("rbc,mbc->mrb", codes.astype(np.int64).reshape(R, -1, 32), q.astype(np.int64).reshape(M, -1, 32))
    assert np.array_equal(acc, ref)
    Y = orc.q8_out(acc, rows, R, C, d)
    w = sc.view(np.float16).astype(np.float64)
    yref = np.einsum("mrb,rb,mb->mr", acc.astype(np.float64), w, d.astype(np.float64))
    assert np.allclose(Y, yref, rtol=1e-5, atol=1e-6 * np.abs(yref).max())
    # the canonical chain is the split tree with one split and one slice (q8_0 form)
    assert np.array_equal(orc.out_tree(acc, d, np.ascontiguousarray(w.astype(np.float32).T), 1, 1, 1), Y)
    # the AVX2 baseline and the reference's k_q8g agree with it to rounding
    for n in range(M):
        ya = orc.q8_gemv_avx2(rows, R, C, q[n], d[n])
        assert np.allclose(ya, Y[n], rtol=1e-5, atol=1e-6 * np.abs(Y).max())
        if orc.ref_dsv41() is not None:
            yk = orc.ref_k_q8g(orc.q8_0_group4(rows, R, C), R, C, q[n], d[n])
            assert np.allclose(yk, Y[n], rtol=1e-5, atol=1e-6 * np.abs(Y).max())


# ------------------------------------------------------------------------------------------- MoE
def test_moe_sort_invariants(orc):
    M, k, E = 37, 6, 128
    r = rng(81)
    ids = np.stack([r.choice(E, k, replace=False) for _ in range(M)]).astype(np.int32)
    cnt, off, xrow, where = orc.moe_sort(ids, E)
    assert cnt.sum() == M * k and np.array_equal(cnt, np.bincount(ids.ravel(), minlength=E))
    assert np.array_equal(off, np.concatenate([[0], np.cumsum(cnt)[:-1]]))
    assert sorted(where.tolist()) == list(range(M * k))            # a permutation
    for i in range(M * k):
        e, p = ids.ravel()[i], where[i]
        assert off[e] <= p < off[e] + cnt[e] and xrow[p] == i // k
    for e in range(E):                                               # stable: ascending flat index inside a range
        seg = [i for i in range(M * k) if ids.ravel()[i] == e]
        assert [where[i] for i in seg] == list(range(off[e], off[e] + cnt[e]))


def test_moe_combine_brute_force(orc):
    M, k, cols = 5, 6, 33
    r = rng(82)
    where = r.permutation(M * k).astype(np.int32)
    gw = r.random((M, k)).astype(np.float32)
    yd = r.normal(0, 1, (M * k, cols)).astype(np.float32)
    ysh = r.normal(0, 1, (M, cols)).astype(np.float32)
    x = r.normal(0, 1, (M, cols)).astype(np.float32)
    out = orc.moe_combine(yd, ysh, where, gw, x)
    ref = x.astype(np.float64) + np.einsum("mj,mjc->mc", gw.astype(np.float64),
                                           yd[where.reshape(M, k)].astype(np.float64)) + ysh
    assert np.allclose(out, ref, rtol=1e-5, atol=1e-6)


def test_router_softmax_topk(orc):
    """against a float64 softmax over all E, top-k by probability, renormalized"""
    M, E, k = 50, 128, 6
    lg = rng(83).normal(0, 1, (M, E)).astype(np.float32)
    ids, gw = orc.router_topk(lg, k)
    p = np.exp(lg.astype(np.float64) - lg.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    top = np.argsort(-p, axis=1, kind="stable")[:, :k]
    assert np.array_equal(ids, top)
    sel = np.take_along_axis(p, top, 1)
    assert np.allclose(gw, sel / sel.sum(1, keepdims=True), rtol=1e-6)
    # ties go to the lower expert index
    t = np.zeros((1, 8), np.float32)
    t[0, [5, 2, 6]] = 1.0
    ids, gw = orc.router_topk(t, 2)
    assert ids.tolist() == [[2, 5]] and np.allclose(gw, 0.5)


def test_router_sigmoid_bias(orc):
    """Kindi's Lightning router (lt_topk, lightning.cu:373-412) against a float64 restatement: sigmoid, bias added
    for the choice only, the k largest choices, weights = chosen scores / their sum * scale"""
    M, E, k, scale = 64, 128, 6, 2.5
    lg = rng(84).normal(0, 1, (M, E)).astype(np.float32)
    bias = rng(85).normal(0, 0.3, E).astype(np.float32)
    ids, gw = orc.router_sig(lg, bias, scale, k)
    s = 1.0 / (1.0 + np.exp(-lg.astype(np.float64)))
    ch = s + bias
    top = np.argsort(-ch, axis=1, kind="stable")[:, :k]
    assert np.array_equal(ids, top)
    sel = np.take_along_axis(s, top, 1)
    assert np.allclose(gw, sel / sel.sum(1, keepdims=True) * scale, rtol=1e-6)
    assert np.allclose(gw.sum(1), scale, rtol=1e-6)
    # the bias moves the choice but not the weight: a large bias on expert 3 makes it the first pick of every token,
    # weighted by its own score
    b2 = np.zeros(E, np.float32)
    b2[3] = 10.0
    ids, gw = orc.router_sig(lg, b2, 1.0, k)
    assert (ids[:, 0] == 3).all()
    s3 = 1.0 / (1.0 + np.exp(-lg[:, 3].astype(np.float64)))
    assert np.allclose(gw[:, 0], s3 / np.take_along_axis(s, ids, 1).sum(1), rtol=1e-6)
    # ties (equal logits, zero bias) go to the lower index; softmax and sigmoid agree on the choice with zero bias
    t = np.zeros((1, 8), np.float32)
    t[0, [5, 2, 6]] = 1.0
    ids, gw = orc.router_sig(t, np.zeros(8, np.float32), 1.0, 2)
    assert ids.tolist() == [[2, 5]] and np.allclose(gw, 0.5)
    ids2, _ = orc.router_topk(lg, k)
    ids3, _ = orc.router_sig(lg, np.zeros(E, np.float32), 1.0, k)
    assert np.array_equal(ids2, ids3)


def test_router_nan_ranks_last(orc):
    """a NaN logit ranks below every number; with fewer numbers than k the NaN entries follow, lowest index first, so
    the picks stay distinct"""
    lg = np.full((1, 16), np.nan, np.float32)
    lg[0, [9, 4]] = [-3.0, 1.0]
    ids, gw = orc.router_topk(lg, 4)
    assert ids.tolist() == [[4, 9, 0, 1]]
    ids, gw = orc.router_sig(lg, np.zeros(16, np.float32), 1.0, 4)
    assert ids.tolist() == [[4, 9, 0, 1]]


# ------------------------------------------------------------------------------------------- fused producers
def hadamard(n):
    """Sylvester's Hadamard matrix H[i, j] = (-1)^popcount(i & j) (float64)"""
    i = np.arange(n)
    bits = np.bitwise_and.outer(i, i)
    pc = np.zeros_like(bits)
    while bits.any():
        pc += bits & 1
        bits >>= 1
    return np.where(pc & 1, -1.0, 1.0)


@pytest.mark.parametrize("HB", [512, 1024, 4096])
def test_fwht_blocks_is_the_normalised_hadamard(orc, HB):
    """the in-place butterflies give H v / sqrt(HB) per block (natural order), and the transform is its own inverse"""
    C = 2 * HB
    v = rng(HB).standard_normal(C).astype(np.float32)
    out = orc.fwht_blocks(v, HB)
    H = hadamard(HB)
    want = np.concatenate([H @ v[b:b + HB].astype(np.float64) for b in range(0, C, HB)]) / np.sqrt(HB)
    assert np.abs(out - want).max() < 2e-5 * np.abs(want).max()
    back = orc.fwht_blocks(out, HB)
    assert np.abs(back - v).max() < 1e-5 * np.abs(v).max()
    # a unit vector at column HB + 3 becomes the block's row 3 of H (+-1 / sqrt(HB)), the first block stays zero
    e = np.zeros(C, np.float32)
    e[HB + 3] = 1.0
    o = orc.fwht_blocks(e, HB)
    assert not o[:HB].any()
    assert np.array_equal(o[HB:], (H[3] * np.float32(1.0 / np.sqrt(HB))).astype(np.float32))


def test_sumsq_covers_every_column_exactly(orc):
    """integer columns: the double sum is exact whatever the order, so it must equal sum e^2 (no dropped index)"""
    for C in (512, 2048, 5120, 8192):
        x = np.arange(C, dtype=np.float32)
        assert orc.sumsq(x) == float(sum(int(e) * int(e) for e in range(C)))
    x = rng(5).standard_normal(5120).astype(np.float32)
    import math
    assert abs(orc.sumsq(x) - math.fsum(float(v) * float(v) for v in x)) < 1e-12 * orc.sumsq(x)


def test_rmsfold_closed_forms(orc):
    """xw = x + parts in part order; xn = x / sqrt(mean x^2 + 1e-6) * w (float64); xo = fold(sg * xn); the int8 row
    is the pinned quantizer of xo"""
    M, C, HB, np_ = 3, 5120, 1024, 3
    r = rng(11)
    x = r.standard_normal((M, C)).astype(np.float32)
    parts = (r.standard_normal((M, np_, C)) * 1e3).astype(np.float32)
    parts[:, 1] = -parts[:, 0] + r.standard_normal((M, C)).astype(np.float32) * 1e-3   # order-revealing
    w = (1.0 + 0.1 * r.standard_normal(C)).astype(np.float32)
    sg = np.where(r.random(C) < 0.5, -1.0, 1.0).astype(np.float32)
    d = orc.rmsfold_q8(x, parts.reshape(M, -1), np_, w, sg, HB)
    rv = parts[:, 0].copy()
    for p in range(1, np_):
        rv = (rv + parts[:, p]).astype(np.float32)
    xf = (x + rv).astype(np.float32)
    assert np.array_equal(d["xw"], xf)
    alt = (x + (parts[:, 0] + (parts[:, 1] + parts[:, 2]).astype(np.float32))).astype(np.float32)
    assert not np.array_equal(alt, xf)                  # the case does tell the two orders apart
    x64 = xf.astype(np.float64)
    want = x64 / np.sqrt((x64 * x64).mean(1, keepdims=True) + 1e-6) * w
    assert np.abs(d["xn"] - want).max() < 2e-6 * np.abs(want).max()
    for n in range(M):
        assert np.array_equal(d["xo"][n], orc.fwht_blocks(sg * d["xn"][n], HB))
    Q, XS, XA = orc.quant_q8(d["xo"])
    assert np.array_equal(Q, d["Q"]) and np.array_equal(XS, d["XS"]) and np.array_equal(XA, d["XA"])
    # without parts: the same row from x alone
    d0 = orc.rmsfold_q8(xf, None, 0, w, sg, HB)
    assert np.array_equal(d0["xo"], d["xo"]) and d0["xw"] is None


def test_fold_and_smfold_closed_forms(orc):
    M, C, HB = 2, 4096, 4096
    r = rng(12)
    x = r.standard_normal((M, C)).astype(np.float32)
    sg = np.where(r.random(C) < 0.5, -1.0, 1.0).astype(np.float32)
    H = hadamard(HB) / np.sqrt(HB)
    d = orc.fold_q8(x, sg, HB)
    want = (sg * x).astype(np.float64) @ H.T
    assert np.abs(d["xo"] - want).max() < 2e-5 * np.abs(want).max()
    # SiLU(a) * b under the grouped-head order: output (k, rep, h) <- source (rep, k, h)
    hd, nk, rep = 128, 4, 8
    a = r.standard_normal((M, C)).astype(np.float32) * 3
    b = r.standard_normal((M, C)).astype(np.float32)
    src = np.arange(C).reshape(rep, nk, hd).transpose(1, 0, 2).reshape(-1)
    assert all(orc.lib().or_perm_src(e, hd, nk, rep) == src[e] for e in range(0, C, 7))
    d = orc.smfold_q8(a, b, sg, HB, (hd, nk, rep))
    a64, b64 = a.astype(np.float64)[:, src], b.astype(np.float64)[:, src]
    m = a64 / (1.0 + np.exp(-a64)) * b64
    want = (sg * m) @ H.T
    assert np.abs(d["xo"] - want).max() < 2e-5 * np.abs(want).max()
    Q, XS, XA = orc.quant_q8(d["xo"])
    assert np.array_equal(Q, d["Q"]) and np.array_equal(XA, d["XA"])

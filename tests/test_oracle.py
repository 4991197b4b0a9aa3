"""Pins the CPU oracle (oracle/nnr_oracle.c) before it is trusted as the
parity checker. Each test checks the oracle against something it does not
share code with: brute-force integer arithmetic in numpy, exact rational
arithmetic (fractions), the ONNX specification's published examples, or
hand-derived known answers that separate the reference's formula variants
(RNE vs roundf, zero point before vs after rounding, fma vs mul+add,
multiply-by-reciprocal vs divide)."""
from fractions import Fraction

import numpy as np
import pytest

from oracle import pyoracle as O


def f32(v):
    return np.float32(v)


def rne_f32(fr: Fraction) -> np.float32:
    """Round an exact rational to the nearest binary32 (ties to even)."""
    x = np.float32(float(fr))          # correctly rounded to f64 then f32: fix by search
    cands = [np.nextafter(x, np.float32(-np.inf)), x, np.nextafter(x, np.float32(np.inf))]
    best = min(cands, key=lambda c: (abs(Fraction(float(c)) - fr),
                                     int(np.array(c).view(np.uint32)) & 1))
    return np.float32(best)


def exact_fma(a, b, c):
    return rne_f32(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c)))


def rne_int(fr: Fraction) -> int:
    fl = fr.numerator // fr.denominator
    rem = fr - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        return fl + 1
    return fl


# --------------------------------------------------------------------------
# integer accumulators: brute force in int64


def brute_conv(x_nchw, w, x_zp, w_zp_oc, stride, dil, pads, group):
    N, C, H, W = x_nchw.shape
    OC, Cg, kH, kW = w.shape
    oH = (H + pads[0] + pads[2] - ((kH - 1) * dil[0] + 1)) // stride[0] + 1
    oW = (W + pads[1] + pads[3] - ((kW - 1) * dil[1] + 1)) // stride[1] + 1
    xp = np.full((N, C, H + pads[0] + pads[2], W + pads[1] + pads[3]), x_zp, np.int64)
    xp[:, :, pads[0]:pads[0] + H, pads[1]:pads[1] + W] = x_nchw
    xp -= x_zp
    out = np.zeros((N, OC, oH, oW), np.int64)
    OCg = OC // group
    for oc in range(OC):
        g = oc // OCg
        wk = w[oc].astype(np.int64) - w_zp_oc[oc]
        for a in range(kH):
            for b in range(kW):
                patch = xp[:, g * Cg:(g + 1) * Cg,
                           a * dil[0]: a * dil[0] + (oH - 1) * stride[0] + 1: stride[0],
                           b * dil[1]: b * dil[1] + (oW - 1) * stride[1] + 1: stride[1]]
                out[:, oc] += np.einsum("nchw,c->nhw", patch, wk[:, a, b])
    return out


CONV_CASES = [
    # N C H W OC k group stride dil pads  w_zp
    (2, 8, 7, 6, 5, 3, 1, (1, 1), (1, 1), (1, 1, 1, 1), ()),
    (1, 6, 9, 9, 6, 3, 6, (2, 2), (1, 1), (1, 1, 1, 1), (3,)),
    (2, 4, 8, 8, 8, 3, 2, (1, 2), (2, 1), (2, 0, 1, 2), ()),
    (1, 3, 11, 10, 16, 7, 1, (2, 2), (1, 1), (3, 3, 3, 3), ()),
    (1, 5, 5, 5, 4, 1, 1, (1, 1), (1, 1), (0, 0, 0, 0), (-7, 2, 0, 5)),
]


@pytest.mark.parametrize("case", CONV_CASES)
@pytest.mark.parametrize("x_nhwc", [0, 1])
def test_conv_acc_bruteforce(case, x_nhwc):
    N, C, H, W, OC, k, G, st, dl, pads, wzp = case
    rng = np.random.default_rng(7)
    x = rng.integers(0, 256, (N, C, H, W), dtype=np.uint8)
    w = rng.integers(-128, 128, (OC, C // G, k, k), dtype=np.int8)
    cv = O.Conv(N, C, H, W, OC, k, k, group=G, stride=st, dil=dl, pads=pads, x_nhwc=x_nhwc,
                x_zp=131, w_zp=np.array(wzp, np.int8) if wzp else ())
    br = cv.dispatch()
    # the VNNI branches read w_zp through the activation type (uint8)
    raw = np.array(wzp if wzp else [0], np.int64)
    if br != O.BR["FLOAT"]:
        raw = raw.astype(np.int8).astype(np.uint8).astype(np.int64)
    zp_oc = np.broadcast_to(raw, (OC,)) if raw.size == 1 else raw
    xin = x.transpose(0, 2, 3, 1).copy() if x_nhwc else x
    acc = cv.acc(xin, w)
    ref = brute_conv(x.astype(np.int64), w, 131, zp_oc, st, dl, pads, G)
    assert np.array_equal(acc.astype(np.int64), ref)


def test_matmul_integer_bruteforce():
    rng = np.random.default_rng(3)
    for (ad, bd, at, bt) in [((5, 7), (7, 3), np.uint8, np.int8),
                             ((2, 4, 9), (9, 6), np.int8, np.uint8),
                             ((3, 1, 4, 5), (2, 5, 2), np.uint8, np.uint8),
                             ((6,), (6, 4), np.int8, np.int8)]:
        a = rng.integers(np.iinfo(at).min, np.iinfo(at).max + 1, ad, dtype=at)
        b = rng.integers(np.iinfo(bt).min, np.iinfo(bt).max + 1, bd, dtype=bt)
        y = O.matmul_integer(a, b, 12, -5)
        ref = np.matmul(a.astype(np.int64) - 12, b.astype(np.int64) + 5)
        assert np.array_equal(y.reshape(ref.shape), ref)


# --------------------------------------------------------------------------
# requantize known answers


def test_rq_b_rne_vs_roundf():
    L = O.lib()
    # os = 0.5: acc 1 -> 0.5, 5 -> 2.5: RNE gives 0 / 2, roundf gives 1 / 3
    assert L.orc_rq_b(1, 0, 0.5, 0, 0, 255) == 0
    assert L.orc_rq_b_roundf(1, 0, 0.5, 0, 0, 255) == 1
    assert L.orc_rq_b(5, 0, 0.5, 0, 0, 255) == 2
    assert L.orc_rq_b_roundf(5, 0, 0.5, 0, 0, 255) == 3
    # bias is added in int32 before scaling, zero point after rounding
    assert L.orc_rq_b(3, 2, 0.5, 127, 0, 255) == 127 + 2      # 2.5 -> 2
    # saturation at both ends and the [lo-zp, hi-zp] clamp
    assert L.orc_rq_b(10**6, 0, 1.0, 10, 0, 255) == 255
    assert L.orc_rq_b(-10**6, 0, 1.0, 10, 0, 255) == 0
    # int32 wrap of acc + bias
    assert L.orc_rq_b(2**31 - 1, 1, 1e-9, 0, 0, 255) == 0        # wraps to -2^31 -> -2.1 -> 0


def test_rq_d_zero_point_before_rounding():
    L = O.lib()
    # RQ-D adds y_zp before rounding: 0.5 + 127 = 127.5 -> 128 (RNE)
    assert L.orc_rq_d(1, 0.5, 127, 0, 255) == 128
    # RQ-B adds it after: rne(0.5) + 127 = 127
    assert L.orc_rq_b(1, 0, 0.5, 127, 0, 255) == 127
    assert L.orc_rq_d(1, 0.5, 128, 0, 255) == 128               # 128.5 -> 128
    assert L.orc_rq_d(-3, 1.0, -126, -128, 127) == -128


def test_rq_a_clamp_floor_and_tail():
    L = O.lib()
    # L = qmin (fused Relu with y_zp 10) vs lo
    assert L.orc_rq_a(-100, 1.0, 0.0, 1.0, 10, 10, 255) == 10
    assert L.orc_rq_a(-100, 1.0, 0.0, 1.0, 10, 0, 255) == 0
    assert L.orc_rq_a_tail(-100, 1.0, 0.0, 1.0, 10, 10, 255) == 10
    # RQ-C: y_zp inside the second fma, clamp before rounding
    assert L.orc_rq_c(5, 0.5, 0.0, 1.0, 3, 0, 255) == 6        # 2.5 + 3 = 5.5 -> 6
    assert L.orc_rq_a(5, 0.5, 0.0, 1.0, 3, 0, 255) == 5        # rne(2.5) + 3 = 5


def test_rq_a_single_rounding_fma():
    """RQ-A rounds acc*cs+bf once; RQ-A' (uncontracted) twice. Find inputs
    where that changes the output and check both against exact arithmetic."""
    L = O.lib()
    rng = np.random.default_rng(11)
    found = 0
    for _ in range(20000):
        acc = int(rng.integers(-2**20, 2**20))
        cs = f32(rng.uniform(1e-4, 1e-2))
        bf = f32(rng.uniform(-5, 5))
        inv = f32(1.0) / f32(rng.uniform(0.01, 0.1))
        fm = exact_fma(f32(acc), cs, bf)
        two = f32(f32(f32(acc) * cs) + bf)
        q1 = rne_int(Fraction(float(f32(fm * inv))))
        q2 = rne_int(Fraction(float(f32(two * inv))))
        exp_a = int(np.clip(q1 + 7, 0, 255))
        assert L.orc_rq_a(acc, cs, bf, inv, 7, 0, 255) == exp_a
        assert L.orc_rq_a_tail(acc, cs, bf, inv, 7, 0, 255) == int(np.clip(q2 + 7, 0, 255))
        if q1 != q2:
            found += 1
    assert found > 0


# --------------------------------------------------------------------------
# Quantize / Dequantize / DynamicQuantize


def _div_mul_disagree(rng):
    """x, s with rne(x*fl(1/s)) != rne(x/s)."""
    while True:
        s = f32(rng.uniform(0.003, 0.2))
        k = int(rng.integers(-100, 100))
        x = f32((k + 0.5) * float(s))
        for cand in (x, np.nextafter(x, f32(np.inf)), np.nextafter(x, f32(-np.inf))):
            a = rne_int(Fraction(float(f32(cand * (f32(1.0) / s)))))
            b = rne_int(Fraction(float(f32(cand / s))))
            if a != b and 0 <= a + 100 <= 255 and 0 <= b + 100 <= 255:
                return cand, s, a, b


def test_quantize_body_vs_tail():
    rng = np.random.default_rng(5)
    x0, s, q_mul, q_div = _div_mul_disagree(rng)
    for n in (40, 64, 70, 4096 + 21):
        x = np.full(n, x0, np.float32)
        y = O.quantize_linear(x, s, 100).astype(int)
        if n < 64:
            assert (y == q_div + 100).all()
        else:
            body = n - n % 16
            assert (y[:body] == q_mul + 100).all()
            assert (y[body:] == q_div + 100).all()


def test_quantize_saturation_int8():
    y = O.quantize_linear(np.array([-1e6, 1e6, 0.26, -0.26] * 20, np.float32), 0.1, -3, np.int8)
    assert list(y[:4]) == [-128, 127, 0, -6]


def test_dequantize_exact():
    q = np.arange(256, dtype=np.uint8)
    y = O.dequantize_linear(q, 0.37, 129)
    assert np.array_equal(y, ((q.astype(np.float32) - np.float32(129)) * np.float32(0.37)))


# ONNX operator documentation examples (DynamicQuantizeLinear)
DQL_SPEC = [
    ([0, 2, -3, -2.5, 1.34, 0.5], [153, 255, 0, 26, 221, 179], 0.0196078438, 153),
    ([-1.0, -2.1, -1.3, -2.5, -3.34, -4.0], [191, 121, 172, 96, 42, 0], 0.0156862754, 255),
    ([1, 2.1, 1.3, 2.5, 3.34, 4.0, 1.5, 2.6, 3.9, 4.0, 3.0, 2.345],
     [64, 134, 83, 159, 213, 255, 96, 166, 249, 255, 191, 149], 0.0156862754, 0),
]


@pytest.mark.parametrize("x,y,s,z", DQL_SPEC)
def test_dynamic_quantize_spec(x, y, s, z):
    yy, ss, zz = O.dynamic_quantize_linear(np.array(x, np.float32))
    assert list(yy) == y and zz == z
    assert abs(ss - s) < 1e-9


def test_dynamic_quantize_formula():
    rng = np.random.default_rng(2)
    x = rng.normal(0, 3, 1000).astype(np.float32)
    y, s, z = O.dynamic_quantize_linear(x)
    mn, mx = min(0.0, float(x.min())), max(0.0, float(x.max()))
    assert s == f32(f32(mx - mn) / f32(255.0))
    for v, q in zip(x[:200], y[:200]):
        assert q == np.clip(rne_int(Fraction(float(f32(v / f32(s))))) + z, 0, 255)


# --------------------------------------------------------------------------
# QLinearMatMul

def test_qlinear_matmul_spec_example():
    a = np.array([[208, 236, 0, 238], [3, 214, 255, 29]], np.uint8)
    b = np.array([[152, 51, 244], [60, 26, 255], [0, 127, 246], [127, 254, 247]], np.uint8)
    y = O.qlinear_matmul(a, 0.0066, 113, b, 0.00705, 114, 0.0107, 118)
    assert y.tolist() == [[168, 115, 255], [1, 66, 151]]


def test_qlinear_matmul_exact_against_rationals():
    rng = np.random.default_rng(9)
    a = rng.integers(0, 256, (3, 17), dtype=np.uint8)
    b = rng.integers(-127, 128, (17, 5), dtype=np.int8)
    y = O.qlinear_matmul(a, 0.02, 128, b, 0.005, 0, 0.05, 128)
    acc = (a.astype(np.int64) - 128) @ b.astype(np.int64)
    cm = f32(f32(f32(0.02) * f32(0.005)) / f32(0.05))
    for i in range(3):
        for j in range(5):
            v = f32(f32(f32(acc[i, j]) * cm) + f32(128))
            assert y[i, j] == np.clip(rne_int(Fraction(float(v))), 0, 255)


def test_f16_conversion_matches_numpy():
    rng = np.random.default_rng(4)
    vals = np.concatenate([rng.uniform(-70000, 70000, 3000), rng.uniform(-1, 1, 3000),
                           rng.uniform(-1e-4, 1e-4, 3000)]).astype(np.float32)
    L = O.lib()
    for v in vals:
        if abs(v) < 2.0 ** -24:       # the reference flushes below 2^-24 (nnrconf.h:172)
            continue
        h = L.orc_f32_to_f16(float(v))
        with np.errstate(over="ignore"):
            ref = np.float16(v)
        assert h == int(np.array(ref).view(np.uint16)), v
        assert L.orc_f16_to_f32(h) == np.float32(ref)


def test_combined_scale_fp16():
    cm = O.qmatmul_combined_scale(0.1, 0.2, 0.3, np.float16)
    h = np.float16(np.float32(np.float16(np.float32(np.float16(0.1)) * np.float32(np.float16(0.2))))
                   / np.float32(np.float16(0.3)))
    assert cm == np.float32(h)


# --------------------------------------------------------------------------
# QLinearAdd

def test_qlinear_add_identity_scales():
    rng = np.random.default_rng(1)
    a = rng.integers(0, 256, 1000, dtype=np.uint8)
    b = rng.integers(0, 256, 1000, dtype=np.uint8)
    y = O.qlinear_add(0, a, b, 0.1, 0, 0.1, 0, 0.1, 0)
    assert np.array_equal(y, np.clip(a.astype(int) + b, 0, 255).astype(np.uint8))


def test_qlinear_add_same_shape_exact():
    rng = np.random.default_rng(8)
    n = 16 * 10 + 7
    a = rng.integers(0, 256, n, dtype=np.uint8)
    b = rng.integers(0, 256, n, dtype=np.uint8)
    a_s, b_s, y_s = f32(0.031), f32(0.017), f32(0.043)
    y = O.qlinear_add(0, a, b, a_s, 117, b_s, 131, y_s, 3)
    sa, sb = f32(a_s / y_s), f32(b_s / y_s)
    fixed = f32(f32(3) - f32(f32(sa * f32(117)) + f32(sb * f32(131))))
    body = n - n % 16
    for i in range(n):
        if i < body:
            v = exact_fma(f32(a[i]), sa, exact_fma(f32(b[i]), sb, fixed))
        else:
            v = f32(f32(f32(sa * f32(int(a[i]) - 117)) + f32(sb * f32(int(b[i]) - 131))) + f32(3))
        assert y[i] == np.clip(rne_int(Fraction(float(v))), 0, 255)


# --------------------------------------------------------------------------
# MaxPool

def test_maxpool_bruteforce():
    rng = np.random.default_rng(6)
    x = rng.integers(0, 256, (2, 9, 10, 5), dtype=np.uint8)
    y = O.maxpool_u8_nhwc(x, 3, 3, 2, 2, 1, 1, 5, 5)
    for n in range(2):
        for oh in range(5):
            for ow in range(5):
                h0, w0 = oh * 2 - 1, ow * 2 - 1
                win = x[n, max(0, h0):h0 + 3, max(0, w0):w0 + 3]
                assert np.array_equal(y[n, oh, ow], win.reshape(-1, 5).max(0))


# --------------------------------------------------------------------------
# QLinearConv: dispatch table and closed forms


def _w(OC, Cg, k):
    return np.zeros((OC, Cg, k, k), np.int8)


@pytest.mark.parametrize("kw,expect", [
    # cfg2: 3x3 s1 p1, IC/OC 64, NHWC out -> NR16 direct
    (dict(N=32, C=64, H=56, W=56, OC=64, k=3, pads=(1, 1, 1, 1), y_nhwc=1), "NR16"),
    # ResNet stem 7x7 s2 IC3, NCHW in -> first layer
    (dict(N=1, C=3, H=224, W=224, OC=64, k=7, stride=(2, 2), pads=(3, 3, 3, 3), y_nhwc=1), "FIRST"),
    # 1x1 / strided 3x3 -> packed NR48
    (dict(N=1, C=256, H=56, W=56, OC=64, k=1, y_nhwc=1), "PACKED"),
    (dict(N=1, C=128, H=56, W=56, OC=128, k=3, stride=(2, 2), pads=(1, 1, 1, 1), y_nhwc=1), "PACKED"),
    # small spatial with NCHW output -> direct
    (dict(N=1, C=64, H=14, W=14, OC=64, k=3, pads=(1, 1, 1, 1), y_nhwc=0), "DIRECT"),
    # same with NHWC output -> NR16
    (dict(N=1, C=64, H=14, W=14, OC=64, k=3, pads=(1, 1, 1, 1), y_nhwc=1), "NR16"),
    # depthwise NHWC -> DW; depthwise NCHW out -> im2col
    (dict(N=1, C=32, H=8, W=8, OC=32, k=3, group=32, pads=(1, 1, 1, 1), y_nhwc=1), "DW"),
    (dict(N=1, C=32, H=8, W=8, OC=32, k=3, group=32, pads=(1, 1, 1, 1), y_nhwc=0), "IM2COL_S1"),
    (dict(N=1, C=32, H=8, W=8, OC=32, k=3, group=32, stride=(2, 2), pads=(1, 1, 1, 1)), "IM2COL"),
    # grouped conv
    (dict(N=1, C=8, H=8, W=8, OC=8, k=3, group=2, pads=(1, 1, 1, 1)), "IM2COL_S1"),
    # int8 activations / per-channel w_zp -> float fallback
    (dict(N=1, C=8, H=8, W=8, OC=8, k=3, act_dtype=np.int8, x_zp=0), "FLOAT"),
    (dict(N=1, C=8, H=8, W=8, OC=4, k=1, w_zp=(1, 2, 3, 4)), "FLOAT"),
    # all-equal per-channel zp collapses to per-tensor
    (dict(N=1, C=8, H=8, W=8, OC=4, k=1, w_zp=(2, 2, 2, 2), y_nhwc=1), "PACKED"),
])
def test_conv_dispatch_table(kw, expect):
    kw = dict(kw)
    k = kw.pop("k")
    args = [kw.pop(n) for n in ("N", "C", "H", "W", "OC")]
    cv = O.Conv(*args[:5], k, k, **kw)
    assert cv.dispatch() == O.BR[expect]


@pytest.mark.parametrize("y_nhwc", [0, 1])
def test_conv_unit_scale_closed_form(y_nhwc):
    """scales 1 and zero points 0: every branch reduces to clamp(acc + bias)."""
    rng = np.random.default_rng(12)
    x = rng.integers(0, 4, (1, 8, 6, 6), dtype=np.uint8)
    w = rng.integers(-3, 4, (16, 8, 3, 3), dtype=np.int8)
    bias = rng.integers(-20, 20, 16).astype(np.int32)
    cv = O.Conv(1, 8, 6, 6, 16, 3, 3, pads=(1, 1, 1, 1), y_nhwc=y_nhwc, x_scale=1.0, x_zp=0,
                w_scale=[1.0], y_scale=1.0, y_zp=0, bias=bias)
    y, br = cv.run(x, w)
    ref = brute_conv(x.astype(np.int64), w, 0, np.zeros(16, np.int64), (1, 1), (1, 1),
                     (1, 1, 1, 1), 1) + bias[None, :, None, None]
    ref = np.clip(ref, 0, 255)
    if y_nhwc:
        ref = ref.transpose(0, 2, 3, 1)
    assert np.array_equal(y.astype(np.int64), ref)


def test_conv_branch_formulas_from_acc():
    """Each branch applies its own formula to the same accumulators."""
    rng = np.random.default_rng(13)
    N, C, H, W, OC = 1, 64, 4, 5, 48 + 40      # OC % 48 = 40 > 32: RQ-B' columns exist
    cv = O.Conv(N, C, H, W, OC, 1, 1, y_nhwc=1, x_scale=0.013, x_zp=120,
                w_scale=rng.uniform(0.001, 0.01, OC).astype(np.float32), y_scale=0.031, y_zp=5,
                bias=rng.integers(-4096, 4096, OC))
    assert cv.dispatch() == O.BR["PACKED"]
    acc = rng.integers(-200000, 200000, (N, OC, H, W)).astype(np.int32)
    y, br = cv.from_acc(acc)
    L = O.lib()
    cs = (np.float32(0.013) * cv.w_scale).astype(np.float32)
    os_ = (cs * (np.float32(1) / np.float32(0.031))).astype(np.float32)
    for oc in range(OC):
        for h in range(H):
            for w_ in range(W):
                a = int(acc[0, oc, h, w_])
                v = a + int(cv.bias[oc])
                f = f32(f32(v) * os_[oc])
                f = min(max(f, f32(-5)), f32(250))
                if oc >= 48 + 32:     # third sub-panel of the partial block: roundf
                    q = int(np.sign(f) * np.floor(abs(float(f)) + 0.5)) + 5
                else:
                    q = rne_int(Fraction(float(f))) + 5
                assert y[0, h, w_, oc] == np.clip(q, 0, 255)
    # the roundf columns really differ somewhere from an RNE epilogue
    assert L.orc_rq_b_roundf(5, 0, 0.5, 0, 0, 255) != L.orc_rq_b(5, 0, 0.5, 0, 0, 255)


# ---------------------------------------------------------------------------
# QLinearConv on 3-D tensors (exec_typed, RQ-S)

def _conv1d_acc_via_2d(N, C, W, OC, k, group, stride, dil, pads, x, w, x_zp, w_zp, act):
    """accumulators of the independently written 2-D oracle on the H = 1 view"""
    cv = O.Conv(N, C, 1, W, OC, 1, k, group=group, stride=(1, stride), dil=(1, dil),
                pads=(0, pads[0], 0, pads[1]), act_dtype=act, x_zp=x_zp, w_zp=w_zp)
    return cv.acc(x[:, :, None, :], w[:, :, None, :])[:, :, 0, :]


@pytest.mark.parametrize("act", [np.int8, np.uint8])
@pytest.mark.parametrize("case", [(2, 8, 23, 12, 3, 1, 1, 1, (1, 1)), (1, 12, 40, 6, 5, 3, 2, 2, (4, 3)),
                                  (3, 4, 9, 4, 3, 4, 1, 1, (2, 0))])
def test_conv1d_acc_matches_2d_oracle(case, act):
    """With scale 1 / zero point 0 the RQ-S output is clamp(acc), so the 1-D
    path's accumulation (taps, padding, stride, dilation, groups) is pinned by
    the 2-D oracle's. uint8 activations use non-negative weights and w_zp so
    the reference's weight-through-T read does not change them."""
    N, C, W, OC, k, group, stride, dil, pads = case
    rng = np.random.default_rng(sum(case[:5]))
    lo, hi = (-128, 128) if act == np.int8 else (0, 256)
    x = rng.integers(lo, hi, (N, C, W), dtype=act)
    wl = -20 if act == np.int8 else 0
    w = rng.integers(wl, 21, (OC, C // group, k), dtype=np.int8)
    x_zp = 3 if act == np.int8 else 131
    acc = _conv1d_acc_via_2d(N, C, W, OC, k, group, stride, dil, pads, x, w, x_zp, (2,), act)
    cv = O.Conv1d(N, C, W, OC, k, group=group, stride=stride, dil=dil, pads=pads, act_dtype=act,
                  x_scale=1.0, x_zp=x_zp, w_scale=(1.0,), w_zp=(2,), y_scale=1.0, y_zp=0)
    y, br = cv.run(x, w)
    assert br == 9
    info = np.iinfo(act)
    assert np.array_equal(y.astype(np.int64), np.clip(acc, info.min, info.max))


def test_conv1d_rounding_and_division():
    """RQ-S known answers: ties go to even (nearbyint, not roundf), and the
    division by y_scale is not a multiplication by fl(1/y_scale): a case
    where the two round to different integers is searched and checked."""
    # one input channel, kernel 1: acc = (x - x_zp) * w
    def run(xv, wv, y_scale, y_zp=0, act=np.int8):
        cv = O.Conv1d(1, 1, 1, 1, 1, act_dtype=act, x_scale=1.0, x_zp=0, w_scale=(1.0,),
                      y_scale=y_scale, y_zp=y_zp)
        y, _ = cv.run(np.array([[[xv]]], act), np.array([[[wv]]], np.int8))
        return int(y.reshape(-1)[0])
    assert run(5, 1, 2.0) == 2 and run(7, 1, 2.0) == 4 and run(-3, 1, 2.0) == -2
    assert run(-5, 1, 2.0, y_zp=9) == 7
    # acc = -80 * 113 = -9040 and y_scale = fl(128.22694): acc / s is exactly
    # -70.5 (a tie, rounds to -70) while acc * fl(1/s) = -70.5000076 (rounds
    # to -71), so this pins the division of RQ-S against RQ-A's reciprocal
    s = np.float32(128.22694)
    assert np.float32(-9040) / s == np.float32(-70.5)
    assert np.rint(np.float32(-9040) * (np.float32(1) / s)) == -71
    assert run(-80, 113, float(s)) == -70


def test_conv1d_weights_read_through_activation_type():
    """exec_typed reads the int8 weights through the uint8 activation type
    (QLinearConv.cpp:206, `const T* pw = (const T*)w->data`): a weight byte of
    -1 counts as 255, and w_zp -2 as 254."""
    def run(x, w, w_zp, act):
        cv = O.Conv1d(1, 1, 1, 1, 1, act_dtype=act, x_scale=1.0, x_zp=0, w_scale=(1.0,),
                      w_zp=(w_zp,), y_scale=1.0, y_zp=0)
        y, _ = cv.run(np.array([[[x]]], act), np.array([[[w]]], np.int8))
        return int(y.reshape(-1)[0])
    assert run(1, -1, 0, np.uint8) == 255          # 1 * (255 - 0)
    assert run(1, -1, -2, np.uint8) == 1            # 1 * (255 - 254)
    assert run(1, -1, 0, np.int8) == -1             # int8 activations: the weight stays -1


# ---------------------------------------------------------------------------
# the rest of the QLinear family: closed forms that fix the structure (the
# golden fixtures, an exact-rational restatement, fix the roundings)

def test_qgap_constant_image_is_its_value():
    """Power-of-two scales, spatial 16: sum*rs is exact, so a constant image
    pools to its own value; a zero-point offset shifts it by the same."""
    for v in (0, 7, 128, 255):
        x = np.full((2, 3, 4, 4), v, np.uint8)
        assert np.array_equal(O.qlinear_global_avgpool(x, 0.25, 10, 0.25, 10), np.full((2, 3), v))
        assert np.array_equal(O.qlinear_global_avgpool(x, 0.25, 10, 0.25, 0), np.full((2, 3), max(v - 10, 0)))
    x = np.arange(16, dtype=np.uint8).reshape(1, 1, 4, 4)
    # mean 7.5 -> nearbyint ties to even: 8
    assert O.qlinear_global_avgpool(x, 1.0, 0, 1.0, 0)[0, 0] == 8
    # NHWC input gives the same sums
    xn = np.random.default_rng(3).integers(0, 256, (2, 5, 6, 7), dtype=np.uint8)
    assert np.array_equal(O.qlinear_global_avgpool(xn, 0.03, 9, 0.02, 4, nhwc=1),
                          O.qlinear_global_avgpool(xn.transpose(0, 3, 1, 2), 0.03, 9, 0.02, 4))


def test_qavgpool_identity_and_padding_count():
    rng = np.random.default_rng(4)
    x = rng.integers(0, 256, (2, 3, 5, 6), dtype=np.uint8)
    # 1x1 window, stride 1, equal power-of-two scales and zero points: identity
    assert np.array_equal(O.qlinear_avgpool(x, (1, 1), (1, 1), (0, 0), 5, 6, 0.5, 9, 0.5, 9), x)
    # a 3x3 window at a corner averages only the in-image taps (count_include_pad 0)
    c = np.full((1, 1, 3, 3), 0, np.uint8)
    c[0, 0, 0, 0], c[0, 0, 0, 1], c[0, 0, 1, 0], c[0, 0, 1, 1] = 4, 8, 12, 16
    y = O.qlinear_avgpool(c, (3, 3), (1, 1), (1, 1), 3, 3, 1.0, 0, 1.0, 0)
    assert y[0, 0, 0, 0] == 10   # (4 + 8 + 12 + 16) / 4
    # NHWC equals NCHW
    xn = x.transpose(0, 2, 3, 1).copy()
    a = O.qlinear_avgpool(x, (3, 3), (2, 2), (1, 1), 3, 3, 0.02, 7, 0.03, 5)
    b = O.qlinear_avgpool(xn, (3, 3), (2, 2), (1, 1), 3, 3, 0.02, 7, 0.03, 5, nhwc=1)
    assert np.array_equal(a, b.transpose(0, 3, 1, 2))


def test_qconcat_copy_and_identity():
    rng = np.random.default_rng(5)
    xs = [rng.integers(0, 256, 4 * c, dtype=np.uint8) for c in (3, 17, 32)]
    cat = np.concatenate([x.reshape(4, -1) for x in xs], 1).reshape(-1)
    # matching scale and zero point: a copy
    y = O.qlinear_concat(xs, [3, 17, 32], 4, [0.1] * 3, [5] * 3, 0.1, 5)
    assert np.array_equal(y, cat)
    # scale ratio 1 with another zero point: x - zp + y_zp, clamped, in body and tail
    y = O.qlinear_concat(xs, [3, 17, 32], 4, [0.25] * 3, [10] * 3, 0.25, 0)
    assert np.array_equal(y, np.clip(cat.astype(int) - 10, 0, 255))


def test_qmul_identity_and_kinds():
    rng = np.random.default_rng(6)
    a = rng.integers(0, 256, 100, dtype=np.uint8)
    one = np.full(100, 65, np.uint8)    # b - b_zp = 1
    # cs = 0.5 * 2 / 1 = 1: y = a exactly, in the 16-wide body and in the tail
    assert np.array_equal(O.qlinear_mul(0, a, one, 0.5, 0, 2.0, 64, 1.0, 0), a)
    # scalar B equals the same-shape result when cs * (b - zp) is exact
    b1 = np.array([66], np.uint8)
    y_sc = O.qlinear_mul(1, a, b1, 0.5, 7, 1.0, 64, 1.0, 3)
    y_full = O.qlinear_mul(0, a, np.full(100, 66, np.uint8), 0.5, 7, 1.0, 64, 1.0, 3)
    assert np.array_equal(y_sc, y_full)
    # per channel, NCHW and NHWC, agree on exact products
    x = rng.integers(0, 256, (2, 4, 3, 5), dtype=np.uint8)
    ch = rng.integers(60, 70, 4, dtype=np.uint8)
    n1 = O.qlinear_mul(3, x, ch, 0.25, 0, 1.0, 64, 1.0, 0, C=4, HW=15, y_nhwc=0)
    n2 = O.qlinear_mul(3, x.transpose(0, 2, 3, 1).copy(), ch, 0.25, 0, 1.0, 64, 1.0, 0, C=4, HW=15, y_nhwc=1)
    assert np.array_equal(n1, n2.transpose(0, 3, 1, 2))
    ref = np.clip(np.rint(x.astype(np.float64) * 0.25 * (ch.astype(np.float64) - 64)[None, :, None, None]), 0, 255)
    assert np.array_equal(n1, ref)


# ---------------------------------------------------------------------------
# fold_bn_qdq and the folded BatchNormalization (fold_bn_qdq.cpp:138-147,
# BatchNormalization.cpp:248-376)

def test_fold_bn_identity():
    """scale 1, bias 0, mean 0, var + eps = 1 and equal DQ / Q parameters
    (power-of-two scale) give A = 1, B = 0 exactly: y = x in every layout."""
    C = 40
    one, zero = np.ones(C, np.float32), np.zeros(C, np.float32)
    A, B = O.fold_bn(one, zero, zero, one, 0.0, 0.03125, 7, dq=(0.03125, 7))
    assert np.all(A == 1.0) and np.all(B == 0.0)
    x = np.random.default_rng(1).integers(0, 256, (2, C, 5, 7), dtype=np.uint8)
    for nhwc in (0, 1):
        xi = x.transpose(0, 2, 3, 1).copy() if nhwc else x
        assert np.array_equal(O.batchnorm_u8(xi, A, B, nhwc=nhwc), xi)


def test_fold_bn_formula():
    """A and B against the algebra in float64 (a dropped or misplaced term
    moves them by far more than float rounding)."""
    rng = np.random.default_rng(2)
    C = 33
    sc, bias, mean = rng.uniform(0.5, 2, C), rng.normal(0, 1, C), rng.normal(0, 1, C)
    var = rng.uniform(0.1, 3, C)
    eps, dq_s, dq_zp, q_s, q_zp = 1e-3, 0.021, 131, 0.047, 9
    A, B = O.fold_bn(sc, bias, mean, var, eps, q_s, q_zp, dq=(dq_s, dq_zp))
    g = sc / np.sqrt(var + eps)
    beta = bias - g * mean
    np.testing.assert_allclose(A, dq_s * g / q_s, rtol=1e-5)
    np.testing.assert_allclose(B, (beta - dq_zp * dq_s * g) / q_s + q_zp, rtol=1e-4, atol=1e-4)
    A2, B2 = O.fold_bn(sc, bias, mean, var, eps, q_s, q_zp)
    np.testing.assert_allclose(A2, g / q_s, rtol=1e-5)
    np.testing.assert_allclose(B2, beta / q_s + q_zp, rtol=1e-4, atol=1e-4)


def test_folded_bn_rounding_per_layout():
    """x + 0.5 exactly (A = 1, B = 0.5): nearest even in the 16-wide bodies and
    the NHWC tail (lrintf), away from zero in the NCHW tail (roundf)."""
    C, H, W = 20, 1, 18       # NHWC: 16 body + 4 tail channels; NCHW: 16 body + 2 tail pixels
    x = (np.arange(2 * C * H * W) % 250).astype(np.uint8).reshape(2, C, H, W)
    A, B = np.ones(C, np.float32), np.full(C, 0.5, np.float32)
    rne = lambda v: (v + (v & 1)).astype(np.uint8)          # (v + 0.5) to even
    y = O.batchnorm_u8(x, A, B, nhwc=0)
    assert np.array_equal(y[..., :16], rne(x[..., :16].astype(np.int32)))
    assert np.array_equal(y[..., 16:], (x[..., 16:].astype(np.int32) + 1).astype(np.uint8))
    xn = x.transpose(0, 2, 3, 1).copy()
    yn = O.batchnorm_u8(xn, A, B, nhwc=1)
    assert np.array_equal(yn, rne(xn.astype(np.int32)))


def test_folded_bn_negative_saturation():
    """A negative result: 0 everywhere except the NHWC 16-wide body with
    uint8 input, whose unsigned saturation (cvtusepi32_epi8 of a negative
    int32) gives 255."""
    C = 20
    x = np.random.default_rng(3).integers(0, 200, (1, C, 2, 3), dtype=np.uint8)
    A, B = np.ones(C, np.float32), np.full(C, -300.0, np.float32)
    assert np.all(O.batchnorm_u8(x, A, B, nhwc=0) == 0)
    yn = O.batchnorm_u8(x.transpose(0, 2, 3, 1).copy(), A, B, nhwc=1)
    assert np.all(yn[..., :16] == 255) and np.all(yn[..., 16:] == 0)
    xf = x.transpose(0, 2, 3, 1).astype(np.float32).copy()
    assert np.all(O.batchnorm_u8(xf, A, B, nhwc=1) == 0)     # fp32 input: clamped first


# ---------------------------------------------------------------------------
# ConvInteger (ConvInteger.cpp:146-354)

def _conv_int_numpy(x, w, x_zp, w_zp, s, p, d, group):
    """int64 brute force over zero-padded (x - x_zp) windows."""
    N, C, H, W = x.shape
    OC, CC, kH, kW = w.shape
    xs = np.pad(x.astype(np.int64) - x_zp, ((0, 0), (0, 0), (p[0], p[0]), (p[1], p[1])))
    ws = w.astype(np.int64) - np.broadcast_to(np.asarray(w_zp, np.int64).reshape(-1), (OC,))[:, None, None, None]
    oH = (H + 2 * p[0] - ((kH - 1) * d[0] + 1)) // s[0] + 1
    oW = (W + 2 * p[1] - ((kW - 1) * d[1] + 1)) // s[1] + 1
    y = np.zeros((N, OC, oH, oW), np.int64)
    MM = OC // group
    for oc in range(OC):
        g = oc // MM
        for kh in range(kH):
            for kw in range(kW):
                win = xs[:, g * CC:(g + 1) * CC, kh * d[0]: kh * d[0] + s[0] * (oH - 1) + 1: s[0],
                         kw * d[1]: kw * d[1] + s[1] * (oW - 1) + 1: s[1]]
                y[:, oc] += np.einsum("nchw,c->nhw", win, ws[oc, :, kh, kw])
    return y.astype(np.int32)


@pytest.mark.parametrize("xdt,wdt,per_ch,s,p,d,group", [
    (np.uint8, np.int8, False, (1, 1), (1, 1), (1, 1), 1),
    (np.uint8, np.uint8, True, (2, 1), (0, 2), (1, 2), 2),
    (np.int8, np.int8, True, (1, 2), (2, 1), (2, 1), 4)])
def test_conv_integer_matches_brute_force(xdt, wdt, per_ch, s, p, d, group):
    rng = np.random.default_rng(7)
    info = lambda t: (0, 256) if t == np.uint8 else (-128, 128)
    x = rng.integers(*info(xdt), (2, 8, 9, 11), dtype=xdt)
    w = rng.integers(*info(wdt), (12, 8 // group, 3, 3), dtype=wdt)
    x_zp = 131 if xdt == np.uint8 else -3
    w_zp = rng.integers(*info(wdt), 12) if per_ch else (7 if wdt == np.uint8 else -2)
    y = O.conv_integer(x, w, x_zp, w_zp, s, p, d, group)
    assert np.array_equal(y, _conv_int_numpy(x, w, x_zp, w_zp, s, p, d, group))


def test_conv_integer_1x1_is_matmul_integer():
    """A 1x1 ConvInteger is MatMulInteger of the weights with the pixels."""
    rng = np.random.default_rng(8)
    x = rng.integers(0, 256, (1, 16, 5, 6), dtype=np.uint8)
    w = rng.integers(-128, 128, (10, 16, 1, 1), dtype=np.int8)
    y = O.conv_integer(x, w, 100, -4)
    mm = O.matmul_integer(w.reshape(10, 16), x.reshape(16, 30), -4, 100)
    assert np.array_equal(y.reshape(10, 30), mm)


def test_folded_bn_half_below_zero():
    """The NHWC uint8 body rounds before it saturates: -0.5 is -0 -> 0, but
    -0.51 is -1 -> 255."""
    C = 16
    x = np.zeros((1, 2, 2, C), np.uint8)
    A = np.ones(C, np.float32)
    assert np.all(O.batchnorm_u8(x, A, np.full(C, -0.5, np.float32), nhwc=1) == 0)
    assert np.all(O.batchnorm_u8(x, A, np.full(C, -0.51, np.float32), nhwc=1) == 255)


# ---------------------------------------------------------------------------
# HardSwish, fp32 (HardSwish.cpp:18-50, vec_ops_avx512.h:74-117)

def _hs_exact(x, body):
    """HardSwish by exact rational arithmetic, one RNE rounding per IEEE
    operation: body fl(fl(x * fl(1/6)) + 1/2), tail fl(fl(x / 6) + 1/2), each
    clamped to [0, 1], times x."""
    X = Fraction(float(x))
    if body:
        u = rne_f32(Fraction(float(rne_f32(X * Fraction(float(rne_f32(Fraction(1, 6))))))) + Fraction(1, 2))
    else:
        u = rne_f32(Fraction(float(rne_f32(X / 6))) + Fraction(1, 2))
    t = min(max(Fraction(float(u)), Fraction(0)), Fraction(1))
    return rne_f32(X * t)


def test_hardswish_closed_forms():
    """x >= 3 passes through, x <= -3 gives (negative) zero, 0 stays 0, at
    body (first n - n % 16) and tail positions alike; NaN and -inf give NaN
    (-inf * 0), +inf stays +inf."""
    vals = np.array([3, 4.5, 100, 1e30, -3, -4, -1e30, 0.0, np.inf, -np.inf, np.nan], np.float32)
    x = np.concatenate([vals, np.zeros(16 - len(vals) % 16, np.float32), vals])   # body copy, tail copy
    y = O.hardswish(x)
    n_t = len(vals)
    for part in (y[:n_t], y[-n_t:]):
        assert np.array_equal(part[:4], vals[:4])
        assert np.all(part[4:7] == 0) and np.all(np.signbit(part[4:7]))
        assert part[7] == 0 and part[8] == np.inf
        assert np.isnan(part[9]) and np.isnan(part[10])


def test_hardswish_matches_float64_within_ulps():
    rng = np.random.default_rng(5)
    x = rng.uniform(-4, 4, 1003).astype(np.float32)
    y = O.hardswish(x).astype(np.float64)
    x64 = x.astype(np.float64)
    ref = x64 * np.clip(x64 / 6 + 0.5, 0, 1)
    # t = x/6 + 1/2 carries an absolute error of about one ulp of 1/2 (it
    # cancels near x = -3), which x then scales
    tol = 4 * np.spacing(np.abs(ref).astype(np.float32)).astype(np.float64) + np.abs(x64) * 2.0 ** -23
    assert np.all(np.abs(y - ref) <= tol)


def test_hardswish_body_and_tail_known_answers():
    """Values where multiplying by fl(1/6) (the 16-wide body) and dividing by
    6 (the scalar tail) round differently: the oracle must give each
    position its own expression, as exact rational arithmetic does."""
    cand = np.linspace(-2.99, 2.99, 4001).astype(np.float32)
    diff = [v for v in cand if _hs_exact(v, True) != _hs_exact(v, False)]
    assert len(diff) > 5
    for v in diff[:: max(1, len(diff) // 20)]:
        x = np.full(17, v, np.float32)           # 16 body elements, 1 tail element
        y = O.hardswish(x)
        assert y[0] == _hs_exact(v, True) and y[15] == _hs_exact(v, True)
        assert y[16] == _hs_exact(v, False) and y[16] != y[0]


def test_hardswish_post_op_adds_zero_bias():
    """The fused form adds the zero bias of bias_hardswish: -0.0 becomes +0.0
    (and stays -0.0 * 0.5 = -0.0 in the standalone operator)."""
    x = np.full(20, -0.0, np.float32)
    assert np.all(np.signbit(O.hardswish(x)))
    assert not np.any(np.signbit(O.hardswish(x, post_op=True)))
    rng = np.random.default_rng(1)
    x = rng.uniform(-4, 4, 100).astype(np.float32)
    assert np.array_equal(O.hardswish(x), O.hardswish(x, post_op=True))


# ---------------------------------------------------------------------------
# the AVX-512 VNNI restatement (the CPU baseline) against the scalar loops

def _vnni_or_skip():
    if not O.vnni_available():
        pytest.skip("host has no AVX-512 VNNI")


@pytest.mark.parametrize("N,C,H,W,OC,k,s,p,d,nhwc,act,wzp", [
    (2, 64, 9, 11, 72, 3, 1, 1, 1, 1, np.uint8, 0),     # NR16-like, OC not a multiple of 48
    (1, 3, 23, 19, 16, 7, 2, 3, 1, 0, np.uint8, 0),     # first layer, NCHW input
    (2, 40, 7, 7, 50, 1, 1, 0, 1, 1, np.uint8, 0),      # 1x1, K % 4 != 0
    (1, 16, 12, 10, 24, 3, 2, 1, 2, 1, np.int8, 3),     # int8 activations, dilation, w_zp
    (3, 8, 6, 5, 96, 5, 1, 2, 1, 0, np.uint8, 250),     # w_zp read through uint8
])
def test_vnni_conv_acc_equals_scalar(N, C, H, W, OC, k, s, p, d, nhwc, act, wzp):
    _vnni_or_skip()
    rng = np.random.default_rng(N * C + H + OC)
    lo, hi = (0, 256) if act == np.uint8 else (-128, 128)
    shape = (N, H, W, C) if nhwc else (N, C, H, W)
    x = rng.integers(lo, hi, shape, dtype=act)
    w = rng.integers(-128, 128, (OC, C, k, k), dtype=np.int8)
    cv = O.Conv(N, C, H, W, OC, k, k, stride=(s, s), dil=(d, d), pads=(p, p, p, p), x_nhwc=nhwc,
                act_dtype=act, x_zp=int(rng.integers(lo, hi)), w_zp=(np.int8(np.uint8(wzp).view(np.int8)),))
    ref = cv.acc(x, w)
    try:
        O.set_vnni(True)
        got = cv.acc(x, w)
    finally:
        O.set_vnni(False)
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("C,k,s", [(32, 3, 1), (40, 3, 2), (16, 5, 1)])
def test_vnni_depthwise_acc_equals_scalar(C, k, s):
    _vnni_or_skip()
    rng = np.random.default_rng(C + k)
    N, H, W = 2, 9, 13
    x = rng.integers(0, 256, (N, H, W, C), dtype=np.uint8)
    w = rng.integers(-128, 128, (C, 1, k, k), dtype=np.int8)
    cv = O.Conv(N, C, H, W, C, k, k, group=C, stride=(s, s), pads=(k // 2,) * 4, x_nhwc=1, y_nhwc=1,
                x_zp=117, w_zp=rng.integers(-5, 5, C).astype(np.int8))
    ref = cv.acc(x, w)
    try:
        O.set_vnni(True)
        got = cv.acc(x, w)
    finally:
        O.set_vnni(False)
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("adt,bdt,azp,bzp", [(np.uint8, np.int8, 131, 0), (np.int8, np.int8, -9, 4),
                                             (np.uint8, np.uint8, 7, 200), (np.int8, np.uint8, 0, 128)])
def test_vnni_matmul_equals_scalar(adt, bdt, azp, bzp):
    _vnni_or_skip()
    rng = np.random.default_rng(abs(azp) + bzp)
    rnd = lambda dt, shape: rng.integers(0 if dt == np.uint8 else -128, 256 if dt == np.uint8 else 128, shape,
                                         dtype=dt)
    a = rnd(adt, (3, 53, 70))
    b = rnd(bdt, (70, 101))
    ref = O.matmul_integer(a, b, azp, bzp)
    try:
        O.set_vnni(True)
        got = O.matmul_integer(a, b, azp, bzp)
        q = O.qlinear_matmul(a[0], 0.02, azp, b, 0.005, bzp, 0.05, 128) if adt == np.uint8 else None
    finally:
        O.set_vnni(False)
    assert np.array_equal(got, ref)
    if q is not None:
        assert np.array_equal(q, O.qlinear_matmul(a[0], 0.02, azp, b, 0.005, bzp, 0.05, 128))


@pytest.mark.parametrize("xdt,s,p,d", [(np.uint8, 1, 1, 1), (np.int8, 2, 0, 1), (np.uint8, 1, 2, 2)])
def test_vnni_conv_integer_equals_scalar(xdt, s, p, d):
    _vnni_or_skip()
    rng = np.random.default_rng(s + 3 * p + 7 * d)
    lo, hi = (0, 256) if xdt == np.uint8 else (-128, 128)
    x = rng.integers(lo, hi, (2, 24, 11, 9), dtype=xdt)
    w = rng.integers(-128, 128, (40, 24, 3, 3), dtype=np.int8)
    wz = rng.integers(-8, 8, 40).astype(np.int32)
    xz = int(rng.integers(lo, hi))
    ref = O.conv_integer(x, w, xz, wz, (s, s), (p, p), (d, d))
    try:
        O.set_vnni(True)
        got = O.conv_integer(x, w, xz, wz, (s, s), (p, p), (d, d))
    finally:
        O.set_vnni(False)
    assert np.array_equal(got, ref)


def test_int8_compute_threads_heuristic():
    """thread_pool.h:725-737: serial below 2^20 ops, physical cores below
    phys * 2^22 ops, every logical thread above, never more than the work."""
    O.lib().orc_set_host_threads(8, 16)
    try:
        f = O.lib().orc_int8_compute_threads
        assert f(100, (1 << 20) - 1) == 1
        assert f(100, 1 << 20) == 8
        assert f(100, 8 * (1 << 22) - 1) == 8
        assert f(100, 8 * (1 << 22)) == 16
        assert f(3, 1 << 40) == 3
    finally:
        O.lib().orc_set_host_threads(0, 0)

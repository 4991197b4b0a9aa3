"""Writes the golden fixtures of this directory (tests/golden/*.npz).

NNR ships no test vectors for its int8 path and cannot be built here, so the
fixtures are computed by an independent restatement of the reference's
arithmetic that shares no code with oracle/: integer accumulators by brute
force in numpy int64, every float operation as an exact rational rounded
once to binary32 (ties to even), and each operator's expression written out
from the reference lines cited next to it. The oracle and the HIP kernels
are both checked against these files (tests/test_golden.py).

Run from the repository root:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import json
import os
from fractions import Fraction

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))

# ---------------------------------------------------------------------------
# binary32 arithmetic on exact rationals


def f32r(fr) -> float:
    """Round a rational (or float) to the nearest binary32, ties to even."""
    fr = Fraction(fr)
    x = np.float32(float(fr))
    best = None
    for c in (np.nextafter(x, np.float32(-np.inf)), x, np.nextafter(x, np.float32(np.inf))):
        key = (abs(Fraction(float(c)) - fr), int(np.array(c, np.float32).view(np.uint32)) & 1)
        if best is None or key < best[0]:
            best = (key, c)
    return float(np.float32(best[1]))


def mul(a, b):
    return f32r(Fraction(a) * Fraction(b))


def add(a, b):
    return f32r(Fraction(a) + Fraction(b))


def div(a, b):
    return f32r(Fraction(a) / Fraction(b))


def fma(a, b, c):
    return f32r(Fraction(a) * Fraction(b) + Fraction(c))


def i2f(v: int) -> float:
    return f32r(Fraction(int(v)))


def rne(x) -> int:
    """Round half to even (cvtps2dq / roundscale NEAREST / nearbyint)."""
    fr = Fraction(x)
    fl = fr.numerator // fr.denominator
    rem = fr - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        return fl + 1
    return fl


def roundf(x) -> int:
    """Half away from zero (std::roundf)."""
    fr = Fraction(x)
    a = abs(fr)
    r = (a.numerator * 2 + a.denominator) // (2 * a.denominator)
    return r if fr >= 0 else -r


def x86_int(r: int) -> int:
    """cvtps2dq / (int) of an integral float: INT_MIN when out of range."""
    return r if -2**31 <= r < 2**31 else -2**31


def clamp(v, lo, hi):
    return lo if v < lo else (hi if v > hi else v)


def wrap32(v: int) -> int:
    v &= 0xFFFFFFFF
    return v - 2**32 if v >= 2**31 else v


# ---------------------------------------------------------------------------
# requantize expressions (SURVEY notation; reference lines cited)


def rq_a(acc, cs, bf, inv_y, y_zp, L, hi):
    # QLinearConv.cpp:630-638 / :1171-1179, depthwise_int8_avx512.h:249-255:
    # fmadd, mul, roundscale, add zp, max/min, convert
    q = mul(fma(i2f(acc), cs, bf), inv_y)
    q = add(rne(q), y_zp)
    return int(clamp(q, L, hi))


def rq_a_tail(acc, cs, bf, inv_y, y_zp, L, hi):
    # QLinearConv.cpp:640-645 (scalar tail, no contraction)
    val = add(mul(i2f(acc), cs), bf)
    t = mul(val, inv_y)
    return clamp(wrap32(x86_int(rne(t)) + y_zp), L, hi)


def rq_b(acc, bias, os_, y_zp, lo, hi, use_roundf=False):
    # jit_conv_int8_ukernel.cpp:950-964 (RQ-B); gemm_int8_avx512.h:1505 (RQ-B')
    v = wrap32(acc + bias)
    f = mul(i2f(v), os_)
    f = max(f, float(lo - y_zp))
    f = min(f, float(hi - y_zp))
    if use_roundf:
        return clamp(roundf(f) + y_zp, 0, 255)
    return rne(f) + y_zp


def rq_c(acc, cs, bf, inv_y, y_zp, qmin, qmax):
    # conv_first_layer_int8_avx512.h:262-273
    t = fma(i2f(acc), cs, bf)
    f = fma(t, inv_y, float(y_zp))
    f = clamp(f, float(qmin), float(qmax))
    return rne(f)


def rq_d(acc, cm, y_zp, lo, hi):
    # QLinearMatMul.cpp:188-198 (no contraction)
    val = add(mul(i2f(acc), cm), float(y_zp))
    return clamp(x86_int(rne(val)), lo, hi)


# ---------------------------------------------------------------------------
# integer accumulators by brute force


def conv_acc(x_nchw, w, x_zp, w_zp, stride, pads, group):
    N, C, H, W = x_nchw.shape
    OC, Cg, kH, kW = w.shape
    oH = (H + pads[0] + pads[2] - kH) // stride[0] + 1
    oW = (W + pads[1] + pads[3] - kW) // stride[1] + 1
    xp = np.full((N, C, H + pads[0] + pads[2], W + pads[1] + pads[3]), x_zp, np.int64)
    xp[:, :, pads[0]:pads[0] + H, pads[1]:pads[1] + W] = x_nchw
    xp -= x_zp
    OCg = OC // group
    acc = np.zeros((N, OC, oH, oW), np.int64)
    for oc in range(OC):
        g = oc // OCg
        wk = w[oc].astype(np.int64) - w_zp
        for a in range(kH):
            for b in range(kW):
                patch = xp[:, g * Cg:(g + 1) * Cg, a:a + stride[0] * (oH - 1) + 1:stride[0],
                           b:b + stride[1] * (oW - 1) + 1:stride[1]]
                acc[:, oc] += np.einsum("nchw,c->nhw", patch, wk[:, a, b])
    return ((acc + 2**31) % 2**32 - 2**31).astype(np.int64)


# ---------------------------------------------------------------------------
# fixtures


def conv_case(name, branch, rng, N, C, H, W, OC, k, group=1, stride=(1, 1), pads=(0, 0, 0, 0),
              x_nhwc=0, y_nhwc=0, post_fn=0, x_zp=128, y_zp=0, x_scale=0.02, y_scale=0.03,
              bias=True):
    x = rng.integers(0, 256, (N, C, H, W), dtype=np.uint8)
    w = rng.integers(-127, 128, (OC, C // group, k, k), dtype=np.int8)
    w_scale = rng.uniform(0.001, 0.01, OC).astype(np.float32)
    b = rng.integers(-4096, 4097, OC).astype(np.int32) if bias else np.zeros(0, np.int32)
    acc = conv_acc(x.astype(np.int64), w, x_zp, 0, stride, pads, group)
    _, _, oH, oW = acc.shape
    lo, hi = 0, 255
    qmin = max(lo, y_zp) if post_fn else lo
    inv_y = div(1.0, float(np.float32(y_scale)))
    xs = float(np.float32(x_scale))
    cs = [mul(xs, float(w_scale[oc])) for oc in range(OC)]
    bf = [mul(i2f(int(b[oc])), cs[oc]) if bias else 0.0 for oc in range(OC)]
    os_ = [mul(cs[oc], inv_y) for oc in range(OC)]
    sp = oH * oW
    y = np.zeros((N, OC, oH, oW), np.int64)
    bprime_from = OC - OC % 48 + 32 if OC % 48 > 32 else OC
    for n in range(N):
        for oc in range(OC):
            for oh in range(oH):
                for ow in range(oW):
                    a = int(acc[n, oc, oh, ow])
                    s = oh * oW + ow
                    if branch == "DW":
                        q = rq_a(a, cs[oc], bf[oc], inv_y, y_zp, lo, hi)
                    elif branch == "FIRST":
                        if y_nhwc or ow < oW - oW % 16:
                            q = rq_c(a, cs[oc], bf[oc], inv_y, y_zp, qmin, hi)
                        else:
                            q = rq_a_tail(a, cs[oc], bf[oc], inv_y, y_zp, qmin, hi)
                    elif branch == "DIRECT":
                        if s < sp - sp % 16:
                            q = rq_a(a, cs[oc], bf[oc], inv_y, y_zp, qmin, hi)
                        else:
                            q = rq_a_tail(a, cs[oc], bf[oc], inv_y, y_zp, qmin, hi)
                    elif branch == "IM2COL_S1":
                        q = rq_a(a, cs[oc], bf[oc], inv_y, y_zp, lo, hi)
                    elif branch == "IM2COL":
                        # one tile (tile_h = oH for these sizes): tail = last sp % 16
                        if s < sp - sp % 16:
                            q = rq_a(a, cs[oc], bf[oc], inv_y, y_zp, qmin, hi)
                        else:
                            q = rq_a_tail(a, cs[oc], bf[oc], inv_y, y_zp, qmin, hi)
                    elif branch in ("PACKED", "NR16"):
                        q = rq_b(a, int(b[oc]) if bias else 0, os_[oc], y_zp, lo, hi,
                                 use_roundf=(branch == "PACKED" and oc >= bprime_from))
                    else:
                        raise ValueError(branch)
                    y[n, oc, oh, ow] = q
    y = y.astype(np.uint8)
    xin = x.transpose(0, 2, 3, 1).copy() if x_nhwc else x
    yout = y.transpose(0, 2, 3, 1).copy() if y_nhwc else y
    params = dict(op="QLinearConv", branch=branch, N=N, C=C, H=H, W=W, OC=OC, k=k, group=group,
                  stride=list(stride), pads=list(pads), x_nhwc=x_nhwc, y_nhwc=y_nhwc,
                  post_fn=post_fn, x_zp=x_zp, y_zp=y_zp, x_scale=x_scale, y_scale=y_scale,
                  bias=bool(bias))
    return name, params, dict(x=xin, w=w, w_scale=w_scale, bias=b, y=yout,
                              acc=acc.astype(np.int32))


def qmatmul_case(rng):
    # QLinearMatMul.cpp:124-135: cm = fl(fl(a_s*b_s)/y_s)
    a_s, a_zp, b_s, b_zp, y_s, y_zp = 0.02, 121, 0.0047, 0, 0.31, 128
    A = rng.integers(0, 256, (2, 5, 40), dtype=np.uint8)
    B = rng.integers(-127, 128, (40, 23), dtype=np.int8)
    acc = np.einsum("bmk,kn->bmn", A.astype(np.int64) - a_zp, B.astype(np.int64) - b_zp)
    cm = div(mul(float(np.float32(a_s)), float(np.float32(b_s))), float(np.float32(y_s)))
    y = np.vectorize(lambda v: rq_d(int(v), cm, y_zp, 0, 255))(acc).astype(np.uint8)
    params = dict(op="QLinearMatMul", a_scale=a_s, a_zp=a_zp, b_scale=b_s, b_zp=b_zp,
                  y_scale=y_s, y_zp=y_zp)
    return "qlinear_matmul", params, dict(a=A, b=B, y=y, acc=acc.astype(np.int32))


def qadd_case(rng):
    # QLinearAdd.cpp:46-47,66-67 (constants), :79-104 (16-wide body, scalar tail)
    a_s, a_zp, b_s, b_zp, y_s, y_zp = 0.041, 7, 0.023, 131, 0.06, 2
    n = 37
    a = rng.integers(0, 256, n, dtype=np.uint8)
    b = rng.integers(0, 256, n, dtype=np.uint8)
    sa = div(float(np.float32(a_s)), float(np.float32(y_s)))
    sb = div(float(np.float32(b_s)), float(np.float32(y_s)))
    fixed = add(float(y_zp), -add(mul(sa, float(a_zp)), mul(sb, float(b_zp))))
    y = np.zeros(n, np.uint8)
    body = n - n % 16
    for i in range(n):
        if i < body:
            v = fma(float(a[i]), sa, fma(float(b[i]), sb, fixed))
            y[i] = clamp(x86_int(rne(v)), 0, 255)
        else:
            t1 = mul(sa, i2f(int(a[i]) - a_zp))
            t2 = mul(sb, i2f(int(b[i]) - b_zp))
            v = add(add(t1, t2), float(y_zp))
            y[i] = clamp(x86_int(rne(v)), 0, 255)
    params = dict(op="QLinearAdd", a_scale=a_s, a_zp=a_zp, b_scale=b_s, b_zp=b_zp,
                  y_scale=y_s, y_zp=y_zp)
    return "qlinear_add", params, dict(a=a, b=b, y=y)


def quantize_case(rng):
    # QuantizeLinear.cpp:128-194: body multiplies by fl(1/s), last n%16 divide
    s, zp = 0.037, 9
    n = 100
    x = (rng.standard_normal(n) * 3).astype(np.float32)
    inv = div(1.0, float(np.float32(s)))
    body = n - n % 16
    y = np.zeros(n, np.uint8)
    for i in range(n):
        if i < body:
            q = rne(mul(float(x[i]), inv))
        else:
            q = rne(div(float(x[i]), float(np.float32(s))))
        y[i] = clamp(q + zp, 0, 255)
    return "quantize", dict(op="QuantizeLinear", scale=s, zp=zp), dict(x=x, y=y)


def dynq_case(rng):
    # DynamicQuantizeLinear.cpp:37-58
    n = 70
    x = (rng.standard_normal(n) * 2 + 0.5).astype(np.float32)
    xmin = min(0.0, float(x.min()))
    xmax = max(0.0, float(x.max()))
    s = div(add(xmax, -xmin), 255.0)
    if s == 0.0:
        s = 1.0
    zp = clamp(rne(div(-xmin, s)), 0, 255)
    y = np.array([clamp(rne(div(float(v), s)) + zp, 0, 255) for v in x], np.uint8)
    return "dynamic_quantize", dict(op="DynamicQuantizeLinear"), dict(
        x=x, y=y, y_scale=np.array([s], np.float32), y_zp=np.array([zp], np.uint8))


def qgap_case(rng):
    # QLinearGlobalAveragePool.cpp:46 (rs), :52-57 (int sum, zero-point term, RQ-F)
    N, C, H, W = 2, 5, 3, 4
    x_s, x_zp, y_s, y_zp = 0.031, 100, 0.017, 3
    x = rng.integers(0, 256, (N, C, H, W), dtype=np.uint8)
    sp = H * W
    rs = div(float(np.float32(x_s)), mul(float(np.float32(y_s)), float(sp)))
    y = np.zeros((N, C, 1, 1), np.uint8)
    for n in range(N):
        for c in range(C):
            sm = wrap32(int(x[n, c].astype(np.int64).sum()) - x_zp * sp)
            q = wrap32(x86_int(rne(mul(i2f(sm), rs))) + y_zp)
            y[n, c, 0, 0] = clamp(q, 0, 255)
    return "qlinear_global_avgpool", dict(op="QLinearGlobalAveragePool", x_scale=x_s, x_zp=x_zp,
                                          y_scale=y_s, y_zp=y_zp), dict(x=x, y=y)


def qavgpool_case(rng):
    # QLinearAveragePool.cpp:90-110: in-image taps only, fl(fl(sum * x_s) / count),
    # nearbyint(fl(avg / y_s)) + y_zp
    N, C, H, W, k, st, pd = 1, 3, 6, 7, 3, 2, 1
    x_s, x_zp, y_s, y_zp = 0.02, 128, 0.013, 128
    x = rng.integers(0, 256, (N, C, H, W), dtype=np.uint8)
    oH = (H + 2 * pd - k) // st + 1
    oW = (W + 2 * pd - k) // st + 1
    y = np.zeros((N, C, oH, oW), np.uint8)
    for c in range(C):
        for oh in range(oH):
            for ow in range(oW):
                sm, cnt = 0, 0
                for kh in range(k):
                    ih = oh * st - pd + kh
                    if not 0 <= ih < H:
                        continue
                    for kw in range(k):
                        iw = ow * st - pd + kw
                        if 0 <= iw < W:
                            sm += int(x[0, c, ih, iw]) - x_zp
                            cnt += 1
                avg = div(mul(i2f(sm), float(np.float32(x_s))), float(max(cnt, 1)))
                q = wrap32(x86_int(rne(div(avg, float(np.float32(y_s))))) + y_zp)
                y[0, c, oh, ow] = clamp(q, 0, 255)
    return "qlinear_avgpool", dict(op="QLinearAveragePool", k=k, stride=st, pad=pd, x_scale=x_s,
                                   x_zp=x_zp, y_scale=y_s, y_zp=y_zp), dict(x=x, y=y)


def qconcat_case(rng):
    # QLinearConcat.cpp:147 (copy when scale and zero point match), :84-104
    # (16-wide body fma(rs, x - zp, y_zp), clamp, rne; scalar tail)
    outer = 3
    counts = [21, 5, 16]
    scales = [0.05, 0.02, 0.031]
    zps = [10, 3, 7]
    y_s, y_zp = 0.031, 7   # the third input is copied
    xs = [rng.integers(0, 256, (outer, c), dtype=np.uint8) for c in counts]
    rows = []
    for o in range(outer):
        row = []
        for t, cnt in enumerate(counts):
            if scales[t] == y_s and zps[t] == y_zp:
                row += [int(v) for v in xs[t][o]]
                continue
            rs = div(float(np.float32(scales[t])), float(np.float32(y_s)))
            body = cnt - cnt % 16 if cnt >= 16 else 0
            for i in range(cnt):
                xv = int(xs[t][o, i])
                if i < body:
                    v = fma(rs, float(xv - zps[t]), float(y_zp))
                    v = min(max(v, 0.0), 255.0)
                    row.append(rne(v))
                else:
                    v = add(mul(rs, i2f(xv - zps[t])), float(y_zp))
                    row.append(clamp(x86_int(rne(v)), 0, 255))
        rows.append(row)
    y = np.array(rows, np.uint8)
    arrays = {f"x{t}": xs[t] for t in range(len(xs))}
    arrays["y"] = y
    return "qlinear_concat", dict(op="QLinearConcat", scales=scales, zps=zps, y_scale=y_s,
                                  y_zp=y_zp), arrays


def qmul_case(rng):
    # QLinearMul.cpp:39 (cs), :54-74 (16-wide body), :76-79 (scalar tail)
    a_s, a_zp, b_s, b_zp, y_s, y_zp = 0.043, 120, 0.029, 135, 0.052, 128
    n = 37
    a = rng.integers(0, 256, n, dtype=np.uint8)
    b = rng.integers(0, 256, n, dtype=np.uint8)
    cs = div(mul(float(np.float32(a_s)), float(np.float32(b_s))), float(np.float32(y_s)))
    body = n - n % 16
    y = np.zeros(n, np.uint8)
    for i in range(n):
        da, db = int(a[i]) - a_zp, int(b[i]) - b_zp
        if i < body:
            v = fma(mul(float(da), float(db)), cs, float(y_zp))
            y[i] = clamp(rne(v), 0, 255)
        else:
            v = add(mul(mul(cs, i2f(da)), i2f(db)), float(y_zp))
            y[i] = clamp(x86_int(rne(v)), 0, 255)
    return "qlinear_mul", dict(op="QLinearMul", a_scale=a_s, a_zp=a_zp, b_scale=b_s, b_zp=b_zp,
                               y_scale=y_s, y_zp=y_zp), dict(a=a, b=b, y=y)


def main():
    rng = np.random.default_rng(20240611)
    cases = [
        conv_case("conv_packed_bprime", "PACKED", rng, 1, 64, 3, 4, 88, 1, x_nhwc=1, y_nhwc=1,
                  x_zp=120, y_zp=5),
        conv_case("conv_nr16", "NR16", rng, 1, 64, 4, 5, 64, 3, pads=(1, 1, 1, 1), x_nhwc=1,
                  y_nhwc=1, post_fn=1, y_zp=0),
        conv_case("conv_first_nchw_tail", "FIRST", rng, 1, 3, 6, 19, 16, 3, pads=(1, 1, 1, 1),
                  post_fn=1, y_zp=4),
        conv_case("conv_direct_tail", "DIRECT", rng, 1, 16, 5, 7, 24, 3, pads=(1, 1, 1, 1),
                  y_zp=20),
        conv_case("conv_dw", "DW", rng, 1, 32, 5, 6, 32, 3, group=32, pads=(1, 1, 1, 1),
                  x_nhwc=1, y_nhwc=1, y_zp=3),
        conv_case("conv_im2col_s1", "IM2COL_S1", rng, 1, 16, 5, 5, 32, 3, group=2,
                  pads=(1, 1, 1, 1), y_zp=6),
        conv_case("conv_im2col_s2", "IM2COL", rng, 1, 16, 9, 9, 32, 3, group=2, stride=(2, 2),
                  pads=(1, 1, 1, 1), post_fn=1, y_zp=12),
        qmatmul_case(rng),
        qadd_case(rng),
        quantize_case(rng),
        dynq_case(rng),
    ]
    # the QOperator family (a separate stream, so the fixtures above stay as committed)
    rng2 = np.random.default_rng(20261201)
    cases += [qgap_case(rng2), qavgpool_case(rng2), qconcat_case(rng2), qmul_case(rng2)]
    for name, params, arrays in cases:
        path = os.path.join(HERE, name + ".npz")
        np.savez_compressed(path, params=np.array(json.dumps(params, sort_keys=True)), **arrays)
        print(f"{path}: {os.path.getsize(path)} bytes")


if __name__ == "__main__":
    main()

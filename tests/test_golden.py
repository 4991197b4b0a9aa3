"""The committed golden fixtures (tests/golden/*.npz, written by
tests/golden/make_golden.py from an independent exact-rational restatement)
against the CPU oracle and, on a GPU, against the HIP kernels."""
import glob
import json
import os

import numpy as np
import pytest

from oracle import pyoracle as O

HERE = os.path.dirname(os.path.abspath(__file__))
FILES = sorted(glob.glob(os.path.join(HERE, "golden", "*.npz")))


def load(path):
    z = np.load(path, allow_pickle=False)
    return json.loads(str(z["params"])), {k: z[k] for k in z.files if k != "params"}


def conv_kwargs(p, d):
    return dict(group=p["group"], stride=tuple(p["stride"]), pads=tuple(p["pads"]),
                x_nhwc=p["x_nhwc"], y_nhwc=p["y_nhwc"], post_fn=p["post_fn"],
                x_scale=p["x_scale"], x_zp=p["x_zp"], w_scale=d["w_scale"],
                y_scale=p["y_scale"], y_zp=p["y_zp"], bias=d["bias"] if p["bias"] else None)


def test_fixtures_present():
    names = {os.path.basename(f)[:-4] for f in FILES}
    assert {"conv_packed_bprime", "conv_nr16", "conv_first_nchw_tail", "conv_direct_tail",
            "conv_dw", "conv_im2col_s1", "conv_im2col_s2", "qlinear_matmul", "qlinear_add",
            "quantize", "dynamic_quantize", "qlinear_global_avgpool", "qlinear_avgpool",
            "qlinear_concat", "qlinear_mul"} <= names


@pytest.mark.parametrize("path", FILES, ids=[os.path.basename(f)[:-4] for f in FILES])
def test_oracle_matches_golden(path):
    p, d = load(path)
    op = p["op"]
    if op == "QLinearConv":
        cv = O.Conv(p["N"], p["C"], p["H"], p["W"], p["OC"], p["k"], p["k"], **conv_kwargs(p, d))
        assert cv.dispatch() == O.BR[p["branch"]]
        y, br = cv.run(d["x"], d["w"])
        assert br == O.BR[p["branch"]]
        assert np.array_equal(y, d["y"])
    elif op == "QLinearMatMul":
        y = O.qlinear_matmul(d["a"], p["a_scale"], p["a_zp"], d["b"], p["b_scale"], p["b_zp"],
                             p["y_scale"], p["y_zp"], np.uint8)
        assert np.array_equal(y, d["y"])
    elif op == "QLinearAdd":
        y = O.qlinear_add(0, d["a"], d["b"], p["a_scale"], p["a_zp"], p["b_scale"], p["b_zp"],
                          p["y_scale"], p["y_zp"])
        assert np.array_equal(y, d["y"])
    elif op == "QuantizeLinear":
        y = O.quantize_linear(d["x"], p["scale"], p["zp"], np.uint8)
        assert np.array_equal(y, d["y"])
    elif op == "QLinearGlobalAveragePool":
        y = O.qlinear_global_avgpool(d["x"], p["x_scale"], p["x_zp"], p["y_scale"], p["y_zp"])
        assert np.array_equal(y.reshape(d["y"].shape), d["y"])
    elif op == "QLinearAveragePool":
        k, st, pd = p["k"], p["stride"], p["pad"]
        oH, oW = d["y"].shape[2:]
        y = O.qlinear_avgpool(d["x"], (k, k), (st, st), (pd, pd), oH, oW, p["x_scale"], p["x_zp"],
                              p["y_scale"], p["y_zp"])
        assert np.array_equal(y, d["y"])
    elif op == "QLinearConcat":
        xs = [d[f"x{t}"] for t in range(len(p["scales"]))]
        outer = xs[0].shape[0]
        y = O.qlinear_concat([x.reshape(-1) for x in xs], [x.shape[1] for x in xs], outer, p["scales"],
                             p["zps"], p["y_scale"], p["y_zp"])
        assert np.array_equal(y.reshape(d["y"].shape), d["y"])
    elif op == "QLinearMul":
        y = O.qlinear_mul(0, d["a"], d["b"], p["a_scale"], p["a_zp"], p["b_scale"], p["b_zp"],
                          p["y_scale"], p["y_zp"])
        assert np.array_equal(y, d["y"])
    elif op == "DynamicQuantizeLinear":
        y, s, z = O.dynamic_quantize_linear(d["x"])
        assert np.float32(s) == d["y_scale"][0] and int(z) == int(d["y_zp"][0])
        assert np.array_equal(y, d["y"])
    else:
        raise AssertionError(op)


@pytest.mark.gpu
@pytest.mark.parametrize("path", FILES, ids=[os.path.basename(f)[:-4] for f in FILES])
def test_hip_matches_golden(dev, path):
    import torch

    import nnr_amd as H
    p, d = load(path)
    op = p["op"]
    to = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    if op == "QLinearConv":
        kw = conv_kwargs(p, d)
        qc = H.QLinearConv(p["N"], p["C"], p["H"], p["W"], d["w"], **kw)
        assert H.BRANCH_NAMES[qc.branch] == p["branch"]
        y = qc(to(d["x"])).cpu().numpy()
    elif op == "QLinearMatMul":
        a = d["a"]
        mm = H.QLinearMatMul(d["b"], p["a_scale"], p["a_zp"], p["b_scale"], p["b_zp"],
                             p["y_scale"], p["y_zp"], m=a.shape[1])
        y = mm(to(a)).cpu().numpy()
    elif op == "QLinearAdd":
        y = H.qlinear_add(0, to(d["a"]), to(d["b"]), p["a_scale"], p["a_zp"], p["b_scale"],
                          p["b_zp"], p["y_scale"], p["y_zp"]).cpu().numpy()
    elif op == "QuantizeLinear":
        y = H.quantize_linear(to(d["x"]), p["scale"], p["zp"], np.uint8).cpu().numpy()
    elif op == "QLinearGlobalAveragePool":
        y = H.qlinear_global_avgpool(to(d["x"]), p["x_scale"], p["x_zp"], p["y_scale"],
                                     p["y_zp"]).cpu().numpy().reshape(d["y"].shape)
    elif op == "QLinearAveragePool":
        k, st, pd = p["k"], p["stride"], p["pad"]
        oH, oW = d["y"].shape[2:]
        y = H.qlinear_avgpool(to(d["x"]), (k, k), (st, st), (pd, pd), oH, oW, p["x_scale"], p["x_zp"],
                              p["y_scale"], p["y_zp"]).cpu().numpy()
    elif op == "QLinearConcat":
        xs = [d[f"x{t}"] for t in range(len(p["scales"]))]
        y = H.qlinear_concat([to(x.reshape(-1)) for x in xs], [x.shape[1] for x in xs], xs[0].shape[0],
                             p["scales"], p["zps"], p["y_scale"], p["y_zp"]).cpu().numpy().reshape(d["y"].shape)
    elif op == "QLinearMul":
        y = H.qlinear_mul(0, to(d["a"]), to(d["b"]), p["a_scale"], p["a_zp"], p["b_scale"],
                          p["b_zp"], p["y_scale"], p["y_zp"]).cpu().numpy()
    elif op == "DynamicQuantizeLinear":
        yt, s, z = H.dynamic_quantize_linear(to(d["x"]))
        assert np.float32(s.cpu().numpy().reshape(-1)[0]) == d["y_scale"][0]
        assert int(z.cpu().numpy().reshape(-1)[0]) == int(d["y_zp"][0])
        y = yt.cpu().numpy()
    else:
        raise AssertionError(op)
    assert np.array_equal(y, d["y"]), f"{np.count_nonzero(y != d['y'])} of {y.size} differ"

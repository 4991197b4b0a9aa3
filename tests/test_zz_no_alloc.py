"""DynamicQuantizeLinear through the entry point that allocates nothing
(nnrh_dynamic_quantize_linear_noalloc), against the workspace entry point
(nnrh_dynamic_quantize_linear) and the oracle, through the C ABI.

Two calls in a row on one stream, the second on a smaller input whose range
is far narrower than the first's: the library's scratch array still holds
the first call's 1024 (min, max) partials, and reading any stale one would
change the second call's scale."""
import ctypes as C

import numpy as np
import pytest

from nnr_amd import _lib
from oracle import pyoracle as O

pytestmark = pytest.mark.gpu


def _dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _outs(n, dev):
    import torch
    return (torch.empty(n, dtype=torch.uint8, device=dev),
            torch.empty(1, dtype=torch.float32, device=dev),
            torch.empty(1, dtype=torch.uint8, device=dev))


def test_dynamic_quantize_noalloc_matches_workspace_entry(dev):
    import torch
    L = _lib.lib()
    stream = torch.cuda.current_stream().cuda_stream
    rng = np.random.default_rng(7)
    n1, n2 = 3_000_017, 1_001
    x1 = (rng.normal(0, 40.0, n1) - 3.0).astype(np.float32)
    x2 = (rng.normal(0, 0.5, n2) + 0.2).astype(np.float32)
    xs = [_dev(x1, dev), _dev(x2, dev)]
    ws = torch.empty(int(L.nnrh_dynamic_quantize_workspace()), dtype=torch.uint8, device=dev)
    got = [_outs(n1, dev), _outs(n2, dev)]
    want = [_outs(n1, dev), _outs(n2, dev)]
    torch.cuda.synchronize()
    # the two no-allocation calls back to back, then the workspace entry point
    for x, (y, s, z) in zip(xs, got):
        print(f"noalloc call n={x.numel()}", flush=True)
        _lib.check(L.nnrh_dynamic_quantize_linear_noalloc(x.data_ptr(), x.numel(), y.data_ptr(),
                                                          s.data_ptr(), z.data_ptr(), stream))
    for x, (y, s, z) in zip(xs, want):
        _lib.check(L.nnrh_dynamic_quantize_linear(x.data_ptr(), x.numel(), y.data_ptr(), s.data_ptr(),
                                                  z.data_ptr(), ws.data_ptr(), stream))
    torch.cuda.synchronize()
    for xh, g, w in zip((x1, x2), got, want):
        y_ref, s_ref, z_ref = O.dynamic_quantize_linear(xh)
        gy, gs, gz = (t.cpu().numpy() for t in g)
        wy, wsc, wz = (t.cpu().numpy() for t in w)
        assert gs[0] == wsc[0] == np.float32(s_ref)
        assert int(gz[0]) == int(wz[0]) == z_ref
        assert np.array_equal(gy, wy) and np.array_equal(gy, y_ref)


def test_dynamic_quantize_noalloc_rejects_oversize(dev):
    import torch
    L = _lib.lib()
    y, s, z = _outs(16, dev)
    x = torch.zeros(16, dtype=torch.float32, device=dev)
    too_many = (1 << 40) + 1
    rc = L.nnrh_dynamic_quantize_linear_noalloc(x.data_ptr(), too_many, y.data_ptr(), s.data_ptr(),
                                                z.data_ptr(), torch.cuda.current_stream().cuda_stream)
    assert rc == _lib.NNRH_ERR_INVALID
    assert b"maximum" in L.nnrh_last_error()


def test_dynamic_quantize_noalloc_in_hip_graph(dev):
    """The no-allocation entry point captured into a HIP graph after one
    eager call on the device (which looks up this GPU's scratch address):
    each replay, on new data copied into the captured input between
    replays, equals the workspace entry point's eager result."""
    import torch
    L = _lib.lib()
    rng = np.random.default_rng(11)
    n = 200_003
    x = torch.empty(n, dtype=torch.float32, device=dev)
    y, s, z = _outs(n, dev)
    ws = torch.empty(int(L.nnrh_dynamic_quantize_workspace()), dtype=torch.uint8, device=dev)
    wy, wsc, wz = _outs(n, dev)
    x.copy_(_dev(rng.normal(0, 3.0, n).astype(np.float32), dev))
    _lib.check(L.nnrh_dynamic_quantize_linear_noalloc(x.data_ptr(), n, y.data_ptr(), s.data_ptr(), z.data_ptr(),
                                                      torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        _lib.check(L.nnrh_dynamic_quantize_linear_noalloc(x.data_ptr(), n, y.data_ptr(), s.data_ptr(),
                                                          z.data_ptr(), torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    for rep, (mu, sd) in enumerate(((-2.0, 7.0), (5.0, 0.25), (0.0, 40.0))):
        print(f"graph replay {rep}", flush=True)
        xh = (rng.normal(mu, sd, n)).astype(np.float32)
        x.copy_(_dev(xh, dev))
        y.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        _lib.check(L.nnrh_dynamic_quantize_linear(x.data_ptr(), n, wy.data_ptr(), wsc.data_ptr(), wz.data_ptr(),
                                                  ws.data_ptr(), torch.cuda.current_stream().cuda_stream))
        torch.cuda.synchronize()
        assert s.cpu().numpy()[0] == wsc.cpu().numpy()[0]
        assert int(z.cpu().numpy()[0]) == int(wz.cpu().numpy()[0])
        assert np.array_equal(y.cpu().numpy(), wy.cpu().numpy())
        y_ref, s_ref, z_ref = O.dynamic_quantize_linear(xh)
        assert s.cpu().numpy()[0] == np.float32(s_ref) and np.array_equal(y.cpu().numpy(), y_ref)

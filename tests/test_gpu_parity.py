"""GPU parity: every HIP path against the CPU oracle, bit-exact, through the C
ABI (nnr_amd is a ctypes view of include/nnr_hip.h). Covers every kernel
branch of QLinearConv's dispatch, QLinearMatMul / MatMulInteger shapes and
dtypes, and the element-wise ops, including tails and edge shapes."""
import numpy as np
import pytest

import nnr_amd as H
from oracle import pyoracle as O

pytestmark = pytest.mark.gpu


def to_dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def to_np(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


# ---------------------------------------------------------------------------
# QLinearMatMul

def test_qmatmul_config1(dev):
    """cfg1: A u8[1024,768] x B i8[768,3072] -> u8, per-tensor scales."""
    rng = np.random.default_rng(1)
    a = rng.integers(0, 256, (1024, 768), dtype=np.uint8)
    b = rng.integers(-127, 128, (768, 3072), dtype=np.int8)
    ref = O.qlinear_matmul(a, 0.02, 128, b, 0.005, 0, 0.05, 128)
    op = H.QLinearMatMul(b, 0.02, 128, 0.005, 0, 0.05, 128, m=1024)
    y = to_np(op(to_dev(a, dev)))
    assert np.array_equal(y, ref)


MM_CASES = [
    # m, n, k, batch, a_dt, b_dt, y_dt, b_zp, scale_dt
    (5, 70, 100, 1, np.uint8, np.int8, np.uint8, 0, np.float32),
    (33, 64, 3, 1, np.uint8, np.int8, np.uint8, 0, np.float32),
    (128, 768, 768, 4, np.uint8, np.int8, np.uint8, 0, np.float32),
    (17, 130, 72, 3, np.int8, np.int8, np.int8, -3, np.float32),
    (64, 96, 64, 1, np.uint8, np.uint8, np.uint8, 114, np.float32),
    (7, 50, 40, 2, np.uint8, np.int8, np.uint8, 0, np.float16),
    (300, 257, 129, 1, np.int8, np.uint8, np.uint8, 7, np.float32),
    # K % 128 == 0 and few 128 x 128 tiles: K split over two waves a sub-tile
    (300, 200, 384, 1, np.uint8, np.int8, np.uint8, 0, np.float32),
    (257, 130, 512, 2, np.int8, np.int8, np.int8, -3, np.float32),
]


@pytest.mark.parametrize("m,n,k,batch,adt,bdt,ydt,bzp,sdt", MM_CASES)
def test_qmatmul_shapes(dev, m, n, k, batch, adt, bdt, ydt, bzp, sdt):
    rng = np.random.default_rng(m * 1000 + n + k)
    info = lambda t: (np.iinfo(t).min, np.iinfo(t).max + 1)
    a = rng.integers(*info(adt), (batch, m, k), dtype=adt)
    b = rng.integers(*info(bdt), (k, n), dtype=bdt)
    a_zp = 121 if adt == np.uint8 else -9
    y_zp = 128 if ydt == np.uint8 else 3
    ref = O.qlinear_matmul(a, 0.021, a_zp, b, 0.0047, bzp, 0.31, y_zp, ydt, sdt)
    op = H.QLinearMatMul(b, 0.021, a_zp, 0.0047, bzp, 0.31, y_zp, m=m, a_dtype=adt, y_dtype=ydt,
                         scale_dtype=sdt)
    y = to_np(op(to_dev(a, dev)))
    assert np.array_equal(y, ref)


def test_qmatmul_device_quant_params(dev):
    """a_scale / a_zp from device memory (the DynamicQuantizeLinear hand-off)."""
    import torch
    rng = np.random.default_rng(21)
    a = rng.integers(0, 256, (2, 40, 96), dtype=np.uint8)
    b = rng.integers(-127, 128, (96, 80), dtype=np.int8)
    ref = O.qlinear_matmul(a, np.float32(0.0133), 77, b, 0.004, 0, 0.02, 128)
    op = H.QLinearMatMul(b, 1.0, 0, 0.004, 0, 0.02, 128, m=40)
    s = torch.tensor([0.0133], dtype=torch.float32, device=dev)
    z = torch.tensor([77], dtype=torch.uint8, device=dev)
    y = to_np(op(to_dev(a, dev), a_scale_dev=s, a_zp_dev=z))
    assert np.array_equal(y, ref)


@pytest.mark.parametrize("m,n,k,adt,bdt,azp,bzp,batch", [
    (64, 64, 64, np.uint8, np.int8, 128, 0, 1),
    (19, 45, 27, np.int8, np.uint8, -4, 200, 1),
    (128, 200, 300, np.uint8, np.uint8, 3, 250, 3),
    (50, 33, 16, np.int8, np.int8, 0, -7, 2),
    # int32 output with the K split (K % 128 == 0, few tiles)
    (257, 130, 512, np.uint8, np.int8, 7, 0, 1),
    (200, 384, 1024, np.int8, np.int8, -3, 0, 2),
])
def test_matmul_integer(dev, m, n, k, adt, bdt, azp, bzp, batch):
    rng = np.random.default_rng(5 + m)
    info = lambda t: (np.iinfo(t).min, np.iinfo(t).max + 1)
    a = rng.integers(*info(adt), (batch, m, k), dtype=adt)
    b = rng.integers(*info(bdt), (batch, k, n), dtype=bdt)
    ref = O.matmul_integer(a, b, azp, bzp)
    op = H.MatMulInteger(m, n, k, adt, bdt, max_batch=batch)
    y = to_np(op(to_dev(a, dev), to_dev(b, dev), azp, bzp, batch=batch))
    assert np.array_equal(y.reshape(ref.shape), ref)


# ---------------------------------------------------------------------------
# QLinearConv

def run_conv_case(dev, N, C, Hh, W, OC, k, seed, expect=None, x_nhwc=0, bias=True, **kw):
    rng = np.random.default_rng(seed)
    act = kw.get("act_dtype", np.uint8)
    G = kw.get("group", 1)
    info = (0, 256) if act == np.uint8 else (-128, 128)
    x = rng.integers(*info, (N, C, Hh, W), dtype=act)
    w = rng.integers(-127, 128, (OC, C // G, k, k), dtype=np.int8)
    kw.setdefault("w_scale", rng.uniform(0.001, 0.01, OC).astype(np.float32))
    kw.setdefault("x_scale", 0.02)
    kw.setdefault("x_zp", 128 if act == np.uint8 else -5)
    kw.setdefault("y_scale", 0.03)
    b = rng.integers(-4096, 4097, OC).astype(np.int32) if bias else None
    xin = x.transpose(0, 2, 3, 1).copy() if x_nhwc else x
    ocv = O.Conv(N, C, Hh, W, OC, k, k, x_nhwc=x_nhwc, bias=b, **kw)
    ref, br = ocv.run(xin, w)
    op = H.QLinearConv(N, C, Hh, W, w, x_nhwc=x_nhwc, bias=b, **kw)
    assert op.branch == br
    if expect is not None:
        assert H.BRANCH_NAMES[br] == expect
    y = to_np(op(to_dev(xin, dev)))
    assert y.shape == ref.shape
    mism = np.count_nonzero(y != ref)
    assert mism == 0, f"{mism} of {y.size} differ (branch {H.BRANCH_NAMES[br]})"


def test_qconv_config2(dev):
    """cfg2: 3x3 s1 p1, x u8[32,64,56,56] NCHW, per-channel w scales, Relu via
    y_zp 0 and a fused Relu (post_fn) -> NR16 NHWC-direct, RQ-B."""
    run_conv_case(dev, 32, 64, 56, 56, 64, 3, seed=2, expect="NR16", pads=(1, 1, 1, 1),
                  y_nhwc=1, post_fn=1, y_zp=0, x_zp=128)


@pytest.mark.parametrize("N,C,Hh,W,OC,k,kw", [
    # 1x1 as a dense GEMM, ragged last row tile (M = 46800), three column tiles
    (13, 64, 60, 60, 384, 1, dict(x_nhwc=1, y_zp=5)),
    # 3x3 uniform tap walk (C % 64 == 0), NR16
    (11, 64, 48, 48, 512, 3, dict(pads=(1, 1, 1, 1), x_nhwc=1, post_fn=1, y_zp=0)),
    # 3x3 with C = 48: the per-chunk tap walk
    (11, 48, 48, 48, 512, 3, dict(pads=(1, 1, 1, 1), x_nhwc=1, y_zp=9)),
    # stride 2
    (40, 64, 48, 48, 640, 3, dict(stride=(2, 2), pads=(1, 1, 1, 1), x_nhwc=1, y_zp=2))])
def test_qconv_tile_256x128(dev, N, C, Hh, W, OC, k, kw):
    """Convolutions big enough for the 8-wave 256x128 tile (N >= 256 and at
    least 384 such tiles): bit-exact with the oracle like the 4-wave tiles."""
    x_nhwc = kw.pop("x_nhwc", 0)
    run_conv_case(dev, N, C, Hh, W, OC, k, seed=N + OC, y_nhwc=1, x_nhwc=x_nhwc, **kw)


def test_conv_integer_tile_256x128(dev):
    """ConvInteger on the 8-wave tile: the in-kernel row sums of the weight
    zero-point term with 8 waves (per-channel w_zp), int32 NCHW output."""
    rng = np.random.default_rng(88)
    N, C, HW, OC = 6, 64, 64, 512
    x = rng.integers(0, 256, (N, C, HW, HW), dtype=np.uint8)
    w = rng.integers(-128, 128, (OC, C, 3, 3), dtype=np.int8)
    wz = rng.integers(-128, 128, OC)
    ref = O.conv_integer(x, w, 113, wz, (1, 1), (1, 1), (1, 1), 1)
    y = H.conv_integer(to_dev(x, dev), to_dev(w, dev), 113, wz, (1, 1), (1, 1), (1, 1), 1)
    assert np.array_equal(to_np(y), ref)


CONV_CASES = [
    # name, N, C, H, W, OC, k, kwargs
    ("nr16_nhwc_in", 2, 64, 14, 15, 128, 3, dict(pads=(1, 1, 1, 1), y_nhwc=1, x_nhwc=1, y_zp=3)),
    ("packed_1x1", 2, 256, 7, 9, 64, 1, dict(y_nhwc=1, x_nhwc=1, y_zp=7)),
    ("packed_bprime", 1, 32, 6, 7, 48 + 40, 1, dict(y_nhwc=1, x_nhwc=1, y_zp=11)),
    ("packed_s2", 2, 64, 13, 13, 96, 3, dict(stride=(2, 2), pads=(1, 1, 1, 1), y_nhwc=1)),
    ("packed_wzp", 1, 48, 9, 9, 40, 3, dict(pads=(1, 1, 1, 1), y_nhwc=1, w_zp=(3,))),
    # a negative int8 w_zp is read through the uint8 activation type (253)
    ("packed_wzp_neg", 1, 32, 7, 7, 24, 1, dict(y_nhwc=1, w_zp=(-3,), y_scale=3.0, y_zp=40)),
    ("first_s1_pad", 2, 3, 20, 21, 48, 5, dict(pads=(2, 1, 2, 1), y_nhwc=1, y_zp=17)),
    ("packed_nchw_out", 1, 32, 20, 20, 24, 3, dict(pads=(1, 1, 1, 1), y_nhwc=0)),
    # NCHW input through the 16 x 16 register transpose (HW % 16 == 0): 40
    # channels padded to 48 with the zero point; 64 channels, 3 images
    ("nchw16_c40_pad", 2, 40, 8, 12, 64, 3, dict(pads=(1, 1, 1, 1), y_nhwc=1, y_zp=4)),
    ("nchw16_c64", 3, 64, 16, 16, 32, 1, dict(y_nhwc=1, x_zp=200)),
    ("packed_dil", 1, 16, 12, 12, 32, 3, dict(pads=(2, 2, 2, 2), dil=(2, 2), y_nhwc=1)),
    ("packed_c24", 2, 24, 10, 10, 144, 1, dict(y_nhwc=1, x_nhwc=1)),
    # the short-K direct kernel: 1x1 NHWC with one 64-byte K step, rows read
    # unpadded in 8-byte pieces (C = 24, 40) or 16-byte chunks (C = 16, 64);
    # ragged column blocks, zero point 0 (saturating store) and odd
    ("direct_c24", 3, 24, 19, 21, 144, 1, dict(y_nhwc=1, x_nhwc=1, y_zp=3)),
    ("direct_c40_oc72", 2, 40, 13, 17, 72, 1, dict(y_nhwc=1, x_nhwc=1, y_zp=0, post_fn=1)),
    ("direct_c16_oc96", 4, 16, 24, 24, 96, 1, dict(y_nhwc=1, x_nhwc=1, y_zp=128)),
    ("direct_c64_oc16", 2, 64, 30, 30, 16, 1, dict(y_nhwc=1, x_nhwc=1, y_zp=7)),
    # 32- and 16-column blocks of the direct kernel: 32 and 24 channels (a
    # ragged 8-byte chunk), 8 channels with K = 24
    ("direct_c32_oc32", 3, 32, 17, 19, 32, 1, dict(y_nhwc=1, x_nhwc=1, y_zp=0, post_fn=1)),
    ("direct_c48_oc24", 2, 48, 21, 13, 24, 1, dict(y_nhwc=1, x_nhwc=1, y_zp=9)),
    ("direct_c24_oc8", 2, 24, 11, 12, 8, 1, dict(y_nhwc=1, x_nhwc=1, y_zp=130)),
    ("direct", 2, 64, 12, 12, 64, 3, dict(pads=(1, 1, 1, 1), y_nhwc=0, post_fn=1, y_zp=9)),
    ("direct_tail", 1, 20, 9, 7, 30, 3, dict(pads=(1, 1, 1, 1), y_nhwc=0, y_zp=20)),
    ("first_nhwc", 2, 3, 40, 40, 64, 7, dict(stride=(2, 2), pads=(3, 3, 3, 3), y_nhwc=1)),
    ("first_nchw", 1, 3, 37, 37, 32, 3, dict(stride=(2, 2), pads=(1, 1, 1, 1), y_nhwc=0,
                                               post_fn=1, y_zp=4)),
    ("dw_s1", 2, 32, 10, 11, 32, 3, dict(group=32, pads=(1, 1, 1, 1), y_nhwc=1, x_nhwc=1)),
    ("dw_s2", 1, 96, 15, 15, 96, 3, dict(group=96, stride=(2, 2), pads=(1, 1, 1, 1), y_nhwc=1,
                                          x_nhwc=1, y_zp=2)),
    ("dw_nchw_s1", 1, 16, 9, 9, 16, 3, dict(group=16, pads=(1, 1, 1, 1), y_nhwc=0)),
    ("dw_nchw_s2", 1, 16, 9, 9, 16, 3, dict(group=16, stride=(2, 2), pads=(1, 1, 1, 1),
                                            y_nhwc=0, post_fn=1, y_zp=6)),
    ("grouped_s1", 1, 16, 8, 8, 32, 3, dict(group=4, pads=(1, 1, 1, 1))),
    ("grouped_s2", 1, 32, 11, 11, 16, 3, dict(group=2, stride=(2, 2), pads=(1, 1, 1, 1),
                                              post_fn=1, y_zp=12)),
    ("float_int8act", 1, 16, 9, 9, 24, 3, dict(pads=(1, 1, 1, 1), act_dtype=np.int8, y_zp=-4)),
    ("float_pcz", 1, 16, 8, 8, 4, 1, dict(w_zp=(1, -2, 3, 0))),
    # direct-to-LDS pipelined GEMM: taps spanning a 64-byte K step (C=48),
    # a ragged last column block (OC=72), more tiles than resident blocks
    # (several tiles per persistent block), strided 3x3, grouped RQ-A
    ("dma_c48_oc72", 2, 48, 11, 13, 72, 3, dict(pads=(1, 1, 1, 1), y_nhwc=1, x_nhwc=1, y_zp=5)),
    ("dma_persistent_1x1", 16, 64, 56, 56, 256, 1, dict(y_nhwc=1, x_nhwc=1, y_zp=2)),
    ("dma_s2_3x3", 4, 128, 28, 28, 128, 3, dict(stride=(2, 2), pads=(1, 1, 1, 1), y_nhwc=1,
                                                x_nhwc=1)),
    ("dma_grouped_c16", 1, 64, 8, 8, 64, 3, dict(group=4, pads=(1, 1, 1, 1))),
    # few 128 x 128 tiles, K % 128 == 0: two waves a sub-tile, one per K half
    # (uniform taps with C = 128; 1x1 dense; stride 2; ragged rows / columns)
    ("ksplit_3x3_c128", 3, 128, 17, 19, 192, 3, dict(pads=(1, 1, 1, 1), y_nhwc=1, x_nhwc=1, y_zp=7)),
    ("ksplit_1x1_c256", 2, 256, 14, 14, 320, 1, dict(y_nhwc=1, x_nhwc=1, post_fn=1)),
    ("ksplit_3x3_s2", 4, 128, 28, 28, 256, 3, dict(stride=(2, 2), pads=(1, 1, 1, 1), y_nhwc=1, x_nhwc=1)),
    # uniform-tap convs split K on grids larger than the resident blocks too:
    # several tiles per persistent block (552 and 588 tiles; a ragged last
    # column block)
    ("ksplit_persistent_2x2", 16, 128, 24, 25, 1024, 2, dict(y_nhwc=1, x_nhwc=1, y_zp=3)),
    ("ksplit_persistent_3x3", 48, 128, 28, 28, 192, 3, dict(pads=(1, 1, 1, 1), y_nhwc=1, x_nhwc=1,
                                                            x_zp=77)),
    # 256 x 64 tiles with 2 stages (3 blocks per CU): a 3x3 uniform-tap conv
    # with several tiles per persistent block (784 tiles), a one-step 1x1
    # with a ragged column block
    ("tall2_persistent_3x3", 64, 64, 56, 56, 64, 3, dict(pads=(1, 1, 1, 1), y_nhwc=1, x_nhwc=1,
                                                          y_zp=6)),
    ("tall2_1x1_k64", 16, 64, 56, 56, 48, 1, dict(y_nhwc=1, x_nhwc=1, y_zp=5)),
    # first layer on the padded multi-copy image: strides 2, 3 (4 copies), 4
    # (1 copy), 4 input channels
    ("first_mbv2_stem", 2, 3, 32, 32, 32, 3, dict(stride=(2, 2), pads=(1, 1, 1, 1), y_nhwc=1)),
    ("first_s3", 1, 3, 33, 30, 32, 3, dict(stride=(3, 3), pads=(1, 1, 1, 1), y_nhwc=1, post_fn=1,
                                          y_zp=6)),
    ("first_s4_c4", 1, 4, 17, 19, 16, 3, dict(stride=(4, 4), y_nhwc=1, y_zp=1)),
    # one-kernel stem on a uint8 image (width % 16 == 0): 4 channels, odd
    # stride, fused Relu (RQ-C bounds [zp, 255]), 48 output channels
    ("first_stem_u8_s3_c4", 2, 4, 30, 48, 48, 3, dict(stride=(3, 3), pads=(1, 1, 1, 1), y_nhwc=1, post_fn=1,
                                                       y_zp=6)),
    # depthwise dot4 kernel: 2x2 taps (one tap group), dilation, odd zero points,
    # channels over several 16-channel chunks; 5x5 (25 taps) takes the VALU kernel
    ("dw16_k2_zpodd", 1, 48, 9, 10, 48, 2, dict(group=48, pads=(0, 0, 1, 1), y_nhwc=1, x_nhwc=1,
                                               x_zp=3, y_zp=7)),
    ("dw16_dil2", 2, 64, 11, 12, 64, 3, dict(group=64, dil=(2, 2), pads=(2, 2, 2, 2), y_nhwc=1,
                                             x_nhwc=1, y_zp=5, post_fn=1)),
    ("dw16_c960_s2", 1, 960, 7, 8, 960, 3, dict(group=960, stride=(2, 2), pads=(1, 1, 1, 1),
                                                y_nhwc=1, x_nhwc=1)),
    ("dw_k5_valu", 1, 32, 9, 9, 32, 5, dict(group=32, pads=(2, 2, 2, 2), y_nhwc=1, x_nhwc=1)),
    # 3x3 depthwise, one dot4 per filter row over 4 pixels' shared columns:
    # ragged last pixel group, asymmetric pads, x_zp != 0, int8 activations,
    # one / many 8-channel chunks, even and odd widths at stride 2
    ("dw3_s1_tail_zp", 2, 16, 7, 13, 16, 3, dict(group=16, pads=(1, 1, 1, 1), y_nhwc=1, x_nhwc=1,
                                                  x_zp=37, y_zp=3, post_fn=1)),
    ("dw3_s2_even_asym", 1, 144, 16, 16, 144, 3, dict(group=144, stride=(2, 2), pads=(0, 0, 1, 1),
                                                       y_nhwc=1, x_nhwc=1, y_zp=11)),
    ("dw3_s2_odd_w", 3, 32, 13, 17, 32, 3, dict(group=32, stride=(2, 2), pads=(1, 1, 1, 1), y_nhwc=1,
                                                 x_nhwc=1, x_zp=200)),
    ("dw3_s1_int8", 1, 48, 9, 10, 48, 3, dict(group=48, pads=(1, 1, 1, 1), y_nhwc=1, x_nhwc=1,
                                               act_dtype=np.int8, x_zp=-5, y_zp=-2)),
    ("dw3_s1_c960_wide", 1, 960, 5, 29, 960, 3, dict(group=960, pads=(1, 1, 1, 1), y_nhwc=1,
                                                      x_nhwc=1)),
    # 24 channels (three 8-channel chunks), one / three 16-pixel spans a row,
    # odd zero points, int8 at stride 2, a larger batch
    ("dw3_s1_c24", 2, 24, 9, 11, 24, 3, dict(group=24, pads=(1, 1, 1, 1), y_nhwc=1, x_nhwc=1,
                                              x_zp=9, y_zp=4)),
    ("dw3_s1_c144_7x7", 3, 144, 7, 7, 144, 3, dict(group=144, pads=(1, 1, 1, 1), y_nhwc=1, x_nhwc=1,
                                                    x_zp=113, y_zp=7)),
    ("dw3_s1_c64_w40", 2, 64, 11, 40, 64, 3, dict(group=64, pads=(1, 1, 1, 1), y_nhwc=1, x_nhwc=1,
                                                   post_fn=1)),
    ("dw3_s2_int8_c32", 2, 32, 15, 21, 32, 3, dict(group=32, stride=(2, 2), pads=(1, 1, 1, 1), y_nhwc=1,
                                                    x_nhwc=1, act_dtype=np.int8, x_zp=-7, y_zp=3)),
    ("dw3_s1_c384_b16", 16, 384, 14, 14, 384, 3, dict(group=384, pads=(1, 1, 1, 1), y_nhwc=1, x_nhwc=1)),
    # ten 8-channel chunks, an odd output zero point; stride 2 onto 7 x 7 maps
    # of five images with a fused Relu
    ("dw3_c80_yzp128", 2, 80, 9, 9, 80, 3, dict(group=80, pads=(1, 1, 1, 1), y_nhwc=1, x_nhwc=1,
                                              x_zp=3, y_zp=128)),
    ("dw3_s2_c96_b5", 5, 96, 14, 14, 96, 3, dict(group=96, stride=(2, 2), pads=(1, 1, 1, 1), y_nhwc=1,
                                                   x_nhwc=1, y_zp=5, post_fn=1)),
    # channel counts off the 16-byte grid run on an x_zp-padded copy
    ("cpad_c8_3x3", 2, 8, 10, 11, 40, 3, dict(pads=(1, 1, 1, 1), x_nhwc=1, y_nhwc=1, y_zp=9)),
    ("cpad_c24_wzp", 1, 24, 7, 9, 32, 1, dict(x_nhwc=1, y_nhwc=1, w_zp=(5,), y_zp=2)),
]


@pytest.mark.parametrize("case", CONV_CASES, ids=[c[0] for c in CONV_CASES])
def test_qconv_branches(dev, case):
    name, N, C, Hh, W, OC, k, kw = case
    kw = dict(kw)
    x_nhwc = kw.pop("x_nhwc", 0)
    run_conv_case(dev, N, C, Hh, W, OC, k, seed=sum(name.encode()), x_nhwc=x_nhwc, **kw)


def test_qconv_no_bias(dev):
    run_conv_case(dev, 1, 64, 10, 10, 64, 3, seed=5, bias=False, pads=(1, 1, 1, 1), y_nhwc=1)


FUSED_ADD_CASES = [
    # name, N, C, H, W, OC, k, pads, conv_is_a
    ("1x1_conv_a", 2, 64, 14, 15, 256, 1, (0, 0, 0, 0), 1),
    # a ragged last column block (80 of 128) and conv as the add's B input
    ("3x3_conv_b", 1, 64, 9, 7, 80, 3, (1, 1, 1, 1), 0),
    # uniform-tap conv (C % 64 == 0), several K steps per tile
    ("3x3_c256_a", 2, 256, 10, 9, 192, 3, (1, 1, 1, 1), 1),
    ("persistent", 16, 64, 56, 56, 256, 1, (0, 0, 0, 0), 1),
    # K = 64 / 128 with the weights in registers (one column block per
    # persistent block): ragged last column block (64 of 128) and ragged
    # rows, conv as B; four column blocks, conv as A
    ("kr1_n192_b", 8, 64, 30, 31, 192, 1, (0, 0, 0, 0), 0),
    ("kr2_c128_a", 6, 128, 28, 28, 512, 1, (0, 0, 0, 0), 1),
]


@pytest.mark.parametrize("case", FUSED_ADD_CASES, ids=[c[0] for c in FUSED_ADD_CASES])
def test_qconv_fused_add(dev, case):
    """conv + same-shape QLinearAdd in one kernel == oracle conv, then oracle add."""
    name, N, C, Hh, W, OC, k, pads, conv_is_a = case
    rng = np.random.default_rng(sum(name.encode()))
    x = rng.integers(0, 256, (N, Hh, W, C), dtype=np.uint8)
    w = rng.integers(-127, 128, (OC, C, k, k), dtype=np.int8)
    b = rng.integers(-4096, 4097, OC).astype(np.int32)
    kw = dict(pads=pads, x_nhwc=1, y_nhwc=1, x_scale=0.02, x_zp=128, y_scale=0.05, y_zp=3,
              w_scale=rng.uniform(0.001, 0.01, OC).astype(np.float32), bias=b)
    conv_ref, _ = O.Conv(N, C, Hh, W, OC, k, k, **kw).run(x, w)
    other = rng.integers(0, 256, conv_ref.shape, dtype=np.uint8)
    # add: A, B scales / zps; the conv side's are independent of its y quant
    sa, za, sb, zb, sy, zy = 0.041, 7, 0.023, 131, 0.06, 2
    a_, b_ = (conv_ref, other) if conv_is_a else (other, conv_ref)
    ref = O.qlinear_add(0, a_, b_, sa, za, sb, zb, sy, zy)
    op = H.QLinearConv(N, C, Hh, W, w, **kw)
    assert op.fuse_add(conv_is_a, sa, za, sb, zb, sy, zy)
    y = to_np(op.run_add(to_dev(x, dev), to_dev(other, dev)))
    mism = np.count_nonzero(y != ref)
    assert mism == 0, f"{mism} of {y.size} differ"


def test_qconv_fuse_add_unsupported(dev):
    """Convolutions whose kernel has no fused add say so and stay usable."""
    rng = np.random.default_rng(11)
    x = rng.integers(0, 256, (1, 3, 20, 20), dtype=np.uint8)
    w = rng.integers(-127, 128, (16, 3, 3, 3), dtype=np.int8)
    kw = dict(pads=(1, 1, 1, 1), y_nhwc=1, x_scale=0.02, x_zp=128, y_scale=0.05, y_zp=0,
              w_scale=np.full(16, 0.004, np.float32))
    op = H.QLinearConv(1, 3, 20, 20, w, **kw)   # first-layer branch
    assert not op.fuse_add(1, 0.05, 0, 0.05, 0, 0.05, 0)
    ref, _ = O.Conv(1, 3, 20, 20, 16, 3, 3, **kw).run(x, w)
    assert np.array_equal(to_np(op(to_dev(x, dev))), ref)
    # output channels off the 16-byte grid: the residual cannot travel in
    # whole 16-byte chunks, so the add stays a separate operator
    x2 = rng.integers(0, 256, (1, 9, 7, 64), dtype=np.uint8)
    w2 = rng.integers(-127, 128, (72, 64, 3, 3), dtype=np.int8)
    kw2 = dict(pads=(1, 1, 1, 1), x_nhwc=1, y_nhwc=1, x_scale=0.02, x_zp=128, y_scale=0.05,
               y_zp=3, w_scale=np.full(72, 0.004, np.float32))
    op2 = H.QLinearConv(1, 64, 9, 7, w2, **kw2)
    assert not op2.fuse_add(0, 0.041, 7, 0.023, 131, 0.06, 2)
    ref2, _ = O.Conv(1, 64, 9, 7, 72, 3, 3, **kw2).run(x2, w2)
    assert np.array_equal(to_np(op2(to_dev(x2, dev))), ref2)


# ---------------------------------------------------------------------------
# element-wise

@pytest.mark.parametrize("n", [40, 64, 70, 4096 + 21, 300000])
@pytest.mark.parametrize("dt", [np.uint8, np.int8])
def test_quantize(dev, n, dt):
    rng = np.random.default_rng(n)
    x = rng.normal(0, 2, n).astype(np.float32)
    zp = 128 if dt == np.uint8 else -3
    ref = O.quantize_linear(x, 0.0173, zp, dt)
    y = to_np(H.quantize_linear(to_dev(x, dev), 0.0173, zp, dt))
    assert np.array_equal(y, ref)


def test_dequantize(dev):
    rng = np.random.default_rng(3)
    for dt in (np.uint8, np.int8):
        q = rng.integers(np.iinfo(dt).min, np.iinfo(dt).max + 1, 10007, dtype=dt)
        ref = O.dequantize_linear(q, 0.0371, 17)
        y = to_np(H.dequantize_linear(to_dev(q, dev), 0.0371, 17))
        assert np.array_equal(y, ref)


@pytest.mark.parametrize("n", [6, 1000, 98304 * 3 + 5])
def test_dynamic_quantize(dev, n):
    rng = np.random.default_rng(n)
    x = (rng.normal(0, 1.5, n) + 0.3).astype(np.float32)
    y_ref, s_ref, z_ref = O.dynamic_quantize_linear(x)
    y, s, z = H.dynamic_quantize_linear(to_dev(x, dev))
    assert to_np(s)[0] == np.float32(s_ref) and int(to_np(z)[0]) == z_ref
    assert np.array_equal(to_np(y), y_ref)


def dyn_quant_ties(n, seed):
    """Data whose scale is exactly 2^-4 (min -4, max 11.9375: range 255 / 16)
    with most values at or one ulp off a half-integer multiple of it, so
    x / scale is an exact tie or within 2^-18 of one: the cases where
    rounding a product by 1/scale instead of the quotient could differ,
    beside ordinary values and a few with |x / scale| near 255."""
    rng = np.random.default_rng(seed)
    k = rng.integers(-64, 191, n).astype(np.float32)
    x = ((k + 0.5) * np.float32(0.0625)).astype(np.float32)
    step = rng.integers(-1, 2, n)
    x = np.where(step < 0, np.nextafter(x, np.float32(-np.inf)), np.where(step > 0, np.nextafter(x, np.float32(np.inf)), x)).astype(np.float32)
    plain = rng.random(n) < 0.25
    x[plain] = rng.uniform(-4, 11.9375, plain.sum()).astype(np.float32)
    x[:2] = (-4.0, 11.9375)
    x[2:6] = (11.9375, np.nextafter(np.float32(11.9375), np.float32(0)), -4.0, np.float32(-3.96875))
    return x


@pytest.mark.parametrize("n", [4096, 70001])
def test_dynamic_quantize_ties(dev, n):
    """DynamicQuantizeLinear on exact and near ties of x / scale, both the
    two-pass form and the one from producer pairs: bytes equal the oracle's
    (the kernels take the division for elements near a half-integer)."""
    x = dyn_quant_ties(n, n)
    y_ref, s_ref, z_ref = O.dynamic_quantize_linear(x)
    assert np.float32(s_ref) == np.float32(0.0625)
    y, s, z = H.dynamic_quantize_linear(to_dev(x, dev))
    assert to_np(s)[0] == np.float32(s_ref) and int(to_np(z)[0]) == z_ref
    assert np.array_equal(to_np(y), y_ref)
    pr = np.array([[x.min(), 0.0], [0.0, x.max()]], np.float32)
    y2, s2, z2 = H.dynamic_quantize_linear_parts(to_dev(x, dev), to_dev(pr.reshape(-1), dev))
    assert to_np(s2)[0] == np.float32(s_ref) and int(to_np(z2)[0]) == z_ref
    assert np.array_equal(to_np(y2), y_ref)


@pytest.mark.parametrize("kind", [0, 1, 2, 3])
@pytest.mark.parametrize("y_nhwc", [0, 1])
def test_qlinear_add(dev, kind, y_nhwc):
    rng = np.random.default_rng(kind * 10 + y_nhwc)
    N, C, HW = 3, 40, 37
    n = N * C * HW
    a = rng.integers(0, 256, n, dtype=np.uint8)
    b = rng.integers(0, 256, {0: n, 1: 1, 2: n, 3: C}[kind], dtype=np.uint8)
    if kind == 2:
        a, b = rng.integers(0, 256, 1, dtype=np.uint8), a
    args = (0.031, 117, 0.017, 131, 0.043, 3)
    ref = O.qlinear_add(kind, a, b, *args, C=C, HW=HW, y_nhwc=y_nhwc)
    y = to_np(H.qlinear_add(kind, to_dev(a, dev), to_dev(b, dev), *args, C=C, HW=HW,
                            y_nhwc=y_nhwc))
    assert np.array_equal(y, ref)


# ---------------------------------------------------------------------------
# the rest of the QLinear family, bit-exact against the oracle

@pytest.mark.parametrize("kind,shape_b,nhwc", [(0, None, 0), (1, (1,), 0), (2, "a1", 0), (3, "c", 0), (3, "c", 1)])
@pytest.mark.parametrize("dt", [np.uint8, np.int8])
@pytest.mark.parametrize("N,C,Hh,W", [(2, 19, 5, 7),     # 665 per image: ragged 16-wide body, one byte a thread
                                      (3, 32, 4, 8)])    # 16 elements a thread (n, C and HW multiples of 16)
def test_qlinear_mul(dev, kind, shape_b, nhwc, dt, N, C, Hh, W):
    rng = np.random.default_rng(kind * 7 + nhwc + (dt == np.int8) + C)
    info = (0, 256) if dt == np.uint8 else (-128, 128)
    full = rng.integers(*info, (N, C, Hh, W) if not nhwc else (N, Hh, W, C), dtype=dt)
    if kind == 0:
        a, b = full, rng.integers(*info, full.shape, dtype=dt)
    elif kind == 1:
        a, b = full, rng.integers(*info, (1,), dtype=dt)
    elif kind == 2:
        a, b = rng.integers(*info, (1,), dtype=dt), full
    else:
        a, b = full, rng.integers(*info, (C,), dtype=dt)
    zps = (13, 200, 128) if dt == np.uint8 else (-7, 20, 3)
    args = (0.037, zps[0], 0.021, zps[1], 0.043, zps[2])
    kw = dict(C=C, HW=Hh * W, y_nhwc=nhwc) if kind == 3 else {}
    ref = O.qlinear_mul(kind, a, b, *args, **kw)
    y = H.qlinear_mul(kind, to_dev(a, dev), to_dev(b, dev), *args, **kw)
    assert np.array_equal(to_np(y), ref)


@pytest.mark.parametrize("nhwc", [0, 1])
@pytest.mark.parametrize("dt,N,C,Hh,W", [(np.uint8, 3, 70, 7, 7), (np.int8, 2, 16, 1, 1), (np.uint8, 1, 5, 13, 17),
                                         # 16-byte paths: pixel lanes + two-level LDS sums (C 32), one-level
                                         # (C 1024), 16-bit lanes flushed past 256 pixels a thread (400x400),
                                         # one group a thread (C 4800), channel slices over blocks (C 8192)
                                         (np.uint8, 3, 32, 56, 56), (np.int8, 2, 32, 12, 12),
                                         (np.uint8, 2, 1024, 7, 7), (np.int8, 1, 16, 400, 400),
                                         (np.uint8, 1, 16, 400, 400), (np.int8, 2, 4800, 2, 2),
                                         (np.uint8, 2, 8192, 3, 1)])
def test_qlinear_global_avgpool(dev, nhwc, dt, N, C, Hh, W):
    rng = np.random.default_rng(N * C + nhwc)
    info = (0, 256) if dt == np.uint8 else (-128, 128)
    x = rng.integers(*info, (N, Hh, W, C) if nhwc else (N, C, Hh, W), dtype=dt)
    zx, zy = (100, 3) if dt == np.uint8 else (-9, 4)
    ref = O.qlinear_global_avgpool(x, 0.031, zx, 0.017, zy, nhwc=nhwc)
    y = H.qlinear_global_avgpool(to_dev(x, dev), 0.031, zx, 0.017, zy, nhwc=nhwc)
    assert np.array_equal(to_np(y), ref)


@pytest.mark.parametrize("nhwc", [0, 1])
@pytest.mark.parametrize("k,st,pad,H_,W_", [((3, 3), (2, 2), (1, 1), 9, 10), ((2, 2), (2, 2), (0, 0), 8, 8),
                                             ((3, 2), (1, 1), (1, 0), 6, 7), ((7, 7), (1, 1), (0, 0), 7, 7),
                                             ((3, 3), (1, 1), (1, 1), 5, 6)])
@pytest.mark.parametrize("C,dt", [(24, np.uint8),    # one byte a thread
                                  (32, np.uint8), (48, np.int8)])   # NHWC: 16 channels a thread
def test_qlinear_avgpool(dev, nhwc, k, st, pad, H_, W_, C, dt):
    rng = np.random.default_rng(H_ * W_ + nhwc + C)
    N = 2
    info = (0, 256) if dt == np.uint8 else (-128, 128)
    x = rng.integers(*info, (N, H_, W_, C) if nhwc else (N, C, H_, W_), dtype=dt)
    oH = (H_ + 2 * pad[0] - k[0]) // st[0] + 1
    oW = (W_ + 2 * pad[1] - k[1]) // st[1] + 1
    zx, zy = (128, 120) if dt == np.uint8 else (-5, 9)
    ref = O.qlinear_avgpool(x, k, st, pad, oH, oW, 0.02, zx, 0.013, zy, nhwc=nhwc)
    y = H.qlinear_avgpool(to_dev(x, dev), k, st, pad, oH, oW, 0.02, zx, 0.013, zy, nhwc=nhwc)
    assert np.array_equal(to_np(y), ref)


@pytest.mark.parametrize("counts,outer", [([3, 17, 32], 5), ([64, 64], 1), ([15, 1, 16, 33], 37),
                                          # 16-, 8- and 4-byte units (NHWC pixels of 24 + 8 channels)
                                          ([16, 32, 48], 7), ([24, 8], 50), ([4, 12], 9),
                                          # more parts than one launch takes: part by part
                                          ([8, 16, 8, 24, 8, 16, 8, 8, 16], 11), ([0, 16, 5], 4)])
@pytest.mark.parametrize("dt", [np.uint8, np.int8])
def test_qlinear_concat(dev, counts, outer, dt):
    rng = np.random.default_rng(sum(counts) + outer)
    info = (0, 256) if dt == np.uint8 else (-128, 128)
    xs = [rng.integers(*info, outer * c, dtype=dt) for c in counts]
    scales = [[0.05, 0.031, 0.02, 0.07][t % 4] for t in range(len(counts))]
    zps = [([10, 7, 3, 200] if dt == np.uint8 else [10, 7, -3, -100])[t % 4] for t in range(len(counts))]
    y_s, y_zp = 0.031, 7                   # input 1 (if present) is copied
    ref = O.qlinear_concat(xs, counts, outer, scales, zps, y_s, y_zp)
    y = H.qlinear_concat([to_dev(x, dev) for x in xs], counts, outer, scales, zps, y_s, y_zp)
    assert np.array_equal(to_np(y), ref)


@pytest.mark.parametrize("C,k,st,pad", [(64, (3, 3), 2, 1),   # fixed 3x3 window (ResNet stem)
                                        (48, (2, 2), 2, 0),   # fixed 2x2
                                        (32, (3, 2), 1, 1),   # any window, 16-channel groups
                                        (20, (3, 3), 2, 1)])  # 4-channel path
def test_maxpool(dev, C, k, st, pad):
    rng = np.random.default_rng(6 + C)
    x = rng.integers(0, 256, (4, 23, 21, C), dtype=np.uint8)
    oH = (23 + 2 * pad - k[0]) // st + 1
    oW = (21 + 2 * pad - k[1]) // st + 1
    ref = O.maxpool_u8_nhwc(x, k[0], k[1], st, st, pad, pad, oH, oW)
    y = to_np(H.maxpool_u8_nhwc(to_dev(x, dev), k[0], k[1], st, st, pad, pad, oH, oW))
    assert np.array_equal(y, ref)


# ---------------------------------------------------------------------------
# fp32 glue: Gemm with every broadcast mode and transpose, against float64
# numpy; the reference's float tolerance (tensor_equal, 1e-3 abs)

@pytest.mark.parametrize("M,N,K", [(37, 70, 300),     # the general strided kernel (K % 64 != 0)
                                   (37, 70, 320),     # the small-GEMM kernel: 5 K chunks over 4 waves
                                   (5, 3, 64),        # one chunk, clamped rows / columns
                                   (600, 1030, 77),   # general kernel, many tiles, ragged M / N / K
                                   (37, 70, 1344),    # 21 K chunks over 4 waves
                                   (256, 1000, 1280),  # MobileNetV2's classifier
                                   (256, 1000, 2048)])  # ResNet-50's classifier
@pytest.mark.parametrize("ta,tb,c_mode", [(0, 1, 2), (0, 0, 0), (1, 0, 1), (1, 1, 3), (0, 1, 4)])
def test_gemm_f32(dev, ta, tb, c_mode, M, N, K):
    import torch
    from nnr_amd import _lib
    rng = np.random.default_rng(ta * 10 + tb * 3 + c_mode + M)
    A = rng.standard_normal((K, M) if ta else (M, K)).astype(np.float32) * 0.1
    B = rng.standard_normal((N, K) if tb else (K, N)).astype(np.float32) * 0.1
    Cs = {0: (1,), 1: (1,), 2: (N,), 3: (M, N), 4: (M,)}[c_mode]
    Cb = rng.standard_normal(Cs).astype(np.float32)
    alpha, beta = 0.75, 1.5
    ref = alpha * ((A.T if ta else A).astype(np.float64) @ (B.T if tb else B).astype(np.float64))
    if c_mode:
        cb = Cb.astype(np.float64)
        ref = ref + beta * (cb[:, None] if c_mode == 4 else cb)
    y = torch.empty((M, N), dtype=torch.float32, device=dev)
    # keep the device copies alive until the asynchronous call has run
    Ad, Bd, Cd = to_dev(A, dev), to_dev(B, dev), to_dev(Cb, dev)
    _lib.check(_lib.lib().nnrh_gemm_f32(_lib.ptr(Ad), _lib.ptr(Bd), _lib.ptr(Cd), _lib.ptr(y),
                                        M, N, K, ta, tb, alpha, beta, c_mode, _lib.cur_stream()))
    np.testing.assert_allclose(to_np(y), ref, atol=1e-3, rtol=1e-4)


@pytest.mark.parametrize("ta,tb,shared", [(0, 0, False), (1, 0, True), (0, 1, False), (1, 1, True)])
def test_gemm_f32_batched(dev, ta, tb, shared):
    """Batched MatMul on the general strided kernel: per-batch A, B per batch
    or shared, every transpose, a per-column C, against float64 numpy."""
    import torch
    from nnr_amd import _lib
    rng = np.random.default_rng(ta * 2 + tb + 7 * shared)
    nb, M, N, K = 5, 45, 67, 83
    A = rng.standard_normal((nb, K, M) if ta else (nb, M, K)).astype(np.float32) * 0.1
    Bs = (K, N) if not tb else (N, K)
    B = rng.standard_normal(Bs if shared else (nb,) + Bs).astype(np.float32) * 0.1
    Cb = rng.standard_normal(N).astype(np.float32)
    opA = np.swapaxes(A, -1, -2) if ta else A
    opB = np.swapaxes(B, -1, -2) if tb else B
    ref = 0.5 * np.matmul(opA.astype(np.float64), opB.astype(np.float64)) + 2.0 * Cb.astype(np.float64)
    y = torch.empty((nb, M, N), dtype=torch.float32, device=dev)
    Ad, Bd, Cd = to_dev(A, dev), to_dev(B, dev), to_dev(Cb, dev)
    _lib.check(_lib.lib().nnrh_gemm_f32_batched(_lib.ptr(Ad), _lib.ptr(Bd), _lib.ptr(Cd), _lib.ptr(y), M, N, K, ta,
                                                tb, 0.5, 2.0, 2, nb, M * K, 0 if shared else K * N, M * N,
                                                _lib.cur_stream()))
    np.testing.assert_allclose(to_np(y), ref, atol=1e-3, rtol=1e-4)


def test_qmatmul_fused_dq_bias(dev):
    """QLinearMatMul -> DequantizeLinear -> + bias in one kernel (fp32 out),
    against the oracle's three operators; device-side activation quantization
    parameters as produced by DynamicQuantizeLinear."""
    import torch
    rng = np.random.default_rng(23)
    a = rng.integers(0, 256, (3, 40, 96), dtype=np.uint8)
    b = rng.integers(-127, 128, (96, 136), dtype=np.int8)
    bias = rng.standard_normal(136).astype(np.float32)
    ys, yz = 0.031, 121
    q = O.qlinear_matmul(a, np.float32(0.0133), 77, b, 0.004, 0, ys, yz)
    deq = O.dequantize_linear(q, ys, yz)
    ref = (deq + bias).astype(np.float32)
    op = H.QLinearMatMul(b, 1.0, 0, 0.004, 0, ys, yz, m=40)
    from nnr_amd import _lib
    _lib.check(_lib.lib().nnrh_qmatmul_fuse_dq_bias(op.h, ys, yz, bias.ctypes.data_as(
        __import__("ctypes").POINTER(__import__("ctypes").c_float))))
    s = torch.tensor([0.0133], dtype=torch.float32, device=dev)
    z = torch.tensor([77], dtype=torch.uint8, device=dev)
    y = torch.empty((3, 40, 136), dtype=torch.float32, device=dev)
    ad = to_dev(a, dev)
    op(ad, y=y, a_scale_dev=s, a_zp_dev=z)
    got = to_np(y)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), \
        f"{np.count_nonzero(got != ref)} of {got.size} differ"


@pytest.mark.parametrize("m,n,batch", [(40, 136, 3), (8192 // 64, 3072, 2), (70, 64, 1)])
def test_qmatmul_fused_gelu_minmax(dev, m, n, batch):
    """QLinearMatMul -> DequantizeLinear -> + bias -> Gelu in one kernel that
    also writes the (min, max) pairs of its output: the Gelu bits equal the
    standalone Gelu kernel on the unfused result (and the erf form within
    fp32 rounding of the float64 formula); the pairs cover exactly the
    output's min / max, and DynamicQuantizeLinear from them matches the
    two-pass one byte for byte."""
    import ctypes
    import math
    import torch
    from nnr_amd import _lib
    rng = np.random.default_rng(m + n)
    k = 96
    a = rng.integers(0, 256, (batch, m, k), dtype=np.uint8)
    b = rng.integers(-127, 128, (k, n), dtype=np.int8)
    bias = rng.standard_normal(n).astype(np.float32)
    ys, yz = 0.031, 121
    s = torch.tensor([0.0133], dtype=torch.float32, device=dev)
    z = torch.tensor([77], dtype=torch.uint8, device=dev)
    ad = to_dev(a, dev)
    plain = H.QLinearMatMul(b, 1.0, 0, 0.004, 0, ys, yz, m=m)
    plain.fuse_dq_bias(ys, yz, bias)
    f = plain(ad, a_scale_dev=s, a_zp_dev=z)
    g_ref = torch.empty_like(f)
    _lib.check(_lib.lib().nnrh_gelu_f32(f.data_ptr(), g_ref.data_ptr(), f.numel(), _lib.cur_stream()))
    op = H.QLinearMatMul(b, 1.0, 0, 0.004, 0, ys, yz, m=m)
    op.fuse_dq_bias(ys, yz, bias)
    op.fuse_gelu()
    cnt = op.minmax_count(batch)
    assert cnt == 4 * batch * -(-m // (256 if n <= 64 else 128)) * -(-n // (64 if n <= 64 else 128))
    parts = torch.full((2 * cnt,), float("nan"), dtype=torch.float32, device=dev)
    op.set_minmax_out(parts[: 2 * cnt - 2])
    with pytest.raises(H.NnrHipError):   # a buffer one pair short is refused
        op(ad, a_scale_dev=s, a_zp_dev=z)
    op.set_minmax_out(parts)
    for _ in range(2):   # the second run rewrites every pair
        y = op(ad, a_scale_dev=s, a_zp_dev=z)
        got, ref = to_np(y), to_np(g_ref)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
        fv = to_np(f).astype(np.float64)
        erf = np.vectorize(math.erf)
        np.testing.assert_allclose(got, 0.5 * fv * (1.0 + erf(fv / math.sqrt(2.0))), rtol=2e-6, atol=1e-7)
        pr = to_np(parts).reshape(-1, 2)
        assert not np.isnan(pr).any()
        assert pr[:, 0].min() == min(0.0, got.min()) and pr[:, 1].max() == max(0.0, got.max())
        q1, s1, z1 = H.dynamic_quantize_linear_parts(y, parts)
        q0, s0, z0 = H.dynamic_quantize_linear(y)
        assert to_np(s1)[0] == to_np(s0)[0] and to_np(z1)[0] == to_np(z0)[0]
        assert np.array_equal(to_np(q1), to_np(q0))
        parts.fill_(float("nan"))
    op.set_minmax_out(None)


@pytest.mark.parametrize("m,n,batch,gelu", [(40, 136, 3, True), (8192 // 64, 3072, 2, True), (70, 64, 1, False),
                                             (50, 320, 2, True), (33, 200, 2, False), (21, 131, 2, True)])
def test_qmatmul_codes_dynamic_quantize(dev, m, n, batch, gelu):
    """The fused QLinearMatMul -> DequantizeLinear -> + bias (-> Gelu) chain
    in codes mode: a run stores the uint8 QLinearMatMul bytes (equal to the
    unfused QLinearMatMul's) and the chain values' (min, max) pairs, and
    DynamicQuantizeLinear from the bytes gives the bytes, scale and zero
    point of DynamicQuantizeLinear over the fp32 chain output. Two inputs in a
    row (the per-column table is rebuilt), N % 16 != 0 (ragged GEMM stores),
    N % 4 != 0 (bytewise gather), a last column slice of 64, rows not a
    multiple of the gather's 256."""
    import torch
    rng = np.random.default_rng(m * n + batch)
    k = 96
    b = rng.integers(-127, 128, (k, n), dtype=np.int8)
    bias = (rng.standard_normal(n) * 0.5).astype(np.float32)
    ys, yz = 0.031, 121
    s = torch.tensor([0.0133], dtype=torch.float32, device=dev)
    z = torch.tensor([77], dtype=torch.uint8, device=dev)
    plain = H.QLinearMatMul(b, 1.0, 0, 0.004, 0, ys, yz, m=m)

    def chain(codes):
        op = H.QLinearMatMul(b, 1.0, 0, 0.004, 0, ys, yz, m=m)
        op.fuse_dq_bias(ys, yz, bias)
        if gelu:
            op.fuse_gelu()
        cnt = op.minmax_count(batch)
        parts = torch.full((2 * cnt,), float("nan"), dtype=torch.float32, device=dev)
        op.set_minmax_out(parts)
        if codes:
            op.set_codes_out()
        return op, parts

    f32op, f32parts = chain(False)
    cop, cparts = chain(True)
    for rep in range(2):
        a = to_dev(rng.integers(0, 256, (batch, m, k), dtype=np.uint8), dev)
        q = to_np(plain(a, a_scale_dev=s, a_zp_dev=z))
        f = f32op(a, a_scale_dev=s, a_zp_dev=z)
        q0, s0, z0 = H.dynamic_quantize_linear_parts(f, f32parts)
        c = cop(a, a_scale_dev=s, a_zp_dev=z)
        assert c.dtype == torch.uint8 and tuple(c.shape) == (batch, m, n)
        assert np.array_equal(to_np(c), q), rep
        # the codes run's pairs are the fp32 run's (same values, same tiles)
        assert np.array_equal(to_np(cparts), to_np(f32parts)), rep
        q1, s1, z1 = cop.dynamic_quantize_codes(c)
        assert to_np(s1)[0] == to_np(s0)[0] and to_np(z1)[0] == to_np(z0)[0], rep
        mism = np.count_nonzero(to_np(q1) != to_np(q0))
        assert mism == 0, f"rep {rep}: {mism} of {q1.numel()} bytes differ"
    # back to fp32 output: the same bits as the fp32 handle
    cop.set_codes_out(False)
    assert np.array_equal(to_np(cop(a, a_scale_dev=s, a_zp_dev=z)).view(np.uint32), to_np(f).view(np.uint32))


def _chain_pair(dev, rng, m, n, k=96, batch=1):
    """A fused QLinearMatMul -> DequantizeLinear -> + bias chain twice: one
    handle writing fp32 values, one writing its uint8 bytes (no pairs), on
    the same A; returns (fp32 output, bytes, bytes handle)."""
    import torch
    b = rng.integers(-127, 128, (k, n), dtype=np.int8)
    bias = (rng.standard_normal(n) * 0.5).astype(np.float32)
    ys, yz = float(rng.uniform(0.01, 0.05)), int(rng.integers(90, 160))
    s = torch.tensor([0.0133], dtype=torch.float32, device=dev)
    z = torch.tensor([77], dtype=torch.uint8, device=dev)
    a = to_dev(rng.integers(0, 256, (batch, m, k), dtype=np.uint8), dev)
    f32op = H.QLinearMatMul(b, 1.0, 0, 0.004, 0, ys, yz, m=m)
    f32op.fuse_dq_bias(ys, yz, bias)
    cop = H.QLinearMatMul(b, 1.0, 0, 0.004, 0, ys, yz, m=m)
    cop.fuse_dq_bias(ys, yz, bias)
    cop.set_codes_out()
    f = f32op(a, a_scale_dev=s, a_zp_dev=z)
    c = cop(a, a_scale_dev=s, a_zp_dev=z)
    assert c.dtype == torch.uint8
    # the bytes are the unfused QLinearMatMul's
    q = H.QLinearMatMul(b, 1.0, 0, 0.004, 0, ys, yz, m=m)(a, a_scale_dev=s, a_zp_dev=z)
    assert np.array_equal(to_np(c), to_np(q))
    return f, c, cop


@pytest.mark.parametrize("rows,D,side", [(256, 768, 0), (96, 768, 1), (40, 130, 0), (33, 130, 1), (64, 200, 2)])
def test_layernorm_codes(dev, rows, D, side):
    """LayerNormalization (with its residual Add) reading one operand as the
    uint8 bytes of a fused dequantize chain: the output and the (min, max)
    pairs equal, bit for bit, those of the fp32 kernel on the chain's fp32
    values (side 0: the normalized input, 1: the residual operand, 2: no
    residual). D = 130: the strided kernel (rows not 4-byte aligned)."""
    import torch
    rng = np.random.default_rng(rows * D + side)
    f, c, cop = _chain_pair(dev, rng, rows, D)
    f, c = f.reshape(rows, D), c.reshape(rows, D)
    gamma = to_dev(rng.uniform(0.5, 1.5, D).astype(np.float32), dev)
    beta = to_dev(rng.standard_normal(D).astype(np.float32), dev)
    r = None if side == 2 else to_dev(rng.standard_normal((rows, D)).astype(np.float32), dev)
    p0 = torch.full((2 * rows,), float("nan"), dtype=torch.float32, device=dev)
    p1 = torch.full((2 * rows,), float("nan"), dtype=torch.float32, device=dev)
    if side == 1:
        y0 = H.layernorm(r, gamma, beta, r=f, parts=p0)
        y1 = H.layernorm_codes((c, cop), gamma, beta, r=r, parts=p1)
    else:
        y0 = H.layernorm(f, gamma, beta, r=r, parts=p0)
        y1 = H.layernorm_codes((c, cop), gamma, beta, r=r, parts=p1)
    assert np.array_equal(to_np(y1).view(np.uint32), to_np(y0).view(np.uint32))
    assert np.array_equal(to_np(p1).view(np.uint32), to_np(p0).view(np.uint32))


@pytest.mark.parametrize("B,S", [(3, 128), (2, 77)])
def test_mha_codes(dev, B, S):
    """The fused attention reading q, k and v as the uint8 bytes of three
    fused dequantize chains: y and its (min, max) pairs equal, bit for bit,
    those of the fp32 kernel on the chains' fp32 values."""
    import ctypes as C
    import torch
    from nnr_amd import _lib
    heads, hidden = 12, 768
    rng = np.random.default_rng(B * S)
    fq, cq, oq = _chain_pair(dev, rng, S, hidden, batch=B)
    fk, ck, ok_ = _chain_pair(dev, rng, S, hidden, batch=B)
    fv, cv, ov = _chain_pair(dev, rng, S, hidden, batch=B)
    scale = 0.125
    pairs = 4 * B * heads
    p0 = torch.full((2 * pairs,), float("nan"), dtype=torch.float32, device=dev)
    p1 = torch.full((2 * pairs,), float("nan"), dtype=torch.float32, device=dev)
    y0 = torch.empty((B, S, hidden), dtype=torch.float32, device=dev)
    _lib.check(_lib.lib().nnrh_multihead_attention_f32(_lib.ptr(fq), _lib.ptr(fk), _lib.ptr(fv), _lib.ptr(y0), B, S,
                                                       hidden, heads, scale, _lib.ptr(p0), None, _lib.cur_stream()))
    y1 = H.multihead_attention_codes((cq, oq), (ck, ok_), (cv, ov), heads, scale, parts=p1)
    assert np.array_equal(to_np(y1).view(np.uint32), to_np(y0).view(np.uint32))
    assert np.array_equal(to_np(p1).view(np.uint32), to_np(p0).view(np.uint32))
    # other shapes are refused
    with pytest.raises(H.NnrHipError):
        H.multihead_attention_codes((cq, oq), (ck, ok_), (cv, ov), 6, scale)


def test_qmatmul_group_codes(dev):
    """A grouped launch of three fused-dequantize QLinearMatMuls in codes
    mode writes each member's uint8 QLinearMatMul bytes: those of the member
    run unfused."""
    import torch
    rng = np.random.default_rng(57)
    rows, k, n = 300, 96, 768
    a = to_dev(rng.integers(0, 256, (rows, k), dtype=np.uint8), dev)
    s = torch.tensor([0.0173], dtype=torch.float32, device=dev)
    z = torch.tensor([119], dtype=torch.uint8, device=dev)
    members, plain = [], []
    for i in range(3):
        b = rng.integers(-127, 128, (k, n), dtype=np.int8)
        bias = rng.standard_normal(n).astype(np.float32)
        ys, yz = [0.031, 0.047, 0.022][i], [121, 90, 140][i]
        op = H.QLinearMatMul(b, 1.0, 0, 0.004, 0, ys, yz, m=rows)
        op.fuse_dq_bias(ys, yz, bias)
        members.append(op)
        plain.append(to_np(H.QLinearMatMul(b, 1.0, 0, 0.004, 0, ys, yz, m=rows)(a, a_scale_dev=s, a_zp_dev=z)))
    g = H.QLinearMatMulGroup(members)
    g.set_codes_out()
    ys_ = [torch.empty((rows, n), dtype=torch.uint8, device=dev) for _ in range(3)]
    g(a, ys_, a_scale_dev=s, a_zp_dev=z)
    for i in range(3):
        assert np.array_equal(to_np(ys_[i]), plain[i]), i


def test_qmatmul_codes_errors(dev):
    """Codes mode needs the fused dequantize; the quantize call needs the
    pairs, then codes mode; a later fusion turns codes mode off; readers'
    parameters exist for chains without Gelu only."""
    import torch
    b = np.ones((64, 64), np.int8)
    op = H.QLinearMatMul(b, 1.0, 0, 0.004, 0, 0.03, 128, m=16)
    with pytest.raises(H.NnrHipError):   # no fused dequantize
        op.set_codes_out()
    with pytest.raises(H.NnrHipError):
        op.dq_params()
    op.fuse_dq_bias(0.03, 128, None)
    op.set_codes_out()
    c = torch.zeros((16, 64), dtype=torch.uint8, device=dev)
    with pytest.raises(H.NnrHipError):   # the quantizer needs the pairs
        op.dynamic_quantize_codes(c)
    parts = torch.zeros(2 * op.minmax_count(1), dtype=torch.float32, device=dev)
    op.set_minmax_out(parts)
    with pytest.raises(H.NnrHipError):   # ... set before codes mode
        op.dynamic_quantize_codes(c)
    op.set_codes_out()
    op.dynamic_quantize_codes(c)
    op.fuse_gelu()   # a later fusion turns codes mode off
    with pytest.raises(H.NnrHipError):
        op.dynamic_quantize_codes(c)
    with pytest.raises(H.NnrHipError):   # no parameters for readers of a Gelu chain
        op.dq_params()


@pytest.mark.parametrize("rows,n,device_q", [(8192 // 64, 768, True), (200, 136, True), (77, 64, False)])
def test_qmatmul_group(dev, rows, n, device_q):
    """Three fused-dequantize QLinearMatMuls reading the same A (different
    weights, scales, zero points, biases) as one grouped launch: every
    member's fp32 output equals its own launch bit for bit, with the
    activation quantization on the device (after DynamicQuantizeLinear) or
    on the host."""
    import torch
    rng = np.random.default_rng(rows + n)
    k = 96
    a = rng.integers(0, 256, (rows, k), dtype=np.uint8)
    a_s, a_z = np.float32(0.0173), 119
    members = []
    for i in range(3):
        b = rng.integers(-127, 128, (k, n), dtype=np.int8)
        bias = rng.standard_normal(n).astype(np.float32)
        ys, yz = [0.031, 0.047, 0.022][i], [121, 90, 140][i]
        if device_q:
            op = H.QLinearMatMul(b, 1.0, 0, [0.004, 0.0031, 0.0057][i], 0, ys, yz, m=rows)
        else:
            op = H.QLinearMatMul(b, a_s, a_z, [0.004, 0.0031, 0.0057][i], 0, ys, yz, m=rows)
        op.fuse_dq_bias(ys, yz, bias)
        members.append(op)
    ad = to_dev(a, dev)
    sd = torch.tensor([a_s], dtype=torch.float32, device=dev) if device_q else None
    zd = torch.tensor([a_z], dtype=torch.uint8, device=dev) if device_q else None
    refs = [to_np(op(ad, a_scale_dev=sd, a_zp_dev=zd)) for op in members]
    grp = H.QLinearMatMulGroup(members)
    for _ in range(2):
        ys = [torch.full((rows, n), float("nan"), dtype=torch.float32, device=dev) for _ in members]
        grp(ad, ys, a_scale_dev=sd, a_zp_dev=zd)
        for i, (y, ref) in enumerate(zip(ys, refs)):
            got = to_np(y)
            assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (i, np.count_nonzero(got != ref))
    # members that differ in shape are refused
    other = H.QLinearMatMul(rng.integers(-127, 128, (k, n + 64), dtype=np.int8), 1.0, 0, 0.004, 0, 0.03, 0, m=rows)
    other.fuse_dq_bias(0.03, 0, None)
    with pytest.raises(H.NnrHipError):
        H.QLinearMatMulGroup([members[0], other])


@pytest.mark.parametrize("rows,D,res,beta", [(37, 768, True, True), (9, 2048, True, False),
                                             (5, 102, True, True), (3, 3000, False, True),
                                             (130, 768, False, False)])
def test_add_layernorm(dev, rows, D, res, beta):
    """LayerNormalization of x (+ r), register-resident (D % 4 == 0, D <= 2048)
    and strided rows, against a float64 restatement of LayerNormalization.cpp;
    the (min, max) pairs are the exact extremes of each group of 4 output
    rows, and DynamicQuantizeLinear from them matches the two-pass one."""
    import torch
    rng = np.random.default_rng(rows * D)
    x = rng.normal(0.2, 1.3, (rows, D)).astype(np.float32)
    r = rng.normal(0, 0.7, (rows, D)).astype(np.float32) if res else None
    gm = rng.normal(1, 0.2, D).astype(np.float32)
    bt = rng.normal(0, 0.2, D).astype(np.float32) if beta else None
    parts = torch.full((2 * rows,), float("nan"), dtype=torch.float32, device=dev)
    y = H.layernorm(to_dev(x, dev), to_dev(gm, dev), None if bt is None else to_dev(bt, dev), 1e-5,
                    r=None if r is None else to_dev(r, dev), parts=parts)
    v = (x + r if res else x).astype(np.float64)   # the fp32 sum, as the Add stores it
    mu = v.mean(-1, keepdims=True)
    ref = (v - mu) / np.sqrt(((v - mu) ** 2).mean(-1, keepdims=True) + 1e-5) * gm
    if beta:
        ref = ref + bt
    got = to_np(y)
    np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-5)
    ng = (rows + 3) // 4
    pr = to_np(parts).reshape(rows, 2)
    assert np.isnan(pr[ng:]).all()   # one pair per 4 rows, nothing past them
    for i in range(ng):
        blk = got[4 * i:4 * i + 4]
        assert pr[i, 0] == min(0.0, blk.min()) and pr[i, 1] == max(0.0, blk.max()), i
    parts = parts[:2 * ng]
    q1, s1, z1 = H.dynamic_quantize_linear_parts(y, parts)
    q0, s0, z0 = H.dynamic_quantize_linear(y)
    assert to_np(s1)[0] == to_np(s0)[0] and to_np(z1)[0] == to_np(z0)[0]
    assert np.array_equal(to_np(q1), to_np(q0))


@pytest.mark.parametrize("n,nparts", [(6, 1), (1000, 7), (98304 * 3 + 5, 300), (4096 * 17, 6144)])
def test_dynamic_quantize_from_parts(dev, n, nparts):
    """DynamicQuantizeLinear from (min, max) pairs of any split of x (the
    extremes are exact in any order): bytes, scale and zero point equal the
    oracle's, including all-positive data (the 0 the operator adds)."""
    import torch
    rng = np.random.default_rng(n + nparts)
    for shift in (0.3, 4.0):
        x = (rng.normal(0, 1.5, n) + shift).astype(np.float32)
        cuts = np.sort(rng.integers(0, n + 1, nparts - 1)) if nparts > 1 else np.array([], int)
        pr = np.zeros((nparts, 2), np.float32)
        for i, c in enumerate(np.split(x, cuts)):
            if c.size:
                pr[i] = (min(0.0, c.min()), max(0.0, c.max()))
        y_ref, s_ref, z_ref = O.dynamic_quantize_linear(x)
        y, s, z = H.dynamic_quantize_linear_parts(to_dev(x, dev), to_dev(pr.reshape(-1), dev))
        assert to_np(s)[0] == np.float32(s_ref) and int(to_np(z)[0]) == z_ref
        assert np.array_equal(to_np(y), y_ref)


# ---------------------------------------------------------------------------
# QuantizeLinear fused into the first layer's input layout, DequantizeLinear
# fused into GlobalAveragePool

QFIRST_CASES = [
    # name, N, C, H, W, OC, k, stride, pads, q_scale, q_zp
    ("rn50_stem", 2, 3, 40, 36, 64, 7, 2, (3, 3, 3, 3), 1.0 / 255, 0),
    ("mbv2_stem", 3, 3, 33, 31, 32, 3, 2, (1, 1, 1, 1), 0.0237, 131),
    # 1*3*21*21 = 1323 elements: the last 11 take QuantizeLinear's divide tail
    ("tail_s1", 1, 3, 21, 21, 16, 3, 1, (1, 1, 1, 1), 0.0113, 17),
    # ResNet-50's stem at its real size: 4-row groups, 14 groups a strip
    ("rn50_stem_224", 2, 3, 224, 224, 64, 7, 2, (3, 3, 3, 3), 0.0187, 114),
    # one-kernel stem with 1*3*21*20 = 1260 elements (12 in the divide tail),
    # stride 1 (4-byte LDS fragment reads), several row groups a strip
    ("tail_w20", 1, 3, 21, 20, 16, 3, 1, (1, 1, 1, 1), 0.0113, 17),
    # output zero point 9 (the RQ-C clamp is not the saturating convert's),
    # fp32 input, even stride (8-byte fragment reads); then odd stride
    ("rn50_stem_yzp", 2, 3, 40, 36, 64, 7, 2, (3, 3, 3, 3), 0.0187, 114, 9),
    ("stem_s1_yzp", 2, 3, 20, 24, 32, 3, 1, (1, 1, 1, 1), 0.0213, 128, 3),
    # stride above the kernel height: each row group stages more new rows
    # (R * sH) than its span; the one-kernel stem takes it at width 64 ...
    ("stem_s4_k3", 2, 3, 30, 64, 32, 3, 4, (1, 1, 1, 1), 0.0213, 128),
    # ... and refuses it at width 640, where 5 staged fp32 rows (38,400 B)
    # overflow the staging area although a 3-row span (23,040 B) fits: the
    # multi-copy GEMM path runs it
    ("stem_s5_w640", 1, 3, 12, 640, 16, 3, 5, (1, 1, 1, 1), 0.0213, 128),
]

# the first-layer cases the one-kernel stem must take (True) or refuse
QFIRST_STEM = {"stem_s4_k3": True, "stem_s5_w640": False, "rn50_stem_224": True}


@pytest.mark.parametrize("case", QFIRST_CASES, ids=[c[0] for c in QFIRST_CASES])
def test_qconv_fused_quantize(dev, case):
    """fp32 NCHW input -> QuantizeLinear -> first-layer QLinearConv, with the
    quantization inside the conv's input layout kernel == oracle Q, then
    oracle conv."""
    import torch
    name, N, C, Hh, W, OC, k, st, pads, qs, qz = case[:11]
    yz = case[11] if len(case) > 11 else 0
    rng = np.random.default_rng(sum(name.encode()))
    x = (rng.standard_normal((N, C, Hh, W)) * 1.3).astype(np.float32)
    # exact ties of x / s land on .5 so the rounding mode is exercised
    x.reshape(-1)[::7] = (np.arange(x.size)[::7] % 40 - 20 + 0.5).astype(np.float32) * np.float32(qs)
    w = rng.integers(-127, 128, (OC, C, k, k), dtype=np.int8)
    kw = dict(stride=(st, st), pads=pads, y_nhwc=1, x_scale=qs, x_zp=qz, y_scale=0.05, y_zp=yz,
              w_scale=rng.uniform(0.001, 0.01, OC).astype(np.float32),
              bias=rng.integers(-4096, 4097, OC).astype(np.int32))
    xq = O.quantize_linear(x, qs, qz, np.uint8)
    ref, br = O.Conv(N, C, Hh, W, OC, k, k, **kw).run(xq, w)
    op = H.QLinearConv(N, C, Hh, W, w, **kw)
    assert H.BRANCH_NAMES[op.branch] == "FIRST"
    assert op.fuse_quantize(qs, qz)
    xd = to_dev(x, dev)
    from nnr_amd import _lib
    _lib.profile_reset()
    _lib.profile_enable(True)
    y = to_np(op.run_f32(xd))
    _lib.profile_enable(False)
    kernels = _lib.profile_read()
    _lib.profile_reset()
    mism = np.count_nonzero(y != ref)
    assert mism == 0, f"{mism} of {y.size} differ"
    if name in QFIRST_STEM:
        assert ("stem_conv" in kernels) == QFIRST_STEM[name], sorted(kernels)


QPOOL_CASES = [
    # name, N, C, H, W, OC, fp32 input (quantize fused), y_zp
    ("rn50_small_f32", 2, 3, 40, 36, 64, True, 0),
    # ResNet-50's stem at its real size: 14-group strips of pooled rows
    ("rn50_224_f32", 2, 3, 224, 224, 64, True, 0),
    # uint8 image, 4 channels, RQ-C clamp not the saturating convert's
    ("u8_c4_zp", 3, 4, 48, 64, 32, False, 5),
    # odd conv output height (the last pooled row's third conv row is
    # padding), 48 channels
    ("odd_rows_f32", 1, 3, 42, 36, 48, True, 9),
]


@pytest.mark.parametrize("case", QPOOL_CASES, ids=[c[0] for c in QPOOL_CASES])
def test_qconv_fused_maxpool(dev, case):
    """first-layer QLinearConv (7x7 / 2, pad 3) with the 3x3 / 2 / pad 1
    MaxPool after it in the same kernel == oracle conv, then oracle MaxPool."""
    name, N, C, Hh, W, OC, f32, yz = case
    rng = np.random.default_rng(sum(name.encode()))
    qs, qz = 0.0187, 114
    w = rng.integers(-127, 128, (OC, C, 7, 7), dtype=np.int8)
    kw = dict(stride=(2, 2), pads=(3, 3, 3, 3), y_nhwc=1, x_scale=qs, x_zp=qz, y_scale=0.05, y_zp=yz,
              w_scale=rng.uniform(0.001, 0.01, OC).astype(np.float32),
              bias=rng.integers(-4096, 4097, OC).astype(np.int32))
    if f32:
        x = (rng.standard_normal((N, C, Hh, W)) * 1.3).astype(np.float32)
        xq = O.quantize_linear(x, qs, qz, np.uint8)
    else:
        xq = rng.integers(0, 256, (N, C, Hh, W), dtype=np.uint8)
    conv, _ = O.Conv(N, C, Hh, W, OC, 7, 7, **kw).run(xq, w)
    oH, oW = conv.shape[1], conv.shape[2]
    pH, pW = (oH - 1) // 2 + 1, (oW - 1) // 2 + 1
    ref = O.maxpool_u8_nhwc(conv, 3, 3, 2, 2, 1, 1, pH, pW)
    op = H.QLinearConv(N, C, Hh, W, w, **kw)
    assert H.BRANCH_NAMES[op.branch] == "FIRST"
    if f32:
        assert op.fuse_quantize(qs, qz)
    assert op.fuse_maxpool()
    y = to_np(op.run_f32(to_dev(x, dev)) if f32 else op(to_dev(xq, dev)))
    assert y.shape == ref.shape
    mism = np.count_nonzero(y != ref)
    assert mism == 0, f"{mism} of {y.size} differ"


def test_qconv_fuse_maxpool_unsupported(dev):
    """other windows, and convolutions that are not the one-kernel first
    layer, are refused with the handle unchanged"""
    rng = np.random.default_rng(3)
    w = rng.integers(-127, 128, (64, 3, 7, 7), dtype=np.int8)
    kw = dict(stride=(2, 2), pads=(3, 3, 3, 3), y_nhwc=1, x_scale=0.02, x_zp=128, y_scale=0.05, y_zp=0,
              w_scale=np.full(64, 0.004, np.float32))
    op = H.QLinearConv(1, 3, 32, 32, w, **kw)
    assert not op.fuse_maxpool(k=(2, 2), s=(2, 2), pads=(0, 0, 0, 0))
    assert not op.fuse_maxpool(pads=(0, 0, 0, 0))
    # 7x7 at stride 8: a group's 32 new rows exceed its ring of one 31-row
    # span, so the pooled kernel refuses it (the plain stem still runs it)
    kw8 = dict(kw, stride=(8, 8))
    op8 = H.QLinearConv(1, 3, 64, 64, w, **kw8)
    assert H.BRANCH_NAMES[op8.branch] == "FIRST"
    assert not op8.fuse_maxpool()
    w2 = rng.integers(-127, 128, (64, 64, 1, 1), dtype=np.int8)
    op2 = H.QLinearConv(1, 64, 16, 16, w2, x_nhwc=1, y_nhwc=1, x_scale=0.02, x_zp=128, y_scale=0.05,
                        y_zp=0, w_scale=np.full(64, 0.004, np.float32))
    assert not op2.fuse_maxpool()


@pytest.mark.parametrize("nhwc,dt,C", [(1, np.uint8, 72), (0, np.uint8, 72), (1, np.int8, 72),
                                       (1, np.uint8, 70)])
def test_global_avgpool_dequant(dev, nhwc, dt, C):
    """DequantizeLinear + GlobalAveragePool in one pass == the two HIP ops
    run separately (bit for bit) and the oracle within fp32 tolerance; NHWC
    with C % 4 == 0 reads 4 channels a load, other C one byte."""
    import torch
    from nnr_amd import _lib
    rng = np.random.default_rng(41 + nhwc + C)
    N, Hh, W = 3, 7, 7
    info = (0, 256) if dt == np.uint8 else (-128, 128)
    shape = (N, Hh, W, C) if nhwc else (N, C, Hh, W)
    q = rng.integers(*info, shape, dtype=dt)
    s, z = 0.0371, (9 if dt == np.uint8 else -4)
    qd = to_dev(q, dev)
    y = torch.empty((N, C), dtype=torch.float32, device=dev)
    xdt = H.U8 if dt == np.uint8 else H.S8
    _lib.check(_lib.lib().nnrh_global_avgpool_dequant(_lib.ptr(qd), _lib.ptr(y), N, C, Hh * W, nhwc, xdt,
                                                      s, z, _lib.cur_stream()))
    f = torch.empty(shape, dtype=torch.float32, device=dev)
    _lib.check(_lib.lib().nnrh_dequantize_linear(_lib.ptr(qd), xdt, q.size, s, z, _lib.ptr(f),
                                                 _lib.cur_stream()))
    y2 = torch.empty((N, C), dtype=torch.float32, device=dev)
    _lib.check(_lib.lib().nnrh_global_avgpool_f32(_lib.ptr(f), _lib.ptr(y2), N, C, Hh * W, nhwc,
                                                  _lib.cur_stream()))
    got, sep = to_np(y), to_np(y2)
    assert np.array_equal(got.view(np.uint32), sep.view(np.uint32))
    deq = O.dequantize_linear(q, s, z)
    ref = deq.mean(axis=(1, 2) if nhwc else (2, 3), dtype=np.float64)
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-6)


# ---------------------------------------------------------------------------
# QLinearConv on 3-D tensors: the reference's exec_typed path (RQ-S)

CONV1D_CASES = [
    # name, N, C, W, OC, k, group, stride, dil, pads, act, w_zp, bias, y_zp
    ("u8_k3", 2, 16, 37, 24, 3, 1, 1, 1, (1, 1), np.uint8, (0,), True, 7),
    ("u8_wzp_s2_d2", 3, 12, 50, 9, 5, 3, 2, 2, (4, 3), np.uint8, (3,), True, 130),
    ("s8_pcz_nobias", 1, 8, 21, 8, 4, 2, 3, 1, (0, 2), np.int8, tuple(range(-4, 4)), False, -5),
    ("u8_depthwise", 2, 32, 64, 32, 7, 32, 1, 1, (3, 3), np.uint8, (0,), True, 0),
]


@pytest.mark.parametrize("case", CONV1D_CASES, ids=[c[0] for c in CONV1D_CASES])
def test_qconv1d(dev, case):
    name, N, C, W, OC, k, group, stride, dil, pads, act, wzp, bias, y_zp = case
    rng = np.random.default_rng(sum(name.encode()))
    info = np.iinfo(act)
    x = rng.integers(info.min, info.max + 1, (N, C, W), dtype=act)
    w = rng.integers(-127, 128, (OC, C // group, k), dtype=np.int8)
    b = rng.integers(-5000, 5000, OC).astype(np.int32) if bias else None
    ws = rng.uniform(0.001, 0.01, OC).astype(np.float32)
    kw = dict(group=group, pads=pads, act_dtype=act, x_scale=0.02, x_zp=int(info.min + 100),
              w_scale=ws, w_zp=wzp, y_scale=0.04, y_zp=y_zp, bias=b)
    ref, br = O.Conv1d(N, C, W, OC, k, stride=stride, dil=dil, **kw).run(x, w)
    assert br == 9
    op = H.QLinearConv(N, C, 1, W, w, stride=(1, stride), dil=(1, dil), spatial_dims=1,
                       **dict(kw, pads=(0, pads[0], 0, pads[1])))
    assert H.BRANCH_NAMES[op.branch] == "TYPED"
    xd = to_dev(x, dev)
    y = to_np(op(xd))
    assert y.shape == ref.shape
    mism = np.count_nonzero(y != ref)
    assert mism == 0, f"{mism} of {y.size} differ"


@pytest.mark.parametrize("B,S,hidden,heads,scale", [
    (3, 37, 96, 4, 0.2),          # head size 24: two strided GEMMs + scaled softmax
    (2, 160, 128, 2, 0.1),        # S > 128: the same
    (2, 128, 768, 12, 0.125),     # head size 64, S <= 128: the fused kernel
    (3, 50, 128, 2, 0.3),         # fused, padded key rows and idle waves
    (2, 1, 64, 1, 0.5),           # fused, one token
    (1, 97, 192, 3, -0.7),        # fused, negative scale
])
def test_multihead_attention_f32(dev, B, S, hidden, heads, scale):
    """MultiHeadAttention (heads read and written in place; the fused fp32
    MFMA kernel for head size 64 and S <= 128, two strided fp32 MFMA GEMMs
    over a (batch, head) grid and a scaled softmax otherwise) against float64
    numpy."""
    import torch
    from nnr_amd import _lib
    import ctypes as C
    rng = np.random.default_rng(B * 100 + S)
    q, k, v = (rng.standard_normal((B, S, hidden)).astype(np.float32) for _ in range(3))
    hd = hidden // heads
    split = lambda t: t.astype(np.float64).reshape(B, S, heads, hd).transpose(0, 2, 1, 3)
    sc = np.matmul(split(q), split(k).transpose(0, 1, 3, 2)) * np.float32(scale)
    e = np.exp(sc - sc.max(-1, keepdims=True))
    ref = np.matmul(e / e.sum(-1, keepdims=True), split(v)).transpose(0, 2, 1, 3).reshape(B, S, hidden)
    nbytes = C.c_size_t()
    _lib.check(_lib.lib().nnrh_multihead_attention_workspace(B, S, hidden, heads, C.byref(nbytes)))
    fused = hidden == 64 * heads and S <= 128
    # the fused kernel needs no workspace: NULL is passed
    assert (nbytes.value == 0) == fused
    wsp = None
    if not fused:
        ws = torch.empty(nbytes.value + 256, dtype=torch.uint8, device=dev)
        wsp = (ws.data_ptr() + 255) & ~255
    qd, kd, vd = to_dev(q, dev), to_dev(k, dev), to_dev(v, dev)
    y = torch.empty((B, S, hidden), dtype=torch.float32, device=dev)
    _lib.check(_lib.lib().nnrh_multihead_attention_f32(_lib.ptr(qd), _lib.ptr(kd), _lib.ptr(vd), _lib.ptr(y), B, S,
                                                       hidden, heads, scale, None, wsp, _lib.cur_stream()))
    np.testing.assert_allclose(to_np(y), ref, atol=1e-4, rtol=1e-4)
    pairs = C.c_int()
    _lib.check(_lib.lib().nnrh_multihead_attention_minmax_count(B, S, hidden, heads, C.byref(pairs)))
    if not fused:
        assert pairs.value == 0
        return
    # the fused kernel's (min, max) pairs: the same output bits, and a
    # DynamicQuantizeLinear from them equals the two-pass operator
    assert pairs.value == 4 * B * heads
    parts = torch.empty(2 * pairs.value, dtype=torch.float32, device=dev)
    y2 = torch.empty_like(y)
    _lib.check(_lib.lib().nnrh_multihead_attention_f32(_lib.ptr(qd), _lib.ptr(kd), _lib.ptr(vd), _lib.ptr(y2), B, S,
                                                       hidden, heads, scale, _lib.ptr(parts), None,
                                                       _lib.cur_stream()))
    yh = to_np(y2)
    assert np.array_equal(yh.view(np.uint32), to_np(y).view(np.uint32))
    pr = to_np(parts).reshape(-1, 2)
    assert pr[:, 0].min() == min(0.0, yh.min()) and pr[:, 1].max() == max(0.0, yh.max())
    yq, ys, yz = H.dynamic_quantize_linear_parts(y2, parts)
    y_ref, s_ref, z_ref = O.dynamic_quantize_linear(yh)
    assert to_np(ys)[0] == np.float32(s_ref) and int(to_np(yz)[0]) == z_ref
    assert np.array_equal(to_np(yq), y_ref.reshape(to_np(yq).shape))


@pytest.mark.parametrize("nhwc", [0, 1])
@pytest.mark.parametrize("f32_in", [False, True])
@pytest.mark.parametrize("N,C,Hh,W", [(2, 40, 13, 13), (1, 16, 4, 4), (3, 7, 5, 3),
                                      (2, 48, 8, 6),    # 16 elements a thread in both layouts
                                      (2, 64, 5, 7), (3, 32, 4, 8)])   # NHWC: a thread's channels fixed
def test_batchnorm_folded(dev, nhwc, f32_in, N, C, Hh, W):
    """Folded BatchNormalization (uint8 or fp32 in, uint8 out) bit-exact with
    the oracle: 16-wide bodies and scalar tails in both layouts, offsets that
    drive results below 0 and above 255, and exact .5 ties."""
    rng = np.random.default_rng(N * C + nhwc + f32_in)
    shape = (N, Hh, W, C) if nhwc else (N, C, Hh, W)
    if f32_in:
        x = (rng.normal(0, 60, shape) + 0.5 * rng.integers(0, 2, shape)).astype(np.float32)
    else:
        x = rng.integers(0, 256, shape, dtype=np.uint8)
    A = rng.uniform(-2.0, 2.0, C).astype(np.float32)
    A[::5] = 1.0
    B = rng.uniform(-300.0, 300.0, C).astype(np.float32)
    B[::3] = 0.5
    # x = 0 with B = -0.5: the result -0.5 rounds to -0, i.e. 0 (not the 255 a
    # negative value saturates to in the NHWC uint8 body)
    B[1::7] = -0.5
    x.reshape(-1)[::11] = 0
    if not f32_in and C > 2:
        # an infinite A (host folding with a tiny output scale): inf * 0 is
        # NaN, which the fast NHWC body must not see; other x saturate
        A[2] = np.inf
        ch = x[..., 2] if nhwc else x[:, 2]   # a view into x
        zero = np.zeros(ch.shape, bool)
        zero.reshape(-1)[::3] = True
        ch[zero] = 0
    ref = O.batchnorm_u8(x, A, B, nhwc=nhwc)
    y = H.batchnorm_u8(to_dev(x, dev), to_dev(A, dev), to_dev(B, dev), nhwc=nhwc)
    assert np.array_equal(to_np(y), ref)


@pytest.mark.parametrize("xdt,wdt,per_ch,s,p,d,group,shape", [
    (np.uint8, np.int8, False, (1, 1), (1, 1), (1, 1), 1, (32, 64, 56, 56)),   # cfg2's shape
    (np.uint8, np.int8, True, (1, 1), (1, 1), (1, 1), 1, (2, 16, 15, 15)),
    (np.uint8, np.uint8, True, (2, 1), (0, 2), (1, 2), 2, (3, 8, 9, 11)),
    (np.int8, np.int8, True, (1, 2), (2, 1), (2, 1), 4, (2, 8, 9, 11)),
    (np.int8, np.uint8, False, (2, 2), (0, 0), (1, 1), 1, (1, 3, 7, 7))])
def test_conv_integer(dev, xdt, wdt, per_ch, s, p, d, group, shape):
    """ConvInteger (im2col + the i8 MFMA MatMulInteger GEMM, per-channel
    weight zero points by a correction pass) bit-exact with the oracle's
    integer convolution, in the range where the reference's float path is
    exact (K * 255 * 255 < 2^24 here)."""
    rng = np.random.default_rng(sum(shape) + group)
    info = lambda t: (0, 256) if t == np.uint8 else (-128, 128)
    N, C, Hh, W = shape
    OC = 64 if C == 64 else 12
    x = rng.integers(*info(xdt), shape, dtype=xdt)
    w = rng.integers(*info(wdt), (OC, C // group, 3, 3), dtype=wdt)
    x_zp = 131 if xdt == np.uint8 else -3
    w_zp = rng.integers(*info(wdt), OC) if per_ch else (7 if wdt == np.uint8 else -2)
    ref = O.conv_integer(x, w, x_zp, w_zp, s, p, d, group)
    y = H.conv_integer(to_dev(x, dev), to_dev(w, dev), x_zp, w_zp, s, p, d, group)
    assert np.array_equal(to_np(y), ref)


@pytest.mark.parametrize("xdt,wdt,wz_mode,k,s,p,group,shape,OC", [
    # w_zp equal to the packed weights' shift: no patch-sum term
    (np.uint8, np.int8, "shift", 3, (1, 1), (1, 1), 1, (4, 64, 20, 20), 64),
    (np.uint8, np.uint8, "shift", 3, (1, 1), (1, 1), 1, (2, 32, 13, 13), 48),
    # groups of 64 channels (uniform tap walk), stride 2
    (np.uint8, np.int8, "pc", 3, (2, 2), (1, 1), 2, (2, 128, 17, 17), 128),
    (np.int8, np.int8, "pc", 5, (1, 1), (2, 2), 1, (2, 64, 14, 14), 96),
    (np.uint8, np.int8, "scalar", 7, (2, 2), (3, 3), 1, (2, 16, 30, 30), 64),
    (np.uint8, np.int8, "pc", 1, (1, 1), (0, 0), 1, (3, 256, 7, 7), 200),
    # K = 2304: 128-byte K stages
    (np.uint8, np.int8, "pc", 3, (1, 1), (1, 1), 1, (2, 256, 14, 14), 256)])
def test_conv_integer_shapes(dev, xdt, wdt, wz_mode, k, s, p, group, shape, OC):
    """ConvInteger on the implicit-GEMM kernel over kernel sizes, groups,
    strides and the three weight zero-point forms: bit-exact against the
    oracle's integer convolution."""
    rng = np.random.default_rng(sum(shape) + k * 7 + OC)
    info = lambda t: (0, 256) if t == np.uint8 else (-128, 128)
    N, C, Hh, W = shape
    x = rng.integers(*info(xdt), shape, dtype=xdt)
    w = rng.integers(*info(wdt), (OC, C // group, k, k), dtype=wdt)
    x_zp = 97 if xdt == np.uint8 else 5
    shift = 128 if wdt == np.uint8 else 0
    w_zp = {"shift": shift, "scalar": shift + 3, "pc": rng.integers(*info(wdt), OC)}[wz_mode]
    ref = O.conv_integer(x, w, x_zp, w_zp, s, p, (1, 1), group)
    y = H.conv_integer(to_dev(x, dev), to_dev(w, dev), x_zp, w_zp, s, p, (1, 1), group)
    assert np.array_equal(to_np(y), ref)


def test_conv_integer_handle_reuse(dev):
    """One handle, three calls in a row: per-channel zero points (patch sums
    computed), then the shift zero point (patch sums skipped, their
    coefficients 0) with other inputs, then per-channel again with another
    x_zp; each equals the oracle."""
    import ctypes as ct
    import torch
    from nnr_amd import _lib
    L = _lib.lib()
    rng = np.random.default_rng(77)
    N, C, HW, OC = 3, 64, 15, 80
    h = ct.c_void_p()
    _lib.check(L.nnrh_conv_integer_create(ct.byref(h), N, C, HW, HW, OC, 3, 3, 1, 1, 1, 1, 1, 1, HW, HW, 1,
                                          H.U8, H.S8))
    try:
        for x_zp, wz_mode in ((128, "pc"), (0, "shift"), (201, "pc")):
            x = rng.integers(0, 256, (N, C, HW, HW), dtype=np.uint8)
            w = rng.integers(-128, 128, (OC, C, 3, 3), dtype=np.int8)
            wz = rng.integers(-128, 128, OC).astype(np.int32) if wz_mode == "pc" else np.zeros(1, np.int32)
            xd, wd = to_dev(x, dev), to_dev(w, dev)
            wzd = to_dev(wz, dev) if wz.size > 1 else None
            y = torch.empty((N, OC, HW, HW), dtype=torch.int32, device=dev)
            _lib.check(L.nnrh_conv_integer_run(h, _lib.ptr(xd), _lib.ptr(wd), x_zp, 0,
                                               _lib.ptr(wzd) if wzd is not None else None, _lib.ptr(y),
                                               _lib.cur_stream()))
            ref = O.conv_integer(x, w, x_zp, wz if wz.size > 1 else 0, (1, 1), (1, 1), (1, 1), 1)
            assert np.array_equal(to_np(y), ref), (x_zp, wz_mode)
    finally:
        L.nnrh_conv_integer_destroy(h)


@pytest.mark.parametrize("m,n,k,batch,a_dt,b_dt,bias", [
    (40, 136, 96, 3, np.uint8, np.int8, True), (128, 768, 768, 2, np.uint8, np.int8, True),
    (70, 64, 48, 1, np.int8, np.int8, False), (33, 200, 64, 2, np.uint8, np.uint8, True)])
def test_matmul_integer_scaled(dev, m, n, k, batch, a_dt, b_dt, bias):
    """MatMulInteger (constant B, device zero point of A) -> Cast -> Mul by
    fl(a_scale * w_scale[n]) -> Add(bias[n]) in one kernel: the bits equal
    the oracle's exact int32 MatMulInteger followed by the same three IEEE
    binary32 operations (MatMulInteger.cpp:11-150, Cast.cpp, binary_math)."""
    import torch
    rng = np.random.default_rng(m * n + k)
    lo, hi = (0, 256) if a_dt == np.uint8 else (-128, 128)
    a = rng.integers(lo, hi, (batch, m, k), dtype=a_dt)
    b = rng.integers(-127, 128, (k, n), dtype=np.int8) if b_dt == np.int8 else \
        rng.integers(0, 256, (k, n), dtype=np.uint8)
    b_zp = 128 if b_dt == np.uint8 else 0
    ws = rng.uniform(1e-4, 2e-3, n).astype(np.float32)
    bi = rng.standard_normal(n).astype(np.float32) if bias else None
    a_s, a_zp = np.float32(0.0173), (91 if a_dt == np.uint8 else -7)
    op = H.MatMulIntegerScaled(b, ws, bi, m=m, a_dtype=a_dt, b_zp=b_zp)
    s = torch.tensor([a_s], dtype=torch.float32, device=dev)
    z = torch.tensor([a_zp], dtype=torch.uint8 if a_dt == np.uint8 else torch.int8, device=dev)
    y = to_np(op(to_dev(a, dev), a_scale_dev=s, a_zp_dev=z))
    acc = O.matmul_integer(a, b, a_zp, b_zp)
    ref = acc.astype(np.float32) * (a_s * ws).astype(np.float32)
    if bias:
        ref = (ref + bi).astype(np.float32)
    assert np.array_equal(y.view(np.uint32), ref.astype(np.float32).view(np.uint32))


def test_matmul_integer_scaled_group_gelu_minmax(dev):
    """Three scaled MatMulIntegers sharing A as one grouped launch, each
    member equal to its own launch bit for bit; and one with Gelu and
    min / max pairs whose DynamicQuantizeLinear matches the two-pass one."""
    import torch
    rng = np.random.default_rng(41)
    m, k, n, batch = 128, 192, 136, 2
    a = to_dev(rng.integers(0, 256, (batch, m, k), dtype=np.uint8), dev)
    s = torch.tensor([0.021], dtype=torch.float32, device=dev)
    z = torch.tensor([133], dtype=torch.uint8, device=dev)
    ops = [H.MatMulIntegerScaled(rng.integers(-127, 128, (k, n), dtype=np.int8),
                                 rng.uniform(1e-4, 2e-3, n).astype(np.float32),
                                 rng.standard_normal(n).astype(np.float32), m=m) for _ in range(3)]
    singles = [to_np(o(a, a_scale_dev=s, a_zp_dev=z)) for o in ops]
    grp = H.QLinearMatMulGroup(ops)
    ys = [torch.empty((batch, m, n), dtype=torch.float32, device=dev) for _ in ops]
    grp(a, ys, a_scale_dev=s, a_zp_dev=z)
    for y, ref in zip(ys, singles):
        assert np.array_equal(to_np(y).view(np.uint32), ref.view(np.uint32))
    g = H.MatMulIntegerScaled(rng.integers(-127, 128, (k, n), dtype=np.int8),
                              rng.uniform(1e-4, 2e-3, n).astype(np.float32),
                              rng.standard_normal(n).astype(np.float32), m=m)
    plain = to_dev(to_np(g(a, a_scale_dev=s, a_zp_dev=z)), dev)
    g_ref = torch.empty_like(plain)
    from nnr_amd import _lib
    _lib.check(_lib.lib().nnrh_gelu_f32(plain.data_ptr(), g_ref.data_ptr(), plain.numel(), _lib.cur_stream()))
    g.fuse_gelu()
    cnt = g.minmax_count(batch)
    parts = torch.full((2 * cnt,), float("nan"), dtype=torch.float32, device=dev)
    g.set_minmax_out(parts)
    y = g(a, a_scale_dev=s, a_zp_dev=z)
    assert np.array_equal(to_np(y).view(np.uint32), to_np(g_ref).view(np.uint32))
    q1, s1, z1 = H.dynamic_quantize_linear_parts(y, parts)
    q0, s0, z0 = H.dynamic_quantize_linear(y)
    assert to_np(s1)[0] == to_np(s0)[0] and to_np(z1)[0] == to_np(z0)[0]
    assert np.array_equal(to_np(q1), to_np(q0))

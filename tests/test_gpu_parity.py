"""Parity of the HIP kernels (libomt_hip.so, called through its C ABI) with the CPU oracle (oracle/omt_oracle.c).

Criterion: rel-L2 = ||dev - ref||_2 / ||ref||_2 <= 1e-4 per op for float32 results; int64
pooling indices must match exactly. Small shapes are checked against the full oracle; the BASELINE full-size shapes
(config 1 AlexNet conv1 at batch 16, config 5 ResNet-50 body layers at batch 256) against oracle values at sampled
output points plus the size-independent adjoint identity <conv(x,w), gy> = <x, dgrad(gy,w)> = <w, wgrad(x,gy)>.
Shape lists follow the reference's own check scripts (notes/scripts/conv_kinds_check.py:5,
notes/scripts/alexnet_ops_check.py:6-16, tools/gemm_bench.py:8-9).
"""

import numpy as np
import pytest
import torch

from oracle import oracle as orc

pytestmark = pytest.mark.gpu

TOL = 1e-4


def rnd(rng, *shape, scale=1.0):
    return (rng.standard_normal(shape) * scale).astype(np.float32)


def dev(a, cuda):
    return torch.from_numpy(np.ascontiguousarray(a)).to(cuda)


def host(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


@pytest.fixture(scope="module")
def ops():
    from omarchy_mac_torch import hip_ops
    return hip_ops


# ---- dense conv: full oracle at small sizes ----

CONV_SHAPES = [
    # (n, ci, co, h, w, ks, stride, pad)
    (4, 6, 10, 14, 14, 5, 1, 2), (4, 6, 10, 14, 14, 3, 1, 1), (4, 6, 10, 14, 14, 1, 1, 0),   # conv_kinds_check.py:5
    (3, 3, 8, 63, 63, 11, 4, 2), (3, 3, 6, 15, 15, 3, 2, 1), (3, 5, 7, 21, 21, 5, 2, 0),     # alexnet_ops_check.py:6
    (2, 64, 192, 27, 27, 5, 1, 2), (2, 192, 64, 13, 13, 3, 1, 1), (2, 32, 32, 16, 16, 3, 1, 1),  # gemm_bench.py:8-9
    (2, 3, 64, 224, 224, 11, 4, 2),                      # config 1 AlexNet conv1 at batch 2
    (2, 64, 64, 56, 56, 3, 1, 1), (2, 128, 128, 28, 28, 3, 1, 1),  # config 5 layers at batch 2
    (2, 256, 256, 14, 14, 3, 1, 1), (2, 512, 512, 7, 7, 3, 1, 1),
    (2, 64, 256, 56, 56, 1, 1, 0), (2, 256, 64, 56, 56, 1, 1, 0),
    (4, 3, 64, 64, 64, 7, 2, 3), (4, 64, 128, 16, 16, 3, 2, 1), (4, 64, 128, 16, 16, 1, 2, 0),  # ResNet-18 stem/down
    (4, 512, 512, 2, 2, 3, 1, 1),                        # ResNet-18 layer4 at 64x64 input
    (3, 7, 9, 13, 11, 3, 3, 2), (2, 5, 3, 9, 17, 4, 4, 4), (2, 17, 33, 10, 7, 2, 1, 0),   # ragged / odd
    # grad input as one super-pixel GEMM (C_in <= 4 at stride > 1): one input channel, 4 x 4 phases x 4 channels
    # (64 rows), stride 3 on a ragged non-square image
    (2, 1, 16, 19, 23, 3, 2, 1), (2, 4, 32, 18, 18, 4, 4, 0), (3, 3, 8, 17, 13, 5, 3, 2),
]


def _ids(s):
    return "n{}c{}o{}h{}w{}k{}s{}p{}".format(*s)


@pytest.mark.parametrize("shape", CONV_SHAPES, ids=_ids)
def test_conv_fwd_dgrad_wgrad(cuda, ops, shape):
    n, ci, co, h, w, ks, s, p = shape
    rng = np.random.default_rng(hash(shape) % 2**32)
    scale = (ci * ks * ks) ** -0.5
    x, wt, b = rnd(rng, n, ci, h, w), rnd(rng, co, ci, ks, ks, scale=scale), rnd(rng, co, scale=0.1)
    y = ops.conv2d(dev(x, cuda), dev(wt, cuda), dev(b, cuda), s, p)
    y_ref = orc.conv_fwd(x, wt, b, s, p)
    assert orc.rel_l2(host(y), y_ref) <= TOL
    gy = rnd(rng, *y_ref.shape)
    gx = ops.conv2d_dgrad(dev(gy, cuda), dev(wt, cuda), x.shape, s, p)
    assert orc.rel_l2(host(gx), orc.conv_dgrad(gy, wt, x.shape, s, p)) <= TOL
    gw = ops.conv2d_wgrad(dev(x, cuda), dev(gy, cuda), ks, s, p)
    assert orc.rel_l2(host(gw), orc.conv_wgrad(x, gy, ks, s, p)) <= TOL
    gb = ops.bias_grad(dev(gy, cuda))
    assert orc.rel_l2(host(gb), orc.bias_grad(gy)) <= TOL


@pytest.mark.parametrize("n,c,hw", [(32, 1000, 1), (7, 5, 3), (3, 300, 16), (2, 4, 17), (1, 1, 1), (5, 70, 9)])
def test_bias_grad(cuda, ops, n, c, hw):
    """Bias gradient: per-channel columns for planes of up to 16 elements (a linear layer's bias, hw = 1), one
    workgroup per channel above."""
    rng = np.random.default_rng(n * c + hw)
    gy = rnd(rng, n, c, hw, 1)
    assert orc.rel_l2(host(ops.bias_grad(dev(gy, cuda))), orc.bias_grad(gy)) <= TOL


@pytest.mark.parametrize("ks", range(1, 12))
def test_conv_geometry_sweep(cuda, ops, ks):
    """Every stride 1..4 and pad 0..ks the dense path accepts at this kernel size (csrc/conv.cpp:173), on tiny
    non-square images, including stride phases that no tap reaches."""
    rng = np.random.default_rng(ks)
    for s in range(1, 5):
        for p in range(0, ks + 1):
            for ih, iw in ((ks + 1, ks + 2), (ks + 5, ks + 3)):
                if ih + 2 * p < ks or iw + 2 * p < ks:
                    continue
                x, wt, b = rnd(rng, 2, 3, ih, iw), rnd(rng, 5, 3, ks, ks), rnd(rng, 5)
                case = (ks, s, p, ih, iw)
                y = ops.conv2d(dev(x, cuda), dev(wt, cuda), dev(b, cuda), s, p, relu=True)
                y_ref = orc.conv_fwd(x, wt, b, s, p, relu=True)
                assert orc.rel_l2(host(y), y_ref) <= TOL, case
                gy = rnd(rng, *y_ref.shape)
                gx = ops.conv2d_dgrad(dev(gy, cuda), dev(wt, cuda), x.shape, s, p)
                assert orc.rel_l2(host(gx), orc.conv_dgrad(gy, wt, x.shape, s, p)) <= TOL, case
                gw = ops.conv2d_wgrad(dev(x, cuda), dev(gy, cuda), ks, s, p)
                assert orc.rel_l2(host(gw), orc.conv_wgrad(x, gy, ks, s, p)) <= TOL, case


def test_memset_zero_kernel_and_graph_replay(cuda):
    """omt_memset_zero on odd sizes and unaligned addresses, eagerly and replayed from a captured HIP graph; the bytes
    around the range are untouched."""
    import ctypes
    from omarchy_mac_torch import _lib
    buf = torch.full((4096,), 0xAB, dtype=torch.uint8, device=cuda)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for off, n in ((0, 4096 - 16), (3, 1001), (16, 1), (5, 0)):
        buf.fill_(0xAB)
        _lib.check(_lib.L.omt_memset_zero(ctypes.c_void_p(buf.data_ptr() + off), n, stream), "omt_memset_zero")
        h = buf.cpu().numpy()
        assert (h[off:off + n] == 0).all() and (h[:off] == 0xAB).all() and (h[off + n:] == 0xAB).all(), (off, n)
    buf.fill_(0xAB)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        _lib.L.omt_memset_zero(ctypes.c_void_p(buf.data_ptr() + 7), 2000,
                               ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    for _ in range(3):
        buf.fill_(0xAB)
        g.replay()
        h = buf.cpu().numpy()
        assert (h[7:2007] == 0).all() and (h[:7] == 0xAB).all() and (h[2007:] == 0xAB).all()


PLAN_SHAPES = [
    (4, 512, 512, 2, 2, 3, 1, 1),   # ResNet-18 layer4 at 64x64: the cost model splits K
    (3, 64, 128, 9, 9, 3, 2, 1),    # stride 2: grad-input phases with different K
    (2, 24, 20, 7, 7, 3, 1, 1),     # channel-major K order (C % 16 != 0) with a K tail
    (2, 32, 48, 6, 5, 1, 1, 0),     # 1x1
]


@pytest.mark.parametrize("shape", PLAN_SHAPES, ids=_ids)
def test_conv_every_plan(cuda, ops, shape):
    """Every tile with 1, 2, 3 and 7 K slices (split-K partials summed by the slice reduce, bias + ReLU applied
    there) for forward and grad input; every wgrad tile with 1, 2 and 5 slices: all plans the tuner may pick."""
    n, ci, co, h, w, ks, s, p = shape
    rng = np.random.default_rng(sum(shape))
    x, wt, b = rnd(rng, n, ci, h, w), rnd(rng, co, ci, ks, ks, scale=(ci * ks * ks) ** -0.5), rnd(rng, co)
    y_ref = orc.conv_fwd(x, wt, b, s, p, relu=True)
    gy = rnd(rng, *y_ref.shape)
    gx_ref, gw_ref = orc.conv_dgrad(gy, wt, x.shape, s, p), orc.conv_wgrad(x, gy, ks, s, p)
    tx, tw, tb, tgy = dev(x, cuda), dev(wt, cuda), dev(b, cuda), dev(gy, cuda)
    try:
        for tile in range(ops.conv_num_tiles("fwd")):
            for slices in (1, 2, 3, 7):
                case = (tile, slices)
                ops.set_conv_plan("fwd", x.shape, wt.shape, s, p, tile, slices)
                ops.set_conv_plan("dgrad", x.shape, wt.shape, s, p, tile, slices)
                assert ops.conv_plan("fwd", x.shape, wt.shape, s, p)[0] == tile
                y = ops.conv2d(tx, tw, tb, s, p, relu=True)
                assert orc.rel_l2(host(y), y_ref) <= TOL, case
                gx = ops.conv2d_dgrad(tgy, tw, x.shape, s, p)
                assert orc.rel_l2(host(gx), gx_ref) <= TOL, case
        for tile in range(ops.conv_num_tiles("wgrad")):
            for slices in (1, 2, 5):
                ops.set_conv_plan("wgrad", x.shape, wt.shape, s, p, tile, slices)
                gw = ops.conv2d_wgrad(tx, tgy, ks, s, p)
                assert orc.rel_l2(host(gw), gw_ref) <= TOL, (tile, slices)
    finally:
        ops.clear_conv_plans()


STREAM_TILE = 13  # the 1x1 streaming tile (conv1x1_stream_kernel); tile 2 is the staged tile of the same shape
STREAM_SHAPES = [
    (32, 64, 256, 56),   # ResNet-50 1x1 expansion at 56^2: runs of 4 pixel tiles per workgroup
    (17, 32, 272, 46),   # P not a multiple of 64, N*H*W not a multiple of 128, a short last run
    (3, 48, 20, 10),     # one run, K of three blocks
    (17, 32, 272, 45),   # H*W % 4 != 0: the row epilogue does not apply and the plan runs as tile 2
]


@pytest.mark.parametrize("shape", STREAM_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_conv1x1_stream_tile_matches_staged_tile(cuda, ops, shape):
    """The streaming 1x1 kernel sums each output's K terms in the staged tile's order and stores whole float4 rows
    through LDS: forward (bias + ReLU) and grad input bit-identical to tile 2, and both against the oracle."""
    n, ci, co, h = shape
    rng = np.random.default_rng(sum(shape))
    x, wt, b = rnd(rng, n, ci, h, h), rnd(rng, co, ci, 1, 1, scale=ci ** -0.5), rnd(rng, co)
    gy = rnd(rng, n, co, h, h)
    tx, tw, tb, tgy = dev(x, cuda), dev(wt, cuda), dev(b, cuda), dev(gy, cuda)
    out = {}
    try:
        for tile in (STREAM_TILE, 2):
            ops.set_conv_plan("fwd", x.shape, wt.shape, 1, 0, tile, 1)
            ops.set_conv_plan("dgrad", x.shape, wt.shape, 1, 0, tile, 1)
            out[tile] = (ops.conv2d(tx, tw, tb, 1, 0, relu=True), ops.conv2d_dgrad(tgy, tw, x.shape, 1, 0))
    finally:
        ops.clear_conv_plans()
    assert torch.equal(out[STREAM_TILE][0], out[2][0]) and torch.equal(out[STREAM_TILE][1], out[2][1])
    assert orc.rel_l2(host(out[STREAM_TILE][0]), orc.conv_fwd(x, wt, b, 1, 0, relu=True)) <= TOL
    assert orc.rel_l2(host(out[STREAM_TILE][1]), orc.conv_dgrad(gy, wt, x.shape, 1, 0)) <= TOL


WST_TILES = (17, 18, 19)  # the filter-stationary 1x1 tiles (conv1x1_wst_kernel, K of 64 or 128)
WST_TILE = WST_TILES[0]
WST_SHAPES = [
    (32, 64, 256, 56),   # ResNet-50 1x1 expansion at 56^2: forward K = 64 (grad input K = 256 runs as the stream tile)
    (32, 256, 64, 56),   # its reduction: grad input K = 64
    (8, 128, 512, 28),   # expansion at 28^2: forward K = 128, four workgroups' channel groups per pixel tile
    (8, 512, 128, 28),   # grad input K = 128
    (5, 64, 272, 18),    # P not a multiple of 256 (a second channel group of 16), 1620 pixels: a partial last tile
    (3, 128, 40, 10),    # P below one workgroup's channels, grad input K = 40 (stream tile)
    (7, 64, 100, 15),    # H W % 4 != 0: runs as tile 2
]


@pytest.mark.parametrize("shape", WST_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_conv1x1_wst_tile_matches_staged_tile(cuda, ops, shape):
    """The filter-stationary 1x1 kernel (filter rows in registers, pixels as the MFMA rows, float4 stores from the
    accumulators) sums each output's K terms in the staged tiles' order: forward (bias + ReLU) and grad input of its
    three tile shapes bit-identical to tile 2 and to the stream tile, and against the oracle; where it does not apply
    it runs as the stream tile or tile 2."""
    n, ci, co, h = shape
    rng = np.random.default_rng(sum(shape) + 7)
    x, wt, b = rnd(rng, n, ci, h, h), rnd(rng, co, ci, 1, 1, scale=ci ** -0.5), rnd(rng, co)
    gy = rnd(rng, n, co, h, h)
    tx, tw, tb, tgy = dev(x, cuda), dev(wt, cuda), dev(b, cuda), dev(gy, cuda)
    out = {}
    try:
        for tile in WST_TILES + (STREAM_TILE, 2):
            ops.set_conv_plan("fwd", x.shape, wt.shape, 1, 0, tile, 1)
            ops.set_conv_plan("dgrad", x.shape, wt.shape, 1, 0, tile, 1)
            out[tile] = (ops.conv2d(tx, tw, tb, 1, 0, relu=True), ops.conv2d_dgrad(tgy, tw, x.shape, 1, 0))
    finally:
        ops.clear_conv_plans()
    for d in range(2):
        for tile in WST_TILES + (STREAM_TILE,):
            assert torch.equal(out[tile][d], out[2][d]), (tile, d)
    assert orc.rel_l2(host(out[WST_TILE][0]), orc.conv_fwd(x, wt, b, 1, 0, relu=True)) <= TOL
    assert orc.rel_l2(host(out[WST_TILE][1]), orc.conv_dgrad(gy, wt, x.shape, 1, 0)) <= TOL


def test_conv1x1_wst_tile_input_off_16_bytes(cuda, ops):
    """An input 4 bytes past a 16-byte boundary cannot take the filter-stationary tile's float4 loads: the plan runs
    as the stream tile, with the aligned input's results."""
    n, ci, co, h = 4, 64, 256, 12
    rng = np.random.default_rng(12)
    x, wt = rnd(rng, n, ci, h, h), rnd(rng, co, ci, 1, 1, scale=ci ** -0.5)
    tx, tw = dev(x, cuda), dev(wt, cuda)
    base = torch.zeros(x.size + 1, device=cuda)
    tx_off = base[1:].view(*x.shape)
    tx_off.copy_(tx)
    assert tx_off.data_ptr() % 16 == 4
    try:
        ops.set_conv_plan("fwd", x.shape, wt.shape, 1, 0, WST_TILE, 1)
        y_off, y = ops.conv2d(tx_off, tw), ops.conv2d(tx, tw)
    finally:
        ops.clear_conv_plans()
    assert torch.equal(y_off, y)
    assert orc.rel_l2(host(y), orc.conv_fwd(x, wt, None, 1, 0)) <= TOL


@pytest.mark.parametrize("tile", [0, 2, 5, 10, STREAM_TILE, WST_TILE])
def test_conv1x1_filter_used_in_place_off_16_bytes(cuda, ops, tile):
    """A 1x1 filter is read in place; from a view 4 bytes past a 16-byte boundary the tap-major tiles' 16-byte filter
    loads (4-byte alignment suffices) and the stream tile give the aligned filter's results, and a direct-to-LDS tile
    (tile 10) runs as its staged form."""
    n, ci, co, h = 4, 64, 96, 12
    rng = np.random.default_rng(11)
    x, wt = rnd(rng, n, ci, h, h), rnd(rng, co, ci, 1, 1, scale=ci ** -0.5)
    tx, tw = dev(x, cuda), dev(wt, cuda)
    base = torch.zeros(co * ci + 1, device=cuda)
    tw_off = base[1:].view(co, ci, 1, 1)
    tw_off.copy_(tw)
    assert tw_off.data_ptr() % 16 == 4
    try:
        ops.set_conv_plan("fwd", x.shape, wt.shape, 1, 0, tile, 1)
        y_off, y = ops.conv2d(tx, tw_off), ops.conv2d(tx, tw)
    finally:
        ops.clear_conv_plans()
    assert torch.equal(y_off, y)
    assert orc.rel_l2(host(y), orc.conv_fwd(x, wt, None, 1, 0)) <= TOL


@pytest.mark.parametrize("slices", [2, 3])
def test_super_pixel_dgrad_split_k(cuda, ops, slices):
    """The super-pixel grad input split over K: the slices' partials on the ceil(63 / 4)^2 grid are summed and
    scattered to the 63 x 63 image (AlexNet conv1's shape), for two tiles."""
    n, ci, co, h, ks, s, p = 3, 3, 8, 63, 11, 4, 2
    rng = np.random.default_rng(slices + 40)
    wt = rnd(rng, co, ci, ks, ks, scale=(ci * ks * ks) ** -0.5)
    o = (h + 2 * p - ks) // s + 1
    gy = rnd(rng, n, co, o, o)
    x_shape = (n, ci, h, h)
    ref = orc.conv_dgrad(gy, wt, x_shape, s, p)
    try:
        for tile in (4, 5):
            ops.set_conv_plan("dgrad", x_shape, wt.shape, s, p, tile, slices)
            gx = ops.conv2d_dgrad(dev(gy, cuda), dev(wt, cuda), x_shape, s, p)
            assert orc.rel_l2(host(gx), ref) <= TOL, tile
    finally:
        ops.clear_conv_plans()


BWD_SHAPES = [
    (4, 512, 512, 2, 2, 3, 1, 1),   # ResNet-18 layer4: both GEMMs split K
    (3, 64, 128, 9, 9, 3, 2, 1),    # stride 2: grad-input stride phases
    (2, 24, 20, 7, 7, 3, 1, 1),     # channel-major K order (C % 16 != 0)
    (2, 32, 48, 6, 5, 1, 1, 0),     # 1x1
    (3, 64, 96, 8, 6, 1, 1, 0),     # 1x1, planes of 48: the separate grad weight loads four pixels per lane (16 bytes)
    (2, 36, 50, 8, 8, 1, 1, 0),     # the same with rows (50 output channels) and columns (36) past a group of four
    (2, 64, 48, 12, 12, 3, 1, 1),   # 3x3 pad 1, tap-major grad weight over rows of 12
    (3, 32, 40, 4, 4, 3, 1, 1),     # rows of 4: every output's side taps reach the padding
    (2, 64, 64, 8, 8, 1, 2, 0),     # 1x1 stride 2: phases no tap reaches
    (2, 3, 64, 20, 20, 3, 2, 1),    # super-pixel grad input (3 channels, stride 2), split K summed by the scatter
    (16, 16, 24, 32, 32, 3, 1, 1),  # grad weight over 16384 pixels: 40 and 100 slices take the grouped slice sum
    (16, 3, 5, 32, 32, 3, 1, 1),    # the same with 135 outputs (scalar vectors, a partial last group)
]


@pytest.mark.parametrize("shape", BWD_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_conv_bwd_matches_separate_calls(cuda, ops, shape):
    """omt_conv_bwd (grad input and grad weight in one call; one launch when both plans use 64x64 tiles) is
    bit-identical to omt_conv_dgrad + omt_conv_wgrad under the same plans, and matches the oracle: dual and non-dual
    plan pairs, tap-major and channel-major grad input, split K on either side (grad weight up to 100 slices, whose
    sums go by groups of slices). On stride-1 1x1 layers whose planes are a multiple of 4 the separate grad weight loads
    four reduction pixels per lane and the one-launch kernel one: the same LDS layout, the same sums to the bit."""
    n, ci, co, h, w, ks, s, p = shape
    rng = np.random.default_rng(sum(shape) + 5)
    x, wt = rnd(rng, n, ci, h, w), rnd(rng, co, ci, ks, ks, scale=(ci * ks * ks) ** -0.5)
    oh, ow = (h + 2 * p - ks) // s + 1, (w + 2 * p - ks) // s + 1
    gy = rnd(rng, n, co, oh, ow)
    gx_ref, gw_ref = orc.conv_dgrad(gy, wt, x.shape, s, p), orc.conv_wgrad(x, gy, ks, s, p)
    tx, tw, tgy = dev(x, cuda), dev(wt, cuda), dev(gy, cuda)
    ng = ops.conv_num_tiles("dgrad") // 2
    try:
        for dtile in (5, 6, 5 + ng, 6 + ng, 0):
            for dslices in (1, 3):
                for wtile, wslices in ((2, 1), (2, 4), (0, 2), (2, 40), (2, 100)):
                    case = (dtile, dslices, wtile, wslices)
                    ops.set_conv_plan("dgrad", x.shape, wt.shape, s, p, dtile, dslices)
                    ops.set_conv_plan("wgrad", x.shape, wt.shape, s, p, wtile, wslices)
                    gx, gw = ops.conv2d_bwd(tx, tgy, tw, s, p)
                    gx1 = ops.conv2d_dgrad(tgy, tw, x.shape, s, p)
                    gw1 = ops.conv2d_wgrad(tx, tgy, ks, s, p)
                    torch.cuda.synchronize()
                    assert torch.equal(gx, gx1) and torch.equal(gw, gw1), case
                    assert orc.rel_l2(host(gx), gx_ref) <= TOL, case
                    assert orc.rel_l2(host(gw), gw_ref) <= TOL, case
    finally:
        ops.clear_conv_plans()


CONV_BN_BWD_SHAPES = [
    (4, 512, 512, 2, 2, 3, 1, 1),    # ResNet-18 layer4: channels of 16 elements, one vector per thread
    (8, 64, 64, 16, 16, 3, 1, 1),    # channels of 2048 elements: several vectors per thread
    (8, 64, 128, 16, 16, 3, 2, 1),   # stride 2: grad-input stride phases
    (32, 24, 20, 7, 7, 3, 1, 1),     # 7x7 planes (scalar vectors), channel-major K order
    (32, 64, 64, 16, 16, 1, 1, 0),   # 1x1, channels of exactly 8192 elements
]


@pytest.mark.parametrize("shape", CONV_BN_BWD_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_conv_bwd_into_bn_bwd_matches_separate_calls(cuda, ops, shape):
    """omt_conv_bwd_parts + omt_bn_bwd_parts (the BatchNorm backward summing the convolution's grad-input partials,
    the grad weight's slice sum on its extra workgroups or through omt_slice_sums) equal omt_conv_bwd followed by
    omt_bn_bwd_act / omt_bn_bwd_res: every output, bit for bit, under grad-input plans of 1 to 32 slices (past the
    fold limit the convolution sums them itself) and grad-weight plans of 1 to 40 slices, for activations none, ReLU
    and hardswish and a residual block's end with and without g2; the grad weight against the oracle."""
    from omarchy_mac_torch import _lib
    n, ci, co, h, w, ks, s, p = shape
    rng = np.random.default_rng(sum(shape) + 9)
    cx, cw = rnd(rng, n, ci, h, w), rnd(rng, co, ci, ks, ks, scale=(ci * ks * ks) ** -0.5)
    oh = (h + 2 * p - ks) // s + 1
    gy = rnd(rng, n, co, oh, (w + 2 * p - ks) // s + 1)
    x, a_in, g2 = rnd(rng, n, ci, h, w) * 2 + 1, rnd(rng, n, ci, h, w) * 3, rnd(rng, n, ci, h, w)
    gam, bet = rnd(rng, ci), rnd(rng, ci)
    tcx, tcw, tgy, tx, tg2, tgam = (dev(a, cuda) for a in (cx, cw, gy, x, g2, gam))
    y, sm, si = ops.batch_norm_train(tx, tgam, dev(bet, cuda), dev(rnd(rng, ci), cuda),
                                     dev(np.abs(rnd(rng, ci)) + 0.5, cuda), 0.1, 1e-5, True)
    relu_y = dev(np.maximum(a_in, 0), cuda)
    gw_ref = orc.conv_wgrad(cx, gy, ks, s, p)
    ng = ops.conv_num_tiles("dgrad") // 3
    folded = set()
    try:
        for dtile, dslices in ((5, 1), (5, 2), (5 + ng, 3), (6, 4), (0, 8), (5, 32)):
            for wtile, wslices in ((2, 1), (2, 4), (2, 40)):
                ops.set_conv_plan("dgrad", cx.shape, cw.shape, s, p, dtile, dslices)
                ops.set_conv_plan("wgrad", cx.shape, cw.shape, s, p, wtile, wslices)
                gx_c, gw_c = ops.conv2d_bwd(tcx, tgy, tcw, s, p)
                for act, res, with_g2 in ((_lib.OMT_ACT_NONE, False, False), (_lib.OMT_ACT_RELU, False, False),
                                          (_lib.OMT_ACT_HARDSWISH, False, False), (_lib.OMT_ACT_RELU, True, True),
                                          (_lib.OMT_ACT_RELU, True, False)):
                    case = (dtile, dslices, wtile, wslices, act, res, with_g2)
                    ain = relu_y if act == _lib.OMT_ACT_RELU else dev(a_in, cuda)
                    if res:
                        ref = ops.batch_norm_backward_res(gx_c, tg2 if with_g2 else None, tx, sm, si, tgam, ain)
                    else:
                        ref = ops.batch_norm_backward_act(gx_c, tx, act, ain, sm, si, tgam) + (None,)
                    out = ops.conv2d_bwd_bn(tcx, tgy, tcw, s, p, tx, sm, si, tgam, act, ain,
                                            tg2 if with_g2 else None, res, max_gx_slices=32 if dslices == 32 else 8,
                                            side_sum=wslices != 4)
                    if out[5] > 1:
                        folded.add(out[5])
                    assert torch.equal(out[0], gw_c), case
                    for a, b in zip(out[1:5], ref):
                        assert (a is None) == (b is None) and (a is None or torch.equal(a, b)), case
                assert orc.rel_l2(host(gw_c), gw_ref) <= TOL
    finally:
        ops.clear_conv_plans()
    assert folded, "no plan left its grad input unsummed"


def test_conv_split_k_bn_loader(cuda, ops):
    """The eval BN + ReLU input loader with K split over slices."""
    rng = np.random.default_rng(11)
    x, wt, b = rnd(rng, 2, 40, 4, 4), rnd(rng, 24, 40, 3, 3, scale=0.05), rnd(rng, 24)
    bn = (rnd(rng, 40), np.abs(rnd(rng, 40)) + 0.5, rnd(rng, 40), rnd(rng, 40))
    y_ref = orc.conv_fwd(x, wt, b, 1, 1, relu=True, bn=bn)
    try:
        for slices in (1, 4, 9):
            ops.set_conv_plan("fwd", x.shape, wt.shape, 1, 1, 5, slices)
            y = ops.conv2d(dev(x, cuda), dev(wt, cuda), dev(b, cuda), 1, 1, relu=True, bn=[dev(t, cuda) for t in bn])
            assert orc.rel_l2(host(y), y_ref) <= TOL, slices
    finally:
        ops.clear_conv_plans()


STATS_SHAPES = [
    (4, 16, 32, 20, 20, 3, 1, 1), (3, 24, 40, 33, 35, 3, 1, 1),   # column groups with a partial last one
    (4, 16, 24, 17, 17, 3, 2, 1), (2, 64, 256, 28, 28, 1, 1, 0),  # stride 2; 1x1 (the streaming tile applies)
    (2, 40, 72, 9, 9, 5, 1, 2),                                   # channels not a multiple of the tile's rows
]


@pytest.mark.parametrize("shape", STATS_SHAPES, ids=_ids)
def test_conv_epilogue_bn_statistics(cuda, ops, shape):
    """omt_conv_fwd_stats under every tile (tap-major, channel-major and in-place variants, the direct-to-LDS and
    streaming tiles) with one K slice: y bit-identical to omt_conv_fwd under the same plan; the epilogue's sums of y
    and y^2 per (output channel, group of the tile's wave columns) equal float64 sums of y over the same groups; then
    omt_bn_train_fwd_stats (with ReLU, and with a residual) matches the oracle's training BatchNorm of the conv output,
    running statistics included. A plan that splits K is refused."""
    n, ci, co, h, w, ks, s, p = shape
    rng = np.random.default_rng(sum(shape) + 77)
    x, wt = rnd(rng, n, ci, h, w), rnd(rng, co, ci, ks, ks, scale=(ci * ks * ks) ** -0.5)
    gam, bet, rm, rv = rnd(rng, co), rnd(rng, co), rnd(rng, co), np.abs(rnd(rng, co)) + 0.5
    tx, tw = dev(x, cuda), dev(wt, cuda)
    ntile = ops.conv_num_tiles("fwd")
    try:
        for tile in range(ntile):
            ops.set_conv_plan("fwd", x.shape, wt.shape, s, p, tile, 1)
            y, st, groups = ops.conv2d_stats(tx, tw, s, p)
            y1 = ops.conv2d(tx, tw, None, s, p)
            torch.cuda.synchronize()
            assert torch.equal(y, y1), tile
            yh = host(y).astype(np.float64)
            q = n * y.shape[2] * y.shape[3]
            wq = 32 if groups == -(-q // 32) else 64
            assert groups == -(-q // wq), (tile, groups, q)
            cols = yh.transpose(1, 0, 2, 3).reshape(co, q)  # GEMM columns: n-major output pixels
            pad = np.zeros((co, groups * wq))
            pad[:, :q] = cols
            g = pad.reshape(co, groups, wq)
            ref = np.stack([g.sum(2), (g * g).sum(2)], 2)
            got = host(st)
            assert np.allclose(got, ref, rtol=1e-12, atol=1e-12 * np.abs(ref).max()), tile
        y_ref_in = orc.conv_fwd(x, wt, None, s, p)
        r = rnd(rng, *y_ref_in.shape)
        for relu, res in ((True, None), (False, None), (True, r)):
            trm, trv = dev(rm, cuda), dev(rv, cuda)
            yb, sm, si = ops.batch_norm_train_stats(y, st, groups, dev(gam, cuda), dev(bet, cuda), trm, trv, 0.1,
                                                    1e-5, relu, None if res is None else dev(res, cuda))
            y_bn, m_ref, i_ref, nrm, nrv = orc.bn_train(y_ref_in, gam, bet, rm, rv, 0.1, 1e-5, False)
            want = y_bn + (0 if res is None else res)
            if relu:
                want = np.maximum(want, 0)
            case = (relu, res is not None)
            assert orc.rel_l2(host(yb), want) <= TOL, case
            assert orc.rel_l2(host(sm), m_ref) <= 1e-5 and orc.rel_l2(host(si), i_ref) <= 1e-5, case
            assert orc.rel_l2(host(trm), nrm) <= 1e-5 and orc.rel_l2(host(trv), nrv) <= 1e-5, case
        ops.set_conv_plan("fwd", x.shape, wt.shape, s, p, 5, 3)
        if ops.conv_plan("fwd", x.shape, wt.shape, s, p)[1] > 1:
            from omarchy_mac_torch import _lib
            with pytest.raises(_lib.Unsupported):
                ops.conv2d_stats(tx, tw, s, p)
    finally:
        ops.clear_conv_plans()


def test_conv_epilogue_bn_statistics_large_mean(cuda, ops):
    """The epilogue's statistics are unshifted float64 sums of y and y^2 (finalized with shift 0), where the
    three-pass path subtracts a per-channel shift first. Outputs whose mean is 75-90 times their spread (positive
    inputs, offset by 4, and positive filters, no padding) still normalize to the oracle's: fp32 squares of fp32
    values are exact in float64 and their sums lose ~1e-16 each, so E[y^2] - E[y]^2 keeps ~1e-16 * (mean / std)^2
    ~ 1e-12 relative, far under the test's bounds."""
    shape = (4, 16, 24, 12, 12, 3, 1, 0)  # no padding: every window sums all its taps
    n, ci, co, h, w, ks, s, p = shape
    rng = np.random.default_rng(2024)
    x = np.abs(rnd(rng, n, ci, h, w)) + 4.0  # every window sums many positive terms: mean >> spread
    wt = np.abs(rnd(rng, co, ci, ks, ks, scale=(ci * ks * ks) ** -0.5))
    gam, bet, rm, rv = rnd(rng, co), rnd(rng, co), rnd(rng, co), np.abs(rnd(rng, co)) + 0.5
    try:
        ops.set_conv_plan("fwd", x.shape, wt.shape, s, p, 5, 1)
        y, st, groups = ops.conv2d_stats(dev(x, cuda), dev(wt, cuda), s, p)
        y_in = orc.conv_fwd(x, wt, None, s, p)
        assert (y_in.mean(axis=(0, 2, 3)) / y_in.std(axis=(0, 2, 3))).min() > 50
        trm, trv = dev(rm, cuda), dev(rv, cuda)
        yb, sm, si = ops.batch_norm_train_stats(y, st, groups, dev(gam, cuda), dev(bet, cuda), trm, trv, 0.1, 1e-5,
                                                False, None)
        y_bn, m_ref, i_ref, nrm, nrv = orc.bn_train(y_in, gam, bet, rm, rv, 0.1, 1e-5, False)
        assert orc.rel_l2(host(yb), y_bn) <= TOL
        assert orc.rel_l2(host(sm), m_ref) <= 1e-6 and orc.rel_l2(host(si), i_ref) <= 1e-5
        assert orc.rel_l2(host(trm), nrm) <= 1e-6 and orc.rel_l2(host(trv), nrv) <= 1e-5
    finally:
        ops.clear_conv_plans()


def test_autotune_caches_a_plan(cuda, ops):
    """omt_conv_autotune times the candidates and caches the fastest; calls then use it (reference autotune,
    csrc/conv.cpp:116-155)."""
    rng = np.random.default_rng(12)
    shape = (8, 256, 256, 4, 4, 3, 1, 1)
    n, ci, co, h, w, ks, s, p = shape
    x, wt = rnd(rng, n, ci, h, w), rnd(rng, co, ci, ks, ks, scale=(ci * 9) ** -0.5)
    try:
        for d in ("fwd", "dgrad", "wgrad"):
            tile, slices = ops.autotune_conv(d, x.shape, wt.shape, s, p)
            assert ops.conv_plan(d, x.shape, wt.shape, s, p)[2]
            assert 0 <= tile < ops.conv_num_tiles(d) and slices >= 1
        assert len(ops.conv_plans()) == 3
        y = ops.conv2d(dev(x, cuda), dev(wt, cuda), None, s, p)
        y_ref = orc.conv_fwd(x, wt, None, s, p)
        assert orc.rel_l2(host(y), y_ref) <= TOL
        gy = rnd(rng, *y_ref.shape)
        gx = ops.conv2d_dgrad(dev(gy, cuda), dev(wt, cuda), x.shape, s, p)
        assert orc.rel_l2(host(gx), orc.conv_dgrad(gy, wt, x.shape, s, p)) <= TOL
        gw = ops.conv2d_wgrad(dev(x, cuda), dev(gy, cuda), ks, s, p)
        assert orc.rel_l2(host(gw), orc.conv_wgrad(x, gy, ks, s, p)) <= TOL
    finally:
        ops.clear_conv_plans()


def test_autotune_bwd_caches_a_pair(cuda, ops):
    """omt_conv_autotune_bwd tunes grad input and grad weight together (through omt_conv_bwd) and caches the pair;
    conv2d_bwd then uses it and matches the oracle."""
    rng = np.random.default_rng(13)
    for shape in ((32, 128, 128, 8, 8, 3, 1, 1), (8, 64, 128, 9, 9, 3, 2, 1)):
        n, ci, co, h, w, ks, s, p = shape
        x, wt = rnd(rng, n, ci, h, w), rnd(rng, co, ci, ks, ks, scale=(ci * ks * ks) ** -0.5)
        oh, ow = (h + 2 * p - ks) // s + 1, (w + 2 * p - ks) // s + 1
        gy = rnd(rng, n, co, oh, ow)
        try:
            (dt, ds), (wt_, ws) = ops.autotune_conv_bwd(x.shape, wt.shape, s, p)
            assert ops.conv_plan("dgrad", x.shape, wt.shape, s, p) == (dt, ds, True), shape
            assert ops.conv_plan("wgrad", x.shape, wt.shape, s, p) == (wt_, ws, True), shape
            gx, gw = ops.conv2d_bwd(dev(x, cuda), dev(gy, cuda), dev(wt, cuda), s, p)
            assert orc.rel_l2(host(gx), orc.conv_dgrad(gy, wt, x.shape, s, p)) <= TOL, shape
            assert orc.rel_l2(host(gw), orc.conv_wgrad(x, gy, ks, s, p)) <= TOL, shape
        finally:
            ops.clear_conv_plans()


def test_conv_bn_loader_and_relu_epilogue(cuda, ops):
    """Kind-3 loader (eval BN + ReLU of the input, padding stays zero) and the bias + ReLU epilogue."""
    rng = np.random.default_rng(7)
    for ks, s, p in ((1, 1, 0), (3, 1, 1), (3, 2, 1)):
        x, wt, b = rnd(rng, 3, 8, 12, 10), rnd(rng, 6, 8, ks, ks), rnd(rng, 6)
        bn = (rnd(rng, 8), np.abs(rnd(rng, 8)) + 0.5, rnd(rng, 8), rnd(rng, 8))
        y = ops.conv2d(dev(x, cuda), dev(wt, cuda), dev(b, cuda), s, p, relu=True, bn=[dev(t, cuda) for t in bn])
        y_ref = orc.conv_fwd(x, wt, b, s, p, relu=True, bn=bn)
        assert orc.rel_l2(host(y), y_ref) <= TOL, (ks, s, p)


def test_fold_bn(cuda, ops):
    rng = np.random.default_rng(3)
    cw, cb = rnd(rng, 16, 8, 3, 3), rnd(rng, 16)
    g, b, m, v = rnd(rng, 16), rnd(rng, 16), rnd(rng, 16), np.abs(rnd(rng, 16)) + 0.2
    for bias in (cb, None):
        fw, fb = ops.fold_bn(dev(cw, cuda), None if bias is None else dev(bias, cuda), *[dev(t, cuda) for t in (g, b, m, v)])
        rw, rb = orc.fold_bn(cw, bias, g, b, m, v)
        assert orc.rel_l2(host(fw), rw) <= 1e-6 and orc.rel_l2(host(fb), rb) <= 1e-6


# ---- dense conv at the BASELINE full sizes ----

FULL = [
    ("C1_alexnet_conv1", (16, 3, 64, 224, 224, 11, 4, 2)),
    ("C5_3x3_56", (256, 64, 64, 56, 56, 3, 1, 1)),
    ("C5_3x3_28", (256, 128, 128, 28, 28, 3, 1, 1)),
    ("C5_3x3_14", (256, 256, 256, 14, 14, 3, 1, 1)),
    ("C5_3x3_7", (256, 512, 512, 7, 7, 3, 1, 1)),
    ("C5_1x1_exp_56", (256, 64, 256, 56, 56, 1, 1, 0)),
    ("C5_1x1_red_56", (256, 256, 64, 56, 56, 1, 1, 0)),
    ("C5_1x1_exp_28", (256, 128, 512, 28, 28, 1, 1, 0)),
    ("C5_1x1_red_28", (256, 512, 128, 28, 28, 1, 1, 0)),
    ("C5_1x1_exp_14", (256, 256, 1024, 14, 14, 1, 1, 0)),
    ("C5_1x1_red_14", (256, 1024, 256, 14, 14, 1, 1, 0)),
    ("C5_1x1_exp_7", (256, 512, 2048, 7, 7, 1, 1, 0)),
    ("C5_1x1_red_7", (256, 2048, 512, 7, 7, 1, 1, 0)),
]
# (fwd, dgrad, wgrad) plans [tile, K slices] that bench.py's tuner picked for the C5 layers on an MI355X
BENCH_PLANS = {
    "C5_3x3_56": ([5, 1], [5, 1], [2, 114]), "C5_3x3_28": ([5, 1], [5, 1], [0, 112]),
    "C5_3x3_14": ([5, 1], [5, 1], [2, 16]), "C5_3x3_7": ([5, 4], [5, 4], [2, 4]),
    "C5_1x1_exp_56": ([17, 1], [2, 1], [2, 256]), "C5_1x1_red_56": ([2, 1], [17, 1], [0, 256]),
    "C5_1x1_exp_28": ([2, 1], [5, 1], [2, 64]), "C5_1x1_red_28": ([5, 1], [2, 1], [0, 64]),
    "C5_1x1_exp_14": ([5, 1], [5, 1], [0, 16]), "C5_1x1_red_14": ([5, 1], [5, 1], [2, 16]),
    "C5_1x1_exp_7": ([5, 1], [5, 1], [0, 4]), "C5_1x1_red_7": ([5, 1], [5, 1], [0, 4]),
}
FULL_CASES = [(name, shape, mode) for name, shape in FULL for mode in ("model", "tuned", "bench")
              if mode != "bench" or name in BENCH_PLANS]


def block_points(rng, rows, cols, to_flat, br=16, bc=32):
    """One random point in every br x bc block of a rows x cols GEMM output (every row tile of every plan is a
    multiple of 16 rows, every column tile and wave tile a multiple of 32 columns, so each output tile and each
    wave's part of it holds sampled points), mapped to flat tensor indices by to_flat(row, col)."""
    r0 = np.arange(0, rows, br)
    c0 = np.arange(0, cols, bc)
    rr, cc = np.meshgrid(r0, c0, indexing="ij")
    r = rr.ravel() + rng.integers(0, br, rr.size) % np.minimum(br, rows - rr.ravel())
    c = cc.ravel() + rng.integers(0, bc, cc.size) % np.minimum(bc, cols - cc.ravel())
    return to_flat(r.astype(np.int64), c.astype(np.int64))


def nchw_flat(n_ch, hw):
    """GEMM (channel row, pixel column q = n*hw + pix) -> flat index of an [N][n_ch][hw] tensor."""
    return lambda r, c: ((c // hw) * n_ch + r) * hw + c % hw


@pytest.mark.parametrize("name,shape,mode", FULL_CASES, ids=[f"{c[0]}-{c[2]}" for c in FULL_CASES])
def test_conv_full_size(cuda, ops, name, shape, mode):
    """A BASELINE full-size layer (config 1 at batch 16, config 5 at batch 256) under one plan per direction: the
    cost model's ("model"), the tuner's ("tuned", as bench.py tunes before timing) or the plans bench.py's tuner picked
    on an MI355X ("bench"). Checked against the oracle at sampled points stratified so that every 16 x 32 block of
    each direction's GEMM output holds a point (grad weight: in both K orders; grad input: every stride phase), which
    puts points in every output tile and every wave's part of it; every sampled output sums every K slice of a split
    plan. Plus the float64 adjoint identity <conv(x, w), gy> = <x, dgrad(gy, w)> = <w, wgrad(x, gy)>."""
    n, ci, co, h, w, ks, s, p = shape
    xs, ws = (n, ci, h, w), (co, ci, ks, ks)
    ops.clear_conv_plans()
    try:
        if mode == "tuned":
            for d in ("fwd", "dgrad", "wgrad"):
                ops.autotune_conv(d, xs, ws, s, p)
        elif mode == "bench":
            for d, plan in zip(("fwd", "dgrad", "wgrad"), BENCH_PLANS[name]):
                ops.set_conv_plan(d, xs, ws, s, p, *plan)
        plans = {d: ops.conv_plan(d, xs, ws, s, p)[:2] for d in ("fwd", "dgrad", "wgrad")}
        gen = torch.Generator(device=cuda).manual_seed(1)
        scale = (ci * ks * ks) ** -0.5
        x = torch.randn(xs, device=cuda, generator=gen)
        wt = torch.randn(ws, device=cuda, generator=gen) * scale
        b = torch.rand((co,), device=cuda, generator=gen) * 0.2 - 0.1
        y = ops.conv2d(x, wt, b, s, p)
        gy = torch.randn(y.shape, device=cuda, generator=gen) * scale
        gx = ops.conv2d_dgrad(gy, wt, xs, s, p)
        gw = ops.conv2d_wgrad(x, gy, ks, s, p)
        torch.cuda.synchronize()
    finally:
        ops.clear_conv_plans()
    case = (name, mode, plans)
    # adjoint identity in float64 (bias removed from y)
    yb = (y - b.view(1, -1, 1, 1)).double()
    a1 = (yb * gy.double()).sum().item()
    a2 = (x.double() * gx.double()).sum().item()
    a3 = (wt.double() * gw.double()).sum().item()
    norm = (yb.norm() * gy.double().norm()).item()
    assert abs(a1 - a2) <= 1e-5 * norm and abs(a1 - a3) <= 1e-5 * norm, (case, a1, a2, a3, norm)
    rng = np.random.default_rng(0)
    xh, wh, bh, gyh = host(x), host(wt), host(b), host(gy)
    oh, ow = y.shape[2], y.shape[3]
    # forward: rows = output channels, columns = n * oh * ow pixels
    pts = block_points(rng, co, n * oh * ow, nchw_flat(co, oh * ow))
    ref = orc.conv_fwd_points(xh, wh, pts, bh, s, p)
    assert orc.rel_l2(host(y).ravel()[pts], ref) <= TOL, case
    # grad input: rows = input channels, columns = n * h * w pixels, plus points on every stride phase
    pts = [block_points(rng, ci, n * h * w, nchw_flat(ci, h * w))]
    for py in range(s if s > 1 else 0):
        for px in range(s):
            ys = rng.integers(0, (h - py + s - 1) // s, 256) * s + py
            xs_ = rng.integers(0, (w - px + s - 1) // s, 256) * s + px
            pts.append(((rng.integers(0, n, 256) * ci + rng.integers(0, ci, 256)) * h + ys) * w + xs_)
    pts = np.concatenate(pts)
    ref = orc.conv_dgrad_points(gyh, wh, xs, pts, s, p)
    assert orc.rel_l2(host(gx).ravel()[pts], ref) <= TOL, case
    # grad weight: rows = output channels, columns = taps in the channel-major order (ci, ky, kx) and in the tap-major
    # order (ky, kx, ci), topped up with random points to at least 2000
    kk = ks * ks
    kcols = ci * kk
    cm = block_points(rng, co, kcols, lambda r, c: r * kcols + c)
    tm = block_points(rng, co, kcols, lambda r, c: r * kcols + (c % ci) * kk + c // ci)
    pts = np.concatenate([cm, tm, rng.integers(0, gw.numel(), max(0, 2000 - cm.size - tm.size))])
    ref = orc.conv_wgrad_points(xh, gyh, ks, pts, s, p)
    assert orc.rel_l2(host(gw).ravel()[pts], ref) <= TOL, case


def test_conv_batch_past_2gib_runs_in_chunks(cuda, ops):
    """A batch whose input and output pass 2 GiB (3 images of 876 MB: the kernels' offsets are 32-bit) runs on the
    HIP kernels as batch chunks of 2 images, then 1. Forward and grad input are bit-identical to the chunks convolved
    one by one; grad weight (alone and through the one-call backward) to the in-order sum of the chunks' filter
    gradients; the channels-last entry points likewise. Checked against the oracle at sampled points of every image
    and by the float64 adjoint identity."""
    n, c, h, ks, s, p = 3, 16, 3700, 3, 1, 1
    xs, ws = (n, c, h, h), (c, c, ks, ks)
    assert n * c * h * h * 4 >= 2**31 and 2 * c * h * h * 4 < 2**31
    chunks = ((0, 2), (2, 3))
    assert ops.conv_plan("fwd", xs, ws, s, p)[:2] == ops.conv_plan("fwd", (2, c, h, h), ws, s, p)[:2]
    gen = torch.Generator(device=cuda).manual_seed(3)
    x = torch.randn(xs, device=cuda, generator=gen)
    wt = torch.randn(ws, device=cuda, generator=gen) * (c * ks * ks) ** -0.5
    gy = torch.randn(xs, device=cuda, generator=gen)
    print(f"chunked conv {xs} x {ws}", flush=True)
    y = ops.conv2d(x, wt, None, s, p)
    gx = ops.conv2d_dgrad(gy, wt, xs, s, p)
    gw = ops.conv2d_wgrad(x, gy, ks, s, p)
    gx2, gw2 = ops.conv2d_bwd(x, gy, wt, s, p)
    gws = []
    for a, b in chunks:
        assert torch.equal(y[a:b], ops.conv2d(x[a:b], wt, None, s, p)), (a, b)
        assert torch.equal(gx[a:b], ops.conv2d_dgrad(gy[a:b], wt, (b - a, c, h, h), s, p)), (a, b)
        gws.append(ops.conv2d_wgrad(x[a:b], gy[a:b], ks, s, p))
    assert torch.equal(gw, gws[0] + gws[1])
    gxb, gwb = zip(*(ops.conv2d_bwd(x[a:b], gy[a:b], wt, s, p) for a, b in chunks))
    assert torch.equal(gx2, torch.cat(gxb)) and torch.equal(gw2, gwb[0] + gwb[1])
    # adjoint identity in float64
    a1 = (y.double() * gy.double()).sum().item()
    a2 = (x.double() * gx.double()).sum().item()
    a3 = (wt.double() * gw.double()).sum().item()
    norm = (y.double().norm() * gy.double().norm()).item()
    assert abs(a1 - a2) <= 1e-5 * norm and abs(a1 - a3) <= 1e-5 * norm, (a1, a2, a3, norm)
    # the oracle at points of every image (and the first and last element)
    rng = np.random.default_rng(7)
    xh, wh, gyh = host(x), host(wt), host(gy)
    per = c * h * h
    pts = np.concatenate([[0, n * per - 1], rng.integers(0, per, 3 * 256) + np.repeat(np.arange(n) * per, 256)])
    assert orc.rel_l2(host(y).ravel()[pts], orc.conv_fwd_points(xh, wh, pts, None, s, p)) <= TOL
    assert orc.rel_l2(host(gx).ravel()[pts], orc.conv_dgrad_points(gyh, wh, xs, pts, s, p)) <= TOL
    wpts = rng.integers(0, gw.numel(), 24)
    assert orc.rel_l2(host(gw).ravel()[wpts], orc.conv_wgrad_points(xh, gyh, ks, wpts, s, p)) <= TOL
    del xh, gyh
    # channels-last: chunks of the same images, against the NCHW results
    xc, wc, gyc = (t.contiguous(memory_format=torch.channels_last) for t in (x, wt, gy))
    del gx2, gxb
    yc = ops.conv2d_nhwc(xc, wc, None, s, p)
    gxc = ops.conv2d_dgrad_nhwc(gyc, wc, xs, s, p)
    gwc = ops.conv2d_wgrad_nhwc(xc, gyc, ks, s, p)
    gwcs = []
    for a, b in chunks:
        assert torch.equal(yc[a:b], ops.conv2d_nhwc(xc[a:b], wc, None, s, p)), (a, b)
        assert torch.equal(gxc[a:b], ops.conv2d_dgrad_nhwc(gyc[a:b], wc, (b - a, c, h, h), s, p)), (a, b)
        gwcs.append(ops.conv2d_wgrad_nhwc(xc[a:b], gyc[a:b], ks, s, p))
    assert torch.equal(gwc, gwcs[0] + gwcs[1])
    for got, ref in ((yc, y), (gxc, gx), (gwc, gw)):
        assert orc.rel_l2(host(got.contiguous()), host(ref)) <= TOL


# ---- depthwise ----

DW = [(3, 1, 1), (5, 1, 2), (7, 1, 3), (3, 2, 1), (5, 2, 0), (11, 4, 5), (2, 3, 1), (9, 1, 0)]


@pytest.mark.parametrize("ks,s,p", DW)
def test_depthwise(cuda, ops, ks, s, p):
    rng = np.random.default_rng(ks * 10 + s)
    c = 12
    x, wt, b = rnd(rng, 3, c, 17, 15), rnd(rng, c, 1, ks, ks), rnd(rng, c)
    y = ops.depthwise_conv2d(dev(x, cuda), dev(wt, cuda), dev(b, cuda), s, p)
    y_ref = orc.dw_fwd(x, wt, b, s, p)
    assert orc.rel_l2(host(y), y_ref) <= TOL
    gy = rnd(rng, *y_ref.shape)
    gx = ops.depthwise_dgrad(dev(gy, cuda), dev(wt, cuda), x.shape, s, p)
    assert orc.rel_l2(host(gx), orc.dw_dgrad(gy, wt, x.shape, s, p)) <= TOL
    gw = ops.depthwise_wgrad(dev(x, cuda), dev(gy, cuda), ks, s, p)
    assert orc.rel_l2(host(gw), orc.dw_wgrad(x, gy, ks, s, p)) <= TOL


@pytest.mark.parametrize("ks", [3, 5, 7])
def test_depthwise_tiled_stride1(cuda, ops, ks):
    """The stride-1 "same" kernels. Forward and grad input: rows of a multiple of 4 run register-blocked (56x56,
    13x300, 20x20, 70x400; rows of exactly 4, where both side runs are padding; 6 and 1 rows, a partial last row
    block); other planes of up to 256 elements run several images of a channel per workgroup (64 of 14x14 in batches
    of 20, leaving a short last batch), larger ones LDS-tiled in row chunks (72x65, 70x41). Grad weight stages several
    small planes per batch: image counts that leave a short last batch (13 images of 9x9 in batches of 6) and a short
    last group (37 of 20x20 in batches of 5, 64 of 14x14 in batches of up to 10). The eval BN + ReLU loader on every
    forward kernel."""
    rng = np.random.default_rng(ks)
    p = ks // 2
    for (n, c, h, w) in ((2, 3, 1, 1), (3, 4, 2, 3), (2, 5, 7, 7), (2, 3, 11, 9), (2, 4, 56, 56), (1, 3, 13, 300),
                         (1, 2, 70, 41), (13, 3, 9, 9), (37, 2, 20, 20), (64, 2, 14, 14), (1, 2, 72, 65),
                         (1, 1, 70, 400), (2, 3, 5, 4), (3, 2, 6, 8), (1, 2, 1, 12)):
        case = (ks, n, c, h, w)
        x, wt, b = rnd(rng, n, c, h, w), rnd(rng, c, 1, ks, ks), rnd(rng, c)
        y = ops.depthwise_conv2d(dev(x, cuda), dev(wt, cuda), dev(b, cuda), 1, p)
        assert orc.rel_l2(host(y), orc.dw_fwd(x, wt, b, 1, p)) <= TOL, case
        gy = rnd(rng, n, c, h, w)
        gx = ops.depthwise_dgrad(dev(gy, cuda), dev(wt, cuda), x.shape, 1, p)
        assert orc.rel_l2(host(gx), orc.dw_dgrad(gy, wt, x.shape, 1, p)) <= TOL, case
        gw = ops.depthwise_wgrad(dev(x, cuda), dev(gy, cuda), ks, 1, p)
        assert orc.rel_l2(host(gw), orc.dw_wgrad(x, gy, ks, 1, p)) <= TOL, case
    for shape in ((2, 6, 60, 33), (3, 5, 12, 9), (1, 3, 80, 70), (2, 4, 28, 28), (3, 2, 5, 4)):
        x, wt = rnd(rng, *shape), rnd(rng, shape[1], 1, ks, ks)
        c = shape[1]
        bn = (rnd(rng, c), np.abs(rnd(rng, c)) + 0.5, rnd(rng, c), rnd(rng, c))
        y = ops.depthwise_conv2d(dev(x, cuda), dev(wt, cuda), None, 1, p, bn=[dev(t, cuda) for t in bn])
        assert orc.rel_l2(host(y), orc.dw_fwd(x, wt, None, 1, p, bn=bn)) <= TOL, shape


@pytest.mark.parametrize("ks", [3, 5, 7])
def test_depthwise_wgrad_image_slices(cuda, ops, ks):
    """Grad weight over image slices summed in slice order by a second launch: 13 images in 13 slices, 27 in 27
    (256-thread workgroups), 4 in 2 slices of 1024-thread workgroups (4- or 2-row blocks; the slice count capped by
    the 640 channels); one slice at 1024 threads (1 x 1280 x 128^2) and at 256 (5 x 64 x 12^2). A workspace left
    full of other bytes, results bit-identical across calls and across replays of a captured graph with other
    grad-weight calls in between."""
    import ctypes
    from omarchy_mac_torch import _lib
    rng = np.random.default_rng(100 + ks)
    p = ks // 2
    stream = lambda: ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)  # noqa: E731
    for (n, c, h, w), split in (((13, 16, 64, 64), 13), ((27, 24, 64, 64), 27), ((4, 640, 96, 96), 2),
                                ((1, 1280, 128, 128), 1), ((5, 64, 12, 12), 1)):
        x, gy = rnd(rng, n, c, h, w), rnd(rng, n, c, h, w)
        ref = orc.dw_wgrad(x, gy, ks, 1, p)
        tx, tgy = dev(x, cuda), dev(gy, cuda)
        g = _lib.conv_geo(n, c, c, h, w, ks, 1, p)
        nb = _lib.L.omt_dw_wgrad_workspace(ctypes.byref(g))
        assert nb == (0 if split == 1 else split * c * ks * ks * 4), ("slices", n, c, h, w, nb)
        outs = []
        for fill in (0xFF, 0x00, 0x3F):
            ws = torch.full((max(nb, 1),), fill, dtype=torch.uint8, device=cuda)
            gw = torch.empty((c, 1, ks, ks), device=cuda)
            _lib.check(_lib.L.omt_dw_wgrad(ctypes.byref(g), ctypes.c_void_p(tx.data_ptr()),
                                           ctypes.c_void_p(tgy.data_ptr()), ctypes.c_void_p(gw.data_ptr()),
                                           ctypes.c_void_p(ws.data_ptr()), nb, stream()), "omt_dw_wgrad")
            outs.append(host(gw))
        assert orc.rel_l2(outs[0], ref) <= TOL, (ks, n, c, h, w)
        assert all(np.array_equal(o, outs[0]) for o in outs[1:])
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            gw_g = ops.depthwise_wgrad(tx, tgy, ks, 1, p)
        for _ in range(3):
            graph.replay()
            torch.cuda.synchronize()
            assert np.array_equal(host(gw_g), outs[0]), (ks, n, c, h, w)
            other = ops.depthwise_wgrad(tgy, tx, ks, 1, p)  # an eager grad-weight call in between
            torch.cuda.synchronize()
            assert orc.rel_l2(host(other), orc.dw_wgrad(gy, x, ks, 1, p)) <= TOL


def test_depthwise_bn_loader_and_mobilenet_size(cuda, ops):
    rng = np.random.default_rng(5)
    c = 8
    x, wt = rnd(rng, 2, c, 11, 11), rnd(rng, c, 1, 3, 3)
    bn = (rnd(rng, c), np.abs(rnd(rng, c)) + 0.5, rnd(rng, c), rnd(rng, c))
    y = ops.depthwise_conv2d(dev(x, cuda), dev(wt, cuda), None, 1, 1, bn=[dev(t, cuda) for t in bn])
    assert orc.rel_l2(host(y), orc.dw_fwd(x, wt, None, 1, 1, bn=bn)) <= TOL
    # a MobileNetV3-Small-style layer at batch 32 (config 4): dw 5x5 over 96 channels at 28x28
    x, wt = rnd(rng, 32, 96, 28, 28), rnd(rng, 96, 1, 5, 5)
    y = ops.depthwise_conv2d(dev(x, cuda), dev(wt, cuda), None, 1, 2)
    y_ref = orc.dw_fwd(x, wt, None, 1, 2)
    assert orc.rel_l2(host(y), y_ref) <= TOL
    gy = rnd(rng, *y_ref.shape)
    gw = ops.depthwise_wgrad(dev(x, cuda), dev(gy, cuda), 5, 1, 2)
    assert orc.rel_l2(host(gw), orc.dw_wgrad(x, gy, 5, 1, 2)) <= TOL


# ---- batch norm ----

@pytest.mark.parametrize("n,c,h,w", [(4, 6, 5, 7), (16, 8, 4, 4), (2, 3, 1, 1), (9, 4, 3, 3), (128, 32, 32, 32),
                                     (32, 64, 16, 16), (32, 512, 2, 2), (1, 16, 57, 31), (3, 5, 37, 41),
                                     (64, 16, 28, 28), (8, 3, 7, 9), (9, 5, 33, 35), (4, 8, 56, 56),
                                     (64, 64, 64, 64), (64, 64, 63, 65), (32, 96, 7, 7), (8, 16, 16, 16),
                                     (9, 12, 15, 15), (2, 8, 33, 32), (32, 24, 28, 28), (32, 8, 32, 32),
                                     (7, 3, 64, 64), (29, 4, 31, 33)])
@pytest.mark.parametrize("relu", [False, True])
def test_batch_norm_train_and_backward(cuda, ops, n, c, h, w, relu):
    rng = np.random.default_rng(n * 1000 + c)
    x = rnd(rng, n, c, h, w) * 3 + 5  # large mean: the shifted statistics must stay accurate
    g, b, rm, rv = rnd(rng, c), rnd(rng, c), rnd(rng, c), np.abs(rnd(rng, c)) + 0.5
    trm, trv = dev(rm, cuda), dev(rv, cuda)
    y, sm, si = ops.batch_norm_train(dev(x, cuda), dev(g, cuda), dev(b, cuda), trm, trv, 0.1, 1e-5, relu)
    y_ref, m_ref, i_ref, nrm, nrv = orc.bn_train(x, g, b, rm, rv, 0.1, 1e-5, relu)
    assert orc.rel_l2(host(y), y_ref) <= TOL
    assert orc.rel_l2(host(sm), m_ref) <= 1e-6 and orc.rel_l2(host(si), i_ref) <= 1e-5
    assert orc.rel_l2(host(trm), nrm) <= 1e-6 and orc.rel_l2(host(trv), nrv) <= 1e-6
    gy = rnd(rng, n, c, h, w)
    gx, dg, db = ops.batch_norm_backward(dev(gy, cuda), dev(x, cuda), sm, si, dev(g, cuda),
                                         relu_y=y if relu else None)
    gx_ref, dg_ref, db_ref = orc.bn_bwd(gy, x, host(sm), host(si), g, relu_y=host(y) if relu else None)
    # gx is a difference of near-equal terms (exactly 0 when m = 2), so its error is normalized by the gradient scale
    gz = gy * (y_ref > 0) if relu else gy
    scale = np.linalg.norm(gz.astype(np.float64)) * np.abs(g * i_ref).max()
    assert np.linalg.norm(host(gx).astype(np.float64) - gx_ref) <= TOL * max(scale, 1e-30)
    assert orc.rel_l2(host(dg), dg_ref) <= TOL and orc.rel_l2(host(db), db_ref) <= TOL


@pytest.mark.parametrize("n,c,h,w", [(32, 64, 4, 4), (8, 3, 7, 9), (16, 8, 32, 32), (4, 6, 5, 7), (1024, 2, 3, 3),
                                     (5, 3, 45, 41)])
@pytest.mark.parametrize("with_g2", [True, False])
def test_batch_norm_backward_res(cuda, ops, n, c, h, w, with_g2):
    """omt_bn_bwd_res: gz = (g + g2) masked by y > 0 returned exactly as the masked sum, and BatchNorm's grads of gz
    against the oracle's backward of that gz, on the one-launch (<= 8192 elements per channel) and split paths, with
    and without grad input."""
    rng = np.random.default_rng(n + c + h)
    x = rnd(rng, n, c, h, w) * 2 + 1
    gam, bet, rm, rv = rnd(rng, c), rnd(rng, c), rnd(rng, c), np.abs(rnd(rng, c)) + 0.5
    y, sm, si = ops.batch_norm_train(dev(x, cuda), dev(gam, cuda), dev(bet, cuda), dev(rm, cuda), dev(rv, cuda), 0.1,
                                     1e-5, True)
    g, g2 = rnd(rng, n, c, h, w), rnd(rng, n, c, h, w) if with_g2 else None
    for mask in ((True, True, True), (False, True, True)):
        gx, dg, db, gz = ops.batch_norm_backward_res(dev(g, cuda), None if g2 is None else dev(g2, cuda), dev(x, cuda),
                                                     sm, si, dev(gam, cuda), y, mask)
        gsum = g + g2 if with_g2 else g
        gz_ref = np.where(host(y) > 0, gsum, np.float32(0)).astype(np.float32)
        assert np.array_equal(host(gz), gz_ref), mask
        gx_ref, dg_ref, db_ref = orc.bn_bwd(gz_ref, x, host(sm), host(si), gam)
        assert orc.rel_l2(host(dg), dg_ref) <= TOL and orc.rel_l2(host(db), db_ref) <= TOL
        if mask[0]:
            scale = np.linalg.norm(gz_ref.astype(np.float64)) * np.abs(gam * host(si)).max()
            assert np.linalg.norm(host(gx).astype(np.float64) - gx_ref) <= TOL * max(scale, 1e-30)
        else:
            assert gx is None


@pytest.mark.parametrize("n,c,h,w", [(32, 16, 16, 16), (8, 24, 56, 56), (64, 8, 20, 20), (3, 5, 37, 41),
                                     (32, 96, 7, 7)])
def test_batch_norm_hardswish(cuda, ops, n, c, h, w):
    """BatchNorm with hardswish fused into its apply (MobileNetV3's BatchNorms): z = the BatchNorm output against the
    oracle, y = hardswish(z) as PyTorch CPU computes it from z, and the backward through the hardswish (gradient from z,
    0 at and below -3, unchanged at and above 3) against PyTorch CPU's hardswish_backward followed by the oracle's
    BatchNorm backward; on the one-launch, two-pass and flat-apply paths, the same via ReLU as act 1."""
    from omarchy_mac_torch import _lib
    rng = np.random.default_rng(n + 7 * c + h)
    x = rnd(rng, n, c, h, w) * 2 + 1
    gam, bet, rm, rv = rnd(rng, c) * 2, rnd(rng, c), rnd(rng, c), np.abs(rnd(rng, c)) + 0.5
    tx, tg = dev(x, cuda), dev(gam, cuda)
    z_ref = orc.bn_train(x, gam, bet, rm, rv, 0.1, 1e-5)[0]
    gy = rnd(rng, n, c, h, w)
    for act in (_lib.OMT_ACT_HARDSWISH, _lib.OMT_ACT_RELU):
        y, sm, si, z = ops.batch_norm_train(tx, tg, dev(bet, cuda), dev(rm, cuda), dev(rv, cuda), 0.1, 1e-5, act=act,
                                            return_z=True)
        assert orc.rel_l2(host(z), z_ref) <= TOL
        tz = torch.from_numpy(host(z))
        y_ref = torch.nn.functional.hardswish(tz) if act == _lib.OMT_ACT_HARDSWISH else torch.relu(tz)
        yd = torch.from_numpy(host(y))
        assert torch.equal(yd, y_ref) or orc.rel_l2(yd.numpy(), y_ref.numpy()) <= 1e-6, act
        gx, dg, db = ops.batch_norm_backward_act(dev(gy, cuda), tx, act, z if act == _lib.OMT_ACT_HARDSWISH else y,
                                                 sm, si, tg)
        gz = (torch.ops.aten.hardswish_backward(torch.from_numpy(gy), tz) if act == _lib.OMT_ACT_HARDSWISH
              else torch.ops.aten.threshold_backward(torch.from_numpy(gy), y_ref, 0)).numpy()
        gx_ref, dg_ref, db_ref = orc.bn_bwd(gz, x, host(sm), host(si), gam)
        assert orc.rel_l2(host(dg), dg_ref) <= TOL and orc.rel_l2(host(db), db_ref) <= TOL
        scale = np.linalg.norm(gz.astype(np.float64)) * np.abs(gam * host(si)).max()
        assert np.linalg.norm(host(gx).astype(np.float64) - gx_ref) <= TOL * max(scale, 1e-30)


BN_POOL = [
    ((32, 16, 16, 16), 2, 2, 0), ((8, 24, 7, 7), 2, 2, 0), ((16, 8, 12, 12), 3, 2, 1), ((2, 4, 64, 64), 3, 2, 1),
    ((32, 64, 32, 32), 3, 2, 1), ((128, 32, 32, 32), 2, 2, 0), ((4, 8, 45, 37), 3, 2, 1), ((2, 3, 150, 150), 3, 2, 0),
    ((3, 5, 9, 11), 3, 3, 1),
]


@pytest.mark.parametrize("shape,k,s,p", BN_POOL, ids=lambda v: "x".join(map(str, v)) if isinstance(v, tuple) else str(v))
def test_batch_norm_train_pool_matches_separate_calls(cuda, ops, shape, k, s, p):
    """omt_bn_train_fwd_pool (training BatchNorm -> activation -> max pool in one pass) against omt_bn_train_fwd_res
    followed by omt_maxpool_fwd, bit for bit (y, statistics, running statistics, pooled values, indices): channels of
    up to 8192 elements (one launch, pooled from LDS; scalar loads on odd planes) and larger ones (runs of pooled
    rows, odd planes, many runs), 2x2 / 3x3 windows with and without padding, activations none (NaN inputs
    propagating through the pool), ReLU and hardswish; and against PyTorch CPU's max_pool2d_with_indices."""
    from omarchy_mac_torch import _lib
    n, c, h, w = shape
    rng = np.random.default_rng(n + c + h + w + k)
    x = rnd(rng, *shape) * 2 + 0.5
    flat = x.reshape(-1)
    tie = np.arange(0, flat.size - 1, 97)
    flat[tie] = flat[tie + 1]  # repeated neighbours: ties inside windows
    gam, bet, rm, rv = rnd(rng, c), rnd(rng, c), rnd(rng, c), np.abs(rnd(rng, c)) + 0.5
    for act in (_lib.OMT_ACT_NONE, _lib.OMT_ACT_RELU, _lib.OMT_ACT_HARDSWISH):
        xa = x.copy()
        if act == _lib.OMT_ACT_NONE:
            xa.reshape(-1)[5] = np.nan
        tx = dev(xa, cuda)
        rm1, rv1, rm2, rv2 = dev(rm, cuda), dev(rv, cuda), dev(rm, cuda), dev(rv, cuda)
        y1, m1, i1, out1, idx1 = ops.batch_norm_train_pool(tx, dev(gam, cuda), dev(bet, cuda), rm1, rv1, 0.1, 1e-5,
                                                           act, k, s, p)
        y2, m2, i2 = ops.batch_norm_train(tx, dev(gam, cuda), dev(bet, cuda), rm2, rv2, 0.1, 1e-5, act=act)
        out2, idx2 = ops.max_pool2d(y2, k, s, p)
        for a, b in ((y1, y2), (m1, m2), (i1, i2), (rm1, rm2), (rv1, rv2), (out1, out2), (idx1, idx2)):
            assert torch.equal(a.cpu(), b.cpu()) or (act == _lib.OMT_ACT_NONE and torch.equal(a.cpu().nan_to_num(7.0),
                                                                                          b.cpu().nan_to_num(7.0))), act
        ref, ref_idx = torch.nn.functional.max_pool2d(y2.cpu(), k, s, p, return_indices=True)
        assert torch.equal(out1.cpu().nan_to_num(7.0), ref.nan_to_num(7.0)) and torch.equal(idx1.cpu(), ref_idx), act


def test_batch_norm_functional_and_eval(cuda, ops):
    rng = np.random.default_rng(11)
    x, g, b, rm, rv = rnd(rng, 8, 5, 6, 6), rnd(rng, 5), rnd(rng, 5), rnd(rng, 5), np.abs(rnd(rng, 5)) + 0.2
    trm, trv = dev(rm, cuda), dev(rv, cuda)
    y, sm, si, nrm, nrv = ops.batch_norm_train(dev(x, cuda), dev(g, cuda), dev(b, cuda), trm, trv, 0.3, 1e-5,
                                               functional=True)
    _, _, _, rnm, rnv = orc.bn_train(x, g, b, rm, rv, 0.3, 1e-5)
    assert np.array_equal(host(trm), rm) and np.array_equal(host(trv), rv)  # inputs untouched
    assert orc.rel_l2(host(nrm), rnm) <= 1e-6 and orc.rel_l2(host(nrv), rnv) <= 1e-6
    for relu in (False, True):
        ye = ops.batch_norm_eval(dev(x, cuda), dev(g, cuda), dev(b, cuda), trm, trv, 1e-3, relu)
        assert orc.rel_l2(host(ye), orc.bn_eval(x, g, b, rm, rv, 1e-3, relu)) <= 1e-6


# ---- pooling ----

MAXPOOL = [((3, 3), (2, 2), (0, 0), (1, 1), False, 13), ((3, 3), (2, 2), (0, 0), (1, 1), False, 27),
           ((3, 3), (2, 2), (1, 1), (1, 1), False, 14), ((3, 3), (1, 1), (1, 1), (1, 1), False, 9),
           ((2, 2), (2, 2), (0, 0), (1, 1), False, 12), ((5, 5), (3, 3), (2, 2), (1, 1), False, 17),
           ((3, 3), (2, 2), (1, 1), (2, 2), False, 15), ((3, 2), (2, 1), (1, 0), (1, 1), True, 11),
           ((2, 2), (2, 2), (0, 0), (1, 1), True, 13),
           # rows of a multiple of 4 (four inputs per thread in the backward; with output rows of a multiple of 4,
           # four outputs per thread in the forward): 2x2 s2 (one output per four inputs' rows, two across), 3x3 s2 p1
           # (two by three), the same 2x2 with a partial last window, 3x3 s2 p0 in ceil mode (partial last window,
           # aligned runs), and 3x3 s1 whose cover (three by six) takes the per-input kernel
           ((2, 2), (2, 2), (0, 0), (1, 1), False, 15), ((3, 3), (2, 2), (1, 1), (1, 1), False, 31),
           ((2, 2), (2, 2), (0, 0), (1, 1), True, 15), ((3, 3), (2, 2), (0, 0), (1, 1), True, 15),
           ((3, 3), (1, 1), (1, 1), (1, 1), False, 11),
           # output rows of 12 (three four-output runs per row; eight-input backward on rows of 24)
           ((3, 3), (2, 2), (1, 1), (1, 1), False, 23)]


@pytest.mark.parametrize("k,s,p,d,ceil,hw", MAXPOOL)
def test_maxpool(cuda, ops, k, s, p, d, ceil, hw):
    rng = np.random.default_rng(hw)
    x = rnd(rng, 2, 4, hw, hw + 1)
    x[0, 0, 0, :3] = x[0, 0, 0, 0]  # ties: the first maximum wins
    x[1, 2, 3, 4] = np.nan          # NaN propagates with its index
    y, idx = ops.max_pool2d(dev(x, cuda), k, s, p, d, ceil)
    y_ref, idx_ref = orc.maxpool_fwd(x, k, s, p, d, ceil)
    np.testing.assert_array_equal(host(idx), idx_ref)
    yh = host(y)
    np.testing.assert_array_equal(np.isnan(yh), np.isnan(y_ref))
    np.testing.assert_array_equal(yh[~np.isnan(yh)], y_ref[~np.isnan(y_ref)])
    gy = rnd(rng, *y_ref.shape)
    gx = ops.max_pool2d_backward(dev(gy, cuda), x.shape, idx, k, s, p, d)
    assert orc.rel_l2(host(gx), orc.maxpool_bwd(gy, idx_ref, x.shape)) <= 1e-6


AVGPOOL = [((3, 3), (2, 2), (1, 1), False, True, None, 14), ((3, 3), (2, 2), (1, 1), False, False, None, 14),
           ((2, 2), (2, 2), (0, 0), False, True, None, 12), ((3, 3), (2, 2), (1, 1), True, False, None, 15),
           ((3, 2), (1, 2), (1, 1), True, True, None, 9), ((3, 3), (2, 2), (1, 1), False, True, 5, 10)]


@pytest.mark.parametrize("k,s,p,ceil,incl,div,hw", AVGPOOL)
def test_avgpool(cuda, ops, k, s, p, ceil, incl, div, hw):
    rng = np.random.default_rng(hw + 100)
    x = rnd(rng, 2, 3, hw, hw + 2)
    y = ops.avg_pool2d(dev(x, cuda), k, s, p, ceil, incl, div)
    y_ref = orc.avgpool_fwd(x, k, s, p, ceil, incl, div)
    assert orc.rel_l2(host(y), y_ref) <= 1e-6
    gy = rnd(rng, *y_ref.shape)
    gx = ops.avg_pool2d_backward(dev(gy, cuda), x.shape, k, s, p, incl, div)
    assert orc.rel_l2(host(gx), orc.avgpool_bwd(gy, x.shape, k, s, p, incl, div)) <= 1e-6


def test_global_avgpool_many_planes(cuda, ops):
    """Global average pooling over thousands of planes (several LDS-staged workgroups, a partial last one), plane
    sizes on both sides of the 64-element staging limit, and an input view not aligned to 16 bytes."""
    rng = np.random.default_rng(3)
    for (n, c, h, w) in ((3, 700, 7, 7), (2, 300, 4, 4), (5, 129, 1, 1), (2, 260, 7, 9), (2, 300, 8, 8),
                         (2, 70, 9, 9)):
        x = rnd(rng, n, c, h, w)
        y = ops.adaptive_avg_pool2d(dev(x, cuda), 1)
        assert orc.rel_l2(host(y), orc.adapool_fwd(x, 1, 1)) <= 1e-6, (n, c, h, w)
        gy = rnd(rng, n, c, 1, 1)
        gx = ops.adaptive_avg_pool2d_backward(dev(gy, cuda), x.shape)
        assert orc.rel_l2(host(gx), orc.adapool_bwd(gy, x.shape)) <= 1e-6, (n, c, h, w)
    x = rnd(rng, 3, 300, 7, 7)
    flat = torch.from_numpy(np.concatenate([np.zeros(1, np.float32), x.ravel()])).to(cuda)
    xv = flat[1:].view(3, 300, 7, 7)  # contiguous, 4 bytes past an aligned allocation
    assert xv.data_ptr() % 16 != 0
    assert orc.rel_l2(host(ops.adaptive_avg_pool2d(xv, 1)), orc.adapool_fwd(x, 1, 1)) <= 1e-6


@pytest.mark.parametrize("hw,o", [(6, 6), (13, 6), (10, 4), (7, 1), (5, 3), (2, 1), (56, 1)])
def test_adaptive_avgpool(cuda, ops, hw, o):
    rng = np.random.default_rng(hw * 7 + o)
    x = rnd(rng, 3, 5, hw, hw + (0 if o == 1 else 1))
    y = ops.adaptive_avg_pool2d(dev(x, cuda), o)
    y_ref = orc.adapool_fwd(x, o, o)
    assert orc.rel_l2(host(y), y_ref) <= 1e-6
    gy = rnd(rng, *y_ref.shape)
    gx = ops.adaptive_avg_pool2d_backward(dev(gy, cuda), x.shape)
    assert orc.rel_l2(host(gx), orc.adapool_bwd(gy, x.shape)) <= 1e-6

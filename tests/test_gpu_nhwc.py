"""Parity of the channels-last (NHWC) convolution kernels (omt_conv_fwd_nhwc / omt_conv_dgrad_nhwc /
omt_conv_wgrad_nhwc, called through the C ABI) with the CPU oracle, and of the device's channels-last convolutions
through autograd with PyTorch CPU.

Criterion: rel-L2 <= 1e-4 per op. The channels-last forward and grad input run the tap-major
reduction of the NCHW gather tiles over the same LDS layout and MFMA order, so under the same plan they must be
bit-identical to the NCHW kernels (which tests/test_gpu_parity.py pins to the oracle at every size); grad weight
reduces in another order and is checked against the oracle only. Full-size cases (BASELINE config 5 layers at batch
256) use stratified oracle points and the float64 adjoint identity.
"""

import numpy as np
import pytest
import torch

from oracle import oracle as orc

pytestmark = pytest.mark.gpu

TOL = 1e-4
CL = torch.channels_last


def rnd(rng, *shape, scale=1.0):
    return (rng.standard_normal(shape) * scale).astype(np.float32)


def dev_cl(a, cuda):
    return torch.from_numpy(np.ascontiguousarray(a)).to(cuda).contiguous(memory_format=CL)


def host(t):
    torch.cuda.synchronize()
    return np.ascontiguousarray(t.detach().cpu().contiguous().numpy())


@pytest.fixture(scope="module")
def ops():
    from omarchy_mac_torch import hip_ops
    return hip_ops


NHWC_SHAPES = [
    # (n, ci, co, h, w, ks, stride, pad)
    (2, 16, 16, 9, 7, 3, 1, 1),       # ragged, one K-block of channels
    (2, 32, 48, 14, 14, 3, 1, 1),
    (3, 64, 32, 13, 11, 5, 2, 2),     # stride 2: phases with different K
    (2, 32, 64, 16, 16, 1, 2, 0),     # 1x1 stride 2: three of four grad-input phases have no tap
    (2, 16, 32, 20, 20, 7, 2, 3),     # the ResNet stem's window
    (2, 48, 16, 11, 11, 4, 3, 1),     # stride 3, even kernel
    (2, 64, 64, 56, 56, 3, 1, 1),     # config 5 layers at batch 2
    (2, 64, 256, 56, 56, 1, 1, 0),
    (2, 256, 64, 28, 28, 1, 1, 0),
    (4, 512, 512, 2, 2, 3, 1, 1),     # ResNet-18 layer4 at 64x64: the cost model splits K
    (3, 16, 36, 10, 10, 3, 1, 1),     # 36 output channels: a partial row tile (grad input then not covered)
    (2, 32, 18, 8, 6, 11, 4, 5),      # 11x11 stride 4, 18 output channels: scalar stores, neither grad covered
]


def _ids(s):
    return "n{}c{}o{}h{}w{}k{}s{}p{}".format(*s)


@pytest.mark.parametrize("shape", NHWC_SHAPES, ids=_ids)
def test_conv_nhwc_fwd_dgrad_wgrad(cuda, ops, shape):
    """Forward (bias + ReLU), grad input and grad weight of channels-last tensors against the oracle; the outputs
    come back channels_last. Grad input needs co % 16 == 0 and grad weight ci, co multiples of 4: other shapes raise
    Unsupported (the device then runs the NCHW kernels)."""
    from omarchy_mac_torch._lib import Unsupported
    n, ci, co, h, w, ks, s, p = shape
    rng = np.random.default_rng(sum(shape))
    x, wt, b = rnd(rng, n, ci, h, w), rnd(rng, co, ci, ks, ks, scale=(ci * ks * ks) ** -0.5), rnd(rng, co, scale=0.1)
    y = ops.conv2d_nhwc(dev_cl(x, cuda), dev_cl(wt, cuda), torch.from_numpy(b).to(cuda), s, p, relu=True)
    assert y.is_contiguous(memory_format=CL)
    y_ref = orc.conv_fwd(x, wt, b, s, p, relu=True)
    assert orc.rel_l2(host(y), y_ref) <= TOL
    gy = rnd(rng, *y_ref.shape)
    if co % 16 == 0:
        gx = ops.conv2d_dgrad_nhwc(dev_cl(gy, cuda), dev_cl(wt, cuda), x.shape, s, p)
        assert gx.is_contiguous(memory_format=CL)
        assert orc.rel_l2(host(gx), orc.conv_dgrad(gy, wt, x.shape, s, p)) <= TOL
    else:
        with pytest.raises(Unsupported):
            ops.conv2d_dgrad_nhwc(dev_cl(gy, cuda), dev_cl(wt, cuda), x.shape, s, p)
    if co % 4 == 0:
        gw = ops.conv2d_wgrad_nhwc(dev_cl(x, cuda), dev_cl(gy, cuda), ks, s, p)
        assert gw.is_contiguous(memory_format=CL)
        assert orc.rel_l2(host(gw), orc.conv_wgrad(x, gy, ks, s, p)) <= TOL
    else:
        with pytest.raises(Unsupported):
            ops.conv2d_wgrad_nhwc(dev_cl(x, cuda), dev_cl(gy, cuda), ks, s, p)


def test_conv_nhwc_input_channels_not_covered(cuda, ops):
    """Forward needs ci % 16 == 0 and grad weight ci % 4 == 0: other inputs raise Unsupported, nothing runs."""
    from omarchy_mac_torch._lib import Unsupported
    rng = np.random.default_rng(3)
    x, wt = rnd(rng, 2, 6, 8, 8), rnd(rng, 16, 6, 3, 3)
    with pytest.raises(Unsupported):
        ops.conv2d_nhwc(dev_cl(x, cuda), dev_cl(wt, cuda), None, 1, 1)
    with pytest.raises(Unsupported):
        ops.conv2d_wgrad_nhwc(dev_cl(x, cuda), dev_cl(rnd(rng, 2, 16, 8, 8), cuda), 3, 1, 1)


NHWC_PLAN_SHAPES = [
    (4, 512, 512, 2, 2, 3, 1, 1),   # tiny images: K splits up to the maximum
    (3, 64, 128, 9, 9, 3, 2, 1),    # stride 2: grad-input phases with different K
    (2, 32, 48, 6, 5, 1, 1, 0),     # 1x1, channels a multiple of 16 but not of 32 (the deeper K-blocks fall back)
    (2, 128, 64, 12, 10, 3, 1, 1),
]


@pytest.mark.parametrize("shape", NHWC_PLAN_SHAPES, ids=_ids)
def test_conv_nhwc_every_plan_matches_nchw_bit_for_bit(cuda, ops, shape):
    """Every channels-last tile with 1, 2, 3 and 7 K slices, forward (bias + ReLU) and grad input, against the oracle;
    where the tile's K-block divides the gathered channels, also bit-identical to the NCHW kernels under the same plan
    (both then run the tap-major K order over the same LDS layout and MFMA sequence; elsewhere the NHWC plan runs as
    tile 5 and the NCHW one in channel-major order). Every grad-weight tile with 1, 2 and 5 slices against the
    oracle."""
    n, ci, co, h, w, ks, s, p = shape
    rng = np.random.default_rng(sum(shape))
    x, wt, b = rnd(rng, n, ci, h, w), rnd(rng, co, ci, ks, ks, scale=(ci * ks * ks) ** -0.5), rnd(rng, co)
    y_ref = orc.conv_fwd(x, wt, b, s, p, relu=True)
    gy = rnd(rng, *y_ref.shape)
    gx_ref, gw_ref = orc.conv_dgrad(gy, wt, x.shape, s, p), orc.conv_wgrad(x, gy, ks, s, p)
    tx, tw, tgy = dev_cl(x, cuda), dev_cl(wt, cuda), dev_cl(gy, cuda)
    tb = torch.from_numpy(b).to(cuda)
    nx, nw, ngy = tx.contiguous(), tw.contiguous(), tgy.contiguous()
    tile_bk = {0: 16, 1: 16, 2: 16, 3: 16, 4: 16, 5: 16, 6: 64, 7: 32, 8: 32}
    try:
        assert ops.conv_num_tiles("fwd_nhwc") == 9 and ops.conv_num_tiles("dgrad_nhwc") == 9
        for tile in range(9):
            for slices in (1, 2, 3, 7):
                case = (tile, slices)
                for d in ("fwd", "dgrad", "fwd_nhwc", "dgrad_nhwc"):
                    ops.set_conv_plan(d, x.shape, wt.shape, s, p, tile, slices)
                y = ops.conv2d_nhwc(tx, tw, tb, s, p, relu=True)
                gx = ops.conv2d_dgrad_nhwc(tgy, tw, x.shape, s, p)
                assert orc.rel_l2(host(y), y_ref) <= TOL, case
                assert orc.rel_l2(host(gx), gx_ref) <= TOL, case
                if ci % tile_bk[tile] == 0:
                    assert torch.equal(y.contiguous(), ops.conv2d(nx, nw, tb, s, p, relu=True)), case
                if co % tile_bk[tile] == 0:
                    assert torch.equal(gx.contiguous(), ops.conv2d_dgrad(ngy, nw, x.shape, s, p)), case
        assert ops.conv_num_tiles("wgrad_nhwc") == 4
        for tile in range(4):
            for slices in (1, 2, 5):
                ops.set_conv_plan("wgrad_nhwc", x.shape, wt.shape, s, p, tile, slices)
                gw = ops.conv2d_wgrad_nhwc(tx, tgy, ks, s, p)
                assert orc.rel_l2(host(gw), gw_ref) <= TOL, (tile, slices)
    finally:
        ops.clear_conv_plans()


def test_conv_nhwc_autotune_caches_plans(cuda, ops):
    """The tuner times the channels-last candidates and caches the winner under the NHWC directions only."""
    xs, ws = (8, 64, 14, 14), (64, 64, 3, 3)
    ops.clear_conv_plans()
    try:
        for d in ("fwd_nhwc", "dgrad_nhwc", "wgrad_nhwc"):
            tile, slices = ops.autotune_conv(d, xs, ws, 1, 1)
            assert ops.conv_plan(d, xs, ws, 1, 1) == (tile, slices, True)
            assert tile < ops.conv_num_tiles(d)
        for d in ("fwd", "dgrad", "wgrad"):
            assert not ops.conv_plan(d, xs, ws, 1, 1)[2]
    finally:
        ops.clear_conv_plans()


FULL_NHWC = [
    ("C5_3x3_56", (256, 64, 64, 56, 56, 3, 1, 1)),
    ("C5_3x3_7", (256, 512, 512, 7, 7, 3, 1, 1)),
    ("C5_1x1_exp_56", (256, 64, 256, 56, 56, 1, 1, 0)),
    ("C5_1x1_red_14", (256, 1024, 256, 14, 14, 1, 1, 0)),
]


def block_points(rng, rows, cols, to_flat, br=16, bc=32):
    """One random point in every br x bc block of a rows x cols GEMM output, mapped to flat NCHW indices."""
    rr, cc = np.meshgrid(np.arange(0, rows, br), np.arange(0, cols, bc), indexing="ij")
    r = rr.ravel() + rng.integers(0, br, rr.size) % np.minimum(br, rows - rr.ravel())
    c = cc.ravel() + rng.integers(0, bc, cc.size) % np.minimum(bc, cols - cc.ravel())
    return to_flat(r.astype(np.int64), c.astype(np.int64))


@pytest.mark.parametrize("name,shape", FULL_NHWC, ids=[c[0] for c in FULL_NHWC])
def test_conv_nhwc_full_size(cuda, ops, name, shape):
    """A config 5 layer at batch 256 in channels-last order under the tuner's plans (as bench.py runs them):
    stratified oracle points in every 16 x 32 block of each direction's GEMM output (grad weight over its tap-major
    columns, which are the channels-last filter's memory order) and the float64 adjoint identity."""
    n, ci, co, h, w, ks, s, p = shape
    xs, ws = (n, ci, h, w), (co, ci, ks, ks)
    ops.clear_conv_plans()
    try:
        for d in ("fwd_nhwc", "dgrad_nhwc", "wgrad_nhwc"):
            ops.autotune_conv(d, xs, ws, s, p)
        plans = {d: ops.conv_plan(d, xs, ws, s, p)[:2] for d in ("fwd_nhwc", "dgrad_nhwc", "wgrad_nhwc")}
        gen = torch.Generator(device=cuda).manual_seed(2)
        scale = (ci * ks * ks) ** -0.5
        x = torch.randn(xs, device=cuda, generator=gen).contiguous(memory_format=CL)
        wt = (torch.randn(ws, device=cuda, generator=gen) * scale).contiguous(memory_format=CL)
        b = torch.rand((co,), device=cuda, generator=gen) * 0.2 - 0.1
        y = ops.conv2d_nhwc(x, wt, b, s, p)
        gy = (torch.randn(y.shape, device=cuda, generator=gen) * scale).contiguous(memory_format=CL)
        gx = ops.conv2d_dgrad_nhwc(gy, wt, xs, s, p)
        gw = ops.conv2d_wgrad_nhwc(x, gy, ks, s, p)
        torch.cuda.synchronize()
    finally:
        ops.clear_conv_plans()
    case = (name, plans)
    yb = (y - b.view(1, -1, 1, 1)).double()
    a1 = (yb * gy.double()).sum().item()
    a2 = (x.double() * gx.double()).sum().item()
    a3 = (wt.double() * gw.double()).sum().item()
    norm = (yb.norm() * gy.double().norm()).item()
    assert abs(a1 - a2) <= 1e-5 * norm and abs(a1 - a3) <= 1e-5 * norm, (case, a1, a2, a3, norm)
    rng = np.random.default_rng(0)
    xh, wh, bh, gyh = host(x), host(wt), host(b), host(gy)
    oh, ow = y.shape[2], y.shape[3]
    hw, ohw = h * w, oh * ow
    # rows = channels, columns = pixels n * hw + pixel (the NHWC GEMM's pixel order), as flat NCHW indices
    pts = block_points(rng, co, n * ohw, lambda r, c: ((c // ohw) * co + r) * ohw + c % ohw)
    assert orc.rel_l2(host(y).ravel()[pts], orc.conv_fwd_points(xh, wh, pts, bh, s, p)) <= TOL, case
    pts = block_points(rng, ci, n * hw, lambda r, c: ((c // hw) * ci + r) * hw + c % hw)
    assert orc.rel_l2(host(gx).ravel()[pts], orc.conv_dgrad_points(gyh, wh, xs, pts, s, p)) <= TOL, case
    kk = ks * ks
    kcols = ci * kk
    tm = block_points(rng, co, kcols, lambda r, c: r * kcols + (c % ci) * kk + c // ci)
    pts = np.concatenate([tm, rng.integers(0, gw.numel(), max(0, 2000 - tm.size))])
    assert orc.rel_l2(host(gw).ravel()[pts], orc.conv_wgrad_points(xh, gyh, ks, pts, s, p)) <= TOL, case


# ---- through the device and autograd ----

CL_CASES = [
    # (n, ci, co, h, ks, s, p, bias): covered by the NHWC kernels in every direction
    (2, 32, 64, 14, 3, 1, 1, False), (2, 64, 32, 9, 1, 2, 0, True), (3, 16, 48, 11, 5, 2, 2, False),
    # input channels not a multiple of 16 (forward in NCHW, output converted), 36 output channels (grad input in NCHW)
    (2, 3, 16, 23, 7, 2, 3, False), (2, 16, 36, 10, 3, 1, 1, True),
]


@pytest.mark.parametrize("case", CL_CASES, ids=lambda c: "n{}c{}o{}h{}k{}s{}p{}b{}".format(*c))
def test_channels_last_conv_through_autograd(cuda, case):
    """A channels_last nn.Conv2d on the device: output and both gradients channels_last (torch's convolution
    convention), values within 1e-4 of PyTorch CPU, the convolutions run on this library's kernels (nothing delegated
    to torch's, no FALLBACKS entry)."""
    import omarchy_mac_torch as omt
    from omarchy_mac_torch import stacks
    n, ci, co, h, ks, s, p, bias = case
    prev = stacks.set_auto_fuse(False)
    omt.FALLBACKS.clear()
    omt._native.core.count_delegated(True)
    try:
        torch.manual_seed(sum(case[:7]))
        conv = torch.nn.Conv2d(ci, co, ks, s, p, bias=bias)
        x = torch.randn(n, ci, h, h)
        ref = torch.nn.Conv2d(ci, co, ks, s, p, bias=bias)
        ref.load_state_dict(conv.state_dict())
        xr = x.clone().requires_grad_()
        yr = ref(xr)
        gy = torch.randn(yr.shape)
        yr.backward(gy)
        dconv = conv.to(omt.DEVICE).to(memory_format=CL)
        dx = x.to(omt.DEVICE).contiguous(memory_format=CL).requires_grad_()
        y = dconv(dx)
        assert y.is_contiguous(memory_format=CL)
        y.backward(gy.to(omt.DEVICE).contiguous(memory_format=CL))
        assert dx.grad.is_contiguous(memory_format=CL)
        for got, want in ((y, yr), (dx.grad, xr.grad), (dconv.weight.grad, ref.weight.grad)):
            assert orc.rel_l2(got.detach().cpu().numpy(), want.detach().numpy()) <= TOL
        if bias:
            assert orc.rel_l2(dconv.bias.grad.cpu().numpy(), ref.bias.grad.numpy()) <= TOL
        delegated = omt._native.core.delegated_counts()
        assert not any(k.startswith("convolution") for k in delegated), delegated
        assert not omt.FALLBACKS, dict(omt.FALLBACKS.items())
    finally:
        omt._native.core.count_delegated(False)
        omt.FALLBACKS.clear()
        stacks.set_auto_fuse(prev)

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
    (3, 16, 36, 10, 10, 3, 1, 1),     # 36 output channels: a partial row tile, a narrow grad input
    (2, 32, 18, 8, 6, 11, 4, 5),      # 11x11 stride 4, 18 output channels: scalar stores, grad weight not covered
    # input channels not a multiple of 16: the forward gathers element by element; of 4: so do grad weight's columns
    (2, 3, 64, 32, 32, 7, 2, 3),      # the ResNet stem (at 64x64 input: 32x32 here)
    (3, 6, 16, 9, 11, 3, 1, 1),
    (2, 20, 32, 10, 10, 3, 2, 1),     # 20 channels: narrow forward, float4 grad-weight columns
    (2, 1, 16, 12, 12, 5, 1, 2),      # one input channel
    (2, 24, 88, 14, 14, 1, 1, 0),     # MobileNetV3's expand: 88 output channels, a narrow grad input
    (2, 16, 24, 9, 9, 3, 2, 1),       # stride 2, narrow grad input over four phases
]


def _ids(s):
    return "n{}c{}o{}h{}w{}k{}s{}p{}".format(*s)


@pytest.mark.parametrize("shape", NHWC_SHAPES, ids=_ids)
def test_conv_nhwc_fwd_dgrad_wgrad(cuda, ops, shape):
    """Forward (bias + ReLU), grad input and grad weight of channels-last tensors against the oracle; the outputs
    come back channels_last. Any channel counts but grad weight's co % 4 != 0, which raises Unsupported (the device
    then runs the NCHW kernel)."""
    from omarchy_mac_torch._lib import Unsupported
    n, ci, co, h, w, ks, s, p = shape
    rng = np.random.default_rng(sum(shape))
    x, wt, b = rnd(rng, n, ci, h, w), rnd(rng, co, ci, ks, ks, scale=(ci * ks * ks) ** -0.5), rnd(rng, co, scale=0.1)
    y = ops.conv2d_nhwc(dev_cl(x, cuda), dev_cl(wt, cuda), torch.from_numpy(b).to(cuda), s, p, relu=True)
    assert y.is_contiguous(memory_format=CL)
    y_ref = orc.conv_fwd(x, wt, b, s, p, relu=True)
    assert orc.rel_l2(host(y), y_ref) <= TOL
    gy = rnd(rng, *y_ref.shape)
    gx = ops.conv2d_dgrad_nhwc(dev_cl(gy, cuda), dev_cl(wt, cuda), x.shape, s, p)
    assert gx.is_contiguous(memory_format=CL)
    assert orc.rel_l2(host(gx), orc.conv_dgrad(gy, wt, x.shape, s, p)) <= TOL
    if co % 4 == 0:
        gw = ops.conv2d_wgrad_nhwc(dev_cl(x, cuda), dev_cl(gy, cuda), ks, s, p)
        assert gw.is_contiguous(memory_format=CL)
        assert orc.rel_l2(host(gw), orc.conv_wgrad(x, gy, ks, s, p)) <= TOL
    else:
        with pytest.raises(Unsupported):
            ops.conv2d_wgrad_nhwc(dev_cl(x, cuda), dev_cl(gy, cuda), ks, s, p)


def test_conv_nhwc_output_channels_not_covered(cuda, ops):
    """Grad weight needs co % 4 == 0: other outputs raise Unsupported, nothing runs."""
    from omarchy_mac_torch._lib import Unsupported
    rng = np.random.default_rng(3)
    x, gy = rnd(rng, 2, 6, 8, 8), rnd(rng, 2, 18, 8, 8)
    with pytest.raises(Unsupported):
        ops.conv2d_wgrad_nhwc(dev_cl(x, cuda), dev_cl(gy, cuda), 3, 1, 1)


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
    # 3 input channels (the narrow NHWC forward and grad weight), 36 output channels (a narrow grad input)
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


# ---- channels-last BatchNorm, pools, plane sums and mixed-order pointwise -------------------------------------------

def dev(a, cuda):
    return torch.from_numpy(np.ascontiguousarray(a)).to(cuda)


BN_NHWC = [(4, 6, 5, 7), (16, 8, 4, 4), (32, 64, 16, 16), (32, 512, 2, 2), (3, 5, 37, 41), (64, 16, 28, 28),
           (8, 3, 7, 9), (4, 8, 56, 56), (32, 96, 7, 7), (2, 576, 7, 7), (1, 16, 57, 31), (9, 12, 15, 15),
           (128, 32, 32, 32), (2, 260, 3, 5), (8, 64, 16, 16), (1, 12, 41, 50)]


@pytest.mark.parametrize("n,c,h,w", BN_NHWC, ids=lambda v: str(v))
def test_batch_norm_nhwc(cuda, ops, n, c, h, w):
    """omt_bn_train_fwd_nhwc / omt_bn_eval_fwd_nhwc / omt_bn_bwd_nhwc over channels_last tensors (float4 channel runs
    when c % 4 == 0, scalar otherwise; one and several channel blocks per row; one launch up to 2048 rows, three
    above: 8 x 16², 2048 rows, and 41 x 50, 2050) against the oracle (the statistics
    from inputs of large mean), and against the NCHW kernels on the same data: the statistics agree to float64
    rounding (rel 1e-6), eval is the same arithmetic bit for bit, and the backward's gz (the gradient through the
    activation, with a second gradient added) is exact."""
    from omarchy_mac_torch import _lib
    rng = np.random.default_rng(n * 7 + c * 3 + h)
    x = rnd(rng, n, c, h, w) * 3 + 5
    gam, bet, rm, rv = rnd(rng, c), rnd(rng, c), rnd(rng, c), np.abs(rnd(rng, c)) + 0.5
    res = rnd(rng, n, c, h, w)
    z_plain, m_ref, i_ref, nrm, nrv = orc.bn_train(x, gam, bet, rm, rv, 0.1, 1e-5)
    tg, tb = dev(gam, cuda), dev(bet, cuda)
    for act in (_lib.OMT_ACT_NONE, _lib.OMT_ACT_RELU, _lib.OMT_ACT_HARDSWISH):
        r = res if act == _lib.OMT_ACT_RELU else None
        trm, trv = dev(rm, cuda), dev(rv, cuda)
        y, sm, si, z = ops.batch_norm_train_nhwc(dev_cl(x, cuda), tg, tb, trm, trv, 0.1, 1e-5, act=act,
                                                 residual=None if r is None else dev_cl(r, cuda), return_z=True)
        assert y.is_contiguous(memory_format=CL) and z.is_contiguous(memory_format=CL)
        z_ref = z_plain + r if r is not None else z_plain
        assert orc.rel_l2(host(z), z_ref) <= TOL, act
        assert orc.rel_l2(host(sm), m_ref) <= 1e-6 and orc.rel_l2(host(si), i_ref) <= 1e-5
        assert orc.rel_l2(host(trm), nrm) <= 1e-6 and orc.rel_l2(host(trv), nrv) <= 1e-6
        y2, sm2, si2, z2 = ops.batch_norm_train(dev(x, cuda), tg, tb, dev(rm, cuda), dev(rv, cuda), 0.1, 1e-5,
                                                act=act, residual=None if r is None else dev(r, cuda), return_z=True)
        assert orc.rel_l2(host(sm), host(sm2)) <= 1e-6 and orc.rel_l2(host(si), host(si2)) <= 1e-6
        assert orc.rel_l2(host(z), host(z2)) <= 1e-6 and orc.rel_l2(host(y), host(y2)) <= 1e-6
        tz = torch.from_numpy(host(z))
        want = {_lib.OMT_ACT_NONE: tz, _lib.OMT_ACT_RELU: torch.relu(tz),
                _lib.OMT_ACT_HARDSWISH: torch.nn.functional.hardswish(tz)}[act]
        yd = torch.from_numpy(host(y))
        assert torch.equal(yd, want) or (act == _lib.OMT_ACT_HARDSWISH and orc.rel_l2(yd.numpy(), want.numpy()) <= 1e-6)
        # backward through the activation, with a second incoming gradient and gz returned
        g, g2 = rnd(rng, n, c, h, w), rnd(rng, n, c, h, w)
        act_in = y if act == _lib.OMT_ACT_RELU else z
        gx, dg, db, gz = ops.batch_norm_backward_nhwc(dev_cl(g, cuda), dev_cl(x, cuda), sm, si, tg, act=act,
                                                      act_in=act_in, g2=dev_cl(g2, cuda), want_gz=True)
        assert gx.is_contiguous(memory_format=CL) and gz.is_contiguous(memory_format=CL)
        gsum = torch.from_numpy(g + g2)
        gz_ref = {_lib.OMT_ACT_NONE: gsum, _lib.OMT_ACT_RELU: torch.ops.aten.threshold_backward(gsum, want, 0),
                  _lib.OMT_ACT_HARDSWISH: torch.ops.aten.hardswish_backward(gsum, tz)}[act].numpy()
        assert np.array_equal(host(gz), gz_ref) or (act == _lib.OMT_ACT_HARDSWISH and
                                                     orc.rel_l2(host(gz), gz_ref) <= 1e-6), act
        gx_ref, dg_ref, db_ref = orc.bn_bwd(gz_ref, x, host(sm), host(si), gam)
        assert orc.rel_l2(host(dg), dg_ref) <= TOL and orc.rel_l2(host(db), db_ref) <= TOL
        scale = np.linalg.norm(gz_ref.astype(np.float64)) * np.abs(gam * host(si)).max()
        assert np.linalg.norm(host(gx).astype(np.float64) - gx_ref) <= TOL * max(scale, 1e-30)
        # the incoming gradient in NCHW order (a global pool's broadcast gradient), read in place: the same results
        gx4, dg4, db4, gz4 = ops.batch_norm_backward_nhwc(dev(g, cuda), dev_cl(x, cuda), sm, si, tg, act=act,
                                                          act_in=act_in, g2=dev_cl(g2, cuda), want_gz=True,
                                                          g_nchw=True)
        for a_, b_ in ((gx4, gx), (dg4, dg), (db4, db), (gz4, gz)):
            assert torch.equal(a_.cpu(), b_.cpu()), act
        # grads only (no gx, no gz): the apply pass is skipped
        _, dg3, db3, _ = ops.batch_norm_backward_nhwc(dev_cl(g, cuda), dev_cl(x, cuda), sm, si, tg, act=act,
                                                      act_in=act_in, g2=dev_cl(g2, cuda),
                                                      output_mask=(False, True, True))
        assert torch.equal(dg3.cpu(), dg.cpu()) and torch.equal(db3.cpu(), db.cpu())
    ye = ops.batch_norm_eval_nhwc(dev_cl(x, cuda), tg, tb, dev(rm, cuda), dev(rv, cuda), 1e-5, act=_lib.OMT_ACT_RELU)
    ye2 = ops.batch_norm_eval(dev(x, cuda), tg, tb, dev(rm, cuda), dev(rv, cuda), 1e-5, relu=True)
    assert np.array_equal(host(ye), host(ye2))
    assert orc.rel_l2(host(ye), orc.bn_eval(x, gam, bet, rm, rv, 1e-5, True)) <= TOL


POOL_NHWC = [
    # (n, c, h, w, kernel, stride, padding, dilation, ceil)
    (2, 64, 32, 32, 3, 2, 1, 1, False),  # the ResNet stem's pool
    (4, 16, 16, 16, 2, 2, 0, 1, False),
    (3, 5, 13, 11, 3, 2, 1, 1, True),    # c % 4 != 0, ceil mode
    (2, 8, 15, 17, 3, 1, 1, 2, False),   # dilation
    (2, 12, 9, 9, 4, 3, 2, 1, False),
]


@pytest.mark.parametrize("case", POOL_NHWC, ids=lambda c: "n{}c{}h{}w{}k{}s{}p{}d{}ceil{}".format(*c))
def test_pools_nhwc_match_nchw_bit_for_bit(cuda, ops, case):
    """Max pool (with ties and a NaN), average pool (padding counted or not, a divisor override) and adaptive
    average pool, forward and backward, over channels_last tensors: the NCHW kernels' values and int64 indices
    transposed, bit for bit (the NCHW kernels are pinned to the oracle in tests/test_gpu_parity.py)."""
    n, c, h, w, k, s, p, d, ceil = case
    rng = np.random.default_rng(sum(case[:8]))
    x = rnd(rng, n, c, h, w)
    x[0, 0, 0, :4] = 7.0  # ties: the first maximum in row-major order wins
    x[-1, -1, h // 2, w // 2] = np.nan
    tx, tcl = dev(x, cuda), dev_cl(x, cuda)
    y, idx = ops.max_pool2d_nhwc(tcl, k, s, p, d, ceil)
    y2, idx2 = ops.max_pool2d(tx, k, s, p, d, ceil)
    assert y.is_contiguous(memory_format=CL) and idx.is_contiguous(memory_format=CL)
    assert np.array_equal(host(y), host(y2), equal_nan=True)
    assert np.array_equal(idx.cpu().contiguous().numpy(), idx2.cpu().numpy())
    gy = rnd(rng, *y2.shape)
    gx = ops.max_pool2d_backward_nhwc(dev_cl(gy, cuda), x.shape, idx, k, s, p, d)
    gx2 = ops.max_pool2d_backward(dev(gy, cuda), x.shape, idx2, k, s, p, d)
    assert gx.is_contiguous(memory_format=CL) and np.array_equal(host(gx), host(gx2))
    x = rnd(rng, n, c, h, w)
    tx, tcl = dev(x, cuda), dev_cl(x, cuda)
    if d == 1 and 2 * p <= k:
        for incl, div in ((True, None), (False, None), (True, 3)):
            ya = ops.avg_pool2d_nhwc(tcl, k, s, p, ceil, incl, div)
            ya2 = ops.avg_pool2d(tx, k, s, p, ceil, incl, div)
            assert np.array_equal(host(ya), host(ya2)), (incl, div)
            gy = rnd(rng, *ya2.shape)
            ga = ops.avg_pool2d_backward_nhwc(dev_cl(gy, cuda), x.shape, k, s, p, incl, div)
            ga2 = ops.avg_pool2d_backward(dev(gy, cuda), x.shape, k, s, p, incl, div)
            assert np.array_equal(host(ga), host(ga2)), (incl, div)
    for out in ((1, 1), (3, 2), (max(1, h // 2), max(1, w // 3))):
        yd = ops.adaptive_avg_pool2d_nhwc(tcl, out)
        yd2 = ops.adaptive_avg_pool2d(tx, out)
        if out != (1, 1) or h * w <= 64:  # larger global pools: the NCHW kernel reduces by wave, in another order
            assert np.array_equal(host(yd), host(yd2)), out
        assert orc.rel_l2(host(yd), orc.adapool_fwd(x, *out)) <= 1e-6
        gy = rnd(rng, n, c, *out)
        gd = ops.adaptive_avg_pool2d_backward_nhwc(dev_cl(gy, cuda), x.shape)
        gd2 = ops.adaptive_avg_pool2d_backward(dev(gy, cuda), x.shape)
        assert np.array_equal(host(gd), host(gd2)), out


def test_plane_sum_nhwc_and_mixed_order_pointwise(cuda, ops):
    """omt_plane_sum_nhwc (a channels_last model's global average pool through mean) against a float64 sum; and
    omt_pointwise_layouts, an NCHW operand meeting a channels_last one (the pool's broadcast gradient meeting the ReLU
    mask), equal to PyTorch CPU's op bit for bit with the output in either order."""
    from omarchy_mac_torch import _lib
    rng = np.random.default_rng(11)
    for n, c, h, w in ((32, 512, 2, 2), (4, 96, 7, 7), (2, 3, 56, 56), (5, 70, 9, 11), (3, 300, 1, 2)):
        x = rnd(rng, n, c, h, w) + 2
        got = ops.plane_sum_nhwc(dev_cl(x, cuda), 1.0 / (h * w))
        want = x.astype(np.float64).mean(axis=(2, 3))
        assert orc.rel_l2(got.cpu().numpy(), want) <= 1e-6, (n, c, h, w)
    g, y = rnd(rng, 4, 24, 5, 6), rnd(rng, 4, 24, 5, 6)
    tg, ty = torch.from_numpy(g), torch.from_numpy(y)
    for out_nhwc in (True, False):
        out = ops.pointwise_layouts(_lib.OMT_PW_THRESHOLD_BWD, dev(g, cuda), dev_cl(y, cuda), 0.0, out_nhwc)
        assert out.is_contiguous(memory_format=CL if out_nhwc else torch.contiguous_format)
        assert torch.equal(out.cpu(), torch.ops.aten.threshold_backward(tg, ty, 0.0))
        out = ops.pointwise_layouts(_lib.OMT_PW_ADD, dev_cl(g, cuda), dev(y, cuda), 0.5, out_nhwc)
        assert torch.equal(out.cpu(), torch.add(tg, ty, alpha=0.5))
        out = ops.pointwise_layouts(_lib.OMT_PW_RELU, dev_cl(g, cuda), None, 0.0, out_nhwc)
        assert torch.equal(out.cpu(), torch.relu(tg))


DW_NHWC = [
    # (n, c, h, w, ks, stride, pad)
    (2, 96, 28, 28, 5, 1, 2),   # MobileNetV3 layers
    (4, 16, 56, 56, 3, 2, 1),
    (2, 576, 7, 7, 5, 1, 2),
    (2, 6, 9, 11, 3, 1, 1),     # c % 4 != 0: one channel per thread
    (3, 40, 14, 14, 7, 1, 3),
    (2, 8, 10, 10, 4, 3, 1),
    (1, 12, 5, 5, 11, 1, 5),    # the largest filter
]


@pytest.mark.parametrize("case", DW_NHWC, ids=lambda c: "n{}c{}h{}w{}k{}s{}p{}".format(*c))
def test_depthwise_nhwc(cuda, ops, case):
    """omt_dw_fwd_nhwc (with bias) / omt_dw_dgrad_nhwc / omt_dw_wgrad_nhwc over channels_last tensors against the
    oracle, outputs channels_last; forward and grad input equal to the general NCHW kernels' results bit for bit
    where those run (stride != 1 or an unmatched padding: not the LDS-tiled stride-1 kernels)."""
    n, c, h, w, ks, s, p = case
    rng = np.random.default_rng(sum(case))
    x, wt, b = rnd(rng, n, c, h, w), rnd(rng, c, 1, ks, ks, scale=ks ** -1.0), rnd(rng, c, scale=0.1)
    tw, tb = dev(wt, cuda), dev(b, cuda)
    y = ops.depthwise_conv2d_nhwc(dev_cl(x, cuda), tw, tb, s, p)
    assert y.is_contiguous(memory_format=CL)
    y_ref = orc.dw_fwd(x, wt, b, s, p)
    assert orc.rel_l2(host(y), y_ref) <= TOL
    gy = rnd(rng, *y_ref.shape)
    gx = ops.depthwise_dgrad_nhwc(dev_cl(gy, cuda), tw, x.shape, s, p)
    assert gx.is_contiguous(memory_format=CL)
    assert orc.rel_l2(host(gx), orc.dw_dgrad(gy, wt, x.shape, s, p)) <= TOL
    gw = ops.depthwise_wgrad_nhwc(dev_cl(x, cuda), dev_cl(gy, cuda), ks, s, p)
    assert orc.rel_l2(host(gw), orc.dw_wgrad(x, gy, ks, s, p)) <= TOL
    if s != 1 or 2 * p != ks - 1:
        assert np.array_equal(host(y), host(ops.depthwise_conv2d(dev(x, cuda), tw, tb, s, p)))
        assert np.array_equal(host(gx), host(ops.depthwise_dgrad(dev(gy, cuda), tw, x.shape, s, p)))


def test_channel_scale_nhwc(cuda, ops):
    """The squeeze-excite scale over channels_last planes, x * s with s [n, c, 1, 1], equal to PyTorch CPU's product
    bit for bit (float4 and scalar channel runs)."""
    rng = np.random.default_rng(5)
    for n, c, h, w in ((4, 96, 14, 14), (2, 6, 5, 7), (3, 576, 7, 7)):
        x, sc = rnd(rng, n, c, h, w), rnd(rng, n, c, 1, 1)
        y = ops.channel_scale_nhwc(dev_cl(x, cuda), dev(sc, cuda))
        assert y.is_contiguous(memory_format=CL)
        assert torch.equal(y.cpu(), torch.from_numpy(x) * torch.from_numpy(sc))

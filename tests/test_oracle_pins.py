"""Pins the CPU oracle (oracle/omt_oracle.c) before it is trusted as the checker of the HIP kernels.

Each oracle function is checked three ways, chosen so that a dropped term, a wrong sign or index, or a transposed
operand fails at least one of them:
  * PyTorch CPU float32, the reference's own correctness oracle (README.md:65-70, tools/conformance.py:55-103);
  * float64 brute force written independently here (direct scatter loops) on tiny shapes, sweeping every kernel
    size 1..11, stride 1..4 and padding 0..ks the reference's dense path accepts (csrc/conv.cpp:173);
  * closed-form identities: the stride-phase grad input (csrc/conv.cpp:79-94) equals the stride-skipping kind-1 map
    (gemm.py:43-59) and the unstrided grad input of the zero-upsampled gradient; the conv adjoint identity
    <conv(x, w), gy> = <x, dgrad(gy, w)> = <w, wgrad(x, gy)>; BN folding (csrc/fused.cpp:34-40).
The reference ships no golden vectors for this path (its checks are live CPU comparisons), so these are the pins.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import oracle as orc

rng = np.random.default_rng(0)


def rnd(*shape, scale=1.0):
    return (rng.standard_normal(shape) * scale).astype(np.float32)


def t(a):
    return torch.from_numpy(np.ascontiguousarray(a))


# ---- brute force (float64, direct loops, written independently of the implicit-GEMM maps) ----

def bf_conv(x, w, b, s, p):
    x, w = x.astype(np.float64), w.astype(np.float64)
    n, ci, ih, iw = x.shape
    co, _, ks, _ = w.shape
    oh, ow = (ih + 2 * p - ks) // s + 1, (iw + 2 * p - ks) // s + 1
    xp = np.zeros((n, ci, ih + 2 * p + s * ks, iw + 2 * p + s * ks))
    xp[:, :, p:p + ih, p:p + iw] = x
    y = np.zeros((n, co, oh, ow))
    for ky in range(ks):
        for kx in range(ks):
            patch = xp[:, :, ky:ky + s * oh:s, kx:kx + s * ow:s]  # n ci oh ow
            y += np.einsum("ncij,oc->noij", patch, w[:, :, ky, kx])
    if b is not None:
        y += b.astype(np.float64)[None, :, None, None]
    return y


def bf_conv_grads(x, w, gy, s, p):
    """dgrad and wgrad by scattering each output tap back (the adjoint of bf_conv's gather)."""
    x, w, gy = x.astype(np.float64), w.astype(np.float64), gy.astype(np.float64)
    n, ci, ih, iw = x.shape
    co, _, ks, _ = w.shape
    oh, ow = gy.shape[2:]
    H, W = ih + 2 * p + s * ks, iw + 2 * p + s * ks
    xp = np.zeros((n, ci, H, W))
    xp[:, :, p:p + ih, p:p + iw] = x
    gxp = np.zeros((n, ci, H, W))
    gw = np.zeros_like(w)
    for ky in range(ks):
        for kx in range(ks):
            gxp[:, :, ky:ky + s * oh:s, kx:kx + s * ow:s] += np.einsum("noij,oc->ncij", gy, w[:, :, ky, kx])
            gw[:, :, ky, kx] = np.einsum("noij,ncij->oc", gy, xp[:, :, ky:ky + s * oh:s, kx:kx + s * ow:s])
    return gxp[:, :, p:p + ih, p:p + iw], gw


def err(a, b):
    return orc.rel_l2(a, b)


# ---- conv ----

# notes/scripts/conv_kinds_check.py:5 (dense entries), notes/scripts/alexnet_ops_check.py:6, tools/gemm_bench.py:8-9
# (reduced batch), plus BASELINE C1 at batch 1.
TORCH_SHAPES = [
    # (n, ci, co, hw, ks, stride, pad)
    (4, 6, 10, 14, 5, 1, 2), (4, 6, 10, 14, 3, 1, 1), (4, 6, 10, 14, 1, 1, 0),
    (3, 3, 8, 63, 11, 4, 2), (3, 4, 6, 17, 5, 1, 2), (3, 3, 6, 15, 3, 2, 1), (3, 4, 6, 9, 1, 1, 0),
    (3, 6, 10, 12, 3, 1, 0), (3, 5, 7, 21, 5, 2, 0),
    (2, 64, 192, 27, 5, 1, 2), (1, 192, 64, 13, 3, 1, 1), (2, 32, 32, 16, 3, 1, 1),
    (1, 3, 64, 224, 11, 4, 2),
]


@pytest.mark.parametrize("shape", TORCH_SHAPES, ids=lambda s: "n{}c{}o{}h{}k{}s{}p{}".format(*s))
def test_conv_vs_torch_cpu(shape):
    n, ci, co, hw, ks, s, p = shape
    x, w, b = rnd(n, ci, hw, hw), rnd(co, ci, ks, ks, scale=(ci * ks * ks) ** -0.5), rnd(co)
    y = orc.conv_fwd(x, w, b, s, p)
    ty = F.conv2d(t(x), t(w), t(b), stride=s, padding=p)
    assert y.shape == tuple(ty.shape)
    assert err(y, ty.numpy()) < 1e-5
    gy = rnd(*y.shape)
    gx_ref, gw_ref, gb_ref = torch.ops.aten.convolution_backward(
        t(gy), t(x), t(w), [co], [s, s], [p, p], [1, 1], False, [0, 0], 1, [True, True, True])
    assert err(orc.conv_dgrad(gy, w, x.shape, s, p), gx_ref.numpy()) < 1e-5
    assert err(orc.conv_wgrad(x, gy, ks, s, p), gw_ref.numpy()) < 1e-5
    assert err(orc.bias_grad(gy), gb_ref.numpy()) < 1e-5


SWEEP = [(ks, s, p) for ks in range(1, 12) for s in range(1, 5) for p in range(0, ks + 1)]


@pytest.mark.parametrize("ks", range(1, 12))
def test_conv_bruteforce_sweep(ks):
    """Every (stride, pad) the dense path accepts at this kernel size, on tiny ragged images, against float64."""
    for _, s, p in [c for c in SWEEP if c[0] == ks]:
        for hw in (ks + 1, ks + 4):
            ih, iw = hw, hw + 1  # non-square images
            if ih + 2 * p < ks or iw + 2 * p < ks:
                continue
            x, w, b = rnd(2, 3, ih, iw), rnd(4, 3, ks, ks), rnd(4)
            ref = bf_conv(x, w, b, s, p)
            y = orc.conv_fwd(x, w, b, s, p)
            assert y.shape == ref.shape, (ks, s, p, hw)
            assert err(y, ref) < 1e-6, (ks, s, p, hw)
            gy = rnd(*y.shape)
            gx_ref, gw_ref = bf_conv_grads(x, w, gy, s, p)
            assert err(orc.conv_dgrad(gy, w, x.shape, s, p), gx_ref) < 1e-6, (ks, s, p, hw)
            assert err(orc.conv_wgrad(x, gy, ks, s, p), gw_ref) < 1e-6, (ks, s, p, hw)


@pytest.mark.parametrize("ks,s,p", [(11, 4, 2), (3, 2, 1), (1, 2, 0), (5, 3, 2), (7, 2, 3), (4, 4, 4), (2, 3, 0)])
def test_stride_phase_identity(ks, s, p):
    """Phase dgrad (kind 5) == stride-skipping map (kind 1) == unstrided dgrad of the zero-upsampled gy."""
    n, ci, co, ih, iw = 2, 3, 5, 19, 17
    w = rnd(co, ci, ks, ks)
    oh, ow = (ih + 2 * p - ks) // s + 1, (iw + 2 * p - ks) // s + 1
    gy = rnd(n, co, oh, ow)
    gx = orc.conv_dgrad(gy, w, (n, ci, ih, iw), s, p)
    every = np.arange(gx.size)
    assert err(gx, orc.conv_dgrad_points(gy, w, (n, ci, ih, iw), every, s, p).reshape(gx.shape)) < 1e-6
    oh1, ow1 = ih + 2 * p - ks + 1, iw + 2 * p - ks + 1
    up = np.zeros((n, co, oh1, ow1), np.float32)
    up[:, :, : s * (oh - 1) + 1: s, : s * (ow - 1) + 1: s] = gy
    assert err(gx, orc.conv_dgrad(up, w, (n, ci, ih, iw), 1, p)) < 1e-6


@pytest.mark.parametrize("ks,s,p", [(3, 1, 1), (11, 4, 2), (1, 2, 0), (5, 2, 2)])
def test_adjoint_identity(ks, s, p):
    """<conv(x, w), gy> = <x, dgrad(gy, w)> = <w, wgrad(x, gy)>, each side from a different oracle map."""
    x, w = rnd(3, 4, 23, 21), rnd(6, 4, ks, ks)
    y = orc.conv_fwd(x, w, None, s, p)
    gy = rnd(*y.shape)
    a = np.vdot(y.astype(np.float64), gy)
    b = np.vdot(x.astype(np.float64), orc.conv_dgrad(gy, w, x.shape, s, p))
    c = np.vdot(w.astype(np.float64), orc.conv_wgrad(x, gy, ks, s, p))
    assert abs(a - b) <= 1e-5 * abs(a) and abs(a - c) <= 1e-5 * abs(a)


def test_points_agree_with_full():
    x, w, b = rnd(2, 5, 13, 11), rnd(7, 5, 3, 3), rnd(7)
    y = orc.conv_fwd(x, w, b, 2, 1, relu=True)
    idx = np.arange(y.size)
    assert err(orc.conv_fwd_points(x, w, idx, b, 2, 1, relu=True), y.ravel()) < 1e-6
    gy = rnd(*y.shape)
    gw = orc.conv_wgrad(x, gy, 3, 2, 1)
    assert err(orc.conv_wgrad_points(x, gy, 3, np.arange(gw.size), 2, 1), gw.ravel()) < 1e-6


def test_wgrad_split_invariance_and_rule():
    """The split-K partition only decides which terms share a partial, never the sum; and it covers K exactly."""
    x, gy_shape = rnd(4, 3, 12, 12), (4, 5, 12, 12)
    gy = rnd(*gy_shape)
    base = orc.conv_wgrad(x, gy, 3, 1, 1, slices=1, kslice=4 * 144)
    for slices, kslice in [(0, 0), (9, 64), (36, 16)]:
        assert err(orc.conv_wgrad(x, gy, 3, 1, 1, slices, kslice), base) < 1e-7
    for geo_args in [(256, 64, 64, 56, 56, 3, 1, 1), (16, 3, 64, 224, 224, 11, 4, 2), (32, 512, 512, 2, 2, 3, 1, 1)]:
        g = orc.geo(*geo_args)
        M, N, K = orc.mnk(2, g)
        for mult in (0.25, 0.5, 1.0, 2.0):
            bm, bn = orc.default_tile(2, g)
            slices, kslice = orc.wgrad_split(g, bm, bn, mult)
            assert kslice % 16 == 0 and slices * kslice >= K and (slices - 1) * kslice < K and slices >= 1


def test_conv_epilogue_and_bn_loader():
    x, w, b = rnd(2, 4, 9, 9), rnd(6, 4, 3, 3), rnd(6)
    y = orc.conv_fwd(x, w, b, 1, 1, relu=True)
    assert err(y, torch.relu(F.conv2d(t(x), t(w), t(b), padding=1)).numpy()) < 1e-6
    # kind 3: padding applies to the post-BN/ReLU tensor (out-of-bounds taps are 0, not relu(bn(0)))
    m, v, g, bb = rnd(4), np.abs(rnd(4)) + 0.5, rnd(4), rnd(4)
    z = torch.relu(F.batch_norm(t(x), t(m), t(v), t(g), t(bb), training=False, eps=1e-5))
    ref = F.conv2d(z, t(w), padding=1)
    assert err(orc.conv_fwd(x, w, None, 1, 1, bn=(m, v, g, bb)), ref.numpy()) < 1e-5


def test_fold_bn():
    x, cw, cb = rnd(2, 4, 8, 8), rnd(6, 4, 3, 3), rnd(6)
    w, b, rm, rv = rnd(6), rnd(6), rnd(6), np.abs(rnd(6)) + 0.3
    fw, fb = orc.fold_bn(cw, cb, w, b, rm, rv, 1e-5)
    ref = F.batch_norm(F.conv2d(t(x), t(cw), t(cb), padding=1), t(rm), t(rv), t(w), t(b), training=False, eps=1e-5)
    assert err(orc.conv_fwd(x, fw, fb, 1, 1), ref.numpy()) < 1e-5
    fw0, fb0 = orc.fold_bn(cw, None, w, b, rm, rv, 1e-5)
    ref0 = F.batch_norm(F.conv2d(t(x), t(cw), padding=1), t(rm), t(rv), t(w), t(b), training=False, eps=1e-5)
    assert err(orc.conv_fwd(x, fw0, fb0, 1, 1), ref0.numpy()) < 1e-5


def test_conv_kind_table():
    k = orc.conv_kind
    assert k(3, 64, 11, 11, (4, 4), (2, 2), (1, 1), False, 1) == 1
    assert k(3, 64, 11, 11, (5, 5), (2, 2), (1, 1), False, 1) == 0      # stride 5
    assert k(3, 64, 12, 12, (1, 1), (0, 0), (1, 1), False, 1) == 0      # ks 12
    assert k(3, 64, 3, 3, (1, 1), (4, 4), (1, 1), False, 1) == 0        # pad > ks
    assert k(3, 64, 3, 3, (1, 1), (1, 1), (2, 2), False, 1) == 0        # dilated
    assert k(3, 64, 3, 5, (1, 1), (1, 1), (1, 1), False, 1) == 0        # non-square
    assert k(3, 64, 3, 3, (1, 2), (1, 1), (1, 1), False, 1) == 0        # unequal strides
    assert k(3, 64, 3, 3, (1, 1), (1, 1), (1, 1), True, 1) == 0         # transposed
    assert k(8, 8, 3, 3, (1, 1), (1, 1), (1, 1), False, 8) == 2
    assert k(8, 8, 5, 5, (1, 1), (2, 2), (1, 1), False, 8) == 2
    assert k(8, 8, 7, 7, (1, 1), (3, 3), (1, 1), False, 8) == 2
    assert k(8, 8, 3, 3, (2, 2), (1, 1), (1, 1), False, 8) == 3
    assert k(8, 8, 9, 9, (1, 1), (4, 4), (1, 1), False, 8) == 3
    assert k(8, 16, 3, 3, (1, 1), (1, 1), (1, 1), False, 8) == 0        # channel multiplier
    assert k(8, 8, 3, 3, (1, 1), (1, 1), (1, 1), False, 2) == 0         # grouped, not depthwise


# ---- depthwise ----

@pytest.mark.parametrize("ks,s,p", [(3, 1, 1), (5, 1, 2), (7, 1, 3), (3, 2, 1), (5, 2, 0), (11, 4, 5), (2, 3, 1)])
def test_depthwise_vs_torch_cpu(ks, s, p):
    c = 6
    x, w, b = rnd(3, c, 14, 13), rnd(c, 1, ks, ks), rnd(c)
    tx, tw = t(x).requires_grad_(), t(w).requires_grad_()
    ty = F.conv2d(tx, tw, t(b), stride=s, padding=p, groups=c)
    y = orc.dw_fwd(x, w, b, s, p)
    assert err(y, ty.detach().numpy()) < 1e-5
    gy = rnd(*y.shape)
    ty.backward(t(gy))
    assert err(orc.dw_dgrad(gy, w, x.shape, s, p), tx.grad.numpy()) < 1e-5
    assert err(orc.dw_wgrad(x, gy, ks, s, p), tw.grad.numpy()) < 1e-5


def test_depthwise_bn_loader():
    c = 5
    x, w = rnd(2, c, 9, 9), rnd(c, 1, 3, 3)
    m, v, g, bb = rnd(c), np.abs(rnd(c)) + 0.5, rnd(c), rnd(c)
    z = torch.relu(F.batch_norm(t(x), t(m), t(v), t(g), t(bb), training=False, eps=1e-5))
    ref = F.conv2d(z, t(w), padding=1, groups=c)
    assert err(orc.dw_fwd(x, w, None, 1, 1, bn=(m, v, g, bb)), ref.numpy()) < 1e-5


# ---- batch norm ----

@pytest.mark.parametrize("n,c,h,w", [(4, 6, 5, 7), (16, 8, 4, 4), (2, 3, 1, 1), (9, 4, 3, 3)])
@pytest.mark.parametrize("relu", [False, True])
def test_bn_train_vs_torch_cpu(n, c, h, w, relu):
    x = rnd(n, c, h, w) * 3 + 5  # large mean: the shifted statistics must stay accurate
    g, b, rm, rv = rnd(c), rnd(c), rnd(c), np.abs(rnd(c)) + 0.5
    y, mean, invstd, nrm, nrv = orc.bn_train(x, g, b, rm, rv, 0.1, 1e-5, relu)
    trm, trv = t(rm.copy()), t(rv.copy())
    ty, tmean, tinv = torch.native_batch_norm(t(x), t(g), t(b), trm, trv, True, 0.1, 1e-5)
    if relu:
        ty = torch.relu(ty)
    assert err(y, ty.numpy()) < 1e-5
    assert err(mean, tmean.numpy()) < 1e-6 and err(invstd, tinv.numpy()) < 1e-5
    assert err(nrm, trm.numpy()) < 1e-6 and err(nrv, trv.numpy()) < 1e-6
    gy = rnd(n, c, h, w)
    gz = gy * (y > 0) if relu else gy
    tg, tgg, tgb = torch.ops.aten.native_batch_norm_backward(t(gz), t(x), t(g), trm, trv, tmean, tinv, True, 1e-5,
                                                             [True, True, True])
    gx, dg, db = orc.bn_bwd(gy, x, mean, invstd, g, relu_y=y if relu else None)
    # dx is a difference of near-equal terms (exactly 0 when m = 2), so it is normalized by the gradient's scale
    scale = np.linalg.norm(gz.astype(np.float64)) * np.abs(g * invstd).max()
    assert np.linalg.norm(gx.astype(np.float64) - tg.numpy()) <= 1e-5 * scale
    assert err(dg, tgg.numpy()) < 1e-5 and err(db, tgb.numpy()) < 1e-5


def test_bn_eval_vs_torch_cpu():
    x, g, b, rm, rv = rnd(3, 5, 4, 6), rnd(5), rnd(5), rnd(5), np.abs(rnd(5)) + 0.2
    ref = F.batch_norm(t(x), t(rm), t(rv), t(g), t(b), training=False, eps=1e-3)
    assert err(orc.bn_eval(x, g, b, rm, rv, 1e-3), ref.numpy()) < 1e-6
    assert err(orc.bn_eval(x, g, b, rm, rv, 1e-3, relu=True), torch.relu(ref).numpy()) < 1e-6


# ---- pooling ----

# notes/scripts/alexnet_ops_check.py:12 (max pool) plus dilation / ceil / asymmetric cases
MAXPOOL = [((3, 3), (2, 2), (0, 0), (1, 1), False, 13), ((3, 3), (2, 2), (0, 0), (1, 1), False, 27),
           ((3, 3), (2, 2), (1, 1), (1, 1), False, 14), ((3, 3), (1, 1), (1, 1), (1, 1), False, 9),
           ((2, 2), (2, 2), (0, 0), (1, 1), False, 12), ((5, 5), (3, 3), (2, 2), (1, 1), False, 17),
           ((3, 3), (2, 2), (1, 1), (2, 2), False, 15), ((3, 2), (2, 1), (1, 0), (1, 1), True, 11),
           ((2, 2), (2, 2), (0, 0), (1, 1), True, 13)]


@pytest.mark.parametrize("k,s,p,d,ceil,hw", MAXPOOL)
def test_maxpool_vs_torch_cpu(k, s, p, d, ceil, hw):
    x = rnd(2, 4, hw, hw + 1)
    x[0, 0, 0, :3] = x[0, 0, 0, 0]  # ties: the first maximum wins
    x[1, 2, 3, 4] = np.nan          # NaN propagates with its index
    tx = t(x).requires_grad_()
    ty, tidx = F.max_pool2d(tx, k, s, p, d, ceil_mode=ceil, return_indices=True)
    y, idx = orc.maxpool_fwd(x, k, s, p, d, ceil)
    np.testing.assert_array_equal(idx, tidx.numpy())
    np.testing.assert_array_equal(np.isnan(y), np.isnan(ty.detach().numpy()))
    fin = ~np.isnan(y)
    np.testing.assert_array_equal(y[fin], ty.detach().numpy()[fin])
    gy = rnd(*y.shape)
    ty.backward(t(gy))
    assert err(orc.maxpool_bwd(gy, idx, x.shape), tx.grad.numpy()) < 1e-6


AVGPOOL = [((3, 3), (2, 2), (1, 1), False, True, None, 14), ((3, 3), (2, 2), (1, 1), False, False, None, 14),
           ((2, 2), (2, 2), (0, 0), False, True, None, 12), ((3, 3), (2, 2), (1, 1), True, False, None, 15),
           ((3, 2), (1, 2), (1, 1), True, True, None, 9), ((3, 3), (2, 2), (1, 1), False, True, 5, 10)]


@pytest.mark.parametrize("k,s,p,ceil,incl,div,hw", AVGPOOL)
def test_avgpool_vs_torch_cpu(k, s, p, ceil, incl, div, hw):
    x = rnd(2, 3, hw, hw + 2)
    tx = t(x).requires_grad_()
    ty = F.avg_pool2d(tx, k, s, p, ceil_mode=ceil, count_include_pad=incl, divisor_override=div)
    y = orc.avgpool_fwd(x, k, s, p, ceil, incl, div)
    assert err(y, ty.detach().numpy()) < 1e-6
    gy = rnd(*y.shape)
    ty.backward(t(gy))
    assert err(orc.avgpool_bwd(gy, x.shape, k, s, p, incl, div), tx.grad.numpy()) < 1e-6


@pytest.mark.parametrize("hw,o", [(6, 6), (13, 6), (10, 4), (7, 1), (5, 3)])  # alexnet_ops_check.py:16 + (5, 3)
def test_adaptive_avgpool_vs_torch_cpu(hw, o):
    x = rnd(2, 5, hw, hw + 1)
    tx = t(x).requires_grad_()
    ty = F.adaptive_avg_pool2d(tx, o)
    y = orc.adapool_fwd(x, o, o)
    assert err(y, ty.detach().numpy()) < 1e-6
    gy = rnd(*y.shape)
    ty.backward(t(gy))
    assert err(orc.adapool_bwd(gy, x.shape), tx.grad.numpy()) < 1e-6

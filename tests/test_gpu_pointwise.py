"""The training steps' ops outside the convolution path (residual add, ReLU / hardswish / hardsigmoid and their
gradients, the squeeze-excite channel scale, plane means and sums, the linear layers' matrix products and bias
gradient, log-softmax and the NLL loss, scalar adds of step counts and batch counters): libomt_hip.so's kernels against PyTorch CPU fp32 (the reference's own oracle for these ops:
tools/conformance.py:55-103), through the C ABI and through the device's aten registrations, checked to run on the
library's kernels rather than torch's. Criterion: rel-L2 <= 1e-4 (most results are bit-identical)."""

import ctypes

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import oracle as orc

pytestmark = pytest.mark.gpu

TOL = 1e-4


@pytest.fixture(scope="module")
def omt(cuda):
    import omarchy_mac_torch
    return omarchy_mac_torch


def rel(a, b):
    return orc.rel_l2(a.detach().cpu().double().numpy(), b.detach().cpu().double().numpy())


def activations_input(n, seed):
    """Values around the activations' break points (-3, 0, 3 exactly) plus Gaussian noise at several scales."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(n, generator=g) * 3
    edge = torch.tensor([-3.0, 3.0, 0.0, -0.0, -3.0000002, 2.9999998, 1e-30, -1e-30])
    x[:min(n, 8)] = edge[:min(n, 8)]
    return x


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


@pytest.mark.parametrize("n,offset", [(4096, 0), (1001, 0), (4099, 1), (7, 3)])
def test_pointwise_c_abi(cuda, n, offset):
    """Every omt_pointwise op against PyTorch CPU, on float4-aligned and unaligned operands with ragged tails."""
    from omarchy_mac_torch import _lib
    L = _lib.L
    x = activations_input(n, n)
    g = torch.randn(n, generator=torch.Generator().manual_seed(n + 1))
    cases = {
        _lib.OMT_PW_ADD: (x, g, 0.5, x + 0.5 * g),
        _lib.OMT_PW_MUL: (x, g, 0.0, x * g),
        _lib.OMT_PW_RELU: (x, None, 0.0, torch.relu(x)),
        _lib.OMT_PW_THRESHOLD_BWD: (g, x, 0.25, torch.ops.aten.threshold_backward(g, x, 0.25)),
        _lib.OMT_PW_HARDSWISH: (x, None, 0.0, F.hardswish(x)),
        _lib.OMT_PW_HARDSWISH_BWD: (g, x, 0.0, torch.ops.aten.hardswish_backward(g, x)),
        _lib.OMT_PW_HARDSIGMOID: (x, None, 0.0, F.hardsigmoid(x)),
        _lib.OMT_PW_HARDSIGMOID_BWD: (g, x, 0.0, torch.ops.aten.hardsigmoid_backward(g, x)),
        _lib.OMT_PW_SCALE: (x, None, -1.75, x * -1.75),
        _lib.OMT_PW_FILL: (x, None, 2.5, torch.full((n,), 2.5)),
    }
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for op, (a, b, alpha, ref) in cases.items():
        da = torch.empty(n + offset, device=cuda)[offset:].copy_(a)
        db = torch.empty(n + offset, device=cuda)[offset:].copy_(b) if b is not None else None
        out = torch.full((n + offset,), float("nan"), device=cuda)[offset:]
        _lib.check(L.omt_pointwise(op, n, _ptr(da), _ptr(db) if db is not None else None, alpha, _ptr(out), stream),
                   "omt_pointwise")
        got = out.cpu()
        assert torch.equal(got, ref) or rel(got, ref) <= TOL, (op, rel(got, ref))
    # relu keeps NaN, as PyTorch's does
    nan = torch.tensor([float("nan"), -1.0, 2.0, float("nan")], device=cuda)
    _lib.check(L.omt_pointwise(_lib.OMT_PW_RELU, 4, _ptr(nan), None, 0.0, _ptr(nan), stream), "omt_pointwise")
    assert torch.equal(torch.isnan(nan.cpu()), torch.tensor([True, False, False, True]))


@pytest.mark.parametrize("shape", [(32, 16, 112, 112), (4, 96, 7, 7), (3, 5, 3, 5), (2, 3, 33, 35), (2, 4, 20, 20)])
def test_channel_scale_plane_sum_and_broadcast(cuda, shape):
    """Channel scale, plane sums (a wave per plane below 1024 elements, a workgroup per plane from there, float4 or
    scalar loads) and the plane broadcast of the mean's gradient."""
    from omarchy_mac_torch import _lib
    L = _lib.L
    n, c, h, w = shape
    gen = torch.Generator().manual_seed(sum(shape))
    x, s = torch.randn(shape, generator=gen), torch.rand(n, c, 1, 1, generator=gen)
    dx, ds = x.to(cuda), s.to(cuda)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    y = torch.empty(shape, device=cuda)
    _lib.check(L.omt_channel_scale(n * c, h * w, _ptr(dx), _ptr(ds), _ptr(y), stream), "omt_channel_scale")
    assert torch.equal(y.cpu(), x * s)
    m = torch.empty(n, c, device=cuda)
    _lib.check(L.omt_plane_sum(n * c, h * w, _ptr(dx), 1.0 / (h * w), _ptr(m), stream), "omt_plane_sum")
    assert rel(m, x.mean((2, 3))) <= 1e-6
    _lib.check(L.omt_plane_sum(n * c, h * w, _ptr(dx), 1.0, _ptr(m), stream), "omt_plane_sum")
    assert rel(m, x.double().sum((2, 3))) <= 1e-6
    b = torch.empty(shape, device=cuda)
    _lib.check(L.omt_plane_broadcast(n * c, h * w, _ptr(ds), 0.25, _ptr(b), stream), "omt_plane_broadcast")
    assert torch.equal(b.cpu(), (s * 0.25).expand(shape))


@pytest.mark.parametrize("rows,cols", [(32, 1000), (128, 10), (5, 1), (3, 130), (4, 3000), (3, 5000), (7, 1024)])
def test_log_softmax_and_nll_c_abi(cuda, rows, cols):
    from omarchy_mac_torch import _lib
    L = _lib.L
    gen = torch.Generator().manual_seed(rows * cols)
    x = torch.randn(rows, cols, generator=gen) * 4
    t = torch.randint(0, cols, (rows,), generator=gen)
    t[0] = -100  # ignore_index
    w = torch.rand(cols, generator=gen) + 0.5
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    dx, dt, dw = x.to(cuda), t.to(cuda), w.to(cuda)
    y = torch.empty(rows, cols, device=cuda)
    _lib.check(L.omt_log_softmax_fwd(rows, cols, _ptr(dx), _ptr(y), stream), "omt_log_softmax_fwd")
    ref = torch.log_softmax(x, 1)
    assert rel(y, ref) <= TOL
    g = torch.randn(rows, cols, generator=gen)
    gx = torch.empty(rows, cols, device=cuda)
    _lib.check(L.omt_log_softmax_bwd(rows, cols, _ptr(g.to(cuda)), _ptr(y), _ptr(gx), stream), "omt_log_softmax_bwd")
    assert rel(gx, torch.ops.aten._log_softmax_backward_data(g, ref, 1, torch.float32)) <= TOL
    for weight in (None, w):
        for red in (0, 1, 2):
            out = torch.empty(rows if red == 0 else 1, device=cuda)
            tw = torch.empty(1, device=cuda)
            _lib.check(L.omt_nll_loss_fwd(rows, cols, _ptr(y), _ptr(dt), _ptr(dw) if weight is not None else None,
                                          -100, red, _ptr(out), _ptr(tw), stream), "omt_nll_loss_fwd")
            r_out, r_tw = torch.ops.aten.nll_loss_forward(ref, t, weight, red, -100)
            assert rel(out.cpu().reshape(r_out.shape), r_out) <= TOL and rel(tw.cpu()[0], r_tw) <= TOL, (red, weight)
            go = torch.randn(r_out.shape, generator=gen)
            gx = torch.full((rows, cols), float("nan"), device=cuda)
            _lib.check(L.omt_nll_loss_bwd(rows, cols, _ptr(go.to(cuda).contiguous()), _ptr(dt),
                                          _ptr(dw) if weight is not None else None, -100, red, _ptr(tw), _ptr(gx),
                                          stream), "omt_nll_loss_bwd")
            r_gx = torch.ops.aten.nll_loss_backward(go, ref, t, weight, red, -100, r_tw)
            assert torch.equal(gx.cpu(), r_gx) or rel(gx, r_gx) <= TOL, (red, weight)


DEVICE_OPS = ["add", "add_", "mul", "mul_channel", "div_scalar", "div_plane", "relu", "relu_", "threshold_backward",
              "hardswish", "hardswish_", "hardswish_backward", "hardsigmoid", "hardsigmoid_backward", "fill_", "zero_",
              "sum_planes", "sum_rows", "mean_planes", "log_softmax", "log_softmax_backward", "nll", "nll_backward"]


@pytest.mark.parametrize("case", DEVICE_OPS)
def test_device_ops_run_on_the_library_kernels(omt, case):
    """The aten ops on device tensors: same results as PyTorch CPU, and not delegated to torch's HIP kernels."""
    core = omt.native.core
    dev = omt.DEVICE
    gen = torch.Generator().manual_seed(len(case))
    x = activations_input(2 * 24 * 9 * 11, len(case)).reshape(2, 24, 9, 11)
    y = torch.randn(2, 24, 9, 11, generator=gen)
    s = torch.rand(2, 24, 1, 1, generator=gen)
    logits = torch.randn(16, 37, generator=gen)
    t = torch.randint(0, 37, (16,), generator=gen)
    lp = torch.log_softmax(logits, 1)
    go = torch.randn(16, 37, generator=gen)
    D = (lambda v: v.to(dev))
    fns = {
        "add": lambda d: d(x) + d(y) if d is D else x + y,
        "add_": lambda d: d(x).clone().add_(d(y), alpha=-2.0),
        "mul": lambda d: d(x) * d(y),
        "mul_channel": lambda d: d(x) * d(s),
        "div_scalar": lambda d: d(x) / 7.0,
        "div_plane": lambda d: d(s).expand(2, 24, 9, 11) / 99,
        "relu": lambda d: torch.relu(d(x)),
        "relu_": lambda d: d(x).clone().relu_(),
        "threshold_backward": lambda d: torch.ops.aten.threshold_backward(d(y), d(x), 0.0),
        "hardswish": lambda d: F.hardswish(d(x)),
        "hardswish_": lambda d: F.hardswish(d(x).clone(), inplace=True),
        "hardswish_backward": lambda d: torch.ops.aten.hardswish_backward(d(y), d(x)),
        "hardsigmoid": lambda d: F.hardsigmoid(d(x)),
        "hardsigmoid_backward": lambda d: torch.ops.aten.hardsigmoid_backward(d(y), d(x)),
        "fill_": lambda d: d(x).clone().fill_(-1.5),
        "zero_": lambda d: d(x).clone().zero_(),
        "sum_planes": lambda d: d(x).sum((2, 3), keepdim=True),
        "sum_rows": lambda d: d(logits).sum(0),
        "mean_planes": lambda d: F.adaptive_avg_pool2d(d(x), 1),
        "log_softmax": lambda d: torch.log_softmax(d(logits), 1),
        "log_softmax_backward": lambda d: torch.ops.aten._log_softmax_backward_data(d(go), d(lp), 1, torch.float32),
        "nll": lambda d: F.nll_loss(d(lp), d(t)),
        "nll_backward": lambda d: torch.ops.aten.nll_loss_backward(d(torch.tensor(0.7)), d(lp), d(t), None, 1, -100,
                                                                  d(torch.tensor(16.0))),
    }
    ref = fns[case](lambda v: v)
    torch.cuda.synchronize()
    core.count_delegated(True)
    try:
        got = fns[case](D)
        torch.cuda.synchronize()
        delegated = dict(core.delegated_counts())
    finally:
        core.count_delegated(False)
    assert torch.equal(got.cpu(), ref) or rel(got, ref) <= TOL, case
    ours = ("add", "mul", "div", "relu", "threshold", "hardswish", "hardsigmoid", "fill", "zero", "sum", "mean",
            "softmax", "nll")
    assert not [k for k in delegated if any(o in k for o in ours)], delegated


def test_cross_entropy_training_step_ops_are_native(omt):
    """One MobileNetV3-style training step (hardswish, squeeze-excite, residual adds, linear layers, cross entropy,
    BatchNorm batch counters, AdamW's step counts): no op is left on torch's kernels."""
    from omarchy_mac_torch import models, stacks
    core = omt.native.core
    prev = stacks.set_auto_fuse(False)
    try:
        torch.manual_seed(0)
        model = models.mobilenet_v3_small(1000).to(omt.DEVICE)
        opt = torch.optim.AdamW(model.parameters(), lr=1e-3, weight_decay=0.01)
        x = torch.randn(4, 3, 64, 64).to(omt.DEVICE)
        t = torch.randint(0, 1000, (4,)).to(omt.DEVICE)
        core.count_delegated(True)
        opt.zero_grad(set_to_none=True)
        F.cross_entropy(model(x), t).backward()
        opt.step()
        torch.cuda.synchronize()
        delegated = dict(core.delegated_counts())
    finally:
        core.count_delegated(False)
        stacks.set_auto_fuse(prev)
    assert not delegated, delegated
    assert not omt.FALLBACKS, dict(omt.FALLBACKS.items())


LINEAR_SHAPES = [(32, 512, 1000), (128, 256, 10), (32, 16, 8), (32, 8, 16), (32, 576, 1024), (1, 7, 3), (5, 1, 9),
                 (3, 9, 1)]


@pytest.mark.parametrize("m,k,n", LINEAR_SHAPES)
def test_linear_products_run_on_the_convolution_gemms(omt, m, k, n):
    """The three matrix products of a linear layer's training step (forward addmm with bias, grad input mm, grad
    weight mm in the layouts PyTorch's autograd requests them) against PyTorch CPU, through the device's aten
    registrations, none delegated to torch's GEMMs; ResNet-18's FC (32 x 512 -> 1000), PlainCNN's (128 x 256 -> 10),
    squeeze-excite FCs and single rows / columns."""
    core = omt.native.core
    gen = torch.Generator().manual_seed(m * 7919 + k * 31 + n)
    x, w, b = torch.randn(m, k, generator=gen), torch.randn(n, k, generator=gen), torch.randn(n, generator=gen)
    gy = torch.randn(m, n, generator=gen)
    D = (lambda v: v.to(omt.DEVICE))
    refs = {"forward": torch.addmm(b, x, w.t()), "grad_input": gy @ w, "grad_weight": gy.t() @ x,
            "no_bias": x @ w.t(), "beta0": torch.addmm(torch.full((n,), float("nan")), x, w.t(), beta=0)}
    torch.cuda.synchronize()
    core.count_delegated(True)
    try:
        got = {"forward": torch.addmm(D(b), D(x), D(w).t()), "grad_input": D(gy) @ D(w),
               "grad_weight": D(gy).t() @ D(x), "no_bias": D(x) @ D(w).t(),
               "beta0": torch.addmm(D(torch.full((n,), float("nan"))), D(x), D(w).t(), beta=0)}
        torch.cuda.synchronize()
        delegated = dict(core.delegated_counts())
    finally:
        core.count_delegated(False)
    for key, ref in refs.items():
        assert got[key].shape == ref.shape and rel(got[key], ref) <= TOL, (key, rel(got[key], ref))
    assert not [k for k in delegated if k.split(".")[0] in ("mm", "addmm")], delegated


def test_linear_products_outside_the_covered_layouts(omt):
    """Both operands column-major, strided rows and a general addmm (alpha, beta, a matrix) still give PyTorch's
    results (on torch's GEMMs)."""
    gen = torch.Generator().manual_seed(3)
    a, b = torch.randn(6, 5, generator=gen), torch.randn(7, 6, generator=gen)
    D = (lambda v: v.to(omt.DEVICE))
    assert rel(D(a).t() @ D(b).t(), a.t() @ b.t()) <= TOL
    big = torch.randn(12, 10, generator=gen)
    assert rel(D(big)[::2, :6] @ D(a), big[::2, :6] @ a) <= TOL
    c = torch.randn(6, 7, generator=gen)
    assert rel(torch.addmm(D(c), D(a), D(b).t()[:5], beta=0.5, alpha=2.0),
               torch.addmm(c, a, b.t()[:5], beta=0.5, alpha=2.0)) <= TOL


@pytest.mark.parametrize("m,k,n", [(32, 512, 1000), (128, 256, 10), (32, 16, 8)])
def test_linear_layer_autograd(omt, m, k, n):
    """nn.Linear forward and backward (input, weight and bias gradients) on the device against PyTorch CPU."""
    torch.manual_seed(m + k + n)
    lin = torch.nn.Linear(k, n)
    dlin = torch.nn.Linear(k, n).to(omt.DEVICE)
    dlin.load_state_dict(lin.state_dict())
    x = torch.randn(m, k, requires_grad=True)
    dx = x.detach().to(omt.DEVICE).requires_grad_()
    gy = torch.randn(m, n)
    y, dy = lin(x), dlin(dx)
    y.backward(gy)
    dy.backward(gy.to(omt.DEVICE))
    for got, ref in ((dy, y), (dx.grad, x.grad), (dlin.weight.grad, lin.weight.grad), (dlin.bias.grad, lin.bias.grad)):
        assert got.shape == ref.shape and rel(got, ref) <= TOL
    assert dlin.weight.grad.is_contiguous()


def test_foreach_and_scalar_adds(omt):
    """_foreach_add_ over float32 step counts and int64 batch counters (one launch per 64 tensors; 70 tensors here),
    add_(1) on a 0-dim int64 counter, x + 1.5 and x += 2: exact, and on the library's kernels."""
    core = omt.native.core
    D = (lambda v: v.to(omt.DEVICE))
    steps = [torch.tensor(float(i)) for i in range(70)]
    counts = [torch.tensor(10 ** 12 + i, dtype=torch.int64) for i in range(70)]
    small = torch.arange(300, dtype=torch.float32)
    dsteps, dcounts, dsmall = [D(t) for t in steps], [D(t) for t in counts], D(small)
    torch.cuda.synchronize()
    core.count_delegated(True)
    try:
        torch._foreach_add_(dsteps, 1)
        torch._foreach_add_(dcounts, 3)
        dcounts[0].add_(1)
        y = dsmall + 1.5
        dsmall += 2
        torch.cuda.synchronize()
        delegated = dict(core.delegated_counts())
    finally:
        core.count_delegated(False)
    assert [float(t) for t in dsteps] == [float(i) + 1 for i in range(70)]
    assert [int(t) for t in dcounts] == [10 ** 12 + i + 3 + (i == 0) for i in range(70)]
    assert torch.equal(y.cpu(), small + 1.5) and torch.equal(dsmall.cpu(), small + 2)
    assert not delegated, delegated


@pytest.mark.parametrize("n,c,r", [(32, 16, 8), (32, 96, 24), (32, 576, 144), (5, 2048, 1024), (3, 40, 10), (1, 7, 1)])
def test_squeeze_excite_mlp(omt, n, c, r):
    """omt::se_mlp (s = hardsigmoid(a2), a2 = W2 h + b2, h = relu(W1 z + b1), two launches, returning s, h, a2) and
    omt::se_mlp_backward (two launches, from the saved z, h, a2) on the device against PyTorch CPU's linear -> relu ->
    linear -> hardsigmoid and its autograd, at rel-L2 1e-5 (the sums run in another order than the CPU's GEMMs), at
    MobileNetV3's sizes and the kernels' limits (2048 channels, 1024 hidden); a hidden unit exactly zero (the ReLU
    mask) for every image; no fallback."""
    omt.FALLBACKS.clear()
    g = torch.Generator().manual_seed(n + c + r)
    z = torch.randn(n, c, generator=g)
    w1, b1 = torch.randn(r, c, generator=g) * c ** -0.5, torch.randn(r, generator=g)
    w2, b2 = torch.randn(c, r, generator=g) * r ** -0.5 * 3, torch.randn(c, generator=g)
    b1[0] = -1e4  # hidden unit 0 exactly zero (ReLU mask) for every image
    cpu = [t.clone().requires_grad_() for t in (z, w1, b1, w2, b2)]
    h = F.relu(F.linear(cpu[0], cpu[1], cpu[2]))
    a2 = F.linear(h, cpu[3], cpu[4])
    s = F.hardsigmoid(a2)
    gs = torch.randn(n, c, generator=g)
    grads = torch.autograd.grad(s, cpu, gs)
    dev = [t.to(omt.DEVICE) for t in (z, w1, b1, w2, b2)]
    ds, dh, da2 = torch.ops.omt.se_mlp(*dev)
    assert rel(ds, s) <= 1e-5 and rel(dh, h) <= 1e-5 and rel(da2, a2) <= 1e-5
    assert torch.all(dh.cpu()[:, 0] == 0)
    dgrads = torch.ops.omt.se_mlp_backward(gs.to(omt.DEVICE), dev[0], dh, da2, dev[1], dev[3])
    for got, ref in zip(dgrads, grads):
        assert got.shape == ref.shape and rel(got, ref) <= 1e-5
    assert not omt.FALLBACKS, dict(omt.FALLBACKS)


@pytest.mark.parametrize("n,c,h,w", [(32, 576, 7, 7), (32, 16, 112, 112), (3, 5, 9, 11), (32, 96, 28, 28)])
def test_squeeze_excite_backward_ops(omt, n, c, h, w):
    """omt::plane_dot (the gate's gradient, sum over each plane of g * x) and omt::se_gate_backward (g * s plus the
    plane mean's broadcast gradient v / hw) on the device: the same bits as the separate multiply, plane sum,
    channel scale, broadcast and add they replace (wave-per-plane and workgroup-per-plane sums, float4 and scalar
    planes, channels-last planes), and against float64 CPU sums; no fallback."""
    omt.FALLBACKS.clear()
    g = torch.Generator().manual_seed(n + c + h)
    go, x = torch.randn(n, c, h, w, generator=g), torch.randn(n, c, h, w, generator=g)
    s, v = torch.rand(n, c, 1, 1, generator=g), torch.randn(n, c, 1, 1, generator=g)
    dg, dx, ds, dv = (t.to(omt.DEVICE) for t in (go, x, s, v))
    dot = torch.ops.omt.plane_dot(dg, dx)
    assert torch.equal(dot.cpu(), (dg * dx).sum((2, 3), keepdim=True).cpu())
    assert rel(dot, (go.double() * x.double()).sum((2, 3), keepdim=True)) <= 1e-6
    gate = torch.ops.omt.se_gate_backward(dg, ds, dv, 1.0 / (h * w))
    assert torch.equal(gate.cpu(), (dg * ds + dv.expand(n, c, h, w) / (h * w)).cpu())
    assert rel(gate, go.double() * s.double() + v.double() / (h * w)) <= 1e-6
    gate_cl = torch.ops.omt.se_gate_backward(dg.contiguous(memory_format=torch.channels_last), ds, dv, 1.0 / (h * w))
    assert gate_cl.is_contiguous(memory_format=torch.channels_last) and torch.equal(gate_cl.cpu(), gate.cpu())
    assert not omt.FALLBACKS, dict(omt.FALLBACKS)

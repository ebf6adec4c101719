"""The torch.compile backend's graph rewrites, on the CPU: hand-built aten graphs of the shape AOTAutograd hands the
backend (training BatchNorm with its running-stat and batch-counter updates kept in the graph as copies into the
inputs), with fake device tensors as node metadata so that the rewrites apply. Each rewritten graph is then run on
CPU tensors (omt.bn_train_ has a composite CPU implementation) against the original graph on the same inputs:
outputs and every mutated buffer must agree. Reference pattern rules: omarchy_mac_torch/compile.py:67-161."""

import copy
import operator

import pytest
import torch
from torch.fx import Graph, GraphModule
from torch._subclasses.fake_tensor import FakeTensorMode

aten = torch.ops.aten


@pytest.fixture(scope="module")
def oc():
    from omarchy_mac_torch import compile as oc
    return oc


def _fake(mode, dev, shape, dtype=torch.float32):
    with mode:
        return torch.empty(shape, dtype=dtype, device=dev)


def _block_tail_graph(oc, tail, save_stats=False):
    """Forward graph of BatchNorm(x) followed by `tail` ("relu", "add_relu", "add", "hardswish" or "none"), plus two
    batch counters.
    save_stats: the new running statistics are also graph outputs (AOTAutograd saves them for the backward)."""
    dev = oc.DEVICE
    mode = FakeTensorMode()
    g = Graph()
    shp, c = (2, 4, 3, 3), 4

    def ph(name, shape, dtype=torch.float32):
        n = g.placeholder(name)
        n.meta["val"] = _fake(mode, dev, shape, dtype)
        return n

    x, w, b, rm, rv, r = ph("x", shp), ph("w", (c,)), ph("b", (c,)), ph("rm", (c,)), ph("rv", (c,)), ph("r", shp)
    t1, t2 = ph("nbt1", (), torch.int64), ph("nbt2", (), torch.int64)
    bn = g.call_function(aten._native_batch_norm_legit_functional.default, (x, w, b, rm, rv, True, 0.1, 1e-5))
    gi = [g.call_function(operator.getitem, (bn, i)) for i in range(5)]
    gi[0].meta["val"] = _fake(mode, dev, shp)
    y = gi[0]
    if tail == "relu":
        y = g.call_function(aten.relu.default, (gi[0],))
    elif tail == "hardswish":
        y = g.call_function(aten.hardswish.default, (gi[0],))
    elif tail == "add_relu":
        s = g.call_function(aten.add.Tensor, (gi[0], r))
        s.meta["val"] = _fake(mode, dev, shp)
        y = g.call_function(aten.relu.default, (s,))
    elif tail == "add":  # a residual add with no activation (MobileNetV3's inverted residuals)
        y = g.call_function(aten.add.Tensor, (r, gi[0]))
    y.meta["val"] = _fake(mode, dev, shp)
    a1 = g.call_function(aten.add.Tensor, (t1, 1))
    a2 = g.call_function(aten.add.Tensor, (t2, 1))
    g.call_function(aten.copy_.default, (rm, gi[3]))
    g.call_function(aten.copy_.default, (rv, gi[4]))
    g.call_function(aten.copy_.default, (t1, a1))
    g.call_function(aten.copy_.default, (t2, a2))
    # hardswish: its input is saved for its backward, a graph output too
    g.output((y, gi[1], gi[2]) + ((gi[3], gi[4]) if save_stats else ()) + ((gi[0],) if tail == "hardswish" else ()))
    return GraphModule(torch.nn.Module(), g)


def _inputs(seed):
    gen = torch.Generator().manual_seed(seed)
    shp, c = (2, 4, 3, 3), 4
    return [torch.randn(shp, generator=gen), torch.rand(c, generator=gen) + 0.5, torch.randn(c, generator=gen),
            torch.randn(c, generator=gen), torch.rand(c, generator=gen) + 0.5, torch.randn(shp, generator=gen),
            torch.tensor(3, dtype=torch.int64), torch.tensor(7, dtype=torch.int64)]


def _targets(gm):
    return [n.target for n in gm.graph.nodes if n.op == "call_function"]


@pytest.mark.parametrize("save_stats", [False, True])
@pytest.mark.parametrize("tail", ["relu", "add_relu", "add", "none", "hardswish"])
def test_bn_train_in_place_and_counters(oc, tail, save_stats):
    gm = _block_tail_graph(oc, tail, save_stats)
    ref = copy.deepcopy(gm)
    stats = oc.fuse_bn_train_in_place(gm.graph)
    assert stats["bn"] == 1 and stats["add_relu"] == (tail == "add_relu") and stats["relu"] == (tail == "relu")
    assert stats["add"] == (tail == "add")
    assert stats["hardswish"] == (tail == "hardswish")
    assert oc.merge_batch_counters(gm.graph) == 2
    gm.graph.eliminate_dead_code()
    gm.graph.lint()
    gm.recompile()
    t = _targets(gm)
    assert t.count(torch.ops.omt.bn_train_.default) == 1 and t.count(aten._foreach_add_.Scalar) == 1
    assert aten.copy_.default not in t and aten._native_batch_norm_legit_functional.default not in t
    assert aten.relu.default not in t and aten.add.Tensor not in t and aten.hardswish.default not in t
    fused = next(n for n in gm.graph.nodes if n.target is torch.ops.omt.bn_train_.default)
    assert fused.args[7] == {"none": 0, "relu": 1, "add_relu": 1, "add": 0, "hardswish": 2}[tail]
    assert (fused.args[8] is not None) == (tail in ("add_relu", "add"))
    # same results and buffer updates as the original graph, on CPU tensors
    a, b = _inputs(1), _inputs(1)
    out_ref, out_new = ref(*a), gm(*b)
    for o_ref, o_new in zip(out_ref, out_new):
        torch.testing.assert_close(o_new, o_ref, rtol=1e-5, atol=1e-6)
    for i in (3, 4, 6, 7):  # rm, rv, both counters
        torch.testing.assert_close(b[i], a[i], rtol=1e-6, atol=1e-7)
    assert int(b[6]) == 4 and int(b[7]) == 8


def test_bn_in_place_needs_sole_copies(oc):
    """A running-stat input read elsewhere in the graph keeps the functional BatchNorm (no in-place update)."""
    gm = _block_tail_graph(oc, "relu")
    rm = next(n for n in gm.graph.nodes if n.op == "placeholder" and n.name == "rm")
    out = next(n for n in gm.graph.nodes if n.op == "output")
    with gm.graph.inserting_before(out):
        extra = gm.graph.call_function(aten.mul.Tensor, (rm, 2))
    out.args = (out.args[0] + (extra,),)
    assert oc.fuse_bn_train_in_place(gm.graph)["bn"] == 0
    # the ReLU still fuses through the functional rewrite
    assert oc.fuse_bn_relu_train(gm.graph) == 1


def test_bn_hardswish_backward(oc):
    """native_batch_norm_backward(hardswish_backward(g, z), x, ...) becomes one omt.bn_act_backward (act 2) that takes
    the hardswish gradient itself; the rewritten graph gives the original's gradients on CPU tensors, with z at the
    hardswish's break points -3 and 3 and between them."""
    dev = oc.DEVICE
    mode = FakeTensorMode()
    g = Graph()
    shp, c = (2, 4, 3, 3), 4

    def ph(name, shape):
        n = g.placeholder(name)
        n.meta["val"] = _fake(mode, dev, shape)
        return n

    gy, z, x, w, mean, invstd = ph("g", shp), ph("z", shp), ph("x", shp), ph("w", (c,)), ph("mean", (c,)), \
        ph("invstd", (c,))
    hb = g.call_function(aten.hardswish_backward.default, (gy, z))
    hb.meta["val"] = _fake(mode, dev, shp)
    bn = g.call_function(aten.native_batch_norm_backward.default,
                         (hb, x, w, None, None, mean, invstd, True, 1e-5, [True, True, True]))
    g.output(tuple(g.call_function(operator.getitem, (bn, i)) for i in range(3)))
    gm = GraphModule(torch.nn.Module(), g)
    ref = copy.deepcopy(gm)
    assert oc.fuse_bn_hardswish_backward(gm.graph) == 1
    gm.graph.eliminate_dead_code()
    gm.graph.lint()
    gm.recompile()
    t = _targets(gm)
    assert torch.ops.omt.bn_act_backward.default in t and aten.hardswish_backward.default not in t
    assert aten.native_batch_norm_backward.default not in t
    gen = torch.Generator().manual_seed(4)
    zv = torch.randn(shp, generator=gen) * 3
    zv.view(-1)[:4] = torch.tensor([-3.0, 3.0, 0.0, -1.5])
    args = [torch.randn(shp, generator=gen), zv, torch.randn(shp, generator=gen), torch.rand(c, generator=gen) + 0.5,
            torch.randn(c, generator=gen), torch.rand(c, generator=gen) + 0.5]
    for o_ref, o_new in zip(ref(*args), gm(*args)):
        torch.testing.assert_close(o_new, o_ref, rtol=1e-6, atol=1e-7)


def _block_end_backward_graph(oc, with_add, second_user):
    """Backward graph of a residual block's end, relu(bn(x) + r): t = threshold_backward(a, y, 0) with
    a = g_main + g_res (with_add) or a plain input, feeding the block's BatchNorm backward and a second user:
    the shortcut's add ("add") or the projection shortcut's BatchNorm backward ("bn")."""
    dev = oc.DEVICE
    mode = FakeTensorMode()
    g = Graph()
    shp, c = (2, 4, 3, 3), 4

    def ph(name, shape):
        n = g.placeholder(name)
        n.meta["val"] = _fake(mode, dev, shape)
        return n

    gm_, gr, y, x, w, mean, invstd = (ph("g_main", shp), ph("g_res", shp), ph("y", shp), ph("x", shp), ph("w", (c,)),
                                      ph("mean", (c,)), ph("invstd", (c,)))
    x2, w2, mean2, invstd2, other = ph("x2", shp), ph("w2", (c,)), ph("mean2", (c,)), ph("invstd2", (c,)), ph("o", shp)
    a = gm_
    if with_add:
        a = g.call_function(aten.add.Tensor, (gm_, gr))
        a.meta["val"] = _fake(mode, dev, shp)
    yd = g.call_function(aten.detach.default, (y,))  # as AOTAutograd emits it: after the add, right before the mask
    yd.meta["val"] = _fake(mode, dev, shp)
    t = g.call_function(aten.threshold_backward.default, (a, yd, 0))
    t.meta["val"] = _fake(mode, dev, shp)
    bn = g.call_function(aten.native_batch_norm_backward.default,
                         (t, x, w, None, None, mean, invstd, True, 1e-5, [True, True, True]))
    outs = [g.call_function(operator.getitem, (bn, i)) for i in range(3)]
    if second_user == "add":
        u = g.call_function(aten.add.Tensor, (t, other))
        extra = (u,)
    else:
        bn2 = g.call_function(aten.native_batch_norm_backward.default,
                              (t, x2, w2, None, None, mean2, invstd2, True, 1e-5, [True, True, True]))
        extra = tuple(g.call_function(operator.getitem, (bn2, i)) for i in range(3))
    g.output(tuple(outs) + extra)
    return GraphModule(torch.nn.Module(), g)


@pytest.mark.parametrize("with_add", [True, False])
@pytest.mark.parametrize("second_user", ["add", "bn"])
def test_bn_relu_res_backward(oc, with_add, second_user):
    """The masked gradient of a block's end feeds its BatchNorm backward and the shortcut: add + threshold_backward +
    that BatchNorm backward become one omt.bn_relu_res_backward whose fourth output feeds the shortcut; the rewritten
    graph gives the original's results on CPU tensors."""
    gm = _block_end_backward_graph(oc, with_add, second_user)
    ref = copy.deepcopy(gm)
    assert oc.fuse_bn_relu_res_backward(gm.graph) == 1
    gm.graph.eliminate_dead_code()
    gm.graph.lint()
    gm.recompile()
    t = _targets(gm)
    assert t.count(torch.ops.omt.bn_relu_res_backward.default) == 1 and aten.threshold_backward.default not in t
    assert t.count(aten.native_batch_norm_backward.default) == (1 if second_user == "bn" else 0)
    assert t.count(aten.add.Tensor) == (1 if second_user == "add" else 0)
    fused = next(n for n in gm.graph.nodes if n.target is torch.ops.omt.bn_relu_res_backward.default)
    assert (fused.args[1] is not None) == with_add
    gen = torch.Generator().manual_seed(3)
    shp, c = (2, 4, 3, 3), 4
    args = [torch.randn(shp, generator=gen) for _ in range(4)] + [torch.rand(c, generator=gen) + 0.5,
                                                                  torch.randn(c, generator=gen),
                                                                  torch.rand(c, generator=gen) + 0.5]
    args += [torch.randn(shp, generator=gen), torch.rand(c, generator=gen) + 0.5, torch.randn(c, generator=gen),
             torch.rand(c, generator=gen) + 0.5, torch.randn(shp, generator=gen)]
    for o_ref, o_new in zip(ref(*args), gm(*args)):
        torch.testing.assert_close(o_new, o_ref, rtol=1e-5, atol=1e-6)


def _conv_bn_graph(oc, bias, early_user, res):
    """Forward graph of convolution -> omt.bn_train_ (as rewrite 0 leaves it), the convolution's output also a graph
    output (saved for the BatchNorm backward); `early_user`: an op reads the convolution output before the BatchNorm."""
    dev = oc.DEVICE
    mode = FakeTensorMode()
    g = Graph()
    xs, ws, ys, c = (2, 3, 6, 6), (4, 3, 3, 3), (2, 4, 6, 6), 4

    def ph(name, shape):
        n = g.placeholder(name)
        n.meta["val"] = _fake(mode, dev, shape)
        return n

    x, cw, cb, w, b, rm, rv, r = (ph("x", xs), ph("cw", ws), ph("cb", (c,)), ph("w", (c,)), ph("b", (c,)),
                                  ph("rm", (c,)), ph("rv", (c,)), ph("r", ys))
    conv = g.call_function(aten.convolution.default, (x, cw, cb if bias else None, [1, 1], [1, 1], [1, 1], False,
                                                      [0, 0], 1))
    conv.meta["val"] = _fake(mode, dev, ys)
    extra = ()
    if early_user:
        e = g.call_function(aten.mul.Tensor, (conv, 2.0))
        e.meta["val"] = _fake(mode, dev, ys)
        extra = (e,)
    bn = g.call_function(torch.ops.omt.bn_train_.default, (conv, w, b, rm, rv, 0.1, 1e-5, 1, r if res else None))
    outs = []
    for i, shp in enumerate((ys, (c,), (c,))):
        gi = g.call_function(operator.getitem, (bn, i))
        gi.meta["val"] = _fake(mode, dev, shp)
        outs.append(gi)
    g.output(tuple(outs) + (conv,) + extra)
    return GraphModule(torch.nn.Module(), g)


@pytest.mark.parametrize("case", ["plain", "residual", "bias", "early_user"])
def test_conv_bn_train(oc, case):
    """A bias-free dense convolution feeding omt.bn_train_ becomes one omt.conv_bn_train_ whose fifth output replaces
    the convolution's other uses; with a bias, or a use of the convolution before the BatchNorm, the graph stays as it
    is. The rewritten graph gives the original's outputs and running statistics on CPU tensors."""
    gm = _conv_bn_graph(oc, case == "bias", case == "early_user", case == "residual")
    ref = copy.deepcopy(gm)
    expect = 1 if case in ("plain", "residual") else 0
    assert oc.fuse_conv_bn_train(gm.graph) == expect
    gm.graph.eliminate_dead_code()
    gm.graph.lint()
    gm.recompile()
    t = _targets(gm)
    assert t.count(torch.ops.omt.conv_bn_train_.default) == expect
    assert t.count(aten.convolution.default) == 1 - expect and t.count(torch.ops.omt.bn_train_.default) == 1 - expect
    gen = torch.Generator().manual_seed(5)
    args = [torch.randn(2, 3, 6, 6, generator=gen), torch.randn(4, 3, 3, 3, generator=gen) * 0.3,
            torch.randn(4, generator=gen), torch.rand(4, generator=gen) + 0.5, torch.randn(4, generator=gen),
            torch.randn(4, generator=gen), torch.rand(4, generator=gen) + 0.5, torch.randn(2, 4, 6, 6, generator=gen)]
    a, b = [t.clone() for t in args], [t.clone() for t in args]
    for o_ref, o_new in zip(ref(*a), gm(*b)):
        torch.testing.assert_close(o_new, o_ref, rtol=1e-5, atol=1e-6)
    for i in (5, 6):  # running statistics, updated in place
        torch.testing.assert_close(b[i], a[i], rtol=1e-6, atol=1e-7)


def test_conv_bn_train_after_a_rewrite_that_uses_the_conv(oc):
    """Two bias-free convolutions of x: the first feeds a BatchNorm whose residual is the second convolution's raw
    output, and the second feeds a BatchNorm of its own. Rewriting the first pair inserts a fused node that uses the
    second convolution before its BatchNorm, so the second pair must stay as it is (the pass looks nodes up in a fresh
    order after each rewrite). The rewritten graph gives the original's outputs and running statistics on CPU."""
    dev = oc.DEVICE
    mode = FakeTensorMode()
    g = Graph()
    xs, ys, c = (2, 3, 6, 6), (2, 4, 6, 6), 4

    def ph(name, shape):
        n = g.placeholder(name)
        n.meta["val"] = _fake(mode, dev, shape)
        return n

    x, wa, wb = ph("x", xs), ph("wa", (c, 3, 3, 3)), ph("wb", (c, 3, 3, 3))
    bn_args = [[ph(f"{k}{j}", (c,)) for k in ("w", "b", "rm", "rv")] for j in (1, 2)]
    convs = []
    for w in (wa, wb):
        cv = g.call_function(aten.convolution.default, (x, w, None, [1, 1], [1, 1], [1, 1], False, [0, 0], 1))
        cv.meta["val"] = _fake(mode, dev, ys)
        convs.append(cv)
    outs = []
    for (w, b, rm, rv), src, res in zip(bn_args, convs, (convs[1], None)):
        bn = g.call_function(torch.ops.omt.bn_train_.default, (src, w, b, rm, rv, 0.1, 1e-5, 1, res))
        for i, shp in enumerate((ys, (c,), (c,))):
            gi = g.call_function(operator.getitem, (bn, i))
            gi.meta["val"] = _fake(mode, dev, shp)
            outs.append(gi)
    g.output(tuple(outs))
    gm = GraphModule(torch.nn.Module(), g)
    ref = copy.deepcopy(gm)
    assert oc.fuse_conv_bn_train(gm.graph) == 1
    gm.graph.eliminate_dead_code()
    gm.graph.lint()
    gm.recompile()
    t = _targets(gm)
    assert t.count(torch.ops.omt.conv_bn_train_.default) == 1 and t.count(aten.convolution.default) == 1
    gen = torch.Generator().manual_seed(9)
    args = [torch.randn(xs, generator=gen), torch.randn(c, 3, 3, 3, generator=gen) * 0.3,
            torch.randn(c, 3, 3, 3, generator=gen) * 0.3]
    for _ in range(2):
        args += [torch.rand(c, generator=gen) + 0.5, torch.randn(c, generator=gen), torch.randn(c, generator=gen),
                 torch.rand(c, generator=gen) + 0.5]
    a, b = [v.clone() for v in args], [v.clone() for v in args]
    for o_ref, o_new in zip(ref(*a), gm(*b)):
        torch.testing.assert_close(o_new, o_ref, rtol=1e-5, atol=1e-6)
    for i in (5, 6, 9, 10):  # running statistics, updated in place
        torch.testing.assert_close(b[i], a[i], rtol=1e-6, atol=1e-7)


def _conv_bn_backward_graph(oc, kind, case):
    """Backward graph of BatchNorm -> activation -> convolution: convolution_backward(gy, cx, cw) whose grad input
    feeds the BatchNorm backward `kind` ("relu", "hardswish", "res_g", "res_g2", "plain"). case: "fusable", or what
    keeps it apart: "second_use" (the grad input used elsewhere too), "bias" (a bias grad asked for), "early_gw" (the
    grad weight used before the BatchNorm backward)."""
    dev = oc.DEVICE
    mode = FakeTensorMode()
    g = Graph()
    xs, c, ys = (2, 4, 5, 5), 4, (2, 6, 3, 3)

    def ph(name, shape):
        n = g.placeholder(name)
        n.meta["val"] = _fake(mode, dev, shape)
        return n

    gy, cx, cw = ph("gy", ys), ph("cx", xs), ph("cw", (6, 4, 3, 3))
    x, r, w, mean, invstd, other = ph("x", xs), ph("r", xs), ph("w", (c,)), ph("mean", (c,)), ph("invstd", (c,)), \
        ph("other", xs)
    mask = [True, True, case == "bias"]
    cb = g.call_function(aten.convolution_backward.default,
                         (gy, cx, cw, [6] if case == "bias" else None, [2, 2], [1, 1], [1, 1], False, [0, 0], 1, mask))
    gx = g.call_function(operator.getitem, (cb, 0))
    gx.meta["val"] = _fake(mode, dev, xs)
    gw = g.call_function(operator.getitem, (cb, 1))
    gw.meta["val"] = _fake(mode, dev, (6, 4, 3, 3))
    extra = ()
    if case == "bias":
        extra = (g.call_function(operator.getitem, (cb, 2)),)
    if case == "early_gw":
        extra = (g.call_function(aten.mul.Tensor, (gw, 2.0)),)
    if case == "second_use":
        extra = (g.call_function(aten.mul.Tensor, (gx, 3.0)),)
    m3 = [True, True, True]
    if kind == "relu":
        bn = g.call_function(torch.ops.omt.bn_relu_backward.default, (gx, x, r, w, mean, invstd, m3))
    elif kind == "hardswish":
        bn = g.call_function(torch.ops.omt.bn_act_backward.default, (gx, x, r, w, mean, invstd, 2, m3))
    elif kind == "res_g":
        bn = g.call_function(torch.ops.omt.bn_relu_res_backward.default, (gx, other, x, r, w, mean, invstd, m3))
    elif kind == "res_g2":
        bn = g.call_function(torch.ops.omt.bn_relu_res_backward.default, (other, gx, x, r, w, mean, invstd, m3))
    else:
        bn = g.call_function(aten.native_batch_norm_backward.default,
                             (gx, x, w, None, None, mean, invstd, True, 1e-5, m3))
    outs = tuple(g.call_function(operator.getitem, (bn, i)) for i in range(4 if kind.startswith("res") else 3))
    g.output((gw,) + outs + extra)
    return GraphModule(torch.nn.Module(), g)


@pytest.mark.parametrize("kind", ["relu", "hardswish", "res_g", "res_g2", "plain"])
@pytest.mark.parametrize("case", ["fusable", "second_use", "bias", "early_gw"])
def test_conv_bn_backward(oc, kind, case):
    """A convolution backward whose grad input only feeds a BatchNorm backward becomes, with it, one
    omt.conv_bn_backward (outputs: the grad weight, then the BatchNorm backward's); at a block's end either gradient may
    be the convolution's. The rewritten graph gives the original's results on CPU tensors (the composite reference);
    a grad input used elsewhere, a bias grad, or a grad weight used before the BatchNorm backward keeps them apart."""
    gm = _conv_bn_backward_graph(oc, kind, case)
    ref = copy.deepcopy(gm)
    fused = oc.fuse_conv_bn_backward(gm.graph)
    gm.graph.eliminate_dead_code()
    gm.graph.lint()
    gm.recompile()
    t = _targets(gm)
    assert fused == (1 if case == "fusable" else 0)
    assert t.count(torch.ops.omt.conv_bn_backward.default) == fused
    assert t.count(aten.convolution_backward.default) == 1 - fused
    if fused:
        node = next(n for n in gm.graph.nodes if n.target is torch.ops.omt.conv_bn_backward.default)
        assert node.args[11] == {"relu": 1, "hardswish": 2, "plain": 0}.get(kind, 1)
        assert node.args[12] == kind.startswith("res") and (node.args[5] is not None) == kind.startswith("res")
    gen = torch.Generator().manual_seed(5)
    xs, c = (2, 4, 5, 5), 4
    r = torch.randn(xs, generator=gen) * 3
    if kind != "hardswish":
        r = r.relu()  # a ReLU's output, zeros included
    args = [torch.randn((2, 6, 3, 3), generator=gen), torch.randn(xs, generator=gen),
            torch.randn((6, 4, 3, 3), generator=gen), torch.randn(xs, generator=gen), r,
            torch.rand(c, generator=gen) + 0.5, torch.randn(c, generator=gen), torch.rand(c, generator=gen) + 0.5,
            torch.randn(xs, generator=gen)]
    for o_ref, o_new in zip(ref(*args), gm(*args)):
        torch.testing.assert_close(o_new, o_ref, rtol=1e-6, atol=1e-6)


def _bn_pool_graph(oc, residual, z_used, pool_args):
    """Forward graph of omt.bn_train_ (as rewrite 0 leaves it) whose output feeds max_pool2d_with_indices and is also
    a graph output (saved for the backward's mask)."""
    dev = oc.DEVICE
    mode = FakeTensorMode()
    g = Graph()
    shp, c = (2, 4, 9, 9), 4

    def ph(name, shape):
        n = g.placeholder(name)
        n.meta["val"] = _fake(mode, dev, shape)
        return n

    x, w, b, rm, rv, r = ph("x", shp), ph("w", (c,)), ph("b", (c,)), ph("rm", (c,)), ph("rv", (c,)), ph("r", shp)
    bn = g.call_function(torch.ops.omt.bn_train_.default, (x, w, b, rm, rv, 0.1, 1e-5, 1, r if residual else None))
    outs = [g.call_function(operator.getitem, (bn, i)) for i in range(4 if z_used else 3)]
    outs[0].meta["val"] = _fake(mode, dev, shp)
    mp = g.call_function(aten.max_pool2d_with_indices.default, (outs[0],) + pool_args)
    pooled = [g.call_function(operator.getitem, (mp, i)) for i in range(2)]
    g.output(tuple(outs) + tuple(pooled))
    return GraphModule(torch.nn.Module(), g)


@pytest.mark.parametrize("case", ["3x3s2p1", "2x2", "k1_list", "residual", "z_used", "dilated", "ceil"])
def test_bn_train_pool(oc, case):
    """omt.bn_train_ -> max_pool2d_with_indices of its output becomes one omt.bn_train_pool_ (outputs: the BatchNorm's,
    then the pool's), the BatchNorm output kept for its other users; the rewritten graph gives the original's outputs
    and running statistics on CPU tensors. A residual, a used fourth output, dilation or ceil mode keeps them apart."""
    pool_args = {"3x3s2p1": ([3, 3], [2, 2], [1, 1]), "2x2": ([2, 2],), "k1_list": ([2], [2]),
                 "dilated": ([3, 3], [2, 2], [1, 1], [2, 2]), "ceil": ([3, 3], [2, 2], [0, 0], [1, 1], True)}
    args = pool_args.get(case, ([3, 3], [2, 2], [1, 1]))
    gm = _bn_pool_graph(oc, case == "residual", case == "z_used", tuple(args))
    ref = copy.deepcopy(gm)
    fused = oc.fuse_bn_train_pool(gm.graph)
    gm.graph.eliminate_dead_code()
    gm.graph.lint()
    gm.recompile()
    t = _targets(gm)
    apart = case in ("residual", "z_used", "dilated", "ceil")
    assert fused == (0 if apart else 1)
    assert t.count(aten.max_pool2d_with_indices.default) == (1 if apart else 0)
    gen = torch.Generator().manual_seed(6)
    shp, c = (2, 4, 9, 9), 4
    inputs = [torch.randn(shp, generator=gen), torch.rand(c, generator=gen) + 0.5, torch.randn(c, generator=gen),
              torch.randn(c, generator=gen), torch.rand(c, generator=gen) + 0.5, torch.randn(shp, generator=gen)]
    a1, a2 = [t.clone() for t in inputs], [t.clone() for t in inputs]
    for o_ref, o_new in zip(ref(*a1), gm(*a2)):
        if o_ref is None:
            assert o_new is None
            continue
        assert torch.equal(o_new, o_ref)
    for i in (3, 4):  # running statistics updated in place the same way
        assert torch.equal(a1[i], a2[i])


def _se_graph(oc, case):
    """Dynamo-style graph (torch-level calls, example values on the device) of a squeeze-excite excitation:
    hardsigmoid(linear(relu(linear(z, w1, b1)), w2, b2)), with the variations `case` names."""
    dev = oc.DEVICE
    mode = FakeTensorMode()
    g = Graph()
    n, c, r = 4, (2100 if case == "too_wide" else 16), 4

    def ph(name, shape):
        node = g.placeholder(name)
        node.meta["example_value"] = _fake(mode, dev, shape)
        return node

    z, w1, b1, w2, b2 = ph("z", (n, c)), ph("w1", (r, c)), ph("b1", (r,)), ph("w2", (c, r)), ph("b2", (c,))
    l1 = g.call_function(torch._C._nn.linear, (z, w1, None if case == "no_bias" else b1))
    h = g.call_function(torch.nn.functional.relu, (l1,), {"inplace": True} if case == "inplace" else {})
    l2 = g.call_function(torch._C._nn.linear, (h, w2, b2))
    s = g.call_function(torch.nn.functional.hardsigmoid, (l2,))
    outs = (s,) + ((h,) if case == "second_use" else ())
    g.output(outs)
    return GraphModule(torch.nn.Module(), g), (n, c, r)


@pytest.mark.parametrize("case", ["fusable", "second_use", "no_bias", "inplace", "too_wide"])
def test_squeeze_excite_rewrite(oc, case):
    """Dynamo's graph of a squeeze-excite excitation (linear -> relu -> linear -> hardsigmoid) becomes one omt.se_mlp,
    whose output and gradients (its registered backward, omt.se_mlp_backward) equal the original's on CPU tensors;
    a second use of an intermediate, a missing bias, an in-place ReLU or more than 2048 channels keeps it apart."""
    gm, (n, c, r) = _se_graph(oc, case)
    ref = copy.deepcopy(gm)
    fused = oc.fuse_squeeze_excite(gm.graph)
    gm.graph.lint()
    gm.recompile()
    assert fused == (1 if case == "fusable" else 0)
    assert _targets(gm).count(torch.ops.omt.se_mlp.default) == fused
    if case != "fusable":
        return
    gen = torch.Generator().manual_seed(8)
    args = [torch.randn(s, generator=gen, requires_grad=True) for s in ((n, c), (r, c), (r,), (c, r), (c,))]
    args2 = [a.detach().clone().requires_grad_() for a in args]
    (y_ref,), (y,) = ref(*args), gm(*args2)
    assert torch.equal(y, y_ref)
    gy = torch.randn(y.shape, generator=gen)
    for a, b in zip(torch.autograd.grad(y_ref, args, gy), torch.autograd.grad(y, args2, gy)):
        torch.testing.assert_close(b, a, rtol=1e-6, atol=1e-6)


def _se_backward_graph(oc, case):
    """Backward graph of a squeeze-excite block x * s (s the gate, [N, C, 1, 1]) as AOTAutograd traces it: the gate's
    gradient sum(mul(g, x), [2, 3], keepdim) and the input's gradient mul(g, s) + div(expand(v), hw), with the
    variations `case` names."""
    dev = oc.DEVICE
    mode = FakeTensorMode()
    g = Graph()
    n, c, h, w = 2, 3, 4, 5

    def ph(name, shape):
        node = g.placeholder(name)
        node.meta["val"] = _fake(mode, dev, shape)
        return node

    def call(target, args, shape):
        node = g.call_function(target, args)
        node.meta["val"] = _fake(mode, dev, shape)
        return node

    go, x, s4, v4 = ph("g", (n, c, h, w)), ph("x", (n, c, h, w)), ph("s", (n, c, 1, 1)), ph("v", (n, c, 1, 1))
    m1 = call(aten.mul.Tensor, (go, x), (n, c, h, w))
    sm = call(aten.sum.dim_IntList, (m1, [2, 3] if case != "other_dims" else [1, 2], True),
              (n, c, 1, 1) if case != "other_dims" else (n, 1, 1, w))
    m2 = call(aten.mul.Tensor, (s4, go) if case == "gate_first" else (go, s4), (n, c, h, w))
    e = call(aten.expand.default, (v4, [n, c, h, w]), (n, c, h, w))
    d = call(aten.div.Scalar, (e, h * w), (n, c, h, w))
    a = call(aten.add.Tensor, (d, m2) if case == "gate_first" else (m2, d), (n, c, h, w))
    outs = (sm, a) + ((m2,) if case == "second_use" else ())
    g.output(outs)
    return GraphModule(torch.nn.Module(), g), (n, c, h, w)


@pytest.mark.parametrize("case", ["plain", "gate_first", "second_use", "other_dims"])
def test_se_backward_rewrite(oc, case):
    """The squeeze-excite backward becomes omt.plane_dot (gate gradient) and omt.se_gate_backward (input gradient),
    with the same values on CPU tensors; a second use of the gated product keeps the input gradient apart, a sum over
    other dims keeps the gate gradient apart."""
    gm, (n, c, h, w) = _se_backward_graph(oc, case)
    ref = copy.deepcopy(gm)
    stats = oc.fuse_se_backward(gm.graph)
    gm.graph.eliminate_dead_code()
    gm.graph.lint()
    gm.recompile()
    assert stats == {"plane_dot": 0 if case == "other_dims" else 1, "gate": 0 if case == "second_use" else 1}
    t = _targets(gm)
    assert t.count(torch.ops.omt.plane_dot.default) == stats["plane_dot"]
    assert t.count(torch.ops.omt.se_gate_backward.default) == stats["gate"]
    if stats["gate"]:
        assert aten.div.Scalar not in t and aten.expand.default not in t and aten.add.Tensor not in t
    gen = torch.Generator().manual_seed(5)
    args = [torch.randn(n, c, h, w, generator=gen), torch.randn(n, c, h, w, generator=gen),
            torch.randn(n, c, 1, 1, generator=gen), torch.randn(n, c, 1, 1, generator=gen)]
    for got, want in zip(gm(*args), ref(*args)):
        torch.testing.assert_close(got, want, rtol=1e-6, atol=1e-7)

"""torch.compile backend: `torch.compile(model, backend="omarchy_mac_torch")` (reference: omarchy_mac_torch/compile.py).

Dynamo captures the model and AOTAutograd produces aten graphs for the forward and backward passes, with the
buffer updates (BatchNorm running statistics and batch counters) kept inside the graph as copies into the inputs.
The rewrites then route the hot path to fused device ops, and the graph runs op by op on the device:

  0. training BatchNorm whose new running statistics are only copied back into its running-stat inputs
     -> omt.bn_train_ (statistics updated in place, no copies), taking along a following ReLU, residual add + ReLU
     (y = relu(bn(x) + r), the end of a ResNet basic block), residual add (y = bn(x) + r, the end of a MobileNetV3
     inverted residual) or hardswish (MobileNetV3; the hardswish's input, saved for its backward, comes out as a
     fourth output); the batch counters' increments (one add and one copy each) become a single _foreach_add_;
  1. training BatchNorm (`_native_batch_norm_legit_functional`) whose normalized output only feeds a ReLU
     -> omt.bn_relu_train (statistics, normalize and ReLU in the library's BN kernels);
  2. its backward, `native_batch_norm_backward(threshold_backward(g, y, 0), ...)` -> omt.bn_relu_backward (the ReLU
     mask read from y inside the BN backward reductions and apply), `native_batch_norm_backward(hardswish_backward(g,
     z), ...)` -> omt.bn_act_backward (the hardswish gradient likewise); where the masked gradient also feeds a residual
     branch (the end of a ResNet basic block) -> omt.bn_relu_res_backward, which returns it as a fourth output and
     takes along the add of the block output's two gradients in front of the mask;
  3. a dense convolution whose only user is a ReLU -> omt.conv_act (ReLU in the GEMM epilogue), or an eval BatchNorm
     (`_native_batch_norm_legit_no_training`, optionally followed by ReLU) -> omt.conv_bn_act_eval (BatchNorm folded
     into the conv's weights and bias); a bias-free dense convolution feeding omt.bn_train_ -> omt.conv_bn_train_,
     where the BatchNorm sums a K-split convolution's partials itself (no slice-sum launch), unless its output is
     max-pooled: omt.bn_train_ -> max_pool2d_with_indices -> omt.bn_train_pool_ (the pool inside the BatchNorm's
     apply pass: the ResNet stem); a BatchNorm backward
     (2, or a plain training one) whose incoming gradient is a dense convolution's grad input -> omt.conv_bn_backward,
     where the BatchNorm backward sums the convolution's grad-input partials and runs its grad-weight slice sum;
  4. a squeeze-excite block's backward: sum(mul(g, x), [2, 3]) -> omt.plane_dot, and mul(g, gate) plus the plane
     mean's broadcast gradient -> omt.se_gate_backward (one launch each instead of two and three).

Before AOTAutograd, on the graph Dynamo hands the backend: a squeeze-excite block's excitation MLP,
hardsigmoid(linear(relu(linear(z)))) -> omt.se_mlp (two launches; its registered backward, omt.se_mlp_backward, two).

Each omt op falls back to its plain aten composition when the device kernels do not cover the case, so a rewritten
graph is always correct. The rewritten graphs then run as HIP graphs: a few calls op by op, then captured once and
replayed (omarchy_mac_torch/replay.py; OMARCHY_MAC_TORCH_COMPILE_GRAPHS=0 keeps them op by op).
OMARCHY_MAC_TORCH_COMPILE_DEBUG=1 prints what each rewrite did. (The reference's fourth
pass, generated pointwise kernels, is elementwise work outside the convolution path.)
"""

import operator
import os

import torch
from torch._dynamo import register_backend
from torch._dynamo.backends.common import aot_autograd
from torch.fx import Node

from omarchy_mac_torch import replay
from omarchy_mac_torch.native import DEVICE

aten = torch.ops.aten
omt = torch.ops.omt
_DEBUG = os.environ.get("OMARCHY_MAC_TORCH_COMPILE_DEBUG", "0") == "1"


def _meta(n):
    return n.meta.get("val") if isinstance(n, Node) else None


def _on_device_f32(n, dim=None):
    v = _meta(n)
    return (isinstance(v, torch.Tensor) and v.device.type == DEVICE and v.dtype == torch.float32
            and (dim is None or v.dim() == dim))


def _getitem_users(n):
    """{index: getitem node} for a multi-output node."""
    return {u.args[1]: u for u in n.users if u.op == "call_function" and u.target is operator.getitem}


def _sole_user(n):
    users = list(n.users)
    return users[0] if len(users) == 1 else None


def _call_before(graph, anchor, target, args, meta_from=None):
    with graph.inserting_before(anchor):
        node = graph.call_function(target, tuple(args))
    if meta_from is not None:
        node.meta = dict(meta_from.meta)
    return node


def _move_getitems(graph, old, new):
    """Re-point every getitem of multi-output node `old` at the same index of `new`."""
    for i, gi in _getitem_users(old).items():
        ngi = _call_before(graph, gi, operator.getitem, (new, i), meta_from=gi)
        gi.replace_all_uses_with(ngi)
        graph.erase_node(gi)


# ---- rewrite 0: in-place training BatchNorm (+ residual) (+ ReLU), batch counters ----

def _sole_copy_into(value, dst):
    """The copy_ of `value` into graph input `dst` when that is value's only use, else None."""
    users = list(value.users) if value is not None else []
    if (len(users) == 1 and users[0].op == "call_function" and users[0].target is aten.copy_.default
            and users[0].args[0] is dst and users[0].args[1] is value):
        return users[0]
    return None


def _copy_back(value, dst):
    """The copy_ of `value` into graph input `dst` when value's other uses are graph outputs only (new running
    statistics saved for the BatchNorm backward, which does not read them in training), else None."""
    if value is None:
        return None
    copies = [u for u in value.users if u.op == "call_function" and u.target is aten.copy_.default
              and u.args[0] is dst and u.args[1] is value]
    if len(copies) == 1 and all(u is copies[0] or u.op == "output" for u in value.users):
        return copies[0]
    return None


def _same_shape(a, b):
    va, vb = _meta(a), _meta(b)
    return isinstance(va, torch.Tensor) and isinstance(vb, torch.Tensor) and tuple(va.shape) == tuple(vb.shape)


def fuse_bn_train_in_place(graph):
    count = {"bn": 0, "relu": 0, "add_relu": 0, "add": 0, "hardswish": 0}
    for n in list(graph.nodes):
        if n.op != "call_function" or n.target is not aten._native_batch_norm_legit_functional.default:
            continue
        order = {v: i for i, v in enumerate(graph.nodes)}  # fresh: earlier rewrites inserted nodes
        x, w, b, rm, rv, training, momentum, eps = n.args[:8]
        if not training or any(a is None for a in (w, b, rm, rv)) or not _on_device_f32(x, 4):
            continue
        if not (isinstance(rm, Node) and rm.op == "placeholder" and isinstance(rv, Node) and rv.op == "placeholder"):
            continue
        outs = _getitem_users(n)
        c3, c4 = _copy_back(outs.get(3), rm), _copy_back(outs.get(4), rv)
        out0 = outs.get(0)
        if c3 is None or c4 is None or out0 is None:
            continue
        # nothing else may read the running statistics (graph outputs see them after the update in either form)
        if any(u not in (n, c3) and u.op != "output" for u in rm.users) or \
                any(u not in (n, c4) and u.op != "output" for u in rv.users):
            continue
        act, res, last, add, anchor = 0, None, out0, None, n
        u = _sole_user(out0)
        hs = [v for v in out0.users if v.op == "call_function" and v.target is aten.hardswish.default]
        if u is not None and u.op == "call_function" and u.target is aten.relu.default:
            act, last = 1, u
        elif len(hs) == 1 and all(v is hs[0] or v.op == "output" for v in out0.users):
            # hardswish, its input saved for the backward (a graph output) or not: the fused node returns it as z
            act, last = 2, hs[0]
        elif (u is not None and u.op == "call_function" and u.target is aten.add.Tensor and len(u.args) == 2
              and not u.kwargs):
            other = u.args[1] if u.args[0] is out0 else u.args[0]
            relu = _sole_user(u)
            # the fused node sits at the add (the residual may be computed after the BatchNorm): every use of the
            # saved statistics must come later
            stats_later = all(order[v] > order[u] for i in (1, 2) if outs.get(i) is not None for v in outs[i].users)
            if (other is not out0 and isinstance(other, Node) and _on_device_f32(other, 4) and _same_shape(other, x)
                    and stats_later):
                if relu is not None and relu.op == "call_function" and relu.target is aten.relu.default:
                    act, res, last, add, anchor = 1, other, relu, u, u
                else:  # a residual add with no activation after it (MobileNetV3's inverted residuals)
                    act, res, last, anchor = 0, other, u, u
        fused = _call_before(graph, anchor, omt.bn_train_.default, (x, w, b, rm, rv, momentum, eps, act, res))
        y = _call_before(graph, anchor, operator.getitem, (fused, 0), meta_from=last)
        for i in (1, 2):
            gi = outs.get(i)
            if gi is not None:
                ngi = _call_before(graph, anchor, operator.getitem, (fused, i), meta_from=gi)
                gi.replace_all_uses_with(ngi)
                graph.erase_node(gi)
        last.replace_all_uses_with(y)
        graph.erase_node(last)
        if act == 2 and out0.users:
            z = _call_before(graph, anchor, operator.getitem, (fused, 3), meta_from=out0)
            out0.replace_all_uses_with(z)
        graph.erase_node(c3)
        graph.erase_node(c4)
        outs[3].replace_all_uses_with(rm)  # outputs: the updated buffers
        outs[4].replace_all_uses_with(rv)
        if add is not None:
            graph.erase_node(add)
        if out0 is not last:
            graph.erase_node(out0)
        for dead in (outs[3], outs[4], n):
            graph.erase_node(dead)
        count["bn"] += 1
        if res is not None:
            count["add_relu" if act == 1 else "add"] += 1
        elif act:
            count["relu" if act == 1 else "hardswish"] += 1
    return count


def merge_batch_counters(graph):
    """`copy_(t, add(t, 1))` on 0-dim int64 graph inputs (BatchNorm's num_batches_tracked) -> one _foreach_add_."""
    found = []
    for n in list(graph.nodes):
        if n.op != "call_function" or n.target is not aten.add.Tensor or len(n.args) != 2 or n.kwargs:
            continue
        t, one = n.args
        v = _meta(t)
        if not (isinstance(t, Node) and t.op == "placeholder" and isinstance(v, torch.Tensor) and v.dim() == 0
                and v.dtype == torch.int64 and one == 1):
            continue
        cp = _sole_copy_into(n, t)
        if cp is not None:
            found.append((t, n, cp))
    if len(found) < 2:
        return 0
    with graph.inserting_before(found[-1][2]):
        graph.call_function(aten._foreach_add_.Scalar, ([t for t, _, _ in found], 1))
    for t, add, cp in found:
        graph.erase_node(cp)
        graph.erase_node(add)
    return len(found)


# ---- rewrite 1: training BatchNorm + ReLU ----

def fuse_bn_relu_train(graph):
    count = 0
    for n in list(graph.nodes):
        if n.op != "call_function" or n.target is not aten._native_batch_norm_legit_functional.default:
            continue
        x, w, b, rm, rv, training, momentum, eps = n.args[:8]
        if not training or any(a is None for a in (w, b, rm, rv)) or not _on_device_f32(x, 4):
            continue
        out0 = _getitem_users(n).get(0)
        relu = _sole_user(out0) if out0 is not None else None
        if relu is None or relu.op != "call_function" or relu.target is not aten.relu.default:
            continue
        fused = _call_before(graph, n, omt.bn_relu_train.default, (x, w, b, rm, rv, momentum, eps))
        y = _call_before(graph, relu, operator.getitem, (fused, 0), meta_from=relu)
        relu.replace_all_uses_with(y)
        graph.erase_node(relu)
        graph.erase_node(out0)
        _move_getitems(graph, n, fused)
        graph.erase_node(n)
        count += 1
    return count


# ---- rewrite 2: its backward ----

def fuse_bn_relu_backward(graph):
    count = 0
    for n in list(graph.nodes):
        if n.op != "call_function" or n.target is not aten.native_batch_norm_backward.default:
            continue
        g, x, w, rm, rv, mean, invstd, train, eps, mask = n.args[:10]
        if not train or w is None or not _on_device_f32(x, 4):
            continue
        if not (isinstance(g, Node) and g.op == "call_function" and g.target is aten.threshold_backward.default
                and g.args[2] == 0 and len(g.users) == 1):
            continue
        gout, y = g.args[0], g.args[1]
        fused = _call_before(graph, n, omt.bn_relu_backward.default, (gout, x, y, w, mean, invstd, list(mask)))
        _move_getitems(graph, n, fused)
        graph.erase_node(n)
        graph.erase_node(g)
        count += 1
    return count


def fuse_bn_hardswish_backward(graph):
    """native_batch_norm_backward(hardswish_backward(g, z), x, ...) -> omt.bn_act_backward(g, x, z, ..., act 2): the
    hardswish gradient taken inside the BatchNorm backward's reads (z, the hardswish's input, is the fused forward's
    fourth output)."""
    count = 0
    for n in list(graph.nodes):
        if n.op != "call_function" or n.target is not aten.native_batch_norm_backward.default:
            continue
        g, x, w, rm, rv, mean, invstd, train, eps, mask = n.args[:10]
        if not train or w is None or not _on_device_f32(x, 4):
            continue
        if not (isinstance(g, Node) and g.op == "call_function" and g.target is aten.hardswish_backward.default
                and len(g.users) == 1 and _on_device_f32(g.args[1], 4)):
            continue
        gout, z = g.args[0], g.args[1]
        fused = _call_before(graph, n, omt.bn_act_backward.default, (gout, x, z, w, mean, invstd, 2, list(mask)))
        _move_getitems(graph, n, fused)
        graph.erase_node(n)
        graph.erase_node(g)
        count += 1
    return count


def fuse_bn_relu_res_backward(graph):
    """t = threshold_backward(a, y, 0) with several users, one of them native_batch_norm_backward(t, ...): that BN
    backward and the mask become one omt.bn_relu_res_backward(g, g2, ...), whose fourth output replaces t for the other
    users; a = add(g, g2) feeding only t goes in as well. The fused node takes t's place in the graph (the BN
    backward's other operands are saved tensors, defined earlier; y, often a detach of one, comes before t)."""
    count = 0
    for t in list(graph.nodes):
        if t.op != "call_function" or t.target is not aten.threshold_backward.default or t.args[2] != 0:
            continue
        if len(t.users) < 2 or not _on_device_f32(t, 4):
            continue
        bn = next((u for u in t.users if u.op == "call_function" and u.target is aten.native_batch_norm_backward.default
                   and u.args[0] is t and u.args[7] and u.args[2] is not None and _on_device_f32(u.args[1], 4)), None)
        if bn is None:
            continue
        a, y = t.args[0], t.args[1]
        g, g2 = a, None
        if (isinstance(a, Node) and a.op == "call_function" and a.target is aten.add.Tensor and len(a.users) == 1
                and len(a.args) == 2 and not a.kwargs and _meta(a.args[0]) is not None and _meta(a.args[1]) is not None
                and tuple(_meta(a.args[0]).shape) == tuple(_meta(a.args[1]).shape)
                and _on_device_f32(a.args[0], 4) and _on_device_f32(a.args[1], 4)):
            g, g2 = a.args
        _, x, w, rm, rv, mean, invstd, train, eps, mask = bn.args[:10]
        order = {nd: i for i, nd in enumerate(graph.nodes)}
        if any(isinstance(v, Node) and order[v] >= order[t] for v in (x, w, mean, invstd)):
            continue
        fused = _call_before(graph, t, omt.bn_relu_res_backward.default, (g, g2, x, y, w, mean, invstd, list(mask)))
        gz = _call_before(graph, t, operator.getitem, (fused, 3), meta_from=t)
        _move_getitems(graph, bn, fused)
        graph.erase_node(bn)
        t.replace_all_uses_with(gz)
        graph.erase_node(t)
        if g2 is not None:
            graph.erase_node(a)
        count += 1
    return count


# ---- rewrite 3: conv epilogues ----

def _is_dense_conv(n):
    if n.op != "call_function" or n.target is not aten.convolution.default:
        return False
    x, w, b, stride, padding, dilation, transposed, output_padding, groups = n.args[:9]
    wv = _meta(w)
    return (_on_device_f32(x, 4) and not transposed and groups == 1 and list(dilation) == [1, 1] and wv is not None
            and wv.dim() == 4 and wv.shape[2] == wv.shape[3] and len(set(stride)) == 1 and len(set(padding)) == 1)


def fuse_conv_epilogues(graph):
    count = 0
    for n in list(graph.nodes):
        if not _is_dense_conv(n):
            continue
        x, w, b, stride, padding = n.args[:5]
        user = _sole_user(n)
        if user is None or user.op != "call_function":
            continue
        if user.target is aten.relu.default:
            fused = _call_before(graph, n, omt.conv_act.default, (x, w, b, list(stride), list(padding), 1),
                                 meta_from=user)
            user.replace_all_uses_with(fused)
            graph.erase_node(user)
            graph.erase_node(n)
            count += 1
        elif user.target is aten._native_batch_norm_legit_no_training.default and user.args[0] is n:
            _, bw, bb, rm, rv, momentum, eps = user.args[:7]
            outs = _getitem_users(user)
            out0 = outs.get(0)
            if any(a is None for a in (bw, bb, rm, rv)) or out0 is None or len(outs) != 1:
                continue
            relu = _sole_user(out0)
            act = 1 if relu is not None and relu.op == "call_function" and relu.target is aten.relu.default else 0
            last = relu if act else out0
            fused = _call_before(graph, n, omt.conv_bn_act_eval.default,
                                 (x, w, b, bw, bb, rm, rv, eps, list(stride), list(padding), act), meta_from=last)
            last.replace_all_uses_with(fused)
            for dead in ([relu] if act else []) + [out0, user, n]:
                graph.erase_node(dead)
            count += 1
    return count


def _two(v, default=()):
    """A 2-D pooling argument as a list of two ints (one int stands for both; empty or missing: default)."""
    if not v:
        return list(default)
    v = [int(t) for t in v]
    return v * 2 if len(v) == 1 else v


def _pool_args(mp):
    """(kernel, stride, padding) of a max_pool2d_with_indices node without dilation or ceil mode, else None."""
    a = list(mp.args) + [None] * (6 - len(mp.args))
    k = _two(a[1])
    s = _two(a[2], k)
    p = _two(a[3], [0, 0])
    d = _two(a[4], [1, 1])
    if mp.kwargs or len(k) != 2 or len(s) != 2 or len(p) != 2 or d != [1, 1] or bool(a[5]):
        return None
    return k, s, p


def fuse_bn_train_pool(graph):
    """max_pool2d_with_indices(y) of an omt.bn_train_ output y (no residual) -> one omt.bn_train_pool_, whose outputs 0-2
    are the BatchNorm's (y stays for its other users: the backward's activation mask) and 3-4 the pool's: the pool
    runs inside the BatchNorm's apply pass (the ResNet stem). Before fuse_conv_bn_train, which would otherwise take
    the BatchNorm."""
    count = 0
    for bn in list(graph.nodes):
        if bn.op != "call_function" or bn.target is not omt.bn_train_.default or bn.args[8] is not None:
            continue
        outs = _getitem_users(bn)
        y = outs.get(0)
        if y is None or 3 in outs:
            continue
        mp = next((u for u in y.users if u.op == "call_function" and u.target is aten.max_pool2d_with_indices.default
                   and u.args[0] is y), None)
        if mp is None:
            continue
        pa = _pool_args(mp)
        if pa is None:
            continue
        x, w, b, rm, rv, momentum, eps, act = bn.args[:8]
        fused = _call_before(graph, bn, omt.bn_train_pool_.default, (x, w, b, rm, rv, momentum, eps, act) + pa)
        _move_getitems(graph, bn, fused)
        graph.erase_node(bn)
        for i, gi in _getitem_users(mp).items():
            new = _call_before(graph, gi, operator.getitem, (fused, 3 + i), meta_from=gi)
            gi.replace_all_uses_with(new)
            graph.erase_node(gi)
        graph.erase_node(mp)
        count += 1
    return count


def fuse_conv_bn_train(graph):
    """bn_train_(convolution(x, cw, None, ...), ...) -> omt.conv_bn_train_(x, cw, stride, padding, ...), whose fifth
    output is the convolution's (the BatchNorm backward reads it): with a K-split plan the BatchNorm sums the
    convolution's partials itself (one launch fewer). The convolution's other uses must come after the BatchNorm."""
    count = 0
    for n in list(graph.nodes):
        if n.op != "call_function" or n.target is not omt.bn_train_.default:
            continue
        order = {v: i for i, v in enumerate(graph.nodes)}  # fresh: earlier rewrites inserted nodes
        conv = n.args[0]
        if not (isinstance(conv, Node) and _is_dense_conv(conv) and conv.args[2] is None):
            continue
        if any(u is not n and u.op != "output" and order[u] < order[n] for u in conv.users):
            continue
        cx, cw, _, stride, padding = conv.args[:5]
        w, b, rm, rv, momentum, eps, act, res = n.args[1:9]
        fused = _call_before(graph, n, omt.conv_bn_train_.default,
                             (cx, cw, list(stride), list(padding), w, b, rm, rv, momentum, eps, act, res))
        out = _call_before(graph, n, operator.getitem, (fused, 4), meta_from=conv)
        n.replace_all_uses_with(fused)  # its users are getitems 0-3, the same outputs of the fused node
        graph.erase_node(n)
        conv.replace_all_uses_with(out)
        graph.erase_node(conv)
        count += 1
    return count


def _dgrad_of(gi, before, order):
    """The convolution_backward node when gi is its grad input and the fused op can take it over: a dense convolution,
    both grads asked for and no bias grad, gi used once, and every use of its grad weight after node `before`."""
    if not (isinstance(gi, Node) and gi.op == "call_function" and gi.target is operator.getitem and gi.args[1] == 0
            and len(gi.users) == 1):
        return None
    cb = gi.args[0]
    if not (isinstance(cb, Node) and cb.op == "call_function" and cb.target is aten.convolution_backward.default):
        return None
    gy, cx, cw, _, stride, padding, dilation, transposed, _, groups, mask = cb.args[:11]
    outs = _getitem_users(cb)
    wv = _meta(cw)
    if not (mask[0] and mask[1] and not mask[2]) or set(outs) - {0, 1}:
        return None
    if (transposed or groups != 1 or list(dilation) != [1, 1] or wv is None or wv.dim() != 4
            or wv.shape[2] != wv.shape[3] or len(set(stride)) != 1 or len(set(padding)) != 1
            or not _on_device_f32(cx, 4) or not _on_device_f32(gy, 4)):
        return None
    if 1 in outs and any(order[u] < order[before] for u in outs[1].users):
        return None
    return cb


def fuse_conv_bn_backward(graph):
    """A BatchNorm backward (omt.bn_relu_backward, bn_act_backward, bn_relu_res_backward, or a training
    native_batch_norm_backward) whose incoming gradient is a dense convolution's grad input -> one
    omt.conv_bn_backward: the BatchNorm backward sums the convolution's K-split grad-input partials as it reads them and
    runs the grad weight's slice sum on workgroups of its own launch (the convolution's slice-sum launch goes). Its
    outputs: the convolution's grad weight, then the BatchNorm backward's. At a residual block's end either of the two
    gradients may be the convolution's (the other goes in as `other`)."""
    count = 0
    for bn in list(graph.nodes):
        if bn.op != "call_function":
            continue
        if bn.target is omt.bn_relu_backward.default:
            g, x, r, w, mean, invstd, mask = bn.args
            cands, act, res = [(g, None)], 1, False
        elif bn.target is omt.bn_act_backward.default:
            g, x, r, w, mean, invstd, act, mask = bn.args
            cands, res = [(g, None)], False
        elif bn.target is omt.bn_relu_res_backward.default:
            g, g2, x, r, w, mean, invstd, mask = bn.args
            cands, act, res = [(g, g2), (g2, g)], 1, True
        elif bn.target is aten.native_batch_norm_backward.default:
            g, x, w, _, _, mean, invstd, train, _, mask = bn.args[:10]
            if not train or w is None or not _on_device_f32(x, 4):
                continue
            cands, act, res, r = [(g, None)], 0, False, x
        else:
            continue
        order = {v: i for i, v in enumerate(graph.nodes)}
        cb = other = None
        for gi, o in cands:
            cb = _dgrad_of(gi, bn, order)
            if cb is not None:
                other = o
                break
        if cb is None:
            continue
        gy, cx, cw, _, stride, padding = cb.args[:6]
        fused = _call_before(graph, bn, omt.conv_bn_backward.default,
                             (gy, cx, cw, list(stride), list(padding), other, x, r, w, mean, invstd, act, res,
                              list(mask)))
        outs = _getitem_users(cb)
        if 1 in outs:
            gw = _call_before(graph, bn, operator.getitem, (fused, 0), meta_from=outs[1])
            outs[1].replace_all_uses_with(gw)
            graph.erase_node(outs[1])
        for i, gi in _getitem_users(bn).items():
            new = _call_before(graph, gi, operator.getitem, (fused, i + 1), meta_from=gi)
            gi.replace_all_uses_with(new)
            graph.erase_node(gi)
        graph.erase_node(bn)
        graph.erase_node(outs[0])
        graph.erase_node(cb)
        count += 1
    return count


# ---- the squeeze-excite backward ----

def _shape(n):
    v = _meta(n)
    return tuple(v.shape) if isinstance(v, torch.Tensor) else None


def fuse_se_backward(graph):
    """The backward of a squeeze-excite block x * gate(mean(x)) as AOTAutograd traces it, in two rewrites:
    sum(mul(g, x), [2, 3], keepdim) -> omt.plane_dot(g, x) (the gate's gradient, one launch instead of two), and
    add(mul(g, s), div(expand(v), hw)) with s, v [N, C, 1, 1] -> omt.se_gate_backward(g, s, v, 1 / hw) (the input's
    gradient through the gate and through the mean, one launch instead of three). The intermediate values must have
    no other use; float32 device tensors."""
    count = {"plane_dot": 0, "gate": 0}
    for n in list(graph.nodes):
        if n.op != "call_function":
            continue
        if n.target is aten.sum.dim_IntList and len(n.args) >= 3 and n.args[2] is True and not n.kwargs:
            m = n.args[0]
            dims = sorted(d % 4 for d in n.args[1]) if isinstance(n.args[1], (list, tuple)) else None
            if (dims == [2, 3] and isinstance(m, Node) and m.op == "call_function" and m.target is aten.mul.Tensor
                    and _sole_user(m) is n and len(m.args) == 2 and not m.kwargs
                    and all(_on_device_f32(a, 4) for a in m.args) and _shape(m.args[0]) == _shape(m.args[1])):
                fused = _call_before(graph, n, omt.plane_dot.default, m.args, meta_from=n)
                n.replace_all_uses_with(fused)
                graph.erase_node(n)
                graph.erase_node(m)
                count["plane_dot"] += 1
            continue
        if n.target is not aten.add.Tensor or len(n.args) != 2 or n.kwargs or not _on_device_f32(n, 4):
            continue
        shape = _shape(n)
        mul = div = None
        for a in n.args:
            if not (isinstance(a, Node) and a.op == "call_function" and _sole_user(a) is n):
                continue
            if a.target is aten.mul.Tensor and len(a.args) == 2 and not a.kwargs:
                mul = a
            elif a.target is aten.div.Scalar and len(a.args) == 2 and not a.kwargs:
                div = a
        if mul is None or div is None:
            continue
        e = div.args[0]
        if not (isinstance(e, Node) and e.op == "call_function" and e.target is aten.expand.default
                and _sole_user(e) is div and isinstance(div.args[1], (int, float)) and div.args[1] != 0):
            continue
        v = e.args[0]
        gate = [a for a in mul.args if _shape(a) == shape[:2] + (1, 1)]
        big = [a for a in mul.args if _shape(a) == shape]
        if len(gate) != 1 or len(big) != 1 or _shape(v) != shape[:2] + (1, 1):
            continue
        if not all(_on_device_f32(t, 4) for t in (gate[0], big[0], v)):
            continue
        fused = _call_before(graph, n, omt.se_gate_backward.default, (big[0], gate[0], v, 1.0 / div.args[1]),
                             meta_from=n)
        n.replace_all_uses_with(fused)
        for dead in (n, mul, div, e):
            graph.erase_node(dead)
        count["gate"] += 1
    return count


def _rewrite(gm):
    g = gm.graph
    stats = {"bn_train_in_place": fuse_bn_train_in_place(g), "batch_counters": merge_batch_counters(g),
             "bn_relu": fuse_bn_relu_train(g), "bn_relu_res_backward": fuse_bn_relu_res_backward(g),
             "bn_relu_backward": fuse_bn_relu_backward(g), "bn_hardswish_backward": fuse_bn_hardswish_backward(g),
             "bn_train_pool": fuse_bn_train_pool(g), "conv_bn_train": fuse_conv_bn_train(g),
             "conv_bn_backward": fuse_conv_bn_backward(g), "se_backward": fuse_se_backward(g),
             "conv_epilogue": fuse_conv_epilogues(g)}
    g.eliminate_dead_code()
    g.lint()
    gm.recompile()
    if _DEBUG:
        print("[omarchy-mac-torch compile]", stats)
    return gm


def _compiler(kind):
    def compile_graph(gm, example_inputs):
        return replay.wrap(_rewrite(gm).forward, kind)
    return compile_graph


# ---- before AOTAutograd: the squeeze-excite MLP ----

def _se_setup(ctx, inputs, output):
    z, w1, _, w2, _ = inputs
    _, h, a2 = output
    ctx.mark_non_differentiable(h, a2)
    ctx.set_materialize_grads(False)
    ctx.save_for_backward(z, h, a2, w1, w2)


def _se_backward(ctx, gs, _gh, _ga2):
    return tuple(omt.se_mlp_backward(gs, *ctx.saved_tensors))


# omt::se_mlp's backward is omt::se_mlp_backward (both defined in the extension): AOTAutograd traces through this
# formula, so the forward graph holds omt.se_mlp and the backward graph omt.se_mlp_backward; the op's second and third
# outputs (the hidden layer and the pre-activation) are saved for the backward, not differentiated
torch.library.register_autograd("omt::se_mlp", _se_backward, setup_context=_se_setup)

_LINEAR = (torch._C._nn.linear, torch.nn.functional.linear)
_RELU = (torch.nn.functional.relu, torch.relu)
_HARDSIGMOID = (torch.nn.functional.hardsigmoid,)
_SE_MAX_C, _SE_MAX_R = 2048, 1024  # the kernels' limits (omt_se_fwd)


def _example(n):
    return n.meta.get("example_value") if isinstance(n, Node) else None


def _only_use(n, user):
    return isinstance(n, Node) and list(n.users) == [user]


def _plain_call(n, targets, nargs):
    """n calls one of `targets` with `nargs` positional arguments and no in-place flag."""
    return (n.op == "call_function" and n.target in targets and len(n.args) == nargs
            and not n.kwargs.get("inplace", False) and all(k == "inplace" for k in n.kwargs))


def fuse_squeeze_excite(graph):
    """hardsigmoid(linear(relu(linear(z, w1, b1)), w2, b2)), the excitation MLP of a squeeze-excite block, over float32
    device tensors -> omt.se_mlp(z, w1, b1, w2, b2), in the graph Dynamo hands the backend (before AOTAutograd, which
    then traces the op's registered backward, omt.se_mlp_backward, into the backward graph). The two intermediate
    values must have no other use, both biases be present, and the sizes be within the kernels' (C <= 2048,
    R <= 1024): two launches forward and two backward instead of about five and ten."""
    count = 0
    for hs in list(graph.nodes):
        if not _plain_call(hs, _HARDSIGMOID, 1):
            continue
        l2 = hs.args[0]
        if not (_only_use(l2, hs) and _plain_call(l2, _LINEAR, 3)):
            continue
        h, w2, b2 = l2.args
        if not (_only_use(h, l2) and _plain_call(h, _RELU, 1)):
            continue
        l1 = h.args[0]
        if not (_only_use(l1, h) and _plain_call(l1, _LINEAR, 3)):
            continue
        z, w1, b1 = l1.args
        ez, e1, eb1, e2, eb2 = (_example(v) for v in (z, w1, b1, w2, b2))
        if not all(isinstance(v, torch.Tensor) and v.device.type == DEVICE and v.dtype == torch.float32
                   for v in (ez, e1, eb1, e2, eb2)):
            continue
        if ez.dim() != 2 or e1.dim() != 2 or e2.dim() != 2:
            continue
        c, r = ez.shape[1], e1.shape[0]
        if c > _SE_MAX_C or r > _SE_MAX_R or tuple(e2.shape) != (c, r):
            continue
        with graph.inserting_before(hs):
            fused = graph.call_function(omt.se_mlp.default, (z, w1, b1, w2, b2))
            out = graph.call_function(operator.getitem, (fused, 0))
        out.meta = dict(hs.meta)
        hs.replace_all_uses_with(out)
        for dead in (hs, l2, h, l1):
            graph.erase_node(dead)
        count += 1
    return count


# buffer mutations stay in the graph (as copy_ into the inputs) so that rewrite 0 can turn them into in-place updates;
# every rewritten graph is replayed as a HIP graph after its warm-up calls (replay.py)
_aot = aot_autograd(fw_compiler=_compiler("forward"), bw_compiler=_compiler("backward"),
                    inference_compiler=_compiler("inference"), keep_inference_input_mutations=True)


def backend(gm, example_inputs):
    """The backend: the squeeze-excite rewrite on Dynamo's graph, then AOTAutograd with the rewrites above on its
    forward and backward graphs."""
    if fuse_squeeze_excite(gm.graph):
        gm.graph.lint()
        gm.recompile()
    return _aot(gm, example_inputs)


register_backend(name=DEVICE)(backend)

"""torch.compile backend: `torch.compile(model, backend="omarchy_mac_torch")` (reference: omarchy_mac_torch/compile.py).

Dynamo captures the model and AOTAutograd produces aten graphs for the forward and backward passes. Three rewrites
then route the hot path to fused device ops, and the graph runs op by op on the device:

  1. training BatchNorm (`_native_batch_norm_legit_functional`) whose normalized output only feeds a ReLU
     -> omt.bn_relu_train (statistics, normalize and ReLU in the library's BN kernels);
  2. its backward, `native_batch_norm_backward(threshold_backward(g, y, 0), ...)` -> omt.bn_relu_backward (the ReLU
     mask read from y inside the BN backward reductions and apply);
  3. a dense convolution whose only user is a ReLU -> omt.conv_act (ReLU in the GEMM epilogue), or an eval BatchNorm
     (`_native_batch_norm_legit_no_training`, optionally followed by ReLU) -> omt.conv_bn_act_eval (BatchNorm folded
     into the conv's weights and bias).

Each omt op falls back to its plain aten composition when the device kernels do not cover the case, so a rewritten
graph is always correct. OMARCHY_MAC_TORCH_COMPILE_DEBUG=1 prints what each rewrite did. (The reference's fourth
pass, generated pointwise kernels, is elementwise work outside the convolution path.)
"""

import operator
import os

import torch
from torch._dynamo import register_backend
from torch._dynamo.backends.common import aot_autograd
from torch.fx import Node

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


def _compile(gm, example_inputs):
    g = gm.graph
    stats = {"bn_relu": fuse_bn_relu_train(g), "bn_relu_backward": fuse_bn_relu_backward(g),
             "conv_epilogue": fuse_conv_epilogues(g)}
    g.eliminate_dead_code()
    g.lint()
    gm.recompile()
    if _DEBUG:
        print("[omarchy-mac-torch compile]", stats)
    from functorch.compile import make_boxed_func
    return make_boxed_func(gm.forward)


backend = aot_autograd(fw_compiler=_compile, bw_compiler=_compile, inference_compiler=_compile)
register_backend(name=DEVICE)(backend)

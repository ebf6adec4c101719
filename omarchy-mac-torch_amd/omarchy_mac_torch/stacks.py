"""Fused Conv / BatchNorm+ReLU / pool stacks (reference: omarchy_mac_torch/stacks.py).

`accelerate(model)` turns every `nn.Sequential` whose layers all have a plan implementation into a `FusedSequential`
(same modules, parameters and state_dict) that runs from a native plan: a fixed list of libomt_hip.so launches over
plan-owned device buffers, built once per (input shape, training, input-grad) and reused. With
OMARCHY_MAC_TORCH_AUTO_FUSE unset or 1, the same swap happens automatically the first time such a Sequential runs on
a device tensor.

Supported layers (the reference's fusability rules, stacks.py:41-63): a first layer that is a conv; dense convs with
odd kernel 1/3/5, stride 1, "same" zero padding and no bias; depthwise 3/5/7 convs, stride 1, "same" padding, no
bias; BatchNorm2d (affine, tracking running stats, momentum set, eps 1e-5) immediately followed by ReLU (fused);
2x2 stride-2 max and average pools; AdaptiveAvgPool2d(1).
"""

import os
import weakref

import torch
from torch import nn

from omarchy_mac_torch.native import DEVICE, core


def _pair(v):
    return tuple(v) if isinstance(v, (tuple, list)) else (v, v)


def _is_maxpool2(m):
    return (type(m) is nn.MaxPool2d and _pair(m.kernel_size) == (2, 2) and _pair(m.stride or m.kernel_size) == (2, 2)
            and _pair(m.padding) == (0, 0) and _pair(m.dilation) == (1, 1) and not m.ceil_mode
            and not m.return_indices)


def _is_avgpool2(m):
    return (type(m) is nn.AvgPool2d and _pair(m.kernel_size) == (2, 2) and _pair(m.stride or m.kernel_size) == (2, 2)
            and _pair(m.padding) == (0, 0) and not m.ceil_mode and m.divisor_override is None)


def _same_conv(m, sizes):
    k = m.kernel_size
    return (k[0] == k[1] and k[0] in sizes and m.stride == (1, 1) and m.dilation == (1, 1)
            and m.padding == (k[0] // 2, k[0] // 2) and m.padding_mode == "zeros" and m.weight.dtype == torch.float32
            and m.bias is None)


def _is_depthwise(m):
    return type(m) is nn.Conv2d and m.groups == m.in_channels == m.out_channels > 1 and _same_conv(m, (3, 5, 7))


def _is_dense(m):
    return type(m) is nn.Conv2d and m.groups == 1 and _same_conv(m, (1, 3, 5))


def _is_bn(m):
    return (type(m) is nn.BatchNorm2d and m.affine and m.track_running_stats and m.momentum is not None
            and m.eps == 1e-5)


def _is_gap(m):
    return type(m) is nn.AdaptiveAvgPool2d and m.output_size in (1, (1, 1), [1, 1])


def fusable(seq):
    """Whether every layer of nn.Sequential `seq` has a plan implementation."""
    mods = list(seq)
    if not mods or not isinstance(mods[0], nn.Conv2d):
        return False
    i = 0
    while i < len(mods):
        m = mods[i]
        if isinstance(m, nn.Conv2d):
            ok = _is_dense(m) or _is_depthwise(m)
        elif type(m) is nn.BatchNorm2d:
            ok = _is_bn(m) and i + 1 < len(mods) and type(mods[i + 1]) is nn.ReLU
            i += 1  # its ReLU is part of the BatchNorm step
        else:
            ok = _is_maxpool2(m) or _is_avgpool2(m) or _is_gap(m)
        if not ok:
            return False
        i += 1
    return True


def _params(seq):
    out = []
    for m in seq:
        if isinstance(m, nn.Conv2d):
            out.append(m.weight)
        elif isinstance(m, nn.BatchNorm2d):
            out += [m.weight, m.bias]
    return out


def _layer_specs(seq):
    """(kind, in channels, out channels, kernel size, momentum) per plan layer."""
    specs, mods, i = [], list(seq), 0
    while i < len(mods):
        m = mods[i]
        if isinstance(m, nn.Conv2d):
            specs.append(("dw" if m.groups > 1 else "conv", m.in_channels, m.out_channels, m.kernel_size[0], 0.0))
        elif isinstance(m, nn.BatchNorm2d):
            specs.append(("bn", m.num_features, m.num_features, 0, float(m.momentum)))
            i += 1
        elif _is_gap(m):
            specs.append(("gap", 0, 0, 0, 0.0))
        elif _is_avgpool2(m):
            specs.append(("apool", 0, 0, 0, 0.0))
        else:
            specs.append(("pool", 0, 0, 0, 0.0))
        i += 1
    return specs


_plans = weakref.WeakKeyDictionary()


def _plan(seq, shape, train, input_grad):
    """The plan for (shape, train, input_grad); a plan whose backward is still pending is never reused, a second
    one is built for re-entrant use (e.g. the same stack applied twice before backward)."""
    cache = _plans.setdefault(seq, {})
    key = (tuple(shape), train, input_grad)
    plan = cache.get(key)
    if plan is None or plan.busy:
        bns = [m for m in seq if isinstance(m, nn.BatchNorm2d)]
        plan = core.make_plan(_layer_specs(seq), list(shape), train, input_grad, list(_params(seq)),
                              [m.running_mean for m in bns], [m.running_var for m in bns])
        if key not in cache:
            cache[key] = plan
    return plan


class _StackFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, seq, *params):
        plan = _plan(seq, x.shape, True, ctx.needs_input_grad[0])
        out = plan.forward(x)
        plan.busy = True
        ctx.plan = plan
        return out

    @staticmethod
    def backward(ctx, gout):
        plan = ctx.plan
        gx, grads = plan.backward(gout)
        plan.busy = False
        return (gx, None, *grads)


class FusedSequential(nn.Sequential):
    """The nn.Sequential it replaces (same modules and state_dict), run from a native plan on device tensors."""

    def _count_batch(self):
        for m in self:  # what nn.BatchNorm2d.forward would have done
            if isinstance(m, nn.BatchNorm2d) and m.num_batches_tracked is not None:
                m.num_batches_tracked.add_(1)

    def forward(self, x):
        if x.device.type == DEVICE and x.dtype == torch.float32 and x.dim() == 4:
            if self.training and torch.is_grad_enabled():
                self._count_batch()
                return _StackFn.apply(x, self, *_params(self))
            if not self.training and not torch.is_grad_enabled():
                return _plan(self, x.shape, False, False).forward(x)
        return super().forward(x)


def accelerate(model):
    """Swap every nn.Sequential of `model` made only of supported layers for a FusedSequential, in place. Parameters,
    buffers and state_dict are unchanged. Returns a short description."""
    count = 0
    for m in model.modules():
        if type(m) is nn.Sequential and fusable(m):
            m.__class__ = FusedSequential
            count += 1
    name = torch.cuda.get_device_name(0) if torch.cuda.is_available() else "no GPU"
    return f"{count} fused stacks on {name}"


_checked = weakref.WeakSet()
_auto = {"on": os.environ.get("OMARCHY_MAC_TORCH_AUTO_FUSE", "1") != "0"}


def set_auto_fuse(on):
    """Turns automatic fusion on or off at run time (OMARCHY_MAC_TORCH_AUTO_FUSE sets the initial state). Returns the
    previous state."""
    prev = _auto["on"]
    _auto["on"] = bool(on)
    return prev


def _auto_fuse(module, args):
    if not _auto["on"] or type(module) is not nn.Sequential or module in _checked:
        return None
    x = args[0] if args else None
    if not (isinstance(x, torch.Tensor) and x.device.type == DEVICE):
        return None
    _checked.add(module)
    if fusable(module):
        module.__class__ = FusedSequential
    return None


nn.modules.module.register_module_forward_pre_hook(_auto_fuse)

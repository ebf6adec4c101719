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

How a stack runs: the Sequential is compiled once into a `_Program` (the plan layer records in order, and the
tensors the native plans bind: conv weights, BatchNorm affine parameters and running statistics). A program keeps a
pool of idle plans per (shape, training, input-grad). A training forward leases a plan from that pool for as long as
its autograd graph lives: the lease returns the plan after backward, or when the graph is freed without one, so a
stack applied twice before backward runs two plans and none is lost. Reassigning a parameter or buffer (a new
tensor, or new `.data`) drops the program's plans, which hold the tensors they were built with.

From its second run on, a plan replays each of its step lists (forward, backward) as one captured HIP graph (the
input copied into the plan's input buffer first); OMARCHY_MAC_TORCH_PLAN_GRAPHS=0 keeps them step by step.
"""

import os
import weakref

import torch
from torch import nn

from omarchy_mac_torch.native import DEVICE, core


# ---- layer records -------------------------------------------------------------------------------------------------

def _two(v):
    return tuple(v) if isinstance(v, (tuple, list)) else (v, v)


def _conv_record(m):
    """("conv" | "dw", C_in, C_out, ks, 0.0) for a convolution a plan runs, else None."""
    if type(m) is not nn.Conv2d or m.bias is not None or m.weight.dtype != torch.float32:
        return None
    ks = m.kernel_size[0]
    same = (m.kernel_size == (ks, ks) and m.stride == (1, 1) and m.dilation == (1, 1) and m.padding == (ks // 2, ks // 2)
            and m.padding_mode == "zeros")
    if not same:
        return None
    if m.groups == 1 and ks in (1, 3, 5):
        return ("conv", m.in_channels, m.out_channels, ks, 0.0)
    if m.groups == m.in_channels == m.out_channels > 1 and ks in (3, 5, 7):
        return ("dw", m.in_channels, m.out_channels, ks, 0.0)
    return None


def _bn_record(m):
    """("bn", C, C, 0, momentum) for a BatchNorm2d a plan runs (its ReLU fused), else None."""
    ok = (type(m) is nn.BatchNorm2d and m.affine and m.track_running_stats and m.momentum is not None
          and m.eps == 1e-5)
    return ("bn", m.num_features, m.num_features, 0, float(m.momentum)) if ok else None


def _pool_record(m):
    """("pool" | "apool" | "gap", 0, 0, 0, 0.0) for a 2x2 stride-2 max / average pool or a global average pool."""
    t = type(m)
    if t is nn.AdaptiveAvgPool2d:
        return ("gap", 0, 0, 0, 0.0) if _two(m.output_size) == (1, 1) else None
    if t not in (nn.MaxPool2d, nn.AvgPool2d) or m.ceil_mode:
        return None
    window = _two(m.kernel_size) == (2, 2) and _two(m.stride or m.kernel_size) == (2, 2) and _two(m.padding) == (0, 0)
    if not window:
        return None
    if t is nn.MaxPool2d:
        return ("pool", 0, 0, 0, 0.0) if _two(m.dilation) == (1, 1) and not m.return_indices else None
    return ("apool", 0, 0, 0, 0.0) if m.divisor_override is None else None


# ---- programs and their plans --------------------------------------------------------------------------------------

class _Program:
    """A Sequential compiled for the native plans: layer records, the tensors the plans bind, and idle plans."""

    def __init__(self, records, params, bns):
        self.records = records
        self.params = params      # conv weights, BatchNorm (weight, bias) pairs, in layer order
        self.bns = bns            # the BatchNorm2d modules, in layer order
        self.binding = None       # identity of the bound tensors when the plans in `idle` were built
        self.idle = {}            # (shape, training, input_grad) -> [plan]

    def tensors(self):
        return self.params + [m.running_mean for m in self.bns] + [m.running_var for m in self.bns]

    def lease(self, shape, train, input_grad):
        """An idle plan for the key, or a new one; the caller hands it back with `restore`."""
        binding = tuple((id(t), t.data_ptr()) for t in self.tensors())
        if binding != self.binding:
            self.idle.clear()
            self.binding = binding
        key = (tuple(shape), train, input_grad)
        free = self.idle.get(key)
        if free:
            return key, free.pop()
        plan = core.make_plan(self.records, list(shape), train, input_grad, self.params,
                              [m.running_mean for m in self.bns], [m.running_var for m in self.bns])
        return key, plan

    def restore(self, key, plan, binding):
        if binding == self.binding:
            self.idle.setdefault(key, []).append(plan)


def _compile(seq):
    """The _Program of nn.Sequential `seq`, or None when a layer has no plan implementation."""
    mods = list(seq)
    if not mods or not isinstance(mods[0], nn.Conv2d):
        return None
    records, params, bns = [], [], []
    fused_relu = False
    for m, nxt in zip(mods, mods[1:] + [None]):
        if fused_relu:  # the ReLU after a BatchNorm runs inside the BatchNorm step
            fused_relu = False
            continue
        if isinstance(m, nn.Conv2d):
            rec = _conv_record(m)
            params.append(m.weight)
        elif isinstance(m, nn.BatchNorm2d):
            rec = _bn_record(m) if type(nxt) is nn.ReLU else None
            params += [m.weight, m.bias]
            bns.append(m)
            fused_relu = True
        else:
            rec = _pool_record(m)
        if rec is None:
            return None
        records.append(rec)
    return _Program(records, params, bns)


def fusable(seq):
    """Whether every layer of nn.Sequential `seq` has a plan implementation."""
    return _compile(seq) is not None


_programs = weakref.WeakKeyDictionary()  # FusedSequential -> _Program


def _program_of(seq):
    prog = _programs.get(seq)
    if prog is None:
        prog = _compile(seq)
        if prog is None:
            raise RuntimeError("omarchy-mac-torch: this Sequential no longer has a plan implementation")
        _programs[seq] = prog
    return prog


class _Lease:
    """A plan held for one autograd graph: handed back to its program after backward, or when the graph that holds the
    lease is freed without a backward."""

    __slots__ = ("prog", "key", "plan", "binding")

    def __init__(self, prog, key, plan):
        self.prog, self.key, self.plan, self.binding = prog, key, plan, prog.binding

    def give_back(self):
        if self.plan is not None:
            self.prog.restore(self.key, self.plan, self.binding)
            self.plan = None

    def __del__(self):
        self.give_back()


class _RunStack(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, prog, *params):
        key, plan = prog.lease(x.shape, True, ctx.needs_input_grad[0])
        ctx.lease = _Lease(prog, key, plan)
        return plan.forward(x)

    @staticmethod
    def backward(ctx, gout):
        lease = ctx.lease
        gx, grads = lease.plan.backward(gout)
        lease.give_back()
        return (gx, None, *grads)


class FusedSequential(nn.Sequential):
    """The nn.Sequential it replaces (same modules and state_dict), run from a native plan on device tensors."""

    def forward(self, x):
        # the plans run NCHW: a channels-last input or layer (model.to(memory_format=torch.channels_last)) runs the
        # layers one by one, on the device's channels-last kernels
        on_device = (x.device.type == DEVICE and x.dtype == torch.float32 and x.dim() == 4 and x.is_contiguous()
                     and all(p.is_contiguous() for p in self.parameters()))
        grad = torch.is_grad_enabled()
        if on_device and self.training and grad:
            prog = _program_of(self)
            counters = [m.num_batches_tracked for m in prog.bns if m.num_batches_tracked is not None]
            if counters:  # nn.BatchNorm2d.forward counts the batch; all of them in one launch here
                torch._foreach_add_(counters, 1)
            return _RunStack.apply(x, prog, *prog.params)
        if on_device and not self.training and not grad:
            prog = _program_of(self)
            key, plan = prog.lease(x.shape, False, False)
            try:
                return plan.forward(x)
            finally:
                prog.restore(key, plan, prog.binding)
        return super().forward(x)


def accelerate(model):
    """Swap every nn.Sequential of `model` made only of supported layers for a FusedSequential, in place. Parameters,
    buffers and state_dict are unchanged. Returns a short description."""
    swapped = [m for m in model.modules() if type(m) is nn.Sequential and fusable(m)]
    for m in swapped:
        m.__class__ = FusedSequential
    name = torch.cuda.get_device_name(0) if torch.cuda.is_available() else "no GPU"
    return f"{len(swapped)} fused stacks on {name}"


# ---- automatic fusion ----------------------------------------------------------------------------------------------

_seen = weakref.WeakSet()
_auto = {"on": os.environ.get("OMARCHY_MAC_TORCH_AUTO_FUSE", "1") != "0"}


def set_auto_fuse(on):
    """Turns automatic fusion on or off at run time (OMARCHY_MAC_TORCH_AUTO_FUSE sets the initial state). Returns the
    previous state."""
    prev, _auto["on"] = _auto["on"], bool(on)
    return prev


def _fuse_on_first_device_call(module, args):
    """Global forward pre-hook: the first time a plain nn.Sequential runs on a device tensor, it becomes a
    FusedSequential if every layer is supported (decided once per module)."""
    if not _auto["on"] or type(module) is not nn.Sequential or module in _seen:
        return None
    if not (args and isinstance(args[0], torch.Tensor) and args[0].device.type == DEVICE):
        return None
    _seen.add(module)
    if fusable(module):
        module.__class__ = FusedSequential
    return None


nn.modules.module.register_module_forward_pre_hook(_fuse_on_first_device_call)

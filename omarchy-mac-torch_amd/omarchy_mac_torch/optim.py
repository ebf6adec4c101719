"""Fused optimizers by default on the device (reference: omarchy_mac_torch/optim.py).

torch.optim.SGD, Adam and AdamW pick their per-tensor (foreach) implementation unless told otherwise; on this device
the fused one (`_fused_sgd_` / `_fused_adam_` / `_fused_adamw_`, one multi-tensor launch per step) is cheaper. PyTorch
has no hook for a device's preferred implementation, so `enable_fused_defaults` wraps the constructors: a call whose
parameters are all on the device, and that chose neither fused= nor foreach= (nor differentiable=, nor a tensor lr),
gets fused=True. `keeps_torch_default` says why a call is left alone. OMARCHY_MAC_TORCH_FUSED_OPTIM=0 leaves
torch.optim untouched.
"""

import functools
import os

import torch

from omarchy_mac_torch.native import DEVICE

_MARK = "_omarchy_mac_torch_fused_default"
DEFAULT_CLASSES = (torch.optim.SGD, torch.optim.Adam, torch.optim.AdamW)


def _tensors_of(params):
    """The tensors of a constructor's params argument: tensors, or param-group dicts (whose "params" is a tensor or
    an iterable of them)."""
    for item in params:
        if not isinstance(item, dict):
            yield item
        elif isinstance(item["params"], torch.Tensor):
            yield item["params"]
        else:
            yield from item["params"]


def keeps_torch_default(tensors, options):
    """Why a constructor call keeps torch's own choice of implementation, or None when it defaults to fused=True."""
    if not tensors:
        return "no parameters"
    if not all(isinstance(t, torch.Tensor) and t.device.type == DEVICE for t in tensors):
        return "parameters not all on the device"
    chosen = [k for k in ("fused", "foreach") if options.get(k) is not None]
    if chosen:
        return f"{chosen[0]}= given by the caller"
    if options.get("differentiable", False):
        return "differentiable=True"
    if isinstance(options.get("lr"), torch.Tensor):
        return "a tensor learning rate"
    return None


def fused_default(cls):
    """Wraps cls.__init__ (once) so that device-resident parameter sets default to fused=True."""
    original = cls.__init__
    if getattr(original, _MARK, False):
        return cls

    @functools.wraps(original)
    def __init__(self, params, *args, **kwargs):
        params = list(params)  # an iterator is consumed here and by the original constructor
        if keeps_torch_default(list(_tensors_of(params)), kwargs) is None:
            kwargs["fused"] = True
        original(self, params, *args, **kwargs)

    setattr(__init__, _MARK, True)
    cls.__init__ = __init__
    return cls


def enable_fused_defaults(classes=DEFAULT_CLASSES):
    """Applies fused_default to each class (the package does this on import unless OMARCHY_MAC_TORCH_FUSED_OPTIM=0);
    returns the classes."""
    return [fused_default(cls) for cls in classes]


if os.environ.get("OMARCHY_MAC_TORCH_FUSED_OPTIM", "1") != "0":
    enable_fused_defaults()

"""Fused optimizers by default on the device (reference: omarchy_mac_torch/optim.py).

torch.optim.SGD, Adam and AdamW pick their per-tensor (foreach) implementation unless told otherwise; on this device
the fused one (`_fused_sgd_` / `_fused_adam_` / `_fused_adamw_`, one multi-tensor launch per step) is cheaper, so the
constructors are wrapped to pass fused=True when every parameter is on the device and the caller chose neither
fused= nor foreach= (nor differentiable=, nor a tensor lr). OMARCHY_MAC_TORCH_FUSED_OPTIM=0 leaves torch.optim
untouched.
"""

import functools
import os

import torch

from omarchy_mac_torch.native import DEVICE

_WRAPPED = "_omarchy_mac_torch_fused_default"


def _all_params(params):
    out = []
    for item in params:
        if isinstance(item, dict):
            out.extend(item["params"] if not isinstance(item["params"], torch.Tensor) else [item["params"]])
        else:
            out.append(item)
    return out


def fused_default(cls):
    """Wraps cls.__init__ (once) so device-resident parameter sets default to fused=True."""
    init = cls.__init__
    if getattr(init, _WRAPPED, False):
        return cls

    @functools.wraps(init)
    def __init__(self, params, *args, **kwargs):
        params = list(params)
        flat = _all_params(params)
        if (flat and all(isinstance(p, torch.Tensor) and p.device.type == DEVICE for p in flat)
                and kwargs.get("fused") is None and kwargs.get("foreach") is None
                and not kwargs.get("differentiable", False) and not isinstance(kwargs.get("lr"), torch.Tensor)):
            kwargs["fused"] = True
        init(self, params, *args, **kwargs)

    setattr(__init__, _WRAPPED, True)
    cls.__init__ = __init__
    return cls


if os.environ.get("OMARCHY_MAC_TORCH_FUSED_OPTIM", "1") != "0":
    for _cls in (torch.optim.SGD, torch.optim.Adam, torch.optim.AdamW):
        fused_default(_cls)

"""omarchy-mac-torch's convolution hot path on AMD Instinct MI355X (gfx950), as hand-written HIP.

    import omarchy_mac_torch                 # registers the "omarchy_mac_torch" device
    model = model.to("omarchy_mac_torch")
    omarchy_mac_torch.accelerate(model)      # optional: fused conv/BN/ReLU/pool stacks
    torch.compile(model, backend="omarchy_mac_torch")

The same API as the reference package (omarchy_mac_torch/__init__.py): DEVICE, FALLBACKS, accelerate,
FusedSequential, synchronize, empty_cache, memory_allocated, memory_reserved, set_queue_depth, validate_kernels.
`hip_ops` exposes the tensor-level entry points over libomt_hip.so's C ABI directly; `graphs` replays captured steps
as HIP graphs.
"""

from omarchy_mac_torch import _lib  # noqa: F401  (libomt_hip.so; ImportError when it is not built)
from omarchy_mac_torch import hip_ops  # noqa: F401
from omarchy_mac_torch import native as _native  # noqa: F401  (registers the device)
from omarchy_mac_torch import compile as _compile  # noqa: F401  (torch.compile backend "omarchy_mac_torch")
from omarchy_mac_torch import optim as _optim  # noqa: F401  (fused SGD / Adam / AdamW by default on the device)
from omarchy_mac_torch import graphs  # noqa: F401  (captured steps replayed as HIP graphs)
from omarchy_mac_torch.native import (DEVICE, FALLBACKS, empty_cache, memory_allocated, memory_reserved,
                                      set_queue_depth, synchronize, validate_kernels)
from omarchy_mac_torch.stacks import FusedSequential, accelerate

__version__ = "0.2.0"
__all__ = ["DEVICE", "FALLBACKS", "FusedSequential", "accelerate", "empty_cache", "graphs", "hip_ops", "memory_allocated",
           "memory_reserved", "set_queue_depth", "synchronize", "validate_kernels"]

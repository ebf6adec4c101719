"""omarchy-mac-torch for AMD Instinct MI355X (gfx950): the reference's convolution hot path as hand-written HIP.

    import omarchy_mac_torch
    from omarchy_mac_torch import hip_ops      # tensor-level entry points over libomt_hip.so
"""

from omarchy_mac_torch import _lib  # noqa: F401  (loads libomt_hip.so; raises ImportError when it is not built)
from omarchy_mac_torch import hip_ops  # noqa: F401

__version__ = "0.2.0"

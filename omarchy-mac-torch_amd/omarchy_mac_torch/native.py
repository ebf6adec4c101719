"""Loads the torch extension (_native) and registers the "omarchy_mac_torch" PrivateUse1 device with PyTorch, as the
reference's omarchy_mac_torch/native.py does (device module, generated tensor/module methods, FALLBACKS).

The device's memory is HBM on the MI355X, allocated by libomt_hip.so. Its convolution hot path runs that library's
HIP kernels; every other op is delegated to torch's own HIP kernels on the same memory. Both native libraries are
required: a missing build raises ImportError instead of running anything elsewhere.
"""

import atexit
import collections.abc
import contextlib
import functools
import json
import os
import pathlib
import tempfile
import types

import torch

from omarchy_mac_torch import _lib  # noqa: F401  (loads libomt_hip.so before the extension that links it)

_HERE = pathlib.Path(__file__).resolve().parent
DEVICE = "omarchy_mac_torch"


def _check_build():
    if not (_HERE / "_native.so").exists():
        raise ImportError("omarchy-mac-torch: the torch extension is not built; run "
                          "`python omarchy-mac-torch_amd/build_native.py` (or __graft_entry__.build())")


_check_build()
from omarchy_mac_torch import _native as core  # noqa: E402

if core.built_with_torch.split("+")[0] != torch.__version__.split("+")[0]:
    raise ImportError(f"omarchy-mac-torch was built against torch {core.built_with_torch} but torch "
                      f"{torch.__version__} is installed; rebuild with omarchy-mac-torch_amd/build_native.py")

if torch._C._get_privateuse1_backend_name() != DEVICE:
    torch.utils.rename_privateuse1_backend(DEVICE)
    # tensor.omarchy_mac_torch(), module.omarchy_mac_torch(), storage methods, is_omarchy_mac_torch
    torch.utils.generate_methods_for_privateuse1_backend(for_tensor=True, for_module=True, for_packed_sequence=True,
                                                         for_storage=True)

core.set_fold(int(os.environ.get("OMARCHY_MAC_TORCH_FOLD", "1")))
core.set_tuning(os.environ.get("OMARCHY_MAC_TORCH_TUNE", "1") != "0", 0)
core.set_debug(os.environ.get("OMARCHY_MAC_TORCH_DEBUG", "0") == "1")


# ---- the device module: torch.omarchy_mac_torch.* ----
_mod = types.ModuleType("torch." + DEVICE)
_mod.is_available = lambda: torch.cuda.is_available()
_mod.is_initialized = lambda: True
_mod._lazy_init = lambda: None
_mod._is_in_bad_fork = lambda: False
_mod.device_count = lambda: 1
_mod.current_device = lambda: 0
_mod.set_device = lambda d: None
_mod.get_amp_supported_dtype = lambda: [torch.float32]
_mod.synchronize = lambda device=None: core.sync()
_mod.empty_cache = core.empty_cache
_mod.memory_allocated = lambda device=None: core.memory_allocated()
_mod.memory_reserved = lambda device=None: core.memory_reserved()
# random numbers come from torch's HIP generator (the device's RNG ops run on torch's HIP kernels). torch.cuda only
# queues a seed until torch.cuda itself is initialized, which a program that uses this device alone never triggers:
# torch.manual_seed (which calls manual_seed_all below) would then leave the generator unseeded, so every RNG entry
# initializes torch.cuda first.


def _hip_rng(fn):
    def call(*args, **kwargs):
        if torch.cuda.is_available():  # without a GPU the calls stay queued, as torch.cuda's own do
            torch.cuda._lazy_init()
        return fn(*args, **kwargs)
    return call


_mod.manual_seed = _hip_rng(lambda seed: torch.cuda.manual_seed(int(seed)))
_mod.manual_seed_all = _hip_rng(lambda seed: torch.cuda.manual_seed_all(int(seed)))
_mod.seed = _hip_rng(lambda: torch.cuda.seed())
_mod.seed_all = _hip_rng(lambda: torch.cuda.seed_all())
_mod.initial_seed = _hip_rng(lambda: torch.cuda.initial_seed())
_mod.get_rng_state = _hip_rng(lambda device=None: torch.cuda.get_rng_state())
_mod.set_rng_state = _hip_rng(lambda state, device=None: torch.cuda.set_rng_state(state))


class _DeviceContext:
    def __init__(self, device):
        pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        return False


_mod.device = _DeviceContext
if not hasattr(torch, DEVICE):
    torch._register_device_module(DEVICE, _mod)


# ---- autograd over torch.cuda tensors ----
# With this PrivateUse1 device registered, PyTorch takes it as the process's accelerator and its autograd engine keeps
# streams for this device type only: a backward pass over torch.cuda tensors then stops on an internal assertion of
# the engine ("opt_ready_stream && opt_parent_stream", torch/csrc/autograd/engine.cpp). A backward or grad call whose
# roots (or requested inputs) are torch.cuda tensors is refused up front with an error that says why.

CUDA_AUTOGRAD_MSG = ("omarchy-mac-torch: autograd over torch.cuda tensors is not supported in a process that has "
                     "registered the omarchy_mac_torch device (PyTorch then takes that device as the accelerator, and "
                     "its autograd engine stops on an internal assertion for cuda tensors). Train on the "
                     "omarchy_mac_torch device (model.to('omarchy_mac_torch')); forward work and explicit aten calls "
                     "on cuda tensors are unaffected.")


def _checked(g):
    """g (a tensor, a gradient edge or a collection of them; an iterator is read into a tuple, which the caller passes
    on), after refusing torch.cuda tensors in it."""
    if g is None:
        return g
    items = (g,) if isinstance(g, torch.Tensor) else g if isinstance(g, (list, tuple)) else tuple(g)
    if any(isinstance(t, torch.Tensor) and t.device.type == "cuda" for t in items):
        raise RuntimeError(CUDA_AUTOGRAD_MSG)
    return g if isinstance(g, (torch.Tensor, list, tuple)) else items


_autograd_backward, _autograd_grad = torch.autograd.backward, torch.autograd.grad


@functools.wraps(_autograd_backward)
def _backward(tensors, grad_tensors=None, retain_graph=None, create_graph=False, grad_variables=None, inputs=None):
    return _autograd_backward(_checked(tensors), grad_tensors, retain_graph, create_graph, grad_variables,
                              inputs=_checked(inputs))


@functools.wraps(_autograd_grad)
def _grad(outputs, inputs, *args, **kwargs):
    return _autograd_grad(_checked(outputs), _checked(inputs), *args, **kwargs)


_backward.omt_cuda_guard = _grad.omt_cuda_guard = True
if not getattr(torch.autograd.backward, "omt_cuda_guard", False):
    torch.autograd.backward, torch.autograd.grad = _backward, _grad


def synchronize():
    core.sync()


def set_queue_depth(depth=3, chunk=64):
    """Kept for the reference's API (it bounded its Vulkan submission queue). HIP streams are already asynchronous
    and the driver bounds them, so there is nothing to configure."""
    return None


def empty_cache():
    core.empty_cache()


def memory_allocated():
    return core.memory_allocated()


def memory_reserved():
    return core.memory_reserved()


def validate_kernels():
    """The reference compiled WGSL at run time; here every kernel is compiled ahead of time for gfx950. Returns the
    failures: always none once the library has loaded."""
    return []


class _FallbackView(collections.abc.Mapping):
    """FALLBACKS: hot-path calls that ran on torch's HIP kernels instead of this library's, as a live read-only mapping
    {"op (why)": count} over the extension's counters (clear() resets them)."""

    def __getitem__(self, key):
        return core.fallback_counts()[key]

    def __iter__(self):
        return iter(core.fallback_counts())

    def __len__(self):
        return len(core.fallback_counts())

    def clear(self):
        core.reset_fallbacks()

    def __repr__(self):
        return f"FALLBACKS({core.fallback_counts()!r})"


FALLBACKS = _FallbackView()


# ---- on-disk conv plan cache (reference: omarchy_mac_torch/native.py:185-209) ----
# One JSON object {"dir,n,ci,co,ih,iw,oh,ow,ks,stride,pad": [tile, slices]}, the reference's key format. The values
# index this library's gfx950 tile tables (the file name carries the gather table's size), so the file is not the
# reference's, whose entries name its own tiles and a split-K multiplier.
TUNE_FILE = os.environ.get(
    "OMARCHY_MAC_TORCH_TUNE_FILE",
    os.path.expanduser(f"~/.cache/omarchy-mac-torch/tuning-gfx950-t{_lib.L.omt_conv_num_tiles(_lib.OMT_DIR_FWD) // 3}.json"))


class TuningStore:
    """The conv plan cache's file. `load` feeds the well-formed entries to the plan cache one by one (an entry with a
    malformed key or value, or a plan the tile tables do not have, is skipped and counted in `skipped`); `save` writes
    the file's entries merged with the cache's (the cache wins), through a temporary file renamed over the old one so
    that readers never see half a file."""

    def __init__(self, path=None):
        self.path = pathlib.Path(path or TUNE_FILE)
        self.skipped = 0

    def _read(self):
        try:
            data = json.loads(self.path.read_text())
        except (OSError, ValueError):
            return {}
        return data if isinstance(data, dict) else {}

    def load(self):
        """Returns the number of entries the plan cache accepted."""
        good, self.skipped = {}, 0
        for key, val in self._read().items():
            fields = key.split(",") if isinstance(key, str) else []
            plan = val if isinstance(val, list) and len(val) == 2 else None
            if (len(fields) != 11 or not all(f.strip().lstrip("-").isdigit() for f in fields) or plan is None
                    or not all(isinstance(v, int) and not isinstance(v, bool) for v in plan)):
                self.skipped += 1
                continue
            good[key] = (plan[0], plan[1])
        accepted = core.tune_load(good) if good else 0
        self.skipped += len(good) - accepted
        return accepted

    def save(self):
        merged = self._read()
        merged.update({k: [int(v[0]), int(v[1])] for k, v in core.tune_dump().items()})
        self.path.parent.mkdir(parents=True, exist_ok=True)
        fd, tmp = tempfile.mkstemp(prefix=self.path.name + ".", dir=self.path.parent)
        try:
            with os.fdopen(fd, "w") as f:
                json.dump(merged, f, sort_keys=True)
            os.replace(tmp, self.path)
        except BaseException:
            with contextlib.suppress(OSError):
                os.unlink(tmp)
            raise
        return len(merged)


def _save_at_exit(store):
    try:
        store.save()
    except OSError:  # a read-only home directory must not fail the interpreter's exit
        pass


if core.tuning():
    _store = TuningStore()
    _store.load()
    atexit.register(_save_at_exit, _store)

"""CPU checks of the host runtime (no GPU needed): the on-disk conv plan cache (reference
omarchy_mac_torch/native.py:185-209, csrc/conv.cpp:243-272) and the fused-stack fusability rules (reference
omarchy_mac_torch/stacks.py:41-63)."""

import json
import os
import pathlib
import subprocess
import sys
import textwrap

import pytest
import torch.nn as nn

ROOT = pathlib.Path(__file__).resolve().parent.parent

# 3x3 stride-1 conv, C 64 -> 64 on 56x56 at batch 2 ("dir,n,ci,co,ih,iw,oh,ow,ks,stride,pad")
GEO = "2,64,64,56,56,56,56,3,1,1"


@pytest.fixture()
def core():
    from omarchy_mac_torch import native
    native.core.clear_plans()
    yield native.core
    native.core.clear_plans()


def test_tuning_file_round_trip_in_a_fresh_process(core, tmp_path):
    """Plans saved by one process are loaded by the next and then drive the launches: the workspace queries, which
    resolve the same plan as the launch, change with the loaded K split."""
    from omarchy_mac_torch import native
    path = tmp_path / "tune.json"
    plans = {f"0,{GEO}": (5, 3), f"1,{GEO}": (2, 1), f"2,{GEO}": (1, 49)}
    assert core.tune_load(plans) == 3
    assert native.TuningStore(path).save() == 3
    saved = json.loads(path.read_text())
    assert {k: tuple(v) for k, v in saved.items()} == plans
    core.clear_plans()

    child = textwrap.dedent(f"""
        import ctypes, json, sys
        sys.path[:0] = [{str(ROOT)!r}, {str(ROOT / 'omarchy-mac-torch_amd')!r}]
        from omarchy_mac_torch import native, _lib
        g = _lib.conv_geo(2, 64, 64, 56, 56, 3, 1, 1)
        L = _lib.L
        out = {{"dump": {{k: list(v) for k, v in native.core.tune_dump().items()}},
               "fwd_ws": L.omt_conv_fwd_workspace(ctypes.byref(g)),
               "wgrad_ws": L.omt_conv_wgrad_workspace(ctypes.byref(g))}}
        native.core.clear_plans()
        out["fwd_ws_model"] = L.omt_conv_fwd_workspace(ctypes.byref(g))
        print(json.dumps(out))
    """)
    env = dict(os.environ, OMARCHY_MAC_TORCH_TUNE="1", OMARCHY_MAC_TORCH_TUNE_FILE=str(path))
    r = subprocess.run([sys.executable, "-c", child], capture_output=True, text=True, env=env, timeout=300)
    assert r.returncode == 0, r.stderr
    out = json.loads(r.stdout.strip().splitlines()[-1])
    assert {k: tuple(v) for k, v in out["dump"].items()} == plans
    # forward plan (tile 5, 3 K slices): the tap-major filter, then three slices of partial outputs
    ybytes = 2 * 64 * 56 * 56 * 4
    assert out["fwd_ws"] == 64 * 64 * 9 * 4 + 3 * ybytes != out["fwd_ws_model"]
    # grad-weight plan with 49 slices (128 pixels each): 49 partial filters
    assert out["wgrad_ws"] == 49 * 64 * 64 * 9 * 4


def test_tuning_file_skips_malformed_entries(core, tmp_path):
    from omarchy_mac_torch import native
    path = tmp_path / "tune.json"
    path.write_text(json.dumps({
        f"0,{GEO}": [5, 1],                       # good
        f"2,{GEO}": [3, 16],                      # good
        f"0,{GEO},9": [5, 1],                     # twelve fields
        "0,2,64,64,56,56,56,56,3,1": [5, 1],      # ten fields
        "0,2,x,64,56,56,56,56,3,1,1": [5, 1],     # not a number
        f"1,{GEO}": [5],                          # one value
        f"1,{GEO.replace('3,1,1', '3,1,2')}": [True, 1],    # a bool is not a tile
        f"1,{GEO.replace('64,64', '64,65')}": [999, 1],     # tile out of range
        f"2,{GEO.replace('2,64', '3,64')}": [0, 0],          # no K slice
        "0,2,64,64,56,56,56,56,13,1,6": [0, 1],   # kernel size 13: not a dense conv this library covers
        "7,2,64,64,56,56,56,56,3,1,1": [0, 1],    # no such direction
    }))
    store = native.TuningStore(path)
    assert store.load() == 2
    assert store.skipped == 9
    assert core.tune_dump() == {f"0,{GEO}": (5, 1), f"2,{GEO}": (3, 16)}
    # a file that is not JSON, or not an object, loads nothing and saving replaces it
    path.write_text("{not json")
    assert native.TuningStore(path).load() == 0
    path.write_text("[1, 2]")
    assert native.TuningStore(path).load() == 0
    assert native.TuningStore(path).save() == 2
    assert set(json.loads(path.read_text())) == {f"0,{GEO}", f"2,{GEO}"}


def test_tuning_file_save_merges_and_the_cache_wins(core, tmp_path):
    from omarchy_mac_torch import native
    path = tmp_path / "sub" / "tune.json"
    path.parent.mkdir()
    path.write_text(json.dumps({f"0,{GEO}": [1, 1], f"1,{GEO}": [2, 2]}))
    core.tune_load({f"0,{GEO}": (5, 3)})
    assert native.TuningStore(path).save() == 2
    assert json.loads(path.read_text()) == {f"0,{GEO}": [5, 3], f"1,{GEO}": [2, 2]}
    assert [p.name for p in path.parent.iterdir()] == ["tune.json"]  # no temporary file left behind


def _conv(ci, co, ks, **kw):
    return nn.Conv2d(ci, co, ks, padding=kw.pop("padding", ks // 2), bias=kw.pop("bias", False), **kw)


@pytest.mark.parametrize("layers,ok", [
    ([_conv(3, 8, 3), nn.BatchNorm2d(8), nn.ReLU(), nn.MaxPool2d(2), nn.AdaptiveAvgPool2d(1)], True),
    ([_conv(3, 8, 1), _conv(8, 8, 5), nn.AvgPool2d(2), _conv(8, 8, 7, groups=8)], True),
    ([nn.BatchNorm2d(3), nn.ReLU(), _conv(3, 8, 3)], False),                  # must start with a conv
    ([_conv(3, 8, 3, bias=True)], False),                                      # bias
    ([_conv(3, 8, 7)], False),                                                 # dense 7x7
    ([_conv(8, 8, 9, groups=8)], False),                                       # depthwise 9x9
    ([_conv(3, 8, 3, stride=2)], False),                                       # stride 2
    ([_conv(3, 8, 3, padding=0)], False),                                      # not "same"
    ([_conv(3, 8, 3, padding_mode="reflect")], False),                         # not zero padding
    ([_conv(4, 8, 3, groups=2)], False),                                       # grouped
    ([_conv(3, 8, 3), nn.BatchNorm2d(8)], False),                              # BatchNorm without its ReLU
    ([_conv(3, 8, 3), nn.BatchNorm2d(8, eps=1e-3), nn.ReLU()], False),         # eps
    ([_conv(3, 8, 3), nn.BatchNorm2d(8, momentum=None), nn.ReLU()], False),    # cumulative average
    ([_conv(3, 8, 3), nn.BatchNorm2d(8, affine=False), nn.ReLU()], False),
    ([_conv(3, 8, 3), nn.ReLU()], False),                                      # a ReLU on its own
    ([_conv(3, 8, 3), nn.MaxPool2d(3)], False),
    ([_conv(3, 8, 3), nn.MaxPool2d(2, ceil_mode=True)], False),
    ([_conv(3, 8, 3), nn.MaxPool2d(2, return_indices=True)], False),
    ([_conv(3, 8, 3), nn.AvgPool2d(2, divisor_override=3)], False),
    ([_conv(3, 8, 3), nn.AdaptiveAvgPool2d(2)], False),
    ([_conv(3, 8, 3), nn.AdaptiveAvgPool2d((1, 1))], True),
])
def test_fusability_rules(layers, ok):
    from omarchy_mac_torch import stacks
    seq = nn.Sequential(*layers)
    assert stacks.fusable(seq) is ok
    if ok:
        prog = stacks._compile(seq)
        convs = [m for m in layers if isinstance(m, nn.Conv2d)]
        bns = [m for m in layers if isinstance(m, nn.BatchNorm2d)]
        assert len(prog.params) == len(convs) + 2 * len(bns) and prog.bns == bns
        assert len(prog.records) == len(layers) - len(bns)  # each BatchNorm's ReLU is part of its step


def test_autograd_over_cuda_tensors_is_refused_up_front():
    """backward / grad whose roots or requested inputs are torch.cuda tensors raise the library's explanation (PyTorch's
    engine would stop on an internal assertion once the device is registered); CPU autograd, gradient edges and
    iterators of inputs pass through unchanged. Fake cuda tensors stand in for real ones (no GPU here)."""
    import torch
    from torch._subclasses.fake_tensor import FakeTensorMode
    from omarchy_mac_torch import native
    assert torch.autograd.backward.omt_cuda_guard and torch.autograd.grad.omt_cuda_guard
    with FakeTensorMode(allow_non_fake_inputs=True):
        fake = torch.empty(3, device="cuda")
    for roots in (fake, [fake], (torch.ones(1), fake), iter([fake])):
        with pytest.raises(RuntimeError, match="omarchy_mac_torch device"):
            native._checked(roots)
    x = torch.randn(4, requires_grad=True)
    (x * 3).sum().backward(inputs=iter([x]))  # an iterator of inputs is read once and handed on
    assert torch.equal(x.grad, torch.full((4,), 3.0))
    (gx,) = torch.autograd.grad((x * x).sum(), [x])
    assert torch.allclose(gx, 2 * x.detach())


def test_replay_static_pointer_holds_end_with_the_storage():
    """The compile backend's registry of memory that stays put while a captured graph lives: a graph's own memory is
    held until release(); a caller's storage it reads in place is held only while that storage lives (then a later
    tensor at the same address is not taken for it); two graphs holding one address keep it until both let go."""
    import gc

    import torch

    from omarchy_mac_torch import replay

    own = torch.empty(16)
    param, other = torch.empty(16), torch.empty(16)
    p_own, p_param, p_other = (t.untyped_storage().data_ptr() for t in (own, param, other))
    before = dict(replay._static_ptrs)
    a = replay._Holds({p_own}, [(p_param, param), (p_other, other)])
    b = replay._Holds(set(), [(p_param, param)])
    assert {p_own, p_param, p_other} <= set(replay._static_ptrs) and replay._static_ptrs[p_param] == 2
    del other
    gc.collect()
    assert p_other not in replay._static_ptrs  # freed: dropped by its finalizer
    a.release()
    a.release()  # once only
    assert p_own not in replay._static_ptrs and replay._static_ptrs[p_param] == 1
    del param
    gc.collect()
    assert p_param not in replay._static_ptrs
    b.release()
    assert replay._static_ptrs == before

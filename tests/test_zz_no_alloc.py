"""omt_conv_wgrad_noalloc, the grad-weight entry point that allocates nothing (its split-K partials live in the
library's static device scratch array), against omt_conv_wgrad with a caller workspace: bit-identical on two calls in
a row, the second on a smaller input, through the C ABI; captured into a HIP graph and replayed without allocating. Also:
a plan whose partials exceed the scratch is rejected on the host before any launch."""

import ctypes

import numpy as np
import pytest
import torch

from oracle import oracle as orc

pytestmark = pytest.mark.gpu


def _wgrad_both(cuda, n, ci, co, h, ks, s, p, plan=None):
    from omarchy_mac_torch import _lib, hip_ops
    L = _lib.L
    g = _lib.conv_geo(n, ci, co, h, h, ks, s, p)
    gen = torch.Generator(device=cuda).manual_seed(n * 1000 + ci)
    x = torch.randn((n, ci, h, h), device=cuda, generator=gen)
    gy = torch.randn((n, co, g.oh, g.ow), device=cuda, generator=gen)
    if plan is not None:
        hip_ops.set_conv_plan("wgrad", x.shape, (co, ci, ks, ks), s, p, *plan)
    need = L.omt_conv_wgrad_workspace(ctypes.byref(g))
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device=cuda)
    ref = torch.full((co, ci, ks, ks), float("nan"), device=cuda)
    out = torch.full((co, ci, ks, ks), float("nan"), device=cuda)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    vp = ctypes.c_void_p
    _lib.check(L.omt_conv_wgrad(ctypes.byref(g), vp(x.data_ptr()), vp(gy.data_ptr()), vp(ref.data_ptr()),
                                vp(ws.data_ptr()), need, stream), "omt_conv_wgrad")
    _lib.check(L.omt_conv_wgrad_noalloc(ctypes.byref(g), vp(x.data_ptr()), vp(gy.data_ptr()), vp(out.data_ptr()),
                                        stream), "omt_conv_wgrad_noalloc")
    torch.cuda.synchronize()
    return x, gy, ref, out, need


def test_wgrad_noalloc_matches_wgrad_on_two_calls(cuda):
    from omarchy_mac_torch import hip_ops
    try:
        # first call: a split-K plan with 14 slices (a 3.1 MB partial buffer in the scratch)
        x, gy, ref, out, need = _wgrad_both(cuda, 8, 64, 96, 28, 3, 1, 1, plan=(2, 14))
        assert need == 14 * 96 * 64 * 9 * 4
        assert torch.equal(out, ref)
        orc_gw = orc.conv_wgrad(x.cpu().numpy(), gy.cpu().numpy(), 3, 1, 1)
        assert orc.rel_l2(out.cpu().numpy(), orc_gw) <= 1e-4
        # second call, smaller input and a smaller split: the scratch keeps the first call's larger contents beyond
        # what this call writes and reads
        x, gy, ref, out, need = _wgrad_both(cuda, 4, 16, 24, 20, 3, 2, 1, plan=(0, 3))
        assert need == 3 * 24 * 16 * 9 * 4
        assert torch.equal(out, ref)
        orc_gw = orc.conv_wgrad(x.cpu().numpy(), gy.cpu().numpy(), 3, 2, 1)
        assert orc.rel_l2(out.cpu().numpy(), orc_gw) <= 1e-4
        # a plan without a K split uses no scratch at all
        x, gy, ref, out, need = _wgrad_both(cuda, 4, 16, 24, 20, 3, 2, 1, plan=(0, 1))
        assert need == 0 and torch.equal(out, ref)
    finally:
        hip_ops.clear_conv_plans()


def test_wgrad_noalloc_rejects_partials_beyond_the_scratch(cuda):
    from omarchy_mac_torch import _lib, hip_ops
    L = _lib.L
    g = _lib.conv_geo(256, 64, 64, 56, 56, 3, 1, 1)
    try:
        hip_ops.set_conv_plan("wgrad", (256, 64, 56, 56), (64, 64, 3, 3), 1, 1, 2, 4096)
        need = L.omt_conv_wgrad_workspace(ctypes.byref(g))
        assert need > _lib.NOALLOC_SCRATCH_BYTES
        fake = ctypes.c_void_p(0x1000)  # never dereferenced: the size check comes first
        assert L.omt_conv_wgrad_noalloc(ctypes.byref(g), fake, fake, fake, None) == _lib.OMT_INVALID
        assert b"static scratch" in L.omt_last_error()
    finally:
        hip_ops.clear_conv_plans()


def test_wgrad_noalloc_under_graph_capture_allocates_nothing(cuda):
    """The callers the entry point is for: captured into a HIP graph (torch.cuda.graph) and replayed three times, with
    eager work and a synchronization between the replays, every replay gives omt_conv_wgrad's bits, and neither
    torch's nor the library's allocator holds a byte more than before the capture."""
    from omarchy_mac_torch import _lib, hip_ops
    L = _lib.L
    vp = ctypes.c_void_p
    n, ci, co, h = 8, 32, 48, 14
    g = _lib.conv_geo(n, ci, co, h, h, 3, 1, 1)
    try:
        hip_ops.set_conv_plan("wgrad", (n, ci, h, h), (co, ci, 3, 3), 1, 1, 2, 6)  # a K split: partials in the scratch
        need = L.omt_conv_wgrad_workspace(ctypes.byref(g))
        assert 0 < need <= _lib.NOALLOC_SCRATCH_BYTES
        gen = torch.Generator(device=cuda).manual_seed(5)
        x = torch.randn((n, ci, h, h), device=cuda, generator=gen)
        gy = torch.randn((n, co, h, h), device=cuda, generator=gen)
        ws = torch.empty(need, dtype=torch.uint8, device=cuda)
        ref = torch.empty((co, ci, 3, 3), device=cuda)
        out = torch.full((co, ci, 3, 3), float("nan"), device=cuda)
        stream = vp(torch.cuda.current_stream().cuda_stream)
        _lib.check(L.omt_conv_wgrad(ctypes.byref(g), vp(x.data_ptr()), vp(gy.data_ptr()), vp(ref.data_ptr()),
                                    vp(ws.data_ptr()), need, stream), "omt_conv_wgrad")
        torch.cuda.synchronize()
        torch.cuda.empty_cache()  # as torch.cuda.graph does before it captures
        torch_before, omt_before = torch.cuda.memory_reserved(), L.omt_memory_reserved()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            cap = vp(torch.cuda.current_stream().cuda_stream)
            _lib.check(L.omt_conv_wgrad_noalloc(ctypes.byref(g), vp(x.data_ptr()), vp(gy.data_ptr()),
                                                vp(out.data_ptr()), cap), "omt_conv_wgrad_noalloc (captured)")
        for i in range(3):
            out.fill_(float("nan"))
            x.mul_(1.0)  # eager work between the replays
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, ref), i
        assert torch.cuda.memory_reserved() == torch_before
        assert L.omt_memory_reserved() == omt_before
        graph.reset()
    finally:
        hip_ops.clear_conv_plans()

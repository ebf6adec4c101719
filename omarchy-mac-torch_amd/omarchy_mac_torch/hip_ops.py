"""Tensor-level entry points over libomt_hip.so for float32 NCHW tensors on the HIP device.

Each function validates shapes on the host, allocates outputs (and any workspace the C ABI asks for) with torch's
device allocator, and launches on torch's current stream. They are the operator implementations behind the
reference's convolution_ / convolution_backward_ (csrc/conv.cpp:179-237), batch_norm_ / batch_norm_backward_
(csrc/nn.cpp:25-78), the pooling ops (csrc/nn.cpp:157-222) and the fused ops of csrc/fused.cpp.
"""

import ctypes

import torch

from . import _lib
from ._lib import L, check

_vp = ctypes.c_void_p


def _ptr(t):
    return None if t is None else _vp(t.data_ptr())


def _stream(device=None):
    return _vp(torch.cuda.current_stream(device).cuda_stream)


def _need(t, name, dim=None):
    if t is None:
        return None
    if not t.is_cuda or t.dtype != torch.float32:
        raise TypeError(f"{name}: expected a float32 tensor on the HIP device, got {t.dtype} on {t.device}")
    if dim is not None and t.dim() != dim:
        raise ValueError(f"{name}: expected {dim}-D, got {tuple(t.shape)}")
    return t.contiguous()


def _workspace(nbytes, device):
    if nbytes == 0:
        return None, 0
    return torch.empty(int(nbytes), dtype=torch.uint8, device=device), int(nbytes)


def _pair(v):
    return (v, v) if isinstance(v, int) else tuple(v)


# ---- dense convolution ------------------------------------------------------------------------------------------

def conv_geo_for(x_shape, w_shape, stride, pad):
    n, ci, ih, iw = x_shape
    co, wci, kh, kw = w_shape
    if wci != ci or kh != kw:
        raise ValueError(f"conv: weight {tuple(w_shape)} does not match input {tuple(x_shape)}")
    return _lib.conv_geo(n, ci, co, ih, iw, kh, stride, pad)


def conv2d(x, w, bias=None, stride=1, padding=0, relu=False, bn=None, bn_eps=1e-5):
    """y = conv(x, w) + bias, optional ReLU. bn = (mean, var, gamma, beta) maps the input through eval BatchNorm +
    ReLU on in-bounds taps first (reference kind-3 loader, omarchy_mac_torch/gemm.py:139-141)."""
    x, w, bias = _need(x, "x", 4), _need(w, "w", 4), _need(bias, "bias", 1)
    g = conv_geo_for(x.shape, w.shape, stride, padding)
    y = torch.empty((g.n, g.co, g.oh, g.ow), device=x.device, dtype=torch.float32)
    bnp = [None] * 4 if bn is None else [_need(t, "bn", 1) for t in bn]
    epi = (_lib.OMT_EPI_BIAS if bias is not None else 0) | (_lib.OMT_EPI_RELU if relu else 0)
    ws, nb = _workspace(L.omt_conv_fwd_workspace(ctypes.byref(g)), x.device)
    check(L.omt_conv_fwd(ctypes.byref(g), _ptr(x), _ptr(w), _ptr(bias), epi, *[_ptr(t) for t in bnp], bn_eps,
                         _ptr(y), _ptr(ws), nb, _stream(x.device)), "conv2d")
    return y


def conv2d_stats(x, w, stride=1, padding=0):
    """y = conv(x, w) and the training-BatchNorm sums of y from the epilogue (omt_conv_fwd_stats): returns
    (y, stats [co][groups][2] float64, groups). Raises Unsupported when the layer's plan splits K."""
    x, w = _need(x, "x", 4), _need(w, "w", 4)
    g = conv_geo_for(x.shape, w.shape, stride, padding)
    y = torch.empty((g.n, g.co, g.oh, g.ow), device=x.device, dtype=torch.float32)
    sb = L.omt_conv_fwd_stats_bytes(ctypes.byref(g))
    stats = torch.empty((sb // 8,), device=x.device, dtype=torch.float64)
    groups = ctypes.c_int32(0)
    ws, nb = _workspace(L.omt_conv_fwd_workspace(ctypes.byref(g)), x.device)
    check(L.omt_conv_fwd_stats(ctypes.byref(g), _ptr(x), _ptr(w), _ptr(y), _ptr(stats), sb, ctypes.byref(groups),
                               _ptr(ws), nb, _stream(x.device)), "conv2d_stats")
    gr = groups.value
    return y, stats[:g.co * gr * 2].view(g.co, gr, 2), gr


def conv2d_dgrad(gy, w, x_shape, stride=1, padding=0):
    gy, w = _need(gy, "gy", 4), _need(w, "w", 4)
    g = conv_geo_for(x_shape, w.shape, stride, padding)
    if tuple(gy.shape) != (g.n, g.co, g.oh, g.ow):
        raise ValueError(f"conv dgrad: gy {tuple(gy.shape)} != {(g.n, g.co, g.oh, g.ow)}")
    gx = torch.empty(tuple(x_shape), device=gy.device, dtype=torch.float32)
    ws, nb = _workspace(L.omt_conv_dgrad_workspace(ctypes.byref(g)), gy.device)
    check(L.omt_conv_dgrad(ctypes.byref(g), _ptr(gy), _ptr(w), _ptr(gx), _ptr(ws), nb, _stream(gy.device)),
          "conv2d_dgrad")
    return gx


def conv2d_wgrad(x, gy, ks, stride=1, padding=0):
    x, gy = _need(x, "x", 4), _need(gy, "gy", 4)
    n, ci, ih, iw = x.shape
    co = gy.shape[1]
    g = _lib.conv_geo(n, ci, co, ih, iw, ks, stride, padding)
    if tuple(gy.shape) != (g.n, g.co, g.oh, g.ow):
        raise ValueError(f"conv wgrad: gy {tuple(gy.shape)} != {(g.n, g.co, g.oh, g.ow)}")
    gw = torch.empty((co, ci, ks, ks), device=x.device, dtype=torch.float32)
    ws, nb = _workspace(L.omt_conv_wgrad_workspace(ctypes.byref(g)), x.device)
    check(L.omt_conv_wgrad(ctypes.byref(g), _ptr(x), _ptr(gy), _ptr(gw), _ptr(ws), nb, _stream(x.device)),
          "conv2d_wgrad")
    return gw


def conv2d_bwd(x, gy, w, stride=1, padding=0):
    """(grad input, grad weight) of one dense convolution in one call (omt_conv_bwd: both GEMMs share a launch when
    their plans allow it)."""
    x, gy, w = _need(x, "x", 4), _need(gy, "gy", 4), _need(w, "w", 4)
    g = conv_geo_for(x.shape, w.shape, stride, padding)
    if tuple(gy.shape) != (g.n, g.co, g.oh, g.ow):
        raise ValueError(f"conv bwd: gy {tuple(gy.shape)} != {(g.n, g.co, g.oh, g.ow)}")
    gx = torch.empty(tuple(x.shape), device=x.device, dtype=torch.float32)
    gw = torch.empty(tuple(w.shape), device=x.device, dtype=torch.float32)
    ws, nb = _workspace(L.omt_conv_bwd_workspace(ctypes.byref(g)), x.device)
    check(L.omt_conv_bwd(ctypes.byref(g), _ptr(x), _ptr(gy), _ptr(w), _ptr(gx), _ptr(gw), _ptr(ws), nb,
                         _stream(x.device)), "conv2d_bwd")
    return gx, gw


def conv2d_bwd_bn(cx, gy, cw, stride, padding, x, save_mean, save_invstd, gamma, act=_lib.OMT_ACT_NONE, act_in=None,
                  g2=None, res=False, output_mask=(True, True, True), max_gx_slices=4, side_sum=True):
    """A convolution backward (input cx, filter cw) whose grad input is the incoming gradient of a BatchNorm backward
    (input x), as one pair of launches: omt_conv_bwd_parts leaves grad input's K-split partials (up to max_gx_slices
    slices) unsummed, and omt_bn_bwd_parts sums them as it reads them, adds g2 (res only), takes the activation's
    gradient and runs the grad weight's slice sum on extra workgroups (side_sum; else omt_slice_sums runs it first).
    res: the backward of omt_bn_bwd_res (act ReLU), which also returns gz. Returns (convolution grad weight, gx,
    dgamma, dbeta, gz or None, the number of grad-input slices the BatchNorm summed)."""
    cx, gy, cw = _need(cx, "cx", 4), _need(gy, "gy", 4), _need(cw, "cw", 4)
    x, act_in, g2 = _need(x, "x", 4), _need(act_in, "act_in", 4), _need(g2, "g2", 4)
    g = conv_geo_for(cx.shape, cw.shape, stride, padding)
    if tuple(gy.shape) != (g.n, g.co, g.oh, g.ow) or x.shape != cx.shape:
        raise ValueError(f"conv2d_bwd_bn: gy {tuple(gy.shape)} or x {tuple(x.shape)} does not fit the convolution")
    n, c, h, w = x.shape
    dev = x.device
    cgx, cgw = torch.empty_like(cx), torch.empty(tuple(cw.shape), device=dev, dtype=torch.float32)
    ws, nb = _workspace(L.omt_conv_bwd_workspace(ctypes.byref(g)), dev)
    parts, slices, job = _vp(), ctypes.c_int32(), _lib.SliceSum()
    s = _stream(dev)
    check(L.omt_conv_bwd_parts(ctypes.byref(g), _ptr(cx), _ptr(gy), _ptr(cw), _ptr(cgx), _ptr(cgw), _ptr(ws), nb,
                               int(max_gx_slices), ctypes.byref(parts), ctypes.byref(slices), ctypes.byref(job), s),
          "conv2d_bwd_bn (convolution)")
    count = 1 if job.slices > 0 else 0
    if count and not side_sum:
        check(L.omt_slice_sums(ctypes.byref(job), 1, s), "conv2d_bwd_bn (slice sum)")
        count = 0
    gx = torch.empty_like(x) if output_mask[0] else None
    dg = torch.empty((c,), device=dev, dtype=torch.float32) if output_mask[1] else None
    db = torch.empty((c,), device=dev, dtype=torch.float32) if output_mask[2] else None
    gz = torch.empty_like(x) if res else None
    src = parts if parts.value else _ptr(cgx)
    check(L.omt_bn_bwd_parts(n, c, h * w, src, slices.value, _ptr(g2), _ptr(x), int(act), _ptr(act_in),
                             _ptr(_need(save_mean, "mean", 1)), _ptr(_need(save_invstd, "invstd", 1)),
                             _ptr(_need(gamma, "gamma", 1)), _ptr(gx), _ptr(dg), _ptr(db), _ptr(gz),
                             ctypes.byref(job), count, s), "conv2d_bwd_bn (BatchNorm)")
    return cgw, gx, dg, db, gz, slices.value


# ---- channels-last (NHWC) dense convolution: tensors of the usual NCHW shapes in torch.channels_last memory order
# (filters [co][ky][kx][ci] in memory); outputs come back channels_last -----------------------------------------

_CL = torch.channels_last


def _need_cl(t, name):
    if t is None:
        return None
    if not t.is_cuda or t.dtype != torch.float32 or t.dim() != 4:
        raise TypeError(f"{name}: expected a 4-D float32 tensor on the HIP device")
    return t.contiguous(memory_format=_CL)


def conv2d_nhwc(x, w, bias=None, stride=1, padding=0, relu=False):
    x, w, bias = _need_cl(x, "x"), _need_cl(w, "w"), _need(bias, "bias", 1)
    g = conv_geo_for(x.shape, w.shape, stride, padding)
    y = torch.empty((g.n, g.co, g.oh, g.ow), device=x.device, dtype=torch.float32, memory_format=_CL)
    epi = (_lib.OMT_EPI_BIAS if bias is not None else 0) | (_lib.OMT_EPI_RELU if relu else 0)
    ws, nb = _workspace(L.omt_conv_fwd_nhwc_workspace(ctypes.byref(g)), x.device)
    check(L.omt_conv_fwd_nhwc(ctypes.byref(g), _ptr(x), _ptr(w), _ptr(bias), epi, _ptr(y), _ptr(ws), nb,
                              _stream(x.device)), "conv2d_nhwc")
    return y


def conv2d_dgrad_nhwc(gy, w, x_shape, stride=1, padding=0):
    gy, w = _need_cl(gy, "gy"), _need_cl(w, "w")
    g = conv_geo_for(x_shape, w.shape, stride, padding)
    if tuple(gy.shape) != (g.n, g.co, g.oh, g.ow):
        raise ValueError(f"conv dgrad: gy {tuple(gy.shape)} != {(g.n, g.co, g.oh, g.ow)}")
    gx = torch.empty(tuple(x_shape), device=gy.device, dtype=torch.float32, memory_format=_CL)
    ws, nb = _workspace(L.omt_conv_dgrad_nhwc_workspace(ctypes.byref(g)), gy.device)
    check(L.omt_conv_dgrad_nhwc(ctypes.byref(g), _ptr(gy), _ptr(w), _ptr(gx), _ptr(ws), nb, _stream(gy.device)),
          "conv2d_dgrad_nhwc")
    return gx


def conv2d_wgrad_nhwc(x, gy, ks, stride=1, padding=0):
    x, gy = _need_cl(x, "x"), _need_cl(gy, "gy")
    n, ci, ih, iw = x.shape
    co = gy.shape[1]
    g = _lib.conv_geo(n, ci, co, ih, iw, ks, stride, padding)
    if tuple(gy.shape) != (g.n, g.co, g.oh, g.ow):
        raise ValueError(f"conv wgrad: gy {tuple(gy.shape)} != {(g.n, g.co, g.oh, g.ow)}")
    gw = torch.empty((co, ci, ks, ks), device=x.device, dtype=torch.float32, memory_format=_CL)
    ws, nb = _workspace(L.omt_conv_wgrad_nhwc_workspace(ctypes.byref(g)), x.device)
    check(L.omt_conv_wgrad_nhwc(ctypes.byref(g), _ptr(x), _ptr(gy), _ptr(gw), _ptr(ws), nb, _stream(x.device)),
          "conv2d_wgrad_nhwc")
    return gw


# ---- plan cache (tile / split-K per geometry) and tuning (reference: conv_plan, autotune, tune_dump, tune_load,
# csrc/conv.cpp:45-60, 116-155, 243-272) ------------------------------------------------------------------------

DIRECTIONS = {"fwd": _lib.OMT_DIR_FWD, "dgrad": _lib.OMT_DIR_DGRAD, "wgrad": _lib.OMT_DIR_WGRAD,
              "fwd_nhwc": _lib.OMT_DIR_FWD_NHWC, "dgrad_nhwc": _lib.OMT_DIR_DGRAD_NHWC,
              "wgrad_nhwc": _lib.OMT_DIR_WGRAD_NHWC}


def conv_num_tiles(direction):
    return L.omt_conv_num_tiles(DIRECTIONS[direction])


def conv_plan(direction, x_shape, w_shape, stride=1, padding=0):
    """(tile, slices, cached): the plan the next call of this direction and geometry uses."""
    g = conv_geo_for(x_shape, w_shape, stride, padding)
    p, cached = _lib.ConvPlan(), ctypes.c_int32()
    check(L.omt_conv_get_plan(DIRECTIONS[direction], ctypes.byref(g), ctypes.byref(p), ctypes.byref(cached)),
          "conv_plan")
    return p.tile, p.slices, bool(cached.value)


def set_conv_plan(direction, x_shape, w_shape, stride=1, padding=0, tile=None, slices=1):
    """Pins (tile, slices) for this direction and geometry; tile None removes the entry."""
    g = conv_geo_for(x_shape, w_shape, stride, padding)
    p = None if tile is None else ctypes.byref(_lib.ConvPlan(tile, slices))
    check(L.omt_conv_set_plan(DIRECTIONS[direction], ctypes.byref(g), p), "set_conv_plan")


def autotune_conv(direction, x_shape, w_shape, stride=1, padding=0, max_tiles=0, device=None):
    """Times the candidate plans on scratch buffers and caches the fastest; returns (tile, slices)."""
    g = conv_geo_for(x_shape, w_shape, stride, padding)
    p = _lib.ConvPlan()
    check(L.omt_conv_autotune(DIRECTIONS[direction], ctypes.byref(g), max_tiles, _stream(device), ctypes.byref(p)),
          "autotune_conv")
    return p.tile, p.slices


def autotune_conv_bwd(x_shape, w_shape, stride=1, padding=0, max_tiles=0, device=None):
    """Tunes the grad-input and grad-weight plans together for conv2d_bwd and caches the fastest pair; returns
    ((tile, slices) of grad input, (tile, slices) of grad weight)."""
    g = conv_geo_for(x_shape, w_shape, stride, padding)
    d, w = _lib.ConvPlan(), _lib.ConvPlan()
    check(L.omt_conv_autotune_bwd(ctypes.byref(g), max_tiles, _stream(device), ctypes.byref(d), ctypes.byref(w)),
          "autotune_conv_bwd")
    return (d.tile, d.slices), (w.tile, w.slices)


def conv_plans():
    """The plan cache: {"dir,n,ci,co,ih,iw,oh,ow,ks,stride,pad": (tile, slices)} (the reference's tune_dump key)."""
    out = {}
    for i in range(L.omt_conv_plan_count()):
        d, g, p = ctypes.c_int32(), _lib.ConvGeo(), _lib.ConvPlan()
        if L.omt_conv_plan_entry(i, ctypes.byref(d), ctypes.byref(g), ctypes.byref(p)) == _lib.OMT_OK:
            out[",".join(str(v) for v in (d.value,) + g.astuple())] = (p.tile, p.slices)
    return out


def clear_conv_plans():
    L.omt_conv_clear_plans()


def bias_grad(gy):
    gy = _need(gy, "gy", 4)
    n, c, h, w = gy.shape
    gb = torch.empty((c,), device=gy.device, dtype=torch.float32)
    check(L.omt_bias_grad(n, c, h * w, _ptr(gy), _ptr(gb), _stream(gy.device)), "bias_grad")
    return gb


def fold_bn(cw, cb, gamma, beta, mean, var, eps=1e-5):
    """Eval BatchNorm folded into the preceding conv (fold_bn, csrc/fused.cpp:34-40)."""
    cw, cb = _need(cw, "cw"), _need(cb, "cb", 1)
    gamma, beta, mean, var = (_need(t, "bn", 1) for t in (gamma, beta, mean, var))
    co = cw.shape[0]
    fw, fb = torch.empty_like(cw), torch.empty((co,), device=cw.device, dtype=torch.float32)
    check(L.omt_fold_bn(co, cw.numel() // co, _ptr(cw), _ptr(cb), _ptr(gamma), _ptr(beta), _ptr(mean), _ptr(var),
                        eps, _ptr(fw), _ptr(fb), _stream(cw.device)), "fold_bn")
    return fw, fb


# ---- depthwise --------------------------------------------------------------------------------------------------

def _dw_geo(x_shape, w_shape, stride, pad):
    n, c, ih, iw = x_shape
    if tuple(w_shape[:2]) != (c, 1) or w_shape[2] != w_shape[3]:
        raise ValueError(f"depthwise: weight {tuple(w_shape)} for input {tuple(x_shape)}")
    return _lib.conv_geo(n, c, c, ih, iw, w_shape[2], stride, pad)


def depthwise_conv2d(x, w, bias=None, stride=1, padding=None, bn=None, bn_eps=1e-5):
    x, w, bias = _need(x, "x", 4), _need(w, "w", 4), _need(bias, "bias", 1)
    padding = w.shape[2] // 2 if padding is None else padding
    g = _dw_geo(x.shape, w.shape, stride, padding)
    y = torch.empty((g.n, g.co, g.oh, g.ow), device=x.device, dtype=torch.float32)
    bnp = [None] * 4 if bn is None else [_need(t, "bn", 1) for t in bn]
    check(L.omt_dw_fwd(ctypes.byref(g), _ptr(x), _ptr(w), _ptr(bias), *[_ptr(t) for t in bnp], bn_eps, _ptr(y),
                       _stream(x.device)), "depthwise_conv2d")
    return y


def depthwise_dgrad(gy, w, x_shape, stride=1, padding=None):
    gy, w = _need(gy, "gy", 4), _need(w, "w", 4)
    padding = w.shape[2] // 2 if padding is None else padding
    g = _dw_geo(x_shape, w.shape, stride, padding)
    gx = torch.empty(tuple(x_shape), device=gy.device, dtype=torch.float32)
    check(L.omt_dw_dgrad(ctypes.byref(g), _ptr(gy), _ptr(w), _ptr(gx), _stream(gy.device)), "depthwise_dgrad")
    return gx


def depthwise_wgrad(x, gy, ks, stride=1, padding=None):
    x, gy = _need(x, "x", 4), _need(gy, "gy", 4)
    padding = ks // 2 if padding is None else padding
    n, c, ih, iw = x.shape
    g = _lib.conv_geo(n, c, c, ih, iw, ks, stride, padding)
    gw = torch.empty((c, 1, ks, ks), device=x.device, dtype=torch.float32)
    ws, nb = _workspace(L.omt_dw_wgrad_workspace(ctypes.byref(g)), x.device)
    check(L.omt_dw_wgrad(ctypes.byref(g), _ptr(x), _ptr(gy), _ptr(gw), _ptr(ws), nb, _stream(x.device)),
          "depthwise_wgrad")
    return gw


# ---- batch norm -------------------------------------------------------------------------------------------------

def batch_norm_train(x, gamma, beta, running_mean=None, running_var=None, momentum=0.1, eps=1e-5, relu=False,
                     functional=False, act=None, residual=None, return_z=False):
    """Training BatchNorm, y = act(bn(x) + residual). Returns (y, save_mean, save_invstd) and, when functional, also
    the updated running stats as new tensors (bn_stats_fin_functional); otherwise running_mean / running_var are
    updated in place. act: _lib.OMT_ACT_* (default: ReLU if relu else none); return_z appends the activation's input
    bn(x) + residual."""
    x, residual = _need(x, "x", 4), _need(residual, "residual", 4)
    gamma, beta = _need(gamma, "gamma", 1), _need(beta, "beta", 1)
    act = (_lib.OMT_ACT_RELU if relu else _lib.OMT_ACT_NONE) if act is None else int(act)
    n, c, h, w = x.shape
    y = torch.empty_like(x)
    z = torch.empty_like(x) if return_z else None
    sm = torch.empty((c,), device=x.device, dtype=torch.float32)
    si = torch.empty_like(sm)
    if functional:
        nrm = torch.empty_like(sm) if running_mean is not None else None
        nrv = torch.empty_like(sm) if running_var is not None else None
    else:
        nrm, nrv = running_mean, running_var
    ws, nb = _workspace(L.omt_bn_train_workspace(n, c, h * w), x.device)
    check(L.omt_bn_train_fwd_res(n, c, h * w, _ptr(x), _ptr(gamma), _ptr(beta), _ptr(running_mean),
                                 _ptr(running_var), momentum, eps, act, _ptr(residual), _ptr(y), _ptr(z), _ptr(sm),
                                 _ptr(si), _ptr(nrm), _ptr(nrv), _ptr(ws), nb, _stream(x.device)), "batch_norm_train")
    out = (y, sm, si, nrm, nrv) if functional else (y, sm, si)
    return out + (z,) if return_z else out


def batch_norm_train_pool(x, gamma, beta, running_mean, running_var, momentum=0.1, eps=1e-5, act=_lib.OMT_ACT_RELU,
                          kernel=2, stride=None, padding=0):
    """Training BatchNorm -> activation -> max pool in one pass (omt_bn_train_fwd_pool): running statistics updated in
    place. Returns (y, save_mean, save_invstd, pooled, indices)."""
    x, gamma, beta = _need(x, "x", 4), _need(gamma, "gamma", 1), _need(beta, "beta", 1)
    (kh, kw), (sh, sw), (ph, pw) = _pair(kernel), _pair(stride if stride is not None else kernel), _pair(padding)
    n, c, h, w = x.shape
    oh, ow = (h + 2 * ph - kh) // sh + 1, (w + 2 * pw - kw) // sw + 1
    y = torch.empty_like(x)
    sm, si = (torch.empty((c,), device=x.device, dtype=torch.float32) for _ in range(2))
    out = torch.empty((n, c, oh, ow), device=x.device, dtype=torch.float32)
    idx = torch.empty((n, c, oh, ow), device=x.device, dtype=torch.int64)
    ws, nb = _workspace(L.omt_bn_train_workspace(n, c, h * w), x.device)
    check(L.omt_bn_train_fwd_pool(n, c, h, w, _ptr(x), _ptr(gamma), _ptr(beta), _ptr(running_mean), _ptr(running_var),
                                  momentum, eps, int(act), _ptr(y), _ptr(sm), _ptr(si), _ptr(running_mean),
                                  _ptr(running_var), kh, kw, sh, sw, ph, pw, _ptr(out), _ptr(idx), _ptr(ws), nb,
                                  _stream(x.device)), "batch_norm_train_pool")
    return y, sm, si, out, idx


def batch_norm_train_stats(x, stats, groups, gamma, beta, running_mean=None, running_var=None, momentum=0.1,
                           eps=1e-5, relu=False, residual=None):
    """Training BatchNorm (+ residual, ReLU) of a conv2d_stats output from its epilogue sums (omt_bn_train_fwd_stats:
    x is read once). Updates running_mean / running_var in place; returns (y, save_mean, save_invstd)."""
    x, residual = _need(x, "x", 4), _need(residual, "residual", 4)
    gamma, beta = _need(gamma, "gamma", 1), _need(beta, "beta", 1)
    if not stats.is_contiguous() or stats.dtype != torch.float64:
        raise TypeError("stats: contiguous float64 from conv2d_stats")
    n, c, h, w = x.shape
    y = torch.empty_like(x)
    sm = torch.empty((c,), device=x.device, dtype=torch.float32)
    si = torch.empty_like(sm)
    ws, nb = _workspace(L.omt_bn_train_workspace(n, c, h * w), x.device)
    check(L.omt_bn_train_fwd_stats(n, c, h * w, _ptr(x), _ptr(stats), int(groups), stats.numel() * 8, _ptr(gamma),
                                   _ptr(beta),
                                   _ptr(running_mean), _ptr(running_var), momentum, eps, int(relu), _ptr(residual),
                                   _ptr(y), None, _ptr(sm), _ptr(si), _ptr(running_mean), _ptr(running_var), _ptr(ws),
                                   nb, _stream(x.device)), "batch_norm_train_stats")
    return y, sm, si


def batch_norm_eval(x, gamma, beta, running_mean, running_var, eps=1e-5, relu=False):
    x = _need(x, "x", 4)
    n, c, h, w = x.shape
    y = torch.empty_like(x)
    check(L.omt_bn_eval_fwd(n, c, h * w, _ptr(x), _ptr(_need(gamma, "gamma", 1)), _ptr(_need(beta, "beta", 1)),
                            _ptr(_need(running_mean, "rm", 1)), _ptr(_need(running_var, "rv", 1)), eps, int(relu),
                            _ptr(y), _stream(x.device)), "batch_norm_eval")
    return y


def batch_norm_backward(g, x, save_mean, save_invstd, gamma, relu_y=None, output_mask=(True, True, True)):
    g, x = _need(g, "g", 4), _need(x, "x", 4)
    relu_y = _need(relu_y, "relu_y", 4)
    n, c, h, w = x.shape
    gx = torch.empty_like(x) if output_mask[0] else None
    dg = torch.empty((c,), device=x.device, dtype=torch.float32) if output_mask[1] else None
    db = torch.empty((c,), device=x.device, dtype=torch.float32) if output_mask[2] else None
    ws, nb = _workspace(L.omt_bn_bwd_workspace(n, c, h * w), x.device)
    check(L.omt_bn_bwd(n, c, h * w, _ptr(g), _ptr(x), _ptr(relu_y), _ptr(_need(save_mean, "mean", 1)),
                       _ptr(_need(save_invstd, "invstd", 1)), _ptr(_need(gamma, "gamma", 1)), _ptr(gx), _ptr(dg),
                       _ptr(db), _ptr(ws), nb, _stream(x.device)), "batch_norm_backward")
    return gx, dg, db


def batch_norm_backward_act(g, x, act, act_in, save_mean, save_invstd, gamma, output_mask=(True, True, True)):
    """BatchNorm backward through its activation (omt_bn_bwd_act): act _lib.OMT_ACT_RELU with act_in the ReLU's output,
    OMT_ACT_HARDSWISH with act_in the hardswish's input, OMT_ACT_NONE. Returns (gx, dgamma, dbeta)."""
    g, x, act_in = _need(g, "g", 4), _need(x, "x", 4), _need(act_in, "act_in", 4)
    n, c, h, w = x.shape
    gx = torch.empty_like(x) if output_mask[0] else None
    dg = torch.empty((c,), device=x.device, dtype=torch.float32) if output_mask[1] else None
    db = torch.empty((c,), device=x.device, dtype=torch.float32) if output_mask[2] else None
    ws, nb = _workspace(L.omt_bn_bwd_workspace(n, c, h * w), x.device)
    check(L.omt_bn_bwd_act(n, c, h * w, _ptr(g), _ptr(x), int(act), _ptr(act_in), _ptr(_need(save_mean, "mean", 1)),
                           _ptr(_need(save_invstd, "invstd", 1)), _ptr(_need(gamma, "gamma", 1)), _ptr(gx), _ptr(dg),
                           _ptr(db), _ptr(ws), nb, _stream(x.device)), "batch_norm_backward_act")
    return gx, dg, db


def batch_norm_backward_res(g, g2, x, save_mean, save_invstd, gamma, relu_y, output_mask=(True, True, True)):
    """The backward of a residual block's end: gz = (g + g2) masked by relu_y > 0 (g2 may be None), BatchNorm's
    (gx, dgamma, dbeta) of gz, and gz. Returns (gx, dgamma, dbeta, gz)."""
    g, g2, x, relu_y = _need(g, "g", 4), _need(g2, "g2", 4), _need(x, "x", 4), _need(relu_y, "relu_y", 4)
    n, c, h, w = x.shape
    gx = torch.empty_like(x) if output_mask[0] else None
    dg = torch.empty((c,), device=x.device, dtype=torch.float32) if output_mask[1] else None
    db = torch.empty((c,), device=x.device, dtype=torch.float32) if output_mask[2] else None
    gz = torch.empty_like(x)
    ws, nb = _workspace(L.omt_bn_bwd_workspace(n, c, h * w), x.device)
    check(L.omt_bn_bwd_res(n, c, h * w, _ptr(g), _ptr(g2), _ptr(x), _ptr(relu_y), _ptr(_need(save_mean, "mean", 1)),
                           _ptr(_need(save_invstd, "invstd", 1)), _ptr(_need(gamma, "gamma", 1)), _ptr(gx), _ptr(dg),
                           _ptr(db), _ptr(gz), _ptr(ws), nb, _stream(x.device)), "batch_norm_backward_res")
    return gx, dg, db, gz


# ---- pooling ----------------------------------------------------------------------------------------------------

def pool_out(size, k, s, p, d=1, ceil=False):
    """Output extent of a pooling window (PyTorch's pooling_output_shape)."""
    num = size + 2 * p - d * (k - 1) - 1 + ((s - 1) if ceil else 0)
    out = num // s + 1
    if ceil and (out - 1) * s >= size + p:
        out -= 1
    return out


def max_pool2d(x, kernel, stride=None, padding=0, dilation=1, ceil_mode=False):
    x = _need(x, "x", 4)
    k, s = _pair(kernel), _pair(stride if stride else kernel)
    p, d = _pair(padding), _pair(dilation)
    n, c, ih, iw = x.shape
    oh, ow = pool_out(ih, k[0], s[0], p[0], d[0], ceil_mode), pool_out(iw, k[1], s[1], p[1], d[1], ceil_mode)
    y = torch.empty((n, c, oh, ow), device=x.device, dtype=torch.float32)
    idx = torch.empty((n, c, oh, ow), device=x.device, dtype=torch.int64)
    check(L.omt_maxpool_fwd(n * c, ih, iw, oh, ow, k[0], k[1], s[0], s[1], p[0], p[1], d[0], d[1], _ptr(x), _ptr(y),
                            _ptr(idx), _stream(x.device)), "max_pool2d")
    return y, idx


def max_pool2d_backward(g, x_shape, idx, kernel, stride=None, padding=0, dilation=1):
    g = _need(g, "g", 4)
    idx = idx.contiguous()
    k, s = _pair(kernel), _pair(stride if stride else kernel)
    p, d = _pair(padding), _pair(dilation)
    n, c, ih, iw = x_shape
    gx = torch.empty(tuple(x_shape), device=g.device, dtype=torch.float32)
    check(L.omt_maxpool_bwd(n * c, ih, iw, g.shape[2], g.shape[3], k[0], k[1], s[0], s[1], p[0], p[1], d[0], d[1],
                            _ptr(g), _ptr(idx), _ptr(gx), _stream(g.device)), "max_pool2d_backward")
    return gx


def avg_pool2d(x, kernel, stride=None, padding=0, ceil_mode=False, count_include_pad=True, divisor_override=None):
    x = _need(x, "x", 4)
    k, s, p = _pair(kernel), _pair(stride if stride else kernel), _pair(padding)
    n, c, ih, iw = x.shape
    oh, ow = pool_out(ih, k[0], s[0], p[0], 1, ceil_mode), pool_out(iw, k[1], s[1], p[1], 1, ceil_mode)
    y = torch.empty((n, c, oh, ow), device=x.device, dtype=torch.float32)
    check(L.omt_avgpool_fwd(n * c, ih, iw, oh, ow, k[0], k[1], s[0], s[1], p[0], p[1], int(count_include_pad),
                            divisor_override or 0, _ptr(x), _ptr(y), _stream(x.device)), "avg_pool2d")
    return y


def avg_pool2d_backward(g, x_shape, kernel, stride=None, padding=0, count_include_pad=True, divisor_override=None):
    g = _need(g, "g", 4)
    k, s, p = _pair(kernel), _pair(stride if stride else kernel), _pair(padding)
    n, c, ih, iw = x_shape
    gx = torch.empty(tuple(x_shape), device=g.device, dtype=torch.float32)
    check(L.omt_avgpool_bwd(n * c, ih, iw, g.shape[2], g.shape[3], k[0], k[1], s[0], s[1], p[0], p[1],
                            int(count_include_pad), divisor_override or 0, _ptr(g), _ptr(gx), _stream(g.device)),
          "avg_pool2d_backward")
    return gx


def adaptive_avg_pool2d(x, output_size):
    x = _need(x, "x", 4)
    oh, ow = _pair(output_size)
    n, c, ih, iw = x.shape
    y = torch.empty((n, c, oh, ow), device=x.device, dtype=torch.float32)
    check(L.omt_adapool_fwd(n * c, ih, iw, oh, ow, _ptr(x), _ptr(y), _stream(x.device)), "adaptive_avg_pool2d")
    return y


def adaptive_avg_pool2d_backward(g, x_shape):
    g = _need(g, "g", 4)
    n, c, ih, iw = x_shape
    gx = torch.empty(tuple(x_shape), device=g.device, dtype=torch.float32)
    check(L.omt_adapool_bwd(n * c, ih, iw, g.shape[2], g.shape[3], _ptr(g), _ptr(gx), _stream(g.device)),
          "adaptive_avg_pool2d_backward")
    return gx


# ---- channels-last (NHWC) BatchNorm, pools and plane sums: tensors of the usual NCHW shapes in torch.channels_last
# memory order; outputs come back channels_last ----------------------------------------------------------------------

def batch_norm_train_nhwc(x, gamma, beta, running_mean=None, running_var=None, momentum=0.1, eps=1e-5,
                          act=_lib.OMT_ACT_NONE, residual=None, return_z=False):
    """Training BatchNorm over channels-last x (omt_bn_train_fwd_nhwc), y = act(bn(x) + residual); running statistics
    updated in place. Returns (y, save_mean, save_invstd) and, with return_z, the activation's input."""
    x, residual = _need_cl(x, "x"), _need_cl(residual, "residual")
    gamma, beta = _need(gamma, "gamma", 1), _need(beta, "beta", 1)
    n, c, h, w = x.shape
    y = torch.empty_like(x, memory_format=_CL)
    z = torch.empty_like(x, memory_format=_CL) if return_z else None
    sm = torch.empty((c,), device=x.device, dtype=torch.float32)
    si = torch.empty_like(sm)
    ws, nb = _workspace(L.omt_bn_nhwc_workspace(n, c, h * w), x.device)
    check(L.omt_bn_train_fwd_nhwc(n, c, h * w, _ptr(x), _ptr(gamma), _ptr(beta), _ptr(running_mean),
                                  _ptr(running_var), momentum, eps, int(act), _ptr(residual), _ptr(y), _ptr(z),
                                  _ptr(sm), _ptr(si), _ptr(running_mean), _ptr(running_var), _ptr(ws), nb,
                                  _stream(x.device)), "batch_norm_train_nhwc")
    return (y, sm, si, z) if return_z else (y, sm, si)


def batch_norm_eval_nhwc(x, gamma, beta, running_mean, running_var, eps=1e-5, act=_lib.OMT_ACT_NONE):
    x = _need_cl(x, "x")
    n, c, h, w = x.shape
    y = torch.empty_like(x, memory_format=_CL)
    check(L.omt_bn_eval_fwd_nhwc(n, c, h * w, _ptr(x), _ptr(_need(gamma, "gamma", 1)), _ptr(_need(beta, "beta", 1)),
                                 _ptr(_need(running_mean, "rm", 1)), _ptr(_need(running_var, "rv", 1)), eps, int(act),
                                 _ptr(y), _stream(x.device)), "batch_norm_eval_nhwc")
    return y


def batch_norm_backward_nhwc(g, x, save_mean, save_invstd, gamma, act=_lib.OMT_ACT_NONE, act_in=None, g2=None,
                             want_gz=False, output_mask=(True, True, True), g_nchw=False):
    """BatchNorm backward over channels-last tensors (omt_bn_bwd_nhwc): gz = (g + g2) through the activation's
    gradient, then (gx, dgamma, dbeta) of gz, and gz itself when want_gz. g_nchw: g is read in NCHW order (made
    contiguous), the rest channels-last. Returns (gx, dgamma, dbeta, gz)."""
    g = _need(g, "g", 4) if g_nchw else _need_cl(g, "g")
    x, act_in, g2 = _need_cl(x, "x"), _need_cl(act_in, "act_in"), _need_cl(g2, "g2")
    n, c, h, w = x.shape
    gx = torch.empty_like(x, memory_format=_CL) if output_mask[0] else None
    dg = torch.empty((c,), device=x.device, dtype=torch.float32) if output_mask[1] else None
    db = torch.empty((c,), device=x.device, dtype=torch.float32) if output_mask[2] else None
    gz = torch.empty_like(x, memory_format=_CL) if want_gz else None
    ws, nb = _workspace(L.omt_bn_nhwc_workspace(n, c, h * w), x.device)
    check(L.omt_bn_bwd_nhwc(n, c, h * w, _ptr(g), int(g_nchw), _ptr(g2), _ptr(x), int(act), _ptr(act_in),
                            _ptr(_need(save_mean, "mean", 1)), _ptr(_need(save_invstd, "invstd", 1)),
                            _ptr(_need(gamma, "gamma", 1)), _ptr(gx), _ptr(dg), _ptr(db), _ptr(gz), _ptr(ws), nb,
                            _stream(x.device)), "batch_norm_backward_nhwc")
    return gx, dg, db, gz


def max_pool2d_nhwc(x, kernel, stride=None, padding=0, dilation=1, ceil_mode=False):
    x = _need_cl(x, "x")
    k, s = _pair(kernel), _pair(stride if stride else kernel)
    p, d = _pair(padding), _pair(dilation)
    n, c, ih, iw = x.shape
    oh, ow = pool_out(ih, k[0], s[0], p[0], d[0], ceil_mode), pool_out(iw, k[1], s[1], p[1], d[1], ceil_mode)
    y = torch.empty((n, c, oh, ow), device=x.device, dtype=torch.float32, memory_format=_CL)
    idx = torch.empty((n, c, oh, ow), device=x.device, dtype=torch.int64, memory_format=_CL)
    check(L.omt_maxpool_fwd_nhwc(n, c, ih, iw, oh, ow, k[0], k[1], s[0], s[1], p[0], p[1], d[0], d[1], _ptr(x),
                                 _ptr(y), _ptr(idx), _stream(x.device)), "max_pool2d_nhwc")
    return y, idx


def max_pool2d_backward_nhwc(g, x_shape, idx, kernel, stride=None, padding=0, dilation=1):
    g = _need_cl(g, "g")
    idx = idx.contiguous(memory_format=_CL)
    k, s = _pair(kernel), _pair(stride if stride else kernel)
    p, d = _pair(padding), _pair(dilation)
    n, c, ih, iw = x_shape
    gx = torch.empty(tuple(x_shape), device=g.device, dtype=torch.float32, memory_format=_CL)
    check(L.omt_maxpool_bwd_nhwc(n, c, ih, iw, g.shape[2], g.shape[3], k[0], k[1], s[0], s[1], p[0], p[1], d[0], d[1],
                                 _ptr(g), _ptr(idx), _ptr(gx), _stream(g.device)), "max_pool2d_backward_nhwc")
    return gx


def avg_pool2d_nhwc(x, kernel, stride=None, padding=0, ceil_mode=False, count_include_pad=True,
                    divisor_override=None):
    x = _need_cl(x, "x")
    k, s, p = _pair(kernel), _pair(stride if stride else kernel), _pair(padding)
    n, c, ih, iw = x.shape
    oh, ow = pool_out(ih, k[0], s[0], p[0], 1, ceil_mode), pool_out(iw, k[1], s[1], p[1], 1, ceil_mode)
    y = torch.empty((n, c, oh, ow), device=x.device, dtype=torch.float32, memory_format=_CL)
    check(L.omt_avgpool_fwd_nhwc(n, c, ih, iw, oh, ow, k[0], k[1], s[0], s[1], p[0], p[1], int(count_include_pad),
                                 divisor_override or 0, _ptr(x), _ptr(y), _stream(x.device)), "avg_pool2d_nhwc")
    return y


def avg_pool2d_backward_nhwc(g, x_shape, kernel, stride=None, padding=0, count_include_pad=True,
                             divisor_override=None):
    g = _need_cl(g, "g")
    k, s, p = _pair(kernel), _pair(stride if stride else kernel), _pair(padding)
    n, c, ih, iw = x_shape
    gx = torch.empty(tuple(x_shape), device=g.device, dtype=torch.float32, memory_format=_CL)
    check(L.omt_avgpool_bwd_nhwc(n, c, ih, iw, g.shape[2], g.shape[3], k[0], k[1], s[0], s[1], p[0], p[1],
                                 int(count_include_pad), divisor_override or 0, _ptr(g), _ptr(gx), _stream(g.device)),
          "avg_pool2d_backward_nhwc")
    return gx


def adaptive_avg_pool2d_nhwc(x, output_size):
    x = _need_cl(x, "x")
    oh, ow = _pair(output_size)
    n, c, ih, iw = x.shape
    y = torch.empty((n, c, oh, ow), device=x.device, dtype=torch.float32, memory_format=_CL)
    check(L.omt_adapool_fwd_nhwc(n, c, ih, iw, oh, ow, _ptr(x), _ptr(y), _stream(x.device)),
          "adaptive_avg_pool2d_nhwc")
    return y


def adaptive_avg_pool2d_backward_nhwc(g, x_shape):
    g = _need_cl(g, "g")
    n, c, ih, iw = x_shape
    gx = torch.empty(tuple(x_shape), device=g.device, dtype=torch.float32, memory_format=_CL)
    check(L.omt_adapool_bwd_nhwc(n, c, ih, iw, g.shape[2], g.shape[3], _ptr(g), _ptr(gx), _stream(g.device)),
          "adaptive_avg_pool2d_backward_nhwc")
    return gx


def depthwise_conv2d_nhwc(x, w, bias=None, stride=1, padding=None):
    """Depthwise convolution over channels-last x (omt_dw_fwd_nhwc); y channels_last."""
    x, w, bias = _need_cl(x, "x"), _need(w, "w", 4), _need(bias, "bias", 1)
    padding = w.shape[2] // 2 if padding is None else padding
    g = _dw_geo(x.shape, w.shape, stride, padding)
    y = torch.empty((g.n, g.co, g.oh, g.ow), device=x.device, dtype=torch.float32, memory_format=_CL)
    check(L.omt_dw_fwd_nhwc(ctypes.byref(g), _ptr(x), _ptr(w), _ptr(bias), _ptr(y), _stream(x.device)),
          "depthwise_conv2d_nhwc")
    return y


def depthwise_dgrad_nhwc(gy, w, x_shape, stride=1, padding=None):
    gy, w = _need_cl(gy, "gy"), _need(w, "w", 4)
    padding = w.shape[2] // 2 if padding is None else padding
    g = _dw_geo(x_shape, w.shape, stride, padding)
    gx = torch.empty(tuple(x_shape), device=gy.device, dtype=torch.float32, memory_format=_CL)
    check(L.omt_dw_dgrad_nhwc(ctypes.byref(g), _ptr(gy), _ptr(w), _ptr(gx), _stream(gy.device)),
          "depthwise_dgrad_nhwc")
    return gx


def depthwise_wgrad_nhwc(x, gy, ks, stride=1, padding=None):
    x, gy = _need_cl(x, "x"), _need_cl(gy, "gy")
    padding = ks // 2 if padding is None else padding
    n, c, ih, iw = x.shape
    g = _lib.conv_geo(n, c, c, ih, iw, ks, stride, padding)
    gw = torch.empty((c, 1, ks, ks), device=x.device, dtype=torch.float32)
    ws, nb = _workspace(L.omt_dw_wgrad_nhwc_workspace(ctypes.byref(g)), x.device)
    check(L.omt_dw_wgrad_nhwc(ctypes.byref(g), _ptr(x), _ptr(gy), _ptr(gw), _ptr(ws), nb, _stream(x.device)),
          "depthwise_wgrad_nhwc")
    return gw


def channel_scale_nhwc(x, s):
    """x * s for channels-last x [n, c, h, w] and s [n, c, 1, 1] (omt_channel_scale_nhwc); channels_last output."""
    x, s = _need_cl(x, "x"), _need(s, "s", 4)
    n, c, h, w = x.shape
    y = torch.empty_like(x, memory_format=_CL)
    check(L.omt_channel_scale_nhwc(n, c, h * w, _ptr(x), _ptr(s), _ptr(y), _stream(x.device)), "channel_scale_nhwc")
    return y


def plane_sum_nhwc(x, scale=1.0):
    """scale * the sum of each channels-last plane of x: [n, c] (omt_plane_sum_nhwc)."""
    x = _need_cl(x, "x")
    n, c, h, w = x.shape
    y = torch.empty((n, c), device=x.device, dtype=torch.float32)
    check(L.omt_plane_sum_nhwc(n, c, h * w, _ptr(x), float(scale), _ptr(y), _stream(x.device)), "plane_sum_nhwc")
    return y


def pointwise_layouts(op, a, b=None, alpha=0.0, out_nhwc=True):
    """omt_pointwise_layouts: op over two 4-D tensors of one shape, each NCHW-contiguous or channels_last (read in
    place); the output in channels_last (out_nhwc) or NCHW order."""
    def order(t):
        if t is None:
            return None, 0
        if not t.is_cuda or t.dtype != torch.float32 or t.dim() != 4:
            raise TypeError("pointwise_layouts: 4-D float32 tensors on the HIP device expected")
        if t.is_contiguous():
            return t, 0
        if t.is_contiguous(memory_format=_CL):
            return t, 1
        return t.contiguous(), 0
    a, an = order(a)
    b, bn = order(b)
    n, c, h, w = a.shape
    out = torch.empty(a.shape, device=a.device, dtype=torch.float32,
                      memory_format=_CL if out_nhwc else torch.contiguous_format)
    check(L.omt_pointwise_layouts(int(op), n, c, h * w, _ptr(a), an, _ptr(b), bn, float(alpha), _ptr(out),
                                  int(out_nhwc), _stream(a.device)), "pointwise_layouts")
    return out


# ---- pointwise (reference csrc/elementwise.cpp:702-817) ---------------------------------------------------------

def fill_(t, value):
    """t[:] = value (a contiguous float32 device tensor), through omt_pointwise's fill."""
    if not t.is_cuda or t.dtype != torch.float32 or not t.is_contiguous():
        raise TypeError("fill_: a contiguous float32 tensor on the HIP device expected")
    check(L.omt_pointwise(_lib.OMT_PW_FILL, t.numel(), None, None, float(value), _ptr(t), _stream(t.device)), "fill_")
    return t


# ---- fused optimizers (reference csrc/optim.cpp:12-67) -----------------------------------------------------------

def _scalar_ptr(t, name):
    if t is None:
        return None
    if not t.is_cuda or t.dtype != torch.float32 or t.numel() != 1:
        raise TypeError(f"{name}: expected a one-element float32 tensor on the HIP device")
    return t.data_ptr()


def fused_adam(params, grads, exp_avgs, exp_avg_sqs, steps, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.0,
               amsgrad=False, maximize=False, decoupled=False, max_exp_avg_sqs=None, grad_scale=None, found_inf=None):
    """One Adam (decoupled: AdamW) step over lists of contiguous float32 tensors, in place; steps are one-element
    float32 device tensors already incremented for this step. lr may be a one-element device tensor."""
    n = len(params)
    lists = [grads, exp_avgs, exp_avg_sqs, steps] + ([max_exp_avg_sqs] if amsgrad else [])
    if any(len(x) != n for x in lists):
        raise ValueError("fused_adam: tensor lists of different lengths")
    arr = (_lib.AdamTensor * max(n, 1))()
    for i in range(n):
        ts = [params[i], grads[i], exp_avgs[i], exp_avg_sqs[i]] + ([max_exp_avg_sqs[i]] if amsgrad else [])
        for t in ts:
            if not t.is_cuda or t.dtype != torch.float32 or not t.is_contiguous() or t.numel() != params[i].numel():
                raise TypeError("fused_adam: contiguous float32 HIP tensors of matching sizes expected")
        arr[i] = _lib.AdamTensor(params[i].data_ptr(), grads[i].data_ptr(), exp_avgs[i].data_ptr(),
                                 exp_avg_sqs[i].data_ptr(), max_exp_avg_sqs[i].data_ptr() if amsgrad else None,
                                 _scalar_ptr(steps[i], "step"), params[i].numel())
    lr_dev = _scalar_ptr(lr, "lr") if isinstance(lr, torch.Tensor) else None
    hp = _lib.AdamParams(0.0 if lr_dev else float(lr), lr_dev, betas[0], betas[1], weight_decay, eps, int(amsgrad),
                         int(maximize), int(decoupled), _scalar_ptr(grad_scale, "grad_scale"),
                         _scalar_ptr(found_inf, "found_inf"))
    check(L.omt_fused_adam(ctypes.byref(hp), arr, n, _stream()), "fused_adam")


def fused_sgd(params, grads, momentum_buffers=None, lr=1e-3, momentum=0.0, dampening=0.0, weight_decay=0.0,
              nesterov=False, maximize=False, first_step=False, grad_scale=None, found_inf=None):
    """One SGD step over lists of contiguous float32 tensors, in place (momentum_buffers when momentum != 0)."""
    n = len(params)
    if len(grads) != n or (momentum and len(momentum_buffers or []) != n):
        raise ValueError("fused_sgd: tensor lists of different lengths")
    arr = (_lib.SgdTensor * max(n, 1))()
    for i in range(n):
        ts = [params[i], grads[i]] + ([momentum_buffers[i]] if momentum else [])
        for t in ts:
            if not t.is_cuda or t.dtype != torch.float32 or not t.is_contiguous() or t.numel() != params[i].numel():
                raise TypeError("fused_sgd: contiguous float32 HIP tensors of matching sizes expected")
        arr[i] = _lib.SgdTensor(params[i].data_ptr(), grads[i].data_ptr(),
                                momentum_buffers[i].data_ptr() if momentum else None, params[i].numel())
    lr_dev = _scalar_ptr(lr, "lr") if isinstance(lr, torch.Tensor) else None
    hp = _lib.SgdParams(0.0 if lr_dev else float(lr), lr_dev, momentum, dampening, weight_decay, int(nesterov),
                        int(maximize), int(first_step), _scalar_ptr(grad_scale, "grad_scale"),
                        _scalar_ptr(found_inf, "found_inf"))
    check(L.omt_fused_sgd(ctypes.byref(hp), arr, n, _stream()), "fused_sgd")

"""numpy front end of the CPU oracle (omt_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, never by the
omarchy_mac_torch package. Each wrapper names the reference function it restates; the C file carries the citations.
"""

import ctypes
import os
import pathlib
import subprocess

import numpy as np

_HERE = pathlib.Path(__file__).resolve().parent
_LIB = None

f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
i64p = np.ctypeslib.ndpointer(dtype=np.int64, flags="C_CONTIGUOUS")
f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
I64 = ctypes.c_int64


class Geo(ctypes.Structure):
    """csrc/omt.h:224-226 (Geo)."""
    _fields_ = [(k, ctypes.c_int64) for k in ("n", "ci", "co", "ih", "iw", "oh", "ow", "ks", "stride", "pad")]

    def tuple(self):
        return tuple(getattr(self, k) for k, _ in self._fields_)


def build():
    subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)


def lib():
    global _LIB
    if _LIB is None:
        path = _HERE / "liboracle.so"
        if not path.exists():
            build()
        L = ctypes.CDLL(str(path))
        G = ctypes.POINTER(Geo)
        opt = ctypes.c_void_p  # nullable float arrays are passed as raw pointers
        L.orc_conv_geo.argtypes = [I64] * 8 + [G]
        L.orc_conv_kind.argtypes = [I64] * 10 + [ctypes.c_int, I64]
        L.orc_conv_kind.restype = ctypes.c_int
        L.orc_mnk.argtypes = [ctypes.c_int, G, ctypes.POINTER(I64), ctypes.POINTER(I64), ctypes.POINTER(I64)]
        L.orc_default_tile.argtypes = [ctypes.c_int, G, ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int)]
        L.orc_wgrad_split.argtypes = [G, ctypes.c_int, ctypes.c_int, ctypes.c_double, ctypes.POINTER(I64), ctypes.POINTER(I64)]
        L.orc_conv_fwd.argtypes = [G, f32p, f32p, opt, ctypes.c_uint, opt, opt, opt, opt, ctypes.c_double, f32p]
        L.orc_conv_fwd_points.argtypes = [G, f32p, f32p, opt, ctypes.c_uint, I64, i64p, f64p]
        L.orc_conv_dgrad.argtypes = [G, f32p, f32p, f32p]
        L.orc_conv_dgrad_points.argtypes = [G, f32p, f32p, I64, i64p, f64p]
        L.orc_conv_wgrad.argtypes = [G, f32p, f32p, I64, I64, f32p]
        L.orc_conv_wgrad_points.argtypes = [G, f32p, f32p, I64, i64p, f64p]
        L.orc_bias_grad.argtypes = [I64, I64, I64, f32p, f32p]
        L.orc_dw_fwd.argtypes = [G, f32p, f32p, opt, opt, opt, opt, opt, ctypes.c_double, f32p]
        L.orc_dw_dgrad.argtypes = [G, f32p, f32p, f32p]
        L.orc_dw_wgrad.argtypes = [G, f32p, f32p, f32p]
        L.orc_bn_stats.argtypes = [I64, I64, I64, f32p, ctypes.c_double, opt, opt, f32p, f32p, opt, opt]
        L.orc_bn_apply.argtypes = [I64, I64, I64, f32p, f32p, f32p, ctypes.c_double, f32p, f32p, ctypes.c_int, f32p]
        L.orc_bn_bwd.argtypes = [I64, I64, I64, f32p, f32p, opt, f32p, f32p, f32p, opt, opt, opt]
        L.orc_fold_bn.argtypes = [I64, I64, f32p, opt, f32p, f32p, f32p, f32p, ctypes.c_double, f32p, f32p]
        L.orc_maxpool_fwd.argtypes = [I64] * 13 + [f32p, f32p, i64p]
        L.orc_maxpool_bwd.argtypes = [I64] * 5 + [f32p, i64p, f32p]
        L.orc_avgpool_fwd.argtypes = [I64] * 11 + [ctypes.c_int, I64, f32p, f32p]
        L.orc_avgpool_bwd.argtypes = [I64] * 11 + [ctypes.c_int, I64, f32p, f32p]
        L.orc_adapool_fwd.argtypes = [I64] * 5 + [f32p, f32p]
        L.orc_adapool_bwd.argtypes = [I64] * 5 + [f32p, f32p]
        _LIB = L
    return _LIB


def _c(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _p(a):
    """Nullable float32 array -> raw pointer (keeps no reference: callers hold the array)."""
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def geo(n, ci, co, ih, iw, ks, stride, pad):
    """conv_geo (csrc/conv.cpp:19-21)."""
    g = Geo()
    lib().orc_conv_geo(n, ci, co, ih, iw, ks, stride, pad, ctypes.byref(g))
    return g


def conv_kind(x_c, w_o, kh, kw, stride, padding, dilation, transposed, groups):
    """conv_kind (csrc/conv.cpp:167-177): 0 = not covered, 1 dense, 2 dw, 3 dwg."""
    return lib().orc_conv_kind(x_c, w_o, kh, kw, stride[0], stride[1], padding[0], padding[1], dilation[0],
                               dilation[1], int(transposed), groups)


def mnk(kind, g):
    M, N, K = I64(), I64(), I64()
    lib().orc_mnk(kind, ctypes.byref(g), ctypes.byref(M), ctypes.byref(N), ctypes.byref(K))
    return M.value, N.value, K.value


def default_tile(kind, g):
    bm, bn = ctypes.c_int(), ctypes.c_int()
    lib().orc_default_tile(kind, ctypes.byref(g), ctypes.byref(bm), ctypes.byref(bn))
    return bm.value, bn.value


def wgrad_split(g, bm, bn, mult=1.0):
    s, k = I64(), I64()
    lib().orc_wgrad_split(ctypes.byref(g), bm, bn, mult, ctypes.byref(s), ctypes.byref(k))
    return s.value, k.value


def conv_fwd(x, w, bias=None, stride=1, pad=0, relu=False, bn=None, eps=1e-5):
    """gemm_forward (csrc/conv.cpp:70-77) + _FWD (gemm.py:25-42); bn = (mean, var, gamma, beta) selects the kind-3
    BN+ReLU loader (gemm.py:139-141)."""
    x, w = _c(x), _c(w)
    n, ci, ih, iw = x.shape
    co, _, ks, _ = w.shape
    g = geo(n, ci, co, ih, iw, ks, stride, pad)
    out = np.empty((n, co, g.oh, g.ow), np.float32)
    b = None if bias is None else _c(bias)
    bnp = [None] * 4 if bn is None else [_c(t) for t in bn]
    epi = (1 if b is not None else 0) | (2 if relu else 0)
    lib().orc_conv_fwd(ctypes.byref(g), x, w, _p(b), epi, *[_p(t) for t in bnp], eps, out)
    return out


def conv_fwd_points(x, w, flat, bias=None, stride=1, pad=0, relu=False):
    x, w = _c(x), _c(w)
    n, ci, ih, iw = x.shape
    co, _, ks, _ = w.shape
    g = geo(n, ci, co, ih, iw, ks, stride, pad)
    flat = np.ascontiguousarray(flat, np.int64)
    out = np.empty(len(flat), np.float64)
    b = None if bias is None else _c(bias)
    epi = (1 if b is not None else 0) | (2 if relu else 0)
    lib().orc_conv_fwd_points(ctypes.byref(g), x, w, _p(b), epi, len(flat), flat, out)
    return out


def conv_dgrad(gy, w, x_shape, stride=1, pad=0):
    """gemm_grad_input (csrc/conv.cpp:78-101): kind 1 at stride 1, stride phases (kind 5) otherwise."""
    gy, w = _c(gy), _c(w)
    n, ci, ih, iw = x_shape
    co, _, ks, _ = w.shape
    g = geo(n, ci, co, ih, iw, ks, stride, pad)
    assert gy.shape == (n, co, g.oh, g.ow), (gy.shape, g.tuple())
    gx = np.empty((n, ci, ih, iw), np.float32)
    lib().orc_conv_dgrad(ctypes.byref(g), gy, w, gx)
    return gx


def conv_dgrad_points(gy, w, x_shape, flat, stride=1, pad=0):
    """Selected gx elements by the stride-skipping kind-1 map (gemm.py:43-59)."""
    gy, w = _c(gy), _c(w)
    n, ci, ih, iw = x_shape
    co, _, ks, _ = w.shape
    g = geo(n, ci, co, ih, iw, ks, stride, pad)
    flat = np.ascontiguousarray(flat, np.int64)
    out = np.empty(len(flat), np.float64)
    lib().orc_conv_dgrad_points(ctypes.byref(g), gy, w, len(flat), flat, out)
    return out


def conv_wgrad(x, gy, ks, stride=1, pad=0, slices=0, kslice=0):
    """gemm_grad_weight (csrc/conv.cpp:102-114): split-K partials + gemm_reduce."""
    x, gy = _c(x), _c(gy)
    n, ci, ih, iw = x.shape
    co = gy.shape[1]
    g = geo(n, ci, co, ih, iw, ks, stride, pad)
    assert gy.shape == (n, co, g.oh, g.ow)
    gw = np.empty((co, ci, ks, ks), np.float32)
    lib().orc_conv_wgrad(ctypes.byref(g), x, gy, slices, kslice, gw)
    return gw


def conv_wgrad_points(x, gy, ks, flat, stride=1, pad=0):
    x, gy = _c(x), _c(gy)
    n, ci, ih, iw = x.shape
    co = gy.shape[1]
    g = geo(n, ci, co, ih, iw, ks, stride, pad)
    flat = np.ascontiguousarray(flat, np.int64)
    out = np.empty(len(flat), np.float64)
    lib().orc_conv_wgrad_points(ctypes.byref(g), x, gy, len(flat), flat, out)
    return out


def bias_grad(gy):
    """csum_nchw (csrc/kernels/csum_nchw.wgsl)."""
    gy = _c(gy)
    n, c, h, w = gy.shape
    gb = np.empty(c, np.float32)
    lib().orc_bias_grad(n, c, h * w, gy, gb)
    return gb


def dw_fwd(x, w, bias=None, stride=1, pad=None, bn=None, eps=1e-5):
    """dw_fwd / dwg_fwd / dw_fwd_bn (csrc/kernels/dw_fwd.wgsl, dwg_fwd.wgsl, dw_fwd_bn.wgsl)."""
    x, w = _c(x), _c(w)
    n, c, ih, iw = x.shape
    ks = w.shape[2]
    pad = ks // 2 if pad is None else pad
    g = geo(n, c, c, ih, iw, ks, stride, pad)
    out = np.empty((n, c, g.oh, g.ow), np.float32)
    b = None if bias is None else _c(bias)
    bnp = [None] * 4 if bn is None else [_c(t) for t in bn]
    lib().orc_dw_fwd(ctypes.byref(g), x, w, _p(b), *[_p(t) for t in bnp], eps, out)
    return out


def dw_dgrad(gy, w, x_shape, stride=1, pad=None):
    gy, w = _c(gy), _c(w)
    n, c, ih, iw = x_shape
    ks = w.shape[2]
    pad = ks // 2 if pad is None else pad
    g = geo(n, c, c, ih, iw, ks, stride, pad)
    gx = np.empty(x_shape, np.float32)
    lib().orc_dw_dgrad(ctypes.byref(g), gy, w, gx)
    return gx


def dw_wgrad(x, gy, ks, stride=1, pad=None):
    x, gy = _c(x), _c(gy)
    n, c, ih, iw = x.shape
    pad = ks // 2 if pad is None else pad
    g = geo(n, c, c, ih, iw, ks, stride, pad)
    gw = np.empty((c, 1, ks, ks), np.float32)
    lib().orc_dw_wgrad(ctypes.byref(g), x, gy, gw)
    return gw


def bn_train(x, gamma, beta, rm, rv, momentum=0.1, eps=1e-5, relu=False):
    """native_batch_norm, training (csrc/nn.cpp:38-48) / bn_relu_train (csrc/fused.cpp:68-84).
    Returns (y, mean, invstd, new_rm, new_rv)."""
    x = _c(x)
    n, c, h, w = x.shape
    mean, var = np.empty(c, np.float32), np.empty(c, np.float32)
    nrm, nrv = np.empty(c, np.float32), np.empty(c, np.float32)
    rm, rv = _c(rm), _c(rv)
    lib().orc_bn_stats(n, c, h * w, x, momentum, _p(rm), _p(rv), mean, var, _p(nrm), _p(nrv))
    y = np.empty_like(x)
    lib().orc_bn_apply(n, c, h * w, x, mean, var, eps, _c(gamma), _c(beta), int(relu), y)
    invstd = (1.0 / np.sqrt(var.astype(np.float64) + eps)).astype(np.float32)
    return y, mean, invstd, nrm, nrv


def bn_eval(x, gamma, beta, rm, rv, eps=1e-5, relu=False):
    """native_batch_norm, eval (csrc/nn.cpp:49-54) / bn_relu_rv.wgsl."""
    x = _c(x)
    n, c, h, w = x.shape
    y = np.empty_like(x)
    lib().orc_bn_apply(n, c, h * w, x, _c(rm), _c(rv), eps, _c(gamma), _c(beta), int(relu), y)
    return y


def bn_bwd(g, x, mean, invstd, gamma, relu_y=None, need_gx=True):
    """batch_norm_backward_ (csrc/nn.cpp:60-78) / bn_relu_backward (csrc/fused.cpp:86-115).
    Returns (gx, dgamma, dbeta)."""
    g, x = _c(g), _c(x)
    n, c, h, w = x.shape
    gx = np.empty_like(x) if need_gx else None
    dg, db = np.empty(c, np.float32), np.empty(c, np.float32)
    ry = None if relu_y is None else _c(relu_y)
    lib().orc_bn_bwd(n, c, h * w, g, x, _p(ry), _c(mean), _c(invstd), _c(gamma), _p(gx), _p(dg), _p(db))
    return gx, dg, db


def fold_bn(cw, cb, w, b, rm, rv, eps=1e-5):
    """fold_bn (csrc/fused.cpp:34-40)."""
    cw = _c(cw)
    co = cw.shape[0]
    fw, fb = np.empty_like(cw), np.empty(co, np.float32)
    cbp = None if cb is None else _c(cb)
    lib().orc_fold_bn(co, cw.size // co, cw, _p(cbp), _c(w), _c(b), _c(rm), _c(rv), eps, fw, fb)
    return fw, fb


def pool_out(size, k, s, p, d=1, ceil=False):
    """at::native::pooling_output_shape (used at csrc/nn.cpp:163-164, 185-186)."""
    num = size + 2 * p - d * (k - 1) - 1 + ((s - 1) if ceil else 0)
    out = num // s + 1
    if ceil and (out - 1) * s >= size + p:
        out -= 1
    return out


def maxpool_fwd(x, k, s, p, d=(1, 1), ceil=False):
    """maxpool_gen_fwd.wgsl. Returns (out, int64 idx)."""
    x = _c(x)
    n, c, ih, iw = x.shape
    oh, ow = pool_out(ih, k[0], s[0], p[0], d[0], ceil), pool_out(iw, k[1], s[1], p[1], d[1], ceil)
    out, idx = np.empty((n, c, oh, ow), np.float32), np.empty((n, c, oh, ow), np.int64)
    lib().orc_maxpool_fwd(n * c, ih, iw, oh, ow, k[0], k[1], s[0], s[1], p[0], p[1], d[0], d[1], x, out, idx)
    return out, idx


def maxpool_bwd(g, idx, x_shape):
    g, idx = _c(g), np.ascontiguousarray(idx, np.int64)
    n, c, ih, iw = x_shape
    gx = np.empty(x_shape, np.float32)
    lib().orc_maxpool_bwd(n * c, ih, iw, g.shape[2], g.shape[3], g, idx, gx)
    return gx


def avgpool_fwd(x, k, s, p, ceil=False, include_pad=True, divisor=None):
    """avgpool_gen_fwd.wgsl."""
    x = _c(x)
    n, c, ih, iw = x.shape
    oh, ow = pool_out(ih, k[0], s[0], p[0], 1, ceil), pool_out(iw, k[1], s[1], p[1], 1, ceil)
    out = np.empty((n, c, oh, ow), np.float32)
    lib().orc_avgpool_fwd(n * c, ih, iw, oh, ow, k[0], k[1], s[0], s[1], p[0], p[1], int(include_pad), divisor or 0, x, out)
    return out


def avgpool_bwd(g, x_shape, k, s, p, include_pad=True, divisor=None):
    g = _c(g)
    n, c, ih, iw = x_shape
    gx = np.empty(x_shape, np.float32)
    lib().orc_avgpool_bwd(n * c, ih, iw, g.shape[2], g.shape[3], k[0], k[1], s[0], s[1], p[0], p[1], int(include_pad),
                          divisor or 0, g, gx)
    return gx


def adapool_fwd(x, oh, ow):
    """adapool_fwd.wgsl."""
    x = _c(x)
    n, c, ih, iw = x.shape
    out = np.empty((n, c, oh, ow), np.float32)
    lib().orc_adapool_fwd(n * c, ih, iw, oh, ow, x, out)
    return out


def adapool_bwd(g, x_shape):
    g = _c(g)
    n, c, ih, iw = x_shape
    gx = np.empty(x_shape, np.float32)
    lib().orc_adapool_bwd(n * c, ih, iw, g.shape[2], g.shape[3], g, gx)
    return gx


def rel_l2(a, b):
    """||a - b||_2 / ||b||_2 in float64 (the per-op parity metric, rel-L2 <= 1e-4)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    d = np.linalg.norm((a - b).ravel())
    nb = np.linalg.norm(b.ravel())
    return float(d / nb) if nb > 0 else float(d)


"""ctypes binding of libomt_hip.so (include/omt_hip.h).

The library is required: importing this module raises ImportError when it is missing, so no operator silently runs
anywhere but the HIP kernels.
"""

import ctypes
import pathlib

import torch  # noqa: F401  (loads torch's HIP runtime first; libomt_hip.so then binds to the same libamdhip64.so.7)

_HERE = pathlib.Path(__file__).resolve().parent
LIB_PATH = _HERE / "libomt_hip.so"

OMT_OK, OMT_UNSUPPORTED, OMT_OOM, OMT_DEVICE_ERROR, OMT_INVALID = range(5)
OMT_CONV_NONE, OMT_CONV_DENSE, OMT_CONV_DW, OMT_CONV_DWG = range(4)
OMT_EPI_BIAS, OMT_EPI_RELU = 1, 2
OMT_DIR_FWD, OMT_DIR_DGRAD, OMT_DIR_WGRAD, OMT_DIR_FWD_NHWC, OMT_DIR_DGRAD_NHWC, OMT_DIR_WGRAD_NHWC = range(6)
NOALLOC_SCRATCH_BYTES = 64 << 20  # OMT_NOALLOC_SCRATCH_BYTES
(OMT_PW_ADD, OMT_PW_MUL, OMT_PW_RELU, OMT_PW_THRESHOLD_BWD, OMT_PW_HARDSWISH, OMT_PW_HARDSWISH_BWD, OMT_PW_HARDSIGMOID,
 OMT_PW_HARDSIGMOID_BWD, OMT_PW_SCALE, OMT_PW_FILL, OMT_PW_ADD_SCALAR) = range(11)
OMT_DT_F32, OMT_DT_I64 = 0, 1
OMT_ACT_NONE, OMT_ACT_RELU, OMT_ACT_HARDSWISH = 0, 1, 2
FOREACH_MAX_NUMEL = 1 << 16  # OMT_FOREACH_MAX_NUMEL


class ConvGeo(ctypes.Structure):
    """omt_conv_geo (reference Geo, csrc/omt.h:224-229)."""
    _fields_ = [(k, ctypes.c_int64) for k in ("n", "ci", "co", "ih", "iw", "oh", "ow", "ks", "stride", "pad")]

    def astuple(self):
        return tuple(getattr(self, k) for k, _ in self._fields_)


class ConvPlan(ctypes.Structure):
    """omt_conv_plan: tile index and K slices of a dense convolution GEMM (reference ConvPlan, csrc/omt.h:230-236)."""
    _fields_ = [("tile", ctypes.c_int32), ("slices", ctypes.c_int32)]


class SliceSum(ctypes.Structure):
    """omt_slice_sum: a deferred in-order sum of `slices` arrays of n floats at `parts` into `out`."""
    _fields_ = [("parts", ctypes.c_void_p), ("out", ctypes.c_void_p), ("n", ctypes.c_int64), ("slices", ctypes.c_int32)]


class OmtError(RuntimeError):
    def __init__(self, status, msg):
        super().__init__(msg)
        self.status = status


class Unsupported(OmtError):
    """OMT_UNSUPPORTED: the geometry is outside what the kernels cover (reference: NEED -> Unsupported)."""


class AdamTensor(ctypes.Structure):
    """omt_adam_tensor: one parameter of a fused Adam / AdamW step (reference csrc/optim.cpp:30-50)."""
    _fields_ = [("param", ctypes.c_void_p), ("grad", ctypes.c_void_p), ("exp_avg", ctypes.c_void_p),
                ("exp_avg_sq", ctypes.c_void_p), ("max_exp_avg_sq", ctypes.c_void_p), ("step", ctypes.c_void_p),
                ("numel", ctypes.c_int64)]


class AdamParams(ctypes.Structure):
    """omt_adam_params: hyper-parameters of a fused Adam / AdamW step."""
    _fields_ = [("lr", ctypes.c_float), ("lr_dev", ctypes.c_void_p), ("beta1", ctypes.c_float),
                ("beta2", ctypes.c_float), ("weight_decay", ctypes.c_float), ("eps", ctypes.c_float),
                ("amsgrad", ctypes.c_int), ("maximize", ctypes.c_int), ("decoupled", ctypes.c_int),
                ("grad_scale", ctypes.c_void_p), ("found_inf", ctypes.c_void_p)]


class SgdTensor(ctypes.Structure):
    """omt_sgd_tensor: one parameter of a fused SGD step (reference csrc/optim.cpp:12-28)."""
    _fields_ = [("param", ctypes.c_void_p), ("grad", ctypes.c_void_p), ("momentum_buffer", ctypes.c_void_p),
                ("numel", ctypes.c_int64)]


class SgdParams(ctypes.Structure):
    """omt_sgd_params: hyper-parameters of a fused SGD step."""
    _fields_ = [("lr", ctypes.c_float), ("lr_dev", ctypes.c_void_p), ("momentum", ctypes.c_float),
                ("dampening", ctypes.c_float), ("weight_decay", ctypes.c_float), ("nesterov", ctypes.c_int),
                ("maximize", ctypes.c_int), ("first_step", ctypes.c_int), ("grad_scale", ctypes.c_void_p),
                ("found_inf", ctypes.c_void_p)]


I64, U32, I32, F32, F64, SZ, VP = (ctypes.c_int64, ctypes.c_uint, ctypes.c_int, ctypes.c_float, ctypes.c_double,
                                   ctypes.c_size_t, ctypes.c_void_p)
G = ctypes.POINTER(ConvGeo)
PL = ctypes.POINTER(ConvPlan)

# name -> (restype, argtypes); the full exported surface of include/omt_hip.h
SIGNATURES = {
    "omt_last_error": (ctypes.c_char_p, []),
    "omt_abi_version": (I32, []),
    "omt_set_kernel_timing": (None, [I32]),
    "omt_kernel_stats_reset": (None, [I32]),
    "omt_kernel_stat_count": (I32, []),
    "omt_kernel_stat_entry": (I32, [I32, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(I64),
                                    ctypes.POINTER(F64)]),
    "omt_hip_runtime_version": (I32, []),
    "omt_conv_geo_init": (None, [G, I64, I64, I64, I64, I64, I64, I64, I64]),
    "omt_conv_kind": (I32, [I64] * 10 + [I32, I64]),
    "omt_malloc": (I32, [ctypes.POINTER(VP), SZ]),
    "omt_malloc_on": (I32, [ctypes.POINTER(VP), SZ, VP]),
    "omt_record_stream": (I32, [VP, VP]),
    "omt_free": (I32, [VP]),
    "omt_empty_cache": (I32, []),
    "omt_memory_allocated": (SZ, []),
    "omt_memory_reserved": (SZ, []),
    "omt_set_memory_limit": (None, [SZ]),
    "omt_default_stream": (VP, []),
    "omt_memcpy": (I32, [VP, VP, SZ, I32, VP]),
    "omt_memset_zero": (I32, [VP, SZ, VP]),
    "omt_stream_sync": (I32, [VP]),
    "omt_graph_pool_create": (I32, []),
    "omt_graph_pool_begin": (I32, [I32]),
    "omt_graph_pool_end": (I32, []),
    "omt_graph_pool_release": (I32, [I32]),
    "omt_event_create": (I32, [ctypes.POINTER(VP)]),
    "omt_event_destroy": (I32, [VP]),
    "omt_event_record": (I32, [VP, VP]),
    "omt_event_query": (I32, [VP]),
    "omt_event_sync": (I32, [VP]),
    "omt_event_elapsed_ms": (I32, [VP, VP, ctypes.POINTER(F32)]),
    "omt_conv_fwd_workspace": (SZ, [G]),
    "omt_conv_fwd": (I32, [G, VP, VP, VP, U32, VP, VP, VP, VP, F32, VP, VP, SZ, VP]),
    "omt_conv_fwd_unsummed": (I32, [G, VP, VP, VP, VP, SZ, I32, ctypes.POINTER(VP), ctypes.POINTER(I32), VP]),
    "omt_conv_fwd_stats_bytes": (SZ, [G]),
    "omt_conv_fwd_stats": (I32, [G, VP, VP, VP, VP, SZ, ctypes.POINTER(I32), VP, SZ, VP]),
    "omt_conv_dgrad_workspace": (SZ, [G]),
    "omt_conv_dgrad": (I32, [G, VP, VP, VP, VP, SZ, VP]),
    "omt_conv_wgrad_workspace": (SZ, [G]),
    "omt_conv_wgrad": (I32, [G, VP, VP, VP, VP, SZ, VP]),
    "omt_conv_wgrad_noalloc": (I32, [G, VP, VP, VP, VP]),
    "omt_conv_fwd_nhwc_workspace": (SZ, [G]),
    "omt_conv_fwd_nhwc": (I32, [G, VP, VP, VP, U32, VP, VP, SZ, VP]),
    "omt_conv_dgrad_nhwc_workspace": (SZ, [G]),
    "omt_conv_dgrad_nhwc": (I32, [G, VP, VP, VP, VP, SZ, VP]),
    "omt_conv_wgrad_nhwc_workspace": (SZ, [G]),
    "omt_conv_wgrad_nhwc": (I32, [G, VP, VP, VP, VP, SZ, VP]),
    "omt_pointwise": (I32, [ctypes.c_int, I64, VP, VP, ctypes.c_float, VP, VP]),
    "omt_foreach_add_scalar": (I32, [ctypes.c_int, ctypes.POINTER(VP), ctypes.POINTER(I64), ctypes.c_int, I64,
                                     ctypes.c_float, VP]),
    "omt_channel_scale": (I32, [I64, I64, VP, VP, VP, VP]),
    "omt_plane_broadcast": (I32, [I64, I64, VP, ctypes.c_float, VP, VP]),
    "omt_plane_sum": (I32, [I64, I64, VP, ctypes.c_float, VP, VP]),
    "omt_plane_sum_nhwc": (I32, [I64, I64, I64, VP, ctypes.c_float, VP, VP]),
    "omt_plane_dot": (I32, [I64, I64, VP, VP, ctypes.c_float, VP, VP]),
    "omt_se_gate_bwd": (I32, [I64, I64, VP, VP, VP, ctypes.c_float, VP, VP]),
    "omt_se_gate_bwd_nhwc": (I32, [I64, I64, I64, VP, VP, VP, ctypes.c_float, VP, VP]),
    "omt_channel_scale_nhwc": (I32, [I64, I64, I64, VP, VP, VP, VP]),
    "omt_dw_fwd_nhwc": (I32, [VP, VP, VP, VP, VP, VP]),
    "omt_dw_dgrad_nhwc": (I32, [VP, VP, VP, VP, VP]),
    "omt_dw_wgrad_nhwc_workspace": (SZ, [VP]),
    "omt_dw_wgrad_nhwc": (I32, [VP, VP, VP, VP, VP, SZ, VP]),
    "omt_pointwise_layouts": (I32, [ctypes.c_int, I64, I64, I64, VP, ctypes.c_int, VP, ctypes.c_int, ctypes.c_float, VP,
                                    ctypes.c_int, VP]),
    "omt_log_softmax_fwd": (I32, [I64, I64, VP, VP, VP]),
    "omt_log_softmax_bwd": (I32, [I64, I64, VP, VP, VP, VP]),
    "omt_nll_loss_fwd": (I32, [I64, I64, VP, VP, VP, I64, ctypes.c_int, VP, VP, VP]),
    "omt_nll_loss_bwd": (I32, [I64, I64, VP, VP, VP, I64, ctypes.c_int, VP, VP, VP]),
    "omt_bn_nhwc_workspace": (SZ, [I64, I64, I64]),
    "omt_bn_train_fwd_nhwc": (I32, [I64, I64, I64, VP, VP, VP, VP, VP, F64, F64, I32, VP, VP, VP, VP, VP, VP, VP, VP,
                                    SZ, VP]),
    "omt_bn_eval_fwd_nhwc": (I32, [I64, I64, I64, VP, VP, VP, VP, VP, F64, I32, VP, VP]),
    "omt_bn_bwd_nhwc": (I32, [I64, I64, I64, VP, I32, VP, VP, I32, VP, VP, VP, VP, VP, VP, VP, VP, VP, SZ, VP]),
    "omt_maxpool_fwd_nhwc": (I32, [I64] * 14 + [VP, VP, VP, VP]),
    "omt_maxpool_bwd_nhwc": (I32, [I64] * 14 + [VP, VP, VP, VP]),
    "omt_avgpool_fwd_nhwc": (I32, [I64] * 12 + [I32, I64, VP, VP, VP]),
    "omt_avgpool_bwd_nhwc": (I32, [I64] * 12 + [I32, I64, VP, VP, VP]),
    "omt_adapool_fwd_nhwc": (I32, [I64] * 6 + [VP, VP, VP]),
    "omt_adapool_bwd_nhwc": (I32, [I64] * 6 + [VP, VP, VP]),
    "omt_se_bwd_workspace": (SZ, [I64, I64, I64]),
    "omt_se_fwd": (I32, [I64, I64, I64] + [VP] * 9),
    "omt_se_bwd": (I32, [I64, I64, I64] + [VP] * 12 + [SZ, VP]),
    "omt_conv_bwd_workspace": (SZ, [G]),
    "omt_conv_bwd": (I32, [G, VP, VP, VP, VP, VP, VP, SZ, VP]),
    "omt_conv_bwd_parts": (I32, [G, VP, VP, VP, VP, VP, VP, SZ, I32, ctypes.POINTER(VP), ctypes.POINTER(I32),
                                 ctypes.POINTER(SliceSum), VP]),
    "omt_slice_sums": (I32, [ctypes.POINTER(SliceSum), I32, VP]),
    "omt_conv_num_tiles": (I32, [I32]),
    "omt_conv_get_plan": (I32, [I32, G, PL, ctypes.POINTER(I32)]),
    "omt_conv_set_plan": (I32, [I32, G, PL]),
    "omt_conv_plan_count": (I32, []),
    "omt_conv_plan_entry": (I32, [I32, ctypes.POINTER(I32), G, PL]),
    "omt_conv_clear_plans": (None, []),
    "omt_conv_autotune": (I32, [I32, G, I32, VP, PL]),
    "omt_conv_autotune_bwd": (I32, [G, I32, VP, PL, PL]),
    "omt_bias_grad": (I32, [I64, I64, I64, VP, VP, VP]),
    "omt_fold_bn": (I32, [I64, I64, VP, VP, VP, VP, VP, VP, F32, VP, VP, VP]),
    "omt_dw_fwd": (I32, [G, VP, VP, VP, VP, VP, VP, VP, F32, VP, VP]),
    "omt_dw_dgrad": (I32, [G, VP, VP, VP, VP]),
    "omt_dw_wgrad_workspace": (SZ, [G]),
    "omt_dw_wgrad": (I32, [G, VP, VP, VP, VP, SZ, VP]),
    "omt_bn_train_workspace": (SZ, [I64, I64, I64]),
    "omt_bn_train_fwd": (I32, [I64, I64, I64, VP, VP, VP, VP, VP, F64, F64, I32, VP, VP, VP, VP, VP, VP, SZ, VP]),
    "omt_bn_train_fwd_res": (I32, [I64, I64, I64, VP, VP, VP, VP, VP, F64, F64, I32] + [VP] * 8 + [SZ, VP]),
    "omt_bn_train_fwd_parts": (I32, [I64, I64, I64, VP, I32, VP, VP, VP, VP, VP, F64, F64, I32] + [VP] * 8 + [SZ, VP]),
    "omt_bn_train_fwd_pool": (I32, [I64, I64, I64, I64, VP, VP, VP, VP, VP, F64, F64, I32] + [VP] * 5 + [I64] * 6 +
                              [VP, VP, VP, SZ, VP]),
    "omt_bn_train_fwd_stats": (I32, [I64, I64, I64, VP, VP, I32, SZ, VP, VP, VP, VP, F64, F64, I32] + [VP] * 8 +
                               [SZ, VP]),
    "omt_bn_eval_fwd": (I32, [I64, I64, I64, VP, VP, VP, VP, VP, F64, I32, VP, VP]),
    "omt_bn_bwd_workspace": (SZ, [I64, I64, I64]),
    "omt_bn_bwd": (I32, [I64, I64, I64, VP, VP, VP, VP, VP, VP, VP, VP, VP, VP, SZ, VP]),
    "omt_bn_bwd_act": (I32, [I64, I64, I64, VP, VP, I32, VP, VP, VP, VP, VP, VP, VP, VP, SZ, VP]),
    "omt_bn_bwd_parts": (I32, [I64, I64, I64, VP, I32, VP, VP, I32, VP, VP, VP, VP, VP, VP, VP, VP,
                               ctypes.POINTER(SliceSum), I32, VP]),
    "omt_bn_bwd_res": (I32, [I64, I64, I64, VP, VP, VP, VP, VP, VP, VP, VP, VP, VP, VP, VP, SZ, VP]),
    "omt_maxpool_fwd": (I32, [I64] * 13 + [VP, VP, VP, VP]),
    "omt_maxpool_bwd": (I32, [I64] * 13 + [VP, VP, VP, VP]),
    "omt_avgpool_fwd": (I32, [I64] * 11 + [I32, I64, VP, VP, VP]),
    "omt_avgpool_bwd": (I32, [I64] * 11 + [I32, I64, VP, VP, VP]),
    "omt_adapool_fwd": (I32, [I64] * 5 + [VP, VP, VP]),
    "omt_adapool_bwd": (I32, [I64] * 5 + [VP, VP, VP]),
    "omt_fused_adam": (I32, [ctypes.POINTER(AdamParams), ctypes.POINTER(AdamTensor), I32, VP]),
    "omt_fused_sgd": (I32, [ctypes.POINTER(SgdParams), ctypes.POINTER(SgdTensor), I32, VP]),
}

ABI_VERSION = 5


def _load():
    if not LIB_PATH.exists():
        raise ImportError(f"omarchy_mac_torch: {LIB_PATH} is not built; run `python omarchy-mac-torch_amd/build_native.py`"
                          " (or __graft_entry__.build())")
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.omt_abi_version() != ABI_VERSION:
        raise ImportError(f"libomt_hip.so ABI {lib.omt_abi_version()} != {ABI_VERSION}; rebuild it")
    return lib


L = _load()


def check(status, what=""):
    """Raises on a non-OK status, with the library's message."""
    if status == OMT_OK:
        return
    msg = (L.omt_last_error() or b"").decode(errors="replace")
    if what:
        msg = f"{what}: {msg}"
    if status == OMT_UNSUPPORTED:
        raise Unsupported(status, msg)
    if status == OMT_OOM:
        raise torch.OutOfMemoryError(msg)
    raise OmtError(status, msg)


def conv_geo(n, ci, co, ih, iw, ks, stride, pad):
    g = ConvGeo()
    L.omt_conv_geo_init(ctypes.byref(g), n, ci, co, ih, iw, ks, stride, pad)
    return g

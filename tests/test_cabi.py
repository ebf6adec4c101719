"""CPU checks of the C ABI (no GPU needed): libomt_hip.so loads and exports every function include/omt_hip.h
declares, the ctypes table matches the header, host-side argument validation returns the documented statuses before
any device work, and the fast integer division the kernels use is exact."""

import ctypes
import pathlib
import re
import subprocess

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "omt_hip.h"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(omt_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    from omarchy_mac_torch import _lib
    names = declared_functions()
    assert len(names) >= 40
    lib = ctypes.CDLL(str(_lib.LIB_PATH))
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert sorted(_lib.SIGNATURES) == names


def test_noalloc_scratch_size_matches_the_header():
    from omarchy_mac_torch import _lib
    m = re.search(r"#define OMT_NOALLOC_SCRATCH_BYTES \((\d+)u << (\d+)\)", HEADER.read_text())
    assert m and int(m.group(1)) << int(m.group(2)) == _lib.NOALLOC_SCRATCH_BYTES


def test_geometry_and_kind_table():
    from omarchy_mac_torch import _lib
    g = _lib.conv_geo(16, 3, 64, 224, 224, 11, 4, 2)
    assert (g.oh, g.ow) == (55, 55)
    k = _lib.L.omt_conv_kind
    # (x_c, w_o, kh, kw, sh, sw, ph, pw, dh, dw, transposed, groups) -> kind (csrc/conv.cpp:167-177)
    assert k(3, 64, 11, 11, 4, 4, 2, 2, 1, 1, 0, 1) == _lib.OMT_CONV_DENSE
    assert k(3, 64, 11, 11, 5, 5, 2, 2, 1, 1, 0, 1) == _lib.OMT_CONV_NONE   # stride 5
    assert k(3, 64, 12, 12, 1, 1, 0, 0, 1, 1, 0, 1) == _lib.OMT_CONV_NONE   # ks 12
    assert k(3, 64, 3, 3, 1, 1, 4, 4, 1, 1, 0, 1) == _lib.OMT_CONV_NONE     # pad > ks
    assert k(3, 64, 3, 3, 1, 1, 1, 1, 2, 2, 0, 1) == _lib.OMT_CONV_NONE     # dilated
    assert k(3, 64, 3, 5, 1, 1, 1, 1, 1, 1, 0, 1) == _lib.OMT_CONV_NONE     # non-square
    assert k(3, 64, 3, 3, 1, 1, 1, 1, 1, 1, 1, 1) == _lib.OMT_CONV_NONE     # transposed
    assert k(8, 8, 3, 3, 1, 1, 1, 1, 1, 1, 0, 8) == _lib.OMT_CONV_DW
    assert k(8, 8, 5, 5, 1, 1, 1, 1, 1, 1, 0, 8) == _lib.OMT_CONV_DWG       # dw with non-"same" pad
    assert k(8, 8, 3, 3, 2, 2, 1, 1, 1, 1, 0, 8) == _lib.OMT_CONV_DWG
    assert k(8, 16, 3, 3, 1, 1, 1, 1, 1, 1, 0, 8) == _lib.OMT_CONV_NONE     # channel multiplier
    assert k(8, 8, 3, 3, 1, 1, 1, 1, 1, 1, 0, 2) == _lib.OMT_CONV_NONE      # grouped


def test_host_validation_statuses():
    """Unsupported geometry and bad arguments are rejected on the host, before any kernel launch."""
    from omarchy_mac_torch import _lib
    L = _lib.L
    fake = ctypes.c_void_p(0x1000)  # never dereferenced: validation fails first
    g = _lib.ConvGeo(2, 3, 4, 8, 8, 1, 1, 12, 1, 0)  # ks 12
    assert L.omt_conv_fwd(ctypes.byref(g), fake, fake, None, 0, None, None, None, None, 1e-5, fake, None, 0, None) == \
        _lib.OMT_UNSUPPORTED
    assert b"geometry" in L.omt_last_error()
    g = _lib.conv_geo(2, 3, 4, 8, 8, 3, 1, 1)
    assert L.omt_conv_fwd(ctypes.byref(g), None, fake, None, 0, None, None, None, None, 1e-5, fake, None, 0, None) == \
        _lib.OMT_INVALID
    assert L.omt_conv_fwd(ctypes.byref(g), fake, fake, None, _lib.OMT_EPI_BIAS, None, None, None, None, 1e-5, fake,
                          None, 0, None) == _lib.OMT_INVALID
    assert L.omt_conv_fwd(ctypes.byref(g), fake, fake, None, 0, fake, None, None, None, 1e-5, fake, None, 0, None) == \
        _lib.OMT_INVALID  # partial BN loader
    g64 = _lib.conv_geo(2, 64, 8, 8, 8, 3, 1, 1)  # tap-major order: the re-packed filter needs a workspace
    assert L.omt_conv_set_plan(_lib.OMT_DIR_FWD, ctypes.byref(g64), ctypes.byref(_lib.ConvPlan(0, 1))) == _lib.OMT_OK
    assert L.omt_conv_fwd_workspace(ctypes.byref(g64)) == 8 * 64 * 9 * 4  # one K slice: no partials
    assert L.omt_conv_fwd(ctypes.byref(g64), fake, fake, None, 0, None, None, None, None, 1e-5, fake, None, 0, None) \
        == _lib.OMT_INVALID
    L.omt_conv_clear_plans()
    g.oh = 99  # inconsistent geometry
    assert L.omt_conv_wgrad(ctypes.byref(g), fake, fake, fake, None, 0, None) == _lib.OMT_UNSUPPORTED
    g = _lib.conv_geo(2, 5, 16, 8, 8, 3, 2, 1)  # tap-major grad input (C_out % 16 == 0) re-packs its filter
    assert L.omt_conv_set_plan(_lib.OMT_DIR_DGRAD, ctypes.byref(g), ctypes.byref(_lib.ConvPlan(0, 1))) == _lib.OMT_OK
    assert L.omt_conv_dgrad(ctypes.byref(g), fake, fake, fake, None, 0, None) == _lib.OMT_INVALID  # no workspace
    assert L.omt_conv_dgrad_workspace(ctypes.byref(g)) == 16 * 5 * 3 * 3 * 4
    n_gather = L.omt_conv_num_tiles(_lib.OMT_DIR_DGRAD) // 3  # tiles, each tap-major / channel-major / in place
    # the channel-major twin of tile 0 and its in-place tap-major twin both read w directly
    for tile in (n_gather, 2 * n_gather):
        assert L.omt_conv_set_plan(_lib.OMT_DIR_DGRAD, ctypes.byref(g), ctypes.byref(_lib.ConvPlan(tile, 1))) \
            == _lib.OMT_OK
        assert L.omt_conv_dgrad_workspace(ctypes.byref(g)) == 0, tile
    # forward: the 3 x 3 filter re-packed for tile 0, read in place by its third twin; the 1 x 1 filter is never packed
    gf = _lib.conv_geo(2, 32, 16, 8, 8, 3, 1, 1)
    for tile, ws in ((0, 16 * 32 * 9 * 4), (2 * n_gather, 0)):
        assert L.omt_conv_set_plan(_lib.OMT_DIR_FWD, ctypes.byref(gf), ctypes.byref(_lib.ConvPlan(tile, 1))) \
            == _lib.OMT_OK
        assert L.omt_conv_fwd_workspace(ctypes.byref(gf)) == ws, tile
    # 3 grad-input channels at stride 2: one super-pixel GEMM of 2 x 2 phases x 3 channels over the 2 x 2 window of gy
    # the 3 x 3 filter reaches (phase rows 0 and 1 use gy rows i and i, i + 1); its filter is re-packed in both K
    # orders, and split over K its partials hold the 12 rows on the 4 x 4 grid
    g3 = _lib.conv_geo(2, 3, 16, 8, 8, 3, 2, 1)
    pack = 4 * 3 * 16 * 2 * 2 * 4
    for plan, ws in (((0, 1), pack), ((n_gather, 1), pack), ((2 * n_gather, 1), pack),
                     ((5, 4), pack + 4 * 2 * 12 * 4 * 4 * 4)):
        assert L.omt_conv_set_plan(_lib.OMT_DIR_DGRAD, ctypes.byref(g3), ctypes.byref(_lib.ConvPlan(*plan))) \
            == _lib.OMT_OK
        assert L.omt_conv_dgrad_workspace(ctypes.byref(g3)) == ws, plan
    # AlexNet conv1 (11 x 11, stride 4, pad 2): phase rows py = 0..3 reach gy rows i-2..i, i-1..i, i-1..i+1, i-1..i+1
    # (ky0 = 2, 3, 0, 1), so the window is 4 x 4 and the filter 16 phases x 3 channels by 64 x 16 taps
    g1 = _lib.conv_geo(16, 3, 64, 224, 224, 11, 4, 2)
    assert L.omt_conv_set_plan(_lib.OMT_DIR_DGRAD, ctypes.byref(g1), ctypes.byref(_lib.ConvPlan(4, 1))) == _lib.OMT_OK
    assert L.omt_conv_dgrad_workspace(ctypes.byref(g1)) == 16 * 3 * 64 * 4 * 4 * 4
    L.omt_conv_clear_plans()
    with pytest.raises(_lib.Unsupported):
        _lib.check(_lib.OMT_UNSUPPORTED)


def test_unsummed_backward_validation_host_side():
    """omt_conv_bwd_parts / omt_bn_bwd_parts / omt_slice_sums reject bad arguments on the host, before any launch."""
    from omarchy_mac_torch import _lib
    L = _lib.L
    fake = ctypes.c_void_p(0x1000)  # never dereferenced: validation fails first
    parts, slices, job = ctypes.c_void_p(), ctypes.c_int32(), _lib.SliceSum()
    g = _lib.conv_geo(2, 8, 8, 8, 8, 3, 1, 1)
    out = (ctypes.byref(parts), ctypes.byref(slices), ctypes.byref(job))
    assert L.omt_conv_bwd_parts(ctypes.byref(g), fake, fake, fake, fake, None, None, 0, 4, *out, None) == \
        _lib.OMT_INVALID  # no grad weight
    assert L.omt_conv_bwd_parts(ctypes.byref(g), fake, fake, fake, fake, fake, None, 0, 4, None, ctypes.byref(slices),
                                ctypes.byref(job), None) == _lib.OMT_INVALID
    g.oh = 99
    assert L.omt_conv_bwd_parts(ctypes.byref(g), fake, fake, fake, fake, fake, None, 0, 4, *out, None) == \
        _lib.OMT_UNSUPPORTED
    bad = (_lib.SliceSum * 1)(_lib.SliceSum(None, fake, 16, 2))
    assert L.omt_slice_sums(bad, 1, None) == _lib.OMT_INVALID
    assert L.omt_slice_sums(None, 1, None) == _lib.OMT_INVALID
    assert L.omt_slice_sums(None, 0, None) == _lib.OMT_OK
    none = (_lib.SliceSum * 1)(_lib.SliceSum(None, None, 0, 0))
    assert L.omt_slice_sums(none, 1, None) == _lib.OMT_OK  # nothing to sum: no launch

    def bn(n=2, c=4, hw=16, slices=2, g2=None, act=_lib.OMT_ACT_RELU, act_in=fake, gz=None, sums=None, count=0):
        return L.omt_bn_bwd_parts(n, c, hw, fake, slices, g2, fake, act, act_in, fake, fake, fake, fake, fake, fake,
                                  gz, sums, count, None)
    assert bn(slices=0) == _lib.OMT_INVALID
    assert bn(slices=65) == _lib.OMT_INVALID
    assert bn(act=3) == _lib.OMT_INVALID
    assert bn(act_in=None) == _lib.OMT_INVALID      # ReLU without its output
    assert bn(g2=fake) == _lib.OMT_INVALID          # a second gradient only with gz
    assert bn(count=1) == _lib.OMT_INVALID          # no sums array
    assert bn(count=3, sums=bad) == _lib.OMT_INVALID  # at most two
    assert bn(count=1, sums=bad) == _lib.OMT_INVALID  # a sum without its partials
    assert bn(n=2, hw=4097) == _lib.OMT_UNSUPPORTED  # channels of more than 8192 elements


def test_batch_chunks_host_side():
    """A batch past 2 GiB (3 images of 876 MB in and out) is planned as batch chunks of 2 images, then 1: plan calls
    on it act on the first chunk's geometry, its workspaces are the larger chunk's (grad weight: plus the chunks'
    filter gradients, 256-byte aligned), and one image or a filter of 2 GiB or more is OMT_UNSUPPORTED with no
    workspace, all without a GPU."""
    from omarchy_mac_torch import _lib
    L = _lib.L
    fake = ctypes.c_void_p(0x1000)  # never dereferenced: validation fails first
    L.omt_conv_clear_plans()
    big, two, one = (_lib.conv_geo(n, 16, 16, 3700, 3700, 3, 1, 1) for n in (3, 2, 1))

    def plan(d, g):
        p, c = _lib.ConvPlan(), ctypes.c_int32()
        assert L.omt_conv_get_plan(d, ctypes.byref(g), ctypes.byref(p), ctypes.byref(c)) == _lib.OMT_OK
        return p.tile, p.slices, c.value

    try:
        for d in (_lib.OMT_DIR_FWD, _lib.OMT_DIR_DGRAD, _lib.OMT_DIR_WGRAD, _lib.OMT_DIR_FWD_NHWC):
            assert plan(d, big) == plan(d, two), d
        # a plan set on the whole batch is the first chunk's
        assert L.omt_conv_set_plan(_lib.OMT_DIR_WGRAD, ctypes.byref(big), ctypes.byref(_lib.ConvPlan(2, 3))) == \
            _lib.OMT_OK
        assert plan(_lib.OMT_DIR_WGRAD, two) == (2, 3, 1)
        ws1 = L.omt_conv_wgrad_workspace(ctypes.byref(one))
        ws2 = L.omt_conv_wgrad_workspace(ctypes.byref(two))
        assert ws2 == 3 * 16 * 16 * 9 * 4
        filt = (2 * 16 * 16 * 9 * 4 + 255) // 256 * 256
        assert L.omt_conv_wgrad_workspace(ctypes.byref(big)) == filt + max(ws1, ws2)
        assert L.omt_conv_bwd_workspace(ctypes.byref(big)) == filt + max(L.omt_conv_bwd_workspace(ctypes.byref(g))
                                                                          for g in (one, two))
        for ws in (L.omt_conv_fwd_workspace, L.omt_conv_dgrad_workspace, L.omt_conv_fwd_nhwc_workspace,
                   L.omt_conv_dgrad_nhwc_workspace):
            assert ws(ctypes.byref(big)) == max(ws(ctypes.byref(one)), ws(ctypes.byref(two))), ws
        # the whole-batch check of the entry points accepts it (a missing workspace is the next error)
        assert L.omt_conv_wgrad(ctypes.byref(big), fake, fake, fake, None, 0, None) == _lib.OMT_INVALID
        assert b"workspace" in L.omt_last_error()
        # no chunk fits: one image of 4.5 GB, or a 2.4 GB filter
        for g in (_lib.conv_geo(2, 64, 64, 4200, 4200, 3, 1, 1), _lib.conv_geo(2, 8192, 8192, 8, 8, 3, 1, 1)):
            assert L.omt_conv_fwd_workspace(ctypes.byref(g)) == 0
            assert L.omt_conv_wgrad_workspace(ctypes.byref(g)) == 0
            assert L.omt_conv_fwd(ctypes.byref(g), fake, fake, None, 0, None, None, None, None, 1e-5, fake, None, 0,
                                  None) == _lib.OMT_UNSUPPORTED
            assert b"2 GiB" in L.omt_last_error()
            assert L.omt_conv_bwd(ctypes.byref(g), fake, fake, fake, fake, fake, None, 0, None) == _lib.OMT_UNSUPPORTED
            p = _lib.ConvPlan()
            assert L.omt_conv_get_plan(_lib.OMT_DIR_FWD, ctypes.byref(g), ctypes.byref(p), None) == \
                _lib.OMT_UNSUPPORTED
    finally:
        L.omt_conv_clear_plans()


def test_epilogue_statistics_validation_host_side():
    """omt_conv_fwd_stats / omt_bn_train_fwd_stats reject bad arguments on the host, before any launch: null
    pointers, a statistics buffer smaller than omt_conv_fwd_stats_bytes (one pair per channel and 32 output pixels), a
    plan that splits K, a batch that would run in chunks, zero column groups, and more column groups than the
    statistics buffer holds."""
    from omarchy_mac_torch import _lib
    L = _lib.L
    fake = ctypes.c_void_p(0x1000)  # never dereferenced: validation fails first
    groups = ctypes.c_int32(7)
    g = _lib.conv_geo(2, 16, 24, 10, 10, 3, 1, 1)
    need = L.omt_conv_fwd_stats_bytes(ctypes.byref(g))
    assert need == -(-2 * 10 * 10 // 32) * 24 * 2 * 8
    L.omt_conv_clear_plans()
    try:
        assert L.omt_conv_fwd_stats(ctypes.byref(g), fake, fake, fake, None, need, ctypes.byref(groups), fake, 1 << 30,
                                    None) == _lib.OMT_INVALID
        assert L.omt_conv_fwd_stats(ctypes.byref(g), fake, fake, fake, fake, need - 8, ctypes.byref(groups), fake,
                                    1 << 30, None) == _lib.OMT_INVALID
        assert groups.value == 0
        assert L.omt_conv_set_plan(_lib.OMT_DIR_FWD, ctypes.byref(g), ctypes.byref(_lib.ConvPlan(5, 3))) == _lib.OMT_OK
        assert L.omt_conv_fwd_stats(ctypes.byref(g), fake, fake, fake, fake, need, ctypes.byref(groups), fake, 1 << 30,
                                    None) == _lib.OMT_UNSUPPORTED
        assert b"splits K" in L.omt_last_error()
        big = _lib.conv_geo(3, 16, 16, 3700, 3700, 3, 1, 1)  # past 2 GiB: the batch would run in chunks
        assert L.omt_conv_fwd_stats(ctypes.byref(big), fake, fake, fake, fake, 1 << 40, ctypes.byref(groups), fake,
                                    1 << 30, None) == _lib.OMT_UNSUPPORTED
    finally:
        L.omt_conv_clear_plans()
    ws = L.omt_bn_train_workspace(2, 24, 100)
    stats_bytes = 24 * 3 * 2 * 8  # 24 channels x 3 column groups x (sum, sum of squares)
    args = [2, 24, 100, fake, fake, 3, stats_bytes, fake, fake, None, None, 0.1, 1e-5, 1, None, fake, None, fake, fake,
            None, None, fake, ws, None]
    bad_groups = list(args)
    bad_groups[5] = 0
    assert L.omt_bn_train_fwd_stats(*bad_groups) == _lib.OMT_INVALID
    no_stats = list(args)
    no_stats[4] = None
    assert L.omt_bn_train_fwd_stats(*no_stats) == _lib.OMT_INVALID
    small_ws = list(args)
    small_ws[22] = ws - 8
    assert L.omt_bn_train_fwd_stats(*small_ws) == _lib.OMT_INVALID
    small_stats = list(args)  # a stats buffer sized for fewer groups than claimed
    small_stats[6] = stats_bytes - 8
    assert L.omt_bn_train_fwd_stats(*small_stats) == _lib.OMT_INVALID
    assert b"stats buffer" in L.omt_last_error()
    more_groups = list(args)
    more_groups[5] = 4
    assert L.omt_bn_train_fwd_stats(*more_groups) == _lib.OMT_INVALID
    bad_act = list(args)  # activations are 0 (none), 1 (ReLU) and 2 (hardswish)
    bad_act[13] = 3
    assert L.omt_bn_train_fwd_stats(*bad_act) == _lib.OMT_INVALID and b"activation" in L.omt_last_error()


def test_plan_cache_host_side():
    """The plan cache (tile, K slices per direction and geometry; reference conv_plan / tune_dump / tune_load,
    csrc/conv.cpp:45-60, 243-272) and the cost model's split choice, all host-side."""
    from omarchy_mac_torch import _lib
    L = _lib.L
    L.omt_conv_clear_plans()
    fwd, dgrad, wgrad = _lib.OMT_DIR_FWD, _lib.OMT_DIR_DGRAD, _lib.OMT_DIR_WGRAD
    assert L.omt_conv_num_tiles(fwd) == L.omt_conv_num_tiles(dgrad) >= 4 and L.omt_conv_num_tiles(wgrad) >= 3
    assert L.omt_conv_num_tiles(7) == 0 and L.omt_conv_num_tiles(6) == 0

    def plan(d, g):
        p, c = _lib.ConvPlan(), ctypes.c_int32()
        assert L.omt_conv_get_plan(d, ctypes.byref(g), ctypes.byref(p), ctypes.byref(c)) == _lib.OMT_OK
        return p.tile, p.slices, c.value

    late = _lib.conv_geo(32, 512, 512, 2, 2, 3, 1, 1)    # ResNet-18 layer4 at 64x64: 128 pixels, K = 4608
    big = _lib.conv_geo(256, 64, 64, 56, 56, 3, 1, 1)    # ResNet-50 layer1 at batch 256
    assert plan(fwd, late)[1] > 1 and plan(dgrad, late)[1] > 1 and plan(fwd, late)[2] == 0
    assert plan(fwd, big)[1] == 1 and plan(dgrad, big)[1] == 1
    # the workspace grows by the partials of a split: [packed filter | 256-B aligned slices x N*P*OH*OW floats]
    g = _lib.conv_geo(4, 64, 32, 6, 6, 3, 1, 1)
    pack = 32 * 64 * 9 * 4
    assert L.omt_conv_set_plan(fwd, ctypes.byref(g), ctypes.byref(_lib.ConvPlan(2, 4))) == _lib.OMT_OK
    assert plan(fwd, g) == (2, 4, 1)
    assert L.omt_conv_fwd_workspace(ctypes.byref(g)) == (pack + 255) // 256 * 256 + 4 * 4 * 32 * 6 * 6 * 4
    # slices beyond the K-blocks are clamped (K = 576 = 36 blocks of 16)
    assert L.omt_conv_set_plan(fwd, ctypes.byref(g), ctypes.byref(_lib.ConvPlan(0, 100))) == _lib.OMT_OK
    assert plan(fwd, g) == (0, 36, 1)
    assert L.omt_conv_set_plan(wgrad, ctypes.byref(g), ctypes.byref(_lib.ConvPlan(1, 50))) == _lib.OMT_OK
    assert plan(wgrad, g) == (1, 3, 1)    # K = 144 pixels -> at most 3 slices of 64
    for bad in (_lib.ConvPlan(-1, 1), _lib.ConvPlan(L.omt_conv_num_tiles(fwd), 1), _lib.ConvPlan(0, 0)):
        assert L.omt_conv_set_plan(fwd, ctypes.byref(g), ctypes.byref(bad)) == _lib.OMT_INVALID
    assert L.omt_conv_set_plan(6, ctypes.byref(g), ctypes.byref(_lib.ConvPlan(0, 1))) == _lib.OMT_INVALID
    bad_geo = _lib.ConvGeo(2, 3, 4, 8, 8, 1, 1, 12, 1, 0)
    assert L.omt_conv_set_plan(fwd, ctypes.byref(bad_geo), ctypes.byref(_lib.ConvPlan(0, 1))) == _lib.OMT_UNSUPPORTED
    # enumeration in key order, removal, clear
    assert L.omt_conv_plan_count() == 2
    d, eg, ep = ctypes.c_int32(), _lib.ConvGeo(), _lib.ConvPlan()
    assert L.omt_conv_plan_entry(1, ctypes.byref(d), ctypes.byref(eg), ctypes.byref(ep)) == _lib.OMT_OK
    assert (d.value, eg.astuple(), ep.tile, ep.slices) == (wgrad, g.astuple(), 1, 50)
    assert L.omt_conv_plan_entry(2, None, None, None) == _lib.OMT_INVALID
    assert L.omt_conv_set_plan(wgrad, ctypes.byref(g), None) == _lib.OMT_OK
    assert L.omt_conv_plan_count() == 1 and plan(wgrad, g)[2] == 0
    L.omt_conv_clear_plans()
    assert L.omt_conv_plan_count() == 0 and plan(fwd, g)[2] == 0


FASTDIV_TEST = r"""
#include "omt_internal.h"
#include <cstdio>
#include <random>
int main() {
  std::mt19937 rng(1);
  int bad = 0;
  for (uint32_t d = 1; d < 70000 && !bad; ++d) {
    omt::FastDiv f = omt::make_fastdiv(d);
    for (int i = 0; i < 200; ++i) {
      uint32_t n = i < 100 ? (uint32_t)(rng() % (1u << 31)) : (uint32_t)(i * 97 + d * (i % 7));
      if (omt::fdiv(n, f) != n / d) { printf("bad %u / %u\n", n, d); bad = 1; break; }
    }
    for (uint32_t k = 1; k < 4 && !bad; ++k) {  // around multiples of d
      uint64_t m = (uint64_t)d * (k * 1000003u % 30011u);
      for (int64_t e = -1; e <= 1; ++e) {
        int64_t n = (int64_t)m + e;
        if (n < 0 || n >= (1ll << 31)) continue;
        if (omt::fdiv((uint32_t)n, f) != (uint32_t)n / d) { printf("bad %lld / %u\n", (long long)n, d); bad = 1; }
      }
    }
  }
  for (uint32_t d : {2147483647u, 1u << 30, 3u, 7u, 802816u, 3136u, 49u, 121u})
    for (uint32_t n : {0u, 1u, d - 1, d, d + 1, 2147483647u})
      if (omt::fdiv(n, omt::make_fastdiv(d)) != n / d) { printf("bad %u / %u\n", n, d); bad = 1; }
  printf(bad ? "FAIL\n" : "OK\n");
  return bad;
}
"""


def test_fastdiv_exact(tmp_path):
    """FastDiv (omt_internal.h) against '/' for divisors 1..70000 and 31-bit numerators, built for the host."""
    src = tmp_path / "fastdiv.cpp"
    src.write_text(FASTDIV_TEST)
    exe = tmp_path / "fastdiv"
    subprocess.run(["/opt/rocm/bin/hipcc", "-x", "hip", "--offload-arch=gfx950", "-O2", "-std=c++17",
                    f"-I{ROOT / 'include'}", f"-I{ROOT / 'omarchy-mac-torch_amd' / 'csrc'}", str(src), "-o", str(exe)],
                   check=True, capture_output=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and r.stdout.strip() == "OK", r.stdout


def test_ctypes_structs_match_the_header(tmp_path):
    """Every struct the ctypes layer passes through the C ABI has the header's size and field offsets (a mismatch
    would hand the library shifted pointers)."""
    import shutil
    from omarchy_mac_torch import _lib
    if shutil.which("g++") is None:
        pytest.skip("needs g++")
    structs = {"omt_conv_geo": _lib.ConvGeo, "omt_conv_plan": _lib.ConvPlan, "omt_adam_tensor": _lib.AdamTensor,
               "omt_adam_params": _lib.AdamParams, "omt_sgd_tensor": _lib.SgdTensor, "omt_sgd_params": _lib.SgdParams,
               "omt_slice_sum": _lib.SliceSum}
    lines = ["#include <cstddef>", "#include <cstdio>", '#include "omt_hip.h"', "int main() {"]
    for cname, py in structs.items():
        lines.append(f'  printf("{cname} size %zu\\n", sizeof({cname}));')
        for field, _ in py._fields_:
            lines.append(f'  printf("{cname} {field} %zu\\n", offsetof({cname}, {field}));')
    lines.append("  return 0;\n}")
    src = tmp_path / "structs.cpp"
    src.write_text("\n".join(lines))
    exe = tmp_path / "structs"
    subprocess.run(["g++", "-std=c++17", f"-I{ROOT / 'include'}", str(src), "-o", str(exe)], check=True)
    got = dict((" ".join(l.split()[:2]), int(l.split()[2]))
               for l in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.splitlines())
    for cname, py in structs.items():
        assert got[f"{cname} size"] == ctypes.sizeof(py), cname
        for field, _ in py._fields_:
            assert got[f"{cname} {field}"] == getattr(py, field).offset, (cname, field)


def test_nhwc_plans_and_workspaces_host_side():
    """Channels-last directions: their own tile tables (the nine staged gather tiles; the four grad-weight tiles), a
    plan whose K-block does not divide the gathered channels runs as tile 5, workspaces of the plans' sizes (grad
    input always re-packs the filter), and the coverage condition (grad weight co % 4; a forward of ci % 16 != 0 and
    a grad input of co % 16 != 0 run their fixed element-by-element plan, no K split: the forward needs no
    workspace, grad input only its packed filter) as workspaces and OMT_UNSUPPORTED, all without a GPU."""
    from omarchy_mac_torch import _lib
    L = _lib.L
    L.omt_conv_clear_plans()
    F, D, W = _lib.OMT_DIR_FWD_NHWC, _lib.OMT_DIR_DGRAD_NHWC, _lib.OMT_DIR_WGRAD_NHWC
    assert L.omt_conv_num_tiles(F) == L.omt_conv_num_tiles(D) == 9 and L.omt_conv_num_tiles(W) == 4

    def plan(d, g):
        p, c = _lib.ConvPlan(), ctypes.c_int32()
        assert L.omt_conv_get_plan(d, ctypes.byref(g), ctypes.byref(p), ctypes.byref(c)) == _lib.OMT_OK
        return p.tile, p.slices, c.value

    try:
        g = _lib.conv_geo(4, 48, 32, 6, 6, 3, 1, 1)      # 48 channels: the 32- and 64-deep K-blocks do not divide them
        for t in (6, 7, 8):
            assert L.omt_conv_set_plan(F, ctypes.byref(g), ctypes.byref(_lib.ConvPlan(t, 1))) == _lib.OMT_OK
            assert plan(F, g)[:2] == (5, 1)
        assert L.omt_conv_set_plan(F, ctypes.byref(g), ctypes.byref(_lib.ConvPlan(2, 3))) == _lib.OMT_OK
        assert plan(F, g) == (2, 3, 1)
        assert L.omt_conv_fwd_nhwc_workspace(ctypes.byref(g)) == 3 * 4 * 32 * 6 * 6 * 4
        assert L.omt_conv_plan_count() == 1   # the NCHW directions keep their own entries
        assert plan(_lib.OMT_DIR_FWD, g)[2] == 0
        pack = 32 * 48 * 9 * 4
        assert L.omt_conv_set_plan(D, ctypes.byref(g), ctypes.byref(_lib.ConvPlan(5, 1))) == _lib.OMT_OK
        assert L.omt_conv_dgrad_nhwc_workspace(ctypes.byref(g)) == pack
        assert L.omt_conv_set_plan(D, ctypes.byref(g), ctypes.byref(_lib.ConvPlan(5, 2))) == _lib.OMT_OK
        assert L.omt_conv_dgrad_nhwc_workspace(ctypes.byref(g)) == (pack + 255) // 256 * 256 + 2 * 4 * 48 * 6 * 6 * 4
        assert L.omt_conv_set_plan(W, ctypes.byref(g), ctypes.byref(_lib.ConvPlan(1, 2))) == _lib.OMT_OK
        assert L.omt_conv_wgrad_nhwc_workspace(ctypes.byref(g)) == 2 * 32 * 48 * 9 * 4
        for bad in (_lib.ConvPlan(9, 1), _lib.ConvPlan(-1, 1)):
            assert L.omt_conv_set_plan(F, ctypes.byref(g), ctypes.byref(bad)) == _lib.OMT_INVALID
        assert L.omt_conv_set_plan(W, ctypes.byref(g), ctypes.byref(_lib.ConvPlan(4, 1))) == _lib.OMT_INVALID
        # coverage: no workspace and OMT_UNSUPPORTED before anything is launched (pointers are never touched)
        odd = _lib.conv_geo(2, 6, 18, 8, 8, 3, 1, 1)
        assert L.omt_conv_fwd_nhwc_workspace(ctypes.byref(odd)) == 0
        assert L.omt_conv_wgrad_nhwc_workspace(ctypes.byref(odd)) == 0
        assert L.omt_conv_dgrad_nhwc_workspace(ctypes.byref(odd)) == 18 * 6 * 9 * 4  # the packed filter alone
        fake = ctypes.c_void_p(16)
        assert L.omt_conv_wgrad_nhwc(ctypes.byref(odd), fake, fake, fake, None, 0, None) == _lib.OMT_UNSUPPORTED
        assert L.omt_conv_fwd_nhwc(ctypes.byref(g), None, fake, None, 0, fake, None, 0, None) == _lib.OMT_INVALID
    finally:
        L.omt_conv_clear_plans()

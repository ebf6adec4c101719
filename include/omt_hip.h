/*
 * omt_hip.h -- C ABI of libomt_hip.so, the MI355X (gfx950) implementation of omarchy-mac-torch's convolution hot
 * path: implicit-GEMM conv forward / grad-input / grad-weight on fp32 MFMA, bias grad, depthwise, BatchNorm
 * (train / eval / backward, optional fused ReLU), max / average / adaptive-average pooling, and the device memory
 * and stream services the operator layer needs.
 *
 * Conventions
 *  - Tensors are dense NCHW float32 device pointers (weights [co][ci][ks][ks]); the caller makes inputs contiguous.
 *    Pointers and workspaces need 4-byte alignment only; 16-byte-aligned ones take the vector paths (direct-to-LDS
 *    filter loads, float4 epilogue stores).
 *  - Every compute entry point is asynchronous on `stream` (a hipStream_t; NULL = the HIP null stream, as in the
 *    HIP runtime API) and returns an omt_status. OMT_UNSUPPORTED means "this geometry is not covered" (the operator layer then records a
 *    fallback, as the reference's NEED() does); any other non-zero status carries a message in omt_last_error().
 *  - Entry points that need scratch memory take a caller-provided workspace; its size comes from the matching
 *    *_workspace() query. The library never frees or retains caller pointers.
 *  - Dense convolutions whose input or output reaches 2 GiB run as consecutive batch chunks below 2 GiB (the kernels'
 *    offsets are 32-bit); plan and tuning calls on such a geometry act on its first chunk's. One image or a filter of
 *    2 GiB or more is OMT_UNSUPPORTED.
 *  - Not thread-safe per stream: the caller serializes calls that share a stream (the reference serializes every op
 *    behind one recursive mutex, csrc/omt.h:62-64).
 *
 * Each declaration names the reference interface it replaces (file:line in the omarchy-mac-torch sources).
 */
#ifndef OMT_HIP_H
#define OMT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum omt_status {
  OMT_OK = 0,
  OMT_UNSUPPORTED = 1,  /* not covered: the caller falls back (reference: NEED() -> Unsupported, csrc/omt.h:168-176) */
  OMT_OOM = 2,          /* device allocation failed after emptying the cache (csrc/runtime.cpp:220-225) */
  OMT_DEVICE_ERROR = 3, /* a HIP runtime error (reference: uncaptured wgpu error, csrc/runtime.cpp:60-81) */
  OMT_INVALID = 4       /* bad arguments (shape mismatch, null pointer, workspace too small) */
} omt_status;

/* Convolution geometry: output size oh = (ih + 2*pad - ks) / stride + 1. Replaces Geo (csrc/omt.h:224-229). */
typedef struct omt_conv_geo {
  int64_t n, ci, co, ih, iw, oh, ow, ks, stride, pad;
} omt_conv_geo;

/* conv kinds, as conv_kind() classifies them (csrc/conv.cpp:167-177) */
enum { OMT_CONV_NONE = 0, OMT_CONV_DENSE = 1, OMT_CONV_DW = 2, OMT_CONV_DWG = 3 };

/* forward epilogue bits (omarchy_mac_torch/gemm.py:38-39) */
enum { OMT_EPI_BIAS = 1u, OMT_EPI_RELU = 2u };

/* GEMM directions of a dense convolution, the first field of a plan-cache key (the reference's GEMM kinds 0, 1, 2:
 * omarchy_mac_torch/gemm.py:6-8), and the same three over channels-last tensors (omt_conv_*_nhwc) */
enum {
  OMT_DIR_FWD = 0,
  OMT_DIR_DGRAD = 1,
  OMT_DIR_WGRAD = 2,
  OMT_DIR_FWD_NHWC = 3,
  OMT_DIR_DGRAD_NHWC = 4,
  OMT_DIR_WGRAD_NHWC = 5
};

/* A dense convolution's launch plan: tile index (into the direction's tile table, omt_conv_num_tiles) and number of
 * K slices (split K; rounded to whole K-blocks per slice). Replaces ConvPlan's tile and split-K multiplier
 * (csrc/omt.h:230-236). */
typedef struct omt_conv_plan {
  int32_t tile, slices;
} omt_conv_plan;

/* ---- library, errors, geometry ---------------------------------------------------------------------------- */

/* Message of the last non-OK status returned on this thread ("" if none). */
const char* omt_last_error(void);
/* ABI version (bumped on any signature change) and the HIP runtime version the library was built against.
 * Replaces built_with_torch (csrc/module.cpp:59) as the build guard. */
int omt_abi_version(void);
int omt_hip_runtime_version(void);
/* Fills g; replaces conv_geo (csrc/conv.cpp:19-21). */
void omt_conv_geo_init(omt_conv_geo* g, int64_t n, int64_t ci, int64_t co, int64_t ih, int64_t iw, int64_t ks,
                       int64_t stride, int64_t pad);
/* Replaces conv_kind (csrc/conv.cpp:167-177): returns OMT_CONV_*. x_c = input channels, w_o = weight rows. */
int omt_conv_kind(int64_t x_c, int64_t w_o, int64_t kh, int64_t kw, int64_t sh, int64_t sw, int64_t ph, int64_t pw,
                  int64_t dh, int64_t dw, int transposed, int64_t groups);

/* ---- device memory and streams (replace the wgpu buffer pool and recorder, csrc/runtime.cpp:177-249, 451-527) --- */

/* Caching allocator with size classes. Replaces alloc_buf/free_buf (csrc/runtime.cpp:205-231) and the PrivateUse1
 * Allocator (csrc/device.cpp:18-30). A block belongs to the stream it is allocated on (omt_malloc: the HIP null
 * stream); once freed it is handed out again only to allocations on that stream, so reuse is ordered after every
 * earlier use there. Work on other streams that uses a block must be declared with omt_record_stream (as torch's
 * Tensor.record_stream): freeing such a block records an event on each of those streams, and the block is reused only
 * after all of them have completed. */
int omt_malloc(void** ptr, size_t bytes);
int omt_malloc_on(void** ptr, size_t bytes, void* stream);
int omt_record_stream(void* ptr, void* stream); /* replaces the guard's recordDataPtrOnStream (csrc/device.cpp) */
int omt_free(void* ptr);
int omt_empty_cache(void);                 /* csrc/runtime.cpp:233-240 (empty_cache) */
size_t omt_memory_allocated(void);         /* csrc/runtime.cpp:242 */
size_t omt_memory_reserved(void);          /* csrc/runtime.cpp:243 */
/* Caps the bytes the allocator may hold (0 = no cap); exceeding it behaves as an out-of-memory (OMT_OOM). */
void omt_set_memory_limit(size_t bytes);
/* A non-blocking stream owned by the library (created on first use), for callers without a stream of their own. */
void* omt_default_stream(void);
/* kind: 0 host->device, 1 device->host, 2 device->device. Asynchronous on stream (device->host: synchronous).
 * Replaces upload/download_bytes and copy_dev (csrc/runtime.cpp:614-676). */
int omt_memcpy(void* dst, const void* src, size_t bytes, int kind, void* stream);
/* Zeroes `bytes` at dst on `stream` with a kernel (not a memset node: safe inside a captured HIP graph). */
int omt_memset_zero(void* dst, size_t bytes, void* stream);

/* Graph pools: memory that a captured HIP graph keeps for its replays. No counterpart in the reference, whose command
 * recorder batches submissions instead (csrc/runtime.cpp:451-518); here a captured step is replayed as one graph.
 * Between omt_graph_pool_begin(id) and omt_graph_pool_end() every omt_malloc, from any thread, is served from pool
 * id, and that pool's blocks return to it (never to the general cache) when freed. omt_graph_pool_release hands
 * them back to the general cache; call it only once no graph that uses them can be replayed (it synchronizes the
 * device). One pool receives at a time. omt_graph_pool_create returns the new pool's id (> 0). */
int omt_graph_pool_create(void);
int omt_graph_pool_begin(int id);
int omt_graph_pool_end(void);
int omt_graph_pool_release(int id);
int omt_stream_sync(void* stream);         /* replaces sync_all (csrc/runtime.cpp:520-527) */
/* Events (replace the submission-index events of the device guard, csrc/device.cpp:124-161). */
int omt_event_create(void** ev);
int omt_event_destroy(void* ev);
int omt_event_record(void* ev, void* stream);
int omt_event_query(void* ev);             /* 1 = complete, 0 = pending, <0 = error */
int omt_event_sync(void* ev);
int omt_event_elapsed_ms(void* start, void* end, float* ms);

/* ---- per-kernel launch counts and timings (replace kcount / ktime, kernel_counts / kernel_times /
 * debug_time_kernels: csrc/runtime.cpp:570-610, csrc/module.cpp:30-33) ---------------------------------------------
 * Every launch is counted under its kernel's name. With timing on, each launch is followed by a device
 * synchronization and the wall time since the previous one is added to the kernel: a debug measurement that
 * serializes the program (not for code under stream capture). omt_kernel_stat_count merges the counters by name into a
 * snapshot (name order) and returns its size; omt_kernel_stat_entry reads entry i of it (the name stays valid until the
 * next omt_kernel_stat_count or reset). omt_kernel_stats_reset zeroes the launch counts and / or the times (bits). */
enum { OMT_KSTAT_LAUNCHES = 1, OMT_KSTAT_TIMES = 2 };
void omt_set_kernel_timing(int on);
void omt_kernel_stats_reset(int what);
int omt_kernel_stat_count(void);
int omt_kernel_stat_entry(int i, const char** name, int64_t* launches, double* ms);

/* ---- dense convolution (implicit GEMM on fp32 MFMA) ------------------------------------------------------- */

/* Forward: y[n][co][oh][ow] = sum_{ci,ky,kx} x[n][ci][oy*s+ky-p][ox*s+kx-p] * w[co][ci][ky][kx], then
 * + bias[co] (epilogue & OMT_EPI_BIAS) and ReLU (epilogue & OMT_EPI_RELU).
 * bn_mean/var/gamma/beta non-NULL (all four): the input is first mapped through the previous layer's eval BatchNorm
 * + ReLU, max((x - mean[ci]) * rsqrt(var[ci] + eps) * gamma[ci] + beta[ci], 0), on in-bounds taps only (padding
 * stays zero). Replaces gemm_forward (csrc/conv.cpp:70-77) with kinds 0 and 3 (omarchy_mac_torch/gemm.py:25-42,
 * 139-141). Dense means: ks 1..11, stride 1..4, 0 <= pad <= ks. The workspace (omt_conv_fwd_workspace bytes, possibly 0,
 * with or without the BN loader) holds the filter re-packed for the tap-major reduction order and, for layers with too
 * few output tiles to fill the GPU, the partial sums of a K split (summed in a fixed order: results are deterministic).
 * The grad-input workspace holds the stride-phase filters and, likewise, any K-split partials. */
size_t omt_conv_fwd_workspace(const omt_conv_geo* g);
int omt_conv_fwd(const omt_conv_geo* g, const float* x, const float* w, const float* bias, unsigned epilogue,
                 const float* bn_mean, const float* bn_var, const float* bn_gamma, const float* bn_beta, float bn_eps,
                 float* y, void* workspace, size_t workspace_bytes, void* stream);
/* Forward without bias, epilogue or BN loader whose K-split partial sums stay unsummed, for a consumer that sums
 * them itself (omt_bn_train_fwd_parts): when the plan splits K into 2..max_slices slices, *partials points at the
 * [*slices][n][co][oh][ow] partials inside the workspace and y is not written; otherwise (no split, or more slices:
 * a consumer reading many slices per element is slower than the slice-sum launch) *slices = 1, *partials = NULL and
 * y holds the output, as from omt_conv_fwd. Same workspace as omt_conv_fwd. No counterpart in the reference, whose
 * convolution and BatchNorm are separate ops; the torch.compile backend fuses convolution -> training BatchNorm into
 * the pair, which saves the slice-sum launch. */
int omt_conv_fwd_unsummed(const omt_conv_geo* g, const float* x, const float* w, float* y, void* workspace,
                          size_t workspace_bytes, int max_slices, const float** partials, int* slices, void* stream);
/* Forward without bias, epilogue or BN loader that also writes the training-BatchNorm sums of its output: stats
 * [co][*groups][2] doubles, for each output channel and group of 32 or 64 consecutive output pixels (n-major, as in
 * y; *groups set by the call from the plan's tile) the sum of y and the sum of y^2 over the group, from the
 * accumulators in the epilogue, so omt_bn_train_fwd_stats normalizes y without reading it for its statistics.
 * stats_bytes >= omt_conv_fwd_stats_bytes(g); same workspace as omt_conv_fwd. A plan that splits K, or a batch that
 * would run in chunks, is OMT_UNSUPPORTED (nothing launched). No counterpart in the reference (see
 * omt_conv_fwd_unsummed); the torch.compile backend's convolution -> training BatchNorm op uses it. */
size_t omt_conv_fwd_stats_bytes(const omt_conv_geo* g);
int omt_conv_fwd_stats(const omt_conv_geo* g, const float* x, const float* w, float* y, double* stats,
                       size_t stats_bytes, int* groups, void* workspace, size_t workspace_bytes, void* stream);

/* Grad input: gx = conv_transpose(gy, w). Stride 1 is one GEMM over flipped, transposed weights; stride s > 1 is
 * s*s dense stride-phase GEMMs in one launch (phases no tap reaches write zeros). Replaces gemm_grad_input
 * (csrc/conv.cpp:78-101; kinds 1 and 5, omarchy_mac_torch/gemm.py:43-80). */
size_t omt_conv_dgrad_workspace(const omt_conv_geo* g);
int omt_conv_dgrad(const omt_conv_geo* g, const float* gy, const float* w, float* gx, void* workspace,
                   size_t workspace_bytes, void* stream);

/* Grad weight: gw[co][ci][ky][kx] = sum_{n,oy,ox} gy[n][co][oy][ox] * x[n][ci][oy*s+ky-p][ox*s+kx-p], split-K over
 * n*oh*ow with a deterministic in-order reduction of the partials. Replaces gemm_grad_weight (csrc/conv.cpp:102-114;
 * kind 2, omarchy_mac_torch/gemm.py:81-91; gemm_reduce.wgsl). */
size_t omt_conv_wgrad_workspace(const omt_conv_geo* g);
int omt_conv_wgrad(const omt_conv_geo* g, const float* x, const float* gy, float* gw, void* workspace,
                   size_t workspace_bytes, void* stream);

/* Grad weight for callers that cannot allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). No counterpart in the reference. Same plan, kernels and results as omt_conv_wgrad
 * (bit-identical), but the split-K partials live in a static device array of OMT_NOALLOC_SCRATCH_BYTES that the
 * library owns, one per GPU, held until the process ends; the call allocates nothing. A plan whose partials exceed
 * that size returns OMT_INVALID. Calls that overlap on one GPU (different streams without ordering between them) share
 * the array and race: order them. */
#define OMT_NOALLOC_SCRATCH_BYTES (64u << 20)
int omt_conv_wgrad_noalloc(const omt_conv_geo* g, const float* x, const float* gy, float* gw, void* stream);

/* Grad input and grad weight together: the dense branch of convolution_backward with both outputs requested
 * (csrc/conv.cpp:207-220 calls gemm_grad_input, then gemm_grad_weight). Results are those of omt_conv_dgrad and
 * omt_conv_wgrad (same plans, same summation order). When both plans use 64x64 tiles, the two GEMMs run in one launch,
 * and so do their split-K sums. Workspace: [grad-input workspace | 256-byte aligned grad-weight workspace]. */
size_t omt_conv_bwd_workspace(const omt_conv_geo* g);
int omt_conv_bwd(const omt_conv_geo* g, const float* x, const float* gy, const float* w, float* gx, float* gw,
                 void* workspace, size_t workspace_bytes, void* stream);

/* A deferred in-order slice sum: out[i] = sum over s = 0 .. slices-1, in order, of parts[s * n + i] (slices 0: none).
 * The sum omt_conv_bwd_parts leaves to its caller, which runs it in a later launch (omt_bn_bwd_parts) or alone
 * (omt_slice_sums). */
typedef struct omt_slice_sum {
  const float* parts;
  float* out;
  int64_t n;
  int slices;
} omt_slice_sum;

/* omt_conv_bwd without its slice-sum launch, for a consumer that sums the partials itself: when the grad-input plan
 * splits K into 2..max_gx_slices slices, *gx_parts points at its [*gx_slices][n][ci][ih][iw] partials (inside the
 * workspace) and gx is not written; otherwise gx holds grad input (summed here if split further) and *gx_slices = 1,
 * *gx_parts = NULL. When the grad-weight plan splits K, *gw_sum describes the in-order sum of its partials into gw,
 * which the caller must run (gw_sum->slices = 0 when gw was written). Partials and sums are those of omt_conv_bwd
 * (same plans, same order): the results, once summed, are bit-identical. Same workspace as omt_conv_bwd; a batch that
 * would run in chunks is OMT_UNSUPPORTED. No counterpart in the reference (its convolution backward and BatchNorm
 * backward are separate ops); the torch.compile backend's convolution backward -> BatchNorm backward op uses it. */
int omt_conv_bwd_parts(const omt_conv_geo* g, const float* x, const float* gy, const float* w, float* gx, float* gw,
                       void* workspace, size_t workspace_bytes, int max_gx_slices, const float** gx_parts,
                       int* gx_slices, omt_slice_sum* gw_sum, void* stream);
/* Runs count deferred slice sums (one launch each). */
int omt_slice_sums(const omt_slice_sum* sums, int count, void* stream);

/* ---- channels-last (NHWC) dense convolution ---------------------------------------------------------------------
 * The same convolutions over channels-last tensors: x / gx [n][ih][iw][ci], y / gy [n][oh][ow][co], and the filter
 * and its gradient [co][ks][ks][ci] -- the memory order of PyTorch's channels_last tensors of those shapes, read and
 * written without a layout change. The reference makes every input contiguous NCHW first (base0,
 * csrc/device.cpp:60-66, before gemm_forward / gemm_grad_input / gemm_grad_weight, csrc/conv.cpp:70-114); these
 * entry points replace that copy and those GEMMs for channels-last callers. Coverage beyond the dense geometry:
 * grad weight needs co % 4 == 0 (else OMT_UNSUPPORTED). A forward of ci % 16 != 0 (the 3-channel stem) and a grad
 * input of co % 16 != 0 gather element by element on one fixed plan, a grad weight of ci % 4 != 0 loads its columns
 * one by one: same LDS staging and MFMA order; those gathers are not tuned. Plans: directions OMT_DIR_FWD_NHWC,
 * OMT_DIR_DGRAD_NHWC, OMT_DIR_WGRAD_NHWC (tile indices below omt_conv_num_tiles of the direction). Bias and ReLU
 * epilogue bits as in omt_conv_fwd; no BN loader. */
size_t omt_conv_fwd_nhwc_workspace(const omt_conv_geo* g);
int omt_conv_fwd_nhwc(const omt_conv_geo* g, const float* x, const float* w, const float* bias, unsigned epilogue,
                      float* y, void* workspace, size_t workspace_bytes, void* stream);
size_t omt_conv_dgrad_nhwc_workspace(const omt_conv_geo* g);
int omt_conv_dgrad_nhwc(const omt_conv_geo* g, const float* gy, const float* w, float* gx, void* workspace,
                        size_t workspace_bytes, void* stream);
size_t omt_conv_wgrad_nhwc_workspace(const omt_conv_geo* g);
int omt_conv_wgrad_nhwc(const omt_conv_geo* g, const float* x, const float* gy, float* gw, void* workspace,
                        size_t workspace_bytes, void* stream);

/* ---- plan cache and tuning (replaces conv_plan / autotune / tune_dump / tune_load / tuned_plans,
 * csrc/conv.cpp:45-60, 116-155, 243-282) ---------------------------------------------------------------------
 * Every dense-conv call and workspace query resolves its plan from a process-wide cache keyed by (direction,
 * geometry); without an entry a cost model picks it. Changing an entry between a workspace query and the launch it
 * sized can make the launch fail with OMT_INVALID (workspace too small), never overrun the workspace.
 * omt_conv_autotune times the candidates (every tile of the first max_tiles, <= 0 meaning all, times a few K
 * splits) on scratch buffers, each as replays of a captured HIP graph of several calls on a private stream ordered
 * after `stream` (so a plan's extra launches cost what they cost in a replayed step), stores the fastest in the cache
 * and returns it in *best (may be NULL). It synchronizes `stream`, allocates through omt_malloc, and refuses
 * (OMT_UNSUPPORTED) while `stream` is capturing. The cache is in key order for omt_conv_plan_entry (i < omt_conv_plan_count()). */
int omt_conv_num_tiles(int dir);
int omt_conv_get_plan(int dir, const omt_conv_geo* g, omt_conv_plan* plan, int* cached);
int omt_conv_set_plan(int dir, const omt_conv_geo* g, const omt_conv_plan* plan); /* NULL plan: remove the entry */
int omt_conv_plan_count(void);
int omt_conv_plan_entry(int i, int* dir, omt_conv_geo* g, omt_conv_plan* plan);
void omt_conv_clear_plans(void);
int omt_conv_autotune(int dir, const omt_conv_geo* g, int max_tiles, void* stream, omt_conv_plan* best);
/* Tunes the grad-input and grad-weight plans together for omt_conv_bwd: the pair tuned one direction at a time
 * (omt_conv_autotune of each) against every pair of candidates that shares a launch, timed through omt_conv_bwd;
 * caches the fastest pair in both directions' entries. Same conditions as omt_conv_autotune. Extends the reference's
 * autotune (csrc/conv.cpp:116-155), which tunes each GEMM alone. */
int omt_conv_autotune_bwd(const omt_conv_geo* g, int max_tiles, void* stream, omt_conv_plan* dgrad_best,
                          omt_conv_plan* wgrad_best);

/* Bias grad gb[c] = sum_{n,hw} gy[n][c][hw]. Replaces csum_nchw (csrc/conv.cpp:232-235). */
int omt_bias_grad(int64_t n, int64_t c, int64_t hw, const float* gy, float* gb, void* stream);

/* BatchNorm folding (fold_bn, csrc/fused.cpp:34-40): scale = gamma / sqrt(var + eps) per output channel,
 * fw = cw * scale, fb = (cb - mean) * scale + beta (cb may be NULL). per_out = ci * ks * ks. */
int omt_fold_bn(int64_t co, int64_t per_out, const float* cw, const float* cb, const float* gamma, const float* beta,
                const float* mean, const float* var, float eps, float* fw, float* fb, void* stream);

/* ---- depthwise (groups = C) ------------------------------------------------------------------------------- */

/* Any ks <= 11, stride 1..4, 0 <= pad <= ks (g->ci == g->co == C). Replace dw_fwd / dwg_fwd / dw_fwd_bn,
 * dw_gin / dwg_gin, dw_gwt / dwg_gwt (csrc/conv.cpp:194-198, 222-229; csrc/plans.cpp:145-158). bias may be NULL;
 * bn_* as in omt_conv_fwd (dw_fwd_bn.wgsl). */
int omt_dw_fwd(const omt_conv_geo* g, const float* x, const float* w, const float* bias, const float* bn_mean,
               const float* bn_var, const float* bn_gamma, const float* bn_beta, float bn_eps, float* y, void* stream);
int omt_dw_dgrad(const omt_conv_geo* g, const float* gy, const float* w, float* gx, void* stream);
size_t omt_dw_wgrad_workspace(const omt_conv_geo* g);
int omt_dw_wgrad(const omt_conv_geo* g, const float* x, const float* gy, float* gw, void* workspace,
                 size_t workspace_bytes, void* stream);
/* The same over channels-last tensors: x / gx [n][ih][iw][C], y / gy [n][oh][ow][C], the filter and its gradient
 * [C][ks][ks] (a channels_last [C][1][ks][ks] filter's memory); n * ih * iw * C and n * oh * ow * C below 2^31. No
 * BN loader. Forward and grad input compute each output as the general NCHW kernels do (same taps, same order); grad
 * weight sums pixel slices into a workspace of omt_dw_wgrad_nhwc_workspace bytes, then the slices in order. No
 * counterpart in the reference, which makes every operand contiguous NCHW first (csrc/device.cpp:60-66). */
int omt_dw_fwd_nhwc(const omt_conv_geo* g, const float* x, const float* w, const float* bias, float* y, void* stream);
int omt_dw_dgrad_nhwc(const omt_conv_geo* g, const float* gy, const float* w, float* gx, void* stream);
size_t omt_dw_wgrad_nhwc_workspace(const omt_conv_geo* g);
int omt_dw_wgrad_nhwc(const omt_conv_geo* g, const float* x, const float* gy, float* gw, void* workspace,
                      size_t workspace_bytes, void* stream);

/* ---- BatchNorm (NCHW, affine) ----------------------------------------------------------------------------- */

/* The activation a BatchNorm entry point applies after the normalization (its `relu` / `act` argument): 0 none, 1 ReLU
 * (y = max(z, 0), NaN propagates), 2 hardswish (y = z * min(max(z + 3, 0), 6) / 6, PyTorch's definition). The
 * reference fuses ReLU only (omt::bn_relu_train, csrc/fused.cpp:68-84); hardswish follows MobileNetV3's BatchNorms. */
enum { OMT_ACT_NONE = 0, OMT_ACT_RELU = 1, OMT_ACT_HARDSWISH = 2 };

/* Training forward: per-channel biased mean / variance over n*hw, y = act((x - mean) * invstd * gamma + beta)
 * (relu: the activation, OMT_ACT_*; 1 = ReLU), save_mean / save_invstd written, and the running stats updated
 * rm' = rm + momentum*(mean - rm), rv' = rv + momentum*(var * m/(m-1) - rv) into new_rm / new_rv (which may alias
 * running_mean / running_var for the in-place native_batch_norm form, or be NULL to skip the update).
 * Replaces batch_norm_ training (csrc/nn.cpp:38-48) and omt::bn_relu_train (csrc/fused.cpp:68-84). */
size_t omt_bn_train_workspace(int64_t n, int64_t c, int64_t hw);
int omt_bn_train_fwd(int64_t n, int64_t c, int64_t hw, const float* x, const float* gamma, const float* beta,
                     const float* running_mean, const float* running_var, double momentum, double eps, int relu,
                     float* y, float* save_mean, float* save_invstd, float* new_rm, float* new_rv, void* workspace,
                     size_t workspace_bytes, void* stream);
/* The same with a residual added before the activation: y = act(bn(x) + residual) (residual [n][c][hw] like x, or
 * NULL), and z (NULL to skip) receiving bn(x) + residual, the activation's input (the hardswish backward reads it).
 * No counterpart in the reference, whose residual add and activations are separate ops; the torch.compile backend
 * fuses BatchNorm -> add -> ReLU (the end of a ResNet basic block) and BatchNorm -> hardswish into it. */
int omt_bn_train_fwd_res(int64_t n, int64_t c, int64_t hw, const float* x, const float* gamma, const float* beta,
                         const float* running_mean, const float* running_var, double momentum, double eps, int relu,
                         const float* residual, float* y, float* z, float* save_mean, float* save_invstd,
                         float* new_rm, float* new_rv, void* workspace, size_t workspace_bytes, void* stream);
/* omt_bn_train_fwd_res over a convolution's unsummed K-split partials (omt_conv_fwd_unsummed): x = the sum of the
 * `slices` partials of n*c*hw elements each, in slice order (the convolution's own slice sum, so x is bit-identical
 * to the summed convolution output), is written to x and normalized as by omt_bn_train_fwd_res. Channels of up to
 * 8192 elements run the sum, the statistics and the apply in one launch. parts must not overlap x, y or residual.
 * No counterpart in the reference (see omt_conv_fwd_unsummed). */
int omt_bn_train_fwd_parts(int64_t n, int64_t c, int64_t hw, const float* parts, int slices, float* x,
                           const float* gamma, const float* beta, const float* running_mean, const float* running_var,
                           double momentum, double eps, int relu, const float* residual, float* y, float* z,
                           float* save_mean, float* save_invstd, float* new_rm, float* new_rv, void* workspace,
                           size_t workspace_bytes, void* stream);

/* Training BatchNorm -> activation -> max pool in one pass over x [n][c][h][w]: y, save_mean, save_invstd and the
 * running statistics as omt_bn_train_fwd_res (no residual), and pooled / idx as omt_maxpool_fwd over y (window kh x kw,
 * stride, padding 2 pad <= window, no dilation, floor mode: [n][c][oh][ow]), bit-identical to those two calls. Channels
 * of up to 8192 elements take one launch (the pool read from LDS), larger ones two (statistics, then the apply with
 * the pool). Same workspace as omt_bn_train_fwd. Replaces native_batch_norm -> relu -> max_pool2d_with_indices (the
 * reference's BatchNorm + ReLU and pool are separate steps of its stack plans, csrc/plans.cpp:110-200; the
 * torch.compile backend and the fused stacks call this for the ResNet stem and PlainCNN's blocks). */
int omt_bn_train_fwd_pool(int64_t n, int64_t c, int64_t h, int64_t w, const float* x, const float* gamma,
                          const float* beta, const float* running_mean, const float* running_var, double momentum,
                          double eps, int act, float* y, float* save_mean, float* save_invstd, float* new_rm,
                          float* new_rv, int64_t kh, int64_t kw, int64_t sh, int64_t sw, int64_t ph, int64_t pw,
                          float* pooled, int64_t* idx, void* workspace, size_t workspace_bytes, void* stream);
/* omt_bn_train_fwd_res with the statistics from omt_conv_fwd_stats (stats [c][groups][2] over x = that call's y):
 * one launch reduces each channel's groups to a few partial sums (in a fixed order, into the workspace of
 * omt_bn_train_workspace's size), the next finalizes mean / invstd and the running statistics as it applies, so x is
 * read once. The variance is E[x^2] - E[x]^2 in double (the sums are unshifted). c * groups * 2 doubles must fit in
 * stats_bytes (OMT_INVALID otherwise, before any launch). No counterpart in the reference (see omt_conv_fwd_stats). */
int omt_bn_train_fwd_stats(int64_t n, int64_t c, int64_t hw, const float* x, const double* stats, int groups,
                           size_t stats_bytes, const float* gamma, const float* beta, const float* running_mean,
                           const float* running_var, double momentum, double eps, int relu, const float* residual,
                           float* y, float* z, float* save_mean, float* save_invstd, float* new_rm, float* new_rv,
                           void* workspace, size_t workspace_bytes, void* stream);
/* Eval forward: y = act((x - rm) * rsqrt(rv + eps) * gamma + beta) (relu: OMT_ACT_*). Replaces batch_norm_ eval
 * (csrc/nn.cpp:49-54) and bn_relu_rv.wgsl. */
int omt_bn_eval_fwd(int64_t n, int64_t c, int64_t hw, const float* x, const float* gamma, const float* beta,
                    const float* running_mean, const float* running_var, double eps, int relu, float* y,
                    void* stream);
/* Backward (training statistics): with gz = g (or g masked by relu_y > 0 when relu_y is non-NULL),
 * dgamma = sum gz * xhat, dbeta = sum gz, gx = gamma * invstd / m * (m * gz - dbeta - xhat * dgamma).
 * gx, dgamma, dbeta may each be NULL. Replaces batch_norm_backward_ (csrc/nn.cpp:60-78) and omt::bn_relu_backward
 * (csrc/fused.cpp:86-115). */
size_t omt_bn_bwd_workspace(int64_t n, int64_t c, int64_t hw);
int omt_bn_bwd(int64_t n, int64_t c, int64_t hw, const float* g, const float* x, const float* relu_y,
               const float* save_mean, const float* save_invstd, const float* gamma, float* gx, float* dgamma,
               float* dbeta, void* workspace, size_t workspace_bytes, void* stream);

/* The backward of BatchNorm -> activation: gz = g through the activation's gradient, act_in its operand (act
 * OMT_ACT_RELU: the ReLU's output, gz = g where act_in > 0, else 0, as omt_bn_bwd's relu_y; OMT_ACT_HARDSWISH: the
 * hardswish's input z, gz = g * hardswish'(z), 0 at and below -3, g at and above 3; OMT_ACT_NONE: act_in unused), then
 * the BatchNorm backward of gz, as omt_bn_bwd. Replaces hardswish_backward -> native_batch_norm_backward (the
 * reference runs them as two ops; it fuses ReLU only, csrc/fused.cpp:86-115). */
int omt_bn_bwd_act(int64_t n, int64_t c, int64_t hw, const float* g, const float* x, int act, const float* act_in,
                   const float* save_mean, const float* save_invstd, const float* gamma, float* gx, float* dgamma,
                   float* dbeta, void* workspace, size_t workspace_bytes, void* stream);

/* The same with a residual branch's gradient: gz = (g + g2) masked by relu_y > 0 (g2 may be NULL), written to gz for
 * the residual branch, and the BatchNorm backward of gz. No counterpart in the reference, whose ReLU backward, residual
 * add and BatchNorm backward are separate ops; the torch.compile backend fuses add -> threshold_backward ->
 * native_batch_norm_backward (the backward of a ResNet basic block's end) into it. gz must not be NULL. */
int omt_bn_bwd_res(int64_t n, int64_t c, int64_t hw, const float* g, const float* g2, const float* x,
                   const float* relu_y, const float* save_mean, const float* save_invstd, const float* gamma, float* gx,
                   float* dgamma, float* dbeta, float* gz, void* workspace, size_t workspace_bytes, void* stream);

/* The BatchNorm backward of omt_bn_bwd_act (gz NULL) or omt_bn_bwd_res (gz not NULL; g2 only then) with its incoming
 * gradient g given as `slices` consecutive arrays of n*c*hw floats, g = their sum in slice order (omt_conv_bwd_parts'
 * grad-input partials; slices 1: g itself), to which g2 is added after the sum. Runs the `count` (at most 2) deferred
 * slice sums in the same launch, on workgroups of their own. One launch: channels of n*hw <= 8192 elements only
 * (OMT_UNSUPPORTED above). With the partials of omt_conv_bwd_parts the results equal omt_conv_bwd followed by
 * omt_bn_bwd_act / omt_bn_bwd_res (the same additions in the same order). No counterpart in the reference (its
 * convolution backward and BatchNorm backward are separate ops); the torch.compile backend's fused convolution
 * backward -> BatchNorm backward op (omt::conv_bn_backward) uses it. No workspace. */
int omt_bn_bwd_parts(int64_t n, int64_t c, int64_t hw, const float* g_parts, int slices, const float* g2,
                     const float* x, int act, const float* act_in, const float* save_mean, const float* save_invstd,
                     const float* gamma, float* gx, float* dgamma, float* dbeta, float* gz, const omt_slice_sum* sums,
                     int count, void* stream);

/* Channels-last (NHWC) BatchNorm: x, y, z, residual, g, g2, act_in, gx, gz [n][hw][c] (the memory of a channels_last
 * [n][c][h][w] tensor). Same operations, arguments and statistics as omt_bn_train_fwd_res, omt_bn_eval_fwd and the
 * backward of omt_bn_bwd_act / omt_bn_bwd_res (g2 and gz may be NULL; gz, when set, receives the gradient through
 * the activation, for a residual branch; g_nchw: g alone is in NCHW order, read in place, as a channels-last
 * model's global-average-pool gradient arrives); the shifted float64 sums run in another order than the NCHW kernels', so
 * the results agree with theirs to float64 rounding. Three launches each way (partial sums, finalize, apply; the
 * backward with gx and gz NULL stops after the finalize); workspace of omt_bn_nhwc_workspace bytes. No counterpart
 * in the reference, which makes every operand contiguous NCHW (csrc/device.cpp:60-66) and runs batch_norm_ /
 * batch_norm_backward_ (csrc/nn.cpp:25-78) on that. */
size_t omt_bn_nhwc_workspace(int64_t n, int64_t c, int64_t hw);
int omt_bn_train_fwd_nhwc(int64_t n, int64_t c, int64_t hw, const float* x, const float* gamma, const float* beta,
                          const float* running_mean, const float* running_var, double momentum, double eps, int act,
                          const float* residual, float* y, float* z, float* save_mean, float* save_invstd,
                          float* new_rm, float* new_rv, void* workspace, size_t workspace_bytes, void* stream);
int omt_bn_eval_fwd_nhwc(int64_t n, int64_t c, int64_t hw, const float* x, const float* gamma, const float* beta,
                         const float* running_mean, const float* running_var, double eps, int act, float* y,
                         void* stream);
int omt_bn_bwd_nhwc(int64_t n, int64_t c, int64_t hw, const float* g, int g_nchw, const float* g2, const float* x,
                    int act, const float* act_in, const float* save_mean, const float* save_invstd, const float* gamma,
                    float* gx, float* dgamma, float* dbeta, float* gz, void* workspace, size_t workspace_bytes,
                    void* stream);

/* ---- pooling (planes = n * c) ----------------------------------------------------------------------------- */

/* Max pool, any window / stride / padding / dilation; idx = int64 flat position in the input plane, first maximum
 * wins ties, NaN propagates. Replaces max_pool2d_with_indices(_backward) (csrc/nn.cpp:157-178). */
int omt_maxpool_fwd(int64_t planes, int64_t ih, int64_t iw, int64_t oh, int64_t ow, int64_t kh, int64_t kw,
                    int64_t sh, int64_t sw, int64_t ph, int64_t pw, int64_t dh, int64_t dw, const float* x, float* y,
                    int64_t* idx, void* stream);
int omt_maxpool_bwd(int64_t planes, int64_t ih, int64_t iw, int64_t oh, int64_t ow, int64_t kh, int64_t kw,
                    int64_t sh, int64_t sw, int64_t ph, int64_t pw, int64_t dh, int64_t dw, const float* g,
                    const int64_t* idx, float* gx, void* stream);
/* Average pool with PyTorch's divisor rules (count_include_pad, divisor_override > 0). Replaces
 * avg_pool2d(_backward) (csrc/nn.cpp:180-204). */
int omt_avgpool_fwd(int64_t planes, int64_t ih, int64_t iw, int64_t oh, int64_t ow, int64_t kh, int64_t kw,
                    int64_t sh, int64_t sw, int64_t ph, int64_t pw, int count_include_pad, int64_t divisor_override,
                    const float* x, float* y, void* stream);
int omt_avgpool_bwd(int64_t planes, int64_t ih, int64_t iw, int64_t oh, int64_t ow, int64_t kh, int64_t kw,
                    int64_t sh, int64_t sw, int64_t ph, int64_t pw, int count_include_pad, int64_t divisor_override,
                    const float* g, float* gx, void* stream);
/* Adaptive average pool, bins [floor(o*in/out), ceil((o+1)*in/out)). Replaces _adaptive_avg_pool2d(_backward)
 * (csrc/nn.cpp:206-222). */
int omt_adapool_fwd(int64_t planes, int64_t ih, int64_t iw, int64_t oh, int64_t ow, const float* x, float* y,
                    void* stream);
int omt_adapool_bwd(int64_t planes, int64_t ih, int64_t iw, int64_t oh, int64_t ow, const float* g, float* gx,
                    void* stream);

/* Channels-last (NHWC) pools: x, gx [n][ih][iw][c], y, g, idx [n][oh][ow][c] (channels_last tensors' memory). The
 * same windows, rules and index meaning (flat y * iw + x within a plane) as the NCHW entry points above, and the same
 * visiting order, so the results are theirs transposed, bit for bit. n * ih * iw * c and n * oh * ow * c below 2^31
 * (OMT_UNSUPPORTED otherwise). No counterpart in the reference, which pools contiguous NCHW copies (csrc/nn.cpp:157-222,
 * csrc/device.cpp:60-66). */
int omt_maxpool_fwd_nhwc(int64_t n, int64_t c, int64_t ih, int64_t iw, int64_t oh, int64_t ow, int64_t kh, int64_t kw,
                         int64_t sh, int64_t sw, int64_t ph, int64_t pw, int64_t dh, int64_t dw, const float* x,
                         float* y, int64_t* idx, void* stream);
int omt_maxpool_bwd_nhwc(int64_t n, int64_t c, int64_t ih, int64_t iw, int64_t oh, int64_t ow, int64_t kh, int64_t kw,
                         int64_t sh, int64_t sw, int64_t ph, int64_t pw, int64_t dh, int64_t dw, const float* g,
                         const int64_t* idx, float* gx, void* stream);
int omt_avgpool_fwd_nhwc(int64_t n, int64_t c, int64_t ih, int64_t iw, int64_t oh, int64_t ow, int64_t kh, int64_t kw,
                         int64_t sh, int64_t sw, int64_t ph, int64_t pw, int count_include_pad,
                         int64_t divisor_override, const float* x, float* y, void* stream);
int omt_avgpool_bwd_nhwc(int64_t n, int64_t c, int64_t ih, int64_t iw, int64_t oh, int64_t ow, int64_t kh, int64_t kw,
                         int64_t sh, int64_t sw, int64_t ph, int64_t pw, int count_include_pad,
                         int64_t divisor_override, const float* g, float* gx, void* stream);
int omt_adapool_fwd_nhwc(int64_t n, int64_t c, int64_t ih, int64_t iw, int64_t oh, int64_t ow, const float* x,
                         float* y, void* stream);
int omt_adapool_bwd_nhwc(int64_t n, int64_t c, int64_t ih, int64_t iw, int64_t oh, int64_t ow, const float* g,
                         float* gx, void* stream);

/* ---- pointwise, reduction and loss ops of the training steps (outside the convolution path) ------------------------
 * Contiguous float32 operands. Replace the reference's general elementwise kernel and op table
 * (csrc/elementwise.cpp:79-112, 702-817), its softmax / log-softmax and NLL loss (csrc/reduce.cpp:128-202). */

/* out[i] = op(a[i], b[i], alpha); out may alias a or b (the in-place forms). Activations follow PyTorch's definitions:
 * relu(a) = max(a, 0) (NaN propagates); threshold_backward(grad a, input b) = b <= alpha ? 0 : a;
 * hardswish(a) = a * min(max(a + 3, 0), 6) / 6 and its gradient g * (a / 3 + 1/2) on (-3, 3) (0 at and below -3,
 * g at and above 3);
 * hardsigmoid(a) = min(max(a + 3, 0), 6) / 6 and its gradient g / 6 on (-3, 3) (0 elsewhere). */
enum {
  OMT_PW_ADD = 0,             /* a + alpha * b */
  OMT_PW_MUL = 1,             /* a * b */
  OMT_PW_RELU = 2,            /* relu(a) */
  OMT_PW_THRESHOLD_BWD = 3,   /* b <= alpha ? 0 : a */
  OMT_PW_HARDSWISH = 4,       /* hardswish(a) */
  OMT_PW_HARDSWISH_BWD = 5,   /* gradient a at input b */
  OMT_PW_HARDSIGMOID = 6,     /* hardsigmoid(a) */
  OMT_PW_HARDSIGMOID_BWD = 7, /* gradient a at input b */
  OMT_PW_SCALE = 8,           /* a * alpha */
  OMT_PW_FILL = 9,            /* alpha (a, b unused) */
  OMT_PW_ADD_SCALAR = 10      /* a + alpha */
};
int omt_pointwise(int op, int64_t n, const float* a, const float* b, float alpha, float* out, void* stream);
/* t += value for each of `count` small contiguous tensors (ptrs[i], numels[i] elements, at most
 * OMT_FOREACH_MAX_NUMEL each; host arrays) in one launch per 64 tensors: dtype OMT_DT_F32 adds fvalue, OMT_DT_I64 adds
 * ivalue. The optimizers' step counts and BatchNorm's batch counters. Replaces the reference's _foreach_* handling,
 * which loops the per-tensor add on the device (csrc/device.cpp:220-225). */
enum { OMT_DT_F32 = 0, OMT_DT_I64 = 1 };
#define OMT_FOREACH_MAX_NUMEL (1 << 16)
int omt_foreach_add_scalar(int count, void* const* ptrs, const int64_t* numels, int dtype, int64_t ivalue,
                           float fvalue, void* stream);
/* Squeeze-excite channel scale: y[p][i] = x[p][i] * scale[p] over `planes` planes (n * c) of hw elements. */
int omt_channel_scale(int64_t planes, int64_t hw, const float* x, const float* scale, float* y, void* stream);
/* y[p][i] = v[p] * scale: a per-plane value broadcast over its plane (the gradient of a plane mean). */
int omt_plane_broadcast(int64_t planes, int64_t hw, const float* v, float scale, float* y, void* stream);
/* y[p] = scale * sum_i x[p][i] (sum or mean over the last two dims of an NCHW tensor). */
int omt_plane_sum(int64_t planes, int64_t hw, const float* x, float scale, float* y, void* stream);
/* y[p] = scale * sum_i a[p][i] * b[p][i], each product rounded and the terms summed as omt_plane_sum sums (so equal to
 * omt_pointwise(OMT_PW_MUL) followed by omt_plane_sum): a squeeze-excite gate's gradient, sum over a plane of g * x, in
 * one launch. No counterpart in the reference (a multiply and a sum, csrc/elementwise.cpp, reduce.cpp). */
int omt_plane_dot(int64_t planes, int64_t hw, const float* a, const float* b, float scale, float* y, void* stream);
/* y[p][i] = g[p][i] * s[p] + v[p] * scale, each product rounded, then added (equal to omt_channel_scale,
 * omt_plane_broadcast and an add): the gradient reaching a squeeze-excite block's input through the gate and through
 * the plane mean, in one launch. No counterpart in the reference (three ops there). */
int omt_se_gate_bwd(int64_t planes, int64_t hw, const float* g, const float* s, const float* v, float scale, float* y,
                    void* stream);
/* The same over channels-last planes: g, y [n][hw][c], s, v [n][c]. */
int omt_se_gate_bwd_nhwc(int64_t n, int64_t c, int64_t hw, const float* g, const float* s, const float* v, float scale,
                         float* y, void* stream);
/* The same over channels-last planes: y[img][ch] = scale * sum_p x[img][p][ch], x [n][hw][c] (a channels_last
 * tensor's memory), y [n][c]; n <= 65535. No counterpart in the reference, which reduces contiguous NCHW copies
 * (csrc/reduce.cpp, csrc/device.cpp:60-66). */
int omt_plane_sum_nhwc(int64_t n, int64_t c, int64_t hw, const float* x, float scale, float* y, void* stream);
/* y[img][p][ch] = x[img][p][ch] * s[img][ch]: omt_channel_scale over channels-last planes (x, y [n][hw][c], s [n][c]).
 * No counterpart in the reference (see omt_plane_sum_nhwc). */
int omt_channel_scale_nhwc(int64_t n, int64_t c, int64_t hw, const float* x, const float* scale, float* y,
                           void* stream);
/* omt_pointwise over [n][c][hw] operands stored in different orders: each of a, b and out NCHW (flag 0) or
 * channels-last NHWC (flag 1); out[i] = op(a, b) at the same logical element. Unary and binary ops only (not
 * OMT_PW_FILL). For the one op per step where a channels-last model meets an NCHW gradient (a global average pool's
 * backward, broadcast over its planes, meeting the ReLU mask). No counterpart in the reference (its operands are
 * contiguous NCHW copies, csrc/device.cpp:60-66). */
int omt_pointwise_layouts(int op, int64_t n, int64_t c, int64_t hw, const float* a, int a_nhwc, const float* b,
                          int b_nhwc, float alpha, float* out, int out_nhwc, void* stream);
/* Row-wise log-softmax of x[rows][cols] and its gradient gx = g - exp(y) * sum_j g (y the forward's output). */
int omt_log_softmax_fwd(int64_t rows, int64_t cols, const float* x, float* y, void* stream);
int omt_log_softmax_bwd(int64_t rows, int64_t cols, const float* g, const float* y, float* gx, void* stream);
/* NLL loss over log-probabilities logp[rows][cols] and int64 targets, optional class weights, rows whose target is
 * ignore_index excluded. reduction 0 (none): out[rows]; 1 (mean): out[0] = sum / total weight; 2 (sum): out[0].
 * *total_weight receives the sum of the counted rows' weights (0 for reduction none). Backward: gx[r][t_r] =
 * -w[t_r] * g' with g' = g[0] / *total_weight (mean), g[0] (sum) or g[r] (none); every other element 0. */
int omt_nll_loss_fwd(int64_t rows, int64_t cols, const float* logp, const int64_t* target, const float* weight,
                     int64_t ignore_index, int reduction, float* out, float* total_weight, void* stream);
int omt_nll_loss_bwd(int64_t rows, int64_t cols, const float* g, const int64_t* target, const float* weight,
                     int64_t ignore_index, int reduction, const float* total_weight, float* gx, void* stream);

/* The squeeze-excite block's excitation MLP, per image n: h[n] = relu(W1 z[n] + b1), a2[n] = W2 h[n] + b2,
 * s[n] = hardsigmoid(a2[n]), z [n][c] the squeezed channels, W1 [r][c], b1 [r], W2 [c][r], b2 [c] (nn.Linear
 * layouts), c <= 2048, r <= 1024 (OMT_UNSUPPORTED otherwise); h [n][r] and a2 [n][c] are kept for the backward. Two
 * launches. The backward, from gs = dL/ds and the forward's z, h, a2: gz [n][c], gw1, gb1, gw2, gb2 (two launches;
 * workspace of omt_se_bwd_workspace bytes). Every sum runs in a fixed order. No counterpart in the reference, whose
 * squeeze-excite runs as linear -> relu -> linear -> hardsigmoid ops (csrc/linalg.cpp:25-79, elementwise.cpp); the
 * torch.compile backend's omt::se_mlp. */
size_t omt_se_bwd_workspace(int64_t n, int64_t c, int64_t r);
int omt_se_fwd(int64_t n, int64_t c, int64_t r, const float* z, const float* w1, const float* b1, const float* w2,
               const float* b2, float* s, float* h, float* a2, void* stream);
int omt_se_bwd(int64_t n, int64_t c, int64_t r, const float* gs, const float* z, const float* h, const float* a2,
               const float* w1, const float* w2, float* gz, float* gw1, float* gb1, float* gw2, float* gb2,
               void* workspace, size_t workspace_bytes, void* stream);

/* ---- fused optimizers (float32, contiguous parameters; many tensors per launch) -------------------------------- */

/* One parameter of an Adam / AdamW step: the step count (a float on the device) has already been incremented.
 * max_exp_avg_sq is read only with amsgrad; grad is written back (unscaled) only with grad_scale. */
typedef struct omt_adam_tensor {
  float* param;
  float* grad;
  float* exp_avg;
  float* exp_avg_sq;
  float* max_exp_avg_sq;
  const float* step;
  int64_t numel;
} omt_adam_tensor;
/* lr_dev (a float on the device) overrides lr when set; grad_scale divides the gradients, and found_inf == 1 on the
 * device skips the step (both optional, AMP). decoupled = AdamW. */
typedef struct omt_adam_params {
  float lr;
  const float* lr_dev;
  float beta1, beta2, weight_decay, eps;
  int amsgrad, maximize, decoupled;
  const float* grad_scale;
  const float* found_inf;
} omt_adam_params;
/* Replaces _fused_adam_ / _fused_adamw_ (csrc/optim.cpp:30-67): p -= lr/(1-b1^t) m / (sqrt(v)/sqrt(1-b2^t) + eps). */
int omt_fused_adam(const omt_adam_params* params, const omt_adam_tensor* tensors, int count, void* stream);

/* One parameter of an SGD step; momentum_buffer is read and written only when momentum != 0. */
typedef struct omt_sgd_tensor {
  float* param;
  float* grad;
  float* momentum_buffer;
  int64_t numel;
} omt_sgd_tensor;
/* first_step: the momentum buffers start as the (decayed) gradient. lr_dev, grad_scale, found_inf as for Adam. */
typedef struct omt_sgd_params {
  float lr;
  const float* lr_dev;
  float momentum, dampening, weight_decay;
  int nesterov, maximize, first_step;
  const float* grad_scale;
  const float* found_inf;
} omt_sgd_params;
/* Replaces _fused_sgd_ (csrc/optim.cpp:12-28). */
int omt_fused_sgd(const omt_sgd_params* params, const omt_sgd_tensor* tensors, int count, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* OMT_HIP_H */

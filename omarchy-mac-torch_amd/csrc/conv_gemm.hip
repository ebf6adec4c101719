// Dense convolution as im2col-free implicit GEMM on gfx950 fp32 MFMA (v_mfma_f32_16x16x4_f32).
//
// Forward and grad-input share one kernel, conv_gather_kernel: C[p][q] = sum_k Wt[p][k] * X(k, q), where p is an
// output channel, q = (n, oy, ox) an output pixel and k = (c, ky, kx) a tap; X(k, q) gathers the source image at
// (oy*S + ky - PH, ox*S + kx - PW), zero outside. Grad input is the same contraction over gy with re-packed weights,
// split into stride phases (reference: gemm_grad_input, csrc/conv.cpp:78-101, and the phase loader,
// omarchy_mac_torch/gemm.py:60-80): for phase (py, px) of stride s,
//   gx[n, ci, py + s*i, px + s*j] = sum_{co, a < jy, b < jx} gy[n, co, i + qy - a, j + qx - b] * w[co, ci, ky0 + s*a, kx0 + s*b]
// with ky0 = (py + pad) mod s, jy = ceil((ks - ky0) / s), qy = (py + pad - ky0) / s. Writing a' = jy - 1 - a turns
// each phase into a stride-1 gather with window jy x jx and padding jy - 1 - qy over weights
// W'[ci][co][a'][b'] = w[co][ci][ky0 + s*(jy-1-a')][kx0 + s*(jx-1-b')]. Stride 1 is the single phase (0, 0), whose
// W' is the flipped, transposed filter. All phases run in one launch (grid z).
//
// Grad weight, conv_wgrad_kernel: C[co][q'] = sum_k gy[k][co] * X(k, q') with k = (n, oy, ox) the reduction over
// output pixels and q' = (ci, ky, kx), split over k into grid-z slices whose partials are summed in slice order by
// split_reduce_kernel (reference: gemm_grad_weight + gemm_reduce, csrc/conv.cpp:102-114).
//
// Split K. A layer with too few output tiles to fill the chip (late, low-resolution layers) splits its reduction into
// grid-z slices of whole K-blocks; each slice writes its raw partial tile into a [slices][N][P][YH][YW] workspace and
// gather_reduce_kernel sums the slices in slice order (deterministic) and applies the bias / ReLU epilogue.
//
// Tiling: a 256-thread workgroup computes a BP x BQ tile of C as 4 waves, each a WP x WQ block of 16x16 MFMA tiles,
// with the operands staged through LDS. MFMA 16x16x4 lane layout: lane l supplies A[l%16][l/16] and B[l/16][l%16];
// the accumulator holds D[4*(l/16) + r][l%16] in element r. Because the reduction order inside a K-block is free,
// lane group g = l/16 supplies K-index g*(BK/4) + s at MFMA step s. Both operands sit in LDS as rows of K
// (k contiguous, pitch BK + 4 floats), so one ds_read_b128 hands a lane four consecutive steps' operands, and the
// pitch (5 or 17 x 16 bytes) puts the eight rows one b128 access phase touches on distinct banks.
//
// Operand loads are raw buffer loads: an offset at or beyond the buffer's byte size returns 0 in hardware, so taps in
// the zero padding, K-tails and pixels past the end are all loaded branch-free with an out-of-range offset (kOOB),
// and no computed offset can reach memory outside the tensor. Tensors read this way must stay below 2 GiB.
//
// Reduction order. With C a multiple of the K-block, K is ordered tap-major, k = (ky, kx, c), over weights re-packed
// to [co][ky][kx][ci] (tap-major mode). A K-block (or a wave's run of tap columns in wgrad) then shares one tap: one
// bounds test per lane per block yields the vector offset, and each element is a bare buffer load whose channel
// offset c*H*W travels in the scalar offset. Other C use the channel-major order k = (c, ky, kx) of the reference's
// index maps (generic mode) with a per-element bounds test.
#include <algorithm>
#include <map>
#include <mutex>
#include <tuple>
#include <type_traits>
#include <vector>

#include "omt_internal.h"
#include "slice_sum.h"
#include "lds_dma.h"
#include "tile_map.h"

namespace omt {

constexpr int kMaxPhases = 16;

__device__ __forceinline__ TileId xcd_block_tile(int gm) {
  return xcd_tile((int)(blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z)), (int)gridDim.x,
                  (int)gridDim.y, (int)gridDim.z, gm);
}
// Tile rows per group: 8 output-channel (gather) or grad-weight row (wgrad) tiles.
constexpr int kTileGroup = 8;


__device__ __forceinline__ float f4get(const float4& v, int s) { return s == 0 ? v.x : s == 1 ? v.y : s == 2 ? v.z : v.w; }

// Gather K orders: channel-major (generic), tap-major over a re-packed filter, tap-major reading the filter in place
// (grad weight uses the first two), tap-major over a channels-last (NHWC) source, whose K-blocks of channels are
// contiguous runs of each pixel, and tap-major over a channels-last source of too few channels for whole K-blocks
// (kNhwcNarrow: the ResNet stem's 3; element by element like the generic order, k = (ky, kx, c), which is also the
// memory order of a channels-last filter).
enum { kGeneric = 0, kTapMajor = 1, kTapInPlace = 2, kNhwc = 3, kNhwcNarrow = 4, kPix4 = 5 };

struct Phase {
  int KH, KW, S, PH, PW;  // gather window, stride and (signed) padding
  int OH, OW;             // output grid of this phase; q = (n, oy, ox) decomposes over it
  int K, Q;               // C * KH * KW, n * OH * OW
  int os, oy0, ox0;       // output scatter: y row = oy * os + oy0, column = ox * os + ox0
  int woff;               // offset of this phase's [P][K] weights (floats)
  int ky0, kx0;           // grad input read straight from w: the phase's first filter tap
  FastDiv div_ohw, div_ow, div_kk, div_kw;
};

struct GatherArgs {
  const float* x;  // gather source [N][C][H][W]
  const float* w;  // weights, per phase [P][K] at woff
  const float* bias;
  const float *bn_mean, *bn_var, *bn_gamma, *bn_beta;  // previous layer's eval BN + ReLU on the source, or null
  float bn_eps;
  int relu;
  float* y;  // [N][P][YH][YW]
  uint32_t x_bytes, w_bytes;
  int C, H, W, P, YH, YW;
  FastDiv div_c;
  int nphase;
  int kslice;            // K elements per grid-z slice (a multiple of the K-block)
  int tpw;               // conv1x1_stream_kernel: pixel tiles per workgroup
  int rows;              // row epilogue: one phase written in place, no split K, OH OW % 4 == 0, y 16-byte aligned
  int d2s, d2s_ci;       // grad input as one super-pixel GEMM: its stride (0: off) and the grad-input channels;
  int d2s_h, d2s_w;      //   the grad-input image (YH x YW is then the super-pixel grid, as its K-split partials)
  int wdirect;           // grad input, channel-major: A[ci][(co, a', b')] read from w[co][ci][ks][ks] (no re-pack)
  int ks, s;             //   the filter size and stride for that read (and for wplace 2)
  int wplace;            // tap-major order with the filter read in place: 1 forward, A[co][(tap, ci)] from
                         //   w[co][ci][ky][kx]; 2 grad input, A[ci][(a', b', co)] from w[co][ci][ky][kx] through the
                         //   phase's flip map (ky = ky0 + s (KH - 1 - a')); 0 the [P][K] filter at w (re-packed)
  uint32_t w_rowst, w_cst;  // wplace: bytes between A rows and between consecutive channels of one tap
  float* part;           // split K: raw partials [slices][N][P][YH][YW], else null (epilogue writes y)
  int64_t part_stride;   // elements per slice
  int nhwc;              // channels-last source [N][H][W][C] and output [N][YH][YW][P] (partials likewise)
  int vec_out;           // nhwc: P % 4 == 0 and y (and the partials) 16-byte aligned: float4 stores of four channels
  double* stats;         // forward, one phase, no split K, bias or ReLU: training-BN sums of y (epilogue_stats)
  int stats_groups;      //   over column groups of WQ GEMM columns: [P][stats_groups][2]
  Phase ph[kMaxPhases];
};

// LDS floats of a gather tile: both operands double-buffered, rows of BK + 4.
template <int BP, int BQ, int BK>
constexpr int gather_lds_floats() { return 2 * (BP + BQ) * (BK + 4); }

// The bias of a lane's accumulator rows (channel p0 + wp WP + 16 i + 4 (lane / 16) + r4), loaded together before the
// epilogue: a bias load per element inside the stores' bounds branches compiled to one `s_waitcnt vmcnt(0)` per
// element, each draining every load and store in flight. 0 where there is no bias or the channel is past P.
template <int TI, int WP>
__device__ __forceinline__ void epilogue_bias(const GatherArgs& a, int p0, int wp, int lane, float (&bv)[TI][4]) {
  const int pb = p0 + wp * WP + 4 * (lane >> 4);
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      const int p = pb + 16 * i + r4;
      bv[i][r4] = a.bias && p < a.P ? a.bias[p] : 0.f;
    }
}

// Training-BatchNorm statistics of a forward's output (a.stats; one phase, no split K, no bias or ReLU): for output
// channel p and column group cg (the WQ consecutive GEMM columns of one wave of one tile: cg = (q0 + wq WQ) / WQ),
// the double sums of y and y^2 over the group's valid columns go to a.stats[(p groups + cg) 2 + {0, 1}] (each
// channel's groups contiguous, for the BatchNorm's per-channel sum). Each lane sums its
// TJ columns of a row (the squares of floats are exact in double), the 16 lanes of its lane group (the MFMA tile's
// columns) combine by DPP steps within the row, in a fixed order, and the group's first lane writes the pair: every
// (cg, p) pair has one writer, so the result does not depend on scheduling. Every lane of the wave takes part.
template <int TI, int TJ, int WP, int WQ>
__device__ __forceinline__ void epilogue_stats(const GatherArgs& a, const Phase& ph, const omt_f32x4 (&acc)[TI][TJ],
                                               int q0, int p0, int wp, int wq, int lane) {
  const int grp = lane >> 4, cg = q0 / WQ + wq;
  bool qok[TJ];
#pragma unroll
  for (int j = 0; j < TJ; ++j) qok[j] = q0 + wq * WQ + 16 * j + (lane & 15) < ph.Q;
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      double s1 = 0.0, s2 = 0.0;
#pragma unroll
      for (int j = 0; j < TJ; ++j) {
        const double v = qok[j] ? (double)acc[i][j][r4] : 0.0;
        s1 += v;
        s2 += v * v;
      }
      s1 = row16_sum(s1);
      s2 = row16_sum(s2);
      const int p = p0 + wp * WP + 16 * i + 4 * grp + r4;
      if ((lane & 15) == 0 && p < a.P && cg < a.stats_groups) {  // a wave past the last column writes nothing
        typedef double f64x2 __attribute__((ext_vector_type(2)));
        *reinterpret_cast<f64x2*>(a.stats + ((int64_t)p * a.stats_groups + cg) * 2) = f64x2{s1, s2};
      }
    }
}

// Gather epilogue: bias, ReLU, scatter to NCHW (phase outputs land on their stride grid); split K: raw partials of
// slice zs. acc[i][j] is the wave's 16x16 MFMA tile (i, j): element r4 of lane l is row 4 (l / 16) + r4, column l % 16.
template <int TI, int TJ, int WP, int WQ, bool BIAS>
__device__ __forceinline__ void gather_epilogue_b(const GatherArgs& a, const Phase& ph, const omt_f32x4 (&acc)[TI][TJ],
                                                  int q0, int p0, int wp, int wq, int lane, int zs,
                                                  const float (&bv)[TI][4]) {
  const int P = a.P, grp = lane >> 4;
  const int64_t yhw = (int64_t)a.YH * a.YW;
  float* const ydst = a.part ? a.part + zs * a.part_stride : a.y;
  const uint32_t ohw = (uint32_t)(ph.OH * ph.OW);
#pragma unroll
  for (int j = 0; j < TJ; ++j) {
    const int q = q0 + wq * WQ + 16 * j + (lane & 15);
    if (q >= ph.Q) continue;
    const uint32_t n = fdiv((uint32_t)q, ph.div_ohw), r = (uint32_t)q - n * ohw;
    const uint32_t oy = fdiv(r, ph.div_ow), ox = r - oy * (uint32_t)ph.OW;
    float* yb = ydst + (int64_t)n * P * yhw + (int64_t)((int)oy * ph.os + ph.oy0) * a.YW + (int)ox * ph.os + ph.ox0;
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int p = p0 + wp * WP + 16 * i + 4 * grp + r4;
        if (p < P) {
          float v = acc[i][j][r4];
          if (!a.part) {
            if (BIAS) v += bv[i][r4];
            if (a.relu) v = fmaxf(v, 0.f);
          }
          yb[(int64_t)p * yhw] = v;
        }
      }
  }
}
// The epilogues branch once on the bias: with one, its loads are issued together and waited for once; without, no
// load is pending at the stores (a merged path would wait for every load and store in flight at each tile's end).
template <int TI, int TJ, int WP, int WQ>
__device__ __forceinline__ void gather_epilogue(const GatherArgs& a, const Phase& ph, const omt_f32x4 (&acc)[TI][TJ],
                                                int q0, int p0, int wp, int wq, int lane, int zs) {
  float bv[TI][4];
  if (a.stats) epilogue_stats<TI, TJ, WP, WQ>(a, ph, acc, q0, p0, wp, wq, lane);
  if (a.bias && !a.part) {
    epilogue_bias<TI, WP>(a, p0, wp, lane, bv);
    gather_epilogue_b<TI, TJ, WP, WQ, true>(a, ph, acc, q0, p0, wp, wq, lane, zs, bv);
  } else {
    gather_epilogue_b<TI, TJ, WP, WQ, false>(a, ph, acc, q0, p0, wp, wq, lane, zs, bv);
  }
}

// Channels-last gather epilogue: output pixel (n, oy os + oy0, ox os + ox0) holds its P channels contiguously, so the
// four accumulator rows of a lane (channels 4 (l / 16) + r4 of one pixel) are one 16-byte store where a.vec_out holds.
template <int TI, int TJ, int WP, int WQ, bool BIAS>
__device__ __forceinline__ void gather_epilogue_nhwc_b(const GatherArgs& a, const Phase& ph,
                                                       const omt_f32x4 (&acc)[TI][TJ], int q0, int p0, int wp, int wq,
                                                       int lane, int zs, const float (&bv)[TI][4]) {
  const int P = a.P, grp = lane >> 4;
  float* const ydst = a.part ? a.part + zs * a.part_stride : a.y;
  const uint32_t ohw = (uint32_t)(ph.OH * ph.OW);
#pragma unroll
  for (int j = 0; j < TJ; ++j) {
    const int q = q0 + wq * WQ + 16 * j + (lane & 15);
    if (q >= ph.Q) continue;
    const uint32_t n = fdiv((uint32_t)q, ph.div_ohw), r = (uint32_t)q - n * ohw;
    const uint32_t oy = fdiv(r, ph.div_ow), ox = r - oy * (uint32_t)ph.OW;
    float* const yb =
        ydst + (((int64_t)n * a.YH + (int)oy * ph.os + ph.oy0) * a.YW + (int)ox * ph.os + ph.ox0) * P;
#pragma unroll
    for (int i = 0; i < TI; ++i) {
      const int p = p0 + wp * WP + 16 * i + 4 * grp;
      float v[4];
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        v[r4] = acc[i][j][r4];
        if (!a.part) {
          if (BIAS && p + r4 < P) v[r4] += bv[i][r4];
          if (a.relu) v[r4] = fmaxf(v[r4], 0.f);
        }
      }
      if (a.vec_out) {
        if (p < P) *reinterpret_cast<float4*>(yb + p) = make_float4(v[0], v[1], v[2], v[3]);
      } else {
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4)
          if (p + r4 < P) yb[p + r4] = v[r4];
      }
    }
  }
}
template <int TI, int TJ, int WP, int WQ>
__device__ __forceinline__ void gather_epilogue_nhwc(const GatherArgs& a, const Phase& ph,
                                                     const omt_f32x4 (&acc)[TI][TJ], int q0, int p0, int wp, int wq,
                                                     int lane, int zs) {
  float bv[TI][4];
  if (a.bias && !a.part) {
    epilogue_bias<TI, WP>(a, p0, wp, lane, bv);
    gather_epilogue_nhwc_b<TI, TJ, WP, WQ, true>(a, ph, acc, q0, p0, wp, wq, lane, zs, bv);
  } else {
    gather_epilogue_nhwc_b<TI, TJ, WP, WQ, false>(a, ph, acc, q0, p0, wp, wq, lane, zs, bv);
  }
}

// Grad input as one super-pixel GEMM (a.d2s = stride s > 1, a.d2s_ci = C channels): GEMM row p = (py s + px) C + c
// at pixel (n, i, j) of the ceil(H / s) x ceil(W / s) grid is grad input (n, c, s i + py, s j + px), stored where it
// lies inside the image (y: [N][C][d2s_h][d2s_w]). Split over K, the raw partials take the gather epilogue's
// [N][rows][grid] layout and the slice sum scatters.
template <int TI, int TJ, int WP, int WQ>
__device__ __forceinline__ void d2s_epilogue(const GatherArgs& a, const Phase& ph, const omt_f32x4 (&acc)[TI][TJ],
                                             int q0, int p0, int wp, int wq, int lane) {
  const int S = a.d2s, CI = a.d2s_ci, grp = lane >> 4, IH = a.d2s_h, IW = a.d2s_w;
  const int64_t yhw = (int64_t)IH * IW;
  int64_t off[TI][4];  // c IH IW + py IW + px of each row this lane stores, -1 past the GEMM's rows
  int dy[TI][4], dx[TI][4];
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      const int p = p0 + wp * WP + 16 * i + 4 * grp + r4;
      const int c = p % CI, f = p / CI, py = f / S, px = f - py * S;
      off[i][r4] = p < a.P ? c * yhw + (int64_t)py * IW + px : -1;
      dy[i][r4] = py;
      dx[i][r4] = px;
    }
  const uint32_t ohw = (uint32_t)(ph.OH * ph.OW);
#pragma unroll
  for (int j = 0; j < TJ; ++j) {
    const int q = q0 + wq * WQ + 16 * j + (lane & 15);
    if (q >= ph.Q) continue;
    const uint32_t n = fdiv((uint32_t)q, ph.div_ohw), r = (uint32_t)q - n * ohw;
    const uint32_t oy = fdiv(r, ph.div_ow), ox = r - oy * (uint32_t)ph.OW;
    const int y0 = (int)oy * S, x0 = (int)ox * S;
    float* const yb = a.y + (int64_t)n * CI * yhw + (int64_t)y0 * IW + x0;
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4)
        if (off[i][r4] >= 0 && y0 + dy[i][r4] < IH && x0 + dx[i][r4] < IW) yb[off[i][r4]] = acc[i][j][r4];
  }
}

// Row epilogue, where a.rows holds: bias and ReLU, then the wave's WP x WQ outputs pass through its 8 x (WQ + 8)
// floats of LDS at ep, 8 rows at a time, and leave as float4 runs along the output rows. WQ / 4 lanes write WQ * 4
// contiguous bytes of one row per instruction, where the MFMA layout writes 64-byte pieces of four rows; that pattern
// reaches about 70% of the row pattern's store bandwidth. Pass (i, h) stages rows 4 g + 2 h + {0, 1} of MFMA tile row
// i (lane group g) as staged rows 2 g + {0, 1}; the pitch WQ + 8 puts the four groups on disjoint banks. The caller
// makes ep free before (no wave still reads it) and, where LDS is used again, waits for the reads after.
template <int WQ>
constexpr int row_epi_floats() { return 8 * (WQ + 8); }
template <int TI, int TJ, int WP, int WQ, bool BIAS>
__device__ __forceinline__ void row_epilogue_b(const GatherArgs& a, const Phase& ph, const omt_f32x4 (&acc)[TI][TJ],
                                               int q0, int p0, int wp, int wq, int lane, float* __restrict__ ep,
                                               const float (&bv)[TI][4]) {
  constexpr int EP = WQ + 8, LPR = WQ / 4, RPI = 64 / LPR;  // LDS row pitch; lanes per row, rows per store
  static_assert(WQ == 32 || WQ == 64, "row runs");
  const int P = a.P, grp = lane >> 4;
  const uint32_t ohw = (uint32_t)(ph.OH * ph.OW);
  const int q = q0 + wq * WQ + 4 * (lane % LPR);
  const uint32_t n = fdiv((uint32_t)min(q, ph.Q - 1), ph.div_ohw);
  float* const yq = a.y + (int64_t)n * P * ohw + (q - (int)(n * ohw));
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int j = 0; j < TJ; ++j)
#pragma unroll
        for (int r2 = 0; r2 < 2; ++r2) {
          const int p = p0 + wp * WP + 16 * i + 4 * grp + 2 * h + r2;
          float v = acc[i][j][2 * h + r2];
          if (BIAS && p < P) v += bv[i][2 * h + r2];
          if (a.relu) v = fmaxf(v, 0.f);
          ep[(2 * grp + r2) * EP + 16 * j + (lane & 15)] = v;
        }
      __builtin_amdgcn_wave_barrier();  // LDS runs one wave's accesses in order: its rows are there for the reads
      asm volatile("" ::: "memory");
#pragma unroll
      for (int t = 0; t < 8 / RPI; ++t) {
        const int sr = lane / LPR + RPI * t;  // staged row: tile row 4 (sr / 2) + 2 h + sr % 2
        const int p = p0 + wp * WP + 16 * i + 4 * (sr >> 1) + 2 * h + (sr & 1);
        const float4 v = *reinterpret_cast<const float4*>(&ep[sr * EP + 4 * (lane % LPR)]);
        if (p < P && q < ph.Q) *reinterpret_cast<float4*>(yq + (int64_t)p * ohw) = v;
      }
      asm volatile("" ::: "memory");
      __builtin_amdgcn_wave_barrier();  // the next pass writes these rows
    }
}
// STATS false: no statistics code at all (the persistent 1x1 kernel keeps its register budget without it).
template <int TI, int TJ, int WP, int WQ, bool STATS = true>
__device__ __forceinline__ void row_epilogue(const GatherArgs& a, const Phase& ph, const omt_f32x4 (&acc)[TI][TJ],
                                             int q0, int p0, int wp, int wq, int lane, float* __restrict__ ep) {
  float bv[TI][4];
  if constexpr (STATS)
    if (a.stats) epilogue_stats<TI, TJ, WP, WQ>(a, ph, acc, q0, p0, wp, wq, lane);
  if (a.bias) {
    epilogue_bias<TI, WP>(a, p0, wp, lane, bv);
    row_epilogue_b<TI, TJ, WP, WQ, true>(a, ph, acc, q0, p0, wp, wq, lane, ep, bv);
  } else {
    row_epilogue_b<TI, TJ, WP, WQ, false>(a, ph, acc, q0, p0, wp, wq, lane, ep, bv);
  }
}

// One workgroup's tile (bx, by) of grid-z index bz (slice * nphase + phase); lds holds gather_lds_floats(). PF: K-blocks
// of operand loads in flight ahead of the MFMAs: 2 (one block measured slower on every layer, four slower still),
// or 1 where the second register set would spill (the BN loader on the 64 x 256 tile).
template <int BP, int BQ, int WP, int WQ, int BK, int MODE, bool BN, int PF = 2>
__device__ __forceinline__ void gather_tile(const GatherArgs& a, const int bx, const int by, const int bz,
                                            float* __restrict__ lds) {
  constexpr int NT = 256;
  static_assert(BK % 16 == 0 && NT % BK == 0, "K-block");
  constexpr int WGQ = BQ / WQ;
  static_assert((BP / WP) * (BQ / WQ) == 4, "four waves per workgroup");
  static_assert(WP % 16 == 0 && WQ % 16 == 0 && BQ >= 64 && NT % BQ == 0, "tile shape");
  constexpr int TI = WP / 16, TJ = WQ / 16;
  constexpr int PK = BK + 4;        // LDS row pitch (floats) of both operands: rows are output channels / pixels
  constexpr int AR = BP * BK / NT;  // weight elements per thread
  constexpr int BR = BQ * BK / NT;  // gathered k-rows per thread (a multiple of 4: stored as b128)
  static_assert(AR >= 1 && BR >= 4 && BR % 4 == 0, "tile too small");
  float(*const As)[BP * PK] = reinterpret_cast<float(*)[BP * PK]>(lds);
  float(*const Bs)[BQ * PK] = reinterpret_cast<float(*)[BQ * PK]>(lds + 2 * BP * PK);

  const int zs = bz / a.nphase;  // K slice
  // a register copy: reads through the dynamically indexed kernel argument would each become a scalar load at its
  // use, some inside the per-element bounds branches of the loaders
  const Phase ph = a.ph[bz - zs * a.nphase];
  const int q0 = bx * BQ, p0 = by * BP;
  if (q0 >= ph.Q) return;  // this phase has fewer pixel tiles than the largest one
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int wp = wave / WGQ, wq = wave % WGQ;
  const int KH = ph.KH, KW = ph.KW, K = ph.K, KK = KH * KW, woff = ph.woff;
  const int H = a.H, W = a.W, HW = H * W, P = a.P;
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, a.x_bytes);
  const __amdgpu_buffer_rsrc_t wr = make_rsrc(a.w, a.w_bytes);

  // this thread's output pixel (column of the gathered operand): byte offset of x[n][0][iy0][ix0]
  const int qc = t % BQ;
  const int rbase = __builtin_amdgcn_readfirstlane((t / BQ) * BR);
  int iy0 = -(1 << 28), ix0 = -(1 << 28);  // pixels past Q gather nothing
  uint32_t lbase = kOOB;
  {
    const int q = q0 + qc;
    if (q < ph.Q) {
      const uint32_t ohw = (uint32_t)(ph.OH * ph.OW);
      const uint32_t n = fdiv((uint32_t)q, ph.div_ohw), r = (uint32_t)q - n * ohw;
      const uint32_t oy = fdiv(r, ph.div_ow), ox = r - oy * (uint32_t)ph.OW;
      iy0 = (int)oy * ph.S - ph.PH;
      ix0 = (int)ox * ph.S - ph.PW;
      lbase = MODE == kNhwcNarrow ? (uint32_t)((((int)n * H + iy0) * W + ix0) * a.C * 4)
                                  : (uint32_t)(((int)n * a.C * HW + iy0 * W + ix0) * 4);
    }
  }
  // Channels-last source: thread t loads channels 4 (t % KQN) .. + 3 of each K-block at the NPX tile pixels
  // t / KQN + (NT / KQN) j, so KQN consecutive lanes read one pixel's K-block as one contiguous run of 4 BK bytes.
  // nlb: byte offset of x[n][iy0][ix0][4 (t % KQN)] (wraps below zero for padding rows; a tap in bounds brings it back).
  constexpr int KQN = BK / 4, NPX = MODE == kNhwc ? BQ * KQN / NT : 1;
  static_assert(MODE != kNhwc || (NT % KQN == 0 && BQ % (NT / KQN) == 0), "NHWC pixel slots");
  int niy[NPX], nix[NPX];
  uint32_t nlb[NPX];
  if constexpr (MODE == kNhwc) {
#pragma unroll
    for (int j = 0; j < NPX; ++j) {
      const int q = q0 + t / KQN + (NT / KQN) * j;
      niy[j] = nix[j] = -(1 << 28);
      nlb[j] = kOOB;
      if (q < ph.Q) {
        const uint32_t ohw = (uint32_t)(ph.OH * ph.OW);
        const uint32_t n = fdiv((uint32_t)q, ph.div_ohw), r = (uint32_t)q - n * ohw;
        const uint32_t oy = fdiv(r, ph.div_ow), ox = r - oy * (uint32_t)ph.OW;
        niy[j] = (int)oy * ph.S - ph.PH;
        nix[j] = (int)ox * ph.S - ph.PW;
        nlb[j] = (uint32_t)((((int)n * H + niy[j]) * W + nix[j]) * a.C * 4 + 16 * (t % KQN));
      }
    }
  }

  // channel-major: wave-uniform tap state (c, ky, kx), decomposed afresh at the start of every K-block
  int sc = 0, sky = 0, skx = 0;
  // tap-major: the wave-uniform tap (ky, kx) and first channel c0 of the next K-block gload reads. gload runs over
  // consecutive K-blocks, so the state advances by one block per call (set from kbeg below) instead of being divided
  // out of k every time.
  int nc0 = 0, nky = 0, nkx = 0;
  const int wrow0 = t / BK, wk = t % BK;  // weight tile element: rows wrow0 + 16 i, column wk
  uint32_t aoff[AR];  // byte offsets of this thread's weight elements at k = 0 (out of range for rows past P)
#pragma unroll
  for (int i = 0; i < AR; ++i) {
    const int p = p0 + wrow0 + (NT / BK) * i;
    aoff[i] = p < P ? (uint32_t)((woff + p * K + wk) * 4) : kOOB;
  }
  // Tap-major weights (whole K-blocks, K and woff multiples of 16): each thread loads runs of four k of one row as
  // one 16-byte load (a multi-dword buffer load needs 4-byte alignment only, so a filter used in place may sit
  // anywhere) and stores them with one b128 LDS write: element e = t + NT i of the tile's BP x BK / 4 runs is row
  // e / (BK / 4), k 4 (e % (BK / 4)).
  // With the filter read in place (a.wplace) a run is four channels of one tap, w_cst bytes apart: four 4-byte loads
  // whose block-uniform part (first channel, tap) travels in the scalar offset.
  constexpr bool TAP = MODE != kGeneric && MODE != kNhwcNarrow;  // tap-major K order in whole K-blocks
  constexpr bool A4 = TAP && BP * BK >= 4 * NT;
  constexpr int AR4 = A4 ? BP * BK / (4 * NT) : 1, KQ = BK / 4;
  uint32_t aoff4[AR4];
#pragma unroll
  for (int i = 0; i < AR4; ++i) {
    const int e = t + NT * i, p = p0 + e / KQ;
    if (MODE == kTapInPlace)
      aoff4[i] = p < P ? (uint32_t)p * a.w_rowst + (uint32_t)(4 * (e % KQ)) * a.w_cst : kOOB;
    else
      aoff4[i] = p < P ? (uint32_t)((woff + p * K + 4 * (e % KQ)) * 4) : kOOB;
  }

  float ra[PF][AR], rb[PF][BR];  // PF register sets: loads PF K-blocks ahead of the MFMAs
  float4 ra4[PF][AR4], rb4[PF][NPX];
  auto gload = [&](int k0, const int set) {
    if constexpr (A4) {
      if constexpr (MODE == kTapInPlace) {
        // this K-block: its channels at tap (nky, nkx) of the gather window (the B loader below advances them).
        // Look-ahead blocks past the last tap, and phases no tap reaches (their values are never used), read filter
        // tap (0, 0), so that every address stays inside the filter: nc0 < C always, and a window tap maps into
        // [0, ks) x [0, ks) (ky0 + s (KH - 1) < ks by the phase's window).
        int tky = 0, tkx = 0;
        if (nky < KH && ph.K > 0) {
          tky = a.wplace == 1 ? nky : ph.ky0 + a.s * (KH - 1 - nky);
          tkx = a.wplace == 1 ? nkx : ph.kx0 + a.s * (KW - 1 - nkx);
        }
        // nc0 is the channel of this thread's first k-row (k0 + rbase, one tap per block): the block starts rbase back
        const uint32_t sb = (uint32_t)(nc0 - rbase) * a.w_cst + (uint32_t)((tky * a.ks + tkx) * 4);
#pragma unroll
        for (int i = 0; i < AR4; ++i)
          ra4[set][i] = make_float4(bload(wr, aoff4[i], sb), bload(wr, aoff4[i], sb + a.w_cst),
                                    bload(wr, aoff4[i], sb + 2 * a.w_cst), bload(wr, aoff4[i], sb + 3 * a.w_cst));
      } else {
#pragma unroll
        for (int i = 0; i < AR4; ++i) ra4[set][i] = bload4(wr, aoff4[i] + (uint32_t)(k0 * 4), 0);
      }
    } else {
#pragma unroll
    for (int i = 0; i < AR; ++i) {
      const int p = p0 + wrow0 + (NT / BK) * i, k = k0 + wk;
      uint32_t off;
      if (MODE == kGeneric && !BN && a.wdirect) {
        // W'[p = ci][k = (co, a', b')] = w[co][ci][ky0 + s (KH-1-a')][kx0 + s (KW-1-b')]
        const int co = (int)fdiv((uint32_t)k, ph.div_kk), tt = k - co * KK;
        const int ap = (int)fdiv((uint32_t)tt, ph.div_kw), bp = tt - ap * KW;
        const int ky = ph.ky0 + a.s * (KH - 1 - ap), kx = ph.kx0 + a.s * (KW - 1 - bp);
        off = (p < P && k < K) ? (uint32_t)((((co * P + p) * a.ks + ky) * a.ks + kx) * 4) : kOOB;
      } else {
        // tap-major K-blocks are all whole (C, and so K, is a multiple of BK): no K-tail test
        off = aoff[i] + (uint32_t)(k0 * 4);
        if (!TAP && k >= K) off = kOOB;
      }
      ra[set][i] = bload(wr, off, 0);
    }
    }
    if (TAP) {
      // k = tap * C + c with C % BK == 0: this thread's BR rows share one tap and K has no tail
      const int c0 = nc0, ky = nky, kx = nkx;
      nc0 += BK;
      if (nc0 >= a.C) {
        nc0 -= a.C;
        if (++nkx == KW) {
          nkx = 0;
          ++nky;
        }
      }
      if constexpr (MODE == kNhwc) {
        // the block's channels c0 .. c0 + BK - 1 of tap (ky, kx): the tap moves the pixel, the channel is scalar
        const uint32_t toff = (uint32_t)((ky * W + kx) * a.C * 4);
#pragma unroll
        for (int j = 0; j < NPX; ++j) {
          const bool ok = (unsigned)(niy[j] + ky) < (unsigned)H && (unsigned)(nix[j] + kx) < (unsigned)W;
          rb4[set][j] = bload4(xr, ok ? nlb[j] + toff : kOOB, (uint32_t)(c0 * 4));
        }
        return;
      }
      const bool ok = (unsigned)(iy0 + ky) < (unsigned)H && (unsigned)(ix0 + kx) < (unsigned)W;
      const uint32_t voff = ok ? lbase + (uint32_t)((ky * W + kx) * 4) : kOOB;
#pragma unroll
      for (int j = 0; j < BR; ++j) rb[set][j] = bload(xr, voff, (uint32_t)((c0 + j) * HW * 4));
      return;
    }
    if constexpr (MODE == kNhwcNarrow) {  // k = (ky, kx, c)
      const uint32_t kb = (uint32_t)(k0 + rbase);
      const int tap = (int)fdiv(kb, a.div_c);
      sc = (int)kb - tap * a.C;
      sky = (int)fdiv((uint32_t)tap, ph.div_kw);
      skx = tap - sky * KW;
#pragma unroll
      for (int j = 0; j < BR; ++j) {
        const bool ok = k0 + rbase + j < K && (unsigned)(iy0 + sky) < (unsigned)H && (unsigned)(ix0 + skx) < (unsigned)W;
        rb[set][j] = bload(xr, ok ? lbase + (uint32_t)(((sky * W + skx) * a.C + sc) * 4) : kOOB, 0);
        if (++sc == a.C) {
          sc = 0;
          if (++skx == KW) {
            skx = 0;
            ++sky;
          }
        }
      }
      return;
    }
    {
      const uint32_t kb = (uint32_t)(k0 + rbase);
      sc = (int)fdiv(kb, ph.div_kk);
      const uint32_t r = kb - (uint32_t)sc * (uint32_t)KK;
      sky = (int)fdiv(r, ph.div_kw);
      skx = (int)r - sky * KW;
    }
#pragma unroll
    for (int j = 0; j < BR; ++j) {
      const bool kval = k0 + rbase + j < K;
      float v = 0.f;
      {
        const bool ok = kval && (unsigned)(iy0 + sky) < (unsigned)H && (unsigned)(ix0 + skx) < (unsigned)W;
        v = bload(xr, ok ? lbase + (uint32_t)((sc * HW + sky * W + skx) * 4) : kOOB, 0);
        if (BN) {
          const int cc = min(sc, a.C - 1);  // K-tail and look-ahead taps run past the last channel (v is dropped)
          const float inv = rsqrtf(a.bn_var[cc] + a.bn_eps);
          const float z = fmaxf((v - a.bn_mean[cc]) * inv * a.bn_gamma[cc] + a.bn_beta[cc], 0.f);
          v = ok ? z : 0.f;  // padding taps stay zero: BN + ReLU applies to in-bounds taps only
        }
        if (++skx == KW) {
          skx = 0;
          if (++sky == KH) {
            sky = 0;
            ++sc;
          }
        }
      }
      rb[set][j] = v;
    }
  };
  auto sstore = [&](int buf, const int set) {
    if constexpr (A4) {
#pragma unroll
      for (int i = 0; i < AR4; ++i) {
        const int e = t + NT * i;
        *reinterpret_cast<float4*>(&As[buf][(e / KQ) * PK + 4 * (e % KQ)]) = ra4[set][i];
      }
    } else {
#pragma unroll
      for (int i = 0; i < AR; ++i) As[buf][(wrow0 + (NT / BK) * i) * PK + wk] = ra[set][i];
    }
    if constexpr (MODE == kNhwc) {
#pragma unroll
      for (int j = 0; j < NPX; ++j)
        *reinterpret_cast<float4*>(&Bs[buf][(t / KQN + (NT / KQN) * j) * PK + 4 * (t % KQN)]) = rb4[set][j];
    } else {
#pragma unroll
      for (int j = 0; j < BR; j += 4)
        *reinterpret_cast<float4*>(&Bs[buf][qc * PK + rbase + j]) =
            make_float4(rb[set][j], rb[set][j + 1], rb[set][j + 2], rb[set][j + 3]);
    }
  };

  omt_f32x4 acc[TI][TJ];
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j) acc[i][j] = omt_f32x4{0.f, 0.f, 0.f, 0.f};

  const int kbeg = zs * a.kslice, kend = min(K, kbeg + a.kslice);
  const int nk = kend > kbeg ? (kend - kbeg + BK - 1) / BK : 0;  // an empty slice still writes its (zero) tile
  if (TAP) {
    const uint32_t kb = (uint32_t)(kbeg + (MODE == kNhwc ? 0 : rbase));  // NHWC: the block's first channel
    const int tap = (int)fdiv(kb, a.div_c);
    nc0 = (int)kb - tap * a.C;
    nky = (int)fdiv((uint32_t)tap, ph.div_kw);
    nkx = tap - nky * KW;
  }
  // lane group grp supplies k = grp * (BK / 4) + s at MFMA step s: BK / 16 b128 reads per operand row
  const int la = wp * WP + (lane & 15), lb = wq * WQ + (lane & 15), grp = lane >> 4;
  auto mfma_block = [&](int cur) {
#pragma unroll
    for (int q = 0; q < BK / 16; ++q) {
      float4 av[TI], bv[TJ];
      const int ko = grp * (BK / 4) + 4 * q;
#pragma unroll
      for (int i = 0; i < TI; ++i) av[i] = *reinterpret_cast<const float4*>(&As[cur][(la + 16 * i) * PK + ko]);
#pragma unroll
      for (int j = 0; j < TJ; ++j) bv[j] = *reinterpret_cast<const float4*>(&Bs[cur][(lb + 16 * j) * PK + ko]);
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
          for (int j = 0; j < TJ; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(f4get(av[i], s), f4get(bv[j], s), acc[i][j], 0, 0, 0);
    }
  };
  if constexpr (PF == 1) {
    if (nk > 0) {
      gload(kbeg, 0);
      sstore(0, 0);
    }
    __syncthreads();
    for (int it = 0; it < nk; ++it) {
      const int cur = it & 1;
      if (it + 1 < nk) gload(kbeg + (it + 1) * BK, 0);
      mfma_block(cur);
      if (it + 1 < nk) sstore(cur ^ 1, 0);
      __syncthreads();
    }
  } else {
    // K-block b uses register set and LDS buffer b & 1; the loads of b + 2 are issued before the MFMAs of b, so two
    // blocks' loads are in flight while the MFMAs run. The loads are issued on every step, past the last block too
    // (range-checked buffer loads: the values are never stored): behind a branch, the compiler's wait before the LDS
    // store of block b + 1 cannot count the later blocks' loads as issued after it and waits for them as well.
    static_assert(PF == 2, "two register sets");
    gload(kbeg, 0);
    gload(kbeg + BK, 1);
    if (nk > 0) sstore(0, 0);
    __syncthreads();
    auto step = [&](int it, auto setc) {
      constexpr int S = decltype(setc)::value;  // it & 1
      gload(kbeg + (it + 2) * BK, S);
      mfma_block(S);
      if (it + 1 < nk) sstore(S ^ 1, S ^ 1);
      __syncthreads();
    };
    for (int it = 0; it < nk; it += 2) {
      step(it, std::integral_constant<int, 0>{});
      if (it + 1 < nk) step(it + 1, std::integral_constant<int, 1>{});
    }
  }

  static_assert(4 * row_epi_floats<WQ>() <= gather_lds_floats<BP, BQ, BK>(), "row epilogue fits the tile's LDS");
  if constexpr (MODE == kNhwc || MODE == kNhwcNarrow)
    gather_epilogue_nhwc<TI, TJ, WP, WQ>(a, ph, acc, q0, p0, wp, wq, lane, zs);
  else if (a.d2s && !a.part)
    d2s_epilogue<TI, TJ, WP, WQ>(a, ph, acc, q0, p0, wp, wq, lane);
  else if (a.rows)  // the K loop's last barrier: no wave reads LDS
    row_epilogue<TI, TJ, WP, WQ>(a, ph, acc, q0, p0, wp, wq, lane, lds + wave * row_epi_floats<WQ>());
  else
    gather_epilogue<TI, TJ, WP, WQ>(a, ph, acc, q0, p0, wp, wq, lane, zs);
}

// 1x1, stride 1, unpadded convolutions (and their grad input, a 1x1 convolution with the transposed filter) with a
// short reduction (K = C of 64 or 128: four or eight K-blocks per tile): Y[n][p][pix] = sum_c A[p][c] X[n][c][pix].
// Launched one tile at a time, such a GEMM spends about as long in each workgroup's first-load latency and store
// drain as in its MFMAs. Here a workgroup keeps one output-channel tile and walks `tpw` consecutive pixel tiles, and
// its two-block prefetch runs on across the tile boundaries: the next tile's first K-blocks are loading while the
// current tile finishes, and its output stores drain under the next tile's MFMAs. One phase, no split K, no BN
// loader; K a multiple of the K-block (the host checks). Same LDS layout and MFMA order as the staged gather tiles,
// so each output sums its K terms in the same order as there.
template <int BP, int BQ, int WP, int WQ, bool STATS>
__global__ void __launch_bounds__(256, 2) conv1x1_stream_kernel(const GatherArgs a, const int tpw) {
  constexpr int NT = 256, BK = 16;
  constexpr int WGQ = BQ / WQ, TI = WP / 16, TJ = WQ / 16, PK = BK + 4;
  constexpr int AR = BP * BK / NT, BR = BQ * BK / NT;
  static_assert((BP / WP) * (BQ / WQ) == 4 && BQ >= 64 && NT % BQ == 0 && BR % 4 == 0 && AR >= 1, "tile shape");
  __shared__ __attribute__((aligned(16))) float lds[gather_lds_floats<BP, BQ, BK>()];
  float(*const As)[BP * PK] = reinterpret_cast<float(*)[BP * PK]>(lds);
  float(*const Bs)[BQ * PK] = reinterpret_cast<float(*)[BQ * PK]>(lds + 2 * BP * PK);

  const TileId tile = xcd_block_tile(kTileGroup);
  const Phase ph = a.ph[0];
  const int ntq = (ph.Q + BQ - 1) / BQ;
  const int tq0 = tile.x * tpw, ntiles = min(ntq, tq0 + tpw) - tq0;
  if (ntiles <= 0) return;
  const int p0 = tile.y * BP, C = a.C, HW = a.H * a.W, P = a.P, K = ph.K;
  const int nk = K / BK, nv = ntiles * nk;  // K-blocks per tile; virtual blocks (tile, K-block) of this workgroup
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int wp = wave / WGQ, wq = wave % WGQ;
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, a.x_bytes);
  const __amdgpu_buffer_rsrc_t wr = make_rsrc(a.w, a.w_bytes);

  const int qc = t % BQ;
  const int rbase = __builtin_amdgcn_readfirstlane((t / BQ) * BR);
  const int wrow0 = t / BK, wk = t % BK;
  uint32_t aoff[AR];
#pragma unroll
  for (int i = 0; i < AR; ++i) {
    const int p = p0 + wrow0 + (NT / BK) * i;
    aoff[i] = p < P ? (uint32_t)((ph.woff + p * K + wk) * 4) : kOOB;
  }
  // byte offset of x[n][0][pix] for this thread's pixel of pixel tile `tq` (past Q: out of range)
  auto xbase = [&](int tq) -> uint32_t {
    const int q = tq * BQ + qc;
    if (q >= ph.Q) return kOOB;
    const uint32_t n = fdiv((uint32_t)q, ph.div_ohw);
    return (uint32_t)(((int)n * C * HW + (q - (int)n * HW)) * 4);
  };

  // load side: the next virtual block to load is K-block lkb of pixel tile ltq. It runs PF = 2 blocks ahead of the
  // MFMAs and past the workgroup's last tile (those loads read in-range or out-of-range values that are never
  // stored), so every load is issued unconditionally and the compiler's waits count them exactly.
  int ltq = tq0, lkb = 0;
  uint32_t lxb = xbase(ltq);
  float ra[2][AR], rb[2][BR];
  auto gload = [&](const int set) {
#pragma unroll
    for (int i = 0; i < AR; ++i) ra[set][i] = bload(wr, aoff[i] == kOOB ? kOOB : aoff[i] + (uint32_t)(lkb * BK * 4), 0);
#pragma unroll
    for (int j = 0; j < BR; ++j) rb[set][j] = bload(xr, lxb, (uint32_t)((lkb * BK + rbase + j) * HW * 4));
    if (++lkb == nk) {
      lkb = 0;
      lxb = xbase(++ltq);
    }
  };
  auto sstore = [&](int buf, const int set) {
#pragma unroll
    for (int i = 0; i < AR; ++i) As[buf][(wrow0 + (NT / BK) * i) * PK + wk] = ra[set][i];
#pragma unroll
    for (int j = 0; j < BR; j += 4)
      *reinterpret_cast<float4*>(&Bs[buf][qc * PK + rbase + j]) =
          make_float4(rb[set][j], rb[set][j + 1], rb[set][j + 2], rb[set][j + 3]);
  };

  omt_f32x4 acc[TI][TJ];
  auto zero = [&]() {
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
      for (int j = 0; j < TJ; ++j) acc[i][j] = omt_f32x4{0.f, 0.f, 0.f, 0.f};
  };
  zero();
  const int la = wp * WP + (lane & 15), lb = wq * WQ + (lane & 15), grp = lane >> 4;
  auto mfma_block = [&](int cur) {
    float4 av[TI], bv[TJ];
    const int ko = grp * (BK / 4);
#pragma unroll
    for (int i = 0; i < TI; ++i) av[i] = *reinterpret_cast<const float4*>(&As[cur][(la + 16 * i) * PK + ko]);
#pragma unroll
    for (int j = 0; j < TJ; ++j) bv[j] = *reinterpret_cast<const float4*>(&Bs[cur][(lb + 16 * j) * PK + ko]);
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(f4get(av[i], s), f4get(bv[j], s), acc[i][j], 0, 0, 0);
  };

  // the row epilogue stages each wave's rows in the two LDS buffers (both free at a tile's end: the last block's
  // MFMAs are done after a barrier, and the next block is stored only afterwards); the host checks a.rows
  static_assert(4 * row_epi_floats<WQ>() <= gather_lds_floats<BP, BQ, BK>(), "row epilogue fits the tile's LDS");
  float* const ep = lds + wave * row_epi_floats<WQ>();

  gload(0);
  gload(1);
  sstore(0, 0);
  __syncthreads();
  int ckb = 0, ctq = tq0;  // compute side: K-block and pixel tile of the block the MFMAs take next
  auto step = [&](int v, auto setc) {
    constexpr int S = decltype(setc)::value;  // v & 1: register set and LDS buffer of block v
    gload(S);                                 // block v + 2 into the set block v vacated
    mfma_block(S);
    if (++ckb == nk) {
      __syncthreads();  // every wave's MFMAs of this block have read buffer S
      row_epilogue<TI, TJ, WP, WQ, STATS>(a, ph, acc, ctq * BQ, p0, wp, wq, lane, ep);
      zero();
      ckb = 0;
      ++ctq;
      __syncthreads();  // the staged rows are read before block v + 1 lands in LDS
    }
    if (v + 1 < nv) sstore(S ^ 1, S ^ 1);
    __syncthreads();
  };
  for (int v = 0; v < nv; v += 2) {
    step(v, std::integral_constant<int, 0>{});
    if (v + 1 < nv) step(v + 1, std::integral_constant<int, 1>{});
  }
}

// 1x1, stride 1, unpadded convolutions (and their grad input) whose reduction K = C is 64 or 128: at ResNet-50's
// 56^2 and 28^2 expansions the output is four times the input, and a launch that computes a tile and then stores it
// adds the store time to the MFMA time (the workgroups of a CU run in step and store together). Filter-stationary:
// each wave keeps its 16 TJ output channels' whole filter rows in registers for the workgroup's life, and only the
// input streams, pixel tile by pixel tile (BQ pixels x K), through two LDS buffers: the loads of tile v + 2 are
// issued when tile v starts and tile v + 1 goes to LDS before tile v's MFMAs, one barrier per tile. Two accumulator
// sets: tile v - 1's outputs leave 16 channels at a time between tile v's K-blocks, so the stores stream out while
// the MFMAs run. The GEMM runs transposed, pixels as the MFMA rows: accumulator rows 4 g + r of lane group g are
// four consecutive pixels of one output channel, staged through the wave's LDS rows into whole row runs. At MFMA step s
// lane group g supplies k = 16 b + 4 g + s of K-block b, the staged tiles' k order, so each output sums its K terms in
// their order. The host checks: one 1x1 s1 unpadded phase, no split, no BN loader or epilogue statistics, H W % 4 == 0
// (float4 pixel runs stay in one image), x and y 16-byte aligned, y below 2 GiB.
template <int K, int TJ, int BQ, int OCC>
__global__ void __launch_bounds__(256, OCC) conv1x1_wst_kernel(const GatherArgs a, const int tpw) {
  constexpr int KP = K + 4, TI = BQ / 16, KB = K / 16, NP = K * BQ / 2048;  // NP: float4 pairs per thread per tile
  static_assert(BQ == 32 || BQ == 64, "pixel tile");
  constexpr int GPB = (TJ + KB - 1) / KB;  // 16-channel store groups after each K-block
  constexpr int SP = BQ + 4, LPR = BQ / 4, RPI = 64 / LPR;  // staging pitch; lanes per output row, rows per store
  static_assert(K == 64 || K == 128, "K");
  // row pitch K + 4: the 16 lanes of a ds_read_b128 quarter read rows 16 i + 0..15 at 16-byte offsets 4 apart mod 64
  // banks, disjoint
  __shared__ __attribute__((aligned(16))) float xs[2][BQ * KP];
  __shared__ __attribute__((aligned(16))) float stg_all[4][16 * SP];  // each wave's output staging rows

  const TileId tile = xcd_block_tile(kTileGroup);
  const Phase ph = a.ph[0];
  const int Q = ph.Q, ntq = (Q + BQ - 1) / BQ;
  const int tq0 = tile.x * tpw, ntiles = min(ntq, tq0 + tpw) - tq0;
  if (ntiles <= 0) return;
  const int t = threadIdx.x, lane = t & 63, g = lane >> 4, l16 = lane & 15;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int P = a.P, HW = a.H * a.W, C = a.C;
  const int pw = tile.y * (64 * TJ) + wave * (16 * TJ);  // the wave's first output channel
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, a.x_bytes);
  const __amdgpu_buffer_rsrc_t wr = make_rsrc(a.w, a.w_bytes);
  const __amdgpu_buffer_rsrc_t yr = make_rsrc(a.y, (uint32_t)((int64_t)Q * P * 4));
  float* const stg = stg_all[wave];

  // the wave's filter rows: wv[j][4 b + s] = A[pw + 16 j + l16][16 b + 4 g + s], 0 past P
  float wv[TJ][K / 4], bj[TJ];
#pragma unroll
  for (int j = 0; j < TJ; ++j) {
    const int p = pw + 16 * j + l16;
#pragma unroll
    for (int b = 0; b < KB; ++b)
#pragma unroll
      for (int s = 0; s < 4; ++s)
        wv[j][4 * b + s] = bload(wr, p < P ? (uint32_t)((ph.woff + p * K + 16 * b + 4 * g + s) * 4) : kOOB, 0);
    bj[j] = a.bias && p < P ? a.bias[p] : 0.f;
  }

  // input tile loads: thread t takes pixel quad pq = t % (BQ / 4) of the tile and k rows KR r + 2 kp + {0, 1}
  // (kp = t / (BQ / 4), KR = 512 / BQ k rows per pass)
  constexpr int NQ = BQ / 4, KR = 2 * 256 / NQ;
  const int pq = t % NQ, kp = t / NQ;
  // byte offset of x[n][2 kp][pixel] for the thread's quad of tile tq (past Q: out of range; the rows' uniform terms
  // go in the scalar offset)
  auto xbase = [&](int tq) __attribute__((always_inline)) -> uint32_t {
    const int q = tq * BQ + 4 * pq;
    if (q >= Q) return kOOB;
    const uint32_t n = fdiv((uint32_t)q, ph.div_ohw);
    return (uint32_t)(((int)n * C * HW + 2 * kp * HW + (q - (int)n * HW)) * 4);
  };
  float4 ld[2][NP][2];
  auto gload = [&](int tq, const int set) __attribute__((always_inline)) {
    const uint32_t xb = xbase(tq);
#pragma unroll
    for (int r = 0; r < NP; ++r)
#pragma unroll
      for (int u = 0; u < 2; ++u) ld[set][r][u] = bload4(xr, xb, (uint32_t)((KR * r + u) * HW * 4));
  };
  // transposed into xs[buf][pixel][k]: each of the four pixels' k pair as one 8-byte store
  auto sstore = [&](int buf, const int set) __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < NP; ++r)
#pragma unroll
      for (int v = 0; v < 4; ++v)
        *reinterpret_cast<float2*>(&xs[buf][(4 * pq + v) * KP + KR * r + 2 * kp]) =
            make_float2(f4get(ld[set][r][0], v), f4get(ld[set][r][1], v));
  };

  omt_f32x4 acc[2][TI][TJ];
#pragma unroll
  for (int c = 0; c < 2; ++c)
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
      for (int j = 0; j < TJ; ++j) acc[c][i][j] = omt_f32x4{0.f, 0.f, 0.f, 0.f};

  // Store group j of a tile: acc[c][i][j][r] is output channel pw + 16 j + l16 at pixel tq BQ + 16 i + 4 g + r. Bias
  // and ReLU, then the 16 channels x BQ pixels pass through the wave's staging rows (as [channel][pixel]) and leave as
  // whole row runs, LPR lanes x 16 bytes per output row, RPI rows per store: a store of 16 rows x 64 bytes straight
  // from the MFMA layout measured a quarter slower at these sizes. The registers are cleared for the tile after next.
  // Range-checked buffer stores issued by every lane (past P or Q at an out-of-range offset, dropped): stores behind
  // branches would leave the compiler unsure how many are in flight, and its wait for the next tile's loads would
  // then drain them all. The staging rows are the wave's own, and LDS runs a wave's accesses in order.
  auto store_group = [&](const int c, int tq, const int j) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < TI; ++i) {
      float v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        v[r] = acc[c][i][j][r] + bj[j];
        if (a.relu) v[r] = fmaxf(v[r], 0.f);
        acc[c][i][j][r] = 0.f;
      }
      *reinterpret_cast<float4*>(&stg[l16 * SP + 16 * i + 4 * g]) = make_float4(v[0], v[1], v[2], v[3]);
    }
    __builtin_amdgcn_wave_barrier();
    asm volatile("" ::: "memory");
    const int q = tq * BQ + 4 * (lane % LPR);
    const uint32_t n = fdiv((uint32_t)min(max(q, 0), Q - 1), ph.div_ohw);
    const uint32_t yq = (uint32_t)(((int)n * P * HW + (q - (int)n * HW)) * 4);
#pragma unroll
    for (int h = 0; h < TI; ++h) {
      const int row = RPI * h + lane / LPR, p = pw + 16 * j + row;
      const float4 w4 = *reinterpret_cast<const float4*>(&stg[row * SP + 4 * (lane % LPR)]);
      const uint32_t off = tq >= 0 && p < P && q < Q ? yq + (uint32_t)(p * HW * 4) : kOOB;
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(omt_u32x4, w4), yr, (int)off, 0, 0);
    }
    asm volatile("" ::: "memory");
    __builtin_amdgcn_wave_barrier();
  };
  // tile v's MFMAs into acc[c] from buffer c, tile v - 1's stores from acc[c ^ 1] between its K-blocks (before the
  // first tile, tq_prev = -1: every store out of range, issued all the same so that the count in flight is fixed)
  auto mfma_tile = [&](const int c, int tq_prev) __attribute__((always_inline)) {
#pragma unroll
    for (int b = 0; b < KB; ++b) {
      float4 xv[TI];
#pragma unroll
      for (int i = 0; i < TI; ++i) xv[i] = *reinterpret_cast<const float4*>(&xs[c][(16 * i + l16) * KP + 16 * b + 4 * g]);
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
          for (int j = 0; j < TJ; ++j)
            acc[c][i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(f4get(xv[i], s), wv[j][4 * b + s], acc[c][i][j], 0, 0, 0);
#pragma unroll
      for (int j = b * GPB; j < (b + 1) * GPB && j < TJ; ++j) store_group(c ^ 1, tq_prev, j);
    }
  };

  // Tile v uses register set, LDS buffer and accumulator set v & 1. Loads run two tiles ahead and past the run's end
  // (tiles past it are never stored to y: they fill a buffer no MFMA reads), so every load and LDS store is
  // unconditional and the compiler's waits count them exactly.
  gload(tq0, 0);
  gload(tq0 + 1, 1);
  sstore(0, 0);
  __syncthreads();
  auto step = [&](int v, auto setc) __attribute__((always_inline)) {
    constexpr int S = decltype(setc)::value;
    gload(tq0 + v + 2, S);  // the set tile v vacated when it went to LDS
    sstore(S ^ 1, S ^ 1);   // tile v + 1 into the buffer tile v - 1 read before the last barrier
    mfma_tile(S, v > 0 ? tq0 + v - 1 : -1);
    __syncthreads();  // tile v + 1 in LDS for every wave; buffer S free for tile v + 2
  };
  for (int v = 0; v < ntiles; v += 2) {
    step(v, std::integral_constant<int, 0>{});
    if (v + 1 < ntiles) step(v + 1, std::integral_constant<int, 1>{});
  }
  // the last tile's stores
  if ((ntiles - 1) & 1) {
#pragma unroll
    for (int j = 0; j < TJ; ++j) store_group(1, tq0 + ntiles - 1, j);
  } else {
#pragma unroll
    for (int j = 0; j < TJ; ++j) store_group(0, tq0 + ntiles - 1, j);
  }
}

template <int BP, int BQ, int WP, int WQ, int BK, int MODE, bool BN, int PF>
__global__ void __launch_bounds__(256, 2) conv_gather_kernel(const GatherArgs a) {
  __shared__ __attribute__((aligned(16))) float lds[gather_lds_floats<BP, BQ, BK>()];
  const TileId t = xcd_block_tile(kTileGroup);
  gather_tile<BP, BQ, WP, WQ, BK, MODE, BN, PF>(a, t.x, t.y, t.z, lds);
}

// ---- gather with direct global -> LDS loads (tap-major order only) ------------------------------------------------
// The operand loads go straight into an LDS ring of NS K-block stages (buffer_load ... lds), so NS - 1 blocks of loads
// are in flight while the MFMAs of one run, at no VGPR cost and with no LDS store instructions. Tile: 64 output
// channels x BQ pixels, K-block BK (16 or 32), four waves of WP x WQ. MFMA lane group g supplies k = g BK/4 + s at
// step s (s < BK/4).
//  - weights, 16-byte loads (lane = row) of four consecutive k into As[stage][k / 4][row][4]; a lane reads its BK/4
//    k-steps of one row with BK/16 ds_read_b128;
//  - gathered input, dword loads: lane = pixel, one instruction per k-row of 64 pixels, into Bs[stage][k][pixel]. Row
//    pitch BQ + 4 (BK 16) or BQ + 2 (BK 32) makes the stride between the lane groups' rows g BK/4 + s 16 banks mod 64,
//    so the four groups' ds_read_b32 fall on disjoint bank ranges.
// All K-blocks are whole (C is a multiple of BK in tap-major order). One barrier per K-block: after it, the stage
// consumed by the previous block is free for the loads NS - 1 blocks ahead.
template <int BK>
constexpr int dl_pad() { return BK == 16 ? 4 : 2; }
template <int BQ, int BK>
constexpr int gather_dl_stage_floats() { return 64 * BK + BK * (BQ + dl_pad<BK>()); }

// stg[s]: the NS stages, each its own LDS array (so that the compiler can tell a stage's reads from the loads in
// flight into the others, and wait for the right ones only); the K loop is unrolled by NS so every access names one.
template <int BQ, int WP, int WQ, int BK, int NS>
__device__ __forceinline__ void gather_tile_dl(const GatherArgs& a, const int bx, const int by, const int bz,
                                               float* const (&stg)[NS]) {
  constexpr int BP = 64, NH = BQ / 64;
  constexpr int WGQ = BQ / WQ;
  static_assert((BP / WP) * (BQ / WQ) == 4 && WP % 16 == 0 && WQ % 16 == 0 && BQ % 64 == 0, "tile shape");
  static_assert(BK == 16 || BK == 32, "K-block");
  constexpr int TI = WP / 16, TJ = WQ / 16, BPITCH = BQ + dl_pad<BK>();
  constexpr int KQ = BK / 16;                  // weight loads (16-byte rows of 4 k) per wave; k-rows per wave: 4 KQ
  constexpr int ASZ = BP * BK;                 // floats of a stage's weight part; the gathered part follows
  constexpr int LOADS = KQ + BK / 4 * NH;      // load instructions per wave per stage
  static_assert(NS >= 2 && NS <= 4, "stages");

  const int zs = bz / a.nphase;
  const Phase ph = a.ph[bz - zs * a.nphase];
  const int q0 = bx * BQ, p0 = by * BP;
  if (q0 >= ph.Q) return;
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int wp = wave / WGQ, wq = wave % WGQ;
  const int KW = ph.KW, K = ph.K, H = a.H, W = a.W, HW = H * W, P = a.P, C = a.C;
  const omt_u32x4 xr = rsrc_words(a.x, a.x_bytes);
  const omt_u32x4 wr = rsrc_words(a.w, a.w_bytes);

  // this lane's pixels (one per 64-pixel half) and weight row
  int iy0[NH], ix0[NH];
  uint32_t lbase[NH];
#pragma unroll
  for (int h = 0; h < NH; ++h) {
    iy0[h] = ix0[h] = -(1 << 28);
    lbase[h] = kOOB;
    const int q = q0 + 64 * h + lane;
    if (q < ph.Q) {
      const uint32_t ohw = (uint32_t)(ph.OH * ph.OW);
      const uint32_t n = fdiv((uint32_t)q, ph.div_ohw), r = (uint32_t)q - n * ohw;
      const uint32_t oy = fdiv(r, ph.div_ow), ox = r - oy * (uint32_t)ph.OW;
      iy0[h] = (int)oy * ph.S - ph.PH;
      ix0[h] = (int)ox * ph.S - ph.PW;
      lbase[h] = (uint32_t)(((int)n * C * HW + iy0[h] * W + ix0[h]) * 4);
    }
  }
  const int prow = p0 + lane;
  const uint32_t abase = prow < P ? (uint32_t)((ph.woff + prow * K) * 4) : kOOB;

  const int kbeg = zs * a.kslice, kend = min(K, kbeg + a.kslice);
  const int nk = kend > kbeg ? (kend - kbeg) / BK : 0;
  // tap state (c0, ky, kx) of the next K-block to load: consecutive blocks advance it by 16 channels
  int nc0, nky, nkx;
  {
    const int tap = (int)fdiv((uint32_t)kbeg, a.div_c);
    nc0 = kbeg - tap * C;
    nky = (int)fdiv((uint32_t)tap, ph.div_kw);
    nkx = tap - nky * KW;
  }
  int kload = kbeg;
  auto issue = [&](float* st) {
#pragma unroll
    for (int u = 0; u < KQ; ++u) {  // weight k-quads wave + 4 u
      const int kq = wave + 4 * u;
      lds_load_b128(wr, lds_addr(st + kq * (BP * 4)), abase == kOOB ? kOOB : abase + (uint32_t)((kload + 4 * kq) * 4));
    }
    const int c0 = nc0, ky = nky, kx = nkx;
#pragma unroll
    for (int h = 0; h < NH; ++h) {
      const bool ok = (unsigned)(iy0[h] + ky) < (unsigned)H && (unsigned)(ix0[h] + kx) < (unsigned)W;
      const uint32_t voff = ok ? lbase[h] + (uint32_t)((ky * W + kx) * 4) : kOOB;
#pragma unroll
      for (int j = 0; j < BK / 4; ++j) {  // input k-rows wave BK/4 + j
        const int k = wave * (BK / 4) + j;
        lds_load_b32(xr, lds_addr(st + ASZ + k * BPITCH + 64 * h), voff, (uint32_t)((c0 + k) * HW * 4));
      }
    }
    kload += BK;
    nc0 += BK;
    if (nc0 >= C) {
      nc0 -= C;
      if (++nkx == KW) {
        nkx = 0;
        ++nky;
      }
    }
  };

  omt_f32x4 acc[TI][TJ];
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j) acc[i][j] = omt_f32x4{0.f, 0.f, 0.f, 0.f};

  const int grp = lane >> 4, m16 = lane & 15;
  auto mfma_stage = [&](const float* st) {
#pragma unroll
    for (int q = 0; q < KQ; ++q) {  // k-steps 4 q .. 4 q + 3 of this lane group
      float4 av[TI];
#pragma unroll
      for (int i = 0; i < TI; ++i)
        av[i] = *reinterpret_cast<const float4*>(st + ((grp * KQ + q) * BP + wp * WP + 16 * i + m16) * 4);
      float bv[TJ][4];
#pragma unroll
      for (int j = 0; j < TJ; ++j)
#pragma unroll
        for (int s = 0; s < 4; ++s)
          bv[j][s] = st[ASZ + (grp * (BK / 4) + 4 * q + s) * BPITCH + wq * WQ + 16 * j + m16];
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
          for (int j = 0; j < TJ; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(f4get(av[i], s), bv[j][s], acc[i][j], 0, 0, 0);
    }
  };
  // block it: wait for this wave's loads of it (the blocks issued after it stay in flight), barrier, issue block
  // it + NS - 1 into the stage block it - 1 used, MFMAs of block it
  auto step = [&](int it, auto stc) {
    constexpr int S = decltype(stc)::value;
    const int after = min(NS - 2, nk - 1 - it);
    asm volatile("" ::: "memory");
    if (after >= 2)
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * LOADS));
    else if (after == 1)
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(LOADS));
    else
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    // a bare barrier: the wait above covers this wave's loads of block it, and a __syncthreads() fence would wait for
    // every load in flight, the later blocks' included. After it, block it is in LDS for every wave and no wave still
    // reads the stage of block it - 1 (its MFMAs consumed their reads before it got here).
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (it + NS - 1 < nk) issue(stg[(S + NS - 1) % NS]);
    mfma_stage(stg[S]);
  };

#pragma unroll
  for (int s = 0; s < NS - 1; ++s)
    if (s < nk) issue(stg[s]);
  // unrolled by 2 NS: the compiler's own wait bookkeeping for the loads in flight is merged at the loop header, and
  // the step after the merge waits for them all; the longer body makes that once per 2 NS blocks
  auto steps = [&](int it0, auto offc) {
    constexpr int O = decltype(offc)::value;
    if (it0 + O < nk) step(it0 + O, std::integral_constant<int, O % NS>{});
  };
  for (int it = 0; it < nk; it += 2 * NS) {
    steps(it, std::integral_constant<int, 0>{});
    steps(it, std::integral_constant<int, 1>{});
    steps(it, std::integral_constant<int, 2>{});
    steps(it, std::integral_constant<int, 3>{});
    if constexpr (NS > 2) {
      steps(it, std::integral_constant<int, 4>{});
      steps(it, std::integral_constant<int, 5>{});
    }
    if constexpr (NS > 3) {
      steps(it, std::integral_constant<int, 6>{});
      steps(it, std::integral_constant<int, 7>{});
    }
  }
  static_assert(4 * row_epi_floats<WQ>() <= gather_dl_stage_floats<BQ, BK>(), "row epilogue fits one stage");
  if (a.rows) {
    __syncthreads();  // every wave's MFMAs have read their last stage
    row_epilogue<TI, TJ, WP, WQ>(a, ph, acc, q0, p0, wp, wq, lane, stg[0] + wave * row_epi_floats<WQ>());
  } else {
    gather_epilogue<TI, TJ, WP, WQ>(a, ph, acc, q0, p0, wp, wq, lane, zs);
  }
}

template <int BQ, int WP, int WQ, int BK, int NS>
__global__ void __launch_bounds__(256, 2) conv_gather_dl_kernel(const GatherArgs a) {
  constexpr int F = gather_dl_stage_floats<BQ, BK>();
  __shared__ __attribute__((aligned(16))) float s0[F];
  __shared__ __attribute__((aligned(16))) float s1[F];
  __shared__ __attribute__((aligned(16))) float s2[NS > 2 ? F : 4];
  __shared__ __attribute__((aligned(16))) float s3[NS > 3 ? F : 4];
  float* stages[4] = {s0, s1, s2, s3};
  float* const(&stg)[NS] = *reinterpret_cast<float* const(*)[NS]>(&stages);
  const TileId t = xcd_block_tile(kTileGroup);
  gather_tile_dl<BQ, WP, WQ, BK, NS>(a, t.x, t.y, t.z, stg);
}

// ---- grad weight ------------------------------------------------------------------------------------------------

struct WgradArgs {
  const float* x;   // [N][C][H][W]
  const float* gy;  // [N][P][OH][OW]
  float* out;       // [slices][P][Q]
  uint32_t x_bytes, gy_bytes;
  int C, H, W, P, OH, OW, KS, S, PAD;
  int Q, K;    // C * KS * KS, N * OH * OW
  int kslice;  // pixels per slice, a multiple of the K-block
  FastDiv div_ohw, div_ow, div_kk, div_ks, div_c;
  int step_n, step_oy, step_ox;  // 64 output pixels as (images, rows, columns): 64 = (step_n OH + step_oy) OW + step_ox
};

// LDS floats of a grad-weight tile: both operands, rows of 64 + 4.
template <int BP, int BQ>
constexpr int wgrad_lds_floats() { return (BP + BQ) * (64 + 4); }

// One workgroup's tile (bx, by) of K slice bz; lds holds wgrad_lds_floats(). PF: K-blocks of operand loads in flight
// ahead of the MFMAs.
template <int BP, int BQ, int WP, int WQ, int MODE, int PF = 1>
__device__ __forceinline__ void wgrad_tile(const WgradArgs& a, const int bx, const int by, const int bz,
                                           float* __restrict__ lds) {
  constexpr int BK = 64;  // one reduction pixel per lane
  constexpr int WGQ = BQ / WQ;
  static_assert((BP / WP) * (BQ / WQ) == 4, "four waves per workgroup");
  static_assert(WP % 16 == 0 && WQ % 16 == 0 && BP % 4 == 0 && BQ % 4 == 0, "tile shape");
  constexpr int TI = WP / 16, TJ = WQ / 16;
  constexpr int PK = BK + 4;               // LDS row pitch (floats): rows are gy channels / tap columns, k contiguous
  constexpr int AR = BP / 4, BR = BQ / 4;  // rows (cols) each wave stages per K-block, contiguous per wave
  float* const As = lds;
  float* const Bs = lds + BP * PK;

  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int wp = wave / WGQ, wq = wave % WGQ;
  const int q0 = bx * BQ, p0 = by * BP;
  const int kbeg = bz * a.kslice;
  const int kend = min(a.K, kbeg + a.kslice);
  const int H = a.H, W = a.W, HW = H * W, P = a.P, Q = a.Q, KS = a.KS;
  const int ohw = a.OH * a.OW;
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, a.x_bytes);
  const __amdgpu_buffer_rsrc_t gr = make_rsrc(a.gy, a.gy_bytes);
  const int pw0 = p0 + wave * AR;  // this wave's first staged gy row
  const int qw0 = q0 + wave * BR;  // this wave's first staged tap column
  // tap state of column qw0 (wave-uniform, constant over the K loop). Generic: q = (c, ky, kx). Tap-major:
  // q = (ky, kx, c) with C % BR == 0, so the wave's BR columns share the tap (ky0, kx0) over channels c0 ...
  int c0, ky0, kx0;
  if (MODE == kTapMajor) {
    const int tap = (int)fdiv((uint32_t)qw0, a.div_c);
    c0 = qw0 - tap * a.C;
    ky0 = (int)fdiv((uint32_t)tap, a.div_ks);
    kx0 = tap - ky0 * KS;
  } else {
    c0 = (int)fdiv((uint32_t)qw0, a.div_kk);
    const int r0 = qw0 - c0 * KS * KS;
    ky0 = (int)fdiv((uint32_t)r0, a.div_ks);
    kx0 = r0 - ky0 * KS;
  }

  // PF register sets: loads PF K-blocks ahead of the MFMAs. kPix4 (1x1, stride 1, unpadded, OH OW % 4 == 0): four
  // consecutive reduction pixels of one row are contiguous in x and gy, so a lane loads them as one 16-byte load
  // (lane: row rr = lane / 16 of four, pixels 4 kq .. 4 kq + 3 of the K-block, kq = lane % 16): a quarter of the load
  // instructions, so four times the bytes in flight per outstanding-load slot, into the same LDS layout
  constexpr bool P4 = MODE == kPix4;
  float ra[PF][P4 ? 1 : AR], rb[PF][P4 ? 1 : BR];
  float4 ra4[PF][P4 ? AR / 4 : 1], rb4[PF][P4 ? BR / 4 : 1];
  const int rr = lane >> 4, kq = lane & 15;
  auto gload = [&](int k0, const int set) {
    if constexpr (P4) {
      const int k = k0 + 4 * kq;  // K and the slice bounds are multiples of 4: the run is whole or past kend
      uint32_t gbase = kOOB, xbase = kOOB;
      if (k < kend) {
        const uint32_t n = fdiv((uint32_t)k, a.div_ohw), r = (uint32_t)k - n * (uint32_t)ohw;
        gbase = (uint32_t)(((int)n * P * ohw + (int)r) * 4) + (uint32_t)(rr * ohw * 4);
        xbase = (uint32_t)(((int)n * a.C * HW + (int)r) * 4) + (uint32_t)(rr * HW * 4);  // pixel = output pixel
      }
#pragma unroll
      for (int i = 0; i < AR / 4; ++i)
        ra4[set][i] = bload4(gr, pw0 + 4 * i + rr < P ? gbase : kOOB, (uint32_t)((pw0 + 4 * i) * ohw * 4));
#pragma unroll
      for (int j = 0; j < BR / 4; ++j)
        rb4[set][j] = bload4(xr, qw0 + 4 * j + rr < Q ? xbase : kOOB, (uint32_t)((qw0 + 4 * j) * HW * 4));
      return;
    }
    const int k = k0 + lane;
    const bool kval = k < kend;
    uint32_t gbase = kOOB, xbase = kOOB;
    int iy0 = -(1 << 28), ix0 = -(1 << 28);
    if (kval) {
      const uint32_t n = fdiv((uint32_t)k, a.div_ohw), r = (uint32_t)k - n * (uint32_t)ohw;
      const uint32_t oy = fdiv(r, a.div_ow), ox = r - oy * (uint32_t)a.OW;
      gbase = (uint32_t)(((int)n * P * ohw + (int)r) * 4);
      iy0 = (int)oy * a.S - a.PAD;
      ix0 = (int)ox * a.S - a.PAD;
      xbase = (uint32_t)(((int)n * a.C * HW + iy0 * W + ix0) * 4);
    }
    // every load is issued (rows and columns past the tile's end at offset kOOB, which reads 0): a load behind a
    // branch leaves the compiler unable to count it at the LDS stores, which then wait for every load in flight
#pragma unroll
    for (int i = 0; i < AR; ++i)
      ra[set][i] = bload(gr, pw0 + i < P ? gbase : kOOB, (uint32_t)((pw0 + i) * ohw * 4));
    if (MODE == kTapMajor) {
      const bool ok = qw0 < Q && (unsigned)(iy0 + ky0) < (unsigned)H && (unsigned)(ix0 + kx0) < (unsigned)W;
      const uint32_t voff = ok ? xbase + (uint32_t)((ky0 * W + kx0) * 4) : kOOB;
#pragma unroll
      for (int j = 0; j < BR; ++j) rb[set][j] = bload(xr, voff, (uint32_t)((c0 + j) * HW * 4));
      return;
    }
    int c = c0, ky = ky0, kx = kx0;
#pragma unroll
    for (int j = 0; j < BR; ++j) {
      const bool ok = qw0 + j < Q && (unsigned)(iy0 + ky) < (unsigned)H && (unsigned)(ix0 + kx) < (unsigned)W;
      rb[set][j] = bload(xr, ok ? xbase + (uint32_t)((c * HW + ky * W + kx) * 4) : kOOB, 0);
      if (++kx == KS) {
        kx = 0;
        if (++ky == KS) {
          ky = 0;
          ++c;
        }
      }
    }
  };
  auto sstore = [&](const int set) {
    if constexpr (P4) {
#pragma unroll
      for (int i = 0; i < AR / 4; ++i)
        *reinterpret_cast<float4*>(&As[(wave * AR + 4 * i + rr) * PK + 4 * kq]) = ra4[set][i];
#pragma unroll
      for (int j = 0; j < BR / 4; ++j)
        *reinterpret_cast<float4*>(&Bs[(wave * BR + 4 * j + rr) * PK + 4 * kq]) = rb4[set][j];
      return;
    }
#pragma unroll
    for (int i = 0; i < AR; ++i) As[(wave * AR + i) * PK + lane] = ra[set][i];
#pragma unroll
    for (int j = 0; j < BR; ++j) Bs[(wave * BR + j) * PK + lane] = rb[set][j];
  };

  omt_f32x4 acc[TI][TJ];
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j) acc[i][j] = omt_f32x4{0.f, 0.f, 0.f, 0.f};

  const int la = wp * WP + (lane & 15), lb = wq * WQ + (lane & 15), grp = lane >> 4;
  auto mfma_block = [&]() {
#pragma unroll
    for (int m = 0; m < BK / 16; ++m) {
      const int kc = grp * (BK / 4) + 4 * m;  // this lane group's next four K-indices
      float4 av[TI], bv[TJ];
#pragma unroll
      for (int i = 0; i < TI; ++i) av[i] = *reinterpret_cast<const float4*>(&As[(la + 16 * i) * PK + kc]);
#pragma unroll
      for (int j = 0; j < TJ; ++j) bv[j] = *reinterpret_cast<const float4*>(&Bs[(lb + 16 * j) * PK + kc]);
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
          for (int j = 0; j < TJ; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(f4get(av[i], s), f4get(bv[j], s), acc[i][j], 0, 0, 0);
    }
  };
  if constexpr (PF == 1) {
    if (kbeg < kend) gload(kbeg, 0);
    for (int k0 = kbeg; k0 < kend; k0 += BK) {
      sstore(0);
      __syncthreads();
      if (k0 + BK < kend) gload(k0 + BK, 0);
      mfma_block();
      __syncthreads();
    }
  } else {
    // K-block b is loaded into register set b % PF, PF blocks ahead: while the MFMAs of b run, the loads of b + 1
    // .. b + PF are in flight. The loads are issued on every step (past kend they load zeros): behind a branch, the
    // compiler's wait before the LDS store of block b + 1 cannot count the later blocks' loads as issued after it.
    static_assert(PF == 2, "two register sets");
#pragma unroll
    for (int b = 0; b < PF; ++b) gload(kbeg + b * BK, b);
    auto step = [&](int k0, auto setc) {
      constexpr int S = decltype(setc)::value;  // block % PF
      sstore(S);
      __syncthreads();
      gload(k0 + PF * BK, S);
      mfma_block();
      __syncthreads();
    };
    for (int k0 = kbeg; k0 < kend; k0 += PF * BK) {
      step(k0, std::integral_constant<int, 0>{});
      if (k0 + BK < kend) step(k0 + BK, std::integral_constant<int, 1>{});
    }
  }

  // store in the [co][ci][ky][kx] order of the weight gradient (tap-major columns are permuted back)
  float* out = a.out + (int64_t)bz * P * Q;
#pragma unroll
  for (int j = 0; j < TJ; ++j) {
    const int q = q0 + wq * WQ + 16 * j + (lane & 15);
    if (q >= Q) continue;
    int col = q;
    if (MODE == kTapMajor) {
      const int tap = (int)fdiv((uint32_t)q, a.div_c);
      col = (q - tap * a.C) * KS * KS + tap;
    }
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int p = p0 + wp * WP + 16 * i + 4 * grp + r4;
        if (p < P) out[(int64_t)p * Q + col] = acc[i][j][r4];
      }
  }
}

template <int BP, int BQ, int WP, int WQ, int MODE, int PF>
__global__ void __launch_bounds__(256, 2) conv_wgrad_kernel(const WgradArgs a) {
  __shared__ __attribute__((aligned(16))) float lds[wgrad_lds_floats<BP, BQ>()];
  const TileId t = xcd_block_tile(kTileGroup);
  wgrad_tile<BP, BQ, WP, WQ, MODE, PF>(a, t.x, t.y, t.z, lds);
}

// Channels-last grad weight: C[co][q'] = sum_k gy[k][co] * X(k, q') with k = (n, oy, ox) and the tap-major column
// q' = (ky, kx, ci), which is also the column order of a channels-last filter gradient gw[co][ky][kx][ci]. Both
// operands are contiguous along their GEMM rows / columns (gy along co, x along ci), not along k: each K-block of 64
// pixels is staged as rows of k (pitch BP + 16 and BQ + 16 floats: the four lane groups of an MFMA operand read, at
// rows 4 s + g, fall on disjoint banks), loaded as float4 runs of four co / four ci of one pixel, and the MFMA
// operands are read one float per lane. Lane group g supplies k = 4 s + g of the block at MFMA step s. Needs
// P % 4 == 0, and C % 4 == 0 (a run of four ci stays inside one tap) unless NARROW: then each of a thread's four
// columns is its own tap and channel (a 3-channel stem's columns cross taps), loaded element by element into the same
// float4 slot, so the staging and the MFMA order are unchanged.
template <int BP, int BQ>
constexpr int wgrad_nhwc_lds_floats() { return 64 * ((BP + 16) + (BQ + 16)); }

template <int BP, int BQ, int WP, int WQ, int PF, bool NARROW = false>
__device__ __forceinline__ void wgrad_nhwc_tile(const WgradArgs& a, const int bx, const int by, const int bz,
                                                float* __restrict__ lds) {
  constexpr int NT = 256, BK = 64;
  constexpr int WGQ = BQ / WQ;
  static_assert((BP / WP) * (BQ / WQ) == 4, "four waves per workgroup");
  static_assert(WP % 16 == 0 && WQ % 16 == 0, "tile shape");
  constexpr int TI = WP / 16, TJ = WQ / 16;
  constexpr int PA = BP + 16, PB = BQ + 16;          // LDS row pitches (floats); rows are the K-block's pixels
  constexpr int AQ = BP / 4, BQN = BQ / 4;           // float4 runs per row
  constexpr int ARW = NT / AQ, BRW = NT / BQN;       // rows one pass of the workgroup loads
  constexpr int NA = BK / ARW, NB = BK / BRW;        // float4 loads per thread and K-block
  static_assert(NT % AQ == 0 && NT % BQN == 0 && BK % ARW == 0 && BK % BRW == 0, "load shape");
  float* const As = lds;
  float* const Bs = lds + BK * PA;

  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int wp = wave / WGQ, wq = wave % WGQ;
  const int q0 = bx * BQ, p0 = by * BP;
  const int kbeg = bz * a.kslice;
  const int kend = min(a.K, kbeg + a.kslice);
  const int H = a.H, W = a.W, P = a.P, Q = a.Q, C = a.C;
  const uint32_t ohw = (uint32_t)(a.OH * a.OW);
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, a.x_bytes);
  const __amdgpu_buffer_rsrc_t gr = make_rsrc(a.gy, a.gy_bytes);
  // this thread's gy run: channels pa .. pa + 3 of pixel rows ar + ARW i
  const int ar = t / AQ, pa = p0 + 4 * (t % AQ);
  const bool pok = pa < P;
  // this thread's x run: columns qb .. qb + 3 = tap (ky, kx), channels ci .. ci + 3, of pixel rows br + BRW j
  const int br = t / BQN, qb = q0 + 4 * (t % BQN);
  const bool qok = qb < Q;
  int ky = 0, kx = 0, ci = 0;
  if (qok) {
    const int tap = (int)fdiv((uint32_t)qb, a.div_c);
    ci = qb - tap * C;
    ky = (int)fdiv((uint32_t)tap, a.div_ks);
    kx = tap - ky * a.KS;
  }
  // NARROW: column qb + e is tap (eky, ekx), channel eci (eq: inside the filter's columns)
  int eky[4] = {0, 0, 0, 0}, ekx[4] = {0, 0, 0, 0}, eci[4] = {0, 0, 0, 0};
  bool eq[4] = {false, false, false, false};
  if constexpr (NARROW) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      eq[e] = qb + e < Q;
      if (eq[e]) {
        const int tap = (int)fdiv((uint32_t)(qb + e), a.div_c);
        eci[e] = qb + e - tap * C;
        eky[e] = (int)fdiv((uint32_t)tap, a.div_ks);
        ekx[e] = tap - eky[e] * a.KS;
      }
    }
  }

  // The pixel (n, oy, ox) of each of this thread's x rows, for the next K-block gload reads: decomposed once, then
  // advanced by one block (64 pixels) per call as a mixed-radix addition with one carry per digit.
  int rn[NB], roy[NB], rox[NB];
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    const uint32_t k = (uint32_t)min(kbeg + br + BRW * j, a.K - 1);
    const uint32_t n = fdiv(k, a.div_ohw), r = k - n * ohw;
    const uint32_t oy = fdiv(r, a.div_ow);
    rn[j] = (int)n;
    roy[j] = (int)oy;
    rox[j] = (int)(r - oy * (uint32_t)a.OW);
  }

  float4 ra4[PF][NA], rb4[PF][NB];
  // Every load is issued and the loaders are branch-free (out-of-range rows and columns select offset kOOB, which
  // reads 0): a load or an index computation behind a branch splits the loop into blocks, and the compiler's waits
  // before the LDS stores then drain every load in flight (see conv_wgrad_kernel).
  auto gload = [&](int k0, const int set) {
    // (the conditions combine with & rather than &&: a short-circuit turns into branches around the offsets)
#pragma unroll
    for (int i = 0; i < NA; ++i) {
      const int k = k0 + ar + ARW * i;
      const uint32_t off = (uint32_t)((k * P + pa) * 4);
      ra4[set][i] = bload4(gr, (pok & (k < kend)) ? off : kOOB, 0);
    }
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int k = k0 + br + BRW * j;
      if constexpr (NARROW) {
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int iy = roy[j] * a.S - a.PAD + eky[e], ix = rox[j] * a.S - a.PAD + ekx[e];
          const bool ok = eq[e] & (k < kend) & ((unsigned)iy < (unsigned)H) & ((unsigned)ix < (unsigned)W);
          v[e] = bload(xr, ok ? (uint32_t)((((rn[j] * H + iy) * W + ix) * C + eci[e]) * 4) : kOOB, 0);
        }
        rb4[set][j] = make_float4(v[0], v[1], v[2], v[3]);
      } else {
        const int iy = roy[j] * a.S - a.PAD + ky, ix = rox[j] * a.S - a.PAD + kx;
        const bool ok = qok & (k < kend) & ((unsigned)iy < (unsigned)H) & ((unsigned)ix < (unsigned)W);
        const uint32_t off = (uint32_t)((((rn[j] * H + iy) * W + ix) * C + ci) * 4);
        rb4[set][j] = bload4(xr, ok ? off : kOOB, 0);
      }
      // the next block's pixel of this row
      int ox = rox[j] + a.step_ox, oy = roy[j] + a.step_oy, n = rn[j] + a.step_n;
      const int cx = ox >= a.OW;
      ox -= cx ? a.OW : 0;
      oy += cx;
      const int cy = oy >= a.OH;
      oy -= cy ? a.OH : 0;
      rox[j] = ox;
      roy[j] = oy;
      rn[j] = n + cy;
    }
  };
  auto sstore = [&](const int set) {
#pragma unroll
    for (int i = 0; i < NA; ++i) *reinterpret_cast<float4*>(&As[(ar + ARW * i) * PA + 4 * (t % AQ)]) = ra4[set][i];
#pragma unroll
    for (int j = 0; j < NB; ++j) *reinterpret_cast<float4*>(&Bs[(br + BRW * j) * PB + 4 * (t % BQN)]) = rb4[set][j];
  };

  omt_f32x4 acc[TI][TJ];
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j) acc[i][j] = omt_f32x4{0.f, 0.f, 0.f, 0.f};

  const int la = wp * WP + (lane & 15), lb = wq * WQ + (lane & 15), grp = lane >> 4;
  auto mfma_block = [&]() {
#pragma unroll
    for (int s = 0; s < BK / 4; ++s) {
      const int k = 4 * s + grp;
      float av[TI], bv[TJ];
#pragma unroll
      for (int i = 0; i < TI; ++i) av[i] = As[k * PA + la + 16 * i];
#pragma unroll
      for (int j = 0; j < TJ; ++j) bv[j] = Bs[k * PB + lb + 16 * j];
#pragma unroll
      for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[i], bv[j], acc[i][j], 0, 0, 0);
    }
  };
  if constexpr (PF == 1) {
    if (kbeg < kend) gload(kbeg, 0);
    for (int k0 = kbeg; k0 < kend; k0 += BK) {
      sstore(0);
      __syncthreads();
      if (k0 + BK < kend) gload(k0 + BK, 0);
      mfma_block();
      __syncthreads();
    }
  } else {
    // Whole pairs of blocks in the loop and an odd last block after it: a conditional second step in the loop body
    // merges two load histories at the loop head, where the compiler then waits for every load in flight.
    static_assert(PF == 2, "two register sets");
#pragma unroll
    for (int b = 0; b < PF; ++b) gload(kbeg + b * BK, b);
    auto step = [&](int k0, auto setc) {
      constexpr int S = decltype(setc)::value;
      sstore(S);
      __syncthreads();
      gload(k0 + PF * BK, S);
      mfma_block();
      __syncthreads();
    };
    int k0 = kbeg;
    for (; k0 + BK < kend; k0 += PF * BK) {
      step(k0, std::integral_constant<int, 0>{});
      step(k0 + BK, std::integral_constant<int, 1>{});
    }
    if (k0 < kend) step(k0, std::integral_constant<int, 0>{});
  }

  float* out = a.out + (int64_t)bz * P * Q;
#pragma unroll
  for (int j = 0; j < TJ; ++j) {
    const int q = q0 + wq * WQ + 16 * j + (lane & 15);
    if (q >= Q) continue;
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int p = p0 + wp * WP + 16 * i + 4 * grp + r4;
        if (p < P) out[(int64_t)p * Q + q] = acc[i][j][r4];
      }
  }
}

template <int BP, int BQ, int WP, int WQ, int PF, bool NARROW = false>
__global__ void __launch_bounds__(256, 2) conv_wgrad_nhwc_kernel(const WgradArgs a) {
  __shared__ __attribute__((aligned(16))) float lds[wgrad_nhwc_lds_floats<BP, BQ>()];
  const TileId t = xcd_block_tile(kTileGroup);
  wgrad_nhwc_tile<BP, BQ, WP, WQ, PF, NARROW>(a, t.x, t.y, t.z, lds);
}

// Grad input and grad weight of one convolution in one launch (omt_conv_bwd), both on 64 x 64 tiles: the first
// gx * gy * gz workgroups run grad-input tiles, the rest grad-weight tiles over wx * wy * wz (each part through the
// XCD tile mapping). On late,
// low-resolution layers each GEMM alone puts about one workgroup on a CU, which then waits on its loads; in one launch
// every CU also holds a workgroup of the other GEMM to run meanwhile.
struct DualGrid {
  int gx, gy, gz, wx, wy, wz;
};
template <int GBK, int GMODE, int WMODE>
__global__ void __launch_bounds__(256, 2) conv_bwd_dual_kernel(const GatherArgs ga, const WgradArgs wa, const DualGrid d) {
  constexpr int kG = gather_lds_floats<64, 64, GBK>(), kW = wgrad_lds_floats<64, 64>();
  __shared__ __attribute__((aligned(16))) float lds[kG > kW ? kG : kW];
  const int b = (int)blockIdx.x;
  const int ng = d.gx * d.gy * d.gz;
  if (b < ng) {
    const TileId t = xcd_tile(b, d.gx, d.gy, d.gz, kTileGroup);
    gather_tile<64, 64, 32, 32, GBK, GMODE, false, 2>(ga, t.x, t.y, t.z, lds);
  } else {
    const TileId t = xcd_tile(b - ng, d.wx, d.wy, d.wz, kTileGroup);
    wgrad_tile<64, 64, 32, 32, WMODE, 2>(wa, t.x, t.y, t.z, lds);
  }
}

// Split-K gather epilogue: y[i] = act(sum_z part[z][i] + bias[c(i)]), slices summed in order; y is NCHW with
// planes of `plane` elements over `P` channels. VEC 4 needs plane % 4 == 0 (a float4 then stays in one plane).
struct GatherSum {
  const float* part;
  float* y;
  int64_t total, plane;
  int slices, P;
  const float* bias;
  int relu;
  bool vec4;
  int64_t blocks;  // workgroups of its launch
  int d2s, d2s_ci, img_h, img_w, grid_w;  // super-pixel grad input: scatter [N][s^2 C][grid] to [N][C][img]
  int nhwc;  // channels-last y [N][YH][YW][P]
};
template <int VEC>
__device__ __forceinline__ void gather_sum(const GatherSum& r, int64_t b0, int64_t nb) {
  using T = typename VecF<VEC>::T;
  const int64_t nv = r.total / VEC;
  for (int64_t i = b0 * blockDim.x + threadIdx.x; i < nv; i += nb * blockDim.x) {
    float v[VEC];
    sum_slices<VEC>(reinterpret_cast<const T*>(r.part), nv, i, r.slices, v);
    if (VEC == 1 && r.d2s) {  // 64-bit image index: the grid of s^2 C rows can exceed the image on tiny images
      const int64_t pl = r.plane, rows = (int64_t)r.P * pl, n = i / rows, rem = i - n * rows;
      const int p = (int)(rem / pl), q = (int)(rem - p * pl);
      const int oy = q / r.grid_w, ox = q - oy * r.grid_w;
      const int c = p % r.d2s_ci, f = p / r.d2s_ci, py = f / r.d2s, px = f - py * r.d2s;
      const int row = oy * r.d2s + py, col = ox * r.d2s + px;
      if (row < r.img_h && col < r.img_w) r.y[((n * r.d2s_ci + c) * r.img_h + row) * r.img_w + col] = v[0];
      continue;
    }
    if (r.nhwc) {  // channels last: element i VEC + e is channel (i VEC + e) % P
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        if (r.bias) v[e] += r.bias[(i * VEC + e) % r.P];
        if (r.relu) v[e] = fmaxf(v[e], 0.f);
      }
      reinterpret_cast<T*>(r.y)[i] = VecF<VEC>::pack(v);
      continue;
    }
    const float b = r.bias ? r.bias[(i * VEC / r.plane) % r.P] : 0.f;
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      v[e] += b;
      if (r.relu) v[e] = fmaxf(v[e], 0.f);
    }
    reinterpret_cast<T*>(r.y)[i] = VecF<VEC>::pack(v);
  }
}

template <int VEC>
__global__ void __launch_bounds__(256) split_reduce_kernel(const SplitSum r) {
  split_sum_any<VEC>(r, blockIdx.x, gridDim.x);
}
template <int VEC>
__global__ void __launch_bounds__(256) gather_reduce_kernel(const GatherSum r) {
  gather_sum<VEC>(r, blockIdx.x, gridDim.x);
}
// Both split-K sums of a convolution backward in one launch: the first g.blocks workgroups sum grad input.
template <int GV, int WV>
__global__ void __launch_bounds__(256) dual_reduce_kernel(const GatherSum g, const SplitSum w) {
  const int64_t b = blockIdx.x;
  if (b < g.blocks)
    gather_sum<GV>(g, b, g.blocks);
  else
    split_sum_any<WV>(w, b - g.blocks, (int64_t)gridDim.x - g.blocks);
}

// Re-packs w[co][ci][ks][ks] into the per-phase grad-input weights W'[ci][co][a'][b'] described at the top.
struct PackPhase {
  int ky0, kx0, jy, jx, woff;
};
struct PackArgs {
  const float* w;
  float* out;
  int CO, CI, KS, S, nphase;
  int tap_major;  // 1: W'[ci][a'][b'][co], else W'[ci][co][a'][b']
  int src_krsc;   // 1: w is a channels-last filter [co][ks][ks][ci]
  PackPhase ph[kMaxPhases];
};
__global__ void __launch_bounds__(256) pack_dgrad_weights_kernel(const PackArgs a) {
  const int total = a.CO * a.CI * a.KS * a.KS;
  for (int e = blockIdx.x * blockDim.x + threadIdx.x; e < total; e += gridDim.x * blockDim.x) {
    int f = 0;
    while (f + 1 < a.nphase && e >= a.ph[f + 1].woff) ++f;
    const PackPhase& p = a.ph[f];
    const int jj = p.jy * p.jx, kph = a.CO * jj;
    const int r = e - p.woff;
    const int ci = r / kph, rem = r % kph;
    const int co = a.tap_major ? rem % a.CO : rem / jj, tap = a.tap_major ? rem / a.CO : rem % jj;
    const int ap = tap / p.jx, bp = tap % p.jx;
    const int ky = p.ky0 + a.S * (p.jy - 1 - ap), kx = p.kx0 + a.S * (p.jx - 1 - bp);
    a.out[e] = a.src_krsc ? a.w[((co * a.KS + ky) * a.KS + kx) * a.CI + ci]
                          : a.w[((co * a.CI + ci) * a.KS + ky) * a.KS + kx];
  }
}

// The stride-1 case of pack_dgrad_weights_kernel for a channels-last filter in tap-major order (one phase, all KK
// taps, ky0 = kx0 = 0): out[ci][t][co] = w[co][KK - 1 - t][ci], a transpose of (co, ci) per tap, run as 32 x 32 tiles
// through LDS (grid: ci tiles, co tiles, taps) so that the reads (runs of ci) and the writes (runs of co) are whole
// 128-byte lines instead of one line per element on the read side.
__global__ void __launch_bounds__(256) pack_dgrad_krsc_s1_kernel(const float* __restrict__ w, float* __restrict__ out,
                                                                 int CO, int CI, int KK) {
  __shared__ float tile[32][33];
  const int tap = blockIdx.z, co0 = blockIdx.y * 32, ci0 = blockIdx.x * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
  for (int r = ty; r < 32; r += 8) {
    const int co = co0 + r, ci = ci0 + tx;
    if (co < CO && ci < CI) tile[r][tx] = w[((int64_t)co * KK + tap) * CI + ci];
  }
  __syncthreads();
  const int t = KK - 1 - tap;  // the flipped tap
  for (int r = ty; r < 32; r += 8) {
    const int ci = ci0 + r, co = co0 + tx;
    if (co < CO && ci < CI) out[((int64_t)ci * KK + t) * CO + co] = tile[tx][r];
  }
}

// Super-pixel grad-input filter W'[p = (py s + px) CI + c][k]: k = (dy L + dx) CO + co (tap-major) or
// co L L + dy L + dx, the L x L window of gy rows i + dy - PH around grid pixel i. Phase (py, px) reaches gy row
// i + qy - a' through filter row ky0 + s a' (a' < jy; ky0 = (py + pad) mod s, qy = (py + pad - ky0) / s), so window row
// dy holds a' = qy - (dy - PH), and zero where no tap of the phase lands.
struct PackD2S {
  const float* w;
  float* out;
  int CO, CI, KS, S, PAD, L, PH, tap_major;
};
__global__ void __launch_bounds__(256) pack_d2s_weights_kernel(const PackD2S a) {
  const int LL = a.L * a.L, K = a.CO * LL, total = a.S * a.S * a.CI * K;
  for (int e = blockIdx.x * blockDim.x + threadIdx.x; e < total; e += gridDim.x * blockDim.x) {
    const int p = e / K, k = e - p * K;
    const int c = p % a.CI, f = p / a.CI, py = f / a.S, px = f - py * a.S;
    const int co = a.tap_major ? k % a.CO : k / LL, tap = a.tap_major ? k / a.CO : k % LL;
    const int dy = tap / a.L, dx = tap - dy * a.L;
    const int ky0 = (py + a.PAD) % a.S, kx0 = (px + a.PAD) % a.S;
    const int jy = ky0 < a.KS ? (a.KS - ky0 + a.S - 1) / a.S : 0, jx = kx0 < a.KS ? (a.KS - kx0 + a.S - 1) / a.S : 0;
    const int ay = (py + a.PAD - ky0) / a.S - (dy - a.PH), ax = (px + a.PAD - kx0) / a.S - (dx - a.PH);
    float v = 0.f;
    if (ay >= 0 && ay < jy && ax >= 0 && ax < jx)
      v = a.w[((co * a.CI + c) * a.KS + ky0 + a.S * ay) * a.KS + kx0 + a.S * ax];
    a.out[e] = v;
  }
}

// Forward weights in tap-major order: wt[co][ky][kx][ci] = w[co][ci][ky][kx].
__global__ void __launch_bounds__(256) pack_tapmajor_kernel(const float* __restrict__ w, float* __restrict__ out,
                                                            int co, int ci, int kk) {
  const int total = co * ci * kk;
  for (int e = blockIdx.x * blockDim.x + threadIdx.x; e < total; e += gridDim.x * blockDim.x) {
    const int o = e / (kk * ci), r = e - o * kk * ci, tap = r / ci, c = r - tap * ci;
    out[e] = w[(o * ci + c) * kk + tap];
  }
}

// gb[c] = sum over n and hw of gy[n][c][hw]: one workgroup per channel, fp32 lanes, tree reduction.
__global__ void __launch_bounds__(256) bias_grad_kernel(const float* __restrict__ gy, float* __restrict__ gb, int n,
                                                        int c, int hw) {
  const int ch = blockIdx.x;
  float s = 0.f;
  for (int nn = 0; nn < n; ++nn) {
    const float* row = gy + ((int64_t)nn * c + ch) * hw;
    for (int e = threadIdx.x; e < hw; e += blockDim.x) s += row[e];
  }
  __shared__ float red[256];
  red[threadIdx.x] = s;
  __syncthreads();
  for (int off = 128; off > 0; off >>= 1) {
    if ((int)threadIdx.x < off) red[threadIdx.x] += red[threadIdx.x + off];
    __syncthreads();
  }
  if (threadIdx.x == 0) gb[ch] = red[0];
}

// Small planes (a linear layer's bias: hw = 1): thread per channel, summing n then hw in order; consecutive threads
// read consecutive channels of a row, and every load of a group of 8 is in flight together.
__global__ void __launch_bounds__(256) bias_grad_cols_kernel(const float* __restrict__ gy, float* __restrict__ gb, int n,
                                                             int c, int hw) {
  const int ch = blockIdx.x * 256 + threadIdx.x;
  if (ch >= c) return;
  const int total = n * hw;
  float s = 0.f;
  for (int i0 = 0; i0 < total; i0 += 8) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = i0 + u, nn = i / hw, e = i - nn * hw;
      v[u] = i < total ? gy[((int64_t)nn * c + ch) * hw + e] : 0.f;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (i0 + u < total) s += v[u];
  }
  gb[ch] = s;
}
constexpr int kBiasColsHW = 16;  // planes up to this size take bias_grad_cols_kernel

__global__ void __launch_bounds__(256) fold_bn_kernel(int co, int per_out, const float* __restrict__ cw,
                                                      const float* __restrict__ cb, const float* __restrict__ gamma,
                                                      const float* __restrict__ beta, const float* __restrict__ mean,
                                                      const float* __restrict__ var, float eps, float* __restrict__ fw,
                                                      float* __restrict__ fb) {
  const int64_t total = (int64_t)co * per_out;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
    const int o = (int)(e / per_out);
    const float scale = gamma[o] / sqrtf(var[o] + eps);
    fw[e] = cw[e] * scale;
    if (e % per_out == 0) fb[o] = ((cb ? cb[o] : 0.f) - mean[o]) * scale + beta[o];
  }
}

// ---- tile selection and launch ----------------------------------------------------------------------------------

struct Tile {
  int bp, bq, wp, wq;
  float eff;    // relative MFMA efficiency of the wave tile (operand reuse)
  int bk = 16;  // K-block (gather kernels)
  int ns = 0;   // > 0: direct global -> LDS loads into an ns-stage ring (tap-major order; else the staged kernel)
  int stream = 0;  // 1x1 stride-1 convolutions only: 1 conv1x1_stream_kernel (runs of pixel tiles per workgroup),
                   // 2 conv1x1_wst_kernel (K of 64 or 128, the filter held in registers)
};

// Picks the tile with the smallest estimated makespan: rounds of `slots` concurrent workgroups times the padded
// tile work, over the tile's efficiency.
template <size_t N>
static int pick_tile(const Tile (&tiles)[N], int64_t P, int64_t Q, int64_t z, int64_t slots) {
  int best = 0;
  double best_cost = 1e300;
  for (size_t i = 0; i < N; ++i) {
    const Tile& tl = tiles[i];
    int64_t blocks = cdiv(P, tl.bp) * cdiv(Q, tl.bq) * z;
    int64_t rounds = cdiv(blocks, slots);
    double cost = (double)rounds * tl.bp * tl.bq / tl.eff;
    if (cost < best_cost * 0.999) {
      best_cost = cost;
      best = (int)i;
    }
  }
  return best;
}

// Tiles 6-8 carry deeper K-blocks: more MFMA work per load round trip for grids of about one workgroup per CU,
// where the loads' latency is not hidden by other workgroups. Tiles 14-16 (32 x 64) give small layers (ResNet-18 at
// 64x64 input: 64 channels over 8192 pixels) twice the workgroups of the 64 x 64 tile, so that every CU holds one
// without a K split.
static const Tile kGatherTiles[] = {
    {64, 256, 64, 64, 1.00f},     {128, 128, 64, 64, 1.00f},    {64, 128, 32, 64, 0.92f},
    {32, 256, 32, 64, 0.90f},     {16, 256, 16, 64, 0.80f},     {64, 64, 32, 32, 0.80f},
    {64, 64, 32, 32, 0.90f, 64},  {64, 128, 32, 64, 0.95f, 32}, {128, 64, 64, 32, 0.95f, 32},
    {64, 64, 32, 32, 0.85f, 16, 4}, {64, 128, 32, 64, 0.95f, 16, 3}, {64, 64, 32, 32, 0.90f, 32, 3},
    {64, 128, 32, 64, 0.97f, 32, 2}, {64, 128, 32, 64, 0.95f, 16, 0, 1},
    {32, 64, 16, 32, 0.60f}, {32, 64, 16, 32, 0.65f, 32}, {32, 64, 16, 32, 0.65f, 64},
    {256, 32, 64, 32, 1.00f, 16, 0, 2}, {128, 32, 32, 32, 1.00f, 16, 0, 2}, {128, 64, 32, 64, 1.00f, 16, 0, 2},
};
// Plan tile index t < 3 * kNGather: kGatherTiles[t % kNGather] in one of three variants. t < kNGather: tap-major K
// order where it applies, over a re-packed filter; kNGather <= t < 2 kNGather: channel-major order (no filter
// re-pack, one launch fewer; the tap-major order gathers faster on large layers); t >= 2 kNGather: tap-major order
// reading the filter in place (no re-pack launch, four 4-byte filter loads per run of four k instead of one 16-byte
// load), on tiles whose filter tile has whole runs per thread (BP BK >= 1024) and that are not the 1x1 streaming
// tile; elsewhere it runs as the first variant.
constexpr int kNGather = (int)(sizeof(kGatherTiles) / sizeof(kGatherTiles[0]));
constexpr int kStreamTile = 13;
// The filter-stationary tiles 17-19 (conv1x1_wst_kernel): 64 TJ output channels per workgroup at K 64 (TJ 4, 2, 2),
// half as many at K 128 (the same filter registers), pixel tiles of 32, 32 and 64; their resident workgroups per CU
// (waves per SIMD) at K 64 and 128, the kernels' launch bounds.
constexpr int kWstFirst = 17;
constexpr int kWstOcc[3][2] = {{2, 3}, {4, 3}, {2, 1}};  // as registers and LDS (input + staging) allow
static int wst_shape(int t) { return t % kNGather - kWstFirst; }  // conv1x1_stream_kernel; tile 17 (conv1x1_wst_kernel) runs as it where it does not apply
static const Tile& gtile(int t) { return kGatherTiles[t % kNGather]; }
static bool gcm(int t) { return t >= kNGather && t < 2 * kNGather; }
static bool wplace_tile(int t) {
  const Tile& tl = gtile(t);
  return t >= 2 * kNGather && !tl.stream && tl.bp * tl.bk >= 1024;
}

static const Tile kWgradTiles[] = {
    {64, 128, 32, 64, 1.00f}, {128, 64, 32, 64, 1.00f}, {64, 64, 32, 32, 0.85f}, {32, 128, 16, 64, 0.85f},
};

constexpr int64_t kCUs = 256;

template <int MODE, bool BN>
static void gather_dispatch(int ti, const GatherArgs& a, dim3 grid, hipStream_t s) {
  switch (ti) {
    case 0: hipLaunchKernelGGL((conv_gather_kernel<64, 256, 64, 64, 16, MODE, BN, BN ? 1 : 2>), grid, dim3(256), 0, s, a); break;
    case 1: hipLaunchKernelGGL((conv_gather_kernel<128, 128, 64, 64, 16, MODE, BN, 2>), grid, dim3(256), 0, s, a); break;
    case 2: hipLaunchKernelGGL((conv_gather_kernel<64, 128, 32, 64, 16, MODE, BN, 2>), grid, dim3(256), 0, s, a); break;
    case 3: hipLaunchKernelGGL((conv_gather_kernel<32, 256, 32, 64, 16, MODE, BN, 2>), grid, dim3(256), 0, s, a); break;
    case 4: hipLaunchKernelGGL((conv_gather_kernel<16, 256, 16, 64, 16, MODE, BN, 2>), grid, dim3(256), 0, s, a); break;
    case 5: hipLaunchKernelGGL((conv_gather_kernel<64, 64, 32, 32, 16, MODE, BN, 2>), grid, dim3(256), 0, s, a); break;
    case 6: hipLaunchKernelGGL((conv_gather_kernel<64, 64, 32, 32, 64, MODE, BN, 2>), grid, dim3(256), 0, s, a); break;
    case 7: hipLaunchKernelGGL((conv_gather_kernel<64, 128, 32, 64, 32, MODE, BN, 2>), grid, dim3(256), 0, s, a); break;
    case 8: hipLaunchKernelGGL((conv_gather_kernel<128, 64, 64, 32, 32, MODE, BN, 2>), grid, dim3(256), 0, s, a); break;
    // the direct-LDS tiles when their kernel does not apply (channel-major order, BN loader): the staged kernel
    case 9: hipLaunchKernelGGL((conv_gather_kernel<64, 64, 32, 32, 16, MODE, BN, 2>), grid, dim3(256), 0, s, a); break;
    case 10: hipLaunchKernelGGL((conv_gather_kernel<64, 128, 32, 64, 16, MODE, BN, 2>), grid, dim3(256), 0, s, a); break;
    case 11: hipLaunchKernelGGL((conv_gather_kernel<64, 64, 32, 32, 16, MODE, BN, 2>), grid, dim3(256), 0, s, a); break;
    case 14: hipLaunchKernelGGL((conv_gather_kernel<32, 64, 16, 32, 16, MODE, BN, 2>), grid, dim3(256), 0, s, a); break;
    case 15: hipLaunchKernelGGL((conv_gather_kernel<32, 64, 16, 32, 32, MODE, BN, 2>), grid, dim3(256), 0, s, a); break;
    case 16: hipLaunchKernelGGL((conv_gather_kernel<32, 64, 16, 32, 64, MODE, BN, 2>), grid, dim3(256), 0, s, a); break;
    default: hipLaunchKernelGGL((conv_gather_kernel<64, 128, 32, 64, 32, MODE, BN, 2>), grid, dim3(256), 0, s, a); break;
  }
}
// Tap-major tiles reading the filter in place (wplace_tile: whole runs of four k per thread, not the streaming tile);
// the direct-to-LDS tiles run as the staged kernel of their shape, as in gather_dispatch.
static void gather_inplace_dispatch(int ti, const GatherArgs& a, dim3 grid, hipStream_t s) {
  constexpr int M = kTapInPlace;
  switch (ti) {
    case 0: hipLaunchKernelGGL((conv_gather_kernel<64, 256, 64, 64, 16, M, false, 2>), grid, dim3(256), 0, s, a); break;
    case 1: hipLaunchKernelGGL((conv_gather_kernel<128, 128, 64, 64, 16, M, false, 2>), grid, dim3(256), 0, s, a); break;
    case 6: hipLaunchKernelGGL((conv_gather_kernel<64, 64, 32, 32, 64, M, false, 2>), grid, dim3(256), 0, s, a); break;
    case 8: hipLaunchKernelGGL((conv_gather_kernel<128, 64, 64, 32, 32, M, false, 2>), grid, dim3(256), 0, s, a); break;
    case 2: case 10: hipLaunchKernelGGL((conv_gather_kernel<64, 128, 32, 64, 16, M, false, 2>), grid, dim3(256), 0, s, a); break;
    case 7: case 12: hipLaunchKernelGGL((conv_gather_kernel<64, 128, 32, 64, 32, M, false, 2>), grid, dim3(256), 0, s, a); break;
    case 15: hipLaunchKernelGGL((conv_gather_kernel<32, 64, 16, 32, 32, M, false, 2>), grid, dim3(256), 0, s, a); break;
    case 16: hipLaunchKernelGGL((conv_gather_kernel<32, 64, 16, 32, 64, M, false, 2>), grid, dim3(256), 0, s, a); break;
    default: hipLaunchKernelGGL((conv_gather_kernel<64, 64, 32, 32, 16, M, false, 2>), grid, dim3(256), 0, s, a); break;  // 5, 9, 11
  }
}
static void gather_dl_dispatch(int ti, const GatherArgs& a, dim3 grid, hipStream_t s) {
  switch (ti) {
    case 9: hipLaunchKernelGGL((conv_gather_dl_kernel<64, 32, 32, 16, 4>), grid, dim3(256), 0, s, a); break;
    case 10: hipLaunchKernelGGL((conv_gather_dl_kernel<128, 32, 64, 16, 3>), grid, dim3(256), 0, s, a); break;
    case 11: hipLaunchKernelGGL((conv_gather_dl_kernel<64, 32, 32, 32, 3>), grid, dim3(256), 0, s, a); break;
    default: hipLaunchKernelGGL((conv_gather_dl_kernel<128, 32, 64, 32, 2>), grid, dim3(256), 0, s, a); break;
  }
}

// Channels-last gathers: the staged tiles 0 .. 8 (the tile's K-block divides the source channels).
static void gather_nhwc_dispatch(int ti, const GatherArgs& a, dim3 grid, hipStream_t s) {
  constexpr int M = kNhwc;
  switch (ti) {
    case 0: hipLaunchKernelGGL((conv_gather_kernel<64, 256, 64, 64, 16, M, false, 2>), grid, dim3(256), 0, s, a); break;
    case 1: hipLaunchKernelGGL((conv_gather_kernel<128, 128, 64, 64, 16, M, false, 2>), grid, dim3(256), 0, s, a); break;
    case 2: hipLaunchKernelGGL((conv_gather_kernel<64, 128, 32, 64, 16, M, false, 2>), grid, dim3(256), 0, s, a); break;
    case 3: hipLaunchKernelGGL((conv_gather_kernel<32, 256, 32, 64, 16, M, false, 2>), grid, dim3(256), 0, s, a); break;
    case 4: hipLaunchKernelGGL((conv_gather_kernel<16, 256, 16, 64, 16, M, false, 2>), grid, dim3(256), 0, s, a); break;
    case 6: hipLaunchKernelGGL((conv_gather_kernel<64, 64, 32, 32, 64, M, false, 2>), grid, dim3(256), 0, s, a); break;
    case 7: hipLaunchKernelGGL((conv_gather_kernel<64, 128, 32, 64, 32, M, false, 2>), grid, dim3(256), 0, s, a); break;
    case 8: hipLaunchKernelGGL((conv_gather_kernel<128, 64, 64, 32, 32, M, false, 2>), grid, dim3(256), 0, s, a); break;
    default: hipLaunchKernelGGL((conv_gather_kernel<64, 64, 32, 32, 16, M, false, 2>), grid, dim3(256), 0, s, a); break;
  }
}

// Tap-major order needs whole K-blocks of channels (so K has no tail); the BN loader keeps the channel-major order.
static bool gather_tap_major(int64_t c, bool bn, int bk) { return !bn && c % bk == 0; }

// Tile and K split of a gather launch: P rows, Q columns (the largest phase), K the longest reduction, z phases.
struct GatherPlan {
  int tile;
  int64_t slices, kslice;
};
static const int kSliceChoices[] = {1, 2, 3, 4, 6, 8, 12, 16, 24, 32, 48, 64};

// Estimated makespan in clocks, over tiles and slice counts:
// - workgroups run two per CU at ~34 fp32 FMA/clock each times the tile's efficiency, or ~1.6x that alone on a CU;
// - a K-block takes at least ~2000 clocks alone on a CU (~1000 with a second workgroup to hide behind): the operand
//   loads' latency, which only deeper K-blocks amortize;
// - each workgroup carries ~2 K-blocks of fixed cost (prologue, epilogue); a split needs >= 96 K per slice;
// - a split pays the partial round trip through HBM (~1.7 KB/clock) and one more launch (~7000 clocks).
// `fixed` (a tuned or requested plan) replaces the estimate: its slice count is rounded to whole K-blocks per slice.
// nhwc_c > 0: a channels-last gather over nhwc_c source channels, which runs the staged tiles 0 .. kNhwcTiles - 1 whose
// K-block divides nhwc_c (a fixed plan outside them runs as tile kNhwcDefault).
constexpr int kNhwcTiles = 9, kNhwcDefault = 5;
static bool nhwc_tile_ok(int t, int64_t c) { return t >= 0 && t < kNhwcTiles && c % kGatherTiles[t].bk == 0; }
static GatherPlan gather_plan(int64_t P, int64_t Q, int64_t K, int64_t z, const omt_conv_plan* fixed,
                              int64_t nhwc_c = 0) {
  const int64_t kk = K > 0 ? K : 1;
  if (fixed) {
    const int tile = nhwc_c && !nhwc_tile_ok(fixed->tile, nhwc_c) ? kNhwcDefault : fixed->tile;
    const int64_t nkb = cdiv(kk, gtile(tile).bk);
    const int64_t kb = cdiv(nkb, std::max<int64_t>(1, std::min<int64_t>(fixed->slices, nkb)));
    return {tile, cdiv(nkb, kb), kb * gtile(tile).bk};
  }
  GatherPlan best{nhwc_c ? kNhwcDefault : 0, 1, cdiv(kk, 16) * 16};
  double best_cost = 1e300;
  for (int ti = 0; ti < kNGather; ++ti) {
    const Tile& tl = kGatherTiles[ti];
    if (tl.stream) continue;  // chosen by tuning only
    if (nhwc_c && !nhwc_tile_ok(ti, nhwc_c)) continue;
    const int64_t tiles = cdiv(P, tl.bp) * cdiv(Q, tl.bq) * z, nkb = cdiv(kk, tl.bk);
    for (int sc : kSliceChoices) {
      const int64_t kb = cdiv(nkb, sc);
      if (sc > 1 && kb * tl.bk < 96) break;
      const int64_t slices = cdiv(nkb, kb);
      if (slices != sc) continue;
      const int64_t blocks = tiles * slices;
      const bool alone = blocks <= kCUs;
      const double blk = std::max((double)tl.bp * tl.bq * tl.bk / (34.0 * tl.eff) / (alone ? 1.6 : 1.0),
                                  alone ? 2000.0 : 1000.0);
      double cost = blk * (kb + 2) * (alone ? 1.0 : (double)cdiv(blocks, 2 * kCUs));
      if (slices > 1) cost += 7000.0 + (double)(2 * slices) * P * Q * z * 4 / 1700.0;
      if (cost < best_cost * 0.999) {
        best_cost = cost;
        best = {ti, slices, kb * tl.bk};
      }
    }
  }
  return best;
}

static size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

// The row epilogue applies to one phase written in place (no stride grid, no split K) whose float4 runs of output
// pixels stay inside one image and are 16-byte aligned.
static bool rows_ok(const GatherArgs& a, bool split) {
  const Phase& p = a.ph[0];
  return !split && !a.d2s && a.nphase == 1 && p.os == 1 && p.oy0 == 0 && p.ox0 == 0 && a.YH == p.OH && a.YW == p.OW &&
         (p.OH * p.OW) % 4 == 0 && (uintptr_t)a.y % 16 == 0;
}
// Completes a gather launch's arguments for its plan: K slice length and, split over K, the partials `part` (the
// workspace of the plan's size). Returns the grid.
static dim3 gather_grid(GatherArgs& a, const GatherPlan& pl, int64_t n, int64_t maxq, float* part) {
  const Tile& tl = gtile(pl.tile);
  a.kslice = (int)pl.kslice;
  a.part = pl.slices > 1 ? part : nullptr;
  a.part_stride = n * a.P * a.YH * a.YW;
  a.tpw = 0;
  a.rows = rows_ok(a, pl.slices > 1);
  if (tl.stream == 2) {  // the shape's resident workgroups per CU; tl.bp output channels per workgroup at K 64, half
    const int sh = wst_shape(pl.tile), k64 = a.ph[0].K == 64;
    const int64_t ntq = cdiv(maxq, tl.bq), ntp = cdiv(a.P, k64 ? tl.bp : tl.bp / 2);
    a.tpw = (int)std::max<int64_t>(1, cdiv(ntq * ntp, kWstOcc[sh][k64 ? 0 : 1] * kCUs));
    return dim3((unsigned)cdiv(ntq, a.tpw), (unsigned)ntp, 1);
  }
  if (tl.stream) {  // a workgroup per resident slot (four per CU, three with the statistics' registers)
    const int64_t ntq = cdiv(maxq, tl.bq), ntp = cdiv(a.P, tl.bp);
    a.tpw = (int)std::max<int64_t>(1, cdiv(ntq * ntp, (a.stats ? 3 : 4) * kCUs));
    return dim3((unsigned)cdiv(ntq, a.tpw), (unsigned)ntp, 1);
  }
  return dim3((unsigned)cdiv(maxq, tl.bq), (unsigned)cdiv(a.P, tl.bp), (unsigned)(a.nphase * pl.slices));
}
// The 1x1 streaming tile runs only where its kernel applies (one 1x1 stride-1 unpadded phase, the [P][K] filter in
// place or re-packed, no BN loader, no split K, whole K-blocks, float4 runs of output pixels inside one image and
// 16-byte aligned); anywhere else its plan runs as the staged tile of the same shape and K-block (tile 2).
static bool stream_ok(const GatherArgs& a, const GatherPlan& pl) {
  const Phase& p = a.ph[0];
  return !gcm(pl.tile) && pl.slices == 1 && !a.bn_mean && !a.wdirect && !a.wplace && p.KH == 1 && p.KW == 1 && p.S == 1 &&
         p.PH == 0 && p.PW == 0 && p.K % 16 == 0 && rows_ok(a, false);
}
// The filter-stationary 1x1 tile: the streaming tile's conditions, K of 64 or 128, no epilogue statistics, x 16-byte
// aligned (float4 loads of four pixels).
static bool wst_ok(const GatherArgs& a, const GatherPlan& pl) {
  const int K = a.ph[0].K;
  return stream_ok(a, pl) && (K == 64 || K == 128) && !a.stats && (uintptr_t)a.x % 16 == 0 &&
         (int64_t)a.ph[0].Q * a.P * 4 <= kMaxBufBytes;
}
static GatherPlan eff_plan(const GatherArgs& a, GatherPlan pl) {
  if (gtile(pl.tile).stream == 2 && !wst_ok(a, pl)) pl.tile = pl.tile - pl.tile % kNGather + kStreamTile;
  if (gtile(pl.tile).stream && !stream_ok(a, pl)) pl.tile = pl.tile - pl.tile % kNGather + 2;
  return pl;
}
// Tap-major K order of a gather launch (the BN loader keeps the channel-major order).
static bool gather_uses_tap_major(const GatherArgs& a, const GatherPlan& pl) {
  return !a.bn_mean && !gcm(pl.tile) && gather_tap_major(a.C, false, gtile(pl.tile).bk);
}
// The slice sum of a split gather launch (blocks 0 if the plan does not split).
static GatherSum gather_sum_of(const GatherArgs& a, const GatherPlan& pl) {
  GatherSum r{};
  if (pl.slices <= 1) return r;
  r.part = a.part;
  r.y = a.y;
  r.total = a.part_stride;
  r.plane = (int64_t)a.YH * a.YW;
  r.slices = (int)pl.slices;
  r.P = a.P;
  r.bias = a.bias;
  r.relu = a.relu;
  r.nhwc = a.nhwc;
  r.vec4 = (a.nhwc ? r.total % 4 == 0 : r.plane % 4 == 0) && (uintptr_t)a.y % 16 == 0 && !a.d2s;
  r.d2s = a.d2s;
  r.d2s_ci = a.d2s_ci;
  r.img_h = a.d2s_h;
  r.img_w = a.d2s_w;
  r.grid_w = a.ph[0].OW;
  r.blocks = grid1d(r.vec4 ? r.total / 4 : r.total, 256, 8192);
  return r;
}
static int launch_gather_sum(const GatherSum& r, hipStream_t s) {
  if (!r.blocks) return OMT_OK;
  if (r.vec4)
    hipLaunchKernelGGL(gather_reduce_kernel<4>, dim3((unsigned)r.blocks), dim3(256), 0, s, r);
  else
    hipLaunchKernelGGL(gather_reduce_kernel<1>, dim3((unsigned)r.blocks), dim3(256), 0, s, r);
  return launch_check("gather_reduce_kernel");
}

// Launches the gather (and, split over K, the slice reduce); `part` is the partial workspace of the plan's size. With
// `unsummed` set to a slice limit, a launch split into at most that many slices leaves its partials unsummed; the
// count is reported back there (1: y was written).
static int run_gather(GatherArgs& a, const GatherPlan& plan, int64_t n, int64_t maxq, float* part, hipStream_t s,
                      int* unsummed = nullptr) {
  const GatherPlan pl = eff_plan(a, plan);
  if (unsummed) {
    const int lim = *unsummed;
    *unsummed = 1;
    if (pl.slices > 1 && pl.slices <= lim) *unsummed = (int)pl.slices;
    else unsummed = nullptr;
  }
  const dim3 grid = gather_grid(a, pl, n, maxq, part);
  if (gtile(pl.tile).stream == 2) {
    const bool k64 = a.ph[0].K == 64;
    switch (wst_shape(pl.tile)) {
      case 0:
        if (k64) hipLaunchKernelGGL((conv1x1_wst_kernel<64, 4, 32, kWstOcc[0][0]>), grid, dim3(256), 0, s, a, a.tpw);
        else hipLaunchKernelGGL((conv1x1_wst_kernel<128, 2, 32, kWstOcc[0][1]>), grid, dim3(256), 0, s, a, a.tpw);
        break;
      case 1:
        if (k64) hipLaunchKernelGGL((conv1x1_wst_kernel<64, 2, 32, kWstOcc[1][0]>), grid, dim3(256), 0, s, a, a.tpw);
        else hipLaunchKernelGGL((conv1x1_wst_kernel<128, 1, 32, kWstOcc[1][1]>), grid, dim3(256), 0, s, a, a.tpw);
        break;
      default:
        if (k64) hipLaunchKernelGGL((conv1x1_wst_kernel<64, 2, 64, kWstOcc[2][0]>), grid, dim3(256), 0, s, a, a.tpw);
        else hipLaunchKernelGGL((conv1x1_wst_kernel<128, 1, 64, kWstOcc[2][1]>), grid, dim3(256), 0, s, a, a.tpw);
    }
    return launch_check("conv1x1_wst_kernel");
  }
  if (gtile(pl.tile).stream) {
    if (a.stats)
      hipLaunchKernelGGL((conv1x1_stream_kernel<64, 128, 32, 64, true>), grid, dim3(256), 0, s, a, a.tpw);
    else
      hipLaunchKernelGGL((conv1x1_stream_kernel<64, 128, 32, 64, false>), grid, dim3(256), 0, s, a, a.tpw);
    return launch_check("conv1x1_stream_kernel");
  }
  if (a.bn_mean)
    gather_dispatch<kGeneric, true>(pl.tile % kNGather, a, grid, s);
  else if (a.wplace)
    gather_inplace_dispatch(pl.tile % kNGather, a, grid, s);
  else if (gather_uses_tap_major(a, pl) && gtile(pl.tile).ns && (uintptr_t)a.w % 16 == 0 && !a.d2s)
    gather_dl_dispatch(pl.tile % kNGather, a, grid, s);
  else if (gather_uses_tap_major(a, pl))
    gather_dispatch<kTapMajor, false>(pl.tile % kNGather, a, grid, s);
  else
    gather_dispatch<kGeneric, false>(pl.tile % kNGather, a, grid, s);
  if (int st = launch_check("conv_gather_kernel")) return st;
  if (unsummed) return OMT_OK;  // the partials stay for the caller
  return launch_gather_sum(gather_sum_of(a, pl), s);
}

static bool dense_geo_ok(const omt_conv_geo* g) {
  return g->n >= 1 && g->ci >= 1 && g->co >= 1 && g->ks >= 1 && g->ks <= 11 && g->stride >= 1 && g->stride <= 4 &&
         g->pad >= 0 && g->pad <= g->ks && g->oh >= 1 && g->ow >= 1 &&
         g->oh == (g->ih + 2 * g->pad - g->ks) / g->stride + 1 && g->ow == (g->iw + 2 * g->pad - g->ks) / g->stride + 1;
}

// Offsets inside the kernels are 32-bit: every tensor the kernels read or write must stay below 2 GiB.
static bool fits_i32(const omt_conv_geo* g) {
  return g->n * g->ci * g->ih * g->iw * 4 <= kMaxBufBytes && g->n * g->co * g->oh * g->ow * 4 <= kMaxBufBytes &&
         g->co * g->ci * g->ks * g->ks * 4 <= kMaxBufBytes;
}

// ---- batches past 2 GiB ------------------------------------------------------------------------------------------
//
// A batch whose input or output reaches 2 GiB runs as consecutive batch chunks that each fit the 32-bit offsets (the
// batch index is the outermost dimension in both memory formats, so a chunk is a contiguous run of images). Forward
// and grad input convolve chunk by chunk; grad weight writes each chunk's filter gradient to the workspace and sums
// the chunks in chunk order. One image and the filter must each stay below 2 GiB. Chunks are as equal as the batch
// allows (at most two sizes: the first count - 1 chunks, then the last), and each runs under its own geometry's plan.
struct Chunks {
  int64_t count, size;  // count 1: the batch fits as it is; count 0: one image or the filter does not fit
};
static Chunks batch_chunks(const omt_conv_geo* g) {
  if (fits_i32(g)) return {1, g->n};
  const int64_t img = std::max(g->ci * g->ih * g->iw, g->co * g->oh * g->ow) * 4;
  if (img > kMaxBufBytes || g->co * g->ci * g->ks * g->ks * 4 > kMaxBufBytes) return {0, 0};
  const int64_t count = cdiv(g->n, kMaxBufBytes / img);
  return {count, cdiv(g->n, count)};
}
static omt_conv_geo chunk_geo(const omt_conv_geo* g, const Chunks& c, int64_t i) {
  omt_conv_geo r = *g;
  r.n = std::min(c.size, g->n - i * c.size);
  return r;
}
// The largest of the chunks' workspaces by `one`, the workspace of a geometry that fits (0 when nothing fits).
template <class F>
static size_t chunks_max(const omt_conv_geo* g, F one) {
  const Chunks c = batch_chunks(g);
  if (!c.count) return 0;
  if (c.count == 1) return one(g);
  const omt_conv_geo a = chunk_geo(g, c, 0), b = chunk_geo(g, c, c.count - 1);
  return std::max(one(&a), one(&b));
}
// Runs one(chunk geometry, first image) over the chunks in order.
template <class F>
static int for_chunks(const omt_conv_geo* g, const Chunks& c, F one) {
  for (int64_t i = 0; i < c.count; ++i) {
    const omt_conv_geo cg = chunk_geo(g, c, i);
    if (int st = one(&cg, i * c.size)) return st;
  }
  return OMT_OK;
}
// The geometry plans are kept and tuned under: the first chunk's when the batch is chunked.
static const omt_conv_geo* plan_geo(const omt_conv_geo* g, omt_conv_geo& tmp) {
  const Chunks c = batch_chunks(g);
  if (c.count <= 1) return g;
  tmp = chunk_geo(g, c, 0);
  return &tmp;
}

// Wgrad split: about four waves of workgroups per CU over the tiles, each slice at least four K-blocks long.
struct WgradPlan {
  int tile;
  int64_t slices, kslice;
};
// The estimate's slice count for tile ti.
static int64_t wgrad_model_slices(const omt_conv_geo* g, int ti) {
  const int64_t P = g->co, Q = g->ci * g->ks * g->ks, K = g->n * g->oh * g->ow;
  const Tile& tl = kWgradTiles[ti];
  const int64_t tiles = cdiv(P, tl.bp) * cdiv(Q, tl.bq);
  return std::max<int64_t>(1, std::min<int64_t>(cdiv(kCUs * 4, tiles), cdiv(K, 64 * 4)));
}
static bool cached_plan(int dir, const omt_conv_geo* g, omt_conv_plan* p);
static WgradPlan wgrad_plan(const omt_conv_geo* g, int dir = OMT_DIR_WGRAD) {
  const int64_t P = g->co, Q = g->ci * g->ks * g->ks, K = g->n * g->oh * g->ow;
  omt_conv_plan cp;
  int ti;
  int64_t slices;
  if (cached_plan(dir, g, &cp)) {
    ti = cp.tile;
    slices = std::max<int64_t>(1, std::min<int64_t>(cp.slices, cdiv(K, 64)));
  } else {
    ti = pick_tile(kWgradTiles, P, Q, 1, kCUs * 2);
    slices = wgrad_model_slices(g, ti);
  }
  const int64_t kslice = cdiv(cdiv(K, slices), 64) * 64;
  return {ti, cdiv(K, kslice), kslice};
}

template <int MODE>
static void wgrad_dispatch(int ti, const WgradArgs& a, dim3 grid, hipStream_t s) {
  switch (ti) {
    case 0: hipLaunchKernelGGL((conv_wgrad_kernel<64, 128, 32, 64, MODE, 1>), grid, dim3(256), 0, s, a); break;
    case 1: hipLaunchKernelGGL((conv_wgrad_kernel<128, 64, 32, 64, MODE, 1>), grid, dim3(256), 0, s, a); break;
    case 2: hipLaunchKernelGGL((conv_wgrad_kernel<64, 64, 32, 32, MODE, 2>), grid, dim3(256), 0, s, a); break;
    default: hipLaunchKernelGGL((conv_wgrad_kernel<32, 128, 16, 64, MODE, 2>), grid, dim3(256), 0, s, a); break;
  }
}

template <bool NARROW>
static void wgrad_nhwc_dispatch(int ti, const WgradArgs& a, dim3 grid, hipStream_t s) {
  switch (ti) {
    case 0: hipLaunchKernelGGL((conv_wgrad_nhwc_kernel<64, 128, 32, 64, 1, NARROW>), grid, dim3(256), 0, s, a); break;
    case 1: hipLaunchKernelGGL((conv_wgrad_nhwc_kernel<128, 64, 32, 64, 1, NARROW>), grid, dim3(256), 0, s, a); break;
    case 2: hipLaunchKernelGGL((conv_wgrad_nhwc_kernel<64, 64, 32, 32, 2, NARROW>), grid, dim3(256), 0, s, a); break;
    default: hipLaunchKernelGGL((conv_wgrad_nhwc_kernel<32, 128, 16, 64, 2, NARROW>), grid, dim3(256), 0, s, a); break;
  }
}

// ---- plan cache: the tile and K split per (direction, geometry), set by tuning --------------------------------

struct PlanKey {
  int dir;
  int64_t n, ci, co, ih, iw, oh, ow, ks, stride, pad;
  auto tie() const { return std::tie(dir, n, ci, co, ih, iw, oh, ow, ks, stride, pad); }
  bool operator<(const PlanKey& o) const { return tie() < o.tie(); }
};
static std::mutex g_plan_mu;
static std::map<PlanKey, omt_conv_plan> g_plans;
// The candidates under test while tuning, per direction (both dgrad and wgrad when the backward is tuned jointly).
constexpr int kNDirs = 6;  // OMT_DIR_FWD .. OMT_DIR_WGRAD_NHWC
static thread_local const omt_conv_plan* t_force[kNDirs] = {};

static PlanKey key_of(int dir, const omt_conv_geo* g) {
  return {dir, g->n, g->ci, g->co, g->ih, g->iw, g->oh, g->ow, g->ks, g->stride, g->pad};
}
static bool cached_plan(int dir, const omt_conv_geo* g, omt_conv_plan* p) {
  if (t_force[dir]) {
    *p = *t_force[dir];
    return true;
  }
  std::lock_guard<std::mutex> lk(g_plan_mu);
  auto it = g_plans.find(key_of(dir, g));
  if (it == g_plans.end()) return false;
  *p = it->second;
  return true;
}
static bool wgrad_dir(int dir) { return dir == OMT_DIR_WGRAD || dir == OMT_DIR_WGRAD_NHWC; }
static int num_tiles(int dir) {
  if (wgrad_dir(dir)) return (int)(sizeof(kWgradTiles) / sizeof(kWgradTiles[0]));
  return dir == OMT_DIR_FWD_NHWC || dir == OMT_DIR_DGRAD_NHWC ? kNhwcTiles : 3 * kNGather;
}

}  // namespace omt

using namespace omt;

static GatherPlan fwd_plan(const omt_conv_geo* g) {
  omt_conv_plan cp;
  const bool have = cached_plan(OMT_DIR_FWD, g, &cp);
  return gather_plan(g->co, g->n * g->oh * g->ow, g->ci * g->ks * g->ks, 1, have ? &cp : nullptr);
}
// Forward workspace: the tap-major filter (when the plan's K-block divides C and ks > 1), then, 256-byte aligned,
// the split-K partials.
static size_t fwd_pack_bytes(const omt_conv_geo* g, const GatherPlan& pl) {
  if (g->ks == 1 || gcm(pl.tile) || wplace_tile(pl.tile) || !gather_tap_major(g->ci, false, gtile(pl.tile).bk))
    return 0;
  return (size_t)(g->co * g->ci * g->ks * g->ks) * sizeof(float);
}

static size_t fwd_workspace_one(const omt_conv_geo* g) {
  const GatherPlan pl = fwd_plan(g);
  const size_t part = pl.slices > 1 ? (size_t)(pl.slices * g->n * g->co * g->oh * g->ow) * sizeof(float) : 0;
  return part ? align256(fwd_pack_bytes(g, pl)) + part : fwd_pack_bytes(g, pl);
}

OMT_EXPORT size_t omt_conv_fwd_workspace(const omt_conv_geo* g) {
  return g && dense_geo_ok(g) ? chunks_max(g, fwd_workspace_one) : 0;
}

// The forward GEMM over a batch that fits the 32-bit offsets; with `unsummed` (no bias, epilogue or BN loader), a plan
// that splits K leaves its partials in the workspace (*parts) and sets *unsummed to its slice count, else writes y and
// sets it to 1.
static int conv_fwd_one(const omt_conv_geo* g, const float* x, const float* w, const float* bias, unsigned epilogue,
                        const float* bn_mean, const float* bn_var, const float* bn_gamma, const float* bn_beta,
                        float bn_eps, float* y, void* workspace, size_t workspace_bytes, void* stream,
                        const float** parts, int* unsummed, double* stats = nullptr, int* groups = nullptr) {
  const bool bn = bn_mean || bn_var || bn_gamma || bn_beta;
  if (bn && !(bn_mean && bn_var && bn_gamma && bn_beta))
    return fail(OMT_INVALID, "omt_conv_fwd: BN loader needs mean, var, gamma and beta");
  if ((epilogue & OMT_EPI_BIAS) && !bias) return fail(OMT_INVALID, "omt_conv_fwd: bias epilogue without bias");
  const size_t need = omt_conv_fwd_workspace(g);
  if (need && (!workspace || workspace_bytes < need))
    return fail(OMT_INVALID, "omt_conv_fwd: workspace of %zu bytes needed", need);
  hipStream_t s = stream_of(stream);
  const GatherPlan pl = fwd_plan(g);
  if (stats && pl.slices > 1) return fail(OMT_UNSUPPORTED, "omt_conv_fwd_stats: the plan splits K");
  GatherArgs a{};
  a.x = x;
  a.w = w;
  // tap-major order: re-pack the filter to [co][ky][kx][ci] (1x1 filters already are)
  if (!bn && fwd_pack_bytes(g, pl)) {
    const int total = (int)(g->co * g->ci * g->ks * g->ks);
    hipLaunchKernelGGL(pack_tapmajor_kernel, dim3(grid1d(total, 256, 4096)), dim3(256), 0, s, w, (float*)workspace,
                       (int)g->co, (int)g->ci, (int)(g->ks * g->ks));
    if (int st = launch_check("pack_tapmajor_kernel")) return st;
    a.w = (const float*)workspace;
  }
  if (!bn && g->ks > 1 && wplace_tile(pl.tile) && gather_tap_major(g->ci, false, gtile(pl.tile).bk)) {
    a.wplace = 1;  // A[co][(ky, kx, ci)] = w[co][ci][ky][kx]
    a.ks = (int)g->ks;
    a.w_rowst = (uint32_t)(g->ci * g->ks * g->ks * 4);
    a.w_cst = (uint32_t)(g->ks * g->ks * 4);
  }
  a.bias = (epilogue & OMT_EPI_BIAS) ? bias : nullptr;
  a.bn_mean = bn ? bn_mean : nullptr;
  a.bn_var = bn_var;
  a.bn_gamma = bn_gamma;
  a.bn_beta = bn_beta;
  a.bn_eps = bn_eps;
  a.relu = (epilogue & OMT_EPI_RELU) ? 1 : 0;
  a.y = y;
  a.x_bytes = (uint32_t)(g->n * g->ci * g->ih * g->iw * 4);
  a.w_bytes = (uint32_t)(g->co * g->ci * g->ks * g->ks * 4);
  a.C = (int)g->ci;
  a.H = (int)g->ih;
  a.W = (int)g->iw;
  a.P = (int)g->co;
  a.YH = (int)g->oh;
  a.YW = (int)g->ow;
  a.nphase = 1;
  Phase& p = a.ph[0];
  p.KH = p.KW = (int)g->ks;
  p.S = (int)g->stride;
  p.PH = p.PW = (int)g->pad;
  p.OH = (int)g->oh;
  p.OW = (int)g->ow;
  p.K = (int)(g->ci * g->ks * g->ks);
  p.Q = (int)(g->n * g->oh * g->ow);
  p.os = 1;
  p.oy0 = p.ox0 = 0;
  p.woff = 0;
  p.div_ohw = make_fastdiv((uint32_t)(g->oh * g->ow));
  p.div_ow = make_fastdiv((uint32_t)g->ow);
  p.div_kk = make_fastdiv((uint32_t)(g->ks * g->ks));
  p.div_kw = make_fastdiv((uint32_t)g->ks);
  a.div_c = make_fastdiv((uint32_t)a.C);
  float* part = (float*)((char*)workspace + align256(fwd_pack_bytes(g, pl)));
  if (parts) *parts = part;
  if (stats) {  // the statistics come from the epilogue of an unsplit plan (checked above, before any launch)
    a.stats = stats;  // first: the tile that runs depends on it (the filter-stationary 1x1 tiles have no statistics)
    const GatherPlan ep = eff_plan(a, pl);
    a.stats_groups = (int)cdiv(p.Q, gtile(ep.tile).wq);
    *groups = a.stats_groups;
  }
  return run_gather(a, pl, g->n, p.Q, part, s, unsummed);
}

// The forward GEMM, chunk by chunk past 2 GiB (a chunked batch is always summed: *unsummed 1).
static int conv_fwd_impl(const omt_conv_geo* g, const float* x, const float* w, const float* bias, unsigned epilogue,
                         const float* bn_mean, const float* bn_var, const float* bn_gamma, const float* bn_beta,
                         float bn_eps, float* y, void* workspace, size_t workspace_bytes, void* stream,
                         const float** parts, int* unsummed) {
  if (!g || !x || !w || !y) return fail(OMT_INVALID, "omt_conv_fwd: null pointer");
  if (!dense_geo_ok(g)) return fail(OMT_UNSUPPORTED, "omt_conv_fwd: geometry not covered (ks 1..11, stride 1..4, pad 0..ks)");
  const Chunks ch = batch_chunks(g);
  if (!ch.count) return fail(OMT_UNSUPPORTED, "omt_conv_fwd: one image or the filter is 2 GiB or more");
  if (ch.count == 1)
    return conv_fwd_one(g, x, w, bias, epilogue, bn_mean, bn_var, bn_gamma, bn_beta, bn_eps, y, workspace,
                        workspace_bytes, stream, parts, unsummed);
  if (unsummed) *unsummed = 1;
  const int64_t xi = g->ci * g->ih * g->iw, yi = g->co * g->oh * g->ow;
  return for_chunks(g, ch, [&](const omt_conv_geo* c, int64_t n0) {
    return conv_fwd_one(c, x + n0 * xi, w, bias, epilogue, bn_mean, bn_var, bn_gamma, bn_beta, bn_eps, y + n0 * yi,
                        workspace, workspace_bytes, stream, nullptr, nullptr);
  });
}

OMT_EXPORT int omt_conv_fwd(const omt_conv_geo* g, const float* x, const float* w, const float* bias,
                            unsigned epilogue, const float* bn_mean, const float* bn_var, const float* bn_gamma,
                            const float* bn_beta, float bn_eps, float* y, void* workspace, size_t workspace_bytes,
                            void* stream) {
  return conv_fwd_impl(g, x, w, bias, epilogue, bn_mean, bn_var, bn_gamma, bn_beta, bn_eps, y, workspace,
                       workspace_bytes, stream, nullptr, nullptr);
}

OMT_EXPORT size_t omt_conv_fwd_stats_bytes(const omt_conv_geo* g) {
  if (!g || !dense_geo_ok(g)) return 0;
  return (size_t)(cdiv(g->n * g->oh * g->ow, 32) * g->co) * 2 * sizeof(double);
}

OMT_EXPORT int omt_conv_fwd_stats(const omt_conv_geo* g, const float* x, const float* w, float* y, double* stats,
                                  size_t stats_bytes, int* groups, void* workspace, size_t workspace_bytes,
                                  void* stream) {
  if (!g || !x || !w || !y || !stats || !groups) return fail(OMT_INVALID, "omt_conv_fwd_stats: null pointer");
  *groups = 0;
  if (!dense_geo_ok(g) || !fits_i32(g))
    return fail(OMT_UNSUPPORTED, "omt_conv_fwd_stats: geometry not covered (a batch below 2 GiB)");
  if (stats_bytes < omt_conv_fwd_stats_bytes(g))
    return fail(OMT_INVALID, "omt_conv_fwd_stats: %zu bytes of statistics needed", omt_conv_fwd_stats_bytes(g));
  return conv_fwd_one(g, x, w, nullptr, 0, nullptr, nullptr, nullptr, nullptr, 0.f, y, workspace, workspace_bytes,
                      stream, nullptr, nullptr, stats, groups);
}

OMT_EXPORT int omt_conv_fwd_unsummed(const omt_conv_geo* g, const float* x, const float* w, float* y, void* workspace,
                                     size_t workspace_bytes, int max_slices, const float** partials, int* slices,
                                     void* stream) {
  if (!partials || !slices) return fail(OMT_INVALID, "omt_conv_fwd_unsummed: null pointer");
  *partials = nullptr;
  int lim = max_slices < 1 ? 1 : max_slices;  // in: the slice limit; out: the slices left unsummed, or 1
  const int st = conv_fwd_impl(g, x, w, nullptr, 0, nullptr, nullptr, nullptr, nullptr, 0.f, y, workspace,
                               workspace_bytes, stream, partials, &lim);
  *slices = lim;
  if (lim == 1) *partials = nullptr;
  return st;
}

// Stride-phase table of the grad-input GEMMs (see the top of this file).
static int dgrad_phases(const omt_conv_geo* g, GatherArgs& a, PackArgs& pk, int64_t& maxq) {
  const int s = (int)g->stride, ks = (int)g->ks, pad = (int)g->pad;
  int nph = 0, woff = 0;
  maxq = 0;
  for (int py = 0; py < s; ++py)
    for (int px = 0; px < s; ++px) {
      const int hi = (int)cdiv(g->ih - py, s), wi = (int)cdiv(g->iw - px, s);
      const int ky0 = (py + pad) % s, kx0 = (px + pad) % s;
      const int jy = ky0 < ks ? (int)cdiv(ks - ky0, s) : 0, jx = kx0 < ks ? (int)cdiv(ks - kx0, s) : 0;
      const int qy = (py + pad - ky0) / s, qx = (px + pad - kx0) / s;
      Phase& p = a.ph[nph];
      p.KH = jy > 0 ? jy : 1;
      p.KW = jx > 0 ? jx : 1;
      p.S = 1;
      p.PH = jy - 1 - qy;
      p.PW = jx - 1 - qx;
      p.OH = hi > 0 ? hi : 1;
      p.OW = wi > 0 ? wi : 1;
      p.K = (int)g->co * jy * jx;  // 0: no tap reaches this phase, it writes zeros
      p.Q = (hi > 0 && wi > 0) ? (int)g->n * hi * wi : 0;
      p.os = s;
      p.oy0 = py;
      p.ox0 = px;
      p.woff = woff;
      p.ky0 = ky0;
      p.kx0 = kx0;
      p.div_ohw = make_fastdiv((uint32_t)(p.OH * p.OW));
      p.div_ow = make_fastdiv((uint32_t)p.OW);
      p.div_kk = make_fastdiv((uint32_t)(p.KH * p.KW));
      p.div_kw = make_fastdiv((uint32_t)p.KW);
      pk.ph[nph] = PackPhase{ky0, kx0, jy, jx, woff};
      woff += (int)(g->ci * g->co) * jy * jx;
      if (p.Q > maxq) maxq = p.Q;
      ++nph;
    }
  a.nphase = nph;
  pk.nphase = nph;
  return woff;
}

// Grad input as one super-pixel GEMM. With few grad-input channels C and a stride s > 1, each of the s^2 stride phases
// fills only C of an MFMA tile's 16 rows. Side by side, the phases' s^2 C rows over one L x L window of gy (the union
// of every phase's taps, zero where a phase has none) fill whole tiles, for L^2 / (taps of a phase) times the FLOPs:
// AlexNet conv1's grad input (C = 3, s = 4, 11 x 11) becomes 48 rows over a 4 x 4 window, 2.2x the FLOPs on 16x the
// rows per tile.
static bool dgrad_d2s(const omt_conv_geo* g) {
  return g->stride > 1 && g->ci <= 4 && g->stride * g->stride * g->ci <= 64;
}
// The window: gy rows i + r for r in [lo, hi] over all phases (phase py reaches rows i + qy - a', a' < jy); L rows
// starting at PH = -lo above the grid row.
static void d2s_window(const omt_conv_geo* g, int& L, int& PH) {
  const int s = (int)g->stride, ks = (int)g->ks, pad = (int)g->pad;
  int lo = 1 << 30, hi = -(1 << 30);
  for (int py = 0; py < s; ++py) {
    const int ky0 = (py + pad) % s;
    if (ky0 >= ks) continue;
    const int jy = (int)cdiv(ks - ky0, s), qy = (py + pad - ky0) / s;
    lo = std::min(lo, qy - jy + 1);
    hi = std::max(hi, qy);
  }
  L = hi - lo + 1;
  PH = -lo;
}
static void dgrad_d2s_phase(const omt_conv_geo* g, GatherArgs& a, int64_t& maxq) {
  const int s = (int)g->stride;
  int L = 1, PH = 0;
  d2s_window(g, L, PH);
  Phase& p = a.ph[0];
  p = Phase{};
  p.KH = p.KW = L;
  p.S = 1;
  p.PH = p.PW = PH;
  p.OH = (int)cdiv(g->ih, s);
  p.OW = (int)cdiv(g->iw, s);
  p.K = (int)g->co * L * L;
  p.Q = (int)g->n * p.OH * p.OW;
  p.os = 1;
  p.div_ohw = make_fastdiv((uint32_t)(p.OH * p.OW));
  p.div_ow = make_fastdiv((uint32_t)p.OW);
  p.div_kk = make_fastdiv((uint32_t)(L * L));
  p.div_kw = make_fastdiv((uint32_t)L);
  a.nphase = 1;
  maxq = p.Q;
}

// Grad-input workspace: the per-phase packed filters, then, 256-byte aligned, the split-K partials.
static GatherPlan dgrad_plan(const omt_conv_geo* g) {
  GatherArgs a{};
  PackArgs pk{};
  int64_t maxq = 0, maxk = 0;
  omt_conv_plan cp;
  const bool have = cached_plan(OMT_DIR_DGRAD, g, &cp);
  if (dgrad_d2s(g)) {
    dgrad_d2s_phase(g, a, maxq);
    return gather_plan(g->stride * g->stride * g->ci, maxq, a.ph[0].K, 1, have ? &cp : nullptr);
  }
  dgrad_phases(g, a, pk, maxq);
  for (int i = 0; i < a.nphase; ++i) maxk = a.ph[i].K > maxk ? a.ph[i].K : maxk;
  return gather_plan(g->ci, maxq, maxk, a.nphase, have ? &cp : nullptr);
}

// Grad input re-packs its filter for the tap-major order only (the channel-major order reads w directly), and always
// in the super-pixel form.
static size_t dgrad_pack_bytes(const omt_conv_geo* g, const GatherPlan& pl) {
  if (dgrad_d2s(g)) {
    int L = 1, PH = 0;
    d2s_window(g, L, PH);
    return (size_t)(g->stride * g->stride * g->ci * g->co * L * L) * sizeof(float);
  }
  if (gcm(pl.tile) || wplace_tile(pl.tile) || !gather_tap_major(g->co, false, gtile(pl.tile).bk)) return 0;
  return (size_t)(g->co * g->ci * g->ks * g->ks) * sizeof(float);
}

static size_t dgrad_workspace_one(const omt_conv_geo* g) {
  const GatherPlan pl = dgrad_plan(g);
  const size_t pack = dgrad_pack_bytes(g, pl);
  // the super-pixel form keeps its partials on the ceil(ih / s) x ceil(iw / s) grid, s^2 ci rows
  const int64_t s = g->stride, plane = dgrad_d2s(g) ? s * s * g->ci * cdiv(g->ih, s) * cdiv(g->iw, s)
                                                    : g->ci * g->ih * g->iw;
  return pl.slices > 1 ? align256(pack) + (size_t)(pl.slices * g->n * plane) * sizeof(float) : pack;
}

OMT_EXPORT size_t omt_conv_dgrad_workspace(const omt_conv_geo* g) {
  return g && dense_geo_ok(g) ? chunks_max(g, dgrad_workspace_one) : 0;
}

// Geometry check of an entry point that runs whole batches only.
static int geo_check(const omt_conv_geo* g, const char* fn) {
  if (!dense_geo_ok(g)) return fail(OMT_UNSUPPORTED, "%s: geometry not covered", fn);
  if (!fits_i32(g)) return fail(OMT_UNSUPPORTED, "%s: a tensor of 2 GiB or more", fn);
  return OMT_OK;
}
// Geometry check of an entry point that runs a batch past 2 GiB in chunks: the chunks (count 1: the whole batch).
static int chunk_check(const omt_conv_geo* g, const char* fn, Chunks& c) {
  if (!dense_geo_ok(g)) return fail(OMT_UNSUPPORTED, "%s: geometry not covered", fn);
  c = batch_chunks(g);
  if (!c.count) return fail(OMT_UNSUPPORTED, "%s: one image or the filter is 2 GiB or more", fn);
  return OMT_OK;
}

// Grad-input launch arguments over `workspace` (of omt_conv_dgrad_workspace's size); launches the filter re-pack of the
// tap-major order. The gather itself is left to the caller (gather_grid, then a launch).
static int dgrad_prepare(const omt_conv_geo* g, const float* gy, const float* w, float* gx, void* workspace,
                         hipStream_t s, GatherArgs& a, GatherPlan& pl, int64_t& maxq, float*& part) {
  PackArgs pk{};
  a = GatherArgs{};
  const bool d2s = dgrad_d2s(g);
  const int packed = d2s ? 0 : dgrad_phases(g, a, pk, maxq);
  pl = dgrad_plan(g);
  const size_t pack = dgrad_pack_bytes(g, pl);
  if (d2s) {
    dgrad_d2s_phase(g, a, maxq);
    PackD2S pd{};
    pd.w = w;
    pd.out = (float*)workspace;
    pd.CO = (int)g->co;
    pd.CI = (int)g->ci;
    pd.KS = (int)g->ks;
    pd.S = (int)g->stride;
    pd.PAD = (int)g->pad;
    pd.L = a.ph[0].KH;
    pd.PH = a.ph[0].PH;
    pd.tap_major = !gcm(pl.tile) && gather_tap_major(g->co, false, gtile(pl.tile).bk);
    const int64_t total = (int64_t)(pack / sizeof(float));
    hipLaunchKernelGGL(pack_d2s_weights_kernel, dim3(grid1d(total, 256, 4096)), dim3(256), 0, s, pd);
    if (int st = launch_check("pack_d2s_weights_kernel")) return st;
    a.w = (const float*)workspace;
    a.w_bytes = (uint32_t)pack;
    a.d2s = (int)g->stride;
    a.d2s_ci = (int)g->ci;
  } else if (pack) {
    pk.w = w;
    pk.out = (float*)workspace;
    pk.CO = (int)g->co;
    pk.CI = (int)g->ci;
    pk.KS = (int)g->ks;
    pk.S = (int)g->stride;
    pk.tap_major = 1;
    hipLaunchKernelGGL(pack_dgrad_weights_kernel, dim3(grid1d(packed, 256, 4096)), dim3(256), 0, s, pk);
    if (int st = launch_check("pack_dgrad_weights_kernel")) return st;
    a.w = (const float*)workspace;
    a.w_bytes = (uint32_t)(packed * 4);
  } else {
    a.w = w;
    a.w_bytes = (uint32_t)(g->co * g->ci * g->ks * g->ks * 4);
    a.ks = (int)g->ks;
    a.s = (int)g->stride;
    if (wplace_tile(pl.tile) && gather_tap_major(g->co, false, gtile(pl.tile).bk)) {
      a.wplace = 2;  // A[ci][(a', b', co)] = w[co][ci][ky0 + s (KH - 1 - a')][kx0 + s (KW - 1 - b')]
      a.w_rowst = (uint32_t)(g->ks * g->ks * 4);
      a.w_cst = (uint32_t)(g->ci * g->ks * g->ks * 4);
    } else {
      a.wdirect = 1;
    }
  }
  a.x = gy;
  a.y = gx;
  a.x_bytes = (uint32_t)(g->n * g->co * g->oh * g->ow * 4);
  a.C = (int)g->co;
  a.H = (int)g->oh;
  a.W = (int)g->ow;
  a.P = (int)(d2s ? g->stride * g->stride * g->ci : g->ci);  // GEMM rows
  a.YH = d2s ? a.ph[0].OH : (int)g->ih;  // super-pixel form: the grid (its partials' plane); the image below
  a.YW = d2s ? a.ph[0].OW : (int)g->iw;
  a.d2s_h = (int)g->ih;
  a.d2s_w = (int)g->iw;
  a.div_c = make_fastdiv((uint32_t)a.C);
  part = workspace ? (float*)((char*)workspace + align256(pack)) : nullptr;
  return OMT_OK;
}

OMT_EXPORT int omt_conv_dgrad(const omt_conv_geo* g, const float* gy, const float* w, float* gx, void* workspace,
                              size_t workspace_bytes, void* stream) {
  if (!g || !gy || !w || !gx) return fail(OMT_INVALID, "omt_conv_dgrad: null pointer");
  Chunks ch;
  if (int st = chunk_check(g, "omt_conv_dgrad", ch)) return st;
  const size_t need = omt_conv_dgrad_workspace(g);
  if (need && (!workspace || workspace_bytes < need))
    return fail(OMT_INVALID, "omt_conv_dgrad: workspace of %zu bytes needed", need);
  hipStream_t s = stream_of(stream);
  const int64_t yi = g->co * g->oh * g->ow, xi = g->ci * g->ih * g->iw;
  return for_chunks(g, ch, [&](const omt_conv_geo* c, int64_t n0) {
    GatherArgs a;
    GatherPlan pl;
    int64_t maxq = 0;
    float* part = nullptr;
    if (int st = dgrad_prepare(c, gy + n0 * yi, w, gx + n0 * xi, workspace, s, a, pl, maxq, part)) return st;
    return run_gather(a, pl, c->n, maxq, part, s);
  });
}

static size_t wgrad_workspace_one(const omt_conv_geo* g) {
  WgradPlan pl = wgrad_plan(g);
  if (pl.slices <= 1) return 0;
  return (size_t)(pl.slices * g->co * g->ci * g->ks * g->ks) * sizeof(float);
}
// Workspace of a grad weight over batch chunks: the chunks' filter gradients [count][filter], then, 256-byte aligned,
// the largest workspace `one` gives a chunk.
template <class F>
static size_t wgrad_chunks_workspace(const omt_conv_geo* g, F one) {
  const Chunks c = batch_chunks(g);
  if (c.count <= 1) return c.count ? one(g) : 0;
  return align256((size_t)(c.count * g->co * g->ci * g->ks * g->ks) * sizeof(float)) + chunks_max(g, one);
}

OMT_EXPORT size_t omt_conv_wgrad_workspace(const omt_conv_geo* g) {
  return g && dense_geo_ok(g) ? wgrad_chunks_workspace(g, wgrad_workspace_one) : 0;
}

// Grad-weight launch arguments over `workspace` (of omt_conv_wgrad_workspace's size) and the launch's grid.
static dim3 wgrad_prepare(const omt_conv_geo* g, const float* x, const float* gy, float* gw, void* workspace,
                          WgradArgs& a, WgradPlan& pl, int dir = OMT_DIR_WGRAD) {
  pl = wgrad_plan(g, dir);
  a = WgradArgs{};
  a.x = x;
  a.gy = gy;
  a.out = pl.slices > 1 ? (float*)workspace : gw;
  a.x_bytes = (uint32_t)(g->n * g->ci * g->ih * g->iw * 4);
  a.gy_bytes = (uint32_t)(g->n * g->co * g->oh * g->ow * 4);
  a.C = (int)g->ci;
  a.H = (int)g->ih;
  a.W = (int)g->iw;
  a.P = (int)g->co;
  a.OH = (int)g->oh;
  a.OW = (int)g->ow;
  a.KS = (int)g->ks;
  a.S = (int)g->stride;
  a.PAD = (int)g->pad;
  a.Q = (int)(g->ci * g->ks * g->ks);
  a.K = (int)(g->n * g->oh * g->ow);
  a.kslice = (int)pl.kslice;
  a.div_ohw = make_fastdiv((uint32_t)(g->oh * g->ow));
  a.div_ow = make_fastdiv((uint32_t)g->ow);
  a.div_kk = make_fastdiv((uint32_t)(g->ks * g->ks));
  a.div_ks = make_fastdiv((uint32_t)g->ks);
  a.div_c = make_fastdiv((uint32_t)g->ci);
  a.step_ox = (int)(64 % g->ow);
  a.step_oy = (int)((64 / g->ow) % g->oh);
  a.step_n = (int)((64 / g->ow) / g->oh);
  const Tile& tl = kWgradTiles[pl.tile];
  return dim3((unsigned)cdiv(a.Q, tl.bq), (unsigned)cdiv(a.P, tl.bp), (unsigned)pl.slices);
}
// Tap-major column order of a grad-weight launch: each wave's BQ / 4 staged columns share one tap.
static bool wgrad_uses_tap_major(const omt_conv_geo* g, const WgradPlan& pl) {
  return g->ci % (kWgradTiles[pl.tile].bq / 4) == 0;
}
// The grad-weight GEMM of a plan in its loader mode: 16-byte loads of four reduction pixels for 1x1 stride-1 unpadded
// layers whose planes are a multiple of 4 (kPix4), else one pixel per lane in tap-major or channel-major order.
static void launch_wgrad_gemm(const omt_conv_geo* g, const WgradPlan& pl, const WgradArgs& a, dim3 grid,
                              hipStream_t s) {
  if (g->ks == 1 && g->stride == 1 && g->pad == 0 && (g->oh * g->ow) % 4 == 0)
    wgrad_dispatch<kPix4>(pl.tile, a, grid, s);
  else if (wgrad_uses_tap_major(g, pl))
    wgrad_dispatch<kTapMajor>(pl.tile, a, grid, s);
  else
    wgrad_dispatch<kGeneric>(pl.tile, a, grid, s);
}
// The slice sum of a split grad-weight launch (blocks 0 if the plan does not split).
static SplitSum wgrad_sum_of(const WgradArgs& a, const WgradPlan& pl, float* gw) {
  if (pl.slices <= 1) return SplitSum{};
  return split_sum_of(a.out, gw, (int64_t)a.P * a.Q, pl.slices);
}
static int launch_split_sum(const SplitSum& r, hipStream_t s) {
  if (!r.blocks) return OMT_OK;
  if (r.vec4)
    hipLaunchKernelGGL(split_reduce_kernel<4>, dim3((unsigned)r.blocks), dim3(256), 0, s, r);
  else
    hipLaunchKernelGGL(split_reduce_kernel<1>, dim3((unsigned)r.blocks), dim3(256), 0, s, r);
  return launch_check("split_reduce_kernel");
}

// The grad-weight GEMM and its slice sum over a workspace of the plan's size (already checked by the caller).
static int run_wgrad(const omt_conv_geo* g, const float* x, const float* gy, float* gw, void* workspace,
                     hipStream_t s) {
  WgradArgs a;
  WgradPlan pl;
  const dim3 grid = wgrad_prepare(g, x, gy, gw, workspace, a, pl);
  launch_wgrad_gemm(g, pl, a, grid, s);
  if (int st = launch_check("conv_wgrad_kernel")) return st;
  return launch_split_sum(wgrad_sum_of(a, pl, gw), s);
}

// Grad weight over batch chunks (more than one): one(chunk geometry, first image, filter gradient out, workspace) for
// each chunk into the workspace's chunk gradients, then their sum in chunk order into gw.
template <class F>
static int wgrad_chunks(const omt_conv_geo* g, const Chunks& ch, float* gw, void* workspace, hipStream_t s, F one) {
  const int64_t f = g->co * g->ci * g->ks * g->ks;
  float* parts = (float*)workspace;
  void* ws = (char*)workspace + align256((size_t)(ch.count * f) * sizeof(float));
  if (int st = for_chunks(g, ch, [&](const omt_conv_geo* c, int64_t n0) { return one(c, n0, parts + n0 / ch.size * f, ws); }))
    return st;
  return launch_split_sum(split_sum_of(parts, gw, f, ch.count), s);
}

OMT_EXPORT int omt_conv_wgrad(const omt_conv_geo* g, const float* x, const float* gy, float* gw, void* workspace,
                              size_t workspace_bytes, void* stream) {
  if (!g || !x || !gy || !gw) return fail(OMT_INVALID, "omt_conv_wgrad: null pointer");
  Chunks ch;
  if (int st = chunk_check(g, "omt_conv_wgrad", ch)) return st;
  const size_t need = omt_conv_wgrad_workspace(g);
  if (need && (!workspace || workspace_bytes < need))
    return fail(OMT_INVALID, "omt_conv_wgrad: workspace of %zu bytes needed", need);
  hipStream_t s = stream_of(stream);
  if (ch.count == 1) return run_wgrad(g, x, gy, gw, workspace, s);
  const int64_t xi = g->ci * g->ih * g->iw, yi = g->co * g->oh * g->ow;
  return wgrad_chunks(g, ch, gw, workspace, s, [&](const omt_conv_geo* c, int64_t n0, float* out, void* ws) {
    return run_wgrad(c, x + n0 * xi, gy + n0 * yi, out, ws, s);
  });
}

// ---- grad weight without allocation ------------------------------------------------------------------------------
//
// omt_conv_wgrad_noalloc keeps the split-K partials in `scratch`, a static device array the library owns: one copy per
// GPU, allocated with the code object and held until the process ends. Host code never passes `scratch` itself (on the
// host the name is a stand-in, not a device address): the first call on a device resolves that device's copy with
// hipGetSymbolAddress, with the device current, and every launch then takes that address. Every partial a slice sum
// reads was written by the same call's grad-weight launch, so the array needs no clearing; calls that overlap on one
// GPU share it and race.
static __device__ __align__(256) unsigned char scratch[OMT_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxScratchDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxScratchDevices];

// The current device's copy of `scratch` (resolved once per device).
static int scratch_of_current_device(void** out) {
  int dev = -1;
  OMT_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxScratchDevices) return fail(OMT_INVALID, "omt_conv_wgrad_noalloc: device %d", dev);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    // a first call may come under stream capture: the lookup runs in relaxed capture mode, which lets this thread
    // make the (non-stream) runtime call while a capture is in progress, then the caller's mode is restored
    void* p = nullptr;
    hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
    OMT_HIP(hipThreadExchangeStreamCaptureMode(&mode));
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    OMT_HIP(hipThreadExchangeStreamCaptureMode(&mode));
    OMT_HIP(e);
    if (!p) return fail(OMT_DEVICE_ERROR, "omt_conv_wgrad_noalloc: no address for the scratch array on device %d", dev);
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return OMT_OK;
}

OMT_EXPORT int omt_conv_wgrad_noalloc(const omt_conv_geo* g, const float* x, const float* gy, float* gw, void* stream) {
  if (!g || !x || !gy || !gw) return fail(OMT_INVALID, "omt_conv_wgrad_noalloc: null pointer");
  if (int st = geo_check(g, "omt_conv_wgrad_noalloc")) return st;
  const size_t need = omt_conv_wgrad_workspace(g);
  if (need > (size_t)OMT_NOALLOC_SCRATCH_BYTES)
    return fail(OMT_INVALID,
                "omt_conv_wgrad_noalloc: the plan's split-K partials need %zu bytes, more than the %zu-byte static "
                "scratch (use omt_conv_wgrad with a workspace, or a plan with fewer K slices)",
                need, (size_t)OMT_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  if (need)
    if (int st = scratch_of_current_device(&ws)) return st;
  return run_wgrad(g, x, gy, gw, ws, stream_of(stream));
}

// ---- grad input and grad weight together ------------------------------------------------------------------------

// One launch for both GEMMs when their plans use the 64 x 64 tiles of conv_bwd_dual_kernel.
static bool dual_tiles(const GatherPlan& dp, const WgradPlan& wp) {
  const Tile& gt = gtile(dp.tile);
  const Tile& wt = kWgradTiles[wp.tile];
  return gt.bp == 64 && gt.bq == 64 && gt.wp == 32 && gt.wq == 32 && (gt.bk == 16 || gt.bk == 64) && wt.bp == 64 &&
         wt.bq == 64 && wt.wp == 32 && wt.wq == 32;
}

static size_t bwd_workspace_one(const omt_conv_geo* g) {
  const size_t d = dgrad_workspace_one(g), w = wgrad_workspace_one(g);
  return w ? align256(d) + w : d;
}

OMT_EXPORT size_t omt_conv_bwd_workspace(const omt_conv_geo* g) {
  return g && dense_geo_ok(g) ? wgrad_chunks_workspace(g, bwd_workspace_one) : 0;
}

// Grad input and grad weight of a batch that fits the 32-bit offsets, over a workspace of bwd_workspace_one's size.
static int conv_bwd_one(const omt_conv_geo* g, const float* x, const float* gy, const float* w, float* gx, float* gw,
                        void* workspace, hipStream_t s) {
  const size_t dbytes = dgrad_workspace_one(g);
  void* dws = dbytes ? workspace : nullptr;
  void* wws = wgrad_workspace_one(g) ? (char*)workspace + align256(dbytes) : nullptr;
  GatherArgs ga;
  GatherPlan dp;
  int64_t maxq = 0;
  float* part = nullptr;
  if (int st = dgrad_prepare(g, gy, w, gx, dws, s, ga, dp, maxq, part)) return st;
  WgradArgs wa;
  WgradPlan wp;
  const dim3 wgrid = wgrad_prepare(g, x, gy, gw, wws, wa, wp);
  if (!dual_tiles(dp, wp)) {
    if (int st = run_gather(ga, dp, g->n, maxq, part, s)) return st;
    launch_wgrad_gemm(g, wp, wa, wgrid, s);
    if (int st = launch_check("conv_wgrad_kernel")) return st;
    return launch_split_sum(wgrad_sum_of(wa, wp, gw), s);
  }
  const dim3 ggrid = gather_grid(ga, dp, g->n, maxq, part);
  const DualGrid d{(int)ggrid.x, (int)ggrid.y, (int)ggrid.z, (int)wgrid.x, (int)wgrid.y, (int)wgrid.z};
  const int64_t blocks = (int64_t)d.gx * d.gy * d.gz + (int64_t)d.wx * d.wy * d.wz;
  if (blocks >= ((int64_t)1 << 31)) return fail(OMT_UNSUPPORTED, "omt_conv_bwd: grid too large");
  const bool gtap = gather_uses_tap_major(ga, dp), wtap = wgrad_uses_tap_major(g, wp);
  const bool deep = gtile(dp.tile).bk == 64;
  const dim3 grid((unsigned)blocks);
#define OMT_DUAL(BK, GM, WM) hipLaunchKernelGGL((conv_bwd_dual_kernel<BK, GM, WM>), grid, dim3(256), 0, s, ga, wa, d)
  if (ga.wplace) {
    switch ((deep ? 2 : 0) + (wtap ? 1 : 0)) {
      case 3: OMT_DUAL(64, kTapInPlace, kTapMajor); break;
      case 2: OMT_DUAL(64, kTapInPlace, kGeneric); break;
      case 1: OMT_DUAL(16, kTapInPlace, kTapMajor); break;
      default: OMT_DUAL(16, kTapInPlace, kGeneric); break;
    }
  } else switch ((deep ? 4 : 0) + (gtap ? 2 : 0) + (wtap ? 1 : 0)) {
    case 7: OMT_DUAL(64, kTapMajor, kTapMajor); break;
    case 6: OMT_DUAL(64, kTapMajor, kGeneric); break;
    case 5: OMT_DUAL(64, kGeneric, kTapMajor); break;
    case 4: OMT_DUAL(64, kGeneric, kGeneric); break;
    case 3: OMT_DUAL(16, kTapMajor, kTapMajor); break;
    case 2: OMT_DUAL(16, kTapMajor, kGeneric); break;
    case 1: OMT_DUAL(16, kGeneric, kTapMajor); break;
    default: OMT_DUAL(16, kGeneric, kGeneric); break;
  }
#undef OMT_DUAL
  if (int st = launch_check("conv_bwd_dual_kernel")) return st;
  const GatherSum gsum = gather_sum_of(ga, dp);
  const SplitSum wsum = wgrad_sum_of(wa, wp, gw);
  if (!gsum.blocks || !wsum.blocks) {
    if (int st = launch_gather_sum(gsum, s)) return st;
    return launch_split_sum(wsum, s);
  }
  const dim3 rgrid((unsigned)(gsum.blocks + wsum.blocks));
  if (gsum.vec4 && wsum.vec4)
    hipLaunchKernelGGL((dual_reduce_kernel<4, 4>), rgrid, dim3(256), 0, s, gsum, wsum);
  else if (gsum.vec4)
    hipLaunchKernelGGL((dual_reduce_kernel<4, 1>), rgrid, dim3(256), 0, s, gsum, wsum);
  else if (wsum.vec4)
    hipLaunchKernelGGL((dual_reduce_kernel<1, 4>), rgrid, dim3(256), 0, s, gsum, wsum);
  else
    hipLaunchKernelGGL((dual_reduce_kernel<1, 1>), rgrid, dim3(256), 0, s, gsum, wsum);
  return launch_check("dual_reduce_kernel");
}

// conv_bwd_one without its slice sums: grad input's partials stay unsummed when split into 2..max_gx slices and their
// sum is plain (no bias, ReLU or super-pixel scatter: a grad input's always is); grad weight's sum is returned as a job.
static int conv_bwd_one_parts(const omt_conv_geo* g, const float* x, const float* gy, const float* w, float* gx,
                              float* gw, void* workspace, hipStream_t s, int max_gx, const float** gx_parts,
                              int* gx_slices, SplitSum& wjob) {
  const size_t dbytes = dgrad_workspace_one(g);
  void* dws = dbytes ? workspace : nullptr;
  void* wws = wgrad_workspace_one(g) ? (char*)workspace + align256(dbytes) : nullptr;
  GatherArgs ga;
  GatherPlan dp;
  int64_t maxq = 0;
  float* part = nullptr;
  if (int st = dgrad_prepare(g, gy, w, gx, dws, s, ga, dp, maxq, part)) return st;
  WgradArgs wa;
  WgradPlan wp;
  const dim3 wgrid = wgrad_prepare(g, x, gy, gw, wws, wa, wp);
  *gx_parts = nullptr;
  *gx_slices = 1;
  wjob = wgrad_sum_of(wa, wp, gw);
  if (!dual_tiles(dp, wp)) {
    int unsummed = ga.d2s ? 1 : max_gx;
    if (int st = run_gather(ga, dp, g->n, maxq, part, s, &unsummed)) return st;
    if (unsummed > 1) {
      *gx_parts = ga.part;
      *gx_slices = unsummed;
    }
    launch_wgrad_gemm(g, wp, wa, wgrid, s);
    return launch_check("conv_wgrad_kernel");
  }
  const dim3 ggrid = gather_grid(ga, dp, g->n, maxq, part);
  const DualGrid d{(int)ggrid.x, (int)ggrid.y, (int)ggrid.z, (int)wgrid.x, (int)wgrid.y, (int)wgrid.z};
  const int64_t blocks = (int64_t)d.gx * d.gy * d.gz + (int64_t)d.wx * d.wy * d.wz;
  if (blocks >= ((int64_t)1 << 31)) return fail(OMT_UNSUPPORTED, "omt_conv_bwd_parts: grid too large");
  const bool gtap = gather_uses_tap_major(ga, dp), wtap = wgrad_uses_tap_major(g, wp);
  const bool deep = gtile(dp.tile).bk == 64;
  const dim3 grid((unsigned)blocks);
#define OMT_DUAL(BK, GM, WM) hipLaunchKernelGGL((conv_bwd_dual_kernel<BK, GM, WM>), grid, dim3(256), 0, s, ga, wa, d)
  if (ga.wplace) {
    switch ((deep ? 2 : 0) + (wtap ? 1 : 0)) {
      case 3: OMT_DUAL(64, kTapInPlace, kTapMajor); break;
      case 2: OMT_DUAL(64, kTapInPlace, kGeneric); break;
      case 1: OMT_DUAL(16, kTapInPlace, kTapMajor); break;
      default: OMT_DUAL(16, kTapInPlace, kGeneric); break;
    }
  } else switch ((deep ? 4 : 0) + (gtap ? 2 : 0) + (wtap ? 1 : 0)) {
    case 7: OMT_DUAL(64, kTapMajor, kTapMajor); break;
    case 6: OMT_DUAL(64, kTapMajor, kGeneric); break;
    case 5: OMT_DUAL(64, kGeneric, kTapMajor); break;
    case 4: OMT_DUAL(64, kGeneric, kGeneric); break;
    case 3: OMT_DUAL(16, kTapMajor, kTapMajor); break;
    case 2: OMT_DUAL(16, kTapMajor, kGeneric); break;
    case 1: OMT_DUAL(16, kGeneric, kTapMajor); break;
    default: OMT_DUAL(16, kGeneric, kGeneric); break;
  }
#undef OMT_DUAL
  if (int st = launch_check("conv_bwd_dual_kernel")) return st;
  const GatherSum gsum = gather_sum_of(ga, dp);
  if (!gsum.blocks) return OMT_OK;
  if (gsum.slices <= max_gx && !gsum.bias && !gsum.relu && !gsum.d2s && !gsum.nhwc) {
    *gx_parts = gsum.part;
    *gx_slices = gsum.slices;
    return OMT_OK;
  }
  return launch_gather_sum(gsum, s);
}

OMT_EXPORT int omt_conv_bwd_parts(const omt_conv_geo* g, const float* x, const float* gy, const float* w, float* gx,
                                  float* gw, void* workspace, size_t workspace_bytes, int max_gx_slices,
                                  const float** gx_parts, int* gx_slices, omt_slice_sum* gw_sum, void* stream) {
  if (!g || !x || !gy || !w || !gx || !gw || !gx_parts || !gx_slices || !gw_sum)
    return fail(OMT_INVALID, "omt_conv_bwd_parts: null pointer");
  Chunks ch;
  if (int st = chunk_check(g, "omt_conv_bwd_parts", ch)) return st;
  if (ch.count != 1) return fail(OMT_UNSUPPORTED, "omt_conv_bwd_parts: the batch runs in chunks");
  const size_t need = omt_conv_bwd_workspace(g);
  if (need && (!workspace || workspace_bytes < need))
    return fail(OMT_INVALID, "omt_conv_bwd_parts: workspace of %zu bytes needed", need);
  SplitSum job{};
  if (int st = conv_bwd_one_parts(g, x, gy, w, gx, gw, workspace, stream_of(stream), max_gx_slices, gx_parts,
                                  gx_slices, job))
    return st;
  *gw_sum = omt_slice_sum{job.part, job.out, job.blocks ? job.n : 0, job.blocks ? job.slices : 0};
  return OMT_OK;
}

OMT_EXPORT int omt_slice_sums(const omt_slice_sum* sums, int count, void* stream) {
  if (count < 0 || (count > 0 && !sums)) return fail(OMT_INVALID, "omt_slice_sums: arguments");
  for (int i = 0; i < count; ++i) {
    const omt_slice_sum& j = sums[i];
    if (j.slices <= 0) continue;
    if (!j.parts || !j.out || j.n < 0) return fail(OMT_INVALID, "omt_slice_sums: sum %d", i);
    if (int st = launch_split_sum(split_sum_of(j.parts, j.out, j.n, j.slices), stream_of(stream))) return st;
  }
  return OMT_OK;
}

OMT_EXPORT int omt_conv_bwd(const omt_conv_geo* g, const float* x, const float* gy, const float* w, float* gx,
                            float* gw, void* workspace, size_t workspace_bytes, void* stream) {
  if (!g || !x || !gy || !w || !gx || !gw) return fail(OMT_INVALID, "omt_conv_bwd: null pointer");
  Chunks ch;
  if (int st = chunk_check(g, "omt_conv_bwd", ch)) return st;
  const size_t need = omt_conv_bwd_workspace(g);
  if (need && (!workspace || workspace_bytes < need))
    return fail(OMT_INVALID, "omt_conv_bwd: workspace of %zu bytes needed", need);
  hipStream_t s = stream_of(stream);
  if (ch.count == 1) return conv_bwd_one(g, x, gy, w, gx, gw, workspace, s);
  const int64_t xi = g->ci * g->ih * g->iw, yi = g->co * g->oh * g->ow;
  return wgrad_chunks(g, ch, gw, workspace, s, [&](const omt_conv_geo* c, int64_t n0, float* out, void* ws) {
    return conv_bwd_one(c, x + n0 * xi, gy + n0 * yi, w, gx + n0 * xi, out, ws, s);
  });
}

// ---- channels-last (NHWC) convolution --------------------------------------------------------------------------
//
// The same three GEMMs over channels-last tensors: x [n][ih][iw][ci], y / gy [n][oh][ow][co], filter and filter
// gradient [co][ks][ks][ci] (the memory order of channels-last tensors of those shapes). The filter already is the
// tap-major [P][K] operand of the forward gather; the grad-input phases re-pack it; grad weight writes its
// tap-major columns in place. Plans live under their own directions (OMT_DIR_*_NHWC).

// Narrow channels-last gathers (channels not a multiple of 16: the forward's input channels, e.g. the ResNet stem's
// 3, or grad input's source channels co): one plan, the 64 x 64 staged tile gathering element by element
// (kNhwcNarrow), no K split.
constexpr int kNarrowTile = 5;
static bool nhwc_narrow(const omt_conv_geo* g) { return g->ci % 16 != 0; }
static bool nhwc_dgrad_narrow(const omt_conv_geo* g) { return g->co % 16 != 0; }
// grad weight: output channels a multiple of 4 (float4 runs of gy); input channels not a multiple of 4 take the
// element-by-element column loads (NARROW)
static bool nhwc_wgrad_ok(const omt_conv_geo* g) { return g->co % 4 == 0; }

static GatherPlan fwd_nhwc_plan(const omt_conv_geo* g) {
  omt_conv_plan cp;
  const bool have = cached_plan(OMT_DIR_FWD_NHWC, g, &cp);
  return gather_plan(g->co, g->n * g->oh * g->ow, g->ci * g->ks * g->ks, 1, have ? &cp : nullptr, g->ci);
}
static GatherPlan dgrad_nhwc_plan(const omt_conv_geo* g) {
  GatherArgs a{};
  PackArgs pk{};
  int64_t maxq = 0, maxk = 0;
  dgrad_phases(g, a, pk, maxq);
  for (int i = 0; i < a.nphase; ++i) maxk = std::max<int64_t>(maxk, a.ph[i].K);
  if (nhwc_dgrad_narrow(g)) return GatherPlan{kNarrowTile, 1, std::max<int64_t>(16, cdiv(maxk, 16) * 16)};
  omt_conv_plan cp;
  const bool have = cached_plan(OMT_DIR_DGRAD_NHWC, g, &cp);
  return gather_plan(g->ci, maxq, maxk, a.nphase, have ? &cp : nullptr, g->co);
}


// Launches a channels-last gather (and, split over K, its slice sum); `part`: the partials of the plan's size.
static int run_gather_nhwc(GatherArgs& a, const GatherPlan& pl, int64_t n, int64_t maxq, float* part,
                           hipStream_t s, bool narrow = false) {
  const Tile& tl = gtile(pl.tile);
  a.nhwc = 1;
  a.kslice = (int)pl.kslice;
  a.part = pl.slices > 1 ? part : nullptr;
  a.part_stride = n * a.P * a.YH * a.YW;
  a.tpw = 0;
  a.rows = 0;
  a.vec_out = a.P % 4 == 0 && (uintptr_t)a.y % 16 == 0 && (uintptr_t)a.part % 16 == 0;
  const dim3 grid((unsigned)cdiv(maxq, tl.bq), (unsigned)cdiv(a.P, tl.bp), (unsigned)(a.nphase * pl.slices));
  if (narrow)
    hipLaunchKernelGGL((conv_gather_kernel<64, 64, 32, 32, 16, kNhwcNarrow, false, 2>), grid, dim3(256), 0, s, a);
  else
    gather_nhwc_dispatch(pl.tile, a, grid, s);
  if (int st = launch_check("conv_gather_kernel (nhwc)")) return st;
  return launch_gather_sum(gather_sum_of(a, pl), s);
}

static size_t fwd_nhwc_workspace_one(const omt_conv_geo* g) {
  if (nhwc_narrow(g)) return 0;
  const GatherPlan pl = fwd_nhwc_plan(g);
  return pl.slices > 1 ? (size_t)(pl.slices * g->n * g->co * g->oh * g->ow) * sizeof(float) : 0;
}

OMT_EXPORT size_t omt_conv_fwd_nhwc_workspace(const omt_conv_geo* g) {
  return g && dense_geo_ok(g) ? chunks_max(g, fwd_nhwc_workspace_one) : 0;
}

static int conv_fwd_nhwc_one(const omt_conv_geo* g, const float* x, const float* w, const float* bias,
                             unsigned epilogue, float* y, void* workspace, hipStream_t s) {
  const bool narrow = nhwc_narrow(g);
  const GatherPlan pl =
      narrow ? GatherPlan{kNarrowTile, 1, cdiv(g->ci * g->ks * g->ks, 16) * 16} : fwd_nhwc_plan(g);
  GatherArgs a{};
  a.x = x;
  a.w = w;  // [co][ky][kx][ci]: the tap-major [P][K] operand as it is
  a.bias = (epilogue & OMT_EPI_BIAS) ? bias : nullptr;
  a.relu = (epilogue & OMT_EPI_RELU) ? 1 : 0;
  a.y = y;
  a.x_bytes = (uint32_t)(g->n * g->ci * g->ih * g->iw * 4);
  a.w_bytes = (uint32_t)(g->co * g->ci * g->ks * g->ks * 4);
  a.C = (int)g->ci;
  a.H = (int)g->ih;
  a.W = (int)g->iw;
  a.P = (int)g->co;
  a.YH = (int)g->oh;
  a.YW = (int)g->ow;
  a.nphase = 1;
  Phase& p = a.ph[0];
  p.KH = p.KW = (int)g->ks;
  p.S = (int)g->stride;
  p.PH = p.PW = (int)g->pad;
  p.OH = (int)g->oh;
  p.OW = (int)g->ow;
  p.K = (int)(g->ci * g->ks * g->ks);
  p.Q = (int)(g->n * g->oh * g->ow);
  p.os = 1;
  p.div_ohw = make_fastdiv((uint32_t)(g->oh * g->ow));
  p.div_ow = make_fastdiv((uint32_t)g->ow);
  p.div_kk = make_fastdiv((uint32_t)(g->ks * g->ks));
  p.div_kw = make_fastdiv((uint32_t)g->ks);
  a.div_c = make_fastdiv((uint32_t)a.C);
  return run_gather_nhwc(a, pl, g->n, p.Q, (float*)workspace, s, narrow);
}

OMT_EXPORT int omt_conv_fwd_nhwc(const omt_conv_geo* g, const float* x, const float* w, const float* bias,
                                 unsigned epilogue, float* y, void* workspace, size_t workspace_bytes, void* stream) {
  if (!g || !x || !w || !y) return fail(OMT_INVALID, "omt_conv_fwd_nhwc: null pointer");
  Chunks ch;
  if (int st = chunk_check(g, "omt_conv_fwd_nhwc", ch)) return st;
  if ((epilogue & OMT_EPI_BIAS) && !bias) return fail(OMT_INVALID, "omt_conv_fwd_nhwc: bias epilogue without bias");
  const size_t need = omt_conv_fwd_nhwc_workspace(g);
  if (need && (!workspace || workspace_bytes < need))
    return fail(OMT_INVALID, "omt_conv_fwd_nhwc: workspace of %zu bytes needed", need);
  hipStream_t s = stream_of(stream);
  const int64_t xi = g->ci * g->ih * g->iw, yi = g->co * g->oh * g->ow;
  return for_chunks(g, ch, [&](const omt_conv_geo* c, int64_t n0) {
    return conv_fwd_nhwc_one(c, x + n0 * xi, w, bias, epilogue, y + n0 * yi, workspace, s);
  });
}

// Grad-input workspace: the per-phase filters W'[ci][a'][b'][co] (all of the filter's elements), then, 256-byte
// aligned, any split-K partials [slices][n][ih][iw][ci].
static size_t dgrad_nhwc_workspace_one(const omt_conv_geo* g) {
  const GatherPlan pl = dgrad_nhwc_plan(g);
  const size_t pack = (size_t)(g->co * g->ci * g->ks * g->ks) * sizeof(float);
  return pl.slices > 1 ? align256(pack) + (size_t)(pl.slices * g->n * g->ci * g->ih * g->iw) * sizeof(float) : pack;
}

OMT_EXPORT size_t omt_conv_dgrad_nhwc_workspace(const omt_conv_geo* g) {
  return g && dense_geo_ok(g) ? chunks_max(g, dgrad_nhwc_workspace_one) : 0;
}

static int conv_dgrad_nhwc_one(const omt_conv_geo* g, const float* gy, const float* w, float* gx, void* workspace,
                               hipStream_t s) {
  GatherArgs a{};
  PackArgs pk{};
  int64_t maxq = 0;
  const int packed = dgrad_phases(g, a, pk, maxq);
  const GatherPlan pl = dgrad_nhwc_plan(g);
  pk.w = w;
  pk.out = (float*)workspace;
  pk.CO = (int)g->co;
  pk.CI = (int)g->ci;
  pk.KS = (int)g->ks;
  pk.S = (int)g->stride;
  pk.tap_major = 1;
  pk.src_krsc = 1;
  const int kk = (int)(g->ks * g->ks);
  if (g->stride == 1 && pk.nphase == 1 && pk.ph[0].ky0 == 0 && pk.ph[0].kx0 == 0 && pk.ph[0].jy == (int)g->ks &&
      pk.ph[0].jx == (int)g->ks && pk.ph[0].woff == 0 && (int64_t)packed == g->co * g->ci * kk) {
    hipLaunchKernelGGL(pack_dgrad_krsc_s1_kernel, dim3((unsigned)cdiv(g->ci, 32), (unsigned)cdiv(g->co, 32), (unsigned)kk),
                       dim3(256), 0, s, w, (float*)workspace, (int)g->co, (int)g->ci, kk);
    if (int st = launch_check("pack_dgrad_krsc_s1_kernel")) return st;
  } else {
    hipLaunchKernelGGL(pack_dgrad_weights_kernel, dim3(grid1d(packed, 256, 4096)), dim3(256), 0, s, pk);
    if (int st = launch_check("pack_dgrad_weights_kernel")) return st;
  }
  a.x = gy;
  a.w = (const float*)workspace;
  a.w_bytes = (uint32_t)(packed * 4);
  a.y = gx;
  a.x_bytes = (uint32_t)(g->n * g->co * g->oh * g->ow * 4);
  a.C = (int)g->co;
  a.H = (int)g->oh;
  a.W = (int)g->ow;
  a.P = (int)g->ci;
  a.YH = (int)g->ih;
  a.YW = (int)g->iw;
  a.div_c = make_fastdiv((uint32_t)a.C);
  float* part = (float*)((char*)workspace + align256((size_t)packed * sizeof(float)));
  return run_gather_nhwc(a, pl, g->n, maxq, part, s, nhwc_dgrad_narrow(g));
}

OMT_EXPORT int omt_conv_dgrad_nhwc(const omt_conv_geo* g, const float* gy, const float* w, float* gx, void* workspace,
                                   size_t workspace_bytes, void* stream) {
  if (!g || !gy || !w || !gx) return fail(OMT_INVALID, "omt_conv_dgrad_nhwc: null pointer");
  Chunks ch;
  if (int st = chunk_check(g, "omt_conv_dgrad_nhwc", ch)) return st;
  const size_t need = omt_conv_dgrad_nhwc_workspace(g);
  if (!workspace || workspace_bytes < need)
    return fail(OMT_INVALID, "omt_conv_dgrad_nhwc: workspace of %zu bytes needed", need);
  hipStream_t s = stream_of(stream);
  const int64_t yi = g->co * g->oh * g->ow, xi = g->ci * g->ih * g->iw;
  return for_chunks(g, ch, [&](const omt_conv_geo* c, int64_t n0) {
    return conv_dgrad_nhwc_one(c, gy + n0 * yi, w, gx + n0 * xi, workspace, s);
  });
}

static size_t wgrad_nhwc_workspace_one(const omt_conv_geo* g) {
  const WgradPlan pl = wgrad_plan(g, OMT_DIR_WGRAD_NHWC);
  return pl.slices > 1 ? (size_t)(pl.slices * g->co * g->ci * g->ks * g->ks) * sizeof(float) : 0;
}

OMT_EXPORT size_t omt_conv_wgrad_nhwc_workspace(const omt_conv_geo* g) {
  return g && dense_geo_ok(g) && nhwc_wgrad_ok(g) ? wgrad_chunks_workspace(g, wgrad_nhwc_workspace_one) : 0;
}

static int conv_wgrad_nhwc_one(const omt_conv_geo* g, const float* x, const float* gy, float* gw, void* workspace,
                               hipStream_t s) {
  WgradArgs a;
  WgradPlan pl;
  const dim3 grid = wgrad_prepare(g, x, gy, gw, workspace, a, pl, OMT_DIR_WGRAD_NHWC);
  if (g->ci % 4 == 0)
    wgrad_nhwc_dispatch<false>(pl.tile, a, grid, s);
  else
    wgrad_nhwc_dispatch<true>(pl.tile, a, grid, s);
  if (int st = launch_check("conv_wgrad_nhwc_kernel")) return st;
  return launch_split_sum(wgrad_sum_of(a, pl, gw), s);
}

OMT_EXPORT int omt_conv_wgrad_nhwc(const omt_conv_geo* g, const float* x, const float* gy, float* gw, void* workspace,
                                   size_t workspace_bytes, void* stream) {
  if (!g || !x || !gy || !gw) return fail(OMT_INVALID, "omt_conv_wgrad_nhwc: null pointer");
  Chunks ch;
  if (int st = chunk_check(g, "omt_conv_wgrad_nhwc", ch)) return st;
  if (!nhwc_wgrad_ok(g)) return fail(OMT_UNSUPPORTED, "omt_conv_wgrad_nhwc: output channels not a multiple of 4");
  const size_t need = omt_conv_wgrad_nhwc_workspace(g);
  if (need && (!workspace || workspace_bytes < need))
    return fail(OMT_INVALID, "omt_conv_wgrad_nhwc: workspace of %zu bytes needed", need);
  hipStream_t s = stream_of(stream);
  if (ch.count == 1) return conv_wgrad_nhwc_one(g, x, gy, gw, workspace, s);
  const int64_t xi = g->ci * g->ih * g->iw, yi = g->co * g->oh * g->ow;
  return wgrad_chunks(g, ch, gw, workspace, s, [&](const omt_conv_geo* c, int64_t n0, float* out, void* ws) {
    return conv_wgrad_nhwc_one(c, x + n0 * xi, gy + n0 * yi, out, ws, s);
  });
}

OMT_EXPORT int omt_bias_grad(int64_t n, int64_t c, int64_t hw, const float* gy, float* gb, void* stream) {
  if (!gy || !gb) return fail(OMT_INVALID, "omt_bias_grad: null pointer");
  if (n < 0 || c < 0 || hw < 0 || n * c * hw >= ((int64_t)1 << 31)) return fail(OMT_UNSUPPORTED, "omt_bias_grad: size");
  if (c == 0) return OMT_OK;
  if (hw <= kBiasColsHW) {
    hipLaunchKernelGGL(bias_grad_cols_kernel, dim3((unsigned)cdiv(c, 256)), dim3(256), 0, stream_of(stream), gy, gb,
                       (int)n, (int)c, (int)hw);
    return launch_check("bias_grad_cols_kernel");
  }
  hipLaunchKernelGGL(bias_grad_kernel, dim3((unsigned)c), dim3(256), 0, stream_of(stream), gy, gb, (int)n, (int)c,
                     (int)hw);
  return launch_check("bias_grad_kernel");
}

OMT_EXPORT int omt_fold_bn(int64_t co, int64_t per_out, const float* cw, const float* cb, const float* gamma,
                           const float* beta, const float* mean, const float* var, float eps, float* fw, float* fb,
                           void* stream) {
  if (!cw || !gamma || !beta || !mean || !var || !fw || !fb) return fail(OMT_INVALID, "omt_fold_bn: null pointer");
  if (co <= 0 || per_out <= 0) return OMT_OK;
  hipLaunchKernelGGL(fold_bn_kernel, dim3(grid1d(co * per_out, 256, 4096)), dim3(256), 0, stream_of(stream), (int)co,
                     (int)per_out, cw, cb, gamma, beta, mean, var, eps, fw, fb);
  return launch_check("fold_bn_kernel");
}

// ---- plan cache and tuning --------------------------------------------------------------------------------------

// Checks a plan call's arguments and points g at the geometry its plans are kept under (for a batch past 2 GiB, the
// first chunk's, in `tmp`).
static int plan_args_ok(int dir, const omt_conv_geo*& g, omt_conv_geo& tmp, const char* what) {
  if (!g) return fail(OMT_INVALID, "%s: null geometry", what);
  if (dir < OMT_DIR_FWD || dir > OMT_DIR_WGRAD_NHWC) return fail(OMT_INVALID, "%s: direction %d", what, dir);
  if (!dense_geo_ok(g) || !batch_chunks(g).count) return fail(OMT_UNSUPPORTED, "%s: geometry not covered", what);
  g = plan_geo(g, tmp);
  return OMT_OK;
}

OMT_EXPORT int omt_conv_num_tiles(int dir) {
  return dir >= OMT_DIR_FWD && dir <= OMT_DIR_WGRAD_NHWC ? num_tiles(dir) : 0;
}

OMT_EXPORT int omt_conv_get_plan(int dir, const omt_conv_geo* g, omt_conv_plan* plan, int* cached) {
  omt_conv_geo tmp;
  if (int st = plan_args_ok(dir, g, tmp, "omt_conv_get_plan")) return st;
  if (!plan) return fail(OMT_INVALID, "omt_conv_get_plan: null plan");
  omt_conv_plan cp;
  if (cached) *cached = cached_plan(dir, g, &cp) ? 1 : 0;
  if (wgrad_dir(dir)) {
    const WgradPlan pl = wgrad_plan(g, dir);
    *plan = {pl.tile, (int32_t)pl.slices};
  } else {
    const GatherPlan pl = dir == OMT_DIR_FWD        ? fwd_plan(g)
                          : dir == OMT_DIR_DGRAD    ? dgrad_plan(g)
                          : dir == OMT_DIR_FWD_NHWC ? fwd_nhwc_plan(g)
                                                    : dgrad_nhwc_plan(g);
    *plan = {pl.tile, (int32_t)pl.slices};
  }
  return OMT_OK;
}

OMT_EXPORT int omt_conv_set_plan(int dir, const omt_conv_geo* g, const omt_conv_plan* plan) {
  omt_conv_geo tmp;
  if (int st = plan_args_ok(dir, g, tmp, "omt_conv_set_plan")) return st;
  std::lock_guard<std::mutex> lk(g_plan_mu);
  if (!plan) {
    g_plans.erase(key_of(dir, g));
    return OMT_OK;
  }
  if (plan->tile < 0 || plan->tile >= num_tiles(dir) || plan->slices < 1 || plan->slices > 4096)
    return fail(OMT_INVALID, "omt_conv_set_plan: tile %d (of %d) / slices %d out of range", plan->tile, num_tiles(dir),
                plan->slices);
  g_plans[key_of(dir, g)] = *plan;
  return OMT_OK;
}

OMT_EXPORT int omt_conv_plan_count(void) {
  std::lock_guard<std::mutex> lk(g_plan_mu);
  return (int)g_plans.size();
}

OMT_EXPORT int omt_conv_plan_entry(int i, int* dir, omt_conv_geo* g, omt_conv_plan* plan) {
  std::lock_guard<std::mutex> lk(g_plan_mu);
  if (i < 0 || i >= (int)g_plans.size()) return fail(OMT_INVALID, "omt_conv_plan_entry: index %d", i);
  auto it = g_plans.begin();
  std::advance(it, i);
  const PlanKey& k = it->first;
  if (dir) *dir = k.dir;
  if (g) *g = omt_conv_geo{k.n, k.ci, k.co, k.ih, k.iw, k.oh, k.ow, k.ks, k.stride, k.pad};
  if (plan) *plan = it->second;
  return OMT_OK;
}

OMT_EXPORT void omt_conv_clear_plans(void) {
  std::lock_guard<std::mutex> lk(g_plan_mu);
  g_plans.clear();
}

namespace {

// Candidate plans of one direction: each tile with the K splits worth timing (distinct after rounding to whole
// K-blocks, at most 512 MiB of partials); wgrad: the estimate's slice count times 1/4, 1/2, 1 and 2, like the
// reference's split-K multipliers (csrc/conv.cpp:129).
std::vector<omt_conv_plan> tune_candidates(int dir, const omt_conv_geo* g, int ntile) {
  std::vector<omt_conv_plan> out;
  if (wgrad_dir(dir)) {
    const int64_t K = g->n * g->oh * g->ow, kmax = cdiv(K, 64);
    for (int t = 0; t < ntile; ++t) {
      const int64_t base = wgrad_model_slices(g, t);
      int64_t last = -1;
      for (double m : {0.25, 0.5, 1.0, 2.0}) {
        const int64_t sl = std::max<int64_t>(1, std::min<int64_t>(kmax, (int64_t)(base * m + 0.5)));
        const int64_t eff = cdiv(K, cdiv(cdiv(K, sl), 64) * 64);
        if (eff == last || eff * g->co * g->ci * g->ks * g->ks * 4 > ((int64_t)512 << 20)) continue;
        last = eff;
        out.push_back({t, (int32_t)eff});
      }
    }
    return out;
  }
  const bool nhwc = dir == OMT_DIR_FWD_NHWC || dir == OMT_DIR_DGRAD_NHWC;
  const bool fwd = dir == OMT_DIR_FWD || dir == OMT_DIR_FWD_NHWC;
  int64_t P, Q, K, z = 1, plane;
  if (fwd) {
    P = g->co, Q = g->n * g->oh * g->ow, K = g->ci * g->ks * g->ks, plane = g->n * g->co * g->oh * g->ow;
  } else if (!nhwc && dgrad_d2s(g)) {  // the super-pixel GEMM
    GatherArgs a{};
    dgrad_d2s_phase(g, a, Q);
    K = a.ph[0].K;
    P = g->stride * g->stride * g->ci, plane = P * Q;
  } else {
    GatherArgs a{};
    PackArgs pk{};
    dgrad_phases(g, a, pk, Q);
    K = 0;
    for (int i = 0; i < a.nphase; ++i) K = std::max<int64_t>(K, a.ph[i].K);
    P = g->ci, z = a.nphase, plane = g->n * g->ci * g->ih * g->iw;
  }
  // the 1x1 streaming tile: one 1x1 stride-1 unpadded phase with whole K-blocks, tap-major order, no split
  const bool stream_geo = g->ks == 1 && g->stride == 1 && g->pad == 0 && K % 16 == 0 && (g->ih * g->iw) % 4 == 0;
  // the in-place filter variant differs from the re-packing one only where a re-pack would run: tap-major order
  // (C a multiple of the K-block), no super-pixel grad input, a filter larger than 1x1 in the forward
  const int64_t gather_c = fwd ? g->ci : g->co;
  const bool packs = !(dir == OMT_DIR_FWD && g->ks == 1) && !(dir == OMT_DIR_DGRAD && dgrad_d2s(g));
  for (int t = 0; t < ntile; ++t) {
    const Tile& tl = gtile(t);
    if (nhwc && !nhwc_tile_ok(t, gather_c)) continue;
    if (t >= 2 * kNGather && !(wplace_tile(t) && packs && gather_tap_major(gather_c, false, tl.bk))) continue;
    if (tl.stream) {
      if (stream_geo && t < kNGather && (tl.stream == 1 || K == 64 || K == 128)) out.push_back({t, 1});
      continue;
    }
    const int64_t tiles = cdiv(P, tl.bp) * cdiv(Q, tl.bq) * z, nkb = cdiv(std::max<int64_t>(K, 1), tl.bk);
    // A grid that already fills the GPU is split only to even out its last round: a few workgroups per CU, all
    // resident at once, finish when the CUs holding one more than the rest do (1568 tiles: 7 on some CUs, 6.125 on
    // average); 2-4 slices of at least 8 K-blocks each spread them more evenly.
    const bool full = tiles >= 2 * kCUs;
    int64_t last = -1;
    for (int sc : {1, 2, 3, 4, 8, 16, 32, 64}) {
      const int64_t kb = cdiv(nkb, sc), eff = cdiv(nkb, kb);
      if (sc > 1 && kb < 2) break;
      if (full && sc > 1 && (sc > 4 || tiles >= 16 * kCUs || kb < 8)) break;
      if (!full && sc == 3) continue;
      if (eff == last || (eff > 1 && eff * plane * 4 > ((int64_t)512 << 20))) continue;
      last = eff;
      out.push_back({t, (int32_t)eff});
    }
  }
  return out;
}

bool forcing() {
  for (const auto* f : t_force)
    if (f) return true;
  return false;
}

struct ForceGuard {
  ~ForceGuard() {
    for (auto& f : t_force) f = nullptr;
  }
};

// Scratch buffers, events and a private stream of one tuning run: zero inputs (fp32 MFMA timing does not depend on
// the values). Candidates are timed as replays of a captured HIP graph on the private stream, the way a training step
// runs: each extra launch of a plan (filter re-pack, split-K slice sum) then costs what a graph node costs, which
// back-to-back stream launches hide. The destructor synchronizes both streams, so nothing queued still uses the buffers
// when they return to the cache.
struct TuneScratch {
  hipStream_t s, cs = nullptr;
  void *x = nullptr, *w = nullptr, *gy = nullptr, *o1 = nullptr, *o2 = nullptr, *ws = nullptr;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  explicit TuneScratch(hipStream_t st) : s(st) {}
  int init(const omt_conv_geo* g, size_t ws_bytes) {
    const size_t xb = (size_t)(g->n * g->ci * g->ih * g->iw) * 4, wb = (size_t)(g->co * g->ci * g->ks * g->ks) * 4,
                 yb = (size_t)(g->n * g->co * g->oh * g->ow) * 4;
    const size_t ob = std::max(xb, std::max(wb, yb));
    if (int st = omt_malloc_on(&x, xb, s)) return st;
    if (int st = omt_malloc_on(&w, wb, s)) return st;
    if (int st = omt_malloc_on(&gy, yb, s)) return st;
    if (int st = omt_malloc_on(&o1, ob, s)) return st;
    if (int st = omt_malloc_on(&o2, wb, s)) return st;
    if (ws_bytes)
      if (int st = omt_malloc_on(&ws, ws_bytes, s)) return st;
    if (int st = hip_check(hipMemsetAsync(x, 0, xb, s), "hipMemsetAsync")) return st;
    if (int st = hip_check(hipMemsetAsync(w, 0, wb, s), "hipMemsetAsync")) return st;
    if (int st = hip_check(hipMemsetAsync(gy, 0, yb, s), "hipMemsetAsync")) return st;
    if (int st = hip_check(hipEventCreate(&e0), "hipEventCreate")) return st;
    if (int st = hip_check(hipEventCreate(&e1), "hipEventCreate")) return st;
    if (int st = hip_check(hipStreamCreateWithFlags(&cs, hipStreamNonBlocking), "hipStreamCreateWithFlags")) return st;
    // the private stream starts after the zeroing queued on s
    if (int st = hip_check(hipEventRecord(e0, s), "hipEventRecord")) return st;
    return hip_check(hipStreamWaitEvent(cs, e0, 0), "hipStreamWaitEvent");
  }
  ~TuneScratch() {
    if (cs) (void)hipStreamSynchronize(cs);
    (void)hipStreamSynchronize(s);
    if (cs) (void)hipStreamDestroy(cs);
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    for (void* p : {x, w, gy, o1, o2, ws})
      if (p) omt_free(p);
  }
  // Average ms of one `run(stream)` call: kReps calls captured into a graph on the private stream, replayed once to
  // warm up and then twice between events.
  template <class Run>
  int time(Run run, float* ms) {
    constexpr int kReps = 8, kTimed = 2;
    if (int e = hip_check(hipStreamBeginCapture(cs, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture"))
      return e;
    int st = OMT_OK;
    for (int r = 0; r < kReps && st == OMT_OK; ++r) st = run(cs);
    hipGraph_t graph = nullptr;
    const hipError_t ce = hipStreamEndCapture(cs, &graph);
    if (st != OMT_OK || ce != hipSuccess) {
      if (graph) (void)hipGraphDestroy(graph);
      (void)hipGetLastError();
      return st != OMT_OK ? st : hip_check(ce, "hipStreamEndCapture");
    }
    hipGraphExec_t exec = nullptr;
    const hipError_t ie = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    if (int e = hip_check(ie, "hipGraphInstantiate")) return e;
    auto replays = [&]() -> int {
      if (int e = hip_check(hipGraphLaunch(exec, cs), "hipGraphLaunch")) return e;
      if (int e = hip_check(hipEventRecord(e0, cs), "hipEventRecord")) return e;
      for (int r = 0; r < kTimed; ++r)
        if (int e = hip_check(hipGraphLaunch(exec, cs), "hipGraphLaunch")) return e;
      if (int e = hip_check(hipEventRecord(e1, cs), "hipEventRecord")) return e;
      if (int e = hip_check(hipEventSynchronize(e1), "hipEventSynchronize")) return e;
      if (int e = hip_check(hipEventElapsedTime(ms, e0, e1), "hipEventElapsedTime")) return e;
      *ms /= (float)(kReps * kTimed);
      return OMT_OK;
    };
    st = replays();
    (void)hipGraphExecDestroy(exec);
    return st;
  }
};

size_t dir_workspace(int dir, const omt_conv_geo* g) {
  switch (dir) {
    case OMT_DIR_FWD: return omt_conv_fwd_workspace(g);
    case OMT_DIR_DGRAD: return omt_conv_dgrad_workspace(g);
    case OMT_DIR_WGRAD: return omt_conv_wgrad_workspace(g);
    case OMT_DIR_FWD_NHWC: return omt_conv_fwd_nhwc_workspace(g);
    case OMT_DIR_DGRAD_NHWC: return omt_conv_dgrad_nhwc_workspace(g);
    default: return omt_conv_wgrad_nhwc_workspace(g);
  }
}

int refuse_capture(hipStream_t s, const char* what) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  OMT_HIP(hipStreamIsCapturing(s, &cs));
  if (cs != hipStreamCaptureStatusNone) return fail(OMT_UNSUPPORTED, "%s: stream is capturing", what);
  return OMT_OK;
}

}  // namespace

OMT_EXPORT int omt_conv_autotune(int dir, const omt_conv_geo* g, int max_tiles, void* stream, omt_conv_plan* best) {
  omt_conv_geo tmp;
  if (int st = plan_args_ok(dir, g, tmp, "omt_conv_autotune")) return st;
  if (forcing()) return fail(OMT_INVALID, "omt_conv_autotune: re-entered");
  hipStream_t s = stream_of(stream);
  if (int st = refuse_capture(s, "omt_conv_autotune")) return st;
  const int ntile = max_tiles <= 0 ? num_tiles(dir) : std::min(max_tiles, num_tiles(dir));
  const std::vector<omt_conv_plan> cands = tune_candidates(dir, g, ntile);
  if (cands.empty()) return fail(OMT_UNSUPPORTED, "omt_conv_autotune: no candidate plan");

  ForceGuard guard;
  size_t ws_bytes = 0;
  for (const omt_conv_plan& c : cands) {
    t_force[dir] = &c;
    ws_bytes = std::max(ws_bytes, dir_workspace(dir, g));
  }
  t_force[dir] = nullptr;
  omt_conv_plan win = cands[0];
  {
    TuneScratch sc(s);
    if (int st = sc.init(g, ws_bytes)) return st;
    auto run = [&](hipStream_t rs) -> int {
      const size_t need = dir_workspace(dir, g);
      const float *x = (const float*)sc.x, *w = (const float*)sc.w, *gy = (const float*)sc.gy;
      float* o = (float*)sc.o1;
      switch (dir) {
        case OMT_DIR_FWD:
          return omt_conv_fwd(g, x, w, nullptr, 0, nullptr, nullptr, nullptr, nullptr, 1e-5f, o, sc.ws, need, rs);
        case OMT_DIR_DGRAD: return omt_conv_dgrad(g, gy, w, o, sc.ws, need, rs);
        case OMT_DIR_WGRAD: return omt_conv_wgrad(g, x, gy, o, sc.ws, need, rs);
        case OMT_DIR_FWD_NHWC: return omt_conv_fwd_nhwc(g, x, w, nullptr, 0, o, sc.ws, need, rs);
        case OMT_DIR_DGRAD_NHWC: return omt_conv_dgrad_nhwc(g, gy, w, o, sc.ws, need, rs);
        default: return omt_conv_wgrad_nhwc(g, x, gy, o, sc.ws, need, rs);
      }
    };
    float win_ms = 1e30f;
    for (const omt_conv_plan& c : cands) {
      t_force[dir] = &c;
      float ms = 0.f;
      if (int st = sc.time(run, &ms)) return st;
      if (ms < win_ms) {
        win_ms = ms;
        win = c;
      }
    }
    t_force[dir] = nullptr;
  }
  {
    std::lock_guard<std::mutex> lk(g_plan_mu);
    g_plans[key_of(dir, g)] = win;
  }
  if (best) *best = win;
  return OMT_OK;
}

OMT_EXPORT int omt_conv_autotune_bwd(const omt_conv_geo* g, int max_tiles, void* stream, omt_conv_plan* dgrad_best,
                                     omt_conv_plan* wgrad_best) {
  omt_conv_geo tmp;
  if (int st = plan_args_ok(OMT_DIR_DGRAD, g, tmp, "omt_conv_autotune_bwd")) return st;
  if (forcing()) return fail(OMT_INVALID, "omt_conv_autotune_bwd: re-entered");
  hipStream_t s = stream_of(stream);
  if (int st = refuse_capture(s, "omt_conv_autotune_bwd")) return st;
  // the pair tuned one direction at a time, then the pairs that share a launch
  omt_conv_plan dsep, wsep;
  if (int st = omt_conv_autotune(OMT_DIR_DGRAD, g, max_tiles, stream, &dsep)) return st;
  if (int st = omt_conv_autotune(OMT_DIR_WGRAD, g, max_tiles, stream, &wsep)) return st;
  std::vector<std::pair<omt_conv_plan, omt_conv_plan>> cands{{dsep, wsep}};
  const int dtiles = max_tiles <= 0 ? num_tiles(OMT_DIR_DGRAD) : std::min(max_tiles, num_tiles(OMT_DIR_DGRAD));
  const int wtiles = max_tiles <= 0 ? num_tiles(OMT_DIR_WGRAD) : std::min(max_tiles, num_tiles(OMT_DIR_WGRAD));
  {
    std::vector<omt_conv_plan> ds, wsv;
    for (const omt_conv_plan& d : tune_candidates(OMT_DIR_DGRAD, g, dtiles)) {
      const Tile& t = gtile(d.tile);
      if (t.bp == 64 && t.bq == 64 && t.wp == 32 && t.wq == 32 && (t.bk == 16 || t.bk == 64)) ds.push_back(d);
    }
    for (const omt_conv_plan& w : tune_candidates(OMT_DIR_WGRAD, g, wtiles)) {
      const Tile& t = kWgradTiles[w.tile];
      if (t.bp == 64 && t.bq == 64 && t.wp == 32 && t.wq == 32) wsv.push_back(w);
    }
    for (const omt_conv_plan& d : ds)
      for (const omt_conv_plan& w : wsv) cands.push_back({d, w});
  }
  ForceGuard guard;
  size_t ws_bytes = 0;
  for (const auto& c : cands) {
    t_force[OMT_DIR_DGRAD] = &c.first;
    t_force[OMT_DIR_WGRAD] = &c.second;
    ws_bytes = std::max(ws_bytes, omt_conv_bwd_workspace(g));
  }
  t_force[OMT_DIR_DGRAD] = t_force[OMT_DIR_WGRAD] = nullptr;
  std::pair<omt_conv_plan, omt_conv_plan> win = cands[0];
  {
    TuneScratch sc(s);
    if (int st = sc.init(g, ws_bytes)) return st;
    auto run = [&](hipStream_t rs) -> int {
      return omt_conv_bwd(g, (const float*)sc.x, (const float*)sc.gy, (const float*)sc.w, (float*)sc.o1,
                          (float*)sc.o2, sc.ws, omt_conv_bwd_workspace(g), rs);
    };
    float win_ms = 1e30f;
    for (const auto& c : cands) {
      t_force[OMT_DIR_DGRAD] = &c.first;
      t_force[OMT_DIR_WGRAD] = &c.second;
      float ms = 0.f;
      if (int st = sc.time(run, &ms)) return st;
      if (ms < win_ms) {
        win_ms = ms;
        win = c;
      }
    }
    t_force[OMT_DIR_DGRAD] = t_force[OMT_DIR_WGRAD] = nullptr;
  }
  {
    std::lock_guard<std::mutex> lk(g_plan_mu);
    g_plans[key_of(OMT_DIR_DGRAD, g)] = win.first;
    g_plans[key_of(OMT_DIR_WGRAD, g)] = win.second;
  }
  if (dgrad_best) *dgrad_best = win.first;
  if (wgrad_best) *wgrad_best = win.second;
  return OMT_OK;
}

/*
 * omt_oracle.c -- CPU restatement of omarchy-mac-torch's convolution hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the checker the HIP kernels are compared against. Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg load it; the product (libomt_hip.so and the
 * omarchy_mac_torch package) never links, imports or calls it.
 *
 * Every function restates one reference function or shader (file:line under the reference repo) in plain C.
 * Arithmetic is float64 throughout (inputs and outputs are float32 arrays, accumulation is double), so the oracle
 * is more accurate than any float32 summation order; the reference's float32 split-K / split-statistics structure
 * is kept where it decides *which* terms are summed, never *how precisely*.
 *
 * Parity pinning (tests/test_oracle_pins.py): every function is checked against PyTorch CPU float32 (the
 * reference's own correctness oracle), against float64 brute force on tiny shapes, and against closed-form
 * identities (stride-phase dgrad vs the stride-skipping dgrad map, the conv adjoint identity, BN folding).
 *
 * Build: make -C oracle   (gcc -O2 -fopenmp -shared -fPIC)
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

typedef struct {
  int64_t n, ci, co, ih, iw, oh, ow, ks, stride, pad;
} orc_geo; /* csrc/omt.h:224-226 (Geo) */

static int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

/* ---------------------------------------------------------------------------------------------------------------
 * geometry and classification
 * ------------------------------------------------------------------------------------------------------------- */

/* conv_geo (csrc/conv.cpp:19-21): oh = (ih + 2p - ks) / s + 1 */
void orc_conv_geo(int64_t n, int64_t ci, int64_t co, int64_t ih, int64_t iw, int64_t ks, int64_t stride, int64_t pad,
                  orc_geo* g) {
  g->n = n; g->ci = ci; g->co = co; g->ih = ih; g->iw = iw;
  g->oh = (ih + 2 * pad - ks) / stride + 1;
  g->ow = (iw + 2 * pad - ks) / stride + 1;
  g->ks = ks; g->stride = stride; g->pad = pad;
}

/* conv_kind (csrc/conv.cpp:167-177). Returns 0 = "" (not covered), 1 = dense, 2 = dw, 3 = dwg.
 * x_c = input channels, w_o = weight out channels; the float32 / 4-D test is the caller's. */
int orc_conv_kind(int64_t x_c, int64_t w_o, int64_t kh, int64_t kw, int64_t sh, int64_t sw, int64_t ph, int64_t pw,
                  int64_t dh, int64_t dw, int transposed, int64_t groups) {
  if (transposed) return 0;
  if (dh != 1 || dw != 1 || kh != kw) return 0;
  if (sh != sw || ph != pw) return 0;
  int64_t ks = kh, s = sh, p = ph;
  if (groups == 1 && ks <= 11 && s >= 1 && s <= 4 && p <= ks) return 1;
  if (groups == x_c && groups == w_o && groups > 1 && (ks == 3 || ks == 5 || ks == 7) && s == 1 && p == ks / 2) return 2;
  if (groups == x_c && groups == w_o && groups > 1 && ks <= 11 && s >= 1 && s <= 4 && p <= ks) return 3;
  return 0;
}

/* mnk (csrc/conv.cpp:23-27): the GEMM view per kind (0/3 forward, 1 grad input, 2 grad weight) */
void orc_mnk(int kind, const orc_geo* g, int64_t* M, int64_t* N, int64_t* K) {
  if (kind == 0 || kind == 3) { *M = g->n * g->oh * g->ow; *N = g->co; *K = g->ci * g->ks * g->ks; }
  else if (kind == 1) { *M = g->n * g->ih * g->iw; *N = g->ci; *K = g->co * g->ks * g->ks; }
  else { *M = g->co; *N = g->ci * g->ks * g->ks; *K = g->n * g->oh * g->ow; }
}

/* The planner's untuned default tile (omarchy_mac_torch/native.py:46-58 over gemm.py:18-19 TILES): least padded
 * M*N, then the larger register block. Kind 5 (one stride phase) uses M = n*ceil(ih/s)*ceil(iw/s), N = ci. */
static const int TILES[10][4] = {{64, 64, 4, 4},  {256, 16, 4, 4}, {16, 256, 4, 4}, {128, 32, 4, 4},  {32, 128, 4, 4},
                                 {128, 64, 8, 4}, {64, 128, 4, 8}, {128, 128, 8, 8}, {256, 32, 8, 4}, {32, 256, 4, 8}};
void orc_default_tile(int kind, const orc_geo* g, int* bm, int* bn) {
  int64_t M, N;
  if (kind == 0 || kind == 3) { M = g->n * g->oh * g->ow; N = g->co; }
  else if (kind == 1) { M = g->n * g->ih * g->iw; N = g->ci; }
  else if (kind == 5) { M = g->n * cdiv(g->ih, g->stride) * cdiv(g->iw, g->stride); N = g->ci; }
  else { M = g->co; N = g->ci * g->ks * g->ks; }
  int best = 0;
  int64_t best_pad = -1, best_reg = 0;
  for (int t = 0; t < 10; t++) {
    int64_t padded = cdiv(M, TILES[t][0]) * TILES[t][0] * cdiv(N, TILES[t][1]) * TILES[t][1];
    int64_t reg = (int64_t)TILES[t][2] * TILES[t][3];
    if (best_pad < 0 || padded < best_pad || (padded == best_pad && reg > best_reg)) { best = t; best_pad = padded; best_reg = reg; }
  }
  *bm = TILES[best][0];
  *bn = TILES[best][1];
}

/* Split-K partition of the weight-gradient GEMM (csrc/conv.cpp:106-109): slices and kslice for tile (bm, bn) and
 * the autotuned multiplier mult. */
void orc_wgrad_split(const orc_geo* g, int bm, int bn, double mult, int64_t* slices_out, int64_t* kslice_out) {
  int64_t M, N, K;
  orc_mnk(2, g, &M, &N, &K);
  int64_t tiles = cdiv(M, bm) * cdiv(N, bn);
  int64_t a = (int64_t)((double)(512 / tiles) * mult);
  int64_t slices = a < K / 64 ? a : K / 64;
  if (slices < 1) slices = 1;
  int64_t kslice = cdiv(cdiv(K, slices), 16) * 16;
  slices = cdiv(K, kslice);
  *slices_out = slices;
  *kslice_out = kslice;
}

/* ---------------------------------------------------------------------------------------------------------------
 * dense convolution: implicit-GEMM index maps
 * ------------------------------------------------------------------------------------------------------------- */

/* A loader of the forward GEMM, kinds 0 and 3 (omarchy_mac_torch/gemm.py:26-33, 139-141): im2col of x with zero
 * padding; kind 3 applies the previous layer's eval BatchNorm + ReLU to in-bounds taps only. */
static double fwd_aval(const orc_geo* g, const float* x, int64_t m, int64_t k, const float* bn_m, const float* bn_v,
                       const float* bn_g, const float* bn_b, double eps) {
  int64_t ohw = g->oh * g->ow, n = m / ohw, r = m % ohw, oy = r / g->ow, ox = r % g->ow;
  int64_t kk = g->ks * g->ks, c = k / kk, kr = k % kk, ky = kr / g->ks, kx = kr % g->ks;
  int64_t yy = oy * g->stride + ky - g->pad, xx = ox * g->stride + kx - g->pad;
  if (yy < 0 || yy >= g->ih || xx < 0 || xx >= g->iw) return 0.0;
  double v = x[((n * g->ci + c) * g->ih + yy) * g->iw + xx];
  if (bn_m) {
    v = (v - bn_m[c]) * (1.0 / sqrt((double)bn_v[c] + eps)) * bn_g[c] + bn_b[c];
    if (v < 0) v = 0;
  }
  return v;
}

/* Forward convolution, gemm_forward (csrc/conv.cpp:70-77) with the _FWD maps (gemm.py:25-42):
 * C[m, nn] = sum_k A[m, k] * w[nn * K + k]; store out[((m / ohw) * co + nn) * ohw + m % ohw].
 * epilogue bit 0: + bias[nn]; bit 1: ReLU (gemm.py:38-39). bn_* non-null: kind 3 loader (BN + ReLU of the input). */
void orc_conv_fwd(const orc_geo* g, const float* x, const float* w, const float* bias, unsigned epilogue,
                  const float* bn_m, const float* bn_v, const float* bn_g, const float* bn_b, double eps, float* out) {
  int64_t M, N, K;
  orc_mnk(0, g, &M, &N, &K);
  int64_t ohw = g->oh * g->ow;
#pragma omp parallel for schedule(static)
  for (int64_t m = 0; m < M; m++) {
    for (int64_t nn = 0; nn < N; nn++) {
      double acc = 0.0;
      for (int64_t k = 0; k < K; k++) {
        double a = fwd_aval(g, x, m, k, bn_m, bn_v, bn_g, bn_b, eps);
        if (a != 0.0) acc += a * (double)w[nn * K + k];
      }
      if ((epilogue & 1u) && bias) acc += bias[nn];
      if ((epilogue & 2u) && acc < 0) acc = 0;
      out[((m / ohw) * g->co + nn) * ohw + m % ohw] = (float)acc;
    }
  }
}

/* Selected forward outputs (flat NCHW indices into y), float64: the same map as orc_conv_fwd, for spot checks of
 * full-size outputs. */
void orc_conv_fwd_points(const orc_geo* g, const float* x, const float* w, const float* bias, unsigned epilogue,
                         int64_t npts, const int64_t* flat, double* out) {
  int64_t M, N, K;
  orc_mnk(0, g, &M, &N, &K);
  int64_t ohw = g->oh * g->ow;
#pragma omp parallel for schedule(dynamic, 16)
  for (int64_t i = 0; i < npts; i++) {
    int64_t f = flat[i], pix = f % ohw, nn = (f / ohw) % g->co, n = f / (ohw * g->co);
    int64_t m = n * ohw + pix;
    double acc = 0.0;
    for (int64_t k = 0; k < K; k++) acc += fwd_aval(g, x, m, k, 0, 0, 0, 0, 0) * (double)w[nn * K + k];
    if ((epilogue & 1u) && bias) acc += bias[nn];
    if ((epilogue & 2u) && acc < 0) acc = 0;
    out[i] = acc;
  }
}

/* A loader of the grad-input GEMM, kind 1 (gemm.py:44-56): gy gathered at (y + p - ky, x + p - kx), keeping only
 * taps on the stride grid (any stride). B = w[((k / kk) * ci + nn) * kk + k % kk] (gemm.py:57). */
static double gin_dot(const orc_geo* g, const float* gy, const float* w, int64_t m, int64_t nn) {
  int64_t ihw = g->ih * g->iw, n = m / ihw, r = m % ihw, y = r / g->iw, x = r % g->iw;
  int64_t kk = g->ks * g->ks, K = g->co * kk;
  double acc = 0.0;
  for (int64_t k = 0; k < K; k++) {
    int64_t co = k / kk, kr = k % kk, ky = kr / g->ks, kx = kr % g->ks;
    int64_t yy = y + g->pad - ky, xx = x + g->pad - kx;
    if (yy < 0 || xx < 0) continue;
    if (g->stride > 1) {
      if (yy % g->stride != 0 || xx % g->stride != 0) continue;
      yy /= g->stride;
      xx /= g->stride;
    }
    if (yy >= g->oh || xx >= g->ow) continue;
    acc += (double)gy[((n * g->co + co) * g->oh + yy) * g->ow + xx] * (double)w[(co * g->ci + nn) * kk + kr];
  }
  return acc;
}

/* Selected grad-input outputs (flat NCHW indices into gx) by the stride-skipping kind-1 map. */
void orc_conv_dgrad_points(const orc_geo* g, const float* gy, const float* w, int64_t npts, const int64_t* flat,
                           double* out) {
  int64_t ihw = g->ih * g->iw;
#pragma omp parallel for schedule(dynamic, 16)
  for (int64_t i = 0; i < npts; i++) {
    int64_t f = flat[i], pix = f % ihw, nn = (f / ihw) % g->ci, n = f / (ihw * g->ci);
    out[i] = gin_dot(g, gy, w, n * ihw + pix, nn);
  }
}

/* Grad input, gemm_grad_input (csrc/conv.cpp:78-101). Stride 1: one kind-1 GEMM (gemm.py:43-59). Stride s > 1: one
 * dense GEMM per stride phase (py, px) in [0, s)^2 (csrc/conv.cpp:79-94, gemm.py:60-80):
 *   hi = ceil((ih - py) / s), ky0 = (py + p) mod s, jy = ceil((ks - ky0) / s) (0 if ky0 >= ks), qy = (py + p - ky0) / s
 *   gx[n, ci, py + s*i, px + s*j] = sum_{co, a < jy, b < jx} gy[n, co, i + qy - a, j + qx - b] * w[co, ci, ky0 + s*a, kx0 + s*b]
 * Phases with K = co*jy*jx = 0 write zeros. */
void orc_conv_dgrad(const orc_geo* g, const float* gy, const float* w, float* gx) {
  int64_t ihw = g->ih * g->iw;
  if (g->stride == 1) {
    int64_t M = g->n * ihw;
#pragma omp parallel for schedule(static)
    for (int64_t m = 0; m < M; m++)
      for (int64_t nn = 0; nn < g->ci; nn++)
        gx[((m / ihw) * g->ci + nn) * ihw + m % ihw] = (float)gin_dot(g, gy, w, m, nn);
    return;
  }
  int64_t s = g->stride;
  for (int64_t py = 0; py < s; py++)
    for (int64_t px = 0; px < s; px++) {
      int64_t hi = cdiv(g->ih - py, s), wi = cdiv(g->iw - px, s);
      if (hi <= 0 || wi <= 0) continue;
      int64_t ky0 = (py + g->pad) % s, kx0 = (px + g->pad) % s;
      int64_t jy = ky0 < g->ks ? cdiv(g->ks - ky0, s) : 0, jx = kx0 < g->ks ? cdiv(g->ks - kx0, s) : 0;
      int64_t qy = (py + g->pad - ky0) / s, qx = (px + g->pad - kx0) / s;
      int64_t M = g->n * hi * wi, K = g->co * jy * jx;
#pragma omp parallel for schedule(static)
      for (int64_t m = 0; m < M; m++) {
        int64_t hw = hi * wi, n = m / hw, r = m % hw, i = r / wi, j = r % wi;
        for (int64_t nn = 0; nn < g->ci; nn++) {
          double acc = 0.0;
          for (int64_t k = 0; k < K; k++) {
            int64_t jj = jy * jx, co = k / jj, kr = k % jj;
            int64_t oy = i + qy - kr / jx, ox = j + qx - kr % jx;
            if (oy < 0 || oy >= g->oh || ox < 0 || ox >= g->ow) continue;
            int64_t ky = ky0 + s * (kr / jx), kx = kx0 + s * (kr % jx);
            acc += (double)gy[((n * g->co + co) * g->oh + oy) * g->ow + ox] *
                   (double)w[((co * g->ci + nn) * g->ks + ky) * g->ks + kx];
          }
          gx[((n * g->ci + nn) * g->ih + py + s * i) * g->iw + px + s * j] = (float)acc;
        }
      }
    }
}

/* B loader of the grad-weight GEMM, kind 2 (gemm.py:83-89): im2col(x) at k = (n, oy, ox), nn = (c, ky, kx).
 * A = gy[((k / ohw) * co + m) * ohw + k % ohw] (gemm.py:82). */
static double gw_dot(const orc_geo* g, const float* x, const float* gy, int64_t m, int64_t nn, int64_t k0, int64_t k1) {
  int64_t ohw = g->oh * g->ow, kk = g->ks * g->ks;
  int64_t c = nn / kk, kr = nn % kk, ky = kr / g->ks, kx = kr % g->ks;
  double acc = 0.0;
  for (int64_t k = k0; k < k1; k++) {
    int64_t s = k / ohw, r = k % ohw, oy = r / g->ow, ox = r % g->ow;
    int64_t yy = oy * g->stride + ky - g->pad, xx = ox * g->stride + kx - g->pad;
    if (yy < 0 || yy >= g->ih || xx < 0 || xx >= g->iw) continue;
    acc += (double)gy[(s * g->co + m) * ohw + r] * (double)x[((s * g->ci + c) * g->ih + yy) * g->iw + xx];
  }
  return acc;
}

/* Grad weight, gemm_grad_weight (csrc/conv.cpp:102-114): split-K over K = n*oh*ow into `slices` ranges of `kslice`
 * (orc_wgrad_split), partials part[z][m][nn], then gemm_reduce (csrc/kernels/gemm_reduce.wgsl) sums z in order into
 * gw[co][ci][ky][kx]. slices <= 0 uses the reference's rule with the planner's default tile and mult = 1. */
void orc_conv_wgrad(const orc_geo* g, const float* x, const float* gy, int64_t slices, int64_t kslice, float* gw) {
  int64_t M, N, K;
  orc_mnk(2, g, &M, &N, &K);
  if (slices <= 0) {
    int bm, bn;
    orc_default_tile(2, g, &bm, &bn);
    orc_wgrad_split(g, bm, bn, 1.0, &slices, &kslice);
  }
  double* part = (double*)malloc(sizeof(double) * (size_t)(slices * M * N));
#pragma omp parallel for collapse(2) schedule(dynamic, 1)
  for (int64_t z = 0; z < slices; z++)
    for (int64_t m = 0; m < M; m++) {
      int64_t k0 = z * kslice, k1 = k0 + kslice < K ? k0 + kslice : K;
      for (int64_t nn = 0; nn < N; nn++) part[(z * M + m) * N + nn] = gw_dot(g, x, gy, m, nn, k0, k1);
    }
  for (int64_t i = 0; i < M * N; i++) {
    double s = 0.0;
    for (int64_t z = 0; z < slices; z++) s += part[z * M * N + i];
    gw[i] = (float)s;
  }
  free(part);
}

/* Selected grad-weight outputs (flat [co][ci][ky][kx] indices), whole K in one sum. */
void orc_conv_wgrad_points(const orc_geo* g, const float* x, const float* gy, int64_t npts, const int64_t* flat,
                           double* out) {
  int64_t M, N, K;
  orc_mnk(2, g, &M, &N, &K);
#pragma omp parallel for schedule(dynamic, 1)
  for (int64_t i = 0; i < npts; i++) out[i] = gw_dot(g, x, gy, flat[i] / N, flat[i] % N, 0, K);
}

/* Bias gradient, csum_nchw (csrc/kernels/csum_nchw.wgsl:21-27; csrc/conv.cpp:232-235): gb[c] = sum_{n, hw} gy. */
void orc_bias_grad(int64_t n, int64_t c, int64_t hw, const float* gy, float* gb) {
  for (int64_t ch = 0; ch < c; ch++) {
    double s = 0.0;
    for (int64_t nn = 0; nn < n; nn++)
      for (int64_t e = 0; e < hw; e++) s += gy[(nn * c + ch) * hw + e];
    gb[ch] = (float)s;
  }
}

/* ---------------------------------------------------------------------------------------------------------------
 * depthwise
 * ------------------------------------------------------------------------------------------------------------- */

/* General depthwise forward (csrc/kernels/dwg_fwd.wgsl:7-22; dw_fwd.wgsl is its stride-1 same-pad case and
 * dw_fwd_bn.wgsl adds the BN + ReLU loader, as in orc_conv_fwd). Bias added afterwards (csrc/conv.cpp:200-203). */
void orc_dw_fwd(const orc_geo* g, const float* x, const float* w, const float* bias, const float* bn_m,
                const float* bn_v, const float* bn_g, const float* bn_b, double eps, float* out) {
  int64_t C = g->ci, total = g->n * C * g->oh * g->ow;
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < total; i++) {
    int64_t ox = i % g->ow, oy = (i / g->ow) % g->oh, nc = i / (g->oh * g->ow), ch = nc % C;
    int64_t y0 = oy * g->stride - g->pad, x0 = ox * g->stride - g->pad;
    double s = 0.0;
    for (int64_t ky = 0; ky < g->ks; ky++) {
      int64_t sy = y0 + ky;
      if (sy < 0 || sy >= g->ih) continue;
      for (int64_t kx = 0; kx < g->ks; kx++) {
        int64_t sx = x0 + kx;
        if (sx < 0 || sx >= g->iw) continue;
        double v = x[(nc * g->ih + sy) * g->iw + sx];
        if (bn_m) {
          v = (v - bn_m[ch]) * (1.0 / sqrt((double)bn_v[ch] + eps)) * bn_g[ch] + bn_b[ch];
          if (v < 0) v = 0;
        }
        s += v * (double)w[(ch * g->ks + ky) * g->ks + kx];
      }
    }
    if (bias) s += bias[ch];
    out[i] = (float)s;
  }
}

/* General depthwise grad input (csrc/kernels/dwg_gin.wgsl:7-22): taps kept only where (y + p - ky) is on the stride
 * grid; dw_gin.wgsl is the stride-1 same-pad case. */
void orc_dw_dgrad(const orc_geo* g, const float* gy, const float* w, float* gx) {
  int64_t C = g->ci, total = g->n * C * g->ih * g->iw, st = g->stride;
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < total; i++) {
    int64_t xx = i % g->iw, yy = (i / g->iw) % g->ih, nc = i / (g->ih * g->iw), ch = nc % C;
    double s = 0.0;
    for (int64_t ky = 0; ky < g->ks; ky++) {
      int64_t ty = yy + g->pad - ky;
      if (ty < 0 || ty % st != 0 || ty / st >= g->oh) continue;
      for (int64_t kx = 0; kx < g->ks; kx++) {
        int64_t tx = xx + g->pad - kx;
        if (tx < 0 || tx % st != 0 || tx / st >= g->ow) continue;
        s += (double)gy[(nc * g->oh + ty / st) * g->ow + tx / st] * (double)w[(ch * g->ks + ky) * g->ks + kx];
      }
    }
    gx[i] = (float)s;
  }
}

/* General depthwise grad weight (csrc/kernels/dwg_gwt.wgsl:6-26): gw[c, ky, kx] = sum over n, oy, ox. */
void orc_dw_wgrad(const orc_geo* g, const float* x, const float* gy, float* gw) {
  int64_t C = g->ci, kk = g->ks * g->ks, ohw = g->oh * g->ow;
#pragma omp parallel for schedule(static)
  for (int64_t j = 0; j < C * kk; j++) {
    int64_t ch = j / kk, k = j % kk, ky = k / g->ks - g->pad, kx = k % g->ks - g->pad;
    double s = 0.0;
    for (int64_t n = 0; n < g->n; n++)
      for (int64_t r = 0; r < ohw; r++) {
        int64_t yy = (r / g->ow) * g->stride + ky, xx = (r % g->ow) * g->stride + kx;
        if (yy < 0 || yy >= g->ih || xx < 0 || xx >= g->iw) continue;
        s += (double)gy[(n * C + ch) * ohw + r] * (double)x[((n * C + ch) * g->ih + yy) * g->iw + xx];
      }
    gw[j] = (float)s;
  }
}

/* ---------------------------------------------------------------------------------------------------------------
 * batch norm
 * ------------------------------------------------------------------------------------------------------------- */

/* Training statistics: bn_stats_part (csrc/kernels/bn_stats_part.wgsl:21-31) + bn_stats_fin (bn_stats_fin.wgsl:11-22).
 * Shifted sums d = x - x[c*hw] (first element of image 0) over S = (n >= 8 ? 8 : 1) image slices, then
 * mean = shift + s1/m, var = max(s2/m - (s1/m)^2, 0) (biased), and the running-stat update
 * rm += mom*(mean - rm), rv += mom*(var*m/(m-1) - rv) (csrc/nn.cpp:41-45, csrc/plans.cpp:175-176).
 * Writes mean[c], var[c]; new_rm / new_rv may alias rm / rv (in-place, as native_batch_norm) or not (functional,
 * bn_stats_fin_functional.wgsl). */
void orc_bn_stats(int64_t n, int64_t c, int64_t hw, const float* x, double momentum, const float* rm, const float* rv,
                  float* mean, float* var, float* new_rm, float* new_rv) {
  int64_t S = n >= 8 ? 8 : 1;
  double m = (double)(n * hw);
  double corr = (double)(float)((double)(n * hw) / (double)(n * hw - 1 > 1 ? n * hw - 1 : 1));
  for (int64_t ch = 0; ch < c; ch++) {
    double shift = x[ch * hw], s1 = 0.0, s2 = 0.0;
    for (int64_t sl = 0; sl < S; sl++)
      for (int64_t nn = sl; nn < n; nn += S)
        for (int64_t e = 0; e < hw; e++) {
          double d = (double)x[(nn * c + ch) * hw + e] - shift;
          s1 += d;
          s2 += d * d;
        }
    double a = s1 / m, mu = shift + a, vr = s2 / m - a * a;
    if (vr < 0) vr = 0;
    mean[ch] = (float)mu;
    var[ch] = (float)vr;
    if (rm && new_rm) new_rm[ch] = (float)((double)rm[ch] + momentum * (mu - (double)rm[ch]));
    if (rv && new_rv) new_rv[ch] = (float)((double)rv[ch] + momentum * (vr * corr - (double)rv[ch]));
  }
}

/* Normalize: bn_apply (csrc/kernels/bn_apply.wgsl:16-17) y = (x - mean) * invstd * gamma + beta, with
 * invstd = rsqrt(var + eps) (ew RSQRT_EPS, csrc/nn.cpp:46-47) in training and rsqrt(rv + eps) in eval
 * (bn_eval_inv.wgsl:4). relu != 0: bn_relu.wgsl / bn_relu_rv.wgsl (max(., 0)). `var` is the variance. */
void orc_bn_apply(int64_t n, int64_t c, int64_t hw, const float* x, const float* mean, const float* var, double eps,
                  const float* gamma, const float* beta, int relu, float* y) {
  int64_t total = n * c * hw;
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < total; i++) {
    int64_t ch = (i / hw) % c;
    double inv = 1.0 / sqrt((double)var[ch] + eps);
    double z = ((double)x[i] - mean[ch]) * inv * gamma[ch] + beta[ch];
    if (relu && z < 0) z = 0;
    y[i] = (float)z;
  }
}

/* Backward: bnb_reduce + bnb_apply (csrc/kernels/bnb_reduce.wgsl:22-37, bnb_apply.wgsl:13-19), and with relu_y
 * non-null the ReLU-masked form bn_bwd_part / bn_bwd_fin / bn_bwd_apply (gz = g where y > 0, else 0):
 *   dgamma = sum gz * xhat, dbeta = sum gz, xhat = (x - mean) * invstd
 *   dx = gamma * invstd / m * (m * gz - dbeta - xhat * dgamma)
 * `invstd` is the saved inverse std (the second output of the forward). gx may be null (output_mask[0] false). */
void orc_bn_bwd(int64_t n, int64_t c, int64_t hw, const float* g, const float* x, const float* relu_y,
                const float* mean, const float* invstd, const float* gamma, float* gx, float* dgamma, float* dbeta) {
  double m = (double)(n * hw);
  for (int64_t ch = 0; ch < c; ch++) {
    double s1 = 0.0, s2 = 0.0, mu = mean[ch], inv = invstd[ch];
    for (int64_t nn = 0; nn < n; nn++)
      for (int64_t e = 0; e < hw; e++) {
        int64_t i = (nn * c + ch) * hw + e;
        double gz = g[i];
        if (relu_y && !(relu_y[i] > 0.0f)) gz = 0.0;
        s1 += gz;
        s2 += gz * ((double)x[i] - mu) * inv;
      }
    if (dgamma) dgamma[ch] = (float)s2;
    if (dbeta) dbeta[ch] = (float)s1;
    if (gx)
      for (int64_t nn = 0; nn < n; nn++)
        for (int64_t e = 0; e < hw; e++) {
          int64_t i = (nn * c + ch) * hw + e;
          double gz = g[i];
          if (relu_y && !(relu_y[i] > 0.0f)) gz = 0.0;
          double xhat = ((double)x[i] - mu) * inv;
          gx[i] = (float)((double)gamma[ch] * inv / m * (m * gz - s1 - xhat * s2));
        }
  }
}

/* BatchNorm folding into a conv (fold_bn, csrc/fused.cpp:34-40): scale = w / sqrt(rv + eps) per output channel,
 * fw = cw * scale, fb = (cb - rm) * scale + b (cb = 0 when absent). */
void orc_fold_bn(int64_t co, int64_t per_out, const float* cw, const float* cb, const float* w, const float* b,
                 const float* rm, const float* rv, double eps, float* fw, float* fb) {
  for (int64_t o = 0; o < co; o++) {
    double scale = (double)w[o] / sqrt((double)rv[o] + eps);
    for (int64_t e = 0; e < per_out; e++) fw[o * per_out + e] = (float)((double)cw[o * per_out + e] * scale);
    fb[o] = (float)(((cb ? (double)cb[o] : 0.0) - rm[o]) * scale + b[o]);
  }
}

/* ---------------------------------------------------------------------------------------------------------------
 * pooling
 * ------------------------------------------------------------------------------------------------------------- */

/* Max pool, any window / stride / padding / dilation (csrc/kernels/maxpool_gen_fwd.wgsl:8-23; output size from
 * at::native::pooling_output_shape, csrc/nn.cpp:163-164). Indices are int64 flat positions in the input plane. The
 * first maximum wins ties. NaN: PyTorch CPU semantics (a NaN replaces the running max, the last NaN's index is kept);
 * the shader's per-row break agrees whenever a window row holds at most one NaN. */
void orc_maxpool_fwd(int64_t nc, int64_t ih, int64_t iw, int64_t oh, int64_t ow, int64_t kh, int64_t kw, int64_t sh,
                     int64_t sw, int64_t ph, int64_t pw, int64_t dh, int64_t dw, const float* x, float* out,
                     int64_t* idx) {
  int64_t total = nc * oh * ow;
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < total; i++) {
    int64_t ox = i % ow, oy = (i / ow) % oh, p = i / (ow * oh);
    float best = -INFINITY;
    int64_t bi = -1;
    for (int64_t ky = 0; ky < kh; ky++) {
      int64_t y = oy * sh + ky * dh - ph;
      if (y < 0 || y >= ih) continue;
      for (int64_t kx = 0; kx < kw; kx++) {
        int64_t xx = ox * sw + kx * dw - pw;
        if (xx < 0 || xx >= iw) continue;
        float v = x[p * ih * iw + y * iw + xx];
        if (bi < 0 || v > best || isnan(v)) {
          best = v;
          bi = y * iw + xx;
        }
      }
    }
    out[i] = best;
    idx[i] = bi;
  }
}

/* Max pool backward (csrc/kernels/maxpool_gen_bwd.wgsl:6-25): every input element gathers g of the outputs whose
 * saved index points at it. */
void orc_maxpool_bwd(int64_t nc, int64_t ih, int64_t iw, int64_t oh, int64_t ow, const float* g, const int64_t* idx,
                     float* gx) {
  memset(gx, 0, sizeof(float) * (size_t)(nc * ih * iw));
  for (int64_t p = 0; p < nc; p++) {
    double* acc = (double*)calloc((size_t)(ih * iw), sizeof(double));
    for (int64_t o = 0; o < oh * ow; o++) {
      int64_t t = idx[p * oh * ow + o];
      if (t >= 0 && t < ih * iw) acc[t] += g[p * oh * ow + o];
    }
    for (int64_t e = 0; e < ih * iw; e++) gx[p * ih * iw + e] = (float)acc[e];
    free(acc);
  }
}

/* Average-pool divisor (csrc/kernels/avgpool_gen_fwd.wgsl:5-13): divisor_override if > 0, else the window clipped
 * to the padded input (count_include_pad) or to the input. */
static double avg_div(int64_t oy, int64_t ox, int64_t ih, int64_t iw, int64_t kh, int64_t kw, int64_t sh, int64_t sw,
                      int64_t ph, int64_t pw, int include_pad, int64_t divisor) {
  if (divisor > 0) return (double)divisor;
  int64_t hs = oy * sh - ph, ws = ox * sw - pw;
  int64_t he = hs + kh < ih + ph ? hs + kh : ih + ph, we = ws + kw < iw + pw ? ws + kw : iw + pw;
  int64_t pool = (he - hs) * (we - ws);
  if (include_pad) return (double)pool;
  if (hs < 0) hs = 0;
  if (ws < 0) ws = 0;
  if (he > ih) he = ih;
  if (we > iw) we = iw;
  return (double)((he - hs) * (we - ws));
}

/* Average pool forward (csrc/kernels/avgpool_gen_fwd.wgsl:15-28). */
void orc_avgpool_fwd(int64_t nc, int64_t ih, int64_t iw, int64_t oh, int64_t ow, int64_t kh, int64_t kw, int64_t sh,
                     int64_t sw, int64_t ph, int64_t pw, int include_pad, int64_t divisor, const float* x, float* out) {
  int64_t total = nc * oh * ow;
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < total; i++) {
    int64_t ox = i % ow, oy = (i / ow) % oh, p = i / (ow * oh);
    int64_t hs = oy * sh - ph, ws = ox * sw - pw;
    double acc = 0.0;
    for (int64_t y = hs < 0 ? 0 : hs; y < (hs + kh < ih ? hs + kh : ih); y++)
      for (int64_t xx = ws < 0 ? 0 : ws; xx < (ws + kw < iw ? ws + kw : iw); xx++) acc += x[(p * ih + y) * iw + xx];
    out[i] = (float)(acc / avg_div(oy, ox, ih, iw, kh, kw, sh, sw, ph, pw, include_pad, divisor));
  }
}

/* Average pool backward (csrc/kernels/avgpool_gen_bwd.wgsl:15-31): scatter g / divisor over each window. */
void orc_avgpool_bwd(int64_t nc, int64_t ih, int64_t iw, int64_t oh, int64_t ow, int64_t kh, int64_t kw, int64_t sh,
                     int64_t sw, int64_t ph, int64_t pw, int include_pad, int64_t divisor, const float* g, float* gx) {
  for (int64_t p = 0; p < nc; p++) {
    double* acc = (double*)calloc((size_t)(ih * iw), sizeof(double));
    for (int64_t oy = 0; oy < oh; oy++)
      for (int64_t ox = 0; ox < ow; ox++) {
        double v = g[(p * oh + oy) * ow + ox] / avg_div(oy, ox, ih, iw, kh, kw, sh, sw, ph, pw, include_pad, divisor);
        int64_t hs = oy * sh - ph, ws = ox * sw - pw;
        for (int64_t y = hs < 0 ? 0 : hs; y < (hs + kh < ih ? hs + kh : ih); y++)
          for (int64_t xx = ws < 0 ? 0 : ws; xx < (ws + kw < iw ? ws + kw : iw); xx++) acc[y * iw + xx] += v;
      }
    for (int64_t e = 0; e < ih * iw; e++) gx[p * ih * iw + e] = (float)acc[e];
    free(acc);
  }
}

/* Adaptive average pool (csrc/kernels/adapool_fwd.wgsl:4-13, adapool_bwd.wgsl:4-19): bin o covers
 * [floor(o*in/out), ceil((o+1)*in/out)). */
void orc_adapool_fwd(int64_t nc, int64_t ih, int64_t iw, int64_t oh, int64_t ow, const float* x, float* out) {
  for (int64_t i = 0; i < nc * oh * ow; i++) {
    int64_t ox = i % ow, oy = (i / ow) % oh, p = i / (ow * oh);
    int64_t y0 = (oy * ih) / oh, y1 = ((oy + 1) * ih + oh - 1) / oh;
    int64_t x0 = (ox * iw) / ow, x1 = ((ox + 1) * iw + ow - 1) / ow;
    double acc = 0.0;
    for (int64_t y = y0; y < y1; y++)
      for (int64_t xx = x0; xx < x1; xx++) acc += x[(p * ih + y) * iw + xx];
    out[i] = (float)(acc / (double)((y1 - y0) * (x1 - x0)));
  }
}

void orc_adapool_bwd(int64_t nc, int64_t ih, int64_t iw, int64_t oh, int64_t ow, const float* g, float* gx) {
  for (int64_t i = 0; i < nc * ih * iw; i++) {
    int64_t xx = i % iw, y = (i / iw) % ih, p = i / (iw * ih);
    double acc = 0.0;
    for (int64_t oy = 0; oy < oh; oy++) {
      int64_t y0 = (oy * ih) / oh, y1 = ((oy + 1) * ih + oh - 1) / oh;
      if (y < y0 || y >= y1) continue;
      for (int64_t ox = 0; ox < ow; ox++) {
        int64_t x0 = (ox * iw) / ow, x1 = ((ox + 1) * iw + ow - 1) / ow;
        if (xx < x0 || xx >= x1) continue;
        acc += g[(p * oh + oy) * ow + ox] / (double)((y1 - y0) * (x1 - x0));
      }
    }
    gx[i] = (float)acc;
  }
}

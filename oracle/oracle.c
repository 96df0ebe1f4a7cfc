/*
 * CPU oracle for the conv-chain upscaler path.
 *
 * TEST INFRASTRUCTURE ONLY. This file is a plain-C restatement of the
 * reference's per-op arithmetic, used as the checker for the HIP engine and as
 * the CPU baseline timed beside it. The product library never links, loads or
 * calls it; only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may.
 *
 * Semantics follow the ONNX operators the reference engine accepts, computed
 * in fp32 with fp16 storage between nodes (the behaviour of ONNX Runtime's CPU
 * EP on an fp16 model, which the reference is judged against):
 *   conv3x3      ONNX Conv, 3x3, stride 1, dilation 1, group 1, pads 1/1/1/1
 *                (reference: src/vapoursynth/hip_engine.cc:397-433 accepts only
 *                this geometry; tests/correctness/harness/reference.py:67-81
 *                restates it in float64)
 *   relu/silu/sigmoid/add/mul/clip
 *                elementwise (hip_kernels.h:75-83 silu, 493-519 unary/binary;
 *                hip_engine.h:47-52 clip defaults to +/-inf)
 *   depth_to_space_dcr
 *                ONNX DepthToSpace mode DCR: out(c, h*b+r, w*b+q) =
 *                in((r*b+q)*Cout + c, h, w) (hip_kernels.h:521-546;
 *                reference.py:84-93)
 *   f32<->f16    IEEE-754 round-to-nearest-even (hip_engine.cc:1190-1276)
 *   winograd_*   F(2x2,3x3) transforms U = G g G^T, V = B^T d B,
 *                Y = A^T M A (hip_engine.cc:995-1016; hip_kernels.h:86-96,
 *                133-141), used only to pin the GPU kernel's pieces.
 *
 * Every function is pinned by tests/test_oracle.py against library routines
 * (numpy float16 casts, torch conv2d/pixel_shuffle/silu), brute force on tiny
 * inputs, and closed-form invariants.
 *
 * Layouts: activations are NCHW float32 (batch n, channel c, row h, col w),
 * weights are OIHW float32.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ---------------------------------------------------------------------- */
/* fp16 <-> fp32 (IEEE binary16, round to nearest, ties to even)           */
/* ---------------------------------------------------------------------- */

/* Follows src/vapoursynth/hip_engine.cc:1190-1232: NaN stays NaN (quiet bit
 * set), overflow goes to inf, values below half the smallest subnormal go to
 * signed zero, subnormals are rounded with ties-to-even. */
uint16_t or_f32_to_f16(float f) {
  uint32_t b;
  memcpy(&b, &f, 4);
  const uint32_t sign = (b >> 16) & 0x8000u;
  const uint32_t exp = (b >> 23) & 0xffu;
  const uint32_t man = b & 0x7fffffu;
  if (exp == 0xffu) return (uint16_t)(sign | 0x7c00u | (man ? 0x200u : 0u));
  int e = (int)exp - 127 + 15;
  if (e >= 31) return (uint16_t)(sign | 0x7c00u);
  if (e <= 0) {
    if (e < -10) return (uint16_t)sign;
    const uint32_t full = man | 0x800000u;
    const uint32_t shift = (uint32_t)(14 - e);
    uint32_t q = full >> shift;
    const uint32_t rem = full & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (q & 1u))) ++q;
    return (uint16_t)(sign | q);
  }
  uint32_t q = man >> 13;
  const uint32_t rem = man & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) ++q;
  if (q == 0x400u) {
    q = 0;
    ++e;
  }
  if (e >= 31) return (uint16_t)(sign | 0x7c00u);
  return (uint16_t)(sign | ((uint32_t)e << 10) | q);
}

/* Exact widening; follows hip_engine.cc:1251-1276. */
float or_f16_to_f32(uint16_t h) {
  const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1fu;
  const uint32_t man = h & 0x3ffu;
  uint32_t out;
  if (exp == 0) {
    if (man == 0) {
      out = sign;
    } else {
      uint32_t e = 127 - 15 + 1;
      uint32_t m = man;
      while ((m & 0x400u) == 0) {
        m <<= 1;
        --e;
      }
      out = sign | (e << 23) | ((m & 0x3ffu) << 13);
    }
  } else if (exp == 0x1fu) {
    out = sign | 0x7f800000u | (man ? 0x400000u : 0u);
  } else {
    out = sign | ((exp + 127 - 15) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &out, 4);
  return f;
}

void or_f32_to_f16_array(const float* x, uint16_t* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = or_f32_to_f16(x[i]);
}

void or_f16_to_f32_array(const uint16_t* x, float* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = or_f16_to_f32(x[i]);
}

/* Round every element to the nearest fp16 value, in place (fp16 storage of an
 * fp32-computed tensor). */
void or_round_f16(float* x, int64_t n) {
  for (int64_t i = 0; i < n; ++i) x[i] = or_f16_to_f32(or_f32_to_f16(x[i]));
}

/* ---------------------------------------------------------------------- */
/* 3x3 SAME convolution (ONNX Conv = cross-correlation), NCHW, fp32 math   */
/* ---------------------------------------------------------------------- */

/* y[n][m][h][w] = bias[m] + sum_{c,r,s} w[m][c][r][s] * x[n][c][h+r-1][w+s-1]
 * with zero padding (reference.py:67-81). Each output row accumulates in
 * fp32 (acc_f64 = 0) or fp64 (acc_f64 = 1) along the (c, r, s) order. bias may
 * be NULL. Parallel over (n, m). */
void or_conv3x3(const float* x, int N, int C, int H, int W, const float* wt, const float* bias,
                int M, float* y, int acc_f64) {
  const int64_t plane = (int64_t)H * W;
  const int Wp = W + 2;
#ifdef _OPENMP
#pragma omp parallel
#endif
  {
    float* accf = (float*)malloc(sizeof(float) * (size_t)W);
    double* accd = (double*)malloc(sizeof(double) * (size_t)W);
    float* row = (float*)malloc(sizeof(float) * (size_t)Wp);
#ifdef _OPENMP
#pragma omp for schedule(dynamic) collapse(2)
#endif
    for (int n = 0; n < N; ++n) {
      for (int m = 0; m < M; ++m) {
        for (int h = 0; h < H; ++h) {
          const float b = bias ? bias[m] : 0.0f;
          for (int i = 0; i < W; ++i) {
            accf[i] = b;
            accd[i] = b;
          }
          for (int c = 0; c < C; ++c) {
            const float* xp = x + ((int64_t)n * C + c) * plane;
            const float* wk = wt + ((int64_t)m * C + c) * 9;
            for (int r = 0; r < 3; ++r) {
              const int hh = h + r - 1;
              if (hh < 0 || hh >= H) continue;
              row[0] = 0.0f;
              row[Wp - 1] = 0.0f;
              memcpy(row + 1, xp + (int64_t)hh * W, sizeof(float) * (size_t)W);
              for (int s = 0; s < 3; ++s) {
                const float k = wk[r * 3 + s];
                const float* src = row + s;
                if (acc_f64) {
                  for (int i = 0; i < W; ++i) accd[i] += (double)k * (double)src[i];
                } else {
                  for (int i = 0; i < W; ++i) accf[i] += k * src[i];
                }
              }
            }
          }
          float* yo = y + ((int64_t)n * M + m) * plane + (int64_t)h * W;
          if (acc_f64) {
            for (int i = 0; i < W; ++i) yo[i] = (float)accd[i];
          } else {
            for (int i = 0; i < W; ++i) yo[i] = accf[i];
          }
        }
      }
    }
    free(accf);
    free(accd);
    free(row);
  }
}

/* ---------------------------------------------------------------------- */
/* Elementwise ops                                                         */
/* ---------------------------------------------------------------------- */

void or_relu(float* x, int64_t n) {
  for (int64_t i = 0; i < n; ++i) x[i] = x[i] > 0.0f ? x[i] : 0.0f;
}

/* sigmoid(x) = 1 / (1 + e^-x), evaluated in double then rounded to fp32. */
void or_sigmoid(float* x, int64_t n) {
  for (int64_t i = 0; i < n; ++i) x[i] = (float)(1.0 / (1.0 + exp(-(double)x[i])));
}

/* silu(x) = x * sigmoid(x) (the Sigmoid+Mul pair fused at hip_engine.cc:493-522). */
void or_silu(float* x, int64_t n) {
  for (int64_t i = 0; i < n; ++i) x[i] = (float)((double)x[i] / (1.0 + exp(-(double)x[i])));
}

void or_add(const float* a, const float* b, float* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = a[i] + b[i];
}

void or_mul(const float* a, const float* b, float* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = a[i] * b[i];
}

/* Clip with ONNX semantics: NaN propagates, bounds default to +/-inf
 * (hip_engine.h:47-52). */
void or_clip(float* x, int64_t n, float lo, float hi) {
  for (int64_t i = 0; i < n; ++i) {
    float v = x[i];
    if (v != v) continue;
    if (v < lo) v = lo;
    if (v > hi) v = hi;
    x[i] = v;
  }
}

/* ONNX DepthToSpace, DCR: x is [N][C][H][W] with C = Cout*b*b; y is
 * [N][Cout][H*b][W*b]; y[n][c][h*b+r][w*b+q] = x[n][(r*b+q)*Cout+c][h][w]. */
void or_depth_to_space_dcr(const float* x, int N, int C, int H, int W, int b, float* y) {
  const int Cout = C / (b * b);
  const int Ho = H * b, Wo = W * b;
  for (int n = 0; n < N; ++n)
    for (int c = 0; c < Cout; ++c)
      for (int oh = 0; oh < Ho; ++oh)
        for (int ow = 0; ow < Wo; ++ow) {
          const int h = oh / b, r = oh % b, w = ow / b, q = ow % b;
          const int cin = (r * b + q) * Cout + c;
          y[(((int64_t)n * Cout + c) * Ho + oh) * Wo + ow] =
              x[(((int64_t)n * C + cin) * H + h) * W + w];
        }
}

/* ---------------------------------------------------------------------- */
/* Winograd F(2x2,3x3) transforms (double precision), for pinning          */
/* ---------------------------------------------------------------------- */

/* U = G g G^T, G = [[1,0,0],[1/2,1/2,1/2],[1/2,-1/2,1/2],[0,0,1]]
 * (hip_engine.cc:995-1016). g and U are row-major 3x3 / 4x4. */
void or_winograd_filter(const double* g, double* U) {
  static const double G[4][3] = {{1, 0, 0}, {0.5, 0.5, 0.5}, {0.5, -0.5, 0.5}, {0, 0, 1}};
  double Gg[4][3];
  for (int i = 0; i < 4; ++i)
    for (int j = 0; j < 3; ++j) {
      double s = 0;
      for (int k = 0; k < 3; ++k) s += G[i][k] * g[k * 3 + j];
      Gg[i][j] = s;
    }
  for (int i = 0; i < 4; ++i)
    for (int j = 0; j < 4; ++j) {
      double s = 0;
      for (int k = 0; k < 3; ++k) s += Gg[i][k] * G[j][k];
      U[i * 4 + j] = s;
    }
}

/* V = B^T d B, B^T = [[1,0,-1,0],[0,1,1,0],[0,-1,1,0],[0,1,0,-1]]
 * (hip_kernels.h:86-96). d and V are row-major 4x4. */
void or_winograd_input(const double* d, double* V) {
  static const double BT[4][4] = {{1, 0, -1, 0}, {0, 1, 1, 0}, {0, -1, 1, 0}, {0, 1, 0, -1}};
  double t[4][4];
  for (int i = 0; i < 4; ++i)
    for (int j = 0; j < 4; ++j) {
      double s = 0;
      for (int k = 0; k < 4; ++k) s += BT[i][k] * d[k * 4 + j];
      t[i][j] = s;
    }
  for (int i = 0; i < 4; ++i)
    for (int j = 0; j < 4; ++j) {
      double s = 0;
      for (int k = 0; k < 4; ++k) s += t[i][k] * BT[j][k];
      V[i * 4 + j] = s;
    }
}

/* Y = A^T M A, A^T = [[1,1,1,0],[0,1,-1,-1]] (hip_kernels.h:133-141). */
void or_winograd_output(const double* Mm, double* Y) {
  static const double AT[2][4] = {{1, 1, 1, 0}, {0, 1, -1, -1}};
  double t[2][4];
  for (int i = 0; i < 2; ++i)
    for (int j = 0; j < 4; ++j) {
      double s = 0;
      for (int k = 0; k < 4; ++k) s += AT[i][k] * Mm[k * 4 + j];
      t[i][j] = s;
    }
  for (int i = 0; i < 2; ++i)
    for (int j = 0; j < 2; ++j) {
      double s = 0;
      for (int k = 0; k < 4; ++k) s += t[i][k] * AT[j][k];
      Y[i * 2 + j] = s;
    }
}

int or_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

void or_set_num_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}

// gfx950 (CDNA4) kernels for the conv-chain upscaler path.
//
// Replaces the reference's device code (src/common/hip_kernels.h): the
// Winograd conv (winograd_conv 143-396), the single-channel head conv
// (direct_conv 402-483), DepthToSpace (dts_kernel* 532-616), the unfused
// pointwise ops (unary_kernel/binary_kernel 493-519) and the NCHW<->NHWC IO
// kernels (629-670). Written for 64-wide wavefronts and the
// v_mfma_f32_16x16x32_f16 matrix instruction; nothing here is shared with the
// reference's wave32 WMMA design.
//
// winograd_conv data flow (F(2x2,3x3), one persistent workgroup per slot):
//   * Each wave owns one 16-wide block of output channels and keeps its share
//     of the transformed filters U' (16 positions x C x 16 outputs, fp16) in
//     VGPRs for the whole launch, so U is read from HBM/L2 once per workgroup.
//   * Per work item (1 tile row x 16*tb tile columns): all threads load 4x4
//     input patches (4 channels per lane, NHWC fp16, zero padded), apply
//     V' = (B^T d B)/4 in packed fp16 and write V' to LDS as
//     [position][tile][channel] with a 16-byte row pad (conflict-free 16-byte
//     reads for the MFMA B operand).
//   * Each wave runs, per position, KC chained MFMAs over 32-channel chunks
//     (A = U' rows = output channels, B = V' columns = tiles) and folds the
//     16 position results into the 2x2 output tile with A^T M A in fp32.
//   * Epilogue in fp32: bias, ReLU/SiLU, up to two residual inputs, Clip, one
//     rounding; stores NHWC fp16, or the NCHW boundary layout (fp16/fp32),
//     optionally through a fused DepthToSpace.
//
// Scaling: V is computed as (B^T d B)/4 (exact in fp16 away from subnormals)
// so that |V'| <= max|d| never overflows fp16; the host packs U' = 4*U to
// compensate. Column-3 positions come out with the opposite sign (that keeps
// the scaled transform at one fused multiply-add per value); the output fold
// absorbs the sign, so U' is not negated.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "conv_args.h"
#include "pack.h"

namespace arthip {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

// Workgroup barrier that first retires this wave's outstanding LDS traffic.
// s_barrier alone orders control flow only; a ds_write still in flight could
// otherwise be read stale by another wave after the barrier.
__device__ __forceinline__ void lds_sync() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __syncthreads();
}

__device__ __forceinline__ float apply_act(float y, int act) {
  if (act == kActRelu) return (y < 0.0f) ? 0.0f : y;  // NaN propagates
  if (act == kActSilu) return y * __builtin_amdgcn_rcpf(1.0f + __expf(-y));
  return y;
}

__device__ __forceinline__ float apply_clip(float y, float lo, float hi) {
  // Comparisons are false for NaN, so NaN passes through (ONNX Clip).
  return (y < lo) ? lo : ((y > hi) ? hi : y);
}

// Epilogue for 4 consecutive output channels [ch0, ch0+4) of one pixel.
// ch0 is a multiple of 4 and ch0 < M; lanes for channels >= M keep out.
__device__ __forceinline__ void store4(const Epilogue& e, int M, int H, int W, int n, int oh,
                                       int ow, int ch0, f4 v) {
  const int64_t pix = ((int64_t)n * H + oh) * W + ow;
  const bool vec = (M & 3) == 0;  // then ch0 + 3 < M
  v += *reinterpret_cast<const f4*>(e.bias + ch0);
#pragma unroll
  for (int q = 0; q < 4; ++q) v[q] = apply_act(v[q], e.act);
  const _Float16* sk[2] = {reinterpret_cast<const _Float16*>(e.skip0),
                           reinterpret_cast<const _Float16*>(e.skip1)};
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    if (sk[s] == nullptr) continue;
    const _Float16* p = sk[s] + pix * M + ch0;
    if (vec) {
      const h4 x = *reinterpret_cast<const h4*>(p);
#pragma unroll
      for (int q = 0; q < 4; ++q) v[q] += (float)x[q];
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (ch0 + q < M) v[q] += (float)p[q];
    }
  }
  if (e.do_clip) {
#pragma unroll
    for (int q = 0; q < 4; ++q) v[q] = apply_clip(v[q], e.clip_lo, e.clip_hi);
  }
  if (e.dts_b >= 2) {
    // DepthToSpace DCR: channel k = (r*b + q)*Cout + c lands at
    // (c, oh*b + r, ow*b + q) of the NCHW [n][Cout][H*b][W*b] output.
    const int b = e.dts_b;
    const int cout = M / (b * b);
    const int64_t Ho = (int64_t)H * b, Wo = (int64_t)W * b;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int k = ch0 + q;
      if (k >= M) break;
      const int rq = k / cout;
      const int c = k - rq * cout;
      const int r = rq / b;
      const int qq = rq - r * b;
      const int64_t idx = (((int64_t)n * cout + c) * Ho + (int64_t)oh * b + r) * Wo +
                          (int64_t)ow * b + qq;
      if (e.out_kind == kOutNchwF32)
        reinterpret_cast<float*>(e.out)[idx] = v[q];
      else
        reinterpret_cast<_Float16*>(e.out)[idx] = (_Float16)v[q];
    }
    return;
  }
  if (e.out_kind == kOutNhwcF16) {
    _Float16* o = reinterpret_cast<_Float16*>(e.out) + pix * M + ch0;
    if (vec) {
      h4 r;
#pragma unroll
      for (int q = 0; q < 4; ++q) r[q] = (_Float16)v[q];
      *reinterpret_cast<h4*>(o) = r;
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (ch0 + q < M) o[q] = (_Float16)v[q];
    }
    return;
  }
  // NCHW boundary layout.
  const int64_t plane = (int64_t)H * W;
  const int64_t base = ((int64_t)n * M + ch0) * plane + (int64_t)oh * W + ow;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    if (ch0 + q >= M) break;
    if (e.out_kind == kOutNchwF32)
      reinterpret_cast<float*>(e.out)[base + q * plane] = v[q];
    else
      reinterpret_cast<_Float16*>(e.out)[base + q * plane] = (_Float16)v[q];
  }
}

// ---------------------------------------------------------------------------
// Winograd F(2x2,3x3)
// ---------------------------------------------------------------------------

// 4x4 input patch with top-left input pixel (h0, w0), channels [c0, c0+4).
// Out-of-image pixels and channels >= C read as zero (SAME padding and the
// channel padding of the last 32-channel chunk).
__device__ __forceinline__ void load_patch(const WinoArgs& a, int n, int h0, int w0, int c0,
                                           h4 d[16]) {
  const _Float16* in = reinterpret_cast<const _Float16*>(a.in);
  const bool cvec = (a.C & 3) == 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int h = h0 + i;
    const bool hok = (h >= 0) && (h < a.H);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int w = w0 + j;
      h4 v = {0, 0, 0, 0};
      if (hok && w >= 0 && w < a.W && c0 < a.C) {
        const _Float16* p = in + (((int64_t)n * a.H + h) * a.W + w) * a.C + c0;
        if (cvec) {
          v = *reinterpret_cast<const h4*>(p);
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q)
            if (c0 + q < a.C) v[q] = p[q];
        }
      }
      d[i * 4 + j] = v;
    }
  }
}

// V' for positions p = 4*i + j: V'_{i,j} = (B^T d B)_{i,j} / 4 for j < 3 and
// -(B^T d B)_{i,3} / 4 for j == 3, with B^T = [[1,0,-1,0],[0,1,1,0],
// [0,-1,1,0],[0,1,0,-1]]. First stage (columns) in plain fp16; the second
// stage folds the 1/4 into one fma per value.
__device__ __forceinline__ void input_transform(const h4 d[16], h4 v[16]) {
  h4 t[16];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    t[0 * 4 + j] = d[0 * 4 + j] - d[2 * 4 + j];
    t[1 * 4 + j] = d[1 * 4 + j] + d[2 * 4 + j];
    t[2 * 4 + j] = d[2 * 4 + j] - d[1 * 4 + j];
    t[3 * 4 + j] = d[1 * 4 + j] - d[3 * 4 + j];
  }
  const h4 qp = {0.25f16, 0.25f16, 0.25f16, 0.25f16};
  const h4 qn = {-0.25f16, -0.25f16, -0.25f16, -0.25f16};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const h4 n1 = t[i * 4 + 1] * qn;
    const h4 n2 = t[i * 4 + 2] * qn;
    v[i * 4 + 0] = __builtin_elementwise_fma(t[i * 4 + 0], qp, n2);   // (t0 - t2)/4
    v[i * 4 + 1] = __builtin_elementwise_fma(t[i * 4 + 1], qp, -n2);  // (t1 + t2)/4
    v[i * 4 + 2] = __builtin_elementwise_fma(t[i * 4 + 2], qp, n1);   // (t2 - t1)/4
    v[i * 4 + 3] = __builtin_elementwise_fma(t[i * 4 + 3], qp, n1);   // (t3 - t1)/4
  }
}

template <int KC>
__global__ void __launch_bounds__(512) winograd_conv(WinoArgs a) {
  extern __shared__ __attribute__((aligned(16))) _Float16 vlds[];
  constexpr int CP = KC * 32;  // padded input channels
  constexpr int TS = CP + 8;   // LDS halfs per tile row (16-byte pad)
  constexpr int QUADS = CP / 4;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int ob = wave % a.n_ob;
  const int tbi = wave / a.n_ob;
  const int ntile = 16 * a.tb;
  const int wps = ntile * TS;  // LDS halfs per position

  // This wave's U' slice, laid out by the host in MFMA A-operand order:
  // [ob][position][kc][lane][8 halfs].
  h8 u[16][KC];
  {
    const h8* up = reinterpret_cast<const h8*>(a.u) + (size_t)ob * (16 * KC * 64) + lane;
#pragma unroll
    for (int p = 0; p < 16; ++p)
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) u[p][kc] = up[(p * KC + kc) * 64];
  }

  // Persistent schedule. Workgroups are dispatched round-robin over the 8
  // XCDs, so workgroup id % 8 is its XCD; each XCD walks one contiguous band
  // of work items so that vertically adjacent tile rows (which share input
  // halo rows) meet in the same L2. gridDim.x is a multiple of 8.
  const int xcd = blockIdx.x & 7;
  const int slot = blockIdx.x >> 3;
  const int nslot = gridDim.x >> 3;
  const int sb_begin = (int)(((int64_t)a.n_sb * xcd) >> 3);
  const int sb_end = (int)(((int64_t)a.n_sb * (xcd + 1)) >> 3);
  const int ntask = ntile * QUADS;

  for (int sb = sb_begin + slot; sb < sb_end; sb += nslot) {
    const int tws = sb % a.sb_w;
    const int rest = sb / a.sb_w;
    const int th = rest % a.tiles_h;
    const int n = rest / a.tiles_h;
    const int tw0 = tws * ntile;

    // ---- input transform into LDS
    for (int task = tid; task < ntask; task += blockDim.x) {
      const int t = task / QUADS;
      const int c0 = (task - t * QUADS) * 4;
      h4 d[16];
      load_patch(a, n, 2 * th - 1, 2 * (tw0 + t) - 1, c0, d);
      h4 v[16];
      input_transform(d, v);
      _Float16* dst = vlds + t * TS + c0;
#pragma unroll
      for (int p = 0; p < 16; ++p) *reinterpret_cast<h4*>(dst + p * wps) = v[p];
    }
    lds_sync();

    // ---- 16 position GEMMs on MFMA, folded row by row into the 2x2 tile
    f4 y00 = {0, 0, 0, 0}, y01 = y00, y10 = y00, y11 = y00;
    const _Float16* vb = vlds + (tbi * 16 + (lane & 15)) * TS + (lane >> 4) * 8;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      f4 m0 = {0, 0, 0, 0}, m1 = m0, m2 = m0, m3 = m0;
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) {
        const _Float16* p = vb + kc * 32 + (r * 4) * wps;
        const h8 b0 = *reinterpret_cast<const h8*>(p);
        const h8 b1 = *reinterpret_cast<const h8*>(p + wps);
        const h8 b2 = *reinterpret_cast<const h8*>(p + 2 * wps);
        const h8 b3 = *reinterpret_cast<const h8*>(p + 3 * wps);
        m0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(u[r * 4 + 0][kc], b0, m0, 0, 0, 0);
        m1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(u[r * 4 + 1][kc], b1, m1, 0, 0, 0);
        m2 = __builtin_amdgcn_mfma_f32_16x16x32_f16(u[r * 4 + 2][kc], b2, m2, 0, 0, 0);
        m3 = __builtin_amdgcn_mfma_f32_16x16x32_f16(u[r * 4 + 3][kc], b3, m3, 0, 0, 0);
      }
      // Column fold with A = [[1,0],[1,1],[1,-1],[0,-1]]. m3 holds -M_r3
      // (V' of column 3 is negated), so s1 = M_r1 - M_r2 - M_r3 = m1 - m2 + m3.
      const f4 s0 = m0 + m1 + m2;
      const f4 s1 = m1 - m2 + m3;
      if (r == 0) {
        y00 += s0;
        y01 += s1;
      } else if (r == 1) {
        y00 += s0;
        y01 += s1;
        y10 += s0;
        y11 += s1;
      } else if (r == 2) {
        y00 += s0;
        y01 += s1;
        y10 -= s0;
        y11 -= s1;
      } else {
        y10 -= s0;
        y11 -= s1;
      }
    }

    // ---- epilogue: lane holds 4 channels x 4 pixels of one tile
    {
      const int ch0 = ob * 16 + 4 * (lane >> 4);
      const int tw = tw0 + tbi * 16 + (lane & 15);
      if (ch0 < a.M && tw < a.tiles_w) {
        const int oh = 2 * th;
        const int ow = 2 * tw;
        const bool w1 = ow + 1 < a.W;
        store4(a.epi, a.M, a.H, a.W, n, oh, ow, ch0, y00);
        if (w1) store4(a.epi, a.M, a.H, a.W, n, oh, ow + 1, ch0, y01);
        if (oh + 1 < a.H) {
          store4(a.epi, a.M, a.H, a.W, n, oh + 1, ow, ch0, y10);
          if (w1) store4(a.epi, a.M, a.H, a.W, n, oh + 1, ow + 1, ch0, y11);
        }
      }
    }
    lds_sync();  // V' of this item is dead before the next item overwrites it
  }
}

// ---------------------------------------------------------------------------
// Direct 3x3 conv with one input channel (head conv)
// ---------------------------------------------------------------------------

// Each thread owns 8 output channels (g = thread % g8) for the whole launch and
// keeps their 9 taps (as 5 half2 pairs, the 10th tap zero) in VGPRs; the 9 input
// pixels are multiplied with v_dot2_f32_f16 (fp16 products, fp32 sums).
__global__ void __launch_bounds__(256) direct_conv_c1(DirectArgs a) {
  const int g = threadIdx.x & (a.g8 - 1);
  const int ppb = blockDim.x / a.g8;
  const int pl = threadIdx.x / a.g8;
  const int ch0 = g * 8;
  if (ch0 >= a.M) return;  // no barriers in this kernel
  h2 wr[8][5];
  {
    const h2* wp = reinterpret_cast<const h2*>(a.w) + (size_t)g * 40;
#pragma unroll
    for (int c = 0; c < 8; ++c)
#pragma unroll
      for (int k = 0; k < 5; ++k) wr[c][k] = wp[c * 5 + k];
  }
  const _Float16* in = reinterpret_cast<const _Float16*>(a.in);
  const int64_t npix = (int64_t)a.N * a.H * a.W;
  const int64_t step = (int64_t)gridDim.x * ppb;
  for (int64_t p = (int64_t)blockIdx.x * ppb + pl; p < npix; p += step) {
    const int ow = (int)(p % a.W);
    const int64_t rest = p / a.W;
    const int oh = (int)(rest % a.H);
    const int n = (int)(rest / a.H);
    _Float16 x[10];
#pragma unroll
    for (int r = 0; r < 3; ++r) {
      const int h = oh + r - 1;
#pragma unroll
      for (int s = 0; s < 3; ++s) {
        const int w = ow + s - 1;
        x[r * 3 + s] = (h >= 0 && h < a.H && w >= 0 && w < a.W)
                           ? in[((int64_t)n * a.H + h) * a.W + w]
                           : (_Float16)0.0f;
      }
    }
    x[9] = (_Float16)0.0f;
    h2 xv[5];
#pragma unroll
    for (int k = 0; k < 5; ++k) xv[k] = h2{x[2 * k], x[2 * k + 1]};
    f4 acc0, acc1;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
      for (int k = 0; k < 5; ++k) {
        s0 = __builtin_amdgcn_fdot2(xv[k], wr[c][k], s0, false);
        s1 = __builtin_amdgcn_fdot2(xv[k], wr[c + 4][k], s1, false);
      }
      acc0[c] = s0;
      acc1[c] = s1;
    }
    store4(a.epi, a.M, a.H, a.W, n, oh, ow, ch0, acc0);
    if (ch0 + 4 < a.M) store4(a.epi, a.M, a.H, a.W, n, oh, ow, ch0 + 4, acc1);
  }
}

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------

namespace {

int g_cu_count = 0;

int cu_count() {
  if (g_cu_count == 0) {
    int dev = 0;
    hipGetDevice(&dev);
    hipDeviceProp_t p{};
    if (hipGetDeviceProperties(&p, dev) == hipSuccess) g_cu_count = p.multiProcessorCount;
    if (g_cu_count <= 0) g_cu_count = 256;
  }
  return g_cu_count;
}

template <int KC>
hipError_t launch_wino_kc(const WinoArgs& a, int threads, size_t lds, int grid, hipStream_t s) {
  auto fn = winograd_conv<KC>;
  if (lds > 65536) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(fn, dim3(grid), dim3(threads), lds, s, a);
  return hipGetLastError();
}

template <int KC>
int wino_occupancy(int threads, size_t lds) {
  int blocks = 0;
  auto fn = winograd_conv<KC>;
  if (lds > 65536)
    hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                        hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, fn, threads, lds) != hipSuccess)
    blocks = 1;
  return blocks < 1 ? 1 : blocks;
}

}  // namespace

// Launch geometry of winograd_conv for one (C, M) pair.
WinoGeom winograd_geom(int C, int M) {
  WinoGeom g{};
  g.kc = (C + 31) / 32;
  g.n_ob = (M + 15) / 16;
  const int cp = g.kc * 32;
  int tb = (g.n_ob >= 4) ? 1 : 4 / g.n_ob;
  while (tb > 1 && 16 * 16 * tb * (cp + 8) * 2 > 80 * 1024) tb /= 2;
  g.tb = tb;
  g.threads = 64 * g.n_ob * g.tb;
  g.lds = (size_t)16 * 16 * tb * (cp + 8) * 2;
  return g;
}

int winograd_max_kc() { return 3; }
int winograd_max_m() { return 128; }

hipError_t launch_winograd(WinoArgs a, hipStream_t s) {
  const WinoGeom g = winograd_geom(a.C, a.M);
  a.n_ob = g.n_ob;
  a.tb = g.tb;
  a.tiles_h = (a.H + 1) / 2;
  a.tiles_w = (a.W + 1) / 2;
  a.sb_w = (a.tiles_w + 16 * g.tb - 1) / (16 * g.tb);
  a.n_sb = a.N * a.tiles_h * a.sb_w;
  int occ = 1;
  switch (g.kc) {
    case 1: occ = wino_occupancy<1>(g.threads, g.lds); break;
    case 2: occ = wino_occupancy<2>(g.threads, g.lds); break;
    case 3: occ = wino_occupancy<3>(g.threads, g.lds); break;
    default: return hipErrorInvalidValue;
  }
  int grid = cu_count() * occ;
  const int need = (a.n_sb + 7) / 8 * 8;
  if (grid > need) grid = need;
  grid = (grid + 7) / 8 * 8;
  switch (g.kc) {
    case 1: return launch_wino_kc<1>(a, g.threads, g.lds, grid, s);
    case 2: return launch_wino_kc<2>(a, g.threads, g.lds, grid, s);
    case 3: return launch_wino_kc<3>(a, g.threads, g.lds, grid, s);
    default: return hipErrorInvalidValue;
  }
}

int direct_g8(int M) {
  int g = 1;
  while (g * 8 < M) g *= 2;
  return g;
}

hipError_t launch_direct(DirectArgs a, hipStream_t s) {
  a.g8 = direct_g8(a.M);
  if (a.g8 > 256) return hipErrorInvalidValue;
  const int threads = 256;
  const int ppb = threads / a.g8;
  const int64_t npix = (int64_t)a.N * a.H * a.W;
  int64_t blocks = (npix + ppb - 1) / ppb;
  const int64_t cap = (int64_t)cu_count() * 8;
  if (blocks > cap) blocks = cap;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL(direct_conv_c1, dim3((unsigned)blocks), dim3(threads), 0, s, a);
  return hipGetLastError();
}

}  // namespace arthip

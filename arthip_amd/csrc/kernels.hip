// gfx950 (CDNA4) kernels for the conv-chain upscaler path.
//
// Replaces the reference's device code (src/common/hip_kernels.h): the
// Winograd conv (winograd_conv 143-396), the single-channel head conv
// (direct_conv 402-483), DepthToSpace (dts_kernel* 532-616), the unfused
// pointwise ops (unary_kernel/binary_kernel 493-519) and the NCHW<->NHWC IO
// kernels (629-670). Written for 64-wide wavefronts and the
// v_mfma_f32_16x16x32_f16 matrix instruction; nothing here follows the
// reference's wave32 WMMA design.
//
// winograd_conv data flow (F(2x2,3x3), persistent workgroups):
//   * Each wave owns one 16-wide block of output channels and keeps its share
//     of the transformed filters U' (16 positions x C x 16 outputs, fp16) in
//     VGPRs for the whole launch, so U' is read from HBM/L2 once per workgroup.
//   * Per work item (1 tile row x 16*tb tile columns) every thread owns input
//     tasks of one tile x 4 channels: it loads the 4x4 patch from the padded
//     NHWC input (no bounds checks), applies V' = (B^T d B)/4 in packed fp16
//     and writes V' to LDS as [position][tile][channel] with a 16-byte row pad
//     (conflict-free 16-byte reads for the MFMA B operand). When each thread
//     has exactly one task, the next item's patch is loaded into registers
//     while the current item runs on the matrix cores.
//   * Each wave runs, per position, KC chained MFMAs over 32-channel chunks
//     (A = U' rows = output channels, B = V' columns = tiles) and folds the
//     16 position results into the 2x2 output tile with A^T M A in fp32.
//   * Epilogue: bias, ReLU/SiLU, up to two residual inputs, Clip; stores the
//     padded NHWC layout, or the NCHW boundary layout (fp16/fp32), optionally
//     through a fused DepthToSpace.
//
// Scaling: V is computed as (B^T d B)/4 (exact in fp16 away from subnormals)
// so that |V'| <= 2 max|d| never overflows fp16 where d does not; the host packs
// U' = 4*U to compensate. Column-3 positions come out with the opposite sign
// (that keeps the scaled transform at one fused multiply-add per value); the
// output fold absorbs the sign, so U' is not negated.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdint>
#include <type_traits>

#include "conv_args.h"
#include "launch.h"
#include "pack.h"
#include "plan_rules.h"
#include "wino_dev.h"

namespace arthip {

// ---------------------------------------------------------------------------
// Epilogues
// ---------------------------------------------------------------------------

// General epilogue for 4 consecutive output channels [ch0, ch0+4) of pixel
// (oh, ow); fp32 until one final rounding. ch0 % 4 == 0 and ch0 < M.
__device__ __forceinline__ void store4(const Epilogue& e, int M, int H, int W, int Hp, int Wp,
                                       int n, int oh, int ow, int ch0, f4 v) {
  const int64_t ppix = ((int64_t)n * Hp + oh + 1) * Wp + ow + 1;  // padded pixel
  const bool vec = (M & 3) == 0;                                  // then ch0 + 3 < M
  v += *reinterpret_cast<const f4*>(e.bias + ch0);
#pragma unroll
  for (int q = 0; q < 4; ++q) v[q] = apply_act(v[q], e.act);
  const _Float16* sk[2] = {reinterpret_cast<const _Float16*>(e.skip0),
                           reinterpret_cast<const _Float16*>(e.skip1)};
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    if (sk[s] == nullptr) continue;
    const _Float16* p = sk[s] + ppix * M + ch0;
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
  if (e.out_kind == kOutPadded) {
    _Float16* o = reinterpret_cast<_Float16*>(e.out) + ppix * M + ch0;
    if (vec) {
      *reinterpret_cast<h4*>(o) = to_h4(v);
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (ch0 + q < M) o[q] = (_Float16)v[q];
    }
    return;
  }
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

// Fast epilogue for 4 channels of one pixel: round acc + bias to fp16, then
// act and the residual adds in packed fp16. s0/s1 are zero when absent.
template <int ACT>
__device__ __forceinline__ h4 fast4(f4 y, f4 bias4, h4 s0, h4 s1) {
  h4 r = to_h4(y + bias4);
  if (ACT == kActRelu) r = __builtin_elementwise_max(r, h4{0, 0, 0, 0});
  if (ACT == kActSilu) r = silu4(r);
  r += s0;
  r += s1;
  return r;
}

// ---------------------------------------------------------------------------
// Winograd F(2x2,3x3)
// ---------------------------------------------------------------------------

// 4x4 patch of input task `task` (tile t of the item, channel quad c0) from
// the padded input; tasks past the last tile column or channel read as zero.
template <int KC, bool CVEC>
__device__ __forceinline__ void load_task(const WinoArgs& a, int n, int th, int tw0, int task,
                                          h4 d[16]) {
  constexpr int QUADS = KC * 8;
  const int t = task / QUADS;
  const int c0 = (task - t * QUADS) * 4;
  const bool ok = (tw0 + t < a.tiles_w) && (c0 < a.C);
  const _Float16* p = reinterpret_cast<const _Float16*>(a.in) +
                      (((int64_t)n * a.Hp + 2 * th) * a.Wp + 2 * (tw0 + t)) * a.C + c0;
  const int64_t rs = (int64_t)a.Wp * a.C;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      h4 v = {0, 0, 0, 0};
      if (ok) {
        const _Float16* q = p + i * rs + j * a.C;
        if (CVEC) {
          v = *reinterpret_cast<const h4*>(q);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (c0 + e < a.C) v[e] = q[e];
        }
      }
      d[i * 4 + j] = v;
    }
  }
}

// Writes V' of one task: V'_{i,j} = (B^T d B)_{i,j}/4 for j < 3 and
// -(B^T d B)_{i,3}/4, with B^T = [[1,0,-1,0],[0,1,1,0],[0,-1,1,0],[0,1,0,-1]].
// First stage (columns) in plain fp16; the second stage folds the 1/4 into one
// fma per value and streams each output row to LDS.
template <int KC>
__device__ __forceinline__ void store_v(_Float16* vlds, int wps, int task, const h4 d[16]) {
  constexpr int TS = KC * 32 + 8;
  constexpr int QUADS = KC * 8;
  const int t = task / QUADS;
  const int c0 = (task - t * QUADS) * 4;
  _Float16* dst = vlds + t * TS + c0;
  h4 tt[16];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    tt[0 * 4 + j] = d[0 * 4 + j] - d[2 * 4 + j];
    tt[1 * 4 + j] = d[1 * 4 + j] + d[2 * 4 + j];
    tt[2 * 4 + j] = d[2 * 4 + j] - d[1 * 4 + j];
    tt[3 * 4 + j] = d[1 * 4 + j] - d[3 * 4 + j];
  }
  const h4 qp = {0.25f16, 0.25f16, 0.25f16, 0.25f16};
  const h4 qn = {-0.25f16, -0.25f16, -0.25f16, -0.25f16};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const h4 n1 = tt[i * 4 + 1] * qn;
    const h4 n2 = tt[i * 4 + 2] * qn;
    _Float16* row = dst + (i * 4) * wps;
    *reinterpret_cast<h4*>(row) = __builtin_elementwise_fma(tt[i * 4 + 0], qp, n2);
    *reinterpret_cast<h4*>(row + wps) = __builtin_elementwise_fma(tt[i * 4 + 1], qp, -n2);
    *reinterpret_cast<h4*>(row + 2 * wps) = __builtin_elementwise_fma(tt[i * 4 + 2], qp, n1);
    *reinterpret_cast<h4*>(row + 3 * wps) = __builtin_elementwise_fma(tt[i * 4 + 3], qp, n1);
  }
}

struct WinoSched {
  FastDiv sb_w, tiles_h;
};

// Item index -> (n, tile row, first tile column).
__device__ __forceinline__ void item_coords(const WinoSched& sc, int sb, int ntile, int& n,
                                            int& th, int& tw0) {
  const uint32_t rest = fdiv((uint32_t)sb, sc.sb_w);
  const uint32_t tws = (uint32_t)sb - rest * sc.sb_w.d;
  const uint32_t nn = fdiv(rest, sc.tiles_h);
  th = (int)(rest - nn * sc.tiles_h.d);
  n = (int)nn;
  tw0 = (int)tws * ntile;
}

// KC:    32-channel input chunks (C <= 32*KC); U' of this wave lives in VGPRs.
// CVEC:  C % 4 == 0 (8-byte input loads).
// FAST:  padded NHWC output with M % 4 == 0 and no clip (the inner layers);
//        else the general epilogue (boundary layouts, fused DepthToSpace, odd M).
template <int KC, bool CVEC, bool FAST>
__global__ void __launch_bounds__(512) winograd_conv(WinoArgs a, WinoSched sc) {
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
  const int ntask = ntile * QUADS;

  // Persistent schedule. Workgroups are dispatched round-robin over the 8
  // XCDs, so workgroup id % 8 is its XCD; each XCD walks one contiguous band
  // of work items so that vertically adjacent tile rows (which share input
  // halo rows) meet in the same L2. gridDim.x is a multiple of 8.
  const int xcd = blockIdx.x & 7;
  const int nslot = gridDim.x >> 3;
  const int sb_end = (int)(((int64_t)a.n_sb * (xcd + 1)) >> 3);
  int sb = (int)(((int64_t)a.n_sb * xcd) >> 3) + (blockIdx.x >> 3);
  if (sb >= sb_end) return;  // uniform across the workgroup

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

  // Lane's output coordinates within an item: 4 channels x one tile.
  const int ch0 = ob * 16 + 4 * (lane >> 4);
  const int tcol = tbi * 16 + (lane & 15);
  f4 bias4 = {0, 0, 0, 0};
  if (FAST && ch0 < a.M) bias4 = *reinterpret_cast<const f4*>(a.epi.bias + ch0);

  int n, th, tw0;
  item_coords(sc, sb, ntile, n, th, tw0);
  h4 d[16];

  for (;;) {
    // ---- input transform into LDS
    for (int task = tid; task < ntask; task += blockDim.x) {
      load_task<KC, CVEC>(a, n, th, tw0, task, d);
      store_v<KC>(vlds, wps, task, d);
    }
    lds_sync();

    const int nsb = sb + nslot;
    const bool more = nsb < sb_end;
    int nn = n, nth = th, ntw0 = tw0;
    if (more) item_coords(sc, nsb, ntile, nn, nth, ntw0);

    const int tw = tw0 + tcol;
    const bool valid = (ch0 < a.M) && (tw < a.tiles_w);
    const int oh = 2 * th, ow = 2 * tw;
    const bool h1 = oh + 1 < a.H, w1 = ow + 1 < a.W;
    const int64_t ppix = ((int64_t)n * a.Hp + oh + 1) * a.Wp + ow + 1;
    const int64_t prow = (int64_t)a.Wp * a.M;
    // Residual inputs for the fast epilogue, loaded after the MFMA work (before
    // it they would hold 16 more VGPRs across it).
    h4 sk[2][4];
    auto load_skips = [&]() {
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const _Float16* sp = reinterpret_cast<const _Float16*>(s == 0 ? a.epi.skip0 : a.epi.skip1);
#pragma unroll
        for (int q = 0; q < 4; ++q) sk[s][q] = h4{0, 0, 0, 0};
        if (sp != nullptr && valid) {
          const _Float16* b = sp + ppix * a.M + ch0;
          sk[s][0] = *reinterpret_cast<const h4*>(b);
          if (w1) sk[s][1] = *reinterpret_cast<const h4*>(b + a.M);
          if (h1) {
            sk[s][2] = *reinterpret_cast<const h4*>(b + prow);
            if (w1) sk[s][3] = *reinterpret_cast<const h4*>(b + prow + a.M);
          }
        }
      }
    };

    // ---- 16 position GEMMs on MFMA, folded row by row into the 2x2 tile
    f4 y[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) y[q] = f4{0, 0, 0, 0};
    const _Float16* vb = vlds + tcol * TS + (lane >> 4) * 8;
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
        y[0] += s0;
        y[1] += s1;
      } else if (r == 1) {
        y[0] += s0;
        y[1] += s1;
        y[2] += s0;
        y[3] += s1;
      } else if (r == 2) {
        y[0] += s0;
        y[1] += s1;
        y[2] -= s0;
        y[3] -= s1;
      } else {
        y[2] -= s0;
        y[3] -= s1;
      }
    }

    // ---- epilogue: lane holds 4 channels x the 4 pixels of one tile
    if (FAST) load_skips();
    if (valid) {
      if (FAST) {
        _Float16* o = reinterpret_cast<_Float16*>(a.epi.out) + ppix * a.M + ch0;
        const int64_t off[4] = {0, a.M, prow, prow + a.M};
        const bool ok[4] = {true, w1, h1, h1 && w1};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          if (!ok[q]) continue;
          h4 r;
          if (a.epi.act == kActRelu)
            r = fast4<kActRelu>(y[q], bias4, sk[0][q], sk[1][q]);
          else if (a.epi.act == kActSilu)
            r = fast4<kActSilu>(y[q], bias4, sk[0][q], sk[1][q]);
          else
            r = fast4<kActNone>(y[q], bias4, sk[0][q], sk[1][q]);
          *reinterpret_cast<h4*>(o + off[q]) = r;
        }
      } else {
        store4(a.epi, a.M, a.H, a.W, a.Hp, a.Wp, n, oh, ow, ch0, y[0]);
        if (w1) store4(a.epi, a.M, a.H, a.W, a.Hp, a.Wp, n, oh, ow + 1, ch0, y[1]);
        if (h1) {
          store4(a.epi, a.M, a.H, a.W, a.Hp, a.Wp, n, oh + 1, ow, ch0, y[2]);
          if (w1) store4(a.epi, a.M, a.H, a.W, a.Hp, a.Wp, n, oh + 1, ow + 1, ch0, y[3]);
        }
      }
    }
    lds_sync();  // V' of this item is dead before the next item overwrites it
    if (!more) break;
    sb = nsb;
    n = nn;
    th = nth;
    tw0 = ntw0;
  }
}

// ---------------------------------------------------------------------------
// Winograd F(2x2,3x3), sliding-window variant for C == M in {32, 64}
// ---------------------------------------------------------------------------
//
// A workgroup of 2*KC waves (one 16-wide output-channel block each) walks a
// contiguous range of work items, each 1 tile row x 16 tile columns, ordered
// down a 16-tile-wide strip. Consecutive items of a strip share two of their
// four input rows, so a thread keeps the lower two rows of its 4x4 patch in
// registers and loads only the two new rows; the loads are issued right after
// the item's barrier and land while the item runs on the matrix cores. V' is
// double-buffered in LDS, so one barrier per item suffices: a wave writing
// buffer b for item i+2 has passed the barrier of item i+1, which every wave
// reaches only after its MFMA reads of item i.
//
// Fold: with m_rc the product at position (r, c) (column 3 negated by the
// input transform), row r needs P_r = m_r0 + m_r1 + m_r2 and
// Q_r = m_r1 - m_r2 + m_r3. Chaining the accumulators gives
// X = m_r2, b = X + m_r1, P_r = b + m_r0, c = b + m_r3 and Q_r = c - 2X with
// one fused multiply-add per value. Row 1 starts from the bias instead
// (Y = bias + m_11; b = Y + m_12; P_1 = b + m_10; c = Y + m_13; Q_1 = c - b + Y):
// (1,1) is the one position every output takes with coefficient +1, so the
// bias lands exactly once in each output. Then
//   y00 = P0 + P1 + P2, y01 = Q0 + Q1 + Q2, y10 = P1 - P2 - P3, y11 = Q1 - Q2 - Q3,
// accumulated row by row.

template <int KC, int ACT, int NSKIP>
__global__ void __launch_bounds__(128 * KC) __attribute__((amdgpu_waves_per_eu(2, 2)))
winograd_strip(StripArgs a) {
  constexpr int C = 32 * KC;   // input channels = output channels
  constexpr int WPS = StripLds<KC>::WPS;
  constexpr int VBUF = StripLds<KC>::VBUF;
  constexpr int SBUF = StripStage<KC>::SBUF;
  constexpr int GR = StripStage<KC>::G;
  constexpr int QUADS = C / 4;
  constexpr int PX = 2 * C;    // bytes per pixel
  extern __shared__ __attribute__((aligned(16))) _Float16 vlds[];  // 2 V' + 2 staging buffers
  _Float16* const stg = vlds + 2 * VBUF;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;

  // Contiguous item range; workgroup id % 8 is the XCD, and each XCD takes a
  // contiguous eighth of the items.
  const int G = gridDim.x;
  const int slot = (blockIdx.x & 7) * (G >> 3) + (blockIdx.x >> 3);
  const int begin = (int)((int64_t)a.n_items * slot / G);
  const int end = (int)((int64_t)a.n_items * (slot + 1) / G);
  if (begin >= end) return;  // uniform across the workgroup

  h8 u[16][KC];
  {
    const h8* up = reinterpret_cast<const h8*>(a.u) + (size_t)wave * (16 * KC * 64) + lane;
#pragma unroll
    for (int p = 0; p < 16; ++p)
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) u[p][kc] = up[(p * KC + kc) * 64];
  }

  // Input task: tile tt of the item, channels [4*tq, 4*tq + 4).
  const int tt = tid / QUADS;
  const int tq = tid - tt * QUADS;
  // MFMA lane: tile tcol; B rows 8*kq.. of each 32-channel chunk; output
  // channels [ch0, ch0 + 4) of the tile's four pixels.
  const int tcol = lane & 15;
  const int kq = lane >> 4;
  const int ch0 = 16 * wave + 4 * kq;
  const f4 bias4 = *reinterpret_cast<const f4*>(a.bias + ch0);
  _Float16* const vw0 = vlds + StripLds<KC>::at(tt, 4 * tq);
  _Float16* const vw1 = vw0 + VBUF;
  const _Float16* vr0[KC];
  const _Float16* vr1[KC];
#pragma unroll
  for (int kc = 0; kc < KC; ++kc) {
    vr0[kc] = vlds + StripLds<KC>::at(tcol, 32 * kc + 8 * kq);
    vr1[kc] = vr0[kc] + VBUF;
  }
  // Staging write offset of (row 0, pixel 2*tcol); the other three pixels of
  // the tile are +C, +32C, +33C halfs (same swizzle: x >> 1 == tcol).
  const int sw0 = StripStage<KC>::at(0, 2 * tcol, ch0 >> 3) + (ch0 & 7);
  // Store phase: thread handles group sg of pixel sx in both rows.
  const int sx = tid / GR;
  const int sg = tid - sx * GR;
  const int sr0 = StripStage<KC>::at(0, sx, sg);
  const uint32_t s_lane = (uint32_t)(sx * C + sg * 8) * 2;  // bytes from the row's first pixel
  const int64_t row_bytes = (int64_t)a.Wp * PX;

  int n, s, th;
  auto decode = [&](int item) {
    const uint32_t sgl = fdiv((uint32_t)item, a.fd_tiles_h);
    th = item - (int)(sgl * (uint32_t)a.tiles_h);
    const uint32_t nn = fdiv(sgl, a.fd_strips);
    s = (int)(sgl - nn * (uint32_t)a.n_strips);
    n = (int)nn;
  };
  // Byte offset of this thread's patch within a strip row; tiles past the
  // right edge read tile 0's patch (their outputs are never stored).
  uint32_t in_lane = 0;
  auto in_row = [&](int r) {
    return reinterpret_cast<const char*>(a.in) + (((int64_t)n * a.Hp + r) * a.Wp + 32 * s) * PX;
  };
  // Input rows are nontemporal: in the model's residual layers nothing reads
  // them again, and bypassing the caches keeps the residual input (which the
  // previous layer just read) cached (1080p 64 -> 64: 152 -> 146 us).
  auto load2 = [&](h2 (&x)[16], const char* rb) {
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const h4 v = __builtin_nontemporal_load(reinterpret_cast<const h4*>(rb + r * row_bytes + in_lane + j * PX));
        x[2 * (4 * r + j)] = __builtin_shufflevector(v, v, 0, 1);
        x[2 * (4 * r + j) + 1] = __builtin_shufflevector(v, v, 2, 3);
      }
  };

  // Coordinates of the item whose output sits in staging, and its residual
  // inputs (loaded after the next item's barrier, consumed after that item's
  // MFMA work). Residual loads and output stores go through buffer resources
  // spanning the item's two output rows: pixels past the right edge and the
  // second row past the bottom get an offset beyond the resource's size, which
  // the hardware drops (stores) or reads as zero (loads). Every thread thus
  // issues the same number of memory instructions on every path, and the
  // waits before the next transform count exactly the input-row loads instead
  // of also waiting on this item's stores.
  int pn = 0, ps = 0, pth = 0;
  bool have_prev = false;  // uniform: staging holds an item not yet stored
  h8 skr[2][2];
  constexpr uint32_t kOob = 0x80000000u;
  const uint32_t rb32 = (uint32_t)row_bytes;
  const int n_rec = (int)(rb32 + 32 * PX);
  auto st_off = [&](int r) -> uint32_t {
    const bool ok = have_prev && (32 * ps + sx < a.W) && (r == 0 || 2 * pth + 1 < a.H);
    return ok ? (uint32_t)r * rb32 + s_lane : kOob;
  };
  auto item_pix = [&]() {
    return ((int64_t)pn * a.Hp + 2 * pth + 1) * a.Wp + 32 * ps + 1;
  };
  auto load_skips = [&]() {
#pragma unroll
    for (int k = 0; k < 2; ++k)
#pragma unroll
      for (int r = 0; r < 2; ++r) skr[k][r] = h8{0, 0, 0, 0, 0, 0, 0, 0};
    if (NSKIP > 0) {
      const int64_t pix0 = item_pix();
      const uint32_t o0 = st_off(0), o1 = st_off(1);
#pragma unroll
      for (int k = 0; k < NSKIP; ++k) {
        const char* sb = reinterpret_cast<const char*>(k == 0 ? a.skip0 : a.skip1) + pix0 * PX;
        const __amdgpu_buffer_rsrc_t rs =
            __builtin_amdgcn_make_buffer_rsrc((void*)sb, (short)0, n_rec, 0x00020000);
        skr[k][0] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(rs, o0, 0, kNonTemporal));
        skr[k][1] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(rs, o1, 0, kNonTemporal));
      }
    }
  };
  auto store_phase = [&](int SB) {
    char* ob = reinterpret_cast<char*>(a.out) + item_pix() * PX;
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void*)ob, (short)0, n_rec, 0x00020000);
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      h8 v = *reinterpret_cast<const h8*>(stg + SB * SBUF + sr0 + r * 32 * C);
      if (NSKIP > 0) v += skr[0][r];
      if (NSKIP > 1) v += skr[1][r];
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, v), rs, st_off(r), 0,
                                             kNonTemporal);
    }
  };

  // One item: transform, barrier, loads (the previous item's residual inputs,
  // the next item's rows), MFMA work, store of the previous item's output,
  // staging of this item's output. The first item of a run has no previous
  // item in staging (the run start drained it); its store phase is issued with
  // out-of-range offsets, keeping the instruction count of every path equal.
  // The next item's two new rows go into `top` (the rows the transform just
  // consumed); past the last item of the run the row index is clamped to the
  // last two rows of the padded image, which are loaded and never used, so the
  // loop body has no data-dependent branch around a load.
  h2 A[16], B[16];
  auto body = [&](auto buf_tag, h2 (&top)[16], h2 (&bot)[16]) {
    constexpr int BUF = decltype(buf_tag)::value;
    _Float16* const vw = BUF ? vw1 : vw0;
    const _Float16* const* vr = BUF ? vr1 : vr0;
    strip_transform<KC>(vw, top, bot);
    lds_sync();
    load_skips();
    {
      const int r = 2 * th + 4;
      load2(top, in_row(r < a.Hp - 2 ? r : a.Hp - 2));
    }

    // 16 position GEMMs, folded through the accumulator chains.
    auto mm = [&](int p, f4 acc) {
#pragma unroll
      for (int kc = 0; kc < KC; ++kc)
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(
            u[p][kc], *reinterpret_cast<const h8*>(vr[kc] + p * WPS), acc, 0, 0, 0);
      return acc;
    };
    const f4 z = {0, 0, 0, 0};
    const f4 m2 = {-2.0f, -2.0f, -2.0f, -2.0f};
    // Row by row, accumulated into the four outputs as each row completes.
    f4 y00, y01, y10, y11;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      f4 P, Q;
      if (r == 1) {
        const f4 Y = mm(5, bias4);
        const f4 b = mm(6, Y);
        P = mm(4, b);
        const f4 c = mm(7, Y);
        Q = (c - b) + Y;
      } else {
        const f4 X = mm(4 * r + 2, z);
        const f4 b = mm(4 * r + 1, X);
        P = mm(4 * r, b);
        const f4 c = mm(4 * r + 3, b);
        Q = __builtin_elementwise_fma(X, m2, c);
      }
      if (r == 0) {
        y00 = P;
        y01 = Q;
      } else if (r == 1) {
        y00 += P;
        y01 += Q;
        y10 = P;
        y11 = Q;
      } else if (r == 2) {
        y00 += P;
        y01 += Q;
        y10 -= P;
        y11 -= Q;
      } else {
        y10 -= P;
        y11 -= Q;
      }
    }
    store_phase(BUF ^ 1);
    _Float16* sw = stg + BUF * SBUF + sw0;
    *reinterpret_cast<h4*>(sw) = strip_act4<ACT>(y00);
    *reinterpret_cast<h4*>(sw + C) = strip_act4<ACT>(y01);
    *reinterpret_cast<h4*>(sw + 32 * C) = strip_act4<ACT>(y10);
    *reinterpret_cast<h4*>(sw + 33 * C) = strip_act4<ACT>(y11);
    pn = n;
    ps = s;
    pth = th;
    have_prev = true;
    ++th;
  };

  // Runs: maximal stretches of the item range within one strip. Each run
  // starts by storing the previous run's last item (after its initial loads,
  // so that the loop is entered with the same memory-instruction order as its
  // back edge: input rows, then two stores); the range ends with a final drain.
  int last_buf = 0;
  for (int it = begin; it < end;) {
    decode(it);
    const int len = min(end - it, a.tiles_h - th);
    {
      const int t = (16 * s + tt < a.tiles_w) ? tt : 0;
      in_lane = (uint32_t)(2 * t * C + 4 * tq) * 2;
    }
    load2(A, in_row(2 * th));
    load2(B, in_row(2 * th + 2));
    load_skips();
    // Orders the previous run's staging writes before the store below and its
    // last V' reads before this run's first transform (buffer parity restarts).
    lds_sync();
    store_phase(last_buf);
    have_prev = false;
    for (int k = len;;) {
      body(IntC<0>{}, A, B);
      last_buf = 0;
      if (--k == 0) break;
      body(IntC<1>{}, B, A);
      last_buf = 1;
      if (--k == 0) break;
    }
    it += len;
  }
  load_skips();
  lds_sync();
  store_phase(last_buf);
}

// ---------------------------------------------------------------------------
// Producer/consumer strip conv (C = M in {64, 96})
// ---------------------------------------------------------------------------
//
// The items (1 tile row x 16 tiles), fold and output staging of
// winograd_strip, split over two kinds of waves of one 512-thread workgroup
// per CU:
//   * waves 0 .. 2*KC-1 (consumers) keep U' of 16 output channels each in
//     VGPRs and run the MFMA fold into staging;
//   * the other waves (producers) load input rows and write V'. Holding no U',
//     they keep PipeL<KC>::NW - 1 row pairs in flight ahead of the transform,
//     so HBM latency hides behind that many items of work.
// Step j (one barrier each): the producers transform item j, the consumers
// fold item j-1, and item j-2 leaves staging for HBM. V' and staging are
// double-buffered by item parity, so each buffer's writes and reads are a
// barrier apart. A run (the items of one strip) restarts the producers' row
// window.
//
// Who moves item j-2 to HBM depends on C. At C = 64 the consumers apply the
// activation in the fold and store (four producer waves, one task each, have
// no room for it: 138 us instead of 122 with producer stores). At C = 96 the
// six consumer waves are the critical path, so the producers take the store
// phase: activation on the staged fp16 values, the residual inputs (loaded into
// registers one step ahead, added in graph order) and the stores. That took
// the one-residual 96 -> 96 layer from 312 to 279 us.
//
// Measured on the 1080p 64 -> 64 ReLU conv: 145 us with winograd_strip, 122 us
// here. Items of 32 tiles (two MFMA column blocks per wave) ran at 146 us: at
// 256 VGPRs the compiler keeps only one or two B reads ahead of the MFMAs.
// Splitting the fold by position rows over 8 consumer waves (12 waves, half of
// U' each, partial sums exchanged through LDS) ran at 137 us.
//
// C = 96: six consumer waves (192 VGPRs of U' each) and two producer waves,
// each transforming three (tile, 4-channel) tasks per item.
//
// Boundary layouts (C = M = 64 without residual inputs; IO bit 0 / bit 1):
// the producers can read the engine's NCHW fp16 input and the consumers write
// the NCHW fp16 output, so that a lone 64 -> 64 conv between boundary tensors
// needs no layout passes (W % 8 == 0). NCHW input: the producers copy the
// strip's rows into an LDS row ring (below) and repack each patch into the
// channel-pair layout of the transform; a producer wave's lanes take tiles
// 0-7 of four channel quads, then tiles 8-15, so that its V' writes hit
// distinct LDS banks. NCHW output:
// the fold stages the item channel-major ([row][channel][32 pixels], 80-byte
// channel rows so the fold's 4-byte writes of four channel quads land on
// distinct banks), and each consumer thread stores 8 pixels of one channel as
// a 16-byte word.
template <int KC>
struct PipeL;
template <>
struct PipeL<2> {
  static constexpr int TS = 64;  // halfs per tile row of V' (swizzled groups)
  static constexpr int NW = 6;   // producer row-pair slots
  __host__ __device__ static constexpr int at(int t, int c) { return StripLds<2>::at(t, c); }
  __host__ __device__ static constexpr int st(int row, int x, int g) {
    return StripStage<2>::at(row, x, g);
  }
};
template <>
struct PipeL<3> {
  // 224-byte tile rows (14 of the 16 bank quads). A ds_read_b128 serves 16
  // lanes per cycle: 8 consecutive lanes of one half of the wave together with
  // the same 8 of the other half (tiles t..t+7, channel groups g and g+1 for
  // the B reads), which with 14 quads per row land on 16 distinct quads (14 t
  // even, +1 odd). 208-byte rows (13 quads) doubled every B read: the counters
  // read 0.9 conflict cycles per LDS cycle. Staging rotates the 12 groups of
  // pixel x by x >> 1.
  static constexpr int TS = 112;
  static constexpr int NW = 3;
  __host__ __device__ static constexpr int at(int t, int c) { return t * TS + c; }
  __host__ __device__ static constexpr int st(int row, int x, int g) {
    return (row * 32 + x) * 96 + (((g + (x >> 1)) % 12) << 3);
  }
};

template <int KC>
struct PipeLds {
  static constexpr int C = 32 * KC;
  static constexpr int TILES = 16;
  static constexpr int PXS = 32;            // pixels per staged row
  static constexpr int WPS = TILES * PipeL<KC>::TS;  // halfs per position
  static constexpr int VBUF = 16 * WPS;     // halfs per V' buffer
  static constexpr int SBUF = 2 * PXS * C;  // halfs per staging buffer
  static constexpr int NCW = 2 * KC;        // consumer waves
  static constexpr int NPT = 64 * (8 - NCW);  // producer threads
  static constexpr int UP = 16 * 8 * KC / NPT;  // producer tasks per thread
  static constexpr int OCH = 2 * PXS * (C / 8) / NPT;  // 16-byte output chunks per producer thread
  // Channel-major staging of the NCHW output: [row][channel][NCS halfs].
  static constexpr int NCS = 40;
  static constexpr int SBUF_NCHW = 2 * C * NCS;
  // Row ring of the NCHW input (C = 64): NSL_NCHW slots of 12 KB after the
  // staging buffers.
  static constexpr int NSL_NCHW = 6;
  static constexpr size_t RING_NCHW_BYTES = (size_t)NSL_NCHW * 2 * 64 * 96;
  static constexpr size_t lds_bytes(bool out_nchw = false, bool in_nchw = false) {
    return (size_t)2 * (VBUF + (out_nchw ? SBUF_NCHW : SBUF)) * 2 +
           (in_nchw ? RING_NCHW_BYTES : 0);
  }
};

template <int KC, int ACT, int NSKIP, int IO = 0>
__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
winograd_pipe(StripArgs a) {
  using L = PipeLds<KC>;
  using LL = PipeL<KC>;
  constexpr int C = L::C;
  constexpr int NCW = L::NCW;
  constexpr bool IN_NCHW = (IO & 1) != 0;
  constexpr bool OUT_NCHW = (IO & 2) != 0;
  static_assert(IO == 0 || (KC == 2 && NSKIP == 0), "boundary layouts: 64 channels, no residuals");
  // With two residual inputs at C = 96 the producers' 3-slot row ring and
  // residual registers exceed 256 VGPRs and spill; a 2-slot ring does not
  // (1080p: 378 -> 327 us). Shallower rings elsewhere measured slower.
  constexpr int NW = (KC == 3 && NSKIP == 2) ? 2 : LL::NW;
  constexpr int UP = L::UP;
  constexpr int WPS = L::WPS;
  constexpr int VBUF = L::VBUF;
  constexpr int SBUF = OUT_NCHW ? L::SBUF_NCHW : L::SBUF;
  constexpr int PXS = L::PXS;
  constexpr int GR = C / 8;  // 16-byte groups per pixel
  constexpr int QUADS = C / 4;
  constexpr int PX = 2 * C;
  constexpr int OCH = L::OCH;
  // Who stores: the producers at C = 96 (six consumer waves are the critical
  // path there), the consumers at C = 64 (one producer wave per SIMD has no
  // room for the store phase).
  constexpr bool PS = KC == 3;
  static_assert(PS || NSKIP == 0, "residual inputs go through the producer store");
  static_assert(L::NPT * UP == 16 * QUADS, "producer tasks cover the item");
  static_assert(L::NPT * OCH == 2 * PXS * GR, "producer stores cover the item");
  // 2 V' | 2 staging
  extern __shared__ __attribute__((aligned(16))) _Float16 vlds[];
  _Float16* const stg = vlds + 2 * VBUF;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;

  const int G = gridDim.x;
  const int slot = (blockIdx.x & 7) * (G >> 3) + (blockIdx.x >> 3);
  const int begin = (int)((int64_t)a.n_items * slot / G);
  const int end = (int)((int64_t)a.n_items * (slot + 1) / G);
  if (begin >= end) return;  // uniform across the workgroup
  const int K = end - begin;

  const int64_t row_bytes = (int64_t)a.Wp * PX;
  const uint32_t rb32 = (uint32_t)row_bytes;
  const int n_rec = (int)(rb32 + L::PXS * PX);  // bytes of an item's two output rows
  constexpr uint32_t kOob = 0x80000000u;
  auto decode = [&](int item, int& n, int& s, int& th) {
    const uint32_t sgl = fdiv((uint32_t)item, a.fd_tiles_h);
    th = item - (int)(sgl * (uint32_t)a.tiles_h);
    const uint32_t nn = fdiv(sgl, a.fd_strips);
    s = (int)(sgl - nn * (uint32_t)a.n_strips);
    n = (int)nn;
  };

  if (wave < NCW) {
    // ---- consumers: step j folds item j-1 ----------------------------------
    h8 u[16][KC];
    {
      const h8* up = reinterpret_cast<const h8*>(a.u) + (size_t)wave * (16 * KC * 64) + lane;
#pragma unroll
      for (int p = 0; p < 16; ++p)
#pragma unroll
        for (int kc = 0; kc < KC; ++kc) u[p][kc] = up[(p * KC + kc) * 64];
    }
    const int tcol = lane & 15;
    const int kq = lane >> 4;
    const int ch0 = 16 * wave + 4 * kq;
    const f4 bias4 = *reinterpret_cast<const f4*>(a.bias + ch0);
    const _Float16* vr0[KC];
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) vr0[kc] = vlds + LL::at(tcol, 32 * kc + 8 * kq);
    // Pixels 2*tcol and 2*tcol + 1 share the staging rotation.
    const int sw0 = LL::st(0, 2 * tcol, ch0 >> 3) + (ch0 & 7);
    // Consumer store (C = 64): thread handles 16-byte group sg of pixel sx in
    // both rows; absent items and pixels past the edges get out-of-range
    // offsets, so every step issues the same two stores.
    const int sx = tid / GR;
    const int sg = tid - sx * GR;
    const int sr0 = LL::st(0, sx, sg);
    const uint32_t s_lane = (uint32_t)(sx * C + sg * 8) * 2;
    auto store_item = [&](int item, bool live, int SB) {
      int n, s, th;
      decode(item, n, s, th);
      if constexpr (OUT_NCHW) {
        // Thread: channel tid / 4, pixels 8 (tid % 4) .. + 7 of the item's
        // strip, in both rows; the row in the scalar offset.
        const uint32_t plane = (uint32_t)a.H * (uint32_t)a.W * 2;
        const char* ob = reinterpret_cast<const char*>(a.out) + (int64_t)n * C * plane;
        const __amdgpu_buffer_rsrc_t rs =
            __builtin_amdgcn_make_buffer_rsrc((void*)ob, (short)0, (int)(C * plane), 0x00020000);
        const int ch = tid >> 2, k = tid & 3;
        const int x = PXS * s + 8 * k;
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          const h8 v = *reinterpret_cast<const h8*>(stg + SB * SBUF + (r * C + ch) * L::NCS + 8 * k);
          const bool ok = live && x < a.W && 2 * th + r < a.H;
          __builtin_amdgcn_raw_buffer_store_b128(
              __builtin_bit_cast(u4, v), rs, ok ? (uint32_t)ch * plane + (uint32_t)x * 2 : kOob,
              (uint32_t)(2 * th + r) * (uint32_t)a.W * 2, kNonTemporal);
        }
        return;
      }
      const int64_t pix0 = ((int64_t)n * a.Hp + 2 * th + 1) * a.Wp + PXS * s + 1;
      char* ob = reinterpret_cast<char*>(a.out) + pix0 * PX;
      const __amdgpu_buffer_rsrc_t rs =
          __builtin_amdgcn_make_buffer_rsrc((void*)ob, (short)0, n_rec, 0x00020000);
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const h8 v = *reinterpret_cast<const h8*>(stg + SB * SBUF + sr0 + r * PXS * C);
        const bool ok = live && (PXS * s + sx < a.W) && (r == 0 || 2 * th + 1 < a.H);
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, v), rs,
                                               ok ? (uint32_t)r * rb32 + s_lane : kOob, 0,
                                               kNonTemporal);
      }
    };

    auto fold = [&](auto buf_tag) {
      constexpr int BUF = decltype(buf_tag)::value;
      auto mm = [&](int p, f4 acc) {
#pragma unroll
        for (int kc = 0; kc < KC; ++kc)
          acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(
              u[p][kc], *reinterpret_cast<const h8*>(vr0[kc] + BUF * VBUF + p * WPS), acc, 0, 0,
              0);
        return acc;
      };
      const f4 z = {0, 0, 0, 0};
      const f4 m2 = {-2.0f, -2.0f, -2.0f, -2.0f};
      f4 y00, y01, y10, y11;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        f4 P, Q;
        if (r == 1) {
          const f4 Y = mm(5, bias4);
          const f4 b = mm(6, Y);
          P = mm(4, b);
          const f4 c = mm(7, Y);
          Q = (c - b) + Y;
        } else {
          const f4 X = mm(4 * r + 2, z);
          const f4 b = mm(4 * r + 1, X);
          P = mm(4 * r, b);
          const f4 c = mm(4 * r + 3, b);
          Q = __builtin_elementwise_fma(X, m2, c);
        }
        if (r == 0) {
          y00 = P;
          y01 = Q;
        } else if (r == 1) {
          y00 += P;
          y01 += Q;
          y10 = P;
          y11 = Q;
        } else if (r == 2) {
          y00 += P;
          y01 += Q;
          y10 -= P;
          y11 -= Q;
        } else {
          y10 -= P;
          y11 -= Q;
        }
      }
      // With producer stores the activation is theirs (on the rounded value,
      // the same arithmetic).
      constexpr int FA = PS ? 0 : ACT;
      if constexpr (OUT_NCHW) {
        // Channel-major: pixels 2 tcol and 2 tcol + 1 of channel ch0 + e, per row.
        const h4 a0 = strip_act4<FA>(y00), a1 = strip_act4<FA>(y01);
        const h4 b0 = strip_act4<FA>(y10), b1 = strip_act4<FA>(y11);
        _Float16* sc = stg + BUF * SBUF + ch0 * L::NCS + 2 * tcol;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          *reinterpret_cast<h2*>(sc + e * L::NCS) = h2{a0[e], a1[e]};
          *reinterpret_cast<h2*>(sc + (C + e) * L::NCS) = h2{b0[e], b1[e]};
        }
        return;
      }
      _Float16* sw = stg + BUF * SBUF + sw0;
      *reinterpret_cast<h4*>(sw) = strip_act4<FA>(y00);
      *reinterpret_cast<h4*>(sw + C) = strip_act4<FA>(y01);
      *reinterpret_cast<h4*>(sw + PXS * C) = strip_act4<FA>(y10);
      *reinterpret_cast<h4*>(sw + (PXS + 1) * C) = strip_act4<FA>(y11);
    };

    // Step j folds item j-1 into buffer (j-1)&1 and, with consumer stores,
    // first stores item j-2 from buffer j&1. Steps alternate odd/even so both
    // parities are static.
    lds_sync();  // step 0
    for (int j = 1;; ++j) {
      if constexpr (!PS) store_item(begin + (j >= 2 ? j - 2 : 0), j >= 2, 1);  // odd j
      fold(IntC<0>{});
      lds_sync();
      if (j == K) break;
      ++j;
      if constexpr (!PS) store_item(begin + j - 2, true, 0);  // even j
      fold(IntC<1>{});
      lds_sync();
      if (j == K) break;
    }
    if constexpr (!PS) {
      store_item(begin + K - 1, true, (K + 1) & 1);  // step K + 1
      lds_sync();
    }
    return;
  }

  // ---- producers: step j transforms item j and stores item j-2 ---------------
  // Task v of thread p: flat index p + NPT * v -> tile, 4-channel quad.
  const int ptid = tid - 64 * NCW;
  int tt[UP];
  uint32_t tq4[UP];
  _Float16* vw0[UP];
#pragma unroll
  for (int v = 0; v < UP; ++v) {
    const int f = ptid + L::NPT * v;
    if constexpr (IN_NCHW) {
      // Lane l of producer wave w: tile (l & 7) + 8 (l >> 5), quad 4 w + ((l >> 3) & 3).
      const int l = ptid & 63;
      tt[v] = (l & 7) + 8 * (l >> 5);
      tq4[v] = (uint32_t)(4 * (4 * (ptid >> 6) + ((l >> 3) & 3)));
    } else {
      tt[v] = f / QUADS;
      tq4[v] = (uint32_t)(4 * (f - tt[v] * QUADS));
    }
    vw0[v] = vlds + LL::at(tt[v], (int)tq4[v]);
  }
  int n, s, th;  // the item being transformed
  uint32_t in_lane[UP];
  auto in_row = [&](int r) {
    if (r > a.Hp - 2) r = a.Hp - 2;
    return reinterpret_cast<const char*>(a.in) + (((int64_t)n * a.Hp + r) * a.Wp + PXS * s) * PX;
  };
  auto load2 = [&](h2 (&x)[UP][16], const char* rb) {
#pragma unroll
    for (int v = 0; v < UP; ++v)
#pragma unroll
      for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const h4 q = *reinterpret_cast<const h4*>(rb + r * row_bytes + in_lane[v] + j * PX);
          x[v][2 * (4 * r + j)] = __builtin_shufflevector(q, q, 0, 1);
          x[v][2 * (4 * r + j) + 1] = __builtin_shufflevector(q, q, 2, 3);
        }
  };
  int par = 0;  // parity of step j = parity of item j
  int js = 0;   // step j

  // Output chunks of this thread: chunk f = ptid + NPT * i -> row, pixel,
  // 16-byte group; its offset in the staging layout and in the item's two
  // output rows. Residual chunks use the same mapping.
  int oc_lds[OCH];
  uint32_t oc_off[OCH];
  int oc_x[OCH], oc_r[OCH];
#pragma unroll
  for (int i = 0; i < OCH; ++i) {
    const int f = ptid + L::NPT * i;
    const int r = f / (PXS * GR);
    const int x = (f / GR) % PXS;
    const int g = f % GR;
    oc_lds[i] = LL::st(r, x, g);
    oc_off[i] = (uint32_t)r * rb32 + (uint32_t)(x * C + g * 8) * 2;
    oc_x[i] = x;
    oc_r[i] = r;
  }
  // Buffer resource spanning item `item`'s two output rows in `base`, and the
  // chunk offsets: chunks past the right or bottom edge (or of an absent item)
  // get an offset beyond the resource, which reads as zero and drops stores,
  // so every step issues the same memory instructions.
  auto item_rsrc = [&](const void* base, int item) {
    int in_, is_, ith;
    decode(item, in_, is_, ith);
    const int64_t pix0 = ((int64_t)in_ * a.Hp + 2 * ith + 1) * a.Wp + PXS * is_ + 1;
    return __builtin_amdgcn_make_buffer_rsrc(
        (void*)(reinterpret_cast<const char*>(base) + pix0 * PX), (short)0, n_rec, 0x00020000);
  };
  auto chunk_off = [&](int item, bool live, int i) {
    int in_, is_, ith;
    decode(item, in_, is_, ith);
    const bool ok = live && (PXS * is_ + oc_x[i] < a.W) && (oc_r[i] == 0 || 2 * ith + 1 < a.H);
    return ok ? oc_off[i] : kOob;
  };
  h8 skv[NSKIP > 0 ? NSKIP : 1][OCH];
  // Residual chunks of item `item` (issued one step before its store).
  auto load_skips = [&](int item, bool live) {
    if (NSKIP == 0) return;
    const int it = live ? item : begin;
#pragma unroll
    for (int k = 0; k < NSKIP; ++k) {
      const __amdgpu_buffer_rsrc_t rs = item_rsrc(k == 0 ? a.skip0 : a.skip1, it);
#pragma unroll
      for (int i = 0; i < OCH; ++i)
        skv[k][i] = __builtin_bit_cast(
            h8, __builtin_amdgcn_raw_buffer_load_b128(rs, chunk_off(it, live, i), 0, kNonTemporal));
    }
  };
  // Item `item` from staging buffer SB: activation, residual inputs, store.
  auto store_item = [&](int item, bool live, int SB) {
    const int it = live ? item : begin;
    const __amdgpu_buffer_rsrc_t rs = item_rsrc(a.out, it);
#pragma unroll
    for (int i = 0; i < OCH; ++i) {
      h8 v = act8<ACT>(*reinterpret_cast<const h8*>(stg + SB * SBUF + oc_lds[i]));
      if (NSKIP > 0) v += skv[0][i];
      if (NSKIP > 1) v += skv[1][i];
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, v), rs,
                                             chunk_off(it, live, i), 0, kNonTemporal);
    }
  };

  if constexpr (IN_NCHW) {
    // NCHW boundary input through an LDS row ring: slot m % NSL holds image
    // rows 2 m - 1 and 2 m of the strip, 48 pixels from 32 s - 8 (16-byte
    // aligned; the patches use 32 s - 1 .. 32 s + 32). Each producer wave
    // copies the rows of its own 16 channels (the ones its lanes transform)
    // with three 16-byte buffer -> LDS loads per row pair (out-of-image
    // chunks read as zero), and reads only what it copied: no barrier orders
    // the ring, only the wave's own load count. Within a wave's region a
    // channel row (96 bytes) sits at position p = 2 j + 8 (c & 1) + (c >> 1)
    // for quad j, channel c of the quad, so that each dword read of the
    // transform (one row and channel, 16 tiles x 4 quads) hits 64 distinct
    // banks. Row pair m + 4 is requested while pairs m and m + 1 are read.
    constexpr int NSL = L::NSL_NCHW;
    constexpr int RP = 24;                // dwords per channel row
    constexpr int WREG = 2 * 16 * RP;     // dwords of one wave's region per slot
    constexpr int SLOT = 4 * WREG;        // dwords per slot
    constexpr int AHEAD = NSL - 2;        // row pairs requested ahead of the first read
    uint32_t* const ring = reinterpret_cast<uint32_t*>(stg + 2 * SBUF);
    const uint32_t plane = (uint32_t)a.H * (uint32_t)a.W * 2;
    const int pw = wave - NCW;  // uniform (ptid >> 6)
    const int l = ptid & 63;
    const int jq = (l >> 3) & 3;
    // The three copies of lane l: chunk q = 64 i + l of the wave's region,
    // row r = q / 96, position p = (q / 6) % 16, 16-byte chunk k = q % 6.
    int d_row[3], d_k[3];
    uint32_t d_ch[3], d_base[3];
    bool d_ok[3];
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      const int q = 64 * i + l;
      const int pp = (q / 6) % 16;
      const int c = ((pp & 1) << 1) | ((pp >> 3) & 1);
      const int j = (pp >> 1) & 3;
      d_row[i] = q / 96;
      d_k[i] = q % 6;
      d_ch[i] = (uint32_t)(16 * pw + 4 * j + c) * plane;
    }
    __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)a.in, (short)0, 0, 0x00020000);
    auto issue = [&](int pair) {
      const uint32_t dst = lds_byte_addr(ring + (pair % NSL) * SLOT + pw * WREG);
#pragma unroll
      for (int i = 0; i < 3; ++i) {
        const int y = 2 * pair - 1 + d_row[i];
        const bool ok = d_ok[i] && y >= 0 && y < a.H;
        dma16_buf(dst + 1024 * i, rs, ok ? d_base[i] + (uint32_t)y * (uint32_t)a.W * 2 : kOob);
      }
    };
    // Dword offsets of this lane's reads in a slot: row r, channel c of its quad.
    auto rd = [&](int r, int c) { return pw * WREG + (r * 16 + 2 * jq + 8 * (c & 1) + (c >> 1)) * RP + 3 + tt[0]; };
    for (int it = begin; it < end;) {
      decode(it, n, s, th);
      const int len = min(end - it, a.tiles_h - th);
      const char* ib = reinterpret_cast<const char*>(a.in) + (int64_t)n * C * plane;
      rs = __builtin_amdgcn_make_buffer_rsrc((void*)ib, (short)0, (int)(C * plane), 0x00020000);
#pragma unroll
      for (int i = 0; i < 3; ++i) {
        const int x = PXS * s - 8 + 8 * d_k[i];
        d_ok[i] = x >= 0 && x < a.W;
        d_base[i] = d_ch[i] + (uint32_t)x * 2;
      }
      for (int m = 0; m < AHEAD; ++m) issue(th + m);
      for (int k = 0; k < len; ++k) {
        issue(th + AHEAD);
        wait_vmcnt<3 * (AHEAD - 1)>();  // row pairs th and th + 1 have landed
        const uint32_t* sa = ring + (th % NSL) * SLOT;
        const uint32_t* sb = ring + ((th + 1) % NSL) * SLOT;
        h2 top[16], bot[16];
#pragma unroll
        for (int pr = 0; pr < 4; ++pr) {
          const uint32_t* sl = pr < 2 ? sa : sb;
          uint32_t x[4][3];
#pragma unroll
          for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int d = 0; d < 3; ++d) x[c][d] = sl[rd(pr & 1, c) + d];
          // Column j of the patch is pixel pair (j + 1) / 2, half (j + 1) % 2;
          // element 2 (4 r + j) + e holds channels 2 e and 2 e + 1.
          h2* row = (pr < 2 ? top : bot) + 8 * (pr & 1);
#pragma unroll
          for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int e = 0; e < 2; ++e) {
              const int d = (j + 1) >> 1;
              const uint32_t sel = ((j + 1) & 1) ? 0x07060302u : 0x05040100u;
              row[2 * j + e] =
                  __builtin_bit_cast(h2, __builtin_amdgcn_perm(x[2 * e + 1][d], x[2 * e][d], sel));
            }
        }
        v_transform<WPS>(vw0[0] + par * VBUF, top, bot);
        ++th;
        par ^= 1;
        lds_sync();
      }
      wait_vmcnt<0>();  // the copies requested past the run have landed
      it += len;
    }
    lds_sync();  // step K: the consumers fold item K-1
    lds_sync();  // step K + 1: they store it
    return;
  }

  auto step = [&](h2 (&top)[UP][16], h2 (&bot)[UP][16]) {
    if constexpr (PS) {
      store_item(begin + js - 2, js >= 2, par);  // item j-2 sits in buffer j & 1
      load_skips(begin + js - 1, js >= 1);       // item j-1, stored next step
    }
#pragma unroll
    for (int v = 0; v < UP; ++v) v_transform<WPS>(vw0[v] + par * VBUF, top[v], bot[v]);
    load2(top, in_row(2 * (th + NW)));
    ++th;
    ++js;
    par ^= 1;
    lds_sync();
  };

  h2 W[NW][UP][16];
  for (int it = begin; it < end;) {
    decode(it, n, s, th);
    const int len = min(end - it, a.tiles_h - th);
#pragma unroll
    for (int v = 0; v < UP; ++v) {
      // Tiles past the right edge read tile 0's patch (never stored).
      const int t = (L::TILES * s + tt[v] < a.tiles_w) ? tt[v] : 0;
      in_lane[v] = (uint32_t)(2 * t * C + (int)tq4[v]) * 2;
    }
#pragma unroll
    for (int m = 0; m < NW; ++m) load2(W[m], in_row(2 * (th + m)));
    // Whole cycles of the slots, then the remainder as nested conditions. A
    // loop with one exit keeps the compiler's count of outstanding loads exact
    // at the loop head (a break after every step would merge all the step
    // states there and force near-complete waits).
    int k = len;
    for (; k >= NW; k -= NW) {
#pragma unroll
      for (int m = 0; m < NW; ++m) step(W[m], W[(m + 1) % NW]);
    }
    auto rest = [&](auto self, auto m_tag) {
      constexpr int M = decltype(m_tag)::value;
      if constexpr (M < NW - 1) {
        if (k > M) {
          step(W[M], W[M + 1]);
          self(self, IntC<M + 1>{});
        }
      }
    };
    rest(rest, IntC<0>{});
    it += len;
  }
  if constexpr (PS) {
    // Step K: store item K-2, load item K-1's residuals; the consumers fold
    // item K-1. Step K + 1: store item K-1.
    store_item(begin + K - 2, K >= 2, par);
    load_skips(begin + K - 1, true);
    lds_sync();
    store_item(begin + K - 1, true, par ^ 1);
  } else {
    lds_sync();  // step K: the consumers fold item K-1
    lds_sync();  // step K + 1: they store it
  }
}


// One 16-byte-per-lane global -> LDS copy: lane l of the wave writes LDS bytes
// [m0 + 16 l, m0 + 16 l + 16) from gbase + voff. Inline assembly, so the
// compiler neither tracks it nor inserts waits for it; the kernels count it.
__device__ __forceinline__ void dma16(uint32_t m0, const char* gbase, uint32_t voff) {
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, %2"
      :
      : "s"(m0), "v"(voff), "s"(gbase)
      : "memory");
}


// ---------------------------------------------------------------------------
// Direct 3x3 conv on MFMA for narrow outputs (M <= 16), boundary layout
// ---------------------------------------------------------------------------
//
// The tail of the upscaler (64 -> 4 channels, then DepthToSpace) has too few
// outputs for the Winograd transform to pay: its cost is per input channel.
// Here each wave computes 16 output pixels x 16 channel slots with
// v_mfma_f32_16x16x32_f16, A = input pixels (one 3x3 tap, 32 channels: 16 B
// per lane straight from LDS), B = the taps (registers, 9 * KC fragments).
// A workgroup walks down a 64-pixel-wide segment; input rows (66 pixels with
// the halo) stream into an LDS ring by global_load_lds, D rows ahead. Each
// item's outputs go through a double-buffered fp32 tile in LDS and leave as
// DepthToSpace-ordered NCHW rows after the next barrier.
//
// Per item k (output row h0 + k; ring row j = padded input row h0 + j):
//   store item k-1 (from tile (k-1)&1)          4 element stores per thread
//   DMA ring row k + D + 2 -> slot (k+D+2) % R   NI instructions per wave
//   MFMA over ring rows k .. k+2, epilogue -> tile k&1
//   wait for ring row k + 3, barrier
// Ring row k + 3 was issued at item k + 1 - D, so (D - 1) * (NI + 4) of this
// wave's vector-memory instructions follow it; the prologue issues its rows in
// the same (4 stores, NI DMA) pattern so that the count holds from item 0.
template <int KC>
struct NarrowRing {
  static constexpr int C = 32 * KC;
  static constexpr int PXB = 2 * C;                // bytes per pixel
  static constexpr int ROWB = 66 * PXB;            // 64 pixels + 2 halo
  static constexpr int D = KC == 1 ? 6 : (KC == 2 ? 5 : 2);
  static constexpr int NSLOT = D + 3;
  static constexpr int CHUNKS = ROWB / 16;
  static constexpr int NI = (CHUNKS + 255) / 256;  // DMA instructions per wave per row
  static constexpr int G = 4 * KC;                 // 16-byte channel groups per pixel
  static constexpr int TILE = 16 * 64;             // fp32 output tile (16 channels x 64 px)
  static constexpr int WAIT = (D - 1) * (NI + 4);
  // Group g of pixel x sits at g ^ swz(x): the 16 lanes of an A read (16
  // consecutive pixels, one group) then cover all 64 banks.
  __host__ __device__ static constexpr int swz(int x) { return KC == 2 ? (x >> 1) & 7 : (x >> 2) & 3; }
  __host__ __device__ static constexpr int first_chunk(int q) { return q * CHUNKS / (4 * NI); }
  static constexpr size_t lds_bytes() { return (size_t)NSLOT * ROWB + 2 * TILE * 4; }
};

template <int KC, bool F32>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
conv3x3_narrow(NarrowArgs a) {
  using R = NarrowRing<KC>;
  extern __shared__ __attribute__((aligned(16))) float nlds[];  // tiles | ring
  float* const tile = nlds;
  char* const ring = reinterpret_cast<char*>(nlds + 2 * R::TILE);
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;

  const int G = gridDim.x;
  const int slot = (blockIdx.x & 7) * (G >> 3) + (blockIdx.x >> 3);
  const int begin = (int)((int64_t)a.n_items * slot / G);
  const int end = (int)((int64_t)a.n_items * (slot + 1) / G);
  if (begin >= end) return;  // uniform across the workgroup

  h8 wb[9][KC];
  {
    const h8* wp = reinterpret_cast<const h8*>(a.w) + lane;
#pragma unroll
    for (int t = 0; t < 9; ++t)
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) wb[t][kc] = wp[(t * KC + kc) * 64];
  }
  const int nch = lane & 15;  // output channel slot of this lane's D column
  const float bias = a.bias[nch];
  const int m = lane & 15, kq = lane >> 4;
  // A reads: pixel 16*wave + m + dx of a ring row, channel group 4*kc + kq.
  uint32_t aoff[3][KC];
#pragma unroll
  for (int dx = 0; dx < 3; ++dx)
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) {
      const int x = 16 * wave + m + dx;
      aoff[dx][kc] = (uint32_t)(x * R::PXB + (((4 * kc + kq) ^ R::swz(x)) << 4));
    }
  // Tile write: channel nch, pixels 16*wave + 4*kq .. +3.
  const int twr = nch * 64 + 16 * wave + 4 * kq;

  // Store phase: this thread's four output elements of an item (element
  // E = ((c*b + r)*64b + xq)) -> tile index and image offset (bytes, without
  // the item's row/segment part), or nothing past the M*64 elements.
  const int b = a.dts_b;
  const int64_t Wo = (int64_t)a.W * b;
  const int64_t Ho = (int64_t)a.H * b;
  constexpr int ELEM = F32 ? 4 : 2;
  int s_tile[4], s_x[4];
  uint32_t s_off[4];
  bool s_live[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int e = 4 * tid + i;
    s_live[i] = e < a.M * 64;
    const int seg = 64 * b;
    const int cr = e / seg;
    const int xq = e - cr * seg;
    const int c = cr / b, r = cr - (cr / b) * b;
    const int x = xq / b, q = xq - (xq / b) * b;
    const int k = (r * b + q) * a.cout + c;
    s_tile[i] = s_live[i] ? k * 64 + x : 0;
    s_x[i] = x;
    s_off[i] = s_live[i] ? (uint32_t)(((int64_t)c * Ho + r) * Wo + xq) * ELEM : 0u;
  }
  constexpr uint32_t kOob = 0x80000000u;

  int n = 0, sg = 0, h0 = 0;
  auto decode = [&](int item) {
    const uint32_t t = fdiv((uint32_t)item, a.fd_H);
    h0 = item - (int)(t * (uint32_t)a.H);
    const uint32_t nn = fdiv(t, a.fd_seg);
    sg = (int)(t - nn * (uint32_t)a.n_seg);
    n = (int)nn;
  };
  // DMA lane offsets for this segment (relative to a ring row's first pixel).
  uint32_t doff[R::NI];
  int dcnt[R::NI];
  auto setup_dma = [&]() {
    const int xmax = a.Wp - 1 - 64 * sg;
#pragma unroll
    for (int j = 0; j < R::NI; ++j) {
      const int q = R::NI * wave + j;
      const int c0 = R::first_chunk(q);
      dcnt[j] = R::first_chunk(q + 1) - c0;
      int c = c0 + lane;
      if (c >= R::CHUNKS) c = R::CHUNKS - 1;
      const int x = c / R::G;
      const int gp = c - x * R::G;
      const int g = gp ^ R::swz(x);
      doff[j] = (uint32_t)((x > xmax ? xmax : x) * R::PXB + g * 16);
    }
  };
  // Ring row j of the run (padded input row h0 + j, clamped) -> slot j % NSLOT.
  auto dma_row = [&](int j) {
    int pr = h0 + j;
    if (pr > a.Hp - 1) pr = a.Hp - 1;
    const char* gb = reinterpret_cast<const char*>(a.in) +
                     (((int64_t)n * a.Hp + pr) * a.Wp + 64 * sg) * R::PXB;
    const uint32_t sb = lds_byte_addr(ring) + (uint32_t)((j % R::NSLOT) * R::ROWB);
#pragma unroll
    for (int q = 0; q < R::NI; ++q) {
      const uint32_t m0 = sb + (uint32_t)R::first_chunk(R::NI * wave + q) * 16;
      if (lane < dcnt[q]) dma16(m0, gb, doff[q]);
    }
  };
  // Four element stores of the item (pn, ps, ph) from tile buffer tb; every
  // thread issues exactly four (out-of-range offsets when absent).
  int pn = 0, ps = 0, ph = 0;
  auto store_item = [&](int tb, bool live) {
    char* ob = reinterpret_cast<char*>(a.out) + (int64_t)pn * a.img_bytes;
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void*)ob, (short)0, (int)a.img_bytes, 0x00020000);
    const uint32_t item_off = (uint32_t)(((int64_t)ph * b * Wo + (int64_t)64 * ps * b) * ELEM);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float v = tile[tb * R::TILE + s_tile[i]];
      const bool ok = live && s_live[i] && (64 * ps + s_x[i] < a.W);
      const uint32_t off = ok ? item_off + s_off[i] : kOob;
      if (F32) {
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), rs, off, 0, 0);
      } else {
        const _Float16 hv = (_Float16)v;
        __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, hv), rs, off, 0, 0);
      }
    }
  };

  int last_tb = 0;
  bool have_prev = false;
  for (int it = begin; it < end;) {
    decode(it);
    const int len = min(end - it, a.H - h0);
    // Retire the previous run (stray ring rows included), store its last item.
    wait_vmcnt<0>();
    lds_sync();
    store_item(last_tb, have_prev);
    have_prev = false;
    setup_dma();
#pragma unroll 1
    for (int j = 0; j < R::D + 2; ++j) {
      store_item(0, false);  // keeps the per-row instruction pattern of the loop
      dma_row(j);
    }
    wait_vmcnt<R::WAIT>();  // ring rows 0..2
    lds_sync();
#pragma unroll 1
    for (int k = 0; k < len; ++k) {
      store_item((k + 1) & 1, have_prev);
      dma_row(k + R::D + 2);
      f4 acc = {0, 0, 0, 0};
#pragma unroll
      for (int dy = 0; dy < 3; ++dy) {
        const char* rowp = ring + ((k + dy) % R::NSLOT) * R::ROWB;
#pragma unroll
        for (int dx = 0; dx < 3; ++dx)
#pragma unroll
          for (int kc = 0; kc < KC; ++kc)
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                *reinterpret_cast<const h8*>(rowp + aoff[dx][kc]), wb[dy * 3 + dx][kc], acc, 0,
                0, 0);
      }
      f4 y;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        float t = apply_act(acc[v] + bias, a.act);
        if (a.do_clip) t = apply_clip(t, a.clip_lo, a.clip_hi);
        y[v] = t;
      }
      *reinterpret_cast<f4*>(tile + (k & 1) * R::TILE + twr) = y;
      pn = n;
      ps = sg;
      ph = h0 + k;
      have_prev = true;
      last_tb = k & 1;
      wait_vmcnt<R::WAIT>();  // ring row k + 3
      lds_sync();
    }
    it += len;
  }
  wait_vmcnt<0>();
  lds_sync();
  store_item(last_tb, have_prev);
}

// Tail conv with the three taps of a kernel row packed into one MFMA (M <= 5).
// B columns are (dx, n) -> dx*M + n, so per kernel row dy and 32-channel chunk
// one MFMA gives D[x][(dx, n)] = sum_c in[dy][x][c] * w[n][c][dy][dx] for the
// wave's 16 pixels x; dy and the chunks accumulate in the MFMA, so a wave
// issues 3 * KC MFMAs per item instead of 9 * KC. The conv output is
// out[x][n] = D[x][(0,n)] + D[x+1][(1,n)] + D[x+2][(2,n)] (+ bias), summed in
// the store phase from an fp32 tile [16 columns][128 pixels] in LDS.
//
// A workgroup walks down a segment of TAIL_SEG = 126 output pixels (one output
// row per item): its eight waves cover the segment's 128 padded input columns,
// halo included (four waves and 62-pixel segments: 65.3 us at 1080p against
// 63.4; sixteen waves: no better). The A fragments (16 pixels x 32 channels, 16 bytes per lane)
// come straight from HBM into a register window of TAIL_ROWS input rows: each
// item consumes three and loads one TAIL_ROWS - 3 rows ahead. (Through an LDS
// ring filled by global_load_lds the same conv ran at 95 us at 1080p, held
// back by the DMA issue and LDS bank conflicts.)
constexpr int TAIL_ROWS = 6;
constexpr int TAIL_WAVES = 8;                  // 16 input columns each
constexpr int TAIL_SEG = 16 * TAIL_WAVES - 2;  // output pixels per segment
// Floats per D tile row: the segment's input columns padded by 8 (two bank
// quads), so that the 16 lanes a ds_write_b128 serves per cycle (columns
// t..t+7 and two adjacent 4-pixel groups) land on 16 distinct quads. Rows of
// 64 floats put every column on the same quads: 8-way conflicts on each write.
constexpr int TAIL_TW = 16 * TAIL_WAVES + 8;

// Four waves per SIMD for C <= 64 (two for C = 96, whose row window needs
// more than 128 VGPRs): at 1080p 64 -> 4 + DepthToSpace, 81 us with two, 70 us
// with four (measured with four-wave workgroups).
template <int KC, bool F32>
__global__ void __launch_bounds__(64 * TAIL_WAVES)
    __attribute__((amdgpu_waves_per_eu(KC == 3 ? 2 : 4, KC == 3 ? 2 : 4)))
conv3x3_tail(NarrowArgs a) {
  constexpr int C = 32 * KC;
  constexpr int PXB = 2 * C;     // bytes per pixel
  constexpr int NR = TAIL_ROWS;  // row slots
  constexpr int SEG = TAIL_SEG;
  constexpr int TW = TAIL_TW;    // tile row: the segment's 64 input columns, padded
  constexpr int TILE = 16 * TW;  // floats per tile buffer
  extern __shared__ __attribute__((aligned(16))) float nlds[];
  float* const tile = nlds;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;

  const int G = gridDim.x;
  const int slot = (blockIdx.x & 7) * (G >> 3) + (blockIdx.x >> 3);
  const int begin = (int)((int64_t)a.n_items * slot / G);
  const int end = (int)((int64_t)a.n_items * (slot + 1) / G);
  if (begin >= end) return;  // uniform across the workgroup

  h8 wb[3][KC];
  {
    const h8* wp = reinterpret_cast<const h8*>(a.w) + lane;
#pragma unroll
    for (int dy = 0; dy < 3; ++dy)
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) wb[dy][kc] = wp[(dy * KC + kc) * 64];
  }
  const int m = lane & 15, kq = lane >> 4;
  // D tile write: column lane & 15, pixels 16*wave + 4*kq .. +3.
  const int twr = (lane & 15) * TW + 16 * wave + 4 * kq;

  // Store phase: element E = ((c*b + r)*SEG*b + xq) of the item -> conv output
  // channel k, pixel x; tile index of D[x][(0,k)], the bias, image offset.
  const int b = a.dts_b;
  const int64_t Wo = (int64_t)a.W * b;
  const int64_t Ho = (int64_t)a.H * b;
  constexpr int ELEM = F32 ? 4 : 2;
  const int dxs = a.M * TW + 1;  // tile step from D[x][(dx,k)] to D[x+1][(dx+1,k)]
  int s_tile[4], s_x[4];
  float s_bias[4];
  uint32_t s_off[4];
  bool s_live[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int e = 4 * tid + i;
    s_live[i] = e < a.M * SEG;
    const int seg = SEG * b;
    const int cr = e / seg;
    const int xq = e - cr * seg;
    const int c = cr / b, r = cr - (cr / b) * b;
    const int x = xq / b, q = xq - (xq / b) * b;
    const int k = (r * b + q) * a.cout + c;
    s_tile[i] = s_live[i] ? k * TW + x : 0;
    s_bias[i] = s_live[i] ? a.bias[k] : 0.0f;
    s_x[i] = x;
    s_off[i] = s_live[i] ? (uint32_t)(((int64_t)c * Ho + r) * Wo + xq) * ELEM : 0u;
  }
  constexpr uint32_t kOob = 0x80000000u;

  int n = 0, sg = 0, h0 = 0;
  auto decode = [&](int item) {
    const uint32_t t = fdiv((uint32_t)item, a.fd_H);
    h0 = item - (int)(t * (uint32_t)a.H);
    const uint32_t nn = fdiv(t, a.fd_seg);
    sg = (int)(t - nn * (uint32_t)a.n_seg);
    n = (int)nn;
  };
  // A fragment loads through a buffer resource over image n; the lane's pixel
  // is clamped to the last padded column (such pixels feed no stored output).
  __amdgpu_buffer_rsrc_t irs;
  uint32_t aoff = 0;
  const uint32_t prow = (uint32_t)(a.Wp * PXB);
  auto setup_run = [&]() {
    const char* base = reinterpret_cast<const char*>(a.in) + (int64_t)n * a.Hp * a.Wp * PXB;
    irs = __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, (int)(a.Hp * prow), 0x00020000);
    int x = SEG * sg + 16 * wave + m;
    if (x > a.Wp - 1) x = a.Wp - 1;
    aoff = (uint32_t)(x * PXB + 16 * kq);
  };
  struct Row {
    h8 v[KC];
  };
  // Window row j of the current run: padded row h0 + j walking down, or
  // h0 + len + 1 - j walking up. Rows past the run's len + 2 are not fetched
  // (out-of-range offset: the load returns zeros and reads no memory).
  int len = 0;
  auto load_row = [&](Row& R, int j, auto rev_tag) {
    constexpr bool REV = decltype(rev_tag)::value;
    int pr = REV ? h0 + len + 1 - j : h0 + j;
    if (pr > a.Hp - 1) pr = a.Hp - 1;
    const uint32_t o = j < len + 2 ? (uint32_t)pr * prow + aoff : kOob;
#pragma unroll
    for (int kc = 0; kc < KC; ++kc)
      R.v[kc] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(irs, o + 64 * kc, 0, 0));
  };
  // A thread's four elements are consecutive output pixels of one output row
  // when SEG * b is a multiple of 4 (b even); with Wo % 4 == 0 and an aligned
  // output they go out as one 4-element store, except where the segment
  // crosses the image's right edge.
  const bool pack4 = (b & 1) == 0 && (Wo & 3) == 0 &&
                     (reinterpret_cast<uintptr_t>(a.out) & (4 * ELEM - 1)) == 0;
  int pn = 0, ps = 0, ph = 0;
  auto store_item = [&](int tb, bool live) {
    char* ob = reinterpret_cast<char*>(a.out) + (int64_t)pn * a.img_bytes;
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void*)ob, (short)0, (int)a.img_bytes, 0x00020000);
    const uint32_t item_off = (uint32_t)(((int64_t)ph * b * Wo + (int64_t)SEG * ps * b) * ELEM);
    const float* tp = tile + tb * TILE;
    float v[4];
    bool ok[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float t = (tp[s_tile[i]] + tp[s_tile[i] + dxs]) + tp[s_tile[i] + 2 * dxs];
      t = apply_act(t + s_bias[i], a.act);
      if (a.do_clip) t = apply_clip(t, a.clip_lo, a.clip_hi);
      v[i] = t;
      ok[i] = live && s_live[i] && (SEG * ps + s_x[i] < a.W);
    }
    // ok[] only falls along i (element index and pixel both rise), so ok[3]
    // means all four.
    if (pack4 && ok[3]) {
      if (F32) {
        const u4 q = {__builtin_bit_cast(uint32_t, v[0]), __builtin_bit_cast(uint32_t, v[1]),
                      __builtin_bit_cast(uint32_t, v[2]), __builtin_bit_cast(uint32_t, v[3])};
        __builtin_amdgcn_raw_buffer_store_b128(q, rs, item_off + s_off[0], 0, 0);
      } else {
        const h4 hv = {(_Float16)v[0], (_Float16)v[1], (_Float16)v[2], (_Float16)v[3]};
        __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u2, hv), rs, item_off + s_off[0],
                                              0, 0);
      }
      return;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t off = ok[i] ? item_off + s_off[i] : kOob;
      if (F32) {
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v[i]), rs, off, 0, 0);
      } else {
        const _Float16 hv = (_Float16)v[i];
        __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, hv), rs, off, 0, 0);
      }
    }
  };

  // Item k of a run uses window rows k, k+1, k+2 (slots k % NR, ...), then
  // loads row k + NR into the slot of row k; one barrier per item (the tile
  // is double-buffered). Walking up, window row k is the conv's bottom tap
  // row, so the slots enter the MFMAs in the opposite order; the MFMA order,
  // and so every result bit, is the same both ways.
  int par = 0;  // tile buffer of the current item
  bool have_prev = false;
  auto item = [&](const Row& r0, const Row& r1, const Row& r2, Row& reload, int k, auto rev_tag) {
    constexpr bool REV = decltype(rev_tag)::value;
    store_item(par ^ 1, have_prev);
    f4 acc = {0, 0, 0, 0};
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) {
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(r0.v[kc], wb[0][kc], acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(r1.v[kc], wb[1][kc], acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(r2.v[kc], wb[2][kc], acc, 0, 0, 0);
    }
    load_row(reload, k + NR, rev_tag);
    *reinterpret_cast<f4*>(tile + par * TILE + twr) = acc;
    pn = n;
    ps = sg;
    ph = REV ? h0 + len - 1 - k : h0 + k;
    have_prev = true;
    par ^= 1;
    lds_sync();
  };

  Row W[NR];
  auto run = [&](auto rev_tag) {
    constexpr bool REV = decltype(rev_tag)::value;
#pragma unroll
    for (int j = 0; j < NR; ++j) load_row(W[j], j, rev_tag);
    auto step = [&](auto j_tag, int k) {
      constexpr int J = decltype(j_tag)::value;
      if constexpr (REV)
        item(W[(J + 2) % NR], W[(J + 1) % NR], W[J], W[J], k, rev_tag);
      else
        item(W[J], W[(J + 1) % NR], W[(J + 2) % NR], W[J], k, rev_tag);
    };
    // Whole cycles of the slots, then the remainder as nested conditions (one
    // loop exit keeps the compiler's count of outstanding loads exact).
    int k = 0;
    for (; k + NR <= len; k += NR) {
      static_for<NR>([&](auto j_tag) { step(j_tag, k + decltype(j_tag)::value); });
    }
    auto rest = [&](auto self, auto j_tag) {
      constexpr int J = decltype(j_tag)::value;
      if constexpr (J < NR) {
        if (k + J < len) {
          step(j_tag, k + J);
          self(self, IntC<J + 1>{});
        }
      }
    };
    rest(rest, IntC<0>{});
  };

  // Odd slots walk their item range backwards (rows upward, runs in reverse),
  // so that the two rows a run boundary shares are read by both neighbouring
  // workgroups (same XCD) near the same time, at both ends of the launch, and
  // the second read hits L2.
  const bool rev = (slot & 1) != 0;
  if (!rev) {
    for (int it = begin; it < end; it += len) {
      decode(it);
      len = min(end - it, a.H - h0);
      setup_run();
      run(IntC<0>{});
    }
  } else {
    for (int it = end; it > begin; it -= len) {
      decode(it - 1);
      len = min(it - begin, h0 + 1);
      h0 = h0 - len + 1;
      setup_run();
      run(IntC<1>{});
    }
  }
  store_item(par ^ 1, have_prev);
}

// ---------------------------------------------------------------------------
// Direct 3x3 conv with one input channel (head conv)
// ---------------------------------------------------------------------------

// Each thread owns 8 output channels (g = thread % g8) for the whole launch and
// keeps their 9 taps (as 5 half2 pairs, the 10th tap zero) in VGPRs; the 9 input
// pixels are multiplied with v_dot2_f32_f16 (fp16 products, fp32 sums).
template <bool FAST>
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
  f4 b0 = {0, 0, 0, 0}, b1 = b0;
  if (FAST) {
    b0 = *reinterpret_cast<const f4*>(a.epi.bias + ch0);
    b1 = *reinterpret_cast<const f4*>(a.epi.bias + ch0 + 4);
  }
  const _Float16* in = reinterpret_cast<const _Float16*>(a.in);
  const int64_t npix = (int64_t)a.N * a.H * a.W;
  const int64_t step = (int64_t)gridDim.x * ppb;
  for (int64_t p = (int64_t)blockIdx.x * ppb + pl; p < npix; p += step) {
    const int ow = (int)(p % a.W);
    const int64_t rest = p / a.W;
    const int oh = (int)(rest % a.H);
    const int n = (int)(rest / a.H);
    // Window rows oh..oh+2, columns ow..ow+2 in padded coordinates.
    const _Float16* src = in + ((int64_t)n * a.Hp + oh) * a.Wp + ow;
    _Float16 x[10];
#pragma unroll
    for (int r = 0; r < 3; ++r)
#pragma unroll
      for (int s = 0; s < 3; ++s) x[r * 3 + s] = src[(int64_t)r * a.Wp + s];
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
    if (FAST) {
      const int64_t o = (((int64_t)n * a.Hp + oh + 1) * a.Wp + ow + 1) * a.M + ch0;
      h4 s00 = {0, 0, 0, 0}, s01 = s00, s10 = s00, s11 = s00;
      if (a.epi.skip0) {
        const _Float16* sp = reinterpret_cast<const _Float16*>(a.epi.skip0) + o;
        s00 = *reinterpret_cast<const h4*>(sp);
        s01 = *reinterpret_cast<const h4*>(sp + 4);
      }
      if (a.epi.skip1) {
        const _Float16* sp = reinterpret_cast<const _Float16*>(a.epi.skip1) + o;
        s10 = *reinterpret_cast<const h4*>(sp);
        s11 = *reinterpret_cast<const h4*>(sp + 4);
      }
      h4 r0, r1;
      if (a.epi.act == kActRelu) {
        r0 = fast4<kActRelu>(acc0, b0, s00, s10);
        r1 = fast4<kActRelu>(acc1, b1, s01, s11);
      } else if (a.epi.act == kActSilu) {
        r0 = fast4<kActSilu>(acc0, b0, s00, s10);
        r1 = fast4<kActSilu>(acc1, b1, s01, s11);
      } else {
        r0 = fast4<kActNone>(acc0, b0, s00, s10);
        r1 = fast4<kActNone>(acc1, b1, s01, s11);
      }
      h8 r = {r0[0], r0[1], r0[2], r0[3], r1[0], r1[1], r1[2], r1[3]};
      *reinterpret_cast<h8*>(reinterpret_cast<_Float16*>(a.epi.out) + o) = r;
    } else {
      store4(a.epi, a.M, a.H, a.W, a.Hp, a.Wp, n, oh, ow, ch0, acc0);
      if (ch0 + 4 < a.M) store4(a.epi, a.M, a.H, a.W, a.Hp, a.Wp, n, oh, ow, ch0 + 4, acc1);
    }
  }
}

// Column-walking variant for the fast epilogue (padded NHWC output, M % 8 ==
// 0): a work item is one output row x SEG pixels, SEG = 4 * 256 / G8, and a
// workgroup's item range walks down a column of segments. Thread t computes
// pixels 4q .. 4q+3 (q = t / G8) for channels 8g .. 8g+7 (g = t % G8). Its 3 x 6
// input window comes straight from HBM: a register ring of HEAD_ROWS padded
// input rows (six halfs each, three 4-byte buffer loads), one row loaded per
// item HEAD_ROWS - 3 rows ahead, so there is no LDS and no barrier. Columns
// past a row's end read the next row (or zero past the image) and feed only
// pixels beyond the right edge, whose stores the output buffer resource drops.
// (With the window staged through LDS per item, 8 items per workgroup: 75-81 us
// at 1080p 1 -> 64.) BIN 1 / 2: the input is the engine's NCHW boundary tensor
// (fp16 / fp32, converted with round-to-nearest-even) instead of the padded
// copy; the window is then read element by element, zero outside the image.
constexpr int HEAD_ROWS = 6;

template <int G8, int ACT, bool SKIP, int BIN>
__global__ void __launch_bounds__(256) direct_conv_c1_walk(DirectArgs a, int n_seg, int n_items,
                                                           FastDiv fd_seg, FastDiv fd_H) {
  constexpr int SEG = 4 * 256 / G8;
  constexpr int NR = HEAD_ROWS;
  const int tid = threadIdx.x;
  const int g = tid % G8;
  const int q = tid / G8;
  const int ch0 = 8 * g;
  const bool live = ch0 < a.M;
  h2 wr[8][5];
  {
    const h2* wp = reinterpret_cast<const h2*>(a.w) + (size_t)g * 40;
#pragma unroll
    for (int c = 0; c < 8; ++c)
#pragma unroll
      for (int k = 0; k < 5; ++k) wr[c][k] = live ? wp[c * 5 + k] : h2{0, 0};
  }
  f4 b0 = {0, 0, 0, 0}, b1 = b0;
  if (live) {
    b0 = *reinterpret_cast<const f4*>(a.epi.bias + ch0);
    b1 = *reinterpret_cast<const f4*>(a.epi.bias + ch0 + 4);
  }

  const int G = gridDim.x;
  const int slot = (blockIdx.x & 7) * (G >> 3) + (blockIdx.x >> 3);
  const int begin = (int)((int64_t)n_items * slot / G);
  const int end = (int)((int64_t)n_items * (slot + 1) / G);
  if (begin >= end) return;

  // Item = (n * n_seg + segment) * H + output row.
  int n = 0, sgm = 0, h0 = 0;
  auto decode = [&](int item) {
    const uint32_t t = fdiv((uint32_t)item, fd_H);
    h0 = item - (int)(t * (uint32_t)a.H);
    const uint32_t nn = fdiv(t, fd_seg);
    sgm = (int)(t - nn * (uint32_t)n_seg);
    n = (int)nn;
  };
  __amdgpu_buffer_rsrc_t irs;
  uint32_t col_off = 0;
  constexpr int EB = BIN == 2 ? 4 : 2;  // bytes per input element
  const uint32_t prow = (uint32_t)(BIN ? a.W : a.Wp) * EB;
  auto setup_run = [&]() {
    const int64_t img = BIN ? (int64_t)a.H * a.W : (int64_t)a.Hp * a.Wp;
    const char* base = reinterpret_cast<const char*>(a.in) + (int64_t)n * img * EB;
    irs = __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, (int)(img * EB), 0x00020000);
    col_off = (uint32_t)(sgm * SEG + 4 * q) * EB;
  };
  struct Row {
    h2 v[3];  // padded columns x .. x+5 of one input row
  };
  auto load_row = [&](Row& R, int pr) {
    if (pr > a.Hp - 1) pr = a.Hp - 1;
    if (BIN == 0) {
      const uint32_t o = (uint32_t)pr * prow + col_off;
#pragma unroll
      for (int i = 0; i < 3; ++i)
        R.v[i] = __builtin_bit_cast(h2, __builtin_amdgcn_raw_buffer_load_b32(irs, o + 4 * i, 0, 0));
    } else {
      // Padded column x + i is image column x + i - 1 of image row pr - 1.
      const int hr = pr - 1;
      const int c0 = sgm * SEG + 4 * q - 1;
      const bool row_ok = hr >= 0 && hr < a.H;
      _Float16 e[6];
#pragma unroll
      for (int i = 0; i < 6; ++i) {
        const int c = c0 + i;
        const uint32_t o =
            row_ok && c >= 0 && c < a.W ? ((uint32_t)hr * (uint32_t)a.W + (uint32_t)c) * EB : 0x80000000u;
        if (BIN == 1)
          e[i] = __builtin_bit_cast(_Float16, __builtin_amdgcn_raw_buffer_load_b16(irs, o, 0, 0));
        else
          e[i] = (_Float16)__builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(irs, o, 0, 0));
      }
#pragma unroll
      for (int i = 0; i < 3; ++i) R.v[i] = h2{e[2 * i], e[2 * i + 1]};
    }
  };
  auto item = [&](Row& r0, const Row& r1, const Row& r2, int k) {
    const int h = h0 + k;
    _Float16 x[3][6];
    const Row* rr[3] = {&r0, &r1, &r2};
#pragma unroll
    for (int r = 0; r < 3; ++r)
#pragma unroll
      for (int i = 0; i < 3; ++i) {
        x[r][2 * i] = rr[r]->v[i][0];
        x[r][2 * i + 1] = rr[r]->v[i][1];
      }
    const int x0 = sgm * SEG;
    char* ob = reinterpret_cast<char*>(a.epi.out) +
               (((int64_t)n * a.Hp + h + 1) * a.Wp + x0 + 1) * a.M * 2;
    const int valid = min(SEG, a.W - x0);
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void*)ob, (short)0, valid * a.M * 2, 0x00020000);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const h2 xv[5] = {h2{x[0][j], x[0][j + 1]}, h2{x[0][j + 2], x[1][j]},
                        h2{x[1][j + 1], x[1][j + 2]}, h2{x[2][j], x[2][j + 1]},
                        h2{x[2][j + 2], (_Float16)0.0f}};
      f4 acc0, acc1;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
        for (int kk = 0; kk < 5; ++kk) {
          s0 = __builtin_amdgcn_fdot2(xv[kk], wr[c][kk], s0, false);
          s1 = __builtin_amdgcn_fdot2(xv[kk], wr[c + 4][kk], s1, false);
        }
        acc0[c] = s0;
        acc1[c] = s1;
      }
      const uint32_t off = (uint32_t)((4 * q + j) * a.M + ch0) * 2;
      h4 s00 = {0, 0, 0, 0}, s01 = s00, s10 = s00, s11 = s00;
      if (SKIP) {
        const int64_t pix = ((int64_t)n * a.Hp + h + 1) * a.Wp + x0 + 1 + 4 * q + j;
        if (live && x0 + 4 * q + j < a.W) {
          if (a.epi.skip0) {
            const _Float16* sp = reinterpret_cast<const _Float16*>(a.epi.skip0) + pix * a.M + ch0;
            s00 = *reinterpret_cast<const h4*>(sp);
            s01 = *reinterpret_cast<const h4*>(sp + 4);
          }
          if (a.epi.skip1) {
            const _Float16* sp = reinterpret_cast<const _Float16*>(a.epi.skip1) + pix * a.M + ch0;
            s10 = *reinterpret_cast<const h4*>(sp);
            s11 = *reinterpret_cast<const h4*>(sp + 4);
          }
        }
      }
      const h4 v0 = fast4<ACT>(acc0, b0, s00, s10);
      const h4 v1 = fast4<ACT>(acc1, b1, s01, s11);
      const h8 rv = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, rv), rs,
                                             live ? off : 0x80000000u, 0, kNonTemporal);
    }
    load_row(r0, h + NR);
  };

  Row W[NR];
  for (int it = begin; it < end;) {
    decode(it);
    const int len = min(end - it, a.H - h0);
    setup_run();
#pragma unroll
    for (int j = 0; j < NR; ++j) load_row(W[j], h0 + j);
    // Whole cycles of the slots, then the remainder as nested conditions (one
    // loop exit keeps the compiler's count of outstanding loads exact).
    int k = 0;
    for (; k + NR <= len; k += NR) {
#pragma unroll
      for (int j = 0; j < NR; ++j) item(W[j], W[(j + 1) % NR], W[(j + 2) % NR], k + j);
    }
    auto rest = [&](auto self, auto j_tag) {
      constexpr int J = decltype(j_tag)::value;
      if constexpr (J < NR) {
        if (k + J < len) {
          item(W[J], W[(J + 1) % NR], W[(J + 2) % NR], k + J);
          self(self, IntC<J + 1>{});
        }
      }
    };
    rest(rest, IntC<0>{});
    it += len;
  }
}

// Head conv on MFMA (C = 1, M = 16 * NB with NB even, fast epilogue, no
// residual inputs). One v_mfma_f32_16x16x16_f16 per 16 pixels and 16 output
// channels: B holds the 16 pixels' 3 x 3 windows as K = 16 slots (kernel row
// q in slots 4q .. 4q+2, slot 4q+3 and row 3 zero), so lane (q, j) supplies
// three input values of pixel j; A holds the taps of 16 output channels in the
// same slots. The channels of block b are permuted (row i = channel
// (i / 4) * 4 NB + 4 b + i % 4) so that lane (q, j) ends with the contiguous
// channels q * 4 NB .. q * 4 NB + 4 NB - 1 of pixel j. Stored from there, each
// 16-byte store instruction would cover half of every pixel line, and such
// partial lines with the nontemporal hint cost 154 us instead of 64 at 1080p
// 1 -> 64. So each wave stages its block (16 pixels, one contiguous stretch of
// the output row) in its own LDS region and stores it linearly, lane l of
// instruction s taking 16-byte chunk 64 s + (l ^ 8 for lanes 16-31 and 48-63):
// whole lines per instruction. LDS operations of one wave complete in order,
// so the region needs no barrier. Chunk g sits at g ^ ((g >> 3) & 7): the
// reads are bank-conflict free, the MFMA-layout writes at most 2-way. The
// stores are plain, not nontemporal: the next two layers read this output
// first (1 -> 64 at 1080p: 63 -> 57 us, and the first residual layer gains).
// An item is one output row x 64 pixels (16 per wave); every lane issues the
// same loads and stores on every path (out-of-range offsets read zero and drop
// stores), and the next item's loads go out before this item's MFMAs. The
// products are exact in fp32 and summed in the matrix unit; the epilogue is
// fast4, as in the other head kernels.
template <int NB, int ACT, int BIN>
__global__ void __launch_bounds__(256) direct_conv_c1_mfma(DirectArgs a, int n_seg, int n_items,
                                                           FastDiv fd_seg, FastDiv fd_H) {
  static_assert(NB % 2 == 0 && NB <= 6, "16 * NB output channels, NB even");
  constexpr int M = 16 * NB;
  constexpr int SEG = 64;
  constexpr int CH = 2 * NB;    // 16-byte chunks per pixel
  constexpr int WCH = 16 * CH;  // chunks of a wave's 16-pixel block
  extern __shared__ __attribute__((aligned(16))) h8 hstage[];
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int j = lane & 15;  // pixel of the wave's 16 (B column, D column)
  const int q = lane >> 4;  // kernel row (B / A slots 4q..4q+3), channel quarter of D
  constexpr uint32_t kOob = 0x80000000u;
  h8* const wl = hstage + wave * WCH;
  auto swz = [](int g) { return g ^ ((g >> 3) & 7); };
  const int rl = lane ^ (((lane >> 4) & 1) << 3);  // chunk of the lane in a store

  h4 wa[NB];
  f4 bias4[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const int ch = (j >> 2) * 4 * NB + 4 * b + (j & 3);  // A row j of block b
    const _Float16* wp = reinterpret_cast<const _Float16*>(a.w) + ch * 10 + 3 * (q < 3 ? q : 0);
    wa[b] = q < 3 ? h4{wp[0], wp[1], wp[2], (_Float16)0.0f} : h4{0, 0, 0, 0};
    bias4[b] = *reinterpret_cast<const f4*>(a.epi.bias + q * 4 * NB + 4 * b);
  }

  const int G = gridDim.x;
  const int slot = (blockIdx.x & 7) * (G >> 3) + (blockIdx.x >> 3);
  const int begin = (int)((int64_t)n_items * slot / G);
  const int end = (int)((int64_t)n_items * (slot + 1) / G);
  if (begin >= end) return;

  // Item = (n * n_seg + segment) * H + output row.
  auto decode = [&](int item, int& n, int& sg, int& y) {
    const uint32_t t = fdiv((uint32_t)item, fd_H);
    y = item - (int)(t * (uint32_t)a.H);
    const uint32_t nn = fdiv(t, fd_seg);
    sg = (int)(t - nn * (uint32_t)n_seg);
    n = (int)nn;
  };
  constexpr int EB = BIN == 2 ? 4 : 2;  // bytes per input element
  // B operand of `item`: input (row y - 1 + q, columns x - 1 .. x + 1) of
  // pixel x, zero outside the image (padded input: the zero border).
  auto load_b = [&](int item, _Float16 (&v)[3]) {
    int n, sg, y;
    decode(item, n, sg, y);
    const int x = SEG * sg + 16 * wave + j;
    const int64_t img = BIN ? (int64_t)a.H * a.W : (int64_t)a.Hp * a.Wp;
    const char* base = reinterpret_cast<const char*>(a.in) + (int64_t)n * img * EB;
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, (int)(img * EB), 0x00020000);
#pragma unroll
    for (int dx = 0; dx < 3; ++dx) {
      uint32_t o;
      if (BIN == 0) {
        // Padded row y + q, column x + dx (x + dx past the row end reads the
        // next row: such pixels are never stored).
        o = q < 3 ? (uint32_t)((y + q) * a.Wp + x + dx) * EB : kOob;
      } else {
        const int hr = y - 1 + q, c = x - 1 + dx;
        o = q < 3 && hr >= 0 && hr < a.H && c >= 0 && c < a.W ? (uint32_t)(hr * a.W + c) * EB : kOob;
      }
      if (BIN == 2)
        v[dx] = (_Float16)__builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, o, 0, 0));
      else
        v[dx] = __builtin_bit_cast(_Float16, __builtin_amdgcn_raw_buffer_load_b16(rs, o, 0, 0));
    }
  };

  // Items go in batches of kBatch: the batch's input loads all go out first
  // (indices clamped to the workgroup's last item, so every load is inside
  // the input), then the items run in order, each waiting only for its own
  // loads while later items' loads and earlier items' stores stay in flight.
  // With one item's loads prefetched per iteration instead, the compiler
  // packed the prefetched values right after requesting them and so waited
  // there, and that wait (vmcnt also counts stores) drained the item's stores
  // as well: one full load latency per item.
  constexpr int kBatch = 4;
  auto item = [&](int it, const _Float16 (&cur)[3]) {
    int n, sg, y;
    decode(it, n, sg, y);
    const int x0 = SEG * sg;
    const h4 bv = {cur[0], cur[1], cur[2], (_Float16)0.0f};
    char* ob = reinterpret_cast<char*>(a.epi.out) + (((int64_t)n * a.Hp + y + 1) * a.Wp + x0 + 1) * M * 2;
    const int valid = min(SEG, a.W - x0);
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void*)ob, (short)0, valid * M * 2, 0x00020000);
#pragma unroll
    for (int m = 0; m < NB / 2; ++m) {
      const f4 z = {0, 0, 0, 0};
      const f4 d0 = __builtin_amdgcn_mfma_f32_16x16x16f16(wa[2 * m], bv, z, 0, 0, 0);
      const f4 d1 = __builtin_amdgcn_mfma_f32_16x16x16f16(wa[2 * m + 1], bv, z, 0, 0, 0);
      const h4 zh = {0, 0, 0, 0};
      const h4 v0 = fast4<ACT>(d0, bias4[2 * m], zh, zh);
      const h4 v1 = fast4<ACT>(d1, bias4[2 * m + 1], zh, zh);
      wl[swz(j * CH + q * (NB / 2) + m)] = h8{v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
    }
    // The wave's block is bytes [16 * wave * M * 2, + 16 * M * 2) of the row
    // segment; pixels past the image's right edge fall outside the resource.
    const uint32_t wbase = (uint32_t)(16 * wave * M * 2);
#pragma unroll
    for (int st = 0; st < WCH / 64; ++st) {
      const int g = 64 * st + rl;
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, wl[swz(g)]), rs, wbase + 16 * g, 0, 0);
    }
  };
  for (int it = begin; it < end; it += kBatch) {
    _Float16 v[kBatch][3];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) load_b(min(it + u, end - 1), v[u]);
#pragma unroll
    for (int u = 0; u < kBatch; ++u)
      if (it + u < end) item(it + u, v[u]);
  }
}

// ---------------------------------------------------------------------------
// Elementwise, DepthToSpace and boundary IO (off the fused hot path)
// ---------------------------------------------------------------------------

__device__ __forceinline__ int64_t padded_index(int64_t i, int H, int W, int C, int Hp, int Wp) {
  const int c = (int)(i % C);
  int64_t r = i / C;
  const int w = (int)(r % W);
  r /= W;
  const int h = (int)(r % H);
  const int64_t n = r / H;
  return ((n * Hp + h + 1) * Wp + w + 1) * C + c;
}

// Unary (Sigmoid / Relu / Clip) and binary (Add / Mul) ops over the interior
// of padded tensors; fp32 math, one rounding (hip_kernels.h:493-519).
__global__ void __launch_bounds__(256) eltwise_kernel(EltArgs a, int binary) {
  const int64_t total = (int64_t)a.N * a.H * a.W * a.C;
  const _Float16* x = reinterpret_cast<const _Float16*>(a.a);
  const _Float16* y = reinterpret_cast<const _Float16*>(a.b);
  _Float16* o = reinterpret_cast<_Float16*>(a.out);
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t k = padded_index(i, a.H, a.W, a.C, a.Hp, a.Wp);
    const float v = (float)x[k];
    float r;
    if (binary) {
      const float w = (float)y[k];
      r = (a.op == kBinaryMul) ? v * w : v + w;
    } else if (a.op == kUnarySigmoid) {
      r = __builtin_amdgcn_rcpf(1.0f + __expf(-v));
    } else if (a.op == kUnaryRelu) {
      r = (v < 0.0f) ? 0.0f : v;
    } else {
      r = apply_clip(v, a.lo, a.hi);
    }
    o[k] = (_Float16)r;
  }
}

// DepthToSpace DCR (hip_kernels.h:521-580): output (n, oh, ow, c) reads input
// channel (r*b + q)*Cout + c at (oh/b, ow/b), r = oh % b, q = ow % b.
__global__ void __launch_bounds__(256) dts_kernel(DtsArgs a) {
  const int b = a.b;
  const int cout = a.C / (b * b);
  const int Ho = a.H * b, Wo = a.W * b;
  const int64_t total = (int64_t)a.N * Ho * Wo * cout;
  const int64_t Hpo = padded_rows(Ho), Wpo = padded_cols(Wo);
  const _Float16* in = reinterpret_cast<const _Float16*>(a.in);
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    // i enumerates the output in its own layout order.
    int n, c, oh, ow;
    if (a.out_kind == kOutPadded) {
      c = (int)(i % cout);
      int64_t r = i / cout;
      ow = (int)(r % Wo);
      r /= Wo;
      oh = (int)(r % Ho);
      n = (int)(r / Ho);
    } else {
      ow = (int)(i % Wo);
      int64_t r = i / Wo;
      oh = (int)(r % Ho);
      r /= Ho;
      c = (int)(r % cout);
      n = (int)(r / cout);
    }
    const int h = oh / b, rr = oh - h * b, w = ow / b, q = ow - w * b;
    const int cin = (rr * b + q) * cout + c;
    float v = (float)in[(((int64_t)n * a.Hp + h + 1) * a.Wp + w + 1) * a.C + cin];
    if (a.do_clip) v = apply_clip(v, a.lo, a.hi);
    if (a.out_kind == kOutPadded)
      reinterpret_cast<_Float16*>(a.out)[(((int64_t)n * Hpo + oh + 1) * Wpo + ow + 1) * cout + c] =
          (_Float16)v;
    else if (a.out_kind == kOutNchwF32)
      reinterpret_cast<float*>(a.out)[i] = v;
    else
      reinterpret_cast<_Float16*>(a.out)[i] = (_Float16)v;
  }
}

// Boundary NCHW (fp16 or fp32) -> padded NHWC fp16 (fp32 rounds to nearest
// even). One thread per NCHW element, so reads are coalesced.
__global__ void __launch_bounds__(256) input_convert(IoArgs a) {
  const int64_t total = (int64_t)a.N * a.C * a.H * a.W;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int w = (int)(i % a.W);
    int64_t r = i / a.W;
    const int h = (int)(r % a.H);
    r /= a.H;
    const int c = (int)(r % a.C);
    const int64_t n = r / a.C;
    const _Float16 v = a.fp32 ? (_Float16)reinterpret_cast<const float*>(a.src)[i]
                              : reinterpret_cast<const _Float16*>(a.src)[i];
    reinterpret_cast<_Float16*>(a.dst)[((n * a.Hp + h + 1) * a.Wp + w + 1) * a.C + c] = v;
  }
}

// Multi-channel boundary conversions, tiled through LDS: a workgroup moves one
// row segment of pixels x C channels (blockIdx.x = segment, then row, then
// image). The NCHW side is accessed per channel (consecutive pixels), the
// padded NHWC side per pixel (C consecutive channels), both coalesced; an
// element-by-element conversion would scatter one of them.
//
// Vector form (C % 8 == 0, W % 8 == 0, so every 8-element group is 16-byte
// aligned on both sides): 128-pixel segments, each lane moves 8 elements per
// global access. LDS holds the segment channel-major, [c][x], rows of
// kIoVecRow halfs (an odd number of dwords): the 8 channels of one pixel that a
// lane gathers, and the 8 lanes of one pixel's channel groups, fall in
// distinct banks.
constexpr int kIoVecSeg = 128;
constexpr int kIoVecRow = kIoVecSeg + 2;

__global__ void __launch_bounds__(256) input_convert_vec(IoArgs a) {
  extern __shared__ __attribute__((aligned(16))) _Float16 iolds[];
  const int C = a.C, cg = a.C >> 3;
  const int nseg = (a.W + kIoVecSeg - 1) / kIoVecSeg;
  const int seg = blockIdx.x % nseg;
  const int64_t rest = blockIdx.x / nseg;
  const int h = (int)(rest % a.H);
  const int64_t n = rest / a.H;
  const int w0 = seg * kIoVecSeg;
  const int ng = min(kIoVecSeg, a.W - w0) >> 3;  // 8-pixel groups in the segment
  // Load: task = (channel c, pixel group g), g fastest.
  for (int i = threadIdx.x; i < C * (kIoVecSeg / 8); i += blockDim.x) {
    const int c = i / (kIoVecSeg / 8), g = i - c * (kIoVecSeg / 8);
    if (g >= ng) continue;
    const int64_t src = ((n * C + c) * a.H + h) * a.W + w0 + 8 * g;
    h8 v;
    if (a.fp32) {
      const f4* p = reinterpret_cast<const f4*>(reinterpret_cast<const float*>(a.src) + src);
      const f4 lo = __builtin_nontemporal_load(p), hi = __builtin_nontemporal_load(p + 1);
      v = h8{(_Float16)lo[0], (_Float16)lo[1], (_Float16)lo[2], (_Float16)lo[3],
             (_Float16)hi[0], (_Float16)hi[1], (_Float16)hi[2], (_Float16)hi[3]};
    } else {
      v = __builtin_nontemporal_load(
          reinterpret_cast<const h8*>(reinterpret_cast<const _Float16*>(a.src) + src));
    }
    const u4 w = __builtin_bit_cast(u4, v);
    uint32_t* d = reinterpret_cast<uint32_t*>(iolds + c * kIoVecRow + 8 * g);
#pragma unroll
    for (int k = 0; k < 4; ++k) d[k] = w[k];
  }
  lds_sync();
  // Store: task = (pixel x, channel group q), q fastest: a wave writes whole
  // pixels, C * 2 consecutive bytes each.
  _Float16* dst = reinterpret_cast<_Float16*>(a.dst) + ((n * a.Hp + h + 1) * a.Wp + w0 + 1) * C;
  for (int i = threadIdx.x; i < 8 * ng * cg; i += blockDim.x) {
    const int x = i / cg, q = i - x * cg;
    h8 v;
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = iolds[(8 * q + k) * kIoVecRow + x];
    // Plain stores: the first conv reads this tensor next, partly from the cache.
    *reinterpret_cast<h8*>(dst + (int64_t)x * C + 8 * q) = v;
  }
}

__global__ void __launch_bounds__(256) output_convert_vec(IoArgs a) {
  extern __shared__ __attribute__((aligned(16))) _Float16 iolds[];
  const int C = a.C, cg = a.C >> 3;
  const int nseg = (a.W + kIoVecSeg - 1) / kIoVecSeg;
  const int seg = blockIdx.x % nseg;
  const int64_t rest = blockIdx.x / nseg;
  const int h = (int)(rest % a.H);
  const int64_t n = rest / a.H;
  const int w0 = seg * kIoVecSeg;
  const int ng = min(kIoVecSeg, a.W - w0) >> 3;
  const _Float16* src =
      reinterpret_cast<const _Float16*>(a.src) + ((n * a.Hp + h + 1) * a.Wp + w0 + 1) * C;
  for (int i = threadIdx.x; i < 8 * ng * cg; i += blockDim.x) {
    const int x = i / cg, q = i - x * cg;
    const h8 v = __builtin_nontemporal_load(reinterpret_cast<const h8*>(src + (int64_t)x * C + 8 * q));
#pragma unroll
    for (int k = 0; k < 8; ++k) iolds[(8 * q + k) * kIoVecRow + x] = v[k];
  }
  lds_sync();
  for (int i = threadIdx.x; i < C * (kIoVecSeg / 8); i += blockDim.x) {
    const int c = i / (kIoVecSeg / 8), g = i - c * (kIoVecSeg / 8);
    if (g >= ng) continue;
    const uint32_t* sp = reinterpret_cast<const uint32_t*>(iolds + c * kIoVecRow + 8 * g);
    const h8 v = __builtin_bit_cast(h8, u4{sp[0], sp[1], sp[2], sp[3]});
    const int64_t dst = ((n * C + c) * a.H + h) * a.W + w0 + 8 * g;
    if (a.fp32) {
      f4* p = reinterpret_cast<f4*>(reinterpret_cast<float*>(a.dst) + dst);
      __builtin_nontemporal_store(f4{(float)v[0], (float)v[1], (float)v[2], (float)v[3]}, p);
      __builtin_nontemporal_store(f4{(float)v[4], (float)v[5], (float)v[6], (float)v[7]}, p + 1);
    } else {
      __builtin_nontemporal_store(v, reinterpret_cast<h8*>(reinterpret_cast<_Float16*>(a.dst) + dst));
    }
  }
}

// Scalar form for any 2 <= C <= 128: 64-pixel segments, one element per lane
// and access; LDS rows hold one pixel's C channels plus one pad element.
constexpr int kIoSeg = 64;

__global__ void __launch_bounds__(256) input_convert_tiled(IoArgs a) {
  extern __shared__ _Float16 iolds[];
  const int C = a.C, cs = a.C + 1;
  const int nseg = (a.W + kIoSeg - 1) / kIoSeg;
  const int seg = blockIdx.x % nseg;
  const int64_t rest = blockIdx.x / nseg;
  const int h = (int)(rest % a.H);
  const int64_t n = rest / a.H;
  const int w0 = seg * kIoSeg;
  const int npx = min(kIoSeg, a.W - w0);
  for (int i = threadIdx.x; i < C * kIoSeg; i += blockDim.x) {
    const int c = i / kIoSeg, x = i - c * kIoSeg;
    if (x >= npx) continue;
    const int64_t src = ((n * C + c) * a.H + h) * a.W + w0 + x;
    iolds[x * cs + c] = a.fp32 ? (_Float16)reinterpret_cast<const float*>(a.src)[src]
                               : reinterpret_cast<const _Float16*>(a.src)[src];
  }
  lds_sync();
  _Float16* dst = reinterpret_cast<_Float16*>(a.dst) + ((n * a.Hp + h + 1) * a.Wp + w0 + 1) * C;
  for (int i = threadIdx.x; i < npx * C; i += blockDim.x) {
    const int x = i / C, c = i - x * C;
    dst[i] = iolds[x * cs + c];
  }
}

__global__ void __launch_bounds__(256) output_convert_tiled(IoArgs a) {
  extern __shared__ _Float16 iolds[];
  const int C = a.C, cs = a.C + 1;
  const int nseg = (a.W + kIoSeg - 1) / kIoSeg;
  const int seg = blockIdx.x % nseg;
  const int64_t rest = blockIdx.x / nseg;
  const int h = (int)(rest % a.H);
  const int64_t n = rest / a.H;
  const int w0 = seg * kIoSeg;
  const int npx = min(kIoSeg, a.W - w0);
  const _Float16* src =
      reinterpret_cast<const _Float16*>(a.src) + ((n * a.Hp + h + 1) * a.Wp + w0 + 1) * C;
  for (int i = threadIdx.x; i < npx * C; i += blockDim.x) {
    const int x = i / C, c = i - x * C;
    iolds[x * cs + c] = src[i];
  }
  lds_sync();
  for (int i = threadIdx.x; i < C * kIoSeg; i += blockDim.x) {
    const int c = i / kIoSeg, x = i - c * kIoSeg;
    if (x >= npx) continue;
    const int64_t dst = ((n * C + c) * a.H + h) * a.W + w0 + x;
    const _Float16 v = iolds[x * cs + c];
    if (a.fp32)
      reinterpret_cast<float*>(a.dst)[dst] = (float)v;
    else
      reinterpret_cast<_Float16*>(a.dst)[dst] = v;
  }
}

// Padded NHWC fp16 -> boundary NCHW (fp16 or fp32).
__global__ void __launch_bounds__(256) output_convert(IoArgs a) {
  const int64_t total = (int64_t)a.N * a.C * a.H * a.W;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int w = (int)(i % a.W);
    int64_t r = i / a.W;
    const int h = (int)(r % a.H);
    r /= a.H;
    const int c = (int)(r % a.C);
    const int64_t n = r / a.C;
    const _Float16 v =
        reinterpret_cast<const _Float16*>(a.src)[((n * a.Hp + h + 1) * a.Wp + w + 1) * a.C + c];
    if (a.fp32)
      reinterpret_cast<float*>(a.dst)[i] = (float)v;
    else
      reinterpret_cast<_Float16*>(a.dst)[i] = v;
  }
}

// Diagnostic fill of a padded NHWC fp16 buffer's interior (rows 1..H, columns
// 1..W, every channel) with one 16-bit pattern; the zero border is not
// touched. One thread per interior element.
__global__ void __launch_bounds__(256) poison_interior(uint16_t* buf, int32_t N, int32_t H,
                                                       int32_t W, int32_t C, int32_t Hp,
                                                       int32_t Wp, uint32_t pattern) {
  const int64_t total = (int64_t)N * H * W * C;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int c = (int)(i % C);
    int64_t r = i / C;
    const int w = (int)(r % W);
    r /= W;
    const int h = (int)(r % H);
    const int64_t n = r / H;
    buf[((n * Hp + h + 1) * Wp + w + 1) * C + c] = (uint16_t)pattern;
  }
}

// Zero fill of everything but the interior of a padded NHWC fp16 buffer: the
// Hp - H rows above and below the image (full width), then, on each image
// row, the Wp - W columns left and right of it. One thread per element.
__global__ void __launch_bounds__(256) zero_border(uint16_t* buf, int32_t N, int32_t H, int32_t W,
                                                   int32_t C, int32_t Hp, int32_t Wp) {
  const int64_t rows_px = (int64_t)(Hp - H) * Wp;  // top row + rows below the image
  const int64_t side = Wp - W;                      // left column + columns right of it
  const int64_t per_img = rows_px + (int64_t)H * side;
  const int64_t total = (int64_t)N * per_img * C;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int c = (int)(i % C);
    const int64_t r = i / C;
    const int64_t n = r / per_img;
    const int64_t k = r % per_img;
    int64_t row, col;
    if (k < rows_px) {
      const int64_t q = k / Wp;
      row = q == 0 ? 0 : H + q;
      col = k % Wp;
    } else {
      const int64_t k2 = k - rows_px;
      row = 1 + k2 / side;
      const int64_t j = k2 % side;
      col = j == 0 ? 0 : W + j;
    }
    buf[((n * Hp + row) * Wp + col) * C + c] = 0;
  }
}

// VapourSynth plane samples <-> NCHW boundary elements, one element per
// thread step (src/vapoursynth/vs_hip.cpp:175-225 packs on the host,
// 347-369 unpacks integer output):
// - integer samples scale by 1/255 (8 bit) or 1/65535 (16 bit) with one fp32
//   multiply, then round to fp16 (nearest even) or stay fp32;
// - fp16 widens exactly to fp32, fp32 rounds to fp16;
// - fp16 -> u16 (integer output) is trunc(v * 65535 + 0.5) in fp32 with no
//   fused multiply-add, clamped to [0, 65535] (NaN -> 0); the reference's cast
//   is undefined outside that range.
__device__ __forceinline__ float plane_load(const void* p, int64_t i, int kind) {
  switch (kind) {
    case kSampleU8: return (float)reinterpret_cast<const uint8_t*>(p)[i] * (1.0f / 255.0f);
    case kSampleU16: return (float)reinterpret_cast<const uint16_t*>(p)[i] * (1.0f / 65535.0f);
    case kSampleF16: return (float)reinterpret_cast<const _Float16*>(p)[i];
    default: return reinterpret_cast<const float*>(p)[i];
  }
}

__global__ void __launch_bounds__(256) plane_convert(PlaneArgs a) {
#pragma clang fp contract(off)
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < a.n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const float v = plane_load(a.src, i, a.src_kind);
    if (a.dst_kind == kSampleF16) {
      reinterpret_cast<_Float16*>(a.dst)[i] = (_Float16)v;
    } else if (a.dst_kind == kSampleF32) {
      reinterpret_cast<float*>(a.dst)[i] = v;
    } else {
      const float x = v * 65535.0f + 0.5f;
      const float c = x >= 65535.0f ? 65535.0f : (x > 0.0f ? x : 0.0f);
      reinterpret_cast<uint16_t*>(a.dst)[i] = (uint16_t)(uint32_t)c;
    }
  }
}

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------

namespace {
constexpr int kMaxDevices = 64;
std::atomic<int> g_cu_count[kMaxDevices];  // 0: not queried yet
}  // namespace

int cu_count() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) dev = 0;
  int n = g_cu_count[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    // Threads that race here all store the same value.
    hipDeviceProp_t p{};
    if (hipGetDeviceProperties(&p, dev) == hipSuccess) n = p.multiProcessorCount;
    if (n <= 0) n = 256;
    g_cu_count[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

FastDiv make_fastdiv(uint32_t d) {
  FastDiv f{d, 0, 0};
  uint32_t s = 0;
  while ((1ull << s) < d) ++s;
  f.s = s;
  f.m = static_cast<uint32_t>(((1ull << 32) * ((1ull << s) - d)) / d + 1);
  return f;
}

namespace {

using WinoKernel = void (*)(WinoArgs, WinoSched);

template <int KC>
WinoKernel pick_kernel(bool cvec, bool fast) {
  if (cvec) return fast ? winograd_conv<KC, true, true> : winograd_conv<KC, true, false>;
  return fast ? winograd_conv<KC, false, true> : winograd_conv<KC, false, false>;
}

WinoKernel wino_kernel(int kc, bool cvec, bool fast) {
  switch (kc) {
    case 1: return pick_kernel<1>(cvec, fast);
    case 2: return pick_kernel<2>(cvec, fast);
    case 3: return pick_kernel<3>(cvec, fast);
    default: return nullptr;
  }
}

int grid_for(int64_t total, int threads) {
  int64_t blocks = (total + threads - 1) / threads;
  const int64_t cap = (int64_t)cu_count() * 16;
  if (blocks > cap) blocks = cap;
  return blocks < 1 ? 1 : (int)blocks;
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

namespace {

using StripKernel = void (*)(StripArgs);

template <int KC, int ACT>
StripKernel strip_kernel_skips(int nskip) {
  switch (nskip) {
    case 0: return winograd_strip<KC, ACT, 0>;
    case 1: return winograd_strip<KC, ACT, 1>;
    case 2: return winograd_strip<KC, ACT, 2>;
    default: return nullptr;
  }
}

template <int KC>
StripKernel strip_kernel_act(int act, int nskip) {
  switch (act) {
    case kActNone: return strip_kernel_skips<KC, kActNone>(nskip);
    case kActRelu: return strip_kernel_skips<KC, kActRelu>(nskip);
    case kActSilu: return strip_kernel_skips<KC, kActSilu>(nskip);
    default: return nullptr;
  }
}

// winograd_strip covers C == M in {32, 64} with the fast epilogue;
// winograd_pipe covers C == M = 64 without residual inputs and C == M = 96.
bool strip_eligible(const WinoArgs& a) {
  const bool fast_epi = a.epi.out_kind == kOutPadded && a.epi.dts_b < 2 && !a.epi.do_clip &&
                        (a.epi.act == kActNone || a.epi.act == kActRelu ||
                         a.epi.act == kActSilu);
  if (!fast_epi || a.C != a.M) return false;
  return a.C == 32 || a.C == 64 || a.C == 96;
}

template <int KC, int NSKIP, int IO = 0>
hipError_t launch_pipe(const StripArgs& a, int act, hipStream_t s) {
  StripKernel pf = act == kActRelu   ? winograd_pipe<KC, kActRelu, NSKIP, IO>
                   : act == kActSilu ? winograd_pipe<KC, kActSilu, NSKIP, IO>
                                     : winograd_pipe<KC, kActNone, NSKIP, IO>;
  const size_t lds = PipeLds<KC>::lds_bytes((IO & 2) != 0, (IO & 1) != 0);
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(pf),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return e;
  int64_t grid = cu_count();  // one 512-thread workgroup per CU
  if (grid > a.n_items) grid = a.n_items;
  if (IO != 0) {
    // NCHW rows are 64 separate planes: every workgroup takes the same share
    // of one strip's rows (a multiple of the strip count, and of 8 for the
    // XCD mapping), so that all of them walk the same image rows together
    // and each plane row is read across the image at once.
    const int64_t per = (int64_t)a.N * a.n_strips;
    for (int64_t q = grid / per; q >= 1; --q)
      if ((per * q) % 8 == 0 && per * q <= a.n_items) {
        grid = per * q;
        break;
      }
  }
  grid = (grid + 7) / 8 * 8;
  hipLaunchKernelGGL(pf, dim3((unsigned)grid), dim3(512), lds, s, a);
  return hipGetLastError();
}

// The 64 -> 64 pipe with an NCHW fp16 boundary input and / or output
// (pipe_boundary_io): no residual inputs, no Clip, no DepthToSpace.
bool pipe_boundary_eligible(const WinoArgs& a) {
  const bool nchw_out = a.epi.out_kind == kOutNchwF16;
  if (!a.in_nchw && !nchw_out) return false;
  if (a.epi.out_kind != kOutPadded && !nchw_out) return false;
  if (a.epi.dts_b >= 2 || a.epi.do_clip || a.epi.skip0 != nullptr || a.epi.skip1 != nullptr)
    return false;
  if (a.epi.act != kActNone && a.epi.act != kActRelu && a.epi.act != kActSilu) return false;
  return (!a.in_nchw || pipe_boundary_io(a.N, a.H, a.W, a.C, a.M, true)) &&
         (!nchw_out || pipe_boundary_io(a.N, a.H, a.W, a.C, a.M, false));
}

hipError_t launch_strip(const WinoArgs& w, hipStream_t s) {
  StripArgs a{};
  a.in = w.in;
  a.u = w.u;
  a.bias = w.epi.bias;
  a.skip0 = w.epi.skip0 ? w.epi.skip0 : w.epi.skip1;
  a.skip1 = w.epi.skip0 ? w.epi.skip1 : nullptr;
  const int nskip = (a.skip0 != nullptr) + (a.skip1 != nullptr);
  a.out = reinterpret_cast<uint16_t*>(w.epi.out);
  a.N = w.N;
  a.H = w.H;
  a.W = w.W;
  a.Hp = (int32_t)padded_rows(w.H);
  a.Wp = (int32_t)padded_cols(w.W);
  a.tiles_h = (w.H + 1) / 2;
  a.tiles_w = (w.W + 1) / 2;
  a.n_strips = (a.tiles_w + 15) / 16;
  const int64_t items = (int64_t)a.N * a.n_strips * a.tiles_h;
  if (items >= (int64_t)1 << 31) return hipErrorInvalidValue;
  a.n_items = (int32_t)items;
  a.fd_tiles_h = make_fastdiv((uint32_t)a.tiles_h);
  a.fd_strips = make_fastdiv((uint32_t)a.n_strips);
  const int kc = w.C / 32;
  const int io = (w.in_nchw ? 1 : 0) | (w.epi.out_kind == kOutNchwF16 ? 2 : 0);
  if (io != 0) {
    if (!pipe_boundary_eligible(w)) return hipErrorInvalidValue;
    if (rowpipe_eligible(64, 64, 0, w.epi.act, w.N, w.H, w.W, io))
      return launch_rowpipe(a, w.epi.act, io, s);
    switch (io) {
      case 1: return launch_pipe<2, 0, 1>(a, w.epi.act, s);
      case 2: return launch_pipe<2, 0, 2>(a, w.epi.act, s);
      default: return launch_pipe<2, 0, 3>(a, w.epi.act, s);
    }
  }
  // 64 channels with residual inputs stay on winograd_strip (it runs at the
  // streaming rate there).
  if (nskip == 0 && kc == 2) {
    if (rowpipe_eligible(64, 64, 0, w.epi.act, w.N, w.H, w.W, 0))
      return launch_rowpipe(a, w.epi.act, 0, s);
    return launch_pipe<2, 0>(a, w.epi.act, s);
  }
  if (kc == 3) {
    // Up to one residual input the row pipe; with two the pipe, whose deeper
    // row lookahead keeps more of the residual reads in flight.
    if (rowpipe96_eligible(w.C, w.M, nskip, w.epi.act, w.N, w.H, w.W, 0))
      return launch_rowpipe96(a, w.epi.act, s);
    switch (nskip) {
      case 0: return launch_pipe<3, 0>(a, w.epi.act, s);
      case 1: return launch_pipe<3, 1>(a, w.epi.act, s);
      default: return launch_pipe<3, 2>(a, w.epi.act, s);
    }
  }
  StripKernel fn = kc == 1 ? strip_kernel_act<1>(w.epi.act, nskip)
                           : strip_kernel_act<2>(w.epi.act, nskip);
  if (fn == nullptr) return hipErrorInvalidValue;
  const int threads = 128 * kc;
  const size_t lds = (size_t)2 *
                     (kc == 1 ? StripLds<1>::VBUF + StripStage<1>::SBUF
                              : StripLds<2>::VBUF + StripStage<2>::SBUF) * 2;
  if (lds > 65536) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
  }
  int occ = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, fn, threads, lds) != hipSuccess ||
      occ < 1)
    occ = 1;
  int64_t grid = (int64_t)cu_count() * occ;
  if (grid > items) grid = items;
  grid = (grid + 7) / 8 * 8;
  hipLaunchKernelGGL(fn, dim3((unsigned)grid), dim3(threads), lds, s, a);
  return hipGetLastError();
}

}  // namespace

namespace {

using NarrowKernel = void (*)(NarrowArgs);

// conv3x3_narrow covers boundary-layout outputs with M <= 16 and no residual
// inputs (the model's tail conv, with or without DepthToSpace and Clip).
bool narrow_launch_eligible(const WinoArgs& w) {
  if (!narrow_eligible(w.C, w.M)) return false;
  if (w.epi.out_kind != kOutNchwF16 && w.epi.out_kind != kOutNchwF32) return false;
  if (w.epi.skip0 != nullptr || w.epi.skip1 != nullptr) return false;
  const int b = w.epi.dts_b >= 2 ? w.epi.dts_b : 1;
  if (w.M % (b * b) != 0) return false;
  const int64_t elem = w.epi.out_kind == kOutNchwF32 ? 4 : 2;
  const int64_t img = (int64_t)w.M * w.H * w.W * elem;  // Cout * (H b) * (W b)
  const int64_t in_img = padded_rows(w.H) * padded_cols(w.W) * w.C * 2;
  return img < ((int64_t)1 << 31) && in_img < ((int64_t)1 << 31);
}

template <int KC>
hipError_t launch_narrow_kc(const NarrowArgs& a, bool f32, hipStream_t s) {
  const bool rows = narrow_row_packed(a.M);
  NarrowKernel fn = rows ? (f32 ? conv3x3_tail<KC, true> : conv3x3_tail<KC, false>)
                         : (f32 ? conv3x3_narrow<KC, true> : conv3x3_narrow<KC, false>);
  // conv3x3_tail keeps only its D tiles ([16][TAIL_TW] floats, two buffers) in LDS.
  const size_t lds = rows ? (size_t)2 * 16 * TAIL_TW * 4 : NarrowRing<KC>::lds_bytes();
  if (lds > 65536) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
  }
  const int threads = rows ? 64 * TAIL_WAVES : 256;
  int occ = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, fn, threads, lds) != hipSuccess ||
      occ < 1)
    occ = 1;
  int64_t grid = (int64_t)cu_count() * occ;
  if (grid > a.n_items) grid = a.n_items;
  grid = (grid + 7) / 8 * 8;
  hipLaunchKernelGGL(fn, dim3((unsigned)grid), dim3(threads), lds, s, a);
  return hipGetLastError();
}

hipError_t launch_narrow(const WinoArgs& w, hipStream_t s) {
  NarrowArgs a{};
  a.in = w.in;
  a.w = w.u + winograd_u_halfs(w.C, w.M);
  a.bias = w.epi.bias;
  a.out = w.epi.out;
  a.N = w.N;
  a.H = w.H;
  a.W = w.W;
  a.Hp = (int32_t)padded_rows(w.H);
  a.Wp = (int32_t)padded_cols(w.W);
  a.M = w.M;
  a.act = w.epi.act;
  a.do_clip = w.epi.do_clip;
  a.clip_lo = w.epi.clip_lo;
  a.clip_hi = w.epi.clip_hi;
  a.dts_b = w.epi.dts_b >= 2 ? w.epi.dts_b : 1;
  a.cout = w.M / (a.dts_b * a.dts_b);
  a.n_seg = narrow_row_packed(w.M) ? (w.W + TAIL_SEG - 1) / TAIL_SEG : (w.W + 63) / 64;
  const int64_t items = (int64_t)w.N * a.n_seg * w.H;
  if (items >= (int64_t)1 << 31) return hipErrorInvalidValue;
  a.n_items = (int32_t)items;
  a.fd_H = make_fastdiv((uint32_t)w.H);
  a.fd_seg = make_fastdiv((uint32_t)a.n_seg);
  const bool f32 = w.epi.out_kind == kOutNchwF32;
  a.img_bytes = (int64_t)w.M * w.H * w.W * (f32 ? 4 : 2);
  switch (w.C / 32) {
    case 1: return launch_narrow_kc<1>(a, f32, s);
    case 2: return launch_narrow_kc<2>(a, f32, s);
    case 3: return launch_narrow_kc<3>(a, f32, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

hipError_t launch_winograd(WinoArgs a, hipStream_t s) {
  // An NCHW boundary input only the 64 -> 64 pipe reads (refused otherwise);
  // an NCHW fp16 output it writes when it can (else the general epilogue).
  if (a.in_nchw) return pipe_boundary_eligible(a) ? launch_strip(a, s) : hipErrorInvalidValue;
  if (a.epi.out_kind == kOutNchwF16 && pipe_boundary_eligible(a)) return launch_strip(a, s);
  if (narrow_launch_eligible(a)) return launch_narrow(a, s);
  if (strip_eligible(a)) return launch_strip(a, s);
  const WinoGeom g = winograd_geom(a.C, a.M);
  a.n_ob = g.n_ob;
  a.tb = g.tb;
  a.tiles_h = (a.H + 1) / 2;
  a.tiles_w = (a.W + 1) / 2;
  a.Hp = (int32_t)padded_rows(a.H);
  a.Wp = (int32_t)padded_cols(a.W);
  a.sb_w = (a.tiles_w + 16 * g.tb - 1) / (16 * g.tb);
  a.n_sb = a.N * a.tiles_h * a.sb_w;
  WinoSched sc{make_fastdiv((uint32_t)a.sb_w), make_fastdiv((uint32_t)a.tiles_h)};
  const bool cvec = (a.C % 4) == 0;
  const bool fast = a.epi.out_kind == kOutPadded && a.epi.dts_b < 2 && (a.M % 4) == 0 &&
                    !a.epi.do_clip;
  WinoKernel fn = wino_kernel(g.kc, cvec, fast);
  if (fn == nullptr) return hipErrorInvalidValue;
  if (g.lds > 65536) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)g.lds);
    if (e != hipSuccess) return e;
  }
  int occ = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, fn, g.threads, g.lds) != hipSuccess ||
      occ < 1)
    occ = 1;
  int grid = cu_count() * occ;
  const int need = (a.n_sb + 7) / 8 * 8;
  if (grid > need) grid = need;
  grid = (grid + 7) / 8 * 8;
  hipLaunchKernelGGL(fn, dim3(grid), dim3(g.threads), g.lds, s, a, sc);
  return hipGetLastError();
}


int direct_g8(int M) { return head_g8(M); }

hipError_t launch_direct(DirectArgs a, hipStream_t s) {
  // Only the column-walking fast path reads the NCHW boundary input; the
  // engine plans that fusion exactly when the fast path applies.
  a.g8 = direct_g8(a.M);
  a.Hp = (int32_t)padded_rows(a.H);
  a.Wp = (int32_t)padded_cols(a.W);
  if (a.g8 > 256) return hipErrorInvalidValue;
  const int threads = 256;
  const int ppb = threads / a.g8;
  const int64_t npix = (int64_t)a.N * a.H * a.W;
  int64_t blocks = (npix + ppb - 1) / ppb;
  const int64_t cap = (int64_t)cu_count() * 8;
  if (blocks > cap) blocks = cap;
  if (blocks < 1) blocks = 1;
  const bool fast = a.epi.out_kind == kOutPadded && a.epi.dts_b < 2 && (a.M % 8) == 0 &&
                    !a.epi.do_clip;
  if (fast && a.g8 <= 16) {
    const int seg = 4 * 256 / a.g8;
    const int n_seg = (a.W + seg - 1) / seg;
    const int64_t items = (int64_t)a.N * n_seg * a.H;
    // The head kernels address one input image through a buffer resource with
    // a 32-bit size (NCHW boundary image, or the padded copy). For the boundary
    // input the planner applies the same rule (head_reads_boundary_input).
    const bool fits = a.in_kind == 0
                          ? items < ((int64_t)1 << 31) && (int64_t)a.Hp * a.Wp * 2 < ((int64_t)1 << 31)
                          : head_reads_boundary_input(a.N, a.H, a.W, a.M, a.in_kind == 2);
    if (fits) {
      const FastDiv fs = make_fastdiv((uint32_t)n_seg), fh = make_fastdiv((uint32_t)a.H);
      using HeadKernel = void (*)(DirectArgs, int, int, FastDiv, FastDiv);
      const bool sk = a.epi.skip0 != nullptr || a.epi.skip1 != nullptr;
      if (a.in_kind != 0 && sk) return hipErrorInvalidValue;
      const int act = a.epi.act == kActRelu ? 1 : (a.epi.act == kActSilu ? 2 : 0);
      // Rows: padded input without / with residual inputs, then the NCHW
      // boundary input in fp16 and fp32 (never with residual inputs).
      const int variant = a.in_kind == 0 ? (sk ? 1 : 0) : 1 + a.in_kind;
      auto pick = [&](auto g_tag) -> HeadKernel {
        constexpr int GG = decltype(g_tag)::value;
        static const HeadKernel t[4][3] = {
            {direct_conv_c1_walk<GG, kActNone, false, 0>, direct_conv_c1_walk<GG, kActRelu, false, 0>,
             direct_conv_c1_walk<GG, kActSilu, false, 0>},
            {direct_conv_c1_walk<GG, kActNone, true, 0>, direct_conv_c1_walk<GG, kActRelu, true, 0>,
             direct_conv_c1_walk<GG, kActSilu, true, 0>},
            {direct_conv_c1_walk<GG, kActNone, false, 1>, direct_conv_c1_walk<GG, kActRelu, false, 1>,
             direct_conv_c1_walk<GG, kActSilu, false, 1>},
            {direct_conv_c1_walk<GG, kActNone, false, 2>, direct_conv_c1_walk<GG, kActRelu, false, 2>,
             direct_conv_c1_walk<GG, kActSilu, false, 2>}};
        return t[variant][act];
      };
      // M = 32, 64, 96 without residual inputs: the MFMA head.
      if (!sk && a.M % 32 == 0 && a.M <= 96) {
        const int ns = (a.W + 63) / 64;
        const int64_t mitems = (int64_t)a.N * ns * a.H;
        if (mitems < ((int64_t)1 << 31)) {
          auto mpick = [&](auto nb_tag) -> HeadKernel {
            constexpr int NB = decltype(nb_tag)::value;
            static const HeadKernel t[3][3] = {
                {direct_conv_c1_mfma<NB, kActNone, 0>, direct_conv_c1_mfma<NB, kActRelu, 0>,
                 direct_conv_c1_mfma<NB, kActSilu, 0>},
                {direct_conv_c1_mfma<NB, kActNone, 1>, direct_conv_c1_mfma<NB, kActRelu, 1>,
                 direct_conv_c1_mfma<NB, kActSilu, 1>},
                {direct_conv_c1_mfma<NB, kActNone, 2>, direct_conv_c1_mfma<NB, kActRelu, 2>,
                 direct_conv_c1_mfma<NB, kActSilu, 2>}};
            return t[a.in_kind][act];
          };
          HeadKernel fn = a.M == 32 ? mpick(IntC<2>{}) : a.M == 64 ? mpick(IntC<4>{}) : mpick(IntC<6>{});
          // Four waves' staging blocks: 16 pixels x M fp16 each.
          const size_t lds = (size_t)4 * 16 * a.M * 2;
          int occ = 0;
          if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, reinterpret_cast<const void*>(fn),
                                                           256, lds) != hipSuccess ||
              occ < 1)
            occ = 1;
          int64_t grid = (int64_t)cu_count() * occ;
          if (grid > mitems) grid = mitems;
          grid = (grid + 7) / 8 * 8;
          const FastDiv fms = make_fastdiv((uint32_t)ns);
          hipLaunchKernelGGL(fn, dim3((unsigned)grid), dim3(256), lds, s, a, ns, (int)mitems, fms, fh);
          return hipGetLastError();
        }
      }
      HeadKernel fn = a.g8 == 1 ? pick(IntC<1>{}) : a.g8 == 2 ? pick(IntC<2>{})
                    : a.g8 == 4 ? pick(IntC<4>{}) : a.g8 == 8 ? pick(IntC<8>{}) : pick(IntC<16>{});
      int occ = 0;
      if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, reinterpret_cast<const void*>(fn), 256,
                                                       0) != hipSuccess ||
          occ < 1)
        occ = 1;
      // Two workgroups per CU at most: longer column walks amortise each
      // workgroup's six-row prologue (1080p 1 -> 64: 68 us with four per CU,
      // 64 us with two, 72 us with one).
      int64_t grid = (int64_t)cu_count() * (occ > 2 ? 2 : occ);
      if (grid > items) grid = items;
      grid = (grid + 7) / 8 * 8;
      hipLaunchKernelGGL(fn, dim3((unsigned)grid), dim3(256), 0, s, a, n_seg, (int)items, fs, fh);
      return hipGetLastError();
    }
  }
  if (a.in_kind != 0) return hipErrorInvalidValue;
  if (fast)
    hipLaunchKernelGGL(direct_conv_c1<true>, dim3((unsigned)blocks), dim3(threads), 0, s, a);
  else
    hipLaunchKernelGGL(direct_conv_c1<false>, dim3((unsigned)blocks), dim3(threads), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_eltwise(EltArgs a, bool binary, hipStream_t s) {
  const int64_t total = (int64_t)a.N * a.H * a.W * a.C;
  hipLaunchKernelGGL(eltwise_kernel, dim3(grid_for(total, 256)), dim3(256), 0, s, a,
                     binary ? 1 : 0);
  return hipGetLastError();
}

hipError_t launch_dts(DtsArgs a, hipStream_t s) {
  const int64_t total = (int64_t)a.N * a.H * a.W * a.C;
  hipLaunchKernelGGL(dts_kernel, dim3(grid_for(total, 256)), dim3(256), 0, s, a);
  return hipGetLastError();
}

// Tiled conversions for 2 <= C <= 128 (one workgroup per row segment, at most
// 2^31 of them); the vector form when C and W are multiples of 8 and both
// buffers 16-byte aligned; otherwise one thread per element.
static int64_t io_blocks(const IoArgs& a, int seg) {
  return (int64_t)a.N * a.H * ((a.W + seg - 1) / seg);
}
static bool io_tiled(const IoArgs& a) {
  return a.C >= 2 && a.C <= 128 && io_blocks(a, kIoSeg) < ((int64_t)1 << 31);
}
static bool io_vec(const IoArgs& a) {
  return io_tiled(a) && a.C % 8 == 0 && a.W % 8 == 0 &&
         reinterpret_cast<uintptr_t>(a.src) % 16 == 0 && reinterpret_cast<uintptr_t>(a.dst) % 16 == 0;
}

hipError_t launch_input_convert(IoArgs a, hipStream_t s) {
  const int64_t total = (int64_t)a.N * a.H * a.W * a.C;
  if (total == 0) return hipSuccess;
  if (io_vec(a)) {
    const size_t lds = (size_t)a.C * kIoVecRow * 2;
    hipLaunchKernelGGL(input_convert_vec, dim3((unsigned)io_blocks(a, kIoVecSeg)), dim3(256), lds,
                       s, a);
    return hipGetLastError();
  }
  if (io_tiled(a)) {
    const size_t lds = (size_t)kIoSeg * (a.C + 1) * 2;
    hipLaunchKernelGGL(input_convert_tiled, dim3((unsigned)io_blocks(a, kIoSeg)), dim3(256), lds,
                       s, a);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(input_convert, dim3(grid_for(total, 256)), dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_output_convert(IoArgs a, hipStream_t s) {
  const int64_t total = (int64_t)a.N * a.H * a.W * a.C;
  if (total == 0) return hipSuccess;
  if (io_vec(a)) {
    const size_t lds = (size_t)a.C * kIoVecRow * 2;
    hipLaunchKernelGGL(output_convert_vec, dim3((unsigned)io_blocks(a, kIoVecSeg)), dim3(256), lds,
                       s, a);
    return hipGetLastError();
  }
  if (io_tiled(a)) {
    const size_t lds = (size_t)kIoSeg * (a.C + 1) * 2;
    hipLaunchKernelGGL(output_convert_tiled, dim3((unsigned)io_blocks(a, kIoSeg)), dim3(256), lds,
                       s, a);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(output_convert, dim3(grid_for(total, 256)), dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_poison(void* buf, int32_t N, int32_t H, int32_t W, int32_t C, uint16_t pattern,
                         hipStream_t s) {
  if (buf == nullptr || N < 0 || H < 0 || W < 0 || C < 0) return hipErrorInvalidValue;
  const int64_t total = (int64_t)N * H * W * C;
  if (total == 0) return hipSuccess;
  hipLaunchKernelGGL(poison_interior, dim3(grid_for(total, 256)), dim3(256), 0, s,
                     static_cast<uint16_t*>(buf), N, H, W, C, (int32_t)padded_rows(H),
                     (int32_t)padded_cols(W), (uint32_t)pattern);
  return hipGetLastError();
}

hipError_t launch_zero_border(void* buf, int32_t N, int32_t H, int32_t W, int32_t C,
                              hipStream_t s) {
  if (buf == nullptr || N < 0 || H < 0 || W < 0 || C < 0) return hipErrorInvalidValue;
  const int64_t Hp = padded_rows(H), Wp = padded_cols(W);
  const int64_t total = (int64_t)N * ((Hp - H) * Wp + (int64_t)H * (Wp - W)) * C;
  if (total == 0) return hipSuccess;
  hipLaunchKernelGGL(zero_border, dim3(grid_for(total, 256)), dim3(256), 0, s,
                     static_cast<uint16_t*>(buf), N, H, W, C, (int32_t)Hp, (int32_t)Wp);
  return hipGetLastError();
}

hipError_t launch_plane_convert(PlaneArgs a, hipStream_t s) {
  const bool src_ok = a.src_kind >= kSampleU8 && a.src_kind <= kSampleF32;
  const bool dst_ok = a.dst_kind == kSampleF16 || a.dst_kind == kSampleF32 ||
                      (a.dst_kind == kSampleU16 && a.src_kind == kSampleF16);
  if (!src_ok || !dst_ok || a.n < 0) return hipErrorInvalidValue;
  if (a.n == 0) return hipSuccess;
  hipLaunchKernelGGL(plane_convert, dim3(grid_for(a.n, 256)), dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace arthip

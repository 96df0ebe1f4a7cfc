// A lone 64 -> 64 conv (bias, activation, no residual input; padded NHWC fp16
// or the NCHW fp16 boundary layout on either side) with the fused block's
// arithmetic and wave layout: Winograd F(2,3) along x with the three kernel
// rows summed in the MFMA, three wave groups per SIMD.

#include <hip/hip_runtime.h>

#include <cstdint>

#include "conv_args.h"
#include "launch.h"
#include "pack.h"
#include "wino_dev.h"

namespace arthip {

// ---------------------------------------------------------------------------
// Row-Winograd pipe: out = act(conv(in) + bias), C = M = 64
// ---------------------------------------------------------------------------
//
// Items are one output tile row (two pixel rows) x 32 tiles (64 pixels),
// ordered (image, 64-pixel strip, tile row) with the tile row fastest; one
// 768-thread workgroup per CU (12 waves, three per SIMD, 128 KB of LDS, up to
// 152 KB with the boundary layouts) walks runs of them down a strip.
//   waves 0-7  fold: wave w holds U' of output channels 16 (w & 3) .. + 15
//              (96 VGPRs, the packed row filters) and folds the 16 tiles
//              16 (w >> 2) .. + 15 of each item into staging, with bias and
//              activation (so each SIMD's two fold waves share one channel
//              block and split the tiles);
//   waves 8-11 load the input rows of the next row pair, transform them into
//              a 3-slot LDS ring of transformed row pairs (4 positions x 32
//              tiles x 64 channels per row), and store the staged item of two
//              phases before.
// Per run (input row pair Q_i = padded rows 2 (j0 + i) and 2 (j0 + i) + 1;
// item i, output rows 2 (j0 + i) and + 1, reads Q_i and Q_{i+1}), after a
// prologue that transforms Q_0 into slot 0 and a barrier, phase k
// (k = 0 .. len+1) ends with the workgroup barrier:
//   fold waves:  fold item k-1 from slots (k-1)%3, k%3 into staging[k&1]
//                (1 <= k <= len)
//   load waves:  store item k-2 from staging[(k-1)&1] (k >= 2); transform
//                Q_{k+1} into slot (k+1)%3 and load the rows of Q_{k+2}
//                (k < len)
// The fold is block_fold's (row_pair_transform's V, chains X / b / P / c): the
// fused block's per-element arithmetic, here on tiles at even columns.
//
// Boundary layouts (IO bit 0: NCHW input, bit 1: NCHW output; W % 8 == 0), the
// same arithmetic in other layouts:
//   NCHW input: load wave w owns channels 16 w .. + 15 (lane: tile l & 15 and
//     + 16, channel quad 4 w + (l >> 4)) and copies its channels' two rows of
//     the next row pair, 80 pixels from 64 s - 8, into a private 5 KB LDS ring
//     with five 16-byte buffer -> LDS loads per lane, one phase ahead; only
//     the wave's own load count orders it. Channel row (c, r) of quad j sits
//     at position 2 j + (m & 1) + 8 (m >> 1), m = 2 c + r, 160 bytes apart, so
//     each dword read of the patches (16 tiles x 4 quads) hits 64 distinct
//     banks.
//   NCHW output: the fold stages channel-major ([row][channel][72 halfs]: its
//     4-byte writes of four channel quads land on distinct banks) and each
//     store thread writes 8 pixels of one channel as a 16-byte word; the
//     channels of lanes 32 .. 63 are those of lanes 0 .. 31 plus 8, so each
//     16-byte read group covers 64 banks.
struct RowPipeL {
  static constexpr int C = 64;
  static constexpr int PX = 2 * C;       // bytes per pixel
  static constexpr int TILES = 32;       // tiles per item
  static constexpr int OPX = 2 * TILES;  // output pixels per item
  static constexpr int THREADS = 768;
  static constexpr int WPS = TILES * 64;  // halfs per position (32 tiles x 64 channels)
  static constexpr int RROW = 4 * WPS;    // halfs per transformed row
  static constexpr int RPAIR = 2 * RROW;  // halfs per ring slot
  static constexpr int NSLOT = 3;
  static constexpr int SBUF = 2 * OPX * C;  // halfs per staging buffer (2 rows x 64 px)
  // Offset (halfs) of the row filters in a 64 -> 64 conv's packed weights.
  static constexpr int UOFF = 4 * 16 * 2 * 64 * 8;
  static constexpr int V = 0;
  static constexpr int STG = NSLOT * RPAIR;
  // Channel-major staging of the NCHW output: [row][channel][NCS halfs].
  static constexpr int NCS = 72;
  static constexpr int SBUF_NCHW = 2 * C * NCS;
  // NCHW input ring: per load wave 32 channel rows of RPW dwords (80 pixels).
  static constexpr int RPW = 40;
  static constexpr int RREG = 32 * RPW;
  static constexpr size_t lds_bytes(int io) {
    return (size_t)(STG + 2 * ((io & 2) ? SBUF_NCHW : SBUF)) * 2 + ((io & 1) ? 4 * RREG * 4 : 0);
  }
  // V' element (tile t < 32, channel c): 128-byte tile rows with the eight
  // 16-byte channel groups of tile t at g ^ (t & 7).
  __host__ __device__ static constexpr int at(int t, int c) {
    return t * 64 + ((((c >> 3) ^ (t & 7))) << 3) + (c & 7);
  }
  // Staging element (row, pixel x < 64, 16-byte group g): groups of pixel x at
  // g ^ ((x >> 1) & 7).
  __host__ __device__ static constexpr int st(int row, int x, int g) {
    return (row * OPX + x) * C + ((g ^ ((x >> 1) & 7)) << 3);
  }
};

// 1-D transform of a task's two input rows (element 2 (4 r + j) + e of x:
// row r, column j, channel pair e) into positions p of two transformed rows:
// V0 = d0 - d2, V1 = d1 + d2, V2 = d2 - d1, V3 = d3 - d1.
__device__ __forceinline__ void rp_transform(_Float16* vw, const h2 (&x)[16]) {
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    h2 o[4][2];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const h2 d0 = x[2 * (4 * r) + e], d1 = x[2 * (4 * r + 1) + e];
      const h2 d2 = x[2 * (4 * r + 2) + e], d3 = x[2 * (4 * r + 3) + e];
      o[0][e] = pk_sub(d0, d2);
      o[1][e] = d1 + d2;
      o[2][e] = pk_sub(d2, d1);
      o[3][e] = pk_sub(d3, d1);
    }
#pragma unroll
    for (int p = 0; p < 4; ++p)
      *reinterpret_cast<h4*>(vw + r * RowPipeL::RROW + p * RowPipeL::WPS) =
          __builtin_shufflevector(o[p][0], o[p][1], 0, 1, 2, 3);
  }
}

// The same transform for one tile and one channel octet (element 4 r + j of
// x: row r, column j, channels 8 g .. 8 g + 7), written as 16-byte groups.
__device__ __forceinline__ void rp_transform8(_Float16* vw, const h8 (&x)[8]) {
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    h2 o[4][4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const h2 d0 = h2{x[4 * r][2 * e], x[4 * r][2 * e + 1]};
      const h2 d1 = h2{x[4 * r + 1][2 * e], x[4 * r + 1][2 * e + 1]};
      const h2 d2 = h2{x[4 * r + 2][2 * e], x[4 * r + 2][2 * e + 1]};
      const h2 d3 = h2{x[4 * r + 3][2 * e], x[4 * r + 3][2 * e + 1]};
      o[0][e] = pk_sub(d0, d2);
      o[1][e] = d1 + d2;
      o[2][e] = pk_sub(d2, d1);
      o[3][e] = pk_sub(d3, d1);
    }
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const h4 lo = __builtin_shufflevector(o[p][0], o[p][1], 0, 1, 2, 3);
      const h4 hi = __builtin_shufflevector(o[p][2], o[p][3], 0, 1, 2, 3);
      *reinterpret_cast<h8*>(vw + r * RowPipeL::RROW + p * RowPipeL::WPS) =
          __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    }
  }
}

// Fold of one item half (16 tiles, two output rows) x 16 output channels from
// row pairs A (rows R0, R1) and B (R2, R3): the fused block's chains.
__device__ __forceinline__ void rp_fold(const h8 (&u)[3][4][2], const _Float16* const (&vr)[2],
                                        int offA, int offB, f4 bias4, f4& y00, f4& y01, f4& y10,
                                        f4& y11) {
  constexpr int WPS = RowPipeL::WPS;
  constexpr int RROW = RowPipeL::RROW;
  auto pos = [&](int p, f4& a0, f4& a1) {
#pragma unroll
    for (int kc = 0; kc < 2; ++kc) {
      const h8 f0 = *reinterpret_cast<const h8*>(vr[kc] + offA + p * WPS);
      const h8 f1 = *reinterpret_cast<const h8*>(vr[kc] + offA + RROW + p * WPS);
      const h8 f2 = *reinterpret_cast<const h8*>(vr[kc] + offB + p * WPS);
      const h8 f3 = *reinterpret_cast<const h8*>(vr[kc] + offB + RROW + p * WPS);
      a0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(u[0][p][kc], f0, a0, 0, 0, 0);
      a1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(u[0][p][kc], f1, a1, 0, 0, 0);
      a0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(u[1][p][kc], f1, a0, 0, 0, 0);
      a1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(u[1][p][kc], f2, a1, 0, 0, 0);
      a0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(u[2][p][kc], f2, a0, 0, 0, 0);
      a1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(u[2][p][kc], f3, a1, 0, 0, 0);
    }
  };
  __builtin_amdgcn_iglp_opt(1);
  const f4 m2 = {-2.0f, -2.0f, -2.0f, -2.0f};
  f4 X0 = {0, 0, 0, 0}, X1 = {0, 0, 0, 0};
  pos(2, X0, X1);
  f4 b0 = X0 + bias4, b1 = X1 + bias4;
  pos(1, b0, b1);
  f4 c0 = b0, c1 = b1;
  pos(0, b0, b1);
  pos(3, c0, c1);
  y00 = b0;
  y10 = b1;
  y01 = __builtin_elementwise_fma(X0, m2, c0);
  y11 = __builtin_elementwise_fma(X1, m2, c1);
}

// Phases k = 0 .. len + 1, six per iteration so that k % 6 (the ring slots
// and the staging parity) is a compile-time constant.
template <class F>
__device__ __forceinline__ void rp_phases(int len, F&& ph) {
  for (int k = 0;;) {
    ph(IntC<0>{}, k);
    if (++k > len + 1) break;
    ph(IntC<1>{}, k);
    if (++k > len + 1) break;
    ph(IntC<2>{}, k);
    if (++k > len + 1) break;
    ph(IntC<3>{}, k);
    if (++k > len + 1) break;
    ph(IntC<4>{}, k);
    if (++k > len + 1) break;
    ph(IntC<5>{}, k);
    if (++k > len + 1) break;
  }
}

template <int ACT, int IO>
__global__ void __launch_bounds__(RowPipeL::THREADS) __attribute__((amdgpu_waves_per_eu(3, 3)))
winograd_rowpipe(StripArgs a) {
  using L = RowPipeL;
  constexpr int C = L::C;
  constexpr int PX = L::PX;
  constexpr bool IN_NCHW = (IO & 1) != 0;
  constexpr bool OUT_NCHW = (IO & 2) != 0;
  constexpr int SBUF = OUT_NCHW ? L::SBUF_NCHW : L::SBUF;
  constexpr int RPAIR = L::RPAIR;
  constexpr uint32_t kOob = 0x80000000u;
  extern __shared__ __attribute__((aligned(16))) _Float16 plds[];
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;

  const int G = gridDim.x;
  const int slot = (blockIdx.x & 7) * (G >> 3) + (blockIdx.x >> 3);
  const int begin = (int)((int64_t)a.n_items * slot / G);
  const int end = (int)((int64_t)a.n_items * (slot + 1) / G);
  if (begin >= end) return;  // uniform across the workgroup

  const int64_t row_bytes = (int64_t)a.Wp * PX;
  const uint32_t rb32 = (uint32_t)row_bytes;
  int n = 0, s = 0, j0 = 0;
  auto decode = [&](int item) {
    const uint32_t sgl = fdiv((uint32_t)item, a.fd_tiles_h);
    j0 = item - (int)(sgl * (uint32_t)a.tiles_h);
    const uint32_t nn = fdiv(sgl, a.fd_strips);
    s = (int)(sgl - nn * (uint32_t)a.n_strips);
    n = (int)nn;
  };
  _Float16* const stg = plds + L::STG;

  if (wave < 8) {
    // ---------------- fold waves ---------------------------------------------
    // MFMA lane: tile 16 half + tcol, B rows 8*kq.. of each 32-channel chunk,
    // output channels [ch0, ch0 + 4) of the tile's four pixels.
    const int blk = wave & 3;
    const int half = wave >> 2;
    const int tcol = lane & 15;
    const int kq = lane >> 4;
    const int ch0 = 16 * blk + 4 * kq;
    h8 u[3][4][2];
    {
      const h8* up = reinterpret_cast<const h8*>(a.u + L::UOFF) + (size_t)blk * (12 * 2 * 64) + lane;
#pragma unroll
      for (int dy = 0; dy < 3; ++dy)
#pragma unroll
        for (int p = 0; p < 4; ++p)
#pragma unroll
          for (int kc = 0; kc < 2; ++kc) u[dy][p][kc] = up[((dy * 4 + p) * 2 + kc) * 64];
    }
    const f4 bias4 = *reinterpret_cast<const f4*>(a.bias + ch0);
    const int t = 16 * half + tcol;
    const _Float16* vr[2];
#pragma unroll
    for (int kc = 0; kc < 2; ++kc) vr[kc] = plds + L::V + L::at(t, 32 * kc + 8 * kq);
    // Staging of this lane's four values: pixels 2 t, 2 t + 1 of rows 0, 1,
    // channels ch0 .. ch0 + 3.
    const int sw0 = L::st(0, 2 * t, ch0 >> 3) + (ch0 & 7);
    auto phase = [&](auto k6_tag, int k, int len) {
      constexpr int K6 = decltype(k6_tag)::value;  // k % 6
      constexpr int P = K6 & 1;
      constexpr int SA = ((K6 + 2) % 3) * RPAIR, SB = (K6 % 3) * RPAIR;
      if (k >= 1 && k <= len) {
        f4 y00, y01, y10, y11;
        rp_fold(u, vr, SA, SB, bias4, y00, y01, y10, y11);
        if constexpr (OUT_NCHW) {
          // Pixels 2 t and 2 t + 1 of channel ch0 + e, per row.
          const h4 a0 = strip_act4<ACT>(y00), a1 = strip_act4<ACT>(y01);
          const h4 b0 = strip_act4<ACT>(y10), b1 = strip_act4<ACT>(y11);
          _Float16* sc = stg + P * SBUF + ch0 * L::NCS + 2 * t;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            *reinterpret_cast<h2*>(sc + e * L::NCS) = h2{a0[e], a1[e]};
            *reinterpret_cast<h2*>(sc + (C + e) * L::NCS) = h2{b0[e], b1[e]};
          }
        } else {
          _Float16* sw = stg + P * SBUF + sw0;
          *reinterpret_cast<h4*>(sw) = strip_act4<ACT>(y00);
          *reinterpret_cast<h4*>(sw + C) = strip_act4<ACT>(y01);
          *reinterpret_cast<h4*>(sw + L::OPX * C) = strip_act4<ACT>(y10);
          *reinterpret_cast<h4*>(sw + (L::OPX + 1) * C) = strip_act4<ACT>(y11);
        }
      }
      lds_sync();
    };
    for (int it = begin; it < end;) {
      decode(it);
      const int len = min(end - it, a.tiles_h - j0);
      lds_sync();  // the prologue
      rp_phases(len, [&](auto pt, int k) { phase(pt, k, len); });
      it += len;
    }
    return;
  }

  // ---------------- load, transform and store waves ---------------------------
  // Transform tasks. Padded input: tile t8 and channel octet g8 per thread,
  // t8 = 8 pw + 2 ((l >> 3) & 3) + (l >> 5), so that lanes l and l + 32,
  // whose 16-byte writes the LDS serves together, take tiles of opposite
  // parity (their two 128-byte tile rows cover all 64 banks). NCHW input:
  // tiles tt and tt + 16, channel quad tq by wave. Store tasks (padded
  // output): 16-byte group sg of pixels sx and sx + 32 in both rows of an item.
  const int gtid = tid - 512;
  const int pw = wave - 8;
  const int tt = lane & 15;
  const int tq = 4 * pw + (lane >> 4);
  const int t8 = 8 * pw + 2 * ((lane >> 3) & 3) + (lane >> 5);
  const int g8 = lane & 7;
  const int sx = gtid >> 3;
  const int sg = gtid & 7;
  _Float16* vw[2];
  vw[0] = plds + L::V + L::at(tt, 4 * tq);
  vw[1] = plds + L::V + L::at(tt + 16, 4 * tq);
  _Float16* const vw8 = plds + L::V + L::at(t8, 8 * g8);
  const uint32_t plane = (uint32_t)a.H * (uint32_t)a.W * 2;  // NCHW channel plane bytes
  // Input patch of tile t8: padded columns pc0 .. pc0 + 3 with pc0 = 64 s +
  // 2 t8, 16 bytes of channel octet g8 each; the row in the scalar offset.
  // Columns past the padded row get an out-of-range lane offset and rows past
  // the image a zero-size resource (both read as zero).
  const int64_t img_bytes = (int64_t)a.Hp * row_bytes;
  __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)a.in, (short)0, 0, 0x00020000);
  __amdgpu_buffer_rsrc_t rs0 = rs;
  uint32_t col_off[4];
  auto load8 = [&](h8 (&x)[8], int pr) {
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const bool row_ok = pr + r < a.Hp;  // uniform
      const __amdgpu_buffer_rsrc_t rr = row_ok ? rs : rs0;
      const uint32_t ro = row_ok ? (uint32_t)(pr + r) * rb32 : 0u;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        x[4 * r + j] =
            __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(rr, col_off[j], ro, 0));
    }
  };
  // NCHW input ring of this wave: the five 16-byte copies of lane l are
  // chunks q = 64 i + l of the region, position p = q / 10, chunk k = q % 10
  // (pixels 64 s - 8 + 8 k ..); position p holds row r = m & 1, channel
  // 16 pw + 4 j + (m >> 1) with j = (p & 7) >> 1, m = (p & 1) + 2 (p >> 3).
  uint32_t* const ring = reinterpret_cast<uint32_t*>(stg + 2 * SBUF) + pw * L::RREG;
  // Per run: byte offset of copy c's channel and pixel in the image (kOob for
  // pixels outside the row: adding a row offset keeps it past the resource),
  // and bit c of d_rows = its row within the pair.
  uint32_t d_base[5];
  uint32_t d_rows = 0;
#pragma unroll
  for (int c = 0; c < 5; ++c) {
    const int pp = (64 * c + lane) / 10;
    d_rows |= (uint32_t)(pp & 1) << c;
  }
  auto set_copies = [&]() {
#pragma unroll
    for (int c = 0; c < 5; ++c) {
      const int q = 64 * c + lane;
      const int pp = q / 10;
      const int ch = 16 * pw + 4 * ((pp & 7) >> 1) + (pp >> 3);
      const int x = L::OPX * s - 8 + 8 * (q - 10 * pp);
      d_base[c] = (x >= 0 && x < a.W) ? (uint32_t)ch * plane + (uint32_t)x * 2 : kOob;
    }
  };
  // Row pair i of the run: image rows 2 (j0 + i) - 1 and 2 (j0 + i).
  auto issue = [&](int i) {
    const uint32_t dst = lds_byte_addr(ring);
#pragma unroll
    for (int c = 0; c < 5; ++c) {
      const int y = 2 * (j0 + i) - 1 + (int)((d_rows >> c) & 1);
      const bool ok = y >= 0 && y < a.H;
      dma16_buf(dst + 1024 * c, rs, ok ? d_base[c] + (uint32_t)y * (uint32_t)a.W * 2 : kOob);
    }
  };
  // The patches of tiles tt, tt + 16 from the ring: channel c of quad tq, row
  // r at position 2 jq + (m & 1) + 8 (m >> 1); pixels 64 s + 2 t - 1 .. + 2
  // are halfs 2 t + 7 .. 2 t + 10 of the row (dwords t + 3 .. t + 5).
  auto read_ring = [&](h2 (&x)[2][16]) {
    const int jq = lane >> 4;
#pragma unroll
    for (int v = 0; v < 2; ++v)
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        h2 w[4][3];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const int m = 2 * c + r;
          const uint32_t* rp = ring + (2 * jq + (m & 1) + 8 * (m >> 1)) * L::RPW + tt + 16 * v + 3;
#pragma unroll
          for (int d = 0; d < 3; ++d) w[c][d] = __builtin_bit_cast(h2, rp[d]);
        }
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const h2* lo = w[2 * e];
          const h2* hi = w[2 * e + 1];
          x[v][2 * (4 * r + 0) + e] = __builtin_shufflevector(lo[0], hi[0], 1, 3);
          x[v][2 * (4 * r + 1) + e] = __builtin_shufflevector(lo[1], hi[1], 0, 2);
          x[v][2 * (4 * r + 2) + e] = __builtin_shufflevector(lo[1], hi[1], 1, 3);
          x[v][2 * (4 * r + 3) + e] = __builtin_shufflevector(lo[2], hi[2], 0, 2);
        }
      }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // reads done before the ring is refilled
  };
  // Stores of an item's two output rows from the run's first row pair: lane
  // offsets of pixels past the right edge (or of a row past the bottom, or of
  // a phase with nothing to store) are out of range, so the stores drop.
  int64_t run_pix = 0;
  uint32_t lane_off[2] = {kOob, kOob};
  const int n_rec = (int)(rb32 + L::OPX * PX);
  // NCHW output: lane l stores 8 pixels from 8 (l & 7) of channel
  // oc[v] = 16 (2 v + (pw >> 1)) + 4 (pw & 1) + ((l >> 3) & 3) + 8 (l >> 5).
  int oc[2];
#pragma unroll
  for (int v = 0; v < 2; ++v)
    oc[v] = 16 * (2 * v + (pw >> 1)) + 4 * (pw & 1) + ((lane >> 3) & 3) + 8 * (lane >> 5);
  const char* out_img = reinterpret_cast<const char*>(a.out);
  auto store_item = [&](bool live, int i, int SB) {
    if constexpr (OUT_NCHW) {
      const __amdgpu_buffer_rsrc_t rsw =
          __builtin_amdgcn_make_buffer_rsrc((void*)out_img, (short)0, (int)(C * plane), 0x00020000);
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const int y = 2 * (j0 + i) + r;
        const bool ok = live && y < a.H;  // uniform
#pragma unroll
        for (int v = 0; v < 2; ++v) {
          const h8 val =
              *reinterpret_cast<const h8*>(stg + SB * SBUF + (r * C + oc[v]) * L::NCS + 8 * (lane & 7));
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, val), rsw,
                                                 ok ? lane_off[v] : kOob,
                                                 ok ? (uint32_t)y * (uint32_t)a.W * 2 : 0u,
                                                 kNonTemporal);
        }
      }
      return;
    }
    const char* p = reinterpret_cast<const char*>(a.out) + run_pix * PX + (int64_t)i * (2 * row_bytes);
    const __amdgpu_buffer_rsrc_t rsw =
        __builtin_amdgcn_make_buffer_rsrc((void*)p, (short)0, n_rec, 0x00020000);
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const bool ok = live && (r == 0 || 2 * (j0 + i) + 1 < a.H);  // uniform
#pragma unroll
      for (int v = 0; v < 2; ++v) {
        const h8 val = *reinterpret_cast<const h8*>(stg + SB * SBUF + L::st(r, sx + 32 * v, sg));
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, val), rsw,
                                               ok ? lane_off[v] + (uint32_t)r * rb32 : kOob, 0,
                                               kNonTemporal);
      }
    }
  };
  h2 X[2][16];  // NCHW input: tiles tt, tt + 16
  h8 X8[8];      // padded input: tile t8
  auto phase = [&](auto k6_tag, int k, int len) {
    constexpr int K6 = decltype(k6_tag)::value;  // k % 6
    constexpr int P = K6 & 1;
    constexpr int SW = ((K6 + 1) % 3) * RPAIR;
    if constexpr (IN_NCHW) {
      // Q_{k+1} has landed in the ring (it and the previous phase's stores are
      // all this wave has in flight); read it, then request Q_{k+2}.
      if (k < len) {
        wait_vmcnt<0>();
        read_ring(X);
        if (k + 2 <= len) issue(k + 2);
      }
    }
    // Item k-2 leaves staging[(k-1)&1] = P^1, where the fold of phase k-1
    // put it.
    store_item(k >= 2, k - 2, P ^ 1);
    if (k < len) {
      if constexpr (IN_NCHW) {
#pragma unroll
        for (int v = 0; v < 2; ++v) rp_transform(vw[v] + SW, X[v]);
      } else {
        rp_transform8(vw8 + SW, X8);
        load8(X8, 2 * (j0 + k) + 4);  // Q_{k+2}: padded rows 2 (j0 + k + 2) and + 1
      }
    }
    lds_sync();
  };
  for (int it = begin; it < end;) {
    decode(it);
    const int len = min(end - it, a.tiles_h - j0);
    if constexpr (IN_NCHW) {
      const char* ib = reinterpret_cast<const char*>(a.in) + (int64_t)n * C * plane;
      rs = __builtin_amdgcn_make_buffer_rsrc((void*)ib, (short)0, (int)(C * plane), 0x00020000);
      set_copies();
    } else {
      const char* ib = reinterpret_cast<const char*>(a.in) + (int64_t)n * img_bytes;
      rs = __builtin_amdgcn_make_buffer_rsrc((void*)ib, (short)0, (int)img_bytes, 0x00020000);
      rs0 = __builtin_amdgcn_make_buffer_rsrc((void*)ib, (short)0, 0, 0x00020000);
      const int pc0 = L::OPX * s + 2 * t8;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        col_off[j] = (pc0 + j < a.Wp) ? (uint32_t)((pc0 + j) * PX + g8 * 16) : kOob;
    }
    if constexpr (OUT_NCHW) {
      out_img = reinterpret_cast<const char*>(a.out) + (int64_t)n * C * plane;
#pragma unroll
      for (int v = 0; v < 2; ++v) {
        const int x = L::OPX * s + 8 * (lane & 7);
        lane_off[v] = x < a.W ? (uint32_t)oc[v] * plane + (uint32_t)x * 2 : kOob;
      }
    } else {
#pragma unroll
      for (int v = 0; v < 2; ++v) {
        const int x = L::OPX * s + sx + 32 * v;
        lane_off[v] = x < a.W ? (uint32_t)((sx + 32 * v) * PX + sg * 16) : kOob;
      }
      run_pix = ((int64_t)n * a.Hp + 2 * j0 + 1) * a.Wp + L::OPX * s + 1;
    }
    // Prologue: Q_0 into slot 0, then the rows of Q_1 for phase 0 (NCHW input:
    // requested into the ring). Slot 0 is free: an earlier run's last fold
    // read it at least two barriers ago.
    if constexpr (IN_NCHW) {
      issue(0);
      wait_vmcnt<0>();
      read_ring(X);
      issue(1);
#pragma unroll
      for (int v = 0; v < 2; ++v) rp_transform(vw[v], X[v]);
    } else {
      load8(X8, 2 * j0);
      rp_transform8(vw8, X8);
      load8(X8, 2 * j0 + 2);
    }
    lds_sync();
    rp_phases(len, [&](auto pt, int k) { phase(pt, k, len); });
    it += len;
  }
  if constexpr (IN_NCHW) wait_vmcnt<0>();  // no copy into LDS outlives the workgroup
}

bool rowpipe_eligible(int C, int M, int nskip, int act, int64_t N, int64_t H, int64_t W,
                      int io) {
  if (C != 64 || M != 64 || nskip != 0 || io < 0 || io > 3) return false;
  if (act != kActNone && act != kActRelu && act != kActSilu) return false;
  if (N < 1 || H < 1 || W < 1) return false;
  if (io != 0 && W % 8 != 0) return false;  // 16-byte NCHW rows
  const int64_t lim = (int64_t)1 << 31;
  const int64_t img = padded_rows(H) * padded_cols(W) * 128;
  const int64_t items = N * ((W + RowPipeL::OPX - 1) / RowPipeL::OPX) * ((H + 1) / 2);
  return img < lim && 64 * H * W * 2 < lim && items < lim;
}

hipError_t launch_rowpipe(StripArgs a, int act, int io, hipStream_t s) {
  if (!rowpipe_eligible(64, 64, a.skip0 || a.skip1 ? 1 : 0, act, a.N, a.H, a.W, io))
    return hipErrorInvalidValue;
  if (block_u_offset(64, 64) != (size_t)RowPipeL::UOFF || block_u_halfs(64, 64) == 0)
    return hipErrorInvalidValue;
  a.Hp = (int32_t)padded_rows(a.H);
  a.Wp = (int32_t)padded_cols(a.W);
  a.tiles_h = (a.H + 1) / 2;
  a.n_strips = (a.W + RowPipeL::OPX - 1) / RowPipeL::OPX;
  const int64_t items = (int64_t)a.N * a.n_strips * a.tiles_h;
  a.n_items = (int32_t)items;
  a.fd_tiles_h = make_fastdiv((uint32_t)a.tiles_h);
  a.fd_strips = make_fastdiv((uint32_t)a.n_strips);
  using Fn = void (*)(StripArgs);
  static constexpr Fn table[4][3] = {
      {winograd_rowpipe<kActNone, 0>, winograd_rowpipe<kActRelu, 0>, winograd_rowpipe<kActSilu, 0>},
      {winograd_rowpipe<kActNone, 1>, winograd_rowpipe<kActRelu, 1>, winograd_rowpipe<kActSilu, 1>},
      {winograd_rowpipe<kActNone, 2>, winograd_rowpipe<kActRelu, 2>, winograd_rowpipe<kActSilu, 2>},
      {winograd_rowpipe<kActNone, 3>, winograd_rowpipe<kActRelu, 3>, winograd_rowpipe<kActSilu, 3>}};
  const Fn fn = table[io][act == kActRelu ? 1 : act == kActSilu ? 2 : 0];
  const size_t lds = RowPipeL::lds_bytes(io);
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return e;
  int64_t grid = cu_count();  // one workgroup per CU (12 waves, 128-152 KB of LDS)
  if (grid > items) grid = items;
  if (io != 0) {
    // NCHW rows are 64 separate planes: every workgroup takes the same share
    // of one strip's rows (a multiple of the strip count, and of 8 for the
    // XCD mapping), so that all of them walk the same image rows together.
    const int64_t per = (int64_t)a.N * a.n_strips;
    for (int64_t q = grid / per; q >= 1; --q)
      if ((per * q) % 8 == 0 && per * q <= items) {
        grid = per * q;
        break;
      }
  }
  grid = (grid + 7) / 8 * 8;
  hipLaunchKernelGGL(fn, dim3((unsigned)grid), dim3(RowPipeL::THREADS), lds, s, a);
  return hipGetLastError();
}

}  // namespace arthip

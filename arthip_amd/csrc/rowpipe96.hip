// A lone 96 -> 96 conv (bias, activation, at most one residual input, padded
// NHWC fp16 on both sides) with the row pipe's arithmetic: Winograd F(2,3) along x
// with the three kernel rows summed in the MFMA. One 16-channel block's row
// filters (144 VGPRs at 96 input channels) are split by position pairs over two
// waves, so that three fold waves and one load wave share each SIMD.

#include <hip/hip_runtime.h>

#include <cstdint>

#include "conv_args.h"
#include "launch.h"
#include "pack.h"
#include "wino_dev.h"

namespace arthip {

// ---------------------------------------------------------------------------
// Row-Winograd pipe at 96 channels: out = act(conv(in) + bias) (+ skip0)
// ---------------------------------------------------------------------------
//
// Items are one output tile row (two pixel rows) x 16 tiles (32 pixels),
// ordered (image, 32-pixel strip, tile row) with the tile row fastest; one
// 1024-thread workgroup per CU (16 waves, four per SIMD, 158 KB of LDS) walks
// runs of them down a strip.
//   waves 0-11 fold: wave w holds the row filters of output channels
//     16 (w % 6) .. + 15 at two positions (72 VGPRs): group 0 (w < 6)
//     positions 2 and 1, accumulating X = M2 and T = bias + M1; group 1
//     positions 0 and 3, accumulating P = M0 and Q = M3' (V3 negated). Each
//     output is then y0 = T + X + P, y1 = T - X + Q per output row.
//   waves 12-15 store the staged item of three phases before (adding the
//     residual input loaded one phase ahead), transform the next row pair
//     into a 3-slot ring of transformed row pairs (4 positions x 16 tiles x 96
//     channels per row, 224-byte tile rows) and load the rows of the pair
//     after it.
// Phase k (k = 0 .. len+2 of a run, after a prologue that transforms Q_0 into
// slot 0; Q_i = padded rows 2 (j0 + i), + 1; item i reads Q_i and Q_{i+1})
// ends with the workgroup barrier:
//   group 1: fold item k-1 from slots (k-1)%3, k%3 and write its partials
//            P, Q (fp32) to partial buffer (k-1)&1   (1 <= k <= len)
//   group 0: combine item k-2 (its X, T kept in registers since the last
//            phase, P and Q from partial buffer k&1) with the activation
//            into staging k&1 (2 <= k <= len+1), then fold item k-1
//            (1 <= k <= len)
//   load:    store item k-3 from staging (k-1)&1 with its residual input
//            (3 <= k <= len+2), load that of item k-2, transform Q_{k+1} into
//            slot (k+1)%3 and load the rows of Q_{k+2} (k < len)
// Every buffer's writer and readers are a barrier apart.
struct RowPipe96L {
  static constexpr int C = 96;
  static constexpr int PX = 2 * C;        // bytes per pixel
  static constexpr int KC = C / 32;       // 32-channel MFMA chunks
  static constexpr int TILES = 16;        // tiles per item
  static constexpr int OPX = 2 * TILES;   // output pixels per item
  static constexpr int THREADS = 1024;
  static constexpr int TROW = 112;             // halfs per tile and position (224 bytes)
  static constexpr int WPS = TILES * TROW;     // halfs per position
  static constexpr int RROW = 4 * WPS;         // halfs per transformed row
  static constexpr int RPAIR = 2 * RROW;       // halfs per ring slot
  static constexpr int NSLOT = 3;
  static constexpr int STG = NSLOT * RPAIR;    // staging after the ring
  static constexpr int SPX = 104;              // halfs per staged pixel (208 bytes)
  static constexpr int SBUF = 2 * OPX * SPX;   // halfs per staging buffer
  static constexpr int PART = STG + 2 * SBUF;  // partials after staging (halfs offset)
  static constexpr int PBUF = 6 * 4 * 64 * 4;  // floats per partial buffer
  static constexpr size_t lds_bytes() { return (size_t)PART * 2 + (size_t)2 * PBUF * 4; }
  static constexpr int STORES = 2 * OPX * (C / 8) / 256;  // 16-byte stores per load thread
  // Offset (halfs) of the row filters in a 96 -> 96 conv's packed weights.
  static constexpr int UOFF = 6 * 16 * KC * 64 * 8;
  // V' element (tile t < 16, channel c).
  __host__ __device__ static constexpr int at(int t, int c) { return t * TROW + c; }
  // Staging element (row, pixel x < 32, channel c).
  __host__ __device__ static constexpr int st(int row, int x, int c) {
    return (row * OPX + x) * SPX + c;
  }
};
static_assert(RowPipe96L::lds_bytes() <= 163840, "LDS");
static_assert(RowPipe96L::STORES * 256 == 2 * RowPipe96L::OPX * RowPipe96L::C / 8, "stores");

// Transform of one tile and one channel octet of a row pair (element 4 r + j
// of x: row r, column j, channels 8 g .. 8 g + 7) into the four positions of
// both transformed rows: V0 = d0 - d2, V1 = d1 + d2, V2 = d2 - d1,
// V3 = d3 - d1, written as 16-byte groups.
__device__ __forceinline__ void rp96_transform(_Float16* vw, const h8 (&x)[8]) {
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
      *reinterpret_cast<h8*>(vw + r * RowPipe96L::RROW + p * RowPipe96L::WPS) =
          __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    }
  }
}

// Phases k = 0 .. len + 2 of a run, six per iteration so that k % 6 (the ring
// slots and the buffer parities) is a compile-time constant.
template <class F>
__device__ __forceinline__ void rp96_phases(int len, F&& ph) {
  for (int k = 0;;) {
    ph(IntC<0>{}, k);
    if (++k > len + 2) break;
    ph(IntC<1>{}, k);
    if (++k > len + 2) break;
    ph(IntC<2>{}, k);
    if (++k > len + 2) break;
    ph(IntC<3>{}, k);
    if (++k > len + 2) break;
    ph(IntC<4>{}, k);
    if (++k > len + 2) break;
    ph(IntC<5>{}, k);
    if (++k > len + 2) break;
  }
}

template <int ACT, int NSKIP>
__global__ void __launch_bounds__(RowPipe96L::THREADS) __attribute__((amdgpu_waves_per_eu(4, 4)))
winograd_rowpipe96(StripArgs a) {
  using L = RowPipe96L;
  constexpr int PX = L::PX;
  constexpr int KC = L::KC;
  constexpr int RPAIR = L::RPAIR;
  constexpr int WPS = L::WPS;
  constexpr int RROW = L::RROW;
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
  float* const part = reinterpret_cast<float*>(plds + L::PART);

  if (wave < 12) {
    // ---------------- fold waves ---------------------------------------------
    // MFMA lane: tile tcol, B rows 8*kq.. of each 32-channel chunk, output
    // channels [ch0, ch0 + 4) of the tile's four pixels.
    const int blk = wave % 6;
    const int tcol = lane & 15;
    const int kq = lane >> 4;
    const int ch0 = 16 * blk + 4 * kq;
    const f4 bias4 = *reinterpret_cast<const f4*>(a.bias + ch0);
    const _Float16* vr[KC];
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) vr[kc] = plds + L::at(tcol, 32 * kc + 8 * kq);
    // Partial buffer entry (f4) j of this lane: P row 0, P row 1, Q row 0, Q row 1.
    auto pslot = [&](int buf, int j) { return part + (((buf * 6 + blk) * 4 + j) * 64 + lane) * 4; };
    // Staging of this lane's values: pixels 2 t, 2 t + 1 of rows 0, 1,
    // channels ch0 .. ch0 + 3.
    const int sw0 = L::st(0, 2 * tcol, ch0);
    auto role = [&](auto grp_tag) {
      constexpr int GRP = decltype(grp_tag)::value;
      // The row filters of this wave's two positions (group 0: 2, 1; group 1: 0, 3).
      constexpr int PA = GRP == 0 ? 2 : 0;
      constexpr int PB = GRP == 0 ? 1 : 3;
      h8 u[3][2][KC];
      {
        const h8* up = reinterpret_cast<const h8*>(a.u + L::UOFF) + (size_t)blk * (12 * KC * 64) + lane;
#pragma unroll
        for (int dy = 0; dy < 3; ++dy)
#pragma unroll
          for (int kc = 0; kc < KC; ++kc) {
            u[dy][0][kc] = up[((dy * 4 + PA) * KC + kc) * 64];
            u[dy][1][kc] = up[((dy * 4 + PB) * KC + kc) * 64];
          }
      }
      // The two positions' products for both output rows (row 0 reads
      // transformed rows R0..R2, row 1 R1..R3; A holds R0, R1 and B R2, R3)
      // into (a0, a1) and (b0, b1).
      auto fold = [&](int offA, int offB, f4& a0, f4& a1, f4& b0, f4& b1) {
        __builtin_amdgcn_iglp_opt(1);
        auto pos = [&](int i, int p, f4& r0, f4& r1) {
#pragma unroll
          for (int kc = 0; kc < KC; ++kc) {
            const h8 f0 = *reinterpret_cast<const h8*>(vr[kc] + offA + p * WPS);
            const h8 f1 = *reinterpret_cast<const h8*>(vr[kc] + offA + RROW + p * WPS);
            const h8 f2 = *reinterpret_cast<const h8*>(vr[kc] + offB + p * WPS);
            const h8 f3 = *reinterpret_cast<const h8*>(vr[kc] + offB + RROW + p * WPS);
            r0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(u[0][i][kc], f0, r0, 0, 0, 0);
            r1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(u[0][i][kc], f1, r1, 0, 0, 0);
            r0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(u[1][i][kc], f1, r0, 0, 0, 0);
            r1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(u[1][i][kc], f2, r1, 0, 0, 0);
            r0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(u[2][i][kc], f2, r0, 0, 0, 0);
            r1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(u[2][i][kc], f3, r1, 0, 0, 0);
          }
        };
        pos(0, PA, a0, a1);
        pos(1, PB, b0, b1);
      };
      f4 X0 = {0, 0, 0, 0}, X1 = X0, T0 = X0, T1 = X0;  // group 0: the last fold
      auto phase = [&](auto k6_tag, int k, int len) {
        constexpr int K6 = decltype(k6_tag)::value;  // k % 6
        constexpr int SA = ((K6 + 2) % 3) * RPAIR, SB = (K6 % 3) * RPAIR;
        if constexpr (GRP == 0) {
          if (k >= 2 && k <= len + 1) {
            // Item k-2: its partials went to buffer (k-2)&1 = k&1 last phase.
            const f4 P0 = *reinterpret_cast<const f4*>(pslot(K6 & 1, 0));
            const f4 P1 = *reinterpret_cast<const f4*>(pslot(K6 & 1, 1));
            const f4 Q0 = *reinterpret_cast<const f4*>(pslot(K6 & 1, 2));
            const f4 Q1 = *reinterpret_cast<const f4*>(pslot(K6 & 1, 3));
            _Float16* sw = stg + (K6 & 1) * L::SBUF + sw0;
            *reinterpret_cast<h4*>(sw) = strip_act4<ACT>(T0 + X0 + P0);
            *reinterpret_cast<h4*>(sw + L::SPX) = strip_act4<ACT>(T0 - X0 + Q0);
            *reinterpret_cast<h4*>(sw + L::OPX * L::SPX) = strip_act4<ACT>(T1 + X1 + P1);
            *reinterpret_cast<h4*>(sw + (L::OPX + 1) * L::SPX) = strip_act4<ACT>(T1 - X1 + Q1);
          }
          if (k >= 1 && k <= len) {
            X0 = f4{0, 0, 0, 0};
            X1 = X0;
            T0 = bias4;
            T1 = bias4;
            fold(SA, SB, X0, X1, T0, T1);
          }
        } else {
          if (k >= 1 && k <= len) {
            f4 P0 = {0, 0, 0, 0}, P1 = P0, Q0 = P0, Q1 = P0;
            fold(SA, SB, P0, P1, Q0, Q1);
            // Item k-1 into buffer (k-1)&1.
            constexpr int B = (K6 + 1) & 1;
            *reinterpret_cast<f4*>(pslot(B, 0)) = P0;
            *reinterpret_cast<f4*>(pslot(B, 1)) = P1;
            *reinterpret_cast<f4*>(pslot(B, 2)) = Q0;
            *reinterpret_cast<f4*>(pslot(B, 3)) = Q1;
          }
        }
        lds_sync();
      };
      for (int it = begin; it < end;) {
        decode(it);
        const int len = min(end - it, a.tiles_h - j0);
        lds_sync();  // the prologue
        rp96_phases(len, [&](auto pt, int k) { phase(pt, k, len); });
        it += len;
      }
    };
    if (wave < 6)
      role(IntC<0>{});
    else
      role(IntC<1>{});
    return;
  }

  // ---------------- load, transform and store waves ---------------------------
  // Transform tasks (lanes 0-47 of each load wave): tile t8 = l & 15 and
  // channel octet g8 = 3 (wave - 12) + {0, 2, 1}[l >> 4], so that lanes l and
  // l + 32, whose 16-byte writes the LDS serves together, take octets of
  // opposite parity (with 224-byte tile rows, 8 tiles x 2 such octets cover
  // the 16 bank groups). Store task i of a load thread: 16-byte group
  // q = gtid + 256 i of the item, row q / 384, pixel (q % 384) / 12, group
  // q % 12.
  const int gtid = tid - 768;
  const bool has_task = lane < 48;
  const int t8 = lane & 15;
  const int g8 = 3 * (wave - 12) + ((lane >> 4) == 1 ? 2 : (lane >> 5));
  _Float16* const vw = plds + L::at(t8, 8 * g8);
  // Input patch of tile t8: padded columns pc0 .. pc0 + 3 with pc0 = 32 s +
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
  // Stores (and residual loads) of item i of the run: buffer resources from
  // the run's first output pixel; lane offsets of pixels past the right edge,
  // of the second row past the bottom, or of a phase with nothing to store are
  // out of range (dropped stores, zero loads).
  int64_t run_pix = 0;
  const int n_rec = (int)(rb32 + L::OPX * PX);
  int st_r[L::STORES], st_x[L::STORES], st_g[L::STORES];
  uint32_t st_lane[L::STORES];
#pragma unroll
  for (int i = 0; i < L::STORES; ++i) {
    const int q = gtid + 256 * i;
    st_r[i] = q / 384;
    st_x[i] = (q % 384) / 12;
    st_g[i] = q % 12;
  }
  auto item_rsrc = [&](const void* base, int i) {
    const char* p = reinterpret_cast<const char*>(base) + run_pix * PX + (int64_t)i * (2 * row_bytes);
    return __builtin_amdgcn_make_buffer_rsrc((void*)p, (short)0, n_rec, 0x00020000);
  };
  auto st_off = [&](bool live, int i, int e) -> uint32_t {
    const bool ok = live && (st_r[e] == 0 || 2 * (j0 + i) + 1 < a.H);
    return ok ? st_lane[e] : kOob;
  };
  h8 skr[L::STORES];
  auto load_skip = [&](bool live, int i) {
    if constexpr (NSKIP > 0) {
      const __amdgpu_buffer_rsrc_t rk = item_rsrc(a.skip0, i);
#pragma unroll
      for (int e = 0; e < L::STORES; ++e)
        skr[e] = __builtin_bit_cast(
            h8, __builtin_amdgcn_raw_buffer_load_b128(rk, st_off(live, i, e), 0, kNonTemporal));
    }
  };
  auto store_item = [&](bool live, int i, int SB) {
    const __amdgpu_buffer_rsrc_t rw = item_rsrc(a.out, i);
#pragma unroll
    for (int e = 0; e < L::STORES; ++e) {
      h8 v = *reinterpret_cast<const h8*>(stg + SB * L::SBUF + L::st(st_r[e], st_x[e], 8 * st_g[e]));
      if constexpr (NSKIP > 0) v += skr[e];
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, v), rw, st_off(live, i, e), 0,
                                             kNonTemporal);
    }
  };
  h8 X8[8];
  auto phase = [&](auto k6_tag, int k, int len) {
    constexpr int K6 = decltype(k6_tag)::value;  // k % 6
    constexpr int SW = ((K6 + 1) % 3) * RPAIR;
    // Item k-3 leaves staging (k-3)&1 = (k-1)&1, where group 0 put it last
    // phase, with its residual input loaded last phase; then that of item k-2.
    store_item(k >= 3, k - 3, (K6 + 1) & 1);
    load_skip(k >= 2 && k <= len + 1, k - 2);
    if (has_task && k < len) {
      rp96_transform(vw + SW, X8);
      load8(X8, 2 * (j0 + k) + 4);  // Q_{k+2}: padded rows 2 (j0 + k + 2) and + 1
    }
    lds_sync();
  };
  for (int it = begin; it < end;) {
    decode(it);
    const int len = min(end - it, a.tiles_h - j0);
    const char* ib = reinterpret_cast<const char*>(a.in) + (int64_t)n * img_bytes;
    rs = __builtin_amdgcn_make_buffer_rsrc((void*)ib, (short)0, (int)img_bytes, 0x00020000);
    rs0 = __builtin_amdgcn_make_buffer_rsrc((void*)ib, (short)0, 0, 0x00020000);
    const int pc0 = L::OPX * s + 2 * t8;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      col_off[j] = (pc0 + j < a.Wp) ? (uint32_t)((pc0 + j) * PX + g8 * 16) : kOob;
#pragma unroll
    for (int e = 0; e < L::STORES; ++e)
      st_lane[e] = (L::OPX * s + st_x[e] < a.W)
                       ? (uint32_t)(st_r[e] * rb32 + st_x[e] * PX + st_g[e] * 16)
                       : kOob;
    run_pix = ((int64_t)n * a.Hp + 2 * j0 + 1) * a.Wp + L::OPX * s + 1;
    // Prologue: Q_0 into slot 0, then the rows of Q_1 for phase 0. Slot 0 is
    // free: an earlier run's last fold read it at least two barriers ago.
    if (has_task) {
      load8(X8, 2 * j0);
      rp96_transform(vw, X8);
      load8(X8, 2 * j0 + 2);
    }
    lds_sync();
    rp96_phases(len, [&](auto pt, int k) { phase(pt, k, len); });
    it += len;
  }
}

bool rowpipe96_eligible(int C, int M, int nskip, int act, int64_t N, int64_t H, int64_t W,
                        int io) {
  if (C != 96 || M != 96 || nskip < 0 || nskip > 1 || io != 0) return false;
  if (act != kActNone && act != kActRelu && act != kActSilu) return false;
  if (N < 1 || H < 1 || W < 1) return false;
  const int64_t lim = (int64_t)1 << 31;
  const int64_t img = padded_rows(H) * padded_cols(W) * 2 * RowPipe96L::C;
  const int64_t items = N * ((W + RowPipe96L::OPX - 1) / RowPipe96L::OPX) * ((H + 1) / 2);
  return img < lim && items < lim;
}

hipError_t launch_rowpipe96(StripArgs a, int act, hipStream_t s) {
  const int nskip = (a.skip0 != nullptr) + (a.skip1 != nullptr);
  if (!rowpipe96_eligible(96, 96, nskip, act, a.N, a.H, a.W, 0)) return hipErrorInvalidValue;
  if (block_u_offset(96, 96) != (size_t)RowPipe96L::UOFF || block_u_halfs(96, 96) == 0)
    return hipErrorInvalidValue;
  a.Hp = (int32_t)padded_rows(a.H);
  a.Wp = (int32_t)padded_cols(a.W);
  a.tiles_h = (a.H + 1) / 2;
  a.n_strips = (a.W + RowPipe96L::OPX - 1) / RowPipe96L::OPX;
  const int64_t items = (int64_t)a.N * a.n_strips * a.tiles_h;
  a.n_items = (int32_t)items;
  a.fd_tiles_h = make_fastdiv((uint32_t)a.tiles_h);
  a.fd_strips = make_fastdiv((uint32_t)a.n_strips);
  using Fn = void (*)(StripArgs);
  static constexpr Fn table[2][3] = {
      {winograd_rowpipe96<kActNone, 0>, winograd_rowpipe96<kActRelu, 0>, winograd_rowpipe96<kActSilu, 0>},
      {winograd_rowpipe96<kActNone, 1>, winograd_rowpipe96<kActRelu, 1>, winograd_rowpipe96<kActSilu, 1>}};
  const Fn fn = table[nskip][act == kActRelu ? 1 : act == kActSilu ? 2 : 0];
  const size_t lds = RowPipe96L::lds_bytes();
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return e;
  int64_t grid = cu_count();  // one workgroup per CU (16 waves, 158 KB of LDS)
  if (grid > items) grid = items;
  grid = (grid + 7) / 8 * 8;
  hipLaunchKernelGGL(fn, dim3((unsigned)grid), dim3(RowPipe96L::THREADS), lds, s, a);
  return hipGetLastError();
}

}  // namespace arthip

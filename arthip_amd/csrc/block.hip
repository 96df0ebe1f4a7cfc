// Fused residual block kernels: a residual block's two 64 -> 64 convs in one
// launch, the intermediate tensor kept in LDS (see the comment on BlockL), and
// their host launcher.

#include <hip/hip_runtime.h>

#include <cstdint>

#include "conv_args.h"
#include "launch.h"
#include "pack.h"
#include "wino_dev.h"

namespace arthip {

// ---------------------------------------------------------------------------
// Fused residual block: two 64 -> 64 convs in one kernel (C = M = 64)
// ---------------------------------------------------------------------------
//
//   t   = act1(conv1(in) + bias1)             (fp16, never written to HBM)
//   out = act2(conv2(t) + bias2) + skip0 + skip1
//
// Both convs run Winograd F(2,3) along x and the three kernel rows directly
// along y: for an output row y and a tile of two pixels (2t, 2t + 1),
//   M_p = sum_dy sum_c U_dy[p][m][c] V_{y-1+dy}[p][c][t]    (p = 0..3)
//   out(y, 2t) = M_0 + M_1 + M_2,  out(y, 2t + 1) = M_1 - M_2 - M_3
// with V_r[p] = B^T d the 1-D transform of input row r (pixels 2t-1 .. 2t+2)
// and U_dy = G g_dy that of kernel row dy (block_u_halfs). The MFMA sums over
// dy and the channels, so a tile row needs 48 MFMAs per 16 output channels
// (against 32 for F(2x2,3x3)) but each transformed input row serves the three
// output rows that read it, the input transform is 8 packed ops per row and
// channel quad, and U' of one conv takes 96 VGPRs per wave instead of 128.
//
// One 768-thread workgroup per CU (12 waves, three per SIMD, 128 KB of LDS)
// walks down an output strip of 30 pixels (15 tiles), one output tile row
// per phase. The three waves of a SIMD do different jobs, so that one wave's
// memory and VALU work runs beside the other two waves' MFMA chains:
//   waves 0-3  (conv1 fold) hold U1' of 16 output channels each and fold t
//              for the 32 columns the strip's conv2 tiles read (16 tiles at
//              column offset -1), one t tile row (2 t rows) per phase, into a
//              2-slot LDS ring; t outside the image is stored as zero, which
//              is conv2's padding;
//   waves 4-7  (conv2 fold) hold U2' and fold 16 tiles of which the first 15
//              are the strip's outputs into staging;
//   waves 8-11 load the input rows, transform them and the t rows from the
//              ring, and store the staged rows a phase later with the residual
//              inputs added.
// U' of one conv takes 96 VGPRs per wave, which leaves the fold waves room in
// the 168 VGPRs of three waves per SIMD (F(2x2,3x3)'s 128 did not: the folds
// spilled).
//
// Transformed rows live in two 3-slot LDS rings (V1 for conv1's input, V2 for
// t), a slot holding one row pair (4 positions x 16 tiles x 64 channels per
// row). A fold of output tile row i reads row pairs i and i + 1 (rows 2i - 1
// .. 2i + 2); each fragment read serves both output rows that use it.
//
// conv1's tiles sit at odd column offsets (t columns 30 s - 1 + 2 k), where a
// separate launch tiles at even ones, so t, and the block output, agree with
// two separate launches to fp16 rounding rather than bit for bit. The offsets
// are fixed relative to the image, so results do not depend on the strip or
// workgroup that computes them. HBM traffic per block is the input once (plus
// the 2-column halo of each strip, mostly cache hits), the residual inputs and
// the output.
//
// Per run (one strip, output tile rows j0 .. j0+len-1; input row pair Q_i =
// padded rows 2(j0+i)-1, 2(j0+i); t tile row i covers t rows 2(j0+i)-1 and
// 2(j0+i), i = 0 .. len), after a prologue that transforms Q_0 into V1 slot
// 0 and a barrier, phase k (k = 0 .. len+4) ends with the workgroup barrier:
//   conv1 waves:     fold t_{k-1} from V1 slots (k-1)%3, k%3 into ring slot
//                    (k-1)&1 (1 <= k <= len+1)
//   conv2 waves:     fold output row k-4 from V2 slots (k-1)%3, k%3 (rows of
//                    t_{k-4}, t_{k-3}) into staging[k&1] (4 <= k <= len+3)
//   load and store   read t_{k-2} from ring slot k&1 (2 <= k <= len+2); store
//   waves:           output row k-5 from staging[(k-5)&1] with its residuals
//                    (k >= 5) and load the residuals of row k-4; transform
//                    Q_{k+1} into V1 slot (k+1)%3 (k <= len) and load the
//                    input rows of Q_{k+2}; transform t_{k-2} into V2 slot
//                    (k+1)%3 (2 <= k <= len+2)
// Every buffer's writer and readers are a barrier apart.
struct BlockL {
  static constexpr int C = 64;
  static constexpr int PX = 2 * C;                // bytes per pixel
  static constexpr int OTILES = 15;               // output tiles per strip
  static constexpr int OPX = 2 * OTILES;          // output pixels per strip
  static constexpr int WPS = StripLds<2>::WPS;    // halfs per position (16 tiles)
  static constexpr int RROW = 4 * WPS;            // halfs per transformed row
  static constexpr int RPAIR = 2 * RROW;          // halfs per ring slot (row pair)
  static constexpr int NSLOT = 3;
  static constexpr int THREADS = 768;             // 12 waves, three per SIMD
  static constexpr int SBUF = StripStage<2>::SBUF;
  static constexpr int RSLOT = 2 * 32 * C;        // halfs per t ring slot (2 t rows x 32 px)
  // t ring: pixel pairs m = x >> 1 take 256 bytes, the two pixels' halves
  // swapped on odd m, and the 8-byte channel quads of the pair XORed with m.
  // The conv1 folds' writes (16 tiles, one pixel and quad each) and the conv2
  // reads (2 tiles x 16 quads per 32 lanes) then both hit distinct banks.
  __host__ __device__ static constexpr int at(int row, int x, int q) {
    return row * 32 * C + (x >> 1) * 128 + (((x & 1) ^ ((x >> 1) & 1)) << 6) +
           ((q ^ ((x >> 1) & 15)) << 2);
  }
  // Offset (halfs) of the row filters in a 64 -> 64 conv's packed weights:
  // after U' (4 channel blocks x 16 positions x 2 chunks x 64 lanes x 8).
  static constexpr int UOFF = 4 * 16 * 2 * 64 * 8;
  static constexpr int V1 = 0;
  static constexpr int V2 = NSLOT * RPAIR;
  static constexpr int RING = 2 * NSLOT * RPAIR;
  static constexpr int STG = RING + 2 * RSLOT;
  static constexpr size_t lds_bytes() { return (size_t)(STG + 2 * SBUF) * 2; }
};

// 1-D transform of rows r = 0, 1 of a task's row pair (element 2 (4 r + j) + e
// of x: column j, channel pair e) into positions p of a transformed row:
// V0 = d0 - d2, V1 = d1 + d2, V2 = d2 - d1, V3 = d3 - d1 (the last negated
// against B^T; the fold's chain absorbs it).
__device__ __forceinline__ void row_pair_transform(_Float16* vw, const h2 (&x)[16]) {
  constexpr int WPS = BlockL::WPS;
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
      *reinterpret_cast<h4*>(vw + r * BlockL::RROW + p * WPS) =
          __builtin_shufflevector(o[p][0], o[p][1], 0, 1, 2, 3);
  }
}

// Fold of one tile row (two output rows) x 16 output channels (one wave) from
// transformed row pairs A (rows R0, R1) and B (R2, R3) at vr[kc] + offA / offB:
// output row 0 reads R0..R2 (dy = 0..2), row 1 R1..R3. Chains per output row
// (the accumulator carries them): X = M2, b = X + bias + M1, P = b + M0 and
// c = b + M3' (M3' = -M3 from the negated V3); y0 = P, y1 = c - 2 X.
__device__ __forceinline__ void block_fold(const h8 (&u)[3][4][2], const _Float16* const (&vr)[2],
                                           int offA, int offB, f4 bias4, f4& y00, f4& y01,
                                           f4& y10, f4& y11) {
  constexpr int WPS = BlockL::WPS;
  constexpr int RROW = BlockL::RROW;
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

// Phases k = 0 .. len + 4 of one run, six per iteration so that k % 6, and
// with it the t ring and staging parity and the three row-pair slots, is a
// compile-time constant (every LDS offset an immediate): ph(k6_tag, k).
template <class F>
__device__ __forceinline__ void block_phases(int len, F&& ph) {
  for (int k = 0;;) {
    ph(IntC<0>{}, k);
    if (++k > len + 4) break;
    ph(IntC<1>{}, k);
    if (++k > len + 4) break;
    ph(IntC<2>{}, k);
    if (++k > len + 4) break;
    ph(IntC<3>{}, k);
    if (++k > len + 4) break;
    ph(IntC<4>{}, k);
    if (++k > len + 4) break;
    ph(IntC<5>{}, k);
    if (++k > len + 4) break;
  }
}

template <int ACT1, int ACT2, int NSKIP, bool kCachedOut>
__global__ void __launch_bounds__(BlockL::THREADS) __attribute__((amdgpu_waves_per_eu(3, 3)))
winograd_block(BlockArgs a) {
  using L = BlockL;
  constexpr int C = L::C;
  constexpr int PX = L::PX;
  constexpr int SBUF = L::SBUF;
  constexpr int RPAIR = L::RPAIR;
  constexpr uint32_t kOob = 0x80000000u;
  extern __shared__ __attribute__((aligned(16))) _Float16 blds[];
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
  // MFMA lane of the fold waves: tile tcol, B rows 8*kq.. of each 32-channel
  // chunk, output channels [ch0, ch0 + 4) of the tile's four pixels.
  const int grp = wave & 3;  // 16-channel block within the conv
  const int tcol = lane & 15;
  const int kq = lane >> 4;
  const int ch0 = 16 * grp + 4 * kq;

  if (wave < 8) {
    // ---------------- fold waves ---------------------------------------------
    const bool c1 = wave < 4;
    // U' of this wave: [dy][position][kc], 16 output channels.
    h8 u[3][4][2];
    {
      const h8* up = reinterpret_cast<const h8*>((c1 ? a.u1 : a.u2) + L::UOFF) +
                     (size_t)grp * (12 * 2 * 64) + lane;
#pragma unroll
      for (int dy = 0; dy < 3; ++dy)
#pragma unroll
        for (int p = 0; p < 4; ++p)
#pragma unroll
          for (int kc = 0; kc < 2; ++kc) u[dy][p][kc] = up[((dy * 4 + p) * 2 + kc) * 64];
    }
    const f4 bias4 = *reinterpret_cast<const f4*>((c1 ? a.bias1 : a.bias2) + ch0);
    const int vbase = c1 ? L::V1 : L::V2;
    const _Float16* vr[2];
#pragma unroll
    for (int kc = 0; kc < 2; ++kc) vr[kc] = blds + vbase + StripLds<2>::at(tcol, 32 * kc + 8 * kq);
    if (c1) {
      // ---------------- conv1: V1 -> t ring ------------------------------------
      _Float16* const ring = blds + L::RING;
      // Ring offsets of this lane's four t values (pixel rows 0/1, columns
      // 2 tcol / 2 tcol + 1, channel quad 4 grp + kq).
      int rw[4];
      {
        const int q = 4 * grp + kq;
        rw[0] = L::at(0, 2 * tcol, q);
        rw[1] = L::at(0, 2 * tcol + 1, q);
        rw[2] = L::at(1, 2 * tcol, q);
        rw[3] = L::at(1, 2 * tcol + 1, q);
      }
      // Lane masks (all ones or zero) of this lane's two t columns, per run.
      uint32_t cm0 = 0, cm1 = 0;
      auto phase = [&](auto k6_tag, int k, int len) {
        constexpr int K6 = decltype(k6_tag)::value;  // k % 6
        constexpr int P = K6 & 1;
        constexpr int SA = ((K6 + 2) % 3) * RPAIR, SB = (K6 % 3) * RPAIR;
        if (k >= 1 && k <= len + 1) {
          // Fold t_{k-1}: t rows 2 (j0 + k - 1) - 1 + r, t columns 30 s - 1 + 2 tcol + dx.
          f4 y00, y01, y10, y11;
          block_fold(u, vr, SA, SB, bias4, y00, y01, y10, y11);
          const int tr0 = 2 * (j0 + k - 1) - 1;
          const uint32_t rm0 = (tr0 >= 0 && tr0 < a.H) ? ~0u : 0u;  // uniform
          const uint32_t rm1 = (tr0 + 1 < a.H) ? ~0u : 0u;
          // t outside the image is stored as zero (bitwise, so that no branch
          // splits the phase).
          // SiLU per element: interleaving the four chains here measured
          // slower for the block (226 -> 230 us) while it pays in the pipes.
          auto masked = [&](f4 y, uint32_t m) {
            u2 b = __builtin_bit_cast(u2, strip_act4<ACT1, false>(y));
            b &= u2{m, m};
            return b;
          };
          _Float16* sl = ring + (P ^ 1) * L::RSLOT;
          *reinterpret_cast<u2*>(sl + rw[0]) = masked(y00, rm0 & cm0);
          *reinterpret_cast<u2*>(sl + rw[1]) = masked(y01, rm0 & cm1);
          *reinterpret_cast<u2*>(sl + rw[2]) = masked(y10, rm1 & cm0);
          *reinterpret_cast<u2*>(sl + rw[3]) = masked(y11, rm1 & cm1);
        }
        lds_sync();
      };
      for (int it = begin; it < end;) {
        decode(it);
        const int len = min(end - it, a.tiles_h - j0);
        const int tc0 = L::OPX * s - 1 + 2 * tcol;
        cm0 = (tc0 >= 0 && tc0 < a.W) ? ~0u : 0u;
        cm1 = (tc0 + 1 < a.W) ? ~0u : 0u;
        lds_sync();  // the prologue's transform of Q_0
        block_phases(len, [&](auto pt, int k) { phase(pt, k, len); });
        it += len;
      }
      return;
    }
    // ---------------- conv2: V2 -> staging ------------------------------------
    _Float16* const stg = blds + L::STG;
    const int sw0 = StripStage<2>::at(0, 2 * tcol, ch0 >> 3) + (ch0 & 7);
    auto phase = [&](auto k6_tag, int k, int len) {
      constexpr int K6 = decltype(k6_tag)::value;  // k % 6
      constexpr int P = K6 & 1;
      constexpr int SA = ((K6 + 2) % 3) * RPAIR, SB = (K6 % 3) * RPAIR;
      if (k >= 4 && k <= len + 3) {
        f4 y00, y01, y10, y11;
        block_fold(u, vr, SA, SB, bias4, y00, y01, y10, y11);
        _Float16* sw = stg + P * SBUF + sw0;
        *reinterpret_cast<h4*>(sw) = strip_act4<kActNone>(y00);
        *reinterpret_cast<h4*>(sw + C) = strip_act4<kActNone>(y01);
        *reinterpret_cast<h4*>(sw + 32 * C) = strip_act4<kActNone>(y10);
        *reinterpret_cast<h4*>(sw + 33 * C) = strip_act4<kActNone>(y11);
      }
      lds_sync();
    };
    for (int it = begin; it < end;) {
      decode(it);
      const int len = min(end - it, a.tiles_h - j0);
      lds_sync();  // the prologue
      block_phases(len, [&](auto pt, int k) { phase(pt, k, len); });
      it += len;
    }
    return;
  }

  // ---------------- load, transform and store waves ---------------------------
  // Transform task (both transforms): tile tt, channel quad tq. Store task:
  // 16-byte group sg of pixel sx in both rows of an output row pair.
  const int gtid = tid - 512;
  const int tt = gtid >> 4;
  const int tq = gtid & 15;
  _Float16* const stg = blds + L::STG;
  const int sx = gtid >> 3;
  const int sg = gtid & 7;
  const int sr0 = StripStage<2>::at(0, sx, sg);
  const uint32_t s_lane = (uint32_t)(sx * C + sg * 8) * 2;
  const int n_rec = (int)(rb32 + 32 * PX);
  h8 skr[2][2];
  // Buffer resources over output row pair o's first pixel of the strip, from
  // the run's first row pair (byte offset of o: (o - j0) * 2 row_bytes). Lane
  // offsets past the strip or the right edge, of the second row past the
  // bottom, or of a phase with nothing to store are out of range: dropped
  // stores, zero loads.
  int64_t run_pix = 0;
  uint32_t lane_off = kOob;
  auto row_rsrc = [&](const void* base, int o) {
    const char* p = reinterpret_cast<const char*>(base) + run_pix * PX +
                    (int64_t)(o - j0) * (2 * row_bytes);
    return __builtin_amdgcn_make_buffer_rsrc((void*)p, (short)0, n_rec, 0x00020000);
  };
  auto st_off = [&](bool live, int o, int r) -> uint32_t {
    const bool ok = live && (r == 0 || 2 * o + 1 < a.H);
    return ok ? lane_off + (uint32_t)r * rb32 : kOob;
  };
  auto load_skips = [&](bool live, int o) {
#pragma unroll
    for (int k = 0; k < 2; ++k)
#pragma unroll
      for (int r = 0; r < 2; ++r) skr[k][r] = h8{0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int k = 0; k < NSKIP; ++k) {
      const __amdgpu_buffer_rsrc_t rs = row_rsrc(k == 0 ? a.skip0 : a.skip1, o);
#pragma unroll
      for (int r = 0; r < 2; ++r)
        skr[k][r] = __builtin_bit_cast(
            h8, __builtin_amdgcn_raw_buffer_load_b128(rs, st_off(live, o, r), 0, kNonTemporal));
    }
  };
  auto store_row = [&](bool live, int o, int SB) {
    const __amdgpu_buffer_rsrc_t rs = row_rsrc(a.out, o);
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      h8 v = act8<ACT2>(*reinterpret_cast<const h8*>(stg + SB * SBUF + sr0 + r * 32 * C));
      if (NSKIP > 0) v += skr[0][r];
      if (NSKIP > 1) v += skr[1][r];
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, v), rs, st_off(live, o, r), 0,
                                             kCachedOut ? 0 : kNonTemporal);
    }
  };
  _Float16* const vw1 = blds + L::V1 + StripLds<2>::at(tt, 4 * tq);
  _Float16* const vw2 = blds + L::V2 + StripLds<2>::at(tt, 4 * tq);
  // Input patch of t tile tt: padded columns pc0 .. pc0 + 3 with
  // pc0 = 30 s - 1 + 2 tt, 8 bytes of channel quad tq each. The row goes in
  // the instruction's scalar offset; columns outside the padded row get an
  // out-of-range lane offset and rows outside the image a zero-size
  // resource, both of which read as zero.
  const int64_t img_bytes = (int64_t)a.Hp * row_bytes;
  __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)a.in, (short)0, 0, 0x00020000);
  __amdgpu_buffer_rsrc_t rs0 = rs;
  uint32_t col_off[4];
  auto load2 = [&](h2 (&x)[16], int pr) {
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const bool row_ok = (pr + r >= 0) && (pr + r < a.Hp);
      const __amdgpu_buffer_rsrc_t rr = row_ok ? rs : rs0;
      const uint32_t ro = row_ok ? (uint32_t)(pr + r) * rb32 : 0u;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const h4 v =
            __builtin_bit_cast(h4, __builtin_amdgcn_raw_buffer_load_b64(rr, col_off[j], ro, 0));
        x[2 * (4 * r + j)] = __builtin_shufflevector(v, v, 0, 1);
        x[2 * (4 * r + j) + 1] = __builtin_shufflevector(v, v, 2, 3);
      }
    }
  };
  // Ring pixels of this task's patch: 2 tt .. 2 tt + 3 (tile 15 is not an
  // output of the strip; it reads tile 14's patch). Row 0 addresses of the
  // four pixels; row 1 and the slot are immediate offsets from them.
  const _Float16* const ring = blds + L::RING;
  const _Float16* rp[4];
  {
    const int rx0 = 2 * (tt < L::OTILES ? tt : L::OTILES - 1);
#pragma unroll
    for (int j = 0; j < 4; ++j) rp[j] = ring + L::at(0, rx0 + j, tq);
  }
  // Tile 15 is folded by conv2 (the MFMA takes 16 tiles) but never stored: its
  // transformed input is zero, which the matrix units multiply at less power
  // than a copy of tile 14.
  const uint32_t tmask = tt < L::OTILES ? ~0u : 0u;
  auto ring_load2 = [&](h2 (&x)[16], int sl) {
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        u2 b = *reinterpret_cast<const u2*>(rp[j] + sl * L::RSLOT + r * 32 * C);
        b &= u2{tmask, tmask};
        const h4 v = __builtin_bit_cast(h4, b);
        x[2 * (4 * r + j)] = __builtin_shufflevector(v, v, 0, 1);
        x[2 * (4 * r + j) + 1] = __builtin_shufflevector(v, v, 2, 3);
      }
  };
  h2 X[16];  // input rows of the next row pair to transform
  h2 T[16];  // the t rows read from the ring this phase
  auto phase = [&](auto k6_tag, int k, int len) {
    constexpr int K6 = decltype(k6_tag)::value;  // k % 6
    constexpr int P = K6 & 1;
    constexpr int SW = ((K6 + 1) % 3) * RPAIR;
    // t_{k-2} from ring slot k&1, read first so that it lands during the
    // store and the input transform.
    const bool tr = k >= 2 && k <= len + 2;
    if (tr) ring_load2(T, P);
    // Output row k-5 leaves staging (k-5)&1 = P^1 (the conv2 fold of the last
    // phase) with the residuals loaded last phase; then the residuals of row
    // k-4 (folded this phase, stored next phase).
    store_row(k >= 5, j0 + k - 5, P ^ 1);
    load_skips(k >= 4 && k <= len + 3, j0 + k - 4);
    if (k <= len) {
      row_pair_transform(vw1 + SW, X);
      // Q_{k+2}: padded rows 2 (j0 + k + 2) - 1 and 2 (j0 + k + 2).
      load2(X, 2 * (j0 + k) + 3);
    }
    if (tr) row_pair_transform(vw2 + SW, T);
    lds_sync();
  };
  for (int it = begin; it < end;) {
    decode(it);
    const int len = min(end - it, a.tiles_h - j0);
    {
      const char* ib = reinterpret_cast<const char*>(a.in) + (int64_t)n * img_bytes;
      rs = __builtin_amdgcn_make_buffer_rsrc((void*)ib, (short)0, (int)img_bytes, 0x00020000);
      rs0 = __builtin_amdgcn_make_buffer_rsrc((void*)ib, (short)0, 0, 0x00020000);
      const int pc0 = L::OPX * s - 1 + 2 * tt;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const bool ok = (pc0 + j >= 0) && (pc0 + j < a.Wp);
        col_off[j] = ok ? (uint32_t)((pc0 + j) * PX + tq * 8) : kOob;
      }
      run_pix = ((int64_t)n * a.Hp + 2 * j0 + 1) * a.Wp + L::OPX * s + 1;
      lane_off = (sx < L::OPX && L::OPX * s + sx < a.W) ? s_lane : kOob;
    }
    // Prologue: Q_0 (padded rows 2 j0 - 1, 2 j0) into V1 slot 0, then the
    // rows of Q_1 for phase 0. Slot 0 is free: the last fold of an earlier
    // run read it at least three barriers ago.
    load2(X, 2 * j0 - 1);
    row_pair_transform(vw1, X);
    load2(X, 2 * j0 + 1);
    lds_sync();  // every role: the prologue's barrier
    block_phases(len, [&](auto pt, int k) { phase(pt, k, len); });
    it += len;
  }
}

// ---------------------------------------------------------------------------
// Host launcher
// ---------------------------------------------------------------------------

using BlockKernel = void (*)(BlockArgs);

template <int ACT1, bool kCachedOut>
BlockKernel block_kernel_for(int nskip) {
  switch (nskip) {
    case 0: return winograd_block<ACT1, kActNone, 0, kCachedOut>;
    case 1: return winograd_block<ACT1, kActNone, 1, kCachedOut>;
    default: return winograd_block<ACT1, kActNone, 2, kCachedOut>;
  }
}

template <int ACT1>
BlockKernel block_kernel_for(int nskip, bool cached_out) {
  return cached_out ? block_kernel_for<ACT1, true>(nskip) : block_kernel_for<ACT1, false>(nskip);
}

bool block_eligible(int C, int M, int act1, int act2, int64_t N, int64_t H, int64_t W) {
  if (C != 64 || M != 64 || act2 != kActNone) return false;
  if (act1 != kActNone && act1 != kActRelu && act1 != kActSilu) return false;
  if (N < 1 || H < 1 || W < 1) return false;
  // The input image goes through a buffer resource with a 32-bit size.
  const int64_t img = padded_rows(H) * padded_cols(W) * 128;
  const int64_t items = N * ((W + BlockL::OPX - 1) / BlockL::OPX) * ((H + 1) / 2);
  return img < ((int64_t)1 << 31) && items < ((int64_t)1 << 31);
}

hipError_t launch_block(BlockArgs a, hipStream_t s) {
  if (!block_eligible(64, 64, a.act1, a.act2, a.N, a.H, a.W)) return hipErrorInvalidValue;
  // The kernel finds the row filters at a fixed offset of the packed weights.
  if (block_u_offset(64, 64) != (size_t)BlockL::UOFF || block_u_halfs(64, 64) == 0)
    return hipErrorInvalidValue;
  if (a.skip0 == nullptr && a.skip1 != nullptr) {
    a.skip0 = a.skip1;
    a.skip1 = nullptr;
  }
  const int nskip = (a.skip0 != nullptr) + (a.skip1 != nullptr);
  a.Hp = (int32_t)padded_rows(a.H);
  a.Wp = (int32_t)padded_cols(a.W);
  a.tiles_h = (a.H + 1) / 2;
  a.n_strips = (a.W + BlockL::OPX - 1) / BlockL::OPX;
  const int64_t items = (int64_t)a.N * a.n_strips * a.tiles_h;
  a.n_items = (int32_t)items;
  a.fd_tiles_h = make_fastdiv((uint32_t)a.tiles_h);
  a.fd_strips = make_fastdiv((uint32_t)a.n_strips);
  const bool cached = a.cached_out != 0;
  const BlockKernel fn = a.act1 == kActRelu   ? block_kernel_for<kActRelu>(nskip, cached)
                         : a.act1 == kActSilu ? block_kernel_for<kActSilu>(nskip, cached)
                                              : block_kernel_for<kActNone>(nskip, cached);
  const size_t lds = BlockL::lds_bytes();
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return e;
  int64_t grid = cu_count();  // one workgroup per CU (12 waves, 128 KB of LDS)
  if (grid > items) grid = items;
  grid = (grid + 7) / 8 * 8;
  hipLaunchKernelGGL(fn, dim3((unsigned)grid), dim3(BlockL::THREADS), lds, s, a);
  return hipGetLastError();
}

}  // namespace arthip

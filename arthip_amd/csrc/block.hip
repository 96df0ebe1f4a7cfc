// Fused residual block kernels: a residual block's two 64 -> 64 convs in one
// launch, the intermediate tensor kept in LDS (see the comment on BlockL), and
// their host launcher.

#include <hip/hip_runtime.h>

#include <cstdint>

#include "conv_args.h"
#include "launch.h"
#include "wino_dev.h"

namespace arthip {

// ---------------------------------------------------------------------------
// Fused residual block: two 64 -> 64 convs in one kernel (C = M = 64)
// ---------------------------------------------------------------------------
//
//   t   = act1(conv1(in) + bias1)             (fp16, never written to HBM)
//   out = act2(conv2(t) + bias2) + skip0 + skip1
//
// One 512-thread workgroup per CU walks down an output strip of 30 pixels
// (15 Winograd tiles). Waves 0-3 (conv1) hold U1' of 16 output channels each
// and compute t for the 32 columns the strip's conv2 tiles read (16 tiles at
// column offset -1), one tile row (2 t rows) per step, into a 2-slot LDS ring;
// t outside the image is stored as zero, which is conv2's padding. Waves 4-7
// (conv2) hold U2', transform t from the ring (keeping the previous two rows in
// registers), fold 16 tiles of which the first 15 are the strip's outputs and
// stage them. The staged rows go to HBM a step later with the residual inputs
// added (loaded one step ahead; the block input rows were read by conv1 a few
// steps before and are usually still cached): stored by the conv1 waves, or
// with two residual inputs one row of each pair by each group.
//
// Both halves are winograd_strip's arithmetic: the same V' transform, fold
// order and fp16 roundings. conv1's tiles sit at odd offsets (t columns
// 30 s - 1 + 2 k, t rows 2 i - 1 and 2 i), where a separate launch tiles at
// even ones; F(2x2,3x3) rounds a tile's two outputs differently, so t, and the
// block output, agree with two separate launches to fp16 rounding rather than
// bit for bit. The offsets are fixed relative to the image, so results do not
// depend on the strip or workgroup that computes them. HBM traffic per block is
// the input once (plus the 2-column halo of each strip, mostly cache hits), the
// residual inputs and the output.
//
// Per run (one strip, output tile rows j0 .. j0+len-1; t tile row i covers t
// rows 2(j0+i)-1 and 2(j0+i), i = 0 .. len), phase k (k = 0 .. len+4) ends with
// the workgroup barrier:
//   conv1 waves: store output row k-5 from staging[(k-5)&1] with its
//                residuals (k >= 5) and load the residuals of row k-4 (after
//                the fold in the ReLU / no-activation block with one residual
//                input; with two, only the first row of each pair, and the
//                conv2 waves store and load the second);
//                transform t_k into V1'[k&1] (k <= len) and load the input
//                rows of t_{k+1}; fold t_{k-1} from V1'[(k-1)&1] into ring
//                slot (k-1)&1 (1 <= k <= len+1)
//   conv2 waves: read t_{k-2} from ring slot k&1 (2 <= k <= len+2); fold
//                output row k-4 from V2'[k&1] into staging[k&1]
//                (4 <= k <= len+3); with two residual inputs store the second
//                row of output row pair k-5 and load the residuals of row k-4;
//                transform output row k-3 into V2'[(k-3)&1] (3 <= k <= len+2)
// Every buffer's writer and readers are a barrier apart. The store sits with
// the conv1 waves where it can: with the conv2 waves it made theirs the
// longer chain by about a third of a phase (timestamps per section), and
// moved over it took the 1080p one-residual launch from 240 to 226 us.
// With two residual inputs it is split between the two wave groups.
struct BlockL {
  static constexpr int C = 64;
  static constexpr int PX = 2 * C;                // bytes per pixel
  static constexpr int OTILES = 15;               // output tiles per strip
  static constexpr int OPX = 2 * OTILES;          // output pixels per strip
  static constexpr int WPS = StripLds<2>::WPS;    // halfs per V' position
  static constexpr int VBUF = StripLds<2>::VBUF;  // halfs per V' buffer
  static constexpr int SBUF = StripStage<2>::SBUF;
  static constexpr int RSLOT = 2 * 32 * C;        // halfs per ring slot (2 t rows x 32 px)
  // Ring: pixel pairs m = x >> 1 take 256 bytes, the two pixels' halves
  // swapped on odd m, and the 8-byte channel quads of the pair XORed with m.
  // The conv1 folds' writes (16 tiles, one pixel and quad each) and the conv2
  // reads (2 tiles x 16 quads per 32 lanes) then both hit distinct banks.
  __host__ __device__ static constexpr int at(int row, int x, int q) {
    return row * 32 * C + (x >> 1) * 128 + (((x & 1) ^ ((x >> 1) & 1)) << 6) +
           ((q ^ ((x >> 1) & 15)) << 2);
  }
  static constexpr int V1 = 0;
  static constexpr int V2 = 2 * VBUF;
  static constexpr int RING = 4 * VBUF;
  static constexpr int STG = RING + 2 * RSLOT;
  static constexpr size_t lds_bytes() { return (size_t)(STG + 2 * SBUF) * 2; }
};

// Fold of 16 tiles x 16 output channels (one wave) from V' at vr[kc] + boff:
// the four outputs of each tile, bias already in, fp32.
__device__ __forceinline__ void block_fold(const h8 (&u)[16][2], const _Float16* const (&vr)[2],
                                           int boff, f4 bias4, f4& y00, f4& y01, f4& y10,
                                           f4& y11) {
  constexpr int WPS = BlockL::WPS;
  auto mm = [&](int p, f4 acc) {
#pragma unroll
    for (int kc = 0; kc < 2; ++kc)
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(
          u[p][kc], *reinterpret_cast<const h8*>(vr[kc] + boff + p * WPS), acc, 0, 0, 0);
    return acc;
  };
  // LLVM's single-wave small-GEMM interleave (LDS reads between the MFMAs):
  // one-residual block 231 -> 228 us at 1080p, the SiLU block 271 -> 264 us;
  // preset 0 measured 247 us.
  __builtin_amdgcn_iglp_opt(1);
  const f4 z = {0, 0, 0, 0};
  const f4 m2 = {-2.0f, -2.0f, -2.0f, -2.0f};
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
}

// Phases k = 0 .. len + 4 of one run, two per iteration so that the buffer
// parity is a compile-time constant: ph(parity_tag, k).
template <class F>
__device__ __forceinline__ void block_phases(int len, F&& ph) {
  for (int k = 0;;) {
    ph(IntC<0>{}, k);
    if (++k > len + 4) break;
    ph(IntC<1>{}, k);
    if (++k > len + 4) break;
  }
}

template <int ACT1, int ACT2, int NSKIP, bool kCachedOut>
__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
winograd_block(BlockArgs a) {
  using L = BlockL;
  constexpr int C = L::C;
  constexpr int PX = L::PX;
  constexpr int WPS = L::WPS;
  constexpr int VBUF = L::VBUF;
  constexpr int SBUF = L::SBUF;
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
  // MFMA lane: tile tcol, B rows 8*kq.. of each 32-channel chunk, output
  // channels [ch0, ch0 + 4) of the tile's four pixels.
  const int grp = wave & 3;  // 16-channel block within the conv
  const int tcol = lane & 15;
  const int kq = lane >> 4;
  const int ch0 = 16 * grp + 4 * kq;
  // Transform task (both halves): tile tt, channel quad tq.
  const int gtid = tid & 255;
  const int tt = gtid >> 4;
  const int tq = gtid & 15;

  // Store phase: thread handles 16-byte group sg of pixel sx in a row of the
  // output row pair that left the conv2 fold last phase. With up to one
  // residual input the conv1 waves store both rows (1080p, one residual:
  // 240 us with the conv2 waves storing, 226 with conv1; split, 229). With
  // two, holding both rows' residual registers across the conv1 fold costs
  // more than it saves (280 against 260 us), so the rows are split: the conv1
  // waves store row 0 and the conv2 waves row 1, each holding one row's
  // residuals (259 -> 241 us).
  constexpr int kConv1Rows = NSKIP < 2 ? 2 : 1;  // rows [0, kConv1Rows) in conv1
  // The conv1 waves load the next row's residuals right after the store, or,
  // in the ReLU / no-activation block with one residual input, after their
  // fold, so that those registers are not live across it: that block 227.0
  // -> 224.6 us at 1080p, while the same order took the SiLU block from 265 to
  // 284-293 us and the two-residual block from 240 to 260 us.
  constexpr bool kSkipsAfterFold = ACT1 != kActSilu && NSKIP == 1;
  // With act1 ReLU or none, conv1 runs on U1' / 4 and bias1 / 4 and the ring
  // holds t / 4: the power-of-two scale commutes with the activation and with
  // every fp16 and fp32 rounding (outside the subnormal range), so conv2's
  // transform of the ring equals the 1/4-scaled transform of t and drops its
  // own 1/4 (16 of 64 packed ops per transform). SiLU does not commute.
  constexpr bool kQuarterT = ACT1 != kActSilu;
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
    const bool ok = live && (r == 0 || 2 * o + 1 < a.H);  // uniform
    return ok ? lane_off + (uint32_t)r * rb32 : kOob;
  };
  // Rows [ra, rb) of the pair.
  auto load_skips = [&](bool live, int o, int ra, int rb) {
#pragma unroll
    for (int k = 0; k < 2; ++k)
#pragma unroll
      for (int r = 0; r < 2; ++r) skr[k][r] = h8{0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int k = 0; k < NSKIP; ++k) {
      const __amdgpu_buffer_rsrc_t rs = row_rsrc(k == 0 ? a.skip0 : a.skip1, o);
#pragma unroll
      for (int r = ra; r < rb; ++r)
        skr[k][r] = __builtin_bit_cast(
            h8, __builtin_amdgcn_raw_buffer_load_b128(rs, st_off(live, o, r), 0, kNonTemporal));
    }
  };
  auto store_row = [&](bool live, int o, int SB, int ra, int rb) {
    const __amdgpu_buffer_rsrc_t rs = row_rsrc(a.out, o);
#pragma unroll
    for (int r = ra; r < rb; ++r) {
      h8 v = act8<ACT2>(*reinterpret_cast<const h8*>(stg + SB * SBUF + sr0 + r * 32 * C));
      if (NSKIP > 0) v += skr[0][r];
      if (NSKIP > 1) v += skr[1][r];
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, v), rs, st_off(live, o, r), 0,
                                             kCachedOut ? 0 : kNonTemporal);
    }
  };
  if (wave < 4) {
    // ---------------- conv1: in -> t ----------------------------------------
    h8 u[16][2];
    {
      const h8* up = reinterpret_cast<const h8*>(a.u1) + (size_t)grp * (16 * 2 * 64) + lane;
#pragma unroll
      for (int p = 0; p < 16; ++p)
#pragma unroll
        for (int kc = 0; kc < 2; ++kc) u[p][kc] = up[(p * 2 + kc) * 64];
    }
    f4 bias4 = *reinterpret_cast<const f4*>(a.bias1 + ch0);
    if constexpr (kQuarterT) {
#pragma unroll
      for (int p = 0; p < 16; ++p)
#pragma unroll
        for (int kc = 0; kc < 2; ++kc) u[p][kc] *= (_Float16)0.25f;
      bias4 *= 0.25f;
    }
    _Float16* const vw = blds + L::V1 + StripLds<2>::at(tt, 4 * tq);
    const _Float16* vr[2];
#pragma unroll
    for (int kc = 0; kc < 2; ++kc) vr[kc] = blds + L::V1 + StripLds<2>::at(tcol, 32 * kc + 8 * kq);
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
    // Input patch of t tile tt: padded columns pc0 .. pc0 + 3 with
    // pc0 = 30 s - 1 + 2 tt, 8 bytes of channel quad tq each. The row goes in
    // the instruction's scalar offset; columns outside the padded row get an
    // out-of-range lane offset and rows outside the image a zero-size
    // resource, both of which read as zero.
    const int64_t img_bytes = (int64_t)a.Hp * row_bytes;
    __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void*)a.in, (short)0, 0, 0x00020000);
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
          const h4 v = __builtin_bit_cast(
              h4, __builtin_amdgcn_raw_buffer_load_b64(rr, col_off[j], ro, 0));
          x[2 * (4 * r + j)] = __builtin_shufflevector(v, v, 0, 1);
          x[2 * (4 * r + j) + 1] = __builtin_shufflevector(v, v, 2, 3);
        }
      }
    };
    // Lane masks (all ones or zero) of this lane's two t columns, per run.
    uint32_t cm0 = 0, cm1 = 0;
    h2 A[16], B[16];
    auto phase = [&](auto par_tag, int k, int len) {
      constexpr int P = decltype(par_tag)::value;  // k & 1
      h2(&top)[16] = P ? B : A;
      h2(&bot)[16] = P ? A : B;
      // Output row k-5 leaves staging (k-5)&1 = P^1 (the conv2 fold of the
      // last phase); its residuals were loaded last phase. Then the residuals
      // of row k-4 (folded by conv2 this phase, stored next phase).
      store_row(k >= 5, j0 + k - 5, P ^ 1, 0, kConv1Rows);
      if constexpr (!kSkipsAfterFold)
        load_skips(k >= 4 && k <= len + 3, j0 + k - 4, 0, kConv1Rows);
      // Transform first, fold second: the conv2 wave on the same SIMD folds
      // first, so one wave's VALU transform overlaps the other's MFMA chain
      // (and the next input rows are requested earlier).
      if (k <= len) {
        v_transform<WPS>(vw + P * VBUF, top, bot);
        // t_{k+1} needs padded input rows 2 (j0 + k + 1) + 1 and + 2.
        load2(top, 2 * (j0 + k) + 3);
      }
      if (k >= 1 && k <= len + 1) {
        // Fold t_{k-1}: t rows 2 (j0 + k - 1) - 1 + dy, t columns 30 s - 1 + 2 tcol + dx.
        f4 y00, y01, y10, y11;
        block_fold(u, vr, (P ^ 1) * VBUF, bias4, y00, y01, y10, y11);
        const int tr0 = 2 * (j0 + k - 1) - 1;
        const uint32_t rm0 = (tr0 >= 0 && tr0 < a.H) ? ~0u : 0u;  // uniform
        const uint32_t rm1 = (tr0 + 1 < a.H) ? ~0u : 0u;
        // t outside the image is stored as zero (bitwise, so that no branch
        // splits the phase).
        auto masked = [&](f4 y, uint32_t m) {
          u2 b = __builtin_bit_cast(u2, strip_act4<ACT1>(y));
          b &= u2{m, m};
          return b;
        };
        _Float16* sl = ring + (P ^ 1) * L::RSLOT;
        *reinterpret_cast<u2*>(sl + rw[0]) = masked(y00, rm0 & cm0);
        *reinterpret_cast<u2*>(sl + rw[1]) = masked(y01, rm0 & cm1);
        *reinterpret_cast<u2*>(sl + rw[2]) = masked(y10, rm1 & cm0);
        *reinterpret_cast<u2*>(sl + rw[3]) = masked(y11, rm1 & cm1);
      }
      if constexpr (kSkipsAfterFold)
        load_skips(k >= 4 && k <= len + 3, j0 + k - 4, 0, kConv1Rows);
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
        const int tc0 = L::OPX * s - 1 + 2 * tcol;
        cm0 = (tc0 >= 0 && tc0 < a.W) ? ~0u : 0u;
        cm1 = (tc0 + 1 < a.W) ? ~0u : 0u;
        run_pix = ((int64_t)n * a.Hp + 2 * j0 + 1) * a.Wp + L::OPX * s + 1;
        lane_off = (sx < L::OPX && L::OPX * s + sx < a.W) ? s_lane : kOob;
      }
      // t_0 needs padded rows 2 j0 - 1 .. 2 j0 + 2.
      load2(A, 2 * j0 - 1);
      load2(B, 2 * j0 + 1);
      block_phases(len, [&](auto pt, int k) { phase(pt, k, len); });
      it += len;
    }
    return;
  }

  // ---------------- conv2: t -> out ------------------------------------------
  h8 u[16][2];
  {
    const h8* up = reinterpret_cast<const h8*>(a.u2) + (size_t)grp * (16 * 2 * 64) + lane;
#pragma unroll
    for (int p = 0; p < 16; ++p)
#pragma unroll
      for (int kc = 0; kc < 2; ++kc) u[p][kc] = up[(p * 2 + kc) * 64];
  }
  const f4 bias4 = *reinterpret_cast<const f4*>(a.bias2 + ch0);
  _Float16* const vw = blds + L::V2 + StripLds<2>::at(tt, 4 * tq);
  const _Float16* vr[2];
#pragma unroll
  for (int kc = 0; kc < 2; ++kc) vr[kc] = blds + L::V2 + StripLds<2>::at(tcol, 32 * kc + 8 * kq);
  const _Float16* const ring = blds + L::RING;
  // Ring pixels of this task's patch: 2 tt .. 2 tt + 3 (tile 15 is not an
  // output of the strip; it reads tile 14's patch).
  // Row 0 addresses of the four pixels; row 1 and the slot are immediate
  // offsets from them.
  const _Float16* rp[4];
  {
    const int rx0 = 2 * (tt < L::OTILES ? tt : L::OTILES - 1);
#pragma unroll
    for (int j = 0; j < 4; ++j) rp[j] = ring + L::at(0, rx0 + j, tq);
  }
  auto ring_load2 = [&](h2 (&x)[16], int sl) {
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const h4 v = *reinterpret_cast<const h4*>(rp[j] + sl * L::RSLOT + r * 32 * C);
        x[2 * (4 * r + j)] = __builtin_shufflevector(v, v, 0, 1);
        x[2 * (4 * r + j) + 1] = __builtin_shufflevector(v, v, 2, 3);
      }
  };
  const int sw0 = StripStage<2>::at(0, 2 * tcol, ch0 >> 3) + (ch0 & 7);
  h2 A[16], B[16];
  auto phase = [&](auto par_tag, int k, int len) {
    constexpr int P = decltype(par_tag)::value;  // k & 1
    h2(&cur)[16] = P ? B : A;
    h2(&nxt)[16] = P ? A : B;
    // t_{k-2} from ring slot k&1 into `nxt`; with t_{k-3} in `cur` that is the
    // patch of output row k-3. Read at the start of the phase, so that these
    // LDS reads overlap the fold (the registers they land in are live all phase
    // anyway): one-residual block 222.0 -> 219.8 us, SiLU block 260 -> 255 us,
    // two-residual block (its store after the fold) 230.9 -> 228.6 us.
    if (k >= 2 && k <= len + 2) ring_load2(nxt, P);
    const bool fold = k >= 4 && k <= len + 3;
    if (fold) {
      f4 y00, y01, y10, y11;
      block_fold(u, vr, P * VBUF, bias4, y00, y01, y10, y11);
      _Float16* sw = stg + P * SBUF + sw0;
      *reinterpret_cast<h4*>(sw) = strip_act4<kActNone>(y00);
      *reinterpret_cast<h4*>(sw + C) = strip_act4<kActNone>(y01);
      *reinterpret_cast<h4*>(sw + 32 * C) = strip_act4<kActNone>(y10);
      *reinterpret_cast<h4*>(sw + 33 * C) = strip_act4<kActNone>(y11);
    }
    // With two residual inputs: output row k-5 leaves staging (k-5)&1 = P^1
    // with the residuals loaded last phase (after the fold: 243 -> 235 us
    // against before it), then the residuals of the row just folded (stored
    // next phase), issued after the fold so that they are not live across it.
    if constexpr (kConv1Rows < 2) {
      store_row(k >= 5, j0 + k - 5, P ^ 1, kConv1Rows, 2);
      load_skips(fold, j0 + k - 4, kConv1Rows, 2);
    }
    if (k >= 2 && k <= len + 2) {
      if (k >= 3) v_transform<WPS, !kQuarterT>(vw + (P ^ 1) * VBUF, cur, nxt);
    }
    lds_sync();
  };
  for (int it = begin; it < end;) {
    decode(it);
    const int len = min(end - it, a.tiles_h - j0);
    run_pix = ((int64_t)n * a.Hp + 2 * j0 + 1) * a.Wp + L::OPX * s + 1;
    lane_off = (sx < L::OPX && L::OPX * s + sx < a.W) ? s_lane : kOob;
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
  int64_t grid = cu_count();  // one 512-thread workgroup per CU (all of its LDS)
  if (grid > items) grid = items;
  grid = (grid + 7) / 8 * 8;
  hipLaunchKernelGGL(fn, dim3((unsigned)grid), dim3(512), lds, s, a);
  return hipGetLastError();
}

}  // namespace arthip

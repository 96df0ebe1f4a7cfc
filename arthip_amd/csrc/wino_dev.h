// Device helpers shared by the gfx950 Winograd kernels (kernels.hip and
// block.hip): vector types, the LDS barrier, the V' input transform, the
// fp16 epilogue activations and the strip staging layout.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "conv_args.h"

namespace arthip {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));

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

__device__ __forceinline__ h4 to_h4(f4 v) {
  return h4{(_Float16)v[0], (_Float16)v[1], (_Float16)v[2], (_Float16)v[3]};
}

// Invariant-divisor division for the persistent work-item index (uniform
// values; avoids the long scalar division sequence). Valid for x < 2^31.
__device__ __forceinline__ uint32_t fdiv(uint32_t x, FastDiv f) {
  const uint64_t t = (static_cast<uint64_t>(x) * f.m) >> 32;
  return static_cast<uint32_t>((t + x) >> f.s);
}

// V' of one input task (4 channels x one tile) into the V' buffer; same
// transform and scaling as store_v, with the patch rows split in two halves.
// The patch is held as half2 pairs (element 2*(4*row + col) + e, channel pair
// e) so that loop-carried values stay in the packed form the v_pk_* ops use.
// a - b on a half2 pair in one packed add. Written as a plain subtraction in
// strip_transform, the compiler splits this one into two half-precision
// subtractions and a pack (three instructions instead of one).
__device__ __forceinline__ h2 pk_sub(h2 a, h2 b) {
  h2 r;
  asm("v_pk_add_f16 %0, %1, %2 neg_lo:[0,1] neg_hi:[0,1]" : "=v"(r) : "v"(a), "v"(b));
  return r;
}

// V' tile-row length in halfs. C = 64 uses 128-byte rows with the eight
// 16-byte channel groups of tile t stored at group index g ^ (t & 7): the MFMA
// B reads (16 tiles x one group per lane) then run at about 160 B/clk per CU on
// gfx950, against 112 B/clk with the padded 144-byte rows, which C = 32 keeps.
template <int KC>
struct StripLds {
  static constexpr bool SWZ = KC == 2;
  static constexpr int TS = SWZ ? 32 * KC : 32 * KC + 8;
  static constexpr int WPS = 16 * TS;  // halfs per position
  static constexpr int VBUF = 16 * WPS;
  // Half offset of channel c (multiple of 4) of tile t within a position.
  __host__ __device__ static constexpr int at(int t, int c) {
    return t * TS + (SWZ ? (((c >> 3) ^ (t & 7)) << 3) + (c & 7) : c);
  }
};

// Cache policy of the buffer accesses that stream through once (output
// stores and residual loads): the "nt" bit. Measured on the 1080p body conv
// with one residual input: 180 -> 159 us; on the input-row loads it helps the
// ReLU layers by 2 us but costs the residual layers 16 us, so those stay plain.
constexpr int kNonTemporal = 2;

// V' of one (tile, 4-channel) task from its 4x4 patch (rows 0-1 in top, 2-3
// in bot), written to LDS at vw + position * WPS. With kQuarter false the
// column stage leaves out the 1/4 (for a patch whose values already carry it).
template <int WPS, bool kQuarter = true>
__device__ __forceinline__ void v_transform(_Float16* vw, const h2 (&top)[16],
                                            const h2 (&bot)[16]) {
  const h2 qp = {0.25f16, 0.25f16};
  const h2 qn = {-0.25f16, -0.25f16};
  h2 t[4][4][2];
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const h2 d0 = top[2 * j + e], d1 = top[2 * (4 + j) + e];
      const h2 d2 = bot[2 * j + e], d3 = bot[2 * (4 + j) + e];
      t[0][j][e] = pk_sub(d0, d2);
      t[1][j][e] = d1 + d2;
      t[2][j][e] = d2 - d1;
      t[3][j][e] = d1 - d3;
    }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    h2 o[4][2];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      if constexpr (kQuarter) {
        const h2 n1 = t[i][1][e] * qn;
        const h2 n2 = t[i][2][e] * qn;
        o[0][e] = __builtin_elementwise_fma(t[i][0][e], qp, n2);
        o[1][e] = __builtin_elementwise_fma(t[i][1][e], qp, -n2);
        o[2][e] = __builtin_elementwise_fma(t[i][2][e], qp, n1);
        o[3][e] = __builtin_elementwise_fma(t[i][3][e], qp, n1);
      } else {
        o[0][e] = pk_sub(t[i][0][e], t[i][2][e]);
        o[1][e] = t[i][1][e] + t[i][2][e];
        o[2][e] = pk_sub(t[i][2][e], t[i][1][e]);
        o[3][e] = pk_sub(t[i][3][e], t[i][1][e]);
      }
    }
    _Float16* row = vw + (4 * i) * WPS;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      *reinterpret_cast<h4*>(row + k * WPS) = __builtin_shufflevector(o[k][0], o[k][1], 0, 1, 2, 3);
  }
}

template <int KC>
__device__ __forceinline__ void strip_transform(_Float16* vw, const h2 (&top)[16],
                                                const h2 (&bot)[16]) {
  v_transform<StripLds<KC>::WPS>(vw, top, bot);
}

// SiLU of four fp16 values, x / (1 + exp(-x)) in fp32 and one rounding to
// fp16: exp(-x) as exp2 of x * -log2(e) (what __expf(-x) computes), the
// reciprocal, and x times it. Both products are FMAs with a zero addend, which
// take x in fp16 directly (v_fma_mix_f32), so x is never converted on its own;
// the values equal plain products except that a zero result is +0.
// kInterleave writes the four chains stage by stage (four exps, four
// reciprocals, four products), which the compiler then issues side by side;
// written per element, it runs them one after another, each waiting on its
// transcendentals. The arithmetic is the same either way.
template <bool kInterleave = true>
__device__ __forceinline__ h4 silu4(h4 r) {
  f4 q, t;
  if constexpr (kInterleave) {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      q[e] = __builtin_amdgcn_exp2f(__builtin_fmaf((float)r[e], -1.44269502f, 0.0f));
#pragma unroll
    for (int e = 0; e < 4; ++e) q[e] = __builtin_amdgcn_rcpf(1.0f + q[e]);
#pragma unroll
    for (int e = 0; e < 4; ++e) t[e] = __builtin_fmaf((float)r[e], q[e], 0.0f);
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float x = (float)r[e];
      q[e] = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(__builtin_fmaf(x, -1.44269502f, 0.0f)));
      t[e] = __builtin_fmaf(x, q[e], 0.0f);
    }
  }
  return __builtin_convertvector(t, h4);
}

// fp16 rounding and activation of 4 channels whose accumulator holds the bias.
template <int ACT, bool kInterleave = true>
__device__ __forceinline__ h4 strip_act4(f4 y) {
  h4 r = to_h4(y);
  if (ACT == kActRelu) r = __builtin_elementwise_max(r, h4{0, 0, 0, 0});
  if (ACT == kActSilu) r = silu4<kInterleave>(r);
  return r;
}

// LDS byte address of a pointer into shared memory.
__device__ __forceinline__ uint32_t lds_byte_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)(p);
}

// One 16-byte-per-lane buffer -> LDS copy: lane l of the wave writes LDS bytes
// [m0 + 16 l, m0 + 16 l + 16) from the buffer resource at byte voff; an offset
// past the resource's size copies zeros. Inline assembly, so the compiler
// neither tracks it nor inserts waits for it; the kernels count it.
__device__ __forceinline__ void dma16_buf(uint32_t m0, __amdgpu_buffer_rsrc_t rs, uint32_t voff) {
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %1, %2, 0 offen lds"
      :
      : "s"(m0), "v"(voff), "s"(rs)
      : "memory");
}

// Waits until at most N of this wave's vector-memory instructions are
// outstanding (they complete in issue order). Inline assembly with a memory
// clobber, so that the compiler moves no memory access across it.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt field");
  asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}

template <int N>
struct IntC {
  static constexpr int value = N;
};

// f(IntC<0>{}), ..., f(IntC<N-1>{}): a loop whose index is a compile-time
// constant in every iteration.
template <int N, int I = 0, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(IntC<I>{});
    static_for<N, I + 1>(f);
  }
}

// Two waves per SIMD: at most 256 registers per lane (U' takes 64 * KC).
// Output staging: after act and the fp16 rounding, each item's 2 x 32 x C
// output tile goes to LDS as [row][pixel][C] (16-byte channel groups of pixel x
// at group index g ^ ((x >> 1) & (C/8 - 1)), which spreads the 8-byte writes of
// the MFMA lanes over the banks). After the next barrier every thread moves
// 16-byte groups to HBM, a wave covering whole 128-byte lines, and adds the
// residual inputs on the way with loads of the same shape.
template <int KC>
struct StripStage {
  static constexpr int C = 32 * KC;
  static constexpr int G = C / 8;          // 16-byte groups per pixel
  static constexpr int SBUF = 2 * 32 * C;  // halfs per staging buffer
  __host__ __device__ static constexpr int at(int row, int x, int g) {
    return (row * 32 + x) * C + ((g ^ ((x >> 1) & (G - 1))) << 3);
  }
};

// Activation of 8 fp16 values, each computed from the fp16 value in fp32 and
// rounded back (the same arithmetic as strip_act4 after its rounding).
template <int ACT>
__device__ __forceinline__ h8 act8(h8 r) {
  if (ACT == kActRelu) r = __builtin_elementwise_max(r, h8{0, 0, 0, 0, 0, 0, 0, 0});
  if (ACT == kActSilu) {
    const h4 lo = silu4(__builtin_shufflevector(r, r, 0, 1, 2, 3));
    const h4 hi = silu4(__builtin_shufflevector(r, r, 4, 5, 6, 7));
    r = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  }
  return r;
}

}  // namespace arthip

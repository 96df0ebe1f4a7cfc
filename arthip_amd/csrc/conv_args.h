// Launch arguments shared by the host launchers and the gfx950 kernels.
//
// Internal activations are "padded NHWC" fp16: [n][Hp][Wp][c] with a zero
// border, Hp = 2*ceil(H/2) + 2 and Wp = 2*ceil(W/2) + 2, pixel (h, w) stored
// at row h+1, column w+1. Every 4x4 Winograd input patch and every 3x3 direct
// window then lies inside the buffer, so the conv kernels load without bounds
// checks. The border is zeroed once when a buffer is allocated and is never
// written afterwards.
//
// The graph boundary (engine input and output) is plain NCHW in fp16 or fp32,
// like the reference's host interface (src/vapoursynth/hip_engine.h:98-103).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace arthip {

enum Act : int32_t { kActNone = 0, kActRelu = 1, kActSilu = 2 };

enum OutKind : int32_t {
  kOutPadded = 0,   // internal padded NHWC fp16
  kOutNchwF16 = 1,  // boundary layout, fp16
  kOutNchwF32 = 2,  // boundary layout, fp32 (a folded output Cast)
};

__host__ __device__ inline int64_t padded_rows(int64_t h) { return 2 * ((h + 1) / 2) + 2; }
__host__ __device__ inline int64_t padded_cols(int64_t w) { return 2 * ((w + 1) / 2) + 2; }

// Epilogue applied to every conv output element:
//   y = acc + bias[m]; y = act(y); y += skip0; y += skip1; y = clip(y)
// The fast path (padded NHWC output, M % 4 == 0, no clip) rounds acc + bias to
// fp16 once and applies act and the residual adds in fp16 arithmetic (each add
// rounds once, like the fp16 tensors between ONNX nodes); the general path keeps
// fp32 until one final rounding. A fused DepthToSpace permutes the destination
// index of a boundary-layout output.
struct Epilogue {
  const float* bias;      // [m_pad] fp32, zero padded (never null)
  const uint16_t* skip0;  // padded NHWC fp16 with the output's geometry, or null
  const uint16_t* skip1;
  void* out;
  int32_t act;       // Act
  int32_t out_kind;  // OutKind
  int32_t dts_b;     // >= 2: fused DepthToSpace(DCR) (boundary output only); else 0
  int32_t do_clip;
  float clip_lo, clip_hi;
};

// Winograd F(2x2,3x3) conv, C > 1 (winograd_conv in kernels.hip).
struct WinoArgs {
  // in_nchw 0: padded NHWC fp16 [N][Hp][Wp][C]; 1: the engine's NCHW fp16
  // boundary input [N][C][H][W] (a 64 -> 64 pipe conv reading it directly).
  const uint16_t* in;
  int32_t in_nchw;
  const uint16_t* u;   // packed transformed filters (winograd_pack)
  Epilogue epi;
  int32_t N, H, W, C, M;
  int32_t Hp, Wp;            // padded geometry shared by input, skips and padded output
  int32_t tiles_h, tiles_w;  // ceil(H/2), ceil(W/2)
  int32_t n_ob;              // 16-wide output-channel blocks (= waves per tile block)
  int32_t tb;                // 16-tile column blocks per work item
  int32_t sb_w;              // work items per tile row = ceil(tiles_w / (16*tb))
  int32_t n_sb;              // total work items = N * tiles_h * sb_w
};

// Invariant-divisor division x / d = (((x * m) >> 32) + x) >> s for uniform
// divisors (valid for x < 2^31); built on the host by make_fastdiv.
struct FastDiv {
  uint32_t d, m, s;
};

// Winograd F(2x2,3x3) conv with C == M in {32, 64} and the fast epilogue
// (winograd_strip in kernels.hip). Work items are 1 tile row x 16 tile columns,
// ordered (n, strip of 16 tile columns, tile row) with the tile row fastest, so
// consecutive items of a workgroup slide down one strip.
struct StripArgs {
  const uint16_t* in;  // padded NHWC fp16 [N][Hp][Wp][C] (or NCHW fp16, winograd_pipe IO bit 0)
  const uint16_t* u;   // packed transformed filters (winograd_pack)
  const float* bias;   // [C] fp32
  const uint16_t* skip0;
  const uint16_t* skip1;
  uint16_t* out;  // padded NHWC fp16, same geometry as the input (or NCHW fp16, IO bit 1)
  int32_t N, H, W, Hp, Wp;
  int32_t tiles_h, tiles_w, n_strips;
  int32_t n_items;  // N * n_strips * tiles_h
  FastDiv fd_tiles_h, fd_strips;
};

// Fused residual block of two 64 -> 64 convs (winograd_block in block.hip):
// out = act2(conv2(act1(conv1(in) + bias1)) + bias2) + skip0 + skip1, every
// tensor padded NHWC fp16 with the input's geometry. Work items are 1 output
// tile row x 15 tiles (a 30-pixel strip), ordered (n, strip, tile row) with the
// tile row fastest.
struct BlockArgs {
  const uint16_t* in;
  const uint16_t* u1;  // packed transformed filters of conv1 (winograd_pack)
  const float* bias1;  // [64] fp32
  const uint16_t* u2;
  const float* bias2;
  const uint16_t* skip0;  // or null
  const uint16_t* skip1;  // or null (only with skip0)
  uint16_t* out;
  int32_t N, H, W, Hp, Wp;
  int32_t act1, act2;
  // 0: output stores carry the non-temporal hint; 1: plain stores, for an
  // output that the next kernel reads while much of it is still cached.
  int32_t cached_out;
  int32_t tiles_h, n_strips;
  int32_t n_items;  // N * n_strips * tiles_h
  FastDiv fd_tiles_h, fd_strips;
};

// Direct 3x3 conv on MFMA for M <= 16 outputs written to the boundary NCHW
// layout (conv3x3_narrow in kernels.hip). Work items are 1 output row x 64
// pixels, ordered (n, 64-pixel segment, row) with the row fastest.
struct NarrowArgs {
  const uint16_t* in;  // padded NHWC fp16 [N][Hp][Wp][C]
  const uint16_t* w;   // narrow taps (narrow_packed_halfs layout)
  const float* bias;   // [>= 16] fp32, zero padded
  void* out;           // NCHW [N][Cout][H*b][W*b], fp16 or fp32
  int32_t N, H, W, Hp, Wp, M;
  int32_t act, do_clip;
  float clip_lo, clip_hi;
  int32_t dts_b, cout;       // DepthToSpace block (1 = none); Cout = M / b^2
  int32_t n_seg, n_items;    // ceil(W / 64); N * n_seg * H
  FastDiv fd_H, fd_seg;
  int64_t img_bytes;         // bytes of one output image (< 2^31)
};

// Direct 3x3 conv for a single input channel (the model's head conv).
struct DirectArgs {
  // in_kind 0: padded NHWC fp16 [N][Hp][Wp][1]; 1 / 2: the engine's NCHW
  // boundary input [N][1][H][W] in fp16 / fp32 (head conv reading it directly).
  const void* in;
  int32_t in_kind;
  const uint16_t* w;   // packed taps: [g8][8 ch][5 x half2] (direct_pack)
  Epilogue epi;
  int32_t N, H, W, M;
  int32_t Hp, Wp;
  int32_t g8;  // threads per pixel (power of two >= ceil(M/8))
};

// Elementwise / layout kernels for the ops the conv epilogues do not absorb.
enum UnaryOp : int32_t { kUnarySigmoid = 0, kUnaryRelu = 1, kUnaryClip = 2 };
enum BinaryOp : int32_t { kBinaryAdd = 0, kBinaryMul = 1 };

struct EltArgs {
  const uint16_t* a;  // padded NHWC fp16
  const uint16_t* b;  // second operand (binary) or null
  uint16_t* out;      // padded NHWC fp16, same geometry
  int32_t N, H, W, C, Hp, Wp;
  int32_t op;
  float lo, hi;
};

struct DtsArgs {
  const uint16_t* in;  // padded NHWC fp16 [N][Hp][Wp][C]
  void* out;           // padded NHWC fp16 (kOutPadded) or boundary NCHW
  int32_t N, H, W, C, Hp, Wp;  // input geometry
  int32_t b;                   // block size; output channels = C / (b*b)
  int32_t out_kind;
  int32_t do_clip;
  float lo, hi;
};

struct IoArgs {
  const void* src;
  void* dst;
  int32_t N, H, W, C, Hp, Wp;
  int32_t fp32;  // boundary side is fp32
};

// Element types of VapourSynth plane samples and of the engine boundary.
enum SampleKind : int32_t { kSampleU8 = 0, kSampleU16 = 1, kSampleF16 = 2, kSampleF32 = 3 };

// Element-wise conversion between plane samples and the NCHW boundary:
// u8 / u16 / f16 / f32 -> f16 / f32 (input side) and f16 -> u16 (output side).
struct PlaneArgs {
  const void* src;
  void* dst;
  int64_t n;  // elements
  int32_t src_kind, dst_kind;  // SampleKind
};

}  // namespace arthip

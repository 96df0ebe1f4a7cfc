// Launch arguments shared by the host launchers and the gfx950 kernels.
//
// Activations inside the engine are NHWC fp16 ([n][h][w][c], channels
// contiguous). The final op of a graph may instead write the public NCHW
// boundary layout directly, in fp16 or fp32, optionally through a fused
// DepthToSpace (DCR) and Clip.
#pragma once

#include <cstdint>

namespace arthip {

enum Act : int32_t { kActNone = 0, kActRelu = 1, kActSilu = 2 };

enum OutKind : int32_t {
  kOutNhwcF16 = 0,  // internal activation layout
  kOutNchwF16 = 1,  // boundary layout, fp16
  kOutNchwF32 = 2,  // boundary layout, fp32 (a folded output Cast)
};

// Epilogue applied to every conv output element, in this order, all in fp32:
//   y = acc + bias[m]; y = act(y); y += skip0; y += skip1; y = clip(y);
// then one rounding to the output dtype. A fused DepthToSpace permutes the
// destination index only.
struct Epilogue {
  const float* bias;       // [m_pad] fp32, zero padded (never null)
  const uint16_t* skip0;   // NHWC fp16 [n][h][w][M], or null
  const uint16_t* skip1;   // NHWC fp16 [n][h][w][M], or null
  void* out;
  int32_t act;             // Act
  int32_t out_kind;        // OutKind
  int32_t dts_b;           // >= 2: fused DepthToSpace(DCR) with this block size; else 0
  int32_t do_clip;
  float clip_lo, clip_hi;
};

// Winograd F(2x2,3x3) conv, C > 1 (see winograd_conv in kernels.hip).
struct WinoArgs {
  const uint16_t* in;  // NHWC fp16 [N][H][W][C]
  const uint16_t* u;   // packed transformed filters (winograd_pack)
  Epilogue epi;
  int32_t N, H, W, C, M;
  int32_t tiles_h, tiles_w;  // ceil(H/2), ceil(W/2)
  int32_t n_ob;              // 16-wide output-channel blocks (= waves per tile block)
  int32_t tb;                // 16-tile column blocks per work item
  int32_t sb_w;              // work items per tile row = ceil(tiles_w / (16*tb))
  int32_t n_sb;              // total work items = N * tiles_h * sb_w
};

// Direct 3x3 conv for a single input channel (the model's head conv).
struct DirectArgs {
  const uint16_t* in;  // NHWC fp16 [N][H][W][1]
  const uint16_t* w;   // packed taps: [g8][8 ch][5 x half2] (direct_pack)
  Epilogue epi;
  int32_t N, H, W, M;
  int32_t g8;          // threads per pixel (power of two >= ceil(M/8))
};

}  // namespace arthip

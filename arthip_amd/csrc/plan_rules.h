// Plan-time rules shared by the engine's planner and the kernel launchers.
// Host-only C++ (no HIP types), so a CPU test can compile and check them.
#pragma once

#include <cstdint>

namespace arthip {

// Threads per pixel of the column-walking head conv: the smallest power of two
// g with 8 * g >= M (each thread computes 8 output channels).
inline int head_g8(int64_t M) {
  int g = 1;
  while (g * 8 < M) g *= 2;
  return g;
}

// True when the one-channel head conv (padded output, no Clip, no DepthToSpace,
// no residual input) can read the engine's NCHW boundary input itself, in fp16
// or fp32, instead of a padded copy. The fast head kernels need M % 8 == 0 and
// at most 16 threads per pixel (M <= 128); their work-item count
// N * ceil(W / segment) * H and the byte size of one boundary input image
// (addressed through a 32-bit buffer resource) must both stay below 2^31.
// launch_direct refuses the boundary input whenever this is false, so the
// planner must never bind it then.
inline bool head_reads_boundary_input(int64_t N, int64_t H, int64_t W, int64_t M, bool fp32) {
  if (N < 1 || H < 1 || W < 1 || M < 1) return false;
  if (M % 8 != 0 || M > 128) return false;
  const int64_t seg = 4 * 256 / head_g8(M);
  const int64_t items = N * ((W + seg - 1) / seg) * H;
  const int64_t img = H * W * (fp32 ? 4 : 2);
  const int64_t lim = static_cast<int64_t>(1) << 31;
  return items < lim && img < lim;
}

// True when a 64 -> 64 conv on the producer/consumer pipe (no residual
// input, no Clip, no DepthToSpace) can read the engine's NCHW fp16 boundary
// input itself (input_side) or write the NCHW fp16 boundary output itself,
// instead of a padded NHWC copy and a layout pass. The producers copy input
// rows in 8-pixel (16-byte) chunks and the consumers store 8-pixel groups of
// one channel as 16-byte words, so either side needs W % 8 == 0. One image (64 planes of H x W fp16) is addressed
// through a 32-bit buffer resource and must stay below 2^31 bytes; the item
// count N * ceil(ceil(W/2) / 16) * ceil(H/2) below 2^31 as well. launch_winograd
// refuses the boundary layouts whenever this is false.
inline bool pipe_boundary_io(int64_t N, int64_t H, int64_t W, int64_t C, int64_t M,
                             bool input_side) {
  if (N < 1 || H < 1 || W < 1 || C != 64 || M != 64) return false;
  (void)input_side;
  if (W % 8 != 0) return false;
  const int64_t lim = static_cast<int64_t>(1) << 31;
  const int64_t items = N * (((W + 1) / 2 + 15) / 16) * ((H + 1) / 2);
  return 64 * H * W * 2 < lim && items < lim;
}

}  // namespace arthip

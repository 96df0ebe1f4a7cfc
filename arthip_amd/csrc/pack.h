// Compile-time weight transforms for the conv kernels.
//
// Winograd: U = G g G^T per (output, input) channel pair, done once when a
// plan is built (the reference does the same on the host:
// src/vapoursynth/hip_engine.cc:972-1018, src/onnxruntime-hip/hip_graph.cc:923-989).
// The packed layout is this build's own: MFMA A-operand order for
// v_mfma_f32_16x16x32_f16, scaled by 4 to match the kernel's V/4 transform.
#pragma once

#include <cstddef>
#include <cstdint>

namespace arthip {

struct WinoGeom {
  int kc, n_ob, tb, threads;
  size_t lds;
};

// Launch geometry / packed sizes (defined in kernels.hip).
WinoGeom winograd_geom(int C, int M);
int direct_g8(int M);

// Convs with C % 32 == 0 (C <= 96) and M <= 16 can also run as a direct conv
// on MFMA (conv3x3_tail / conv3x3_narrow, used for boundary outputs such as the
// model's tail).
bool narrow_eligible(int C, int M);
// M <= 5: the three taps of a kernel row share one MFMA (conv3x3_tail).
bool narrow_row_packed(int M);
// Halfs of the direct-conv taps, in v_mfma_f32_16x16x32_f16 B-operand order
// (lane = col + 16*q holds channels 32*kc + 8*q + e, e < 8):
//   row-packed: [3 rows dy][kc][64 lanes][8], col = dx*M + n holding
//               w[n][32*kc + 8*q + e][dy][dx] (zero for col >= 3M);
//   otherwise:  [9 taps][kc][64 lanes][8], col = n holding w[n][...][tap].
size_t narrow_packed_halfs(int C, int M);

// Halfs in the packed buffer: U' as [n_ob][16 positions][kc][64 lanes][8],
// followed by the narrow taps when narrow_eligible(C, M), followed for
// C = M = 64 and C = M = 96 by the row-Winograd filters (block_u_halfs).
size_t winograd_packed_halfs(int C, int M);
// The row-Winograd kernels (the fused residual block and the row pipes,
// C = M = 64 or 96) run F(2,3) along x and sum the three kernel rows in the
// MFMA: per kernel row dy the 1-D transform U_dy = G (w[dy][0], w[dy][1],
// w[dy][2]) (G as above, unscaled), packed as [n_ob][3 dy][4 positions][kc]
// [64 lanes][8] in MFMA A-operand order. Its offset in the packed buffer is
// block_u_offset(C, M); 0 halfs for other shapes.
size_t block_u_halfs(int C, int M);
size_t block_u_offset(int C, int M);
// Halfs of the U' part alone (offset of the narrow taps).
size_t winograd_u_halfs(int C, int M);
// w is OIHW [M][C][3][3] fp32 (exact fp16 values from the model).
void winograd_pack(const float* w, int M, int C, uint16_t* out);

// Halfs in the packed direct-conv taps: [g8][8 channels][5 pairs][2].
size_t direct_packed_halfs(int M);
// w is OIHW [M][1][3][3] fp32.
void direct_pack(const float* w, int M, uint16_t* out);

// Bias padded with zeros to the kernels' channel granularity (16), fp32.
size_t bias_padded_len(int M);
void bias_pad(const float* bias, int M, float* out);

}  // namespace arthip

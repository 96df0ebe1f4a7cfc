#include "pack.h"

#include <cstring>

#include "half.h"

namespace arthip {

bool narrow_eligible(int C, int M) { return C % 32 == 0 && C <= 96 && M >= 1 && M <= 16; }

bool narrow_row_packed(int M) { return M >= 1 && 3 * M <= 16; }

size_t narrow_packed_halfs(int C, int M) {
  if (!narrow_eligible(C, M)) return 0;
  return static_cast<size_t>(narrow_row_packed(M) ? 3 : 9) * (C / 32) * 64 * 8;
}

size_t winograd_u_halfs(int C, int M) {
  const WinoGeom g = winograd_geom(C, M);
  return static_cast<size_t>(g.n_ob) * 16 * g.kc * 64 * 8;
}

size_t block_u_halfs(int C, int M) {
  const bool rows = C == M && (C == 64 || C == 96);
  return rows ? static_cast<size_t>(M / 16) * 12 * (C / 32) * 64 * 8 : 0;
}

size_t block_u_offset(int C, int M) { return winograd_u_halfs(C, M) + narrow_packed_halfs(C, M); }

size_t winograd_packed_halfs(int C, int M) {
  return winograd_u_halfs(C, M) + narrow_packed_halfs(C, M) + block_u_halfs(C, M);
}

void winograd_pack(const float* w, int M, int C, uint16_t* out) {
  const WinoGeom g = winograd_geom(C, M);
  const size_t total = winograd_packed_halfs(C, M);
  std::memset(out, 0, total * sizeof(uint16_t));
  if (narrow_eligible(C, M)) {
    uint16_t* nb = out + winograd_u_halfs(C, M);
    const int kcn = C / 32;
    const bool rows = narrow_row_packed(M);
    for (int n = 0; n < M; ++n)
      for (int c = 0; c < C; ++c)
        for (int t = 0; t < 9; ++t) {
          const int kc = c / 32, q = (c % 32) / 8, e = c % 8;
          const int slot = rows ? t / 3 : t;             // B operand index
          const int col = rows ? (t % 3) * M + n : n;    // B column
          const size_t idx = ((static_cast<size_t>(slot) * kcn + kc) * 64 + col + 16 * q) * 8 + e;
          nb[idx] = f32_to_f16(w[(static_cast<size_t>(n) * C + c) * 9 + t]);
        }
  }
  // G = [[1,0,0],[1/2,1/2,1/2],[1/2,-1/2,1/2],[0,0,1]]; U = G g G^T in double,
  // scaled by 4 (exact), rounded once to fp16.
  static const double G[4][3] = {{1, 0, 0}, {0.5, 0.5, 0.5}, {0.5, -0.5, 0.5}, {0, 0, 1}};
  if (block_u_halfs(C, M) != 0) {
    // Row filters of the fused block: U_dy[p] = G[p] . w[dy][0..2], rounded once.
    uint16_t* bu = out + block_u_offset(C, M);
    const int kcn = C / 32;
    for (int m = 0; m < M; ++m) {
      const int ob = m / 16, row = m % 16;
      for (int c = 0; c < C; ++c) {
        const float* k = w + (static_cast<size_t>(m) * C + c) * 9;
        const int kc = c / 32, kk = c % 32;
        const int lane = row + 16 * (kk / 8), e = kk % 8;
        for (int dy = 0; dy < 3; ++dy)
          for (int p = 0; p < 4; ++p) {
            const double u = G[p][0] * k[dy * 3] + G[p][1] * k[dy * 3 + 1] + G[p][2] * k[dy * 3 + 2];
            const size_t idx =
                ((((static_cast<size_t>(ob) * 3 + dy) * 4 + p) * kcn + kc) * 64 + lane) * 8 + e;
            bu[idx] = f32_to_f16(static_cast<float>(u));
          }
      }
    }
  }
  for (int m = 0; m < M; ++m) {
    const int ob = m / 16, row = m % 16;
    for (int c = 0; c < C; ++c) {
      const float* k = w + (static_cast<size_t>(m) * C + c) * 9;
      double Gg[4][3];
      for (int i = 0; i < 4; ++i)
        for (int j = 0; j < 3; ++j)
          Gg[i][j] = G[i][0] * k[0 * 3 + j] + G[i][1] * k[1 * 3 + j] + G[i][2] * k[2 * 3 + j];
      const int kc = c / 32, kk = c % 32;
      const int lane = row + 16 * (kk / 8), e = kk % 8;
      for (int i = 0; i < 4; ++i)
        for (int j = 0; j < 4; ++j) {
          const double u = Gg[i][0] * G[j][0] + Gg[i][1] * G[j][1] + Gg[i][2] * G[j][2];
          const int p = i * 4 + j;
          const size_t idx = ((((static_cast<size_t>(ob) * 16 + p) * g.kc + kc) * 64) + lane) * 8 + e;
          out[idx] = f32_to_f16(static_cast<float>(4.0 * u));
        }
    }
  }
}

size_t direct_packed_halfs(int M) { return static_cast<size_t>(direct_g8(M)) * 8 * 5 * 2; }

void direct_pack(const float* w, int M, uint16_t* out) {
  const size_t total = direct_packed_halfs(M);
  std::memset(out, 0, total * sizeof(uint16_t));
  for (int m = 0; m < M; ++m) {
    const int g = m / 8, c = m % 8;
    for (int t = 0; t < 9; ++t) {
      const size_t idx = ((static_cast<size_t>(g) * 8 + c) * 5 + t / 2) * 2 + (t % 2);
      out[idx] = f32_to_f16(w[static_cast<size_t>(m) * 9 + t]);
    }
  }
}

size_t bias_padded_len(int M) {
  size_t n = (static_cast<size_t>(M) + 15) / 16 * 16;
  const size_t d = static_cast<size_t>(direct_g8(M)) * 8;
  return n > d ? n : d;
}

void bias_pad(const float* bias, int M, float* out) {
  const size_t n = bias_padded_len(M);
  for (size_t i = 0; i < n; ++i) out[i] = (bias != nullptr && i < static_cast<size_t>(M)) ? bias[i] : 0.0f;
}

}  // namespace arthip

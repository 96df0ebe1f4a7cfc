// extern "C" kernel-level entry points and helpers (include/arthip.h).
#include <hip/hip_runtime.h>

#include <string>
#include <vector>

#include "arthip.h"
#include "half.h"
#include "launch.h"
#include "pack.h"

namespace {

thread_local std::string t_last_error;

int fail(const std::string& msg, int code) {
  t_last_error = msg;
  return code;
}

}  // namespace

extern "C" {

uint16_t arthip_f32_to_f16(float f) { return arthip::f32_to_f16(f); }
float arthip_f16_to_f32(uint16_t h) { return arthip::f16_to_f32(h); }
const char* arthip_last_error(void) { return t_last_error.c_str(); }
const char* arthip_version(void) { return "arthip-mi355x 0.1.0 (gfx950)"; }

int arthip_conv3x3_limits(int* max_c, int* max_m) {
  if (max_c) *max_c = 32 * arthip::winograd_max_kc();
  if (max_m) *max_m = arthip::winograd_max_m();
  return ARTHIP_OK;
}

size_t arthip_conv3x3_packed_halfs(int M, int C) {
  if (M <= 0 || C <= 0) return 0;
  return C == 1 ? arthip::direct_packed_halfs(M) : arthip::winograd_packed_halfs(C, M);
}

size_t arthip_conv3x3_bias_len(int M) { return M <= 0 ? 0 : arthip::bias_padded_len(M); }

int arthip_conv3x3_pack(const uint16_t* w_oihw, const uint16_t* bias, int M, int C,
                        uint16_t* packed, size_t packed_cap, float* bias_out, size_t bias_cap) {
  if (w_oihw == nullptr || packed == nullptr || bias_out == nullptr || M <= 0 || C <= 0)
    return fail("arthip_conv3x3_pack: null buffer or non-positive channel count", ARTHIP_ERR_BUILD);
  if (packed_cap < arthip_conv3x3_packed_halfs(M, C) || bias_cap < arthip_conv3x3_bias_len(M))
    return fail("arthip_conv3x3_pack: output buffer too small", ARTHIP_ERR_BUILD);
  std::vector<float> w(static_cast<size_t>(M) * C * 9);
  for (size_t i = 0; i < w.size(); ++i) w[i] = arthip::f16_to_f32(w_oihw[i]);
  std::vector<float> b(static_cast<size_t>(M), 0.0f);
  if (bias)
    for (int i = 0; i < M; ++i) b[i] = arthip::f16_to_f32(bias[i]);
  if (C == 1)
    arthip::direct_pack(w.data(), M, packed);
  else
    arthip::winograd_pack(w.data(), M, C, packed);
  arthip::bias_pad(b.data(), M, bias_out);
  return ARTHIP_OK;
}

int arthip_conv3x3_f16_nhwc(const void* in, const void* packed, const float* bias, int act,
                            const void* skip0, const void* skip1, void* out, int N, int H, int W,
                            int C, int M, void* stream) {
  if (in == nullptr || packed == nullptr || bias == nullptr || out == nullptr)
    return fail("arthip_conv3x3_f16_nhwc: null buffer", ARTHIP_ERR_BUILD);
  if (N < 1 || H < 1 || W < 1 || C < 1 || M < 1)
    return fail("arthip_conv3x3_f16_nhwc: non-positive dimension", ARTHIP_ERR_BUILD);
  if (act < 0 || act > 2) return fail("arthip_conv3x3_f16_nhwc: unknown activation", ARTHIP_ERR_BUILD);
  if (C > 32 * arthip::winograd_max_kc() || M > arthip::winograd_max_m())
    return fail("arthip_conv3x3_f16_nhwc: channel count beyond kernel limits", ARTHIP_ERR_BUILD);
  arthip::Epilogue e{};
  e.bias = bias;
  e.skip0 = static_cast<const uint16_t*>(skip0);
  e.skip1 = static_cast<const uint16_t*>(skip1);
  e.out = out;
  e.act = act;
  e.out_kind = arthip::kOutNhwcF16;
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t err;
  if (C == 1) {
    arthip::DirectArgs a{};
    a.in = static_cast<const uint16_t*>(in);
    a.w = static_cast<const uint16_t*>(packed);
    a.epi = e;
    a.N = N; a.H = H; a.W = W; a.M = M;
    err = arthip::launch_direct(a, s);
  } else {
    arthip::WinoArgs a{};
    a.in = static_cast<const uint16_t*>(in);
    a.u = static_cast<const uint16_t*>(packed);
    a.epi = e;
    a.N = N; a.H = H; a.W = W; a.C = C; a.M = M;
    err = arthip::launch_winograd(a, s);
  }
  if (err != hipSuccess)
    return fail(std::string("conv3x3 launch failed: ") + hipGetErrorString(err), ARTHIP_ERR_RUN);
  return ARTHIP_OK;
}

}  // extern "C"

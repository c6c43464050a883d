// CPU parts of the ABI: QuantDecoders (AnimaXS/Runtime/Animapk/QuantDecoders.swift:
// 17-164) and the RoPE table builders (DitRoPE.generate, Runtime/Text/DitRoPE.swift:
// 58-107; QwenEncoderMetal.makeRope, Runtime/Metal/QwenEncoderMetal.swift:126-143).
// Pure C++: no HIP headers, no device work.
#include <cmath>
#include <cstdint>
#include <cstring>

#include "anima_hip.h"
#include "status.hpp"

namespace anima {

// binary16 payload -> fp32, subnormals preserved (Float(Float16(bitPattern:))).
static float f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1fu;
  const uint32_t man = h & 0x3ffu;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else {
      const float mag = (float)man * 5.9604644775390625e-8f;  // man * 2^-24, exact
      std::memcpy(&bits, &mag, 4);
      bits |= sign;
    }
  } else if (exp == 0x1f) {
    bits = sign | 0x7f800000u | (man << 13);
  } else {
    bits = sign | ((exp + 112u) << 23) | (man << 13);
  }
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

static void check_decoder(const void* d, const void* s, const void* z, const void* out, int64_t a, int64_t b,
                          int64_t group) {
  if (a < 0 || b < 0 || group <= 0) fail(ANIMA_E_INVALID_SHAPE, "invalid dequant shape or group size");
  if ((a > 0 && b > 0) && (!d || !s || !z || !out)) fail(ANIMA_E_INVALID_ARGUMENT, "dequant pointer is null");
}

}  // namespace anima

using namespace anima;

extern "C" {

anima_status anima_fp16_to_float32(const uint16_t* bits, int64_t count, float* out) {
  return guarded([&] {
    if (count < 0) fail(ANIMA_E_INVALID_SHAPE, "fp16 count must be >= 0");
    if (count > 0 && (!bits || !out)) fail(ANIMA_E_INVALID_ARGUMENT, "fp16 pointer is null");
    for (int64_t i = 0; i < count; ++i) out[i] = f16_to_f32(bits[i]);
  });
}

anima_status anima_dequant_w4(const uint8_t* data, const uint16_t* scale, const uint16_t* zero, int64_t k,
                              int64_t group_size, float* out) {
  return guarded([&] {
    check_decoder(data, scale, zero, out, k, 1, group_size);
    for (int64_t i = 0; i < k; ++i) {
      const uint8_t b = data[i >> 1];
      const uint32_t q = (i & 1) == 0 ? (b & 0x0Fu) : (b >> 4);
      const int64_t g = i / group_size;
      out[i] = (float)q * f16_to_f32(scale[g]) + f16_to_f32(zero[g]);
    }
  });
}

anima_status anima_dequant_w4_matrix(const uint8_t* data, const uint16_t* scale, const uint16_t* zero, int64_t rows,
                                     int64_t cols, int64_t group_size, float* out) {
  return guarded([&] {
    check_decoder(data, scale, zero, out, rows, cols, group_size);
    const int64_t bytes_per_row = (cols + 1) / 2;
    const int64_t groups = (cols + group_size - 1) / group_size;
    for (int64_t r = 0; r < rows; ++r)
      for (int64_t c = 0; c < cols; ++c) {
        const uint8_t b = data[r * bytes_per_row + (c >> 1)];
        const uint32_t q = (c & 1) == 0 ? (b & 0x0Fu) : (b >> 4);
        const int64_t g = r * groups + c / group_size;
        out[r * cols + c] = (float)q * f16_to_f32(scale[g]) + f16_to_f32(zero[g]);
      }
  });
}

anima_status anima_dequant_w8(const uint8_t* data, const uint16_t* scale, const uint16_t* zero, int64_t k,
                              int64_t group_size, float* out) {
  return guarded([&] {
    check_decoder(data, scale, zero, out, k, 1, group_size);
    for (int64_t i = 0; i < k; ++i) {
      const int64_t g = i / group_size;
      out[i] = (float)data[i] * f16_to_f32(scale[g]) + f16_to_f32(zero[g]);
    }
  });
}

anima_status anima_dequant_w8_matrix(const uint8_t* data, const uint16_t* scale, const uint16_t* zero, int64_t rows,
                                     int64_t cols, int64_t group_size, float* out) {
  return guarded([&] {
    check_decoder(data, scale, zero, out, rows, cols, group_size);
    const int64_t groups = (cols + group_size - 1) / group_size;
    for (int64_t r = 0; r < rows; ++r)
      for (int64_t c = 0; c < cols; ++c) {
        const int64_t g = r * groups + c / group_size;
        out[r * cols + c] = (float)data[r * cols + c] * f16_to_f32(scale[g]) + f16_to_f32(zero[g]);
      }
  });
}

anima_status anima_rope_dit3d(int64_t T, int64_t H, int64_t W, float* out) {
  return guarded([&] {
    if (T <= 0 || H <= 0 || W <= 0) fail(ANIMA_E_INVALID_SHAPE, "RoPE grid dims must be positive");
    if (!out) fail(ANIMA_E_INVALID_ARGUMENT, "RoPE output pointer is null");
    const int head_dim = 128;
    const int dim_h = head_dim / 6 * 2, dim_w = dim_h, dim_t = head_dim - 2 * dim_h;  // 42, 42, 44
    const float h_theta = (float)(10000.0 * std::pow(4.0, 42.0 / 40.0));
    const float w_theta = h_theta;
    const float t_theta = (float)(10000.0 * std::pow(1.0, 44.0 / 42.0));
    float f_t[32], f_h[32], f_w[32];
    for (int d = 0; d < dim_t / 2; ++d) f_t[d] = 1.0f / std::pow(t_theta, (float)(d * 2) / (float)dim_t);
    for (int d = 0; d < dim_h / 2; ++d) f_h[d] = 1.0f / std::pow(h_theta, (float)(d * 2) / (float)dim_h);
    for (int d = 0; d < dim_w / 2; ++d) f_w[d] = 1.0f / std::pow(w_theta, (float)(d * 2) / (float)dim_w);
    const int nf = dim_t / 2 + dim_h / 2 + dim_w / 2;  // 64
    int64_t tok = 0;
    auto put = [&](int f, float angle) {
      const float c = std::cos(angle), s = std::sin(angle);
      float* b = out + (tok * nf + f) * 4;
      b[0] = c; b[1] = -s; b[2] = s; b[3] = c;
    };
    for (int64_t t = 0; t < T; ++t)
      for (int64_t h = 0; h < H; ++h)
        for (int64_t w = 0; w < W; ++w) {
          int f = 0;
          for (int d = 0; d < dim_t / 2; ++d) put(f++, (float)t * f_t[d]);
          for (int d = 0; d < dim_h / 2; ++d) put(f++, (float)h * f_h[d]);
          for (int d = 0; d < dim_w / 2; ++d) put(f++, (float)w * f_w[d]);
          ++tok;
        }
  });
}

anima_status anima_rope_neox(int64_t tokens, int64_t head_dim, float theta, float* out) {
  return guarded([&] {
    if (tokens <= 0 || head_dim <= 0 || head_dim % 2) fail(ANIMA_E_INVALID_SHAPE, "invalid NeoX RoPE shape");
    if (!(theta > 0.f) || !std::isfinite(theta)) fail(ANIMA_E_INVALID_ARGUMENT, "RoPE theta must be positive");
    if (!out) fail(ANIMA_E_INVALID_ARGUMENT, "RoPE output pointer is null");
    const int64_t pairs = head_dim / 2;
    for (int64_t t = 0; t < tokens; ++t)
      for (int64_t j = 0; j < pairs; ++j) {
        const float inv = 1.0f / std::pow(theta, (float)(2 * j) / (float)head_dim);
        const float angle = (float)t * inv;
        const float c = std::cos(angle), s = std::sin(angle);
        float* b = out + (t * pairs + j) * 4;
        b[0] = c; b[1] = -s; b[2] = s; b[3] = c;
      }
  });
}

}  // extern "C"

// quant.h -- host-side weight encoders of the product library (run once at
// weight registration; the decode hot path never calls them).
//
//   quant_rows_i8   Lin::load int8 branch (opt125m_decode.rs:41-62) on an
//                   out-major [m,k] matrix: scale = max|row|/127 (1.0 for an
//                   all-zero row), q = round-half-away(w/scale) clamped +-127.
//   f32_to_bf16_bits  npu-xrt/src/lib.rs:809-817 (RNE by integer bias).
//   bfp16_encode    bfp16ebs8 of ffn_bfp16/golden_ffn_gemm.py:21-49: bf16 RNE
//                   first, blocks of 8 along k share e = floor(log2 max|x|),
//                   mantissa = round-half-even(x / 2^(e-6)); +128 (the sim's
//                   overflow case) saturates to 127; stored exponent e + 127.
//   quant_rows_i4   Lin::load int4 branch (opt125m_decode.rs:63-79) on [m,k]:
//                   scale = max|row|/7 (1.0 for an all-zero row), q =
//                   round-half-away(w/scale) clamped +-7, two's-complement
//                   nibbles packed along k (byte j: k = 2j low, 2j+1 high).
//   quant_scale / quant_i8 / dequant_epi   W8A8 (ctx2.rs:1352-1435).
#pragma once

#include <cmath>
#include <cstdint>
#include <cstring>

namespace xe {

inline uint16_t f32_to_bf16_bits(float x) {
  uint32_t bits;
  std::memcpy(&bits, &x, 4);
  if ((bits & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((bits >> 16) | 0x0040u);
  const uint32_t bias = 0x00007fffu + ((bits >> 16) & 1u);
  return static_cast<uint16_t>((bits + bias) >> 16);
}

inline float bf16_round(float x) {
  const uint32_t b = static_cast<uint32_t>(f32_to_bf16_bits(x)) << 16;
  float r;
  std::memcpy(&r, &b, 4);
  return r;
}

inline int8_t quant_i8(float x, float scale) {
  float v = std::round(x / scale);
  if (v != v) return 0;  // Rust's saturating `as i8` maps NaN to 0
  v = v < -127.0f ? -127.0f : (v > 127.0f ? 127.0f : v);
  return static_cast<int8_t>(v);
}

inline float quant_scale(const float *a, size_t n) {
  float amax = 0.f;
  for (size_t i = 0; i < n; i++) {
    const float v = std::fabs(a[i]);
    amax = v > amax ? v : amax;
  }
  return amax > 0.0f ? amax / 127.0f : 1.0f;
}

inline void quant_rows_i8(const float *w, int m, int k, int8_t *q, float *s) {
  for (int r = 0; r < m; r++) {
    const float *row = w + static_cast<size_t>(r) * k;
    float amax = 0.f;
    for (int j = 0; j < k; j++) {
      const float v = std::fabs(row[j]);
      amax = v > amax ? v : amax;
    }
    const float sc = amax > 0.0f ? amax / 127.0f : 1.0f;
    s[r] = sc;
    for (int j = 0; j < k; j++) q[static_cast<size_t>(r) * k + j] = quant_i8(row[j], sc);
  }
}

// qrow of route_b_kernels/decode_fused/gen_decode.py:158-165 (the fused
// decode ELF's static int8 rows): fp32 s = max|row| / 127 (1.0 for an all-zero
// row), q = round half to even of w / s, clamped to +-127; the scale applied
// to the GEMV output is stored as bf16 (w_or_i8, :291-298).
inline void quant_rows_i8_elf(const float *w, int m, int k, int8_t *q, float *s) {
  for (int r = 0; r < m; r++) {
    const float *row = w + static_cast<size_t>(r) * k;
    float amax = 0.f;
    for (int j = 0; j < k; j++) {
      const float v = std::fabs(row[j]);
      amax = v > amax ? v : amax;
    }
    float sc = amax / 127.0f;
    if (!(sc > 0.0f)) sc = 1.0f;
    for (int j = 0; j < k; j++) {
      float v = std::nearbyint(row[j] / sc);
      if (v != v) v = 0.0f;
      v = v < -127.0f ? -127.0f : (v > 127.0f ? 127.0f : v);
      q[static_cast<size_t>(r) * k + j] = static_cast<int8_t>(v);
    }
    s[r] = bf16_round(sc);
  }
}

inline void quant_rows_i4(const float *w, int m, int k, uint8_t *packed, float *s) {
  for (int r = 0; r < m; r++) {
    const float *row = w + static_cast<size_t>(r) * k;
    float amax = 0.f;
    for (int j = 0; j < k; j++) {
      const float v = std::fabs(row[j]);
      amax = v > amax ? v : amax;
    }
    const float sc = amax > 0.0f ? amax / 7.0f : 1.0f;
    s[r] = sc;
    for (int j = 0; j < k; j += 2) {
      unsigned nib[2];
      for (int h = 0; h < 2; h++) {
        float v = std::round(row[j + h] / sc);
        if (v != v) v = 0.0f;
        v = v < -7.0f ? -7.0f : (v > 7.0f ? 7.0f : v);
        nib[h] = static_cast<unsigned>(static_cast<int>(v)) & 0x0Fu;
      }
      packed[static_cast<size_t>(r) * (k / 2) + j / 2] = static_cast<uint8_t>(nib[0] | (nib[1] << 4));
    }
  }
}

inline void bfp16_encode(const float *w, int m, int k, int8_t *mant, uint8_t *exps) {
  const int nb = k / 8;
  for (int r = 0; r < m; r++)
    for (int bk = 0; bk < nb; bk++) {
      float v[8];
      float maxabs = 0.f;
      for (int i = 0; i < 8; i++) {
        v[i] = bf16_round(w[static_cast<size_t>(r) * k + bk * 8 + i]);
        const float a = std::fabs(v[i]);
        maxabs = a > maxabs ? a : maxabs;
      }
      if (maxabs == 0.0f) maxabs = 1.0f;
      int e2 = 0;
      (void)std::frexp(maxabs, &e2);  // maxabs = f * 2^e2, f in [0.5, 1)
      int e = e2 - 1;                 // floor(log2(maxabs))
      e = e < -127 ? -127 : (e > 127 ? 127 : e);
      const float quantum = std::ldexp(1.0f, e - 6);
      for (int i = 0; i < 8; i++) {
        float qv = std::nearbyint(v[i] / quantum);
        qv = qv > 127.0f ? 127.0f : (qv < -128.0f ? -128.0f : qv);
        mant[static_cast<size_t>(r) * k + bk * 8 + i] = static_cast<int8_t>(qv);
      }
      exps[static_cast<size_t>(r) * nb + bk] = static_cast<uint8_t>(e + 127);
    }
}

inline void dequant_epi(const int32_t *acc, int mp, int n, float scale_a, const float *ws,
                        const float *bias, float *out) {
  for (int r = 0; r < mp; r++)
    for (int c = 0; c < n; c++) {
      const float v = static_cast<float>(acc[static_cast<size_t>(r) * n + c]) * scale_a * ws[c];
      out[static_cast<size_t>(r) * n + c] = bias ? v + bias[c] : v;
    }
}

}  // namespace xe

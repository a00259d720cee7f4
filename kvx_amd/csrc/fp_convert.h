// Bit-exact scalar conversions shared by the HIP kernels and host code.
//
// FP8 formats are the OCP ones:
//   E4M3 ("e4m3fn"): 1 sign, 4 exponent (bias 7), 3 mantissa bits; no
//     infinities; S.1111.111 is NaN; largest finite magnitude 448
//     (S.1111.110); subnormals are m * 2^-9.
//   E5M2: 1 sign, 5 exponent (bias 15), 2 mantissa bits, the top byte of an
//     IEEE binary16; S.11111.00 is infinity, S.11111.{01,10,11} NaN; largest
//     finite magnitude 57344 (S.11110.11); subnormals are m * 2^-16.
// Conversions to FP8 saturate: out-of-range values and infinities become the
// largest finite magnitude of the format.  Every routine is written from the
// IEEE-754 / OCP definitions with round-to-nearest-even and is callable on
// both host and device, so the exact device code can be checked exhaustively
// on the CPU.
//
// NaN results are canonical and positive in every format (E4M3 0x7F, E5M2
// 0x7E, bf16 0x7FC0, f16 0x7E00, f32 0x7FC00000): host and device disagree
// on the sign and payload of NaNs produced by arithmetic, so nothing
// downstream may depend on them.
#pragma once

#include <stdint.h>
#include <string.h>

#if defined(__HIPCC__)
#define KVX_HD __host__ __device__ __forceinline__
#else
#define KVX_HD inline
#endif

namespace kvx {

KVX_HD uint32_t f32_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

KVX_HD float bits_f32(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

// f32 -> E4M3 with saturation to +-448 (infinities included), NaN -> 0x7F,
// round-to-nearest-even otherwise.
KVX_HD uint8_t f32_to_e4m3(float v) {
  const uint32_t u = f32_bits(v);
  const uint8_t sign = (uint8_t)((u >> 24) & 0x80u);
  const uint32_t a = u & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return (uint8_t)0x7Fu;                // NaN
  if (a >= 0x43E00000u) return (uint8_t)(sign | 0x7Eu);      // >= 448, inf
  if (a < 0x3C800000u) {                                     // < 2^-6
    // Subnormal range: the code is round_even(|v| * 2^9), an integer in
    // [0, 8]; the value 8 is the smallest normal 2^-6 = code 0x08.
    // |v| * 512 is exact (power-of-two scale of a value >= 2^-149).
    const float scaled = bits_f32(a) * 512.0f;
    const uint32_t q = (uint32_t)scaled;                     // truncation
    const float rem = scaled - (float)q;                      // exact, < 1
    uint32_t r = q;
    if (rem > 0.5f || (rem == 0.5f && (q & 1u))) r = q + 1u;
    return (uint8_t)(sign | r);
  }
  // Normal: keep 3 of the 23 mantissa bits, ties to even; a carry out of the
  // mantissa bumps the exponent, which is the right encoding.  a < 448 so
  // the result never exceeds 0x7E.
  const uint32_t rounded = a + 0x7FFFFu + ((a >> 20) & 1u);
  const uint32_t e8m3 = rounded >> 20;            // (biased exp << 3) | mant
  return (uint8_t)(sign | (uint8_t)(e8m3 - ((127u - 7u) << 3)));
}

// E4M3 -> f32, exact.  Both NaN codes (0x7F, 0xFF) map to 0x7FC00000.
KVX_HD float e4m3_to_f32(uint8_t q) {
  const uint32_t sign = (uint32_t)(q & 0x80u) << 24;
  const uint32_t e = (q >> 3) & 0xFu;
  const uint32_t m = q & 7u;
  if (e == 0xFu && m == 7u) return bits_f32(0x7FC00000u);
  if (e == 0u) {
    const float mag = (float)m * 0.001953125f;  // m * 2^-9, exact
    return bits_f32(sign | f32_bits(mag));
  }
  return bits_f32(sign | ((e + 120u) << 23) | (m << 20));
}

// f32 -> E5M2 with saturation to +-57344 (infinities included), NaN -> 0x7E,
// round-to-nearest-even otherwise.
KVX_HD uint8_t f32_to_e5m2(float v) {
  const uint32_t u = f32_bits(v);
  const uint8_t sign = (uint8_t)((u >> 24) & 0x80u);
  const uint32_t a = u & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return (uint8_t)0x7Eu;                // NaN
  if (a >= 0x47600000u) return (uint8_t)(sign | 0x7Bu);      // >= 57344, inf
  if (a < 0x38800000u) {                                     // < 2^-14
    // Subnormal range: code = round_even(|v| * 2^16), in [0, 4]; 4 is the
    // smallest normal 2^-14 = code 0x04.  |v| * 2^16 is exact.
    const float scaled = bits_f32(a) * 65536.0f;
    const uint32_t q = (uint32_t)scaled;
    const float rem = scaled - (float)q;
    uint32_t r = q;
    if (rem > 0.5f || (rem == 0.5f && (q & 1u))) r = q + 1u;
    return (uint8_t)(sign | r);
  }
  // Normal: keep 2 of the 23 mantissa bits, ties to even; a < 57344 keeps
  // the result at or below 0x7B.
  const uint32_t rounded = a + 0xFFFFFu + ((a >> 21) & 1u);
  const uint32_t e8m2 = rounded >> 21;            // (biased exp << 2) | mant
  return (uint8_t)(sign | (uint8_t)(e8m2 - ((127u - 15u) << 2)));
}

// E5M2 -> f32, exact; infinities kept, every NaN code -> 0x7FC00000.
KVX_HD float e5m2_to_f32(uint8_t q) {
  const uint32_t sign = (uint32_t)(q & 0x80u) << 24;
  const uint32_t e = (q >> 2) & 0x1Fu;
  const uint32_t m = q & 3u;
  if (e == 0x1Fu) return m ? bits_f32(0x7FC00000u) : bits_f32(sign | 0x7F800000u);
  if (e == 0u) {
    const float mag = (float)m * 1.52587890625e-05f;  // m * 2^-16, exact
    return bits_f32(sign | f32_bits(mag));
  }
  return bits_f32(sign | ((e + 112u) << 23) | (m << 21));
}

// f32 -> bf16 bits, round-to-nearest-even; NaN -> 0x7FC0.
KVX_HD uint16_t f32_to_bf16(float f) {
  const uint32_t u = f32_bits(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)0x7FC0u;
  return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

KVX_HD float bf16_to_f32(uint16_t h) { return bits_f32((uint32_t)h << 16); }

// f32 -> IEEE binary16 bits, round-to-nearest-even, overflow -> inf,
// NaN -> 0x7E00, subnormals kept.
KVX_HD uint16_t f32_to_f16(float f) {
  const uint32_t u = f32_bits(f);
  const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  const uint32_t a = u & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return (uint16_t)0x7E00u;
  if (a >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);  // >= 65520
  if (a < 0x38800000u) {                                     // < 2^-14
    // Subnormal: code = round_even(|f| * 2^24), in [0, 1024]; 1024 is the
    // smallest normal.  |f| * 2^24 is exact for |f| >= 2^-149.
    const float scaled = bits_f32(a) * 16777216.0f;
    const uint32_t q = (uint32_t)scaled;
    const float rem = scaled - (float)q;
    uint32_t r = q;
    if (rem > 0.5f || (rem == 0.5f && (q & 1u))) r = q + 1u;
    return (uint16_t)(sign | r);
  }
  const uint32_t rounded = a + 0xFFFu + ((a >> 13) & 1u);
  return (uint16_t)(sign | (uint16_t)((rounded >> 13) - ((127u - 15u) << 10)));
}

// Canonical positive quiet NaN for any NaN input, identity otherwise.
KVX_HD float canon_nan_f32(float f) {
  return ((f32_bits(f) & 0x7FFFFFFFu) > 0x7F800000u) ? bits_f32(0x7FC00000u)
                                                    : f;
}

KVX_HD float f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1Fu;
  const uint32_t m = h & 0x3FFu;
  if (e == 0x1Fu) return bits_f32(sign | 0x7F800000u | (m << 13));
  if (e == 0u) {
    const float mag = (float)m * 5.9604644775390625e-08f;  // m * 2^-24
    return bits_f32(sign | f32_bits(mag));
  }
  return bits_f32(sign | ((e + 112u) << 23) | (m << 13));
}

}  // namespace kvx

// Host-side check of the kernels' scalar casts (kvx_amd/csrc/fp_convert.h,
// the exact source the HIP kernels compile) against the oracle's
// nearest-value casts (oracle/kvx_oracle.c).  Built and run by
// tests/test_oracle.py; prints "<check> <mismatches>" lines.
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <random>

#include "fp_convert.h"
#include "kvx_oracle.h"

using namespace kvx;

static float f_of(uint32_t u) { return bits_f32(u); }

// Every f32 within +-span ulps of x (same sign side).
template <class F>
static void around(float x, int span, F &&f) {
  const uint32_t u = f32_bits(x);
  for (int d = -span; d <= span; ++d) {
    const int64_t v = (int64_t)(u & 0x7FFFFFFFu) + d;
    if (v < 0 || v > 0x7F800000) continue;
    f(f_of((u & 0x80000000u) | (uint32_t)v));
  }
}

int main() {
  std::mt19937_64 rng(12345);
  const float scales[] = {1.0f, 0.25f, 3.0f, 0.0078125f, 0.013671875f,
                          1e-3f, 37.5f, 0.0044642857f, 1e-30f, 6e4f};
  long bad = 0, n = 0;

  // f32 -> e4m3: all bf16 and f16 patterns divided by each scale, random
  // bit patterns, and +-64 ulps around every e4m3 value and midpoint.
  auto chk8 = [&](float v) {
    ++n;
    if (f32_to_e4m3(v) != oracle_f32_to_e4m3(v)) {
      if (bad < 5) fprintf(stderr, "e4m3 %08x: %02x vs %02x\n", f32_bits(v),
                           f32_to_e4m3(v), oracle_f32_to_e4m3(v));
      ++bad;
    }
  };
  for (float s : scales) {
    for (uint32_t h = 0; h < 65536; ++h) {
      volatile float q1 = bf16_to_f32((uint16_t)h) / s;
      chk8(q1);
      volatile float q2 = oracle_f16_to_f32((uint16_t)h) / s;
      chk8(q2);
    }
  }
  for (int i = 0; i < (1 << 22); ++i) chk8(f_of((uint32_t)rng()));
  for (int c = 0; c < 127; ++c) {
    const float v = oracle_e4m3_to_f32((uint8_t)c);
    around(v, 64, chk8);
    around(-v, 64, chk8);
    const float mid = (float)(((double)v + (double)oracle_e4m3_to_f32((uint8_t)(c + 1))) / 2);
    if (c < 126) { around(mid, 64, chk8); around(-mid, 64, chk8); }
  }
  around(448.0f, 4096, chk8);
  around(INFINITY, 4, chk8);
  printf("f32_to_e4m3 %ld of %ld\n", bad, n);

  bad = n = 0;
  for (int c = 0; c < 256; ++c) {
    ++n;
    const float a = e4m3_to_f32((uint8_t)c), b = oracle_e4m3_to_f32((uint8_t)c);
    if (f32_bits(a) != f32_bits(b)) ++bad;
  }
  printf("e4m3_to_f32 %ld of %ld\n", bad, n);

  // f32 -> e5m2: the same input classes, around every e5m2 value and
  // midpoint, the saturation threshold and infinity.
  bad = n = 0;
  auto chk5 = [&](float v) {
    ++n;
    if (f32_to_e5m2(v) != oracle_f32_to_e5m2(v)) {
      if (bad < 5) fprintf(stderr, "e5m2 %08x: %02x vs %02x\n", f32_bits(v),
                           f32_to_e5m2(v), oracle_f32_to_e5m2(v));
      ++bad;
    }
  };
  for (float s : scales) {
    for (uint32_t h = 0; h < 65536; ++h) {
      volatile float q1 = bf16_to_f32((uint16_t)h) / s;
      chk5(q1);
      volatile float q2 = oracle_f16_to_f32((uint16_t)h) / s;
      chk5(q2);
    }
  }
  for (int i = 0; i < (1 << 22); ++i) chk5(f_of((uint32_t)rng()));
  for (int c = 0; c < 124; ++c) {
    const float v = oracle_e5m2_to_f32((uint8_t)c);
    around(v, 64, chk5);
    around(-v, 64, chk5);
    const float mid = (float)(((double)v + (double)oracle_e5m2_to_f32((uint8_t)(c + 1))) / 2);
    if (c < 123) { around(mid, 64, chk5); around(-mid, 64, chk5); }
  }
  around(57344.0f, 1 << 16, chk5);
  around(INFINITY, 4, chk5);
  printf("f32_to_e5m2 %ld of %ld\n", bad, n);

  bad = n = 0;
  for (int c = 0; c < 256; ++c) {
    ++n;
    const float a = e5m2_to_f32((uint8_t)c), b = oracle_e5m2_to_f32((uint8_t)c);
    if (f32_bits(a) != f32_bits(b)) ++bad;
  }
  printf("e5m2_to_f32 %ld of %ld\n", bad, n);

  bad = n = 0;
  auto chkb = [&](float v) {
    ++n;
    if (f32_to_bf16(v) != oracle_f32_to_bf16(v)) ++bad;
  };
  for (int i = 0; i < (1 << 22); ++i) chkb(f_of((uint32_t)rng()));
  for (uint32_t h = 0; h < 65536; ++h) {
    around(f_of((h << 16) | 0x8000u), 2, chkb);  // midpoints
    around(f_of(h << 16), 1, chkb);
  }
  printf("f32_to_bf16 %ld of %ld\n", bad, n);

  bad = n = 0;
  auto chkh = [&](float v) {
    ++n;
    if (f32_to_f16(v) != oracle_f32_to_f16(v)) ++bad;
  };
  for (int i = 0; i < (1 << 22); ++i) chkh(f_of((uint32_t)rng()));
  for (uint32_t h = 0; h < 0x7C00; ++h) {
    const double a = fabs((double)oracle_f16_to_f32((uint16_t)h));
    const double b = (h + 1 < 0x7C00) ? fabs((double)oracle_f16_to_f32((uint16_t)(h + 1)))
                                      : 65536.0;
    around((float)((a + b) / 2), 3, chkh);
    around(-(float)((a + b) / 2), 3, chkh);
  }
  printf("f32_to_f16 %ld of %ld\n", bad, n);

  bad = n = 0;
  for (uint32_t h = 0; h < 65536; ++h) {
    ++n;
    if (f32_bits(f16_to_f32((uint16_t)h)) != f32_bits(oracle_f16_to_f32((uint16_t)h)))
      ++bad;
  }
  printf("f16_to_f32 %ld of %ld\n", bad, n);
  return 0;
}

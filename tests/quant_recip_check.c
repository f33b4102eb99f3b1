// Exhaustive check of the activation quantizers' reciprocal path (quant1_recip in
// llm-serving-engine_amd/csrc/lse_common.h) against their division path (quant1): for every
// positive finite bf16 amax whose scale s = fl32(amax / 127) is at least 2^-100 and every bf16
// v with 0 <= v <= amax,
//   clamp(rne(fl32(v / s)), -127, 127) == clamp(rne(fma(fma(-q0, s, v), y, q0)), -127, 127)
// with y = fl32(1 / s), q0 = fl32(v y). Negative v need no check: every step is odd in v.
// `uncorrected` instead counts how often rne(q0) alone differs (the check must see those).
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float bf16(uint32_t b) {
  const uint32_t u = b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static float clampq(float t) { return fminf(fmaxf(t, -127.0f), 127.0f); }

int main(int argc, char** argv) {
  const int uncorrected = argc > 1 && strcmp(argv[1], "uncorrected") == 0;
  long long rows = 0, pairs = 0, mismatches = 0;
#pragma omp parallel for schedule(dynamic, 64) reduction(+ : rows, pairs, mismatches)
  for (uint32_t ab = 1; ab < 0x7f80; ++ab) {
    const float amax = bf16(ab);
    const float s = amax / 127.0f;
    if (!(s >= 0x1p-100f)) continue;
    ++rows;
    const float y = 1.0f / s;
    for (uint32_t vb = 0; vb <= ab; ++vb) {
      const float v = bf16(vb);
      const float q0 = v * y;
      const float q = uncorrected ? q0 : fmaf(fmaf(-q0, s, v), y, q0);
      mismatches += clampq(rintf(v / s)) != clampq(rintf(q));
      ++pairs;
    }
  }
  printf("rows %lld pairs %lld mismatches %lld\n", rows, pairs, mismatches);
  return 0;
}

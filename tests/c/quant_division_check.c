// Exhaustive check of the quantizer's division by the scale (device function div_by_scale
// in mini-inference-engine_amd/csrc/fp8_common.h) against IEEE single-precision division.
//
// For every amax (positive finite value of the 16-bit format) and every t of the format
// with |t| <= amax (the elements of a group are bounded by its amax) or t NaN:
//   den = max(amax / 448, 1e-12), r = 1 / den            (IEEE, correctly rounded)
//   q0 = t * r, rem = fma(-q0, den, t), q = copysign(fma(rem, r, q0), t)
// must equal t / den bitwise wherever |t / den| >= 2^-12; below that (every such quotient
// becomes an e4m3 zero) only the sign has to match, and NaN must stay NaN with t's sign.
// Usage: quant_division_check b|h   (bf16 or fp16).  Exit status 0 when no mismatch.
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float from_bf16(uint16_t b) {
  const uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static float from_f16(uint16_t h) {
  const int e = (h >> 10) & 0x1f, m = h & 0x3ff;
  float v;
  if (e == 0) v = ldexpf((float)m, -24);
  else if (e == 31) v = m ? NAN : INFINITY;
  else v = ldexpf((float)(m | 0x400), e - 25);
  return (h & 0x8000) ? -v : v;
}

static uint32_t bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

int main(int argc, char** argv) {
  const int fp16 = argc > 1 && argv[1][0] == 'h';
  long long checked = 0, bad = 0;
#pragma omp parallel for schedule(dynamic, 64) reduction(+ : checked, bad)
  for (int ab = 1; ab < 0x8000; ++ab) {
    const float amax = fp16 ? from_f16((uint16_t)ab) : from_bf16((uint16_t)ab);
    if (!isfinite(amax)) continue;
    volatile float k448 = 448.0f;  // keep the division a run-time IEEE division
    const float scale = amax / k448;
    const float den = scale > 1e-12f ? scale : 1e-12f;
    volatile float one = 1.0f;
    const float r = one / den;
    for (int tb = 0; tb < 0x10000; ++tb) {
      const float t = fp16 ? from_f16((uint16_t)tb) : from_bf16((uint16_t)tb);
      if (!isnan(t) && !(fabsf(t) <= amax)) continue;
      const float exact = t / den;
      const float q0 = t * r;
      const float rem = fmaf(-q0, den, t);
      const float q = copysignf(fmaf(rem, r, q0), t);
      ++checked;
      int ok;
      if (isnan(t)) ok = isnan(q) && signbit(q) == signbit(exact);
      else if (fabsf(exact) < 0x1p-12f && fabsf(q) < 0x1p-12f) ok = signbit(q) == signbit(exact);
      else ok = bits(q) == bits(exact);
      if (!ok) {
        if (bad < 5) printf("mismatch amax=%a t=%a exact=%a fast=%a\n", amax, t, exact, q);
        ++bad;
      }
    }
  }
  printf("%s: %lld pairs checked, %lld mismatches\n", fp16 ? "fp16" : "bf16", checked, bad);
  return bad != 0;
}

/* The quantizer kernel's division x / s, computed as q = RN(x y), r = x - q s
 * (one FMA), RN(q + r y) with y = RN(1/s) (Markstein's correction step), must
 * round exactly as the true division for the values the quantizers see.
 * Mode "fp16": every finite fp16 x against every STRIDE-th positive finite
 * fp16 scale s (STRIDE 1 is the exhaustive check, about 2e9 pairs).
 * Mode "fp32": COUNT random fp32 x with s = max(a / qmax, 1e-8) for a row
 * maximum a >= |x|, plus quotients at and next to the rounding ties k + 0.5.
 * The sign of a zero quotient is not compared (rint and the int conversion
 * drop it). Prints the number of pairs and mismatches; exit status 1 on any. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float h2f(uint16_t h) {
  const uint32_t sg = (h >> 15) & 1u, e = (h >> 10) & 31u, m = h & 1023u;
  if (e == 0) {
    const float f = ldexpf((float)m, -24);
    return sg ? -f : f;
  }
  const uint32_t u = (sg << 31) | ((e - 15u + 127u) << 23) | (m << 13);
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static long long bad = 0, pairs = 0;

static void check(float x, float s) {
  const volatile float one = 1.0f, xv = x;
  const float y = one / s;
  const float ref = xv / s;
  const float q = x * y;
  const float got = fmaf(fmaf(-q, s, x), y, q);
  ++pairs;
  if (memcmp(&ref, &got, 4) != 0 && !(ref == 0.0f && got == 0.0f)) {
    if (bad < 5) printf("mismatch x %a s %a: %a vs %a\n", x, s, ref, got);
    ++bad;
  }
}

static uint64_t rs = 88172645463325252ull;
static uint64_t next(void) {
  rs ^= rs << 13;
  rs ^= rs >> 7;
  rs ^= rs << 17;
  return rs;
}

int main(int argc, char** argv) {
  if (argc < 3) return 2;
  if (strcmp(argv[1], "fp16") == 0) {
    const unsigned stride = (unsigned)atoi(argv[2]);
    for (uint32_t sh = 1; sh < 0x7c00u; sh += stride)
      for (uint32_t xh = 0; xh < 0x10000u; ++xh)
        if (((xh >> 10) & 31u) != 31u) check(h2f((uint16_t)xh), h2f((uint16_t)sh));
  } else {
    const long long count = atoll(argv[2]);
    const float inv[2] = {1.0f / 127.0f, 1.0f / 7.0f};
    for (long long i = 0; i < count; ++i) {
      uint32_t u = ((uint32_t)next() & 0xBFFFFFFFu) | 0x20000000u;  /* |x| in [2^-63, 2^65) */
      float x;
      memcpy(&x, &u, 4);
      const float a = fabsf(x) * (1.0f + (float)(next() % 1000000u) * 1e-5f);
      const float s = fmaxf(a * inv[i & 1], 1e-8f);
      check(x, s);
      const float t = ((float)(next() % 127u) + 0.5f) * s;
      check(t, s);
      check(nextafterf(t, 0.0f), s);
      check(nextafterf(t, INFINITY), s);
    }
  }
  printf("pairs %lld mismatches %lld\n", pairs, bad);
  return bad != 0;
}

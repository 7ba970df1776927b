/* Exhaustive check of the quotient the KIVI quantiser forms without a
 * division: for a dividend a >= 0 and divisor b > 0 that are both fp16 (or
 * both bf16) values, with a == 0 or a in [2^-63, 2^63] and b in
 * [2^-63, 2^63],
 *     y = RN(1/b),  q = RN(a * y),  r = fma(-q, b, a),  q' = fma(r, y, q)
 * equals the IEEE fp32 quotient RN(a / b) bit for bit.  Usage: ./check fp16|bf16.
 * Exit status 0 when every pair agrees. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float from_fp16(uint16_t h) {
  const uint32_t e = (h >> 10) & 31, m = h & 1023;
  if (e == 0) return ldexpf((float)m, -24);
  if (e == 31) return m ? NAN : INFINITY;
  return ldexpf((float)(m | 1024), (int)e - 25);
}

static float from_bf16(uint16_t h) {
  const uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static int in_range(float x) { return x >= 0x1p-63f && x <= 0x1p63f; }

int main(int argc, char** argv) {
  const int bf = argc > 1 && strcmp(argv[1], "bf16") == 0;
  const uint32_t top = bf ? 0x7f80u : 0x7c00u; /* first non-finite pattern */
  long long checked = 0, skipped = 0, bad = 0;
  for (uint32_t bh = 1; bh < top; ++bh) {
    const float b = bf ? from_bf16((uint16_t)bh) : from_fp16((uint16_t)bh);
    for (uint32_t ah = 0; ah < top; ++ah) {
      const float a = bf ? from_bf16((uint16_t)ah) : from_fp16((uint16_t)ah);
      if (!in_range(b) || (a != 0.f && !in_range(a))) {
        ++skipped;
        continue;
      }
      const float y = 1.0f / b;
      const float q = a * y;
      const float r = fmaf(-q, b, a);
      const float q1 = fmaf(r, y, q);
      const float want = a / b;
      ++checked;
      if (memcmp(&q1, &want, 4) != 0) {
        if (bad < 5) printf("a=%a b=%a: %a != %a\n", a, b, q1, want);
        ++bad;
      }
    }
  }
  printf("%s: %lld pairs checked, %lld outside the range, %lld differ\n", bf ? "bf16" : "fp16", checked, skipped,
         bad);
  return bad != 0;
}

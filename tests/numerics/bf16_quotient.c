/* Exhaustive check of the bf16 softmax quotient (rowops.hip): for every
 * positive bf16 e <= 1 (denormals included) and every bf16 s in [1, 2^24],
 * the Markstein-corrected product q = fma(fma(-q0, s, e), r, q0), with
 * r = RN(1 / s) and q0 = RN(e * r), rounds to the same bf16 as the IEEE f32
 * quotient e / s (XLA:CPU's bf16 divide).  Prints the number of pairs that
 * differ; exit status 0 when none does.  glibc's fmaf is correctly rounded. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float from_bf16(uint32_t b) {
  const uint32_t u = b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static uint32_t to_bf16(float f) { /* round to nearest even; finite inputs */
  uint32_t u;
  memcpy(&u, &f, 4);
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

int main(void) {
  long bad = 0, n = 0;
  for (uint32_t sb = 0x3F80; sb <= 0x4B80; ++sb) {
    const float s = from_bf16(sb), r = 1.0f / s;
    for (uint32_t eb = 0x0001; eb <= 0x3F80; ++eb) {
      const float e = from_bf16(eb);
      const float q0 = e * r;
      const float q = fmaf(fmaf(-q0, s, e), r, q0);
      if (to_bf16(q) != to_bf16(e / s)) ++bad;
      ++n;
    }
  }
  printf("%ld of %ld pairs differ\n", bad, n);
  return bad != 0;
}

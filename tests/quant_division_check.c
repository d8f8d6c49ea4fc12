/* Exhaustive check of the quotient used by the bf16 row quantizers.
 *
 * The per-token int8 recipe computes code = clamp(rint(x / s), -127, 127) with
 * s = amax / 127 (0 -> 1), x / s correctly rounded.  For bf16 rows the GPU kernels use
 * Markstein's corrected quotient instead of a full division:
 *     r = RN(1 / s)   (one correctly rounded division per row)
 *     y0 = RN(x * r);  rem = fma(-y0, s, x);  y1 = RN(rem * r + y0)
 * (P. Markstein, "Computation of elementary functions on the IBM RISC System/6000
 * processor", IBM J. Res. Dev. 34(1), 1990).  It is used only when s >= 2^-120; rows with
 * a smaller scale keep the division.
 *
 * This program walks every positive finite bf16 amax and every bf16 x with |x| <= amax
 * (about 1.07e9 pairs) and counts pairs whose code differs between the two formulas.
 * Exit status 0 iff no pair with s >= 2^-120 differs.  It also reports the pairs below
 * the cut-off that would differ, which is why the cut-off exists.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float bf16(uint32_t h) {
  uint32_t u = h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static float code(float q) { return fminf(fmaxf(rintf(q), -127.f), 127.f); }

int main(void) {
  long long pairs = 0, bad_fast = 0, bad_below = 0;
#pragma omp parallel for schedule(dynamic, 64) reduction(+ : pairs, bad_fast, bad_below)
  for (int ha = 1; ha < 0x7f80; ++ha) {
    const float amax = bf16((uint32_t)ha);
    float s = amax / 127.0f;
    if (s == 0.f) s = 1.f;
    const float r = 1.0f / s;
    const int fast = s >= 0x1p-120f;
    for (uint32_t hx = 0; hx < 0x10000; ++hx) {
      if ((int)(hx & 0x7fff) > ha) continue;
      const float x = bf16(hx);
      const float y0 = x * r;
      const float y1 = fmaf(fmaf(-y0, s, x), r, y0);
      ++pairs;
      if (code(x / s) != code(y1)) {
        if (fast) ++bad_fast;
        else ++bad_below;
      }
    }
  }
  printf("pairs %lld; code mismatches with s >= 2^-120: %lld; below the cut-off: %lld\n", pairs, bad_fast,
         bad_below);
  return bad_fast != 0 || pairs < 1000000000LL;
}

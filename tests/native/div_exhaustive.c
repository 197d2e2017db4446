/* Exhaustive check of the prologue's three-operation quotient for a constant divisor.
 *
 * For every non-negative finite fp32 x (bit patterns 0 .. 0x7f7fffff), computes
 *     y = RN(1/s), q = RN(x*y), e = RN(q*s - x) (fma), r = RN(q - e*y) (fma)
 * exactly as `div_by` in sageattention-rdna4_amd/csrc/sage_device.h does, and compares r with the
 * IEEE correctly rounded x / s bit for bit. Built with gcc without fast-math (fmaf is the C
 * library's correctly rounded fused multiply-add; SSE float arithmetic rounds each operation once,
 * FLT_EVAL_METHOD 0). Denormals are kept (no FTZ/DAZ), as the gfx950 kernels keep fp32 denormals.
 *
 * The quantizers use the quotient of a row's absmax as a scale floored at 1e-12:
 * max(RN(x / s), floor). So besides the raw mismatches the program counts the mismatches whose
 * correct quotient is a normal number, and the mismatches that survive the floor.
 *
 * usage: div_exhaustive <divisor> <floor> [variant]
 * variant 0 (default) is the device sequence; 1 and 2 are planted mistakes the check must catch:
 * 1 drops the correction (r = q = RN(x*y)), 2 forms the residual without the fma
 * (e = RN(RN(q*s) - x), no longer exact).
 * prints "checked N mismatches M normal_quotient_mismatches A floored_mismatches F max_bad_x X"
 * and up to 8 mismatching x
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float f_of(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t u_of(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

int main(int argc, char** argv) {
  if (argc != 3 && argc != 4) return 2;
  const volatile float s = (float)atof(argv[1]);
  const volatile float floor_ = (float)atof(argv[2]);
  const int variant = argc == 4 ? atoi(argv[3]) : 0;
  const float y = 1.0f / s;
  const uint32_t last = 0x7f7fffffu;
  uint64_t bad = 0, bad_normal = 0, bad_floored = 0;
  uint32_t first_bad[8], max_bad = 0;
#pragma omp parallel for schedule(static, 1 << 20) reduction(+ : bad, bad_normal, bad_floored) reduction(max : max_bad)
  for (int64_t i = 0; i <= (int64_t)last; ++i) {
    const float x = f_of((uint32_t)i);
    const float q = x * y;
    float r;
    if (variant == 1) {
      r = q;
    } else if (variant == 2) {
      volatile float qs = q * s;
      const float e = qs - x;
      r = fmaf(-e, y, q);
    } else {
      const float e = fmaf(q, s, -x);
      r = fmaf(-e, y, q);
    }
    const float ref = x / s;
    if (u_of(r) != u_of(ref)) {
      uint64_t k;
#pragma omp atomic capture
      k = bad++;
      if (k < 8) first_bad[k] = (uint32_t)i;
      if (fabsf(ref) >= 0x1p-126f) bad_normal++;
      if (u_of(fmaxf(r, floor_)) != u_of(fmaxf(ref, floor_))) bad_floored++;
      if ((uint32_t)i > max_bad) max_bad = (uint32_t)i;
    }
  }
  /* the loop's reduction hides the order: the first 8 recorded are some 8 mismatches */
  printf("checked %llu mismatches %llu normal_quotient_mismatches %llu floored_mismatches %llu "
         "max_bad_x %a\n", (unsigned long long)last + 1, (unsigned long long)bad,
         (unsigned long long)bad_normal, (unsigned long long)bad_floored, f_of(max_bad));
  for (uint64_t k = 0; k < bad && k < 8; ++k)
    printf("x=%a (0x%08x) got %a want %a\n", f_of(first_bad[k]), first_bad[k],
           fmaf(-fmaf(f_of(first_bad[k]) * y, s, -f_of(first_bad[k])), y, f_of(first_bad[k]) * y),
           f_of(first_bad[k]) / s);
  return 0;
}

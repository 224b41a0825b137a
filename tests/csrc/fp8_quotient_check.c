/* Exhaustive check of the FP8 pack kernel's quotient for 16-bit inputs.
 *
 * The kernel (morph_amd/csrc/fp8.hip) divides each element x of a 256-element
 * block by the block scale s = max(amax / 448, 1e-30) (streamtrain/precision.py:
 * 27-31) as Markstein's correction of x * (1 / s):
 *     y = RN(1 / s); t = RN(x y); r = RN(x - t s) (an fma); q = RN(t + r y) (an fma)
 * instead of one IEEE division per element.  For every FP16 (or BF16) block
 * maximum amax and every element x with |x| <= amax, this program compares q
 * with the IEEE quotient x / s, and the E4M3FN bytes the two encode to (after
 * the clamp to +-448).  Output: "<pairs> <quotient mismatches> <byte
 * mismatches> <largest |x / s| among the quotient mismatches>".  The kernel
 * runs the sequence on |x| and puts x's sign back (a -0 element stays -0), so
 * the non-negative elements checked here cover the negative ones too.
 * Built with -ffp-contract=off; the C library's fmaf is the IEEE fused
 * multiply-add.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float from_bits(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t to_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

static float half_to_float(uint32_t h) {  /* IEEE binary16, exact */
  const uint32_t e = (h >> 10) & 0x1F, m = h & 0x3FF;
  if (e == 0) return ldexpf((float)m, -24);
  if (e == 31) return m ? NAN : INFINITY;
  return from_bits(((e + 112) << 23) | (m << 13));
}

/* E4M3FN round to nearest even after the clamp (the format definition). */
static uint32_t e4m3fn(float x) {
  if (!isnan(x)) x = x < -448.f ? -448.f : (x > 448.f ? 448.f : x);
  const uint32_t u = to_bits(x), sign = (u >> 24) & 0x80u, a = u & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return sign | 0x7Fu;
  uint32_t r;
  if (a < 0x3C800000u) {
    r = (uint32_t)rintf(from_bits(a) * 512.0f);
  } else {
    r = ((a + 0x7FFFFu + ((a >> 20) & 1u)) >> 20) - (120u << 3);
    if (r > 0x7Eu) r = 0x7Fu;
  }
  return sign | r;
}

int main(int argc, char** argv) {
  const int bf16 = argc > 1 && strcmp(argv[1], "bf16") == 0;
  static float vals[32768];
  int nv = 0;
  for (uint32_t h = 0; h < 0x8000; ++h) {  /* positive patterns, ascending */
    const float f = bf16 ? from_bits(h << 16) : half_to_float(h);
    if (isfinite(f)) vals[nv++] = f;
  }
  long long pairs = 0, qbad = 0, bbad = 0;
  float worst = 0.f;
  for (int a = 0; a < nv; ++a) {
    float s = vals[a] / 448.0f;
    if (s < 1e-30f) s = 1e-30f;
    const float y = 1.0f / s;
    for (int k = 0; k <= a; ++k) {
      const float x = vals[k], ref = x / s;
      const float t = x * y;
      const float r = fmaf(-t, s, x);
      const float q = fmaf(r, y, t);
      ++pairs;
      if (to_bits(q) != to_bits(ref)) {
        ++qbad;
        if (fabsf(ref) > worst) worst = fabsf(ref);
        if (e4m3fn(q) != e4m3fn(ref)) ++bbad;
      }
    }
  }
  printf("%lld %lld %lld %a\n", pairs, qbad, bbad, worst);
  return 0;
}

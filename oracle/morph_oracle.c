/*
 * morph_oracle.c -- CPU restatement of MORPH's optimizer-step arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (morph_amd/) links,
 * loads or calls this file; only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py use it, as the checker.
 *
 * Built with -ffp-contract=off so that every multiply and add rounds
 * separately, and fmaf() appears exactly where torch's CPU kernels fuse.
 * Which torch ops fuse was established by running the installed torch and
 * is pinned by tests/test_oracle_adamw.py against torch.optim.AdamW
 * (bit-exact) and against the reference op sequence of
 * streamtrain/disk.py:209-215 run through torch (bit-exact):
 *   Tensor.lerp_(end, w), w < 0.5    -> fmaf(w, end - self, self)
 *   Tensor.lerp_(end, w), w >= 0.5   -> fmaf(w - 1, end - self, end)
 *   Tensor.addcmul_(a, b, value=c)   -> fmaf(c * a, b, self)
 *   Tensor.addcdiv_(a, b, value=c)   -> self + (c * a) / b
 *   Tensor / python_float            -> true division by (float)scalar
 *   Tensor.mul_(python_float)        -> self * (float)scalar
 *   Tensor.add_(x, alpha=c)          -> fmaf(x, c, self)   (pinned by
 *                                       tests/test_oracle_muon.py, the Muon update)
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#include "../include/morph_optim.h"

static float bits_to_f32(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static uint32_t f32_to_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

/* IEEE binary16 -> binary32, exact (every half is a float). */
static float f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1Fu;
  uint32_t man = h & 0x3FFu;
  if (exp == 0x1Fu) return bits_to_f32(sign | 0x7F800000u | (man << 13));
  if (exp == 0) {
    /* zero or subnormal: man * 2^-24 is exact in binary32 */
    float v = (float)man * 0x1p-24f;
    return sign ? -v : v;
  }
  return bits_to_f32(sign | ((exp + 112u) << 23) | (man << 13));
}

static float bf16_to_f32(uint16_t b) { return bits_to_f32((uint32_t)b << 16); }

/*
 * binary32 -> binary16, round to nearest even, from the IEEE 754 definition:
 * overflow to infinity, gradual underflow, NaN -> canonical quiet NaN (as
 * torch's c10::Half).  Pinned against numpy.astype(float16) for non-NaN input
 * (export.py:33 uses astype('<f2')) and torch .to(float16).
 */
static uint16_t f32_to_f16_rne(float f) {
  uint32_t x = f32_to_bits(f);
  uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  uint32_t ax = x & 0x7FFFFFFFu;
  if (ax > 0x7F800000u) return (uint16_t)(sign | 0x7E00u); /* canonical quiet NaN */
  if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* >= 65520 rounds to inf */
  int e = (int)(ax >> 23) - 127;
  if (e < -25) return sign; /* below half the smallest subnormal: +-0 */
  uint32_t man = (ax & 0x7FFFFFu) | 0x800000u; /* 24-bit significand */
  if (e >= -14) {
    /* normal half: keep 11 bits, drop 13 */
    uint32_t keep = man >> 13, rest = man & 0x1FFFu;
    uint32_t h = ((uint32_t)(e + 15) << 10) + (keep - 0x400u);
    if (rest > 0x1000u || (rest == 0x1000u && (keep & 1u))) h += 1u; /* carry may reach exp */
    return (uint16_t)(sign | h);
  }
  /* subnormal half: value = man * 2^(e-23); unit = 2^-24 -> shift = -e - 1 */
  int shift = -e - 1; /* 14..24 */
  uint32_t keep = man >> shift, rest = man & ((1u << shift) - 1u), half = 1u << (shift - 1);
  if (rest > half || (rest == half && (keep & 1u))) keep += 1u;
  return (uint16_t)(sign | keep);
}

/* binary32 -> bfloat16, round to nearest even; NaN -> quiet NaN (torch c10::BFloat16). */
static uint16_t f32_to_bf16_rne(float f) {
  uint32_t x = f32_to_bits(f);
  if ((x & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u;
  uint32_t lsb = (x >> 16) & 1u;
  return (uint16_t)((x + 0x7FFFu + lsb) >> 16);
}

static float load_grad(const void* g, int dtype, int64_t i) {
  switch (dtype) {
    case MORPH_DTYPE_F16: return f16_to_f32(((const uint16_t*)g)[i]);
    case MORPH_DTYPE_BF16: return bf16_to_f32(((const uint16_t*)g)[i]);
    default: return ((const float*)g)[i];
  }
}

static int is_nonfinite_bits(const void* g, int dtype, int64_t i) {
  switch (dtype) {
    case MORPH_DTYPE_F16: return (((const uint16_t*)g)[i] & 0x7C00u) == 0x7C00u;
    case MORPH_DTYPE_BF16: return (((const uint16_t*)g)[i] & 0x7F80u) == 0x7F80u;
    default: return (((const uint32_t*)g)[i] & 0x7F800000u) == 0x7F800000u;
  }
}

/* ---- exported oracle entry points (ctypes) ---- */

void oracle_f32_to_f16(const float* x, uint16_t* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = f32_to_f16_rne(x[i]);
}

void oracle_f32_to_bf16(const float* x, uint16_t* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = f32_to_bf16_rne(x[i]);
}

void oracle_f16_to_f32(const uint16_t* x, float* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = f16_to_f32(x[i]);
}

/*
 * Any non-finite element.  Restates optimizer.py:49-51 and the norm test of
 * disk.py:466-468 / 485: sqrt(sum(g.double()**2)) is non-finite iff some
 * element is +-inf or NaN (a finite binary32 squared cannot overflow binary64,
 * and fewer than 2^64 of them cannot sum to overflow).
 */
int oracle_nonfinite_any(const void* g, int dtype, int64_t n) {
  for (int64_t i = 0; i < n; ++i)
    if (is_nonfinite_bits(g, dtype, i)) return 1;
  return 0;
}

/*
 * One AdamW step on n elements, in place on w/m/v, optional export.
 * Follows torch/optim/adam.py:414-419 (decay), 457 (lerp), 476 (mul+addcmul),
 * 528-547 (bias-corrected denominator and addcdiv), with the gradient first
 * unscaled (disk.py:447, sparse_disk.py:107: g.float()/loss_scale) and
 * clipped (disk.py:210: gradient * clip).
 */
void oracle_adamw(const void* grad, int grad_dtype, float* w, float* m, float* v, void* out,
                  int out_dtype, int64_t n, const morph_adamw_hp* hp) {
  const uint32_t fl = hp->flags;
  for (int64_t i = 0; i < n; ++i) {
    float g = load_grad(grad, grad_dtype, i);
    g = g / hp->scale;
    if (fl & MORPH_HP_APPLY_CLIP) g = g * hp->clip;
    float p = w[i];
    if (fl & MORPH_HP_APPLY_DECAY) p = p * hp->decay;
    float mm = m[i];
    if (fl & MORPH_HP_LERP_LARGE)
      mm = fmaf(hp->lerp_weight - 1.0f, g - mm, g);
    else
      mm = fmaf(hp->lerp_weight, g - mm, mm);
    float vv = v[i] * hp->beta2;
    vv = fmaf(hp->one_minus_beta2 * g, g, vv);
    float d = sqrtf(vv) / hp->bias_correction2_sqrt + hp->eps;
    p = p + (hp->neg_step_size * mm) / d;
    w[i] = p;
    m[i] = mm;
    v[i] = vv;
    if (out) {
      if (out_dtype == MORPH_DTYPE_F16)
        ((uint16_t*)out)[i] = f32_to_f16_rne(p);
      else if (out_dtype == MORPH_DTYPE_BF16)
        ((uint16_t*)out)[i] = f32_to_bf16_rne(p);
      else if (out_dtype == MORPH_DTYPE_F32)
        ((float*)out)[i] = p;
    }
  }
}

/*
 * Muon momentum + Nesterov blend (optimizer.py:58-59), elementwise:
 *   momentum.lerp_(grad, mom_w)            mom_w = 0.05 < 0.5
 *   u = grad.lerp(momentum, nesterov_w)    nesterov_w = 0.95 >= 0.5
 */
void oracle_muon_momentum(const float* grad, float* momentum, float* u, int64_t n, float mom_w,
                          float nesterov_w) {
  for (int64_t i = 0; i < n; ++i) {
    float g = grad[i];
    float mm = momentum[i];
    mm = (mom_w < 0.5f) ? fmaf(mom_w, g - mm, mm) : fmaf(mom_w - 1.0f, g - mm, g);
    momentum[i] = mm;
    u[i] = (nesterov_w < 0.5f) ? fmaf(nesterov_w, mm - g, g) : fmaf(nesterov_w - 1.0f, mm - g, mm);
  }
}

/*
 * Muon master update (optimizer.py:60-61):
 *   update *= scale;  p.mul_(decay).add_(update, alpha=neg_lr)
 */
void oracle_muon_apply(float* p, const float* update, int64_t n, float scale, float decay,
                       float neg_lr) {
  for (int64_t i = 0; i < n; ++i) {
    float u = update[i] * scale;
    float q = p[i] * decay;
    p[i] = fmaf(u, neg_lr, q);
  }
}

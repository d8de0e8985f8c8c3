/*
 * aicpu_oracle.c -- CPU oracle for the conv-as-GEMM path (TEST INFRASTRUCTURE).
 *
 * Checker only: loaded by tests/, the smoke check and bench.py's cpu_baseline
 * leg, never by the product.  Each function cites the reference file:line it
 * restates; paths are relative to the reference repository root.
 *
 * Arithmetic contract: built with -ffp-contract=off, so `a += x * w` rounds the
 * product and the sum separately, exactly like the reference's x86 scalar
 * F32x4 fallback (crates/ai-cpu/src/simd.rs:220-227) and its naive oracle
 * (crates/ai-core/src/reference/conv.rs:48, Rust never contracts).
 */
#include "aicpu_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* ai-core                                                                   */
/* ------------------------------------------------------------------------ */

static inline uint32_t div_ceil_u32(uint32_t a, uint32_t b) { return (a + b - 1) / b; }
static inline uint32_t next_mult_u32(uint32_t a, uint32_t m) { return div_ceil_u32(a, m) * m; }

/* Conv2d::out_hw -- crates/ai-core/src/ops/conv.rs:49-56 */
void orc_out_hw(const orc_conv2d *op, uint32_t ih, uint32_t iw, uint32_t *oh, uint32_t *ow) {
  uint32_t ekh = op->dil * (op->kh - 1) + 1;
  uint32_t ekw = op->dil * (op->kw - 1) + 1;
  *oh = (ih + op->pad[0] + op->pad[2] - ekh) / op->sh + 1;
  *ow = (iw + op->pad[1] + op->pad[3] - ekw) / op->sw + 1;
}

/* Rust f32::max / f32::min: NaN operands yield the other operand. */
static inline float rmax(float a, float b) { return isnan(a) ? b : (isnan(b) ? a : (a > b ? a : b)); }
static inline float rmin(float a, float b) { return isnan(a) ? b : (isnan(b) ? a : (a < b ? a : b)); }
/* Rust f32::clamp: NaN passes through. */
static inline float rclamp(float x, float lo, float hi) {
  if (x < lo) x = lo;
  if (x > hi) x = hi;
  return x;
}

/* Activation::apply -- crates/ai-core/src/activation.rs:28-43 */
float orc_act_apply(int32_t act, float x) {
  switch (act) {
    case ORC_ACT_NONE: return x;
    case ORC_ACT_RELU: return rmax(x, 0.0f);
    case ORC_ACT_SIGMOID: return 1.0f / (1.0f + expf(-x));
    case ORC_ACT_TANH: return tanhf(x);
    case ORC_ACT_HARDSWISH: return x * rclamp(x / 6.0f + 0.5f, 0.0f, 1.0f);
    case ORC_ACT_HARDSIGMOID: return rclamp(x / 6.0f + 0.5f, 0.0f, 1.0f);
    case ORC_ACT_CLAMP01: return rclamp(x, 0.0f, 1.0f);
    case ORC_ACT_RELU6: return rclamp(x, 0.0f, 6.0f);
    case ORC_ACT_SQRT: return sqrtf(rmax(x, 0.0f));
    case ORC_ACT_NEG: return -x;
    case ORC_ACT_RECIP: return 1.0f / x;
    default: return x;
  }
}

void orc_act_apply_n(int32_t act, const float *x, float *y, size_t n) {
  for (size_t i = 0; i < n; ++i) y[i] = orc_act_apply(act, x[i]);
}

/* ai-cpu apply4 -- crates/ai-cpu/src/kernels/mod.rs:21-50.  Differs from the
 * scalar apply for the hard activations: it multiplies by (1/6) instead of
 * dividing by 6, and chains max/min instead of clamp. */
void orc_act_apply4(int32_t act, float v[4]) {
  const float sixth = 1.0f / 6.0f;
  for (int l = 0; l < 4; ++l) {
    float x = v[l];
    switch (act) {
      case ORC_ACT_NONE: break;
      case ORC_ACT_RELU: x = rmax(x, 0.0f); break;
      case ORC_ACT_HARDSWISH: x = x * rmin(rmax(x * sixth + 0.5f, 0.0f), 1.0f); break;
      case ORC_ACT_HARDSIGMOID: x = rmin(rmax(x * sixth + 0.5f, 0.0f), 1.0f); break;
      case ORC_ACT_CLAMP01: x = rmin(rmax(x, 0.0f), 1.0f); break;
      case ORC_ACT_RELU6: x = rmin(rmax(x, 0.0f), 6.0f); break;
      case ORC_ACT_NEG: x = x * -1.0f; break;
      default: x = orc_act_apply(act, x); break;
    }
    v[l] = x;
  }
}

/* XorShift32 -- crates/ai-core/src/rng.rs:3-35 */
uint32_t orc_xs32_seed(uint32_t seed) { return seed == 0 ? 0x9e3779b9u : seed; }

uint32_t orc_xs32_next(uint32_t *s) {
  uint32_t x = *s;
  x ^= x << 13;
  x ^= x >> 17;
  x ^= x << 5;
  *s = x;
  return x;
}

/* top 24 bits -> [0,1) -> [-1,1) (rng.rs:20-23) */
float orc_xs32_next_f32(uint32_t *s) {
  return (float)(orc_xs32_next(s) >> 8) / (float)(1u << 24) * 2.0f - 1.0f;
}

void orc_xs32_fill(uint32_t seed, float *out, size_t n) {
  uint32_t s = orc_xs32_seed(seed);
  for (size_t i = 0; i < n; ++i) out[i] = orc_xs32_next_f32(&s);
}

/* No reference counterpart (the reference defines no Gaussian).  Box-Muller:
 * u1 = ((x1 >> 8) + 1) / 2^24 in (0,1], u2 = (x2 >> 8) / 2^24 in [0,1),
 * z = sqrt(-2 ln u1) * cos(2 pi u2) in double; one normal per two draws. */
void orc_gauss_fill(uint32_t seed, float mean, float sigma, float *out, size_t n) {
  uint32_t s = orc_xs32_seed(seed);
  const double two_pi = 6.283185307179586476925286766559;
  for (size_t i = 0; i < n; ++i) {
    double u1 = (double)((orc_xs32_next(&s) >> 8) + 1u) / 16777216.0;
    double u2 = (double)(orc_xs32_next(&s) >> 8) / 16777216.0;
    double z = sqrt(-2.0 * log(u1)) * cos(two_pi * u2);
    out[i] = (float)((double)mean + (double)sigma * z);
  }
}

/* f32 -> IEEE binary16, round to nearest even (what half::f16::from_f32 does,
 * crates/ai-core/src/pack.rs:20). */
uint16_t orc_f32_to_f16(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  uint32_t sign = (u >> 16) & 0x8000u;
  uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((a >> 13) & 0x3ffu)); /* NaN */
  if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);                       /* -> inf */
  if (a < 0x38800000u) {                                                           /* f16 subnormal */
    uint32_t e = a >> 23;
    if (e == 0) return (uint16_t)sign;
    uint32_t mant = (a & 0x7fffffu) | 0x800000u;
    uint32_t shift = 126u - e;
    if (shift > 24) return (uint16_t)sign;
    uint32_t q = mant >> shift;
    uint32_t rem = mant & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return (uint16_t)(sign | q);
  }
  uint32_t r = a - 0x38000000u; /* rebias exponent 127 -> 15 */
  r = r + 0xfffu + ((r >> 13) & 1u);
  return (uint16_t)(sign | (r >> 13));
}

float orc_f16_to_f32(uint16_t h) {
  uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 0x1fu;
  uint32_t m = h & 0x3ffu;
  uint32_t u;
  if (e == 0) {
    if (m == 0) {
      u = sign;
    } else { /* subnormal: m * 2^-24 is exact in f32 */
      float f = (float)m * (1.0f / 16777216.0f);
      memcpy(&u, &f, 4);
      u |= sign;
    }
  } else if (e == 31) {
    u = sign | 0x7f800000u | (m << 13);
  } else {
    u = sign | ((e + 112u) << 23) | (m << 13);
  }
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* No reference counterpart (ai-core has no bf16): f32 -> bfloat16 RNE. */
uint16_t orc_f32_to_bf16(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float orc_bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

size_t orc_dtype_bytes(int32_t dt) { return dt == ORC_F32 ? 4 : 2; }

static inline void store_elem(void *out, size_t i, float v, int32_t dt) {
  if (dt == ORC_F32) ((float *)out)[i] = v;
  else if (dt == ORC_F16) ((uint16_t *)out)[i] = orc_f32_to_f16(v);
  else ((uint16_t *)out)[i] = orc_f32_to_bf16(v);
}

static inline float load_elem(const void *in, size_t i, int32_t dt) {
  if (dt == ORC_F32) return ((const float *)in)[i];
  if (dt == ORC_F16) return orc_f16_to_f32(((const uint16_t *)in)[i]);
  return orc_bf16_to_f32(((const uint16_t *)in)[i]);
}

void orc_cvt_from_f32(int32_t dt, const float *in, void *out, size_t n) {
  for (size_t i = 0; i < n; ++i) store_elem(out, i, in[i], dt);
}

void orc_cvt_to_f32(int32_t dt, const void *in, float *out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = load_elem(in, i, dt);
}

/* TensorDesc::size_bytes with the batch added (tensor.rs:51-64) */
size_t orc_nhwc_c4_bytes(uint32_t n, uint32_t h, uint32_t w, uint32_t c, int32_t dt) {
  return (size_t)n * h * w * div_ceil_u32(c, 4) * 4 * orc_dtype_bytes(dt);
}

/* pack_nhwc -- pack.rs:34-47, index TensorDesc::idx (tensor.rs:72-74); batch
 * is the outermost dimension (no reference counterpart: n is always 1 there). */
void orc_pack_nhwc(const float *data, uint32_t n, uint32_t h, uint32_t w, uint32_t c, int32_t dt,
                   void *out) {
  uint32_t cg = div_ceil_u32(c, 4);
  size_t px = (size_t)n * h * w;
  for (size_t p = 0; p < px; ++p)
    for (uint32_t ch = 0; ch < cg * 4; ++ch)
      store_elem(out, p * cg * 4 + ch, ch < c ? data[p * c + ch] : 0.0f, dt);
}

/* unpack_nhwc -- pack.rs:50-64 */
void orc_unpack_nhwc(const void *bytes, uint32_t n, uint32_t h, uint32_t w, uint32_t c, int32_t dt,
                     float *out) {
  uint32_t cg = div_ceil_u32(c, 4);
  size_t px = (size_t)n * h * w;
  for (size_t p = 0; p < px; ++p)
    for (uint32_t ch = 0; ch < c; ++ch) out[p * c + ch] = load_elem(bytes, p * cg * 4 + ch, dt);
}

/* pack_weights_conv -- pack.rs:68-102 (index formula :95, kg padding :78) */
uint32_t orc_pack_weights_conv(const float *w, uint32_t cout, uint32_t cin, uint32_t kh,
                               uint32_t kw, uint32_t kg_align, int32_t dt, void *out) {
  uint32_t kg = next_mult_u32(div_ceil_u32(cin, 4), kg_align ? kg_align : 1);
  uint32_t ng = div_ceil_u32(cout, 4);
  uint32_t taps = kh * kw;
  for (uint32_t t = 0; t < taps; ++t) {
    uint32_t ky = t / kw, kx = t % kw;
    for (uint32_t kgi = 0; kgi < kg; ++kgi)
      for (uint32_t ngi = 0; ngi < ng; ++ngi)
        for (uint32_t j = 0; j < 4; ++j)
          for (uint32_t comp = 0; comp < 4; ++comp) {
            uint32_t oc = ngi * 4 + j, ic = kgi * 4 + comp;
            float v = (oc < cout && ic < cin) ? w[(((size_t)oc * cin + ic) * kh + ky) * kw + kx] : 0.0f;
            store_elem(out, ((((size_t)t * kg + kgi) * ng + ngi) * 4 + j) * 4 + comp, v, dt);
          }
  }
  return kg;
}

/* unpack_weights_conv -- pack.rs:125-156 */
void orc_unpack_weights_conv(const void *bytes, uint32_t cout, uint32_t cin, uint32_t kh,
                             uint32_t kw, uint32_t kg_pad, int32_t dt, float *out) {
  uint32_t ng = div_ceil_u32(cout, 4);
  for (uint32_t t = 0; t < kh * kw; ++t) {
    uint32_t ky = t / kw, kx = t % kw;
    for (uint32_t kgi = 0; kgi < div_ceil_u32(cin, 4); ++kgi)
      for (uint32_t ngi = 0; ngi < ng; ++ngi)
        for (uint32_t j = 0; j < 4; ++j)
          for (uint32_t comp = 0; comp < 4; ++comp) {
            uint32_t oc = ngi * 4 + j, ic = kgi * 4 + comp;
            if (oc < cout && ic < cin)
              out[(((size_t)oc * cin + ic) * kh + ky) * kw + kx] =
                  load_elem(bytes, ((((size_t)t * kg_pad + kgi) * ng + ngi) * 4 + j) * 4 + comp, dt);
          }
  }
}

/* pack_weights_dw -- pack.rs:105-122: tap-major [tap][cg][comp] */
void orc_pack_weights_dw(const float *w, uint32_t c, uint32_t kh, uint32_t kw, int32_t dt,
                         void *out) {
  uint32_t cg = div_ceil_u32(c, 4), taps = kh * kw;
  for (uint32_t cgi = 0; cgi < cg; ++cgi)
    for (uint32_t t = 0; t < taps; ++t)
      for (uint32_t comp = 0; comp < 4; ++comp) {
        uint32_t ch = cgi * 4 + comp;
        store_elem(out, ((size_t)t * cg + cgi) * 4 + comp, ch < c ? w[(size_t)ch * taps + t] : 0.0f, dt);
      }
}

/* unpack_weights_dw -- pack.rs:159-170 */
void orc_unpack_weights_dw(const void *bytes, uint32_t c, uint32_t kh, uint32_t kw, int32_t dt,
                           float *out) {
  uint32_t taps = kh * kw, cg = div_ceil_u32(c, 4);
  for (uint32_t ch = 0; ch < c; ++ch)
    for (uint32_t t = 0; t < taps; ++t)
      out[(size_t)ch * taps + t] = load_elem(bytes, ((size_t)t * cg + ch / 4) * 4 + ch % 4, dt);
}

/* pack_bias -- pack.rs:178-184 */
void orc_pack_bias(const float *b, uint32_t cout, int32_t dt, void *out) {
  uint32_t ng = div_ceil_u32(cout, 4);
  for (uint32_t i = 0; i < ng * 4; ++i) store_elem(out, i, i < cout ? b[i] : 0.0f, dt);
}

/* unpack_bias -- pack.rs:173-175 */
void orc_unpack_bias(const void *bytes, uint32_t cout, int32_t dt, float *out) {
  for (uint32_t i = 0; i < cout; ++i) out[i] = load_elem(bytes, i, dt);
}

/* reference::conv::conv2d -- crates/ai-core/src/reference/conv.rs:9-62:
 * bias-first sequential accumulation over (ky, kx, icg), skip padded taps,
 * then act, then + residual. */
int orc_conv2d_ref(const orc_conv2d *op, uint32_t ih, uint32_t iw, const float *input,
                   const float *weights, const float *bias, const float *residual, float *out) {
  if (op->groups == 0 || op->cin % op->groups || op->cout % op->groups) return -1;
  uint32_t cin_g = op->cin / op->groups, cout_g = op->cout / op->groups;
  uint32_t oh, ow;
  orc_out_hw(op, ih, iw, &oh, &ow);
  for (uint32_t oy = 0; oy < oh; ++oy)
    for (uint32_t ox = 0; ox < ow; ++ox)
      for (uint32_t oc = 0; oc < op->cout; ++oc) {
        uint32_t g = oc / cout_g;
        float acc = bias ? bias[oc] : 0.0f;
        for (uint32_t ky = 0; ky < op->kh; ++ky)
          for (uint32_t kx = 0; kx < op->kw; ++kx) {
            int64_t iy = (int64_t)(oy * op->sh + ky * op->dil) - op->pad[0];
            int64_t ix = (int64_t)(ox * op->sw + kx * op->dil) - op->pad[1];
            if (iy < 0 || iy >= ih || ix < 0 || ix >= iw) continue;
            for (uint32_t icg = 0; icg < cin_g; ++icg) {
              uint32_t ic = g * cin_g + icg;
              float iv = input[((size_t)iy * iw + (size_t)ix) * op->cin + ic];
              float wv = weights[(((size_t)oc * cin_g + icg) * op->kh + ky) * op->kw + kx];
              acc += iv * wv;
            }
          }
        size_t idx = ((size_t)oy * ow + ox) * op->cout + oc;
        float v = orc_act_apply(op->act, acc);
        if (residual) v += residual[idx];
        out[idx] = v;
      }
  return 0;
}

/* ------------------------------------------------------------------------ */
/* ai-cpu kernels                                                            */
/* ------------------------------------------------------------------------ */

#define NR 8
#define MR_BIG 8

/* conv::repack_weights -- crates/ai-cpu/src/kernels/conv.rs:44-66 */
uint32_t orc_cpu_repack_weights(const float *w, uint32_t cout, uint32_t cin, uint32_t cin_pad,
                                uint32_t kh, uint32_t kw, float *out) {
  uint32_t cout_pad = next_mult_u32(cout, NR), taps = kh * kw;
  memset(out, 0, sizeof(float) * (size_t)taps * cin_pad * cout_pad);
  for (uint32_t oc = 0; oc < cout; ++oc)
    for (uint32_t ic = 0; ic < cin; ++ic)
      for (uint32_t t = 0; t < taps; ++t)
        out[((size_t)t * cin_pad + ic) * cout_pad + oc] = w[((size_t)oc * cin + ic) * taps + t];
  return cout_pad;
}

static inline size_t vbase(const orc_view *v, size_t lin_px) { return lin_px * v->stride + v->c_off; }

/* floor division for a positive divisor (i64::div_euclid) */
static inline int64_t div_floor(int64_t a, int64_t b) {
  int64_t q = a / b;
  if ((a % b) != 0 && ((a < 0) != (b < 0))) q -= 1;
  return q;
}

typedef struct {
  const orc_conv2d *op;
  uint32_t ih, iw, ow, cout, cout_pad, cin_total, nparts;
  const orc_view *views;
  const uint32_t *ic0, *c4;
  const float *wts, *bias;
  const orc_view *res;
  float *out;
  size_t px_base;
} std_ctx;

/* conv::epilogue -- conv.rs:190-232 */
static inline __attribute__((always_inline)) void std_epilogue(const std_ctx *c, const float acc[NR],
                                                                size_t px, size_t oc0) {
  size_t cout = c->cout;
  size_t o = (px - c->px_base) * cout + oc0;
  size_t nc = cout - oc0;
  float *out = c->out;
  if (nc >= NR) {
    float v0[4] = {acc[0], acc[1], acc[2], acc[3]};
    float v1[4] = {acc[4], acc[5], acc[6], acc[7]};
    orc_act_apply4(c->op->act, v0);
    orc_act_apply4(c->op->act, v1);
    if (c->res) {
      size_t rb = vbase(c->res, px) + oc0;
      for (int l = 0; l < 4; ++l) {
        v0[l] = v0[l] + c->res->data[rb + l];
        v1[l] = v1[l] + c->res->data[rb + 4 + l];
      }
    }
    for (int l = 0; l < 4; ++l) {
      out[o + l] = v0[l];
      out[o + 4 + l] = v1[l];
    }
  } else {
    size_t l0 = 0;
    if (nc >= 4) {
      float v0[4] = {acc[0], acc[1], acc[2], acc[3]};
      orc_act_apply4(c->op->act, v0);
      if (c->res) {
        size_t rb = vbase(c->res, px) + oc0;
        for (int l = 0; l < 4; ++l) v0[l] = v0[l] + c->res->data[rb + l];
      }
      for (int l = 0; l < 4; ++l) out[o + l] = v0[l];
      l0 = 4;
    }
    for (size_t l = l0; l < nc; ++l) {
      float v = orc_act_apply(c->op->act, acc[l]);
      if (c->res) v += c->res->data[vbase(c->res, px) + oc0 + l];
      out[o + l] = v;
    }
  }
}

/* conv::mr_n -- conv.rs:238-316: MR interior pixels x NR channels, no bounds
 * checks.  Per output the accumulation order is bias, then (ky, kx, part, ic);
 * each step `acc += a * w` rounds twice (x86 fallback, simd.rs:221-227). */
static inline __attribute__((always_inline)) void std_mr_n(const int MR, const std_ctx *c,
                                                            const uint32_t (*ky_list)[2], int n_ky,
                                                            size_t oy, size_t ox, size_t oc0) {
  float acc[MR_BIG][NR];
  for (int p = 0; p < MR; ++p)
    for (int j = 0; j < NR; ++j) acc[p][j] = c->bias[oc0 + j];
  const orc_conv2d *op = c->op;
  size_t sw = op->sw, dil = op->dil, pl = op->pad[1], kw = op->kw, cp = c->cout_pad;
  for (int r = 0; r < n_ky; ++r) {
    size_t t_row = ky_list[r][0], iy = ky_list[r][1];
    for (size_t kx = 0; kx < kw; ++kx) {
      size_t t = t_row + kx;
      size_t ix0 = ox * sw + kx * dil - pl;
      size_t row = iy * c->iw;
      for (uint32_t pi = 0; pi < c->nparts; ++pi) {
        const orc_view *v = &c->views[pi];
        size_t base[MR_BIG];
        for (int p = 0; p < MR; ++p) base[p] = vbase(v, row + ix0 + (size_t)p * sw);
        const float *x = v->data;
        size_t pc = v->c, c4 = c->c4[pi];
        size_t w_idx = (t * c->cin_total + c->ic0[pi]) * cp + oc0;
        size_t ic = 0;
        while (ic + 4 <= c4) {
          float a[MR_BIG][4];
          for (int p = 0; p < MR; ++p)
            for (int l = 0; l < 4; ++l) a[p][l] = x[base[p] + ic + l];
          for (int l = 0; l < 4; ++l) {
            const float *w = c->wts + w_idx;
            for (int p = 0; p < MR; ++p)
              for (int j = 0; j < NR; ++j) acc[p][j] += a[p][l] * w[j];
            w_idx += cp;
          }
          ic += 4;
        }
        while (ic < pc) {
          const float *w = c->wts + w_idx;
          for (int p = 0; p < MR; ++p) {
            float a = x[base[p] + ic];
            for (int j = 0; j < NR; ++j) acc[p][j] += a * w[j];
          }
          w_idx += cp;
          ic += 1;
        }
      }
    }
  }
  for (int p = 0; p < MR; ++p) std_epilogue(c, acc[p], oy * c->ow + ox + p, oc0);
}

/* conv::mr1 -- conv.rs:405-468: one edge pixel with per-kx bounds checks */
static void std_mr1(const std_ctx *c, const uint32_t (*ky_list)[2], int n_ky, size_t oy, size_t ox,
                    size_t oc0) {
  float acc[NR];
  for (int j = 0; j < NR; ++j) acc[j] = c->bias[oc0 + j];
  const orc_conv2d *op = c->op;
  int64_t sw = op->sw, dil = op->dil, pl = op->pad[1];
  size_t kw = op->kw, cp = c->cout_pad;
  for (int r = 0; r < n_ky; ++r) {
    size_t t_row = ky_list[r][0], iy = ky_list[r][1];
    for (size_t kx = 0; kx < kw; ++kx) {
      int64_t ix = (int64_t)ox * sw + (int64_t)kx * dil - pl;
      if (ix < 0 || ix >= (int64_t)c->iw) continue;
      size_t t = t_row + kx;
      size_t lin = iy * c->iw + (size_t)ix;
      for (uint32_t pi = 0; pi < c->nparts; ++pi) {
        const orc_view *v = &c->views[pi];
        size_t base = vbase(v, lin);
        const float *x = v->data;
        size_t pc = v->c, c4 = c->c4[pi];
        size_t w_idx = (t * c->cin_total + c->ic0[pi]) * cp + oc0;
        size_t ic = 0;
        while (ic + 4 <= c4) {
          float a[4] = {x[base + ic], x[base + ic + 1], x[base + ic + 2], x[base + ic + 3]};
          for (int l = 0; l < 4; ++l) {
            const float *w = c->wts + w_idx;
            for (int j = 0; j < NR; ++j) acc[j] += a[l] * w[j];
            w_idx += cp;
          }
          ic += 4;
        }
        while (ic < pc) {
          const float *w = c->wts + w_idx;
          float a = x[base + ic];
          for (int j = 0; j < NR; ++j) acc[j] += a * w[j];
          w_idx += cp;
          ic += 1;
        }
      }
    }
  }
  std_epilogue(c, acc, oy * c->ow + ox, oc0);
}

/* conv::conv_std -- conv.rs:81-185 (native: NR8, MR_BIG 8; the wasm-only
 * mr4_nr16 path is not taken on x86). */
void orc_cpu_conv_std(const orc_conv2d *op, uint32_t ih, uint32_t iw, const orc_view *views,
                      const uint32_t *ic0, const uint32_t *c4, uint32_t nparts, const float *wts,
                      const float *bias, uint32_t cout_pad, const orc_view *residual, float *out,
                      uint32_t y0, uint32_t y1) {
  uint32_t oh, ow;
  orc_out_hw(op, ih, iw, &oh, &ow);
  (void)oh;
  std_ctx c;
  c.op = op;
  c.ih = ih;
  c.iw = iw;
  c.ow = ow;
  c.cout = op->cout;
  c.cout_pad = cout_pad;
  c.cin_total = 0;
  for (uint32_t i = 0; i < nparts; ++i) c.cin_total += c4[i];
  c.nparts = nparts;
  c.views = views;
  c.ic0 = ic0;
  c.c4 = c4;
  c.wts = wts;
  c.bias = bias;
  c.res = residual;
  c.out = out;
  c.px_base = (size_t)y0 * ow;

  int64_t sh = op->sh, sw = op->sw, dil = op->dil, pt = op->pad[0], pl = op->pad[1];
  int64_t kw = op->kw;
  int64_t lo = 0, hi = (int64_t)ow - 1;
  for (int64_t kx = 0; kx < kw; ++kx) {
    int64_t off = kx * dil - pl;
    int64_t mn = div_floor(-off + sw - 1, sw);
    if (mn < 0) mn = 0;
    int64_t mx = div_floor((int64_t)iw - 1 - off, sw);
    if (mn > lo) lo = mn;
    if (mx < hi) hi = mx;
  }

  for (size_t oy = y0; oy < y1; ++oy) {
    uint32_t ky_list[16][2];
    int n_ky = 0;
    for (int64_t ky = 0; ky < (int64_t)op->kh; ++ky) {
      int64_t iy = (int64_t)oy * sh + ky * dil - pt;
      if (iy >= 0 && iy < (int64_t)ih) {
        ky_list[n_ky][0] = (uint32_t)(ky * kw);
        ky_list[n_ky][1] = (uint32_t)iy;
        n_ky++;
      }
    }
    for (size_t oc0 = 0; oc0 < c.cout; oc0 += NR) {
      size_t ox = 0;
      while (ox < ow) {
#define INB(n) ((int64_t)ox >= lo && (int64_t)(ox + (n) - 1) <= hi && ox + (n) <= ow)
        if (INB(MR_BIG)) {
          std_mr_n(MR_BIG, &c, (const uint32_t(*)[2])ky_list, n_ky, oy, ox, oc0);
          ox += MR_BIG;
        } else if (INB(4)) {
          std_mr_n(4, &c, (const uint32_t(*)[2])ky_list, n_ky, oy, ox, oc0);
          ox += 4;
        } else {
          std_mr1(&c, (const uint32_t(*)[2])ky_list, n_ky, oy, ox, oc0);
          ox += 1;
        }
#undef INB
      }
    }
  }
}

/* dw::repack_weights -- crates/ai-cpu/src/kernels/dw.rs:22-34 */
uint32_t orc_cpu_repack_weights_dw(const float *w, uint32_t c, uint32_t kh, uint32_t kw, float *out) {
  uint32_t c_pad = next_mult_u32(c, 4), taps = kh * kw;
  memset(out, 0, sizeof(float) * (size_t)taps * c_pad);
  for (uint32_t ch = 0; ch < c; ++ch)
    for (uint32_t t = 0; t < taps; ++t) out[(size_t)t * c_pad + ch] = w[(size_t)ch * taps + t];
  return c_pad;
}

/* dw::edge_px -- dw.rs:209-264 */
static void dw_edge_px(const orc_conv2d *op, uint32_t iw, const orc_view *in, const float *wts,
                       const float *bias, const orc_view *res, float *out,
                       const uint32_t (*ky_list)[2], int n_ky, size_t oy, size_t ox, size_t ow,
                       size_t px_base, size_t c, size_t c_pad, size_t cv) {
  int64_t sw = op->sw, dil = op->dil, pl = op->pad[1];
  size_t kw = op->kw;
  size_t px_out = oy * ow + ox;
  size_t out_base = (px_out - px_base) * c;
  for (size_t cc = 0; cc < cv; cc += 4) {
    float acc[4] = {bias[cc], bias[cc + 1], bias[cc + 2], bias[cc + 3]};
    for (int r = 0; r < n_ky; ++r) {
      size_t t_row = ky_list[r][0], iy = ky_list[r][1];
      for (size_t kx = 0; kx < kw; ++kx) {
        int64_t ix = (int64_t)ox * sw + (int64_t)kx * dil - pl;
        if (ix < 0 || ix >= (int64_t)iw) continue;
        size_t base = vbase(in, iy * iw + (size_t)ix);
        const float *w = wts + (t_row + kx) * c_pad + cc;
        for (int l = 0; l < 4; ++l) acc[l] += in->data[base + cc + l] * w[l];
      }
    }
    orc_act_apply4(op->act, acc);
    if (res) {
      size_t rb = vbase(res, px_out) + cc;
      for (int l = 0; l < 4; ++l) acc[l] = acc[l] + res->data[rb + l];
    }
    for (int l = 0; l < 4; ++l) out[out_base + cc + l] = acc[l];
  }
  for (size_t ch = cv; ch < c; ++ch) {
    float acc = bias[ch];
    for (int r = 0; r < n_ky; ++r) {
      size_t t_row = ky_list[r][0], iy = ky_list[r][1];
      for (size_t kx = 0; kx < kw; ++kx) {
        int64_t ix = (int64_t)ox * sw + (int64_t)kx * dil - pl;
        if (ix < 0 || ix >= (int64_t)iw) continue;
        size_t base = vbase(in, iy * iw + (size_t)ix);
        acc += in->data[base + ch] * wts[(t_row + kx) * c_pad + ch];
      }
    }
    float v = orc_act_apply(op->act, acc);
    if (res) v += res->data[vbase(res, px_out) + ch];
    out[out_base + ch] = v;
  }
}

/* dw::conv_dw -- dw.rs:40-204: interior pixels use a per-(row, channel block)
 * table of tap offsets and run four pixels at a time; edges check each kx.
 * Per output the order is bias, then taps in (ky, kx) order. */
void orc_cpu_conv_dw(const orc_conv2d *op, uint32_t ih, uint32_t iw, const orc_view *in,
                     const float *wts, const float *bias, const orc_view *res, float *out,
                     uint32_t y0, uint32_t y1) {
  size_t c = op->cout, c_pad = next_mult_u32(op->cout, 4);
  uint32_t oh_u, ow_u;
  orc_out_hw(op, ih, iw, &oh_u, &ow_u);
  size_t ow = ow_u;
  int64_t sh = op->sh, sw = op->sw, dil = op->dil, pt = op->pad[0], pl = op->pad[1];
  size_t cv = c / 4 * 4, kw = op->kw;
  int64_t lo = 0, hi = (int64_t)ow - 1;
  for (int64_t kx = 0; kx < (int64_t)kw; ++kx) {
    int64_t off = kx * dil - pl;
    int64_t mn = div_floor(-off + sw - 1, sw);
    if (mn < 0) mn = 0;
    int64_t mx = div_floor((int64_t)iw - 1 - off, sw);
    if (mn > lo) lo = mn;
    if (mx < hi) hi = mx;
  }
  size_t x_lo = (size_t)(lo < 0 ? 0 : (lo > (int64_t)ow ? (int64_t)ow : lo));
  int64_t xh = hi + 1;
  if (xh < (int64_t)x_lo) xh = (int64_t)x_lo;
  if (xh > (int64_t)ow) xh = (int64_t)ow;
  size_t x_hi = (size_t)xh;
  size_t px_base = (size_t)y0 * ow;
  enum { MAX_TAPS = 32 };

  for (size_t oy = y0; oy < y1; ++oy) {
    uint32_t ky_list[16][2];
    int n_ky = 0;
    for (int64_t ky = 0; ky < (int64_t)op->kh; ++ky) {
      int64_t iy = (int64_t)oy * sh + ky * dil - pt;
      if (iy >= 0 && iy < (int64_t)ih) {
        ky_list[n_ky][0] = (uint32_t)(ky * (int64_t)kw);
        ky_list[n_ky][1] = (uint32_t)iy;
        n_ky++;
      }
    }
    const uint32_t(*kl)[2] = (const uint32_t(*)[2])ky_list;
    for (size_t ox = 0; ox < x_lo; ++ox)
      dw_edge_px(op, iw, in, wts, bias, res, out, kl, n_ky, oy, ox, ow, px_base, c, c_pad, cv);
    if (x_hi > x_lo && op->kh * op->kw <= MAX_TAPS) {
      size_t step = (size_t)sw * in->stride;
      for (size_t cc = 0; cc < cv; cc += 4) {
        size_t off0[MAX_TAPS];
        float wv[MAX_TAPS][4];
        size_t nt = 0;
        for (int r = 0; r < n_ky; ++r)
          for (size_t kx = 0; kx < kw; ++kx) {
            size_t ix = (size_t)((int64_t)x_lo * sw + (int64_t)kx * dil - pl);
            off0[nt] = vbase(in, (size_t)kl[r][1] * iw + ix) + cc;
            for (int l = 0; l < 4; ++l) wv[nt][l] = wts[(kl[r][0] + kx) * c_pad + cc + l];
            nt++;
          }
        size_t out_idx = (oy * ow + x_lo - px_base) * c + cc;
        size_t r_idx = res ? vbase(res, oy * ow + x_lo) + cc : 0;
        size_t px_off = 0;
        size_t ox = x_lo;
        for (; ox + 4 <= x_hi; ox += 4) {
          float acc[4][4];
          for (int p = 0; p < 4; ++p)
            for (int l = 0; l < 4; ++l) acc[p][l] = bias[cc + l];
          for (size_t t = 0; t < nt; ++t) {
            size_t o = off0[t] + px_off;
            for (int p = 0; p < 4; ++p)
              for (int l = 0; l < 4; ++l) acc[p][l] += in->data[o + p * step + l] * wv[t][l];
          }
          for (int p = 0; p < 4; ++p) {
            orc_act_apply4(op->act, acc[p]);
            if (res) {
              for (int l = 0; l < 4; ++l) acc[p][l] = acc[p][l] + res->data[r_idx + l];
              r_idx += res->stride;
            }
            for (int l = 0; l < 4; ++l) out[out_idx + l] = acc[p][l];
            out_idx += c;
          }
          px_off += 4 * step;
        }
        for (; ox < x_hi; ++ox) {
          float acc[4] = {bias[cc], bias[cc + 1], bias[cc + 2], bias[cc + 3]};
          for (size_t t = 0; t < nt; ++t)
            for (int l = 0; l < 4; ++l) acc[l] += in->data[off0[t] + px_off + l] * wv[t][l];
          orc_act_apply4(op->act, acc);
          if (res) {
            for (int l = 0; l < 4; ++l) acc[l] = acc[l] + res->data[r_idx + l];
            r_idx += res->stride;
          }
          for (int l = 0; l < 4; ++l) out[out_idx + l] = acc[l];
          out_idx += c;
          px_off += step;
        }
      }
      for (size_t ch = cv; ch < c; ++ch) {
        size_t off0[MAX_TAPS];
        float ws[MAX_TAPS];
        size_t nt = 0;
        for (int r = 0; r < n_ky; ++r)
          for (size_t kx = 0; kx < kw; ++kx) {
            size_t ix = (size_t)((int64_t)x_lo * sw + (int64_t)kx * dil - pl);
            off0[nt] = vbase(in, (size_t)kl[r][1] * iw + ix) + ch;
            ws[nt] = wts[(kl[r][0] + kx) * c_pad + ch];
            nt++;
          }
        size_t out_idx = (oy * ow + x_lo - px_base) * c + ch;
        size_t r_idx = res ? vbase(res, oy * ow + x_lo) + ch : 0;
        size_t px_off = 0;
        for (size_t ox = x_lo; ox < x_hi; ++ox) {
          float acc = bias[ch];
          for (size_t t = 0; t < nt; ++t) acc += in->data[off0[t] + px_off] * ws[t];
          float v = orc_act_apply(op->act, acc);
          if (res) {
            v += res->data[r_idx];
            r_idx += res->stride;
          }
          out[out_idx] = v;
          out_idx += c;
          px_off += step;
        }
      }
    } else {
      for (size_t ox = x_lo; ox < x_hi; ++ox)
        dw_edge_px(op, iw, in, wts, bias, res, out, kl, n_ky, oy, ox, ow, px_base, c, c_pad, cv);
    }
    for (size_t ox = x_hi; ox < ow; ++ox)
      dw_edge_px(op, iw, in, wts, bias, res, out, kl, n_ky, oy, ox, ow, px_base, c, c_pad, cv);
  }
}

/* im2row::im2row -- crates/ai-cpu/src/kernels/im2row.rs:22-86: patches
 * [out_px][k_pad] in (ky, kx, ic) order; out holds oh*ow*k_pad + 4 floats. */
void orc_cpu_im2row(const orc_conv2d *op, uint32_t ih, uint32_t iw, const orc_view *input,
                    uint32_t k_pad, float *out) {
  uint32_t oh, ow;
  orc_out_hw(op, ih, iw, &oh, &ow);
  size_t c = input->c, kh = op->kh, kw = op->kw, sh = op->sh, sw = op->sw;
  int64_t pt = op->pad[0], pl = op->pad[1];
  size_t row_k = kw * c;
  const float *d = input->data;
  for (size_t oy = 0; oy < oh; ++oy) {
    size_t iy_of[16];
    for (size_t ky = 0; ky < 16; ++ky) iy_of[ky] = (size_t)-1;
    for (size_t ky = 0; ky < kh && ky < 16; ++ky) {
      int64_t iy = (int64_t)(oy * sh + ky) - pt;
      if (iy >= 0 && iy < (int64_t)ih) iy_of[ky] = (size_t)iy;
    }
    for (size_t ox = 0; ox < ow; ++ox) {
      int64_t ix0 = (int64_t)(ox * sw) - pl;
      size_t dst_px = (oy * ow + ox) * k_pad;
      int interior_x = ix0 >= 0 && ix0 + (int64_t)kw <= (int64_t)iw;
      for (size_t ky = 0; ky < kh; ++ky) {
        size_t dst = dst_px + ky * row_k;
        size_t iy = iy_of[ky];
        if (iy == (size_t)-1) {
          for (size_t o = 0; o < row_k; o += 4)
            for (int l = 0; l < 4; ++l) out[dst + o + l] = 0.0f;
          continue;
        }
        if (interior_x) {
          size_t src = (iy * iw + (size_t)ix0) * c;
          for (size_t o = 0; o < row_k; o += 4)
            for (int l = 0; l < 4; ++l) out[dst + o + l] = d[src + o + l];
        } else {
          for (size_t kx = 0; kx < kw; ++kx) {
            int64_t ix = ix0 + (int64_t)kx;
            for (size_t ch = 0; ch < c; ++ch)
              out[dst + kx * c + ch] = (ix >= 0 && ix < (int64_t)iw) ? d[(iy * iw + (size_t)ix) * c + ch] : 0.0f;
          }
        }
      }
    }
  }
}

/* im2row::permute_weights -- im2row.rs:89-102: OIHW -> [cout][(ky,kx,ic)] */
void orc_cpu_permute_weights(const float *w, uint32_t cout, uint32_t cin, uint32_t kh, uint32_t kw,
                             float *out) {
  size_t k = (size_t)kh * kw * cin;
  for (size_t oc = 0; oc < cout; ++oc)
    for (size_t ic = 0; ic < cin; ++ic)
      for (size_t t = 0; t < (size_t)kh * kw; ++t)
        out[oc * k + t * cin + ic] = w[(oc * cin + ic) * kh * kw + t];
}

/* pw_dot::conv_pw_dot -- crates/ai-cpu/src/kernels/pw_dot.rs:32-61 (weights
 * [cout][k_pad], repack_weights :19-28): 4-lane partial sums, horizontal sum
 * (a0+a1)+(a2+a3) (simd.rs:285-287), then act(sum + bias). */
void orc_cpu_conv_pw_dot(const orc_conv2d *op, const orc_view *input, const float *wts,
                         uint32_t k_pad, const float *bias, uint32_t px, float *out) {
  size_t cout = op->cout;
  for (size_t p = 0; p < px; ++p) {
    size_t b = vbase(input, p);
    float acc[4][4] = {{0}};
    for (size_t kc = 0; kc < k_pad; kc += 4)
      for (size_t oc = 0; oc < cout; ++oc)
        for (int l = 0; l < 4; ++l) acc[oc][l] += input->data[b + kc + l] * wts[oc * k_pad + kc + l];
    for (size_t oc = 0; oc < cout; ++oc) {
      float s = (acc[oc][0] + acc[oc][1]) + (acc[oc][2] + acc[oc][3]);
      out[p * cout + oc] = orc_act_apply(op->act, s + bias[oc]);
    }
  }
}

/* ------------------------------------------------------------------------ */
/* Row-band thread pool (stands in for the rayon pool of model.rs:70-84)     */
/* ------------------------------------------------------------------------ */

typedef void (*band_fn)(void *ctx, uint32_t y0, uint32_t y1, float *out_chunk);

typedef struct {
  pthread_mutex_t mu;
  pthread_cond_t cv_work, cv_done;
  int nthreads; /* workers, excluding the caller */
  pthread_t *th;
  unsigned long gen;
  int pending;
  /* current job */
  band_fn fn;
  void *ctx;
  uint32_t rows, band, nbands;
  size_t chunk_len;
  float *out;
  int next;
} pool_t;

static pool_t g_pool = {PTHREAD_MUTEX_INITIALIZER, PTHREAD_COND_INITIALIZER, PTHREAD_COND_INITIALIZER,
                        0, NULL, 0, 0, NULL, NULL, 0, 0, 0, 0, NULL, 0};

static int pool_take(pool_t *p) {
  int i = __atomic_fetch_add(&p->next, 1, __ATOMIC_RELAXED);
  return i < (int)p->nbands ? i : -1;
}

static void pool_run_band(pool_t *p, int i) {
  uint32_t y0 = (uint32_t)i * p->band;
  uint32_t y1 = y0 + p->band;
  if (y1 > p->rows) y1 = p->rows;
  p->fn(p->ctx, y0, y1, p->out + (size_t)i * p->chunk_len);
}

static void *pool_worker(void *arg) {
  pool_t *p = (pool_t *)arg;
  unsigned long seen = 0;
  for (;;) {
    pthread_mutex_lock(&p->mu);
    while (p->gen == seen) pthread_cond_wait(&p->cv_work, &p->mu);
    seen = p->gen;
    pthread_mutex_unlock(&p->mu);
    int i;
    while ((i = pool_take(p)) >= 0) pool_run_band(p, i);
    pthread_mutex_lock(&p->mu);
    if (--p->pending == 0) pthread_cond_signal(&p->cv_done);
    pthread_mutex_unlock(&p->mu);
  }
  return NULL;
}

static void pool_ensure(int workers) {
  pool_t *p = &g_pool;
  if (p->nthreads >= workers) return;
  pthread_t *th = (pthread_t *)realloc(p->th, sizeof(pthread_t) * (size_t)workers);
  if (!th) return;
  p->th = th;
  for (int i = p->nthreads; i < workers; ++i) {
    pthread_create(&p->th[i], NULL, pool_worker, p);
    pthread_detach(p->th[i]);
  }
  p->nthreads = workers;
}

/* model.rs:421-436: band = ceil(rows / threads); out is cut into chunks of
 * band * row_len floats and chunk i covers rows [i*band, min((i+1)*band, rows)). */
static void run_bands(int threads, uint32_t rows, size_t row_len, float *out, band_fn fn, void *ctx) {
  pool_t *p = &g_pool;
  uint32_t band = div_ceil_u32(rows, (uint32_t)threads);
  uint32_t nbands = div_ceil_u32(rows, band);
  pool_ensure(threads - 1);
  int workers = p->nthreads < threads - 1 ? p->nthreads : threads - 1;
  pthread_mutex_lock(&p->mu);
  p->fn = fn;
  p->ctx = ctx;
  p->rows = rows;
  p->band = band;
  p->nbands = nbands;
  p->chunk_len = (size_t)band * row_len;
  p->out = out;
  p->next = 0;
  p->pending = p->nthreads; /* every worker wakes on a new generation */
  p->gen++;
  pthread_cond_broadcast(&p->cv_work);
  pthread_mutex_unlock(&p->mu);
  (void)workers;
  int i;
  while ((i = pool_take(p)) >= 0) pool_run_band(p, i);
  pthread_mutex_lock(&p->mu);
  while (p->pending > 0) pthread_cond_wait(&p->cv_done, &p->mu);
  pthread_mutex_unlock(&p->mu);
}

/* ------------------------------------------------------------------------ */
/* plan::lower Conv arm + model::dispatch                                    */
/* ------------------------------------------------------------------------ */

struct orc_cpu_op {
  orc_conv2d op, pw;
  uint32_t ih, iw, oh, ow;
  int32_t route, has_res;
  float *wts, *bias;
  uint32_t cout_pad, cin_pad, k_pad, c_pad;
  float *im_scratch;
};

/* plan.rs:462-614, restricted to a dense single input (no concat parts). */
orc_cpu_op *orc_cpu_op_create(const orc_conv2d *op, uint32_t ih, uint32_t iw, const float *w_oihw,
                              const float *bias, int32_t has_res) {
  orc_cpu_op *p = (orc_cpu_op *)calloc(1, sizeof(orc_cpu_op));
  if (!p) return NULL;
  p->op = *op;
  p->ih = ih;
  p->iw = iw;
  p->has_res = has_res;
  orc_out_hw(op, ih, iw, &p->oh, &p->ow);
  uint32_t cout = op->cout, cin = op->cin, kh = op->kh, kw = op->kw;
  if (op->groups > 1) {
    if (op->groups != cin || cin != cout) goto fail;
    p->route = ORC_ROUTE_CONV_DW;
    p->c_pad = next_mult_u32(cout, 4);
    p->wts = (float *)malloc(sizeof(float) * (size_t)kh * kw * p->c_pad);
    p->bias = (float *)calloc(p->c_pad, sizeof(float));
    if (!p->wts || !p->bias) goto fail;
    orc_cpu_repack_weights_dw(w_oihw, cout, kh, kw, p->wts);
    memcpy(p->bias, bias, sizeof(float) * cout);
  } else if (cin <= 4 && kh * kw > 1 && op->dil == 1) {
    p->route = ORC_ROUTE_CONV_STEM;
    uint32_t k = kh * kw * cin;
    p->k_pad = next_mult_u32(k, 4);
    float *perm = (float *)malloc(sizeof(float) * (size_t)cout * k);
    p->cout_pad = next_mult_u32(cout, NR);
    p->wts = (float *)malloc(sizeof(float) * (size_t)p->k_pad * p->cout_pad);
    p->bias = (float *)calloc(p->cout_pad, sizeof(float));
    p->im_scratch = (float *)calloc((size_t)p->oh * p->ow * p->k_pad + 4, sizeof(float));
    if (!perm || !p->wts || !p->bias || !p->im_scratch) {
      free(perm);
      goto fail;
    }
    orc_cpu_permute_weights(w_oihw, cout, cin, kh, kw, perm);
    orc_cpu_repack_weights(perm, cout, k, p->k_pad, 1, 1, p->wts);
    free(perm);
    memcpy(p->bias, bias, sizeof(float) * cout);
    orc_conv2d pw = {k, cout, 1, 1, 1, 1, {0, 0, 0, 0}, 1, 1, op->act};
    p->pw = pw;
  } else if (kh == 1 && kw == 1 && op->sh == 1 && op->sw == 1 && !has_res && cout <= 4) {
    p->route = ORC_ROUTE_PW_DOT;
    p->k_pad = next_mult_u32(cin, 4);
    p->wts = (float *)calloc((size_t)cout * p->k_pad, sizeof(float));
    p->bias = (float *)malloc(sizeof(float) * cout);
    if (!p->wts || !p->bias) goto fail;
    for (uint32_t oc = 0; oc < cout; ++oc) memcpy(p->wts + (size_t)oc * p->k_pad, w_oihw + (size_t)oc * cin, sizeof(float) * cin);
    memcpy(p->bias, bias, sizeof(float) * cout);
  } else {
    p->route = ORC_ROUTE_CONV_STD;
    p->cin_pad = cin % 4 ? next_mult_u32(cin, 4) : cin;
    p->cout_pad = next_mult_u32(cout, NR);
    p->wts = (float *)malloc(sizeof(float) * (size_t)kh * kw * p->cin_pad * p->cout_pad);
    p->bias = (float *)calloc(p->cout_pad, sizeof(float));
    if (!p->wts || !p->bias) goto fail;
    orc_cpu_repack_weights(w_oihw, cout, cin, p->cin_pad, kh, kw, p->wts);
    memcpy(p->bias, bias, sizeof(float) * cout);
  }
  return p;
fail:
  orc_cpu_op_free(p);
  return NULL;
}

int32_t orc_cpu_op_route(const orc_cpu_op *p) { return p->route; }

void orc_cpu_op_free(orc_cpu_op *p) {
  if (!p) return;
  free(p->wts);
  free(p->bias);
  free(p->im_scratch);
  free(p);
}

typedef struct {
  const orc_cpu_op *p;
  const orc_conv2d *op;
  uint32_t ih, iw;
  orc_view view;
  uint32_t ic0, c4;
  const orc_view *res;
} run_ctx;

static void band_std(void *vc, uint32_t y0, uint32_t y1, float *out) {
  run_ctx *c = (run_ctx *)vc;
  orc_cpu_conv_std(c->op, c->ih, c->iw, &c->view, &c->ic0, &c->c4, 1, c->p->wts, c->p->bias,
                   c->p->cout_pad, c->res, out, y0, y1);
}

static void band_dw(void *vc, uint32_t y0, uint32_t y1, float *out) {
  run_ctx *c = (run_ctx *)vc;
  orc_cpu_conv_dw(c->op, c->ih, c->iw, &c->view, c->p->wts, c->p->bias, c->res, out, y0, y1);
}

/* model.rs:403-549: ConvStd folds k1s1p0 into one row at T<=1 (:413-418) and
 * cuts row bands at T>1 when oh >= T (:421-436); ConvDw bands the same way;
 * ConvStem runs im2row then a 1x1 conv_std over (oh, ow) (:508-540); PwDot is
 * single-threaded. */
int orc_cpu_op_run(orc_cpu_op *p, uint32_t n, const float *input, const float *res, float *out,
                   int32_t threads) {
  const orc_conv2d *op = &p->op;
  size_t in_px = (size_t)p->ih * p->iw, out_px = (size_t)p->oh * p->ow;
  if (threads < 1) threads = 1;
  for (uint32_t b = 0; b < n; ++b) {
    const float *x = input + (size_t)b * in_px * op->cin;
    float *y = out + (size_t)b * out_px * op->cout;
    orc_view rv;
    const orc_view *rvp = NULL;
    if (res && p->has_res) {
      rv.data = res + (size_t)b * out_px * op->cout;
      rv.c_off = 0;
      rv.stride = op->cout;
      rv.c = op->cout;
      rvp = &rv;
    }
    run_ctx c;
    memset(&c, 0, sizeof(c));
    c.p = p;
    c.res = rvp;
    c.view.data = x;
    c.view.c_off = 0;
    c.view.stride = op->cin;
    c.view.c = op->cin;
    switch (p->route) {
      case ORC_ROUTE_CONV_STD: {
        int pw1 = op->kh == 1 && op->kw == 1 && op->sh == 1 && op->sw == 1 && op->pad[0] == 0 &&
                  op->pad[1] == 0 && op->pad[2] == 0 && op->pad[3] == 0;
        c.op = op;
        c.ic0 = 0;
        c.c4 = p->cin_pad;
        uint32_t ih = p->ih, iw = p->iw, oh = p->oh;
        if (pw1 && threads <= 1) {
          ih = 1;
          iw = p->ih * p->iw;
          oh = 1;
        }
        c.ih = ih;
        c.iw = iw;
        if (threads > 1 && oh >= (uint32_t)threads) {
          run_bands(threads, oh, (size_t)p->ow * op->cout, y, band_std, &c);
        } else {
          band_std(&c, 0, oh, y);
        }
        break;
      }
      case ORC_ROUTE_CONV_DW: {
        c.op = op;
        c.ih = p->ih;
        c.iw = p->iw;
        if (threads > 1 && p->oh >= (uint32_t)threads) {
          run_bands(threads, p->oh, (size_t)p->ow * op->cout, y, band_dw, &c);
        } else {
          band_dw(&c, 0, p->oh, y);
        }
        break;
      }
      case ORC_ROUTE_CONV_STEM: {
        orc_cpu_im2row(op, p->ih, p->iw, &c.view, p->k_pad, p->im_scratch);
        c.op = &p->pw;
        c.ih = p->oh;
        c.iw = p->ow;
        c.view.data = p->im_scratch;
        c.view.stride = p->k_pad;
        c.view.c = p->k_pad;
        c.ic0 = 0;
        c.c4 = p->k_pad;
        if (threads > 1 && p->oh >= (uint32_t)threads) {
          run_bands(threads, p->oh, (size_t)p->ow * op->cout, y, band_std, &c);
        } else {
          band_std(&c, 0, p->oh, y);
        }
        break;
      }
      case ORC_ROUTE_PW_DOT:
        orc_cpu_conv_pw_dot(op, &c.view, p->wts, p->k_pad, p->bias, (uint32_t)out_px, y);
        break;
      default:
        return -1;
    }
  }
  return 0;
}

/* ------------------------------------------------------------------------ */
/* ai-gpu variant policies                                                   */
/* ------------------------------------------------------------------------ */

/* gemm_pw.rs:48-50 */
uint32_t orc_ref_gemv_width(uint32_t kg) {
  uint32_t p = 1;
  while (p < kg) p <<= 1;
  if (p < 32) p = 32;
  if (p > 256) p = 256;
  return p;
}

/* gemm_pw.rs:55-57 */
void orc_ref_splitk_geometry(uint32_t cells, uint32_t *split, uint32_t *cpw) {
  if (cells < 8192) {
    *split = 8;
    *cpw = 32;
  } else {
    *split = 4;
    *cpw = 64;
  }
}

/* gemm_pw.rs:64-73 */
void orc_ref_splitk_tile(uint32_t ng, uint32_t cpw, uint32_t *pxt, uint32_t *ngt) {
  uint32_t t;
  if (ng % 4 == 0 || ng >= 8) t = ng < 4 ? ng : 4;
  else if (ng % 2 == 0) t = 2;
  else t = 1;
  *ngt = t;
  *pxt = cpw / t;
}

/* pick_variant -- gemm_pw.rs:91-102, with the default Splitk NG gate of 4
 * (gemm_pw.rs:112-126; the AI_PW_SPLITK_NG override is not read). */
int32_t orc_ref_pw_variant(uint32_t m, uint32_t kg, uint32_t ng) {
  uint32_t tiles = div_ceil_u32(m, 32) * div_ceil_u32(ng, 8);
  if (m * ng < 512 && kg >= 16) return ORC_PW_GEMV;
  if (kg >= 16 && tiles < 192 && ng >= 4 && m >= 64) return ORC_PW_SPLITK;
  if (ng >= 16 && kg >= 16 && m >= 64) return ORC_PW_TILED;
  return ORC_PW_SMALL;
}

/* ConvIgemmSpec::variant -- conv_igemm.rs:201-233 (out_hw :176-181) */
int32_t orc_ref_igemm_variant(uint32_t ih, uint32_t iw, uint32_t cin, uint32_t cout, uint32_t k,
                              uint32_t s, uint32_t d, const uint32_t pad[4], uint32_t nsrcs,
                              int32_t has_offset_src) {
  uint32_t ek = d * (k - 1) + 1;
  uint32_t oh = (ih + pad[0] + pad[2] - ek) / s + 1;
  uint32_t ow = (iw + pad[1] + pad[3] - ek) / s + 1;
  uint32_t kg = div_ceil_u32(cin, 4), ng = div_ceil_u32(cout, 4);
  if (nsrcs > 1 || has_offset_src || ng <= 20 || oh * ow < 512 || k * k * kg <= 9) {
    uint32_t nblk = oh * div_ceil_u32(ow, 4);
    if (nblk * ng < 4096 && kg >= 16) return ORC_IG_SPLITK;
    return ORC_IG_DIRECT;
  }
  return ORC_IG_TILED;
}

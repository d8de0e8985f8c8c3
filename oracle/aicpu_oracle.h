/*
 * aicpu_oracle.h -- CPU oracle for the conv-as-GEMM path (TEST INFRASTRUCTURE).
 *
 * This library is the checker, never the product: only tests/, the smoke
 * check in __graft_entry__.py and the cpu_baseline leg of bench.py may load
 * it.  The product path (ai_engine_amd/) never links or calls it.
 *
 * It restates, in plain C, the reference's CPU arithmetic for this path:
 *   - ai-core: XorShift32 (crates/ai-core/src/rng.rs:3-35), Activation::apply
 *     (activation.rs:28-43), Conv2d::out_hw (ops/conv.rs:49-56), the NHWC-C4
 *     layout and the packing contract (tensor.rs:36-81, pack.rs:16-185), and the
 *     naive conv oracle reference::conv::conv2d (reference/conv.rs:9-62);
 *   - ai-cpu: conv_std with MR8/MR4/MR1 x NR8 register blocking
 *     (crates/ai-cpu/src/kernels/conv.rs:44-468), conv_pw_dot (pw_dot.rs:19-61),
 *     im2row + permute_weights (im2row.rs:22-104), conv_dw (dw.rs:22-304), the
 *     x86 scalar F32x4 fallback with UNFUSED multiply-add (simd.rs:190-293),
 *     apply4 (kernels/mod.rs:21-50), the routing of plan::lower's Conv arm
 *     (plan.rs:462-614) and model::dispatch's row-band threading
 *     (model.rs:403-549);
 *   - ai-gpu variant policies (pure functions): pick_variant, splitk_geometry,
 *     splitk_tile, gemv_width (kernels/gemm_pw.rs:48-126) and
 *     ConvIgemmSpec::variant (kernels/conv_igemm.rs:201-233).
 *
 * Additions with no reference counterpart (documented where defined): a batch
 * dimension n (outermost) for the layout helpers, bf16 storage (RNE), and a
 * seeded Box-Muller Gaussian on XorShift32 draws.
 *
 * Build: see oracle/Makefile (compiled with -ffp-contract=off so that every
 * `acc += a * b` rounds the product and the sum separately, as the x86
 * fallback of the reference does).
 */
#ifndef AICPU_ORACLE_H
#define AICPU_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Storage dtypes: F32/F16 as ai-core DType (tensor.rs:12-16); BF16 is new. */
enum { ORC_F32 = 0, ORC_F16 = 1, ORC_BF16 = 2 };

/* Activation, same order as ai-core Activation (activation.rs:7-25). */
enum {
  ORC_ACT_NONE = 0,
  ORC_ACT_RELU,
  ORC_ACT_SIGMOID,
  ORC_ACT_TANH,
  ORC_ACT_HARDSWISH,
  ORC_ACT_HARDSIGMOID,
  ORC_ACT_CLAMP01,
  ORC_ACT_RELU6,
  ORC_ACT_SQRT,
  ORC_ACT_NEG,
  ORC_ACT_RECIP,
  ORC_ACT_COUNT
};

/* Conv2d (ops/conv.rs:6-20). pad = [top, left, bottom, right]. */
typedef struct {
  uint32_t cin, cout, kh, kw, sh, sw;
  uint32_t pad[4];
  uint32_t dil, groups;
  int32_t act;
} orc_conv2d;

/* Channel-strided view (ai-cpu view.rs:1-28): element of pixel p, channel c
 * lives at data[p * stride + c_off + c]. */
typedef struct {
  const float *data;
  uint32_t c_off, stride, c;
} orc_view;

/* ---- ai-core ---- */
void orc_out_hw(const orc_conv2d *op, uint32_t ih, uint32_t iw, uint32_t *oh, uint32_t *ow);
float orc_act_apply(int32_t act, float x);
/* orc_act_apply over n values (y may alias x) */
void orc_act_apply_n(int32_t act, const float *x, float *y, size_t n);
void orc_act_apply4(int32_t act, float v[4]);

uint32_t orc_xs32_seed(uint32_t seed);
uint32_t orc_xs32_next(uint32_t *state);
float orc_xs32_next_f32(uint32_t *state);
/* XorShift32::new(seed).vec_f32(n) */
void orc_xs32_fill(uint32_t seed, float *out, size_t n);
/* N(mean, sigma) by Box-Muller on two XorShift32 draws; see definition. */
void orc_gauss_fill(uint32_t seed, float mean, float sigma, float *out, size_t n);

uint16_t orc_f32_to_f16(float x);
float orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_bf16(float x);
float orc_bf16_to_f32(uint16_t h);
size_t orc_dtype_bytes(int32_t dt);
/* bulk conversions (element i of in -> element i of out) */
void orc_cvt_from_f32(int32_t dt, const float *in, void *out, size_t n);
void orc_cvt_to_f32(int32_t dt, const void *in, float *out, size_t n);

/* NHWC-C4 with batch n outermost: vec4 index ((b*H + h)*W + w)*cg + g. */
size_t orc_nhwc_c4_bytes(uint32_t n, uint32_t h, uint32_t w, uint32_t c, int32_t dt);
void orc_pack_nhwc(const float *data, uint32_t n, uint32_t h, uint32_t w, uint32_t c,
                   int32_t dt, void *out);
void orc_unpack_nhwc(const void *bytes, uint32_t n, uint32_t h, uint32_t w, uint32_t c,
                     int32_t dt, float *out);
/* OIHW -> [tap][kg_pad][ng][j][comp]; returns kg_pad. out holds taps*kg_pad*ng*16 elems. */
uint32_t orc_pack_weights_conv(const float *w_oihw, uint32_t cout, uint32_t cin, uint32_t kh,
                               uint32_t kw, uint32_t kg_align, int32_t dt, void *out);
void orc_unpack_weights_conv(const void *bytes, uint32_t cout, uint32_t cin, uint32_t kh,
                             uint32_t kw, uint32_t kg_pad, int32_t dt, float *out);
/* [c][kh][kw] -> [tap][cg][comp] */
void orc_pack_weights_dw(const float *w, uint32_t c, uint32_t kh, uint32_t kw, int32_t dt,
                         void *out);
void orc_unpack_weights_dw(const void *bytes, uint32_t c, uint32_t kh, uint32_t kw, int32_t dt,
                           float *out);
void orc_pack_bias(const float *b, uint32_t cout, int32_t dt, void *out);
void orc_unpack_bias(const void *bytes, uint32_t cout, int32_t dt, float *out);

/* reference::conv::conv2d, one image, logical NHWC. bias/res may be NULL. */
int orc_conv2d_ref(const orc_conv2d *op, uint32_t ih, uint32_t iw, const float *input,
                   const float *weights, const float *bias, const float *residual, float *out);

/* ---- ai-cpu kernels (callers keep +4 floats of slack after every view) ---- */
/* conv::repack_weights -> [tap][cin_pad][cout_pad]; returns cout_pad (multiple of 8). */
uint32_t orc_cpu_repack_weights(const float *w_oihw, uint32_t cout, uint32_t cin,
                                uint32_t cin_pad, uint32_t kh, uint32_t kw, float *out);
/* conv::conv_std over output rows [y0, y1); out starts at row y0. */
void orc_cpu_conv_std(const orc_conv2d *op, uint32_t ih, uint32_t iw, const orc_view *views,
                      const uint32_t *ic0, const uint32_t *c4, uint32_t nparts,
                      const float *wts, const float *bias, uint32_t cout_pad,
                      const orc_view *residual, float *out, uint32_t y0, uint32_t y1);
/* dw::repack_weights -> [tap][c_pad4] */
uint32_t orc_cpu_repack_weights_dw(const float *w, uint32_t c, uint32_t kh, uint32_t kw,
                                   float *out);
void orc_cpu_conv_dw(const orc_conv2d *op, uint32_t ih, uint32_t iw, const orc_view *input,
                     const float *wts, const float *bias, const orc_view *residual, float *out,
                     uint32_t y0, uint32_t y1);
void orc_cpu_im2row(const orc_conv2d *op, uint32_t ih, uint32_t iw, const orc_view *input,
                    uint32_t k_pad, float *out);
void orc_cpu_permute_weights(const float *w_oihw, uint32_t cout, uint32_t cin, uint32_t kh,
                             uint32_t kw, float *out);
void orc_cpu_conv_pw_dot(const orc_conv2d *op, const orc_view *input, const float *wts,
                         uint32_t k_pad, const float *bias, uint32_t px, float *out);

/* ---- ai-cpu plan/dispatch: one conv op prepared at load, run per frame ---- */
enum { ORC_ROUTE_CONV_STD = 0, ORC_ROUTE_CONV_STEM = 1, ORC_ROUTE_PW_DOT = 2, ORC_ROUTE_CONV_DW = 3 };
typedef struct orc_cpu_op orc_cpu_op;
/* Routes like plan::lower (dense single input). has_res selects the residual
 * form of the op. Returns NULL on unsupported ops. */
orc_cpu_op *orc_cpu_op_create(const orc_conv2d *op, uint32_t ih, uint32_t iw,
                              const float *w_oihw, const float *bias, int32_t has_res);
int32_t orc_cpu_op_route(const orc_cpu_op *p);
/* Runs n images one after another (ai-cpu has no batch dimension). input holds
 * n*ih*iw*cin floats (+4 slack), res/out n*oh*ow*cout. threads as set_threads. */
int orc_cpu_op_run(orc_cpu_op *p, uint32_t n, const float *input, const float *res, float *out,
                   int32_t threads);
void orc_cpu_op_free(orc_cpu_op *p);

/* ---- ai-gpu variant policies (pure) ---- */
enum { ORC_PW_TILED = 0, ORC_PW_SMALL = 1, ORC_PW_GEMV = 2, ORC_PW_SPLITK = 3 };
enum { ORC_IG_TILED = 0, ORC_IG_DIRECT = 1, ORC_IG_SPLITK = 2 };
int32_t orc_ref_pw_variant(uint32_t m, uint32_t kg, uint32_t ng);
uint32_t orc_ref_gemv_width(uint32_t kg);
void orc_ref_splitk_geometry(uint32_t cells, uint32_t *split, uint32_t *cpw);
void orc_ref_splitk_tile(uint32_t ng, uint32_t cpw, uint32_t *pxt, uint32_t *ngt);
int32_t orc_ref_igemm_variant(uint32_t ih, uint32_t iw, uint32_t cin, uint32_t cout, uint32_t k,
                              uint32_t s, uint32_t d, const uint32_t pad[4], uint32_t nsrcs,
                              int32_t has_offset_src);

#ifdef __cplusplus
}
#endif
#endif

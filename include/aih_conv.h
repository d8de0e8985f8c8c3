/*
 * aih_conv.h -- C ABI of the MI355X (gfx950) conv-as-GEMM backend.
 *
 * The entry points replace, op for op, what the reference's GPU runtime binds
 * for a SwOp::Conv (crates/ai-gpu-runtime/src/lowering.rs:99-187):
 *   - aih_conv_pw     <- GemmPwSpec + its dispatch (crates/ai-gpu/src/kernels/gemm_pw.rs:129-297)
 *   - aih_conv_igemm  <- ConvIgemmSpec + its dispatch (crates/ai-gpu/src/kernels/conv_igemm.rs:49-558)
 *   - aih_conv_dw     <- ConvDwSpec + its dispatch (crates/ai-gpu/src/kernels/conv_dw.rs:21-216)
 *   - aih_conv        <- the Conv arm of lower_op itself (lowering.rs:99-187):
 *                        routes groups>1 -> dw, 1x1 -> pw, KxK -> igemm
 *   - aih_*_plan      <- the pure variant policies pick_variant (gemm_pw.rs:91-102)
 *                        and ConvIgemmSpec::variant (conv_igemm.rs:201-233), re-tuned
 *                        for MI355X
 *   - aih_pack_*      <- ai-core pack.rs:34-184 (the converter's output contract)
 *
 * Conventions follow the reference's C ABI (crates/ai-ffi/src/lib.rs:45-52,
 * 130-133): every function returns AIH_OK (0) or AIH_ERR (-1) and never lets
 * an exception cross the boundary; aih_last_error() returns the calling
 * thread's message for the last failure.
 *
 * Buffers (all device pointers, caller-owned, never allocated by a conv call):
 *   activations  NHWC-C4: element (b, y, x, c) at ((b*H + y)*W + x)*CG*4 + c,
 *                CG = ceil(C/4), C padded with zeros to a multiple of 4
 *                (tensor.rs:1-6,72-74); b is the batch, outermost (new here).
 *   std weights  [tap][kg_pad][ng][j][comp] vec4, kg_pad = ceil(cin/4) rounded up
 *                to a multiple of 4 (pack.rs:68-102), dtype wdt.
 *   dw weights   [tap][cg][comp] vec4 (pack.rs:105-122), dtype dt.
 *   bias         [ng][4] (pack.rs:178-184), dtype dt; always present.
 *   residual     same layout and dtype as the output; added AFTER the
 *                activation: y = act(acc + bias) + res (reference/conv.rs:53-56).
 * dtypes: AIH_F32 / AIH_F16 as ai-core DType; AIH_BF16 is new. Accumulation
 * is always fp32.
 *
 * Diagnostic environment overrides, read once per process (like the
 * reference's AI_PW_SPLITK_NG, gemm_pw.rs:112-126, and AI_RT_FORCE_DIRECT,
 * lowering.rs:156-160); they apply to AIH_VAR_AUTO calls without a forced
 * split only, and the plan functions report their effect:
 *   AIH_PW_SPLITK=<n>     every AUTO pointwise conv gets n K chunks as a forced split does
 *                         (the one-dispatch split-K kernel where the shape allows, else the
 *                         tiled GEMM; 1 = no split): the narrow, direct, LDS one-tap and
 *                         streamed routes are bypassed while it is set
 *   AIH_IGEMM_NO_SPLIT=1  a KxK conv never splits K
 */
#ifndef AIH_CONV_H
#define AIH_CONV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define AIH_OK 0
#define AIH_ERR (-1)

/* A hipStream_t. NULL selects the null stream. */
typedef void *aih_stream;

enum aih_dtype { AIH_F32 = 0, AIH_F16 = 1, AIH_BF16 = 2 };

/* Same order as ai-core Activation (crates/ai-core/src/activation.rs:7-25). */
enum aih_act {
  AIH_ACT_NONE = 0,
  AIH_ACT_RELU = 1,
  AIH_ACT_SIGMOID = 2,
  AIH_ACT_TANH = 3,
  AIH_ACT_HARDSWISH = 4,
  AIH_ACT_HARDSIGMOID = 5,
  AIH_ACT_CLAMP01 = 6,
  AIH_ACT_RELU6 = 7,
  AIH_ACT_SQRT = 8,
  AIH_ACT_NEG = 9,
  AIH_ACT_RECIP = 10
};

/* Kernel variants chosen by the plan functions (a caller asks for the first
 * three; the plans also report the last two). */
enum aih_variant {
  AIH_VAR_AUTO = 0,    /* let the policy decide */
  AIH_VAR_TILE = 1,    /* one MFMA tile per workgroup over the whole K */
  AIH_VAR_SPLITK = 2,  /* K cut into chunks, fp32 partials reduced in a fixed order */
  AIH_VAR_ROWS = 3,    /* pointwise, ng == 1: one pixel per thread on the VALU */
  AIH_VAR_DIRECT = 4   /* 32 pixels per wavefront, activations from memory into
                          MFMA registers: pointwise with ng <= 16 (short K:
                          weights in registers; K up to 256 fp32 / 512 16-bit
                          channels over >= 2048 pixel blocks: weights resident
                          in LDS); 3x3 igemm with cout <= 64 (weights in LDS);
                          the 3x3 stem over <= 3 input channels */
};

/* Pointwise 1x1 conv GEMM: out[M, N] = act(in[M, K] x W[K, N] + bias) (+ res).
 * Mirrors GemmPwSpec{m, kg, ng, act, residual, dt, wdt} (gemm_pw.rs:129-142). */
typedef struct {
  uint32_t n;       /* images; the reference always has 1 (tensor.rs:37) */
  uint32_t m;       /* pixels per image (= ih*iw, lowering.rs:145) */
  uint32_t kg;      /* ceil(cin/4) */
  uint32_t ng;      /* ceil(cout/4) */
  uint32_t kg_pad;  /* kg of the packed weights (SwOp::Conv.kg_pad); >= kg */
  int32_t act;      /* enum aih_act */
  int32_t residual; /* 0 or 1 */
  int32_t dt;       /* activation / bias / residual / output dtype */
  int32_t wdt;      /* weight dtype (independent of dt, format/model.rs:245-254) */
  int32_t variant;  /* enum aih_variant */
  int32_t splitk;   /* 0 = policy; otherwise the split-K factor (1 = no split) */
} aih_pw_desc;

/* One input part of a KxK conv: `c` channels that start at channel `c_off`
 * of a tensor whose pixels hold `stride_c` channels (SrcView,
 * crates/ai-gpu/src/kernels/common/source.rs:17). c_off and stride_c are
 * multiples of 4. */
typedef struct {
  uint32_t c, stride_c, c_off;
} aih_src;

/* KxK implicit-GEMM conv (groups = 1). Mirrors ConvIgemmSpec (conv_igemm.rs:49-76)
 * plus a batch n; non-square kernels and anisotropic strides are rejected as in
 * ConvIgemmSpec::from_op (conv_igemm.rs:79-83). With AIH_VAR_AUTO and no
 * forced split, a 3x3 conv with dt == wdt, cout <= 64, at most two input
 * parts whose channel counts, offsets and pixel strides are whole 16-byte
 * units (4 fp32 / 8 16-bit channels), at most 10 MFMA steps per tap (80
 * fp32 / 160 16-bit input channels) and 9 * K * N of weights within 160 KB of
 * LDS runs the direct kernel (plan variant
 * AIH_VAR_DIRECT, no workspace); <= 3 input channels of a dense input with
 * d = 1 and 32 or 64 outputs run the stem kernel (also AIH_VAR_DIRECT);
 * everything else the tiled GEMM (TILE / SPLITK). */
typedef struct {
  uint32_t n, ih, iw, cin, cout;
  uint32_t k, s, d;
  uint32_t pad[4]; /* top, left, bottom, right */
  int32_t act, residual, dt, wdt;
  int32_t variant; /* enum aih_variant */
  int32_t splitk;  /* 0 = policy */
  uint32_t nsrcs;  /* 0 = one dense input; 1..3 = srcs[] (channel view / concat parts) */
  aih_src srcs[3];
} aih_igemm_desc;

/* Depthwise conv (groups = cin = cout), any k/s/d/pad. Mirrors ConvDwSpec. */
typedef struct {
  uint32_t n, ih, iw, c;
  uint32_t k, s, d;
  uint32_t pad[4];
  int32_t act, residual, dt;
} aih_dw_desc;

/* A whole SwOp::Conv (format/model.rs:80-111) as lower_op sees it. */
typedef struct {
  uint32_t n, ih, iw, cin, cout;
  uint32_t kh, kw, sh, sw;
  uint32_t pad[4];
  uint32_t d, groups;
  int32_t act, residual;
  int32_t dt, wdt;
  uint32_t kg_pad;
} aih_conv_desc;

/* What a plan function chose; grid is the number of workgroups of the main kernel. */
typedef struct {
  int32_t variant;  /* AIH_VAR_TILE, AIH_VAR_SPLITK, AIH_VAR_ROWS or AIH_VAR_DIRECT */
  uint32_t splitk;  /* K chunks (1 for TILE) */
  uint32_t bm, bn;  /* output tile: pixels x channels */
  uint32_t grid;
  size_t ws_bytes;  /* workspace the call needs */
} aih_plan;

/* Fused inverted-residual block: three consecutive SwOp::Conv that lower_op
 * would dispatch separately (lowering.rs:122-152) -- a 1x1 expand (cin ->
 * cexp), a depthwise 3x3 with stride s over cexp channels, and a 1x1 project
 * (cexp -> cout) -- run as one kernel, so the expanded tensor never goes to
 * HBM. Each stage keeps its unfused arithmetic: fp32 accumulation,
 * y = act(acc + bias) (+ res), intermediates rounded to dt where the unfused
 * ops store them. All weights and biases are in dt, in the converter's
 * layouts (pack_weights_conv kg_align 4 for the 1x1 convs, pack_weights_dw
 * for the depthwise). Residual, if any, is added after act_project. */
typedef struct {
  uint32_t n, ih, iw;
  uint32_t cin, cexp, cout;
  uint32_t s;       /* depthwise stride (1 or 2); the kernel is 3x3 */
  uint32_t pad[4];  /* depthwise padding: top, left, bottom, right */
  int32_t act_expand, act_dw, act_project;
  int32_t residual;
  int32_t dt;
  uint32_t tile_h, tile_w; /* output tile; 0 = chosen by the plan */
  uint32_t ec;             /* expanded channels per chunk; 0 = chosen by the plan */
  int32_t weights;         /* enum aih_ir_weights: where the expand / project weights live */
  int32_t kernel;          /* enum aih_ir_kernel */
  uint32_t waves;          /* wavefronts per workgroup; 0 = chosen by the plan. The split kernel takes
                              1, 2, 4 or 8; the wave kernel 2, 4, 8, or 12 for the stride-1 tiles of
                              32-, 48- and 64-channel blocks (three wavefronts per SIMD sharing one
                              copy of the weights) */
} aih_ir_block_desc;

/* Which fused kernel runs a block: chosen by the plan (the cheaper estimate
 * of the wave and split kernels where they apply, else the tile kernel), the
 * tile kernel (a workgroup shares one output tile of up to 256 pixels and its
 * halo through LDS, any clamp or other activation, f32 / f16 / bf16), the
 * wave kernel (every wavefront owns a tile of up to 32 pixels with a private
 * expanded chunk in LDS, weights shared through LDS; f16 / bf16 storage,
 * clamp-type activations, the instantiated widths), or the split kernel
 * (as the wave kernel, but the 1..8 wavefronts of a workgroup share one tile
 * and divide its expanded channels, weights read from memory, the partial
 * projections added in a fixed order: for launches with few tiles). */
enum aih_ir_kernel { AIH_IR_KERNEL_AUTO = 0, AIH_IR_KERNEL_TILE = 1, AIH_IR_KERNEL_WAVE = 2, AIH_IR_KERNEL_SPLIT = 3 };

/* Weight placement of a fused block: chosen by the plan (resident when they
 * fit), all of them resident in LDS for every tile, or streamed chunk by
 * chunk through two LDS slots. */
enum aih_ir_weights { AIH_IR_WEIGHTS_AUTO = 0, AIH_IR_WEIGHTS_RESIDENT = 1, AIH_IR_WEIGHTS_STREAMED = 2 };

/* Geometry aih_ir_block_plan chose: output tile th x tw, expanded channels
 * per chunk, whether all expand/project weights stay resident in LDS, LDS
 * bytes and workgroups per CU, launched workgroups. */
typedef struct {
  uint32_t th, tw, ec, chunks, resident;
  uint32_t tiles, lds_bytes, occupancy, grid;
  uint32_t kernel; /* enum aih_ir_kernel: AIH_IR_KERNEL_TILE, _WAVE or _SPLIT */
  uint32_t waves;  /* wavefronts per workgroup */
  uint32_t deep;   /* split kernel: operands prefetched a whole chunk ahead (1) or one phase ahead (0) */
} aih_ir_plan;

/* ---- op entry points (asynchronous on `stream`) ---- */

/* Buffer order follows GemmPwSpec::bindings (gemm_pw.rs:276-283): IN, W, BIAS,
 * [RES], OUT. res must be NULL iff residual == 0. ws may be NULL when the plan
 * needs no workspace; otherwise ws_bytes >= aih_plan.ws_bytes. With
 * AIH_VAR_AUTO and splitk == 0 two shapes skip the planned MFMA tile and need
 * no workspace: ng == 1 (at most 4 output channels) runs a VALU kernel (one
 * pixel per thread, the reference's Gemv role); dt == wdt, 2 <= ng <= 16 and
 * at most 128 (16-bit) / 64 (fp32) input channels run a direct MFMA kernel
 * (32 pixels per wavefront, operands from memory into registers); fp32 with
 * at least 256 input channels and enough pixels for eight 32 x 32 wavefront
 * units per CU runs a GEMM whose operands stream through LDS by DMA over
 * the whole K (reported as AIH_VAR_TILE with bm = 96, no workspace). */
int aih_conv_pw(const aih_pw_desc *d, const void *x, const void *w, const void *bias,
                const void *res, void *y, void *ws, size_t ws_bytes, aih_stream stream);
int aih_conv_pw_plan(const aih_pw_desc *d, aih_plan *out);

/* inputs holds max(1, nsrcs) device pointers: the plain input, or one per part
 * (the IN0..IN2 bindings of conv_igemm.rs:141-171). A dense 3x3 conv (d = 1)
 * over at most 3 input channels with cout 32 or 64, AIH_VAR_AUTO, splitk 0 and
 * dt == wdt -- the stem -- runs a dedicated kernel (all 27 tap-channel values
 * in one MFMA operand) instead of the planned implicit GEMM; it needs no
 * workspace. */
int aih_conv_igemm(const aih_igemm_desc *d, const void *const *inputs, const void *w,
                   const void *bias, const void *res, void *y, void *ws, size_t ws_bytes,
                   aih_stream stream);
int aih_conv_igemm_plan(const aih_igemm_desc *d, aih_plan *out);

int aih_conv_dw(const aih_dw_desc *d, const void *x, const void *w, const void *bias,
                const void *res, void *y, aih_stream stream);

/* Routes like lower_op (lowering.rs:122-168): groups > 1 -> dw, 1x1 -> pw
 * (stride or pad rejected, :136-140), otherwise igemm. */
int aih_conv(const aih_conv_desc *d, const void *x, const void *w, const void *bias,
             const void *res, void *y, void *ws, size_t ws_bytes, aih_stream stream);
size_t aih_conv_workspace_size(const aih_conv_desc *d);
/* The plan aih_conv would run for d: the pointwise or implicit-GEMM plan of
 * its route; a depthwise conv reports AIH_VAR_DIRECT with bm = bn = grid = 0
 * (one kernel, no workspace). */
int aih_conv_plan(const aih_conv_desc *d, aih_plan *out);
/* aih_conv for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc). No
 * counterpart in the reference. The split-K workspace aih_conv takes from the
 * caller is instead a static device array of AIH_NOALLOC_SCRATCH_BYTES inside
 * the library, one per device, set up on the first call from that device and
 * held until the process ends. A conv whose workspace (aih_conv_workspace_size)
 * exceeds it fails with AIH_ERR and the size in the message. Calls on one
 * device share the array: calls that overlap on one device (different
 * streams, unordered threads) race; calls ordered on one stream do not. The
 * same kernels as aih_conv, so the same results bit for bit. */
#define AIH_NOALLOC_SCRATCH_BYTES (16u << 20)
int aih_conv_noalloc(const aih_conv_desc *d, const void *x, const void *w, const void *bias,
                     const void *res, void *y, aih_stream stream);
/* Validates a descriptor as aih_conv would (routing, shapes, dtypes, plan)
 * without launching: AIH_OK, or AIH_ERR with the reason (lower_op's load-time
 * rejection of a conv it cannot run, lowering.rs:136-140). */
int aih_conv_check(const aih_conv_desc *d);

/* Fused block (no counterpart op in the reference: a fusion of the three
 * dispatches above). Fails with a message when the shape cannot run fused
 * (cin % 16 (f16/bf16) or % 8 (f32), cin > 128, cexp % 32, cout % 32 or cout > 128,
 * s not in {1, 2}); the caller then runs the three ops unfused. Buffers:
 * x [n][ih][iw][cin], res/y [n][oh][ow][cout], NHWC-C4 in dt. */
int aih_ir_block_plan(const aih_ir_block_desc *d, aih_ir_plan *out);
int aih_ir_block(const aih_ir_block_desc *d, const void *x, const void *w_expand, const void *b_expand,
                 const void *w_dw, const void *b_dw, const void *w_project, const void *b_project,
                 const void *res, void *y, aih_stream stream);

/* Fused depthwise + pointwise: a depthwise 3x3 conv (groups = c, stride s,
 * d = 1) + act_dw and the 1x1 conv that is its output's only reader (c ->
 * cout) + act_pw (+ residual) -- two SwOp::Conv that lower_op dispatches
 * separately (lowering.rs:122-168: conv_dw.rs:21-216, then gemm_pw.rs:129-297)
 * -- as one kernel; the depthwise output never goes to memory. No
 * counterpart op in the reference (a fusion of those two dispatches). Each
 * stage keeps its unfused arithmetic (fp32 accumulation, depthwise sum from
 * the bias over the taps in (ky, kx) order, y = act(acc + bias) (+ res)),
 * and at 16 bit its rounding point: the depthwise result is rounded to dt
 * where the unfused depthwise stores it.
 * Buffers in the unfused ops' layouts: x [n][ih][iw][c] NHWC-C4, w_dw / b_dw
 * as aih_conv_dw takes them, w_pw / b_pw as aih_conv_pw takes them (packed
 * kg_align 4, kg_pad groups), res / y [n][oh][ow][cout] NHWC-C4; every buffer
 * 16-byte aligned. Storage f32, f16 or bf16 (every buffer in dt); cout
 * 1..64; fails with a message otherwise (the caller then runs the two ops). */
typedef struct {
  uint32_t n, ih, iw, c;   /* depthwise input: n images, c channels */
  uint32_t k, s;           /* depthwise kernel (3) and stride (1 or 2) */
  uint32_t pad[4];         /* depthwise padding: top, left, bottom, right (< k) */
  uint32_t cout;           /* pointwise output channels */
  uint32_t kg_pad;         /* kg of the packed pointwise weights (>= ceil(c / 4)) */
  int32_t act_dw, act_pw;  /* enum aih_act */
  int32_t residual;        /* 0 or 1: y = act_pw(...) + res */
  int32_t dt;              /* enum aih_dtype: AIH_F32, AIH_F16 or AIH_BF16 */
  uint32_t tile_h, tile_w; /* output tile (16-column multiples, 1-8 wavefronts); 0 = chosen by the plan */
  uint32_t wave_rows;      /* output rows per wavefront, 2 or 4; 0 = chosen by the plan */
} aih_dwpw_desc;

/* Geometry aih_conv_dwpw_plan chose: output tile th x tw (a wavefront per
 * wave_rows rows x 16 columns), channel chunks of 16 (fp32) or 32 (16-bit),
 * tiles (one workgroup each), LDS bytes and resident workgroups per CU,
 * launched workgroups. */
typedef struct {
  uint32_t th, tw, waves, wave_rows, chunks, tiles, lds_bytes, occupancy, grid;
} aih_dwpw_plan;

int aih_conv_dwpw_plan(const aih_dwpw_desc *d, aih_dwpw_plan *out);
int aih_conv_dwpw(const aih_dwpw_desc *d, const void *x, const void *w_dw, const void *b_dw, const void *w_pw,
                  const void *b_pw, const void *res, void *y, aih_stream stream);

/* ---- host-side packing (ai-core pack.rs; plain host memory) ---- */
/* Output bytes = n*h*w*ceil(c/4)*4*sizeof(dt). */
size_t aih_nhwc_c4_bytes(uint32_t n, uint32_t h, uint32_t w, uint32_t c, int32_t dt);
int aih_pack_nhwc(const float *data, uint32_t n, uint32_t h, uint32_t w, uint32_t c, int32_t dt,
                  void *out);
int aih_unpack_nhwc(const void *bytes, uint32_t n, uint32_t h, uint32_t w, uint32_t c,
                    int32_t dt, float *out);
/* Returns kg_pad (> 0) or 0 on error. */
uint32_t aih_pack_weights_conv(const float *w_oihw, uint32_t cout, uint32_t cin, uint32_t kh,
                               uint32_t kw, uint32_t kg_align, int32_t dt, void *out);
int aih_pack_weights_dw(const float *w, uint32_t c, uint32_t kh, uint32_t kw, int32_t dt,
                        void *out);
int aih_pack_bias(const float *b, uint32_t cout, int32_t dt, void *out);

/* ---- device-side layout kernels ---- */
/* Logical NHWC fp32 (n*h*w*c floats) -> NHWC-C4 in dt, on the device (the
 * upload path of Model::upload_input, crates/ai-gpu-runtime/src/model.rs:387-399). */
int aih_pack_nhwc_device(const float *x, uint32_t n, uint32_t h, uint32_t w, uint32_t c,
                         int32_t dt, void *y, aih_stream stream);

/* The stem conv straight from the model's input: x is logical NHWC fp32
 * (n*ih*iw*cin floats, the layout Model::upload_input takes,
 * crates/ai-gpu-runtime/src/model.rs:387-399), rounded to d->dt as it is
 * read, so y equals aih_pack_nhwc_device into NHWC-C4 followed by
 * aih_conv_igemm bit for bit, without the packed copy. It replaces that
 * pair -- the runtime's input pack and the first Conv's dispatch
 * (lowering.rs:122-168) -- for a descriptor on the stem route (k = 3,
 * d = 1, cin <= 3, cout 32 or 64, one dense input, AIH_VAR_AUTO, splitk 0,
 * dt == wdt); x must stay below 2 GiB and 4-byte aligned. */
int aih_conv_stem_f32in(const aih_igemm_desc *d, const float *x, const void *w, const void *bias,
                        const void *res, void *y, aih_stream stream);

/* The stem conv fused into the inverted-residual block that reads its output
 * as input and residual: one launch in place of aih_conv_stem_f32in followed
 * by aih_ir_block (the reference dispatches the stem conv and the block's
 * three convs separately, lowering.rs:122-168; no counterpart op). For each
 * halo pixel of a block tile the launch computes the stem's output from the
 * logical NHWC fp32 image with the stem kernel's operands, MFMA steps, bias,
 * activation and rounding -- what aih_conv_stem_f32in would store, bit for
 * bit -- and runs the block on it; the stem's output is never stored, so y
 * equals the two calls' result bit for bit. stem: on aih_conv_stem_f32in's
 * route with cin = 3, cout = 32, no residual, a clamp-type activation (none,
 * ReLU, ReLU6, clamp01), image below 2 GiB; blk: 32 -> cexp -> 32 with a
 * stride-1 depthwise, ReLU after the expand and the depthwise, residual = 1
 * (the block's input: the stem's output), ih x iw = the stem's output size,
 * the same n, dt = f16 or bf16 in both (weights in it), kernel AUTO or WAVE
 * (the wave kernel runs it; tile_h / tile_w / weights / waves as for
 * aih_ir_block, waves 2 / 4 / 8 / 12). */
int aih_ir_block_stem_plan(const aih_igemm_desc *stem, const aih_ir_block_desc *blk, aih_ir_plan *out);
int aih_ir_block_stem(const aih_igemm_desc *stem, const aih_ir_block_desc *blk, const float *image,
                      const void *w_stem, const void *b_stem, const void *w_expand, const void *b_expand,
                      const void *w_dw, const void *b_dw, const void *w_project, const void *b_project, void *y,
                      aih_stream stream);

/* The inverted-residual block joined to the pointwise conv that reads its
 * output when that conv has at most 4 outputs (a segmentation head, e.g.
 * 128 -> 2): one launch in place of aih_ir_block followed by aih_conv_pw
 * (the reference dispatches the block's three convs and the head
 * separately, lowering.rs:122-168; no counterpart op). The block runs on the
 * split kernel; each output block, as it is stored, also feeds the head's
 * products, which are summed exactly as aih_conv_pw's narrow route sums them
 * (the same fused multiply-adds per input group, each lane's groups in the
 * same order, the lanes added in the same tree), so y_head equals the two
 * calls' head output bit for bit. y: the block's output, or NULL to not store
 * it (when nothing else reads it). blk: as for aih_ir_block, f16 or bf16,
 * kernel AUTO or SPLIT (tile_h / tile_w / waves 1 / 2 / 4 / 8 as for
 * aih_ir_block); head: n and m = the block's output, kg = cout / 4 >= 16,
 * ng = 1, no residual, AIH_VAR_AUTO, splitk 0, dt = wdt = the block's dt. */
int aih_ir_block_head_plan(const aih_ir_block_desc *blk, const aih_pw_desc *head, aih_ir_plan *out);
int aih_ir_block_head(const aih_ir_block_desc *blk, const aih_pw_desc *head, const void *x, const void *w_expand,
                      const void *b_expand, const void *w_dw, const void *b_dw, const void *w_project,
                      const void *b_project, const void *res, void *y, const void *w_head, const void *b_head,
                      void *y_head, aih_stream stream);

/* ---- errors / info ---- */
const char *aih_last_error(void);
const char *aih_version(void);

#ifdef __cplusplus
}
#endif
#endif

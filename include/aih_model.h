/*
 * aih_model.h -- the graph-level C ABI: a .sw model resident on one MI355X,
 * and the non-conv ops a segmentation graph needs around the conv path.
 *
 * Model verbs replace ai_gpu_runtime::Model (crates/ai-gpu-runtime/src/model.rs):
 *   - aih_model_load          <- Model::load (:56): parse the .sw container
 *                                (crates/ai-core/src/format/header.rs:58-86, model.rs:79-307),
 *                                upload the weight blob once, allocate every tensor,
 *                                lower every op (lower_op, lowering.rs:88-516)
 *   - aih_model_upload_input  <- Model::upload_input (:387-399)
 *   - aih_model_infer         <- Model::infer (:402-426): submit only
 *   - aih_model_read_output   <- Model::read_output (:442-457)
 *   - aih_model_reset         <- Model::reset (:368-385): zero the state tensors
 *   - aih_model_tensor        <- Model::input_storage / output_storage (:465-478):
 *                                the device buffer of a tensor, for zero-copy callers
 *   - aih_model_free          <- Drop
 * Op entry points replace the reference's non-conv lowerings (lowering.rs:188-516):
 *   - aih_resize  <- SwOp::Resize (bilinear, half_pixel / asymmetric, concat parts)
 *   - aih_gpool   <- SwOp::Gpool (channel mean)
 *   - aih_binary  <- SwOp::Binary (add / sub / mul / prelu, six operand kinds) + act
 *   - aih_concat  <- SwOp::Concat (channel concat)
 *   - aih_resize_concat <- a Resize folded into the Concat that alone reads it
 *
 * Supported .sw ops: Conv (all of lower_op's routes, concat parts, residual),
 * Binary, Gpool, Resize, Concat. Any other op kind makes aih_model_load fail
 * with a message naming it. Conventions as in aih_conv.h: AIH_OK / AIH_ERR,
 * aih_last_error(), NHWC-C4 activations with the batch outermost, fp32
 * arithmetic on f32 / f16 / bf16 storage.
 */
#ifndef AIH_MODEL_H
#define AIH_MODEL_H

#include <stddef.h>
#include <stdint.h>

#include "aih_conv.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- non-conv ops (asynchronous on `stream`; caller-owned device buffers) ---- */

/* Bilinear resize (crates/ai-core/src/reference/resize.rs:6-44): src coordinate
 * (dst + 0.5) * in/out - 0.5 (half_pixel) or dst * in/out (asymmetric), taps
 * clamped to the image. The output holds the parts' channels one after the
 * other (concat-into-resize, model.rs:150-159): part i is srcs[i] of
 * inputs[i]; every part but the last has a multiple of 4 channels. */
enum aih_coord { AIH_COORD_HALF_PIXEL = 0, AIH_COORD_ASYMMETRIC = 1 };
typedef struct {
  uint32_t n, ih, iw, oh, ow;
  int32_t mode; /* enum aih_coord */
  int32_t dt;
  uint32_t nsrcs; /* 1..8 */
  aih_src srcs[8];
} aih_resize_desc;
int aih_resize(const aih_resize_desc *d, const void *const *inputs, void *y, aih_stream stream);

/* Global average pool (reference/pool.rs:6-19): y[b][0][0][c] = mean over the
 * h*w pixels of x[b][.][.][c]. */
typedef struct {
  uint32_t n, h, w, c;
  int32_t dt;
} aih_gpool_desc;
int aih_gpool(const aih_gpool_desc *d, const void *x, void *y, aih_stream stream);

/* y = act(a op b) (ops/elementwise.rs:13-27, reference/elementwise.rs:7-30),
 * a and y [n][h][w][c]. The operand b (SwOperand, model.rs:60-78):
 *   TENSOR       [n][h][w][c]
 *   SCALAR       `scalar`; scalar_first = 1 computes scalar op a
 *   CVEC         [c] constant channel vector (NHWC-C4 of 1x1xc, no batch)
 *   CVEC_TENSOR  [n][1][1][b_c] runtime channel vector (an SE gate), b_c = c;
 *                b_c = 1 is a runtime scalar
 *   PVEC_TENSOR  one runtime value per pixel, broadcast over channels:
 *                [n][h][w][1] (b_c = 1) or [n][1][1][h*w] (b_c = h*w)
 *   TILED_TENSOR [n][1][1][b_c] runtime vector, channel k takes element k % b_c
 * (ai-cpu model.rs:478-507). */
enum aih_binop { AIH_BIN_ADD = 0, AIH_BIN_SUB = 1, AIH_BIN_MUL = 2, AIH_BIN_PRELU = 3 };
enum aih_operand {
  AIH_OPND_TENSOR = 0,
  AIH_OPND_SCALAR = 1,
  AIH_OPND_CVEC = 2,
  AIH_OPND_CVEC_TENSOR = 3,
  AIH_OPND_PVEC_TENSOR = 4,
  AIH_OPND_TILED_TENSOR = 5
};
typedef struct {
  uint32_t n, h, w, c;
  int32_t op;      /* enum aih_binop */
  int32_t act;     /* enum aih_act, applied after op */
  int32_t dt;
  int32_t operand; /* enum aih_operand */
  float scalar;
  int32_t scalar_first;
  uint32_t b_c;    /* channels of a tensor operand b (vector kinds) */
} aih_binary_desc;
int aih_binary(const aih_binary_desc *d, const void *a, const void *b, void *y, aih_stream stream);

/* Channel concat (model.rs:160-164): the output holds parts[0] channels, then
 * parts[1] ..., any channel counts. */
typedef struct {
  uint32_t n, h, w;
  int32_t dt;
  uint32_t nparts; /* 1..8 */
  aih_src parts[8];
} aih_concat_desc;
int aih_concat(const aih_concat_desc *d, const void *const *inputs, void *y, aih_stream stream);

/* A Resize whose output only a Concat reads, folded into the concat: one
 * launch writes the h x w concat, part i (parts[i] of inputs[i]) read at
 * ih x iw and resized as aih_resize does when bit i of `resized` is set
 * (the same coordinates, weights and arithmetic, so the same bits), and
 * copied at oh x ow as aih_concat does otherwise. Every part but the last has
 * a multiple of 4 channels. No counterpart in the reference, which runs the
 * two ops as two dispatches (crates/ai-gpu-runtime/src/lowering.rs:335-388,
 * the Resize and Concat arms); aih_model_load uses it for that pattern. */
typedef struct {
  uint32_t n, ih, iw, oh, ow;
  int32_t mode; /* enum aih_coord */
  int32_t dt;
  uint32_t nparts;  /* 1..8 */
  uint32_t resized; /* bit i: part i is resized from ih x iw */
  aih_src parts[8];
} aih_resize_concat_desc;
int aih_resize_concat(const aih_resize_concat_desc *d, const void *const *inputs, void *y, aih_stream stream);

/* ---- model ---- */

typedef struct aih_model aih_model;

/* Parses `bytes` (a whole .sw container, copied; the caller may free it
 * afterwards), uploads the weights and allocates every tensor for a batch of
 * n images (n >= 1; the reference has n = 1). dt = -1 keeps the file's dtypes
 * (dt_default for activations, dt_weights for std conv weights,
 * format/model.rs:245-254); AIH_F16 / AIH_BF16 converts an fp32 file's
 * weights and biases to that dtype at load (round to nearest even) and runs
 * every activation in it. Returns NULL on failure (aih_last_error). The model
 * uses the current HIP device. */
aih_model *aih_model_load(const void *bytes, size_t len, uint32_t n, int32_t dt);

/* aih_model_load with load flags. By default (flags 0, and aih_model_load)
 * every inverted-residual block of the graph runs as one fused launch
 * (aih_ir_block): a 1x1 expand, a 3x3 depthwise reading only the expand's
 * output and a 1x1 projection reading only the depthwise's output,
 * consecutive in the file's op order, whose two intermediate tensors no other
 * op, alias, graph output or state uses, and that aih_ir_block_plan accepts
 * (the plan's deterministic choice of kernel, tile and weight placement).
 * A stem conv reading the graph's fp32 input (the route of
 * aih_conv_stem_f32in) whose output only the next fused block reads, as its
 * input and residual, joins that block's launch (aih_ir_block_stem, where it
 * plans) when the input is uploaded (staged); an input written into its slot
 * instead runs the stem and the block as two launches.
 * A 1x1 conv with at most 4 outputs (a segmentation head) right after a
 * fused block whose output it alone reads joins that block's launch
 * (aih_ir_block_head, the split kernel) where the block's plan is the split
 * kernel, or where load-time tuning finds the joined launch faster.
 * Elsewhere, a 3x3 depthwise and the 1x1 conv after it that alone reads its
 * output run as one aih_conv_dwpw launch when its plan has a tile for every
 * CU (weights in the activation dtype). A Resize whose output only the
 * Concat right after it reads runs inside that concat's launch
 * (aih_resize_concat) when every concat part but the last has a multiple of
 * 4 channels (any dtypes). The intermediates are then never stored:
 * reading, writing or querying them fails, and aih_model_infer_range may not
 * split a fused block. The reference runtime dispatches the convs separately
 * (lowering.rs:122-152); this fusion has no counterpart there and keeps each
 * conv's arithmetic and rounding points. AIH_MODEL_NO_FUSE lowers every op on
 * its own. AIH_MODEL_TUNE times each fused inverted-residual block's launch
 * options at load (the plan's choice; the wave, split and tile kernels at a
 * set of forced tiles, weight placements and wavefront counts; for a stem
 * or a head joined to its block, the two launches against the joined one at
 * those tiles; a few launches each on the model's own buffers) and keeps the
 * fastest, as the
 * reference's Model::load does its per-model device work once
 * (model.rs:56-366); aih_model_fused_block reports the choice. */
enum aih_model_flags { AIH_MODEL_NO_FUSE = 1, AIH_MODEL_TUNE = 2 };
aih_model *aih_model_load_ex(const void *bytes, size_t len, uint32_t n, int32_t dt, uint32_t flags);
void aih_model_free(aih_model *m);

/* Logical NHWC fp32 (n*h*w*c floats) of an input -> its NHWC-C4 tensor. host
 * memory (the copy completes before the call returns) or, for the _device
 * variant, device memory. */
int aih_model_upload_input(aih_model *m, const char *name, const float *host_nhwc, size_t count,
                           aih_stream stream);
int aih_model_upload_input_device(aih_model *m, const char *name, const float *dev_nhwc, size_t count,
                                  aih_stream stream);
/* Runs every op in order on `stream` (asynchronous). */
int aih_model_infer(aih_model *m, aih_stream stream);
/* Runs ops [first, last) only (per-op timing and parity; the reference's
 * ai-cpu profiler times op by op, crates/ai-cpu/src/model.rs:241-272). A
 * fused block's ops run together: a range must hold all of them or none. */
int aih_model_infer_range(aih_model *m, uint32_t first, uint32_t last, aih_stream stream);
/* A tensor (by name; outputs and any other tensor) as logical NHWC fp32,
 * n*h*w*c floats; waits for `stream`. */
int aih_model_read_output(aih_model *m, const char *name, float *host_nhwc, size_t count, aih_stream stream);
/* Overwrites any tensor (a channel view too: the other channels of its
 * backing buffer are kept) with logical NHWC fp32 values, n*h*w*c floats;
 * waits for `stream` and completes before returning. */
int aih_model_write_tensor(aih_model *m, const char *name, const float *host_nhwc, size_t count,
                           aih_stream stream);
/* Zeroes the state tensors (SwState inputs and outputs). */
int aih_model_reset(aih_model *m, aih_stream stream);

typedef struct {
  void *data;       /* device pointer of the tensor's first element (its view start) */
  size_t bytes;     /* bytes of the backing NHWC-C4 buffer from `data` on */
  uint32_t n, h, w, c;
  uint32_t stride_c; /* channels per pixel of the backing buffer (multiple of 4) */
  int32_t dt;
} aih_tensor_info;
int aih_model_tensor(const aih_model *m, const char *name, aih_tensor_info *out);

typedef struct {
  uint32_t n_tensors, n_ops, n_inputs, n_outputs;
  uint32_t n_launches; /* kernel launches of one aih_model_infer from a staged upload: ops, less n_ops - 1 per fused block */
  uint32_t n_fused;    /* fused blocks (every aih_fused_kind) */
  int32_t dt, wdt;
  size_t device_bytes; /* weights + tensors + workspace */
} aih_model_info;
int aih_model_get_info(const aih_model *m, aih_model_info *out);

/* Fused block i (0 <= i < n_fused): its kind, first op and op count (it
 * covers ops first_op .. first_op + n_ops - 1); for an inverted-residual
 * block (n_ops 3) the plan aih_ir_block runs it with, for the stem conv fused
 * into the block after it (n_ops 4, first_op the stem's) the plan of
 * aih_ir_block_stem, for a block joined to the head after it (n_ops 4,
 * first_op the block's expand) the plan of aih_ir_block_head, for a
 * depthwise -> pointwise pair (n_ops 2) the plan of aih_conv_dwpw; a resize
 * folded into a concat (n_ops 2) has no plan (both zeroed). */
enum aih_fused_kind {
  AIH_FUSED_IR_BLOCK = 0,     /* aih_ir_block */
  AIH_FUSED_DWPW = 1,         /* aih_conv_dwpw */
  AIH_FUSED_STEM_BLOCK = 2,   /* aih_ir_block_stem */
  AIH_FUSED_BLOCK_HEAD = 3,   /* aih_ir_block_head */
  AIH_FUSED_RESIZE_CONCAT = 4 /* aih_resize_concat */
};
typedef struct {
  uint32_t first_op;
  uint32_t n_ops;
  aih_ir_plan plan;
  aih_dwpw_plan dwpw;
  int32_t kind; /* enum aih_fused_kind */
} aih_model_fused_info;
int aih_model_fused_block(const aih_model *m, uint32_t i, aih_model_fused_info *out);
/* Name of input / output i (valid while m lives). */
const char *aih_model_input_name(const aih_model *m, uint32_t i);
const char *aih_model_output_name(const aih_model *m, uint32_t i);

/* Parses a .sw container without a device, checks every op's geometry as
 * aih_model_load does before any device work (output / residual / operand /
 * part shapes against the op, weight and bias lengths against the packed
 * layouts), and writes a one-line JSON summary (name, dtypes, tensor / op
 * counts per kind) into buf. Returns the summary's length, or AIH_ERR (the
 * container or graph is invalid, inconsistent or unsupported). */
int aih_sw_describe(const void *bytes, size_t len, char *buf, size_t buflen);

#ifdef __cplusplus
}
#endif

#endif /* AIH_MODEL_H */

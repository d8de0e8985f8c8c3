// sw_ops.hip -- the non-conv ops of a segmentation graph (include/aih_model.h):
// bilinear resize with concat parts (and a resize folded into the concat that
// reads it), global average pool, binary elementwise with the six SwOperand
// kinds, channel concat. All are streaming kernels over NHWC-C4 with fp32
// arithmetic on the storage dtype: one thread per output vec4 (gpool: a
// workgroup per image and channel group; resize: a workgroup per pair of
// output rows, its threads over the rows' vec4s); the grids cover the output
// exactly and every index is checked against it. Output vec4 counts are kept
// below 2^32 (checked on the host) so the index decomposition is 32-bit with
// precomputed divisors.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <string>

#include "../../include/aih_model.h"
#include "aih_device.h"
#include "capi_util.h"

namespace aih {
namespace {

constexpr int kMaxParts = 8;

// One input part: device base, channels per pixel of its buffer, first
// channel, channels, first output channel.
struct PartArg {
  const void *p;
  uint32_t stride_c, c_off, c, out_c0;
};
struct Parts {
  PartArg v[kMaxParts];
  uint32_t n;
  uint32_t resized;  // resize_kernel: bit p set = part p is bilinear-resized
};

template <int DT>
__device__ __forceinline__ float ld1(const void *base, size_t i) {
  if constexpr (DT == DT_F32) return reinterpret_cast<const float *>(base)[i];
  else if constexpr (DT == DT_F16) return f16_to_f32(reinterpret_cast<const uint16_t *>(base)[i]);
  else return bf16_to_f32(reinterpret_cast<const uint16_t *>(base)[i]);
}

// ---------------------------------------------------------------- resize

// reference/resize.rs:13-43: src coordinate, taps clamped to the image,
// weights clamped to [0, 1]; out = top*(1-ty) + bot*ty with top and bot the
// same blend along x. Every product and sum is rounded on its own (no fused
// multiply-add), as the reference's scalar code computes them, so fp32
// results equal the reference's bit for bit. The scales (in / out, one fp32
// division) come from the host, where IEEE division gives the same value.
struct Coord {
  uint32_t i0, i1;
  float t, u;  // weight of i1, and 1 - t (the weight of i0)
};

__device__ __forceinline__ Coord resize_coord(uint32_t o, float scale, int mode, uint32_t in) {
#pragma clang fp contract(off)
  const float of = (float)o;  // exact: sizes are checked below 2^24
  const float f = mode == AIH_COORD_HALF_PIXEL ? (of + 0.5f) * scale - 0.5f : of * scale;
  const float fl = floorf(f);
  const int b = (int)fl;  // -1 <= b <= in: fits
  const int hi = (int)in - 1;
  Coord c;
  c.i0 = (uint32_t)min(max(b, 0), hi);
  c.i1 = (uint32_t)min(max(b + 1, 0), hi);
  c.t = fminf(fmaxf(f - fl, 0.0f), 1.0f);
  c.u = 1.0f - c.t;
  return c;
}

__device__ __forceinline__ f32x4 lerp4(f32x4 a, f32x4 b, float t, float u) {
#pragma clang fp contract(off)
  return a * u + b * t;
}

// Vec4 `idx` of a part: a 32-bit byte offset from the part's base when the
// host found every part below 4 GiB (O32; the loads then take the base in
// scalar registers and one 32-bit offset), else 64-bit indexing.
template <int DT, bool O32>
__device__ __forceinline__ f32x4 part_load(const void *base, size_t idx) {
  if constexpr (O32)
    return Vec4IO<DT>::load(static_cast<const char *>(base) + (uint32_t)idx * (DT == DT_F32 ? 16u : 8u), 0);
  else
    return Vec4IO<DT>::load(base, idx);
}

// One workgroup per group of one or two consecutive output rows of an image
// (`off` = 1: row 0 alone, then rows 2k - 1, 2k -- the pairs a 2x half-pixel
// upsample maps to one source row pair; `off` = 0: rows 2k, 2k + 1). The
// group's source rows and y weights are computed once, and the threads stride
// over the row's ow * cg output vec4s (stores of consecutive threads are
// consecutive). Part p with bit p of parts.resized set is read at ih x iw and
// blended from its four taps -- when both rows of the group have the same
// two source rows, their x blends (top, bot) are computed once and only the y
// blend differs: the same operations on the same values as two separate rows
// -- any other part is read at the output's own pixel (a plain concat part).
// Lanes past a part's channels are stored as 0. The loop over parts is
// uniform, so each part's fields sit in scalar registers; a lane takes the one
// part its vec4 lies in.
template <int DT, bool O32>
__device__ __forceinline__ void resize_vec(const PartArg &pa, bool resized, uint32_t k0, uint32_t ox, size_t pa_row,
                                           size_t pb_row, bool two, bool shared, size_t a0, size_t a1, size_t b0,
                                           size_t b1, const Coord &ca, const Coord &cb, float sx, int mode,
                                           uint32_t iw, f32x4 &va, f32x4 &vb) {
  const uint32_t cgi = pa.stride_c / 4, q = (pa.c_off + k0) / 4;
  if (resized) {
    const Coord cx = resize_coord(ox, sx, mode, iw);
    auto blend_x = [&](size_t r) {
      const f32x4 l = part_load<DT, O32>(pa.p, (r + cx.i0) * cgi + q);
      const f32x4 h = part_load<DT, O32>(pa.p, (r + cx.i1) * cgi + q);
      return lerp4(l, h, cx.t, cx.u);
    };
    const f32x4 top = blend_x(a0), bot = blend_x(a1);
    va = lerp4(top, bot, ca.t, ca.u);
    if (shared) {
      vb = lerp4(top, bot, cb.t, cb.u);
    } else if (two) {
      const f32x4 top_b = blend_x(b0), bot_b = blend_x(b1);
      vb = lerp4(top_b, bot_b, cb.t, cb.u);
    }
  } else {
    va = part_load<DT, O32>(pa.p, (pa_row + ox) * cgi + q);
    if (two) vb = part_load<DT, O32>(pa.p, (pb_row + ox) * cgi + q);
  }
#pragma unroll
  for (int l = 0; l < 4; ++l)
    if (k0 + l >= pa.c) va[l] = vb[l] = 0.0f;
}

// Rows of up to 1024 vec4s take one thread per vec4 (the block rounded up
// to whole wavefronts); longer rows 256 threads that stride over the row.
template <int DT, bool O32>
__global__ __launch_bounds__(1024) void resize_kernel(Parts parts, uint32_t ih, uint32_t iw, uint32_t oh,
                                                      uint32_t ow, float sy, float sx, int mode, uint32_t cg_out,
                                                      FastDiv fd_cg, uint32_t groups, FastDiv fd_groups,
                                                      uint32_t off, void *y) {
  const uint32_t img = fdiv(blockIdx.x, fd_groups);
  const uint32_t k = blockIdx.x - img * groups;
  const uint32_t ra = off ? (k == 0 ? 0u : 2 * k - 1) : 2 * k;
  const bool two = !(off && k == 0) && ra + 1 < oh;
  const Coord ca = resize_coord(ra, sy, mode, ih);
  const Coord cb = resize_coord(two ? ra + 1 : ra, sy, mode, ih);
  const bool shared = two && ca.i0 == cb.i0 && ca.i1 == cb.i1;
  const size_t ib = (size_t)img * ih;
  const size_t a0 = (ib + ca.i0) * iw, a1 = (ib + ca.i1) * iw, b0 = (ib + cb.i0) * iw, b1 = (ib + cb.i1) * iw;
  const size_t row_a = (size_t)img * oh + ra;  // output (and plain part) rows
  const uint32_t nrow = ow * cg_out;
  for (uint32_t j = threadIdx.x; j < nrow; j += blockDim.x) {
    const uint32_t ox = fdiv(j, fd_cg);
    const uint32_t g4 = (j - ox * cg_out) * 4;
    f32x4 va = {}, vb = {};
    for (uint32_t p = 0; p < parts.n; ++p) {
      const PartArg &pa = parts.v[p];
      const uint32_t end = p + 1 < parts.n ? parts.v[p + 1].out_c0 : 0xffffffffu;
      if (g4 >= pa.out_c0 && g4 < end)
        resize_vec<DT, O32>(pa, (parts.resized >> p) & 1u, g4 - pa.out_c0, ox, row_a * ow, (row_a + 1) * ow, two,
                            shared, a0, a1, b0, b1, ca, cb, sx, mode, iw, va, vb);
    }
    Vec4IO<DT>::store(y, row_a * nrow + j, va);
    if (two) Vec4IO<DT>::store(y, (row_a + 1) * nrow + j, vb);
  }
}

// ---------------------------------------------------------------- gpool

// reference/pool.rs:6-19: sum over pixels, times 1/(h*w). One workgroup per
// (image, channel group); the 256 threads stride over the pixels and reduce
// in LDS.
template <int DT>
__global__ __launch_bounds__(256) void gpool_kernel(const void *x, uint32_t hw, uint32_t cg, float inv, void *y) {
  __shared__ f32x4 red[256];
  const uint32_t img = blockIdx.x / cg, g = blockIdx.x % cg;
  f32x4 s = {};
  for (uint32_t p = threadIdx.x; p < hw; p += 256) s += Vec4IO<DT>::load(x, ((size_t)img * hw + p) * cg + g);
  red[threadIdx.x] = s;
  __syncthreads();
  for (uint32_t o = 128; o > 0; o >>= 1) {
    if (threadIdx.x < o) red[threadIdx.x] += red[threadIdx.x + o];
    __syncthreads();
  }
  if (threadIdx.x == 0) Vec4IO<DT>::store(y, (size_t)img * cg + g, red[0] * inv);
}

// ---------------------------------------------------------------- binary

__device__ __forceinline__ float bin_apply(int op, float a, float b) {
  switch (op) {
    case AIH_BIN_ADD: return a + b;
    case AIH_BIN_SUB: return a - b;
    case AIH_BIN_MUL: return a * b;
    default: return a > 0.0f ? a : a * b;  // prelu
  }
}

template <int DT>
__global__ __launch_bounds__(256) void binary_kernel(const void *a, const void *b, void *y, uint32_t total,
                                                     uint32_t hw, uint32_t c, int op, int act, int operand,
                                                     float scalar, int scalar_first, uint32_t b_c, FastDiv fd_cg,
                                                     FastDiv fd_hw) {
  const uint32_t cg = (c + 3) / 4;
  const uint32_t i = blockIdx.x * 256 + threadIdx.x;
  if (i >= total) return;
  const uint32_t pix = fdiv(i, fd_cg);  // image-major pixel index
  const uint32_t g = i - pix * cg;
  const uint32_t img = fdiv(pix, fd_hw);
  const f32x4 va = Vec4IO<DT>::load(a, i);
  f32x4 vb;
  switch (operand) {
    case AIH_OPND_TENSOR: vb = Vec4IO<DT>::load(b, i); break;
    case AIH_OPND_SCALAR: vb = f32x4{scalar, scalar, scalar, scalar}; break;
    case AIH_OPND_CVEC: vb = Vec4IO<DT>::load(b, g); break;
    case AIH_OPND_CVEC_TENSOR: {
      // a one-channel vector is a runtime scalar (ai-cpu model.rs:483-491)
      if (b_c == 1) {
        const float s = ld1<DT>(b, (size_t)img * 4);
        vb = f32x4{s, s, s, s};
      } else {
        vb = Vec4IO<DT>::load(b, (size_t)img * ((b_c + 3) / 4) + g);
      }
      break;
    }
    case AIH_OPND_PVEC_TENSOR: {
      // one value per pixel: a pixel grid with one channel, or a 1x1 vector
      // of hw channels (ai-cpu model.rs:494-500)
      const uint32_t p = pix - img * hw;
      const float s = b_c == 1 ? ld1<DT>(b, (size_t)pix * 4) : ld1<DT>(b, (size_t)img * ((b_c + 3) / 4) * 4 + p);
      vb = f32x4{s, s, s, s};
      break;
    }
    default: {  // tiled: channel k takes b[k % b_c]
      const uint32_t bcg = (b_c + 3) / 4;
#pragma unroll
      for (int l = 0; l < 4; ++l) {
        const uint32_t k = (g * 4 + l) % b_c;
        vb[l] = ld1<DT>(b, ((size_t)img * bcg) * 4 + k);
      }
      break;
    }
  }
  const Act ap = act_params(act);
  float v[4];
#pragma unroll
  for (int l = 0; l < 4; ++l) v[l] = scalar_first ? bin_apply(op, vb[l], va[l]) : bin_apply(op, va[l], vb[l]);
  act_array<4>(ap, v);
  Vec4IO<DT>::store(y, i, f32x4{v[0], v[1], v[2], v[3]});
}

// ---------------------------------------------------------------- concat

// Any channel counts: every output lane finds its part; padding lanes are 0.
// When every part but the last holds a multiple of 4 channels (VEC), each
// output vec4 lies in one part and is one vector copy (padding lanes of the
// last part's vec4 are zeroed).
template <int DT, bool VEC>
__global__ __launch_bounds__(256) void concat_kernel(Parts parts, uint32_t total, uint32_t c_out, FastDiv fd_cg,
                                                     void *y) {
  const uint32_t cg = (c_out + 3) / 4;
  const uint32_t i = blockIdx.x * 256 + threadIdx.x;
  if (i >= total) return;
  const uint32_t pix = fdiv(i, fd_cg);
  const uint32_t g = i - pix * cg;
  if constexpr (VEC) {
    uint32_t p = 0;
    while (p + 1 < parts.n && g * 4 >= parts.v[p + 1].out_c0) ++p;
    const PartArg &pa = parts.v[p];
    const uint32_t k0 = g * 4 - pa.out_c0;
    f32x4 v = Vec4IO<DT>::load(pa.p, ((size_t)pix * pa.stride_c + pa.c_off + k0) / 4);
#pragma unroll
    for (int l = 0; l < 4; ++l)
      if (k0 + l >= pa.c) v[l] = 0.0f;
    Vec4IO<DT>::store(y, i, v);
    return;
  }
  f32x4 v = {};
#pragma unroll
  for (int l = 0; l < 4; ++l) {
    const uint32_t ch = g * 4 + l;
    if (ch >= c_out) continue;
    uint32_t p = 0;
    while (p + 1 < parts.n && ch >= parts.v[p + 1].out_c0) ++p;
    const PartArg &pa = parts.v[p];
    v[l] = ld1<DT>(pa.p, (size_t)pix * pa.stride_c + pa.c_off + (ch - pa.out_c0));
  }
  Vec4IO<DT>::store(y, i, v);
}

// ---------------------------------------------------------------- host side

bool dt_ok(int32_t dt) { return dt == AIH_F32 || dt == AIH_F16 || dt == AIH_BF16; }
bool aligned(const void *p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }
size_t vec_bytes(int32_t dt) { return dt == AIH_F32 ? 16 : 8; }

dim3 grid_for(uint64_t threads) { return dim3((unsigned)((threads + 255) / 256)); }

// Validates parts and fills the kernel's table; out_c = total channels.
int fill_parts(const aih_src *src, uint32_t nsrc, const void *const *inputs, int32_t dt, bool vec_aligned,
               Parts *parts, uint32_t *out_c) {
  if (nsrc == 0 || nsrc > kMaxParts) return api_fail("1 to 8 parts");
  if (!inputs) return api_fail("null inputs");
  uint32_t c0 = 0;
  for (uint32_t i = 0; i < nsrc; ++i) {
    const aih_src &s = src[i];
    if (!inputs[i]) return api_fail("null input part");
    if (s.c == 0 || s.stride_c == 0 || s.stride_c % 4 || s.c_off % 4 || s.c_off + s.c > s.stride_c)
      return api_fail("part view: need c > 0, stride_c and c_off multiples of 4, c_off + c <= stride_c");
    if (vec_aligned && i + 1 < nsrc && s.c % 4) return api_fail("every part but the last needs a multiple of 4 channels");
    if (!aligned(inputs[i], vec_bytes(dt))) return api_fail("misaligned input part");
    parts->v[i] = PartArg{inputs[i], s.stride_c, s.c_off, s.c, c0};
    c0 += s.c;
  }
  parts->n = nsrc;
  parts->resized = 0;
  *out_c = c0;
  return AIH_OK;
}

// Shared by aih_resize (every part resized) and aih_resize_concat. `all`:
// every part is resized; else bit i of `mask` picks part i. Sizes stay below
// 2^24 so output coordinates convert to fp32 exactly.
int launch_resize(const char *what, uint32_t n, uint32_t ih, uint32_t iw, uint32_t oh, uint32_t ow, int32_t mode,
                  int32_t dt, const aih_src *srcs, uint32_t nsrcs, bool all, uint32_t mask,
                  const void *const *inputs, void *y, aih_stream stream) {
  const std::string w(what);
  if (!dt_ok(dt)) return api_fail(w + ": unknown dtype");
  if (!n || !ih || !iw || !oh || !ow) return api_fail(w + ": zero-sized dimension");
  if (ih >= (1u << 24) || iw >= (1u << 24) || oh >= (1u << 24) || ow >= (1u << 24))
    return api_fail(w + ": sizes must stay below 2^24");
  if (mode != AIH_COORD_HALF_PIXEL && mode != AIH_COORD_ASYMMETRIC) return api_fail(w + ": unknown mode");
  if (!y || !aligned(y, vec_bytes(dt))) return api_fail(w + ": null or misaligned output");
  Parts parts;
  uint32_t c = 0;
  if (fill_parts(srcs, nsrcs, inputs, dt, true, &parts, &c)) return AIH_ERR;
  if (!all && (mask >> nsrcs) != 0) return api_fail(w + ": resized bits past the parts");
  parts.resized = all ? (1u << nsrcs) - 1u : mask;
  const uint32_t cg = (c + 3) / 4;
  const uint64_t rows = (uint64_t)n * oh;
  const uint64_t total = rows * ow * cg;
  if (total > 0xffffff00ull || rows > 0x7fffffffull) return api_fail(w + ": output too large");
  const uint32_t nrow = ow * cg;
  const uint32_t threads = nrow <= 1024 ? (nrow + 63) / 64 * 64 : 256u;
  // every part's vec4s (its ih x iw or oh x ow pixels times stride_c / 4) below 4 GiB
  bool o32 = true;
  for (uint32_t i = 0; i < nsrcs; ++i) {
    const bool rs = (parts.resized >> i) & 1u;
    const uint64_t px = (uint64_t)n * (rs ? (uint64_t)ih * iw : (uint64_t)oh * ow);
    o32 = o32 && px * srcs[i].stride_c / 4 * vec_bytes(dt) < (1ull << 32);
  }
  const float sy = (float)ih / (float)oh, sx = (float)iw / (float)ow;
  // row groups: pairs from row 1 where that pairs rows of the same source
  // rows more often than pairs from row 0 (a 2x upsample); only the speed
  // depends on it, the kernel checks each pair
  auto src_row = [&](uint32_t o) {
    const float f = mode == AIH_COORD_HALF_PIXEL ? ((float)o + 0.5f) * sy - 0.5f : (float)o * sy;
    return (int64_t)std::floor(f);
  };
  uint32_t share[2] = {0, 0};
  for (uint32_t o = 0; o + 1 < oh && o < 64; ++o)
    if (src_row(o) == src_row(o + 1)) ++share[o & 1];
  const uint32_t off = share[1] > share[0] ? 1u : 0u;
  const uint32_t groups = off ? 1 + oh / 2 : (oh + 1) / 2;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)(n * groups)), block(threads);
  const FastDiv fcg = make_fastdiv(cg), fgr = make_fastdiv(groups);
#define AIH_RESIZE_LAUNCH(D, O)                                                                                  \
  hipLaunchKernelGGL((resize_kernel<D, O>), grid, block, 0, st, parts, ih, iw, oh, ow, sy, sx, (int)mode, cg, fcg, \
                     groups, fgr, off, y)
  switch (dt) {
    case AIH_F32: if (o32) AIH_RESIZE_LAUNCH(DT_F32, true); else AIH_RESIZE_LAUNCH(DT_F32, false); break;
    case AIH_F16: if (o32) AIH_RESIZE_LAUNCH(DT_F16, true); else AIH_RESIZE_LAUNCH(DT_F16, false); break;
    default: if (o32) AIH_RESIZE_LAUNCH(DT_BF16, true); else AIH_RESIZE_LAUNCH(DT_BF16, false); break;
  }
#undef AIH_RESIZE_LAUNCH
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? AIH_OK : api_fail(w + " launch: " + hipGetErrorString(e));
}

}  // namespace
}  // namespace aih

using namespace aih;

#define AIH_LAUNCH_DT(KERNEL, dt, grid, st, ...)                                           \
  do {                                                                                     \
    switch (dt) {                                                                          \
      case AIH_F32: hipLaunchKernelGGL(KERNEL<DT_F32>, grid, dim3(256), 0, st, __VA_ARGS__); break; \
      case AIH_F16: hipLaunchKernelGGL(KERNEL<DT_F16>, grid, dim3(256), 0, st, __VA_ARGS__); break; \
      default: hipLaunchKernelGGL(KERNEL<DT_BF16>, grid, dim3(256), 0, st, __VA_ARGS__); break;     \
    }                                                                                      \
  } while (0)

#define AIH_LAUNCH_DT2(KERNEL, B, dt, grid, st, ...)                                                  \
  do {                                                                                               \
    switch (dt) {                                                                                    \
      case AIH_F32: hipLaunchKernelGGL((KERNEL<DT_F32, B>), grid, dim3(256), 0, st, __VA_ARGS__); break;  \
      case AIH_F16: hipLaunchKernelGGL((KERNEL<DT_F16, B>), grid, dim3(256), 0, st, __VA_ARGS__); break;  \
      default: hipLaunchKernelGGL((KERNEL<DT_BF16, B>), grid, dim3(256), 0, st, __VA_ARGS__); break;      \
    }                                                                                                \
  } while (0)

extern "C" {

int aih_resize(const aih_resize_desc *d, const void *const *inputs, void *y, aih_stream stream) {
  return api_guarded([&] {
    if (!d) return api_fail("resize: null descriptor");
    return launch_resize("resize", d->n, d->ih, d->iw, d->oh, d->ow, d->mode, d->dt, d->srcs, d->nsrcs, true, 0,
                         inputs, y, stream);
  });
}

int aih_resize_concat(const aih_resize_concat_desc *d, const void *const *inputs, void *y, aih_stream stream) {
  return api_guarded([&] {
    if (!d) return api_fail("resize_concat: null descriptor");
    return launch_resize("resize_concat", d->n, d->ih, d->iw, d->oh, d->ow, d->mode, d->dt, d->parts, d->nparts,
                         false, d->resized, inputs, y, stream);
  });
}

int aih_gpool(const aih_gpool_desc *d, const void *x, void *y, aih_stream stream) {
  return api_guarded([&] {
    if (!d) return api_fail("gpool: null descriptor");
    if (!dt_ok(d->dt)) return api_fail("gpool: unknown dtype");
    if (!d->n || !d->h || !d->w || !d->c) return api_fail("gpool: zero-sized dimension");
    if (!x || !y || !aligned(x, vec_bytes(d->dt)) || !aligned(y, vec_bytes(d->dt)))
      return api_fail("gpool: null or misaligned buffer");
    const uint32_t cg = (d->c + 3) / 4;
    const uint64_t blocks = (uint64_t)d->n * cg;
    if (blocks > 0x7fffffffull || (uint64_t)d->h * d->w > 0xffffffffull) return api_fail("gpool: too large");
    const float inv = 1.0f / (float)(d->h * d->w);
    hipStream_t st = static_cast<hipStream_t>(stream);
    AIH_LAUNCH_DT(gpool_kernel, d->dt, dim3((unsigned)blocks), st, x, d->h * d->w, cg, inv, y);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? AIH_OK : api_fail(std::string("gpool launch: ") + hipGetErrorString(e));
  });
}

int aih_binary(const aih_binary_desc *d, const void *a, const void *b, void *y, aih_stream stream) {
  return api_guarded([&] {
    if (!d) return api_fail("binary: null descriptor");
    if (!dt_ok(d->dt)) return api_fail("binary: unknown dtype");
    if (!d->n || !d->h || !d->w || !d->c) return api_fail("binary: zero-sized dimension");
    if (d->op < AIH_BIN_ADD || d->op > AIH_BIN_PRELU) return api_fail("binary: unknown op");
    if (d->act < AIH_ACT_NONE || d->act > AIH_ACT_RECIP) return api_fail("binary: unknown activation");
    if (d->operand < AIH_OPND_TENSOR || d->operand > AIH_OPND_TILED_TENSOR) return api_fail("binary: unknown operand");
    const bool tensor_b = d->operand == AIH_OPND_CVEC_TENSOR || d->operand == AIH_OPND_PVEC_TENSOR ||
                          d->operand == AIH_OPND_TILED_TENSOR;
    if (tensor_b && d->b_c == 0) return api_fail("binary: vector operands need b_c > 0");
    if (d->operand == AIH_OPND_CVEC_TENSOR && d->b_c != 1 && d->b_c != d->c)
      return api_fail("binary: a channel vector needs 1 or c channels");
    if (d->operand == AIH_OPND_PVEC_TENSOR && d->b_c != 1 && d->b_c != d->h * d->w)
      return api_fail("binary: a pixel vector needs 1 channel or h*w channels");
    const size_t vb = vec_bytes(d->dt);
    if (!a || !y || !aligned(a, vb) || !aligned(y, vb)) return api_fail("binary: null or misaligned a / y");
    if (d->operand != AIH_OPND_SCALAR && (!b || !aligned(b, tensor_b ? vb / 4 : vb)))
      return api_fail("binary: null or misaligned b");
    const uint64_t total = (uint64_t)d->n * d->h * d->w * ((d->c + 3) / 4);
    if (total > 0xffffff00ull) return api_fail("binary: too large");
    hipStream_t st = static_cast<hipStream_t>(stream);
    AIH_LAUNCH_DT(binary_kernel, d->dt, grid_for(total), st, a, b, y, (uint32_t)total, d->h * d->w, d->c,
                  (int)d->op, (int)d->act, (int)d->operand, d->scalar, (int)d->scalar_first, d->b_c,
                  make_fastdiv((d->c + 3) / 4), make_fastdiv(d->h * d->w));
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? AIH_OK : api_fail(std::string("binary launch: ") + hipGetErrorString(e));
  });
}

int aih_concat(const aih_concat_desc *d, const void *const *inputs, void *y, aih_stream stream) {
  return api_guarded([&] {
    if (!d) return api_fail("concat: null descriptor");
    if (!dt_ok(d->dt)) return api_fail("concat: unknown dtype");
    if (!d->n || !d->h || !d->w) return api_fail("concat: zero-sized dimension");
    if (!y || !aligned(y, vec_bytes(d->dt))) return api_fail("concat: null or misaligned output");
    Parts parts;
    uint32_t c = 0;
    if (fill_parts(d->parts, d->nparts, inputs, d->dt, false, &parts, &c)) return AIH_ERR;
    const uint64_t px = (uint64_t)d->n * d->h * d->w;
    const uint64_t total = px * ((c + 3) / 4);
    if (total > 0xffffff00ull) return api_fail("concat: too large");
    bool vec = true;
    for (uint32_t i = 0; i + 1 < d->nparts; ++i) vec = vec && d->parts[i].c % 4 == 0;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const FastDiv fd = make_fastdiv((c + 3) / 4);
    if (vec)
      AIH_LAUNCH_DT2(concat_kernel, true, d->dt, grid_for(total), st, parts, (uint32_t)total, c, fd, y);
    else
      AIH_LAUNCH_DT2(concat_kernel, false, d->dt, grid_for(total), st, parts, (uint32_t)total, c, fd, y);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? AIH_OK : api_fail(std::string("concat launch: ") + hipGetErrorString(e));
  });
}

}  // extern "C"

// aih_device.h -- device-side helpers shared by the gfx950 conv kernels:
// storage dtypes (f32 / f16 / bf16 with fp32 accumulation), 16-byte vector
// types, the fused epilogue activation, and an XCD-aware workgroup remap.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

#include "../../include/aih_conv.h"

namespace aih {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Storage dtype tags (same values as enum aih_dtype).
enum : int { DT_F32 = 0, DT_F16 = 1, DT_BF16 = 2 };

template <int DT> struct Storage;
template <> struct Storage<DT_F32> { using T = float; static constexpr int bytes = 4; };
template <> struct Storage<DT_F16> { using T = uint16_t; static constexpr int bytes = 2; };
template <> struct Storage<DT_BF16> { using T = uint16_t; static constexpr int bytes = 2; };

__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) { return __uint_as_float(bits16 << 16); }

// f32 -> bf16, round to nearest even; NaN stays a quiet NaN.
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

__device__ __forceinline__ float f16_to_f32(uint32_t bits16) {
  _Float16 h;
  uint16_t b = (uint16_t)bits16;
  __builtin_memcpy(&h, &b, 2);
  return (float)h;
}

// f32 -> f16 via the hardware conversion (round to nearest even).
__device__ __forceinline__ uint32_t f32_to_f16(float f) {
  _Float16 h = (_Float16)f;
  uint16_t b;
  __builtin_memcpy(&b, &h, 2);
  return b;
}

// Register-level conversions of 4 packed 16-bit values (one 8-byte vec4).
template <int DT>
__device__ __forceinline__ f32x4 unpack4(u32x2 r) {
  if constexpr (DT == DT_F16)
    return f32x4{f16_to_f32(r.x & 0xffffu), f16_to_f32(r.x >> 16), f16_to_f32(r.y & 0xffffu),
                 f16_to_f32(r.y >> 16)};
  else
    return f32x4{bf16_to_f32(r.x & 0xffffu), bf16_to_f32(r.x >> 16), bf16_to_f32(r.y & 0xffffu),
                 bf16_to_f32(r.y >> 16)};
}

// fp32 -> 4 packed 16-bit values, round to nearest even: gfx950's
// v_cvt_pk_{f16,bf16}_f32 convert two values per instruction.
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

template <int DT>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  if constexpr (DT == DT_F16)
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, f16x2));
  else
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
}

template <int DT>
__device__ __forceinline__ u32x2 pack4(f32x4 v) {
  return u32x2{pack2<DT>(v.x, v.y), pack2<DT>(v.z, v.w)};
}

// 4 consecutive channels (one vec4 of NHWC-C4) <-> fp32.
template <int DT> struct Vec4IO;

template <> struct Vec4IO<DT_F32> {
  static __device__ __forceinline__ f32x4 load(const void *base, size_t vec_idx) {
    return reinterpret_cast<const f32x4 *>(base)[vec_idx];
  }
  static __device__ __forceinline__ void store(void *base, size_t vec_idx, f32x4 v) {
    reinterpret_cast<f32x4 *>(base)[vec_idx] = v;
  }
};

template <> struct Vec4IO<DT_F16> {
  static __device__ __forceinline__ f32x4 load(const void *base, size_t vec_idx) {
    u32x2 r = reinterpret_cast<const u32x2 *>(base)[vec_idx];
    return f32x4{f16_to_f32(r.x & 0xffffu), f16_to_f32(r.x >> 16), f16_to_f32(r.y & 0xffffu),
                 f16_to_f32(r.y >> 16)};
  }
  static __device__ __forceinline__ void store(void *base, size_t vec_idx, f32x4 v) {
    reinterpret_cast<u32x2 *>(base)[vec_idx] = pack4<DT_F16>(v);
  }
};

template <> struct Vec4IO<DT_BF16> {
  static __device__ __forceinline__ f32x4 load(const void *base, size_t vec_idx) {
    u32x2 r = reinterpret_cast<const u32x2 *>(base)[vec_idx];
    return f32x4{bf16_to_f32(r.x & 0xffffu), bf16_to_f32(r.x >> 16), bf16_to_f32(r.y & 0xffffu),
                 bf16_to_f32(r.y >> 16)};
  }
  static __device__ __forceinline__ void store(void *base, size_t vec_idx, f32x4 v) {
    reinterpret_cast<u32x2 *>(base)[vec_idx] = pack4<DT_BF16>(v);
  }
};

// Epilogue activation (ai-core Activation::apply, crates/ai-core/src/activation.rs:28-43).
// `act` is uniform across the grid, so the switch does not diverge. Every
// case is a few instructions (hardware exp2 / rcp / sqrt, ~1 ulp), so the
// fused epilogue stays small: a libm-accurate expf/tanhf inlined at every
// output element multiplies the kernel's code size and register demand.
// tanh clamps its input to +-9 as the reference's WGSL does
// (crates/ai-gpu/src/kernels/common/activation.rs:20); at |x| = 9 tanh is 1
// to within 2e-8.
__device__ __forceinline__ float act_apply(int act, float x) {
  switch (act) {
    case AIH_ACT_NONE: return x;
    case AIH_ACT_RELU: return fmaxf(x, 0.0f);
    case AIH_ACT_SIGMOID: return __builtin_amdgcn_rcpf(1.0f + __expf(-x));
    case AIH_ACT_TANH: {
      const float e = __expf(2.0f * fminf(fmaxf(x, -9.0f), 9.0f));
      return (e - 1.0f) * __builtin_amdgcn_rcpf(e + 1.0f);
    }
    case AIH_ACT_HARDSWISH: return x * fminf(fmaxf(x * (1.0f / 6.0f) + 0.5f, 0.0f), 1.0f);
    case AIH_ACT_HARDSIGMOID: return fminf(fmaxf(x * (1.0f / 6.0f) + 0.5f, 0.0f), 1.0f);
    case AIH_ACT_CLAMP01: return fminf(fmaxf(x, 0.0f), 1.0f);
    case AIH_ACT_RELU6: return fminf(fmaxf(x, 0.0f), 6.0f);
    case AIH_ACT_SQRT: return __builtin_amdgcn_sqrtf(fmaxf(x, 0.0f));
    case AIH_ACT_NEG: return -x;
    case AIH_ACT_RECIP: return __builtin_amdgcn_rcpf(x);
    default: return x;
  }
}

__device__ __forceinline__ f32x4 act_apply4(int act, f32x4 v) {
  return f32x4{act_apply(act, v.x), act_apply(act, v.y), act_apply(act, v.z), act_apply(act, v.w)};
}

// The activation as wave-uniform parameters, so that inner loops apply it
// without a per-element switch: every activation the converter fuses into a
// conv is one of
//   IDENT   v = x                              none
//   LINEAR  v = x*s + t                        neg
//   RELU    v = max(x, 0)                      relu
//   CLAMP0  v = min(max(x, 0), hi)             relu6, clamp01
//   CLAMP   v = min(max(x*s + t, 0), hi)       hardsigmoid
//   XCLAMP  v = x * min(max(x*s + t, 0), hi)   hardswish
// and the transcendental ones (sigmoid, tanh, sqrt, recip) go through act_apply.
// Clamps to [0, hi] with hi >= 0 are taken on the float bits as signed
// integers, whose order agrees with the floats' for non-negative values while
// every negative float (and -0) is a negative integer: one v_max_i32 /
// v_med3_i32 instead of a float max that must first quiet signalling NaNs.
// They return +0 for negative inputs (and -0) like max(x, 0); NaN inputs are
// the one difference from the float form (a NaN with the sign bit clear is
// kept, one with it set becomes 0).
struct Act {
  float s, t, hi;
  int hib;  // bits of hi
  int mode;
  int act;
  float clo, chi;  // clamp-type activations: the clamp interval ([-inf, inf] for the identity)
};
enum : int { ACT_LINEAR = 0, ACT_CLAMP = 1, ACT_XCLAMP = 2, ACT_SPECIAL = 3, ACT_IDENT = 4, ACT_RELU = 5,
             ACT_CLAMP0 = 6 };

// Activations that are a clamp to an interval [clo, chi]: the identity,
// ReLU, ReLU6 and clamp01.
__host__ __device__ __forceinline__ bool act_is_clamp(int act) {
  return act == AIH_ACT_NONE || act == AIH_ACT_RELU || act == AIH_ACT_RELU6 || act == AIH_ACT_CLAMP01;
}

__device__ __forceinline__ Act act_params(int act) {
  Act p{1.0f, -0.0f, 0.0f, 0, ACT_LINEAR, act, 0.0f, 0.0f};
  switch (act) {
    case AIH_ACT_NONE: p.mode = ACT_IDENT; break;
    case AIH_ACT_NEG: p.s = -1.0f; break;
    case AIH_ACT_RELU: p.mode = ACT_RELU; break;
    case AIH_ACT_RELU6: p.mode = ACT_CLAMP0; p.hi = 6.0f; break;
    case AIH_ACT_CLAMP01: p.mode = ACT_CLAMP0; p.hi = 1.0f; break;
    case AIH_ACT_HARDSIGMOID:
      p.mode = ACT_CLAMP; p.s = 1.0f / 6.0f; p.t = 0.5f; p.hi = 1.0f;
      break;
    case AIH_ACT_HARDSWISH:
      p.mode = ACT_XCLAMP; p.s = 1.0f / 6.0f; p.t = 0.5f; p.hi = 1.0f;
      break;
    default: p.mode = ACT_SPECIAL; break;
  }
  p.hib = __float_as_int(p.hi);
  p.clo = p.mode == ACT_IDENT ? -__builtin_huge_valf() : 0.0f;
  p.chi = p.mode == ACT_CLAMP0 ? p.hi : __builtin_huge_valf();
  return p;
}

// A clamp-type activation (act_is_clamp) without a branch: one v_med3_f32
// with the interval [clo, chi] (the identity is [-inf, inf]). Only a zero's
// sign can differ from max / min; a NaN input stays NaN. (A builtin rather
// than inline asm: the values often come straight from an MFMA, and only
// instructions the compiler sees get the wait states an MFMA result needs.)
__device__ __forceinline__ float act_clamp_any(const Act &p, float x) {
  return __builtin_amdgcn_fmed3f(x, p.clo, p.chi);
}

__device__ __forceinline__ float act_relu_bits(float x) { return __int_as_float(max(__float_as_int(x), 0)); }
__device__ __forceinline__ float act_clamp_bits(float x, int hib) {
  return __int_as_float(min(max(__float_as_int(x), 0), hib));
}

// Applies p to N values; the only branch is on the uniform mode.
template <int N>
__device__ __forceinline__ void act_array(const Act &p, float (&v)[N]) {
  switch (p.mode) {
    case ACT_IDENT:
      break;
    case ACT_RELU:
#pragma unroll
      for (int j = 0; j < N; ++j) v[j] = act_relu_bits(v[j]);
      break;
    case ACT_CLAMP0:
#pragma unroll
      for (int j = 0; j < N; ++j) v[j] = act_clamp_bits(v[j], p.hib);
      break;
    case ACT_LINEAR:
#pragma unroll
      for (int j = 0; j < N; ++j) v[j] = v[j] * p.s + p.t;
      break;
    case ACT_CLAMP:
#pragma unroll
      for (int j = 0; j < N; ++j) v[j] = act_clamp_bits(v[j] * p.s + p.t, p.hib);
      break;
    case ACT_XCLAMP:
#pragma unroll
      for (int j = 0; j < N; ++j) v[j] = v[j] * act_clamp_bits(v[j] * p.s + p.t, p.hib);
      break;
    default:
#pragma unroll
      for (int j = 0; j < N; ++j) v[j] = act_apply(p.act, v[j]);
      break;
  }
}

__device__ __forceinline__ f32x4 act4(const Act &p, f32x4 x) {
  float v[4] = {x.x, x.y, x.z, x.w};
  act_array<4>(p, v);
  return f32x4{v[0], v[1], v[2], v[3]};
}

// Division by a launch-uniform divisor d without the ~35-instruction
// integer division: q = (umulhi(n, m) + n) >> s with s = ceil(log2 d) and
// m = floor(2^32 (2^s - d) / d) + 1 (the round-up multiply-high method of
// Granlund and Montgomery, 1994), exact for every 32-bit n and d >= 1.
struct FastDiv {
  uint32_t d, m, s;
};

inline FastDiv make_fastdiv(uint32_t d) {
  uint32_t s = 0;
  while ((1ull << s) < d) ++s;
  const uint64_t m = ((1ull << 32) * ((1ull << s) - d)) / d + 1;
  return FastDiv{d, (uint32_t)m, s};
}

__device__ __forceinline__ uint32_t fdiv(uint32_t n, const FastDiv &f) {
  return (uint32_t)(((uint64_t)__umulhi(n, f.m) + n) >> f.s);
}

// MI355X dispatches consecutive workgroup ids round-robin over its XCDs (8
// on a whole device), each with a private L2. Remap so that every XCD walks a
// contiguous range of logical tiles: neighbouring tiles (which share input
// rows / halos) then hit the same L2. Bijective on [0, n) for any nxcd >= 1.
__device__ __forceinline__ uint32_t xcd_remap(uint32_t bid, uint32_t n, uint32_t nxcd) {
  if (nxcd <= 1) return bid;
  uint32_t per = n / nxcd;
  if (bid >= per * nxcd) return bid;
  return (bid % nxcd) * per + bid / nxcd;
}

// Launch facts of the current device, queried once per device ordinal:
// compute units (grids and split decisions) and XCDs (xcd_remap). A failed
// query falls back to a whole MI355X (256 CUs in 8 XCDs).
struct DeviceInfo {
  uint32_t cus, xcds;
};

inline DeviceInfo device_info() {
  static std::mutex mu;
  static DeviceInfo cache[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return DeviceInfo{256, 8};
  std::lock_guard<std::mutex> lock(mu);
  DeviceInfo &d = cache[dev];
  if (d.cus == 0) {
    int cus = 0, xcds = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    if (hipDeviceGetAttribute(&xcds, hipDeviceAttributeNumberOfXccs, dev) != hipSuccess || xcds <= 0) xcds = 8;
    d = DeviceInfo{(uint32_t)cus, (uint32_t)xcds};
  }
  return d;
}
inline uint32_t device_cus() { return device_info().cus; }
inline uint32_t device_xcds() { return device_info().xcds; }

}  // namespace aih

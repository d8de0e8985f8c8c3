// conv_pw_stream.hip -- fp32 pointwise conv GEMM for long K over many pixels
// (960 -> 160 at 10x18, batch 256: M = 46080, K = 960, N = 160), the role of
// gemm_pw_tiled.wgsl (crates/ai-gpu/src/kernels/gemm_pw.rs) for those shapes,
// with the bias -> act -> +residual epilogue of common/epilogue.rs:13-30.
//
// Work unit: a wavefront owns 32 output pixels x TN blocks of 32 output
// channels over the whole K; a workgroup is WM x WN such wavefronts sharing
// one tile (32 WM pixels x 32 WN TN channels). Small wavefront units keep
// the grid fine-grained -- 960 -> 160 at batch 256 has 7200 of them for the
// 1024 SIMDs instead of the 1440 a 32 x 160 unit gives -- so every SIMD ends
// within one unit of the others without splitting K (the K split that the
// 128 x 160 tiles needed cost 118 MB of partial sums each way and a second
// launch).
//
// K runs in stages of 16 channels (4 kg). A stage's operands -- the tile's
// pixel rows and weight rows -- go from memory into LDS by DMA (buffer loads
// with the LDS as destination, 1 KB per instruction, no registers, no
// address arithmetic beyond one add per stage), NST - 1 stages ahead of the
// MFMAs; one workgroup barrier per stage publishes a landed stage and frees
// the oldest buffer. Pixel rows sit in LDS as 4 16-byte units per pixel with
// the unit index XORed by bits 1-2 of the pixel, so the MFMA operand reads
// (8 pixels, one unit each, per LDS cycle) touch 8 distinct bank groups; the
// DMA lanes still read each pixel's 64 bytes as one contiguous run. Weight
// rows of odd kg hold column n at n ^ 4, so the lanes of the two lane halves
// (kg 2q and 2q + 1 of the same columns) also fall in different banks.
//
// MFMA mapping (v_mfma_f32_32x32x2f32, operands swapped so the result is
// channel-major): A = weights (32 channels x K), B = activations (K x 32
// pixels); lane half h takes unit 2q + h of pair q for both operands, four
// MFMAs per unit (one per fp32 component). Lane l of the result holds pixel
// l%32 and channels 8*(r/4) + 4*(l/32) + r%4 (r = 0..15): one 16-byte
// NHWC-C4 vector per lane and r/4, stored straight from registers.
#include <hip/hip_runtime.h>

#include "aih_device.h"
#include "conv_pw_stream.h"

namespace aih {
namespace {

typedef __attribute__((address_space(3))) void ps_lds_void;
constexpr uint32_t kOob = 0x80000000u;  // a byte offset past both buffers

__device__ __forceinline__ __amdgpu_buffer_rsrc_t ps_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, (int)bytes, 0x00020000);
}

// LDS slot of unit u of tile pixel p is 4p + (u ^ ps_swz(p)): bits 1 and 2
// of p swapped into a 2-bit XOR. The 8 pixels an LDS cycle serves (8
// consecutive lanes, one unit each) land in 8 distinct 16-byte bank groups,
// and so do 4 consecutive lanes together with the 4 lanes 32 above them
// (the same pixels, the neighbouring unit).
__device__ __forceinline__ uint32_t ps_swz(uint32_t p) { return (((p >> 1) & 1) << 1) | ((p >> 2) & 1); }

// s_waitcnt vmcnt(N) (expcnt and lgkmcnt not waited for).
template <int N>
__device__ __forceinline__ void ps_wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
}

// vmcnt(n) for a wavefront-uniform n in [0, MAXN].
template <int MAXN>
__device__ __forceinline__ void ps_wait_vm_n(uint32_t n) {
  if constexpr (MAXN > 0) {
    if (n >= (uint32_t)MAXN) {
      ps_wait_vm<MAXN>();
      return;
    }
    ps_wait_vm_n<MAXN - 1>(n);
  } else {
    ps_wait_vm<0>();
  }
}

template <int WM, int WN, int TN, int NST>
__global__ __launch_bounds__(64 * WM * WN) void pw_stream_kernel(PwStreamArgs a) {
  constexpr int NW = WM * WN;
  constexpr int BM = 32 * WM, BN = 32 * WN * TN;
  constexpr int A_INS = BM / 16, W_INS = BN / 16, NI = A_INS + W_INS;  // 1 KB DMA instructions per stage
  constexpr int MI = (NI + NW - 1) / NW;                              // the most one wavefront issues
  constexpr uint32_t A_BYTES = BM * 64, STAGE = (BM + BN) * 64;
  static_assert(NST >= 2, "stages");
  extern __shared__ __align__(16) char lds[];

  const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, lh = lane >> 5;
  // wavefront-uniform: every branch on it is a scalar branch
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave % WM, wn = wave / WM;

  const uint32_t t = xcd_remap(blockIdx.x, gridDim.x, a.nxcd);
  const uint32_t mt = t / a.ntiles, nt = t - mt * a.ntiles;
  const uint32_t m0 = mt * BM, n0 = nt * BN;
  const uint32_t nst = (a.KG + 3) / 4;

  const __amdgpu_buffer_rsrc_t rs_x = ps_rsrc(a.x, a.x_bytes);
  const __amdgpu_buffer_rsrc_t rs_w = ps_rsrc(a.w, a.w_bytes);

  // This wavefront's DMA instructions (i = wave + k * NW): pixel-row
  // instruction i < A_INS moves pixels 16i .. 16i + 15 (lane -> pixel
  // lane / 4, LDS slot lane % 4 holding unit (lane % 4) ^ bits 1-2 of the
  // pixel); weight instruction i - A_INS moves (kg, column) entries
  // 64 (i - A_INS) + lane of the stage's [4][BN] rows. Per lane: the byte
  // offset at stage 0, its step per stage, the kg inside the stage, and
  // whether the pixel / column exists.
  uint32_t d_off[MI], d_step[MI], d_kg[MI];
  bool d_ok[MI];
  uint32_t nmine = 0;
#pragma unroll
  for (int k = 0; k < MI; ++k) {
    const int i = wave + k * NW;
    d_off[k] = 0;
    d_step[k] = 0;
    d_kg[k] = 0;
    d_ok[k] = false;
    if (i < A_INS) {
      const uint32_t p = 16 * i + (lane >> 2);
      const uint32_t u = (uint32_t)(lane & 3) ^ ps_swz(p);
      const uint32_t m = m0 + p;
      d_ok[k] = m < a.M;
      d_off[k] = (m * a.KG + u) * 16;
      d_step[k] = 64;
      d_kg[k] = u;
      ++nmine;
    } else if (i < NI) {
      const uint32_t e = 64 * (i - A_INS) + lane;
      const uint32_t kgl = e / BN, n = (e - kgl * BN) ^ (4 * (kgl & 1));
      d_ok[k] = n0 + n < a.N4;
      d_off[k] = (kgl * a.N4 + n0 + n) * 16;
      d_step[k] = 64 * a.N4;
      d_kg[k] = kgl;
      ++nmine;
    }
  }
  auto issue = [&](uint32_t s, uint32_t b) {
    char *base = lds + b * STAGE;
#pragma unroll
    for (int k = 0; k < MI; ++k) {
      const int i = wave + k * NW;
      if (i >= NI) break;
      const bool ok = d_ok[k] & (4 * s + d_kg[k] < a.KG);
      const uint32_t off = ok ? d_off[k] + s * d_step[k] : kOob;
      const uint32_t dst = i < A_INS ? (uint32_t)i * 1024 : A_BYTES + (uint32_t)(i - A_INS) * 1024;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(i < A_INS ? rs_x : rs_w, (ps_lds_void *)(base + dst), 16, off, 0, 0,
                                               0);
    }
  };

  // LDS byte offsets (inside a stage) of this lane's operands of pair q
  const uint32_t p = 32 * wm + l32;  // tile pixel of this lane
  uint32_t a_off[2];
  uint32_t w_off[2][TN];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const uint32_t u = 2 * q + lh;
    a_off[q] = (4 * p + (u ^ ps_swz(p))) * 16;
#pragma unroll
    for (int tn = 0; tn < TN; ++tn)
      w_off[q][tn] = A_BYTES + (u * BN + ((32 * TN * wn + 32 * tn + l32) ^ (4 * lh))) * 16;
  }

  f32x16 acc[TN];
#pragma unroll
  for (int tn = 0; tn < TN; ++tn) acc[tn] = f32x16{};

  auto compute = [&](uint32_t b) {
    const char *base = lds + b * STAGE;
    u32x4 bv[2], av[2][TN];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      bv[q] = *reinterpret_cast<const u32x4 *>(base + a_off[q]);
#pragma unroll
      for (int tn = 0; tn < TN; ++tn) av[q][tn] = *reinterpret_cast<const u32x4 *>(base + w_off[q][tn]);
    }
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const f32x4 x4 = __builtin_bit_cast(f32x4, bv[q]);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) {
          const f32x4 w4 = __builtin_bit_cast(f32x4, av[q][tn]);
          acc[tn] = __builtin_amdgcn_mfma_f32_32x32x2f32(w4[c], x4[c], acc[tn], 0, 0, 0);
        }
      }
    }
  };

  // ---- pipeline: stage s + NST - 1 is requested while stage s computes ----
#pragma unroll
  for (int s = 0; s < NST - 1; ++s)
    if ((uint32_t)s < nst) issue((uint32_t)s, (uint32_t)s);
  uint32_t b_cmp = 0, b_iss = NST - 1;  // buffer of the stage computed / requested
  for (uint32_t s = 0; s < nst; ++s) {
    // this wavefront's copies of stage s have landed once at most those of
    // the stages requested after it are still in flight
    const uint32_t later = nst - 1 - s < (uint32_t)(NST - 2) ? nst - 1 - s : (uint32_t)(NST - 2);
    ps_wait_vm_n<MI *(NST - 2)>(later * nmine);
    // every wavefront's copies of stage s are in LDS, and every wavefront is
    // done with stage s - 1, whose buffer the next request reuses (its LDS
    // reads returned before its MFMAs). A bare barrier: __syncthreads()'s
    // workgroup fence would also wait for the copies still in flight.
    __asm__ volatile("s_barrier" ::: "memory");
    if (s + NST - 1 < nst) issue(s + NST - 1, b_iss);
    compute(b_cmp);
    b_cmp = b_cmp + 1 == NST ? 0 : b_cmp + 1;
    b_iss = b_iss + 1 == NST ? 0 : b_iss + 1;
  }

  // ---- epilogue: act(acc + bias) (+ residual), 16 bytes per lane ----
  const Act actp = act_params(a.act);
  const uint32_t m = m0 + p;
  if (m >= a.M) return;
#pragma unroll
  for (int tn = 0; tn < TN; ++tn) {
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      const uint32_t c = n0 + 32 * TN * wn + 32 * tn + 8 * r4 + 4 * lh;
      if (c >= a.N4) continue;
      f32x4 v = f32x4{acc[tn][4 * r4], acc[tn][4 * r4 + 1], acc[tn][4 * r4 + 2], acc[tn][4 * r4 + 3]} +
                reinterpret_cast<const f32x4 *>(a.bias)[c / 4];
      v = act4(actp, v);
      const size_t vi = ((size_t)m * a.N4 + c) / 4;
      if (a.has_res) v += reinterpret_cast<const f32x4 *>(a.res)[vi];
      reinterpret_cast<f32x4 *>(a.y)[vi] = v;
    }
  }
}

template <int WM, int WN, int TN, int NST>
hipError_t launch_inst(const PwStreamArgs &a, hipStream_t st) {
  constexpr uint32_t lds = NST * (32 * WM + 32 * WN * TN) * 64;
  static const hipError_t attr =
      hipFuncSetAttribute(reinterpret_cast<const void *>(pw_stream_kernel<WM, WN, TN, NST>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  if (attr != hipSuccess) return attr;
  hipLaunchKernelGGL((pw_stream_kernel<WM, WN, TN, NST>), dim3(a.mtiles * a.ntiles), dim3(64 * WM * WN), lds, st,
                     a);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_pw_stream(const PwStreamArgs &a, const PwStreamShape &s, hipStream_t st) {
  if (a.M == 0 || a.KG == 0 || a.N4 == 0 || a.N4 % 4 || a.x_bytes >= 0x80000000u || a.w_bytes >= 0x80000000u ||
      (uint64_t)a.M * a.KG * 16 > a.x_bytes || a.mtiles != (a.M + pw_stream_bm(s) - 1) / pw_stream_bm(s) ||
      a.ntiles != (a.N4 + pw_stream_bn(s) - 1) / pw_stream_bn(s) || (uint64_t)a.mtiles * a.ntiles > 0x7fffffffu)
    return hipErrorInvalidValue;
#define AIH_PS_CASE(WM, WN, TN, NST) \
  if (s.wm == WM && s.wn == WN && s.tn == TN && s.nst == NST) return launch_inst<WM, WN, TN, NST>(a, st);
  AIH_PS_CASE(3, 5, 1, 2)
  AIH_PS_CASE(3, 4, 1, 2)
  AIH_PS_CASE(3, 3, 1, 2)
  AIH_PS_CASE(3, 2, 1, 2)
#undef AIH_PS_CASE
  return hipErrorInvalidValue;
}

}  // namespace aih

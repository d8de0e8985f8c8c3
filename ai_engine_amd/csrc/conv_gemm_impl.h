// conv_gemm_impl.h -- the MFMA conv-as-GEMM kernel for gfx950 (CDNA4).
//
// One kernel template serves the pointwise 1x1 GEMM (the role of
// gemm_pw_{tiled,small,gemv,splitk}.wgsl, crates/ai-gpu/src/kernels/gemm_pw.rs)
// and the KxK implicit GEMM (conv_igemm_{tiled,direct,splitk}.wgsl,
// crates/ai-gpu/src/kernels/conv_igemm.rs), with the bias -> act -> +residual
// epilogue of common/epilogue.rs:13-30 fused in registers.
//
// GEMM view:  out[m, n] = sum_k A[m, k] * B[k, n]
//   m = output pixel (batch folded in), n = output channel,
//   k = (tap, input channel); the K loop walks "kg" groups of 4 channels.
//   A is never materialised: each kg of a row is loaded straight from the
//   NHWC-C4 input at the source pixel of that tap (implicit im2col, addresses
//   computed in registers, padding by predication).
//   B is the packed weight [tap][kg_pad][ng][j][comp] (pack.rs:68-102): for a
//   fixed (tap, kg) row, channel n holds 4 consecutive K values, so a 16-byte
//   (f32) or 8-byte (16-bit) vector per (kg, n) is already MFMA-shaped.
//
// MFMA mapping (operands swapped so the accumulator is channel-major):
//   MFMA "A" = weights  (32 output channels x K), MFMA "B" = activations
//   (K x 32 pixels). With v_mfma_f32_32x32x*, lane l of the result holds
//   pixel l%32 and channels 8*(r/4) + 4*(l/32) + r%4 for r = 0..15, i.e. four
//   float4 runs of consecutive channels -> 128-bit NHWC-C4 epilogue stores.
//   fp32:    v_mfma_f32_32x32x2f32, four per 16-byte K unit pair
//   f16/bf16: v_mfma_f32_32x32x16_{f16,bf16}, one per 16-byte K unit pair
//   Lane half h = l/32 always takes K unit 2p+h of pair p for both operands,
//   so the K pairing is consistent whatever order the hardware sums in.
//
// Tiling: 256 threads = 4 wavefronts; block tile BM = 128 pixels x BN
// channels; each wave owns 32 pixels x BN channels (BN/32 accumulator tiles of
// 16 VGPRs). K is staged through LDS in BKU 16-byte units per stage, double
// buffered: global loads of stage s+1 are issued before the MFMAs of stage s
// and written to the other LDS buffer afterwards (one barrier per stage).
//
// Split-K: the grid's third axis cuts K into chunks; each chunk writes fp32
// partials [split][M][N4] and splitk_reduce sums them in split order (a fixed
// order, so results are deterministic) and applies the epilogue.
#pragma once

#include <type_traits>

#include "aih_device.h"

namespace aih {

struct GemmArgs {
  const void *src[3];     // input parts (1 for a plain input)
  uint32_t part_kg[3];    // first kg (within a tap) of each part
  uint32_t stride_kg[3];  // pixel stride of each part, in kg (4-channel) units
  uint32_t off_kg[3];     // first kg of each part inside its pixel
  uint32_t nparts;
  const void *w;          // [tap][KGP][NG][4][4]
  const void *bias;       // [N4]
  const void *res;        // like y, or null
  void *y;                // NHWC-C4 output, N4 channels per pixel
  float *partial;         // [nsplit][M][N4] fp32, split-K only
  uint32_t M;             // output pixels over the whole batch
  uint32_t OHW, OW;       // output pixels per image, output width
  uint32_t IH, IW;        // input height, width
  uint32_t K, S, D;       // kernel size, stride, dilation
  int32_t PT, PL;         // top / left padding
  uint32_t KG, KGP;       // input kg per tap, packed-weight kg per tap
  uint32_t KK;            // taps * KG
  uint32_t N4;            // output channels padded to 4
  uint32_t kk_chunk;      // kg per split chunk (multiple of the stage depth)
  uint32_t nsplit;
  uint32_t mtiles, ntiles;
  int32_t act;
  int32_t has_res;
};

constexpr int GEMM_THREADS = 256;
constexpr int GEMM_BM = 128;

template <int DTA, int DTW, int BN>
struct GemmCfg {
  static constexpr bool F32 = (DTA == DT_F32);
  static constexpr int KU = F32 ? 1 : 2;                  // kg per 16-byte K unit
  static constexpr int BKU = (F32 && BN > 160) ? 4 : 8;   // K units per stage
  static constexpr int BKG = BKU * KU;                    // kg per stage
  static constexpr int TN = BN / 32;                      // accumulator tiles per wave
  static constexpr int AROW = GEMM_BM + 1;                // LDS row pitch (units), +1 against bank conflicts
  static constexpr int WROW = BN + 1;
  // A loads: one kg per item (16 B f32, 8 B 16-bit)
  static constexpr int A_EPR = BKG;                       // items per pixel row per stage
  static constexpr int A_ITEMS = GEMM_BM * A_EPR / GEMM_THREADS;
  // W loads: f32 compute: one (kg, n) per item; 16-bit: one (kg, n pair) per item (16 B)
  static constexpr int W_COLS = F32 ? BN : BN / 2;
  static constexpr int W_ITEMS = BKG * W_COLS / GEMM_THREADS;
  static_assert(GEMM_BM * A_EPR % GEMM_THREADS == 0, "A tile");
  static_assert(BKG * W_COLS % GEMM_THREADS == 0, "W tile");
  static_assert(GEMM_THREADS % A_EPR == 0, "A item mapping");
  static_assert(BN % 32 == 0, "BN");
};

template <int DTA, int DTW, int BN, bool IGEMM>
__global__ __launch_bounds__(GEMM_THREADS) void conv_gemm_kernel(GemmArgs a) {
  using Cfg = GemmCfg<DTA, DTW, BN>;
  constexpr bool F32 = Cfg::F32;
  constexpr int BKU = Cfg::BKU, BKG = Cfg::BKG, TN = Cfg::TN;
  constexpr int AROW = Cfg::AROW, WROW = Cfg::WROW;
  constexpr int A_ITEMS = Cfg::A_ITEMS, W_ITEMS = Cfg::W_ITEMS;
  constexpr int A_EPR = Cfg::A_EPR, W_COLS = Cfg::W_COLS;
  constexpr int AB = Storage<DTA>::bytes * 4;  // bytes of one activation kg vector
  constexpr int WB = Storage<DTW>::bytes * 4;  // bytes of one weight kg vector

  __shared__ u32x4 As[2][BKU][AROW];
  __shared__ u32x4 Ws[2][BKU][WROW];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int l32 = lane & 31;
  const int lh = lane >> 5;

  // ---- tile coordinates (XCD-aware order; channel tiles of one pixel tile
  // are adjacent so they share the A rows in L2) ----
  const uint32_t nblk = a.mtiles * a.ntiles * a.nsplit;
  const uint32_t L = xcd_remap(blockIdx.x, nblk);
  const uint32_t nt = L % a.ntiles;
  const uint32_t mt = (L / a.ntiles) % a.mtiles;
  const uint32_t split = L / (a.ntiles * a.mtiles);
  const uint32_t m0 = mt * GEMM_BM;
  const uint32_t n0 = nt * BN;
  const uint32_t kk_begin = split * a.kk_chunk;
  uint32_t kk_end = kk_begin + a.kk_chunk;
  if (kk_end > a.KK) kk_end = a.KK;

  // ---- per-thread A rows: decode the output pixel once ----
  const int a_e = tid % A_EPR;  // kg slot within a stage (same for every item)
  int a_row[A_ITEMS];
  bool a_ok[A_ITEMS];
  int32_t a_iy0[A_ITEMS], a_ix0[A_ITEMS];
  uint32_t a_px[A_ITEMS];  // IGEMM: first pixel of the image; PW: the pixel itself
#pragma unroll
  for (int i = 0; i < A_ITEMS; ++i) {
    const int r = (i * GEMM_THREADS + tid) / A_EPR;
    a_row[i] = r;
    const uint32_t m = m0 + r;
    a_ok[i] = m < a.M;
    if constexpr (IGEMM) {
      const uint32_t mm = a_ok[i] ? m : 0;
      const uint32_t img = mm / a.OHW;
      const uint32_t rem = mm - img * a.OHW;
      const uint32_t oy = rem / a.OW;
      const uint32_t ox = rem - oy * a.OW;
      a_iy0[i] = (int32_t)(oy * a.S) - a.PT;
      a_ix0[i] = (int32_t)(ox * a.S) - a.PL;
      a_px[i] = img * a.IH * a.IW;
    } else {
      a_iy0[i] = 0;
      a_ix0[i] = 0;
      a_px[i] = m;
    }
  }

  using AReg = typename std::conditional<F32, u32x4, u32x2>::type;
  using WLoad = typename std::conditional<(F32 && DTW != DT_F32), u32x2, u32x4>::type;
  AReg areg[A_ITEMS];
  WLoad wreg[W_ITEMS];

  const char *wbase = reinterpret_cast<const char *>(a.w);
  const uint32_t wrow_vecs = a.N4;  // kg vectors per packed weight row

  auto load_stage = [&](uint32_t k0) {
    // ---- A: one kg of one pixel row per item ----
    const uint32_t kk = k0 + a_e;
    const bool k_ok = kk < kk_end;
    uint32_t tap = 0, kg = kk;
    int32_t dy = 0, dx = 0;
    if constexpr (IGEMM) {
      tap = kk / a.KG;
      kg = kk - tap * a.KG;
      const uint32_t ky = tap / a.K;
      const uint32_t kx = tap - ky * a.K;
      dy = (int32_t)(ky * a.D);
      dx = (int32_t)(kx * a.D);
    }
    // part of this kg (concat parts / channel views)
    uint32_t p = 0;
    if (a.nparts > 1) p = (kg >= a.part_kg[1]) + (a.nparts > 2 && kg >= a.part_kg[2]);
    const char *src = reinterpret_cast<const char *>(p == 0 ? a.src[0] : (p == 1 ? a.src[1] : a.src[2]));
    const uint32_t pstride = p == 0 ? a.stride_kg[0] : (p == 1 ? a.stride_kg[1] : a.stride_kg[2]);
    const uint32_t poff = (p == 0 ? a.off_kg[0] : (p == 1 ? a.off_kg[1] : a.off_kg[2])) +
                          kg - (p == 0 ? a.part_kg[0] : (p == 1 ? a.part_kg[1] : a.part_kg[2]));
#pragma unroll
    for (int i = 0; i < A_ITEMS; ++i) {
      bool ok = k_ok && a_ok[i];
      uint32_t pix = a_px[i];
      if constexpr (IGEMM) {
        const int32_t iy = a_iy0[i] + dy;
        const int32_t ix = a_ix0[i] + dx;
        ok = ok && (uint32_t)iy < a.IH && (uint32_t)ix < a.IW;
        pix = a_px[i] + (uint32_t)iy * a.IW + (uint32_t)ix;
      }
      AReg v = {};
      if (ok) {
        const size_t vidx = (size_t)pix * pstride + poff;
        v = *reinterpret_cast<const AReg *>(src + vidx * AB);
      }
      areg[i] = v;
    }
    // ---- W: row (tap, kg) of the packed weights ----
#pragma unroll
    for (int i = 0; i < W_ITEMS; ++i) {
      const int idx = i * GEMM_THREADS + tid;
      const int col = idx % W_COLS;
      const int kl = idx / W_COLS;
      const uint32_t wkk = k0 + kl;
      const uint32_t n = n0 + (F32 ? col : 2 * col);
      WLoad v = {};
      if (wkk < kk_end && n < a.N4) {
        uint32_t wt = 0, wkg = wkk;
        if constexpr (IGEMM) {
          wt = wkk / a.KG;
          wkg = wkk - wt * a.KG;
        }
        const size_t vidx = (size_t)(wt * a.KGP + wkg) * wrow_vecs + n;
        v = *reinterpret_cast<const WLoad *>(wbase + vidx * WB);
      }
      wreg[i] = v;
    }
  };

  auto store_stage = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_ITEMS; ++i) {
      const int r = a_row[i];
      if constexpr (F32) {
        As[buf][a_e][r] = areg[i];
      } else {
        u32x2 *dst = reinterpret_cast<u32x2 *>(&As[buf][a_e >> 1][r]) + (a_e & 1);
        *dst = areg[i];
      }
    }
#pragma unroll
    for (int i = 0; i < W_ITEMS; ++i) {
      const int idx = i * GEMM_THREADS + tid;
      const int col = idx % W_COLS;
      const int kl = idx / W_COLS;
      if constexpr (F32) {
        if constexpr (DTW == DT_F32) {
          Ws[buf][kl][col] = wreg[i];
        } else {
          const u32x2 h = wreg[i];
          f32x4 f;
          if constexpr (DTW == DT_F16) {
            f = f32x4{f16_to_f32(h.x & 0xffffu), f16_to_f32(h.x >> 16), f16_to_f32(h.y & 0xffffu),
                      f16_to_f32(h.y >> 16)};
          } else {
            f = f32x4{bf16_to_f32(h.x & 0xffffu), bf16_to_f32(h.x >> 16), bf16_to_f32(h.y & 0xffffu),
                      bf16_to_f32(h.y >> 16)};
          }
          Ws[buf][kl][col] = __builtin_bit_cast(u32x4, f);
        }
      } else {
        // (kg, n..n+1) -> half (kg & 1) of units (kg >> 1) at columns n and n+1
        const u32x4 v = wreg[i];
        u32x2 *d0 = reinterpret_cast<u32x2 *>(&Ws[buf][kl >> 1][2 * col]) + (kl & 1);
        u32x2 *d1 = reinterpret_cast<u32x2 *>(&Ws[buf][kl >> 1][2 * col + 1]) + (kl & 1);
        *d0 = u32x2{v.x, v.y};
        *d1 = u32x2{v.z, v.w};
      }
    }
  };

  f32x16 acc[TN];
#pragma unroll
  for (int t = 0; t < TN; ++t) acc[t] = f32x16{};

  const int wm = wave * 32 + l32;  // this lane's pixel row inside the block tile

  auto compute_stage = [&](int buf) {
#pragma unroll
    for (int p = 0; p < BKU / 2; ++p) {
      const int u = 2 * p + lh;
      const u32x4 bv = As[buf][u][wm];
      u32x4 av[TN];
#pragma unroll
      for (int t = 0; t < TN; ++t) av[t] = Ws[buf][u][t * 32 + l32];
      if constexpr (F32) {
        const f32x4 b = __builtin_bit_cast(f32x4, bv);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
#pragma unroll
          for (int t = 0; t < TN; ++t) {
            const f32x4 w4 = __builtin_bit_cast(f32x4, av[t]);
            acc[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(w4[c], b[c], acc[t], 0, 0, 0);
          }
        }
      } else if constexpr (DTA == DT_F16) {
        const f16x8 b = __builtin_bit_cast(f16x8, bv);
#pragma unroll
        for (int t = 0; t < TN; ++t)
          acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, av[t]), b, acc[t], 0, 0, 0);
      } else {
        const bf16x8 b = __builtin_bit_cast(bf16x8, bv);
#pragma unroll
        for (int t = 0; t < TN; ++t)
          acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, av[t]), b, acc[t], 0, 0, 0);
      }
    }
  };

  // ---- double-buffered K loop ----
  const uint32_t nst = kk_end > kk_begin ? (kk_end - kk_begin + BKG - 1) / BKG : 0;
  if (nst > 0) {
    load_stage(kk_begin);
    store_stage(0);
    __syncthreads();
    for (uint32_t s = 0; s < nst; ++s) {
      const bool more = s + 1 < nst;
      if (more) load_stage(kk_begin + (s + 1) * BKG);
      compute_stage(s & 1);
      if (more) store_stage((s + 1) & 1);
      __syncthreads();
    }
  }

  // ---- epilogue: bias -> act -> +residual, 128-bit stores ----
  const uint32_t m = m0 + wm;
  if (m >= a.M) return;
  const size_t row = (size_t)m * a.N4;
#pragma unroll
  for (int t = 0; t < TN; ++t) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t n = n0 + t * 32 + 8 * q + 4 * lh;
      if (n >= a.N4) continue;
      f32x4 v = f32x4{acc[t][4 * q + 0], acc[t][4 * q + 1], acc[t][4 * q + 2], acc[t][4 * q + 3]};
      if (a.nsplit > 1) {
        reinterpret_cast<f32x4 *>(a.partial)[((size_t)split * a.M * a.N4 + row + n) / 4] = v;
      } else {
        v += Vec4IO<DTA>::load(a.bias, n / 4);
        v = act_apply4(a.act, v);
        if (a.has_res) v += Vec4IO<DTA>::load(a.res, (row + n) / 4);
        Vec4IO<DTA>::store(a.y, (row + n) / 4, v);
      }
    }
  }
}

// Sums split-K partials in split order, then bias -> act -> +residual.
template <int DTA>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float *__restrict__ partial, uint32_t nsplit,
                                                            uint32_t M, uint32_t N4, const void *bias,
                                                            const void *res, void *y, int32_t act,
                                                            int32_t has_res) {
  const size_t nvec = (size_t)M * N4 / 4;
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= nvec) return;
  const f32x4 *p = reinterpret_cast<const f32x4 *>(partial);
  f32x4 v = p[i];
  for (uint32_t s = 1; s < nsplit; ++s) v += p[s * nvec + i];
  const uint32_t n = (uint32_t)(i % (N4 / 4)) * 4;
  v += Vec4IO<DTA>::load(bias, n / 4);
  v = act_apply4(act, v);
  if (has_res) v += Vec4IO<DTA>::load(res, i);
  Vec4IO<DTA>::store(y, i, v);
}

}  // namespace aih

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
//   pixel l%32 and channels 8*(r/4) + 4*(l/32) + r%4 for r = 0..15.
//   fp32:    v_mfma_f32_32x32x2f32, four per 16-byte K unit pair
//   f16/bf16: v_mfma_f32_32x32x16_{f16,bf16}, one per 16-byte K unit pair
//   Lane half h = l/32 always takes K unit 2p+h of pair p for both operands,
//   so the K pairing is consistent whatever order the hardware sums in.
//
// Work decomposition: a tile is 128 pixels x BN channels x one K chunk
// (split-K); 256 threads = 4 wavefronts of 32 pixels x BN channels each.
// The grid is persistent: every workgroup walks a contiguous range of tiles
// (ranges are handed out XCD by XCD, so neighbouring tiles -- which share
// input rows and halos -- stay in one L2). Each tile's K is staged through
// LDS in stages of 16 (fp32) or 32 (16-bit) channels, double buffered, and
// the pipeline runs across
// tile boundaries: the global loads of the next (tile, stage) are in flight
// while the current stage's MFMAs and the finished tile's epilogue execute.
//
// Epilogue: bias and activation are applied in the MFMA layout, then every
// wavefront stages its 32x32 fp32 block in a private LDS region and writes
// it back row by row: each lane stores 16 contiguous bytes (4 f32 or 8
// 16-bit channels), loading the residual the same way, so both the output
// stores and the residual loads are full-line 128-bit accesses.
//
// Split-K tiles write fp32 partials [split][M][N4] through the same path and
// splitk_reduce_kernel sums them in split order (deterministic) and applies
// the epilogue.
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
  uint32_t ntiles_total;  // mtiles * ntiles * nsplit
  int32_t act;
  int32_t has_res;
  uint32_t nxcd;          // XCDs of the device (workgroup remap)
  // the divisors above the kernel divides by, prepared on the host
  FastDiv fd_ntiles, fd_mtiles, fd_KG, fd_K, fd_OHW, fd_OW;
};

constexpr int GEMM_THREADS = 256;
constexpr int GEMM_BM = 128;

template <int DTA, int DTW, int BN, bool PAIR>
struct GemmCfg {
  static constexpr bool F32 = (DTA == DT_F32);
  static constexpr int KU = F32 ? 1 : 2;       // kg per 16-byte K unit
  static constexpr int BKU = 4;                // K units per stage (16 f32 / 32 16-bit channels)
  static constexpr int BKG = BKU * KU;         // kg per stage
  static constexpr int TN = BN / 32;           // accumulator tiles per wave
  static constexpr int AROW = GEMM_BM + 1;     // LDS row pitch (units), +1 against bank conflicts
  static constexpr int WROW = BN + 1;
  // A items: f32 -> one kg (16 B); 16-bit paired -> two kg (16 B); unpaired -> one kg (8 B)
  static constexpr int A_KGI = (!F32 && PAIR) ? 2 : 1;
  static constexpr int A_EPR = BKG / A_KGI;    // items per pixel row per stage
  static constexpr int A_ITEMS = GEMM_BM * A_EPR / GEMM_THREADS;
  // W items: f32 compute -> one (kg, n) 16 B (or 8 B 16-bit weights, widened);
  // 16-bit compute -> one (kg, n..n+1) 16 B
  static constexpr int W_COLS = F32 ? BN : BN / 2;
  static constexpr int W_TOTAL = BKG * W_COLS;
  static constexpr int W_ITEMS = (W_TOTAL + GEMM_THREADS - 1) / GEMM_THREADS;
  static constexpr int ST_PITCH = 36;          // staging row pitch in floats (32 + 4)
  static_assert(GEMM_BM * A_EPR % GEMM_THREADS == 0, "A tile");
  static_assert(GEMM_THREADS % A_EPR == 0, "A item mapping");
  static_assert(BN % 32 == 0, "BN");
};

template <int DTA, int DTW, int BN, bool IGEMM, bool PAIR>
__global__ __launch_bounds__(GEMM_THREADS) void conv_gemm_kernel(GemmArgs a) {
  using Cfg = GemmCfg<DTA, DTW, BN, PAIR>;
  constexpr bool F32 = Cfg::F32;
  constexpr int BKU = Cfg::BKU, BKG = Cfg::BKG, TN = Cfg::TN;
  constexpr int AROW = Cfg::AROW, WROW = Cfg::WROW;
  constexpr int A_ITEMS = Cfg::A_ITEMS, W_ITEMS = Cfg::W_ITEMS;
  constexpr int A_EPR = Cfg::A_EPR, A_KGI = Cfg::A_KGI, W_COLS = Cfg::W_COLS, W_TOTAL = Cfg::W_TOTAL;
  constexpr int ST_PITCH = Cfg::ST_PITCH;
  constexpr int AB = Storage<DTA>::bytes * 4;  // bytes of one activation kg vector
  constexpr int WB = Storage<DTW>::bytes * 4;  // bytes of one weight kg vector

  __shared__ u32x4 As[2][BKU][AROW];
  __shared__ u32x4 Ws[2][BKU][WROW];
  __shared__ float St[4][32 * ST_PITCH];
  __shared__ f32x4 Bs[2][BN / 4];  // bias of the tile, by tile parity

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int l32 = lane & 31;
  const int lh = lane >> 5;

  // ---- this workgroup's contiguous range of tiles ----
  const uint32_t blk = xcd_remap(blockIdx.x, gridDim.x, a.nxcd);
  const uint32_t t_begin = (uint32_t)(((uint64_t)blk * a.ntiles_total) / gridDim.x);
  const uint32_t t_end = (uint32_t)(((uint64_t)(blk + 1) * a.ntiles_total) / gridDim.x);
  if (t_begin >= t_end) return;

  struct TileInfo {
    uint32_t m0, n0, split, kk_begin, kk_end, nst;
  };
  auto tile_info = [&](uint32_t T) {
    TileInfo ti;
    const uint32_t q = fdiv(T, a.fd_ntiles);
    const uint32_t nt = T - q * a.ntiles;
    const uint32_t q2 = fdiv(q, a.fd_mtiles);
    const uint32_t mt = q - q2 * a.mtiles;
    ti.split = q2;
    ti.m0 = mt * GEMM_BM;
    ti.n0 = nt * BN;
    ti.kk_begin = ti.split * a.kk_chunk;
    uint32_t e = ti.kk_begin + a.kk_chunk;
    ti.kk_end = e > a.KK ? a.KK : e;
    ti.nst = ti.kk_end > ti.kk_begin ? (ti.kk_end - ti.kk_begin + BKG - 1) / BKG : 0;
    return ti;
  };

  // ---- per-thread A rows of the tile being loaded (decoded once per tile) ----
  const int a_e = tid % A_EPR;  // item slot within a stage (same for every row item)
  bool a_ok[A_ITEMS];
  int32_t a_iy0[A_ITEMS], a_ix0[A_ITEMS];
  uint32_t a_px[A_ITEMS];  // IGEMM: first pixel of the image; PW: the pixel itself
  uint32_t decoded_m0 = 0xffffffffu;
  auto decode_rows = [&](uint32_t m0) {
#pragma unroll
    for (int i = 0; i < A_ITEMS; ++i) {
      const uint32_t m = m0 + (i * GEMM_THREADS + tid) / A_EPR;
      a_ok[i] = m < a.M;
      if constexpr (IGEMM) {
        const uint32_t mm = a_ok[i] ? m : 0;
        const uint32_t img = fdiv(mm, a.fd_OHW);
        const uint32_t rem = mm - img * a.OHW;
        const uint32_t oy = fdiv(rem, a.fd_OW);
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
    decoded_m0 = m0;
  };

  using AReg = typename std::conditional<(F32 || PAIR), u32x4, u32x2>::type;
  using WLoad = typename std::conditional<(F32 && DTW != DT_F32), u32x2, u32x4>::type;
  AReg areg[A_ITEMS];
  WLoad wreg[W_ITEMS];
  f32x4 breg = {};  // bias of the next tile (threads < BN/4, stage 0 only)

  const char *wbase = reinterpret_cast<const char *>(a.w);
  const Act actp = act_params(a.act);

  auto load_stage = [&](const TileInfo &ti, uint32_t s) {
    if (decoded_m0 != ti.m0) decode_rows(ti.m0);
    if (s == 0 && tid < BN / 4) {
      const uint32_t n = ti.n0 + 4 * tid;
      breg = n < a.N4 ? Vec4IO<DTA>::load(a.bias, n / 4) : f32x4{};
    }
    const uint32_t k0 = ti.kk_begin + s * BKG;
    // ---- A: A_KGI kg of one pixel row per item ----
    const uint32_t kk = k0 + a_e * A_KGI;
    const bool k_ok = kk < ti.kk_end;
    uint32_t kg = kk;
    int32_t dy = 0, dx = 0;
    if constexpr (IGEMM) {
      const uint32_t tap = fdiv(kk, a.fd_KG);
      kg = kk - tap * a.KG;
      const uint32_t ky = fdiv(tap, a.fd_K);
      const uint32_t kx = tap - ky * a.K;
      dy = (int32_t)(ky * a.D);
      dx = (int32_t)(kx * a.D);
    }
    uint32_t p = 0;
    if (a.nparts > 1) p = (kg >= a.part_kg[1]) + (a.nparts > 2 && kg >= a.part_kg[2]);
    const char *src = reinterpret_cast<const char *>(p == 0 ? a.src[0] : (p == 1 ? a.src[1] : a.src[2]));
    const uint32_t pstride = p == 0 ? a.stride_kg[0] : (p == 1 ? a.stride_kg[1] : a.stride_kg[2]);
    const uint32_t poff = (p == 0 ? a.off_kg[0] : (p == 1 ? a.off_kg[1] : a.off_kg[2])) + kg -
                          (p == 0 ? a.part_kg[0] : (p == 1 ? a.part_kg[1] : a.part_kg[2]));
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
    // ---- W: rows (tap, kg) of the packed weights ----
#pragma unroll
    for (int i = 0; i < W_ITEMS; ++i) {
      const int idx = i * GEMM_THREADS + tid;
      const int col = idx % W_COLS;
      const int kl = idx / W_COLS;
      const uint32_t wkk = k0 + kl;
      const uint32_t n = ti.n0 + (F32 ? col : 2 * col);
      WLoad v = {};
      if ((W_TOTAL % GEMM_THREADS == 0 || idx < W_TOTAL) && wkk < ti.kk_end && n < a.N4) {
        uint32_t wt = 0, wkg = wkk;
        if constexpr (IGEMM) {
          wt = fdiv(wkk, a.fd_KG);
          wkg = wkk - wt * a.KG;
        }
        const size_t vidx = (size_t)(wt * a.KGP + wkg) * a.N4 + n;
        v = *reinterpret_cast<const WLoad *>(wbase + vidx * WB);
      }
      wreg[i] = v;
    }
  };

  auto store_stage = [&](int buf, uint32_t s, uint32_t tile_parity) {
    if (s == 0 && tid < BN / 4) Bs[tile_parity][tid] = breg;
#pragma unroll
    for (int i = 0; i < A_ITEMS; ++i) {
      const int r = (i * GEMM_THREADS + tid) / A_EPR;
      if constexpr (F32 || PAIR) {
        As[buf][a_e][r] = areg[i];
      } else {
        u32x2 *dst = reinterpret_cast<u32x2 *>(&As[buf][a_e >> 1][r]) + (a_e & 1);
        *dst = areg[i];
      }
    }
#pragma unroll
    for (int i = 0; i < W_ITEMS; ++i) {
      const int idx = i * GEMM_THREADS + tid;
      if (W_TOTAL % GEMM_THREADS != 0 && idx >= W_TOTAL) continue;
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
        // (kg, n..n+1) -> half (kg & 1) of unit (kg >> 1) at columns n and n+1
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

  const int wm = wave * 32 + l32;  // this lane's pixel row inside the tile

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

  float *st = St[wave];
  // Residual rows of one 32-channel block, in the lane layout of the
  // write-back: fp32 -> 4 passes of 8 rows (16 B = 4 channels per lane);
  // 16-bit -> 2 passes of 16 rows (16 B = 8 channels per lane).
  constexpr int PASSES = F32 ? 4 : 2;
  auto wb_row = [&](int pass) { return F32 ? pass * 8 + (lane >> 3) : pass * 16 + (lane >> 2); };
  auto wb_col = [&]() { return F32 ? (lane & 7) * 4 : (lane & 3) * 8; };
  // 16-bit rows start 16-byte aligned only when N4 % 8 == 0; otherwise the
  // 8 channels of a lane are moved as two 8-byte halves.
  const bool row16 = (a.N4 % 8) == 0;
  auto load_res = [&](const TileInfo &ti, int t, u32x4 (&r)[PASSES]) {
#pragma unroll
    for (int pass = 0; pass < PASSES; ++pass) {
      const uint32_t m = ti.m0 + wave * 32 + wb_row(pass);
      const uint32_t n = ti.n0 + t * 32 + wb_col();
      u32x4 v = {};
      if (m < a.M && n < a.N4) {
        const size_t vi = ((size_t)m * a.N4 + n) / 4;  // 4-channel vector index
        if constexpr (F32) {
          v = reinterpret_cast<const u32x4 *>(a.res)[vi];
        } else if (n + 8 <= a.N4 && row16) {
          v = reinterpret_cast<const u32x4 *>(a.res)[vi / 2];
        } else {
          const u32x2 *rp = reinterpret_cast<const u32x2 *>(a.res);
          const u32x2 h0 = rp[vi];
          const u32x2 h1 = n + 8 <= a.N4 ? rp[vi + 1] : u32x2{0u, 0u};
          v = u32x4{h0.x, h0.y, h1.x, h1.y};
        }
      }
      r[pass] = v;
    }
  };

  auto epilogue = [&](const TileInfo &ti, uint32_t tile_parity) {
    const bool split = a.nsplit > 1;
    const bool res = !split && a.has_res;
    // The residual of block t+1 is requested before block t's stores: vector
    // memory operations retire in order, so waiting for it never waits for
    // the stores that follow it.
    u32x4 rcur[PASSES], rnext[PASSES];
    if (res) load_res(ti, 0, rnext);
#pragma unroll
    for (int t = 0; t < TN; ++t) {
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int pass = 0; pass < PASSES; ++pass) rcur[pass] = rnext[pass];
      if (res && t + 1 < TN) load_res(ti, t + 1, rnext);
      // (1) bias + act in the MFMA layout, staged as fp32 [32 px][32 ch]
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int cl = 8 * q + 4 * lh;  // channel inside the 32-channel block
        f32x4 v = f32x4{acc[t][4 * q + 0], acc[t][4 * q + 1], acc[t][4 * q + 2], acc[t][4 * q + 3]};
        if (!split) v = act4(actp, v + Bs[tile_parity][(t * 32 + cl) / 4]);
        *reinterpret_cast<f32x4 *>(st + l32 * ST_PITCH + cl) = v;
      }
      __builtin_amdgcn_wave_barrier();
      // (2) row-wise write-back: 16 contiguous bytes per lane
      const uint32_t nb = ti.n0 + t * 32;
#pragma unroll
      for (int pass = 0; pass < PASSES; ++pass) {
        const int r = wb_row(pass), c = wb_col();
        const uint32_t m = ti.m0 + wave * 32 + r;
        const uint32_t n = nb + c;
        if (m >= a.M || n >= a.N4) continue;
        const size_t vi = ((size_t)m * a.N4 + n) / 4;
        if constexpr (F32) {
          f32x4 v = *reinterpret_cast<const f32x4 *>(st + r * ST_PITCH + c);
          if (split) {
            reinterpret_cast<f32x4 *>(a.partial)[(size_t)ti.split * a.M * (a.N4 / 4) + vi] = v;
          } else {
            if (res) v += __builtin_bit_cast(f32x4, rcur[pass]);
            reinterpret_cast<f32x4 *>(a.y)[vi] = v;
          }
        } else if (split) {
          // fp32 partials, 8 channels per lane
          const f32x4 v0 = *reinterpret_cast<const f32x4 *>(st + r * ST_PITCH + c);
          f32x4 *pp = reinterpret_cast<f32x4 *>(a.partial) + (size_t)ti.split * a.M * (a.N4 / 4) + vi;
          pp[0] = v0;
          if (n + 8 <= a.N4) pp[1] = *reinterpret_cast<const f32x4 *>(st + r * ST_PITCH + c + 4);
        } else {
          f32x4 v0 = *reinterpret_cast<const f32x4 *>(st + r * ST_PITCH + c);
          f32x4 v1 = *reinterpret_cast<const f32x4 *>(st + r * ST_PITCH + c + 4);
          if (res) {
            v0 += unpack4<DTA>(u32x2{rcur[pass].x, rcur[pass].y});
            v1 += unpack4<DTA>(u32x2{rcur[pass].z, rcur[pass].w});
          }
          const u32x2 lo = pack4<DTA>(v0);
          if (n + 8 <= a.N4) {
            const u32x2 hi = pack4<DTA>(v1);
            if (row16) {
              reinterpret_cast<u32x4 *>(a.y)[vi / 2] = u32x4{lo.x, lo.y, hi.x, hi.y};
            } else {
              reinterpret_cast<u32x2 *>(a.y)[vi] = lo;
              reinterpret_cast<u32x2 *>(a.y)[vi + 1] = hi;
            }
          } else {
            reinterpret_cast<u32x2 *>(a.y)[vi] = lo;
          }
        }
      }
      __builtin_amdgcn_wave_barrier();
    }
#pragma unroll
    for (int t = 0; t < TN; ++t) acc[t] = f32x16{};
  };

  // ---- software pipeline over (tile, stage) pairs of this workgroup ----
  uint32_t T = t_begin;
  TileInfo cur = tile_info(T);
  uint32_t s = 0;
  uint32_t parity = 0;  // tile parity: which Bs slot holds this tile's bias
  load_stage(cur, 0);
  store_stage(0, 0, parity);
  __syncthreads();
  int buf = 0;
  for (;;) {
    // next (tile, stage)
    uint32_t nT = T, ns = s + 1;
    TileInfo nxt = cur;
    if (ns >= cur.nst) {
      nT = T + 1;
      ns = 0;
      if (nT < t_end) nxt = tile_info(nT);
    }
    const bool more = nT < t_end;
    if (more) load_stage(nxt, ns);
    if (s < cur.nst) compute_stage(buf);
    if (ns == 0) epilogue(cur, parity);
    if (more) store_stage(buf ^ 1, ns, ns == 0 ? parity ^ 1 : parity);
    __syncthreads();
    if (!more) break;
    if (ns == 0) parity ^= 1;
    T = nT;
    s = ns;
    cur = nxt;
    buf ^= 1;
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
  v = act4(act_params(act), v);
  if (has_res) v += Vec4IO<DTA>::load(res, i);
  Vec4IO<DTA>::store(y, i, v);
}

}  // namespace aih

// dw_pw.hip -- fused depthwise KxK conv + pointwise 1x1 conv, fp32.
//
// The reference dispatches the two convs separately (lower_op's Conv arm,
// crates/ai-gpu-runtime/src/lowering.rs:122-168: conv_dw.wgsl, then
// gemm_pw_*.wgsl), so the depthwise output makes a round trip through memory
// -- for a 256-channel fp32 tensor that is 1 KB written and read again per
// pixel, more than the pointwise conv's own input, output and residual. Here
// one launch computes
//
//   y = act_p( W_p . act_d( dw_K(x) + b_d ) + b_p ) (+ res)
//
// with the depthwise result rounded nowhere (fp32 throughout), in the
// reference's arithmetic order per stage: the depthwise sum starts at the
// bias and adds the taps in (ky, kx) order (reference/conv.rs:131-140,
// crates/ai-cpu/src/kernels/dw.rs:40-204), the pointwise sum is the MFMA's,
// the epilogue act(acc + bias) + res (common/epilogue.rs:13-30).
//
// Decomposition (MI355X): a workgroup owns an output tile of wy * NB rows x
// wx * 16 columns of one image (NB = 4 or 2 rows per wavefront, up to 8
// wavefronts) and walks the depthwise channels in chunks of 16. Per chunk
// the tile's input halo (the chunk's 64 bytes of every pixel)
// and the chunk's weights are copied global -> LDS by LDS-direct buffer loads
// (no registers; zeros outside the image from the range check) into one of
// two buffers, the next chunk's copy overlapping the current chunk's compute,
// one workgroup barrier per chunk (three or four buffers, more chunks in
// flight, measured 1.4-1.9x slower: their LDS costs resident workgroups).
// A wavefront owns a vertical strip of NB 16-pixel row blocks; lane l
// computes the depthwise result of pixel l % 16 of each block for the four
// channels of 16-byte unit l / 16, reading every
// halo row once for the up to K blocks that use it (row reuse), and that
// result is directly the B operand of v_mfma_f32_16x16x4f32 (K index l / 16
// of the MFMA step j = channel 4 (l / 16) + j of the chunk); the pointwise
// weights of the chunk are the A operand (packed layout, pack.rs:68-102: the
// four K of one output channel are one 16-byte group). Accumulators stay in
// registers over all chunks; the epilogue adds the bias, applies the
// activation and the residual and stores 16 bytes per lane.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <map>
#include <mutex>
#include <string>
#include <tuple>

#include "capi_util.h"
#include "dw_pw.h"

namespace aih {
namespace {

typedef __attribute__((address_space(3))) void dp_lds_void;
constexpr uint32_t kOob = 0x80000000u;  // a byte offset past every buffer the kernel reads (< 2 GiB)

__device__ __forceinline__ __amdgpu_buffer_rsrc_t dp_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, (int)bytes, 0x00020000);
}

// One 16-byte LDS-direct load per lane: lane i's bytes land at dst + 16 i.
__device__ __forceinline__ void dp_load16(__amdgpu_buffer_rsrc_t rs, char *dst, uint32_t off, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (dp_lds_void *)dst, 16, off, (int)soff, 0, 0);
}

// K: depthwise kernel size; S: stride; NO: blocks of 16 output channels;
// U: 16-byte units (4 fp32 channels) per chunk and halo pixel; NB: output
// rows (16-pixel row blocks) per wavefront, 4 or 2; CL: both activations are
// clamp-type (one v_med3 each, no mode switch).
template <int K, int S, int NO, int U, int NB, bool CL>
__global__ __launch_bounds__(512) void dw_pw_kernel(DwPwArgs a) {
  constexpr uint32_t ES = 4, EC = 4 * U, COP = 16 * NO, PITCH = (U + 1) * 16;
  constexpr int HR = (NB - 1) * S + K;  // halo rows one wavefront reads
  constexpr int XS = dwpw_slots(S);
  constexpr uint32_t NWD = K * K * U, NWP = U * COP;  // weight slots of a chunk
  extern __shared__ __align__(16) char lds[];
  const uint32_t tid = threadIdx.x, lane = tid & 63, p16 = lane & 15, kq = lane >> 4;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t nthr = blockDim.x, nwaves = nthr >> 6;
  const uint32_t wxi = wave % a.wx, wyi = wave / a.wx;

  // ---- this workgroup's tile ----
  const uint32_t T = xcd_remap(blockIdx.x, gridDim.x, a.nxcd);
  const uint32_t img = fdiv(T, a.fd_pi);
  const uint32_t trem = T - img * a.per_img;
  const uint32_t tyi = fdiv(trem, a.fd_tx);
  const uint32_t ty0 = tyi * a.TH, tx0 = (trem - tyi * a.tiles_x) * a.TW;
  const int32_t iy0 = (int32_t)(ty0 * S) - a.PT, ix0 = (int32_t)(tx0 * S) - a.PL;

  // ---- this thread's halo slots (the same for every chunk) ----
  // slot s = 64 (wave + nwaves k) + lane holds unit s % (U + 1) of halo
  // pixel s / (U + 1) (unit U: the pad; slots past the halo pad the region
  // to whole rows of 64); gsl[k]: the unit's byte offset in the image for
  // channel 0 of a chunk (the chunk's channel offset goes in the scalar
  // offset) plus the unit index (the offset is a multiple of 16), or kOob
  // (outside the image, the pad, past the halo)
  const uint32_t nrows = (a.xrows + nwaves - 1 - wave) / nwaves;  // uniform: 64-slot rows this wavefront copies
  uint32_t gsl[XS];
#pragma unroll
  for (int k = 0; k < XS; ++k) {
    const uint32_t s = 64 * (wave + nwaves * k) + lane;
    const uint32_t P = s / (U + 1), u = s - P * (U + 1);
    const uint32_t hr = fdiv(P, a.fd_hw), hc = P - hr * a.HW;
    uint32_t hx = hc;
    if constexpr (S == 2) hx = hc < a.HWE ? 2 * hc : 2 * (hc - a.HWE) + 1;
    const uint32_t iy = (uint32_t)(iy0 + (int32_t)hr), ix = (uint32_t)(ix0 + (int32_t)hx);
    gsl[k] = (u < U && hr < a.HH && iy < a.IH && ix < a.IW) ? (iy * a.IW + ix) * a.C * ES + 16 * u + u : kOob;
  }

  // the weight copies go out in 64-slot rows, row r from wavefront
  // (first + r) % nwaves: this wavefront's first row
  auto first_row = [&](uint32_t first) { return (wave + nwaves - first % nwaves) % nwaves; };

  // chunk c (channels [EC c, EC c + EC)) -> LDS buffer b
  auto stage = [&](uint32_t c, uint32_t b) {
    char *B = lds + b * a.buf_bytes;
    const uint32_t c0 = c * EC, soff = c0 * ES;
    const __amdgpu_buffer_rsrc_t rs_x = dp_rsrc((const char *)a.x + (size_t)img * a.img_bytes, a.img_bytes);
    if (c0 + EC <= a.C) {
#pragma unroll
      for (int k = 0; k < XS; ++k) {
        if ((uint32_t)k >= nrows) break;
        dp_load16(rs_x, B + 1024 * (wave + nwaves * k), gsl[k] & ~15u, soff);
      }
    } else {
      // the last chunk of a C that is no multiple of EC: units past C read zeros
#pragma unroll
      for (int k = 0; k < XS; ++k) {
        if ((uint32_t)k >= nrows) break;
        const uint32_t g = gsl[k];
        dp_load16(rs_x, B + 1024 * (wave + nwaves * k), c0 + 4 * (g & 15u) < a.C ? g & ~15u : kOob, soff);
      }
    }
    // depthwise weights [tap][U units], its bias [U units], pointwise weights [U groups][COP rows]
    char *W = B + a.off_wd;
    const __amdgpu_buffer_rsrc_t rs_wd = dp_rsrc(a.wd, K * K * a.C * ES);
    for (uint32_t s0 = 64 * first_row(1); s0 < NWD; s0 += nthr) {
      const uint32_t s = s0 + lane;
      if (s < NWD) {
        const uint32_t t = s / U, u = s % U;
        dp_load16(rs_wd, W + s0 * 16, c0 + 4 * u < a.C ? (t * a.C + 4 * u) * ES : kOob, soff);
      }
    }
    if (wave == 0 && lane < U) {
      const __amdgpu_buffer_rsrc_t rs_bd = dp_rsrc(a.bd, a.C * ES);
      dp_load16(rs_bd, W + NWD * 16, c0 + 4 * lane < a.C ? 16 * lane : kOob, soff);
    }
    const __amdgpu_buffer_rsrc_t rs_wp = dp_rsrc(a.wp, a.KGP * a.CO4 * 4 * ES);
    for (uint32_t s0 = 64 * first_row(2); s0 < NWP; s0 += nthr) {
      const uint32_t s = s0 + lane;
      if (s < NWP) {
        const uint32_t g = s / COP, o = s % COP;
        const bool ok = o < a.CO4 && c0 + 4 * g < a.C;
        dp_load16(rs_wp, W + (NWD + U + s0) * 16, ok ? (g * a.CO4 + o) * 16 : kOob, c0 * a.CO4 * ES);
      }
    }
  };

  // LDS byte offset of this lane's halo pixel for tap (0, 0) of its first
  // block, unit kq (stride 2: halo columns stored even first)
  const uint32_t xbase = ((wyi * NB * S) * a.HW + 16 * wxi + p16) * PITCH + kq * 16;

  f32x4 acc[NB][NO];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int o = 0; o < NO; ++o) acc[b][o] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  const Act actd = act_params(a.act_d), actp = act_params(a.act_p);

  // chunk c lives in buffer c % 2; chunk c + 1 goes out once every
  // wavefront is done with chunk c - 1 (the barrier), into that buffer
  const uint32_t nch = a.nchunks;
  stage(0, 0);
  for (uint32_t c = 0; c < nch; ++c) {
    // this wavefront's copies of chunk c have landed, then the barrier
    // publishes every wavefront's
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0); expcnt, lgkmcnt untouched
    __syncthreads();
    if (c + 1 < nch) stage(c + 1, (c + 1) & 1);
    const uint32_t cur = c & 1;
    const char *B = lds + cur * a.buf_bytes;
    const char *W = B + a.off_wd;
    // lane group kq takes unit kq of the chunk (and kq + 4, ... for U > 4)
#pragma unroll
    for (int h = 0; h < U / 4; ++h) {
      const uint32_t u = 4 * h + kq;
      f32x4 w[K * K];
#pragma unroll
      for (int t = 0; t < K * K; ++t) w[t] = *reinterpret_cast<const f32x4 *>(W + (t * U + u) * 16);
      const f32x4 bias = *reinterpret_cast<const f32x4 *>(W + (NWD + u) * 16);
      f32x4 d[NB];
#pragma unroll
      for (int b = 0; b < NB; ++b) d[b] = bias;
      // halo row i feeds block b with kernel row i - S b
#pragma unroll
      for (int i = 0; i < HR; ++i) {
#pragma unroll
        for (int kx = 0; kx < K; ++kx) {
          const uint32_t col = S == 1 ? (uint32_t)kx : (uint32_t)(kx & 1) * a.HWE + (uint32_t)(kx >> 1);
          const f32x4 xv = *reinterpret_cast<const f32x4 *>(B + xbase + h * 64 + (i * a.HW + col) * PITCH);
#pragma unroll
          for (int b = 0; b < NB; ++b) {
            const int ky = i - S * b;
            if (ky >= 0 && ky < K) d[b] += xv * w[ky * K + kx];
          }
        }
      }
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        if constexpr (CL) {
#pragma unroll
          for (int j = 0; j < 4; ++j) d[b][j] = act_clamp_any(actd, d[b][j]);
        } else {
          d[b] = act4(actd, d[b]);
        }
      }
      f32x4 aw[NO];
#pragma unroll
      for (int o = 0; o < NO; ++o)
        aw[o] = *reinterpret_cast<const f32x4 *>(W + (NWD + U + u * COP + 16 * o + p16) * 16);
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
          for (int o = 0; o < NO; ++o)
            acc[b][o] = __builtin_amdgcn_mfma_f32_16x16x4f32(aw[o][j], d[b][j], acc[b][o], 0, 0, 0);
    }
  }

  // ---- epilogue: lane holds output channels 16 o + 4 kq .. + 3 of pixel p16 of each block ----
  f32x4 bp[NO];
#pragma unroll
  for (int o = 0; o < NO; ++o) {
    const uint32_t ch = 16 * o + 4 * kq;
    bp[o] = ch < a.CO4 ? Vec4IO<DT_F32>::load(a.bp, ch / 4) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }
  const uint32_t ox = tx0 + 16 * wxi + p16;
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const uint32_t oy = ty0 + wyi * NB + b;
    if (oy >= a.OH || ox >= a.OW) continue;
    const size_t pix = ((size_t)img * a.OH + oy) * a.OW + ox;
#pragma unroll
    for (int o = 0; o < NO; ++o) {
      const uint32_t ch = 16 * o + 4 * kq;
      if (ch >= a.CO4) continue;
      f32x4 v = acc[b][o] + bp[o];
      if constexpr (CL) {
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = act_clamp_any(actp, v[j]);
      } else {
        v = act4(actp, v);
      }
      const size_t vi = pix * (a.CO4 / 4) + ch / 4;
      if (a.has_res) v += Vec4IO<DT_F32>::load(a.res, vi);
      Vec4IO<DT_F32>::store(a.y, vi, v);
    }
  }
}

template <int K, int S, int NO, int NB, bool CL>
hipError_t prepare_inst() {
  static const hipError_t e =
      hipFuncSetAttribute(reinterpret_cast<const void *>(dw_pw_kernel<K, S, NO, kDpUnits, NB, CL>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
  return e;
}

template <int K, int S, int NO, int NB, bool CL>
hipError_t launch_inst(const DwPwArgs &a, uint32_t waves, uint32_t lds, uint32_t grid, hipStream_t st) {
  const hipError_t e = prepare_inst<K, S, NO, NB, CL>();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((dw_pw_kernel<K, S, NO, kDpUnits, NB, CL>), dim3(grid), dim3(64 * waves), lds, st, a);
  return hipGetLastError();
}

template <int K, int S, int NO, int NB, bool CL>
int occ_inst(uint32_t waves, uint32_t lds) {
  if (prepare_inst<K, S, NO, NB, CL>() != hipSuccess) return -1;
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, dw_pw_kernel<K, S, NO, kDpUnits, NB, CL>,
                                                   (int)(64 * waves), lds) != hipSuccess)
    return -1;
  return per_cu;
}

#define AIH_DP_SHAPES(X) \
  X(3, 1, 1) X(3, 1, 2) X(3, 1, 3) X(3, 1, 4) X(3, 2, 1) X(3, 2, 2) X(3, 2, 3) X(3, 2, 4)

}  // namespace

hipError_t launch_dw_pw(const DwPwArgs &a, int dt, uint32_t k, uint32_t s, uint32_t rows, uint32_t waves,
                        uint32_t lds, uint32_t grid, hipStream_t st) {
  if (dt != DT_F32) return hipErrorInvalidValue;
  const uint32_t no = dwpw_no(a.CO4);
  const bool cl = act_is_clamp(a.act_d) && act_is_clamp(a.act_p);
#define AIH_DP_LAUNCH(K_, S_, NO_)                                                                  \
  if (k == K_ && s == S_ && no == NO_) {                                                            \
    if (rows == 2)                                                                                  \
      return cl ? launch_inst<K_, S_, NO_, 2, true>(a, waves, lds, grid, st)                        \
                : launch_inst<K_, S_, NO_, 2, false>(a, waves, lds, grid, st);                      \
    if (rows == 4)                                                                                  \
      return cl ? launch_inst<K_, S_, NO_, 4, true>(a, waves, lds, grid, st)                        \
                : launch_inst<K_, S_, NO_, 4, false>(a, waves, lds, grid, st);                      \
  }
  AIH_DP_SHAPES(AIH_DP_LAUNCH)
#undef AIH_DP_LAUNCH
  return hipErrorInvalidValue;
}

// Workgroups per CU of an instantiation at a workgroup size and LDS size,
// queried once per device; 0 for a shape without an instantiation.
int dw_pw_occupancy(int dt, uint32_t k, uint32_t s, uint32_t cout, uint32_t rows, bool cl, uint32_t waves,
                    uint32_t lds) {
  if (dt != DT_F32 || (rows != 2 && rows != 4)) return 0;
  const uint32_t no = dwpw_no(cout);
  static std::mutex mu;
  static std::map<std::tuple<uint32_t, uint32_t, uint32_t, uint32_t, bool, uint32_t, uint32_t, int>, int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = -1;
  std::lock_guard<std::mutex> lock(mu);
  const auto key = std::make_tuple(k, s, no, rows, cl, waves, lds, dev);
  auto it = cache.find(key);
  if (it != cache.end()) return it->second;
  int occ = -2;
#define AIH_DP_OCC(K_, S_, NO_)                                                                           \
  if (k == K_ && s == S_ && no == NO_)                                                                      \
    occ = rows == 2 ? (cl ? occ_inst<K_, S_, NO_, 2, true>(waves, lds) : occ_inst<K_, S_, NO_, 2, false>(waves, lds)) \
                    : (cl ? occ_inst<K_, S_, NO_, 4, true>(waves, lds) : occ_inst<K_, S_, NO_, 4, false>(waves, lds));
  AIH_DP_SHAPES(AIH_DP_OCC)
#undef AIH_DP_OCC
  if (occ == -2) return 0;  // no instantiation
  // a failed query (no device to ask): plan for one workgroup per CU, and
  // ask again next time; a real answer, 0 included, is kept
  if (occ < 0) return 1;
  cache[key] = occ;
  return occ;
}

}  // namespace aih

// ---------------------------------------------------------------- the C ABI

namespace {

using aih::DwPwPlan;

int dp_fail(const std::string &m) { return aih::api_fail(m); }

// Output size of the depthwise conv, or false when the descriptor cannot run fused.
bool dp_check(const aih_dwpw_desc *d, uint32_t *oh, uint32_t *ow) {
  if (!d) return dp_fail("dwpw: null descriptor"), false;
  if (d->dt != AIH_F32) return dp_fail("dwpw: only fp32 storage (dt = AIH_F32)"), false;
  if (d->n == 0 || d->ih == 0 || d->iw == 0 || d->c == 0) return dp_fail("dwpw: empty input"), false;
  if (d->k != 3) return dp_fail("dwpw: the depthwise kernel must be 3x3"), false;
  if (d->s != 1 && d->s != 2) return dp_fail("dwpw: stride must be 1 or 2"), false;
  if (!aih::dwpw_has_cout(d->cout)) return dp_fail("dwpw: cout must be 1..64"), false;
  if (d->kg_pad < (d->c + 3) / 4) return dp_fail("dwpw: kg_pad below ceil(c / 4)"), false;
  for (int i = 0; i < 4; ++i)
    if (d->pad[i] >= d->k) return dp_fail("dwpw: padding must be below the kernel size"), false;
  const uint32_t eh = d->ih + d->pad[0] + d->pad[2], ew = d->iw + d->pad[1] + d->pad[3];
  if (eh < d->k || ew < d->k) return dp_fail("dwpw: input smaller than the kernel"), false;
  *oh = (eh - d->k) / d->s + 1;
  *ow = (ew - d->k) / d->s + 1;
  const uint64_t c4 = (d->c + 3) / 4 * 4, co4 = (d->cout + 3) / 4 * 4;
  if ((uint64_t)d->ih * d->iw * c4 * 4 >= (1ull << 31)) return dp_fail("dwpw: an input image must stay below 2 GiB"), false;
  if ((uint64_t)d->kg_pad * co4 * 16 >= (1ull << 31) || 9 * c4 * 4 >= (1ull << 31))
    return dp_fail("dwpw: weights too large"), false;
  return true;
}

// Tile shape (wy x wx wavefronts, each nb = 4 or 2 output rows x 16
// columns): forced by tile_h / tile_w (and wave_rows), else, among the shapes
// whose tiles give every CU one (or, when none does, the most tiles), the one
// keeping the most wavefronts resident per CU (workgroups resident x
// wavefronts, up to 16, or fewer when the launch has fewer tiles: the MFMA
// and depthwise phases of one wavefront and the copies of another overlap),
// then the fewest wavefronts per workgroup (a shorter barrier), the least
// halo copied over all tiles, four rows per wavefront. Measured at batch 64
// (us): 256 -> 64 at 40x72, 8x16 with 2 rows 109, 16x16 with 2 rows (8
// wavefronts) 119, 16x16 with 4 rows 132; 44 -> 24 at 80x144 56 / 65 / 74.
// Two LDS chunk buffers.
bool dp_plan(const aih_dwpw_desc *d, uint32_t oh, uint32_t ow, DwPwPlan *out) {
  // {wx, wy, nb}: 1-8 wavefronts, at most 64 columns and 16 rows
  static const uint32_t shapes[][3] = {{1, 1, 4}, {2, 1, 4}, {1, 2, 4}, {4, 1, 4}, {2, 2, 4}, {1, 4, 4},
                                       {1, 2, 2}, {2, 2, 2}, {1, 4, 2}, {4, 2, 2}, {2, 4, 2}, {1, 8, 2}};
  const uint32_t cus = aih::device_cus();
  bool found = false;
  uint64_t best_halo = 0;
  double best_eff = 0.0;
  for (const auto &sh : shapes) {
    DwPwPlan p{};
    p.wx = sh[0];
    p.wy = sh[1];
    p.nb = sh[2];
    if ((d->tile_h || d->tile_w) && (d->tile_h != p.wy * p.nb || d->tile_w != p.wx * 16)) continue;
    if (d->wave_rows && d->wave_rows != p.nb) continue;
    const uint32_t waves = p.wx * p.wy;
    p.TH = p.wy * p.nb;
    p.TW = p.wx * 16;
    p.HH = (p.TH - 1) * d->s + d->k;
    p.HW = (p.TW - 1) * d->s + d->k;
    p.HWE = d->s == 2 ? (p.HW + 1) / 2 : 0;
    p.xrows = aih::dwpw_xrows(p.HH, p.HW);
    if (p.xrows > waves * aih::dwpw_slots(d->s)) continue;
    p.buf_bytes = aih::dwpw_buf_bytes(d->k, d->s, p.HH, p.HW, d->cout);
    p.lds = 2 * p.buf_bytes;
    if (p.lds > 160u * 1024u) continue;
    p.occ = (uint32_t)aih::dw_pw_occupancy(d->dt, d->k, d->s, d->cout, p.nb,
                                           aih::act_is_clamp(d->act_dw) && aih::act_is_clamp(d->act_pw), waves, p.lds);
    if (p.occ == 0) continue;
    p.tiles_x = (ow + p.TW - 1) / p.TW;
    p.tiles_y = (oh + p.TH - 1) / p.TH;
    const uint64_t nt = (uint64_t)d->n * p.tiles_x * p.tiles_y;
    if (nt >= (1ull << 31)) continue;
    p.ntiles = (uint32_t)nt;
    p.grid = p.ntiles;
    const uint64_t halo = nt * p.HH * p.HW;
    const double eff = std::min({(double)(waves * p.occ), 16.0, (double)nt * waves / cus});
    bool better = !found;
    if (found) {
      const bool fills = p.ntiles >= cus, best_fills = out->ntiles >= cus;
      const uint32_t best_waves = out->wx * out->wy;
      if (fills != best_fills)
        better = fills;
      else if (!fills && p.ntiles != out->ntiles)
        better = p.ntiles > out->ntiles;
      else if (std::fabs(eff - best_eff) > 1e-9)
        better = eff > best_eff;
      else if (waves != best_waves)
        better = waves < best_waves;
      else if (halo != best_halo)
        better = halo < best_halo;
      else
        better = p.nb > out->nb;
    }
    if (better) {
      *out = p;
      best_halo = halo;
      best_eff = eff;
      found = true;
    }
  }
  if (!found) {
    dp_fail(d->tile_h || d->tile_w || d->wave_rows
                ? "dwpw: the forced tile / wave rows are no shape of 1-8 wavefronts of 2 or 4 rows x 16 columns that fits"
                : "dwpw: no tile fits");
    return false;
  }
  return true;
}

bool dp_aligned(const void *p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

}  // namespace

extern "C" {

int aih_conv_dwpw_plan(const aih_dwpw_desc *d, aih_dwpw_plan *out) {
  return aih::api_guarded([&] {
    uint32_t oh, ow;
    if (!dp_check(d, &oh, &ow)) return AIH_ERR;
    if (!out) return dp_fail("dwpw: null plan");
    DwPwPlan p;
    if (!dp_plan(d, oh, ow, &p)) return AIH_ERR;
    const uint32_t ec = 4 * aih::kDpUnits;
    *out = aih_dwpw_plan{p.TH, p.TW, p.wx * p.wy, p.nb, (d->c + ec - 1) / ec, p.ntiles, p.lds, p.occ, p.grid};
    return AIH_OK;
  });
}

int aih_conv_dwpw(const aih_dwpw_desc *d, const void *x, const void *w_dw, const void *b_dw, const void *w_pw,
                  const void *b_pw, const void *res, void *y, aih_stream stream) {
  return aih::api_guarded([&] {
    uint32_t oh, ow;
    if (!dp_check(d, &oh, &ow)) return AIH_ERR;
    if (!x || !w_dw || !b_dw || !w_pw || !b_pw || !y) return dp_fail("dwpw: null buffer");
    if ((d->residual != 0) != (res != nullptr)) return dp_fail("dwpw: res must be given iff residual");
    for (const void *p : {x, w_dw, b_dw, w_pw, b_pw, (const void *)y})
      if (!dp_aligned(p, 16)) return dp_fail("dwpw: misaligned buffer (16 bytes)");
    if (res && !dp_aligned(res, 16)) return dp_fail("dwpw: misaligned residual (16 bytes)");
    DwPwPlan p;
    if (!dp_plan(d, oh, ow, &p)) return AIH_ERR;
    aih::DwPwArgs a{};
    a.x = x;
    a.wd = w_dw;
    a.bd = b_dw;
    a.wp = w_pw;
    a.bp = b_pw;
    a.res = res;
    a.y = y;
    a.IH = d->ih;
    a.IW = d->iw;
    a.C = (d->c + 3) / 4 * 4;
    a.OH = oh;
    a.OW = ow;
    a.CO4 = (d->cout + 3) / 4 * 4;
    a.KGP = d->kg_pad;
    a.img_bytes = d->ih * d->iw * a.C * 4;
    a.PT = (int32_t)d->pad[0];
    a.PL = (int32_t)d->pad[1];
    a.TH = p.TH;
    a.TW = p.TW;
    a.wx = p.wx;
    a.HH = p.HH;
    a.HW = p.HW;
    a.HWE = p.HWE;
    a.tiles_x = p.tiles_x;
    a.per_img = p.tiles_x * p.tiles_y;
    a.ntiles = p.ntiles;
    a.fd_pi = aih::make_fastdiv(a.per_img);
    a.fd_tx = aih::make_fastdiv(p.tiles_x);
    a.fd_hw = aih::make_fastdiv(p.HW);
    a.nchunks = (a.C + 4 * aih::kDpUnits - 1) / (4 * aih::kDpUnits);
    a.xrows = p.xrows;
    a.buf_bytes = p.buf_bytes;
    a.off_wd = p.xrows * 1024;
    a.act_d = d->act_dw;
    a.act_p = d->act_pw;
    a.has_res = d->residual ? 1 : 0;
    a.nxcd = aih::device_xcds();
    const hipError_t e = aih::launch_dw_pw(a, d->dt, d->k, d->s, p.nb, p.wx * p.wy, p.lds, p.grid,
                                           static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return dp_fail(std::string("dwpw launch: ") + hipGetErrorString(e));
    return AIH_OK;
  });
}

}  // extern "C"

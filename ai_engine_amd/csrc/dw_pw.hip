// dw_pw.hip -- fused depthwise KxK conv + pointwise 1x1 conv, fp32 and
// 16-bit storage (the kernel: dw_pw_impl.h; its 16-bit instantiations:
// dw_pw_f16.hip, dw_pw_bf16.hip).
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
// with the depthwise result rounded nowhere at fp32, and rounded to the
// storage dtype at 16 bit exactly where the unfused depthwise stores its
// output, in the reference's arithmetic order per stage: the depthwise sum starts at the
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
//
// 16-bit storage: a 16-byte unit is 8 channels, a chunk 32. Lane l's
// depthwise result (fp32 from the widened taps, rounded to the dtype after
// the activation) for the 8 channels of unit l / 16 is the B operand of one
// v_mfma_f32_16x16x32_{f16,bf16} (K slice l / 16), the projection weights of
// those channels -- packed K groups 2 (l / 16) and 2 (l / 16) + 1 -- the A
// operand; same tiles, LDS bytes and epilogue.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <map>
#include <mutex>
#include <string>
#include <tuple>

#include "capi_util.h"
#include "dw_pw_impl.h"

namespace aih {

hipError_t launch_dw_pw(const DwPwArgs &a, int dt, uint32_t k, uint32_t s, uint32_t rows, uint32_t waves,
                        uint32_t lds, uint32_t grid, hipStream_t st) {
  switch (dt) {
    case DT_F32: return dp_launch_dt<DT_F32>(a, k, s, rows, waves, lds, grid, st);
    case DT_F16: return launch_dw_pw_f16(a, k, s, rows, waves, lds, grid, st);
    case DT_BF16: return launch_dw_pw_bf16(a, k, s, rows, waves, lds, grid, st);
    default: return hipErrorInvalidValue;
  }
}

// Workgroups per CU of an instantiation at a workgroup size and LDS size,
// queried once per device; 0 for a shape without an instantiation.
int dw_pw_occupancy(int dt, uint32_t k, uint32_t s, uint32_t cout, uint32_t rows, bool cl, uint32_t waves,
                    uint32_t lds) {
  if ((dt != DT_F32 && dt != DT_F16 && dt != DT_BF16) || (rows != 2 && rows != 4)) return 0;
  const uint32_t no = dwpw_no(cout);
  static std::mutex mu;
  static std::map<std::tuple<int, uint32_t, uint32_t, uint32_t, uint32_t, bool, uint32_t, uint32_t, int>, int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = -1;
  std::lock_guard<std::mutex> lock(mu);
  const auto key = std::make_tuple(dt, k, s, no, rows, cl, waves, lds, dev);
  auto it = cache.find(key);
  if (it != cache.end()) return it->second;
  const int occ = dt == DT_F32   ? dp_occ_dt<DT_F32>(k, s, no, rows, cl, waves, lds)
                  : dt == DT_F16 ? dw_pw_occ_f16(k, s, no, rows, cl, waves, lds)
                                 : dw_pw_occ_bf16(k, s, no, rows, cl, waves, lds);
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
  if (d->dt != AIH_F32 && d->dt != AIH_F16 && d->dt != AIH_BF16) return dp_fail("dwpw: unknown dtype"), false;
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
// and depthwise phases of one wavefront and the copies of another overlap)
// times the share of the tiles' pixels inside the output (at 20x36, 16x16
// tiles compute 1536 pixels for 720: 9.4 us against 7.7 for 4x16 tiles),
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
    // resident wavefronts, scaled by the share of the tiles' pixels inside
    // the output (tiles overhanging a small image compute for nothing)
    const double used = (double)oh * ow / ((double)p.tiles_y * p.TH * p.tiles_x * p.TW);
    const double eff = std::min({(double)(waves * p.occ), 16.0, (double)nt * waves / cus}) * used;
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
    const uint32_t ec = (d->dt == AIH_F32 ? 4 : 8) * aih::kDpUnits;
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
    const uint32_t es = d->dt == AIH_F32 ? 4 : 2;
    a.img_bytes = d->ih * d->iw * a.C * es;
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
    const uint32_t ec = (16 / es) * aih::kDpUnits;
    a.nchunks = (a.C + ec - 1) / ec;
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

// ir_block.hip -- host side of the fused inverted-residual block: tile and
// chunk planning, LDS layout, and dispatch to the per-dtype instantiations.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <map>
#include <mutex>
#include <tuple>

#include "aih_device.h"
#include "ir_block_impl.h"

namespace aih {

namespace {

uint32_t cdiv(uint32_t a, uint32_t b) { return (a + b - 1) / b; }
uint32_t align16(uint32_t v) { return (v + 15u) & ~15u; }

// Workgroups per CU allowed by registers alone, per instantiation (queried once).
int reg_occupancy(int dt, uint32_t nob, uint32_t npw, bool cl) {
  static std::mutex mu;
  static std::map<std::tuple<int, uint32_t, uint32_t, bool>, int> cache;
  std::lock_guard<std::mutex> lock(mu);
  const auto key = std::make_tuple(dt, nob, npw, cl);
  auto it = cache.find(key);
  if (it != cache.end()) return it->second;
  int occ = 0;
  switch (dt) {
    case DT_F32: occ = ir_occ_f32(nob, npw, cl, 0); break;
    case DT_F16: occ = ir_occ_f16(nob, npw, cl, 0); break;
    case DT_BF16: occ = ir_occ_bf16(nob, npw, cl, 0); break;
    default: break;
  }
  // A failed query (no device to ask): plan for one workgroup per CU, and
  // ask again next time; a real answer, 0 included, is kept (the planner
  // then skips the shape).
  if (occ < 0) return 1;
  cache[key] = occ;
  return occ;
}

// LDS regions of the kernel: input tile, the expanded chunk, and WR/32 weight
// slots, each holding one 32-channel chunk's expand, project (rows of COP
// channels) and depthwise weights and biases in their packed layouts (all of
// E when the weights are resident, else two slots), and the fp32 projection
// bias.
void lds_layout(uint32_t C, uint32_t COP, uint32_t CO, uint32_t WR, uint32_t NPI, int dt, IrPlan *p) {
  const uint32_t es = dt == DT_F32 ? 4 : 2;
  const uint32_t rpx = C * es + 16, rpe = IR_EC * es + 16;
  uint32_t off = 0;
  p->lds_x = off;
  off = align16(off + NPI * 32 * rpx);
  p->lds_xe = off;
  off = align16(off + NPI * 32 * rpe);
  p->lds_we = off;
  off = align16(off + WR * C * es);
  p->lds_wp = off;
  off = align16(off + WR * COP * es);
  p->lds_sm = off;
  off = align16(off + WR * 11 * es);
  p->lds_bp = off;
  off = align16(off + CO * 4);
  p->lds = off;
}

constexpr uint32_t kMaxLds = 160 * 1024;

}  // namespace

// Geometry search. For every candidate output tile TH x TW (32 to 256 pixels,
// at most 8 32-pixel blocks so a wavefront owns at most two) and chunk EC
// dividing E, a per-CU cost in cycles is estimated from the three resources a
// tile uses -- MFMA (expand over the halo tile, project over the output
// tile), VALU (the depthwise taps) and LDS bandwidth -- and multiplied by the
// number of tile rounds the grid needs. The cheapest candidate that fits in
// LDS wins; candidates with a single workgroup per CU pay a latency penalty.
const char *ir_plan(uint32_t N, uint32_t IH, uint32_t IW, uint32_t OH, uint32_t OW, uint32_t C, uint32_t E,
                    uint32_t CO, uint32_t S, int dt, bool cl, uint32_t tile_h, uint32_t tile_w, uint32_t ec_force,
                    int32_t weights, IrPlan *out) {
  if (dt != DT_F32 && dt != DT_F16 && dt != DT_BF16) return "unknown dtype";
  const bool f32 = dt == DT_F32;
  const uint32_t kstep = f32 ? 8 : 16;
  if (C == 0 || E == 0 || CO == 0 || N == 0 || OH == 0 || OW == 0) return "zero-sized block";
  if (C % kstep) return f32 ? "expand input channels must be a multiple of 8" : "expand input channels must be a multiple of 16";
  if (C > 128) return "expand input channels must be at most 128";
  if (E % 32) return "expanded channels must be a multiple of 32";
  if (CO % 16 || CO > 128) return "project output channels must be a multiple of 16 and at most 128";
  if (S != 1 && S != 2) return "depthwise stride must be 1 or 2";
  if (ec_force && ec_force != IR_EC) return "the kernel walks E in chunks of 32 channels";
  if ((tile_h && tile_h > OH) || (tile_w && tile_w > OW)) return "forced tile larger than the output";
  if (tile_h && tile_w && (tile_h * tile_w > 256)) return "forced tile above 256 pixels";
  if (weights != AIH_IR_WEIGHTS_AUTO && weights != AIH_IR_WEIGHTS_RESIDENT && weights != AIH_IR_WEIGHTS_STREAMED)
    return "unknown weight placement";
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = -1;

  // the plan depends on the device (CU count, occupancy) and on the
  // instantiation (clamp-type activations use fewer registers)
  struct Key {
    uint32_t v[16];
    bool operator<(const Key &o) const { return std::memcmp(v, o.v, sizeof(v)) < 0; }
  };
  static std::mutex mu;
  static std::map<Key, IrPlan> cache;
  const Key key{{N, IH, IW, OH, OW, C, E, CO, S, (uint32_t)dt, tile_h, tile_w, ec_force, (uint32_t)cl,
                 (uint32_t)weights, (uint32_t)dev}};
  {
    std::lock_guard<std::mutex> lock(mu);
    auto it = cache.find(key);
    if (it != cache.end()) {
      *out = it->second;
      return nullptr;
    }
  }

  const int cus = (int)device_cus();
  const uint32_t COP = ir_cop(CO), nob = COP / 32;
  const uint32_t ec = IR_EC, chunks = E / IR_EC;
  // Per-wavefront cycle estimates: one 32-channel chunk of the depthwise +
  // projection for a 32-pixel block (VALU-bound: 9 FMAs per channel and ~50%
  // overhead), one MFMA, the expand epilogue of a block, the exposed latency
  // of a global round trip (hidden by co-resident workgroups) and a barrier.
  const double kst = f32 ? 4.0 : 2.0;  // projection K steps per chunk
  const double dw_chunk = kst * 4.0 * (f32 ? 60.0 : 110.0);
  const double mfma = f32 ? 4 * 64.0 : 32.0;
  const double latency = 2500.0, barrier = 250.0;

  bool found = false;
  double best = 0;
  IrPlan bp{};
  for (uint32_t resident = 0; resident < 2; ++resident) {
    if ((weights == AIH_IR_WEIGHTS_RESIDENT && !resident) || (weights == AIH_IR_WEIGHTS_STREAMED && resident)) continue;
    for (uint32_t tw = 4; tw <= 64; tw *= 2) {
      const uint32_t twx = tile_w ? tile_w : std::min(tw, OW);
      for (uint32_t th = 1; th <= 32; ++th) {
        const uint32_t thx = tile_h ? tile_h : std::min(th, OH);
        if (thx != th && !tile_h) continue;
        const uint32_t tpix = thx * twx;
        if ((tpix < 16 && !(tile_h && tile_w)) || tpix > 256) continue;
        const uint32_t npb = cdiv(tpix, 32);
        const uint32_t hh = (thx - 1) * S + 3, hw = (twx - 1) * S + 3;
        const uint32_t npi = cdiv(hh * hw, 32);
        IrPlan p{};
        p.TH = thx;
        p.TW = twx;
        p.HH = hh;
        p.HW = hw;
        p.NPI = npi;
        p.NPB = npb;
        p.EC = ec;
        p.resident = resident;
        lds_layout(C, COP, CO, resident ? E : 2 * ec, npi, dt, &p);
        if (p.lds > kMaxLds) continue;
        const uint32_t npw = cdiv(npb, 4);
        const int occ_r = reg_occupancy(dt, nob, npw, cl);
        const int occ = std::min<int>(occ_r, (int)(kMaxLds / p.lds));
        if (occ < 1) continue;
        p.tiles_y = cdiv(OH, thx);
        p.tiles_x = cdiv(OW, twx);
        const uint64_t nt = (uint64_t)N * p.tiles_y * p.tiles_x;
        if (nt > 0x7fffffffull) continue;
        p.ntiles = (uint32_t)nt;
        p.occ = (uint32_t)occ;
        const double exp_mfma = std::ceil(npi / 4.0) * ((double)C / kstep) * mfma;
        const double exp_valu = std::ceil(npi / 4.0) * 4.0 * 60.0;
        const double dw = npw * (dw_chunk + kst * nob * mfma * 0.25);
        const double per_chunk = std::max(exp_mfma, 0.0) + exp_valu + dw + barrier;
        const double tile = chunks * per_chunk + (latency * (resident ? 1.0 : 2.0)) / occ;
        // the kernel's phases are latency chains: co-resident workgroups on a
        // CU overlap them (measured: 3 workgroups per CU beat 1 by ~1.5x)
        const double overlap = occ >= 3 ? 0.75 : (occ == 2 ? 0.9 : 1.1);
        const double cost = std::ceil((double)p.ntiles / cus) * tile * overlap;
        if (!found || cost < best) {
          found = true;
          best = cost;
          bp = p;
        }
      }
    }
  }
  if (!found) return "no tile geometry fits in LDS";
  bp.grid = (uint32_t)std::min<uint64_t>(bp.ntiles, (uint64_t)cus * bp.occ);
  {
    std::lock_guard<std::mutex> lock(mu);
    cache[key] = bp;
  }
  *out = bp;
  return nullptr;
}

hipError_t launch_ir_block(const IrArgs &a, int dt, uint32_t lds, uint32_t grid, hipStream_t st) {
  switch (dt) {
    case DT_F32: return launch_ir_block_f32(a, lds, grid, st);
    case DT_F16: return launch_ir_block_f16(a, lds, grid, st);
    case DT_BF16: return launch_ir_block_bf16(a, lds, grid, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace aih

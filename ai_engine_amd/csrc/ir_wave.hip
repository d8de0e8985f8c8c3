// ir_wave.hip -- host side of the one-tile-per-wavefront fused block:
// tile choice, weight placement, LDS layout, dispatch per dtype.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <map>
#include <mutex>

#include "aih_device.h"
#include "ir_block.h"
#include "ir_wave_impl.h"

namespace aih {

namespace {

uint32_t cdiv(uint32_t a, uint32_t b) { return (a + b - 1) / b; }
uint32_t align16(uint32_t v) { return (v + 15u) & ~15u; }

int irw_occupancy(int dt, uint32_t ke, uint32_t npi, uint32_t nob, bool rl, uint32_t waves, uint32_t lds) {
  static std::mutex mu;
  static std::map<std::tuple<int, uint32_t, uint32_t, uint32_t, bool, uint32_t, uint32_t, int>, int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = -1;
  std::lock_guard<std::mutex> lock(mu);
  const auto key = std::make_tuple(dt, ke, npi, nob, rl, waves, lds, dev);
  auto it = cache.find(key);
  if (it != cache.end()) return it->second;
  int occ = dt == DT_F16 ? ir_wave_occ_f16(ke, npi, nob, rl, waves, lds)
                         : ir_wave_occ_bf16(ke, npi, nob, rl, waves, lds);
  // without a device the runtime cannot answer: plan for one workgroup per CU
  if (occ <= 0) occ = 1;
  cache[key] = occ;
  return occ;
}

// Output tiles of at most 32 pixels (one MFMA column block) the planner tries.
constexpr uint32_t kTiles[][2] = {{4, 8}, {8, 4}, {5, 6}, {6, 5}, {2, 16}, {16, 2}, {3, 10}, {10, 3},
                                  {4, 7}, {7, 4}, {1, 32}, {32, 1}};

}  // namespace

const char *irw_plan(uint32_t N, uint32_t IH, uint32_t IW, uint32_t OH, uint32_t OW, uint32_t C, uint32_t E,
                     uint32_t CO, uint32_t S, int dt, bool cl, bool rl, uint32_t tile_h, uint32_t tile_w,
                     int32_t weights, IrWavePlan *out) {
  if (dt != DT_F16 && dt != DT_BF16) return "the wave kernel takes f16 / bf16 storage";
  if (!cl) return "the wave kernel takes clamp-type activations (identity, ReLU, ReLU6, clamp01)";
  if (C % 16 || E % 32 || CO % 16 || C == 0 || E == 0 || CO == 0) return "cin % 16, cexp % 32 and cout % 16 needed";
  if (S != 1 && S != 2) return "depthwise stride must be 1 or 2";
  if (weights != AIH_IR_WEIGHTS_AUTO && weights != AIH_IR_WEIGHTS_RESIDENT && weights != AIH_IR_WEIGHTS_STREAMED)
    return "unknown weight placement";
  const uint32_t ke = C / 16, COP = ir_cop(CO), nob = COP / 32;
  if (!irw_has_shape(ke, 2, nob) && !irw_has_shape(ke, 5, nob)) return "no wave-kernel instantiation for this width";
  if ((tile_h && tile_h > OH) || (tile_w && tile_w > OW)) return "forced tile larger than the output";
  if (tile_h && tile_w && tile_h * tile_w > 32) return "the wave kernel's tiles hold at most 32 pixels";
  if ((uint64_t)IH * IW * C * 2 >= 0x80000000ull) return "image of 2 GiB or more";

  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = -1;
  struct Key {
    uint32_t v[15];
    bool operator<(const Key &o) const { return std::memcmp(v, o.v, sizeof(v)) < 0; }
  };
  static std::mutex mu;
  static std::map<Key, IrWavePlan> cache;
  const Key key{{N, IH, IW, OH, OW, C, E, CO, S, (uint32_t)dt, tile_h, tile_w, (uint32_t)weights, (uint32_t)dev,
                 rl ? 1u : 0u}};
  {
    std::lock_guard<std::mutex> lock(mu);
    auto it = cache.find(key);
    if (it != cache.end()) {
      *out = it->second;
      return nullptr;
    }
  }

  const uint32_t cus = device_cus();
  const uint32_t nchunks = E / 32, slot = irw_slot_bytes(C, COP);
  bool found = false;
  double best = 0;
  IrWavePlan bp{};
  auto consider = [&](uint32_t th, uint32_t tw) {
    if (th == 0 || tw == 0 || th * tw > 32) return;
    const uint32_t hh = (th - 1) * S + 3, hw = (tw - 1) * S + 3;
    uint32_t npi = 0;
    for (uint32_t n : {2u, 5u})
      if (hh * hw <= n * 32 && irw_has_shape(ke, n, nob)) {
        npi = n;
        break;
      }
    if (!npi) return;
    for (uint32_t waves : {8u, 4u, 2u})
      for (uint32_t resident = 0; resident < 2; ++resident) {
        if ((weights == AIH_IR_WEIGHTS_RESIDENT && !resident) || (weights == AIH_IR_WEIGHTS_STREAMED && resident))
          continue;
        IrWavePlan p{};
        p.TH = th;
        p.TW = tw;
        p.HH = hh;
        p.HW = hw;
        p.NPI = npi;
        p.resident = resident;
        p.waves = waves;
        p.lds_w = 0;
        p.lds_bp = align16((resident ? nchunks : 2u) * slot);
        p.lds_xe = align16(p.lds_bp + CO * 4);
        p.lds = p.lds_xe + waves * npi * 32 * IRW_RPE;
        if (p.lds > 160u * 1024u) continue;
        const int occ = irw_occupancy(dt, ke, npi, nob, rl, waves, p.lds);
        p.tiles_y = cdiv(OH, th);
        p.tiles_x = cdiv(OW, tw);
        const uint64_t nt = (uint64_t)N * p.tiles_y * p.tiles_x;
        if (nt > 0x7fffffffull) continue;
        p.ntiles = (uint32_t)nt;
        p.occ = (uint32_t)occ;
        p.grid = (uint32_t)std::min<uint64_t>(cdiv(p.ntiles, waves), (uint64_t)cus * p.occ);
        // per tile: expand (NPI blocks of KE + 1 MFMAs, their epilogue), the
        // depthwise of 32 pixels x 32 channels on the VALU, the projection;
        // streamed weights pay a barrier and a copy per chunk. A CU's four
        // SIMDs take its workgroups' tiles side by side: the launch lasts
        // ceil(tiles / (CUs used x 4)) tile times; total work breaks ties.
        const double per_tile = (npi * (ke + 1) * 32.0 + npi * 120.0 + 800.0 + nob * 64.0 +
                                 (resident ? 0.0 : 300.0)) * nchunks;
        const double used = std::min<double>(p.grid, cus) * 4.0;
        const double cost = (std::ceil((double)nt / used) + 1e-3 * (double)nt / (cus * 4.0)) * per_tile;
        if (!found || cost < best * 0.999) {
          found = true;
          best = cost;
          bp = p;
        }
      }
  };
  if (tile_h && tile_w) {
    consider(tile_h, tile_w);
  } else {
    // a tile larger than the output is cut down to it
    for (const auto &t : kTiles) {
      const uint32_t th = tile_h ? tile_h : std::min(t[0], OH), tw = tile_w ? tile_w : std::min(t[1], OW);
      consider(th, tw);
    }
  }
  if (!found) return "no wave-kernel tile fits";
  {
    std::lock_guard<std::mutex> lock(mu);
    cache[key] = bp;
  }
  *out = bp;
  return nullptr;
}

hipError_t launch_ir_wave(const IrWaveArgs &a, int dt, uint32_t npi, uint32_t waves, uint32_t lds, uint32_t grid,
                          hipStream_t st) {
  if (lds > 160u * 1024u || grid == 0 || (waves != 2 && waves != 4 && waves != 8)) return hipErrorInvalidValue;
  switch (dt) {
    case DT_F16: return launch_ir_wave_f16(a, npi, waves, lds, grid, st);
    case DT_BF16: return launch_ir_wave_bf16(a, npi, waves, lds, grid, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace aih

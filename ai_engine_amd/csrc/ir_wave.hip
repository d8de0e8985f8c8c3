// ir_wave.hip -- host side of the one-tile-per-wavefront fused block and of
// its split variant (one tile per workgroup): kernel, tile, weight placement
// and LDS layout choice, dispatch per dtype.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <cmath>
#include <map>
#include <mutex>
#include <tuple>

#include "aih_device.h"
#include "ir_block.h"
#include "ir_split_impl.h"

namespace aih {

namespace {

uint32_t cdiv(uint32_t a, uint32_t b) { return (a + b - 1) / b; }
uint32_t align16(uint32_t v) { return (v + 15u) & ~15u; }

// Workgroups per CU of an instantiation at a workgroup size and LDS size
// (queried once per device).
// split: 0 = wave kernel, 1 = split kernel, 2 = split kernel with the deep
// prefetch, 3 = the stem-fused wave kernel
int irw_occupancy(int split, int dt, uint32_t ke, uint32_t npi, uint32_t nob, bool rl, uint32_t waves,
                  uint32_t lds) {
  static std::mutex mu;
  static std::map<std::tuple<int, int, uint32_t, uint32_t, uint32_t, bool, uint32_t, uint32_t, int>, int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = -1;
  std::lock_guard<std::mutex> lock(mu);
  const auto key = std::make_tuple(split, dt, ke, npi, nob, rl, waves, lds, dev);
  auto it = cache.find(key);
  if (it != cache.end()) return it->second;
  int occ;
  if (split == 3)
    occ = dt == DT_F16 ? ir_wave_stem_occ_f16(waves, lds) : ir_wave_stem_occ_bf16(waves, lds);
  else if (split)
    occ = dt == DT_F16 ? ir_split_occ_f16(ke, npi, nob, rl, split == 2, waves, lds)
                       : ir_split_occ_bf16(ke, npi, nob, rl, split == 2, waves, lds);
  else
    occ = dt == DT_F16 ? ir_wave_occ_f16(ke, npi, nob, rl, waves, lds) : ir_wave_occ_bf16(ke, npi, nob, rl, waves, lds);
  // a failed query (no device to ask): plan for one workgroup per CU, and
  // ask again next time; a real answer, 0 included, is kept
  if (occ < 0) return 1;
  cache[key] = occ;
  return occ;
}

// Output tiles of at most 32 pixels (one MFMA column block) the planner tries.
constexpr uint32_t kTiles[][2] = {{4, 8}, {8, 4}, {5, 6}, {6, 5}, {2, 16}, {16, 2}, {3, 10}, {10, 3},
                                  {4, 7}, {7, 4}, {1, 32}, {32, 1}};

// Throughput of a SIMD that holds n of these latency-bound wavefronts,
// relative to a full one (one wavefront leaves most of each chunk's MFMA,
// LDS and memory latency exposed).
double simd_eff(uint32_t n) { return n <= 1 ? 0.45 : n == 2 ? 0.7 : n == 3 ? 0.85 : 1.0; }

}  // namespace

const char *irw_plan(uint32_t N, uint32_t IH, uint32_t IW, uint32_t OH, uint32_t OW, uint32_t C, uint32_t E,
                     uint32_t CO, uint32_t S, int dt, bool cl, bool rl, uint32_t tile_h, uint32_t tile_w,
                     int32_t weights, int32_t kernel, uint32_t waves_force, IrWavePlan *out, bool stem,
                     bool head) {
  if (head) {
    if (stem) return "a block joins the stem or the head, not both";
    if (kernel != AIH_IR_KERNEL_AUTO && kernel != AIH_IR_KERNEL_SPLIT) return "the head joins the split kernel";
    kernel = AIH_IR_KERNEL_SPLIT;
  }
  if (stem) {
    if (C != 32 || CO != 32 || S != 1) return "the stem-fused block is 32 -> E -> 32 with a stride-1 depthwise";
    if (!rl) return "the stem-fused block takes ReLU after its expand and its depthwise";
    if (kernel != AIH_IR_KERNEL_AUTO && kernel != AIH_IR_KERNEL_WAVE) return "the stem-fused block runs the wave kernel";
    kernel = AIH_IR_KERNEL_WAVE;
  }
  if (dt != DT_F16 && dt != DT_BF16) return "the wave kernels take f16 / bf16 storage";
  if (!cl) return "the wave kernels take clamp-type activations (identity, ReLU, ReLU6, clamp01)";
  if (C % 16 || E % 32 || CO % 16 || C == 0 || E == 0 || CO == 0) return "cin % 16, cexp % 32 and cout % 16 needed";
  if (S != 1 && S != 2) return "depthwise stride must be 1 or 2";
  if (weights != AIH_IR_WEIGHTS_AUTO && weights != AIH_IR_WEIGHTS_RESIDENT && weights != AIH_IR_WEIGHTS_STREAMED)
    return "unknown weight placement";
  if (kernel != AIH_IR_KERNEL_AUTO && kernel != AIH_IR_KERNEL_WAVE && kernel != AIH_IR_KERNEL_SPLIT)
    return "not a wave-family kernel";
  if (kernel == AIH_IR_KERNEL_SPLIT && weights != AIH_IR_WEIGHTS_AUTO)
    return "the split kernel reads its weights from memory (no placement to choose)";
  if (waves_force && waves_force != 1 && waves_force != 2 && waves_force != 4 && waves_force != 8 &&
      waves_force != 12)
    return "wavefronts per workgroup must be 1, 2, 4, 8 or 12 (12: the wave kernel, where its shape allows)";
  const uint32_t ke = C / 16, COP = ir_cop(CO), nob = COP / 32;
  const bool any_wave = irw_has_shape(ke, 2, nob) || irw_has_shape(ke, 5, nob);
  const bool any_split = irs_has_shape(ke, 2, nob) || irs_has_shape(ke, 5, nob);
  if (!(kernel != AIH_IR_KERNEL_SPLIT && any_wave) && !(kernel != AIH_IR_KERNEL_WAVE && any_split))
    return "no wave-kernel instantiation for this width";
  if ((tile_h && tile_h > OH) || (tile_w && tile_w > OW)) return "forced tile larger than the output";
  if (tile_h && tile_w && tile_h * tile_w > 32) return "the wave kernels' tiles hold at most 32 pixels";
  if ((uint64_t)IH * IW * C * 2 >= 0x80000000ull) return "image of 2 GiB or more";
  if ((uint64_t)N * OH * OW >= 0xffffffffull) return "2^32 or more output pixels";

  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = -1;
  struct Key {
    uint32_t v[19];
    bool operator<(const Key &o) const { return std::memcmp(v, o.v, sizeof(v)) < 0; }
  };
  static std::mutex mu;
  static std::map<Key, IrWavePlan> cache;
  const Key key{{N, IH, IW, OH, OW, C, E, CO, S, (uint32_t)dt, tile_h, tile_w, (uint32_t)weights, (uint32_t)dev,
                 rl ? 1u : 0u, (uint32_t)kernel, waves_force, stem ? 1u : 0u, head ? 1u : 0u}};
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
  auto keep = [&](const IrWavePlan &p, double cost) {
    if (!found || cost < best * 0.999) {
      found = true;
      best = cost;
      bp = p;
    }
  };
  auto consider = [&](uint32_t th, uint32_t tw) {
    if (th == 0 || tw == 0 || th * tw > 32) return;
    const uint32_t hh = (th - 1) * S + 3, hw = (tw - 1) * S + 3;
    // halo blocks of the smallest instantiation that holds the halo
    auto npi_of = [&](bool (*has)(uint32_t, uint32_t, uint32_t)) -> uint32_t {
      for (uint32_t n : {2u, 5u})
        if (hh * hw <= n * 32 && has(ke, n, nob)) return n;
      return 0;
    };
    const uint32_t npi_w = npi_of(irw_has_shape), npi_s = npi_of(irs_has_shape);
    const uint32_t tiles_y = cdiv(OH, th), tiles_x = cdiv(OW, tw);
    const uint64_t nt64 = (uint64_t)N * tiles_y * tiles_x;
    if (nt64 > 0x7fffffffull) return;
    const uint32_t nt = (uint32_t)nt64;
    // one chunk of one tile: expand (NPI blocks of KE + 1 MFMAs, their
    // epilogue), the depthwise of 32 pixels x 32 channels (20 16x16x32
    // MFMAs and the operand masking), the projection
    auto chunk_cost = [&](uint32_t npi) { return npi * (ke + 1) * 32.0 + npi * 120.0 + 420.0 + nob * 64.0; };
    if (kernel != AIH_IR_KERNEL_SPLIT && npi_w) {
      const uint32_t npi = npi_w;
      const double chunk = chunk_cost(npi);
      for (uint32_t waves : {12u, 8u, 4u, 2u})
        for (uint32_t resident = 0; resident < 2; ++resident) {
          if (waves_force && waves != waves_force) continue;
          if (waves > irw_max_waves(ke, npi, nob)) continue;
          if ((weights == AIH_IR_WEIGHTS_RESIDENT && !resident) || (weights == AIH_IR_WEIGHTS_STREAMED && resident))
            continue;
          IrWavePlan p{};
          p.split = 0;
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
          p.lds_red = 0;
          p.lds = p.lds_xe + waves * npi * 32 * IRW_XPIX;
          if (stem) {
            if (npi != 2) continue;
            p.lds_stem = p.lds;
            p.lds_res = p.lds_stem + IRW_STEM_LDS;
            p.lds = p.lds_res + waves * IRW_RES_STASH;
          }
          if (resident) {
            p.lds_next = p.lds;
            p.lds += 16;
          }
          if (p.lds > 160u * 1024u) continue;
          p.occ = (uint32_t)irw_occupancy(stem ? 3 : 0, dt, ke, npi, nob, rl, waves, p.lds);
          if (p.occ == 0) continue;  // not resident at this size
          p.tiles_y = tiles_y;
          p.tiles_x = tiles_x;
          p.ntiles = nt;
          p.grid = (uint32_t)std::min<uint64_t>(cdiv(nt, waves), (uint64_t)cus * p.occ);
          // streamed weights pay a barrier and a copy per chunk. A CU's four
          // SIMDs take its workgroups' tiles side by side: the launch lasts
          // `rounds` tile times, slower where a SIMD holds few wavefronts;
          // total work breaks ties.
          const double per_tile = (chunk + (resident ? 0.0 : 300.0)) * nchunks;
          const uint32_t used = std::min(p.grid, cus) * 4;
          const uint32_t rounds = cdiv(nt, used);
          const uint32_t per_simd = std::min<uint32_t>(rounds, cdiv(std::min(p.grid, cus * p.occ) * waves, cus * 4));
          keep(p, (rounds + 1e-3 * (double)nt / (cus * 4.0)) * per_tile / simd_eff(per_simd));
        }
    }
    if (!stem && kernel != AIH_IR_KERNEL_WAVE && weights == AIH_IR_WEIGHTS_AUTO && npi_s) {
      const uint32_t npi = npi_s;
      const double chunk = chunk_cost(npi);
      for (uint32_t w : {1u, 2u, 4u, 8u}) {
        if ((waves_force && w != waves_force) || w > nchunks) continue;
        IrWavePlan p{};
        p.split = 1;
        p.TH = th;
        p.TW = tw;
        p.HH = hh;
        p.HW = hw;
        p.NPI = npi;
        p.resident = 0;
        p.waves = w;
        p.lds_bp = 0;
        p.lds_x = align16(CO * 4);
        p.lds_xe = p.lds_x + npi * 32 * (C * 2 + 16);
        p.lds_w = p.lds_xe + w * npi * 32 * IRW_XPIX;
        p.lds_red = p.lds_x;
        p.lds = p.lds_x + std::max(p.lds_w + w * IRS_RING - p.lds_x, std::min(w, 4u) * nob * IRS_RED_BLOCK);
        if (head) {
          p.lds_head = p.lds;
          p.lds += IRW_HEAD_LDS;
        }
        if (p.lds > 160u * 1024u) continue;
        p.occ = (uint32_t)irw_occupancy(1, dt, ke, npi, nob, rl, w, p.lds);
        if (p.occ == 0) continue;  // not resident at this size
        // the deep prefetch where its registers cost no workgroup this
        // launch would have resident
        const uint32_t occ_deep = (uint32_t)irw_occupancy(2, dt, ke, npi, nob, rl, w, p.lds);
        p.deep = occ_deep > 0 && occ_deep >= std::min(p.occ, cdiv(nt, cus)) ? 1u : 0u;
        if (p.deep) p.occ = occ_deep;
        p.tiles_y = tiles_y;
        p.tiles_x = tiles_x;
        p.ntiles = nt;
        p.grid = nt;
        // a workgroup per tile: the CUs take their share of workgroups in
        // `rounds`, a SIMD then holds per_simd wavefronts of ceil(chunks / W)
        // chunks each, weights read from memory (L2) instead of LDS; the
        // partial sums meet once per tile
        const uint32_t wg_cu = std::min(p.occ, cdiv(nt, cus));
        const uint32_t rounds = cdiv(nt, cus * wg_cu);
        const uint32_t per_simd = cdiv(w * wg_cu, 4);
        const double per_wave = cdiv(nchunks, w) * (chunk + 150.0) + 1500.0 + (w > 1 ? 200.0 * nob * w : 0.0);
        keep(p, rounds * per_simd * per_wave / simd_eff(per_simd));
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

hipError_t launch_ir_wave_stem(const IrWaveArgs &a, int dt, const IrWavePlan &p, hipStream_t st) {
  if (p.lds > 160u * 1024u || p.grid == 0 || p.split || p.NPI != 2 || a.C != 32 || a.COP != 32 ||
      (p.waves != 2 && p.waves != 4 && p.waves != 8 && p.waves != 12) || p.waves > irw_max_waves(2, 2, 1))
    return hipErrorInvalidValue;
  switch (dt) {
    case DT_F16: return launch_ir_wave_stem_f16(a, p.waves, p.lds, p.grid, st);
    case DT_BF16: return launch_ir_wave_stem_bf16(a, p.waves, p.lds, p.grid, st);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_ir_wave(const IrWaveArgs &a, int dt, const IrWavePlan &p, hipStream_t st) {
  if (p.lds > 160u * 1024u || p.grid == 0) return hipErrorInvalidValue;
  if (p.split) {
    if (p.waves != 1 && p.waves != 2 && p.waves != 4 && p.waves != 8) return hipErrorInvalidValue;
    switch (dt) {
      case DT_F16: return launch_ir_split_f16(a, p.NPI, p.deep != 0, p.waves, p.lds, p.grid, st);
      case DT_BF16: return launch_ir_split_bf16(a, p.NPI, p.deep != 0, p.waves, p.lds, p.grid, st);
      default: return hipErrorInvalidValue;
    }
  }
  if ((p.waves != 2 && p.waves != 4 && p.waves != 8 && p.waves != 12) ||
      p.waves > irw_max_waves(a.C / 16, p.NPI, a.COP / 32))
    return hipErrorInvalidValue;
  switch (dt) {
    case DT_F16: return launch_ir_wave_f16(a, p.NPI, p.waves, p.lds, p.grid, st);
    case DT_BF16: return launch_ir_wave_bf16(a, p.NPI, p.waves, p.lds, p.grid, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace aih

// ir_wave_impl.h -- fused inverted-residual block, one output tile per
// wavefront (16-bit storage, clamp-type activations).
//
// The same three convs as ir_block_impl.h (1x1 expand + act, depthwise 3x3
// stride S + act, 1x1 project + act (+ residual); crates/ai-gpu-runtime/src/
// lowering.rs:122-152 dispatches them separately) with the same arithmetic
// and rounding points, decomposed for overlap instead of sharing:
//
//   * every wavefront owns its own output tile of at most 32 pixels (one
//     MFMA column block) and runs expand -> depthwise -> project for it
//     alone; its expanded chunk lives in a private LDS region, so the
//     wavefronts of a workgroup never wait for each other between phases --
//     while one packs its expand results another runs its depthwise MFMAs;
//   * the input tile (with its halo, NPI blocks of 32 pixels) goes from
//     memory straight into MFMA operand registers once per tile (16-byte
//     buffer loads, zeros outside the image through the range check) and
//     is reused by every chunk;
//   * the expand / project / depthwise weights of a 32-channel chunk sit in
//     LDS in the converter's packed layouts (pack.rs:68-122), shared by the
//     workgroup: all chunks resident for the whole launch when they fit (no
//     workgroup barrier after the first), else streamed through two slots,
//     the next chunk's copy (LDS-direct loads) overlapping the current one,
//     with one barrier per chunk.
//
// MFMA convention as in ir_block_impl.h: weights are the A operand (rows =
// channels), pixels the B operand, v_mfma_f32_32x32x16_{f16,bf16}; lane l
// holds pixel l%32 and channels 8*(r/4) + 4*(l/32) + r%4 of a result. The
// expand bias enters as one extra K step against a column that is 1.0 for
// pixels inside the image and 0 outside, so outside pixels expand to exactly
// 0 (the depthwise zero padding; the activations here are all clamp-type,
// act(0) = 0). The depthwise runs on 16x16x32 MFMAs with diagonal weight
// operands (below); its result lane holds exactly the K slice it feeds to
// the projection's MFMAs, so it is their B operand without an LDS round trip.
#pragma once

#include "conv_stem.h"
#include "ir_block_impl.h"

namespace aih {

// Global -> LDS copy of n items of SZ bytes (LDS-direct loads, no
// registers): item g from byte offset src(g) + soff (soff: a wavefront-
// uniform part, added in the scalar offset); the workgroup's `threads`
// take 64-item rows in turn, a row per wavefront. Asynchronous until
// ir_dma_wait() and a barrier.
template <int SZ, class F>
__device__ __forceinline__ void irw_dma(char *dst, uint32_t n, __amdgpu_buffer_rsrc_t rs, int wave, int lane,
                                        uint32_t threads, F src, uint32_t soff = 0) {
  for (uint32_t g0 = (uint32_t)wave * 64; g0 < n; g0 += threads) {
    const uint32_t g = g0 + lane;
    if (g >= n) continue;
    ir_lds_void *d = (ir_lds_void *)(dst + g0 * SZ);
    if constexpr (SZ == 16)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, d, 16, src(g), (int)soff, 0, 0);
    else
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, d, 4, src(g), (int)soff, 0, 0);
  }
}

// ReLU of two 16-bit floats packed in 32 bits, as 16-bit signed integers:
// every negative float (and -0) has its sign bit set, so max(bits, 0) is 0
// exactly where max(x, 0) is, and a non-negative float keeps its bits (one
// v_pk_max_i16 for two values). Rounding is monotone and keeps the sign, so
// relu(round(x)) == round(relu(x)) bit for bit: packing first is exact.
__device__ __forceinline__ uint32_t irw_relu2(uint32_t v) {
  typedef short s16x2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(s16x2, v), s16x2{0, 0}));
}

// act(v) rounded to the storage dtype, 4 values -> 8 bytes: ReLU after the
// conversion on packed 16-bit integers; other clamp-type activations before
// it (one v_med3_f32 each).
template <int DT, bool RELU>
__device__ __forceinline__ u32x2 irw_act_pack4(const Act &p, f32x4 v) {
  if constexpr (RELU) {
    const u32x2 b = pack4<DT>(v);
    return u32x2{irw_relu2(b.x), irw_relu2(b.y)};
  }
  float t[4] = {v.x, v.y, v.z, v.w};
  ir_act<true, 4>(p, t);
  return pack4<DT>(f32x4{t[0], t[1], t[2], t[3]});
}

// Orders this wavefront's LDS accesses on either side (its lanes write the
// expanded chunk that other lanes of the same wavefront read next; a
// wavefront's LDS operations complete in issue order, so only the compiler
// must not move them across).
__device__ __forceinline__ void irw_wave_order() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("" ::: "memory");
}

// ---- depthwise 3x3 and projection on 16x16x32 MFMAs ----
//
// Lane l: l16 = l % 16 is a pixel (B column, result column) or a channel (A
// row); q = l / 16 its K slice of 8 elements. The depthwise of a chunk runs
// as matrix products whose K = 32 holds two taps of 16 channels: slice q is
// channels 8 (q % 2) .. + 7 of tap ta (q < 2) or of its partner tb (q >= 2),
// read as 16 bytes of the expanded chunk (B) and of the tap weights (A). A is
// diagonal -- row c holds w[t][c] at channel c's K position of each tap and
// zeros elsewhere, a lane's 16 weight bytes masked to its own element -- so
// result row c, column p is w[ta][c] x[p + ta][c] + w[tb][c] x[p + tb][c]
// (+ the accumulator): two taps of a 16-channel x 16-pixel depthwise per
// MFMA, fp32 accumulation of exact 16-bit products, the bias entering as the
// first MFMA's accumulator. Nine taps are four pairs and one single whose
// partner is a zero run in the weight slot. The 32 channels of a chunk are
// two 16-channel groups (cg), the 32 output pixels of a tile two 16-pixel
// groups (pg). The result lane (pixel p, slice q) holds rows 4q .. 4q + 3 of
// each group; packed after act_d, group 0's four then group 1's four are
// exactly the projection's B operand for K slice q when the projection's K
// order is channels {4q .. 4q+3, 16+4q .. 16+4q+3}: packed weight groups q and
// q + 4 of the chunk (ir_ld_w with a stride of four groups).
//
// Pairs, taps t = 3 dy + dx:            A (tap weights)      B (expanded chunk)
//   (0, 1) (3, 4) (6+1, 6+2) along a row    wa1 + 64 ta          bc[dy] (+ one pixel for (7, 8))
//   (2, 5) down a column                    wa3 + 64 * 2         br + two pixels
//   (6, zero run)                           wa3 + 64 * 6         bc[2] (partner lanes read tap 7, times 0)
// wa1 / wa3: the word of the lane's row channel, + one / three taps for q >= 2;
// bc[dy] = pixel row + dy rows (+ one pixel for q >= 2); br = pixel row (+ one
// row for q >= 2). Every read stays inside the tile's halo rows. (Reads of the
// expanded chunk: plane 2 cg + q % 2, 16 bytes at the halo pixel.)

template <int DT>
__device__ __forceinline__ f32x4 ir_mma16(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (DT == DT_F16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                  0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
}

// Lane constants of the depthwise MFMAs. The A operand of lane (row c, slice
// q) is zero but for w[t][c] in its own element: the lane reads just the
// 32-bit word holding channel c's weight (and its neighbour's) and masks it
// into the dword of its element.
struct IrDwLane {
  u32x4 mask;         // the lane's diagonal element (0xffff in its half of its dword), or zero
  uint32_t wa1, wa3;  // tap-weight word offsets in a slot: channel c's word, + 1 / 3 taps for q >= 2
};

__device__ __forceinline__ IrDwLane irdw_lane(int lane) {
  const uint32_t l16 = lane & 15, q = lane >> 4, qh = q & 1, qt = q >> 1;
  const uint32_t e = l16 & 7, j = e >> 1;
  const uint32_t hm = (l16 >> 3) == qh ? ((e & 1) ? 0xffff0000u : 0x0000ffffu) : 0u;
  IrDwLane L;
  L.mask = u32x4{j == 0 ? hm : 0u, j == 1 ? hm : 0u, j == 2 ? hm : 0u, j == 3 ? hm : 0u};
  L.wa1 = (l16 & ~1u) * 2 + qt * 64;
  L.wa3 = (l16 & ~1u) * 2 + qt * 192;
  return L;
}

// B-operand byte offsets (within the wavefront's expanded chunk, planes of
// PLANE bytes) of the output pixel whose top-left halo pixel is rp, for lane
// slice q: bc[dy] and br as in the table above (plane q % 2 of the channel
// group; the group's plane offset and the tap column are immediates).
__device__ __forceinline__ void irdw_rows(uint32_t rp, uint32_t hw, int q, uint32_t plane, uint32_t (&bc)[3],
                                          uint32_t &br) {
  const uint32_t qh = q & 1, qt = q >> 1;
  const uint32_t lo = qh * plane + rp * 16;
#pragma unroll
  for (int dy = 0; dy < 3; ++dy) bc[dy] = lo + (dy * hw + qt) * 16;
  br = lo + qt * hw * 16;
}

// The depthwise of one chunk for the wavefront's two 16-pixel groups: tap
// weights and biases of the chunk at sm (slot layout: 9 taps, zero run, bd,
// be), its expanded planes (PLANE bytes each) at xe. Returns the projection
// B operand of each pixel group: act_d of the result in the storage dtype,
// rows 4q .. 4q + 3 of channel group 0, then of group 1.
template <int DT, bool RLD, uint32_t PLANE>
__device__ __forceinline__ void irdw_chunk(const char *xe, const char *sm, const IrDwLane &L,
                                          const uint32_t (&bc)[2][3], const uint32_t (&br)[2], int q,
                                          const Act &act_d, u32x4 (&bop)[2]) {
  // Ten steps s = 5 cg + P: channel group cg (one after the other: half the
  // accumulators live at a time), tap pair P; in each, the two pixel groups'
  // MFMA chains interleave. The operands of step s + 1 are read before the
  // MFMAs of step s, so an MFMA does not wait on the LDS read just issued.
  auto aoff = [&](int P) -> uint32_t {
    return P == 0 ? L.wa1 : P == 1 ? L.wa1 + 3 * 64 : P == 2 ? L.wa1 + 7 * 64 : P == 3 ? L.wa3 + 2 * 64
                                                                                         : L.wa3 + 6 * 64;
  };
  auto boff = [&](int P, int pg) -> uint32_t {
    return P == 0 ? bc[pg][0] : P == 1 ? bc[pg][1] : P == 2 ? bc[pg][2] + 16 : P == 3 ? br[pg] + 32 : bc[pg][2];
  };
  uint32_t A[2];
  u32x4 B[2][2];
  auto load = [&](int s, int slot) {
    const int cg = s / 5, P = s % 5;
    A[slot] = *reinterpret_cast<const uint32_t *>(sm + aoff(P) + 32 * cg);
#pragma unroll
    for (int pg = 0; pg < 2; ++pg)
      B[slot][pg] = *reinterpret_cast<const u32x4 *>(xe + boff(P, pg) + 2 * cg * PLANE);
  };
  u32x2 h[2][2];  // [cg][pg]: act_d of the result, packed
  f32x4 d[2], bias;
  load(0, 0);
#pragma unroll
  for (int s = 0; s < 10; ++s) {
    const int cg = s / 5, P = s % 5, cur = s & 1;
    if (P == 0)  // bias of rows 4q..4q+3: the first MFMA's accumulator
      bias = unpack4<DT>(*reinterpret_cast<const u32x2 *>(sm + IRW_BD + (16 * cg + 4 * q) * 2));
    if (s + 1 < 10) load(s + 1, cur ^ 1);
    const u32x4 Am = u32x4{A[cur], A[cur], A[cur], A[cur]} & L.mask;
#pragma unroll
    for (int pg = 0; pg < 2; ++pg) d[pg] = ir_mma16<DT>(Am, B[cur][pg], P == 0 ? bias : d[pg]);
    if (P == 4) {
#pragma unroll
      for (int pg = 0; pg < 2; ++pg) {
        if constexpr (RLD) {
          const u32x2 b = pack4<DT>(d[pg]);
          h[cg][pg] = u32x2{irw_relu2(b.x), irw_relu2(b.y)};
        } else {
          float t[4] = {d[pg].x, d[pg].y, d[pg].z, d[pg].w};
          ir_act<true, 4>(act_d, t);
          h[cg][pg] = pack4<DT>(f32x4{t[0], t[1], t[2], t[3]});
        }
      }
    }
  }
#pragma unroll
  for (int pg = 0; pg < 2; ++pg) bop[pg] = u32x4{h[0][pg].x, h[0][pg].y, h[1][pg].x, h[1][pg].y};
}

// Bias, act_p, residual and the store of a wavefront's projection results:
// block og (16 output channels) of pixel group pg, lane rows 4q .. 4q + 3 =
// output channels 16 og + 4q .. + 3 of pixel pix[pg]. STEM: the residual
// comes from the wavefront's stash (32 16-bit channels per tile pixel, tile
// pixel pg * 16 + l16), not from memory.
template <int DT, int NOG, bool STEM = false>
__device__ __forceinline__ void irdw_store(const IrWaveArgs &a, const float *BpL, const f32x4 (&acc)[NOG][2],
                                          const bool (&ok)[2], const uint32_t (&pix)[2], int q, const Act &act_p,
                                          const char *ResL = nullptr, int l16 = 0) {
#pragma unroll
  for (int og = 0; og < NOG; ++og) {
    const uint32_t oc = og * 16 + 4 * q;
    if (og * 16 >= (int)a.CO) continue;  // padding channels of the last 32-channel block
#pragma unroll
    for (int pg = 0; pg < 2; ++pg) {
      if (!ok[pg]) continue;
      f32x4 v = acc[og][pg] + *reinterpret_cast<const f32x4 *>(BpL + oc);
      float t4[4] = {v.x, v.y, v.z, v.w};
      ir_act<true, 4>(act_p, t4);
      v = f32x4{t4[0], t4[1], t4[2], t4[3]};
      const size_t vi = (size_t)pix[pg] * (a.CO / 4) + oc / 4;
      if constexpr (STEM)
        v += unpack4<DT>(*reinterpret_cast<const u32x2 *>(ResL + ((pg * 16 + l16) * 32 + oc) * 2));
      else if (a.has_res)
        v += Vec4IO<DT>::load(a.res, vi);
      Vec4IO<DT>::store(a.y, vi, v);
    }
  }
}

// KE: expand K steps (C / 16); NPI: 32-pixel blocks of the halo tile; NOB:
// projection blocks of 32 output channels; RL: the expand and depthwise
// activations are both ReLU (applied to the packed 16-bit results).
// Wavefronts per SIMD the register allocation aims for: three where a
// workgroup may have 12 wavefronts (168 VGPRs; the 32-channel shape, at four
// wavefronts a SIMD within 128, spilled and ran slower), else what the shape
// needs.
__host__ __device__ constexpr int irw_waves_per_simd(int ke, int npi, int nob) {
  return irw_max_waves(ke, npi, nob) == 12 ? 3 : 1;
}

// The kernel body. STEM: the block's input is computed, not read -- each halo
// pixel's 32 channels are the stem conv's output at that pixel (the 3x3
// conv over the 3-channel fp32 image, with the stem kernel's operands,
// MFMA steps, bias, activation and rounding: bit for bit what the stem
// kernel stores), held as the expand's B operands, and the tile's own
// pixels of it stashed in LDS as the projection's residual. The expand's
// operands are the unfused block's, in its K order, so the block's sums are
// the same.
template <int DT, int KE, int NPI, int NOB, bool RL, bool STEM>
__device__ __forceinline__ void ir_wave_body(const IrWaveArgs &a) {
  static_assert(DT == DT_F16 || DT == DT_BF16, "16-bit storage");
  static_assert(!STEM || (KE == 2 && NOB == 1), "the stem feeds a 32-channel block");
  extern __shared__ __align__(16) char lds[];
  constexpr int ES = 2, KSTEP = 16, HK = 8, EC = 32, NOG = 2 * NOB;
  constexpr uint32_t GB = 4 * ES;  // one packed group: 4 K of one channel
  constexpr uint32_t C = KE * KSTEP;
  constexpr uint32_t WES = EC * C * ES;  // expand weights of one chunk
  constexpr bool RLE = RL, RLD = RL;
  const int tid = threadIdx.x;
  const int lane = tid & 63, l32 = lane & 31, lh = lane >> 5, l16 = lane & 15, q = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // wavefronts of this workgroup (2, 4, 8 or 12, chosen by the plan)
  const uint32_t nthr = blockDim.x, nwaves = nthr >> 6;

  const uint32_t WPG = EC * a.CO * ES;         // project weights of one chunk in memory
  const uint32_t WPS = EC * a.COP * ES;        // ... in a slot, rows padded to COP channels
  const uint32_t SLOT = WES + WPS + IRW_SMB;   // 16-byte multiple (C, COP multiples of 16 / 32)
  const uint32_t nchunks = a.E / EC;
  char *WL = lds + a.lds_w;
  float *BpL = reinterpret_cast<float *>(lds + a.lds_bp);
  constexpr uint32_t PLANE = NPI * 32 * 16;  // one 8-channel plane of the expanded chunk
  char *XeL = lds + a.lds_xe + (uint32_t)wave * (4 * PLANE);
  const Act act_e = act_params(a.act_e), act_d = act_params(a.act_d), act_p = act_params(a.act_p);
  const IrDwLane DL = irdw_lane(lane);

  const __amdgpu_buffer_rsrc_t rs_we = ir_rsrc(a.we, C * a.E * ES);
  const __amdgpu_buffer_rsrc_t rs_wp = ir_rsrc(a.wp, a.E * a.CO * ES);
  const __amdgpu_buffer_rsrc_t rs_wd = ir_rsrc(a.wd, 9 * a.E * ES);
  const __amdgpu_buffer_rsrc_t rs_bd = ir_rsrc(a.bd, a.E * ES);
  const __amdgpu_buffer_rsrc_t rs_be = ir_rsrc(a.be, a.E * ES);

  // chunk c's weights (expanded channels [32c, 32c + 32)) -> slot s, byte
  // for byte in the packed layouts: expand element (k, e) at (k/4 * E + e) * 4
  // + k%4 gives C/4 runs of 32 channels; the project weights of K rows
  // [32c, 32c + 32) are one contiguous run (EC/4 runs of CO channels, each
  // to a COP-channel row when CO < COP); depthwise taps 9 runs of 32.
  auto dma_chunk = [&](uint32_t c, uint32_t s) {
    char *slot = WL + s * SLOT;
    constexpr uint32_t GR = EC * GB / 16;  // 16-byte items per expand run
    irw_dma<16>(slot, (C / 4) * GR, rs_we, wave, lane, nthr,
                [&](uint32_t g) -> uint32_t { return ((g / GR) * a.E + EC * c) * GB + (g % GR) * 16; });
    if (a.COP == a.CO) {
      irw_dma<16>(slot + WES, WPS / 16, rs_wp, wave, lane, nthr,
                  [&](uint32_t g) -> uint32_t { return c * WPG + g * 16; });
    } else {
      const uint32_t rb = a.CO * GB;  // bytes of one K group's run
      for (uint32_t qq = 0; qq < EC / 4; ++qq)
        irw_dma<16>(slot + WES + qq * (a.COP * GB), rb / 16, rs_wp, (wave + qq) % nwaves, lane, nthr,
                    [&](uint32_t g) -> uint32_t { return c * WPG + qq * rb + g * 16; });
    }
    constexpr uint32_t TR = EC * ES / 16;  // 16-byte items per depthwise tap run
    char *sm = slot + WES + WPS;
    irw_dma<16>(sm, 9 * TR, rs_wd, wave, lane, nthr,
                [&](uint32_t g) -> uint32_t { return ((g / TR) * a.E + EC * c) * ES + (g % TR) * 16; });
    irw_dma<4>(sm + IRW_BD, EC * ES / 4, rs_bd, wave, lane, nthr,
               [&](uint32_t g) -> uint32_t { return EC * c * ES + g * 4; });
    irw_dma<4>(sm + IRW_BE, EC * ES / 4, rs_be, wave, lane, nthr,
               [&](uint32_t g) -> uint32_t { return EC * c * ES + g * 4; });
  };

  for (uint32_t i = tid; i < a.CO / 4; i += nthr)
    *reinterpret_cast<f32x4 *>(BpL + 4 * i) = Vec4IO<DT>::load(a.bp, i);
  const uint32_t nslots = a.resident ? nchunks : 2u;
  if (a.COP != a.CO) {
    // project weights of channels CO..COP: zero in every slot, for good (the
    // copies write only channels below CO)
    const uint32_t pad16 = (a.COP - a.CO) * GB / 16;
    for (uint32_t i = tid; i < nslots * (EC / 4) * pad16; i += nthr) {
      const uint32_t sq = i / pad16, v = i - sq * pad16;
      *reinterpret_cast<u32x4 *>(WL + (sq / (EC / 4)) * SLOT + WES + (sq % (EC / 4)) * (a.COP * GB) + a.CO * GB +
                                 v * 16) = u32x4{0u, 0u, 0u, 0u};
    }
  }
  // the zero run after each slot's taps (the copies never write it)
  for (uint32_t i = tid; i < nslots * 4; i += nthr)
    *reinterpret_cast<u32x4 *>(WL + (i >> 2) * SLOT + WES + WPS + IRW_TAPS_ZERO + (i & 3) * 16) =
        u32x4{0u, 0u, 0u, 0u};
  if (a.resident) {
    for (uint32_t c = 0; c < nchunks; ++c) dma_chunk(c, c);
  } else {
    dma_chunk(0, 0);
  }
  if constexpr (STEM) {
    // the stem's A operands as the stem kernel builds them (lane (channel
    // l32, half lh), steps 0..2) and its bias in fp32, once per workgroup
    if (tid < 64) {
#pragma unroll
      for (int s = 0; s < 3; ++s)
        *reinterpret_cast<u32x4 *>(lds + a.lds_stem + (s * 64 + lane) * 16) = stem_a16(a.sw, 4, C / 4, l32, lh, s);
    } else if (tid < 64 + (int)C / 4) {
      const int g = tid - 64;
      *reinterpret_cast<f32x4 *>(lds + a.lds_stem + 3 * 64 * 16 + g * 16) = Vec4IO<DT>::load(a.sb, g);
    }
  }
  // this workgroup's contiguous range of tiles (handed out XCD by XCD)
  const uint32_t blk = xcd_remap(blockIdx.x, gridDim.x, a.nxcd);
  const uint32_t t_begin = (uint32_t)(((uint64_t)blk * a.ntiles) / gridDim.x);
  const uint32_t t_end = (uint32_t)(((uint64_t)(blk + 1) * a.ntiles) / gridDim.x);
  // resident weights: after its first tile a wavefront claims the range's
  // next unclaimed tile from this counter
  uint32_t *next_tile = reinterpret_cast<uint32_t *>(lds + a.lds_next);
  if (a.resident && tid == 0) *next_tile = t_begin + nwaves;
  ir_dma_wait();
  __syncthreads();

  const char *xg = reinterpret_cast<const char *>(a.x);
  const uint32_t img_bytes = a.IH * a.IW * C * ES;
  // STEM: the whole fp32 image batch as one buffer (below 2 GiB), and this
  // wavefront's residual stash
  const __amdgpu_buffer_rsrc_t rs_sx = STEM ? ir_rsrc(a.sx, a.sx_bytes) : ir_rsrc(a.we, 0);
  char *ResL = lds + a.lds_res + (uint32_t)wave * IRW_RES_STASH;
  const Act act_s = act_params(a.act_s);

  const uint32_t per_img = a.tiles_y * a.tiles_x;
  const uint32_t HPIX = a.HH * a.HW, TPIX = a.TH * a.TW;
  constexpr uint32_t ONE = DT == DT_F16 ? 0x3C00u : 0x3F80u;

  // ---- per-tile state of this wavefront ----
  u32x4 xop[NPI][KE];  // input halo pixels as expand B operands
  bool inside[NPI];    // this lane's halo pixel of block b lies in the image
  uint32_t bc[2][3], br[2];  // depthwise B offsets per 16-pixel group
  uint32_t pix[2];     // this lane's output pixel of each group
  bool ok[2];
  f32x4 acc[NOG][2];

  auto begin_tile = [&](uint32_t T) {
    const uint32_t img = fdiv(T, a.fd_pi);
    const uint32_t trem = T - img * per_img;
    const uint32_t tyi = fdiv(trem, a.fd_tx);
    const uint32_t ty0 = tyi * a.TH, tx0 = (trem - tyi * a.tiles_x) * a.TW;
    const int32_t iy0 = (int32_t)(ty0 * a.S) - a.PT, ix0 = (int32_t)(tx0 * a.S) - a.PL;
    const __amdgpu_buffer_rsrc_t rs_x = ir_rsrc(xg + (size_t)img * img_bytes, STEM ? 0u : img_bytes);
#pragma unroll
    for (int b = 0; b < NPI; ++b) {
      const uint32_t r = b * 32 + l32;
      const uint32_t hy = fdiv(r, a.fd_hw), hx = r - hy * a.HW;
      const int32_t iy = iy0 + (int32_t)hy, ix = ix0 + (int32_t)hx;
      const bool in = r < HPIX && (uint32_t)iy < a.IH && (uint32_t)ix < a.IW;
      inside[b] = in;
      if constexpr (!STEM) {
        const uint32_t off = in ? ((uint32_t)iy * a.IW + (uint32_t)ix) * (C * ES) + lh * 16 : IR_OOB;
#pragma unroll
        for (int k = 0; k < KE; ++k)
          xop[b][k] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs_x, off + k * 32, 0, 0));
      } else {
        // the stem at block input pixel (iy, ix): its 5 input-pixel slots of
        // this lane half (zeros outside the image, or for a halo pixel
        // outside the block's input), 3 MFMAs from the bias, act, rounded
        const int32_t sy0 = iy * (int32_t)a.SS - a.SPT, sx0 = ix * (int32_t)a.SS - a.SPL;
        // taps inside the image, bit 3 dy + dx: rows times columns
        const uint32_t rk = ((uint32_t)sy0 < a.SIH ? 07u : 0u) | ((uint32_t)(sy0 + 1) < a.SIH ? 070u : 0u) |
                            ((uint32_t)(sy0 + 2) < a.SIH ? 0700u : 0u);
        const uint32_t ck = ((uint32_t)sx0 < a.SIW ? 0111u : 0u) | ((uint32_t)(sx0 + 1) < a.SIW ? 0222u : 0u) |
                            ((uint32_t)(sx0 + 2) < a.SIW ? 0444u : 0u);
        const uint32_t m9 = in ? rk & ck : 0u;
        // 3 x the pixel index of tap (0, 0) (modulo 2^32 where it lies
        // outside the image; every tap read lies inside, below 2 GiB): a
        // tap's byte offset is 4 x that + its wave-uniform offset, shifts and
        // adds instead of a quarter-rate multiply per tap (the empty asm
        // keeps the compiler from folding them back into one)
        const uint32_t vp = ((uint32_t)img * a.SIH + (uint32_t)sy0) * a.SIW + (uint32_t)sx0;
        uint32_t vp2 = vp << 1;
        asm volatile("" : "+v"(vp2));
        const uint32_t vp3 = vp2 + vp;
        // the five loads go out together, converted after (the scheduler
        // would otherwise wait for each before issuing the next)
        typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
        u32x3 sv[5];
#pragma unroll
        for (int i = 0; i < 5; ++i) {
          // the slot's tap in either lane half (compile-time), its byte
          // offset from tap (0, 0) (wave-uniform)
          const int t0 = stem_slot_tap(0, i), t1 = stem_slot_tap(1, i);
          const uint32_t so0 = ((uint32_t)(t0 / 3) * a.SIW + (uint32_t)(t0 % 3)) * 12u;
          const uint32_t so1 = ((uint32_t)(t1 / 3) * a.SIW + (uint32_t)(t1 % 3)) * 12u;
          const bool tin = lh ? (m9 >> t1) & 1u : (m9 >> t0) & 1u;  // bit 9 (no tap) is 0
          sv[i] = __builtin_amdgcn_raw_buffer_load_b96(rs_sx, tin ? (vp3 << 2) + (lh ? so1 : so0) : IR_OOB, 0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
        u32x2 th[6];
#pragma unroll
        for (int i = 0; i < 5; ++i)
          th[i] = pack4<DT>(f32x4{__uint_as_float(sv[i].x), __uint_as_float(sv[i].y), __uint_as_float(sv[i].z), 0.0f});
        th[5] = u32x2{0u, 0u};
        // the accumulator starts at the bias, as in the stem kernel (the same
        // fp32 sums)
        const char *sbl = lds + a.lds_stem + 3 * 64 * 16 + lh * 16;
        const f32x4 sbias[4] = {*reinterpret_cast<const f32x4 *>(sbl), *reinterpret_cast<const f32x4 *>(sbl + 32),
                                *reinterpret_cast<const f32x4 *>(sbl + 64), *reinterpret_cast<const f32x4 *>(sbl + 96)};
        f32x16 sa = stem_acc_init(sbias);
#pragma unroll
        for (int s = 0; s < 3; ++s)
          sa = ir_mma<DT>(*reinterpret_cast<const u32x4 *>(lds + a.lds_stem + (s * 64 + lane) * 16),
                          u32x4{th[2 * s].x, th[2 * s].y, th[2 * s + 1].x, th[2 * s + 1].y}, sa);
        // lane: pixel r, channels 8 qq + 4 lh .. + 3 in sa[4 qq .. 4 qq + 3]
        u32x2 h[4];
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {
          const f32x4 o = f32x4{sa[4 * qq], sa[4 * qq + 1], sa[4 * qq + 2], sa[4 * qq + 3]};
          const u32x2 p = pack4<DT>(f32x4{act_clamp_any(act_s, o.x), act_clamp_any(act_s, o.y),
                                          act_clamp_any(act_s, o.z), act_clamp_any(act_s, o.w)});
          h[qq] = in ? p : u32x2{0u, 0u};
        }
        // the expand's B operand of step k, lane half lh: channels 16k + 8lh
        // .. + 7, as the unfused block loads them (the same K order, so the
        // same MFMA sums); half 0 holds groups 8q + 0..3, half 1 8q + 4..7:
        // each half passes the other the two groups it lacks
        const u32x2 sa0 = lh ? h[0] : h[1], sb0 = lh ? h[2] : h[3];
        const u32x2 ra = u32x2{(uint32_t)__shfl_xor((int)sa0.x, 32), (uint32_t)__shfl_xor((int)sa0.y, 32)};
        const u32x2 rb = u32x2{(uint32_t)__shfl_xor((int)sb0.x, 32), (uint32_t)__shfl_xor((int)sb0.y, 32)};
        xop[b][0] = lh ? u32x4{ra.x, ra.y, h[1].x, h[1].y} : u32x4{h[0].x, h[0].y, ra.x, ra.y};
        xop[b][1] = lh ? u32x4{rb.x, rb.y, h[3].x, h[3].y} : u32x4{h[2].x, h[2].y, rb.x, rb.y};
        // the tile's own pixels: the projection's residual (stride 1, the
        // block's input pixel (iy, ix) = output pixel (iy0 + hy, ix0 + hx)
        // less the padding)
        const uint32_t ry = hy - (uint32_t)a.PT, rx = hx - (uint32_t)a.PL;
        if (r < HPIX && ry < a.TH && rx < a.TW) {
#pragma unroll
          for (int qq = 0; qq < 4; ++qq)
            *reinterpret_cast<u32x2 *>(ResL + ((ry * a.TW + rx) * 32 + 8 * qq + 4 * lh) * 2) = h[qq];
        }
      }
    }
#pragma unroll
    for (int pg = 0; pg < 2; ++pg) {
      const uint32_t op = pg * 16 + l16;
      const bool in_tile = op < TPIX;
      const uint32_t oy = in_tile ? fdiv(op, a.fd_tw) : 0, ox = in_tile ? op - oy * a.TW : 0;
      irdw_rows(oy * a.S * a.HW + ox * a.S, a.HW, q, PLANE, bc[pg], br[pg]);
      const uint32_t gy = ty0 + oy, gx = tx0 + ox;
      ok[pg] = in_tile && gy < a.OH && gx < a.OW;
      pix[pg] = (img * a.OH + gy) * a.OW + gx;
    }
#pragma unroll
    for (int og = 0; og < NOG; ++og) acc[og][0] = acc[og][1] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  };

  // expand of chunk `slot` over the halo tile -> this wavefront's XeL, then
  // its depthwise and projection into acc
  auto run_chunk = [&](const char *slot) {
    // expand A operands of the chunk: channel l32, K groups from 2 * lh; a K
    // step advances 4 groups of 32 channels (1024 bytes)
    const char *ap = slot + ((uint32_t)lh * (HK / 4) * EC + l32) * GB;
    u32x4 aw[KE];
#pragma unroll
    for (int k = 0; k < KE; ++k) aw[k] = ir_ld_w<DT>(ap + k * (KSTEP * EC * ES), EC * GB);
    const char *sm = slot + WES + WPS;
    const uint32_t bw = lh == 0 ? (uint32_t)*reinterpret_cast<const uint16_t *>(sm + IRW_BE + l32 * 2) : 0u;
#pragma unroll
    for (int b = 0; b < NPI; ++b) {
      const u32x4 bx = {(lh == 0 && inside[b]) ? ONE : 0u, 0u, 0u, 0u};
      f32x16 e = ir_mma<DT>(u32x4{bw, 0u, 0u, 0u}, bx, f32x16{});
#pragma unroll
      for (int k = 0; k < KE; ++k) e = ir_mma<DT>(aw[k], xop[b][k], e);
      // channels 8 qq + 4 lh .. + 3: plane qq, the pixel's 16 bytes at 8 lh
      char *px = XeL + (b * 32 + l32) * 16 + lh * 8;
#pragma unroll
      for (int qq = 0; qq < 4; ++qq)
        *reinterpret_cast<u32x2 *>(px + qq * PLANE) =
            irw_act_pack4<DT, RLE>(act_e, f32x4{e[4 * qq], e[4 * qq + 1], e[4 * qq + 2], e[4 * qq + 3]});
    }
    irw_wave_order();

    u32x4 bop[2];
    // a wavefront in its depthwise and projection MFMAs issues ahead of the
    // SIMD's others (their expands and packing): measured against no
    // priority, and against raising it for the expand or for either half
    // alone, this keeps the matrix pipe fed best (encoder +0.6-1.3 % on one
    // box each, the same tiles)
    __builtin_amdgcn_s_setprio(1);
    irdw_chunk<DT, RLD, PLANE>(XeL, sm, DL, bc, br, q, act_d, bop);
    // projection: K slice q = packed groups q and q + 4 of the chunk
    const char *wpp = slot + WES + ((uint32_t)q * a.COP + l16) * GB;
#pragma unroll
    for (int og = 0; og < NOG; ++og) {
      if (og * 16 >= (int)a.CO) continue;
      const u32x4 wv = ir_ld_w<DT>(wpp + og * (16 * GB), 4 * a.COP * GB);
#pragma unroll
      for (int pg = 0; pg < 2; ++pg) acc[og][pg] = ir_mma16<DT>(wv, bop[pg], acc[og][pg]);
    }
    __builtin_amdgcn_s_setprio(0);
    // the next chunk's expand overwrites XeL after these reads
    irw_wave_order();
  };

  if (a.resident) {
    // every chunk in LDS: the wavefronts run their tiles independently, each
    // claiming its next tile while it works on the current one, so the SIMDs
    // whose wavefronts run ahead take more of the range (a fixed
    // round-robin left one SIMD of a CU a tile more than the others)
    for (uint32_t T = t_begin + wave; T < t_end;) {
      uint32_t nx = 0;
      if (lane == 0) nx = __hip_atomic_fetch_add(next_tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      begin_tile(T);
      for (uint32_t c = 0; c < nchunks; ++c) run_chunk(WL + c * SLOT);
      irdw_store<DT, NOG, STEM>(a, BpL, acc, ok, pix, q, act_p, ResL, l16);
      T = __builtin_amdgcn_readfirstlane(nx);
    }
    return;
  }

  // streamed weights: the wavefronts walk the chunks in step (one barrier a
  // chunk), chunk number gc of the workgroup's run in slot gc & 1; the next
  // chunk's copy goes out as soon as every wavefront is done with its slot
  uint32_t gc = 0;
  for (uint32_t T0 = t_begin; T0 < t_end; T0 += nwaves) {
    const uint32_t T = T0 + wave;
    const bool active = T < t_end;  // wave-uniform
    const bool more = T0 + nwaves < t_end;
    if (active) begin_tile(T);
    for (uint32_t c = 0; c < nchunks; ++c, ++gc) {
      // chunk gc has landed (every wavefront's share) and slot (gc + 1) & 1
      // is free: every wavefront finished chunk gc - 1
      ir_dma_wait();
      __syncthreads();
      const bool last = c + 1 == nchunks;
      if (!last || more) dma_chunk(last ? 0 : c + 1, (gc + 1) & 1);
      if (active) run_chunk(WL + (gc & 1) * SLOT);
    }
    if (active) irdw_store<DT, NOG, STEM>(a, BpL, acc, ok, pix, q, act_p, ResL, l16);
  }
  ir_dma_wait();
}

template <int DT, int KE, int NPI, int NOB, bool RL>
__global__ __launch_bounds__(64 * irw_max_waves(KE, NPI, NOB))
__attribute__((amdgpu_waves_per_eu(irw_waves_per_simd(KE, NPI, NOB))))
void ir_wave_kernel(IrWaveArgs a) {
  ir_wave_body<DT, KE, NPI, NOB, RL, false>(a);
}

// The stem conv fused into the first inverted-residual block after it: the
// 32 -> 128 -> 32 stride-1 block (ReLU inside) reading the stem's output as
// its input and residual. The stem's output is never stored.
template <int DT>
__global__ __launch_bounds__(64 * irw_max_waves(2, 2, 1)) __attribute__((amdgpu_waves_per_eu(irw_waves_per_simd(2, 2, 1))))
void ir_wave_stem_kernel(IrWaveArgs a) {
  ir_wave_body<DT, 2, 2, 1, true, true>(a);
}

template <int DT, int KE, int NPI, int NOB, bool RL>
inline hipError_t irw_prepare_inst() {
  static const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(ir_wave_kernel<DT, KE, NPI, NOB, RL>),
                                                  hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
  return e;
}

template <int DT, int KE, int NPI, int NOB, bool RL>
inline hipError_t irw_launch_inst(const IrWaveArgs &a, uint32_t waves, uint32_t lds, uint32_t grid, hipStream_t st) {
  const hipError_t e = irw_prepare_inst<DT, KE, NPI, NOB, RL>();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((ir_wave_kernel<DT, KE, NPI, NOB, RL>), dim3(grid), dim3(64 * waves), lds, st, a);
  return hipGetLastError();
}

template <int DT, int KE, int NPI, int NOB, bool RL>
inline int irw_occ_inst(uint32_t waves, uint32_t lds) {
  if (irw_prepare_inst<DT, KE, NPI, NOB, RL>() != hipSuccess) return -1;
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, ir_wave_kernel<DT, KE, NPI, NOB, RL>, (int)(64 * waves),
                                                   lds) != hipSuccess)
    return -1;
  return per_cu;
}

// The (KE, NPI, NOB) combinations with an instantiation: the inverted-residual
// blocks of the MobileNet-style encoders (C = 16 KE input channels, NPI halo
// blocks: 2 for a stride-1 tile of <= 32 pixels, 5 for stride 2, NOB = COP /
// 32) and the 48 -> 96 -> 48 blocks of the converter's segmentation model.
#define AIH_IRW_SHAPES(X) X(2, 2, 1) X(2, 5, 2) X(3, 2, 2) X(4, 2, 2) X(4, 5, 3) X(6, 2, 3) X(8, 2, 4)

inline bool irw_has_shape(uint32_t ke, uint32_t npi, uint32_t nob) {
#define AIH_IRW_HAS(KE, NPI, NOB) \
  if (ke == KE && npi == NPI && nob == NOB) return true;
  AIH_IRW_SHAPES(AIH_IRW_HAS)
#undef AIH_IRW_HAS
  return false;
}

// Both inner activations ReLU: the instantiation that applies them to packed results.
inline bool irw_relu_inner(int act_e, int act_d) { return act_e == AIH_ACT_RELU && act_d == AIH_ACT_RELU; }

template <int DT>
inline hipError_t irw_launch_dt(const IrWaveArgs &a, uint32_t npi, uint32_t waves, uint32_t lds, uint32_t grid,
                                hipStream_t st) {
  const uint32_t ke = a.C / 16, nob = a.COP / 32;
  const bool rl = irw_relu_inner(a.act_e, a.act_d);
#define AIH_IRW_LAUNCH(KE, NPI, NOB)                                                          \
  if (ke == KE && npi == NPI && nob == NOB)                                                   \
    return rl ? irw_launch_inst<DT, KE, NPI, NOB, true>(a, waves, lds, grid, st)             \
              : irw_launch_inst<DT, KE, NPI, NOB, false>(a, waves, lds, grid, st);
  AIH_IRW_SHAPES(AIH_IRW_LAUNCH)
#undef AIH_IRW_LAUNCH
  return hipErrorInvalidValue;
}

template <int DT>
inline int irw_occ_dt(uint32_t ke, uint32_t npi, uint32_t nob, bool rl, uint32_t waves, uint32_t lds) {
#define AIH_IRW_OCC(KE, NPI, NOB)                                                                        \
  if (ke == KE && npi == NPI && nob == NOB)                                                              \
    return rl ? irw_occ_inst<DT, KE, NPI, NOB, true>(waves, lds) : irw_occ_inst<DT, KE, NPI, NOB, false>(waves, lds);
  AIH_IRW_SHAPES(AIH_IRW_OCC)
#undef AIH_IRW_OCC
  return 0;
}

template <int DT>
inline hipError_t irw_stem_prepare() {
  static const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(ir_wave_stem_kernel<DT>),
                                                  hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
  return e;
}

template <int DT>
inline hipError_t irw_stem_launch(const IrWaveArgs &a, uint32_t waves, uint32_t lds, uint32_t grid, hipStream_t st) {
  const hipError_t e = irw_stem_prepare<DT>();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((ir_wave_stem_kernel<DT>), dim3(grid), dim3(64 * waves), lds, st, a);
  return hipGetLastError();
}

template <int DT>
inline int irw_stem_occ(uint32_t waves, uint32_t lds) {
  if (irw_stem_prepare<DT>() != hipSuccess) return -1;
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, ir_wave_stem_kernel<DT>, (int)(64 * waves), lds) !=
      hipSuccess)
    return -1;
  return per_cu;
}

hipError_t launch_ir_wave_f16(const IrWaveArgs &a, uint32_t npi, uint32_t waves, uint32_t lds, uint32_t grid,
                              hipStream_t st);
hipError_t launch_ir_wave_stem_f16(const IrWaveArgs &a, uint32_t waves, uint32_t lds, uint32_t grid, hipStream_t st);
hipError_t launch_ir_wave_stem_bf16(const IrWaveArgs &a, uint32_t waves, uint32_t lds, uint32_t grid, hipStream_t st);
int ir_wave_stem_occ_f16(uint32_t waves, uint32_t lds);
int ir_wave_stem_occ_bf16(uint32_t waves, uint32_t lds);
hipError_t launch_ir_wave_bf16(const IrWaveArgs &a, uint32_t npi, uint32_t waves, uint32_t lds, uint32_t grid,
                               hipStream_t st);
int ir_wave_occ_f16(uint32_t ke, uint32_t npi, uint32_t nob, bool rl, uint32_t waves, uint32_t lds);
int ir_wave_occ_bf16(uint32_t ke, uint32_t npi, uint32_t nob, bool rl, uint32_t waves, uint32_t lds);

}  // namespace aih

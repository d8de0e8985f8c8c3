// ir_block_impl.h -- fused inverted-residual block for gfx950 (CDNA4).
//
// Three consecutive SwOp::Conv that the reference lowers to three separate
// dispatches (crates/ai-gpu-runtime/src/lowering.rs:122-152: GemmPwSpec,
// ConvDwSpec, GemmPwSpec) run as one kernel, so the 4x-expanded intermediate
// never leaves the CU:
//
//   e = act_e(x . We + be)            1x1 expand, C -> E      (MFMA)
//   d = act_d(dw3x3_S(e) + bd)        depthwise, stride S     (VALU, fp32)
//   y = act_p(d . Wp + bp) (+ res)    1x1 project, E -> CO    (MFMA)
//
// with each stage's arithmetic and rounding matching its unfused kernel:
// fp32 accumulation, bias -> act -> (+ residual) as in common/epilogue.rs:13-30,
// and the e and d intermediates rounded to the storage dtype exactly where the
// unfused path stores them.
//
// Work decomposition. A workgroup (4 wavefronts) owns a TH x TW tile of output
// pixels of one image and walks E in chunks of EC channels:
//   (0) the input tile with its halo, HH x HW pixels x C channels, is copied
//       to LDS once per tile (zeros outside the image);
//   (1) expand: [halo px x (C + 1)] x [(C + 1) x EC] on MFMA, in 32-pixel x
//       32-channel blocks dealt round-robin to the wavefronts, the bias being
//       the extra K row against a column that is 1 inside the image and 0
//       outside; act in the MFMA layout; halo pixels outside the image come
//       out 0 (the depthwise zero padding, not act(expand(0))) -- masked
//       explicitly only for activations with act(0) != 0; the chunk is stored
//       to LDS;
//   (2) depthwise + project: every wavefront owns NPW 32-pixel blocks of the
//       output tile. Lane l computes the depthwise output of pixel l%32 for
//       the K slice that lane l feeds to the projection MFMA, so the
//       depthwise result is the MFMA B operand directly, without a round
//       trip through LDS. The projection accumulates over all chunks in
//       registers: NPW x NOB 32x32 fp32 blocks per wavefront.
// After the last chunk: bias, act, residual and the store to HBM.
//
// MFMA operand convention (as in the conv-GEMM kernel): the weights are the A
// operand (rows = output channels), the pixels the B operand; every operand
// is one 16-byte LDS read per lane at row (l%32), K offset ks*KSTEP + (l/32)*KSTEP/2:
//   f16/bf16: v_mfma_f32_32x32x16_{f16,bf16}, KSTEP = 16, one MFMA per read;
//   fp32:     v_mfma_f32_32x32x2f32,          KSTEP = 8,  four MFMAs per read
//             (MFMA c takes component c: K = 4*(l/32) + c for both operands).
// Result lane l holds pixel l%32 and channels 8*(r/4) + 4*(l/32) + r%4.
// LDS rows are padded by 16 bytes so that 8 consecutive lanes reading 16 bytes
// of 8 consecutive rows hit 32 distinct banks.
#pragma once

#include "aih_device.h"
#include "ir_block.h"

namespace aih {

// Expanded channels per chunk.
constexpr int IR_EC = 32;

template <int DT>
__device__ __forceinline__ f32x16 ir_mma(u32x4 a, u32x4 b, f32x16 c) {
  if constexpr (DT == DT_F16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                  0, 0, 0);
  } else if constexpr (DT == DT_BF16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                   c, 0, 0, 0);
  } else {
    const f32x4 fa = __builtin_bit_cast(f32x4, a), fb = __builtin_bit_cast(f32x4, b);
#pragma unroll
    for (int k = 0; k < 4; ++k) c = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[k], fb[k], c, 0, 0, 0);
    return c;
  }
}

// 16 bytes of storage <-> HK fp32 values (HK = 8 for 16-bit, 4 for fp32).
template <int DT, int HK>
__device__ __forceinline__ void ir_unpack(u32x4 v, float (&out)[HK]) {
  if constexpr (DT == DT_F32) {
    const f32x4 f = __builtin_bit_cast(f32x4, v);
    out[0] = f.x; out[1] = f.y; out[2] = f.z; out[3] = f.w;
  } else {
    const f32x4 lo = unpack4<DT>(u32x2{v.x, v.y}), hi = unpack4<DT>(u32x2{v.z, v.w});
    out[0] = lo.x; out[1] = lo.y; out[2] = lo.z; out[3] = lo.w;
    out[4] = hi.x; out[5] = hi.y; out[6] = hi.z; out[7] = hi.w;
  }
}

template <int DT, int HK>
__device__ __forceinline__ u32x4 ir_pack(const float (&v)[HK]) {
  if constexpr (DT == DT_F32) {
    return __builtin_bit_cast(u32x4, f32x4{v[0], v[1], v[2], v[3]});
  } else {
    const u32x2 lo = pack4<DT>(f32x4{v[0], v[1], v[2], v[3]});
    const u32x2 hi = pack4<DT>(f32x4{v[4], v[5], v[6], v[7]});
    return u32x4{lo.x, lo.y, hi.x, hi.y};
  }
}

// d[j] += x[j] * w[j] for the HK channels in 16 bytes of x and of w (both in
// the storage dtype; f16 products go through v_fma_mix_f32, fp32 accumulate).
template <int DT, int HK>
__device__ __forceinline__ void ir_fma_taps(u32x4 xv, u32x4 wv, float (&d)[HK]) {
  if constexpr (DT == DT_F32) {
    const f32x4 x = __builtin_bit_cast(f32x4, xv), w = __builtin_bit_cast(f32x4, wv);
    d[0] += x.x * w.x; d[1] += x.y * w.y; d[2] += x.z * w.z; d[3] += x.w * w.w;
  } else if constexpr (DT == DT_F16) {
    const f16x8 x = __builtin_bit_cast(f16x8, xv), w = __builtin_bit_cast(f16x8, wv);
#pragma unroll
    for (int j = 0; j < HK; ++j) d[j] += (float)x[j] * (float)w[j];
  } else {
    // bf16: v_dot2c_f32_bf16 against the weight with its other half zeroed,
    // x.lo * w.lo + x.hi * 0 + d (the bf16 product is exact in fp32, so this
    // is the FMA of the widened operands) -- two instructions per channel
    // pair instead of four widenings and two FMAs
    const uint32_t xs[4] = {xv.x, xv.y, xv.z, xv.w}, ws[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bf16x2 x2 = __builtin_bit_cast(bf16x2, xs[j]);
      d[2 * j] = __builtin_amdgcn_fdot2_f32_bf16(x2, __builtin_bit_cast(bf16x2, ws[j] & 0x0000ffffu), d[2 * j], false);
      d[2 * j + 1] =
          __builtin_amdgcn_fdot2_f32_bf16(x2, __builtin_bit_cast(bf16x2, ws[j] & 0xffff0000u), d[2 * j + 1], false);
    }
  }
}

// Global -> LDS copies without registers: buffer_load_dword{,x4} ... lds
// writes lane i's SZ bytes to LDS at a wavefront-uniform base + SZ * i.
// A lane whose offset lies at or past the buffer's size writes zeros.
typedef __attribute__((address_space(3))) void ir_lds_void;
// An offset past every buffer the kernel reads (the host keeps each below 2 GiB).
constexpr uint32_t IR_OOB = 0x80000000u;
// A source offset meaning "leave this item of LDS as it is" (the lane issues nothing).
constexpr uint32_t IR_SKIP = 0xffffffffu;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t ir_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, (int)bytes, 0x00020000);
}

// Copies n items of SZ bytes to dst[0, n * SZ), item g from byte offset src(g)
// of the buffer. The four wavefronts take 64-item rows in turn, the first row
// going to wavefront w0. The copy is asynchronous: ir_dma_wait() and then a
// workgroup barrier publish it.
template <int SZ, class F>
__device__ __forceinline__ void ir_dma(char *dst, uint32_t n, __amdgpu_buffer_rsrc_t rs, int wave, int lane, int w0,
                                       F src) {
  for (uint32_t g0 = (uint32_t)((wave - w0) & 3) * 64; g0 < n; g0 += 256) {
    const uint32_t g = g0 + lane;
    const uint32_t off = g < n ? src(g) : IR_SKIP;
    if (off == IR_SKIP) continue;
    ir_lds_void *d = (ir_lds_void *)(dst + g0 * SZ);
    if constexpr (SZ == 16)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, d, 16, off, 0, 0, 0);
    else
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, d, 4, off, 0, 0, 0);
  }
}

// This wavefront's copies to LDS (and every other global load) have landed.
__device__ __forceinline__ void ir_dma_wait() { __builtin_amdgcn_s_waitcnt(0x0F70); }  // vmcnt(0)

// A weight operand of one lane: HK consecutive K of one output channel, held
// in LDS as packed groups of 4 K (pack.rs:95) -- one 16-byte group for fp32,
// two 8-byte groups `next` bytes apart for 16-bit storage.
template <int DT>
__device__ __forceinline__ u32x4 ir_ld_w(const char *p, uint32_t next) {
  if constexpr (DT == DT_F32) {
    return *reinterpret_cast<const u32x4 *>(p);
  } else {
    const u32x2 lo = *reinterpret_cast<const u32x2 *>(p), hi = *reinterpret_cast<const u32x2 *>(p + next);
    return u32x4{lo.x, lo.y, hi.x, hi.y};
  }
}

// Activation of N values: CL (all three activations of the block are
// clamp-type) applies one integer clamp per value with no branch on the mode.
template <bool CL, int N>
__device__ __forceinline__ void ir_act(const Act &p, float (&v)[N]) {
  if constexpr (CL) {
#pragma unroll
    for (int j = 0; j < N; ++j) v[j] = act_clamp_any(p, v[j]);
  } else {
    act_array<N>(p, v);
  }
}

template <int DT, int NOB, int NPW, bool CL>
__global__ __launch_bounds__(256) void ir_block_kernel(IrArgs a) {
  extern __shared__ __align__(16) char lds[];
  constexpr bool F32 = DT == DT_F32;
  constexpr int ES = F32 ? 4 : 2;       // storage bytes per element
  constexpr int KSTEP = F32 ? 8 : 16;   // K per operand read (both lane halves)
  constexpr int HK = KSTEP / 2;         // K elements in one lane's 16 bytes
  constexpr int EC = IR_EC;             // expanded channels per chunk
  constexpr int NKS = EC / KSTEP;       // projection K steps per chunk
  constexpr int RPE = EC * ES + 16;     // expanded-chunk LDS row pitch
  constexpr uint32_t GB = 4 * ES;       // bytes of one packed weight group (4 K of one channel)
  constexpr uint32_t SMB = 11 * EC * ES;  // per-chunk small tensors: 9 depthwise taps, its bias, expand bias

  const int tid = threadIdx.x;
  const int lane = tid & 63, l32 = lane & 31, lh = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  // Weight slots: resident -> one per chunk (all of E); streamed -> two,
  // chunk c in slot c & 1. Every slot holds the chunk's weights byte for byte
  // as packed by the converter:
  //   WeL [slot][C/4 groups][32 channels][GB]    expand, group kq of channel e
  //   WpL [slot][EC/4 groups][COP][GB]           project (one contiguous range;
  //                                              channels CO..COP zero)
  //   SmL [slot][11][32] x ES                    depthwise taps 0..8, depthwise bias, expand bias
  char *XL = lds + a.lds_x;    // [NPI*32][RPX]   input tile
  char *XeL = lds + a.lds_xe;  // [NPI*32][RPE]   expanded chunk
  char *WeL = lds + a.lds_we;
  char *WpL = lds + a.lds_wp;
  char *SmL = lds + a.lds_sm;
  float *BpL = reinterpret_cast<float *>(lds + a.lds_bp);  // [CO] fp32
  const uint32_t RPX = a.C * ES + 16;
  const uint32_t NVX = a.C * ES / 16;     // 16-byte vectors per input pixel
  const uint32_t nchunks = a.E / EC;
  const uint32_t nks_e = a.C / KSTEP;
  const uint32_t HPIX = a.HH * a.HW;
  const uint32_t TPIX = a.TH * a.TW;
  const uint32_t WES = EC * a.C * ES, WPS = EC * a.COP * ES;  // bytes of one slot
  const uint32_t WPG = EC * a.CO * ES;                        // a chunk's project weights in memory
  const Act act_e = act_params(a.act_e), act_d = act_params(a.act_d), act_p = act_params(a.act_p);

  const uint32_t blk = xcd_remap(blockIdx.x, gridDim.x, a.nxcd);
  const uint32_t t_begin = (uint32_t)(((uint64_t)blk * a.ntiles) / gridDim.x);
  const uint32_t t_end = (uint32_t)(((uint64_t)(blk + 1) * a.ntiles) / gridDim.x);
  if (t_begin >= t_end) return;

  const char *xg = reinterpret_cast<const char *>(a.x);
  const __amdgpu_buffer_rsrc_t rs_we = ir_rsrc(a.we, a.C * a.E * ES);
  const __amdgpu_buffer_rsrc_t rs_wp = ir_rsrc(a.wp, a.E * a.CO * ES);
  const __amdgpu_buffer_rsrc_t rs_wd = ir_rsrc(a.wd, 9 * a.E * ES);
  const __amdgpu_buffer_rsrc_t rs_bd = ir_rsrc(a.bd, a.E * ES);
  const __amdgpu_buffer_rsrc_t rs_be = ir_rsrc(a.be, a.E * ES);

  // ---- weights of chunk c (expanded channels [32c, 32c + 32)) -> slot s ----
  // Packed 1x1 weights hold element (k, n) at (k/4 * Nn + n) * 4 + k%4
  // (pack.rs:95 with one tap): the chunk's expand weights are C/4 runs of
  // 32 * GB bytes, its project weights one run of WPG bytes (EC/4 runs of CO
  // channels, each to a COP-channel row when CO < COP); depthwise weights
  // [tap][E/4][4] give 9 runs of 32 * ES bytes.
  auto dma_chunk = [&](uint32_t c, uint32_t s) {
    constexpr uint32_t GR = EC * GB / 16;  // 16-byte items per expand run
    ir_dma<16>(WeL + s * WES, (a.C / 4) * GR, rs_we, wave, lane, 0, [&](uint32_t g) -> uint32_t {
      return ((g / GR) * a.E + EC * c) * GB + (g % GR) * 16;
    });
    if (a.COP == a.CO) {
      ir_dma<16>(WpL + s * WPS, WPS / 16, rs_wp, wave, lane, 1,
                 [&](uint32_t g) -> uint32_t { return c * WPG + g * 16; });
    } else {
      const uint32_t rb = a.CO * GB;  // bytes of one K group's run
      for (uint32_t q = 0; q < EC / 4; ++q)
        ir_dma<16>(WpL + s * WPS + q * (a.COP * GB), rb / 16, rs_wp, wave, lane, (int)(q & 3),
                   [&](uint32_t g) -> uint32_t { return c * WPG + q * rb + g * 16; });
    }
    constexpr uint32_t TR = EC * ES / 16;  // 16-byte items per depthwise tap run
    char *sm = SmL + s * SMB;
    ir_dma<16>(sm, 9 * TR, rs_wd, wave, lane, 2, [&](uint32_t g) -> uint32_t {
      return ((g / TR) * a.E + EC * c) * ES + (g % TR) * 16;
    });
    // biases need only 4-byte alignment: copied 4 bytes per lane
    ir_dma<4>(sm + 9 * EC * ES, EC * ES / 4, rs_bd, wave, lane, 3,
              [&](uint32_t g) -> uint32_t { return EC * c * ES + g * 4; });
    ir_dma<4>(sm + 10 * EC * ES, EC * ES / 4, rs_be, wave, lane, 0,
              [&](uint32_t g) -> uint32_t { return EC * c * ES + g * 4; });
  };

  for (uint32_t i = tid; i < a.CO / 4; i += 256)
    *reinterpret_cast<f32x4 *>(BpL + 4 * i) = Vec4IO<DT>::load(a.bp, i);
  if (a.COP != a.CO) {
    // project weights of channels CO..COP: zero in every slot, for good (the
    // copies write only channels below CO)
    const uint32_t nslots = a.resident ? nchunks : 2u, pad16 = (a.COP - a.CO) * GB / 16;
    for (uint32_t i = tid; i < nslots * (EC / 4) * pad16; i += 256) {
      const uint32_t sq = i / pad16, v = i - sq * pad16;
      *reinterpret_cast<u32x4 *>(WpL + sq * (a.COP * GB) + a.CO * GB + v * 16) = u32x4{0u, 0u, 0u, 0u};
    }
  }
  if (a.resident)
    for (uint32_t c = 0; c < nchunks; ++c) dma_chunk(c, c);

  const uint32_t img_bytes = a.IH * a.IW * a.C * ES;
  const uint32_t per_img = a.tiles_y * a.tiles_x;
  // output origin of tile T: image, first row, first column
  auto tile_origin = [&](uint32_t T, uint32_t &img, uint32_t &ty0, uint32_t &tx0) {
    img = fdiv(T, a.fd_pi);
    const uint32_t trem = T - img * per_img;
    const uint32_t tyi = fdiv(trem, a.fd_tx);
    ty0 = tyi * a.TH;
    tx0 = (trem - tyi * a.tiles_x) * a.TW;
  };
  // (0) input tile T with halo -> XL: item g is 16 bytes of halo row
  // r = g / (NVX + 1); pixels outside the image read as zeros. The row's
  // last item (the pitch padding) is the bias column of the expand: 1.0 in
  // its first K slot for pixels inside the image, 0 outside, so the expand
  // of an outside pixel is exactly 0. Asynchronous: published by the next
  // ir_dma_wait() and barrier.
  auto load_x = [&](uint32_t T) {
    uint32_t img, ty0, tx0;
    tile_origin(T, img, ty0, tx0);
    const int32_t iy0 = (int32_t)(ty0 * a.S) - a.PT, ix0 = (int32_t)(tx0 * a.S) - a.PL;
    const __amdgpu_buffer_rsrc_t rs_x = ir_rsrc(xg + (size_t)img * img_bytes, img_bytes);
    ir_dma<16>(XL, a.NPI * 32 * (NVX + 1), rs_x, wave, lane, 0, [&](uint32_t g) -> uint32_t {
      const uint32_t r = fdiv(g, a.fd_rpx), v = g - r * (NVX + 1);
      if (v == NVX) return IR_SKIP;
      const uint32_t hy = fdiv(r, a.fd_hw), hx = r - hy * a.HW;
      const int32_t iy = iy0 + (int32_t)hy, ix = ix0 + (int32_t)hx;
      const bool in = r < HPIX && (uint32_t)iy < a.IH && (uint32_t)ix < a.IW;
      return in ? ((uint32_t)iy * a.IW + (uint32_t)ix) * (NVX * 16) + v * 16 : IR_OOB;
    });
    constexpr uint32_t ONE = F32 ? 0x3F800000u : (DT == DT_F16 ? 0x3C00u : 0x3F80u);
    for (uint32_t r = tid; r < a.NPI * 32; r += 256) {
      const uint32_t hy = fdiv(r, a.fd_hw), hx = r - hy * a.HW;
      const int32_t iy = iy0 + (int32_t)hy, ix = ix0 + (int32_t)hx;
      const bool in = r < HPIX && (uint32_t)iy < a.IH && (uint32_t)ix < a.IW;
      *reinterpret_cast<u32x4 *>(XL + r * RPX + NVX * 16) = u32x4{in ? ONE : 0u, 0u, 0u, 0u};
    }
  };

  // Pipeline across tiles: the next tile's input tile (and, streamed, its
  // first chunk's weights) are copied while the current tile's last chunk
  // runs its depthwise and projection, so a tile starts with its operands in
  // LDS. Streamed weights alternate between two slots over the workgroup's
  // whole run of chunks: chunk number gc sits in slot gc & 1.
  load_x(t_begin);
  if (!a.resident) dma_chunk(0, 0);
  uint32_t gc = 0;
  for (uint32_t T = t_begin; T < t_end; ++T) {
    uint32_t img, ty0, tx0;
    tile_origin(T, img, ty0, tx0);
    const int32_t iy0 = (int32_t)(ty0 * a.S) - a.PT, ix0 = (int32_t)(tx0 * a.S) - a.PL;

    // the tile's input (and weights) have landed; every wavefront is done
    // with the previous tile's LDS
    ir_dma_wait();
    __syncthreads();

    // LDS byte addresses of the depthwise tap rows of this wavefront's output
    // pixel blocks (the tap column and the K step add constants: immediate
    // offsets)
    uint32_t rowo[NPW][3];
    bool live[NPW];
#pragma unroll
    for (int i = 0; i < NPW; ++i) {
      const uint32_t pbo = wave + 4 * i;
      live[i] = pbo < a.NPB;
      const uint32_t op = pbo * 32 + l32;
      const bool valid = live[i] && op < TPIX;
      const uint32_t oy = valid ? fdiv(op, a.fd_tw) : 0;
      const uint32_t ox = valid ? op - oy * a.TW : 0;
      const uint32_t base = oy * a.S * a.HW + ox * a.S;
#pragma unroll
      for (int dy = 0; dy < 3; ++dy) rowo[i][dy] = a.lds_xe + (base + dy * a.HW) * RPE + lh * 16;
    }

    // (1) expand chunk c (weights in slot s) over the halo tile -> XeL
    auto expand = [&](uint32_t s) {
      // lane: channel l32 of the chunk, K groups from 2*lh (16-bit) / lh (fp32);
      // a K step advances KSTEP/4 groups = 1024 bytes
      const char *ap = WeL + s * WES + ((uint32_t)lh * (HK / 4) * EC + l32) * GB;
      const char *bes = SmL + s * SMB + 10 * EC * ES;
      for (uint32_t b = wave; b < a.NPI; b += 4) {
        const char *bp = XL + (b * 32 + l32) * RPX + lh * 16;
        // the bias as the first K step: bias of channel l32 (A) x the tile's
        // bias column (B), both in the first K slot of lane half 0
        f32x16 acc;
        {
          const u32x4 bx = *reinterpret_cast<const u32x4 *>(XL + (b * 32 + l32) * RPX + NVX * 16);
          if constexpr (F32) {
            const float bw = lh == 0 ? *reinterpret_cast<const float *>(bes + l32 * 4) : 0.0f;
            const float bo = lh == 0 ? __uint_as_float(bx.x) : 0.0f;
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(bw, bo, f32x16{}, 0, 0, 0);
          } else {
            const uint32_t bw = lh == 0 ? (uint32_t)*reinterpret_cast<const uint16_t *>(bes + l32 * 2) : 0u;
            acc = ir_mma<DT>(u32x4{bw, 0u, 0u, 0u}, lh == 0 ? bx : u32x4{0u, 0u, 0u, 0u}, f32x16{});
          }
        }
#pragma unroll 2
        for (uint32_t ks = 0; ks < nks_e; ++ks)
          acc = ir_mma<DT>(ir_ld_w<DT>(ap + ks * (KSTEP * EC * ES), EC * GB),
                           *reinterpret_cast<const u32x4 *>(bp + ks * 32), acc);
        const uint32_t r = b * 32 + l32;
        // outside pixels are 0 before the activation; only an activation with
        // act(0) != 0 needs them masked (a wave-uniform test skips blocks
        // wholly inside); clamp-type activations all have act(0) = 0
        bool mask = false, inside = true;
        if (!CL && a.mask_e) {
          const uint32_t hy = fdiv(r, a.fd_hw), hx = r - hy * a.HW;
          const int32_t iy = iy0 + (int32_t)hy, ix = ix0 + (int32_t)hx;
          inside = r < HPIX && (uint32_t)iy < a.IH && (uint32_t)ix < a.IW;
          mask = !__all(inside);
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t el = 8 * q + 4 * lh;
          float v[4] = {acc[4 * q], acc[4 * q + 1], acc[4 * q + 2], acc[4 * q + 3]};
          ir_act<CL, 4>(act_e, v);
          if (mask && !inside) v[0] = v[1] = v[2] = v[3] = 0.0f;
          if constexpr (F32)
            *reinterpret_cast<f32x4 *>(XeL + r * RPE + el * 4) = f32x4{v[0], v[1], v[2], v[3]};
          else
            *reinterpret_cast<u32x2 *>(XeL + r * RPE + el * 2) = pack4<DT>(f32x4{v[0], v[1], v[2], v[3]});
        }
      }
    };

    f32x16 acc[NPW][NOB];
#pragma unroll
    for (int i = 0; i < NPW; ++i)
#pragma unroll
      for (int o = 0; o < NOB; ++o) acc[i][o] = f32x16{};

    // output pixel of lane l32 in block i (false: outside the tile or image)
    auto out_pixel = [&](int i, size_t &pix) -> bool {
      const uint32_t pbo = wave + 4 * i;
      if (pbo >= a.NPB) return false;
      const uint32_t op = pbo * 32 + l32;
      const uint32_t oy = fdiv(op, a.fd_tw), ox = op - oy * a.TW;
      const uint32_t gy = ty0 + oy, gx = tx0 + ox;
      if (op >= TPIX || gy >= a.OH || gx >= a.OW) return false;
      pix = ((size_t)img * a.OH + gy) * a.OW + gx;
      return true;
    };

    // Chunk loop: the next chunk's streamed weights (the next tile's first
    // chunk after the last) start towards the other slot (last read by the
    // previous chunk, before the barrier that closed it), then
    // expand(c) | barrier | depthwise + project(c) | copies landed + barrier.
    for (uint32_t c = 0; c < nchunks; ++c) {
      const bool last = c + 1 == nchunks, next_tile = T + 1 < t_end;
      const uint32_t s = a.resident ? c : (gc & 1);
      if (!a.resident && (!last || next_tile)) dma_chunk(last ? 0 : c + 1, (gc + 1) & 1);
      expand(s);
      __syncthreads();
      if (last) {
        // the input tile is no longer read: the next one can land in XL
        if (next_tile) load_x(T + 1);
      }

      // (2) depthwise of chunk c straight into the projection's B operand;
      // the wavefront's pixel blocks share every K step's weight reads
      {
        const char *wdp = SmL + s * SMB + lh * 16;            // tap t at + t * EC * ES
        const char *bdp = SmL + s * SMB + 9 * EC * ES + lh * 16;
        // lane: output channel l32 of block o, K groups as in the expand
        const char *wpp = WpL + s * WPS + ((uint32_t)lh * (HK / 4) * a.COP + l32) * GB;
        const uint32_t wp_ks = KSTEP / 4 * a.COP * GB, wp_next = a.COP * GB;
        // one K step at a time (unrolled, so that every LDS offset is an
        // immediate; the scheduling barrier keeps the next step's 18 operand
        // reads below this one, which would double the live registers)
#pragma unroll 1
        for (int ks = 0; ks < NKS; ++ks) {
          u32x4 wv[9];
#pragma unroll
          for (int t = 0; t < 9; ++t) wv[t] = *reinterpret_cast<const u32x4 *>(wdp + t * (EC * ES) + ks * 32);
          float bias[HK];
          ir_unpack<DT, HK>(*reinterpret_cast<const u32x4 *>(bdp + ks * 32), bias);
          u32x4 bop[NPW];
#pragma unroll
          for (int i = 0; i < NPW; ++i) {
            if (!live[i]) continue;
            float d[HK];
#pragma unroll
            for (int j = 0; j < HK; ++j) d[j] = bias[j];
#pragma unroll
            for (int t = 0; t < 9; ++t)
              ir_fma_taps<DT, HK>(
                  *reinterpret_cast<const u32x4 *>(lds + rowo[i][t / 3] + (t % 3) * RPE + ks * 32), wv[t], d);
            ir_act<CL, HK>(act_d, d);
            bop[i] = ir_pack<DT, HK>(d);
          }
#pragma unroll
          for (int o = 0; o < NOB; ++o) {
            const u32x4 av = ir_ld_w<DT>(wpp + o * (32 * GB) + ks * wp_ks, wp_next);
#pragma unroll
            for (int i = 0; i < NPW; ++i)
              if (live[i]) acc[i][o] = ir_mma<DT>(av, bop[i], acc[i][o]);
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      }

      ++gc;
      if (!last) {
        ir_dma_wait();
        __syncthreads();
      }
    }

    // epilogue: bias -> act -> (+ residual) -> HBM (the next tile's top
    // barrier orders this tile's last LDS reads before its writes)
#pragma unroll
    for (int i = 0; i < NPW; ++i) {
      size_t pix;
      if (!out_pixel(i, pix)) continue;
#pragma unroll
      for (int o = 0; o < NOB; ++o) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t oc = o * 32 + 8 * q + 4 * lh;
          if (o == NOB - 1 && oc >= a.CO) continue;  // padding channels of the last block
          f32x4 v = f32x4{acc[i][o][4 * q], acc[i][o][4 * q + 1], acc[i][o][4 * q + 2], acc[i][o][4 * q + 3]} +
                    *reinterpret_cast<const f32x4 *>(BpL + oc);
          {
            float t[4] = {v.x, v.y, v.z, v.w};
            ir_act<CL, 4>(act_p, t);
            v = f32x4{t[0], t[1], t[2], t[3]};
          }
          const size_t vi = pix * (a.CO / 4) + oc / 4;
          if (a.has_res) v += Vec4IO<DT>::load(a.res, vi);
          Vec4IO<DT>::store(a.y, vi, v);
        }
      }
    }
  }
}

// The kernel may use up to the device's whole LDS (160 KB on gfx950).
template <int DT, int NOB, int NPW, bool CL>
inline hipError_t ir_prepare_inst() {
  static const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(ir_block_kernel<DT, NOB, NPW, CL>),
                                                  hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
  return e;
}

template <int DT, int NOB, int NPW, bool CL>
inline hipError_t ir_launch_inst(const IrArgs &a, uint32_t lds, uint32_t grid, hipStream_t st) {
  hipError_t e = ir_prepare_inst<DT, NOB, NPW, CL>();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((ir_block_kernel<DT, NOB, NPW, CL>), dim3(grid), dim3(256), lds, st, a);
  return hipGetLastError();
}

// Workgroups per CU for this instantiation at `lds` bytes of dynamic LDS
// (registers and LDS both counted by the runtime).
template <int DT, int NOB, int NPW, bool CL>
inline int ir_occ_inst(uint32_t lds) {
  if (ir_prepare_inst<DT, NOB, NPW, CL>() != hipSuccess) return -1;
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, ir_block_kernel<DT, NOB, NPW, CL>, 256, lds) !=
      hipSuccess)
    return -1;
  return per_cu;
}

// Dispatch on the projection width (NOB = COP / 32 output-channel blocks), the
// output pixel blocks per wavefront (NPW) and whether every activation is
// clamp-type.
template <int DT, bool CL>
inline hipError_t ir_launch_cl(const IrArgs &a, uint32_t lds, uint32_t grid, hipStream_t st) {
  const uint32_t nob = a.COP / 32, npw = (a.NPB + 3) / 4;
  switch (nob * 4 + npw) {
    case 1 * 4 + 1: return ir_launch_inst<DT, 1, 1, CL>(a, lds, grid, st);
    case 1 * 4 + 2: return ir_launch_inst<DT, 1, 2, CL>(a, lds, grid, st);
    case 2 * 4 + 1: return ir_launch_inst<DT, 2, 1, CL>(a, lds, grid, st);
    case 2 * 4 + 2: return ir_launch_inst<DT, 2, 2, CL>(a, lds, grid, st);
    case 3 * 4 + 1: return ir_launch_inst<DT, 3, 1, CL>(a, lds, grid, st);
    case 3 * 4 + 2: return ir_launch_inst<DT, 3, 2, CL>(a, lds, grid, st);
    case 4 * 4 + 1: return ir_launch_inst<DT, 4, 1, CL>(a, lds, grid, st);
    case 4 * 4 + 2: return ir_launch_inst<DT, 4, 2, CL>(a, lds, grid, st);
    default: return hipErrorInvalidValue;
  }
}

template <int DT>
inline hipError_t ir_launch_dt(const IrArgs &a, uint32_t lds, uint32_t grid, hipStream_t st) {
  return a.clamp_acts ? ir_launch_cl<DT, true>(a, lds, grid, st) : ir_launch_cl<DT, false>(a, lds, grid, st);
}

template <int DT, bool CL>
inline int ir_occ_cl(uint32_t nob, uint32_t npw, uint32_t lds) {
  switch (nob * 4 + npw) {
    case 1 * 4 + 1: return ir_occ_inst<DT, 1, 1, CL>(lds);
    case 1 * 4 + 2: return ir_occ_inst<DT, 1, 2, CL>(lds);
    case 2 * 4 + 1: return ir_occ_inst<DT, 2, 1, CL>(lds);
    case 2 * 4 + 2: return ir_occ_inst<DT, 2, 2, CL>(lds);
    case 3 * 4 + 1: return ir_occ_inst<DT, 3, 1, CL>(lds);
    case 3 * 4 + 2: return ir_occ_inst<DT, 3, 2, CL>(lds);
    case 4 * 4 + 1: return ir_occ_inst<DT, 4, 1, CL>(lds);
    case 4 * 4 + 2: return ir_occ_inst<DT, 4, 2, CL>(lds);
    default: return 0;
  }
}

template <int DT>
inline int ir_occ_dt(uint32_t nob, uint32_t npw, bool cl, uint32_t lds) {
  return cl ? ir_occ_cl<DT, true>(nob, npw, lds) : ir_occ_cl<DT, false>(nob, npw, lds);
}

hipError_t launch_ir_block_f32(const IrArgs &a, uint32_t lds, uint32_t grid, hipStream_t st);
hipError_t launch_ir_block_f16(const IrArgs &a, uint32_t lds, uint32_t grid, hipStream_t st);
hipError_t launch_ir_block_bf16(const IrArgs &a, uint32_t lds, uint32_t grid, hipStream_t st);
int ir_occ_f32(uint32_t nob, uint32_t npw, bool cl, uint32_t lds);
int ir_occ_f16(uint32_t nob, uint32_t npw, bool cl, uint32_t lds);
int ir_occ_bf16(uint32_t nob, uint32_t npw, bool cl, uint32_t lds);

}  // namespace aih

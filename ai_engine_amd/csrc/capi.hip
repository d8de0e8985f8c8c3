// capi.hip -- the extern "C" boundary of include/aih_conv.h.
//
// Every export validates its descriptor, never throws across the boundary
// (the reference's FFI returns VbResult 0 / -1 behind catch_unwind,
// crates/ai-ffi/src/lib.rs:45-52,130-133), and records a per-thread message
// for aih_last_error().
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <exception>
#include <initializer_list>
#include <string>
#include <utility>

#include "../../include/aih_conv.h"
#include "capi_util.h"
#include "conv_dw.h"
#include "conv_gemm_launch.h"
#include "conv_igemm_direct.h"
#include "conv_pw_direct.h"
#include "conv_pw_narrow.h"
#include "conv_pw_splitk.h"
#include "conv_pw_stream.h"
#include "conv_stem.h"
#include "ir_block.h"

std::string &aih::last_error_slot() {
  thread_local std::string msg;
  return msg;
}

namespace {

int fail(const std::string &msg) { return aih::api_fail(msg); }

template <class F>
int guarded(F &&f) {
  return aih::api_guarded(std::forward<F>(f));
}

inline uint32_t div_ceil(uint32_t a, uint32_t b) { return (a + b - 1) / b; }

bool dtype_ok(int32_t dt) { return dt == AIH_F32 || dt == AIH_F16 || dt == AIH_BF16; }

// Activation storage dt with weight storage wdt: fp32 activations take any
// weight dtype (converted to fp32 in LDS, fp32 MFMA); 16-bit activations need
// weights of the same dtype (f16 / bf16 MFMA).
bool dtype_pair_ok(int32_t dt, int32_t wdt) {
  if (!dtype_ok(dt) || !dtype_ok(wdt)) return false;
  return dt == AIH_F32 || dt == wdt;
}

size_t dsize(int32_t dt) { return dt == AIH_F32 ? 4 : 2; }

// ---------------------------------------------------------------- policy
//
// The reference's policy (gemm_pw.rs:91-102, conv_igemm.rs:201-233) splits K
// when the tile grid cannot fill its 19-core GPU and K is long enough to be
// worth cutting. Re-tuned for MI355X: 256 CUs, one 128-pixel MFMA tile per
// workgroup; split when the tile grid covers fewer than 256 CUs and K holds at
// least 16 channel groups (the reference's own kg >= 16 gate), aiming at two
// workgroups per CU, at most 32 chunks, and at least one full stage per chunk;
// a grid that splitting cannot bring there takes narrower column tiles first.
// The CU count is the current device's (aih::device_cus()).

// kg per K stage of the kernel: 16 channels for fp32, 32 for 16-bit storage.
int stage_kg(int32_t dt) { return dt == AIH_F32 ? 4 : 8; }

int pick_bn(uint32_t n4) {
  int best = 32;
  uint64_t best_cols = ~0ull;
  for (int bn : aih::kGemmBN) {
    const uint64_t cols = (uint64_t)div_ceil(n4, bn) * bn;
    if (cols < best_cols || (cols == best_cols && bn > best)) {
      best = bn;
      best_cols = cols;
    }
  }
  return best;
}

struct GemmPlan {
  int bn;
  uint32_t mtiles, ntiles, nsplit, kk_chunk;
  size_t ws;
};

int plan_gemm(uint32_t M, uint32_t N4, uint32_t KK, int32_t dt, int32_t variant, int32_t splitk,
              GemmPlan *p) {
  const uint32_t kCUs = aih::device_cus();
  if (variant != AIH_VAR_AUTO && variant != AIH_VAR_TILE && variant != AIH_VAR_SPLITK)
    return fail("variant must be AIH_VAR_AUTO, AIH_VAR_TILE or AIH_VAR_SPLITK");
  if (splitk < 0 || splitk > 64) return fail("splitk must be in [0, 64]");
  p->bn = pick_bn(N4);
  p->mtiles = div_ceil(M, aih::GEMM_BM);
  p->ntiles = div_ceil(N4, p->bn);
  const uint32_t bkg = (uint32_t)stage_kg(dt);
  // the most K chunks this call may use
  uint32_t split_cap = 1;
  if (splitk > 0) split_cap = (uint32_t)splitk;
  else if (variant == AIH_VAR_SPLITK) split_cap = 4;
  else if (variant == AIH_VAR_AUTO && KK >= 16) split_cap = std::min<uint32_t>(8, std::max<uint32_t>(KK / bkg, 1));
  if ((uint64_t)p->mtiles * p->ntiles * split_cap < 2 * kCUs) {
    // a grid that splitting K cannot bring to two workgroups per CU: narrower
    // column tiles give more workgroups, as long as the padded columns stay
    // within 25 % of the tightest fit
    const uint64_t best_cols = (uint64_t)p->ntiles * p->bn;
    uint32_t best_tiles = p->mtiles * p->ntiles;
    for (int bn : aih::kGemmBN) {
      const uint32_t nt = div_ceil(N4, bn);
      if ((uint64_t)nt * bn * 4 > best_cols * 5) continue;
      const uint32_t t = std::min<uint32_t>(p->mtiles * nt, kCUs);
      if (t > best_tiles) {
        best_tiles = t;
        p->bn = bn;
        p->ntiles = nt;
      }
    }
  }
  const uint32_t tiles = p->mtiles * p->ntiles;
  uint32_t s = 1;
  if (splitk > 0) {
    s = (uint32_t)splitk;
  } else if (variant == AIH_VAR_SPLITK) {
    s = 4;
  } else if (variant == AIH_VAR_AUTO && tiles < kCUs && KK >= 16) {
    // at most 8 chunks: more only add partial sums to write and reduce
    // (960 -> 160 at 10x18, batch 1: 15.6 us with 8 chunks, 16.9 us with 30)
    s = (2 * kCUs) / tiles;
    if (s > 8) s = 8;
    const uint32_t max_s = KK / bkg;
    if (s > max_s) s = max_s;
    if (s < 1) s = 1;
  } else if (variant == AIH_VAR_AUTO && dt == AIH_F32 && tiles < 2 * kCUs && KK >= 128) {
    // fp32 with long K (>= 512 channels, MFMA-bound) whose tiles fill the CUs
    // once but not twice: the second, partial round of workgroups idles most
    // CUs. Four K chunks make each workgroup's range at most 3/4 of a whole
    // tile's work (960 -> 160 at 10x18 b256: 360 tiles, 236 -> 215 us; two
    // chunks did not help, six and eight cost more in partial sums).
    s = 4;
  }
  if (variant == AIH_VAR_TILE && splitk > 1) return fail("AIH_VAR_TILE with splitk > 1");
  uint32_t chunk = div_ceil(KK, s);
  chunk = div_ceil(chunk, bkg) * bkg;
  p->kk_chunk = chunk;
  p->nsplit = div_ceil(KK, chunk);
  p->ws = p->nsplit > 1 ? (size_t)p->nsplit * M * N4 * sizeof(float) : 0;
  const uint64_t grid = (uint64_t)p->mtiles * p->ntiles * p->nsplit;
  if (grid > 0x7fffffffull) return fail("grid too large");
  return AIH_OK;
}

void fill_plan(const GemmPlan &g, aih_plan *out) {
  out->variant = g.nsplit > 1 ? AIH_VAR_SPLITK : AIH_VAR_TILE;
  out->splitk = g.nsplit;
  out->bm = aih::GEMM_BM;
  out->bn = (uint32_t)g.bn;
  out->grid = g.mtiles * g.ntiles * g.nsplit;
  out->ws_bytes = g.ws;
}

// Diagnostic overrides of the split-K policy, read once per process (so a
// plan stays a pure function of its descriptor within a run), as the
// reference's AI_PW_SPLITK_NG (gemm_pw.rs:112-126) and AI_RT_FORCE_DIRECT
// (lowering.rs:156-160) are:
//   AIH_PW_SPLITK=<n>     every pointwise conv with AIH_VAR_AUTO and no
//                         forced split is given n K chunks, as a forced split
//                         is: the one-dispatch split-K kernel where its shape
//                         allows, else the tiled GEMM (1 = no split); the
//                         narrow, direct, LDS one-tap and streamed routes are
//                         bypassed while it is set;
//   AIH_IGEMM_NO_SPLIT=1  KxK convs with AIH_VAR_AUTO and no forced split
//                         never split K.
int env_int_once(const char *name, int *slot, std::once_flag *once) {
  std::call_once(*once, [&] {
    const char *v = std::getenv(name);
    *slot = 0;
    if (v && *v) {
      char *end = nullptr;
      const long n = std::strtol(v, &end, 10);
      if (end && *end == 0 && n > 0 && n <= 64) *slot = (int)n;
    }
  });
  return *slot;
}

int env_pw_splitk() {
  static int v;
  static std::once_flag once;
  return env_int_once("AIH_PW_SPLITK", &v, &once);
}

bool env_igemm_no_split() {
  static int v;
  static std::once_flag once;
  return env_int_once("AIH_IGEMM_NO_SPLIT", &v, &once) == 1;
}

// Which kernel a pointwise call runs: with AIH_VAR_AUTO and no forced split,
// one output channel group goes to the one-pixel-per-thread kernel and short
// K with at most 64 output channels (same storage for activations and
// weights) to the direct MFMA kernel; everything else to the tiled GEMM.
enum { PW_TILED = 0, PW_ROWS = 1, PW_DIRECT = 2, PW_LDS = 3, PW_SPLITK = 4, PW_STREAM = 5 };

// The pointwise call as a one-tap launch of the direct 3x3 kernel (weights
// resident in LDS, activations straight into MFMA registers): what the
// register-operand kernel does not take, up to 64 output channels (256 at
// fp32, beyond 64 in groups of 64, one group per work item), a kg count in whole 16-byte
// units, 4 to 32 MFMA steps (32-256 fp32 / 64-512 16-bit channels), weights
// within LDS, and enough 32-pixel blocks (>= 2048) that the launch fills every
// CU without splitting K.
bool pw_lds_plan(const aih_pw_desc *d, aih::IgDirectArgs *a) {
  const uint32_t ku = d->dt == AIH_F32 ? 1 : 2, es = d->dt == AIH_F32 ? 4 : 2;
  const uint64_t M = (uint64_t)d->n * d->m;
  // more than 64 outputs only at fp32: at 16 bit the tiled GEMM is as fast
  // there (64 -> 256 f16 at 40x72 b64: 51.8 us tiled, 53.4 us here)
  if (d->dt != d->wdt || d->ng < 2 || d->ng * 4 > (d->dt == AIH_F32 ? 256u : 64u) || d->kg % ku ||
      M < 2048ull * 32 || M > 0xffffff00ull)
    return false;
  const uint64_t bytes = M * d->kg * 4 * es;
  if (bytes >= 0x80000000ull) return false;
  const uint32_t nu = d->kg / ku, nj = div_ceil(nu, 2);
  // at least 4 steps: the shortest instantiation has 8 (padding steps cost MFMAs)
  if (nj < 4 || aih::pw_lds_steps(nj) == 0 || aih::ig_direct_lds_bytes(1, nj, d->ng * 4) > 160u * 1024u) return false;
  std::memset(a, 0, sizeof(*a));
  a->src_bytes[0] = a->src_bytes[1] = (uint32_t)bytes;
  a->stride_u[0] = a->stride_u[1] = nu;
  a->nu[0] = nu;
  a->nj0 = a->nj = nj;
  a->taps = 1;
  a->ncg = aih::ig_direct_ncg(d->ng * 4);
  a->KGP = d->kg_pad;
  a->N4 = d->ng * 4;
  a->M = (uint32_t)M;
  a->OHW = d->m;
  a->OW = d->m;
  a->IH = 1;
  a->IW = d->m;
  a->S = 1;
  a->D = 1;
  a->nblk = (uint32_t)((M + 31) / 32);
  a->act = d->act;
  a->has_res = d->residual ? 1 : 0;
  a->nxcd = aih::device_xcds();
  a->fd_ohw = aih::make_fastdiv(d->m);
  a->fd_ow = aih::make_fastdiv(d->m);
  return true;
}

// The fp32 pointwise call on the LDS-streamed GEMM (conv_pw_stream.hip): long
// K (>= 256 channels, MFMA-bound), whole buffers within 32-bit offsets, and
// at least 8 wavefront units (32 pixels x 32 channels or two such) per CU,
// so the fine-grained grid evens out without splitting K. The tile width is
// the instantiation that pads the output channels least (the wider on ties).
bool pw_stream_plan(const aih_pw_desc *d, aih::PwStreamArgs *a, aih::PwStreamShape *shape) {
  if (d->dt != AIH_F32 || d->wdt != AIH_F32 || d->kg < 64) return false;
  const uint64_t M = (uint64_t)d->n * d->m, N4 = (uint64_t)d->ng * 4;
  const uint64_t xb = M * d->kg * 16, wb = (uint64_t)d->kg_pad * N4 * 16;
  if (xb >= 0x80000000ull || wb >= 0x80000000ull) return false;
  const aih::PwStreamShape *best = nullptr;
  uint64_t best_cols = 0;
  for (const aih::PwStreamShape &sh : aih::kPwStreamShapes) {
    const uint64_t cols = (N4 + aih::pw_stream_bn(sh) - 1) / aih::pw_stream_bn(sh) * aih::pw_stream_bn(sh);
    if (!best || cols < best_cols || (cols == best_cols && aih::pw_stream_bn(sh) > aih::pw_stream_bn(*best))) {
      best = &sh;
      best_cols = cols;
    }
  }
  const uint64_t mtiles = (M + aih::pw_stream_bm(*best) - 1) / aih::pw_stream_bm(*best);
  const uint64_t ntiles = best_cols / aih::pw_stream_bn(*best);
  if (mtiles * ntiles * best->wm * best->wn < 8ull * aih::device_cus() || mtiles * ntiles > 0x7fffffffull)
    return false;
  std::memset(a, 0, sizeof(*a));
  a->x_bytes = (uint32_t)xb;
  a->w_bytes = (uint32_t)wb;
  a->M = (uint32_t)M;
  a->KG = d->kg;
  a->N4 = (uint32_t)N4;
  a->mtiles = (uint32_t)mtiles;
  a->ntiles = (uint32_t)ntiles;
  a->act = d->act;
  a->has_res = d->residual ? 1 : 0;
  a->nxcd = aih::device_xcds();
  *shape = *best;
  return true;
}

// The split factor of a pointwise call: the descriptor's, else (AUTO only)
// the AIH_PW_SPLITK override, else 0 (the policy decides).
int32_t pw_splitk_of(const aih_pw_desc *d) {
  if (d->splitk != 0 || d->variant != AIH_VAR_AUTO) return d->splitk;
  return env_pw_splitk();
}

// Shapes the one-dispatch split-K kernel takes: same storage for activations
// and weights, whole 16-channel output blocks, at most kPwSplitkMaxM pixels.
bool pw_splitk_shape(const aih_pw_desc *d) {
  const uint64_t M = (uint64_t)d->n * d->m;
  return d->dt == d->wdt && (d->ng * 4) % 16 == 0 && M <= aih::kPwSplitkMaxM;
}

bool pw_splitk_waves_ok(int32_t w) {
  for (uint32_t v : aih::kPwSplitkWaves)
    if ((int32_t)v == w) return true;
  return false;
}

int pw_route(const aih_pw_desc *d) {
  const int32_t sk = pw_splitk_of(d);
  if (d->variant == AIH_VAR_AUTO && sk > 0)
    // a forced factor: one dispatch with that many K chunks where the shape
    // allows, else the tiled GEMM with that many chunks
    return pw_splitk_shape(d) && pw_splitk_waves_ok(sk) ? PW_SPLITK : PW_TILED;
  if (d->variant != AIH_VAR_AUTO) return PW_TILED;
  if (d->ng == 1 && d->kg <= aih::kPwNarrowMaxKG) return PW_ROWS;
  const uint32_t kmax = d->dt == AIH_F32 ? aih::kPwDirectMaxK32 : aih::kPwDirectMaxK16;
  if (d->dt == d->wdt && d->ng >= 2 && d->ng * 4 <= aih::kPwDirectMaxN4 && d->kg * 4 <= kmax) {
    // too few 32-pixel blocks to give every SIMD a wavefront: 16x16 output
    // blocks, one wavefront each, spread the same work over 4-8x more waves
    const uint64_t M = (uint64_t)d->n * d->m;
    if ((d->ng * 4) % 16 == 0 && (M + 31) / 32 < 4ull * aih::device_cus() && M <= 0xffffff00ull) return PW_SPLITK;
    return PW_DIRECT;
  }
  aih::IgDirectArgs a;
  if (pw_lds_plan(d, &a)) return PW_LDS;
  aih::PwStreamArgs sa;
  aih::PwStreamShape ss;
  if (pw_stream_plan(d, &sa, &ss)) return PW_STREAM;
  // small M, long K (the reference's kg >= 16 gate, gemm_pw.rs:91-102): the
  // tiled GEMM's 128-pixel tiles cannot fill the CUs and would split K
  // through memory; one dispatch with the split on chip instead
  const uint64_t M = (uint64_t)d->n * d->m;
  if (pw_splitk_shape(d) && d->kg >= 16 &&
      ((M + aih::GEMM_BM - 1) / aih::GEMM_BM) * ((d->ng * 4 + 31) / 32) < aih::device_cus())
    return PW_SPLITK;
  return PW_TILED;
}

// Arguments of the one-dispatch split-K kernel and its K chunks (waves).
aih::PwSplitkArgs pw_splitk_args(const aih_pw_desc *d, uint32_t *waves) {
  aih::PwSplitkArgs a;
  std::memset(&a, 0, sizeof(a));
  a.M = d->n * d->m;
  a.KG = d->kg;
  a.N4 = d->ng * 4;
  a.mblk = (a.M + 15) / 16;
  a.nblk = a.N4 / 16;
  a.steps = aih::pw_splitk_steps(d->kg, d->dt == AIH_F32);
  const int32_t sk = pw_splitk_of(d);
  *waves = sk > 0 ? (uint32_t)sk : aih::pw_splitk_waves(a.steps);
  // short K (the direct route's shapes): one wavefront per 16x16 block
  const uint32_t kmax = d->dt == AIH_F32 ? aih::kPwDirectMaxK32 : aih::kPwDirectMaxK16;
  if (sk <= 0 && d->kg * 4 <= kmax) *waves = 1;
  a.spw = (a.steps + *waves - 1) / *waves;
  a.act = d->act;
  a.has_res = d->residual ? 1 : 0;
  a.nxcd = aih::device_xcds();
  return a;
}

int run_gemm(aih::GemmArgs &a, const GemmPlan &g, int32_t dt, int32_t wdt, bool igemm, bool pair, void *ws,
             size_t ws_bytes, hipStream_t st) {
  a.mtiles = g.mtiles;
  a.ntiles = g.ntiles;
  a.nsplit = g.nsplit;
  a.ntiles_total = g.mtiles * g.ntiles * g.nsplit;
  a.kk_chunk = g.kk_chunk;
  a.fd_ntiles = aih::make_fastdiv(a.ntiles);
  a.fd_mtiles = aih::make_fastdiv(a.mtiles);
  a.fd_KG = aih::make_fastdiv(a.KG);
  a.fd_K = aih::make_fastdiv(a.K);
  a.fd_OHW = aih::make_fastdiv(a.OHW);
  a.fd_OW = aih::make_fastdiv(a.OW);
  a.partial = nullptr;
  a.nxcd = aih::device_xcds();
  if (g.nsplit > 1) {
    if (ws == nullptr || ws_bytes < g.ws)
      return fail("split-K needs a workspace of " + std::to_string(g.ws) + " bytes");
    if (reinterpret_cast<uintptr_t>(ws) % 16) return fail("workspace must be 16-byte aligned");
    a.partial = static_cast<float *>(ws);
  }
  hipError_t e = aih::launch_conv_gemm(a, dt, wdt, g.bn, igemm, pair, st);
  if (e != hipSuccess) return fail(std::string("conv_gemm launch: ") + hipGetErrorString(e));
  if (g.nsplit > 1) {
    e = aih::launch_splitk_reduce(a, dt, st);
    if (e != hipSuccess) return fail(std::string("splitk_reduce launch: ") + hipGetErrorString(e));
  }
  return AIH_OK;
}

bool aligned(const void *p, size_t a) { return reinterpret_cast<uintptr_t>(p) % a == 0; }

// ---------------------------------------------------------------- pw

int check_pw(const aih_pw_desc *d) {
  if (!d) return fail("null descriptor");
  if (d->n == 0 || d->m == 0) return fail("pw: n and m must be > 0");
  if (d->kg == 0 || d->ng == 0) return fail("pw: kg and ng must be > 0");
  if (d->kg_pad < d->kg) return fail("pw: kg_pad < kg");
  if (d->act < AIH_ACT_NONE || d->act > AIH_ACT_RECIP) return fail("pw: unknown activation");
  if (!dtype_pair_ok(d->dt, d->wdt)) return fail("pw: unsupported (dt, wdt) pair");
  if ((uint64_t)d->n * d->m > 0xffffffffull / 4) return fail("pw: too many pixels");
  if ((uint64_t)d->n * d->m * d->kg > 0xffffffffull) return fail("pw: input too large");
  return AIH_OK;
}

int plan_pw(const aih_pw_desc *d, GemmPlan *g) {
  return plan_gemm(d->n * d->m, d->ng * 4, d->kg, d->dt, d->variant, pw_splitk_of(d), g);
}

// ---------------------------------------------------------------- igemm

int igemm_out_hw(const aih_igemm_desc *d, uint32_t *oh, uint32_t *ow) {
  const uint32_t ek = d->d * (d->k - 1) + 1;
  if (d->ih + d->pad[0] + d->pad[2] < ek || d->iw + d->pad[1] + d->pad[3] < ek)
    return fail("igemm: kernel larger than the padded input");
  *oh = (d->ih + d->pad[0] + d->pad[2] - ek) / d->s + 1;
  *ow = (d->iw + d->pad[1] + d->pad[3] - ek) / d->s + 1;
  return AIH_OK;
}

int check_igemm(const aih_igemm_desc *d) {
  if (!d) return fail("null descriptor");
  if (d->n == 0 || d->ih == 0 || d->iw == 0 || d->cin == 0 || d->cout == 0)
    return fail("igemm: zero-sized dimension");
  if (d->k == 0 || d->k > 15 || d->s == 0 || d->d == 0) return fail("igemm: k must be in [1, 15], s and d > 0");
  if (d->act < AIH_ACT_NONE || d->act > AIH_ACT_RECIP) return fail("igemm: unknown activation");
  if (!dtype_pair_ok(d->dt, d->wdt)) return fail("igemm: unsupported (dt, wdt) pair");
  if (d->nsrcs > 3) return fail("igemm: at most 3 input parts (lowering.rs:177-179)");
  if (d->nsrcs > 0) {
    uint32_t csum = 0, kgsum = 0;
    for (uint32_t i = 0; i < d->nsrcs; ++i) {
      const aih_src &s = d->srcs[i];
      if (s.c == 0) return fail("igemm: empty input part");
      if (s.stride_c % 4 || s.c_off % 4) return fail("igemm: part stride_c / c_off must be multiples of 4");
      if (i + 1 < d->nsrcs && s.c % 4) return fail("igemm: only the last part may have c % 4 != 0");
      if (s.c_off + div_ceil(s.c, 4) * 4 > s.stride_c) return fail("igemm: part exceeds its pixel stride");
      csum += s.c;
      kgsum += div_ceil(s.c, 4);
    }
    if (csum != d->cin || kgsum != div_ceil(d->cin, 4)) return fail("igemm: parts do not add up to cin");
  }
  uint32_t oh, ow;
  if (igemm_out_hw(d, &oh, &ow)) return AIH_ERR;
  if ((uint64_t)d->n * oh * ow > 0xffffffffull / 4) return fail("igemm: too many output pixels");
  if ((uint64_t)d->n * d->ih * d->iw * 64 > 0xffffffffull) return fail("igemm: input too large");
  return AIH_OK;
}

// The stem kernel's arguments for a stem-route descriptor (buffers unset).
int stem_args(const aih_igemm_desc *d, uint32_t oh, uint32_t ow, aih::StemArgs *sa) {
  const uint64_t M = (uint64_t)d->n * oh * ow;
  if (M > 0xffffff00ull) return fail("igemm: too many output pixels");
  std::memset(sa, 0, sizeof(*sa));
  sa->IH = d->ih;
  sa->IW = d->iw;
  sa->OHW = oh * ow;
  sa->OW = ow;
  sa->S = d->s;
  sa->PT = (int32_t)d->pad[0];
  sa->PL = (int32_t)d->pad[1];
  sa->CO = d->cout;
  sa->KGP = 4;
  sa->M = (uint32_t)M;
  sa->nblocks = (uint32_t)((M + 31) / 32);
  sa->act = d->act;
  sa->has_res = d->residual ? 1 : 0;
  sa->fd_ohw = aih::make_fastdiv(oh * ow);
  sa->fd_ow = aih::make_fastdiv(ow);
  sa->nxcd = aih::device_xcds();
  return AIH_OK;
}

// The stem route: <= 3 input channels of a dense input, 3x3, 32 or 64 outputs.
bool igemm_is_stem(const aih_igemm_desc *d) {
  const bool dense_in = d->nsrcs == 0 || (d->nsrcs == 1 && d->srcs[0].c_off == 0 && d->srcs[0].stride_c == 4);
  return d->k == 3 && d->d == 1 && d->cin <= 3 && dense_in && d->cout % 32 == 0 && d->cout <= 64 &&
         d->variant == AIH_VAR_AUTO && d->splitk == 0 && d->dt == d->wdt;
}

int plan_igemm(const aih_igemm_desc *d, GemmPlan *g) {
  uint32_t oh, ow;
  if (igemm_out_hw(d, &oh, &ow)) return AIH_ERR;
  int32_t sk = d->splitk;
  if (d->variant == AIH_VAR_AUTO && sk == 0 && env_igemm_no_split()) sk = 1;
  return plan_gemm(d->n * oh * ow, div_ceil(d->cout, 4) * 4, d->k * d->k * div_ceil(d->cin, 4), d->dt,
                   d->variant, sk, g);
}

// The 3x3 direct kernel's arguments for an igemm call (buffers aside), or
// false when the call goes to the tiled GEMM: AIH_VAR_AUTO without a forced
// split, a 3x3 kernel, the same storage for activations and weights, at most
// 64 output channels, at most two input parts whose kg runs, pixel strides
// and offsets are whole 16-byte units (two kg for 16-bit storage), at most 10
// MFMA steps per tap, weights within LDS and every part below 2 GiB.
bool ig_direct_plan(const aih_igemm_desc *d, uint32_t oh, uint32_t ow, aih::IgDirectArgs *a) {
  if (d->variant != AIH_VAR_AUTO || d->splitk != 0 || d->k != 3 || d->dt != d->wdt) return false;
  const uint32_t n4 = div_ceil(d->cout, 4) * 4;
  if (n4 > 64) return false;
  const uint32_t nparts = d->nsrcs ? d->nsrcs : 1;
  if (nparts > 2) return false;
  const uint32_t ku = d->dt == AIH_F32 ? 1 : 2, es = d->dt == AIH_F32 ? 4 : 2;
  std::memset(a, 0, sizeof(*a));
  uint32_t kg0 = 0, nj = 0;
  for (uint32_t i = 0; i < nparts; ++i) {
    const uint32_t kgi = div_ceil(d->nsrcs ? d->srcs[i].c : d->cin, 4);
    const uint32_t stride = d->nsrcs ? d->srcs[i].stride_c / 4 : kgi;
    const uint32_t off = d->nsrcs ? d->srcs[i].c_off / 4 : 0;
    if (kgi % ku || stride % ku || off % ku) return false;
    const uint64_t bytes = (uint64_t)d->n * d->ih * d->iw * stride * 4 * es;
    if (bytes >= 0x80000000ull) return false;
    a->src_bytes[i] = (uint32_t)bytes;
    a->stride_u[i] = stride / ku;
    a->off_u[i] = off / ku;
    a->nu[i] = kgi / ku;
    a->kg_first[i] = kg0;
    kg0 += kgi;
    nj += div_ceil(a->nu[i], 2);
    if (i == 0) a->nj0 = nj;
  }
  if (nparts == 1) {
    a->src_bytes[1] = a->src_bytes[0];
    a->stride_u[1] = a->stride_u[0];
  }
  if (nj == 0 || nj > aih::kIgDirectMaxSteps || aih::ig_direct_lds_bytes(9, nj, n4) > 160u * 1024u) return false;
  a->nj = nj;
  a->taps = 9;
  a->ncg = 1;
  a->KGP = div_ceil(div_ceil(d->cin, 4), 4) * 4;
  a->N4 = n4;
  a->M = d->n * oh * ow;
  a->OHW = oh * ow;
  a->OW = ow;
  a->IH = d->ih;
  a->IW = d->iw;
  a->S = d->s;
  a->D = d->d;
  a->PT = (int32_t)d->pad[0];
  a->PL = (int32_t)d->pad[1];
  a->nblk = div_ceil(a->M, 32);
  a->act = d->act;
  a->has_res = d->residual ? 1 : 0;
  a->nxcd = aih::device_xcds();
  a->fd_ohw = aih::make_fastdiv(oh * ow);
  a->fd_ow = aih::make_fastdiv(ow);
  return true;
}

// ---------------------------------------------------------------- fused inverted-residual block

int check_ir(const aih_ir_block_desc *d, uint32_t *oh, uint32_t *ow) {
  if (!d) return fail("null descriptor");
  if (!d->n || !d->ih || !d->iw || !d->cin || !d->cexp || !d->cout) return fail("ir_block: zero-sized dimension");
  if (!dtype_ok(d->dt)) return fail("ir_block: unknown dtype");
  for (int32_t act : {d->act_expand, d->act_dw, d->act_project})
    if (act < AIH_ACT_NONE || act > AIH_ACT_RECIP) return fail("ir_block: unknown activation");
  if (d->s != 1 && d->s != 2) return fail("ir_block: depthwise stride must be 1 or 2");
  if (d->ih + d->pad[0] + d->pad[2] < 3 || d->iw + d->pad[1] + d->pad[3] < 3)
    return fail("ir_block: kernel larger than the padded input");
  *oh = (d->ih + d->pad[0] + d->pad[2] - 3) / d->s + 1;
  *ow = (d->iw + d->pad[1] + d->pad[3] - 3) / d->s + 1;
  if ((uint64_t)d->n * d->ih * d->iw * d->cin > 0xffffffffull / 4 ||
      (uint64_t)d->n * *oh * *ow * d->cout > 0xffffffffull / 4)
    return fail("ir_block: tensor too large");
  // the kernel addresses one image of x and each weight tensor with 31-bit
  // byte offsets (buffer resources)
  const uint64_t es = d->dt == AIH_F32 ? 4 : 2;
  if ((uint64_t)d->ih * d->iw * d->cin * es >= 0x80000000ull || (uint64_t)d->cin * d->cexp * es >= 0x80000000ull ||
      (uint64_t)d->cexp * d->cout * es >= 0x80000000ull)
    return fail("ir_block: image or weights of 2 GiB or more");
  return AIH_OK;
}

bool ir_clamp_acts(const aih_ir_block_desc *d) {
  return aih::act_is_clamp(d->act_expand) && aih::act_is_clamp(d->act_dw) && aih::act_is_clamp(d->act_project);
}

int plan_ir(const aih_ir_block_desc *d, uint32_t oh, uint32_t ow, aih::IrPlan *p) {
  const char *why = aih::ir_plan(d->n, d->ih, d->iw, oh, ow, d->cin, d->cexp, d->cout, d->s, d->dt,
                                 ir_clamp_acts(d), d->tile_h, d->tile_w, d->ec, d->weights, p);
  if (why) return fail(std::string("ir_block: ") + why);
  return AIH_OK;
}

// The wave or split kernel's plan, when the descriptor selects one (WAVE,
// SPLIT) or leaves the choice (AUTO) and one applies; false: the tile kernel
// runs (AUTO) or the call fails (WAVE / SPLIT, with the reason).
int plan_ir_wave(const aih_ir_block_desc *d, uint32_t oh, uint32_t ow, aih::IrWavePlan *p, bool *use) {
  *use = false;
  if (d->kernel == AIH_IR_KERNEL_TILE) return AIH_OK;
  if (d->kernel != AIH_IR_KERNEL_AUTO && d->kernel != AIH_IR_KERNEL_WAVE && d->kernel != AIH_IR_KERNEL_SPLIT)
    return fail("ir_block: unknown kernel");
  const bool forced = d->kernel != AIH_IR_KERNEL_AUTO;
  if (d->ec && d->ec != 32) {
    if (forced) return fail("ir_block: the wave and split kernels walk E in chunks of 32");
    return AIH_OK;
  }
  const char *why = aih::irw_plan(d->n, d->ih, d->iw, oh, ow, d->cin, d->cexp, d->cout, d->s, d->dt,
                                  ir_clamp_acts(d), d->act_expand == AIH_ACT_RELU && d->act_dw == AIH_ACT_RELU,
                                  d->tile_h, d->tile_w, d->weights, d->kernel, d->waves, p);
  if (why) return forced || d->waves ? fail(std::string("ir_block: ") + why) : AIH_OK;
  *use = true;
  return AIH_OK;
}

// The wave / split kernels' arguments from a block descriptor and its plan
// (buffers aside).
aih::IrWaveArgs wave_args(const aih_ir_block_desc *d, uint32_t oh, uint32_t ow, const aih::IrWavePlan &wp) {
  aih::IrWaveArgs a;
  std::memset(&a, 0, sizeof(a));
  a.N = d->n;
  a.IH = d->ih;
  a.IW = d->iw;
  a.OH = oh;
  a.OW = ow;
  a.C = d->cin;
  a.E = d->cexp;
  a.CO = d->cout;
  a.COP = aih::ir_cop(d->cout);
  a.S = d->s;
  a.PT = (int32_t)d->pad[0];
  a.PL = (int32_t)d->pad[1];
  a.TH = wp.TH;
  a.TW = wp.TW;
  a.HH = wp.HH;
  a.HW = wp.HW;
  a.tiles_y = wp.tiles_y;
  a.tiles_x = wp.tiles_x;
  a.ntiles = wp.ntiles;
  a.resident = wp.resident;
  a.act_e = d->act_expand;
  a.act_d = d->act_dw;
  a.act_p = d->act_project;
  a.has_res = d->residual ? 1 : 0;
  a.nxcd = aih::device_xcds();
  a.lds_w = wp.lds_w;
  a.lds_bp = wp.lds_bp;
  a.lds_xe = wp.lds_xe;
  a.lds_red = wp.lds_red;
  a.lds_x = wp.lds_x;
  a.lds_stem = wp.lds_stem;
  a.lds_res = wp.lds_res;
  a.lds_next = wp.lds_next;
  a.fd_hw = aih::make_fastdiv(wp.HW);
  a.fd_tw = aih::make_fastdiv(wp.TW);
  a.fd_tx = aih::make_fastdiv(wp.tiles_x);
  a.fd_pi = aih::make_fastdiv(wp.tiles_x * wp.tiles_y);
  return a;
}

// The stem-fused block: both descriptors checked against each other and the
// block planned on the stem kernel (aih_ir_block_stem_plan / _stem).
int plan_ir_stem(const aih_igemm_desc *sd, const aih_ir_block_desc *d, uint32_t *oh, uint32_t *ow,
                 aih::StemArgs *sa, aih::IrWavePlan *wp) {
  if (!sd || !d) return fail("ir_block_stem: null descriptor");
  if (check_igemm(sd) || check_ir(d, oh, ow)) return AIH_ERR;
  if (!igemm_is_stem(sd) || sd->nsrcs != 0 || sd->cin != 3 || sd->cout != 32 || sd->residual)
    return fail("ir_block_stem: the stem must be on the stem route (k 3, d 1, AUTO, splitk 0, dt == wdt) with 3 "
                "input and 32 output channels, one dense fp32 input and no residual");
  if (!aih::act_is_clamp(sd->act))
    return fail("ir_block_stem: the stem's activation must be clamp-type (none, relu, relu6, clamp01)");
  if (sd->dt != d->dt || (d->dt != AIH_F16 && d->dt != AIH_BF16))
    return fail("ir_block_stem: the stem and the block must both have f16 or both bf16 storage");
  uint32_t soh, sow;
  if (igemm_out_hw(sd, &soh, &sow)) return AIH_ERR;
  if (sd->n != d->n || soh != d->ih || sow != d->iw || d->cin != 32 || d->cout != 32 || d->s != 1 || !d->residual)
    return fail("ir_block_stem: the block must be 32 -> cexp -> 32 with a stride-1 depthwise and its input as "
                "residual, on the stem's output (same n and size)");
  if ((uint64_t)sd->n * sd->ih * sd->iw * 3 * 4 >= 0x80000000ull) return fail("ir_block_stem: image of 2 GiB or more");
  if (d->kernel != AIH_IR_KERNEL_AUTO && d->kernel != AIH_IR_KERNEL_WAVE)
    return fail("ir_block_stem: the stem-fused block runs the wave kernel");
  if (d->ec && d->ec != 32) return fail("ir_block_stem: the wave kernel walks E in chunks of 32");
  const char *why = aih::irw_plan(d->n, d->ih, d->iw, *oh, *ow, d->cin, d->cexp, d->cout, d->s, d->dt,
                                  ir_clamp_acts(d), d->act_expand == AIH_ACT_RELU && d->act_dw == AIH_ACT_RELU,
                                  d->tile_h, d->tile_w, d->weights, AIH_IR_KERNEL_WAVE, d->waves, wp, true);
  if (why) return fail(std::string("ir_block_stem: ") + why);
  return stem_args(sd, soh, sow, sa);
}

// The head-joined block: the block on the split kernel and a pointwise conv
// on the narrow route (<= 4 outputs, 16 lanes a pixel) reading its output
// (aih_ir_block_head_plan / _head).
int plan_ir_head(const aih_ir_block_desc *d, const aih_pw_desc *h, uint32_t *oh, uint32_t *ow, aih::IrWavePlan *wp) {
  if (!d || !h) return fail("ir_block_head: null descriptor");
  if (check_ir(d, oh, ow) || check_pw(h)) return AIH_ERR;
  if (d->dt != AIH_F16 && d->dt != AIH_BF16) return fail("ir_block_head: the block must have f16 or bf16 storage");
  if (h->dt != d->dt || h->wdt != d->dt) return fail("ir_block_head: the head's dt and wdt must be the block's");
  if (h->n != d->n || h->m != *oh * *ow || h->kg != d->cout / 4 || h->ng != 1 || h->residual)
    return fail("ir_block_head: the head must read the block's output (same n and pixels, kg = cout / 4) and "
                "have at most 4 outputs (ng 1) and no residual");
  if (pw_route(h) != PW_ROWS || aih::pw_narrow_group(h->kg) != 16)
    return fail("ir_block_head: the head must be on the narrow route with 16 lanes a pixel (AUTO, splitk 0, "
                "kg >= 16)");
  if (d->kernel != AIH_IR_KERNEL_AUTO && d->kernel != AIH_IR_KERNEL_SPLIT)
    return fail("ir_block_head: the head-joined block runs the split kernel");
  if (d->ec && d->ec != 32) return fail("ir_block_head: the split kernel walks E in chunks of 32");
  const char *why = aih::irw_plan(d->n, d->ih, d->iw, *oh, *ow, d->cin, d->cexp, d->cout, d->s, d->dt,
                                  ir_clamp_acts(d), d->act_expand == AIH_ACT_RELU && d->act_dw == AIH_ACT_RELU,
                                  d->tile_h, d->tile_w, d->weights, AIH_IR_KERNEL_SPLIT, d->waves, wp, false, true);
  if (why) return fail(std::string("ir_block_head: ") + why);
  return AIH_OK;
}

}  // namespace

extern "C" {

const char *aih_last_error(void) { return aih::last_error_slot().c_str(); }

const char *aih_version(void) { return "aih_conv 0.1 gfx950"; }

int aih_conv_pw_plan(const aih_pw_desc *d, aih_plan *out) {
  return guarded([&] {
    if (check_pw(d)) return AIH_ERR;
    if (!out) return fail("null plan");
    const uint64_t M = (uint64_t)d->n * d->m;
    switch (pw_route(d)) {
      case PW_ROWS: {
        // pw_narrow_group(kg) lanes per pixel: 256 / that many pixels per workgroup
        const uint32_t ppb = 256 / aih::pw_narrow_group(d->kg);
        *out = aih_plan{AIH_VAR_ROWS, 1, ppb, 4, (uint32_t)std::min<uint64_t>((M + ppb - 1) / ppb, 65535), 0};
        return AIH_OK;
      }
      case PW_SPLITK: {
        // one dispatch: 16x16 output blocks, K split across `waves`
        // wavefronts (one wavefront: K whole, reported as a direct launch)
        uint32_t waves;
        const aih::PwSplitkArgs a = pw_splitk_args(d, &waves);
        *out = aih_plan{waves > 1 ? AIH_VAR_SPLITK : AIH_VAR_DIRECT, waves, 16, 16, a.mblk * a.nblk, 0};
        return AIH_OK;
      }
      case PW_LDS: {
        aih::IgDirectArgs a;
        pw_lds_plan(d, &a);
        *out = aih_plan{AIH_VAR_DIRECT, 1, 32, aih::ig_direct_nob(a.N4) * 32u, aih::ig_direct_grid(a.nblk, a.nj, a.N4),
                        0};
        return AIH_OK;
      }
      case PW_STREAM: {
        // a tiled GEMM over the whole K (operands streamed through LDS)
        aih::PwStreamArgs a;
        aih::PwStreamShape sh;
        pw_stream_plan(d, &a, &sh);
        *out = aih_plan{AIH_VAR_TILE, 1, aih::pw_stream_bm(sh), aih::pw_stream_bn(sh), a.mtiles * a.ntiles, 0};
        return AIH_OK;
      }
      case PW_DIRECT: {
        aih::PwDirectArgs da{nullptr, nullptr, nullptr, nullptr, nullptr, (uint32_t)M, d->kg, d->ng * 4,
                             (uint32_t)((M + 31) / 32), d->act, d->residual ? 1 : 0};
        uint32_t grid = 0;
        if (aih::launch_pw_direct(da, d->dt, nullptr, &grid) != hipSuccess) return fail("pw: no direct instantiation");
        *out = aih_plan{AIH_VAR_DIRECT, 1, 32, d->ng * 4 <= 32 ? 32u : 64u, grid, 0};
        return AIH_OK;
      }
      default:
        break;
    }
    GemmPlan g;
    if (plan_pw(d, &g)) return AIH_ERR;
    fill_plan(g, out);
    return AIH_OK;
  });
}

int aih_conv_pw(const aih_pw_desc *d, const void *x, const void *w, const void *bias, const void *res, void *y,
                void *ws, size_t ws_bytes, aih_stream stream) {
  return guarded([&] {
    if (check_pw(d)) return AIH_ERR;
    if (!x || !w || !bias || !y) return fail("pw: null buffer");
    if ((d->residual != 0) != (res != nullptr)) return fail("pw: res must be given iff residual");
    if (!aligned(x, 16) || !aligned(w, 16) || !aligned(y, 16) || !aligned(bias, 8) || (res && !aligned(res, 16)))
      return fail("pw: misaligned buffer (x, w, y, res need 16 bytes, bias 8)");
    const int route = pw_route(d);
    if (route == PW_SPLITK) {
      // small M, long K: K split across the wavefronts of one workgroup,
      // reduced in LDS, one dispatch, no workspace
      uint32_t waves;
      aih::PwSplitkArgs a = pw_splitk_args(d, &waves);
      a.x = x;
      a.w = w;
      a.bias = bias;
      a.res = res;
      a.y = y;
      const hipError_t e = aih::launch_pw_splitk(a, d->dt, waves, static_cast<hipStream_t>(stream));
      return e == hipSuccess ? AIH_OK : fail(std::string("pw split-K launch: ") + hipGetErrorString(e));
    }
    if (route == PW_ROWS) {
      // at most 4 output channels: one pixel per thread on the VALU
      const uint64_t M = (uint64_t)d->n * d->m;
      if (M > 0xffffffffull) return fail("pw: too many pixels");
      aih::PwNarrowArgs na{x, w, bias, res, y, (uint32_t)M, d->kg, d->kg, d->act, d->residual ? 1 : 0};
      const hipError_t e = aih::launch_pw_narrow(na, d->dt, d->wdt, static_cast<hipStream_t>(stream));
      return e == hipSuccess ? AIH_OK : fail(std::string("pw narrow launch: ") + hipGetErrorString(e));
    }
    if (route == PW_LDS) {
      // mid-size K, <= 64 output channels: the direct kernel with one tap
      aih::IgDirectArgs a;
      pw_lds_plan(d, &a);
      a.src[0] = a.src[1] = x;
      a.w = w;
      a.bias = bias;
      a.res = res;
      a.y = y;
      const hipError_t e = aih::launch_ig_direct(a, d->dt, static_cast<hipStream_t>(stream));
      return e == hipSuccess ? AIH_OK : fail(std::string("pw lds-direct launch: ") + hipGetErrorString(e));
    }
    if (route == PW_STREAM) {
      // fp32, long K, many pixels: operands streamed through LDS by DMA
      aih::PwStreamArgs a;
      aih::PwStreamShape sh;
      pw_stream_plan(d, &a, &sh);
      a.x = x;
      a.w = w;
      a.bias = bias;
      a.res = res;
      a.y = y;
      const hipError_t e = aih::launch_pw_stream(a, sh, static_cast<hipStream_t>(stream));
      return e == hipSuccess ? AIH_OK : fail(std::string("pw stream launch: ") + hipGetErrorString(e));
    }
    if (route == PW_DIRECT) {
      // short K and at most 64 output channels: operands from memory straight
      // into MFMA registers, no LDS staging
      const uint64_t M = (uint64_t)d->n * d->m;
      if (M > 0xffffff00ull) return fail("pw: too many pixels");
      aih::PwDirectArgs da{x, w, bias, res, y, (uint32_t)M, d->kg, d->ng * 4, (uint32_t)((M + 31) / 32),
                           d->act, d->residual ? 1 : 0};
      const hipError_t e = aih::launch_pw_direct(da, d->dt, static_cast<hipStream_t>(stream));
      return e == hipSuccess ? AIH_OK : fail(std::string("pw direct launch: ") + hipGetErrorString(e));
    }
    GemmPlan g;
    if (plan_pw(d, &g)) return AIH_ERR;
    aih::GemmArgs a;
    std::memset(&a, 0, sizeof(a));
    a.src[0] = x;
    a.nparts = 1;
    a.stride_kg[0] = d->kg;
    a.w = w;
    a.bias = bias;
    a.res = res;
    a.y = y;
    a.M = d->n * d->m;
    a.OHW = d->m;
    a.OW = d->m;
    a.IH = 1;
    a.IW = d->m;
    a.K = 1;
    a.S = 1;
    a.D = 1;
    a.KG = d->kg;
    a.KGP = d->kg_pad;
    a.KK = d->kg;
    a.N4 = d->ng * 4;
    a.act = d->act;
    a.has_res = d->residual ? 1 : 0;
    // 16-byte A loads take two kg at once: needs an even kg count per pixel
    const bool pair = d->dt != AIH_F32 && d->kg % 2 == 0;
    return run_gemm(a, g, d->dt, d->wdt, false, pair, ws, ws_bytes, static_cast<hipStream_t>(stream));
  });
}

int aih_conv_igemm_plan(const aih_igemm_desc *d, aih_plan *out) {
  return guarded([&] {
    if (check_igemm(d)) return AIH_ERR;
    if (!out) return fail("null plan");
    uint32_t oh, ow;
    if (igemm_out_hw(d, &oh, &ow)) return AIH_ERR;
    if (igemm_is_stem(d)) {
      // the stem kernel: 32 pixels per wavefront, 4 wavefronts per workgroup
      aih::StemArgs sa;
      if (stem_args(d, oh, ow, &sa)) return AIH_ERR;
      uint32_t grid = 0;
      if (aih::launch_conv_stem(sa, d->dt, nullptr, &grid) != hipSuccess) return fail("igemm: no stem instantiation");
      *out = aih_plan{AIH_VAR_DIRECT, 1, 32, d->cout, grid, 0};
      return AIH_OK;
    }
    aih::IgDirectArgs da;
    if (ig_direct_plan(d, oh, ow, &da)) {
      *out = aih_plan{AIH_VAR_DIRECT, 1, 32, da.N4 <= 32 ? 32u : 64u, aih::ig_direct_grid(da.nblk, da.nj, da.N4), 0};
      return AIH_OK;
    }
    GemmPlan g;
    if (plan_igemm(d, &g)) return AIH_ERR;
    fill_plan(g, out);
    return AIH_OK;
  });
}

int aih_conv_igemm(const aih_igemm_desc *d, const void *const *inputs, const void *w, const void *bias,
                   const void *res, void *y, void *ws, size_t ws_bytes, aih_stream stream) {
  return guarded([&] {
    if (check_igemm(d)) return AIH_ERR;
    if (!inputs || !w || !bias || !y) return fail("igemm: null buffer");
    const uint32_t nin = d->nsrcs ? d->nsrcs : 1;
    for (uint32_t i = 0; i < nin; ++i) {
      if (!inputs[i]) return fail("igemm: null input part");
      if (!aligned(inputs[i], 16)) return fail("igemm: misaligned input (16 bytes)");
    }
    if ((d->residual != 0) != (res != nullptr)) return fail("igemm: res must be given iff residual");
    if (!aligned(w, 16) || !aligned(y, 16) || !aligned(bias, 8) || (res && !aligned(res, 16)))
      return fail("igemm: misaligned buffer (w, y, res need 16 bytes, bias 8)");
    uint32_t oh, ow;
    if (igemm_out_hw(d, &oh, &ow)) return AIH_ERR;
    if (igemm_is_stem(d)) {
      // the stem: <= 3 input channels, every (tap, channel) gathered into one
      // 32-deep MFMA operand
      aih::StemArgs sa;
      if (stem_args(d, oh, ow, &sa)) return AIH_ERR;
      sa.x = inputs[0];
      sa.w = w;
      sa.bias = bias;
      sa.res = res;
      sa.y = y;
      const hipError_t e = aih::launch_conv_stem(sa, d->dt, static_cast<hipStream_t>(stream));
      return e == hipSuccess ? AIH_OK : fail(std::string("conv stem launch: ") + hipGetErrorString(e));
    }
    aih::IgDirectArgs da;
    if (ig_direct_plan(d, oh, ow, &da)) {
      // 3x3 with at most 64 output channels: weights resident in LDS,
      // activations straight into MFMA registers, no barriers after the load
      for (uint32_t i = 0; i < (d->nsrcs ? d->nsrcs : 1); ++i) da.src[i] = inputs[i];
      if (!d->nsrcs || d->nsrcs == 1) da.src[1] = da.src[0];
      da.w = w;
      da.bias = bias;
      da.res = res;
      da.y = y;
      const hipError_t e = aih::launch_ig_direct(da, d->dt, static_cast<hipStream_t>(stream));
      return e == hipSuccess ? AIH_OK : fail(std::string("igemm direct launch: ") + hipGetErrorString(e));
    }
    GemmPlan g;
    if (plan_igemm(d, &g)) return AIH_ERR;
    aih::GemmArgs a;
    std::memset(&a, 0, sizeof(a));
    const uint32_t kg = div_ceil(d->cin, 4);
    if (d->nsrcs == 0) {
      a.src[0] = inputs[0];
      a.nparts = 1;
      a.stride_kg[0] = kg;
    } else {
      uint32_t kg0 = 0;
      for (uint32_t i = 0; i < d->nsrcs; ++i) {
        a.src[i] = inputs[i];
        a.part_kg[i] = kg0;
        a.stride_kg[i] = d->srcs[i].stride_c / 4;
        a.off_kg[i] = d->srcs[i].c_off / 4;
        kg0 += div_ceil(d->srcs[i].c, 4);
      }
      a.nparts = d->nsrcs;
    }
    a.w = w;
    a.bias = bias;
    a.res = res;
    a.y = y;
    a.M = d->n * oh * ow;
    a.OHW = oh * ow;
    a.OW = ow;
    a.IH = d->ih;
    a.IW = d->iw;
    a.K = d->k;
    a.S = d->s;
    a.D = d->d;
    a.PT = (int32_t)d->pad[0];
    a.PL = (int32_t)d->pad[1];
    a.KG = kg;
    a.KGP = div_ceil(kg, 4) * 4;
    a.KK = d->k * d->k * kg;
    a.N4 = div_ceil(d->cout, 4) * 4;
    a.act = d->act;
    a.has_res = d->residual ? 1 : 0;
    // 16-byte A loads take two kg at once: every (tap, part) run of kg, every
    // pixel stride and every part offset must be even
    bool pair = d->dt != AIH_F32 && kg % 2 == 0;
    for (uint32_t i = 0; i < a.nparts; ++i)
      pair = pair && a.part_kg[i] % 2 == 0 && a.stride_kg[i] % 2 == 0 && a.off_kg[i] % 2 == 0;
    return run_gemm(a, g, d->dt, d->wdt, true, pair, ws, ws_bytes, static_cast<hipStream_t>(stream));
  });
}

static int check_dw(const aih_dw_desc *d) {
  if (!d) return fail("null descriptor");
  if (d->n == 0 || d->ih == 0 || d->iw == 0 || d->c == 0) return fail("dw: zero-sized dimension");
  if (d->k == 0 || d->s == 0 || d->d == 0) return fail("dw: k, s, d must be > 0");
  if (d->act < AIH_ACT_NONE || d->act > AIH_ACT_RECIP) return fail("dw: unknown activation");
  if (!dtype_ok(d->dt)) return fail("dw: unknown dtype");
  const uint32_t ek = d->d * (d->k - 1) + 1;
  if (d->ih + d->pad[0] + d->pad[2] < ek || d->iw + d->pad[1] + d->pad[3] < ek)
    return fail("dw: kernel larger than the padded input");
  return AIH_OK;
}

int aih_conv_dw(const aih_dw_desc *d, const void *x, const void *w, const void *bias, const void *res, void *y,
                aih_stream stream) {
  return guarded([&] {
    if (check_dw(d)) return AIH_ERR;
    if (!x || !w || !bias || !y) return fail("dw: null buffer");
    if ((d->residual != 0) != (res != nullptr)) return fail("dw: res must be given iff residual");
    if (!aligned(x, 16) || !aligned(w, 16) || !aligned(y, 16) || !aligned(bias, 16) || (res && !aligned(res, 16)))
      return fail("dw: misaligned buffer (16 bytes)");
    const uint32_t ek = d->d * (d->k - 1) + 1;
    aih::DwArgs a;
    a.x = x;
    a.w = w;
    a.bias = bias;
    a.res = res;
    a.y = y;
    a.N = d->n;
    a.IH = d->ih;
    a.IW = d->iw;
    a.OH = (d->ih + d->pad[0] + d->pad[2] - ek) / d->s + 1;
    a.OW = (d->iw + d->pad[1] + d->pad[3] - ek) / d->s + 1;
    a.CG = div_ceil(d->c, 4);
    a.K = d->k;
    a.S = d->s;
    a.D = d->d;
    a.PT = (int32_t)d->pad[0];
    a.PL = (int32_t)d->pad[1];
    a.act = d->act;
    a.has_res = d->residual ? 1 : 0;
    a.nxcd = aih::device_xcds();
    if ((uint64_t)a.N * a.IH * a.IW * a.CG > 0xffffffffull || (uint64_t)a.N * a.OH * a.OW * a.CG > 0xffffffffull)
      return fail("dw: tensor too large");
    hipError_t e = aih::launch_conv_dw(a, d->dt, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return fail(std::string("conv_dw launch: ") + hipGetErrorString(e));
    return AIH_OK;
  });
}

int aih_ir_block_plan(const aih_ir_block_desc *d, aih_ir_plan *out) {
  return guarded([&] {
    uint32_t oh, ow;
    if (check_ir(d, &oh, &ow)) return AIH_ERR;
    if (!out) return fail("null plan");
    aih::IrWavePlan wp;
    bool wave;
    if (plan_ir_wave(d, oh, ow, &wp, &wave)) return AIH_ERR;
    if (wave) {
      *out = aih_ir_plan{wp.TH, wp.TW, 32, d->cexp / 32, wp.resident, wp.ntiles, wp.lds, wp.occ, wp.grid,
                         wp.split ? AIH_IR_KERNEL_SPLIT : AIH_IR_KERNEL_WAVE, wp.waves, wp.deep};
      return AIH_OK;
    }
    if (d->waves) return fail("ir_block: the tile kernel's workgroups have 4 wavefronts (waves must be 0)");
    aih::IrPlan p;
    if (plan_ir(d, oh, ow, &p)) return AIH_ERR;
    *out = aih_ir_plan{p.TH, p.TW, p.EC, d->cexp / p.EC, p.resident, p.ntiles, p.lds, p.occ, p.grid,
                       AIH_IR_KERNEL_TILE, 4, 0};
    return AIH_OK;
  });
}

int aih_ir_block(const aih_ir_block_desc *d, const void *x, const void *w_expand, const void *b_expand,
                 const void *w_dw, const void *b_dw, const void *w_project, const void *b_project, const void *res,
                 void *y, aih_stream stream) {
  return guarded([&] {
    uint32_t oh, ow;
    if (check_ir(d, &oh, &ow)) return AIH_ERR;
    if (!x || !w_expand || !b_expand || !w_dw || !b_dw || !w_project || !b_project || !y)
      return fail("ir_block: null buffer");
    if ((d->residual != 0) != (res != nullptr)) return fail("ir_block: res must be given iff residual");
    for (const void *p : {x, w_expand, w_dw, w_project, (const void *)y})
      if (!aligned(p, 16)) return fail("ir_block: misaligned buffer (x, y and weights need 16 bytes)");
    for (const void *p : {b_expand, b_dw, b_project})
      if (!aligned(p, 8)) return fail("ir_block: misaligned bias (8 bytes)");
    if (res && !aligned(res, 16)) return fail("ir_block: misaligned residual (16 bytes)");
    aih::IrWavePlan wp;
    bool wave;
    if (plan_ir_wave(d, oh, ow, &wp, &wave)) return AIH_ERR;
    if (wave) {
      aih::IrWaveArgs a = wave_args(d, oh, ow, wp);
      a.x = x;
      a.we = w_expand;
      a.be = b_expand;
      a.wd = w_dw;
      a.bd = b_dw;
      a.wp = w_project;
      a.bp = b_project;
      a.res = res;
      a.y = y;
      const hipError_t e = aih::launch_ir_wave(a, d->dt, wp, static_cast<hipStream_t>(stream));
      if (e != hipSuccess) return fail(std::string("ir_block wave launch: ") + hipGetErrorString(e));
      return AIH_OK;
    }
    if (d->waves) return fail("ir_block: the tile kernel's workgroups have 4 wavefronts (waves must be 0)");
    aih::IrPlan p;
    if (plan_ir(d, oh, ow, &p)) return AIH_ERR;
    aih::IrArgs a;
    std::memset(&a, 0, sizeof(a));
    a.x = x;
    a.we = w_expand;
    a.be = b_expand;
    a.wd = w_dw;
    a.bd = b_dw;
    a.wp = w_project;
    a.bp = b_project;
    a.res = res;
    a.y = y;
    a.N = d->n;
    a.IH = d->ih;
    a.IW = d->iw;
    a.OH = oh;
    a.OW = ow;
    a.C = d->cin;
    a.E = d->cexp;
    a.CO = d->cout;
    a.COP = aih::ir_cop(d->cout);
    a.S = d->s;
    a.PT = (int32_t)d->pad[0];
    a.PL = (int32_t)d->pad[1];
    a.TH = p.TH;
    a.TW = p.TW;
    a.HH = p.HH;
    a.HW = p.HW;
    a.NPI = p.NPI;
    a.NPB = p.NPB;
    a.EC = p.EC;
    a.resident = p.resident;
    a.tiles_y = p.tiles_y;
    a.tiles_x = p.tiles_x;
    a.ntiles = p.ntiles;
    a.act_e = d->act_expand;
    a.act_d = d->act_dw;
    a.act_p = d->act_project;
    a.has_res = d->residual ? 1 : 0;
    // activations with act(0) != 0 (the depthwise's zero padding is 0 after
    // the expand's activation, not act(0))
    a.mask_e = (d->act_expand == AIH_ACT_SIGMOID || d->act_expand == AIH_ACT_HARDSIGMOID ||
                d->act_expand == AIH_ACT_RECIP) ? 1 : 0;
    a.clamp_acts = ir_clamp_acts(d) ? 1 : 0;
    a.nxcd = aih::device_xcds();
    a.lds_x = p.lds_x;
    a.lds_xe = p.lds_xe;
    a.lds_we = p.lds_we;
    a.lds_wp = p.lds_wp;
    a.lds_sm = p.lds_sm;
    a.lds_bp = p.lds_bp;
    const uint32_t es = d->dt == AIH_F32 ? 4 : 2;
    a.fd_rpx = aih::make_fastdiv(d->cin * es / 16 + 1);
    a.fd_hw = aih::make_fastdiv(p.HW);
    a.fd_tw = aih::make_fastdiv(p.TW);
    a.fd_tx = aih::make_fastdiv(p.tiles_x);
    a.fd_pi = aih::make_fastdiv(p.tiles_x * p.tiles_y);
    hipError_t e = aih::launch_ir_block(a, d->dt, p.lds, p.grid, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return fail(std::string("ir_block launch: ") + hipGetErrorString(e));
    return AIH_OK;
  });
}

// lower_op's Conv arm (crates/ai-gpu-runtime/src/lowering.rs:122-168).
static int conv_route(const aih_conv_desc *d, aih_pw_desc *pw, aih_igemm_desc *ig, aih_dw_desc *dw) {
  if (!d) return fail("null descriptor");
  if (d->groups == 0) return fail("conv: groups must be > 0");
  if (d->groups > 1) {
    if (d->groups != d->cin || d->cin != d->cout) return fail("conv: grouped conv other than depthwise");
    if (d->kh != d->kw || d->sh != d->sw) return fail("conv: depthwise needs square k and isotropic stride");
    *dw = aih_dw_desc{d->n, d->ih, d->iw, d->cin, d->kh, d->sh, d->d, {d->pad[0], d->pad[1], d->pad[2], d->pad[3]},
                      d->act, d->residual, d->dt};
    return 2;
  }
  if (d->kh == 1 && d->kw == 1) {
    if (d->sh != 1 || d->sw != 1 || d->pad[0] || d->pad[1] || d->pad[2] || d->pad[3])
      return fail("conv: 1x1 conv with stride/pad is not supported (lowering.rs:136-140)");
    *pw = aih_pw_desc{d->n, d->ih * d->iw, div_ceil(d->cin, 4), div_ceil(d->cout, 4), d->kg_pad, d->act,
                      d->residual, d->dt, d->wdt, AIH_VAR_AUTO, 0};
    return 0;
  }
  if (d->kh != d->kw) return fail("conv: square kernels only (conv_igemm.rs:81)");
  if (d->sh != d->sw) return fail("conv: isotropic stride only (conv_igemm.rs:82)");
  std::memset(ig, 0, sizeof(*ig));
  *ig = aih_igemm_desc{d->n, d->ih, d->iw, d->cin, d->cout, d->kh, d->sh, d->d,
                       {d->pad[0], d->pad[1], d->pad[2], d->pad[3]}, d->act, d->residual, d->dt, d->wdt,
                       AIH_VAR_AUTO, 0, 0, {}};
  if (d->kg_pad != div_ceil(div_ceil(d->cin, 4), 4) * 4) return fail("conv: kg_pad must be ceil(cin/4) rounded to 4");
  return 1;
}

int aih_conv_check(const aih_conv_desc *d) {
  return guarded([&] {
    aih_pw_desc pw;
    aih_igemm_desc ig;
    aih_dw_desc dw;
    GemmPlan g;
    const int r = conv_route(d, &pw, &ig, &dw);
    if (r < 0) return AIH_ERR;
    if (r == 0) return check_pw(&pw) ? AIH_ERR : plan_pw(&pw, &g);
    if (r == 1) return check_igemm(&ig) ? AIH_ERR : plan_igemm(&ig, &g);
    return check_dw(&dw);
  });
}

int aih_conv_plan(const aih_conv_desc *d, aih_plan *out) {
  return guarded([&] {
    aih_pw_desc pw;
    aih_igemm_desc ig;
    aih_dw_desc dw;
    const int r = conv_route(d, &pw, &ig, &dw);
    if (r < 0) return AIH_ERR;
    if (!out) return fail("null plan");
    if (r == 0) return aih_conv_pw_plan(&pw, out);
    if (r == 1) return aih_conv_igemm_plan(&ig, out);
    if (check_dw(&dw)) return AIH_ERR;
    *out = aih_plan{AIH_VAR_DIRECT, 1, 0, 0, 0, 0};
    return AIH_OK;
  });
}

size_t aih_conv_workspace_size(const aih_conv_desc *d) {
  aih_pw_desc pw;
  aih_igemm_desc ig;
  aih_dw_desc dw;
  GemmPlan g;
  const int r = conv_route(d, &pw, &ig, &dw);
  if (r == 0 && !check_pw(&pw) && pw_route(&pw) != PW_TILED) return 0;
  if (r == 0 && !check_pw(&pw) && !plan_pw(&pw, &g)) return g.ws;
  if (r == 1 && !check_igemm(&ig)) {
    uint32_t oh, ow;
    aih::IgDirectArgs da;
    if (igemm_out_hw(&ig, &oh, &ow)) return 0;
    if (igemm_is_stem(&ig) || ig_direct_plan(&ig, oh, ow, &da)) return 0;
    if (!plan_igemm(&ig, &g)) return g.ws;
  }
  return 0;
}

int aih_conv(const aih_conv_desc *d, const void *x, const void *w, const void *bias, const void *res, void *y,
             void *ws, size_t ws_bytes, aih_stream stream) {
  return guarded([&] {
    aih_pw_desc pw;
    aih_igemm_desc ig;
    aih_dw_desc dw;
    const int r = conv_route(d, &pw, &ig, &dw);
    if (r < 0) return AIH_ERR;
    if (r == 0) return aih_conv_pw(&pw, x, w, bias, res, y, ws, ws_bytes, stream);
    if (r == 1) {
      const void *ins[1] = {x};
      return aih_conv_igemm(&ig, ins, w, bias, res, y, ws, ws_bytes, stream);
    }
    return aih_conv_dw(&dw, x, w, bias, res, y, stream);
  });
}

// ---------------------------------------------------------------- host packing (ai-core pack.rs)

static inline uint16_t host_f32_to_f16(float f) {
  _Float16 h = (_Float16)f;
  uint16_t b;
  std::memcpy(&b, &h, 2);
  return b;
}

static inline uint16_t host_f32_to_bf16(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

static inline float host_load(const void *p, size_t i, int32_t dt) {
  if (dt == AIH_F32) return static_cast<const float *>(p)[i];
  const uint16_t b = static_cast<const uint16_t *>(p)[i];
  if (dt == AIH_F16) {
    _Float16 h;
    std::memcpy(&h, &b, 2);
    return (float)h;
  }
  uint32_t u = (uint32_t)b << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

static inline void host_store(void *p, size_t i, float v, int32_t dt) {
  if (dt == AIH_F32) static_cast<float *>(p)[i] = v;
  else if (dt == AIH_F16) static_cast<uint16_t *>(p)[i] = host_f32_to_f16(v);
  else static_cast<uint16_t *>(p)[i] = host_f32_to_bf16(v);
}

size_t aih_nhwc_c4_bytes(uint32_t n, uint32_t h, uint32_t w, uint32_t c, int32_t dt) {
  if (!dtype_ok(dt)) return 0;
  return (size_t)n * h * w * div_ceil(c, 4) * 4 * dsize(dt);
}

// pack_nhwc (pack.rs:34-47) with the batch outermost.
int aih_pack_nhwc(const float *data, uint32_t n, uint32_t h, uint32_t w, uint32_t c, int32_t dt, void *out) {
  return guarded([&] {
    if (!data || !out || !dtype_ok(dt)) return fail("pack_nhwc: bad argument");
    const uint32_t c4 = div_ceil(c, 4) * 4;
    const size_t px = (size_t)n * h * w;
    for (size_t p = 0; p < px; ++p)
      for (uint32_t ch = 0; ch < c4; ++ch) host_store(out, p * c4 + ch, ch < c ? data[p * c + ch] : 0.0f, dt);
    return AIH_OK;
  });
}

// unpack_nhwc (pack.rs:50-64).
int aih_unpack_nhwc(const void *bytes, uint32_t n, uint32_t h, uint32_t w, uint32_t c, int32_t dt, float *out) {
  return guarded([&] {
    if (!bytes || !out || !dtype_ok(dt)) return fail("unpack_nhwc: bad argument");
    const uint32_t c4 = div_ceil(c, 4) * 4;
    const size_t px = (size_t)n * h * w;
    for (size_t p = 0; p < px; ++p)
      for (uint32_t ch = 0; ch < c; ++ch) out[p * c + ch] = host_load(bytes, p * c4 + ch, dt);
    return AIH_OK;
  });
}

// pack_weights_conv (pack.rs:68-102): OIHW -> [tap][kg_pad][ng][j][comp].
uint32_t aih_pack_weights_conv(const float *wt, uint32_t cout, uint32_t cin, uint32_t kh, uint32_t kw,
                               uint32_t kg_align, int32_t dt, void *out) {
  if (!wt || !out || !dtype_ok(dt) || !cout || !cin || !kh || !kw) {
    aih::last_error_slot() = "pack_weights_conv: bad argument";
    return 0;
  }
  const uint32_t al = kg_align ? kg_align : 1;
  const uint32_t kg = div_ceil(div_ceil(cin, 4), al) * al;
  const uint32_t ng = div_ceil(cout, 4);
  for (uint32_t t = 0; t < kh * kw; ++t) {
    const uint32_t ky = t / kw, kx = t % kw;
    for (uint32_t g = 0; g < kg; ++g)
      for (uint32_t o = 0; o < ng; ++o)
        for (uint32_t j = 0; j < 4; ++j)
          for (uint32_t comp = 0; comp < 4; ++comp) {
            const uint32_t oc = o * 4 + j, ic = g * 4 + comp;
            const float v = (oc < cout && ic < cin) ? wt[(((size_t)oc * cin + ic) * kh + ky) * kw + kx] : 0.0f;
            host_store(out, ((((size_t)t * kg + g) * ng + o) * 4 + j) * 4 + comp, v, dt);
          }
  }
  return kg;
}

// pack_weights_dw (pack.rs:105-122): [c][kh][kw] -> [tap][cg][comp].
int aih_pack_weights_dw(const float *wt, uint32_t c, uint32_t kh, uint32_t kw, int32_t dt, void *out) {
  return guarded([&] {
    if (!wt || !out || !dtype_ok(dt)) return fail("pack_weights_dw: bad argument");
    const uint32_t cg = div_ceil(c, 4), taps = kh * kw;
    for (uint32_t g = 0; g < cg; ++g)
      for (uint32_t t = 0; t < taps; ++t)
        for (uint32_t comp = 0; comp < 4; ++comp) {
          const uint32_t ch = g * 4 + comp;
          host_store(out, ((size_t)t * cg + g) * 4 + comp, ch < c ? wt[(size_t)ch * taps + t] : 0.0f, dt);
        }
    return AIH_OK;
  });
}

// pack_bias (pack.rs:178-184).
int aih_pack_bias(const float *b, uint32_t cout, int32_t dt, void *out) {
  return guarded([&] {
    if (!b || !out || !dtype_ok(dt)) return fail("pack_bias: bad argument");
    const uint32_t n4 = div_ceil(cout, 4) * 4;
    for (uint32_t i = 0; i < n4; ++i) host_store(out, i, i < cout ? b[i] : 0.0f, dt);
    return AIH_OK;
  });
}

int aih_pack_nhwc_device(const float *x, uint32_t n, uint32_t h, uint32_t w, uint32_t c, int32_t dt, void *y,
                         aih_stream stream) {
  return guarded([&] {
    if (!x || !y || !dtype_ok(dt) || !n || !h || !w || !c) return fail("pack_nhwc_device: bad argument");
    if (!aligned(y, 8) || !aligned(x, 4)) return fail("pack_nhwc_device: misaligned buffer");
    hipError_t e = aih::launch_pack_nhwc(x, (uint64_t)n * h * w, c, dt, y, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return fail(std::string("pack_nhwc launch: ") + hipGetErrorString(e));
    return AIH_OK;
  });
}

int aih_conv_stem_f32in(const aih_igemm_desc *d, const float *x, const void *w, const void *bias,
                        const void *res, void *y, aih_stream stream) {
  return guarded([&] {
    if (check_igemm(d)) return AIH_ERR;
    if (!igemm_is_stem(d) || d->nsrcs != 0)
      return fail("stem_f32in: the descriptor is not on the stem route (k 3, d 1, cin <= 3, cout 32 / 64, "
                  "one dense input, AUTO, splitk 0, dt == wdt)");
    if (!x || !w || !bias || !y) return fail("stem_f32in: null buffer");
    if ((d->residual != 0) != (res != nullptr)) return fail("stem_f32in: res must be given iff residual");
    if (!aligned(x, 4) || !aligned(w, 16) || !aligned(y, 16) || !aligned(bias, 8) || (res && !aligned(res, 16)))
      return fail("stem_f32in: misaligned buffer (x needs 4 bytes, w, y, res 16, bias 8)");
    const uint64_t xb = (uint64_t)d->n * d->ih * d->iw * d->cin * 4;
    if (xb >= 0x80000000ull) return fail("stem_f32in: input of 2 GiB or more");
    uint32_t oh, ow;
    if (igemm_out_hw(d, &oh, &ow)) return AIH_ERR;
    aih::StemArgs sa;
    if (stem_args(d, oh, ow, &sa)) return AIH_ERR;
    sa.x = x;
    sa.cin_f32 = d->cin;
    sa.x_bytes = (uint32_t)xb;
    sa.w = w;
    sa.bias = bias;
    sa.res = res;
    sa.y = y;
    const hipError_t e = aih::launch_conv_stem(sa, d->dt, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? AIH_OK : fail(std::string("conv stem launch: ") + hipGetErrorString(e));
  });
}

int aih_ir_block_head_plan(const aih_ir_block_desc *blk, const aih_pw_desc *head, aih_ir_plan *out) {
  return guarded([&] {
    uint32_t oh, ow;
    aih::IrWavePlan wp;
    if (plan_ir_head(blk, head, &oh, &ow, &wp)) return AIH_ERR;
    if (!out) return fail("null plan");
    *out = aih_ir_plan{wp.TH, wp.TW, 32, blk->cexp / 32, wp.resident, wp.ntiles, wp.lds, wp.occ, wp.grid,
                       AIH_IR_KERNEL_SPLIT, wp.waves, wp.deep};
    return AIH_OK;
  });
}

int aih_ir_block_head(const aih_ir_block_desc *blk, const aih_pw_desc *head, const void *x, const void *w_expand,
                      const void *b_expand, const void *w_dw, const void *b_dw, const void *w_project,
                      const void *b_project, const void *res, void *y, const void *w_head, const void *b_head,
                      void *y_head, aih_stream stream) {
  return guarded([&] {
    uint32_t oh, ow;
    aih::IrWavePlan wp;
    if (plan_ir_head(blk, head, &oh, &ow, &wp)) return AIH_ERR;
    if (!x || !w_expand || !b_expand || !w_dw || !b_dw || !w_project || !b_project || !w_head || !b_head || !y_head)
      return fail("ir_block_head: null buffer");
    if ((blk->residual != 0) != (res != nullptr)) return fail("ir_block_head: res must be given iff residual");
    for (const void *p : {x, w_expand, w_dw, w_project, w_head, (const void *)y_head})
      if (!aligned(p, 16)) return fail("ir_block_head: misaligned buffer (x, y, y_head and weights need 16 bytes)");
    if (y && !aligned(y, 16)) return fail("ir_block_head: misaligned buffer (x, y, y_head and weights need 16 bytes)");
    for (const void *p : {b_expand, b_dw, b_project, b_head})
      if (!aligned(p, 8)) return fail("ir_block_head: misaligned bias (8 bytes)");
    if (res && !aligned(res, 16)) return fail("ir_block_head: misaligned residual (16 bytes)");
    aih::IrWaveArgs a = wave_args(blk, oh, ow, wp);
    a.x = x;
    a.we = w_expand;
    a.be = b_expand;
    a.wd = w_dw;
    a.bd = b_dw;
    a.wp = w_project;
    a.bp = b_project;
    a.res = res;
    a.y = y;
    a.hw = w_head;
    a.hb = b_head;
    a.hy = y_head;
    a.act_h = head->act;
    a.lds_head = wp.lds_head;
    const hipError_t e = aih::launch_ir_wave(a, blk->dt, wp, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? AIH_OK : fail(std::string("ir_block_head launch: ") + hipGetErrorString(e));
  });
}

int aih_ir_block_stem_plan(const aih_igemm_desc *stem, const aih_ir_block_desc *blk, aih_ir_plan *out) {
  return guarded([&] {
    uint32_t oh, ow;
    aih::StemArgs sa;
    aih::IrWavePlan wp;
    if (plan_ir_stem(stem, blk, &oh, &ow, &sa, &wp)) return AIH_ERR;
    if (!out) return fail("null plan");
    *out = aih_ir_plan{wp.TH, wp.TW, 32, blk->cexp / 32, wp.resident, wp.ntiles, wp.lds, wp.occ, wp.grid,
                       AIH_IR_KERNEL_WAVE, wp.waves, 0};
    return AIH_OK;
  });
}

int aih_ir_block_stem(const aih_igemm_desc *stem, const aih_ir_block_desc *blk, const float *image,
                      const void *w_stem, const void *b_stem, const void *w_expand, const void *b_expand,
                      const void *w_dw, const void *b_dw, const void *w_project, const void *b_project, void *y,
                      aih_stream stream) {
  return guarded([&] {
    uint32_t oh, ow;
    aih::StemArgs sa;
    aih::IrWavePlan wp;
    if (plan_ir_stem(stem, blk, &oh, &ow, &sa, &wp)) return AIH_ERR;
    if (!image || !w_stem || !b_stem || !w_expand || !b_expand || !w_dw || !b_dw || !w_project || !b_project || !y)
      return fail("ir_block_stem: null buffer");
    if (!aligned(image, 4)) return fail("ir_block_stem: misaligned image (4 bytes)");
    for (const void *p : {w_stem, w_expand, w_dw, w_project, (const void *)y})
      if (!aligned(p, 16)) return fail("ir_block_stem: misaligned buffer (y and weights need 16 bytes)");
    for (const void *p : {b_stem, b_expand, b_dw, b_project})
      if (!aligned(p, 8)) return fail("ir_block_stem: misaligned bias (8 bytes)");
    aih::IrWaveArgs a = wave_args(blk, oh, ow, wp);
    a.we = w_expand;
    a.be = b_expand;
    a.wd = w_dw;
    a.bd = b_dw;
    a.wp = w_project;
    a.bp = b_project;
    a.y = y;
    a.sx = image;
    a.sw = w_stem;
    a.sb = b_stem;
    a.SIH = stem->ih;
    a.SIW = stem->iw;
    a.SS = stem->s;
    a.SPT = sa.PT;
    a.SPL = sa.PL;
    a.act_s = stem->act;
    a.sx_bytes = (uint32_t)((uint64_t)stem->n * stem->ih * stem->iw * 3 * 4);
    const hipError_t e = aih::launch_ir_wave_stem(a, blk->dt, wp, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? AIH_OK : fail(std::string("ir_block_stem launch: ") + hipGetErrorString(e));
  });
}

}  // extern "C"

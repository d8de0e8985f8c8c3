// sw_model.hip -- a .sw model resident on the GPU (include/aih_model.h), the
// native counterpart of ai_gpu_runtime::Model (crates/ai-gpu-runtime/src/model.rs).
//
// Load (Model::load, model.rs:56-366): parse the container and graph, put the
// weight blob on the device once (converted to 16-bit storage when asked),
// give every tensor that is not an alias its own NHWC-C4 buffer with the
// batch outermost (aliases are views: the backing buffer plus a channel-group
// offset, model.rs:29-35,300-307), and lower every op to a launch closure
// with its descriptor built once (lower_op, lowering.rs:88-516). Conv ops go
// through the conv entry points of aih_conv.h exactly as the op-level boundary
// routes them; the other op kinds through aih_model.h's op entry points.
// The converter has already decided its fusions (conv + act + residual),
// topological order and liveness (format/model.rs:1-9); the runtime keeps one
// buffer per tensor (HBM is not the constraint at these sizes). On top of
// that, one graph rewrite of its own: each inverted-residual block (1x1
// expand -> depthwise 3x3 -> 1x1 project whose intermediates nothing else
// reads) becomes one aih_ir_block launch, its intermediates never stored.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <array>
#include <set>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "../../include/aih_model.h"
#include "aih_device.h"
#include "capi_util.h"
#include "sw_format.h"

namespace aih {
namespace {

size_t es_of(int32_t dt) { return dt == AIH_F32 ? 4 : 2; }
uint32_t c4(uint32_t c) { return (c + 3) / 4 * 4; }

// f32 -> f16 / bf16 bits, round to nearest even (IEEE 754; the half crate's
// from_f32 used by pack.rs:16-31 rounds the same way). NaN stays NaN.
uint16_t f32_to_f16_bits(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);  // rounds to >= 65520: inf
  if (ax < 0x38800000u) {                                    // below the f16 normal range
    if (ax < 0x33000000u) return (uint16_t)sign;             // below half the smallest subnormal
    const uint32_t e = ax >> 23, m = (ax & 0x7fffffu) | 0x800000u;
    const uint32_t shift = 126 - e;                          // 14..24
    uint32_t v = m >> shift;
    const uint32_t rem = m & ((1u << shift) - 1), half = 1u << (shift - 1);
    if (rem > half || (rem == half && (v & 1u))) ++v;
    return (uint16_t)(sign | v);
  }
  uint32_t v = ((ax >> 13) - (112u << 10));
  const uint32_t rem = ax & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (v & 1u))) ++v;
  return (uint16_t)(sign | v);
}

uint16_t f32_to_bf16_bits(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
  x += 0x7fffu + ((x >> 16) & 1u);
  return (uint16_t)(x >> 16);
}

float f16_bits_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  uint32_t x;
  if (e == 0) {
    if (m == 0) {
      x = sign;
    } else {  // subnormal: normalise
      e = 113;
      while (!(m & 0x400u)) {
        m <<= 1;
        --e;
      }
      x = sign | (e << 23) | ((m & 0x3ffu) << 13);
    }
  } else if (e == 31) {
    x = sign | 0x7f800000u | (m << 13);
  } else {
    x = sign | ((e + 112) << 23) | (m << 13);
  }
  float f;
  std::memcpy(&f, &x, 4);
  return f;
}

float bf16_bits_to_f32(uint16_t h) {
  const uint32_t x = (uint32_t)h << 16;
  float f;
  std::memcpy(&f, &x, 4);
  return f;
}

int hip_fail(const char *what, hipError_t e) { return api_fail(std::string(what) + ": " + hipGetErrorString(e)); }

// A JSON string literal of s (quotes, backslashes and control characters escaped).
std::string json_quote(const std::string &s) {
  std::string o = "\"";
  for (unsigned char ch : s) {
    if (ch == '"' || ch == '\\') {
      o.push_back('\\');
      o.push_back((char)ch);
    } else if (ch < 0x20) {
      char b[8];
      std::snprintf(b, sizeof(b), "\\u%04x", ch);
      o += b;
    } else {
      o.push_back((char)ch);
    }
  }
  return o + "\"";
}

}  // namespace
}  // namespace aih

using namespace aih;

struct aih_model {
  sw::Model g;
  uint32_t n = 1;
  int32_t dt = AIH_F32, wdt = AIH_F32;
  std::vector<void *> allocs;
  char *wdev = nullptr;                      // weights on the device
  std::map<uint64_t, uint64_t> woff;         // blob offset -> device offset (identity unless converted)
  int32_t blob_dt = AIH_F32;                 // storage of the blob's float data before conversion
  struct View {
    char *base = nullptr;  // backing buffer
    size_t bytes = 0;      // backing buffer size
    uint32_t stride_c = 0; // channels per pixel of the backing buffer
    uint32_t c_off = 0;    // first channel of the view
  };
  std::vector<View> views;                   // per tid
  void *ws = nullptr;
  size_t ws_bytes = 0;
  float *staging = nullptr;
  size_t staging_floats = 0;
  std::vector<std::function<int(hipStream_t)>> launches;  // per op; empty for a fused block's later ops
  size_t device_bytes = 0;
  uint32_t flags = 0;
  struct Fused {
    uint32_t first;  // ops first .. first + nops - 1
    uint32_t nops;   // 3: inverted-residual block (d, plan); 2: depthwise -> pointwise pair (dp, dpp)
                     // or a resize folded into the concat after it; 4: the stem conv and the block
                     // after it (sd, d, plan: aih_ir_block_stem), or a block and the head after it
    aih_ir_block_desc d;
    aih_ir_plan plan;
    aih_dwpw_desc dp;
    aih_dwpw_plan dpp;
    aih_igemm_desc sd;
    int32_t kind = AIH_FUSED_IR_BLOCK;  // enum aih_fused_kind
  };
  std::vector<Fused> fused;
  std::vector<int32_t> block_of;  // per op: its fused block, or -1
  std::vector<int32_t> internal;  // per tensor: first op of the fused block it stays inside, or -1
  // A stem conv that is the graph's single input's only reader reads the
  // uploaded logical NHWC fp32 values from `staging` itself
  // (aih_conv_stem_f32in: the pack and the conv in one launch, the same
  // result bit for bit). staged: the input's values sit in staging and its
  // NHWC-C4 slot is stale until settle_input packs it.
  int64_t stem_op = -1;
  uint32_t stem_tid = 0;
  bool staged = false;

  ~aih_model() {
    for (void *p : allocs) (void)hipFree(p);
  }

  void *dalloc(size_t bytes) {
    void *p = nullptr;
    const hipError_t e = hipMalloc(&p, bytes ? bytes : 16);
    if (e != hipSuccess) throw std::runtime_error(std::string("hipMalloc: ") + hipGetErrorString(e));
    allocs.push_back(p);
    device_bytes += bytes;
    return p;
  }

  int64_t find(const char *name) const {
    if (!name) return -1;
    for (size_t i = 0; i < g.tensors.size(); ++i)
      if (g.tensors[i].name == name) return (int64_t)i;
    return -1;
  }

  bool dense(uint32_t tid) const {
    const View &v = views[tid];
    return v.c_off == 0 && v.stride_c == c4(g.tensors[tid].c);
  }
  void *ptr(uint32_t tid) const { return views[tid].base + (size_t)views[tid].c_off * es_of(dt); }
  const void *wptr(const sw::WRef &r) const {
    auto it = woff.find(r.off);
    if (it == woff.end()) throw std::runtime_error("weight reference not prepared");
    return wdev + it->second;
  }
  aih_src src_of(uint32_t tid, uint32_t c) const {
    const View &v = views[tid];
    return aih_src{c, v.stride_c, v.c_off};
  }
  // fails for a tensor that stays inside a fused block (never stored)
  void need_stored(uint32_t tid, const char *what) const {
    if (internal[tid] >= 0) {
      const Fused &f = fused[(size_t)block_of[(size_t)internal[tid]]];
      throw std::runtime_error(std::string(what) + ": tensor '" + g.tensors[tid].name +
                               "' stays inside the fused block of ops " + std::to_string(f.first) + ".." +
                               std::to_string(f.first + f.nops - 1) + " (load with AIH_MODEL_NO_FUSE to keep it)");
    }
  }
};

namespace {

// Weight blob -> device. Every WRef the ops use must lie inside the blob; with
// a dtype change its fp32 elements are converted one by one (the packed
// layouts index elements, so the layout is unchanged at the new size).
void prepare_weights(aih_model *m, const sw::Container &c) {
  std::vector<sw::WRef> refs;
  for (const sw::Op &op : m->g.ops) {
    if (op.kind == sw::OP_CONV) refs.push_back(op.w), refs.push_back(op.b);
    if (op.kind == sw::OP_BINARY && op.opnd == sw::OPND_CVEC) refs.push_back(op.cvec);
  }
  for (const sw::WRef &r : refs)
    if (r.off > c.blob_len || r.len > c.blob_len - r.off) throw sw::Error(".sw: weight reference outside the blob");
  const bool convert = m->blob_dt == AIH_F32 && m->dt != AIH_F32;
  if (!convert) {
    m->wdev = static_cast<char *>(m->dalloc(c.blob_len));
    if (c.blob_len) {
      const hipError_t e = hipMemcpy(m->wdev, c.blob, c.blob_len, hipMemcpyHostToDevice);
      if (e != hipSuccess) throw std::runtime_error(std::string("weights upload: ") + hipGetErrorString(e));
    }
    for (const sw::WRef &r : refs) m->woff[r.off] = r.off;
    return;
  }
  std::vector<uint8_t> host;
  for (const sw::WRef &r : refs) {
    if (m->woff.count(r.off)) continue;
    if (r.len % 4) throw sw::Error(".sw: fp32 weight reference with a length not a multiple of 4");
    const size_t off = (host.size() + 255) / 256 * 256;
    const size_t cnt = r.len / 4;
    host.resize(off + cnt * 2);
    for (size_t i = 0; i < cnt; ++i) {
      float f;
      std::memcpy(&f, c.blob + r.off + i * 4, 4);
      const uint16_t h = m->dt == AIH_F16 ? f32_to_f16_bits(f) : f32_to_bf16_bits(f);
      std::memcpy(&host[off + i * 2], &h, 2);
    }
    m->woff[r.off] = off;
  }
  m->wdev = static_cast<char *>(m->dalloc(host.size()));
  if (!host.empty()) {
    const hipError_t e = hipMemcpy(m->wdev, host.data(), host.size(), hipMemcpyHostToDevice);
    if (e != hipSuccess) throw std::runtime_error(std::string("weights upload: ") + hipGetErrorString(e));
  }
}

void alloc_tensors(aih_model *m) {
  const size_t es = es_of(m->dt);
  const auto &T = m->g.tensors;
  m->views.assign(T.size(), aih_model::View{});
  size_t total = 0;
  std::vector<size_t> off(T.size(), 0);
  for (size_t i = 0; i < T.size(); ++i) {
    if (T[i].alias_of >= 0 || m->internal[i] >= 0) continue;
    off[i] = total;
    total += ((size_t)m->n * T[i].h * T[i].w * c4(T[i].c) * es + 255) / 256 * 256;
  }
  char *arena = static_cast<char *>(m->dalloc(total));
  const hipError_t e = hipMemset(arena, 0, total ? total : 16);
  if (e != hipSuccess) throw std::runtime_error(std::string("tensor arena clear: ") + hipGetErrorString(e));
  for (size_t i = 0; i < T.size(); ++i) {
    if (T[i].alias_of >= 0 || m->internal[i] >= 0) continue;
    m->views[i] = aih_model::View{arena + off[i], (size_t)m->n * T[i].h * T[i].w * c4(T[i].c) * es, c4(T[i].c), 0};
  }
  for (size_t i = 0; i < T.size(); ++i) {
    if (T[i].alias_of < 0) continue;
    const auto r = m->g.resolve((uint32_t)i);
    const auto &B = T[r.first];
    aih_model::View v = m->views[r.first];
    v.c_off = r.second * 4;
    if (T[i].h != B.h || T[i].w != B.w || v.c_off + T[i].c > v.stride_c)
      throw sw::Error(".sw: alias '" + T[i].name + "' does not fit inside '" + B.name + "'");
    m->views[i] = v;
  }
}

// Every op's geometry against the tensors and weight ranges the file declares,
// before any device work: the kernels index their buffers by the op's own
// fields, so a mismatched file must not reach them (the reference's wgpu
// runtime gets bounds-checked buffers; here the arena and the weight blob are
// plain device memory). Weight lengths are in the file's element size:
// dt_weights for the packed std-conv weights, dt_default for depthwise
// weights, biases and constant channel vectors (format/model.rs:245-254).
void validate_geometry(const sw::Model &g) {
  const auto &T = g.tensors;
  const uint64_t es_d = g.dt_default == sw::F16 ? 2 : 4, es_w = g.dt_weights == sw::F16 ? 2 : 4;
  auto c4u = [](uint64_t c) { return (c + 3) / 4 * 4; };
  for (size_t k = 0; k < g.ops.size(); ++k) {
    const sw::Op &op = g.ops[k];
    const std::string at = ".sw: op " + std::to_string(k) + ": ";
    auto shape = [&](uint32_t tid) {
      return T[tid].name + " " + std::to_string(T[tid].h) + "x" + std::to_string(T[tid].w) + "x" +
             std::to_string(T[tid].c);
    };
    auto same_hw = [&](uint32_t a, uint32_t b) { return T[a].h == T[b].h && T[a].w == T[b].w; };
    auto parts_c = [&](const std::vector<sw::Part> &ps) {
      uint64_t c = 0;
      for (const sw::Part &p : ps) {
        if (p.c == 0 || p.c > T[p.tid].c) throw sw::Error(at + "part of " + std::to_string(p.c) + " channels in " + shape(p.tid));
        c += p.c;
      }
      return c;
    };
    const auto &O = T[op.out];
    switch (op.kind) {
      case sw::OP_CONV: {
        const auto &I = T[op.in];
        if (!op.groups || !op.kh || !op.kw || !op.sh || !op.sw || !op.d || !op.cin || !op.cout)
          throw sw::Error(at + "conv with a zero-sized attribute");
        const uint64_t ekh = (uint64_t)op.d * (op.kh - 1) + 1, ekw = (uint64_t)op.d * (op.kw - 1) + 1;
        if (I.h + (uint64_t)op.pad[0] + op.pad[2] < ekh || I.w + (uint64_t)op.pad[1] + op.pad[3] < ekw)
          throw sw::Error(at + "kernel larger than the padded input " + shape(op.in));
        const uint64_t oh = (I.h + (uint64_t)op.pad[0] + op.pad[2] - ekh) / op.sh + 1;
        const uint64_t ow = (I.w + (uint64_t)op.pad[1] + op.pad[3] - ekw) / op.sw + 1;
        if (O.h != oh || O.w != ow || O.c != op.cout)
          throw sw::Error(at + "output " + shape(op.out) + " but the conv makes " + std::to_string(oh) + "x" +
                          std::to_string(ow) + "x" + std::to_string(op.cout));
        if (op.srcs.empty()) {
          if (I.c != op.cin) throw sw::Error(at + "input " + shape(op.in) + " but cin " + std::to_string(op.cin));
        } else {
          if (parts_c(op.srcs) != op.cin) throw sw::Error(at + "concat parts do not add up to cin");
          for (const sw::Part &p : op.srcs)
            if (!same_hw(p.tid, op.in)) throw sw::Error(at + "concat part " + shape(p.tid) + " of another size");
        }
        if (op.res >= 0 && (T[op.res].h != O.h || T[op.res].w != O.w || T[op.res].c != O.c))
          throw sw::Error(at + "residual " + shape((uint32_t)op.res) + " is not the output's shape");
        const uint64_t taps = (uint64_t)op.kh * op.kw;
        uint64_t wlen;
        if (op.groups > 1) {
          wlen = taps * c4u(op.cout) * es_d;
        } else {
          if (op.kg_pad < (op.cin + 3) / 4) throw sw::Error(at + "kg_pad below ceil(cin / 4)");
          wlen = taps * op.kg_pad * c4u(op.cout) * 4 * es_w;
        }
        if (op.w.len != wlen)
          throw sw::Error(at + "weights of " + std::to_string(op.w.len) + " bytes, the packed layout needs " +
                          std::to_string(wlen));
        if (op.b.len != c4u(op.cout) * es_d)
          throw sw::Error(at + "bias of " + std::to_string(op.b.len) + " bytes, needs " +
                          std::to_string(c4u(op.cout) * es_d));
        break;
      }
      case sw::OP_BINARY: {
        if (!same_hw(op.in, op.out) || T[op.in].c != O.c)
          throw sw::Error(at + "binary input " + shape(op.in) + " and output " + shape(op.out) + " differ");
        const auto *B = op.opnd == sw::OPND_SCALAR || op.opnd == sw::OPND_CVEC ? nullptr : &T[op.b_tid];
        bool ok = true;
        switch (op.opnd) {
          case sw::OPND_TENSOR: ok = B->h == O.h && B->w == O.w && B->c == O.c; break;
          case sw::OPND_CVEC: ok = op.cvec_c == O.c && op.cvec.len == c4u(O.c) * es_d; break;
          case sw::OPND_CVEC_TENSOR: ok = B->h == 1 && B->w == 1 && (B->c == 1 || B->c == O.c); break;
          case sw::OPND_PVEC_TENSOR:
            ok = (B->c == 1 && B->h == O.h && B->w == O.w) ||
                 (B->h == 1 && B->w == 1 && (uint64_t)B->c == (uint64_t)O.h * O.w);
            break;
          case sw::OPND_TILED_TENSOR: ok = B->h == 1 && B->w == 1 && B->c > 0; break;
          default: break;
        }
        if (!ok) throw sw::Error(at + "binary operand does not fit the output " + shape(op.out));
        break;
      }
      case sw::OP_GPOOL:
        if (O.h != 1 || O.w != 1 || O.c != T[op.in].c)
          throw sw::Error(at + "gpool of " + shape(op.in) + " into " + shape(op.out));
        break;
      case sw::OP_RESIZE: {
        if (O.h != op.oh || O.w != op.ow || !op.oh || !op.ow)
          throw sw::Error(at + "resize to " + std::to_string(op.oh) + "x" + std::to_string(op.ow) + " into " + shape(op.out));
        if (op.srcs.empty()) {
          if (T[op.in].c != O.c) throw sw::Error(at + "resize of " + shape(op.in) + " into " + shape(op.out));
        } else {
          if (parts_c(op.srcs) != O.c) throw sw::Error(at + "resize parts do not add up to the output channels");
          for (const sw::Part &p : op.srcs)
            if (!same_hw(p.tid, op.in)) throw sw::Error(at + "resize part " + shape(p.tid) + " of another size");
        }
        break;
      }
      case sw::OP_CONCAT: {
        if (op.srcs.empty() || parts_c(op.srcs) != O.c)
          throw sw::Error(at + "concat parts do not add up to the output channels");
        for (const sw::Part &p : op.srcs)
          if (!same_hw(p.tid, op.out)) throw sw::Error(at + "concat part " + shape(p.tid) + " of another size");
        break;
      }
    }
  }
}

void need_dense(const aih_model *m, uint32_t tid, const char *role, size_t op_index) {
  if (!m->dense(tid))
    throw sw::Error(".sw: op " + std::to_string(op_index) + ": " + role + " '" + m->g.tensors[tid].name +
                    "' is a channel view; this op needs a whole tensor");
}

// A tensor a kernel can take as a whole NHWC-C4 buffer: its own, or an alias
// covering all of its backing tensor's channel groups from the first.
bool dense_tid(const sw::Model &g, uint32_t tid) {
  const auto r = g.resolve(tid);
  return r.second == 0 && c4(g.tensors[r.first].c) == c4(g.tensors[tid].c);
}

// The tensors each op reads, one entry per operand slot: an op that reads a
// tensor through two slots (a conv whose residual is its own input, a binary
// op of a tensor with itself) counts as two readers of it, so no fusion rule
// that asks for a single reader can drop a tensor the op still needs.
std::vector<uint32_t> reads_of(const sw::Op &op) {
  std::vector<uint32_t> r;
  for (const sw::Part &p : op.srcs) r.push_back(p.tid);
  switch (op.kind) {
    case sw::OP_CONV:
      r.push_back(op.in);
      if (op.res >= 0) r.push_back((uint32_t)op.res);
      break;
    case sw::OP_BINARY:
      r.push_back(op.in);
      if (op.opnd != sw::OPND_SCALAR && op.opnd != sw::OPND_CVEC) r.push_back(op.b_tid);
      break;
    case sw::OP_GPOOL:
    case sw::OP_RESIZE: r.push_back(op.in); break;
    case sw::OP_CONCAT: break;
  }
  return r;
}

bool is_pw(const sw::Op &o) {
  return o.kind == sw::OP_CONV && o.groups == 1 && o.kh == 1 && o.kw == 1 && o.sh == 1 && o.sw == 1 && o.d == 1 &&
         !o.pad[0] && !o.pad[1] && !o.pad[2] && !o.pad[3] && o.srcs.empty();
}

// Ops k, k + 1 as one aih_conv_dwpw launch, by the rule in find_fusions'
// comment (op k a depthwise conv: never the first op of an inverted-residual
// block).
bool fuse_pair(aih_model *m, size_t k, const std::vector<uint32_t> &readers, const std::vector<bool> &pinned) {
  const auto &ops = m->g.ops;
  const auto &T = m->g.tensors;
  if (m->dt != m->wdt || k + 1 >= ops.size()) return false;
  const sw::Op &B = ops[k], &P = ops[k + 1];
  const bool ok = B.kind == sw::OP_CONV && B.kh == 3 && B.kw == 3 && B.sh == B.sw && B.d == 1 &&
                  B.groups == B.cin && B.cin == B.cout && B.srcs.empty() && B.res < 0 && is_pw(P) &&
                  P.in == B.out && P.cin == B.cout && readers[B.out] == 1 && !pinned[B.out] &&
                  dense_tid(m->g, B.in) && dense_tid(m->g, P.out) && (P.res < 0 || dense_tid(m->g, (uint32_t)P.res));
  if (!ok) return false;
  for (const sw::WRef *r : {&B.w, &B.b, &P.w, &P.b})
    if (reinterpret_cast<uintptr_t>(m->wptr(*r)) % 16 != 0) return false;
  aih_dwpw_desc d{};
  d.n = m->n;
  d.ih = T[B.in].h;
  d.iw = T[B.in].w;
  d.c = B.cin;
  d.k = 3;
  d.s = B.sh;
  std::memcpy(d.pad, B.pad, sizeof(d.pad));
  d.cout = P.cout;
  d.kg_pad = P.kg_pad;
  d.act_dw = B.act;
  d.act_pw = P.act;
  d.residual = P.res >= 0 ? 1 : 0;
  d.dt = m->dt;
  aih_dwpw_plan plan;
  if (aih_conv_dwpw_plan(&d, &plan) != AIH_OK || plan.tiles < aih::device_cus()) return false;
  const int32_t bi = (int32_t)m->fused.size();
  m->fused.push_back(aih_model::Fused{(uint32_t)k, 2, aih_ir_block_desc{}, aih_ir_plan{}, d, plan,
                                      aih_igemm_desc{}, AIH_FUSED_DWPW});
  m->block_of[k] = m->block_of[k + 1] = bi;
  m->internal[B.out] = (int32_t)k;
  return true;
}

// The parts of the one aih_resize_concat launch that replaces a Resize (op
// k) and the Concat after it (op k + 1): the concat's parts in order, the
// resize's output replaced by the resize's own parts (its srcs, or its whole
// input), each marked resized.
struct FoldPart {
  sw::Part part;
  bool resized;
};
std::vector<FoldPart> fold_parts(const sw::Model &g, const sw::Op &R, const sw::Op &C) {
  std::vector<FoldPart> out;
  for (const sw::Part &p : C.srcs) {
    if (p.tid != R.out) {
      out.push_back(FoldPart{p, false});
      continue;
    }
    if (R.srcs.empty())
      out.push_back(FoldPart{sw::Part{R.in, g.tensors[R.in].c}, true});
    else
      for (const sw::Part &q : R.srcs) out.push_back(FoldPart{q, true});
  }
  return out;
}

// Ops k, k + 1 as one aih_resize_concat launch: a Resize whose output only
// the Concat right after it reads (no alias, graph output or state), taken
// whole as one of its parts, every part of the folded launch but the last
// with a multiple of 4 channels, at most 8 parts, and a dense concat output.
// The resize output is then never stored: at batch 64, f16, the real
// segmentation model's 40x72x32 -> 80x144 resize and the 44-channel concat
// after it write and read back 47 MB less.
bool fold_resize_concat(aih_model *m, size_t k, const std::vector<uint32_t> &readers,
                        const std::vector<bool> &pinned) {
  const auto &ops = m->g.ops;
  if (k + 1 >= ops.size()) return false;
  const sw::Op &R = ops[k], &C = ops[k + 1];
  if (R.kind != sw::OP_RESIZE || C.kind != sw::OP_CONCAT || readers[R.out] != 1 || pinned[R.out] ||
      !dense_tid(m->g, C.out))
    return false;
  bool whole = false;
  for (const sw::Part &p : C.srcs) whole = whole || (p.tid == R.out && p.c == m->g.tensors[R.out].c);
  if (!whole) return false;
  const std::vector<FoldPart> parts = fold_parts(m->g, R, C);
  if (parts.size() > 8) return false;
  for (size_t i = 0; i + 1 < parts.size(); ++i)
    if (parts[i].part.c % 4) return false;
  const int32_t bi = (int32_t)m->fused.size();
  aih_model::Fused f{};
  f.first = (uint32_t)k;
  f.nops = 2;
  f.kind = AIH_FUSED_RESIZE_CONCAT;
  m->fused.push_back(f);
  m->block_of[k] = m->block_of[k + 1] = bi;
  m->internal[R.out] = (int32_t)k;
  return true;
}

// Inverted-residual blocks that run as one aih_ir_block launch: ops k, k+1,
// k+2 = 1x1 expand (no residual), depthwise 3x3 (d = 1, square stride) on the
// expand's output, 1x1 project on the depthwise's output (residual allowed);
// both intermediates read by exactly that next op and by nothing else (no
// other op, alias, graph output or state); weights in the activation dtype at
// the alignment aih_ir_block needs; and a plan that aih_ir_block_plan accepts.
// The fused kernels take the converter's packed layouts as they are (the
// 1x1 weights' K groups past cin / 4 and the pitch of kg_pad are never read).
//
// Where no such block starts, an fp32 depthwise 3x3 (d = 1, square stride)
// whose output only the next op, a 1x1 conv, reads runs with it as one
// aih_conv_dwpw launch, when its plan has a tile for every CU (with fewer,
// part of the GPU idles through the whole channel walk). Measured at batch
// 64, fused against the two launches: 96 -> 48 stride 2 at 20x36 15 vs 22 us
// (256 tiles), 44 -> 24 at 80x144 56 vs 89 us.
void find_fusions(aih_model *m) {
  const auto &ops = m->g.ops;
  const auto &T = m->g.tensors;
  m->block_of.assign(ops.size(), -1);
  m->internal.assign(T.size(), -1);
  if (m->flags & AIH_MODEL_NO_FUSE) return;
  std::vector<uint32_t> readers(T.size(), 0);
  for (const sw::Op &op : ops)
    for (uint32_t t : reads_of(op)) ++readers[t];
  std::vector<bool> pinned(T.size(), false);
  for (uint32_t t : m->g.outputs) pinned[t] = true;
  for (const auto &st : m->g.states) pinned[st.first] = pinned[st.second] = true;
  for (size_t i = 0; i < T.size(); ++i)
    if (T[i].alias_of >= 0) pinned[i] = pinned[(size_t)T[i].alias_of] = true;
  // resize -> concat folds move no weights: any dtypes
  for (size_t k = 0; k + 1 < ops.size(); ++k)
    if (fold_resize_concat(m, k, readers, pinned)) ++k;
  if (m->wdt != m->dt) return;
  auto aligned = [&](const sw::WRef &r, uintptr_t a) { return (reinterpret_cast<uintptr_t>(m->wptr(r)) % a) == 0; };
  for (size_t k = 0; k + 1 < ops.size();) {
    if (fuse_pair(m, k, readers, pinned)) {
      k += 2;
      continue;
    }
    if (k + 2 >= ops.size()) break;
    const sw::Op &A = ops[k], &B = ops[k + 1], &P = ops[k + 2];
    bool ok = is_pw(A) && A.res < 0 && B.kind == sw::OP_CONV && B.kh == 3 && B.kw == 3 && B.sh == B.sw &&
              B.d == 1 && B.groups == B.cin && B.cin == B.cout && B.cout == A.cout && B.in == A.out &&
              B.srcs.empty() && B.res < 0 && is_pw(P) && P.in == B.out && P.cin == B.cout;
    ok = ok && readers[A.out] == 1 && readers[B.out] == 1 && !pinned[A.out] && !pinned[B.out] &&
         dense_tid(m->g, A.in) && dense_tid(m->g, P.out) && (P.res < 0 || dense_tid(m->g, (uint32_t)P.res));
    ok = ok && aligned(A.w, 16) && aligned(B.w, 16) && aligned(P.w, 16) && aligned(A.b, 8) && aligned(B.b, 8) &&
         aligned(P.b, 8);
    if (ok) {
      aih_ir_block_desc d{};
      d.n = m->n;
      d.ih = T[A.in].h;
      d.iw = T[A.in].w;
      d.cin = A.cin;
      d.cexp = A.cout;
      d.cout = P.cout;
      d.s = B.sh;
      std::memcpy(d.pad, B.pad, sizeof(d.pad));
      d.act_expand = A.act;
      d.act_dw = B.act;
      d.act_project = P.act;
      d.residual = P.res >= 0 ? 1 : 0;
      d.dt = m->dt;
      aih_ir_plan plan;
      if (aih_ir_block_plan(&d, &plan) == AIH_OK) {
        const int32_t bi = (int32_t)m->fused.size();
        m->fused.push_back(aih_model::Fused{(uint32_t)k, 3, d, plan, aih_dwpw_desc{}, aih_dwpw_plan{},
                                            aih_igemm_desc{}, AIH_FUSED_IR_BLOCK});
        m->block_of[k] = m->block_of[k + 1] = m->block_of[k + 2] = bi;
        m->internal[A.out] = m->internal[B.out] = (int32_t)k;
        k += 3;
        continue;
      }
    }
    ++k;
  }
}

// Load-time tuning (AIH_MODEL_TUNE): every fused inverted-residual block's
// launch options -- the plan's own choice, and the wave kernel (weights
// resident and streamed), the split kernel (2 / 4 / 8 wavefronts a tile) and
// the tile kernel at a set of forced output tiles -- are timed on the device
// with the model's own buffers, two warm-up launches and kTuneReps timed ones
// each (the median), in two passes over the candidates (each keeping its
// faster median, so a drift during one pass does not pick the winner), and
// the fastest is kept. The reference's Model::load does its
// per-model device work -- pipeline compilation -- once at load
// (crates/ai-gpu-runtime/src/model.rs:56-366); this is the same kind of
// one-time cost, tens of milliseconds a block. The kernels' arithmetic does not
// depend on the choice beyond the fp32 summation order.
// Launches timed per candidate and pass (the median kept).
constexpr int kTuneReps = 9;
constexpr uint32_t kTuneWaveTiles[][2] = {{0, 0}, {4, 8}, {8, 4}, {5, 6}, {6, 5}, {2, 16}, {16, 2}, {3, 10}};
constexpr uint32_t kTuneTileTiles[][2] = {{0, 0}, {4, 8}, {8, 4}, {8, 8}, {4, 16}, {16, 4}, {8, 16}, {16, 8}};

void tune_blocks(aih_model *m) {
  hipStream_t st = nullptr;
  if (hipStreamCreateWithFlags(&st, hipStreamNonBlocking) != hipSuccess) throw std::runtime_error("tune: hipStreamCreate");
  constexpr int R = kTuneReps;
  hipEvent_t ev[2 * R];
  for (auto &e : ev)
    if (hipEventCreate(&e) != hipSuccess) throw std::runtime_error("tune: hipEventCreate");
  struct Cleanup {
    hipStream_t st;
    hipEvent_t *ev;
    ~Cleanup() {
      for (int i = 0; i < 2 * R; ++i) (void)hipEventDestroy(ev[i]);
      (void)hipStreamDestroy(st);
    }
  } cleanup{st, ev};
  for (aih_model::Fused &f : m->fused) {
    if (f.nops != 3) continue;
    const sw::Op &A = m->g.ops[f.first], &B = m->g.ops[f.first + 1], &P = m->g.ops[f.first + 2];
    const void *x = m->ptr(A.in), *we = m->wptr(A.w), *be = m->wptr(A.b), *wd = m->wptr(B.w), *bd = m->wptr(B.b),
               *wp = m->wptr(P.w), *bp = m->wptr(P.b);
    const void *res = P.res >= 0 ? m->ptr((uint32_t)P.res) : nullptr;
    void *y = m->ptr(P.out);
    std::vector<aih_ir_block_desc> cands;
    auto add = [&](int32_t kernel, const uint32_t (&t)[2], int32_t weights, uint32_t waves) {
      aih_ir_block_desc d = f.d;
      d.tile_h = t[0];
      d.tile_w = t[1];
      d.kernel = kernel;
      d.weights = weights;
      d.waves = waves;
      cands.push_back(d);
    };
    cands.push_back(f.d);
    for (const auto &t : kTuneWaveTiles) {
      for (uint32_t w : {0u, 4u, 8u, 12u}) {  // the plan's wavefronts per workgroup, then forced (12 where allowed)
        add(AIH_IR_KERNEL_WAVE, t, AIH_IR_WEIGHTS_RESIDENT, w);
        add(AIH_IR_KERNEL_WAVE, t, AIH_IR_WEIGHTS_STREAMED, w);
      }
      for (uint32_t w : {2u, 4u, 8u}) add(AIH_IR_KERNEL_SPLIT, t, AIH_IR_WEIGHTS_AUTO, w);
    }
    for (const auto &t : kTuneTileTiles) {
      add(AIH_IR_KERNEL_TILE, t, AIH_IR_WEIGHTS_RESIDENT, 0);
      add(AIH_IR_KERNEL_TILE, t, AIH_IR_WEIGHTS_STREAMED, 0);
    }
    std::set<std::array<uint32_t, 5>> seen;
    std::vector<std::pair<aih_ir_block_desc, aih_ir_plan>> runs;
    for (const aih_ir_block_desc &d : cands) {
      aih_ir_plan plan;
      if (aih_ir_block_plan(&d, &plan) != AIH_OK) continue;  // a forced option this block cannot run
      const std::array<uint32_t, 5> key{plan.kernel, plan.th, plan.tw, plan.resident,
                                        plan.kernel == AIH_IR_KERNEL_TILE ? 0u : plan.waves};
      if (!seen.insert(key).second) continue;
      // the plan's choice, made explicit, so later calls run exactly it
      aih_ir_block_desc dd = d;
      dd.tile_h = plan.th;
      dd.tile_w = plan.tw;
      dd.kernel = (int32_t)plan.kernel;
      if (plan.kernel != AIH_IR_KERNEL_SPLIT) dd.weights = plan.resident ? AIH_IR_WEIGHTS_RESIDENT : AIH_IR_WEIGHTS_STREAMED;
      if (plan.kernel != AIH_IR_KERNEL_TILE) dd.waves = plan.waves;
      runs.emplace_back(dd, plan);
    }
    // median of R launches after two warm-up ones
    auto time = [&](const aih_ir_block_desc &dd) -> float {
      for (int w = 0; w < 2; ++w)
        if (aih_ir_block(&dd, x, we, be, wd, bd, wp, bp, res, y, st) != AIH_OK)
          throw std::runtime_error(std::string("tune: ") + aih_last_error());
      for (int r = 0; r < R; ++r) {
        if (hipEventRecord(ev[2 * r], st) != hipSuccess ||
            aih_ir_block(&dd, x, we, be, wd, bd, wp, bp, res, y, st) != AIH_OK ||
            hipEventRecord(ev[2 * r + 1], st) != hipSuccess)
          throw std::runtime_error("tune: launch");
      }
      if (hipEventSynchronize(ev[2 * R - 1]) != hipSuccess) throw std::runtime_error("tune: hipEventSynchronize");
      float t[R];
      for (int r = 0; r < R; ++r)
        if (hipEventElapsedTime(&t[r], ev[2 * r], ev[2 * r + 1]) != hipSuccess)
          throw std::runtime_error("tune: hipEventElapsedTime");
      std::sort(t, t + R);
      return t[R / 2];
    };
    // two passes over the candidates, each keeping its faster median: a
    // clock or cache drift during one pass does not pick the winner
    std::vector<float> t1, t2;
    for (const auto &rp : runs) t1.push_back(time(rp.first));
    for (const auto &rp : runs) t2.push_back(time(rp.first));
    float best = -1.0f;
    for (size_t i = 0; i < runs.size(); ++i) {
      const float ms = std::min(t1[i], t2[i]);
      if (best < 0 || ms < best) {
        best = ms;
        f.d = runs[i].first;
        f.plan = runs[i].second;
      }
    }
  }
  if (hipStreamSynchronize(st) != hipSuccess) throw std::runtime_error("tune: hipStreamSynchronize");
}

// The stem-from-fp32 route for the graph's input (see aih_model::stem_op):
// one input, read only by op k, a dense 3x3 conv on the stem route (d = 1,
// cin <= 3, cout 32 or 64, weights in the activation dtype), not a graph
// output, state or alias; not under AIH_MODEL_NO_FUSE (every op on its own).
void find_stem_input(aih_model *m) {
  const auto &ops = m->g.ops;
  if ((m->flags & AIH_MODEL_NO_FUSE) || m->g.inputs.size() != 1 || m->dt != m->wdt) return;
  const uint32_t t = m->g.inputs[0];
  if (m->g.tensors[t].alias_of >= 0) return;
  for (uint32_t o : m->g.outputs)
    if (o == t) return;
  for (const auto &st : m->g.states)
    if (st.first == t || st.second == t) return;
  for (const auto &tt : m->g.tensors)
    if (tt.alias_of == (int64_t)t) return;
  int64_t reader = -1;
  size_t nreads = 0;
  for (size_t k = 0; k < ops.size(); ++k)
    for (uint32_t r : reads_of(ops[k]))
      if (r == t) {
        ++nreads;
        reader = (int64_t)k;
      }
  if (nreads != 1 || m->block_of[(size_t)reader] >= 0) return;
  const sw::Op &op = ops[(size_t)reader];
  if (op.kind != sw::OP_CONV || op.in != t || !op.srcs.empty() || op.groups != 1 || op.kh != 3 || op.kw != 3 ||
      op.sh != op.sw || op.d != 1 || op.cin > 3 || (op.cout != 32 && op.cout != 64) || !m->dense(t))
    return;
  m->stem_op = reader;
  m->stem_tid = t;
}

// Packs the staged fp32 input into its NHWC-C4 slot (for a reader of the
// slot other than the stem: read_output, tensor storage).
int settle_input(const aih_model *cm, aih_stream stream) {
  aih_model *m = const_cast<aih_model *>(cm);
  if (!m->staged) return AIH_OK;
  const auto &t = m->g.tensors[m->stem_tid];
  if (aih_pack_nhwc_device(m->staging, m->n, t.h, t.w, t.c, m->dt, m->ptr(m->stem_tid), stream)) return AIH_ERR;
  m->staged = false;
  return AIH_OK;
}

// The stem conv fused into the inverted-residual block after it
// (aih_ir_block_stem): the stem-from-fp32 route's conv (stem_op) whose
// output only that fused block reads -- as its expand input and its
// residual, two reads -- and that is no graph output, state or alias. Runs
// after lower(): op k's launch becomes one aih_ir_block_stem from the
// staged fp32 input, falling back to the stem and the block as two
// launches (the stem's output keeps its slot for that) when the input slot
// holds the input instead; the block's record then covers the stem op
// (n_ops 4) and the stem's output counts as the block's intermediate. With
// AIH_MODEL_TUNE the two launches and the fused one at the tune tiles,
// placements and 4 / 8 wavefronts are timed on the model's buffers (the
// staged input zeroed), the fastest kept; else the fused launch on the
// block's own tile and placement where it plans. Not under AIH_MODEL_NO_FUSE.
void fuse_stem_launch(aih_model *m) {
  if (m->stem_op < 0 || (m->flags & AIH_MODEL_NO_FUSE)) return;
  const size_t k = (size_t)m->stem_op;
  const auto &ops = m->g.ops;
  if (k + 3 >= ops.size() || m->block_of[k + 1] < 0) return;
  const int32_t bi = m->block_of[k + 1];
  aih_model::Fused &f = m->fused[(size_t)bi];
  if (f.first != k + 1 || f.nops != 3) return;
  const sw::Op &S = ops[k], &A = ops[k + 1], &B = ops[k + 2], &P = ops[k + 3];
  const uint32_t t = S.out;
  if (S.res >= 0 || A.in != t || P.res != (int64_t)t || m->g.tensors[t].alias_of >= 0) return;
  for (uint32_t o : m->g.outputs)
    if (o == t) return;
  for (const auto &st : m->g.states)
    if (st.first == t || st.second == t) return;
  for (const auto &tt : m->g.tensors)
    if (tt.alias_of == (int64_t)t) return;
  size_t nreads = 0;
  for (const auto &op : ops)
    for (uint32_t r : reads_of(op)) nreads += r == t;
  if (nreads != 2) return;
  const auto &I = m->g.tensors[S.in];
  aih_igemm_desc sd{};
  sd.n = m->n;
  sd.ih = I.h;
  sd.iw = I.w;
  sd.cin = S.cin;
  sd.cout = S.cout;
  sd.k = 3;
  sd.s = S.sh;
  sd.d = 1;
  std::memcpy(sd.pad, S.pad, sizeof(sd.pad));
  sd.act = S.act;
  sd.dt = m->dt;
  sd.wdt = m->wdt;
  const float *img = m->staging;
  const void *ws = m->wptr(S.w), *bs = m->wptr(S.b), *we = m->wptr(A.w), *be = m->wptr(A.b), *wd = m->wptr(B.w),
             *bd = m->wptr(B.b), *wp = m->wptr(P.w), *bp = m->wptr(P.b);
  void *y = m->ptr(P.out);
  // the candidates: the block's own tile and placement, then (tuning) the tune set
  std::vector<aih_ir_block_desc> cands;
  {
    aih_ir_block_desc d = f.d;
    if (d.kernel != AIH_IR_KERNEL_WAVE) d.kernel = AIH_IR_KERNEL_AUTO, d.tile_h = d.tile_w = 0, d.waves = 0;
    cands.push_back(d);
  }
  const bool tune = (m->flags & AIH_MODEL_TUNE) != 0;
  if (tune)
    for (const auto &tt : kTuneWaveTiles)
      for (int32_t w : {AIH_IR_WEIGHTS_RESIDENT, AIH_IR_WEIGHTS_STREAMED})
        for (uint32_t wv : {0u, 4u, 8u, 12u}) {
          aih_ir_block_desc d = f.d;
          d.kernel = AIH_IR_KERNEL_WAVE;
          d.tile_h = tt[0];
          d.tile_w = tt[1];
          d.weights = w;
          d.waves = wv;
          cands.push_back(d);
        }
  std::function<int(hipStream_t)> sep_stem = m->launches[k], sep_blk = m->launches[k + 1];
  aih_ir_block_desc best{};
  aih_ir_plan best_plan{};
  bool found = false;
  if (!tune) {
    for (const auto &d : cands)
      if (aih_ir_block_stem_plan(&sd, &d, &best_plan) == AIH_OK) {
        best = d;
        found = true;
        break;
      }
  } else {
    hipStream_t st = nullptr;
    if (hipStreamCreateWithFlags(&st, hipStreamNonBlocking) != hipSuccess) throw std::runtime_error("tune: hipStreamCreate");
    constexpr int R = kTuneReps;
    hipEvent_t ev[2 * R];
    for (auto &e : ev)
      if (hipEventCreate(&e) != hipSuccess) throw std::runtime_error("tune: hipEventCreate");
    struct Cleanup {
      hipStream_t st;
      hipEvent_t *ev;
      ~Cleanup() {
        for (int i = 0; i < 2 * R; ++i) (void)hipEventDestroy(ev[i]);
        (void)hipStreamDestroy(st);
      }
    } cleanup{st, ev};
    if (hipMemsetAsync(m->staging, 0, m->staging_floats * 4, st) != hipSuccess) throw std::runtime_error("tune: memset");
    const bool staged0 = m->staged;
    m->staged = true;
    auto time = [&](const std::function<int(hipStream_t)> &fn) -> float {
      for (int w = 0; w < 2; ++w)
        if (fn(st) != AIH_OK) throw std::runtime_error(std::string("tune: ") + aih_last_error());
      for (int r = 0; r < R; ++r)
        if (hipEventRecord(ev[2 * r], st) != hipSuccess || fn(st) != AIH_OK || hipEventRecord(ev[2 * r + 1], st) != hipSuccess)
          throw std::runtime_error("tune: launch");
      if (hipEventSynchronize(ev[2 * R - 1]) != hipSuccess) throw std::runtime_error("tune: hipEventSynchronize");
      float ts[R];
      for (int r = 0; r < R; ++r)
        if (hipEventElapsedTime(&ts[r], ev[2 * r], ev[2 * r + 1]) != hipSuccess) throw std::runtime_error("tune: elapsed");
      std::sort(ts, ts + R);
      return ts[R / 2];
    };
    std::set<std::array<uint32_t, 4>> seen;
    std::vector<std::pair<aih_ir_block_desc, aih_ir_plan>> runs;
    for (const auto &d : cands) {
      aih_ir_plan plan;
      if (aih_ir_block_stem_plan(&sd, &d, &plan) != AIH_OK) continue;
      if (!seen.insert({plan.th, plan.tw, plan.resident, plan.waves}).second) continue;
      aih_ir_block_desc dd = d;
      dd.kernel = AIH_IR_KERNEL_WAVE;
      dd.tile_h = plan.th;
      dd.tile_w = plan.tw;
      dd.weights = plan.resident ? AIH_IR_WEIGHTS_RESIDENT : AIH_IR_WEIGHTS_STREAMED;
      dd.waves = plan.waves;
      runs.emplace_back(dd, plan);
    }
    // two passes (the two launches first), each keeping its faster median
    const auto sep = [&](hipStream_t s) { return sep_stem(s) != AIH_OK ? AIH_ERR : sep_blk(s); };
    auto fused_fn = [&](const aih_ir_block_desc &dd) {
      return [&, dd](hipStream_t s) { return aih_ir_block_stem(&sd, &dd, img, ws, bs, we, be, wd, bd, wp, bp, y, s); };
    };
    float best_ms = time(sep);
    std::vector<float> t1;
    for (const auto &rp : runs) t1.push_back(time(fused_fn(rp.first)));
    best_ms = std::min(best_ms, time(sep));
    for (size_t i = 0; i < runs.size(); ++i) {
      const float ms = std::min(t1[i], time(fused_fn(runs[i].first)));
      if (ms < best_ms) {
        best_ms = ms;
        best = runs[i].first;
        best_plan = runs[i].second;
        found = true;
      }
    }
    m->staged = staged0;
    if (hipStreamSynchronize(st) != hipSuccess) throw std::runtime_error("tune: hipStreamSynchronize");
  }
  if (!found) return;
  aih_model *mm = m;
  const aih_ir_block_desc d = best;
  m->launches[k] = [mm, sd, d, ws, bs, we, be, wd, bd, wp, bp, y, sep_stem, sep_blk](hipStream_t s) {
    // the staged fp32 upload: one launch; else the stem from the input slot, then the block
    if (mm->staged) return aih_ir_block_stem(&sd, &d, mm->staging, ws, bs, we, be, wd, bd, wp, bp, y, s);
    return sep_stem(s) != AIH_OK ? AIH_ERR : sep_blk(s);
  };
  m->launches[k + 1] = {};
  f.first = (uint32_t)k;
  f.nops = 4;
  f.kind = AIH_FUSED_STEM_BLOCK;
  f.sd = sd;
  f.d = best;
  f.plan = best_plan;
  m->block_of[k] = bi;
  m->internal[t] = (int32_t)k;
}

// The narrow head joined to the block before it (aih_ir_block_head): a 1x1
// conv op k (no stride, pad, groups, residual or views; at most 4 outputs)
// right after a three-op fused block (ops k - 3 .. k - 1) whose output t it
// alone reads, t no graph output, state or alias. Runs after lower(): op
// k - 3's launch becomes the joined one on the split kernel and op k's is
// dropped; the block's record then covers the head (n_ops 4) and t counts as
// its intermediate (never stored). Candidates: the block's own tile and
// wavefronts where its plan is the split kernel, and with AIH_MODEL_TUNE the
// split kernel at the tune tiles with 2 / 4 / 8 wavefronts, timed (two
// passes) against the block's and the head's own launches, the fastest
// kept; without tuning the joined launch where the block's own plan is the
// split kernel. Not under AIH_MODEL_NO_FUSE.
void fuse_head_launch(aih_model *m) {
  if (m->flags & AIH_MODEL_NO_FUSE) return;
  const auto &ops = m->g.ops;
  const auto &T = m->g.tensors;
  for (aih_model::Fused &f : m->fused) {
    if (f.nops != 3) continue;
    const size_t k = f.first + 3;
    if (k >= ops.size() || m->block_of[k] >= 0) continue;
    const sw::Op &A = ops[f.first], &B = ops[f.first + 1], &P = ops[f.first + 2], &H = ops[k];
    const uint32_t t = P.out;
    if (H.kind != sw::OP_CONV || H.in != t || !H.srcs.empty() || H.groups != 1 || H.kh != 1 || H.kw != 1 ||
        H.sh != 1 || H.sw != 1 || H.pad[0] || H.pad[1] || H.pad[2] || H.pad[3] || H.res >= 0 || H.cout > 4 ||
        T[t].alias_of >= 0 || !m->dense(t) || !m->dense(H.out))
      continue;
    bool keep = false;
    for (uint32_t o : m->g.outputs) keep |= o == t;
    for (const auto &st : m->g.states) keep |= st.first == t || st.second == t;
    for (const auto &tt : T) keep |= tt.alias_of == (int64_t)t;
    size_t nreads = 0;
    for (const auto &op : ops)
      for (uint32_t r : reads_of(op)) nreads += r == t;
    if (keep || nreads != 1) continue;
    aih_pw_desc hd{m->n, T[t].h * T[t].w, (H.cin + 3) / 4, 1, H.kg_pad, H.act, 0, m->dt, m->wdt, AIH_VAR_AUTO, 0};
    // the candidates: the block's own split plan, then (tuning) the tune set
    std::vector<aih_ir_block_desc> cands;
    if (f.plan.kernel == AIH_IR_KERNEL_SPLIT) cands.push_back(f.d);
    const bool tune = (m->flags & AIH_MODEL_TUNE) != 0;
    if (tune)
      for (const auto &tt : kTuneWaveTiles)
        for (uint32_t wv : {2u, 4u, 8u}) {
          aih_ir_block_desc d = f.d;
          d.kernel = AIH_IR_KERNEL_SPLIT;
          d.weights = AIH_IR_WEIGHTS_AUTO;
          d.tile_h = tt[0];
          d.tile_w = tt[1];
          d.waves = wv;
          cands.push_back(d);
        }
    std::set<std::array<uint32_t, 3>> seen;
    std::vector<std::pair<aih_ir_block_desc, aih_ir_plan>> runs;
    for (const auto &d : cands) {
      aih_ir_plan plan;
      if (aih_ir_block_head_plan(&d, &hd, &plan) != AIH_OK) continue;
      if (!seen.insert({plan.th, plan.tw, plan.waves}).second) continue;
      aih_ir_block_desc dd = d;
      dd.kernel = AIH_IR_KERNEL_SPLIT;
      dd.weights = AIH_IR_WEIGHTS_AUTO;
      dd.tile_h = plan.th;
      dd.tile_w = plan.tw;
      dd.waves = plan.waves;
      runs.emplace_back(dd, plan);
    }
    if (runs.empty()) continue;
    const void *x = m->ptr(A.in), *we = m->wptr(A.w), *be = m->wptr(A.b), *wd = m->wptr(B.w), *bd = m->wptr(B.b),
               *wp = m->wptr(P.w), *bp = m->wptr(P.b), *wh = m->wptr(H.w), *bh = m->wptr(H.b);
    const void *res = P.res >= 0 ? m->ptr((uint32_t)P.res) : nullptr;
    void *yh = m->ptr(H.out);
    size_t best = 0;
    if (tune) {
      hipStream_t st = nullptr;
      if (hipStreamCreateWithFlags(&st, hipStreamNonBlocking) != hipSuccess) throw std::runtime_error("tune: hipStreamCreate");
      constexpr int R = kTuneReps;
      hipEvent_t ev[2 * R];
      for (auto &e : ev)
        if (hipEventCreate(&e) != hipSuccess) throw std::runtime_error("tune: hipEventCreate");
      struct Cleanup {
        hipStream_t st;
        hipEvent_t *ev;
        ~Cleanup() {
          for (int i = 0; i < 2 * R; ++i) (void)hipEventDestroy(ev[i]);
          (void)hipStreamDestroy(st);
        }
      } cleanup{st, ev};
      auto time = [&](const std::function<int(hipStream_t)> &fn) -> float {
        for (int w = 0; w < 2; ++w)
          if (fn(st) != AIH_OK) throw std::runtime_error(std::string("tune: ") + aih_last_error());
        for (int r = 0; r < R; ++r)
          if (hipEventRecord(ev[2 * r], st) != hipSuccess || fn(st) != AIH_OK ||
              hipEventRecord(ev[2 * r + 1], st) != hipSuccess)
            throw std::runtime_error("tune: launch");
        if (hipEventSynchronize(ev[2 * R - 1]) != hipSuccess) throw std::runtime_error("tune: hipEventSynchronize");
        float ts[R];
        for (int r = 0; r < R; ++r)
          if (hipEventElapsedTime(&ts[r], ev[2 * r], ev[2 * r + 1]) != hipSuccess) throw std::runtime_error("tune: elapsed");
        std::sort(ts, ts + R);
        return ts[R / 2];
      };
      const std::function<int(hipStream_t)> sep_blk = m->launches[f.first], sep_head = m->launches[k];
      const auto sep = [&](hipStream_t s) { return sep_blk(s) != AIH_OK ? AIH_ERR : sep_head(s); };
      auto joined = [&](const aih_ir_block_desc &dd) {
        return [&, dd](hipStream_t s) {
          return aih_ir_block_head(&dd, &hd, x, we, be, wd, bd, wp, bp, res, nullptr, wh, bh, yh, s);
        };
      };
      // two passes (the two launches first), each keeping its faster median
      float best_ms = time(sep);
      std::vector<float> t1;
      for (const auto &rp : runs) t1.push_back(time(joined(rp.first)));
      best_ms = std::min(best_ms, time(sep));
      best = runs.size();
      for (size_t i = 0; i < runs.size(); ++i) {
        const float ms = std::min(t1[i], time(joined(runs[i].first)));
        if (ms < best_ms) {
          best_ms = ms;
          best = i;
        }
      }
      if (hipStreamSynchronize(st) != hipSuccess) throw std::runtime_error("tune: hipStreamSynchronize");
      if (best == runs.size()) continue;  // the two launches stay
    }
    const aih_ir_block_desc d = runs[best].first;
    m->launches[f.first] = [d, hd, x, we, be, wd, bd, wp, bp, res, wh, bh, yh](hipStream_t s) {
      return aih_ir_block_head(&d, &hd, x, we, be, wd, bd, wp, bp, res, nullptr, wh, bh, yh, s);
    };
    m->launches[k] = {};
    f.nops = 4;
    f.kind = AIH_FUSED_BLOCK_HEAD;
    f.d = d;
    f.plan = runs[best].second;
    m->block_of[k] = m->block_of[f.first];
    m->internal[t] = (int32_t)f.first;
  }
}

void lower(aih_model *m) {
  const auto &T = m->g.tensors;
  for (size_t k = 0; k < m->g.ops.size(); ++k) {
    const sw::Op &op = m->g.ops[k];
    const auto &O = T[op.out];
    if (m->block_of[k] >= 0) {
      const aih_model::Fused &f = m->fused[(size_t)m->block_of[k]];
      if (f.first != k) {
        m->launches.emplace_back();  // runs in the block's first op
        continue;
      }
      if (f.kind == AIH_FUSED_RESIZE_CONCAT) {
        const sw::Op &C = m->g.ops[k + 1];
        const auto &I = T[op.in];
        aih_resize_concat_desc d{};
        d.n = m->n;
        d.ih = I.h;
        d.iw = I.w;
        d.oh = T[C.out].h;
        d.ow = T[C.out].w;
        d.mode = op.coord;
        d.dt = m->dt;
        std::vector<const void *> ins;
        for (const FoldPart &p : fold_parts(m->g, op, C)) {
          d.resized |= (p.resized ? 1u : 0u) << d.nparts;
          d.parts[d.nparts++] = m->src_of(p.part.tid, p.part.c);
          ins.push_back(m->views[p.part.tid].base);
        }
        void *y = m->ptr(C.out);
        m->launches.push_back([d, ins, y](hipStream_t s) { return aih_resize_concat(&d, ins.data(), y, s); });
        continue;
      }
      if (f.kind == AIH_FUSED_DWPW) {
        const sw::Op &P = m->g.ops[k + 1];
        const aih_dwpw_desc d = f.dp;
        const void *x = m->ptr(op.in), *wd = m->wptr(op.w), *bd = m->wptr(op.b), *wp = m->wptr(P.w),
                   *bp = m->wptr(P.b);
        const void *res = P.res >= 0 ? m->ptr((uint32_t)P.res) : nullptr;
        void *y = m->ptr(P.out);
        m->launches.push_back([d, x, wd, bd, wp, bp, res, y](hipStream_t s) {
          return aih_conv_dwpw(&d, x, wd, bd, wp, bp, res, y, s);
        });
        continue;
      }
      const sw::Op &B = m->g.ops[k + 1], &P = m->g.ops[k + 2];
      const aih_ir_block_desc d = f.d;
      const void *x = m->ptr(op.in), *we = m->wptr(op.w), *be = m->wptr(op.b), *wd = m->wptr(B.w),
                 *bd = m->wptr(B.b), *wp = m->wptr(P.w), *bp = m->wptr(P.b);
      const void *res = P.res >= 0 ? m->ptr((uint32_t)P.res) : nullptr;
      void *y = m->ptr(P.out);
      m->launches.push_back([d, x, we, be, wd, bd, wp, bp, res, y](hipStream_t s) {
        return aih_ir_block(&d, x, we, be, wd, bd, wp, bp, res, y, s);
      });
      continue;
    }
    need_dense(m, op.out, "output", k);
    void *y = m->ptr(op.out);
    switch (op.kind) {
      case sw::OP_CONV: {
        const auto &I = T[op.in];
        const void *w = m->wptr(op.w), *b = m->wptr(op.b);
        const void *res = nullptr;
        if (op.res >= 0) {
          need_dense(m, (uint32_t)op.res, "residual", k);
          res = m->ptr((uint32_t)op.res);
        }
        // std conv weights in dt_weights, dw weights and biases in dt_default
        // (lowering.rs:94-97, format/model.rs:245-254)
        const int32_t wdt = op.groups > 1 ? m->dt : m->wdt;
        if (!op.srcs.empty() || !m->dense(op.in)) {
          // concat-into-conv parts or a channel view: the implicit-GEMM path
          // reads each part through its own view (conv_igemm.rs:141-171)
          if (op.groups != 1 || op.kh != op.kw || op.sh != op.sw || op.kh == 1)
            throw sw::Error(".sw: op " + std::to_string(k) +
                            ": concat parts / channel views feed only KxK (k > 1) dense convs here");
          aih_igemm_desc d{};
          d.n = m->n;
          d.ih = I.h;
          d.iw = I.w;
          d.cin = op.cin;
          d.cout = op.cout;
          d.k = op.kh;
          d.s = op.sh;
          d.d = op.d;
          std::memcpy(d.pad, op.pad, sizeof(d.pad));
          d.act = op.act;
          d.residual = res ? 1 : 0;
          d.dt = m->dt;
          d.wdt = wdt;
          std::vector<const void *> ins;
          if (op.srcs.empty()) {
            d.nsrcs = 1;
            d.srcs[0] = m->src_of(op.in, op.cin);
            ins.push_back(m->views[op.in].base);
          } else {
            if (op.srcs.size() > 3) throw sw::Error(".sw: conv with more than 3 concat parts");
            d.nsrcs = (uint32_t)op.srcs.size();
            for (size_t i = 0; i < op.srcs.size(); ++i) {
              const auto &P = T[op.srcs[i].tid];
              if (P.h != I.h || P.w != I.w) throw sw::Error(".sw: concat part of another size");
              d.srcs[i] = m->src_of(op.srcs[i].tid, op.srcs[i].c);
              ins.push_back(m->views[op.srcs[i].tid].base);
            }
          }
          aih_plan p;
          if (aih_conv_igemm_plan(&d, &p)) throw sw::Error(std::string("op ") + std::to_string(k) + ": " + aih_last_error());
          m->ws_bytes = std::max(m->ws_bytes, p.ws_bytes);
          aih_model *mm = m;
          m->launches.push_back([mm, d, ins, w, b, res, y](hipStream_t s) {
            return aih_conv_igemm(&d, ins.data(), w, b, res, y, mm->ws, mm->ws_bytes, s);
          });
        } else {
          aih_conv_desc d{};
          d.n = m->n;
          d.ih = I.h;
          d.iw = I.w;
          d.cin = op.cin;
          d.cout = op.cout;
          d.kh = op.kh;
          d.kw = op.kw;
          d.sh = op.sh;
          d.sw = op.sw;
          std::memcpy(d.pad, op.pad, sizeof(d.pad));
          d.d = op.d;
          d.groups = op.groups;
          d.act = op.act;
          d.residual = res ? 1 : 0;
          d.dt = m->dt;
          d.wdt = wdt;
          d.kg_pad = op.kg_pad;
          if (c4(I.c) != c4(op.cin)) throw sw::Error(".sw: op " + std::to_string(k) + ": input channels != cin");
          if (aih_conv_check(&d)) throw sw::Error(".sw: op " + std::to_string(k) + ": " + aih_last_error());
          const size_t ws = aih_conv_workspace_size(&d);
          m->ws_bytes = std::max(m->ws_bytes, ws);
          const void *x = m->ptr(op.in);
          aih_model *mm = m;
          if ((int64_t)k == m->stem_op) {
            aih_igemm_desc sd{};
            sd.n = m->n;
            sd.ih = I.h;
            sd.iw = I.w;
            sd.cin = op.cin;
            sd.cout = op.cout;
            sd.k = 3;
            sd.s = op.sh;
            sd.d = 1;
            std::memcpy(sd.pad, op.pad, sizeof(sd.pad));
            sd.act = op.act;
            sd.residual = res ? 1 : 0;
            sd.dt = m->dt;
            sd.wdt = wdt;  // one dense input: no parts (nsrcs 0)
            m->launches.push_back([mm, d, sd, x, w, b, res, y](hipStream_t s) {
              // the staged fp32 upload, read by the stem itself; else the slot
              return mm->staged ? aih_conv_stem_f32in(&sd, mm->staging, w, b, res, y, s)
                                : aih_conv(&d, x, w, b, res, y, mm->ws, mm->ws_bytes, s);
            });
            break;
          }
          m->launches.push_back([mm, d, x, w, b, res, y](hipStream_t s) {
            return aih_conv(&d, x, w, b, res, y, mm->ws, mm->ws_bytes, s);
          });
        }
        break;
      }
      case sw::OP_BINARY: {
        need_dense(m, op.in, "input", k);
        aih_binary_desc d{};
        d.n = m->n;
        d.h = O.h;
        d.w = O.w;
        d.c = O.c;
        d.op = op.bin;
        d.act = op.act;
        d.dt = m->dt;
        d.operand = op.opnd;
        d.scalar = op.scalar;
        d.scalar_first = op.scalar_first ? 1 : 0;
        const void *a = m->ptr(op.in), *b = nullptr;
        if (op.opnd == sw::OPND_CVEC) {
          b = m->wptr(op.cvec);
        } else if (op.opnd != sw::OPND_SCALAR) {
          need_dense(m, op.b_tid, "operand", k);
          b = m->ptr(op.b_tid);
          d.b_c = T[op.b_tid].c;
        }
        m->launches.push_back([d, a, b, y](hipStream_t s) { return aih_binary(&d, a, b, y, s); });
        break;
      }
      case sw::OP_GPOOL: {
        need_dense(m, op.in, "input", k);
        const auto &I = T[op.in];
        aih_gpool_desc d{m->n, I.h, I.w, I.c, m->dt};
        const void *x = m->ptr(op.in);
        m->launches.push_back([d, x, y](hipStream_t s) { return aih_gpool(&d, x, y, s); });
        break;
      }
      case sw::OP_RESIZE: {
        const auto &I = T[op.in];
        aih_resize_desc d{};
        d.n = m->n;
        d.ih = I.h;
        d.iw = I.w;
        d.oh = op.oh;
        d.ow = op.ow;
        d.mode = op.coord;
        d.dt = m->dt;
        std::vector<const void *> ins;
        std::vector<sw::Part> parts = op.srcs;
        if (parts.empty()) parts.push_back(sw::Part{op.in, I.c});
        if (parts.size() > 8) throw sw::Error(".sw: resize with more than 8 parts");
        d.nsrcs = (uint32_t)parts.size();
        for (size_t i = 0; i < parts.size(); ++i) {
          d.srcs[i] = m->src_of(parts[i].tid, parts[i].c);
          ins.push_back(m->views[parts[i].tid].base);
        }
        m->launches.push_back([d, ins, y](hipStream_t s) { return aih_resize(&d, ins.data(), y, s); });
        break;
      }
      case sw::OP_CONCAT: {
        aih_concat_desc d{};
        d.n = m->n;
        d.h = O.h;
        d.w = O.w;
        d.dt = m->dt;
        if (op.srcs.size() > 8) throw sw::Error(".sw: concat with more than 8 parts");
        d.nparts = (uint32_t)op.srcs.size();
        std::vector<const void *> ins;
        for (size_t i = 0; i < op.srcs.size(); ++i) {
          d.parts[i] = m->src_of(op.srcs[i].tid, op.srcs[i].c);
          ins.push_back(m->views[op.srcs[i].tid].base);
        }
        m->launches.push_back([d, ins, y](hipStream_t s) { return aih_concat(&d, ins.data(), y, s); });
        break;
      }
    }
  }
}

}  // namespace

extern "C" {

aih_model *aih_model_load(const void *bytes, size_t len, uint32_t n, int32_t dt) {
  return aih_model_load_ex(bytes, len, n, dt, 0);
}

aih_model *aih_model_load_ex(const void *bytes, size_t len, uint32_t n, int32_t dt, uint32_t flags) {
  aih_model *out = nullptr;
  const int rc = api_guarded([&] {
    if (n == 0) return api_fail("model_load: n must be >= 1");
    if (flags & ~(uint32_t)(AIH_MODEL_NO_FUSE | AIH_MODEL_TUNE)) return api_fail("model_load: unknown flags");
    if (dt != -1 && dt != AIH_F32 && dt != AIH_F16 && dt != AIH_BF16) return api_fail("model_load: unknown dtype");
    sw::Container c = sw::parse_container(bytes, len);
    std::unique_ptr<aih_model> m(new aih_model);
    m->g = sw::parse_model(c.json, c.json_len);
    m->n = n;
    m->flags = flags;
    m->blob_dt = m->g.dt_default == sw::F16 ? AIH_F16 : AIH_F32;
    for (const auto &t : m->g.tensors)
      if (t.dt != m->g.dt_default)
        return api_fail("model_load: tensor '" + t.name + "' has a dtype other than dt_default");
    if (dt == -1) {
      m->dt = m->g.dt_default == sw::F16 ? AIH_F16 : AIH_F32;
      m->wdt = m->g.dt_weights == sw::F16 ? AIH_F16 : AIH_F32;
    } else {
      if (dt != AIH_F32 && (m->g.dt_default != sw::F32 || m->g.dt_weights != sw::F32))
        return api_fail("model_load: a dtype change needs an fp32 file");
      if (dt == AIH_F32 && m->g.dt_default != sw::F32) return api_fail("model_load: cannot widen a 16-bit file");
      m->dt = m->wdt = dt;
    }
    if (!m->g.consts.empty()) return api_fail("model_load: constant tensors are not supported");
    validate_geometry(m->g);
    prepare_weights(m.get(), c);
    find_fusions(m.get());
    alloc_tensors(m.get());
    if (flags & AIH_MODEL_TUNE) tune_blocks(m.get());
    find_stem_input(m.get());
    for (uint32_t t : m->g.inputs)
      m->staging_floats = std::max(m->staging_floats, (size_t)n * m->g.tensors[t].h * m->g.tensors[t].w * m->g.tensors[t].c);
    if (m->staging_floats) m->staging = static_cast<float *>(m->dalloc(m->staging_floats * 4));
    lower(m.get());
    if (m->ws_bytes) m->ws = m->dalloc(m->ws_bytes);
    fuse_stem_launch(m.get());
    fuse_head_launch(m.get());
    out = m.release();
    return AIH_OK;
  });
  return rc == AIH_OK ? out : nullptr;
}

void aih_model_free(aih_model *m) { delete m; }

static int upload(aih_model *m, const char *name, const float *src, size_t count, bool host, aih_stream stream) {
  return api_guarded([&] {
    if (!m || !src) return api_fail("upload_input: null argument");
    const int64_t tid = m->find(name);
    if (tid < 0 || std::find(m->g.inputs.begin(), m->g.inputs.end(), (uint32_t)tid) == m->g.inputs.end())
      return api_fail(std::string("upload_input: no input named '") + (name ? name : "") + "'");
    const auto &t = m->g.tensors[tid];
    const size_t want = (size_t)m->n * t.h * t.w * t.c;
    if (count != want) return api_fail("upload_input: expected " + std::to_string(want) + " floats");
    if (!m->dense((uint32_t)tid)) return api_fail("upload_input: input is a channel view");
    hipStream_t s = static_cast<hipStream_t>(stream);
    const float *x = src;
    if (m->stem_op >= 0 && (uint32_t)tid == m->stem_tid) {
      // the stem reads the fp32 values from staging at infer (a copy, as
      // Model::upload_input copies: the caller's buffer is free afterwards)
      const hipError_t e = hipMemcpyAsync(m->staging, src, count * 4,
                                          host ? hipMemcpyHostToDevice : hipMemcpyDeviceToDevice, s);
      if (e != hipSuccess) return hip_fail("upload_input copy", e);
      m->staged = true;
    } else {
      if (host) {
        const hipError_t e = hipMemcpyAsync(m->staging, src, count * 4, hipMemcpyHostToDevice, s);
        if (e != hipSuccess) return hip_fail("upload_input copy", e);
        x = m->staging;
      }
      if (aih_pack_nhwc_device(x, m->n, t.h, t.w, t.c, m->dt, m->ptr((uint32_t)tid), stream)) return AIH_ERR;
    }
    if (host) {
      const hipError_t e = hipStreamSynchronize(s);
      if (e != hipSuccess) return hip_fail("upload_input", e);
    }
    return AIH_OK;
  });
}

int aih_model_upload_input(aih_model *m, const char *name, const float *host_nhwc, size_t count, aih_stream stream) {
  return upload(m, name, host_nhwc, count, true, stream);
}

int aih_model_upload_input_device(aih_model *m, const char *name, const float *dev_nhwc, size_t count,
                                  aih_stream stream) {
  return upload(m, name, dev_nhwc, count, false, stream);
}

int aih_model_infer(aih_model *m, aih_stream stream) {
  return api_guarded([&] {
    if (!m) return api_fail("infer: null model");
    hipStream_t s = static_cast<hipStream_t>(stream);
    for (size_t i = 0; i < m->launches.size(); ++i)
      if (m->launches[i] && m->launches[i](s) != AIH_OK)
        return api_fail("infer: op " + std::to_string(i) + ": " + aih_last_error());
    return AIH_OK;
  });
}

int aih_model_infer_range(aih_model *m, uint32_t first, uint32_t last, aih_stream stream) {
  return api_guarded([&] {
    if (!m) return api_fail("infer_range: null model");
    if (first > last || last > m->launches.size()) return api_fail("infer_range: bad op range");
    for (uint32_t e : {first, last})
      if (e < m->block_of.size() && m->block_of[e] >= 0 && m->fused[(size_t)m->block_of[e]].first != e)
        return api_fail("infer_range: op " + std::to_string(e) + " is inside the fused block of ops " +
                        std::to_string(m->fused[(size_t)m->block_of[e]].first) + "..; a range holds all of it or none");
    hipStream_t s = static_cast<hipStream_t>(stream);
    for (uint32_t i = first; i < last; ++i)
      if (m->launches[i] && m->launches[i](s) != AIH_OK)
        return api_fail("infer: op " + std::to_string(i) + ": " + aih_last_error());
    return AIH_OK;
  });
}

int aih_model_read_output(aih_model *m, const char *name, float *host_nhwc, size_t count, aih_stream stream) {
  return api_guarded([&] {
    if (!m || !host_nhwc) return api_fail("read_output: null argument");
    const int64_t tid = m->find(name);
    if (tid < 0) return api_fail(std::string("read_output: no tensor named '") + (name ? name : "") + "'");
    m->need_stored((uint32_t)tid, "read_output");
    if ((uint32_t)tid == m->stem_tid && settle_input(m, stream)) return AIH_ERR;
    const auto &t = m->g.tensors[tid];
    const size_t want = (size_t)m->n * t.h * t.w * t.c;
    if (count != want) return api_fail("read_output: expected " + std::to_string(want) + " floats");
    const aih_model::View &v = m->views[tid];
    hipError_t e = hipStreamSynchronize(static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail("read_output", e);
    std::vector<uint8_t> buf(v.bytes);
    e = hipMemcpy(buf.data(), v.base, v.bytes, hipMemcpyDeviceToHost);
    if (e != hipSuccess) return hip_fail("read_output copy", e);
    const size_t es = es_of(m->dt);
    const size_t px = (size_t)m->n * t.h * t.w;
    for (size_t p = 0; p < px; ++p)
      for (uint32_t ch = 0; ch < t.c; ++ch) {
        const uint8_t *q = buf.data() + (p * v.stride_c + v.c_off + ch) * es;
        float f;
        if (m->dt == AIH_F32) {
          std::memcpy(&f, q, 4);
        } else {
          uint16_t h;
          std::memcpy(&h, q, 2);
          f = m->dt == AIH_F16 ? f16_bits_to_f32(h) : bf16_bits_to_f32(h);
        }
        host_nhwc[p * t.c + ch] = f;
      }
    return AIH_OK;
  });
}

int aih_model_write_tensor(aih_model *m, const char *name, const float *host_nhwc, size_t count,
                           aih_stream stream) {
  return api_guarded([&] {
    if (!m || !host_nhwc) return api_fail("write_tensor: null argument");
    const int64_t tid = m->find(name);
    if (tid < 0) return api_fail(std::string("write_tensor: no tensor named '") + (name ? name : "") + "'");
    m->need_stored((uint32_t)tid, "write_tensor");
    if ((uint32_t)tid == m->stem_tid && settle_input(m, stream)) return AIH_ERR;
    const auto &t = m->g.tensors[tid];
    const size_t want = (size_t)m->n * t.h * t.w * t.c;
    if (count != want) return api_fail("write_tensor: expected " + std::to_string(want) + " floats");
    const aih_model::View &v = m->views[tid];
    hipError_t e = hipStreamSynchronize(static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail("write_tensor", e);
    std::vector<uint8_t> buf(v.bytes);
    e = hipMemcpy(buf.data(), v.base, v.bytes, hipMemcpyDeviceToHost);
    if (e != hipSuccess) return hip_fail("write_tensor read", e);
    const size_t es = es_of(m->dt);
    const size_t px = (size_t)m->n * t.h * t.w;
    for (size_t p = 0; p < px; ++p)
      for (uint32_t ch = 0; ch < t.c; ++ch) {
        uint8_t *q = buf.data() + (p * v.stride_c + v.c_off + ch) * es;
        const float f = host_nhwc[p * t.c + ch];
        if (m->dt == AIH_F32) {
          std::memcpy(q, &f, 4);
        } else {
          const uint16_t h = m->dt == AIH_F16 ? f32_to_f16_bits(f) : f32_to_bf16_bits(f);
          std::memcpy(q, &h, 2);
        }
      }
    e = hipMemcpy(v.base, buf.data(), v.bytes, hipMemcpyHostToDevice);
    if (e != hipSuccess) return hip_fail("write_tensor write", e);
    return AIH_OK;
  });
}

int aih_model_reset(aih_model *m, aih_stream stream) {
  return api_guarded([&] {
    if (!m) return api_fail("reset: null model");
    for (const auto &st : m->g.states)
      for (uint32_t tid : {st.first, st.second}) {
        const aih_model::View &v = m->views[tid];
        const hipError_t e = hipMemsetAsync(v.base, 0, v.bytes, static_cast<hipStream_t>(stream));
        if (e != hipSuccess) return hip_fail("reset", e);
      }
    return AIH_OK;
  });
}

int aih_model_tensor(const aih_model *m, const char *name, aih_tensor_info *out) {
  return api_guarded([&] {
    if (!m || !out) return api_fail("tensor: null argument");
    const int64_t tid = m->find(name);
    if (tid < 0) return api_fail(std::string("tensor: no tensor named '") + (name ? name : "") + "'");
    m->need_stored((uint32_t)tid, "tensor");
    if ((uint32_t)tid == m->stem_tid && m->staged) {
      // the caller may read or write the slot directly from now on: it holds
      // the last upload, and infer reads it
      if (settle_input(m, nullptr)) return AIH_ERR;
      const hipError_t e = hipStreamSynchronize(nullptr);
      if (e != hipSuccess) return hip_fail("tensor", e);
    }
    const auto &t = m->g.tensors[tid];
    const aih_model::View &v = m->views[tid];
    const size_t skip = (size_t)v.c_off * es_of(m->dt);
    *out = aih_tensor_info{v.base + skip, v.bytes - skip, m->n, t.h, t.w, t.c, v.stride_c, m->dt};
    return AIH_OK;
  });
}

int aih_model_get_info(const aih_model *m, aih_model_info *out) {
  return api_guarded([&] {
    if (!m || !out) return api_fail("info: null argument");
    uint32_t nl = 0;
    for (const auto &f : m->launches) nl += f ? 1u : 0u;
    *out = aih_model_info{(uint32_t)m->g.tensors.size(), (uint32_t)m->g.ops.size(), (uint32_t)m->g.inputs.size(),
                          (uint32_t)m->g.outputs.size(), nl, (uint32_t)m->fused.size(), m->dt, m->wdt,
                          m->device_bytes};
    return AIH_OK;
  });
}

int aih_model_fused_block(const aih_model *m, uint32_t i, aih_model_fused_info *out) {
  return api_guarded([&] {
    if (!m || !out) return api_fail("fused_block: null argument");
    if (i >= m->fused.size()) return api_fail("fused_block: no fused block " + std::to_string(i));
    const aih_model::Fused &f = m->fused[i];
    *out = aih_model_fused_info{f.first, f.nops, f.plan, f.dpp, f.kind};
    return AIH_OK;
  });
}

const char *aih_model_input_name(const aih_model *m, uint32_t i) {
  return m && i < m->g.inputs.size() ? m->g.tensors[m->g.inputs[i]].name.c_str() : nullptr;
}

const char *aih_model_output_name(const aih_model *m, uint32_t i) {
  return m && i < m->g.outputs.size() ? m->g.tensors[m->g.outputs[i]].name.c_str() : nullptr;
}

int aih_sw_describe(const void *bytes, size_t len, char *buf, size_t buflen) {
  return api_guarded([&] {
    sw::Container c = sw::parse_container(bytes, len);
    sw::Model g = sw::parse_model(c.json, c.json_len);
    validate_geometry(g);
    int counts[5] = {0, 0, 0, 0, 0};
    for (const auto &op : g.ops) ++counts[op.kind];
    int aliases = 0;
    for (const auto &t : g.tensors) aliases += t.alias_of >= 0;
    char tmp[1024];
    const std::string qname = json_quote(g.name.substr(0, 256));
    const int k = std::snprintf(
        tmp, sizeof(tmp),
        "{\"name\": %s, \"h\": %u, \"w\": %u, \"dt_default\": \"%s\", \"dt_weights\": \"%s\", \"tensors\": %zu, "
        "\"aliases\": %d, \"inputs\": %zu, \"outputs\": %zu, \"ops\": %zu, \"conv\": %d, \"binary\": %d, \"gpool\": %d, "
        "\"resize\": %d, \"concat\": %d, \"json_bytes\": %zu, \"blob_bytes\": %zu}",
        qname.c_str(), g.size_h, g.size_w, g.dt_default == sw::F16 ? "f16" : "f32",
        g.dt_weights == sw::F16 ? "f16" : "f32", g.tensors.size(), aliases, g.inputs.size(), g.outputs.size(),
        g.ops.size(), counts[sw::OP_CONV], counts[sw::OP_BINARY], counts[sw::OP_GPOOL], counts[sw::OP_RESIZE],
        counts[sw::OP_CONCAT], c.json_len, c.blob_len);
    if (k < 0 || (size_t)k >= sizeof(tmp)) return api_fail("describe: summary too long");
    if (!buf || buflen <= (size_t)k) return api_fail("describe: buffer too small");
    std::memcpy(buf, tmp, (size_t)k + 1);
    return k;
  });
}

}  // extern "C"

// sw_format.h -- the .sw container (crates/ai-core/src/format/header.rs:1-86)
// and the part of its JSON graph schema (crates/ai-core/src/format/model.rs:
// 20-320) this backend runs: tensors with channel-group aliases, Conv (with
// concat parts and residual), Binary, Gpool, Resize and Concat. Host code only.
#pragma once

#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

#include "sw_json.h"

namespace aih {
namespace sw {

// header.rs:18-22
constexpr char kMagic[4] = {'S', 'W', '1', '\0'};
constexpr uint32_t kVersion = 1;
constexpr size_t kHeaderLen = 32;

struct Error : std::runtime_error {
  using std::runtime_error::runtime_error;
};

// parse_container (header.rs:58-86): magic, version, JSON range, blob at the
// JSON end rounded up to blob_align.
struct Container {
  const char *json = nullptr;
  size_t json_len = 0;
  const uint8_t *blob = nullptr;
  size_t blob_len = 0;
};

inline Container parse_container(const void *bytes, size_t len) {
  const uint8_t *b = static_cast<const uint8_t *>(bytes);
  if (!b || len < kHeaderLen) throw Error(".sw: truncated (header)");
  if (std::memcmp(b, kMagic, 4) != 0) throw Error(".sw: bad magic (not a .sw container)");
  auto u32 = [&](size_t o) {
    uint32_t v;
    std::memcpy(&v, b + o, 4);
    return v;
  };
  auto u64 = [&](size_t o) {
    uint64_t v;
    std::memcpy(&v, b + o, 8);
    return v;
  };
  const uint32_t version = u32(4);
  if (version != kVersion) throw Error(".sw: unsupported version " + std::to_string(version) + " (supported: 1)");
  const uint64_t align = u32(12) ? u32(12) : 1;
  const uint64_t json_off = u64(16), json_len = u64(24);
  if (json_off > len || json_len > len - json_off) throw Error(".sw: truncated (json)");
  const uint64_t json_end = json_off + json_len;
  const uint64_t blob_off = (json_end + align - 1) / align * align;
  if (blob_off > len) throw Error(".sw: truncated (blob)");
  Container c;
  c.json = reinterpret_cast<const char *>(b + json_off);
  c.json_len = (size_t)json_len;
  c.blob = b + blob_off;
  c.blob_len = (size_t)(len - blob_off);
  return c;
}

enum DType : int32_t { F32 = 0, F16 = 1 };  // tensor.rs:10-16 (the file has no bf16)

struct WRef {
  uint64_t off = 0, len = 0;
};

struct Tensor {
  std::string name;
  uint32_t h = 0, w = 0, c = 0;
  int32_t dt = F32;
  int64_t alias_of = -1;  // SwAlias{of, cg_off} (model.rs:29-35)
  uint32_t cg_off = 0;
  uint32_t last_use = 0;
};

struct Part {  // SwConcatPart (model.rs:226-232)
  uint32_t tid = 0, c = 0;
};

enum OpKind { OP_CONV, OP_BINARY, OP_GPOOL, OP_RESIZE, OP_CONCAT };
enum BinOp : int32_t { BIN_ADD = 0, BIN_SUB = 1, BIN_MUL = 2, BIN_PRELU = 3 };  // ops/elementwise.rs:5-11
// SwOperand (model.rs:60-78)
enum OperandKind : int32_t { OPND_TENSOR = 0, OPND_SCALAR = 1, OPND_CVEC = 2, OPND_CVEC_TENSOR = 3,
                             OPND_PVEC_TENSOR = 4, OPND_TILED_TENSOR = 5 };
enum Coord : int32_t { COORD_HALF_PIXEL = 0, COORD_ASYMMETRIC = 1 };  // ops/resize.rs:6-11

struct Op {
  OpKind kind = OP_CONV;
  uint32_t in = 0, out = 0;
  std::vector<Part> srcs;  // Conv / Resize concat parts, Concat parts
  // Conv (model.rs:82-111)
  int64_t res = -1;
  uint32_t cin = 0, cout = 0, kh = 0, kw = 0, sh = 0, sw = 0, pad[4] = {0, 0, 0, 0}, d = 1, groups = 1;
  int32_t act = 0;
  WRef w, b;
  uint32_t kg_pad = 0;
  // Binary (model.rs:112-118)
  int32_t bin = BIN_ADD;
  int32_t opnd = OPND_TENSOR;
  uint32_t b_tid = 0;
  float scalar = 0;
  bool scalar_first = false;
  WRef cvec;
  uint32_t cvec_c = 0;
  // Resize (model.rs:150-159)
  uint32_t oh = 0, ow = 0;
  int32_t coord = COORD_HALF_PIXEL;
};

struct Model {
  std::string name;
  uint32_t size_h = 0, size_w = 0;
  int32_t dt_default = F32, dt_weights = F32;
  std::vector<Tensor> tensors;
  std::vector<uint32_t> inputs, outputs;
  std::vector<std::pair<uint32_t, uint32_t>> states;  // SwState{input, output}
  std::vector<std::pair<uint32_t, WRef>> consts;      // SwConst{tid, w}
  std::vector<Op> ops;

  // resolve_alias (model.rs:300-307): tid -> (backing tid, accumulated cg_off)
  std::pair<uint32_t, uint32_t> resolve(uint32_t tid) const {
    uint32_t cg = 0;
    for (size_t guard = 0; tensors.at(tid).alias_of >= 0; ++guard) {
      if (guard > tensors.size()) throw Error(".sw: alias cycle");
      cg += tensors[tid].cg_off;
      tid = (uint32_t)tensors[tid].alias_of;
    }
    return {tid, cg};
  }
};

inline int32_t parse_dtype(const json::Value &v) {
  const std::string &s = v.s();
  if (s == "f32") return F32;
  if (s == "f16") return F16;
  throw Error(".sw: unknown dtype '" + s + "'");
}

// activation.rs:5-25 (serde lowercase names) -> enum aih_act (same order)
inline int32_t parse_act(const json::Value &v) {
  static const char *names[] = {"none", "relu", "sigmoid", "tanh", "hardswish", "hardsigmoid",
                                "clamp01", "relu6", "sqrt", "neg", "recip"};
  const std::string &s = v.s();
  for (int i = 0; i < 11; ++i)
    if (s == names[i]) return i;
  throw Error(".sw: unknown activation '" + s + "'");
}

inline WRef parse_wref(const json::Value &v) {
  WRef r;
  r.off = v["off"].u64();
  r.len = v["len"].u64();
  return r;
}

inline std::vector<Part> parse_parts(const json::Value &v) {
  std::vector<Part> out;
  for (size_t i = 0; i < v.size(); ++i) out.push_back(Part{v.at(i)["in"].u32(), v.at(i)["c"].u32()});
  return out;
}

inline Op parse_op(const json::Value &v) {
  Op op;
  const std::string &kind = v["kind"].s();
  if (kind == "conv") {
    op.kind = OP_CONV;
    op.in = v["in"].u32();
    op.out = v["out"].u32();
    if (v.has("srcs")) op.srcs = parse_parts(v["srcs"]);
    if (v.has("res") && !v["res"].is_null()) op.res = v["res"].u32();
    op.cin = v["cin"].u32();
    op.cout = v["cout"].u32();
    op.kh = v["kh"].u32();
    op.kw = v["kw"].u32();
    op.sh = v["sh"].u32();
    op.sw = v["sw"].u32();
    for (int i = 0; i < 4; ++i) op.pad[i] = v["pad"].at(i).u32();
    op.d = v.has("d") ? v["d"].u32() : 1;  // default_dil (model.rs:17-19)
    op.groups = v["groups"].u32();
    op.act = parse_act(v["act"]);
    op.w = parse_wref(v["w"]);
    op.b = parse_wref(v["b"]);
    op.kg_pad = v["kg_pad"].u32();
  } else if (kind == "binary") {
    op.kind = OP_BINARY;
    op.in = v["a"].u32();
    op.out = v["out"].u32();
    const std::string &bo = v["op"].s();
    if (bo == "add") op.bin = BIN_ADD;
    else if (bo == "sub") op.bin = BIN_SUB;
    else if (bo == "mul") op.bin = BIN_MUL;
    else if (bo == "prelu") op.bin = BIN_PRELU;
    else throw Error(".sw: unknown binary op '" + bo + "'");
    op.act = parse_act(v["act"]);
    const json::Value &b = v["b"];
    if (b.kind != json::Value::Object || b.size() != 1) throw Error(".sw: binary operand must be one tagged object");
    const std::string &t = b.obj[0].first;
    const json::Value &bv = b.obj[0].second;
    if (t == "tensor") { op.opnd = OPND_TENSOR; op.b_tid = bv["tid"].u32(); }
    else if (t == "scalar") { op.opnd = OPND_SCALAR; op.scalar = bv["v"].f32(); op.scalar_first = bv["first"].b; }
    else if (t == "cvec") { op.opnd = OPND_CVEC; op.cvec = parse_wref(bv["w"]); op.cvec_c = bv["c"].u32(); }
    else if (t == "cvectensor") { op.opnd = OPND_CVEC_TENSOR; op.b_tid = bv["tid"].u32(); }
    else if (t == "pvectensor") { op.opnd = OPND_PVEC_TENSOR; op.b_tid = bv["tid"].u32(); }
    else if (t == "tiledtensor") { op.opnd = OPND_TILED_TENSOR; op.b_tid = bv["tid"].u32(); }
    else throw Error(".sw: unknown binary operand '" + t + "'");
  } else if (kind == "gpool") {
    op.kind = OP_GPOOL;
    op.in = v["in"].u32();
    op.out = v["out"].u32();
  } else if (kind == "resize") {
    op.kind = OP_RESIZE;
    op.in = v["in"].u32();
    op.out = v["out"].u32();
    if (v.has("srcs")) op.srcs = parse_parts(v["srcs"]);
    op.oh = v["oh"].u32();
    op.ow = v["ow"].u32();
    const std::string &m = v["mode"].s();
    if (m == "half_pixel") op.coord = COORD_HALF_PIXEL;
    else if (m == "asymmetric") op.coord = COORD_ASYMMETRIC;
    else throw Error(".sw: unknown resize mode '" + m + "'");
  } else if (kind == "concat") {
    op.kind = OP_CONCAT;
    op.out = v["out"].u32();
    op.srcs = parse_parts(v["parts"]);
    if (op.srcs.empty()) throw Error(".sw: concat without parts");
    op.in = op.srcs[0].tid;
  } else {
    throw Error(".sw: op kind '" + kind + "' is not supported by this backend");
  }
  return op;
}

// SwModel::from_json (model.rs:265-267) for the supported subset, with the
// tensor-id checks a graph needs before anything indexes with them.
inline Model parse_model(const char *json_text, size_t json_len) {
  json::Value root;
  try {
    root = json::parse(json_text, json_len);
  } catch (const std::exception &e) {
    throw Error(std::string(".sw: ") + e.what());
  }
  Model m;
  try {
    m.name = root["name"].s();
    m.size_h = root["size"]["h"].u32();
    m.size_w = root["size"]["w"].u32();
    m.dt_default = parse_dtype(root["dt_default"]);
    m.dt_weights = root.has("dt_weights") && !root["dt_weights"].is_null() ? parse_dtype(root["dt_weights"])
                                                                           : m.dt_default;
    const json::Value &ts = root["tensors"];
    for (size_t i = 0; i < ts.size(); ++i) {
      const json::Value &t = ts.at(i);
      Tensor x;
      x.name = t["name"].s();
      x.h = t["h"].u32();
      x.w = t["w"].u32();
      x.c = t["c"].u32();
      x.dt = parse_dtype(t["dt"]);
      if (t.has("alias") && !t["alias"].is_null()) {
        x.alias_of = t["alias"]["of"].u32();
        x.cg_off = t["alias"]["cg_off"].u32();
      }
      x.last_use = t["last_use"].u32();
      m.tensors.push_back(std::move(x));
    }
    for (size_t i = 0; i < root["inputs"].size(); ++i) m.inputs.push_back(root["inputs"].at(i).u32());
    for (size_t i = 0; i < root["outputs"].size(); ++i) m.outputs.push_back(root["outputs"].at(i).u32());
    if (root.has("states"))
      for (size_t i = 0; i < root["states"].size(); ++i)
        m.states.emplace_back(root["states"].at(i)["input"].u32(), root["states"].at(i)["output"].u32());
    if (root.has("consts") && !root["consts"].is_null())
      for (size_t i = 0; i < root["consts"].size(); ++i)
        m.consts.emplace_back(root["consts"].at(i)["tid"].u32(), parse_wref(root["consts"].at(i)["w"]));
    const json::Value &ops = root["ops"];
    for (size_t i = 0; i < ops.size(); ++i) m.ops.push_back(parse_op(ops.at(i)));
  } catch (const Error &) {
    throw;
  } catch (const std::exception &e) {
    throw Error(std::string(".sw: ") + e.what());
  }
  const size_t nt = m.tensors.size();
  auto chk = [&](uint64_t tid, const char *what) {
    if (tid >= nt) throw Error(std::string(".sw: ") + what + " refers to tensor " + std::to_string(tid) + " of " +
                               std::to_string(nt));
  };
  for (auto &t : m.tensors)
    if (t.alias_of >= 0) chk((uint64_t)t.alias_of, "alias");
  for (uint32_t t : m.inputs) chk(t, "inputs");
  for (uint32_t t : m.outputs) chk(t, "outputs");
  for (auto &s : m.states) chk(s.first, "states"), chk(s.second, "states");
  for (auto &c : m.consts) chk(c.first, "consts");
  for (auto &op : m.ops) {
    chk(op.in, "op input");
    chk(op.out, "op output");
    for (auto &p : op.srcs) chk(p.tid, "op part");
    if (op.res >= 0) chk((uint64_t)op.res, "op residual");
    if (op.kind == OP_BINARY && op.opnd != OPND_SCALAR && op.opnd != OPND_CVEC) chk(op.b_tid, "binary operand");
  }
  for (size_t i = 0; i < nt; ++i) m.resolve((uint32_t)i);  // rejects alias cycles
  return m;
}

}  // namespace sw
}  // namespace aih

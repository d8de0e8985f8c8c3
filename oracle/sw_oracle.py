"""CPU restatement of a .sw graph run (TEST INFRASTRUCTURE).

Only tests/, the smoke check and bench.py's cpu_baseline leg use this module;
the product never does. It reads a .sw container with its own parser
(crates/ai-core/src/format/header.rs:58-86, format/model.rs:79-307) and runs
the graph op by op on logical NHWC fp32 arrays, n images at a time:

* Conv      -> the ai-cpu restatement (oracle.CpuConv: plan.rs:462-614 routing,
               kernels/conv.rs, dw.rs, pw_dot.rs, im2row.rs); concat parts are
               materialised first, which ai-cpu's own tests hold equivalent
               (kernels/conv.rs:572-627);
* Binary    -> reference/elementwise.rs:7-30 with the operand kinds of
               ai-cpu model.rs:478-507;
* Gpool     -> reference/pool.rs:6-19;
* Resize    -> reference/resize.rs:6-44 (concat parts as ai-cpu resize.rs:1-20);
* Concat    -> channel concatenation (format/model.rs:160-164);
* aliases   -> channel slices of their backing tensor (model.rs:29-35,300-307).
Weights are read out of the blob with the oracle's unpack functions (pack.rs).
"""
from __future__ import annotations

import json
import struct

import numpy as np

from . import oracle as orc


def read_container(data: bytes) -> tuple[dict, bytes]:
    if len(data) < 32 or data[:4] != b"SW1\0":
        raise ValueError(".sw: bad magic or truncated header")
    version, _flags, align, joff, jlen = struct.unpack_from("<IIIQQ", data, 4)
    if version != 1:
        raise ValueError(f".sw: unsupported version {version}")
    align = max(align, 1)
    if joff + jlen > len(data):
        raise ValueError(".sw: truncated json")
    blob_off = -(-(joff + jlen) // align) * align
    if blob_off > len(data):
        raise ValueError(".sw: truncated blob")
    return json.loads(data[joff:joff + jlen]), data[blob_off:]


def _f32(blob: bytes, ref: dict) -> np.ndarray:
    return np.frombuffer(blob, np.float32, count=ref["len"] // 4, offset=ref["off"]).copy()


def act_np(act: str, x: np.ndarray) -> np.ndarray:
    """Activation::apply (activation.rs:28-43), elementwise."""
    x = x.astype(np.float32)
    with np.errstate(over="ignore", divide="ignore", invalid="ignore"):
        if act == "none":
            return x
        if act == "relu":
            return np.maximum(x, np.float32(0))
        if act == "sigmoid":
            return (np.float32(1) / (np.float32(1) + np.exp(-x))).astype(np.float32)
        if act == "tanh":
            return np.tanh(x).astype(np.float32)
        if act == "hardswish":
            return (x * np.clip(x / np.float32(6) + np.float32(0.5), 0, 1)).astype(np.float32)
        if act == "hardsigmoid":
            return np.clip(x / np.float32(6) + np.float32(0.5), 0, 1).astype(np.float32)
        if act == "clamp01":
            return np.clip(x, 0, 1).astype(np.float32)
        if act == "relu6":
            return np.clip(x, 0, 6).astype(np.float32)
        if act == "sqrt":
            return np.sqrt(np.maximum(x, 0)).astype(np.float32)
        if act == "neg":
            return -x
        if act == "recip":
            return (np.float32(1) / x).astype(np.float32)
    raise ValueError(f"unknown activation {act}")


def binop_np(op: str, a: np.ndarray, b) -> np.ndarray:
    """BinaryOp::apply (ops/elementwise.rs:14-27)."""
    if op == "add":
        return (a + b).astype(np.float32)
    if op == "sub":
        return (a - b).astype(np.float32)
    if op == "mul":
        return (a * b).astype(np.float32)
    if op == "prelu":
        return np.where(a > 0, a, a * b).astype(np.float32)
    raise ValueError(f"unknown binary op {op}")


def global_avg_pool(x: np.ndarray) -> np.ndarray:
    """reference/pool.rs:6-19 over [n, h, w, c]: sequential fp32 sum over the
    pixels, then times 1/(h*w)."""
    n, h, w, c = x.shape
    acc = np.zeros((n, c), np.float32)
    flat = x.reshape(n, h * w, c)
    for i in range(h * w):
        acc += flat[:, i, :]
    return (acc * np.float32(1.0 / (h * w))).reshape(n, 1, 1, c)


def resize_bilinear(x: np.ndarray, oh: int, ow: int, mode: str) -> np.ndarray:
    """reference/resize.rs:6-44 over [n, h, w, c]."""
    n, ih, iw, c = x.shape
    sy, sx = np.float32(ih) / np.float32(oh), np.float32(iw) / np.float32(ow)

    def coords(o, scale, size):
        o = o.astype(np.float32)
        f = (o + np.float32(0.5)) * scale - np.float32(0.5) if mode == "half_pixel" else o * scale
        fl = np.floor(f)
        i0 = np.clip(fl.astype(np.int64), 0, size - 1)
        i1 = np.clip(fl.astype(np.int64) + 1, 0, size - 1)
        t = np.clip(f - fl, 0, 1).astype(np.float32)
        return i0, i1, t

    y0, y1, ty = coords(np.arange(oh), sy, ih)
    x0, x1, tx = coords(np.arange(ow), sx, iw)
    tx = tx[None, None, :, None]
    ty = ty[None, :, None, None]
    g = lambda ys, xs: x[:, ys][:, :, xs]
    top = g(y0, x0) * (np.float32(1) - tx) + g(y0, x1) * tx
    bot = g(y1, x0) * (np.float32(1) - tx) + g(y1, x1) * tx
    return (top * (np.float32(1) - ty) + bot * ty).astype(np.float32)


class SwGraph:
    """A parsed .sw graph with its convs prepared for the ai-cpu oracle."""

    def __init__(self, data: bytes, round_dt: int | None = None):
        """round_dt (oracle.F16 / oracle.BF16): emulate 16-bit storage -- the
        weights, the input and every op's output rounded to that dtype (round
        to nearest even), the arithmetic staying fp32."""
        self.round_dt = round_dt
        self.g, self.blob = read_container(data)
        self.T = self.g["tensors"]
        if self.g["dt_default"] != "f32" or self.g.get("dt_weights", "f32") not in (None, "f32"):
            raise ValueError("the oracle runs fp32 .sw files")
        self._convs = {}
        for k, op in enumerate(self.g["ops"]):
            if op["kind"] == "conv":
                self._convs[k] = self._conv(op)

    def resolve(self, tid: int) -> tuple[int, int]:
        cg = 0
        while self.T[tid].get("alias"):
            cg += self.T[tid]["alias"]["cg_off"]
            tid = self.T[tid]["alias"]["of"]
        return tid, cg

    def conv_weights(self, op: dict) -> tuple[np.ndarray, np.ndarray]:
        """OIHW weights and bias of a Conv op, unpacked from the blob (pack.rs)."""
        kh, kw, cin, cout = op["kh"], op["kw"], op["cin"], op["cout"]
        wp = _f32(self.blob, op["w"])
        if op["groups"] > 1:
            w = orc.unpack_weights_dw(wp, cout, kh, kw)
        else:
            w = orc.unpack_weights_conv(wp, cout, cin, kh, kw, op["kg_pad"])
        b = orc.unpack_bias(_f32(self.blob, op["b"]), cout)
        if getattr(self, "round_dt", None):
            w, b = self._rd(w), self._rd(b)
        return w, b

    def _rd(self, v):
        if not self.round_dt:
            return v
        return orc.round_to(np.asarray(v, np.float32), self.round_dt).reshape(np.shape(v))

    def _conv(self, op):
        src = op["srcs"][0]["in"] if op.get("srcs") else op["in"]
        ih, iw = self.T[src]["h"], self.T[src]["w"]
        w, b = self.conv_weights(op)
        c2 = orc.conv2d(op["cin"], op["cout"], kh=op["kh"], kw=op["kw"], sh=op["sh"], sw=op["sw"],
                        pad=list(op["pad"]), dil=op.get("d", 1), groups=op["groups"], act=op["act"])
        return orc.CpuConv(c2, ih, iw, w, b, has_res=op.get("res") is not None)

    def run(self, inputs: dict, n: int = 1, threads: int = 8, keep_all: bool = False) -> dict:
        """inputs: name -> [n, h, w, c] fp32. Returns name -> [n, h, w, c] of
        the graph outputs (every tensor with keep_all)."""
        vals: dict[int, np.ndarray] = {}
        names = {t["name"]: i for i, t in enumerate(self.T)}
        for name, x in inputs.items():
            t = self.T[names[name]]
            vals[names[name]] = self._rd(np.asarray(x, np.float32).reshape(n, t["h"], t["w"], t["c"]))

        def get(tid):
            base, cg = self.resolve(tid)
            if base == tid:
                return vals[tid]
            c = self.T[tid]["c"]
            return vals[base][..., cg * 4:cg * 4 + c]

        for k, op in enumerate(self.g["ops"]):
            kind = op["kind"]
            out_t = self.T[op["out"]]
            if kind == "conv":
                cv = self._convs[k]
                if op.get("srcs"):
                    x = np.concatenate([get(p["in"])[..., :p["c"]] for p in op["srcs"]], axis=-1)
                else:
                    x = get(op["in"])
                res = get(op["res"]) if op.get("res") is not None else None
                y = cv.run(np.ascontiguousarray(x).ravel(), n,
                           None if res is None else np.ascontiguousarray(res).ravel(), threads=threads)
                vals[op["out"]] = y.reshape(n, out_t["h"], out_t["w"], out_t["c"])
            elif kind == "binary":
                a = get(op["a"])
                (bk, bv), = op["b"].items()
                if bk == "tensor":
                    b = get(bv["tid"])
                elif bk == "scalar":
                    b = np.float32(bv["v"])
                elif bk == "cvec":
                    b = self._rd(_f32(self.blob, bv["w"])[:bv["c"]].reshape(1, 1, 1, -1))
                elif bk == "cvectensor":
                    t = get(bv["tid"]).reshape(n, -1)
                    b = t[:, :1].reshape(n, 1, 1, 1) if t.shape[1] == 1 else t.reshape(n, 1, 1, -1)
                elif bk == "pvectensor":
                    b = get(bv["tid"]).reshape(n, a.shape[1], a.shape[2], 1)
                elif bk == "tiledtensor":
                    t = get(bv["tid"]).reshape(n, -1)
                    L = t.shape[1]
                    b = t[:, np.arange(a.shape[3]) % L].reshape(n, 1, 1, -1)
                else:
                    raise ValueError(f"operand {bk}")
                if bk == "scalar" and bv.get("first"):
                    r = binop_np(op["op"], np.broadcast_to(b, a.shape), a)
                else:
                    r = binop_np(op["op"], a, b)
                vals[op["out"]] = act_np(op["act"], r)
            elif kind == "gpool":
                vals[op["out"]] = global_avg_pool(get(op["in"]))
            elif kind == "resize":
                parts = op.get("srcs") or [{"in": op["in"], "c": self.T[op["in"]]["c"]}]
                x = np.concatenate([get(p["in"])[..., :p["c"]] for p in parts], axis=-1)
                vals[op["out"]] = resize_bilinear(x, op["oh"], op["ow"], op["mode"])
            elif kind == "concat":
                vals[op["out"]] = np.concatenate([get(p["in"])[..., :p["c"]] for p in op["parts"]], axis=-1)
            else:
                raise ValueError(f"op kind {kind} is not restated")
            vals[op["out"]] = self._rd(vals[op["out"]])
        want = range(len(self.T)) if keep_all else self.g["outputs"]
        out = {}
        for tid in want:
            base, _ = self.resolve(tid)
            if base in vals:
                out[self.T[tid]["name"]] = np.ascontiguousarray(get(tid))
        return out

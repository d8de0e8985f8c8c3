"""Writes the real-weights fixtures of the .sw path (run in a container that
has the reference checkout at /root/reference; the outputs are committed):

* segm_r11_160x288.sw -- the reference converter's own output for the
  MobileNetV4-small segmentation model (reference: web/models/
  segm_r11_160x288.sw, built by `Makefile:83-86` from
  models/segm_mnv4s050_s2_160x288_nhwc.onnx), copied as data;
* segm_r11_onnx_convs.json -- for each Conv node of the ONNX twin
  (web/models/segm_mnv4s050_s2_160x288_nhwc.onnx), in graph order: its
  attributes and the shape and SHA-256 of its float32 weight (OIHW) and bias
  initializers. The ONNX file is read with the minimal protobuf wire-format
  reader below (onnx is not installed); only Conv nodes and float
  initializers are decoded.

The .sw and the ONNX list their 36 convs in the same order; unpacking each
conv's weight reference from the .sw must give the ONNX initializer bit for
bit (tests/test_sw_format.py checks it).
"""
from __future__ import annotations

import hashlib
import json
import os
import shutil
import struct

import numpy as np

REF = "/root/reference"
HERE = os.path.dirname(os.path.abspath(__file__))


def _varint(b: bytes, i: int) -> tuple[int, int]:
    r = s = 0
    while True:
        c = b[i]
        i += 1
        r |= (c & 0x7F) << s
        s += 7
        if c < 0x80:
            return r, i


def _fields(b: bytes):
    """(field number, wire type, value) of one protobuf message."""
    i = 0
    while i < len(b):
        key, i = _varint(b, i)
        f, wt = key >> 3, key & 7
        if wt == 0:
            v, i = _varint(b, i)
        elif wt == 1:
            v, i = b[i:i + 8], i + 8
        elif wt == 2:
            ln, i = _varint(b, i)
            v, i = b[i:i + ln], i + ln
        elif wt == 5:
            v, i = b[i:i + 4], i + 4
        else:
            raise ValueError(f"wire type {wt}")
        yield f, wt, v


def _ints(wt, v) -> list[int]:
    if wt == 0:
        return [v]
    out, j = [], 0
    while j < len(v):
        x, j = _varint(v, j)
        out.append(x)
    return out


def read_onnx(path: str):
    """ModelProto.graph (7): initializers (5, TensorProto) and nodes (1, NodeProto)."""
    data = open(path, "rb").read()
    graph = [v for f, _, v in _fields(data) if f == 7][0]
    inits, nodes = {}, []
    for f, _, v in _fields(graph):
        if f == 5:  # TensorProto: dims 1, data_type 2, float_data 4, name 8, raw_data 9
            dims, dt, name, raw, fd = [], None, None, None, []
            for f2, wt2, v2 in _fields(v):
                if f2 == 1:
                    dims += _ints(wt2, v2)
                elif f2 == 2:
                    dt = v2
                elif f2 == 8:
                    name = v2.decode()
                elif f2 == 9:
                    raw = v2
                elif f2 == 4:
                    fd += list(struct.unpack(f"<{len(v2) // 4}f", v2)) if wt2 == 2 else [struct.unpack("<f", v2)[0]]
            if dt == 1:  # FLOAT
                a = np.frombuffer(raw, np.float32) if raw is not None else np.array(fd, np.float32)
                inits[name] = a.reshape(dims)
        elif f == 1:  # NodeProto: input 1, output 2, op_type 4, attribute 5
            ins, op, attrs = [], None, {}
            for f2, wt2, v2 in _fields(v):
                if f2 == 1:
                    ins.append(v2.decode())
                elif f2 == 4:
                    op = v2.decode()
                elif f2 == 5:  # AttributeProto: name 1, i 3, ints 8
                    an, ai, aints = None, None, []
                    for f3, wt3, v3 in _fields(v2):
                        if f3 == 1:
                            an = v3.decode()
                        elif f3 == 3:
                            ai = v3
                        elif f3 == 8:
                            aints += _ints(wt3, v3)
                    attrs[an] = aints if aints else ai
            nodes.append((op, ins, attrs))
    return inits, nodes


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a, np.float32).tobytes()).hexdigest()


def main():
    sw_src = os.path.join(REF, "web", "models", "segm_r11_160x288.sw")
    shutil.copyfile(sw_src, os.path.join(HERE, "segm_r11_160x288.sw"))
    inits, nodes = read_onnx(os.path.join(REF, "web", "models", "segm_mnv4s050_s2_160x288_nhwc.onnx"))
    convs = []
    for op, ins, attrs in nodes:
        if op != "Conv":
            continue
        w = inits[ins[1]]
        b = inits[ins[2]] if len(ins) > 2 else np.zeros(w.shape[0], np.float32)
        convs.append(dict(weight=ins[1], shape=list(w.shape), weight_sha256=sha(w), bias_sha256=sha(b),
                          strides=attrs.get("strides"), pads=attrs.get("pads"), group=attrs.get("group", 1),
                          dilations=attrs.get("dilations")))
    with open(os.path.join(HERE, "segm_r11_onnx_convs.json"), "w") as f:
        json.dump(dict(source="web/models/segm_mnv4s050_s2_160x288_nhwc.onnx", convs=convs), f, indent=1)
    print(f"wrote {len(convs)} convs")


if __name__ == "__main__":
    main()

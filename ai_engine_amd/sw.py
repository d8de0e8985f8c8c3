"""The .sw model runtime and its non-conv ops, through include/aih_model.h.

`SwModel` mirrors ai_gpu_runtime::Model (crates/ai-gpu-runtime/src/model.rs):
`load` (Model::load, :56), `upload_input` (:387-399), `infer` (:402-426),
`read_output` (:442-457), `reset` (:368-385), `tensor` (input_storage /
output_storage, :465-478). The work happens in the native library
(ai_engine_amd/csrc/sw_model.hip); this module only binds it.

`write_container` and `conv_graph_to_sw` produce .sw containers in the
reference's format (crates/ai-core/src/format/header.rs:37-55,
format/model.rs:79-256) -- used to hand synthetic conv graphs to the native
loader exactly as the reference's converter would.
"""
from __future__ import annotations

import ctypes as C
import json
import struct

import numpy as np

from . import conv


class _Resize(C.Structure):
    _fields_ = [("n", C.c_uint32), ("ih", C.c_uint32), ("iw", C.c_uint32), ("oh", C.c_uint32),
                ("ow", C.c_uint32), ("mode", C.c_int32), ("dt", C.c_int32), ("nsrcs", C.c_uint32),
                ("srcs", conv._Src * 8)]


class _Gpool(C.Structure):
    _fields_ = [("n", C.c_uint32), ("h", C.c_uint32), ("w", C.c_uint32), ("c", C.c_uint32), ("dt", C.c_int32)]


class _Binary(C.Structure):
    _fields_ = [("n", C.c_uint32), ("h", C.c_uint32), ("w", C.c_uint32), ("c", C.c_uint32), ("op", C.c_int32),
                ("act", C.c_int32), ("dt", C.c_int32), ("operand", C.c_int32), ("scalar", C.c_float),
                ("scalar_first", C.c_int32), ("b_c", C.c_uint32)]


class _Concat(C.Structure):
    _fields_ = [("n", C.c_uint32), ("h", C.c_uint32), ("w", C.c_uint32), ("dt", C.c_int32),
                ("nparts", C.c_uint32), ("parts", conv._Src * 8)]


class _ResizeConcat(C.Structure):
    _fields_ = [("n", C.c_uint32), ("ih", C.c_uint32), ("iw", C.c_uint32), ("oh", C.c_uint32),
                ("ow", C.c_uint32), ("mode", C.c_int32), ("dt", C.c_int32), ("nparts", C.c_uint32),
                ("resized", C.c_uint32), ("parts", conv._Src * 8)]


class TensorInfo(C.Structure):
    _fields_ = [("data", C.c_void_p), ("bytes", C.c_size_t), ("n", C.c_uint32), ("h", C.c_uint32),
                ("w", C.c_uint32), ("c", C.c_uint32), ("stride_c", C.c_uint32), ("dt", C.c_int32)]


class ModelInfo(C.Structure):
    _fields_ = [("n_tensors", C.c_uint32), ("n_ops", C.c_uint32), ("n_inputs", C.c_uint32),
                ("n_outputs", C.c_uint32), ("n_launches", C.c_uint32), ("n_fused", C.c_uint32),
                ("dt", C.c_int32), ("wdt", C.c_int32), ("device_bytes", C.c_size_t)]


class FusedInfo(C.Structure):
    _fields_ = [("first_op", C.c_uint32), ("n_ops", C.c_uint32), ("plan", conv.IrPlan), ("dwpw", conv.DwPwPlan),
                ("kind", C.c_int32)]


# aih_fused_kind
FUSED_IR_BLOCK, FUSED_DWPW, FUSED_STEM_BLOCK, FUSED_BLOCK_HEAD, FUSED_RESIZE_CONCAT = range(5)


NO_FUSE, TUNE = 1, 2  # aih_model_flags


EXPORTS = (
    "aih_resize", "aih_gpool", "aih_binary", "aih_concat", "aih_resize_concat", "aih_model_load", "aih_model_load_ex", "aih_model_free",
    "aih_model_upload_input", "aih_model_upload_input_device", "aih_model_infer", "aih_model_infer_range",
    "aih_model_read_output", "aih_model_write_tensor", "aih_model_reset", "aih_model_tensor", "aih_model_get_info", "aih_model_input_name", "aih_model_output_name",
    "aih_sw_describe", "aih_model_fused_block",
)

COORD = {"half_pixel": 0, "asymmetric": 1}
BINOP = {"add": 0, "sub": 1, "mul": 2, "prelu": 3}
OPERAND = {"tensor": 0, "scalar": 1, "cvec": 2, "cvectensor": 3, "pvectensor": 4, "tiledtensor": 5}

_ready = None


def lib() -> C.CDLL:
    """The native library with the model / op signatures declared."""
    global _ready
    L = conv.lib()
    if _ready is L:
        return L
    P, u32, i32, sz = C.c_void_p, C.c_uint32, C.c_int32, C.c_size_t
    sigs = {
        "aih_resize": (C.c_int, [C.POINTER(_Resize), C.POINTER(P), P, P]),
        "aih_gpool": (C.c_int, [C.POINTER(_Gpool), P, P, P]),
        "aih_binary": (C.c_int, [C.POINTER(_Binary), P, P, P, P]),
        "aih_concat": (C.c_int, [C.POINTER(_Concat), C.POINTER(P), P, P]),
        "aih_resize_concat": (C.c_int, [C.POINTER(_ResizeConcat), C.POINTER(P), P, P]),
        "aih_model_load": (P, [C.c_char_p, sz, u32, i32]),
        "aih_model_load_ex": (P, [C.c_char_p, sz, u32, i32, u32]),
        "aih_model_fused_block": (C.c_int, [P, u32, C.POINTER(FusedInfo)]),
        "aih_model_free": (None, [P]),
        "aih_model_upload_input": (C.c_int, [P, C.c_char_p, P, sz, P]),
        "aih_model_upload_input_device": (C.c_int, [P, C.c_char_p, P, sz, P]),
        "aih_model_infer": (C.c_int, [P, P]),
        "aih_model_infer_range": (C.c_int, [P, u32, u32, P]),
        "aih_model_read_output": (C.c_int, [P, C.c_char_p, P, sz, P]),
        "aih_model_write_tensor": (C.c_int, [P, C.c_char_p, P, sz, P]),
        "aih_model_reset": (C.c_int, [P, P]),
        "aih_model_tensor": (C.c_int, [P, C.c_char_p, C.POINTER(TensorInfo)]),
        "aih_model_get_info": (C.c_int, [P, C.POINTER(ModelInfo)]),
        "aih_model_input_name": (C.c_char_p, [P, u32]),
        "aih_model_output_name": (C.c_char_p, [P, u32]),
        "aih_sw_describe": (C.c_int, [C.c_char_p, sz, C.c_char_p, sz]),
        "aih_conv_check": (C.c_int, [C.POINTER(conv._ConvDesc)]),
    }
    for name, (res, args) in sigs.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _ready = L
    return L


def describe(data: bytes) -> dict:
    """Parse a .sw container with the native reader (no device needed)."""
    buf = C.create_string_buffer(1024)
    k = lib().aih_sw_describe(data, len(data), buf, len(buf))
    if k < 0:
        raise conv.AihError(conv.last_error())
    return json.loads(buf.value.decode())


def _srcs(parts):
    arr = (conv._Src * 8)()
    for i, (c, stride_c, c_off) in enumerate(parts):
        arr[i] = conv._Src(c, stride_c, c_off)
    return arr


def _ptrs(ts):
    return (C.c_void_p * len(ts))(*[conv._ptr(t) for t in ts])


# ---------------------------------------------------------------- op entry points

def resize(x_parts, n, ih, iw, oh, ow, mode, dt, y, stream=None):
    """x_parts: [(tensor, c, stride_c, c_off)], concatenated into y along channels."""
    d = _Resize(n, ih, iw, oh, ow, COORD[mode] if isinstance(mode, str) else mode, int(dt), len(x_parts),
                _srcs([(c, s, o) for _, c, s, o in x_parts]))
    conv._check(lib().aih_resize(C.byref(d), _ptrs([p[0] for p in x_parts]), conv._ptr(y), conv._stream(stream)))
    return y


def gpool(x, n, h, w, c, dt, y, stream=None):
    d = _Gpool(n, h, w, c, int(dt))
    conv._check(lib().aih_gpool(C.byref(d), conv._ptr(x), conv._ptr(y), conv._stream(stream)))
    return y


def binary(a, b, n, h, w, c, op, act, dt, y, operand="tensor", scalar=0.0, scalar_first=False, b_c=0,
           stream=None):
    d = _Binary(n, h, w, c, BINOP[op] if isinstance(op, str) else op, int(act), int(dt),
                OPERAND[operand] if isinstance(operand, str) else operand, float(scalar), int(bool(scalar_first)),
                b_c)
    conv._check(lib().aih_binary(C.byref(d), conv._ptr(a), conv._ptr(b), conv._ptr(y), conv._stream(stream)))
    return y


def concat(parts, n, h, w, dt, y, stream=None):
    """parts: [(tensor, c, stride_c, c_off)]."""
    d = _Concat(n, h, w, int(dt), len(parts), _srcs([(c, s, o) for _, c, s, o in parts]))
    conv._check(lib().aih_concat(C.byref(d), _ptrs([p[0] for p in parts]), conv._ptr(y), conv._stream(stream)))
    return y


def resize_concat(parts, n, ih, iw, oh, ow, mode, dt, y, stream=None):
    """parts: [(tensor, c, stride_c, c_off, resized)]; a resized part is read at
    ih x iw and resized to oh x ow, any other is copied at oh x ow."""
    mask = sum(1 << i for i, p in enumerate(parts) if p[4])
    d = _ResizeConcat(n, ih, iw, oh, ow, COORD[mode] if isinstance(mode, str) else mode, int(dt), len(parts), mask,
                      _srcs([(c, s, o) for _, c, s, o, _ in parts]))
    conv._check(lib().aih_resize_concat(C.byref(d), _ptrs([p[0] for p in parts]), conv._ptr(y),
                                        conv._stream(stream)))
    return y


# ---------------------------------------------------------------- model

class SwModel:
    """A .sw model resident on the current HIP device (batch n, outermost).
    fuse=False lowers every op on its own (AIH_MODEL_NO_FUSE); by default each
    inverted-residual block runs as one fused launch. tune=True times each
    fused block's launch options at load and keeps the fastest
    (AIH_MODEL_TUNE)."""

    def __init__(self, data: bytes, n: int = 1, dt: conv.DType | None = None, fuse: bool = True,
                 tune: bool = False):
        L = lib()
        self._h = L.aih_model_load_ex(bytes(data), len(data), n, -1 if dt is None else int(dt),
                                      (0 if fuse else NO_FUSE) | (TUNE if tune else 0))
        if not self._h:
            raise conv.AihError(conv.last_error())
        self.n = n
        info = ModelInfo()
        conv._check(L.aih_model_get_info(self._h, C.byref(info)))
        self.info = info
        self.dt = conv.DType(info.dt)
        self.inputs = [L.aih_model_input_name(self._h, i).decode() for i in range(info.n_inputs)]
        self.outputs = [L.aih_model_output_name(self._h, i).decode() for i in range(info.n_outputs)]

    def close(self):
        if getattr(self, "_h", None):
            lib().aih_model_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:  # interpreter shutdown
            pass

    def fused_blocks(self) -> list[FusedInfo]:
        out = []
        for i in range(self.info.n_fused):
            f = FusedInfo()
            conv._check(lib().aih_model_fused_block(self._h, i, C.byref(f)))
            out.append(f)
        return out

    def tensor(self, name: str) -> TensorInfo:
        t = TensorInfo()
        conv._check(lib().aih_model_tensor(self._h, name.encode(), C.byref(t)))
        return t

    def upload_input(self, name: str, x, stream=None):
        """x: logical NHWC fp32, a numpy array (host) or a torch CUDA tensor."""
        if isinstance(x, np.ndarray):
            a = np.ascontiguousarray(x, np.float32)
            conv._check(lib().aih_model_upload_input(self._h, name.encode(), a.ctypes.data, a.size,
                                                     conv._stream(stream)))
        else:
            x = x.contiguous()
            conv._check(lib().aih_model_upload_input_device(self._h, name.encode(), x.data_ptr(), x.numel(),
                                                            conv._stream(stream)))

    def infer(self, stream=None):
        conv._check(lib().aih_model_infer(self._h, conv._stream(stream)))

    def infer_range(self, first: int, last: int, stream=None):
        conv._check(lib().aih_model_infer_range(self._h, first, last, conv._stream(stream)))

    def write_tensor(self, name: str, x: np.ndarray, stream=None):
        """Overwrite any tensor (a channel view too) with logical NHWC fp32
        values; the copy completes before the call returns."""
        a = np.ascontiguousarray(x, np.float32)
        conv._check(lib().aih_model_write_tensor(self._h, name.encode(), a.ctypes.data, a.size,
                                                 conv._stream(stream)))

    def read_output(self, name: str | None = None, stream=None) -> np.ndarray:
        name = name or self.outputs[0]
        t = self.tensor(name)
        out = np.empty((t.n, t.h, t.w, t.c), np.float32)
        conv._check(lib().aih_model_read_output(self._h, name.encode(), out.ctypes.data, out.size,
                                                conv._stream(stream)))
        return out

    def reset(self, stream=None):
        conv._check(lib().aih_model_reset(self._h, conv._stream(stream)))


# ---------------------------------------------------------------- writing .sw containers

MAGIC, VERSION, BLOB_ALIGN = b"SW1\0", 1, 256


def write_container(graph: dict, blob: bytes) -> bytes:
    """header.rs:37-55: 32-byte header, JSON at 32, blob at the JSON end rounded up to 256."""
    js = json.dumps(graph, separators=(",", ":")).encode()
    blob_off = -(-(32 + len(js)) // BLOB_ALIGN) * BLOB_ALIGN
    head = MAGIC + struct.pack("<IIIQQ", VERSION, 0, BLOB_ALIGN, 32, len(js))
    return head + js + b"\0" * (blob_off - 32 - len(js)) + bytes(blob)


def read_container(data: bytes) -> tuple[dict, bytes]:
    """parse_container (header.rs:58-86) in Python: (graph, blob)."""
    if len(data) < 32:
        raise ValueError(".sw: truncated (header)")
    if data[:4] != MAGIC:
        raise ValueError(".sw: bad magic")
    version, _flags, align, joff, jlen = struct.unpack_from("<IIIQQ", data, 4)
    if version != VERSION:
        raise ValueError(f".sw: unsupported version {version}")
    if joff + jlen > len(data):
        raise ValueError(".sw: truncated (json)")
    blob_off = -(-(joff + jlen) // max(align, 1)) * max(align, 1)
    if blob_off > len(data):
        raise ValueError(".sw: truncated (blob)")
    return json.loads(data[joff:joff + jlen]), data[blob_off:]


def conv_graph_to_sw(name: str, layers, weights, h: int, w: int, c: int) -> bytes:
    """A conv chain (ai_engine_amd.workloads layers + weights) as the .sw the
    reference's converter writes for it: fp32, pack_weights_conv(kg_align=4) /
    pack_weights_dw / pack_bias at 256-aligned offsets (lower.rs:116-193)."""
    tensors = [dict(name="input", h=h, w=w, c=c, dt="f32", alias=None, last_use=0)]
    tid = {"input": 0}
    blob = bytearray()
    ops = []

    def put(a: np.ndarray) -> dict:
        off = -(-len(blob) // BLOB_ALIGN) * BLOB_ALIGN
        blob.extend(b"\0" * (off - len(blob)))
        raw = np.ascontiguousarray(a).tobytes()
        blob.extend(raw)
        return dict(off=off, len=len(raw))

    for i, Lr in enumerate(layers):
        wt, bt = weights.w[Lr.name], weights.b[Lr.name]
        if Lr.depthwise:
            wp = conv.pack_weights_dw(wt, Lr.cout, Lr.k, Lr.k, conv.DType.F32)
            kg_pad = 0
        else:
            wp, kg_pad = conv.pack_weights_conv(wt, Lr.cout, Lr.cin, Lr.k, Lr.k, 4, conv.DType.F32)
        bp = conv.pack_bias(bt, Lr.cout, conv.DType.F32)
        oh, ow = Lr.out_hw()
        tid[Lr.name] = len(tensors)
        tensors.append(dict(name=Lr.name, h=oh, w=ow, c=Lr.cout, dt="f32", alias=None, last_use=0))
        for src in [Lr.src] + ([Lr.res] if Lr.res else []):
            tensors[tid[src]]["last_use"] = i
        ops.append(dict(kind="conv", out=tid[Lr.name], res=tid[Lr.res] if Lr.res else None, cin=Lr.cin,
                        cout=Lr.cout, kh=Lr.k, kw=Lr.k, sh=Lr.s, sw=Lr.s, pad=[Lr.pad] * 4, d=1, groups=Lr.groups,
                        act=Lr.act, w=put(wp), b=put(bp), kg_pad=int(kg_pad), **{"in": tid[Lr.src]}))
    out = tid[layers[-1].name]
    tensors[out]["last_use"] = len(ops)
    graph = dict(name=name, size=dict(h=h, w=w), dt_default="f32", dt_weights="f32", tensors=tensors, inputs=[0],
                 outputs=[out], states=[], ops=ops)
    return write_container(graph, bytes(blob))

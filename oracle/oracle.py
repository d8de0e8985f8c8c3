"""ctypes wrapper of the CPU oracle (TEST INFRASTRUCTURE).

Only tests/, the smoke check in __graft_entry__.py and bench.py's cpu_baseline
leg import this module; the product (ai_engine_amd) never does.  The C library
it loads (oracle/liboracle.so, built by oracle/Makefile) restates the
reference's ai-core / ai-cpu arithmetic; every function cites its reference
file:line in oracle/aicpu_oracle.c.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from dataclasses import dataclass, field

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")

F32, F16, BF16 = 0, 1, 2
ACT = {
    "none": 0, "relu": 1, "sigmoid": 2, "tanh": 3, "hardswish": 4, "hardsigmoid": 5,
    "clamp01": 6, "relu6": 7, "sqrt": 8, "neg": 9, "recip": 10,
}
ROUTE_NAMES = {0: "ConvStd", 1: "ConvStem", 2: "PwDot", 3: "ConvDw"}
PW_VARIANTS = {0: "Tiled", 1: "Small", 2: "Gemv", 3: "Splitk"}
IG_VARIANTS = {0: "Tiled", 1: "Direct", 2: "Splitk"}


def build() -> str:
    """Compile the oracle with its Makefile (gcc only)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


class Conv2d(C.Structure):
    """orc_conv2d == ai-core Conv2d (crates/ai-core/src/ops/conv.rs:6-20)."""

    _fields_ = [
        ("cin", C.c_uint32), ("cout", C.c_uint32), ("kh", C.c_uint32), ("kw", C.c_uint32),
        ("sh", C.c_uint32), ("sw", C.c_uint32), ("pad", C.c_uint32 * 4),
        ("dil", C.c_uint32), ("groups", C.c_uint32), ("act", C.c_int32),
    ]


class View(C.Structure):
    _fields_ = [("data", C.c_void_p), ("c_off", C.c_uint32), ("stride", C.c_uint32), ("c", C.c_uint32)]


def conv2d(cin, cout, k=1, s=1, pad=None, dil=1, groups=1, act="none", kh=None, kw=None, sh=None, sw=None):
    kh = k if kh is None else kh
    kw = k if kw is None else kw
    sh = s if sh is None else sh
    sw = s if sw is None else sw
    if pad is None:
        pad = [0, 0, 0, 0]
    elif isinstance(pad, int):
        pad = [pad] * 4
    act_id = ACT[act] if isinstance(act, str) else int(act)
    return Conv2d(cin, cout, kh, kw, sh, sw, (C.c_uint32 * 4)(*pad), dil, groups, act_id)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = C.CDLL(_LIB_PATH)
        P = C.c_void_p
        u32, i32, sz, f32 = C.c_uint32, C.c_int32, C.c_size_t, C.c_float
        sig = {
            "orc_out_hw": (None, [C.POINTER(Conv2d), u32, u32, C.POINTER(u32), C.POINTER(u32)]),
            "orc_act_apply": (f32, [i32, f32]),
            "orc_act_apply4": (None, [i32, P]),
            "orc_act_apply_n": (None, [i32, P, P, C.c_size_t]),
            "orc_xs32_seed": (u32, [u32]),
            "orc_xs32_next": (u32, [C.POINTER(u32)]),
            "orc_xs32_next_f32": (f32, [C.POINTER(u32)]),
            "orc_xs32_fill": (None, [u32, P, sz]),
            "orc_gauss_fill": (None, [u32, f32, f32, P, sz]),
            "orc_f32_to_f16": (C.c_uint16, [f32]),
            "orc_f16_to_f32": (f32, [C.c_uint16]),
            "orc_f32_to_bf16": (C.c_uint16, [f32]),
            "orc_bf16_to_f32": (f32, [C.c_uint16]),
            "orc_cvt_from_f32": (None, [i32, P, P, sz]),
            "orc_cvt_to_f32": (None, [i32, P, P, sz]),
            "orc_nhwc_c4_bytes": (sz, [u32, u32, u32, u32, i32]),
            "orc_pack_nhwc": (None, [P, u32, u32, u32, u32, i32, P]),
            "orc_unpack_nhwc": (None, [P, u32, u32, u32, u32, i32, P]),
            "orc_pack_weights_conv": (u32, [P, u32, u32, u32, u32, u32, i32, P]),
            "orc_unpack_weights_conv": (None, [P, u32, u32, u32, u32, u32, i32, P]),
            "orc_pack_weights_dw": (None, [P, u32, u32, u32, i32, P]),
            "orc_unpack_weights_dw": (None, [P, u32, u32, u32, i32, P]),
            "orc_pack_bias": (None, [P, u32, i32, P]),
            "orc_unpack_bias": (None, [P, u32, i32, P]),
            "orc_conv2d_ref": (C.c_int, [C.POINTER(Conv2d), u32, u32, P, P, P, P, P]),
            "orc_cpu_repack_weights": (u32, [P, u32, u32, u32, u32, u32, P]),
            "orc_cpu_conv_std": (None, [C.POINTER(Conv2d), u32, u32, C.POINTER(View), P, P, u32, P, P, u32,
                                        C.POINTER(View), P, u32, u32]),
            "orc_cpu_repack_weights_dw": (u32, [P, u32, u32, u32, P]),
            "orc_cpu_conv_dw": (None, [C.POINTER(Conv2d), u32, u32, C.POINTER(View), P, P, C.POINTER(View), P,
                                       u32, u32]),
            "orc_cpu_im2row": (None, [C.POINTER(Conv2d), u32, u32, C.POINTER(View), u32, P]),
            "orc_cpu_permute_weights": (None, [P, u32, u32, u32, u32, P]),
            "orc_cpu_conv_pw_dot": (None, [C.POINTER(Conv2d), C.POINTER(View), P, u32, P, u32, P]),
            "orc_cpu_op_create": (P, [C.POINTER(Conv2d), u32, u32, P, P, i32]),
            "orc_cpu_op_route": (i32, [P]),
            "orc_cpu_op_run": (C.c_int, [P, u32, P, P, P, i32]),
            "orc_cpu_op_free": (None, [P]),
            "orc_ref_pw_variant": (i32, [u32, u32, u32]),
            "orc_ref_gemv_width": (u32, [u32]),
            "orc_ref_splitk_geometry": (None, [u32, C.POINTER(u32), C.POINTER(u32)]),
            "orc_ref_splitk_tile": (None, [u32, u32, C.POINTER(u32), C.POINTER(u32)]),
            "orc_ref_igemm_variant": (i32, [u32, u32, u32, u32, u32, u32, u32, C.POINTER(u32), u32, i32]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def storage_np_dtype(dt: int):
    return np.float32 if dt == F32 else np.uint16


# ---- ai-core ----

def out_hw(op: Conv2d, ih: int, iw: int) -> tuple[int, int]:
    oh, ow = C.c_uint32(), C.c_uint32()
    lib().orc_out_hw(C.byref(op), ih, iw, C.byref(oh), C.byref(ow))
    return oh.value, ow.value


def act_apply(act: str | int, x: float) -> float:
    return lib().orc_act_apply(ACT[act] if isinstance(act, str) else act, x)


def act_array(act: str | int, x) -> np.ndarray:
    """Activation::apply (activation.rs:28-43) element-wise over an array."""
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    lib().orc_act_apply_n(ACT[act] if isinstance(act, str) else act, _p(x), _p(y), x.size)
    return y


def xs32_fill(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().orc_xs32_fill(seed, _p(out), n)
    return out


def xs32_u32(seed: int, n: int) -> list[int]:
    s = C.c_uint32(lib().orc_xs32_seed(seed))
    return [lib().orc_xs32_next(C.byref(s)) for _ in range(n)]


def gauss_fill(seed: int, mean: float, sigma: float, n: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().orc_gauss_fill(seed, mean, sigma, _p(out), n)
    return out


def cvt_from_f32(x, dt: int) -> np.ndarray:
    x = _f32(x).ravel()
    out = np.empty(x.size, storage_np_dtype(dt))
    lib().orc_cvt_from_f32(dt, _p(x), _p(out), x.size)
    return out


def cvt_to_f32(x: np.ndarray, dt: int) -> np.ndarray:
    x = np.ascontiguousarray(x).ravel()
    out = np.empty(x.size, np.float32)
    lib().orc_cvt_to_f32(dt, _p(x), _p(out), x.size)
    return out


def round_to(x, dt: int) -> np.ndarray:
    """Value of x after storage in dt (identity for F32)."""
    x = _f32(x)
    if dt == F32:
        return x.copy()
    return cvt_to_f32(cvt_from_f32(x, dt), dt).reshape(x.shape)


def pack_nhwc(data, n, h, w, c, dt=F32) -> np.ndarray:
    data = _f32(data)
    assert data.size == n * h * w * c
    out = np.empty(n * h * w * ((c + 3) // 4) * 4, storage_np_dtype(dt))
    lib().orc_pack_nhwc(_p(data), n, h, w, c, dt, _p(out))
    return out


def unpack_nhwc(packed: np.ndarray, n, h, w, c, dt=F32) -> np.ndarray:
    packed = np.ascontiguousarray(packed)
    out = np.empty(n * h * w * c, np.float32)
    lib().orc_unpack_nhwc(_p(packed), n, h, w, c, dt, _p(out))
    return out


def pack_weights_conv(w_oihw, cout, cin, kh, kw, kg_align=4, dt=F32) -> tuple[np.ndarray, int]:
    w = _f32(w_oihw)
    kg = -(-((cin + 3) // 4) // max(kg_align, 1)) * max(kg_align, 1)
    ng = (cout + 3) // 4
    out = np.empty(kh * kw * kg * ng * 16, storage_np_dtype(dt))
    kg_pad = lib().orc_pack_weights_conv(_p(w), cout, cin, kh, kw, kg_align, dt, _p(out))
    assert kg_pad == kg
    return out, kg_pad


def unpack_weights_conv(packed, cout, cin, kh, kw, kg_pad, dt=F32) -> np.ndarray:
    packed = np.ascontiguousarray(packed)
    out = np.zeros(cout * cin * kh * kw, np.float32)
    lib().orc_unpack_weights_conv(_p(packed), cout, cin, kh, kw, kg_pad, dt, _p(out))
    return out


def pack_weights_dw(w, c, kh, kw, dt=F32) -> np.ndarray:
    w = _f32(w)
    out = np.empty(kh * kw * ((c + 3) // 4) * 4, storage_np_dtype(dt))
    lib().orc_pack_weights_dw(_p(w), c, kh, kw, dt, _p(out))
    return out


def unpack_weights_dw(packed, c, kh, kw, dt=F32) -> np.ndarray:
    packed = np.ascontiguousarray(packed)
    out = np.empty(c * kh * kw, np.float32)
    lib().orc_unpack_weights_dw(_p(packed), c, kh, kw, dt, _p(out))
    return out


def pack_bias(b, cout, dt=F32) -> np.ndarray:
    b = _f32(b)
    out = np.empty(((cout + 3) // 4) * 4, storage_np_dtype(dt))
    lib().orc_pack_bias(_p(b), cout, dt, _p(out))
    return out


def unpack_bias(packed, cout, dt=F32) -> np.ndarray:
    packed = np.ascontiguousarray(packed)
    out = np.empty(cout, np.float32)
    lib().orc_unpack_bias(_p(packed), cout, dt, _p(out))
    return out


def conv2d_ref(op: Conv2d, ih, iw, x, w, bias=None, res=None, n=1) -> np.ndarray:
    """reference::conv::conv2d over n images (looped; the reference has n=1)."""
    x = _f32(x)
    w = _f32(w)
    b = None if bias is None else _f32(bias)
    oh, ow = out_hw(op, ih, iw)
    out = np.empty(n * oh * ow * op.cout, np.float32)
    in_sz, out_sz = ih * iw * op.cin, oh * ow * op.cout
    r = None if res is None else _f32(res)
    for i in range(n):
        xi = x[i * in_sz:(i + 1) * in_sz]
        ri = None if r is None else r[i * out_sz:(i + 1) * out_sz]
        oi = out[i * out_sz:(i + 1) * out_sz]
        rc = lib().orc_conv2d_ref(C.byref(op), ih, iw, _p(xi), _p(w), _p(b), _p(ri), _p(oi))
        assert rc == 0
    return out


# ---- ai-cpu ----

@dataclass
class CpuConv:
    """One conv op lowered like ai-cpu plan::lower and run like model::dispatch."""

    op: Conv2d
    ih: int
    iw: int
    w_oihw: np.ndarray
    bias: np.ndarray
    has_res: bool = False
    _h: int = field(default=0, repr=False)

    def __post_init__(self):
        self.w_oihw = _f32(self.w_oihw)
        self.bias = _f32(self.bias)
        h = lib().orc_cpu_op_create(C.byref(self.op), self.ih, self.iw, _p(self.w_oihw), _p(self.bias),
                                    1 if self.has_res else 0)
        if not h:
            raise ValueError("ai-cpu oracle: unsupported conv")
        self._h = h
        self.oh, self.ow = out_hw(self.op, self.ih, self.iw)

    @property
    def route(self) -> str:
        return ROUTE_NAMES[lib().orc_cpu_op_route(self._h)]

    def alloc_input(self, n: int) -> np.ndarray:
        """Input slot with the +4 float slack of ai-cpu's slots (model.rs:38-41)."""
        return np.zeros(n * self.ih * self.iw * self.op.cin + 4, np.float32)

    def run(self, x: np.ndarray, n: int = 1, res: np.ndarray | None = None, threads: int = 1,
            out: np.ndarray | None = None) -> np.ndarray:
        in_sz = n * self.ih * self.iw * self.op.cin
        if x.size < in_sz + 4 or x.dtype != np.float32 or not x.flags.c_contiguous:
            buf = self.alloc_input(n)
            buf[:in_sz] = np.asarray(x, np.float32).ravel()[:in_sz]
            x = buf
        if out is None:
            out = np.empty(n * self.oh * self.ow * self.op.cout, np.float32)
        r = None
        if res is not None:
            r = _f32(res)
        rc = lib().orc_cpu_op_run(self._h, n, _p(x), _p(r), _p(out), threads)
        assert rc == 0
        return out

    def __del__(self):
        if getattr(self, "_h", 0):
            lib().orc_cpu_op_free(self._h)
            self._h = 0


# ---- ai-gpu policies ----

def ref_pw_variant(m, kg, ng) -> str:
    return PW_VARIANTS[lib().orc_ref_pw_variant(m, kg, ng)]


def ref_gemv_width(kg) -> int:
    return lib().orc_ref_gemv_width(kg)


def ref_splitk_geometry(cells) -> tuple[int, int]:
    a, b = C.c_uint32(), C.c_uint32()
    lib().orc_ref_splitk_geometry(cells, C.byref(a), C.byref(b))
    return a.value, b.value


def ref_splitk_tile(ng, cpw) -> tuple[int, int]:
    a, b = C.c_uint32(), C.c_uint32()
    lib().orc_ref_splitk_tile(ng, cpw, C.byref(a), C.byref(b))
    return a.value, b.value


def ref_igemm_variant(ih, iw, cin, cout, k, s, d=1, pad=None, nsrcs=0, has_offset=False) -> str:
    if pad is None:
        pad = [(k - 1) // 2] * 4
    p = (C.c_uint32 * 4)(*pad)
    return IG_VARIANTS[lib().orc_ref_igemm_variant(ih, iw, cin, cout, k, s, d, p, nsrcs, 1 if has_offset else 0)]

"""Host-side mirror of the reference's conv op interface, over the C ABI.

The reference's GPU runtime lowers a `SwOp::Conv` into one of three specs
(crates/ai-gpu-runtime/src/lowering.rs:99-187) and dispatches it with the
bindings IN, W, BIAS, [RES], OUT (crates/ai-gpu/src/kernels/gemm_pw.rs:276-283):

* `GemmPwSpec`    (crates/ai-gpu/src/kernels/gemm_pw.rs:129-142)  -> aih_conv_pw
* `ConvIgemmSpec` (crates/ai-gpu/src/kernels/conv_igemm.rs:49-76) -> aih_conv_igemm
* `ConvDwSpec`    (crates/ai-gpu/src/kernels/conv_dw.rs:21-60)    -> aih_conv_dw
* `lower_conv`    (the Conv arm of lower_op)                       -> aih_conv

Buffers are device tensors (torch, for allocation and streams only) or raw
device addresses; every call is asynchronous on the given stream (default:
torch's current stream).  There is no CPU fallback: if the HIP library is
missing this module raises at import of the library.
"""
from __future__ import annotations

import ctypes as C
import enum
import os
from dataclasses import dataclass, field

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libaih_conv.so")


class AihError(RuntimeError):
    """A call through the C ABI returned AIH_ERR; the message is aih_last_error()."""


class DType(enum.IntEnum):
    """ai-core DType (crates/ai-core/src/tensor.rs:12-16) plus BF16."""

    F32 = 0
    F16 = 1
    BF16 = 2

    @property
    def nbytes(self) -> int:
        return 4 if self == DType.F32 else 2


class Activation(enum.IntEnum):
    """ai-core Activation, same order (crates/ai-core/src/activation.rs:7-25)."""

    NONE = 0
    RELU = 1
    SIGMOID = 2
    TANH = 3
    HARDSWISH = 4
    HARDSIGMOID = 5
    CLAMP01 = 6
    RELU6 = 7
    SQRT = 8
    NEG = 9
    RECIP = 10


class IrWeights(enum.IntEnum):
    """Where a fused block keeps its expand / project weights (enum aih_ir_weights)."""

    AUTO = 0
    RESIDENT = 1
    STREAMED = 2


class IrKernel(enum.IntEnum):
    """Which fused kernel runs a block (enum aih_ir_kernel)."""

    AUTO = 0
    TILE = 1
    WAVE = 2
    SPLIT = 3


class Variant(enum.IntEnum):
    AUTO = 0
    TILE = 1
    SPLITK = 2
    ROWS = 3    # reported by the pointwise plan: one pixel per thread (ng == 1)
    DIRECT = 4  # reported by the plans: operands straight into MFMA registers (short-K pointwise, 3x3 <= 64 outputs)


# ---------------------------------------------------------------- ctypes structs (include/aih_conv.h)

class _PwDesc(C.Structure):
    _fields_ = [("n", C.c_uint32), ("m", C.c_uint32), ("kg", C.c_uint32), ("ng", C.c_uint32),
                ("kg_pad", C.c_uint32), ("act", C.c_int32), ("residual", C.c_int32), ("dt", C.c_int32),
                ("wdt", C.c_int32), ("variant", C.c_int32), ("splitk", C.c_int32)]


class _Src(C.Structure):
    _fields_ = [("c", C.c_uint32), ("stride_c", C.c_uint32), ("c_off", C.c_uint32)]


class _IgemmDesc(C.Structure):
    _fields_ = [("n", C.c_uint32), ("ih", C.c_uint32), ("iw", C.c_uint32), ("cin", C.c_uint32),
                ("cout", C.c_uint32), ("k", C.c_uint32), ("s", C.c_uint32), ("d", C.c_uint32),
                ("pad", C.c_uint32 * 4), ("act", C.c_int32), ("residual", C.c_int32), ("dt", C.c_int32),
                ("wdt", C.c_int32), ("variant", C.c_int32), ("splitk", C.c_int32), ("nsrcs", C.c_uint32),
                ("srcs", _Src * 3)]


class _DwDesc(C.Structure):
    _fields_ = [("n", C.c_uint32), ("ih", C.c_uint32), ("iw", C.c_uint32), ("c", C.c_uint32),
                ("k", C.c_uint32), ("s", C.c_uint32), ("d", C.c_uint32), ("pad", C.c_uint32 * 4),
                ("act", C.c_int32), ("residual", C.c_int32), ("dt", C.c_int32)]


class _ConvDesc(C.Structure):
    _fields_ = [("n", C.c_uint32), ("ih", C.c_uint32), ("iw", C.c_uint32), ("cin", C.c_uint32),
                ("cout", C.c_uint32), ("kh", C.c_uint32), ("kw", C.c_uint32), ("sh", C.c_uint32),
                ("sw", C.c_uint32), ("pad", C.c_uint32 * 4), ("d", C.c_uint32), ("groups", C.c_uint32),
                ("act", C.c_int32), ("residual", C.c_int32), ("dt", C.c_int32), ("wdt", C.c_int32),
                ("kg_pad", C.c_uint32)]


class _IrDesc(C.Structure):
    _fields_ = [("n", C.c_uint32), ("ih", C.c_uint32), ("iw", C.c_uint32), ("cin", C.c_uint32),
                ("cexp", C.c_uint32), ("cout", C.c_uint32), ("s", C.c_uint32), ("pad", C.c_uint32 * 4),
                ("act_expand", C.c_int32), ("act_dw", C.c_int32), ("act_project", C.c_int32),
                ("residual", C.c_int32), ("dt", C.c_int32), ("tile_h", C.c_uint32), ("tile_w", C.c_uint32),
                ("ec", C.c_uint32), ("weights", C.c_int32), ("kernel", C.c_int32), ("waves", C.c_uint32)]


class IrPlan(C.Structure):
    _fields_ = [("th", C.c_uint32), ("tw", C.c_uint32), ("ec", C.c_uint32), ("chunks", C.c_uint32),
                ("resident", C.c_uint32), ("tiles", C.c_uint32), ("lds_bytes", C.c_uint32),
                ("occupancy", C.c_uint32), ("grid", C.c_uint32), ("kernel", C.c_uint32), ("waves", C.c_uint32),
                ("deep", C.c_uint32)]

    def __repr__(self):
        return (f"IrPlan({IrKernel(self.kernel).name.lower()}, tile={self.th}x{self.tw}, ec={self.ec}, "
                f"chunks={self.chunks}, resident={self.resident}, tiles={self.tiles}, lds={self.lds_bytes}, "
                f"occ={self.occupancy}, grid={self.grid}x{self.waves} waves{', deep' if self.deep else ''})")


class _DwPwDesc(C.Structure):
    _fields_ = [("n", C.c_uint32), ("ih", C.c_uint32), ("iw", C.c_uint32), ("c", C.c_uint32),
                ("k", C.c_uint32), ("s", C.c_uint32), ("pad", C.c_uint32 * 4), ("cout", C.c_uint32),
                ("kg_pad", C.c_uint32), ("act_dw", C.c_int32), ("act_pw", C.c_int32), ("residual", C.c_int32),
                ("dt", C.c_int32), ("tile_h", C.c_uint32), ("tile_w", C.c_uint32),
                ("wave_rows", C.c_uint32)]


class DwPwPlan(C.Structure):
    _fields_ = [("th", C.c_uint32), ("tw", C.c_uint32), ("waves", C.c_uint32), ("wave_rows", C.c_uint32),
                ("chunks", C.c_uint32),
                ("tiles", C.c_uint32), ("lds_bytes", C.c_uint32), ("occupancy", C.c_uint32), ("grid", C.c_uint32)]

    def __repr__(self):
        return (f"DwPwPlan(tile={self.th}x{self.tw}, waves={self.waves}x{self.wave_rows} rows, chunks={self.chunks}, "
                f"tiles={self.tiles}, lds={self.lds_bytes}, occ={self.occupancy}, grid={self.grid})")


class Plan(C.Structure):
    _fields_ = [("variant", C.c_int32), ("splitk", C.c_uint32), ("bm", C.c_uint32), ("bn", C.c_uint32),
                ("grid", C.c_uint32), ("ws_bytes", C.c_size_t)]

    def __repr__(self):
        return (f"Plan(variant={Variant(self.variant).name}, splitk={self.splitk}, bm={self.bm}, "
                f"bn={self.bn}, grid={self.grid}, ws_bytes={self.ws_bytes})")


EXPORTS = (
    "aih_conv_pw", "aih_conv_pw_plan", "aih_conv_igemm", "aih_conv_igemm_plan", "aih_conv_dw", "aih_conv",
    "aih_conv_workspace_size", "aih_nhwc_c4_bytes", "aih_pack_nhwc", "aih_unpack_nhwc",
    "aih_pack_weights_conv", "aih_pack_weights_dw", "aih_pack_bias", "aih_pack_nhwc_device",
    "aih_ir_block_plan", "aih_ir_block", "aih_last_error", "aih_version", "aih_conv_check", "aih_conv_plan",
    "aih_conv_noalloc", "aih_conv_stem_f32in", "aih_conv_dwpw_plan", "aih_conv_dwpw",
    "aih_ir_block_stem_plan", "aih_ir_block_stem",
    "aih_ir_block_head_plan", "aih_ir_block_head",
)

_lib = None


def lib() -> C.CDLL:
    """Load the HIP library (raises if it was not built: there is no fallback)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise AihError(f"{LIB_PATH} is missing; build it with `python -m ai_engine_amd.build`")
    L = C.CDLL(LIB_PATH)
    P, u32, i32, sz = C.c_void_p, C.c_uint32, C.c_int32, C.c_size_t
    sigs = {
        "aih_conv_pw": (C.c_int, [C.POINTER(_PwDesc), P, P, P, P, P, P, sz, P]),
        "aih_conv_pw_plan": (C.c_int, [C.POINTER(_PwDesc), C.POINTER(Plan)]),
        "aih_conv_igemm": (C.c_int, [C.POINTER(_IgemmDesc), C.POINTER(P), P, P, P, P, P, sz, P]),
        "aih_conv_igemm_plan": (C.c_int, [C.POINTER(_IgemmDesc), C.POINTER(Plan)]),
        "aih_conv_dw": (C.c_int, [C.POINTER(_DwDesc), P, P, P, P, P, P]),
        "aih_conv": (C.c_int, [C.POINTER(_ConvDesc), P, P, P, P, P, P, sz, P]),
        "aih_conv_workspace_size": (sz, [C.POINTER(_ConvDesc)]),
        "aih_conv_plan": (C.c_int, [C.POINTER(_ConvDesc), C.POINTER(Plan)]),
        "aih_conv_noalloc": (C.c_int, [C.POINTER(_ConvDesc), P, P, P, P, P, P]),
        "aih_nhwc_c4_bytes": (sz, [u32, u32, u32, u32, i32]),
        "aih_pack_nhwc": (C.c_int, [P, u32, u32, u32, u32, i32, P]),
        "aih_unpack_nhwc": (C.c_int, [P, u32, u32, u32, u32, i32, P]),
        "aih_pack_weights_conv": (u32, [P, u32, u32, u32, u32, u32, i32, P]),
        "aih_pack_weights_dw": (C.c_int, [P, u32, u32, u32, i32, P]),
        "aih_pack_bias": (C.c_int, [P, u32, i32, P]),
        "aih_pack_nhwc_device": (C.c_int, [P, u32, u32, u32, u32, i32, P, P]),
        "aih_conv_stem_f32in": (C.c_int, [C.POINTER(_IgemmDesc), P, P, P, P, P, P]),
        "aih_ir_block_plan": (C.c_int, [C.POINTER(_IrDesc), C.POINTER(IrPlan)]),
        "aih_ir_block": (C.c_int, [C.POINTER(_IrDesc), P, P, P, P, P, P, P, P, P, P]),
        "aih_ir_block_stem_plan": (C.c_int, [C.POINTER(_IgemmDesc), C.POINTER(_IrDesc), C.POINTER(IrPlan)]),
        "aih_ir_block_stem": (C.c_int, [C.POINTER(_IgemmDesc), C.POINTER(_IrDesc)] + [P] * 11),
        "aih_ir_block_head_plan": (C.c_int, [C.POINTER(_IrDesc), C.POINTER(_PwDesc), C.POINTER(IrPlan)]),
        "aih_ir_block_head": (C.c_int, [C.POINTER(_IrDesc), C.POINTER(_PwDesc)] + [P] * 13),
        "aih_conv_dwpw_plan": (C.c_int, [C.POINTER(_DwPwDesc), C.POINTER(DwPwPlan)]),
        "aih_conv_dwpw": (C.c_int, [C.POINTER(_DwPwDesc), P, P, P, P, P, P, P, P]),
        "aih_last_error": (C.c_char_p, []),
        "aih_version": (C.c_char_p, []),
    }
    for name, (res, args) in sigs.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def last_error() -> str:
    return lib().aih_last_error().decode()


def _check(rc: int):
    if rc != 0:
        raise AihError(last_error())


def _ptr(t) -> int | None:
    """Device address of a torch tensor, an int address, or None."""
    if t is None:
        return None
    if isinstance(t, int):
        return t
    return t.data_ptr()


def _stream(stream) -> int | None:
    if stream is None:
        import torch

        return torch.cuda.current_stream().cuda_stream
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream


def _workspace(nbytes: int, ws, device):
    if nbytes == 0 or ws is not None:
        return ws
    import torch

    return torch.empty(max(nbytes // 4, 1), dtype=torch.float32, device=device)


def _device_of(t):
    return getattr(t, "device", None)


# ---------------------------------------------------------------- specs

@dataclass
class GemmPwSpec:
    """1x1 conv GEMM; fields of GemmPwSpec (gemm_pw.rs:129-142) plus n / kg_pad / variant / splitk."""

    m: int
    kg: int
    ng: int
    act: Activation = Activation.NONE
    residual: bool = False
    dt: DType = DType.F32
    wdt: DType | None = None
    n: int = 1
    kg_pad: int | None = None
    variant: Variant = Variant.AUTO
    splitk: int = 0

    def desc(self) -> _PwDesc:
        wdt = self.dt if self.wdt is None else self.wdt
        kg_pad = self.kg_pad if self.kg_pad is not None else -(-self.kg // 4) * 4
        return _PwDesc(self.n, self.m, self.kg, self.ng, kg_pad, int(self.act), int(bool(self.residual)),
                       int(self.dt), int(wdt), int(self.variant), int(self.splitk))

    def plan(self) -> Plan:
        p = Plan()
        _check(lib().aih_conv_pw_plan(C.byref(self.desc()), C.byref(p)))
        return p

    def run(self, x, w, bias, res, y, ws=None, stream=None):
        d = self.desc()
        p = Plan()
        _check(lib().aih_conv_pw_plan(C.byref(d), C.byref(p)))
        ws = _workspace(p.ws_bytes, ws, _device_of(y))
        _check(lib().aih_conv_pw(C.byref(d), _ptr(x), _ptr(w), _ptr(bias), _ptr(res), _ptr(y), _ptr(ws),
                                 p.ws_bytes if ws is not None else 0, _stream(stream)))
        return y


@dataclass
class SrcView:
    """One input part (SrcView, crates/ai-gpu/src/kernels/common/source.rs:17)."""

    c: int
    stride_c: int | None = None
    c_off: int = 0


@dataclass
class ConvIgemmSpec:
    """KxK implicit-GEMM conv; fields of ConvIgemmSpec (conv_igemm.rs:49-76) plus n."""

    ih: int
    iw: int
    cin: int
    cout: int
    k: int
    s: int = 1
    d: int = 1
    pad: tuple = (0, 0, 0, 0)
    act: Activation = Activation.NONE
    residual: bool = False
    dt: DType = DType.F32
    wdt: DType | None = None
    n: int = 1
    variant: Variant = Variant.AUTO
    splitk: int = 0
    srcs: list = field(default_factory=list)

    def out_hw(self) -> tuple[int, int]:
        ek = self.d * (self.k - 1) + 1
        oh = (self.ih + self.pad[0] + self.pad[2] - ek) // self.s + 1
        ow = (self.iw + self.pad[1] + self.pad[3] - ek) // self.s + 1
        return oh, ow

    def desc(self) -> _IgemmDesc:
        wdt = self.dt if self.wdt is None else self.wdt
        srcs = (_Src * 3)()
        for i, s in enumerate(self.srcs):
            stride = s.stride_c if s.stride_c is not None else -(-s.c // 4) * 4
            srcs[i] = _Src(s.c, stride, s.c_off)
        return _IgemmDesc(self.n, self.ih, self.iw, self.cin, self.cout, self.k, self.s, self.d,
                          (C.c_uint32 * 4)(*self.pad), int(self.act), int(bool(self.residual)), int(self.dt),
                          int(wdt), int(self.variant), int(self.splitk), len(self.srcs), srcs)

    def plan(self) -> Plan:
        p = Plan()
        _check(lib().aih_conv_igemm_plan(C.byref(self.desc()), C.byref(p)))
        return p

    def run(self, inputs, w, bias, res, y, ws=None, stream=None):
        if not isinstance(inputs, (list, tuple)):
            inputs = [inputs]
        d = self.desc()
        p = Plan()
        _check(lib().aih_conv_igemm_plan(C.byref(d), C.byref(p)))
        ws = _workspace(p.ws_bytes, ws, _device_of(y))
        arr = (C.c_void_p * 3)(*[_ptr(t) for t in inputs])
        _check(lib().aih_conv_igemm(C.byref(d), arr, _ptr(w), _ptr(bias), _ptr(res), _ptr(y), _ptr(ws),
                                    p.ws_bytes if ws is not None else 0, _stream(stream)))
        return y

    def run_f32_input(self, x, w, bias, res, y, stream=None):
        """The stem route from a logical NHWC fp32 input (aih_conv_stem_f32in):
        equal to pack_nhwc_device followed by run(), without the packed copy."""
        _check(lib().aih_conv_stem_f32in(C.byref(self.desc()), _ptr(x), _ptr(w), _ptr(bias), _ptr(res), _ptr(y),
                                         _stream(stream)))
        return y


@dataclass
class ConvDwSpec:
    """Depthwise conv; fields of ConvDwSpec (conv_dw.rs:21-60) plus n."""

    ih: int
    iw: int
    c: int
    k: int = 3
    s: int = 1
    d: int = 1
    pad: tuple = (1, 1, 1, 1)
    act: Activation = Activation.NONE
    residual: bool = False
    dt: DType = DType.F32
    n: int = 1

    def out_hw(self) -> tuple[int, int]:
        ek = self.d * (self.k - 1) + 1
        return ((self.ih + self.pad[0] + self.pad[2] - ek) // self.s + 1,
                (self.iw + self.pad[1] + self.pad[3] - ek) // self.s + 1)

    def desc(self) -> _DwDesc:
        return _DwDesc(self.n, self.ih, self.iw, self.c, self.k, self.s, self.d, (C.c_uint32 * 4)(*self.pad),
                       int(self.act), int(bool(self.residual)), int(self.dt))

    def run(self, x, w, bias, res, y, stream=None):
        _check(lib().aih_conv_dw(C.byref(self.desc()), _ptr(x), _ptr(w), _ptr(bias), _ptr(res), _ptr(y),
                                 _stream(stream)))
        return y


@dataclass
class ConvOp:
    """A SwOp::Conv (crates/ai-core/src/format/model.rs:80-111) with a batch n; run() routes like lower_op."""

    ih: int
    iw: int
    cin: int
    cout: int
    kh: int = 1
    kw: int = 1
    sh: int = 1
    sw: int = 1
    pad: tuple = (0, 0, 0, 0)
    d: int = 1
    groups: int = 1
    act: Activation = Activation.NONE
    residual: bool = False
    dt: DType = DType.F32
    wdt: DType | None = None
    n: int = 1

    @property
    def kg_pad(self) -> int:
        return -(-(-(-self.cin // 4)) // 4) * 4

    def out_hw(self) -> tuple[int, int]:
        oh = (self.ih + self.pad[0] + self.pad[2] - (self.d * (self.kh - 1) + 1)) // self.sh + 1
        ow = (self.iw + self.pad[1] + self.pad[3] - (self.d * (self.kw - 1) + 1)) // self.sw + 1
        return oh, ow

    def desc(self) -> _ConvDesc:
        wdt = self.dt if self.wdt is None else self.wdt
        return _ConvDesc(self.n, self.ih, self.iw, self.cin, self.cout, self.kh, self.kw, self.sh, self.sw,
                         (C.c_uint32 * 4)(*self.pad), self.d, self.groups, int(self.act), int(bool(self.residual)),
                         int(self.dt), int(wdt), self.kg_pad)

    def workspace_bytes(self) -> int:
        return lib().aih_conv_workspace_size(C.byref(self.desc()))

    def plan(self) -> Plan:
        """The plan of the route aih_conv takes (aih_conv_plan)."""
        p = Plan()
        _check(lib().aih_conv_plan(C.byref(self.desc()), C.byref(p)))
        return p

    def run(self, x, w, bias, res, y, ws=None, stream=None):
        nb = self.workspace_bytes()
        ws = _workspace(nb, ws, _device_of(y))
        _check(lib().aih_conv(C.byref(self.desc()), _ptr(x), _ptr(w), _ptr(bias), _ptr(res), _ptr(y), _ptr(ws),
                              nb if ws is not None else 0, _stream(stream)))
        return y


@dataclass
class IrBlockSpec:
    """Fused inverted-residual block: the three SwOp::Conv a MobileNet block
    lowers to (1x1 expand, depthwise 3x3 stride s, 1x1 project) in one launch.
    The reference dispatches them separately (GemmPwSpec, ConvDwSpec,
    GemmPwSpec; crates/ai-gpu-runtime/src/lowering.rs:122-152)."""

    ih: int
    iw: int
    cin: int
    cexp: int
    cout: int
    s: int = 1
    pad: tuple = (1, 1, 1, 1)
    act_expand: Activation = Activation.RELU
    act_dw: Activation = Activation.RELU
    act_project: Activation = Activation.NONE
    residual: bool = False
    dt: DType = DType.F32
    n: int = 1
    tile: tuple = (0, 0)  # forced output tile (h, w); (0, 0) = plan's choice
    ec: int = 0           # forced expanded channels per chunk; 0 = plan's choice
    weights: int = 0      # IrWeights: 0 = plan's choice, 1 = resident in LDS, 2 = streamed
    kernel: int = 0       # IrKernel: 0 = plan's choice, 1 = tile, 2 = wave, 3 = split kernel
    waves: int = 0        # wavefronts per workgroup (wave / split kernel); 0 = plan's choice

    def out_hw(self) -> tuple[int, int]:
        return ((self.ih + self.pad[0] + self.pad[2] - 3) // self.s + 1,
                (self.iw + self.pad[1] + self.pad[3] - 3) // self.s + 1)

    def desc(self) -> _IrDesc:
        return _IrDesc(self.n, self.ih, self.iw, self.cin, self.cexp, self.cout, self.s, (C.c_uint32 * 4)(*self.pad),
                       int(self.act_expand), int(self.act_dw), int(self.act_project), int(bool(self.residual)),
                       int(self.dt), self.tile[0], self.tile[1], self.ec, int(self.weights), int(self.kernel),
                       self.waves)

    def plan(self) -> IrPlan:
        p = IrPlan()
        _check(lib().aih_ir_block_plan(C.byref(self.desc()), C.byref(p)))
        return p

    def fusable(self) -> bool:
        p = IrPlan()
        return lib().aih_ir_block_plan(C.byref(self.desc()), C.byref(p)) == 0

    def run(self, x, w_expand, b_expand, w_dw, b_dw, w_project, b_project, res, y, stream=None):
        _check(lib().aih_ir_block(C.byref(self.desc()), _ptr(x), _ptr(w_expand), _ptr(b_expand), _ptr(w_dw),
                                  _ptr(b_dw), _ptr(w_project), _ptr(b_project), _ptr(res), _ptr(y),
                                  _stream(stream)))
        return y


@dataclass
class StemIrBlockSpec:
    """The stem conv (a ConvIgemmSpec on the stem route, 3 -> 32, read from
    the logical NHWC fp32 image) fused into the inverted-residual block that
    reads its output as input and residual (aih_ir_block_stem): one launch,
    the stem's output never stored; bit for bit aih_conv_stem_f32in followed
    by aih_ir_block on the same plan. The reference dispatches the four convs
    separately (crates/ai-gpu-runtime/src/lowering.rs:122-168)."""

    stem: "ConvIgemmSpec"
    block: IrBlockSpec

    def plan(self) -> IrPlan:
        p = IrPlan()
        _check(lib().aih_ir_block_stem_plan(C.byref(self.stem.desc()), C.byref(self.block.desc()), C.byref(p)))
        return p

    def fusable(self) -> bool:
        p = IrPlan()
        return lib().aih_ir_block_stem_plan(C.byref(self.stem.desc()), C.byref(self.block.desc()), C.byref(p)) == 0

    def run(self, image, w_stem, b_stem, w_expand, b_expand, w_dw, b_dw, w_project, b_project, y, stream=None):
        _check(lib().aih_ir_block_stem(C.byref(self.stem.desc()), C.byref(self.block.desc()), _ptr(image),
                                       _ptr(w_stem), _ptr(b_stem), _ptr(w_expand), _ptr(b_expand), _ptr(w_dw),
                                       _ptr(b_dw), _ptr(w_project), _ptr(b_project), _ptr(y), _stream(stream)))
        return y


@dataclass
class IrBlockHeadSpec:
    """An inverted-residual block (an IrBlockSpec, on the split kernel) joined
    to the pointwise conv with at most 4 outputs that reads its output -- a
    GemmPwSpec on the narrow route, e.g. a segmentation head 128 -> 2
    (aih_ir_block_head): one launch; its head output equals aih_ir_block
    followed by aih_conv_pw bit for bit, and the block's own output is
    stored only when y is given. The reference dispatches the block's convs
    and the head separately (crates/ai-gpu-runtime/src/lowering.rs:122-168)."""

    block: IrBlockSpec
    head: GemmPwSpec

    def plan(self) -> IrPlan:
        p = IrPlan()
        _check(lib().aih_ir_block_head_plan(C.byref(self.block.desc()), C.byref(self.head.desc()), C.byref(p)))
        return p

    def fusable(self) -> bool:
        p = IrPlan()
        return lib().aih_ir_block_head_plan(C.byref(self.block.desc()), C.byref(self.head.desc()), C.byref(p)) == 0

    def run(self, x, w_expand, b_expand, w_dw, b_dw, w_project, b_project, res, y, w_head, b_head, y_head,
            stream=None):
        _check(lib().aih_ir_block_head(C.byref(self.block.desc()), C.byref(self.head.desc()), _ptr(x),
                                       _ptr(w_expand), _ptr(b_expand), _ptr(w_dw), _ptr(b_dw), _ptr(w_project),
                                       _ptr(b_project), _ptr(res), _ptr(y), _ptr(w_head), _ptr(b_head),
                                       _ptr(y_head), _stream(stream)))
        return y_head


@dataclass
class DwPwSpec:
    """Fused depthwise 3x3 + pointwise 1x1: a depthwise conv and the 1x1 conv
    that is its output's only reader, in one launch (the depthwise output
    never reaches memory). The reference dispatches them separately
    (ConvDwSpec, then GemmPwSpec; crates/ai-gpu-runtime/src/lowering.rs:122-168).
    Weights in the unfused ops' layouts: depthwise as pack_weights_dw, the
    pointwise as pack_weights_conv (kg_align 4, kg_pad groups)."""

    ih: int
    iw: int
    c: int
    cout: int
    k: int = 3
    s: int = 1
    pad: tuple = (1, 1, 1, 1)
    act_dw: Activation = Activation.RELU
    act_pw: Activation = Activation.NONE
    residual: bool = False
    dt: DType = DType.F32
    n: int = 1
    kg_pad: int = 0       # 0: ceil(c / 4) rounded up to a multiple of 4 (pack_weights_conv's kg_align 4)
    tile: tuple = (0, 0)  # forced output tile (h, w); (0, 0) = plan's choice
    rows: int = 0         # forced output rows per wavefront (2 or 4); 0 = plan's choice

    def out_hw(self) -> tuple[int, int]:
        return ((self.ih + self.pad[0] + self.pad[2] - self.k) // self.s + 1,
                (self.iw + self.pad[1] + self.pad[3] - self.k) // self.s + 1)

    def desc(self) -> _DwPwDesc:
        kgp = self.kg_pad or ((self.c + 3) // 4 + 3) // 4 * 4
        return _DwPwDesc(self.n, self.ih, self.iw, self.c, self.k, self.s, (C.c_uint32 * 4)(*self.pad), self.cout,
                         kgp, int(self.act_dw), int(self.act_pw), int(bool(self.residual)), int(self.dt),
                         self.tile[0], self.tile[1], self.rows)

    def plan(self) -> DwPwPlan:
        p = DwPwPlan()
        _check(lib().aih_conv_dwpw_plan(C.byref(self.desc()), C.byref(p)))
        return p

    def fusable(self) -> bool:
        p = DwPwPlan()
        return lib().aih_conv_dwpw_plan(C.byref(self.desc()), C.byref(p)) == 0

    def run(self, x, w_dw, b_dw, w_pw, b_pw, res, y, stream=None):
        _check(lib().aih_conv_dwpw(C.byref(self.desc()), _ptr(x), _ptr(w_dw), _ptr(b_dw), _ptr(w_pw), _ptr(b_pw),
                                   _ptr(res), _ptr(y), _stream(stream)))
        return y


def pack_nhwc_device(x, n, h, w, c, dt: DType, y, stream=None):
    """Logical NHWC fp32 on the device -> NHWC-C4 in dt (Model::upload_input's pack, on the GPU)."""
    _check(lib().aih_pack_nhwc_device(_ptr(x), n, h, w, c, int(dt), _ptr(y), _stream(stream)))
    return y


# ---------------------------------------------------------------- host packing (pack.rs)

def _np_storage(dt: DType):
    import numpy as np

    return np.float32 if dt == DType.F32 else np.uint16


def pack_nhwc(data, n, h, w, c, dt: DType = DType.F32):
    import numpy as np

    data = np.ascontiguousarray(data, np.float32)
    out = np.empty(n * h * w * (-(-c // 4)) * 4, _np_storage(dt))
    _check(lib().aih_pack_nhwc(data.ctypes.data, n, h, w, c, int(dt), out.ctypes.data))
    return out


def unpack_nhwc(packed, n, h, w, c, dt: DType = DType.F32):
    import numpy as np

    packed = np.ascontiguousarray(packed)
    out = np.empty(n * h * w * c, np.float32)
    _check(lib().aih_unpack_nhwc(packed.ctypes.data, n, h, w, c, int(dt), out.ctypes.data))
    return out


def pack_weights_conv(w_oihw, cout, cin, kh, kw, kg_align=4, dt: DType = DType.F32):
    import numpy as np

    w_oihw = np.ascontiguousarray(w_oihw, np.float32)
    al = max(kg_align, 1)
    kg = -(-(-(-cin // 4)) // al) * al
    out = np.empty(kh * kw * kg * (-(-cout // 4)) * 16, _np_storage(dt))
    kgp = lib().aih_pack_weights_conv(w_oihw.ctypes.data, cout, cin, kh, kw, kg_align, int(dt), out.ctypes.data)
    if kgp == 0:
        raise AihError(last_error())
    return out, kgp


def pack_weights_dw(w, c, kh, kw, dt: DType = DType.F32):
    import numpy as np

    w = np.ascontiguousarray(w, np.float32)
    out = np.empty(kh * kw * (-(-c // 4)) * 4, _np_storage(dt))
    _check(lib().aih_pack_weights_dw(w.ctypes.data, c, kh, kw, int(dt), out.ctypes.data))
    return out


def pack_bias(b, cout, dt: DType = DType.F32):
    import numpy as np

    b = np.ascontiguousarray(b, np.float32)
    out = np.empty(-(-cout // 4) * 4, _np_storage(dt))
    _check(lib().aih_pack_bias(b.ctypes.data, cout, int(dt), out.ctypes.data))
    return out

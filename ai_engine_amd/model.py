"""A conv graph resident on the GPU: the host-side mirror of the reference's
`ai_gpu_runtime::Model` (crates/ai-gpu-runtime/src/model.rs:56-457).

* construction = `Model::load`: weights are packed once in the converter's
  layout (pack.rs) and uploaded; every tensor gets its own NHWC-C4 device
  buffer (the batch is the outermost dimension);
* `upload_input` = `Model::upload_input` (:387-399): logical NHWC fp32 already
  on the device is packed to NHWC-C4 in the model dtype by a device kernel;
* `infer` = `Model::infer` (:402-426): every conv is issued in order on one
  stream through the C ABI (aih_conv routes each op like lower_op);
* `read_output` = `Model::read_output` (:442-457).
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import torch

from . import conv
from .workloads import Layer, Weights

ACT = {"none": conv.Activation.NONE, "relu": conv.Activation.RELU, "relu6": conv.Activation.RELU6,
       "hardswish": conv.Activation.HARDSWISH, "sigmoid": conv.Activation.SIGMOID}


def _storage_torch(dt: conv.DType):
    return torch.float32 if dt == conv.DType.F32 else torch.int16


def _to_device(a: np.ndarray, device) -> torch.Tensor:
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    return torch.from_numpy(a).to(device)


class Model:
    def __init__(self, layers: list[Layer], weights: Weights, n: int, ih: int, iw: int, cin: int,
                 dt: conv.DType = conv.DType.F32, wdt: conv.DType | None = None, device="cuda:0"):
        self.layers = layers
        self.n, self.ih, self.iw, self.cin = n, ih, iw, cin
        self.dt = conv.DType(dt)
        self.wdt = self.dt if wdt is None else conv.DType(wdt)
        self.device = torch.device(device)
        L = conv.lib()
        self._fn = L.aih_conv
        self.tensors: dict[str, torch.Tensor] = {}
        self.shapes: dict[str, tuple[int, int, int]] = {"input": (ih, iw, cin)}
        self.tensors["input"] = self._alloc(ih, iw, cin)
        self.ops = []
        self._keep = []
        for Lr in layers:
            oh, ow = Lr.out_hw()
            assert self.shapes[Lr.src][:2] == (Lr.ih, Lr.iw), Lr.name
            op = conv.ConvOp(ih=Lr.ih, iw=Lr.iw, cin=Lr.cin, cout=Lr.cout, kh=Lr.k, kw=Lr.k, sh=Lr.s, sw=Lr.s,
                             pad=(Lr.pad,) * 4, groups=Lr.groups, act=ACT[Lr.act], residual=Lr.res is not None,
                             dt=self.dt, wdt=self.wdt, n=n)
            w = weights.w[Lr.name]
            if Lr.depthwise:
                wp = conv.pack_weights_dw(w, Lr.cout, Lr.k, Lr.k, self.dt)
            else:
                wp, _ = conv.pack_weights_conv(w, Lr.cout, Lr.cin, Lr.k, Lr.k, 4, self.wdt)
            bp = conv.pack_bias(weights.b[Lr.name], Lr.cout, self.dt)
            wd, bd = _to_device(wp, self.device), _to_device(bp, self.device)
            y = self._alloc(oh, ow, Lr.cout)
            self.tensors[Lr.name] = y
            self.shapes[Lr.name] = (oh, ow, Lr.cout)
            nb = op.workspace_bytes()
            ws = torch.empty(max(nb // 4, 1), dtype=torch.float32, device=self.device) if nb else None
            desc = op.desc()
            res = self.tensors[Lr.res] if Lr.res else None
            args = (C.byref(desc), self.tensors[Lr.src].data_ptr(), wd.data_ptr(), bd.data_ptr(),
                    res.data_ptr() if res is not None else None, y.data_ptr(),
                    ws.data_ptr() if ws is not None else None, nb)
            self._keep += [desc, wd, bd, ws]
            self.ops.append((Lr, op, args))
        self.output = layers[-1].name

    def _alloc(self, h: int, w: int, c: int) -> torch.Tensor:
        return torch.empty(self.n * h * w * (-(-c // 4)) * 4, dtype=_storage_torch(self.dt), device=self.device)

    def upload_input(self, x_nhwc_f32: torch.Tensor, stream=None):
        conv.pack_nhwc_device(x_nhwc_f32, self.n, self.ih, self.iw, self.cin, self.dt, self.tensors["input"], stream)

    def infer(self, stream=None):
        s = conv._stream(stream)
        fn = self._fn
        for Lr, _, args in self.ops:
            if fn(*args, s) != 0:
                raise conv.AihError(f"{Lr.name}: {conv.last_error()}")

    def launch_op(self, i: int, stream=None):
        Lr, _, args = self.ops[i]
        if self._fn(*args, conv._stream(stream)) != 0:
            raise conv.AihError(f"{Lr.name}: {conv.last_error()}")

    def read_output(self, name: str | None = None) -> np.ndarray:
        """Unpacked logical NHWC fp32 of a tensor (default: the graph output)."""
        name = name or self.output
        h, w, c = self.shapes[name]
        a = self.tensors[name].detach().cpu().numpy()
        if a.dtype == np.int16:
            a = a.view(np.uint16)
        return conv.unpack_nhwc(a, self.n, h, w, c, self.dt)

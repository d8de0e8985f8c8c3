"""A conv graph resident on the GPU: the host-side mirror of the reference's
`ai_gpu_runtime::Model` (crates/ai-gpu-runtime/src/model.rs:56-457).

* construction = `Model::load`: weights are packed once in the converter's
  layout (pack.rs) and uploaded; every tensor gets its own NHWC-C4 device
  buffer (the batch is the outermost dimension);
* `upload_input` = `Model::upload_input` (:387-399): logical NHWC fp32 already
  on the device is packed to NHWC-C4 in the model dtype by a device kernel;
* `infer` = `Model::infer` (:402-426): every op is issued in order on one
  stream through the C ABI (aih_conv routes each conv like lower_op);
* `read_output` = `Model::read_output` (:442-457).

Load-time fusion: a 1x1 conv feeding a depthwise 3x3 feeding a 1x1 conv,
whose two intermediates have no other reader, becomes one aih_ir_block launch
(the expanded tensor stays on chip). The fused op reads the same packed
weights; blocks the fused kernel cannot run (aih_ir_block_plan fails) stay
three launches.

Load-time tuning (tune=True, the default): for every fusable block the
candidates -- the three separate launches, the fused launch at the planner's
tile and at a set of forced tiles, each with its weights resident in LDS and
streamed, and (fp32) the expand conv followed by one aih_conv_dwpw launch for
the depthwise and projection at each of its tiles -- are timed on the device
at load, a few launches each,
and the fastest is kept (like the reference's Model::load, which does its
per-model work -- pipeline compilation -- once at load). fuse="auto" lets the
timing choose between fused and separate; True keeps only fused candidates,
False never fuses. With tune=False the planner's tile is used and "auto"
fuses 16-bit models only.

The choice per block is recorded (choice_map()) and can be given back
(choices={block: label}), so a later load runs exactly the same kernels; a
label is "unfused", "fused THxTW" (the tile kernel, streamed weights),
"fused THxTW resident", "wave THxTW[ resident]" (the wave kernel),
"split THxTW wN" (the split kernel, N wavefronts per tile) or "dwpw THxTW rR"
(expand, then the fused depthwise + projection at that tile, R output rows
per wavefront) --
fused_candidates() and dwpw_candidates() list the labels a block can take.
"""
from __future__ import annotations

import ctypes as C
import dataclasses
import re
from dataclasses import dataclass, field

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


@dataclass
class ModelOp:
    """One launch of the graph: a single conv ("conv"), a fused block
    ("ir_block"), a fused depthwise + pointwise pair ("dw_pw"), the stem
    conv fused into the block after it ("stem_ir_block") or a block joined to
    the narrow pointwise head after it ("ir_block_head")."""

    name: str
    kind: str
    layers: list
    fn: object
    args: tuple
    spec: object = None
    keep: list = field(default_factory=list)

    def flops(self, n: int) -> int:
        return sum(L.flops(n) for L in self.layers)

    def bytes(self, n: int, act_bytes: int, w_bytes: int) -> int:
        """Algorithmic HBM bytes of this launch: each tensor it must read or
        write once (a fused block's intermediates never reach HBM)."""
        if self.kind == "conv":
            return self.layers[0].bytes(n, act_bytes, w_bytes)
        c4 = lambda c: -(-c // 4) * 4
        if self.kind == "dw_pw":
            d, p = self.layers
            oh, ow = p.out_hw()
            x = n * d.ih * d.iw * c4(d.cin) * act_bytes
            y = n * oh * ow * p.cout * act_bytes
            r = y if p.res else 0
            w = (d.k * d.k * d.cout + p.cin * p.cout) * w_bytes + (d.cout + p.cout) * act_bytes
            return x + y + r + w
        if self.kind == "stem_ir_block":
            # the fp32 image in, the block's output out, weights once: the
            # stem's output (the block's input and residual) is never stored
            S, e, d, p = self.layers
            oh, ow = p.out_hw()
            x = n * S.ih * S.iw * S.cin * 4
            y = n * oh * ow * p.cout * act_bytes
            w = (S.k * S.k * S.cin * S.cout + e.cin * e.cout + d.k * d.k * d.cout + p.cin * p.cout) * w_bytes
            b = (S.cout + e.cout + d.cout + p.cout) * act_bytes
            return x + y + w + b
        if self.kind == "ir_block_head":
            # the block's input (and a residual that is not it) in, the
            # head's output out, weights once: the block's output (the head's
            # input) is never stored
            e, d, p, H = self.layers
            oh, ow = p.out_hw()
            x = n * e.ih * e.iw * c4(e.cin) * act_bytes
            r = n * oh * ow * p.cout * act_bytes if p.res and p.res != e.src else 0
            y = n * oh * ow * c4(H.cout) * act_bytes
            w = (e.cin * e.cout + d.k * d.k * d.cout + p.cin * p.cout + H.cin * H.cout) * w_bytes
            b = (e.cout + d.cout + p.cout + c4(H.cout)) * act_bytes
            return x + r + y + w + b
        e, d, p = self.layers
        oh, ow = p.out_hw()
        x = n * e.ih * e.iw * c4(e.cin) * act_bytes
        y = n * oh * ow * p.cout * act_bytes
        # a residual that is the block's own input is the tensor already
        # counted in x: each tensor once (crates/ai-cpu/src/model.rs:241-272)
        r = y if p.res and p.res != e.src else 0
        w = (e.cin * e.cout + d.k * d.k * d.cout + p.cin * p.cout) * w_bytes
        b = (e.cout + d.cout + p.cout) * act_bytes
        return x + y + r + w + b


class Model:
    # forced output tiles (h, w) tried for a fused block besides the planner's:
    # for the tile kernel (a workgroup per tile) and the wave kernel (a
    # wavefront per tile of at most 32 pixels)
    TUNE_TILES = [(2, 8), (4, 4), (4, 8), (8, 4), (4, 16), (8, 8), (16, 4), (2, 32), (4, 32), (8, 16), (16, 8),
                  (8, 32), (16, 16)]
    WAVE_TILES = [(4, 8), (8, 4), (5, 6), (6, 5), (2, 16), (16, 2), (3, 10)]
    SPLIT_WAVES = [2, 4, 8]
    WAVE_WAVES = [4, 8, 12]  # wave-kernel workgroup sizes (12: the shapes that allow it)
    # a block's label with this prefix: the stem conv before it fused into its
    # launch (aih_ir_block_stem), the rest naming the block's wave-kernel plan
    STEM_PREFIX = "stem+"
    STEM_WAVES = [4, 8, 12]
    # a block's label with this suffix: the narrow pointwise head after it
    # joined to its launch (aih_ir_block_head), the rest naming the block's
    # split-kernel plan
    HEAD_SUFFIX = "+head"

    def __init__(self, layers: list[Layer], weights: Weights, n: int, ih: int, iw: int, cin: int,
                 dt: conv.DType = conv.DType.F32, wdt: conv.DType | None = None, device="cuda:0",
                 fuse="auto", tune: bool = True, choices: dict[str, str] | None = None):
        self.layers = layers
        self.n, self.ih, self.iw, self.cin = n, ih, iw, cin
        self.dt = conv.DType(dt)
        self.wdt = self.dt if wdt is None else conv.DType(wdt)
        self.device = torch.device(device)
        L = conv.lib()
        self.tensors: dict[str, torch.Tensor] = {}
        self.shapes: dict[str, tuple[int, int, int]] = {"input": (ih, iw, cin)}
        self.tensors["input"] = self._alloc(ih, iw, cin)
        self.ops: list[ModelOp] = []
        self.output = layers[-1].name

        readers: dict[str, int] = {}
        for Lr in layers:
            readers[Lr.src] = readers.get(Lr.src, 0) + 1
            if Lr.res:
                readers[Lr.res] = readers.get(Lr.res, 0) + 1

        packed = {}
        for Lr in layers:
            w = weights.w[Lr.name]
            if Lr.depthwise:
                wp = conv.pack_weights_dw(w, Lr.cout, Lr.k, Lr.k, self.dt)
            else:
                wp, _ = conv.pack_weights_conv(w, Lr.cout, Lr.cin, Lr.k, Lr.k, 4, self.wdt)
            bp = conv.pack_bias(weights.b[Lr.name], Lr.cout, self.dt)
            packed[Lr.name] = (_to_device(wp, self.device), _to_device(bp, self.device))
            self.shapes[Lr.name] = Lr.out_hw() + (Lr.cout,)

        self.choices: dict[str, tuple[str, float]] = {}  # block -> (chosen candidate, us), when tuned
        if fuse == "auto" and not tune:
            fuse = self.dt != conv.DType.F32
        i = 0
        while i < len(layers):
            blk = self._match_block(layers, i, readers) if (fuse or choices) else None
            if blk is not None and choices is not None:
                self.ops.extend(self._chosen_block(blk, packed, L, choices))
                i += 3
                continue
            if blk is not None and (tune and fuse == "auto" or blk[3].fusable()):
                if tune:
                    self.ops.extend(self._tuned_block(blk, packed, L, allow_unfused=fuse == "auto"))
                else:
                    self.ops.append(self._fused_op(blk, packed, L))
                i += 3
                continue
            self.ops.append(self._conv_op(layers[i], packed, L))
            i += 1
        # a stem that is the input's only reader reads the fp32 input itself
        self._x_f32 = None        # the uploaded fp32 input, held until the next upload
        self._x_version = 0       # its version counter at the upload
        self._input_packed = True  # tensors["input"] holds the last upload
        self._stem_in = self._stem_input_op(layers, readers, packed, L)
        # the stem fused into the block after it: op 0 reads the fp32 upload
        self._stem_fused = self._fuse_stem(layers, readers, packed, L, tune, choices)
        # the narrow head joined to the block before it
        self._head_fused = self._fuse_head(readers, packed, L, tune, choices)

    # ------------------------------------------------------------ graph building

    def _match_block(self, layers, i, readers):
        if i + 2 >= len(layers):
            return None
        e, d, p = layers[i:i + 3]
        if e.depthwise or e.k != 1 or e.s != 1:
            return None
        if not d.depthwise or d.k != 3 or d.src != e.name or d.cin != e.cout or d.res:
            return None
        if p.depthwise or p.k != 1 or p.s != 1 or p.src != d.name or e.res:
            return None
        if readers.get(e.name, 0) != 1 or readers.get(d.name, 0) != 1 or self.output in (e.name, d.name):
            return None
        if self.wdt != self.dt:
            return None
        spec = conv.IrBlockSpec(ih=e.ih, iw=e.iw, cin=e.cin, cexp=e.cout, cout=p.cout, s=d.s, pad=(d.pad,) * 4,
                                act_expand=ACT[e.act], act_dw=ACT[d.act], act_project=ACT[p.act],
                                residual=p.res is not None, dt=self.dt, n=self.n)
        if not spec.fusable() and not self.dwpw_candidates(self._dwpw_spec(d, p)):
            return None
        return (e, d, p, spec)

    def _dwpw_spec(self, d, p) -> conv.DwPwSpec:
        return conv.DwPwSpec(ih=d.ih, iw=d.iw, c=d.cin, cout=p.cout, k=d.k, s=d.s, pad=(d.pad,) * 4,
                             act_dw=ACT[d.act], act_pw=ACT[p.act], residual=p.res is not None, dt=self.dt,
                             n=self.n)

    DWPW_TILES = [(4, 16), (8, 16), (4, 32), (16, 16), (8, 32), (4, 64)]

    @classmethod
    def dwpw_candidates(cls, spec: conv.DwPwSpec) -> list[tuple[str, conv.DwPwSpec]]:
        """The fused depthwise + projection launches the tuner times after the
        expand conv: every DWPW_TILES entry with 4 and with 2 output rows per
        wavefront that fits, as (label, spec with tile and rows forced); none
        for a pair aih_conv_dwpw cannot run."""
        out = []
        for t in cls.DWPW_TILES:
            for rows in (4, 2):
                sp = dataclasses.replace(spec, tile=t, rows=rows)
                if sp.fusable():
                    out.append((f"dwpw {t[0]}x{t[1]} r{rows}", sp))
        return out

    @classmethod
    def fused_candidates(cls, spec: conv.IrBlockSpec) -> list[tuple[str, conv.IrBlockSpec]]:
        """The fused launches the tuner times for a block: on the tile kernel
        the planner's tile and every TUNE_TILES entry, on the wave kernel the
        planner's tile and every WAVE_TILES entry, each with resident and
        streamed weights (the ones that fit) and with the planner's or each
        of WAVE_WAVES wavefronts per workgroup, on the split kernel the planner's
        tile and every WAVE_TILES entry with each of SPLIT_WAVES wavefronts,
        as (label, spec with kernel, tile, placement and wavefronts forced);
        duplicates dropped."""
        out, seen = [], set()
        K, Wt = conv.IrKernel, conv.IrWeights
        opts = [(K.TILE, t, w, 0) for t in [(0, 0)] + cls.TUNE_TILES for w in (Wt.RESIDENT, Wt.STREAMED)]
        opts += [(K.WAVE, t, w, n) for t in [(0, 0)] + cls.WAVE_TILES for w in (Wt.RESIDENT, Wt.STREAMED)
                 for n in [0] + cls.WAVE_WAVES]
        opts += [(K.SPLIT, t, Wt.AUTO, n) for t in [(0, 0)] + cls.WAVE_TILES for n in cls.SPLIT_WAVES]
        for kernel, tile, w, waves in opts:
            sp = dataclasses.replace(spec, tile=tile, weights=w, kernel=kernel, waves=waves)
            if not sp.fusable():
                continue
            pl = sp.plan()
            key = (int(kernel), pl.th, pl.tw, pl.resident, pl.waves if kernel in (K.SPLIT, K.WAVE) else 0)
            if key in seen:
                continue
            seen.add(key)
            out.append((cls.label_of(kernel, pl.th, pl.tw, pl.resident, pl.waves),
                        dataclasses.replace(spec, tile=(pl.th, pl.tw), weights=w, kernel=kernel, waves=waves)))
        return out

    @staticmethod
    def label_of(kernel, th: int, tw: int, resident: bool, waves: int = 0) -> str:
        k = conv.IrKernel(kernel)
        if k == conv.IrKernel.SPLIT:
            return f"split {th}x{tw} w{waves}"
        if k == conv.IrKernel.WAVE:
            return f"wave {th}x{tw}{' resident' if resident else ''} w{waves}"
        return f"fused {th}x{tw}{' resident' if resident else ''}"

    @staticmethod
    def parse_label(label: str):
        """"unfused" -> None; "fused THxTW[ resident]", "wave THxTW[ resident][ wN]"
        or "split THxTW wN" -> (IrKernel, (th, tw), IrWeights, wavefronts or 0
        for the plan's choice); "dwpw THxTW rN" -> ("dwpw", (th, tw), None,
        rows per wavefront)."""
        if label == "unfused":
            return None
        if label.startswith(Model.STEM_PREFIX):  # the block fused with the stem before it: the block's part
            label = label[len(Model.STEM_PREFIX):]
        if label.endswith(Model.HEAD_SUFFIX):  # the block joined to the head after it: the block's part
            label = label[:-len(Model.HEAD_SUFFIX)]
        m = re.fullmatch(r"dwpw (\d+)x(\d+) r([24])", label)
        if m:
            return "dwpw", (int(m.group(1)), int(m.group(2))), None, int(m.group(3))
        m = re.fullmatch(r"split (\d+)x(\d+) w(\d+)", label)
        if m:
            return conv.IrKernel.SPLIT, (int(m.group(1)), int(m.group(2))), conv.IrWeights.AUTO, int(m.group(3))
        m = re.fullmatch(r"wave (\d+)x(\d+)( resident)?(?: w(\d+))?", label)
        if m:
            w = conv.IrWeights.RESIDENT if m.group(3) else conv.IrWeights.STREAMED
            return conv.IrKernel.WAVE, (int(m.group(1)), int(m.group(2))), w, int(m.group(4) or 0)
        m = re.fullmatch(r"fused (\d+)x(\d+)( resident)?", label)
        if not m:
            raise ValueError(f"unknown block choice {label!r}")
        w = conv.IrWeights.RESIDENT if m.group(3) else conv.IrWeights.STREAMED
        return conv.IrKernel.TILE, (int(m.group(1)), int(m.group(2))), w, 0

    def choice_map(self) -> dict[str, str]:
        """Block -> the label of the launch it runs (feed back as choices=)."""
        return {k: v[0] for k, v in self.choices.items()}

    def _block_name(self, p) -> str:
        return p.name.rsplit(".", 1)[0]

    def _chosen_block(self, blk, packed, L, choices) -> list:
        """The block as `choices` names it (no timing); a block missing from
        the map runs unfused."""
        e, d, p, spec = blk
        label = choices.get(self._block_name(p), "unfused")
        forced = self.parse_label(label)
        self.choices[self._block_name(p)] = (label, float("nan"))
        if forced is None:
            return [self._conv_op(Lr, packed, L) for Lr in (e, d, p)]
        kernel, tile, w, waves = forced
        if kernel == "dwpw":
            sp = dataclasses.replace(self._dwpw_spec(d, p), tile=tile, rows=waves)
            if not sp.fusable():
                raise conv.AihError(f"{self._block_name(p)}: {label!r}: {conv.last_error()}")
            return [self._conv_op(e, packed, L), self._dwpw_op(d, p, sp, packed, L)]
        sp = dataclasses.replace(spec, tile=tile, weights=w, kernel=kernel, waves=waves)
        pl = sp.plan()
        planned = self.label_of(pl.kernel, pl.th, pl.tw, pl.resident, pl.waves)
        if kernel == conv.IrKernel.WAVE and not waves:
            planned = planned.rsplit(" w", 1)[0]  # a label without a count takes the plan's
        if planned != label.removeprefix(self.STEM_PREFIX).removesuffix(self.HEAD_SUFFIX):
            raise conv.AihError(f"{self._block_name(p)}: {label!r} planned as "
                                f"{self.label_of(pl.kernel, pl.th, pl.tw, pl.resident, pl.waves)!r}")
        return [self._fused_op((e, d, p, sp), packed, L)]

    def _tuned_block(self, blk, packed, L, allow_unfused: bool) -> list:
        """Times the block's candidates on the device and returns the fastest
        one's ops (an unfused winner keeps its intermediates)."""
        e, d, p, spec = blk
        cands = []
        if allow_unfused:
            cands.append(("unfused", [self._conv_op(Lr, packed, L) for Lr in (e, d, p)]))
        else:
            oh, ow = p.out_hw()
            self.tensors[p.name] = self._alloc(oh, ow, p.cout)
        y = self.tensors[p.name]
        if spec.fusable():
            for label, sp in self.fused_candidates(spec):
                cands.append((label, [self._fused_op((e, d, p, sp), packed, L, y=y)]))
        if allow_unfused:
            expand = cands[0][1][0]
            for label, sp in self.dwpw_candidates(self._dwpw_spec(d, p)):
                cands.append((label, [expand, self._dwpw_op(d, p, sp, packed, L, y=y)]))
        # two passes over the candidates, each keeping its faster median: a
        # clock or cache drift during one pass does not pick the winner
        t1 = [self._time_ops(ops) for _, ops in cands]
        t2 = [self._time_ops(ops) for _, ops in cands]
        timed = [(min(a, b), label, ops) for a, b, (label, ops) in zip(t1, t2, cands)]
        us, label, ops = min(timed, key=lambda t: t[0])
        self.choices[self._block_name(p)] = (label, us)
        if label != "unfused":
            for nm in ((d.name,) if label.startswith("dwpw") else (e.name, d.name)):
                self.tensors.pop(nm, None)
        return ops

    def _time_ops(self, ops, reps: int = 9) -> float:
        """Median device time (us) of one pass over ops, on the current stream."""
        s = conv._stream(None)

        def once():
            for op in ops:
                if op.fn(*op.args, s) != 0:
                    raise conv.AihError(f"{op.name}: {conv.last_error()}")

        once()
        once()
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
        for a, b in ev:
            a.record()
            once()
            b.record()
        torch.cuda.synchronize(self.device)
        ts = sorted(a.elapsed_time(b) for a, b in ev)
        return ts[len(ts) // 2] * 1e3

    def _fused_op(self, blk, packed, L, y=None) -> ModelOp:
        e, d, p, spec = blk
        oh, ow = p.out_hw()
        if y is None:
            y = self._alloc(oh, ow, p.cout)
        self.tensors[p.name] = y
        desc = spec.desc()
        res = self.tensors[p.res] if p.res else None
        args = (C.byref(desc), self.tensors[e.src].data_ptr(), packed[e.name][0].data_ptr(),
                packed[e.name][1].data_ptr(), packed[d.name][0].data_ptr(), packed[d.name][1].data_ptr(),
                packed[p.name][0].data_ptr(), packed[p.name][1].data_ptr(),
                res.data_ptr() if res is not None else None, y.data_ptr())
        keep = [desc] + [t for nm in (e.name, d.name, p.name) for t in packed[nm]]
        return ModelOp(p.name.rsplit(".", 1)[0], "ir_block", [e, d, p], L.aih_ir_block, args, spec, keep)

    def _dwpw_op(self, d, p, spec: conv.DwPwSpec, packed, L, y=None) -> ModelOp:
        """The depthwise conv d and the projection p as one aih_conv_dwpw launch."""
        oh, ow = p.out_hw()
        if y is None:
            y = self._alloc(oh, ow, p.cout)
        self.tensors[p.name] = y
        desc = spec.desc()
        res = self.tensors[p.res] if p.res else None
        args = (C.byref(desc), self.tensors[d.src].data_ptr(), packed[d.name][0].data_ptr(),
                packed[d.name][1].data_ptr(), packed[p.name][0].data_ptr(), packed[p.name][1].data_ptr(),
                res.data_ptr() if res is not None else None, y.data_ptr())
        keep = [desc] + [t for nm in (d.name, p.name) for t in packed[nm]]
        return ModelOp(p.name.rsplit(".", 1)[0] + ".dwpw", "dw_pw", [d, p], L.aih_conv_dwpw, args, spec, keep)

    def _conv_op(self, Lr, packed, L) -> ModelOp:
        oh, ow = Lr.out_hw()
        assert self.shapes[Lr.src][:2] == (Lr.ih, Lr.iw), Lr.name
        op = conv.ConvOp(ih=Lr.ih, iw=Lr.iw, cin=Lr.cin, cout=Lr.cout, kh=Lr.k, kw=Lr.k, sh=Lr.s, sw=Lr.s,
                         pad=(Lr.pad,) * 4, groups=Lr.groups, act=ACT[Lr.act], residual=Lr.res is not None,
                         dt=self.dt, wdt=self.wdt, n=self.n)
        wd, bd = packed[Lr.name]
        y = self._alloc(oh, ow, Lr.cout)
        self.tensors[Lr.name] = y
        nb = op.workspace_bytes()
        ws = torch.empty(max(nb // 4, 1), dtype=torch.float32, device=self.device) if nb else None
        desc = op.desc()
        res = self.tensors[Lr.res] if Lr.res else None
        args = (C.byref(desc), self.tensors[Lr.src].data_ptr(), wd.data_ptr(), bd.data_ptr(),
                res.data_ptr() if res is not None else None, y.data_ptr(),
                ws.data_ptr() if ws is not None else None, nb)
        return ModelOp(Lr.name, "conv", [Lr], L.aih_conv, args, op, [desc, wd, bd, ws])

    def _stem_input_op(self, layers, readers, packed, L) -> ModelOp | None:
        """The first op as a stem launch on the logical NHWC fp32 input
        (aih_conv_stem_f32in): the pack of upload_input and the stem in one
        kernel, bit for bit the same result. Only for a first layer on the
        stem route whose input nothing else reads."""
        if not self.ops or self.ops[0].kind != "conv":
            return None
        Lr = layers[0]
        if (Lr.src != "input" or readers.get("input", 0) != 1 or Lr.depthwise or Lr.groups != 1 or Lr.k != 3
                or Lr.cin > 3 or Lr.cout not in (32, 64) or self.wdt != self.dt):
            return None
        spec = conv.ConvIgemmSpec(ih=Lr.ih, iw=Lr.iw, cin=Lr.cin, cout=Lr.cout, k=3, s=Lr.s, pad=(Lr.pad,) * 4,
                                  act=ACT[Lr.act], residual=Lr.res is not None, dt=self.dt, wdt=self.wdt, n=self.n)
        desc = spec.desc()
        wd, bd = packed[Lr.name]
        res = self.tensors[Lr.res] if Lr.res else None
        y = self.tensors[Lr.name]
        args = (C.byref(desc), None, wd.data_ptr(), bd.data_ptr(), res.data_ptr() if res is not None else None,
                y.data_ptr())
        return ModelOp(Lr.name, "conv", [Lr], L.aih_conv_stem_f32in, args, spec, [desc, wd, bd])

    def _stem_block_op(self, blk, sp: conv.StemIrBlockSpec, packed, L, y, image=None) -> ModelOp:
        """The stem conv (op 0) and the block after it (blk) as one
        aih_ir_block_stem launch reading the fp32 image."""
        S = self._stem_in.layers[0]
        e, d, p = blk.layers
        self.tensors[p.name] = y
        sd, bd = sp.stem.desc(), sp.block.desc()
        args = (C.byref(sd), C.byref(bd), image.data_ptr() if image is not None else None,
                packed[S.name][0].data_ptr(), packed[S.name][1].data_ptr()) + tuple(
            packed[nm][k].data_ptr() for nm in (e.name, d.name, p.name) for k in (0, 1)) + (y.data_ptr(),)
        keep = [sd, bd] + [t for nm in (S.name, e.name, d.name, p.name) for t in packed[nm]]
        return ModelOp(f"{S.name}+{blk.name}", "stem_ir_block", [S, e, d, p], L.aih_ir_block_stem, args, sp, keep)

    def _fuse_stem(self, layers, readers, packed, L, tune: bool, choices) -> bool:
        """Fuses the stem conv (op 0, on the fp32 input) into the
        inverted-residual block after it when that block reads the stem's
        output as its input and residual and nothing else does: recorded
        choices fuse it where the block's label carries STEM_PREFIX; the
        tuner times the stem + the chosen block against the fused launch at
        the planner's and the WAVE_TILES tiles, resident and streamed
        weights, the planner's or STEM_WAVES wavefronts, and keeps the
        faster. The stem's output is then never stored."""
        if self._stem_in is None or len(self.ops) < 2 or self.ops[1].kind != "ir_block":
            return False
        S, blk = layers[0], self.ops[1]
        e, d, p = blk.layers
        if e.src != S.name or p.res != S.name or readers.get(S.name, 0) != 2 or self.output == S.name:
            return False
        name = self._block_name(p)
        y = self.tensors[p.name]
        K, Wt = conv.IrKernel, conv.IrWeights
        if choices is not None:
            label = self.choices.get(name, ("", 0.0))[0]
            if not label.startswith(self.STEM_PREFIX):
                return False
            _, tile, w, waves = self.parse_label(label)
            sp = conv.StemIrBlockSpec(self._stem_in.spec,
                                      dataclasses.replace(blk.spec, tile=tile, weights=w, kernel=K.WAVE, waves=waves))
            if not sp.fusable():
                raise conv.AihError(f"{name}: {label!r}: {conv.last_error()}")
            self.ops[0:2] = [self._stem_block_op(blk, sp, packed, L, y)]
            self.tensors.pop(S.name, None)
            return True
        if not tune:
            return False
        # time on a stand-in image (the stem's input slot is the caller's tensor)
        xt = torch.zeros(self.n * self.ih * self.iw * self.cin, dtype=torch.float32, device=self.device)
        a0 = self._stem_in.args
        self._stem_in.args = (a0[0], xt.data_ptr()) + a0[2:]
        cands, seen = [], set()
        for tile in [(0, 0)] + self.WAVE_TILES:
            for w in (Wt.RESIDENT, Wt.STREAMED):
                for waves in [0] + self.STEM_WAVES:
                    sp = conv.StemIrBlockSpec(self._stem_in.spec, dataclasses.replace(
                        blk.spec, tile=tile, weights=w, kernel=K.WAVE, waves=waves))
                    if not sp.fusable():
                        continue
                    pl = sp.plan()
                    if (pl.th, pl.tw, pl.resident, pl.waves) in seen:
                        continue
                    seen.add((pl.th, pl.tw, pl.resident, pl.waves))
                    cands.append((self.STEM_PREFIX + self.label_of(K.WAVE, pl.th, pl.tw, pl.resident, pl.waves),
                                  self._stem_block_op(blk, sp, packed, L, y, image=xt)))
        # two passes, each candidate keeping its faster median (as _tuned_block)
        sep = [self._stem_in, blk]
        best_us = min(self._time_ops(sep), self._time_ops(sep)) if cands else 0.0
        t1 = [self._time_ops([op]) for _, op in cands]
        t2 = [self._time_ops([op]) for _, op in cands]
        best_label, best_op = None, None
        for a_, b_, (label, op) in zip(t1, t2, cands):
            if min(a_, b_) < best_us:
                best_us, best_label, best_op = min(a_, b_), label, op
        self._stem_in.args = a0
        self.tensors[p.name] = y
        if best_op is None:
            return False
        a = best_op.args
        best_op.args = a[:2] + (None,) + a[3:]
        self.choices[name] = (best_label, best_us)
        self.ops[0:2] = [best_op]
        self.tensors.pop(S.name, None)
        return True

    def _head_op(self, blk: ModelOp, hop: ModelOp, sp: conv.IrBlockHeadSpec, packed, L, y=None) -> ModelOp:
        """The block blk and the narrow pointwise head hop after it as one
        aih_ir_block_head launch; y: where the block's output goes, or None
        (not stored)."""
        e, d, p = blk.layers
        H = hop.layers[0]
        bd, hd = sp.block.desc(), sp.head.desc()
        res = self.tensors[p.res] if p.res else None
        yh = self.tensors[H.name]
        args = (C.byref(bd), C.byref(hd), self.tensors[e.src].data_ptr()) + tuple(
            packed[nm][k].data_ptr() for nm in (e.name, d.name, p.name) for k in (0, 1)) + (
            res.data_ptr() if res is not None else None, y.data_ptr() if y is not None else None,
            packed[H.name][0].data_ptr(), packed[H.name][1].data_ptr(), yh.data_ptr())
        keep = [bd, hd] + [t for nm in (e.name, d.name, p.name, H.name) for t in packed[nm]]
        return ModelOp(f"{blk.name}+{H.name}", "ir_block_head", [e, d, p, H], L.aih_ir_block_head, args, sp, keep)

    def _fuse_head(self, readers, packed, L, tune: bool, choices) -> bool:
        """Joins the last op, a 1x1 conv with at most 4 outputs (the
        segmentation head) that alone reads the output of the fused block
        before it, to that block's launch (aih_ir_block_head, the split
        kernel): recorded choices join it where the block's label carries
        HEAD_SUFFIX; the tuner times the block and the head against the
        joined launch at the planner's and the WAVE_TILES tiles with each of
        SPLIT_WAVES wavefronts (two passes) and keeps the faster. The block's
        output is then never stored."""
        if len(self.ops) < 2 or self.ops[-1].kind != "conv" or self.ops[-2].kind != "ir_block":
            return False
        blk, hop = self.ops[-2], self.ops[-1]
        H = hop.layers[0]
        e, d, p = blk.layers
        if (H.depthwise or H.groups != 1 or H.k != 1 or H.s != 1 or H.res or H.cout > 4 or H.src != p.name
                or readers.get(p.name, 0) != 1 or self.output != H.name or self.wdt != self.dt
                or self.dt == conv.DType.F32):
            return False
        name = self._block_name(p)
        oh, ow = p.out_hw()
        hs = conv.GemmPwSpec(m=oh * ow, kg=p.cout // 4, ng=1, act=ACT[H.act], dt=self.dt, wdt=self.wdt, n=self.n)
        K = conv.IrKernel
        label0 = self.choices.get(name, ("", 0.0))[0]
        if choices is not None:
            if not label0.endswith(self.HEAD_SUFFIX):
                return False
            sp = conv.IrBlockHeadSpec(blk.spec, hs)
            if not sp.fusable():
                raise conv.AihError(f"{name}: {label0!r}: {conv.last_error()}")
            self.ops[-2:] = [self._head_op(blk, hop, sp, packed, L)]
            self.tensors.pop(p.name, None)
            return True
        if not tune:
            return False
        cands, seen = [], set()
        for tile in [(0, 0)] + self.WAVE_TILES:
            for waves in self.SPLIT_WAVES:
                sp = conv.IrBlockHeadSpec(dataclasses.replace(blk.spec, tile=tile, kernel=K.SPLIT, waves=waves,
                                                              weights=conv.IrWeights.AUTO), hs)
                if not sp.fusable():
                    continue
                pl = sp.plan()
                if (pl.th, pl.tw, pl.waves) in seen:
                    continue
                seen.add((pl.th, pl.tw, pl.waves))
                sp = conv.IrBlockHeadSpec(dataclasses.replace(sp.block, tile=(pl.th, pl.tw), waves=pl.waves), hs)
                cands.append((self.label_of(K.SPLIT, pl.th, pl.tw, False, pl.waves) + self.HEAD_SUFFIX,
                              self._head_op(blk, hop, sp, packed, L)))
        if not cands:
            return False
        # two passes, each candidate keeping its faster median (as _tuned_block)
        best_us = min(self._time_ops([blk, hop]), self._time_ops([blk, hop]))
        t1 = [self._time_ops([op]) for _, op in cands]
        best_label, best_op = None, None
        for a_, (label, op) in zip(t1, cands):
            us = min(a_, self._time_ops([op]))
            if us < best_us:
                best_us, best_label, best_op = us, label, op
        if best_op is None:
            return False
        self.choices[name] = (best_label, best_us)
        self.ops[-2:] = [best_op]
        self.tensors.pop(p.name, None)
        return True

    def _alloc(self, h: int, w: int, c: int) -> torch.Tensor:
        return torch.empty(self.n * h * w * (-(-c // 4)) * 4, dtype=_storage_torch(self.dt), device=self.device)

    # ------------------------------------------------------------ runtime verbs

    def upload_input(self, x_nhwc_f32: torch.Tensor, stream=None):
        """The next infer()'s input. With a stem as the first op the fp32
        tensor itself is the stem's input (no packed copy; the model holds
        it until the next upload, and it must not change before infer()
        has run: an in-place torch write to it after the upload -- which
        bumps the tensor's version counter -- makes infer() raise instead of
        reading the new values; writes torch does not see, through its raw
        pointer, are the caller's to order); otherwise it is packed into the
        input slot now."""
        if self._stem_in is None:
            conv.pack_nhwc_device(x_nhwc_f32, self.n, self.ih, self.iw, self.cin, self.dt, self.tensors["input"],
                                  stream)
            return
        x = x_nhwc_f32
        if (not isinstance(x, torch.Tensor) or x.device != self.device or x.dtype != torch.float32
                or not x.is_contiguous() or x.numel() != self.n * self.ih * self.iw * self.cin):
            raise conv.AihError(f"upload_input: expected a contiguous float32 tensor of "
                                f"{self.n * self.ih * self.iw * self.cin} values on {self.device}")
        self._x_f32 = x
        self._x_version = x._version
        self._input_packed = False
        a = self._stem_in.args
        self._stem_in.args = (a[0], x.data_ptr()) + a[2:]
        if self._stem_fused:
            f = self.ops[0].args
            self.ops[0].args = f[:2] + (x.data_ptr(),) + f[3:]

    def sync_input(self):
        """Fills tensors["input"] with the last upload when the stem read the
        fp32 tensor directly (for inspecting the stored input; later infer()
        calls then read the slot)."""
        if not self._input_packed:
            conv.pack_nhwc_device(self._x_f32, self.n, self.ih, self.iw, self.cin, self.dt, self.tensors["input"])
            torch.cuda.synchronize(self.device)
            self._input_packed = True

    def _op(self, i: int) -> ModelOp:
        # op 0 reads the fp32 upload while it has not been packed into the
        # input slot; otherwise (no upload yet, or the slot written) the slot.
        # A stem fused into the block after it always reads the upload.
        if i == 0 and self._stem_in is not None and (self._stem_fused or not self._input_packed):
            if self._x_f32 is None:
                raise conv.AihError("infer: the stem fused into the first block reads the fp32 upload: "
                                    "call upload_input first")
            if self._x_f32._version != self._x_version:
                raise conv.AihError("infer: the tensor given to upload_input was modified in place after the "
                                    "upload; call upload_input again")
            return self.ops[0] if self._stem_fused else self._stem_in
        return self.ops[i]

    def infer(self, stream=None):
        s = conv._stream(stream)
        for i in range(len(self.ops)):
            op = self._op(i)
            if op.fn(*op.args, s) != 0:
                raise conv.AihError(f"{op.name}: {conv.last_error()}")

    def launch_op(self, i: int, stream=None):
        op = self._op(i)
        if op.fn(*op.args, conv._stream(stream)) != 0:
            raise conv.AihError(f"{op.name}: {conv.last_error()}")

    def read_output(self, name: str | None = None) -> np.ndarray:
        """Unpacked logical NHWC fp32 of a tensor (default: the graph output)."""
        name = name or self.output
        h, w, c = self.shapes[name]
        if name == "input":
            self.sync_input()
        if name not in self.tensors:
            raise conv.AihError(f"read_output: {name!r} is an intermediate of a fused launch and is not stored")
        a = self.tensors[name].detach().cpu().numpy()
        if a.dtype == np.int16:
            a = a.view(np.uint16)
        return conv.unpack_nhwc(a, self.n, h, w, c, self.dt)

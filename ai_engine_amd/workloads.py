"""Synthetic conv workloads measured on the MI355X, with their algorithmic work.

Each layer is a SwOp::Conv (crates/ai-core/src/format/model.rs:80-111) with
NHWC tensors and the batch outermost.  Work is counted as the reference's
ai-cpu profiler counts it (crates/ai-cpu/src/model.rs:241-272): flops =
2 * MACs (depthwise 2 * M * k^2 * C), bytes = input + weights + bias + output
(+ residual), each touched once at its storage width; the epilogue is free.

Weights are He-initialised N(0, sqrt(2 / (k^2 * cin))), inputs U[-1, 1),
biases N(0, 0.01) -- random-init weights of the named architecture (no
checkpoints are used).
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np


@dataclass
class Layer:
    name: str
    cin: int
    cout: int
    k: int = 1
    s: int = 1
    groups: int = 1
    act: str = "none"
    res: str | None = None   # name of the tensor added after the activation
    src: str | None = None   # input tensor name (default: previous layer's output)
    ih: int = 0
    iw: int = 0

    @property
    def pad(self) -> int:
        return (self.k - 1) // 2

    @property
    def depthwise(self) -> bool:
        return self.groups > 1

    def out_hw(self) -> tuple[int, int]:
        p = self.pad
        return (self.ih + 2 * p - self.k) // self.s + 1, (self.iw + 2 * p - self.k) // self.s + 1

    def macs(self, n: int) -> int:
        oh, ow = self.out_hw()
        if self.depthwise:
            return n * oh * ow * self.k * self.k * self.cout
        return n * oh * ow * self.k * self.k * self.cin * self.cout

    def flops(self, n: int) -> int:
        return 2 * self.macs(n)

    def bytes(self, n: int, act_bytes: int, w_bytes: int) -> int:
        """Algorithmic HBM bytes (logical channel counts; the stem's 3-channel
        input is stored as 4 channels in NHWC-C4 and is counted as stored)."""
        oh, ow = self.out_hw()
        c4 = lambda c: -(-c // 4) * 4
        x = n * self.ih * self.iw * c4(self.cin) * act_bytes
        y = n * oh * ow * self.cout * act_bytes
        r = y if self.res else 0
        if self.depthwise:
            w = self.k * self.k * self.cout * act_bytes
        else:
            w = self.k * self.k * self.cin * self.cout * w_bytes
        return x + w + self.cout * act_bytes + y + r


def _chain(layers: list[Layer], ih: int, iw: int) -> list[Layer]:
    """Fill in spatial sizes and default sources down a sequential chain."""
    h, w = ih, iw
    prev = "input"
    shapes = {"input": (ih, iw)}
    for L in layers:
        if L.src is None:
            L.src = prev
        L.ih, L.iw = shapes[L.src]
        shapes[L.name] = L.out_hw()
        prev = L.name
    return layers


def inverted_residual(prefix: str, cin: int, cout: int, stride: int, expand: int = 4) -> list[Layer]:
    """MobileNet inverted residual: pw expand + ReLU, dw 3x3 (stride) + ReLU, pw
    project (linear) + residual when the shape is kept."""
    hid = cin * expand
    res = "@in" if (stride == 1 and cin == cout) else None
    return [
        Layer(f"{prefix}.expand", cin, hid, 1, 1, act="relu"),
        Layer(f"{prefix}.dw", hid, hid, 3, stride, groups=hid, act="relu"),
        Layer(f"{prefix}.project", hid, cout, 1, 1, act="none", res=res),
    ]


def _resolve_block_inputs(layers: list[Layer]) -> list[Layer]:
    # "@in" = the input of the block (the tensor feeding its expand layer)
    prev = "input"
    block_in = {}
    for L in layers:
        blk = L.name.split(".")[0]
        if L.name.endswith(".expand"):
            block_in[blk] = prev
        if L.res == "@in":
            L.res = block_in[blk]
        prev = L.name
    return layers


def ir_chain_40x72(n: int = 64) -> tuple[list[Layer], dict]:
    """Four stacked inverted-residual blocks at 40x72, 64 channels, expand 4."""
    layers = []
    for b in range(4):
        layers += inverted_residual(f"b{b}", 64, 64, 1)
    layers = _chain(_resolve_block_inputs(layers), 40, 72)
    return layers, dict(n=n, h=40, w=72, c=64, name="ir_block_chain_4x_64c_40x72")


def mnv4_small_encoder_160x288(n: int = 64) -> tuple[list[Layer], dict]:
    """MobileNetV4-small-width segmentation encoder at 160x288: stem 3x3 s2
    3->32, ten inverted-residual blocks (32, 32 | 64 s2, 64, 64 | 96 s2, 96, 96
    | 128 s2, 128; expand 4, stride on the depthwise), 1x1 head 128->2."""
    layers = [Layer("stem", 3, 32, 3, 2, act="relu")]
    spec = [(32, 32, 1), (32, 32, 1), (32, 64, 2), (64, 64, 1), (64, 64, 1), (64, 96, 2), (96, 96, 1),
            (96, 96, 1), (96, 128, 2), (128, 128, 1)]
    for i, (ci, co, s) in enumerate(spec):
        layers += inverted_residual(f"b{i}", ci, co, s)
    layers.append(Layer("head", 128, 2, 1, 1, act="none"))
    layers = _chain(_resolve_block_inputs(layers), 160, 288)
    return layers, dict(n=n, h=160, w=288, c=3, name="mnv4_small_encoder_160x288")


@dataclass
class Weights:
    w: dict = field(default_factory=dict)   # name -> OIHW fp32 ([c,k,k] for depthwise)
    b: dict = field(default_factory=dict)


def make_weights(layers: list[Layer], seed: int = 0) -> Weights:
    rng = np.random.default_rng(seed)
    W = Weights()
    for L in layers:
        fan_in = L.k * L.k * (1 if L.depthwise else L.cin)
        sigma = np.sqrt(2.0 / fan_in)
        shape = (L.cout, 1 if L.depthwise else L.cin, L.k, L.k)
        W.w[L.name] = (rng.standard_normal(shape) * sigma).astype(np.float32).ravel()
        W.b[L.name] = (rng.standard_normal(L.cout) * 0.01).astype(np.float32)
    return W


def totals(layers: list[Layer], n: int, act_bytes: int, w_bytes: int) -> tuple[int, int]:
    return (sum(L.flops(n) for L in layers), sum(L.bytes(n, act_bytes, w_bytes) for L in layers))

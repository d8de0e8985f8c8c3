"""The stem conv fused into the first inverted-residual block
(aih_ir_block_stem): one launch computing the stem's output inside the
block's halo loads, never storing it. The reference runs the stem conv and
the block's three convs as separate dispatches
(crates/ai-gpu-runtime/src/lowering.rs:122-168).

The fused launch must equal, bit for bit, the two launches it replaces on the
same plan: aih_conv_stem_f32in (itself bit-identical to pack-then-stem and
checked against the oracle in test_gpu_parity.py) into a stored stem output,
then aih_ir_block with that output as input and residual (checked against
the oracle's three-op chain in test_gpu_ir_block.py). Cases: the encoder's
shape (160x288 image, stride-2 stem, 32 -> 128 -> 32 block), odd image sizes
(block tiles overhanging the image), a stride-1 stem, asymmetric padding, a
batch of three, each clamp-type stem activation, forced tiles, wavefront
counts and weight placements, f16 and bf16. Outputs start as NaN.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():  # pragma: no cover
    pytest.skip("no GPU", allow_module_level=True)

from tests import gpu_util as G  # noqa: E402

from ai_engine_amd import conv  # noqa: E402

F16, BF16 = 1, 2

# (n, image h, w, stem stride, stem pad, stem act, block tile, waves, weights)
CASES = [
    (2, 160, 288, 2, (0, 0, 1, 1), "relu", (0, 0), 0, 0),
    (2, 160, 288, 2, (0, 0, 1, 1), "relu", (8, 4), 8, 1),
    (1, 37, 53, 2, (1, 1, 1, 1), "relu6", (4, 8), 4, 1),
    (3, 21, 30, 1, (1, 1, 1, 1), "none", (5, 6), 2, 2),
    (1, 45, 17, 2, (0, 1, 1, 0), "relu", (10, 3), 8, 2),
    (2, 16, 16, 2, (1, 1, 1, 1), "clamp01", (0, 0), 0, 0),
]


def _id(c):
    n, h, w, s, pad, act, tile, waves, wts = c
    return f"n{n}_{h}x{w}_s{s}_p{''.join(map(str, pad))}_{act}_t{tile[0]}x{tile[1]}_w{waves}_p{wts}"


def _case(case, dt, seed):
    n, h, w, s, pad, act, tile, waves, wts = case
    stem = conv.ConvIgemmSpec(ih=h, iw=w, cin=3, cout=32, k=3, s=s, pad=pad, act=G.ACT[act], residual=False,
                              dt=conv.DType(dt), n=n)
    oh, ow = stem.out_hw()
    blk = conv.IrBlockSpec(ih=oh, iw=ow, cin=32, cexp=128, cout=32, s=1, pad=(1, 1, 1, 1),
                           act_expand=G.ACT["relu"], act_dw=G.ACT["relu"], act_project=G.ACT["none"], residual=True,
                           dt=conv.DType(dt), n=n, tile=tile, waves=waves, weights=wts, kernel=conv.IrKernel.WAVE)
    o = G.orc
    we = o.gauss_fill(seed + 1, 0.0, float(np.sqrt(2.0 / 32)), 128 * 32)
    wd = o.gauss_fill(seed + 3, 0.0, float(np.sqrt(2.0 / 9)), 128 * 9)
    wp = o.gauss_fill(seed + 5, 0.0, float(np.sqrt(2.0 / 128)), 32 * 128)
    bufs = (G.dev(o.pack_weights_conv(we, 128, 32, 1, 1, 4, dt)[0]),
            G.dev(o.pack_bias(o.gauss_fill(seed + 2, 0.0, 0.01, 128), 128, dt)),
            G.dev(o.pack_weights_dw(wd, 128, 3, 3, dt)),
            G.dev(o.pack_bias(o.gauss_fill(seed + 4, 0.0, 0.01, 128), 128, dt)),
            G.dev(o.pack_weights_conv(wp, 32, 128, 1, 1, 4, dt)[0]),
            G.dev(o.pack_bias(o.gauss_fill(seed + 6, 0.0, 0.01, 32), 32, dt)))
    x, ws, bs, _ = G.stream(seed + 50, n * h * w * 3, 32 * 3 * 9, 32, 0)
    xf = G.dev(np.asarray(x, np.float32))
    wsp, _ = o.pack_weights_conv(ws, 32, 3, 3, 3, 4, dt)
    return stem, blk, bufs, xf, G.dev(wsp), G.dev(o.pack_bias(bs, 32, dt))


@pytest.mark.parametrize("dt", [F16, BF16], ids=["f16", "bf16"])
@pytest.mark.parametrize("case", CASES, ids=_id)
def test_stem_block_equals_stem_then_block(case, dt):
    stem, blk, bufs, xf, wsd, bsd = _case(case, dt, 8800 + 10 * CASES.index(case))
    fused = conv.StemIrBlockSpec(stem, blk)
    fp, bp_ = fused.plan(), blk.plan()
    print(f"case {_id(case)} dt{dt}: fused {fp}, block {bp_}", flush=True)
    # the same tile, placement and wavefronts on both sides
    assert (fp.th, fp.tw, fp.resident, fp.waves) == (bp_.th, bp_.tw, bp_.resident, bp_.waves), (fp, bp_)
    n, oh, ow = blk.n, blk.ih, blk.iw
    we, be, wd, bd, wp, bp = bufs
    mid = G.poisoned(n * oh * ow * 32, dt)
    stem.run_f32_input(xf, wsd, bsd, None, mid)
    want = G.poisoned(n * oh * ow * 32, dt)
    blk.run(mid, we, be, wd, bd, wp, bp, mid, want)
    got = G.poisoned(n * oh * ow * 32, dt)
    fused.run(xf, wsd, bsd, we, be, wd, bd, wp, bp, got)
    torch.cuda.synchronize()
    assert not torch.isnan(got.float()).any()
    assert torch.equal(got.view(-1), want.view(-1))
    # a second launch into the same buffer: the same bits
    fused.run(xf, wsd, bsd, we, be, wd, bd, wp, bp, got)
    torch.cuda.synchronize()
    assert torch.equal(got.view(-1), want.view(-1))


def test_stem_block_rejects_what_it_does_not_take():
    stem, blk, *_ = _case(CASES[0], F16, 8900)
    import dataclasses
    bad = [
        (dataclasses.replace(stem, cout=64), blk, "stem"),
        (dataclasses.replace(stem, act=G.ACT["sigmoid"]), blk, "clamp"),
        (stem, dataclasses.replace(blk, residual=False), "residual"),
        (stem, dataclasses.replace(blk, kernel=conv.IrKernel.SPLIT), "wave kernel"),
        (stem, dataclasses.replace(blk, dt=conv.DType.BF16), "f16 or both bf16"),
        (stem, dataclasses.replace(blk, ih=blk.ih + 1), "stem's output"),
        (dataclasses.replace(stem, dt=conv.DType.F32), dataclasses.replace(blk, dt=conv.DType.F32), "f16 or both bf16"),
    ]
    for s, b, why in bad:
        assert not conv.StemIrBlockSpec(s, b).fusable()
        assert why in conv.last_error(), (why, conv.last_error())

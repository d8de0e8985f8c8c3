"""The inverted-residual block joined to the narrow pointwise conv that reads
its output (aih_ir_block_head): one split-kernel launch computing the head's
products from each output block as it is stored. The reference runs the
block's three convs and the head as separate dispatches
(crates/ai-gpu-runtime/src/lowering.rs:122-168).

The joined launch must equal, bit for bit, the two launches it replaces on
the same plan: aih_ir_block (checked against the oracle's three-op chain in
test_gpu_ir_block.py and test_gpu_ir_tiles.py) into a stored block output,
then aih_conv_pw on the narrow route (checked against the oracle in
test_gpu_parity.py). The block's output, when the joined launch stores it,
must equal aih_ir_block's too. Cases: the encoder's last block and head
(10x18, 128 -> 512 -> 128, residual, head 128 -> 2), the stride-2 block before
it joined to a head instead, a 64-channel block (the narrow kernel's
smallest 16-lane K), odd sizes whose tiles overhang the output, a batch of
three, forced tiles and 1 / 2 / 4 / 8 wavefronts, head activations, the
block output stored or not, f16 and bf16. Outputs start as NaN.
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

# (n, ih, iw, cin, cexp, cout, s, residual, head cout, head act, tile, waves, store y)
CASES = [
    (64, 10, 18, 128, 512, 128, 1, True, 2, "none", (0, 0), 0, False),
    (2, 10, 18, 128, 512, 128, 1, True, 2, "none", (5, 6), 4, True),
    (2, 20, 36, 96, 384, 128, 2, False, 2, "relu", (5, 6), 2, False),
    (3, 13, 11, 64, 256, 64, 1, True, 4, "sigmoid", (4, 8), 8, True),
    (1, 7, 9, 64, 128, 64, 1, False, 1, "relu6", (3, 9), 1, False),
    (2, 9, 17, 96, 384, 128, 2, False, 3, "none", (0, 0), 0, True),
]


def _id(c):
    n, h, w, ci, ce, co, s, r, hc, act, tile, waves, st = c
    return (f"n{n}_{h}x{w}_{ci}-{ce}-{co}_s{s}{'_res' if r else ''}_h{hc}{act}_t{tile[0]}x{tile[1]}_w{waves}"
            f"{'_y' if st else ''}")


def _case(case, dt, seed):
    n, h, w, ci, ce, co, s, r, hc, act, tile, waves, st = case
    blk = conv.IrBlockSpec(ih=h, iw=w, cin=ci, cexp=ce, cout=co, s=s, pad=(1, 1, 1, 1), act_expand=G.ACT["relu"],
                           act_dw=G.ACT["relu"], act_project=G.ACT["none"], residual=r, dt=conv.DType(dt), n=n,
                           tile=tile, waves=waves, kernel=conv.IrKernel.SPLIT)
    oh, ow = blk.out_hw()
    head = conv.GemmPwSpec(m=oh * ow, kg=co // 4, ng=1, act=G.ACT[act], dt=conv.DType(dt), n=n)
    o = G.orc
    we = o.gauss_fill(seed + 1, 0.0, float(np.sqrt(2.0 / ci)), ce * ci)
    wd = o.gauss_fill(seed + 3, 0.0, float(np.sqrt(2.0 / 9)), ce * 9)
    wp = o.gauss_fill(seed + 5, 0.0, float(np.sqrt(2.0 / ce)), co * ce)
    wh = o.gauss_fill(seed + 7, 0.0, float(np.sqrt(2.0 / co)), hc * co)
    bufs = (G.dev(o.pack_weights_conv(we, ce, ci, 1, 1, 4, dt)[0]),
            G.dev(o.pack_bias(o.gauss_fill(seed + 2, 0.0, 0.01, ce), ce, dt)),
            G.dev(o.pack_weights_dw(wd, ce, 3, 3, dt)),
            G.dev(o.pack_bias(o.gauss_fill(seed + 4, 0.0, 0.01, ce), ce, dt)),
            G.dev(o.pack_weights_conv(wp, co, ce, 1, 1, 4, dt)[0]),
            G.dev(o.pack_bias(o.gauss_fill(seed + 6, 0.0, 0.01, co), co, dt)))
    hbufs = (G.dev(o.pack_weights_conv(wh, hc, co, 1, 1, 4, dt)[0]),
             G.dev(o.pack_bias(o.gauss_fill(seed + 8, 0.0, 0.1, hc), hc, dt)))
    x = G.dev(o.pack_nhwc(o.gauss_fill(seed + 50, 0.0, 1.0, n * h * w * ci), n, h, w, ci, dt))
    return blk, head, bufs, hbufs, x


@pytest.mark.parametrize("dt", [F16, BF16], ids=["f16", "bf16"])
@pytest.mark.parametrize("case", CASES, ids=_id)
def test_block_head_equals_block_then_head(case, dt):
    blk, head, bufs, (wh, bh), x = _case(case, dt, 9100 + 10 * CASES.index(case))
    store_y = case[-1]
    joined = conv.IrBlockHeadSpec(blk, head)
    jp, bp_ = joined.plan(), blk.plan()
    print(f"case {_id(case)} dt{dt}: joined {jp}, block {bp_}", flush=True)
    # the same tile and wavefronts on both sides
    assert (jp.th, jp.tw, jp.waves, jp.kernel) == (bp_.th, bp_.tw, bp_.waves, bp_.kernel), (jp, bp_)
    n, (oh, ow), co = blk.n, blk.out_hw(), blk.cout
    we, be, wd, bd, wp, bp = bufs
    res = x if blk.residual else None
    y_ref = G.poisoned(n * oh * ow * co, dt)
    blk.run(x, we, be, wd, bd, wp, bp, res, y_ref)
    h_ref = G.poisoned(n * oh * ow * 4, dt)
    assert head.plan().variant == int(conv.Variant.ROWS)
    head.run(y_ref, wh, bh, None, h_ref)
    y = G.poisoned(n * oh * ow * co, dt) if store_y else None
    h = G.poisoned(n * oh * ow * 4, dt)
    joined.run(x, we, be, wd, bd, wp, bp, res, y, wh, bh, h)
    torch.cuda.synchronize()
    assert not torch.isnan(h_ref.float()).any()
    assert torch.equal(h.view(-1), h_ref.view(-1))
    if store_y:
        assert torch.equal(y.view(-1), y_ref.view(-1))
    # a second launch into the same buffers: the same bits
    joined.run(x, we, be, wd, bd, wp, bp, res, y, wh, bh, h)
    torch.cuda.synchronize()
    assert torch.equal(h.view(-1), h_ref.view(-1))


def test_block_head_rejects_what_it_does_not_take():
    blk, head, *_ = _case(CASES[1], F16, 9900)
    import dataclasses
    bad = [
        (blk, dataclasses.replace(head, ng=2), "at most 4 outputs"),
        (blk, dataclasses.replace(head, kg=16), "kg = cout / 4"),
        (blk, dataclasses.replace(head, residual=True), "no residual"),
        (blk, dataclasses.replace(head, splitk=2), "narrow route"),
        (blk, dataclasses.replace(head, dt=conv.DType.BF16), "dt and wdt"),
        (dataclasses.replace(blk, kernel=conv.IrKernel.WAVE), head, "split kernel"),
        (dataclasses.replace(blk, cout=32, cin=32, cexp=128), dataclasses.replace(head, kg=8), "16 lanes"),
        (dataclasses.replace(blk, dt=conv.DType.F32), dataclasses.replace(head, dt=conv.DType.F32), "f16 or bf16"),
    ]
    for b, hd, why in bad:
        assert not conv.IrBlockHeadSpec(b, hd).fusable()
        assert why in conv.last_error(), (why, conv.last_error())

"""GPU parity of the fused depthwise -> pointwise launch (aih_conv_dwpw)
against the oracle's two ops run separately, as the reference dispatches
them (conv_dw, then the 1x1 conv: crates/ai-gpu-runtime/src/lowering.rs:
122-168): a depthwise 3x3 + act, then a 1x1 conv + act (+ residual), fp32
storage, max relative error <= 1e-4 (the reference's metric,
crates/ai-cpu/tests/synthetic_e2e.rs:113-116). Cases cover both strides,
channel counts with a partial last 16-channel chunk, every output block
count, widths and heights that leave partial tiles, asymmetric padding,
batches, every forced tile shape and the non-clamp activations. 16-bit
storage (f16, bf16): the same cases against the oracle's two ops with the
same storage rounding (inputs, weights, the depthwise output and the result
rounded to the dtype, fp32 arithmetic) within 2e-3 f16 / 8e-3 bf16."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():
    pytest.skip("no GPU", allow_module_level=True)

from ai_engine_amd import conv  # noqa: E402
from oracle import oracle as orc  # noqa: E402
from tests.gpu_util import ACT, dev, host, poisoned, rel_err  # noqa: E402

TOL = 1e-4


class DwPwCase:
    """Seeded depthwise + pointwise pair: the oracle's separate ops on the
    host and the packed device buffers in the unfused ops' layouts."""

    def __init__(self, n, ih, iw, c, cout, s, pad, residual, act_d, act_p, seed, dt=0):
        self.n, self.ih, self.iw, self.c, self.cout, self.s, self.dt = n, ih, iw, c, cout, s, dt
        self.pad, self.residual, self.act_d, self.act_p = tuple(pad), residual, act_d, act_p
        op_d = orc.conv2d(c, c, k=3, s=s, pad=list(pad), groups=c, act=act_d)
        op_p = orc.conv2d(c, cout, act=act_p)
        self.oh, self.ow = orc.out_hw(op_d, ih, iw)
        x = orc.xs32_fill(seed, n * ih * iw * c)
        wd = orc.gauss_fill(seed + 1, 0.0, float(np.sqrt(2.0 / 9)), c * 9)
        bd = orc.gauss_fill(seed + 2, 0.0, 0.01, c)
        wp = orc.gauss_fill(seed + 3, 0.0, float(np.sqrt(2.0 / c)), cout * c)
        bp = orc.gauss_fill(seed + 4, 0.0, 0.01, cout)
        r = orc.xs32_fill(seed + 5, n * self.oh * self.ow * cout) if residual else None
        # 16-bit: the oracle on the stored values, its depthwise output and
        # result rounded where the unfused ops store them
        rd = (lambda v: v) if dt == 0 else (lambda v: orc.round_to(v, dt))
        d = rd(orc.CpuConv(op_d, ih, iw, rd(wd), rd(bd)).run(rd(x), n, threads=8))
        self.want = rd(orc.CpuConv(op_p, self.oh, self.ow, rd(wp), rd(bp), has_res=residual).run(
            d, n, rd(r) if residual else None, threads=8))
        wpp, self.kgp = orc.pack_weights_conv(wp, cout, c, 1, 1, 4, dt)
        self.bufs = (dev(orc.pack_nhwc(x, n, ih, iw, c, dt)), dev(orc.pack_weights_dw(wd, c, 3, 3, dt)),
                     dev(orc.pack_bias(bd, c, dt)), dev(wpp), dev(orc.pack_bias(bp, cout, dt)),
                     dev(orc.pack_nhwc(r, n, self.oh, self.ow, cout, dt)) if residual else None)

    def spec(self, **kw):
        return conv.DwPwSpec(ih=self.ih, iw=self.iw, c=self.c, cout=self.cout, s=self.s, pad=self.pad,
                             act_dw=ACT[self.act_d], act_pw=ACT[self.act_p], residual=self.residual, n=self.n,
                             kg_pad=self.kgp, dt=conv.DType(self.dt), **kw)

    def run(self, spec) -> np.ndarray:
        yd = poisoned(self.n * self.oh * self.ow * (-(-self.cout // 4)) * 4, self.dt)
        spec.run(*self.bufs, yd)
        torch.cuda.synchronize()
        return orc.unpack_nhwc(host(yd, self.dt), self.n, self.oh, self.ow, self.cout, self.dt)


CASES = [
    # (n, ih, iw, c, cout, s, pad, residual, act_d, act_p)
    (2, 40, 72, 256, 64, 1, (1, 1, 1, 1), True, "relu", "none"),      # the fp32 inverted-residual chain's pair
    (1, 80, 144, 44, 24, 1, (1, 1, 1, 1), False, "relu", "relu"),     # the segmentation model's 44 -> 24 head pair
    (2, 20, 36, 96, 48, 2, (1, 1, 1, 1), False, "relu", "none"),      # stride 2
    (1, 21, 37, 96, 48, 2, (0, 0, 1, 1), False, "relu6", "none"),     # stride 2, odd size, bottom/right padding
    (3, 10, 18, 48, 48, 1, (1, 1, 1, 1), True, "none", "relu"),       # the model's 48 -> 48 pair
    (1, 7, 5, 20, 12, 1, (1, 1, 1, 1), False, "relu", "relu6"),       # tiny: one partial tile, 5 channel groups
    (1, 9, 33, 36, 4, 1, (1, 1, 1, 1), True, "relu6", "none"),        # one output block, partial chunk of 4
    (1, 16, 16, 16, 64, 2, (1, 1, 1, 1), False, "none", "none"),      # one chunk, four output blocks
    (2, 13, 29, 64, 40, 1, (0, 1, 2, 1), True, "relu", "relu"),       # asymmetric padding
    (1, 12, 20, 32, 2, 1, (1, 1, 1, 1), False, "relu", "none"),       # two outputs (c4 padding)
    (2, 17, 23, 42, 20, 1, (1, 1, 1, 1), True, "relu6", "relu"),      # channels no multiple of 4 (c4 padding)
    (1, 18, 26, 42, 36, 2, (1, 1, 1, 1), False, "relu", "none"),      # the same at stride 2
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "x".join(str(v) for v in c[:6]) + f"_{c[8]}_{c[9]}")
def test_dwpw_matches_two_ops(case):
    n, ih, iw, c, cout, s, pad, res, act_d, act_p = case
    cs = DwPwCase(n, ih, iw, c, cout, s, pad, res, act_d, act_p, seed=100 + c + cout)
    got = cs.run(cs.spec())
    err = rel_err(got, cs.want)
    assert err <= TOL, (cs.spec().plan(), err)


# (tile, output rows per wavefront): every shape the planner can choose
TILES = [((4, 16), 4), ((4, 32), 4), ((8, 16), 4), ((4, 64), 4), ((8, 32), 4), ((16, 16), 4),
         ((4, 16), 2), ((4, 32), 2), ((8, 16), 2), ((4, 64), 2), ((8, 32), 2), ((16, 16), 2)]


@pytest.mark.parametrize("tile", TILES, ids=lambda t: f"{t[0][0]}x{t[0][1]}r{t[1]}")
@pytest.mark.parametrize("s", [1, 2])
def test_dwpw_every_tile(tile, s):
    """Every tile shape the planner can choose, forced, on one case per stride."""
    (th, tw), rows = tile
    cs = DwPwCase(2, 19, 43, 52, 36, s, (1, 1, 1, 1), True, "relu", "relu6", seed=7 + s)
    spec = cs.spec(tile=(th, tw), rows=rows)
    if not spec.fusable():
        pytest.skip(f"tile {th}x{tw} r{rows} does not fit at stride {s}: {conv.last_error()}")
    p = spec.plan()
    assert (p.th, p.tw, p.wave_rows, p.waves) == (th, tw, rows, th // rows * (tw // 16))
    err = rel_err(cs.run(spec), cs.want)
    assert err <= TOL, (p, err)


@pytest.mark.parametrize("act_p", ["hardswish", "sigmoid", "tanh", "hardsigmoid"])
def test_dwpw_activations(act_p):
    cs = DwPwCase(1, 11, 23, 40, 20, 1, (1, 1, 1, 1), False, "relu6", act_p, seed=31)
    err = rel_err(cs.run(cs.spec()), cs.want)
    assert err <= TOL, err


def test_dwpw_repeat_is_bit_identical():
    """Deterministic: two launches give the same bits (fixed chunk order,
    no atomics)."""
    cs = DwPwCase(2, 40, 72, 256, 64, 1, (1, 1, 1, 1), True, "relu", "none", seed=5)
    a = cs.run(cs.spec())
    b = cs.run(cs.spec())
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("case", [(40, 72, 256, 64, True, "relu", "none"), (80, 144, 44, 24, False, "relu", "relu")],
                         ids=["ir_chain_256to64_40x72", "segm_head_44to24_80x144"])
def test_dwpw_benched_routes_b64(case):
    """The two pairs the bench times at batch 64 (the fp32 inverted-residual
    chain's depthwise + projection, the real model's 44 -> 24 head pair),
    launched over the whole batch with the planner's tile -- 8x16 tiles of
    2-row wavefronts, the tuner's choice there -- and checked on sampled
    images against the oracle's two ops (1e-4)."""
    ih, iw, c, cout, res, act_d, act_p = case
    n = 64
    op_d = orc.conv2d(c, c, k=3, s=1, pad=[1, 1, 1, 1], groups=c, act=act_d)
    op_p = orc.conv2d(c, cout, act=act_p)
    oh, ow = orc.out_hw(op_d, ih, iw)
    x = orc.xs32_fill(900 + c, n * ih * iw * c)
    wd = orc.gauss_fill(901, 0.0, float(np.sqrt(2.0 / 9)), c * 9)
    bd = orc.gauss_fill(902, 0.0, 0.01, c)
    wp = orc.gauss_fill(903, 0.0, float(np.sqrt(2.0 / c)), cout * c)
    bp = orc.gauss_fill(904, 0.0, 0.01, cout)
    r = orc.xs32_fill(905, n * oh * ow * cout) if res else None
    wpp, kgp = orc.pack_weights_conv(wp, cout, c, 1, 1, 4, 0)
    spec = conv.DwPwSpec(ih=ih, iw=iw, c=c, cout=cout, act_dw=ACT[act_d], act_pw=ACT[act_p], residual=res, n=n,
                         kg_pad=kgp)
    p = spec.plan()
    assert (p.th, p.tw, p.wave_rows) == (8, 16, 2), p
    y = poisoned(n * oh * ow * (-(-cout // 4)) * 4, 0)
    spec.run(dev(orc.pack_nhwc(x, n, ih, iw, c, 0)), dev(orc.pack_weights_dw(wd, c, 3, 3, 0)),
             dev(orc.pack_bias(bd, c, 0)), dev(wpp), dev(orc.pack_bias(bp, cout, 0)),
             dev(orc.pack_nhwc(r, n, oh, ow, cout, 0)) if res else None, y)
    torch.cuda.synchronize()
    got = orc.unpack_nhwc(host(y, 0), n, oh, ow, cout, 0).reshape(n, -1)
    img_in, img_out = ih * iw * c, oh * ow * cout
    worst = 0.0
    for i in (0, 21, 42, 63):
        d = orc.CpuConv(op_d, ih, iw, wd, bd).run(x[i * img_in:(i + 1) * img_in], 1, threads=8)
        ri = r[i * img_out:(i + 1) * img_out] if res else None
        want = orc.CpuConv(op_p, oh, ow, wp, bp, has_res=res).run(d, 1, ri, threads=8)
        worst = max(worst, rel_err(got[i], want.reshape(-1)))
    assert worst <= TOL, (p, worst)


@pytest.mark.parametrize("dt", [1, 2], ids=["f16", "bf16"])
@pytest.mark.parametrize("case", CASES, ids=lambda c: "x".join(str(v) for v in c[:6]) + f"_{c[8]}_{c[9]}")
def test_dwpw_16bit_matches_two_ops_with_storage_rounding(case, dt):
    n, ih, iw, c, cout, s, pad, res, act_d, act_p = case
    cs = DwPwCase(n, ih, iw, c, cout, s, pad, res, act_d, act_p, 7700 + c + cout, dt=dt)
    spec = cs.spec()
    if not spec.fusable():
        pytest.skip(f"not fusable: {conv.last_error()}")
    got = cs.run(spec)
    err = rel_err(got, cs.want)
    print(f"dwpw dt{dt} {case}: plan {spec.plan()}, max_rel_err {err:.3e}", flush=True)
    assert err <= (2e-3 if dt == 1 else 8e-3), err

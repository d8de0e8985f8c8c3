"""GPU parity of the fused inverted-residual block (aih_ir_block) against the
oracle: the same three convs the reference runs separately (1x1 expand,
depthwise 3x3, 1x1 project + residual; crates/ai-gpu-runtime/src/lowering.rs:122-152)
restated by the oracle's ai-cpu path, on the same seeded inputs.

Expected values: the oracle chain on the tensors as the GPU stores them --
input, weights and biases rounded to the storage dtype, the expanded and the
depthwise tensors rounded to it after their convs (exactly where the unfused
path stores them). Against that chain the fused kernel differs only by
accumulation order: fp32 <= 1e-4, f16 <= 2e-3, bf16 <= 8e-3
(max |g - c| / max(|c|, 1)). fp32 is also held to 1e-4 against the plain
fp32 chain; f16 to 2e-2 against it (He-init weights).

Shapes cover both strides, residual on/off, odd sizes (tiles overhanging the
image), images smaller than a tile, one- and multi-chunk expansions, every
projection width (32..128) and asymmetric padding. Outputs start as NaN.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():  # pragma: no cover
    pytest.skip("no GPU", allow_module_level=True)

from ai_engine_amd import conv  # noqa: E402
from oracle import oracle as orc  # noqa: E402
from tests import gpu_util as G  # noqa: E402

F32, F16, BF16 = 0, 1, 2
BAR_STORED = {F32: 1e-4, F16: 2e-3, BF16: 8e-3}

# (n, ih, iw, cin, cexp, cout, s, pad, residual, activations): "e" alone is the
# expand's activation with a ReLU depthwise and a linear projection; "e/d/p"
# names all three
CASES = [
    (2, 12, 20, 32, 128, 32, 1, (1, 1, 1, 1), True, "relu"),
    (2, 13, 21, 32, 128, 64, 2, (1, 1, 1, 1), False, "relu"),
    (1, 10, 18, 64, 256, 64, 1, (1, 1, 1, 1), True, "relu6"),
    (2, 9, 17, 64, 256, 96, 2, (1, 1, 1, 1), False, "relu"),
    (1, 5, 9, 96, 384, 96, 1, (1, 1, 1, 1), True, "hardswish"),
    (1, 10, 18, 128, 512, 128, 1, (1, 1, 1, 1), True, "relu"),
    (3, 7, 33, 16, 32, 32, 1, (1, 1, 1, 1), True, "relu"),
    (1, 16, 16, 32, 64, 32, 2, (0, 0, 1, 1), False, "relu"),
    (1, 40, 72, 64, 256, 64, 1, (1, 1, 1, 1), True, "relu"),
    # "expand/dw/project" activations: every one clamp-type (the branch-free
    # instantiation) with the identity and ReLU6 in it, and a sigmoid expand
    # (act(0) != 0: the border mask, generic activations)
    (2, 11, 19, 32, 128, 32, 1, (1, 1, 1, 1), True, "none/relu6/relu"),
    (2, 12, 20, 32, 128, 64, 2, (1, 1, 1, 1), False, "sigmoid/relu6/none"),
]


def _id(c):
    n, ih, iw, cin, cexp, cout, s, pad, res, act = c
    return f"n{n}_{ih}x{iw}_{cin}-{cexp}-{cout}_s{s}_p{''.join(map(str, pad))}{'_res' if res else ''}_{act.replace('/', '-')}"


def run_case(case, dt, seed):
    n, ih, iw, cin, cexp, cout, s, pad, residual, acts = case
    parts = acts.split("/")
    act_e, act_d, act_p = parts if len(parts) == 3 else (parts[0], "relu", "none")
    op_e = orc.conv2d(cin, cexp, act=act_e)
    op_d = orc.conv2d(cexp, cexp, k=3, s=s, pad=list(pad), groups=cexp, act=act_d)
    op_p = orc.conv2d(cexp, cout, act=act_p)
    oh, ow = orc.out_hw(op_d, ih, iw)
    x = orc.xs32_fill(seed, n * ih * iw * cin)
    we = orc.gauss_fill(seed + 1, 0.0, float(np.sqrt(2.0 / cin)), cexp * cin)
    be = orc.gauss_fill(seed + 2, 0.0, 0.01, cexp)
    wd = orc.gauss_fill(seed + 3, 0.0, float(np.sqrt(2.0 / 9)), cexp * 9)
    bd = orc.gauss_fill(seed + 4, 0.0, 0.01, cexp)
    wp = orc.gauss_fill(seed + 5, 0.0, float(np.sqrt(2.0 / cexp)), cout * cexp)
    bp = orc.gauss_fill(seed + 6, 0.0, 0.01, cout)
    r = orc.xs32_fill(seed + 7, n * oh * ow * cout) if residual else None

    def chain(rd):
        e = rd(orc.CpuConv(op_e, ih, iw, rd(we), rd(be)).run(rd(x), n, threads=8))
        d = rd(orc.CpuConv(op_d, ih, iw, rd(wd), rd(bd)).run(e, n, threads=8))
        y = orc.CpuConv(op_p, oh, ow, rd(wp), rd(bp), has_res=residual).run(
            d, n, rd(r) if residual else None, threads=8)
        return rd(y)

    want = chain(lambda v: v)
    want_stored = chain(lambda v: orc.round_to(v, dt))

    yd = G.poisoned(n * oh * ow * cout, dt)
    spec = conv.IrBlockSpec(ih=ih, iw=iw, cin=cin, cexp=cexp, cout=cout, s=s, pad=pad,
                            act_expand=G.ACT[act_e], act_dw=G.ACT[act_d],
                            act_project=G.ACT[act_p], residual=residual, dt=conv.DType(dt), n=n)
    plan = spec.plan()
    print(f"case {_id(case)} dt{dt}: {plan}", flush=True)
    wep, _ = orc.pack_weights_conv(we, cexp, cin, 1, 1, 4, dt)
    wpp, _ = orc.pack_weights_conv(wp, cout, cexp, 1, 1, 4, dt)
    spec.run(G.dev(orc.pack_nhwc(x, n, ih, iw, cin, dt)), G.dev(wep), G.dev(orc.pack_bias(be, cexp, dt)),
             G.dev(orc.pack_weights_dw(wd, cexp, 3, 3, dt)), G.dev(orc.pack_bias(bd, cexp, dt)), G.dev(wpp),
             G.dev(orc.pack_bias(bp, cout, dt)),
             G.dev(orc.pack_nhwc(r, n, oh, ow, cout, dt)) if residual else None, yd)
    torch.cuda.synchronize()
    got = orc.unpack_nhwc(G.host(yd, dt), n, oh, ow, cout, dt)
    return got, want, want_stored


@pytest.mark.parametrize("case", CASES, ids=_id)
@pytest.mark.parametrize("dt", [F32, F16, BF16], ids=["f32", "f16", "bf16"])
def test_ir_block_matches_oracle_chain(case, dt):
    got, want, want_stored = run_case(case, dt, 7000 + 10 * CASES.index(case))
    e_stored = G.rel_err(got, want_stored)
    e = G.rel_err(got, want)
    print(f"  max_rel_err vs stored-dtype chain {e_stored:.3e}, vs fp32 chain {e:.3e}", flush=True)
    assert e_stored <= BAR_STORED[dt], e_stored
    if dt == F32:
        assert e <= 1e-4, e
    elif dt == F16:
        assert e <= 2e-2, e

"""Every activation of the table (crates/ai-core/src/activation.rs:7-43) in
every epilogue that applies one, on the GPU.

The conv arithmetic itself is checked against the oracle by the parity grid;
here the activation is isolated. Each route runs twice on the same seeded
inputs: with no activation, giving the pre-activation z as the kernel stores
it, and with activation f. The second output must equal the oracle's
Activation::apply of z, rounded to the storage dtype:

  fp32:  max |y - f(z)| / max(|f(z)|, 1) <= 1e-5 (the GPU's exp / reciprocal /
         square root against the C library's; the conv bar is 1e-4);
  16-bit: y = round(f(a)) against round(f(round(a))): two roundings apart,
         <= 4 u (u = 2^-11 f16, 2^-8 bf16) relative, plus f's own sensitivity
         to the rounding of a, which the chosen inputs keep small.

Equal infinities and NaN in the same place count as equal (recip of an exact
zero is inf on both sides). The routes are the kernels a conv can land on:
pointwise one-pixel-per-thread (<= 4 outputs), register-operand direct (32-
pixel blocks, and 16x16 blocks for small M),
LDS-weight direct (one tap, large M), tiled GEMM, split-K in one dispatch and
in two (the epilogue runs in the reduction), implicit-GEMM direct, tiled and
split-K, the stem, the depthwise
kernel, and the fused inverted-residual block (its projection epilogue the
same way; its expand and depthwise activations against the oracle's
three-op chain with stored-dtype rounding).
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
ACTS = list(orc.ACT)  # all eleven, in the reference's order
TOL = {F32: 1e-5, F16: 4 * 2.0 ** -11, BF16: 4 * 2.0 ** -8}
V = conv.Variant


def act_err(got, ref) -> float:
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape
    same = (got == ref) | (np.isnan(got) & np.isnan(ref))
    with np.errstate(invalid="ignore", over="ignore"):
        e = np.abs(got - ref) / np.maximum(np.abs(ref), 1.0)
    e = np.where(same, 0.0, e)
    if np.isnan(e).any():
        return float("inf")
    return float(e.max(initial=0.0))


# route -> (runner(act, dt, seed) -> Result, expected plan variant or None)
ROUTES = {
    "pw_rows": (lambda a, dt, s: G.run_pw(16, 16, 24, 2, a, False, dt, s, refs=False), V.ROWS),
    "pw_direct_16x16": (lambda a, dt, s: G.run_pw(16, 16, 32, 16, a, False, dt, s, refs=False), V.DIRECT),
    "pw_direct_32px": (lambda a, dt, s: G.run_pw(128, 256, 32, 16, a, False, dt, s, refs=False), V.DIRECT),
    "pw_lds_direct": (lambda a, dt, s: G.run_pw(256, 256, 64 if dt == F32 else 128, 32, a, False, dt, s,
                                                refs=False), V.DIRECT),
    "pw_tiled": (lambda a, dt, s: G.run_pw(9, 16, 64, 96, a, False, dt, s, variant=1, refs=False), V.TILE),
    "pw_splitk_one_dispatch": (lambda a, dt, s: G.run_pw(9, 16, 256, 64, a, False, dt, s, splitk=4, refs=False),
                               V.SPLITK),
    "pw_splitk_two_launch": (lambda a, dt, s: G.run_pw(9, 16, 256, 64, a, False, dt, s, variant=2, splitk=4,
                                                       refs=False), V.SPLITK),
    "igemm_direct": (lambda a, dt, s: G.run_igemm(12, 20, 16, 32, 3, 1, (1, 1, 1, 1), a, False, dt, s,
                                                  refs=False), V.DIRECT),
    "igemm_tiled": (lambda a, dt, s: G.run_igemm(12, 20, 16, 96, 3, 1, (1, 1, 1, 1), a, False, dt, s,
                                                 variant=1, refs=False), V.TILE),
    "igemm_splitk": (lambda a, dt, s: G.run_igemm(12, 20, 16, 96, 3, 1, (1, 1, 1, 1), a, False, dt, s,
                                                  splitk=3, refs=False), V.SPLITK),
    "igemm_stem": (lambda a, dt, s: G.run_igemm(12, 20, 3, 32, 3, 2, (1, 1, 1, 1), a, False, dt, s,
                                                refs=False), V.DIRECT),
    "dw": (lambda a, dt, s: G.run_dw(12, 20, 32, 3, 1, a, False, dt, s, refs=False), None),
}


@pytest.mark.parametrize("route", list(ROUTES))
@pytest.mark.parametrize("dt", [F32, F16, BF16], ids=["f32", "f16", "bf16"])
def test_epilogue_activation(route, dt):
    run, variant = ROUTES[route]
    seed = 4100 + 10 * list(ROUTES).index(route)
    z = run("none", dt, seed)
    if variant is not None:
        assert z.plan.variant == variant, (route, z.plan)
    worst = {}
    for act in ACTS:
        y = run(act, dt, seed)
        if variant is not None:
            assert y.plan.variant == variant, (route, act, y.plan)
        ref = orc.round_to(orc.act_array(act, z.got), dt)
        worst[act] = act_err(y.got, ref)
    print(f"{route} dt{dt}: " + ", ".join(f"{a} {e:.1e}" for a, e in worst.items()), flush=True)
    bad = {a: e for a, e in worst.items() if e > TOL[dt]}
    assert not bad, bad


# ---------------------------------------------------------------- the fused block

@pytest.mark.parametrize("dt", [F32, F16, BF16], ids=["f32", "f16", "bf16"])
def test_fused_block_projection_activation(dt):
    """Projection epilogue: y(act_p = f) against f(y(act_p = none)), both on
    the tile kernel (the one that takes every activation; the plan would put
    the clamp-type ones on the split kernel, whose partial sums add in
    another order)."""
    tile = conv.IrKernel.TILE
    z = G.IrCase(2, 12, 20, 32, 128, 64, 1, (1, 1, 1, 1), False, ("relu", "relu", "none"), dt, seed=4300)
    zg = z.run(z.spec(kernel=tile))
    worst = {}
    for act in ACTS:
        c = G.IrCase(2, 12, 20, 32, 128, 64, 1, (1, 1, 1, 1), False, ("relu", "relu", act), dt, seed=4300)
        worst[act] = act_err(c.run(c.spec(kernel=tile)), orc.round_to(orc.act_array(act, zg), dt))
    print(f"fused projection dt{dt}: " + ", ".join(f"{a} {e:.1e}" for a, e in worst.items()), flush=True)
    bad = {a: e for a, e in worst.items() if e > TOL[dt]}
    assert not bad, bad


# expand / depthwise activations whose outputs stay well conditioned through
# the following convs (recip of a near-zero expanded value would not be)
INNER_ACTS = [a for a in ACTS if a != "recip"]
BAR_STORED = {F32: 1e-4, F16: 2e-3, BF16: 8e-3}


@pytest.mark.parametrize("stage", ["expand", "dw"])
@pytest.mark.parametrize("dt", [F32, F16, BF16], ids=["f32", "f16", "bf16"])
def test_fused_block_inner_activations(stage, dt):
    """Expand and depthwise activations against the oracle's three-op chain
    (stored-dtype rounding), with the halo both inside and outside the image
    (act(0) != 0 for sigmoid / hardsigmoid exercises the border mask)."""
    worst = {}
    for i, act in enumerate(INNER_ACTS):
        acts = (act, "relu", "none") if stage == "expand" else ("relu", act, "none")
        c = G.IrCase(2, 11, 19, 32, 128, 32, 1, (1, 1, 1, 1), True, acts, dt, seed=4400 + 10 * i)
        worst[act] = G.rel_err(c.run(c.spec()), c.want_stored)
    print(f"fused {stage} dt{dt}: " + ", ".join(f"{a} {e:.1e}" for a, e in worst.items()), flush=True)
    bad = {a: e for a, e in worst.items() if e > BAR_STORED[dt]}
    assert not bad, bad

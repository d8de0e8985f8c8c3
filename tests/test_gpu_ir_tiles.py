"""Every fused launch the load-time tuner can choose, checked: for each of the
ten inverted-residual blocks of the 160x288 encoder (the headline workload's
shapes, two images) and the 48 -> 96 -> 48 block of the converter's
segmentation model, every candidate the tuner times -- the planner's tile
and every forced tile, each with its weights resident in LDS and streamed
(Model.fused_candidates) -- runs through the C ABI and is compared with the
oracle's three-op chain (the convs the reference dispatches separately,
crates/ai-gpu-runtime/src/lowering.rs:122-152) on the same seeded inputs.

Bars (max |g - c| / max(|c|, 1)): against the chain with every stored tensor
rounded to the dtype where the unfused path stores it, fp32 1e-4, f16 2e-3,
bf16 8e-3 (the kernel's own error: accumulation order only); fp32 also 1e-4
against the plain fp32 chain. Whatever tile a tuned load picks, its kernel is
one of these launches.
"""
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():  # pragma: no cover
    pytest.skip("no GPU", allow_module_level=True)

from ai_engine_amd import workloads as W  # noqa: E402
from ai_engine_amd.model import Model  # noqa: E402
from tests import gpu_util as G  # noqa: E402

F32, F16, BF16 = 0, 1, 2
BAR_STORED = {F32: 1e-4, F16: 2e-3, BF16: 8e-3}


def encoder_blocks():
    layers, _ = W.mnv4_small_encoder_160x288(2)
    out = []
    for i in range(1, len(layers) - 1, 3):
        e, d, p = layers[i:i + 3]
        out.append((e.name.split(".")[0], (e.ih, e.iw, e.cin, e.cout, p.cout, d.s, p.res is not None)))
    assert len(out) == 10
    # the four 48 -> 96 -> 48 blocks of the converter's segmentation model
    # (ops 12-23 of segm_r11_160x288.sw), which the native loader fuses
    out.append(("segm_ir48", (10, 18, 48, 96, 48, 1, True)))
    return out


BLOCKS = encoder_blocks()


@pytest.mark.parametrize("blk", BLOCKS, ids=[b[0] for b in BLOCKS])
@pytest.mark.parametrize("dt", [F32, F16, BF16], ids=["f32", "f16", "bf16"])
def test_every_tuner_candidate_matches_oracle(blk, dt):
    name, (ih, iw, cin, cexp, cout, s, res) = blk
    case = G.IrCase(2, ih, iw, cin, cexp, cout, s, (1, 1, 1, 1), res, ("relu", "relu", "none"), dt,
                    seed=9000 + 100 * BLOCKS.index(blk) + dt)
    cands = Model.fused_candidates(case.spec())
    assert cands, f"{name}: no fused candidate"
    labels = [c[0] for c in cands]
    assert len(set(labels)) == len(labels)
    worst = 0.0
    for label, sp in cands:
        got = case.run(sp)
        e_st = G.rel_err(got, case.want_stored)
        worst = max(worst, e_st)
        print(f"{name} dt{dt} {label}: vs stored-dtype chain {e_st:.3e}", flush=True)
        assert e_st <= BAR_STORED[dt], (label, e_st)
        if dt == F32:
            e = G.rel_err(got, case.want)
            assert e <= 1e-4, (label, e)
    print(f"{name} dt{dt}: {len(cands)} candidates, worst {worst:.3e}", flush=True)

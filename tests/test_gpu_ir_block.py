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
fp32 chain; f16 and bf16 to the ideal-storage error of the case (the stored
chain against the fp32 chain) plus the kernel's bar, and f16 to 2e-2, bf16 to
4e-2 outright (He-init weights; bf16's ideal storage alone is 0.9e-2 to
2.3e-2 on these cases).

Shapes cover both strides, residual on/off, odd sizes (tiles overhanging the
image), images smaller than a tile, one- and multi-chunk expansions, every
projection width (32..128, and 16, 48, 80: part of the last 32-channel MFMA
block unused) and asymmetric padding. Outputs start as NaN, so a store into a
padding channel, or a missing one, shows.
"""
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():  # pragma: no cover
    pytest.skip("no GPU", allow_module_level=True)

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
    # projection widths that are not whole 32-channel MFMA blocks: the
    # converter's segmentation model's 48 -> 96 -> 48 block (its shape and
    # activations), 16 and 80 channels
    (2, 10, 18, 48, 96, 48, 1, (1, 1, 1, 1), True, "relu/relu/none"),
    (1, 9, 17, 32, 64, 16, 2, (1, 1, 1, 1), False, "relu"),
    (2, 12, 20, 32, 128, 80, 1, (1, 1, 1, 1), True, "relu6"),
]


def _id(c):
    n, ih, iw, cin, cexp, cout, s, pad, res, act = c
    return f"n{n}_{ih}x{iw}_{cin}-{cexp}-{cout}_s{s}_p{''.join(map(str, pad))}{'_res' if res else ''}_{act.replace('/', '-')}"


def make_case(case, dt, seed):
    n, ih, iw, cin, cexp, cout, s, pad, residual, acts = case
    parts = acts.split("/")
    act3 = tuple(parts) if len(parts) == 3 else (parts[0], "relu", "none")
    return G.IrCase(n, ih, iw, cin, cexp, cout, s, pad, residual, act3, dt, seed)


@pytest.mark.parametrize("case", CASES, ids=_id)
@pytest.mark.parametrize("dt", [F32, F16, BF16], ids=["f32", "f16", "bf16"])
def test_ir_block_matches_oracle_chain(case, dt):
    c = make_case(case, dt, 7000 + 10 * CASES.index(case))
    spec = c.spec()
    print(f"case {_id(case)} dt{dt}: {spec.plan()}", flush=True)
    got = c.run(spec)
    e_stored = G.rel_err(got, c.want_stored)
    e = G.rel_err(got, c.want)
    e_ideal = G.rel_err(c.want_stored, c.want)
    print(f"  max_rel_err vs stored-dtype chain {e_stored:.3e}, vs fp32 chain {e:.3e} "
          f"(ideal {'fp32' if dt == F32 else 'storage'} {e_ideal:.3e})", flush=True)
    assert e_stored <= BAR_STORED[dt], e_stored
    if dt == F32:
        assert e <= 1e-4, e
        return
    # against the fp32 chain: storage rounding (what the stored-dtype chain
    # itself is off by) plus at most the kernel's own error
    assert e <= e_ideal + BAR_STORED[dt], (e, e_ideal)
    if dt == F16:
        assert e <= 2e-2, e
    else:
        # bf16's 8-bit mantissa: ideal storage alone is 0.9e-2 .. 2.3e-2 on these cases
        assert e <= 4e-2, e


@pytest.mark.parametrize("kernel", ["tile", "wave"])
@pytest.mark.parametrize("dt", [F32, F16, BF16], ids=["f32", "f16", "bf16"])
def test_ir_block_48_channel_projection_both_kernels(kernel, dt):
    """The 48 -> 96 -> 48 block (two 32-channel MFMA blocks, the second half
    zero-weighted and never stored) on each kernel that takes it, weights
    resident and streamed."""
    from ai_engine_amd import conv
    if kernel == "wave" and dt == F32:
        pytest.skip("the wave kernel takes 16-bit storage")
    c = G.IrCase(2, 10, 18, 48, 96, 48, 1, (1, 1, 1, 1), True, ("relu", "relu", "none"), dt, seed=7600 + dt)
    k = conv.IrKernel.TILE if kernel == "tile" else conv.IrKernel.WAVE
    for w in (conv.IrWeights.RESIDENT, conv.IrWeights.STREAMED):
        spec = c.spec(kernel=k, weights=w)
        p = spec.plan()
        assert p.kernel == k and p.resident == (w == conv.IrWeights.RESIDENT), p
        e = G.rel_err(c.run(spec), c.want_stored)
        print(f"{kernel} dt{dt} {w.name}: {p} vs stored-dtype chain {e:.3e}", flush=True)
        assert e <= BAR_STORED[dt], (w, e)


@pytest.mark.parametrize("case", CASES, ids=_id)
@pytest.mark.parametrize("dt", [F16, BF16], ids=["f16", "bf16"])
def test_ir_block_split_kernel_every_wave_count(case, dt):
    """The split kernel (a tile per workgroup, its chunks divided among 1, 2,
    4 or 8 wavefronts, partial projections added in wavefront order) on every
    case it takes, against the stored-dtype chain; two runs of one launch
    give the same bits (the order of the partial sums is fixed)."""
    from ai_engine_amd import conv
    c = make_case(case, dt, 7800 + 10 * CASES.index(case))
    ran = 0
    for waves in (1, 2, 4, 8):
        spec = c.spec(kernel=conv.IrKernel.SPLIT, waves=waves)
        if not spec.fusable():
            continue
        p = spec.plan()
        assert p.kernel == conv.IrKernel.SPLIT and p.waves == waves and p.grid == p.tiles, p
        got = c.run(spec)
        e = G.rel_err(got, c.want_stored)
        print(f"case {_id(case)} dt{dt} split w{waves}: {p} vs stored-dtype chain {e:.3e}", flush=True)
        assert e <= BAR_STORED[dt], (waves, e)
        assert (c.run(spec) == got).all()
        ran += 1
    if not ran:
        pytest.skip("not a split-kernel shape (activation, width or instantiation)")

"""The conv launches captured into a HIP graph and replayed, as bench.py times
the per-config kernels: every replay must write exactly what the eager launch
wrote (same kernels, same inputs, so bit for bit). Covered: the direct
pointwise kernel, the tiled pointwise GEMM with its split-K reduction (the
workspace comes from the caller, no memset node), the direct 3x3 kernel (two
input parts, dynamic LDS) and the tiled implicit GEMM. Between replays the
program runs its own eager work, refills the outputs with NaN and
synchronises, so a replay that skipped a node or read stale memory fails.
"""
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():  # pragma: no cover
    pytest.skip("no GPU", allow_module_level=True)

from ai_engine_amd import conv  # noqa: E402

DEV = torch.device("cuda:0")
A, V, D = conv.Activation, conv.Variant, conv.DType


def _rnd(gen, n, dt, scale=1.0):
    v = (torch.rand(n, generator=gen, device=DEV) * 2 - 1) * scale
    if dt == D.F32:
        return v
    return (v.half() if dt == D.F16 else v.bfloat16()).view(torch.int16)


def _nan(n, dt):
    if dt == D.F32:
        return torch.full((n,), float("nan"), device=DEV)
    return torch.full((n,), 0x7e00 if dt == D.F16 else 0x7fc0, dtype=torch.int16, device=DEV)


def _poison(y, dt):
    if dt == D.F32:
        y.fill_(float("nan"))
    else:
        y.fill_(0x7e00 if dt == D.F16 else 0x7fc0)


def _diff(y, ref, dt):
    """Where a replay's output differs from the eager one: how many elements,
    how many of them still hold the NaN poison (never written), the largest
    difference among the written ones and the first differing index."""
    f = y.float() if dt == D.F32 else (y.view(torch.float16) if dt == D.F16 else y.view(torch.bfloat16)).float()
    g = ref.float() if dt == D.F32 else (ref.view(torch.float16) if dt == D.F16 else ref.view(torch.bfloat16)).float()
    bad = (f != g) & ~(torch.isnan(f) & torch.isnan(g))
    nan = bad & torch.isnan(f)
    written = bad & ~torch.isnan(f)
    idx = torch.nonzero(bad)
    md = float((f[written] - g[written]).abs().max()) if written.any() else 0.0
    return (f"{int(bad.sum())} of {f.numel()} elements differ, {int(nan.sum())} unwritten (NaN), "
            f"max |diff| of the written {md:.3e}, first at {int(idx[0]) if len(idx) else -1}")


def _cases(gen):
    """(name, spec, launch(stream), output buffer, its dtype, expected plan variant)"""
    out = []
    # direct pointwise: 32 -> 64 at 80x144, fp32
    sp = conv.GemmPwSpec(m=80 * 144, kg=8, ng=16, act=A.RELU6)
    x, w, b = _rnd(gen, 80 * 144 * 32, D.F32), _rnd(gen, 32 * 64, D.F32, 0.1), _rnd(gen, 64, D.F32, 0.01)
    y = _nan(80 * 144 * 64, D.F32)
    out.append(("pw direct", sp, lambda st, sp=sp, x=x, w=w, b=b, y=y: sp.run(x, w, b, None, y, None, st), y, D.F32,
                V.DIRECT))
    # tiled pointwise with the split-K reduction: 960 -> 160 at 10x18, fp32
    sp = conv.GemmPwSpec(m=180, kg=240, ng=40)
    p = sp.plan()
    x, w, b = _rnd(gen, 180 * 960, D.F32), _rnd(gen, 960 * 160, D.F32, 0.05), _rnd(gen, 160, D.F32, 0.01)
    ws = torch.empty(max(p.ws_bytes // 4, 1), device=DEV)
    y = _nan(180 * 160, D.F32)
    out.append(("pw split-K", sp, lambda st, sp=sp, x=x, w=w, b=b, y=y, ws=ws: sp.run(x, w, b, None, y, ws, st), y,
                D.F32, V.SPLITK))
    # direct 3x3, two input parts (48 + 24 channels), f16, residual
    sp = conv.ConvIgemmSpec(ih=40, iw=72, cin=72, cout=32, k=3, pad=(1, 1, 1, 1), act=A.RELU, residual=True,
                            dt=D.F16, n=2, srcs=[conv.SrcView(c=48), conv.SrcView(c=24)])
    xs = [_rnd(gen, 2 * 40 * 72 * 48, D.F16), _rnd(gen, 2 * 40 * 72 * 24, D.F16)]
    # packed weights [tap][kg_pad][32 outputs][4]: 72 channels = 18 groups, padded to 20
    w, b = _rnd(gen, 9 * 20 * 32 * 4, D.F16, 0.1), _rnd(gen, 32, D.F16, 0.01)
    r = _rnd(gen, 2 * 40 * 72 * 32, D.F16)
    y = _nan(2 * 40 * 72 * 32, D.F16)
    out.append(("igemm direct", sp, lambda st, sp=sp, xs=xs, w=w, b=b, r=r, y=y: sp.run(xs, w, b, r, y, None, st), y,
                D.F16, V.DIRECT))
    # tiled implicit GEMM (forced), fp32, stride 2
    sp = conv.ConvIgemmSpec(ih=36, iw=64, cin=16, cout=32, k=3, s=2, pad=(1, 1, 1, 1), act=A.HARDSWISH, n=2,
                            variant=V.TILE)
    oh, ow = sp.out_hw()
    x, w, b = _rnd(gen, 2 * 36 * 64 * 16, D.F32), _rnd(gen, 9 * 16 * 32, D.F32, 0.1), _rnd(gen, 32, D.F32, 0.01)
    y = _nan(2 * oh * ow * 32, D.F32)
    out.append(("igemm tiled", sp, lambda st, sp=sp, x=x, w=w, b=b, y=y: sp.run([x], w, b, None, y, None, st), y,
                D.F32, V.TILE))
    return out


def test_graph_replays_match_eager():
    gen = torch.Generator(device=DEV)
    gen.manual_seed(4242)
    cases = _cases(gen)
    for name, spec, _, _, _, variant in cases:
        assert conv.Variant(spec.plan().variant) == variant, name
    side = torch.cuda.Stream()
    # eager reference (also the warm-up that sets the kernels' attributes)
    want = []
    for _, _, run, y, dt, _ in cases:
        run(side)
        side.synchronize()
        want.append(y.clone())
        _poison(y, dt)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        for _, _, run, _, _, _ in cases:
            run(side)
    torch.cuda.synchronize()
    scratch = torch.empty(1 << 20, device=DEV)
    for rep in range(3):
        # the program's own eager work between replays
        scratch.uniform_(-1, 1)
        scratch.mul_(2.0).add_(1.0)
        for _, _, _, y, dt, _ in cases:
            _poison(y, dt)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for (name, _, _, y, dt, _), ref in zip(cases, want):
            same = torch.equal(y, ref)
            print(f"replay {rep} {name}: {'bit-identical' if same else 'DIFFERS'}", flush=True)
            assert same, f"replay {rep}: {name} differs from the eager launch: {_diff(y, ref, dt)}"
            assert not torch.isnan(ref if ref.dtype == torch.float32 else ref.view(torch.float16)).any(), name

"""aih_conv_noalloc against aih_conv: the allocation-free entry point runs the
same kernels with its split-K workspace in the library's static device
scratch, so its outputs must equal aih_conv's (given a caller workspace) bit
for bit -- on two calls in a row, the second with a smaller input (the
scratch keeps the first call's partial sums; nothing may leak from them).
Also: a conv that needs no workspace, and a rejection (with the size in the
message) of one whose workspace exceeds the scratch.
"""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():  # pragma: no cover
    pytest.skip("no GPU", allow_module_level=True)

from ai_engine_amd import conv  # noqa: E402
from oracle import oracle as orc  # noqa: E402
from tests import gpu_util as G  # noqa: E402

SCRATCH = 16 << 20  # AIH_NOALLOC_SCRATCH_BYTES


def lib():
    return conv.lib()


def case(n, h, w, cin, cout, k, dt, seed, residual=False):
    op = conv.ConvOp(ih=h, iw=w, cin=cin, cout=cout, kh=k, kw=k, pad=((k - 1) // 2,) * 4,
                     act=conv.Activation.RELU, residual=residual, dt=conv.DType(dt), n=n)
    oh, ow = op.out_hw()
    x = orc.xs32_fill(seed, n * h * w * cin)
    wt = orc.gauss_fill(seed + 1, 0.0, float(np.sqrt(2.0 / (k * k * cin))), cout * cin * k * k)
    b = orc.gauss_fill(seed + 2, 0.0, 0.01, cout)
    r = orc.xs32_fill(seed + 3, n * oh * ow * cout) if residual else None
    wp, _ = orc.pack_weights_conv(wt, cout, cin, k, k, 4, dt)
    bufs = dict(x=G.dev(orc.pack_nhwc(x, n, h, w, cin, dt)), w=G.dev(wp), b=G.dev(orc.pack_bias(b, cout, dt)),
                r=G.dev(orc.pack_nhwc(r, n, oh, ow, cout, dt)) if residual else None)
    return op, bufs, n * oh * ow * (-(-cout // 4)) * 4


def run_both(op, bufs, nout, dt):
    L = lib()
    d = op.desc()
    ws_bytes = op.workspace_bytes()
    y_ref = G.poisoned(nout, dt)
    ws = torch.empty(max(ws_bytes // 4, 1), dtype=torch.float32, device=G.DEV)
    rp = bufs["r"].data_ptr() if bufs["r"] is not None else None
    assert L.aih_conv(C.byref(d), bufs["x"].data_ptr(), bufs["w"].data_ptr(), bufs["b"].data_ptr(), rp,
                      y_ref.data_ptr(), ws.data_ptr(), ws_bytes, None) == 0, conv.last_error()
    y = G.poisoned(nout, dt)
    assert L.aih_conv_noalloc(C.byref(d), bufs["x"].data_ptr(), bufs["w"].data_ptr(), bufs["b"].data_ptr(), rp,
                              y.data_ptr(), None) == 0, conv.last_error()
    torch.cuda.synchronize()
    return G.host(y_ref, dt), G.host(y, dt), ws_bytes


@pytest.mark.parametrize("dt", [0, 1, 2], ids=["f32", "f16", "bf16"])
def test_noalloc_equals_aih_conv_on_two_calls(dt):
    # 960 -> 100 1x1 (100 outputs: not whole 16-channel blocks, so the tiled
    # GEMM splits K through the workspace), at 10x18 batch 2, then a smaller
    # input, 9x16 batch 1, reusing the same scratch
    for n, h, w, seed in ((2, 10, 18, 8100), (1, 9, 16, 8200)):
        op, bufs, nout = case(n, h, w, 960, 100, 1, dt, seed)
        want, got, ws_bytes = run_both(op, bufs, nout, dt)
        print(f"n={n} dt{dt}: plan {op.plan()}, workspace {ws_bytes} bytes", flush=True)
        assert 0 < ws_bytes <= SCRATCH
        assert np.array_equal(want.view(np.uint8), got.view(np.uint8)), f"n={n}: outputs differ"


def test_noalloc_split_igemm_and_plain_conv():
    # a 3x3 conv the policy splits (small M, long K), then one with no workspace
    op, bufs, nout = case(1, 9, 16, 240, 96, 3, 0, 8300)
    want, got, ws_bytes = run_both(op, bufs, nout, 0)
    assert 0 < ws_bytes <= SCRATCH
    assert np.array_equal(want.view(np.uint8), got.view(np.uint8))
    op, bufs, nout = case(2, 20, 36, 32, 64, 1, 1, 8400, residual=True)
    want, got, ws_bytes = run_both(op, bufs, nout, 1)
    assert ws_bytes == 0
    assert np.array_equal(want.view(np.uint8), got.view(np.uint8))
    # the skinny layer at batch 1: K split on chip in one dispatch, no workspace
    op, bufs, nout = case(1, 10, 18, 960, 160, 1, 0, 8500)
    want, got, ws_bytes = run_both(op, bufs, nout, 0)
    assert ws_bytes == 0 and op.plan().bm == 16
    assert np.array_equal(want.view(np.uint8), got.view(np.uint8))


def test_noalloc_rejects_workspace_beyond_scratch():
    L = lib()
    # a 3x3 256 -> 160 fp32 conv at 10x18, batch 256: four K chunks on the
    # tiled implicit GEMM, 118 MB of partial sums
    op = conv.ConvOp(ih=10, iw=18, cin=256, cout=160, kh=3, kw=3, pad=(1, 1, 1, 1), n=256, dt=conv.DType.F32)
    need = op.workspace_bytes()
    assert need > SCRATCH, need
    d = op.desc()
    # real device buffers of the conv's own sizes: were the call accepted,
    # its kernels would read and write inside them (and aih_conv itself
    # rejects a workspace below the plan's), so a regression in the host-side
    # rejection fails the assertion below rather than touching a bad address
    x = torch.zeros(256 * 10 * 18 * 256, dtype=torch.float32, device=G.DEV)
    w = torch.zeros(9 * 256 * 160, dtype=torch.float32, device=G.DEV)
    b = torch.zeros(160, dtype=torch.float32, device=G.DEV)
    y = G.poisoned(256 * 10 * 18 * 160, 0)
    rc = L.aih_conv_noalloc(C.byref(d), x.data_ptr(), w.data_ptr(), b.data_ptr(), None, y.data_ptr(), None)
    torch.cuda.synchronize()
    assert rc == -1
    assert str(need) in conv.last_error() and "scratch" in conv.last_error()
    # nothing was written
    assert bool(torch.isnan(y).all())

"""GPU parity grid through the C ABI: the HIP kernels against the oracle.

Mirrors the reference's shared GPU testsuite (crates/ai-gpu/src/testsuite.rs):
the same (h, w, cin, cout) shapes, activations, seeds and XorShift32 stream
order for run_gemm_pw (:373-414), run_conv_dw (:466-496) and run_conv_igemm
(:722-786), with bf16 added next to every f16 case. Expected values come from
the oracle's restatement of reference::conv::conv2d on the unrounded fp32
inputs. Bars: the reference's compare (atol/rtol 1e-4 f32, 1e-2 f16,
testsuite.rs:21-24) and max |gpu-cpu|/max(|cpu|,1) <= 1e-4 for fp32.
16-bit storage is checked three ways: against the fp32 reference on the
inputs as stored (the kernel's own error: <= 2e-3 f16, <= 8e-3 bf16, a few
output roundings -- this is the check a wrong index or a lost term fails);
element-wise against the unrounded fp32 reference within the error that
storing the inputs can cause, |gpu - ref| <= 3.1 u sum|x||w| + 2 u |ref| with
u the dtype's unit roundoff (2^-11 f16, 2^-9 bf16); and, for f16, with the
reference's own 1e-2 compare. (bf16 has no reference counterpart; its 8-bit
mantissa puts the unrounded error of these U[-1,1]-weight shapes near 1e-1 at
K = 960, so the 2e-2 bar is applied to the He-init workloads of
test_gpu_workloads instead.) Every output buffer starts as NaN.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():  # pragma: no cover - the gpu marker keeps these off CPU runs
    pytest.skip("no GPU", allow_module_level=True)

from tests import gpu_util as G  # noqa: E402

F32, F16, BF16 = 0, 1, 2
# dt: (testsuite atol, rtol, bar vs fp32 on stored inputs, unit roundoff)
TOL = {F32: (1e-4, 1e-4, 1e-4, 0.0), F16: (1e-2, 1e-2, 2e-3, 2.0 ** -11), BF16: (None, None, 8e-3, 2.0 ** -9)}


def check(name, res, dt):
    atol, rtol, bar_r, u = TOL[dt]
    err = G.rel_err(res.got, res.want)
    err_r = G.rel_err(res.got, res.want_r) if res.want_r is not None else err
    print(f"{name}: max_rel_err={err:.3e} vs_stored_inputs={err_r:.3e}", flush=True)
    assert err_r <= bar_r, f"{name}: vs stored inputs {err_r}"
    if dt == F32:
        assert err <= 1e-4, f"{name}: {err}"
    else:
        bound = 3.1 * u * res.mag + 2 * u * np.abs(res.want) + 1e-6
        assert np.all(np.abs(res.got - res.want) <= bound), f"{name}: exceeds the storage-rounding bound"
    if atol is not None:
        assert G.testsuite_ok(res.got, res.want, atol, rtol), f"{name}: testsuite compare failed"


# ---------------------------------------------------------------- pointwise (testsuite.rs:373-414)

PW_SHAPES = [(1, 1, 64, 16), (9, 16, 128, 24), (3, 5, 6, 10), (72, 128, 16, 64), (24, 32, 6, 10),
             (23, 33, 8, 20), (9, 16, 960, 160), (9, 16, 240, 68), (11, 13, 72, 68)]
PW_ACTS = ["none", "relu", "hardswish", "sigmoid"]
PW_CASES = []
_seed = 2000
for _shape in PW_SHAPES:
    for _act in PW_ACTS:
        _seed += 1
        PW_CASES.append((_shape, _act, _seed))


@pytest.mark.parametrize("shape,act,seed", PW_CASES, ids=lambda v: str(v))
def test_pw_f32(shape, act, seed):
    h, w, cin, cout = shape
    res = G.run_pw(h, w, cin, cout, act, False, F32, seed)
    check(f"pw {shape} {act} {res.plan}", res, F32)


@pytest.mark.parametrize("case", [((9, 16, 32, 32), "relu", 3001), ((9, 16, 960, 160), "relu", 3003),
                                  ((72, 128, 16, 16), "hardswish", 3002)], ids=str)
def test_pw_residual_f32(case):
    (h, w, cin, cout), act, seed = case
    res = G.run_pw(h, w, cin, cout, act, True, F32, seed)
    check(f"pw res {case}", res, F32)


PW16 = [((72, 128, 16, 64), "relu", False, 3101), ((9, 16, 128, 24), "hardswish", False, 3102),
        ((24, 32, 16, 16), "relu", True, 3103), ((9, 16, 960, 160), "none", False, 3104),
        # N4 % 8 == 4: 16-bit output rows are 8-byte but not 16-byte aligned
        ((11, 13, 72, 68), "relu", True, 3105), ((7, 9, 20, 12), "none", True, 3106)]


@pytest.mark.parametrize("dt", [F16, BF16], ids=["f16", "bf16"])
@pytest.mark.parametrize("case", PW16, ids=str)
def test_pw_16bit(case, dt):
    (h, w, cin, cout), act, with_res, seed = case
    res = G.run_pw(h, w, cin, cout, act, with_res, dt, seed)
    check(f"pw dt{dt} {case}", res, dt)


@pytest.mark.parametrize("wdt", [F16, BF16], ids=["w_f16", "w_bf16"])
def test_pw_f32_act_16bit_weights(wdt):
    # dt_weights axis (format/model.rs:245-254): f32 activations, 16-bit weights
    res = G.run_pw(9, 16, 240, 68, "relu", True, F32, 3201, wdt=wdt)
    check(f"pw f32/w{wdt}", res, wdt)
    assert G.rel_err(res.got, res.want_r) <= 1e-4  # activations stay fp32: only the weights were rounded


# at most 4 output channels (the segmentation heads 24 -> 2 and 128 -> 2):
# the one-pixel-per-thread kernel
PW_NARROW = [((80, 144, 24, 2), "none", False, 3401), ((10, 18, 128, 2), "sigmoid", False, 3402),
             ((9, 16, 960, 4), "relu", True, 3403), ((5, 7, 6, 1), "hardswish", True, 3404),
             ((13, 11, 44, 3), "relu6", False, 3405)]


@pytest.mark.parametrize("dt", [F32, F16, BF16], ids=["f32", "f16", "bf16"])
@pytest.mark.parametrize("case", PW_NARROW, ids=str)
def test_pw_narrow_cout(case, dt):
    (h, w, cin, cout), act, with_res, seed = case
    res = G.run_pw(h, w, cin, cout, act, with_res, dt, seed, n=2)
    check(f"pw narrow dt{dt} {case}", res, dt)


def test_pw_narrow_f32_act_16bit_weights():
    res = G.run_pw(10, 18, 128, 2, "none", True, F32, 3410, wdt=F16)
    check("pw narrow f32/wf16", res, F16)
    assert G.rel_err(res.got, res.want_r) <= 1e-4


# short K (<= 128 16-bit / 64 fp32 channels) and at most 64 output channels:
# the direct kernel (operands from memory into MFMA registers); K, N and M
# ragged against its 16-channel steps, 32-channel blocks and 32-pixel blocks
PW_DIRECT = [((80, 144, 44, 24), "relu", False, 3501), ((13, 19, 32, 12), "none", True, 3502),
             ((10, 18, 96, 48), "relu6", True, 3503), ((9, 16, 128, 64), "hardswish", False, 3504),
             ((7, 11, 8, 8), "sigmoid", True, 3505), ((5, 9, 60, 36), "none", False, 3506)]


# beyond the register-operand kernel (K, or 65-256 outputs in column groups of
# 64), >= 2048 blocks of 32 pixels: the direct kernel run with one tap
# (weights in LDS); a ragged last block, steps padded up to the instantiation
# (25 -> 32, 13 -> 16), a half-empty last step at 16 bit, 4 and 3 column
# groups (the last one ragged: 136 = 2 x 64 + 8)
PW_LDS = [((257, 257, 256, 64), "relu", True, 3601), ((260, 256, 200, 20), "hardswish", False, 3602),
          ((256, 260, 96, 40), "relu6", True, 3603), ((257, 256, 64, 256), "relu", False, 3604),
          ((256, 257, 72, 136), "none", True, 3605)]


@pytest.mark.parametrize("dt", [F32, F16, BF16], ids=["f32", "f16", "bf16"])
@pytest.mark.parametrize("case", PW_LDS, ids=str)
def test_pw_lds_direct(case, dt):
    (h, w, cin, cout), act, res, seed = case
    r = G.run_pw(h, w, cin, cout, act, res, dt, seed)
    if cout <= 64 or dt == F32:  # more than 64 outputs at 16 bit: the tiled GEMM
        assert r.plan.variant == G.conv.Variant.DIRECT and r.plan.ws_bytes == 0, r.plan
    check(f"pw lds-direct {case} dt{dt} {r.plan}", r, dt)


@pytest.mark.parametrize("dt", [F32, F16, BF16], ids=["f32", "f16", "bf16"])
@pytest.mark.parametrize("case", PW_DIRECT, ids=str)
def test_pw_direct(case, dt):
    (h, w, cin, cout), act, with_res, seed = case
    if dt == F32 and cin > 64:
        cin = 64  # the fp32 direct route takes K <= 64
    res = G.run_pw(h, w, cin, cout, act, with_res, dt, seed, n=2)
    check(f"pw direct dt{dt} {case}", res, dt)


@pytest.mark.parametrize("dt", [F32, F16, BF16], ids=["f32", "f16", "bf16"])
def test_pw_direct_equals_tiled_gemm(dt):
    # the same short-K shapes with the tiled GEMM forced (AIH_VAR_TILE, one
    # tile over the whole K): the direct kernel's 32-pixel blocks run the same
    # MFMA K steps in the same order, so the outputs agree bit for bit (the
    # second shape at batch 16: enough 32-pixel blocks that the 16x16-block
    # launch for small M does not take it)
    for (h, w, cin, cout, res, n), seed in [((13, 19, 44, 24, True, 2), 3510), ((40, 72, 32, 64, False, 16), 3511)]:
        xs = G.stream(seed, n * h * w * cin, cout * cin, cout, n * h * w * cout if res else 0)
        a = G.run_pw(h, w, cin, cout, "relu", res, dt, seed, n=n, xs=xs)
        b = G.run_pw(h, w, cin, cout, "relu", res, dt, seed, n=n, xs=xs, variant=1)
        assert a.plan.variant == G.conv.Variant.DIRECT and a.plan.bm == 32 and b.plan.variant == G.conv.Variant.TILE
        check(f"pw tiled dt{dt}", b, dt)
        assert np.array_equal(np.asarray(a.got), np.asarray(b.got))


@pytest.mark.parametrize("splitk", [1, 4, 8])
@pytest.mark.parametrize("n", [1, 3])
def test_pw_splitk_factors(splitk, n):
    # the skinny 960 -> 160 layer at 10x18 with split-K forced to 1 / 4 / 8
    res = G.run_pw(10, 18, 960, 160, "none", False, F32, 3300 + splitk, n=n, splitk=splitk)
    assert res.plan.splitk == splitk
    check(f"pw splitk={splitk} n={n}", res, F32)


@pytest.mark.parametrize("splitk", [1, 4, 8])
def test_pw_splitk_factors_at_batch_256(splitk):
    """The skinny 960 -> 160 layer at 10x18, batch 256 (46080 pixels), with
    split-K forced to 1 / 4 / 8: the rows the bench times as
    pw_960to160_10x18_b256_splitk{1,4,8}. A forced factor takes the tiled GEMM
    (160-channel tiles) and, above 1, its fp32 partials and the reduction
    launch. Images of a batch never interact, so sampled images are checked
    against the oracle run of each image alone (fp32 bar 1e-4)."""
    n, h, w, cin, cout = 256, 10, 18, 960, 160
    xs = G.stream(3600 + splitk, n * h * w * cin, cout * cin, cout, 0)
    res = G.run_pw(h, w, cin, cout, "none", False, F32, 3600 + splitk, n=n, splitk=splitk, xs=xs, refs=False)
    assert res.plan.splitk == splitk and res.plan.bn == 160, res.plan
    x, wts, b, _ = xs
    op = G.orc.conv2d(cin, cout, act="none")
    got = np.asarray(res.got).reshape(n, -1)
    worst = 0.0
    for i in (0, 1, 97, 200, 255):
        want = G.orc.conv2d_ref(op, h, w, x.reshape(n, -1)[i], wts, b, None, n=1)
        worst = max(worst, G.rel_err(got[i], want))
    print(f"pw 960->160 b256 splitk={splitk} ({res.plan}): sampled images max_rel_err={worst:.3e}", flush=True)
    assert worst <= 1e-4


def test_pw_splitk_is_deterministic():
    a = G.run_pw(9, 16, 960, 160, "relu", True, F32, 3401, splitk=8).got
    b = G.run_pw(9, 16, 960, 160, "relu", True, F32, 3401, splitk=8).got
    assert np.array_equal(a, b)


def test_pw_tail_tiles():
    # M not a multiple of the 128-pixel tile, N4 not a multiple of any channel tile
    res = G.run_pw(7, 37, 44, 300, "relu6", True, F32, 3501)
    check("pw tails", res, F32)


# fp32, K >= 256 channels and enough 32-pixel x 32-channel wavefront units to
# fill every CU eight times over: the LDS-streamed GEMM (96-pixel tiles over
# the whole K, reported as TILE with bm = 96 and no workspace). The cases
# take a ragged last pixel tile, a K tail inside the last 16-channel stage,
# columns padded inside a 128-wide tile, two column tiles, and the 960 -> 160
# layer at batch 80.
PW_STREAM = [((1, 13250, 260, 160, 1), "relu6", True, 3601),
             ((1, 16400, 256, 100, 1), "hardswish", False, 3602),
             ((1, 16400, 272, 256, 1), "none", True, 3603),
             ((10, 18, 960, 160, 80), "none", False, 3604)]


@pytest.mark.parametrize("case", PW_STREAM, ids=str)
def test_pw_stream(case):
    (h, w, cin, cout, n), act, res, seed = case
    r = G.run_pw(h, w, cin, cout, act, res, F32, seed, n=n)
    assert r.plan.variant == G.conv.Variant.TILE and r.plan.bm == 96 and r.plan.ws_bytes == 0, r.plan
    check(f"pw stream {case} {r.plan}", r, F32)


def test_pw_stream_is_deterministic():
    xs = G.stream(3605, 80 * 180 * 960, 160 * 960, 160, 80 * 180 * 160)
    a = G.run_pw(10, 18, 960, 160, "relu", True, F32, 3605, n=80, xs=xs, refs=False)
    b = G.run_pw(10, 18, 960, 160, "relu", True, F32, 3605, n=80, xs=xs, refs=False)
    assert a.plan.bm == 96
    assert np.array_equal(np.asarray(a.got), np.asarray(b.got))


# ---------------------------------------------------------------- depthwise (testsuite.rs:466-496)

DW_SHAPES = [(72, 128, 64, 3, 1), (36, 64, 96, 5, 2), (33, 17, 6, 3, 2), (16, 16, 10, 5, 1)]
DW_CASES = []
_seed = 4000
for _shape in DW_SHAPES:
    for _act in ["none", "relu", "hardswish"]:
        _seed += 1
        DW_CASES.append((_shape, _act, _seed))


@pytest.mark.parametrize("shape,act,seed", DW_CASES, ids=lambda v: str(v))
def test_dw_f32(shape, act, seed):
    ih, iw, c, k, s = shape
    res = G.run_dw(ih, iw, c, k, s, act, False, F32, seed)
    check(f"dw {shape} {act}", res, F32)


def test_dw_residual_and_dilation():
    res = G.run_dw(36, 64, 32, 3, 1, "relu", True, F32, 5001)
    check("dw res", res, F32)
    res = G.run_dw(18, 32, 40, 3, 1, "relu", False, F32, 5201, pad=[2] * 4, d=2)
    check("dw d2", res, F32)


@pytest.mark.parametrize("dt", [F16, BF16], ids=["f16", "bf16"])
def test_dw_16bit(dt):
    res = G.run_dw(72, 128, 64, 3, 1, "relu", False, dt, 5101)
    check("dw16 a", res, dt)
    res = G.run_dw(36, 64, 96, 5, 2, "none", False, dt, 5102)
    check("dw16 b", res, dt)
    # the real segmentation model's small 5x5 layers (one-pixel strips of 4-channel vectors), a batch of 4
    res = G.run_dw(20, 36, 32, 5, 1, "none", True, dt, 5103, n=4)
    check("dw16 c", res, dt)
    res = G.run_dw(20, 36, 96, 5, 2, "relu", False, dt, 5104, n=4)
    check("dw16 d", res, dt)


def test_dw_batch():
    res = G.run_dw(20, 36, 64, 3, 2, "relu", True, F32, 5301, n=3)
    check("dw batch", res, F32)


# ---------------------------------------------------------------- implicit GEMM (testsuite.rs:722-786)

IG_SHAPES = [(36, 64, 3, 16, 3, 2), (24, 32, 16, 24, 3, 1), (40, 64, 20, 32, 3, 1), (17, 23, 6, 8, 3, 2),
             (33, 45, 8, 12, 5, 2), (9, 16, 128, 128, 3, 1), (18, 32, 171, 80, 3, 1)]
IG_CASES = []
_seed = 6000
for _shape in IG_SHAPES:
    for _act in ["none", "relu", "hardswish"]:
        _seed += 1
        IG_CASES.append((_shape, _act, _seed))


@pytest.mark.parametrize("shape,act,seed", IG_CASES, ids=lambda v: str(v))
def test_igemm_f32(shape, act, seed):
    ih, iw, cin, cout, k, s = shape
    p = (k - 1) // 2
    res = G.run_igemm(ih, iw, cin, cout, k, s, [p] * 4, act, False, F32, seed)
    check(f"igemm {shape} {act} {res.plan}", res, F32)


IG_EXTRA = [
    # (ih, iw, cin, cout, k, s, pad, act, residual, seed) -- testsuite.rs:745-770
    (16, 16, 4, 8, 3, 1, [1, 0, 0, 1], "relu", False, 7001),
    (128, 128, 3, 16, 3, 2, [0, 0, 1, 1], "none", False, 7008),
    (32, 32, 3, 16, 3, 2, [0, 0, 1, 1], "none", False, 7005),
    (32, 32, 3, 24, 5, 2, [1, 1, 2, 2], "none", False, 7006),
    (24, 24, 16, 16, 3, 2, [0, 0, 1, 1], "relu", False, 7007),
    (24, 32, 16, 16, 3, 1, [1, 1, 1, 1], "hardswish", True, 7002),
    (9, 16, 8, 8, 3, 1, [1, 1, 1, 1], "none", True, 7003),
    (9, 16, 128, 128, 3, 1, [1, 1, 1, 1], "relu", True, 7004),
]


@pytest.mark.parametrize("case", IG_EXTRA, ids=lambda c: str(c[-1]))
def test_igemm_pads_and_residual(case):
    ih, iw, cin, cout, k, s, pad, act, with_res, seed = case
    res = G.run_igemm(ih, iw, cin, cout, k, s, pad, act, with_res, F32, seed)
    check(f"igemm {case}", res, F32)


@pytest.mark.parametrize("case", [((24, 32), [16, 16], 24, "relu", False, 7101),
                                  ((36, 64), [80, 24, 3], 40, "hardswish", False, 7102),
                                  ((9, 16), [64, 64], 128, "relu", True, 7103)], ids=lambda c: str(c[-1]))
def test_igemm_concat_parts(case):
    (ih, iw), parts, cout, act, with_res, seed = case
    res = G.run_igemm(ih, iw, sum(parts), cout, 3, 1, [1] * 4, act, with_res, F32, seed, parts=parts)
    check(f"igemm concat {case}", res, F32)


def test_igemm_dilated():
    res = G.run_igemm(24, 32, 8, 12, 3, 1, [2] * 4, "hardswish", False, F32, 5202, d=2)
    check("igemm d2", res, F32)


@pytest.mark.parametrize("dt", [F16, BF16], ids=["f16", "bf16"])
@pytest.mark.parametrize("case", [(24, 32, 16, 24, 3, 1, "relu", 7201), (36, 64, 3, 16, 3, 2, "none", 7202),
                                  (18, 32, 171, 80, 3, 1, "relu", 7203)], ids=lambda c: str(c[-1]))
def test_igemm_16bit(case, dt):
    ih, iw, cin, cout, k, s, act, seed = case
    res = G.run_igemm(ih, iw, cin, cout, k, s, [1] * 4, act, False, dt, seed)
    check(f"igemm dt{dt} {case}", res, dt)


@pytest.mark.parametrize("splitk", [2, 4])
def test_igemm_splitk(splitk):
    res = G.run_igemm(9, 16, 128, 128, 3, 1, [1] * 4, "relu", True, F32, 7301, splitk=splitk)
    assert res.plan.splitk == splitk
    check(f"igemm splitk {splitk}", res, F32)


def test_igemm_batch():
    res = G.run_igemm(20, 36, 16, 32, 3, 2, [1] * 4, "relu", True, F32, 7401, n=3)
    check("igemm batch", res, F32)


# ---------------------------------------------------------------- the 3x3 direct route (<= 64 outputs)

# (ih, iw, cin or parts, cout, s, d, pad, act, residual, n, seed): every one is
# routed to the direct kernel in all three dtypes -- odd unit counts per part
# (a half-empty last step), output channels that do not fill a 32-column
# block, two parts, stride 2, dilation 2, asymmetric padding, residual, a
# ragged last block of 32 pixels, the largest K per tap
IG_DIRECT = [
    (20, 36, 16, 32, 1, 1, (1, 1, 1, 1), "relu", False, 2, 7501),
    (21, 37, 32, 64, 2, 1, (0, 1, 1, 0), "hardswish", True, 1, 7502),
    (16, 24, 24, 20, 1, 2, (2, 2, 2, 2), "sigmoid", False, 1, 7503),
    (13, 19, 40, 48, 1, 1, (1, 1, 1, 1), "relu6", True, 3, 7504),
    (24, 32, [32, 24], 32, 1, 1, (1, 1, 1, 1), "relu", False, 1, 7505),
    (17, 29, [16, 8], 12, 2, 1, (1, 1, 1, 1), "none", True, 1, 7506),
    (12, 20, 64, 64, 1, 1, (1, 1, 1, 1), "relu", False, 1, 7507),
    (10, 14, 80, 32, 1, 1, (1, 1, 1, 1), "hardswish", True, 2, 7508),
    (14, 18, [48, 24], 28, 1, 1, (1, 1, 1, 1), "relu", False, 1, 7509),
]


@pytest.mark.parametrize("dt", [F32, F16, BF16], ids=["f32", "f16", "bf16"])
@pytest.mark.parametrize("case", IG_DIRECT, ids=lambda c: str(c[-1]))
def test_igemm_direct(case, dt):
    """3x3, cout <= 64, same storage for activations and weights, whole
    16-byte units per part: the direct route of aih_conv_igemm (weights in
    LDS, activations straight into MFMA registers)."""
    ih, iw, cin, cout, s, d, pad, act, with_res, n, seed = case
    parts = cin if isinstance(cin, list) else None
    res = G.run_igemm(ih, iw, sum(parts) if parts else cin, cout, 3, s, pad, act, with_res, dt, seed, n=n, d=d,
                      parts=parts)
    assert res.plan.variant == G.conv.Variant.DIRECT, res.plan
    check(f"igemm direct dt{dt} {case}", res, dt)


@pytest.mark.parametrize("dt", [F32, F16], ids=["f32", "f16"])
def test_igemm_direct_channel_view(dt):
    """One input part that is a channel view (channels 8..31 of a 48-channel
    tensor, SrcView{c: 24, stride_c: 48, c_off: 8}): the direct route reads the
    view through its pixel stride and offset; checked against the oracle on
    the sliced input."""
    ih, iw, full, c0, c, cout, seed = 15, 21, 48, 8, 24, 20, 7511
    op = G.orc.conv2d(c, cout, k=3, s=1, pad=[1, 1, 1, 1], act="relu")
    xf, wts, b = G.stream(seed, ih * iw * full, cout * c * 9, cout)
    xs = xf.reshape(ih * iw, full)[:, c0:c0 + c].ravel().copy()
    want = G.orc.conv2d_ref(op, ih, iw, xs, wts, b, None)
    wp, _ = G.orc.pack_weights_conv(wts, cout, c, 3, 3, 4, dt)
    spec = G.conv.ConvIgemmSpec(ih=ih, iw=iw, cin=c, cout=cout, k=3, pad=(1, 1, 1, 1), act=G.ACT["relu"],
                                dt=G.conv.DType(dt), srcs=[G.conv.SrcView(c=c, stride_c=full, c_off=c0)])
    assert spec.plan().variant == G.conv.Variant.DIRECT
    yd = G.poisoned(ih * iw * 20, dt)
    spec.run([G.dev(G.orc.pack_nhwc(xf, 1, ih, iw, full, dt))], G.dev(wp), G.dev(G.orc.pack_bias(b, cout, dt)), None, yd)
    torch.cuda.synchronize()
    got = G.orc.unpack_nhwc(G.host(yd, dt), 1, ih, iw, cout, dt)
    err = G.rel_err(got, want)
    print(f"igemm direct channel view dt{dt}: max_rel_err={err:.3e}", flush=True)
    assert err <= (1e-4 if dt == F32 else 2e-2), err


@pytest.mark.parametrize("dt", [F16, BF16], ids=["f16", "bf16"])
def test_igemm_direct_10_steps_16bit(dt):
    """160 16-bit input channels: 10 MFMA steps per tap, the most the direct
    route takes (fp32 stops at 80 channels)."""
    res = G.run_igemm(9, 11, 160, 24, 3, 1, [1, 1, 1, 1], "relu", True, dt, 7510)
    assert res.plan.variant == G.conv.Variant.DIRECT, res.plan
    check(f"igemm direct 160->24 dt{dt}", res, dt)


# ---------------------------------------------------------------- the stem (3x3 over <= 3 channels)

STEM = [((160, 288, 3, 32, 2, (1, 1, 1, 1)), "relu", False, 3601, 2),
        ((33, 17, 3, 64, 1, (0, 1, 2, 1)), "hardswish", True, 3602, 1),
        ((16, 16, 1, 32, 2, (0, 0, 1, 1)), "none", False, 3603, 3),
        ((9, 9, 2, 32, 1, (1, 1, 1, 1)), "sigmoid", True, 3604, 2),
        ((7, 40, 3, 64, 2, (1, 1, 1, 1)), "relu6", False, 3605, 1)]


@pytest.mark.parametrize("dt", [F32, F16, BF16], ids=["f32", "f16", "bf16"])
@pytest.mark.parametrize("case", STEM, ids=str)
def test_stem_kernel(case, dt):
    """dense 3x3, d = 1, <= 3 input channels, cout 32 / 64: the stem route of
    aih_conv_igemm (every tap-channel value in one MFMA operand)."""
    (ih, iw, cin, cout, s, pad), act, with_res, seed, n = case
    res = G.run_igemm(ih, iw, cin, cout, 3, s, pad, act, with_res, dt, seed, n=n)
    check(f"stem dt{dt} {case}", res, dt)


@pytest.mark.parametrize("dt", [F32, F16, BF16], ids=["f32", "f16", "bf16"])
@pytest.mark.parametrize("case", STEM, ids=str)
def test_stem_from_f32_input_equals_pack_then_stem(case, dt):
    """aih_conv_stem_f32in reads the logical NHWC fp32 input and rounds it
    to dt as it loads: its output equals aih_pack_nhwc_device followed by
    aih_conv_igemm bit for bit (the same stored input, the same kernel)."""
    (ih, iw, cin, cout, s, pad), act, with_res, seed, n = case
    spec = G.conv.ConvIgemmSpec(ih=ih, iw=iw, cin=cin, cout=cout, k=3, s=s, pad=pad, act=G.ACT[act],
                                residual=with_res, dt=G.conv.DType(dt), n=n)
    oh, ow = spec.out_hw()
    x, wts, b, r = G.stream(seed, n * ih * iw * cin, cout * cin * 9, cout, n * oh * ow * cout if with_res else 0)
    xf = G.dev(np.asarray(x, np.float32))
    wp, _ = G.orc.pack_weights_conv(wts, cout, cin, 3, 3, 4, dt)
    wd, bd = G.dev(wp), G.dev(G.orc.pack_bias(b, cout, dt))
    rd = G.dev(G.orc.pack_nhwc(r, n, oh, ow, cout, dt)) if with_res else None
    n4 = -(-cout // 4) * 4
    xp = G.poisoned(n * ih * iw * 4, dt)
    G.conv.pack_nhwc_device(xf, n, ih, iw, cin, G.conv.DType(dt), xp)
    want = G.poisoned(n * oh * ow * n4, dt)
    spec.run([xp], wd, bd, rd, want)
    got = G.poisoned(n * oh * ow * n4, dt)
    spec.run_f32_input(xf, wd, bd, rd, got)
    G.torch.cuda.synchronize()
    assert G.torch.equal(got.view(-1), want.view(-1))

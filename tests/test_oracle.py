"""Pins the CPU oracle (oracle/) before anything is checked against it.

Sources of truth, none of which is the oracle's own formula retyped:
  * the reference's own known-answer tests, ported value for value
    (crates/ai-core/src/{rng,activation,tensor,pack,reference/conv}.rs test
    modules, crates/ai-cpu/src/kernels/*.rs test modules, and the variant
    policy KATs of crates/ai-gpu/src/kernels/{gemm_pw,conv_igemm}.rs);
  * textbook values (Marsaglia's xorshift32 sequence, IEEE binary16 /
    bfloat16 round-to-nearest-even as implemented by numpy and torch);
  * an independent float64 convolution (numpy shifted-slice GEMM) and
    torch.nn.functional.conv2d in float64;
  * invariants the reference states (row-split == full, concat parts ==
    materialized concat, pack/unpack round trips).
"""
import math

import numpy as np
import pytest
import torch

F32, F16, BF16 = 0, 1, 2


# ---------------------------------------------------------------- helpers

def conv_f64(x, w, bias, ih, iw, cin, cout, kh, kw, sh, sw, pad, dil, groups, act="none", res=None,
             absval=False):
    """Independent float64 conv (shifted slices + matmul), logical NHWC, OIHW."""
    X = np.asarray(x, np.float64).reshape(ih, iw, cin)
    W = np.asarray(w, np.float64).reshape(cout, cin // groups, kh, kw)
    if absval:
        X, W = np.abs(X), np.abs(W)
    ph, pw_ = ih + pad[0] + pad[2], iw + pad[1] + pad[3]
    Xp = np.zeros((ph, pw_, cin))
    Xp[pad[0]:pad[0] + ih, pad[1]:pad[1] + iw] = X
    oh = (ph - (dil * (kh - 1) + 1)) // sh + 1
    ow = (pw_ - (dil * (kw - 1) + 1)) // sw + 1
    cin_g, cout_g = cin // groups, cout // groups
    out = np.zeros((oh, ow, cout))
    for ky in range(kh):
        for kx in range(kw):
            patch = Xp[ky * dil: ky * dil + sh * (oh - 1) + 1: sh, kx * dil: kx * dil + sw * (ow - 1) + 1: sw, :]
            for g in range(groups):
                out[..., g * cout_g:(g + 1) * cout_g] += (
                    patch[..., g * cin_g:(g + 1) * cin_g] @ W[g * cout_g:(g + 1) * cout_g, :, ky, kx].T)
    if bias is not None:
        out += np.abs(np.asarray(bias, np.float64)) if absval else np.asarray(bias, np.float64)
    if absval:
        return out.ravel()
    if act == "relu":
        out = np.maximum(out, 0)
    elif act == "relu6":
        out = np.clip(out, 0, 6)
    elif act == "none":
        pass
    else:
        raise ValueError(act)
    if res is not None:
        out = out + np.asarray(res, np.float64).reshape(out.shape)
    return out.ravel()


def assert_close_ref(got, want, what=""):
    """ai-cpu's own bar: |a - g| <= 1e-4 * max(|a|, 1) (crates/ai-cpu/src/kernels/conv.rs:502-506)."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    err = np.abs(got - want) / np.maximum(np.abs(want), 1.0)
    assert got.shape == want.shape
    assert err.max(initial=0) <= 1e-4, f"{what}: max rel err {err.max()}"


# ---------------------------------------------------------------- rng

def test_xorshift32_marsaglia_sequence(orc):
    # Marsaglia (2003), xorshift32 with (13, 17, 5) from state 1: 270369, ...
    seq = orc.xs32_u32(1, 3)
    assert seq[0] == 270369
    # second value from the same textbook recurrence on 270369
    x = 270369
    x ^= (x << 13) & 0xFFFFFFFF
    x ^= x >> 17
    x ^= (x << 5) & 0xFFFFFFFF
    assert seq[1] == x


def test_xorshift32_seed_zero_substitution(orc):
    # rng.rs:7: seed 0 -> 0x9e3779b9
    assert orc.xs32_u32(0, 5) == orc.xs32_u32(0x9E3779B9, 5)


def test_xorshift32_deterministic_and_in_range(orc):
    # rng.rs:43-52
    a = orc.xs32_fill(42, 1000)
    b = orc.xs32_fill(42, 1000)
    assert np.array_equal(a, b)
    assert (a >= -1.0).all() and (a < 1.0).all()


def test_xorshift32_f32_quantisation(orc):
    # next_f32 keeps 24 bits: every value is k/2^23 - 1 for an integer k in [0, 2^24)
    v = orc.xs32_fill(7, 10000).astype(np.float64)
    k = (v + 1.0) * 2 ** 23
    assert np.array_equal(k, np.round(k))
    # and it is the top 24 bits of the u32 stream
    u = np.array(orc.xs32_u32(7, 10000), dtype=np.uint64)
    assert np.array_equal(k.astype(np.uint64), u >> np.uint64(8))


def test_gauss_moments(orc):
    z = orc.gauss_fill(123, 0.0, 0.05, 200000).astype(np.float64)
    assert abs(z.mean()) < 0.05 * 4 / math.sqrt(len(z))
    assert abs(z.std() / 0.05 - 1) < 0.01
    # kurtosis of a normal is 3
    assert abs(((z - z.mean()) ** 4).mean() / z.var() ** 2 - 3) < 0.05
    assert np.array_equal(z, orc.gauss_fill(123, 0.0, 0.05, 200000).astype(np.float64))


# ---------------------------------------------------------------- activation

def test_activation_kats(orc):
    # activation.rs:67-76
    assert orc.act_apply("hardsigmoid", 3.0) == 1.0
    assert orc.act_apply("hardsigmoid", -3.0) == 0.0
    assert orc.act_apply("hardsigmoid", 0.0) == 0.5
    assert orc.act_apply("hardswish", 3.0) == 3.0
    assert orc.act_apply("hardswish", -3.0) == 0.0
    assert abs(orc.act_apply("hardswish", 1.0) - 2.0 / 3.0) < 1e-6
    # closed forms for the activations the configs use
    for x in np.array([-7.5, -1.0, -0.0, 0.25, 5.999, 6.0, 6.5, 100.0], np.float32).tolist():
        assert orc.act_apply("relu", x) == max(x, 0.0)
        assert orc.act_apply("relu6", x) == min(max(x, 0.0), 6.0)
        assert orc.act_apply("none", x) == x


def test_activation_closed_forms_and_array(orc):
    """Every activation against its closed form (activation.rs:28-43), and the
    array form (what the GPU activation tests compare with) equal to the
    scalar one element for element."""
    import math

    xs = np.array([-30.0, -7.5, -3.0, -1.0, -0.0, 1e-3, 0.25, 1.0, 2.0, 5.999, 6.0, 9.0, 30.0], np.float32)
    f = {
        "none": lambda x: x, "relu": lambda x: max(x, 0.0), "sigmoid": lambda x: 1.0 / (1.0 + math.exp(-x)),
        "tanh": math.tanh, "hardswish": lambda x: x * min(max(x / 6.0 + 0.5, 0.0), 1.0),
        "hardsigmoid": lambda x: min(max(x / 6.0 + 0.5, 0.0), 1.0), "clamp01": lambda x: min(max(x, 0.0), 1.0),
        "relu6": lambda x: min(max(x, 0.0), 6.0), "sqrt": lambda x: math.sqrt(max(x, 0.0)), "neg": lambda x: -x,
        "recip": lambda x: 1.0 / x if x != 0 else math.copysign(math.inf, x),
    }
    assert set(f) == set(orc.ACT)
    for name, fn in f.items():
        arr = orc.act_array(name, xs)
        for x, y in zip(xs.tolist(), arr.tolist()):
            assert y == orc.act_apply(name, x), (name, x)
            want = fn(x)
            assert abs(y - want) <= 2e-7 * max(abs(want), 1.0) or (math.isinf(want) and y == want), (name, x, y, want)


# ---------------------------------------------------------------- dtype conversion

def test_f16_matches_ieee_rne(orc):
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.standard_normal(100000).astype(np.float32) * np.float32(3.0),
        (rng.standard_normal(20000) * 1e-5).astype(np.float32),  # subnormal range
        (rng.standard_normal(20000) * 7e4).astype(np.float32),   # overflow range
        np.array([0.0, -0.0, 65504, 65519.99, 65520, -65520, 2 ** -24, 2 ** -25, 3 * 2 ** -26,
                  np.inf, -np.inf, 1 + 2 ** -11, 1 + 3 * 2 ** -11], np.float32),
    ])
    got = orc.cvt_from_f32(vals, F16)
    want = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)
    back = orc.cvt_to_f32(got, F16)
    assert np.array_equal(back, want.view(np.float16).astype(np.float32))
    assert np.isnan(orc.cvt_to_f32(orc.cvt_from_f32(np.array([np.nan], np.float32), F16), F16)[0])


def test_bf16_matches_rne(orc):
    rng = np.random.default_rng(1)
    vals = np.concatenate([
        rng.standard_normal(100000).astype(np.float32),
        np.array([1.0, 1 + 2 ** -8, 1 + 3 * 2 ** -8, -(1 + 2 ** -8), 3.4e38, np.finfo(np.float32).max,
                  np.inf, -np.inf, 1e-40, -0.0], np.float32),
    ])
    got = orc.cvt_from_f32(vals, BF16)
    want = torch.from_numpy(vals).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)
    # closed forms: ties go to even, the largest finite f32 rounds to +inf
    assert orc.cvt_from_f32([1 + 2 ** -8], BF16)[0] == 0x3F80
    assert orc.cvt_from_f32([1 + 3 * 2 ** -8], BF16)[0] == 0x3F82
    assert orc.cvt_from_f32([np.finfo(np.float32).max], BF16)[0] == 0x7F80
    nan16 = orc.cvt_from_f32(np.array([np.nan], np.float32), BF16)[0]
    assert (nan16 & 0x7F80) == 0x7F80 and (nan16 & 0x7F) != 0


# ---------------------------------------------------------------- layout / packing

def test_layout_math(orc):
    # tensor.rs:87-110 -- idx(h,w,cg) = (h*W + w)*cg_count + cg; C padded to 4
    h, w, c = 3, 5, 6
    data = np.arange(h * w * c, dtype=np.float32)
    packed = orc.pack_nhwc(data, 1, h, w, c)
    cg = 2
    assert packed.size * 4 == 3 * 5 * 2 * 16
    for (hh, ww, g, want_idx) in [(0, 0, 0, 0), (0, 0, 1, 1), (0, 1, 0, 2), (1, 0, 0, 10), (2, 4, 1, (2 * 5 + 4) * 2 + 1)]:
        assert (hh * w + ww) * cg + g == want_idx
        vec = packed[want_idx * 4: want_idx * 4 + 4]
        for comp in range(4):
            ch = g * 4 + comp
            exp = data[(hh * w + ww) * c + ch] if ch < c else 0.0
            assert vec[comp] == exp
    # f16 sizes (tensor.rs:102-105)
    assert orc.lib().orc_nhwc_c4_bytes(1, 9, 16, 64, F16) == 9 * 16 * 16 * 8
    assert orc.lib().orc_nhwc_c4_bytes(1, 1, 1, 1, F32) == 16


def test_nhwc_roundtrip_f32_odd_shapes(orc):
    # pack.rs:192-199
    data = orc.xs32_fill(1, 3 * 5 * 6)
    packed = orc.pack_nhwc(data, 1, 3, 5, 6)
    assert packed.nbytes == 3 * 5 * 2 * 16
    assert np.array_equal(orc.unpack_nhwc(packed, 1, 3, 5, 6), data)


def test_nhwc_roundtrip_f16_tolerance(orc):
    # pack.rs:201-209
    data = orc.xs32_fill(2, 2 * 3 * 5)
    rt = orc.unpack_nhwc(orc.pack_nhwc(data, 1, 2, 3, 5, F16), 1, 2, 3, 5, F16)
    assert np.abs(rt - data).max() < 1e-3


def test_pack_padding_channels_are_zero(orc):
    # pack.rs:211-220
    packed = orc.pack_nhwc(np.ones(1 * 2 * 3, np.float32), 1, 1, 2, 3)
    assert packed[3] == 0.0 and packed[7] == 0.0


def test_batch_is_outermost(orc):
    n, h, w, c = 3, 2, 3, 5
    data = orc.xs32_fill(9, n * h * w * c)
    packed = orc.pack_nhwc(data, n, h, w, c).reshape(n, h * w, 8)
    for b in range(n):
        one = orc.pack_nhwc(data[b * h * w * c:(b + 1) * h * w * c], 1, h, w, c).reshape(h * w, 8)
        assert np.array_equal(packed[b], one)


def test_conv_weight_layout_pointwise_identity(orc):
    # pack.rs:222-238
    w = np.zeros(16, np.float32)
    for i in range(4):
        w[i * 4 + i] = 1.0
    packed, kg = orc.pack_weights_conv(w, 4, 4, 1, 1, 1)
    assert kg == 1
    for j in range(4):
        for comp in range(4):
            assert packed[j * 4 + comp] == (1.0 if j == comp else 0.0)


def test_conv_weight_kg_alignment_pads_zero(orc):
    # pack.rs:240-254
    w = orc.xs32_fill(3, 8 * 6)
    packed, kg = orc.pack_weights_conv(w, 8, 6, 1, 1, 4)
    assert kg == 4
    ng = 2
    assert (packed[2 * ng * 16: 4 * ng * 16] == 0).all()


def test_pack_weights_index_formula(orc):
    # pack.rs:95 -- out[((((t*KG + kg)*NG + ng)*4 + j)*4 + comp)] = w[oc][ic][ky][kx]
    cout, cin, kh, kw = 10, 7, 3, 2
    w = np.arange(cout * cin * kh * kw, dtype=np.float32) + 1
    packed, kgp = orc.pack_weights_conv(w, cout, cin, kh, kw, 4)
    ng = 3
    W = w.reshape(cout, cin, kh, kw)
    P = packed.reshape(kh * kw, kgp, ng, 4, 4)
    for t in range(kh * kw):
        for oc in range(12):
            for ic in range(kgp * 4):
                v = P[t, ic // 4, oc // 4, oc % 4, ic % 4]
                exp = W[oc, ic, t // kw, t % kw] if (oc < cout and ic < cin) else 0.0
                assert v == exp


def test_pack_unpack_roundtrip_conv_and_dw(orc):
    # pack.rs:256-271 (one XorShift32 stream feeds all three tensors)
    stream = orc.xs32_fill(11, 10 * 6 * 9 + 7 * 9 + 10)
    cout, cin, k = 10, 6, 3
    w = stream[:cout * cin * k * k]
    packed, kg_pad = orc.pack_weights_conv(w, cout, cin, k, k, 4)
    assert np.array_equal(orc.unpack_weights_conv(packed, cout, cin, k, k, kg_pad), w)
    wd = stream[cout * cin * 9: cout * cin * 9 + 7 * 9]
    assert np.array_equal(orc.unpack_weights_dw(orc.pack_weights_dw(wd, 7, 3, 3), 7, 3, 3), wd)
    b = stream[-10:]
    assert np.array_equal(orc.unpack_bias(orc.pack_bias(b, cout), cout), b)


def test_dw_weight_layout(orc):
    # pack.rs:273-288
    c, taps, cg = 5, 9, 2
    w = np.arange(c * taps, dtype=np.float32)
    flat = orc.pack_weights_dw(w, c, 3, 3)
    for t in range(taps):
        assert flat[(t * cg + 1) * 4] == 4 * taps + t
        assert flat[(t * cg + 1) * 4 + 1] == 0.0


# ---------------------------------------------------------------- reference conv2d KATs

def test_conv2d_hand_computed_box_sum(orc):
    # reference/conv.rs:71-91
    op = orc.conv2d(1, 1, k=3, s=1, pad=1)
    out = orc.conv2d_ref(op, 3, 3, np.arange(1, 10, dtype=np.float32), np.ones(9, np.float32))
    assert out[4] == 45.0 and out[0] == 12.0 and out[8] == 28.0


def test_conv2d_pointwise_identity(orc):
    # reference/conv.rs:93-103
    x = np.arange(12, dtype=np.float32) * 0.5
    w = np.eye(3, dtype=np.float32).ravel()
    assert np.array_equal(orc.conv2d_ref(orc.conv2d(3, 3), 2, 2, x, w), x)


def test_conv2d_hand_computed_pointwise_bias_act(orc):
    # reference/conv.rs:105-114
    out = orc.conv2d_ref(orc.conv2d(2, 1, act="relu"), 1, 2, [1.0, -1.0, 0.5, 2.0], [2.0, 3.0], bias=[1.0])
    assert list(out) == [0.0, 8.0]


def test_conv2d_hand_computed_depthwise(orc):
    # reference/conv.rs:116-129
    x = [1.0, 10.0, 2.0, 20.0, 3.0, 30.0, 4.0, 40.0]
    w = np.concatenate([np.ones(9), 2 * np.ones(9)]).astype(np.float32)
    out = orc.conv2d_ref(orc.conv2d(2, 2, k=3, s=1, pad=1, groups=2), 2, 2, x, w)
    assert out[0] == 10.0 and out[1] == 200.0


def test_conv2d_residual_applied_after_activation(orc):
    # reference/conv.rs:131-140
    out = orc.conv2d_ref(orc.conv2d(1, 1, act="relu"), 1, 1, [-1.0], [1.0], res=[5.0])
    assert list(out) == [5.0]


def test_conv2d_stride2_asymmetric_pad(orc):
    # reference/conv.rs:142-165
    op = orc.conv2d(1, 1, k=2, s=2, pad=[1, 0, 0, 1])
    assert orc.out_hw(op, 4, 4) == (2, 2)
    out = orc.conv2d_ref(op, 4, 4, np.arange(1, 17, dtype=np.float32), np.ones(4, np.float32))
    assert out[0] == 3.0 and out[3] == 38.0


SHAPES_F64 = [
    # ih, iw, cin, cout, k, s, pad, dil, groups, act, res
    (6, 7, 3, 5, 1, 1, [0] * 4, 1, 1, "relu", False),
    (5, 9, 8, 16, 1, 1, [0] * 4, 1, 1, "none", True),
    (8, 8, 6, 10, 3, 1, [1] * 4, 1, 1, "none", False),
    (9, 11, 6, 10, 3, 2, [1] * 4, 1, 1, "relu", True),
    (6, 6, 4, 8, 2, 2, [1, 0, 0, 1], 1, 1, "none", False),
    (7, 7, 3, 5, 3, 1, [2] * 4, 2, 1, "relu6", False),
    (10, 12, 3, 8, 3, 2, [1] * 4, 1, 1, "relu", False),
    (7, 9, 8, 8, 3, 1, [1] * 4, 1, 8, "relu", True),
    (8, 8, 7, 7, 3, 2, [1] * 4, 1, 7, "none", False),
    (9, 6, 3, 3, 5, 1, [2] * 4, 1, 3, "none", True),
    (10, 18, 96, 32, 1, 1, [0] * 4, 1, 1, "none", True),
    (12, 14, 32, 24, 3, 1, [1] * 4, 1, 1, "relu", False),
]


@pytest.mark.parametrize("case", SHAPES_F64, ids=lambda c: "x".join(map(str, c[:6])))
def test_conv2d_ref_vs_independent_f64(orc, case):
    ih, iw, cin, cout, k, s, pad, dil, groups, act, with_res = case
    rng = np.random.default_rng(ih * 131 + cin)
    x = rng.uniform(-1, 1, ih * iw * cin).astype(np.float32)
    w = rng.uniform(-1, 1, cout * (cin // groups) * k * k).astype(np.float32)
    b = rng.uniform(-1, 1, cout).astype(np.float32)
    op = orc.conv2d(cin, cout, k=k, s=s, pad=pad, dil=dil, groups=groups, act=act)
    oh, ow = orc.out_hw(op, ih, iw)
    res = rng.uniform(-1, 1, oh * ow * cout).astype(np.float32) if with_res else None
    got = orc.conv2d_ref(op, ih, iw, x, w, b, res)
    want = conv_f64(x, w, b, ih, iw, cin, cout, k, k, s, s, pad, dil, groups, act, res)
    # sequential fp32 summation error <= (K+1) eps sum|terms| (+ one rounding for res)
    mag = conv_f64(x, w, b, ih, iw, cin, cout, k, k, s, s, pad, dil, groups, absval=True)
    K = (cin // groups) * k * k
    bound = 2 * (K + 2) * 2.0 ** -24 * (mag + (np.abs(res) if res is not None else 0))
    assert (np.abs(got - want) <= bound + 1e-30).all()
    # the bound stays far below the average |term|, so a single dropped or
    # misplaced term (a wrong index or padding offset) cannot hide inside it
    assert bound.max() < 0.05 * (mag / (K + 1)).min()


@pytest.mark.parametrize("case", SHAPES_F64[:10], ids=lambda c: "x".join(map(str, c[:6])))
def test_conv2d_ref_vs_torch_f64(orc, case):
    ih, iw, cin, cout, k, s, pad, dil, groups, act, with_res = case
    rng = np.random.default_rng(7 + ih * 17 + cout)
    x = rng.uniform(-1, 1, ih * iw * cin).astype(np.float32)
    w = rng.uniform(-1, 1, cout * (cin // groups) * k * k).astype(np.float32)
    b = rng.uniform(-1, 1, cout).astype(np.float32)
    op = orc.conv2d(cin, cout, k=k, s=s, pad=pad, dil=dil, groups=groups, act=act)
    got = orc.conv2d_ref(op, ih, iw, x, w, b)
    X = torch.from_numpy(x.astype(np.float64)).reshape(1, ih, iw, cin).permute(0, 3, 1, 2)
    X = torch.nn.functional.pad(X, (pad[1], pad[3], pad[0], pad[2]))
    Y = torch.nn.functional.conv2d(X, torch.from_numpy(w.astype(np.float64)).reshape(cout, cin // groups, k, k),
                                   torch.from_numpy(b.astype(np.float64)), stride=s, dilation=dil, groups=groups)
    if act == "relu":
        Y = Y.clamp_min(0)
    elif act == "relu6":
        Y = Y.clamp(0, 6)
    want = Y.permute(0, 2, 3, 1).reshape(-1).numpy()
    assert np.abs(got - want).max() <= 1e-4


# ---------------------------------------------------------------- ai-cpu restatement

AICPU_CASES = [
    # crates/ai-cpu/src/kernels/conv.rs:513-569 test shapes (+ route they take)
    ("pw cin3 cout5 relu", dict(cin=3, cout=5, act="relu"), 6, 7, False, 1),
    ("pw cin8 cout16 hswish res", dict(cin=8, cout=16, act="hardswish"), 5, 9, True, 2),
    ("k3 s1 6->10", dict(cin=6, cout=10, k=3, s=1, pad=1), 8, 8, False, 3),
    ("k3 s2 relu res", dict(cin=6, cout=10, k=3, s=2, pad=1, act="relu"), 9, 11, True, 4),
    ("k2 s2 asym pad", dict(cin=4, cout=8, k=2, s=2, pad=[1, 0, 0, 1]), 6, 6, False, 5),
    ("d2 k3 pad2 sigmoid", dict(cin=5, cout=5, k=3, s=1, pad=2, dil=2, act="sigmoid"), 7, 7, False, 6),
    # im2row stem (im2row.rs:112-154)
    ("stem 3->8 k3 s2 relu", dict(cin=3, cout=8, k=3, s=2, pad=1, act="relu"), 10, 12, False, 9),
    # pw_dot (pw_dot.rs:70-98)
    ("pwdot 24->2", dict(cin=24, cout=2), 5, 6, False, 26),
    ("pwdot 7->3 relu", dict(cin=7, cout=3, act="relu"), 5, 6, False, 10),
    ("pwdot 16->4 sigmoid", dict(cin=16, cout=4, act="sigmoid"), 5, 6, False, 20),
    # dw (dw.rs:305-327)
    ("dw c8 k3 s1 relu", dict(cin=8, cout=8, k=3, s=1, pad=1, groups=8, act="relu"), 7, 9, True, 1),
    ("dw c7 k3 s2 hswish", dict(cin=7, cout=7, k=3, s=2, pad=1, groups=7, act="hardswish"), 8, 8, True, 2),
    ("dw c3 k5 pad2", dict(cin=3, cout=3, k=5, s=1, pad=2, groups=3), 9, 6, True, 3),
    # config-shaped (reduced spatial size)
    ("pw 32->64 relu6", dict(cin=32, cout=64, act="relu6"), 8, 14, False, 101),
    ("pw 960->160", dict(cin=960, cout=160), 10, 18, False, 102),
    ("k3 s2 16->32 relu", dict(cin=16, cout=32, k=3, s=2, pad=1, act="relu"), 16, 29, False, 103),
    ("k3 s1 32->64 relu", dict(cin=32, cout=64, k=3, s=1, pad=1, act="relu"), 8, 14, False, 104),
    ("pw 256->64 res", dict(cin=256, cout=64), 4, 9, True, 105),
    ("dw 256 k3 s1 relu", dict(cin=256, cout=256, k=3, s=1, pad=1, groups=256, act="relu"), 4, 9, False, 106),
    ("head 128->2", dict(cin=128, cout=2), 5, 9, False, 107),
]

EXPECTED_ROUTE = {
    "pw cin3 cout5 relu": "ConvStd", "stem 3->8 k3 s2 relu": "ConvStem", "pwdot 24->2": "PwDot",
    "dw c8 k3 s1 relu": "ConvDw", "head 128->2": "PwDot", "pw 256->64 res": "ConvStd",
}


def _run_aicpu(orc, kw, ih, iw, with_res, seed, threads=1):
    op = orc.conv2d(**kw)
    groups = kw.get("groups", 1)
    k = kw.get("k", 1)
    stream = orc.xs32_fill(seed, ih * iw * op.cin + op.cout * (op.cin // groups) * k * k + op.cout + 10 ** 6)
    o = 0
    x = stream[o:o + ih * iw * op.cin]; o += x.size
    w = stream[o:o + op.cout * (op.cin // groups) * k * k]; o += w.size
    b = stream[o:o + op.cout]; o += b.size
    oh, ow = orc.out_hw(op, ih, iw)
    res = orc.xs32_fill(seed + 7777, oh * ow * op.cout) if with_res else None
    want = orc.conv2d_ref(op, ih, iw, x, w, b, res)
    cc = orc.CpuConv(op, ih, iw, w, b, has_res=with_res)
    got = cc.run(x, 1, res, threads=threads)
    return cc, got, want


@pytest.mark.parametrize("case", AICPU_CASES, ids=lambda c: c[0])
def test_aicpu_matches_reference_conv(orc, case):
    name, kw, ih, iw, with_res, seed = case
    cc, got, want = _run_aicpu(orc, kw, ih, iw, with_res, seed)
    if name in EXPECTED_ROUTE:
        assert cc.route == EXPECTED_ROUTE[name]
    assert_close_ref(got, want, name)
    act = kw.get("act", "none")
    if cc.route != "PwDot" and act in ("none", "relu", "relu6"):
        # on x86 ai-cpu accumulates in the reference's order with unfused
        # multiply-add, so these routes agree bit for bit
        assert np.array_equal(got, want), name


@pytest.mark.parametrize("threads", [2, 3, 4, 8])
def test_aicpu_row_split_equals_full(orc, threads):
    # conv.rs:631-667: banded execution must equal the single-band run
    for kw, ih, iw in [(dict(cin=5, cout=9, k=3, s=2, pad=1, act="relu"), 11, 13),
                       (dict(cin=16, cout=32, k=3, s=2, pad=1, act="relu"), 20, 36),
                       (dict(cin=3, cout=32, k=3, s=2, pad=1, act="relu"), 20, 36),
                       (dict(cin=64, cout=64, k=3, s=1, pad=1, groups=64, act="relu"), 10, 18)]:
        _, full, _ = _run_aicpu(orc, kw, ih, iw, False, 8, threads=1)
        _, split, _ = _run_aicpu(orc, kw, ih, iw, False, 8, threads=threads)
        assert np.array_equal(full, split)


def test_aicpu_concat_parts_match_materialized(orc):
    # conv.rs:572-627: two parts, the second a channel slice of a wider tensor
    import ctypes as C
    ih, iw, c1, c2, big_c, c_off, cout = 5, 6, 3, 5, 8, 2, 12
    stream = orc.xs32_fill(7, ih * iw * (c1 + big_c) + cout * (c1 + c2) * 9 + cout)
    px = ih * iw
    x1 = np.concatenate([stream[:px * c1], np.zeros(4, np.float32)])
    big = np.concatenate([stream[px * c1:px * (c1 + big_c)], np.zeros(4, np.float32)])
    o = px * (c1 + big_c)
    cin = c1 + c2
    w = stream[o:o + cout * cin * 9]
    b = stream[o + cout * cin * 9:o + cout * cin * 9 + cout]
    xcat = np.concatenate([x1[:px * c1].reshape(px, c1), big[:px * big_c].reshape(px, big_c)[:, c_off:c_off + c2]], 1)
    op = orc.conv2d(cin, cout, k=3, s=1, pad=1, act="relu")
    want = orc.conv2d_ref(op, ih, iw, xcat.ravel(), w, b)
    wts = np.zeros(9 * cin * 16, np.float32)
    cout_pad = orc.lib().orc_cpu_repack_weights(w.ctypes.data_as(C.c_void_p), cout, cin, cin, 3, 3,
                                                wts.ctypes.data_as(C.c_void_p))
    bias = np.zeros(cout_pad, np.float32)
    bias[:cout] = b
    views = (orc.View * 2)(orc.View(x1.ctypes.data, 0, c1, c1), orc.View(big.ctypes.data, c_off, big_c, c2))
    ic0 = np.array([0, c1], np.uint32)
    c4 = np.array([c1, c2], np.uint32)
    got = np.zeros_like(want)
    orc.lib().orc_cpu_conv_std(C.byref(op), ih, iw, views, ic0.ctypes.data_as(C.c_void_p),
                               c4.ctypes.data_as(C.c_void_p), 2, wts.ctypes.data_as(C.c_void_p),
                               bias.ctypes.data_as(C.c_void_p), cout_pad, None,
                               got.ctypes.data_as(C.c_void_p), 0, ih)
    assert np.array_equal(got, want)


def test_aicpu_batch_runs_images_in_sequence(orc):
    kw = dict(cin=16, cout=32, k=3, s=2, pad=1, act="relu")
    op = orc.conv2d(**kw)
    ih, iw, n = 12, 20, 3
    x = orc.xs32_fill(5, n * ih * iw * 16)
    w = orc.xs32_fill(6, 32 * 16 * 9)
    b = orc.xs32_fill(7, 32)
    cc = orc.CpuConv(op, ih, iw, w, b)
    got = cc.run(x, n, threads=4)
    want = orc.conv2d_ref(op, ih, iw, x, w, b, n=n)
    assert np.array_equal(got, want)


# ---------------------------------------------------------------- variant policy KATs

def test_reference_pw_variant_policy(orc):
    # gemm_pw.rs:337-354
    assert orc.ref_pw_variant(1, 144, 36) == "Gemv"
    assert orc.ref_pw_variant(144, 240, 40) == "Splitk"
    assert orc.ref_pw_variant(144, 40, 240) == "Splitk"
    assert orc.ref_pw_variant(144, 168, 28) == "Splitk"
    assert orc.ref_pw_variant(9216, 16, 16) == "Tiled"
    assert orc.ref_pw_variant(576, 30, 10) == "Splitk"
    assert orc.ref_pw_variant(2304, 18, 6) == "Splitk"
    assert orc.ref_pw_variant(36864, 6, 4) == "Small"
    assert orc.ref_pw_variant(36864, 1, 4) == "Small"
    assert orc.ref_pw_variant(512, 8, 8) == "Small"


def test_reference_gemv_width(orc):
    # gemm_pw.rs:357-366
    assert orc.ref_gemv_width(60) == 64
    assert orc.ref_gemv_width(30) == 32
    assert orc.ref_gemv_width(240) == 256
    assert orc.ref_gemv_width(400) == 256
    assert orc.ref_gemv_width(9) == 32


def test_reference_splitk_geometry(orc):
    # gemm_pw.rs:55-73 and the SPLIT*CPW == 256 invariant (conv_igemm.rs:462-465)
    for cells in [1, 100, 8191, 8192, 50000]:
        split, cpw = orc.ref_splitk_geometry(cells)
        assert split * cpw == 256
        assert (split, cpw) == ((8, 32) if cells < 8192 else (4, 64))
    assert orc.ref_splitk_tile(40, 32) == (8, 4)
    assert orc.ref_splitk_tile(6, 32) == (16, 2)
    assert orc.ref_splitk_tile(5, 32) == (32, 1)
    assert orc.ref_splitk_tile(2, 32) == (16, 2)


def test_reference_igemm_variant_policy(orc):
    # conv_igemm.rs:606-651
    assert orc.ref_igemm_variant(72, 128, 3, 16, 3, 1) == "Direct"
    assert orc.ref_igemm_variant(24, 32, 16, 16, 3, 1) == "Direct"
    assert orc.ref_igemm_variant(72, 128, 64, 16, 3, 1) == "Direct"
    assert orc.ref_igemm_variant(9, 16, 64, 16, 3, 1) == "Splitk"
    assert orc.ref_igemm_variant(24, 32, 64, 128, 3, 1) == "Tiled"

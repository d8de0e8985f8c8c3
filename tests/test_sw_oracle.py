"""The oracle's restatement of the non-conv .sw ops, pinned by the reference's
own known-answer tests and by properties the mathematics fixes:

* resize  -- reference/resize.rs:52-80 (1x2 -> 1x4 half_pixel [0, .25, .75, 1],
             asymmetric [0, .5, 1, 1]; same size is the identity; a constant
             stays constant), plus separability (a 2-D resize of an outer
             product is the outer product of the 1-D resizes) and a brute-force
             fp64 restatement on a small random case;
* gpool   -- reference/pool.rs:88-93 (2x2, c=2 -> [2.5, 10]) and the fp64 mean;
* binary  -- reference/elementwise.rs:31-45 (add, mul + relu, scalar_first sub)
             and prelu's definition;
* graph   -- the oracle's graph runner on a two-op graph equals the ops run by
             hand, and a conv-only graph equals the ai-cpu conv chain.
"""
import numpy as np
import pytest

from oracle import sw_oracle as so


def r(a):
    return np.asarray(a, np.float32).reshape(1, 1, -1, 1)


def test_resize_known_answers():
    x = r([0.0, 1.0])
    assert so.resize_bilinear(x, 1, 4, "half_pixel").ravel().tolist() == [0.0, 0.25, 0.75, 1.0]
    assert so.resize_bilinear(x, 1, 4, "asymmetric").ravel().tolist() == [0.0, 0.5, 1.0, 1.0]
    c = np.full((1, 5, 7, 2), 3.0, np.float32)
    assert np.array_equal(so.resize_bilinear(c, 5, 7, "half_pixel"), c)
    assert np.all(np.abs(so.resize_bilinear(c, 10, 14, "half_pixel") - 3.0) < 1e-6)


def _resize_fp64(x, oh, ow, mode):
    n, ih, iw, c = x.shape
    out = np.zeros((n, oh, ow, c))
    for oy in range(oh):
        fy = (oy + 0.5) * ih / oh - 0.5 if mode == "half_pixel" else oy * ih / oh
        y0, y1 = min(max(int(np.floor(fy)), 0), ih - 1), min(max(int(np.floor(fy)) + 1, 0), ih - 1)
        ty = min(max(fy - np.floor(fy), 0.0), 1.0)
        for ox in range(ow):
            fx = (ox + 0.5) * iw / ow - 0.5 if mode == "half_pixel" else ox * iw / ow
            x0, x1 = min(max(int(np.floor(fx)), 0), iw - 1), min(max(int(np.floor(fx)) + 1, 0), iw - 1)
            tx = min(max(fx - np.floor(fx), 0.0), 1.0)
            top = x[:, y0, x0] * (1 - tx) + x[:, y0, x1] * tx
            bot = x[:, y1, x0] * (1 - tx) + x[:, y1, x1] * tx
            out[:, oy, ox] = top * (1 - ty) + bot * ty
    return out


@pytest.mark.parametrize("mode", ["half_pixel", "asymmetric"])
@pytest.mark.parametrize("shape", [(5, 7, 10, 14), (10, 18, 20, 36), (9, 9, 4, 5), (3, 8, 3, 8)])
def test_resize_against_fp64_and_separability(mode, shape):
    ih, iw, oh, ow = shape
    rng = np.random.default_rng(ih * 100 + oh)
    x = rng.uniform(-1, 1, (2, ih, iw, 3)).astype(np.float32)
    got = so.resize_bilinear(x, oh, ow, mode)
    assert np.abs(got - _resize_fp64(x.astype(np.float64), oh, ow, mode)).max() < 2e-6
    u = rng.uniform(-1, 1, ih).astype(np.float32)
    v = rng.uniform(-1, 1, iw).astype(np.float32)
    outer = (u[:, None] * v[None, :]).reshape(1, ih, iw, 1)
    ru = so.resize_bilinear(u.reshape(1, ih, 1, 1), oh, 1, mode).ravel()
    if iw == 1:
        return
    rv = so.resize_bilinear(v.reshape(1, 1, iw, 1), 1, ow, mode).ravel()
    assert np.abs(so.resize_bilinear(outer, oh, ow, mode)[0, :, :, 0] - np.outer(ru, rv)).max() < 1e-5


def test_gpool_known_answer_and_mean():
    x = np.array([1.0, 4.0, 2.0, 8.0, 3.0, 12.0, 4.0, 16.0], np.float32).reshape(1, 2, 2, 2)
    assert so.global_avg_pool(x).ravel().tolist() == [2.5, 10.0]
    y = np.random.default_rng(3).uniform(-1, 1, (2, 10, 18, 5)).astype(np.float32)
    assert np.abs(so.global_avg_pool(y).reshape(2, 5) - y.astype(np.float64).mean(axis=(1, 2))).max() < 1e-6


def test_binary_known_answers():
    a = np.array([1.0, -2.0, 3.0], np.float32)
    b = np.array([0.5, 1.0, -1.0], np.float32)
    assert so.act_np("none", so.binop_np("add", a, b)).tolist() == [1.5, -1.0, 2.0]
    assert so.act_np("relu", so.binop_np("mul", a, b)).tolist() == [0.5, 0.0, 0.0]
    assert so.binop_np("sub", np.float32(1.0), a).tolist() == [0.0, 3.0, -2.0]
    assert so.binop_np("prelu", a, b).tolist() == [1.0, -2.0, 3.0]


def test_graph_runner_matches_hand_run(orc):
    """gpool -> cvectensor mul, the SE-gate pattern of the real model (ops 28-30)."""
    from ai_engine_amd import sw

    g = dict(name="se", size=dict(h=6, w=10), dt_default="f32", dt_weights="f32",
             tensors=[dict(name="x", h=6, w=10, c=8, dt="f32", alias=None, last_use=1),
                      dict(name="g", h=1, w=1, c=8, dt="f32", alias=None, last_use=1),
                      dict(name="y", h=6, w=10, c=8, dt="f32", alias=None, last_use=2),
                      dict(name="z", h=12, w=20, c=8, dt="f32", alias=None, last_use=3)],
             inputs=[0], outputs=[3], states=[],
             ops=[{"kind": "gpool", "in": 0, "out": 1},
                  {"kind": "binary", "a": 0, "b": {"cvectensor": {"tid": 1}}, "out": 2, "op": "mul", "act": "relu"},
                  {"kind": "resize", "in": 2, "out": 3, "oh": 12, "ow": 20, "mode": "half_pixel"}])
    G = so.SwGraph(sw.write_container(g, b""))
    x = np.random.default_rng(1).uniform(-1, 1, (2, 6, 10, 8)).astype(np.float32)
    got = G.run({"x": x}, n=2)["z"]
    gate = so.global_avg_pool(x)
    want = so.resize_bilinear(np.maximum(x * gate, 0), 12, 20, "half_pixel")
    assert np.array_equal(got, want)


def test_graph_runner_conv_chain_matches_cpu_conv(orc):
    """A conv-only .sw (written like the converter does) run by the graph
    runner equals the same convs run one by one through the ai-cpu oracle."""
    from ai_engine_amd import sw
    from ai_engine_amd.workloads import Layer, _chain, make_weights

    layers = _chain([Layer("e", 16, 64, act="relu"), Layer("d", 64, 64, k=3, s=2, groups=64, act="relu6"),
                     Layer("p", 64, 24, act="none"), Layer("q", 24, 24, k=3, act="relu", res="p")], 9, 14)
    wts = make_weights(layers, seed=5)
    data = sw.conv_graph_to_sw("chain", layers, wts, 9, 14, 16)
    x = np.random.default_rng(2).uniform(-1, 1, (2, 9, 14, 16)).astype(np.float32)
    got = so.SwGraph(data).run({"input": x}, n=2)["q"]
    vals = {"input": x.ravel()}
    for L in layers:
        cv = orc.CpuConv(orc.conv2d(L.cin, L.cout, k=L.k, s=L.s, pad=[L.pad] * 4, groups=L.groups, act=L.act),
                         L.ih, L.iw, wts.w[L.name], wts.b[L.name], has_res=L.res is not None)
        vals[L.name] = cv.run(vals[L.src], 2, vals[L.res] if L.res else None)
    assert np.array_equal(got.ravel(), vals["q"])

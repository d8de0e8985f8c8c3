"""GPU parity of the .sw path through the C ABI of include/aih_model.h:

* the non-conv ops (aih_resize, aih_gpool, aih_binary, aih_concat) against
  the oracle's restatement (oracle/sw_oracle.py) on seeded inputs, in every
  storage dtype: fp32 <= 1e-4, f16 / bf16 <= 2e-2 against the fp32 oracle on
  the unrounded inputs (max |g - c| / max(|c|, 1));
* the reference converter's real model (tests/golden/segm_r11_160x288.sw, 36
  convs + resize / gpool / binary / concat) loaded by aih_model_load and run
  end to end at batch 1 and 2 against the oracle's graph run on the same
  weights and input: every op, fed the oracle's inputs, within fp32 1e-4;
  the whole graph within 1e-3 on every tensor (accumulated through up to 44
  chained ops); f16 / bf16 (weights converted at load): every op within
  2e-2 of the oracle with the same storage rounding, the end-to-end mask
  agreeing with fp32 on >= 99% of pixels;
  The model runs both as loaded by default -- its four 48 -> 96 -> 48
  inverted-residual blocks (ops 12-23) fused into one aih_ir_block launch
  each, checked block by block against the oracle's three ops -- and with
  AIH_MODEL_NO_FUSE, op by op;
* a synthetic conv chain written as a .sw the way the converter writes one,
  through the native loader.
Outputs of the op tests start as NaN.
"""
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():  # pragma: no cover
    pytest.skip("no GPU", allow_module_level=True)

from ai_engine_amd import conv, sw  # noqa: E402
from oracle import oracle as orc  # noqa: E402
from oracle import sw_oracle as so  # noqa: E402
from tests import gpu_util as G  # noqa: E402

F32, F16, BF16 = 0, 1, 2
BAR = {F32: 1e-4, F16: 2e-2, BF16: 2e-2}
HERE = os.path.dirname(os.path.abspath(__file__))
SEGM = os.path.join(HERE, "golden", "segm_r11_160x288.sw")


def c4(c):
    return -(-c // 4) * 4


def upload(x, dt):
    """logical [n, h, w, c] fp32 -> device NHWC-C4 in dt"""
    n, h, w, c = x.shape
    return G.dev(orc.pack_nhwc(x.ravel(), n, h, w, c, dt))


def download(t, shape, dt):
    n, h, w, c = shape
    return orc.unpack_nhwc(G.host(t, dt), n, h, w, c, dt).reshape(shape)


def rnd(seed, *shape):
    return orc.xs32_fill(seed, int(np.prod(shape))).reshape(shape)


# ---------------------------------------------------------------- ops

def rdt(x, dt):
    """x rounded to the storage dtype (round to nearest even), as fp32."""
    n, h, w, c = x.shape
    return orc.unpack_nhwc(orc.pack_nhwc(x.ravel(), n, h, w, c, dt), n, h, w, c, dt).reshape(x.shape)


RESIZE_CASES = [(10, 18, 20, 36, "half_pixel"), (40, 72, 80, 144, "half_pixel"), (7, 9, 3, 4, "half_pixel"),
                (5, 6, 10, 12, "asymmetric"), (80, 144, 160, 288, "half_pixel"), (3, 7, 10, 11, "half_pixel"),
                (9, 5, 4, 13, "asymmetric")]


@pytest.mark.parametrize("dt", [F32, F16, BF16], ids=["f32", "f16", "bf16"])
@pytest.mark.parametrize("case", RESIZE_CASES, ids=lambda c: "x".join(map(str, c[:4])) + "_" + c[4])
def test_resize_matches_oracle(case, dt):
    """Bit for bit: the kernel rounds every product and sum as the reference's
    scalar code does (reference/resize.rs:36-38), so on inputs already in the
    storage dtype its output is the oracle's fp32 result rounded to that
    dtype. Up- and downscales at non-power-of-two ratios, both modes."""
    ih, iw, oh, ow, mode = case
    n = 2
    # two parts: 8 channels of a 12-channel tensor starting at channel 4 (a
    # view), then a 6-channel tensor -> 14 output channels
    a = rdt(rnd(11, n, ih, iw, 12), dt)
    b = rdt(rnd(12, n, ih, iw, 6), dt)
    y = G.poisoned(n * oh * ow * c4(14), dt)
    print(f"resize {case} dt{dt}", flush=True)
    sw.resize([(upload(a, dt), 8, 12, 4), (upload(b, dt), 6, 8, 0)], n, ih, iw, oh, ow, mode, dt, y)
    torch.cuda.synchronize()
    got = download(y, (n, oh, ow, 14), dt)
    want = rdt(so.resize_bilinear(np.concatenate([a[..., 4:12], b], -1), oh, ow, mode), dt)
    assert np.array_equal(got, want), G.rel_err(got, want)
    raw = G.host(y, dt).reshape(n * oh * ow, c4(14))
    assert not raw[:, 14:].any()  # padding lanes are zero


# (channels, resized) per part; every part but the last a multiple of 4 channels
RC_CASES = [[(32, True), (12, False)], [(12, False), (8, True), (5, True)], [(4, False), (8, False), (3, False)],
            [(8, True)], [(16, True), (4, False), (8, True), (6, False)]]


@pytest.mark.parametrize("dt", [F32, F16, BF16], ids=["f32", "f16", "bf16"])
@pytest.mark.parametrize("parts", RC_CASES, ids=lambda ps: "_".join(f"{c}{'r' if r else 'p'}" for c, r in ps))
@pytest.mark.parametrize("geo", [(40, 72, 80, 144, "half_pixel"), (5, 7, 9, 4, "asymmetric")],
                         ids=lambda g: "x".join(map(str, g[:4])) + "_" + g[4])
def test_resize_concat_equals_resize_then_concat(geo, parts, dt):
    """aih_resize_concat (a resize folded into the concat that reads it) is
    bit for bit aih_resize of the resized parts followed by aih_concat, and
    the oracle's resize and concatenation rounded to the storage dtype; the
    resized parts are channel views (4 channels in, a 4-channel wider
    buffer)."""
    ih, iw, oh, ow, mode = geo
    n = 2
    xs, args, want = [], [], []
    for i, (c, r) in enumerate(parts):
        h, w = (ih, iw) if r else (oh, ow)
        x = rdt(rnd(100 + i, n, h, w, c4(c) + 8), dt)  # the part is channels 4 .. 4 + c of a wider tensor
        xs.append(x)
        args.append((upload(x, dt), c, c4(c) + 8, 4, r))
        want.append(so.resize_bilinear(x[..., 4:4 + c], oh, ow, mode) if r else x[..., 4:4 + c])
    cout = sum(c for c, _ in parts)
    y = G.poisoned(n * oh * ow * c4(cout), dt)
    print(f"resize_concat {geo} {parts} dt{dt}", flush=True)
    sw.resize_concat(args, n, ih, iw, oh, ow, mode, dt, y)
    # the two launches: each resized part on its own, then the concat
    tmp = []
    for (t, c, st, off, r) in args:
        if r:
            z = G.poisoned(n * oh * ow * c4(c), dt)
            sw.resize([(t, c, st, off)], n, ih, iw, oh, ow, mode, dt, z)
            tmp.append((z, c, c4(c), 0))
        else:
            tmp.append((t, c, st, off))
    y2 = G.poisoned(n * oh * ow * c4(cout), dt)
    sw.concat(tmp, n, oh, ow, dt, y2)
    torch.cuda.synchronize()
    assert torch.equal(y.view(-1), y2.view(-1))
    got = download(y, (n, oh, ow, cout), dt)
    assert np.array_equal(got, rdt(np.concatenate(want, -1), dt))


def test_resize_concat_rejects_bad_parts():
    dt = F16
    x = upload(rnd(5, 1, 4, 4, 8), dt)
    y = G.poisoned(8 * 8 * 16, dt)
    bad = [
        ([(x, 8, 8, 0, True)], 2, "resized bits past the parts"),  # mask bit 1 without a part 1
        ([(x, 6, 8, 0, True), (x, 8, 8, 0, False)], None, "multiple of 4"),
        ([(x, 8, 8, 0, True)] * 9, None, "1 to 8 parts"),
    ]
    for parts, mask, why in bad:
        d = sw._ResizeConcat(1, 4, 4, 8, 8, 0, dt, len(parts), mask if mask is not None else
                             sum(1 << i for i, p in enumerate(parts) if p[4]),
                             sw._srcs([(c, s, o) for _, c, s, o, _ in parts[:8]]))
        rc = sw.lib().aih_resize_concat(sw.C.byref(d), sw._ptrs([p[0] for p in parts]), conv._ptr(y),
                                        conv._stream(None))
        assert rc != 0 and why in conv.last_error(), (why, conv.last_error())


@pytest.mark.parametrize("dt", [F32, F16, BF16], ids=["f32", "f16", "bf16"])
@pytest.mark.parametrize("shape", [(1, 10, 18, 48), (3, 40, 72, 30), (2, 1, 1, 5), (2, 160, 288, 8)],
                         ids=lambda s: "x".join(map(str, s)))
def test_gpool_matches_oracle(shape, dt):
    n, h, w, c = shape
    x = rnd(21, *shape)
    y = G.poisoned(n * c4(c), dt)
    sw.gpool(upload(x, dt), n, h, w, c, dt, y)
    torch.cuda.synchronize()
    assert G.rel_err(download(y, (n, 1, 1, c), dt), so.global_avg_pool(x)) <= BAR[dt]


OPERANDS = ["tensor", "scalar", "scalar_first", "cvec", "cvectensor", "cvectensor1", "pvectensor",
            "pvectensor_row", "tiledtensor"]


@pytest.mark.parametrize("dt", [F32, F16, BF16], ids=["f32", "f16", "bf16"])
@pytest.mark.parametrize("operand", OPERANDS)
@pytest.mark.parametrize("op,act", [("add", "none"), ("sub", "relu"), ("mul", "sigmoid"), ("prelu", "none")])
def test_binary_matches_oracle(op, act, operand, dt):
    n, h, w, c = 2, 6, 11, 10
    a = rnd(31, n, h, w, c)
    y = G.poisoned(n * h * w * c4(c), dt)
    kw = dict(operand=operand)
    if operand == "tensor":
        bl = rnd(32, n, h, w, c)
        bd, want_b = upload(bl, dt), bl
    elif operand in ("scalar", "scalar_first"):
        bd, want_b = None, np.float32(-0.375)
        kw = dict(operand="scalar", scalar=-0.375, scalar_first=operand == "scalar_first")
    elif operand == "cvec":
        v = rnd(33, c)
        bd, want_b = G.dev(orc.pack_nhwc(v, 1, 1, 1, c, dt)), v.reshape(1, 1, 1, c)
    elif operand == "cvectensor":
        v = rnd(34, n, 1, 1, c)
        bd, want_b = upload(v, dt), v
        kw["b_c"] = c
    elif operand == "cvectensor1":
        v = rnd(35, n, 1, 1, 1)
        bd, want_b = upload(v, dt), v
        kw = dict(operand="cvectensor", b_c=1)
    elif operand == "pvectensor":
        v = rnd(36, n, h, w, 1)
        bd, want_b = upload(v, dt), v
        kw["b_c"] = 1
    elif operand == "pvectensor_row":
        v = rnd(37, n, 1, 1, h * w)
        bd, want_b = upload(v, dt), v.reshape(n, h, w, 1)
        kw = dict(operand="pvectensor", b_c=h * w)
    else:
        L = 4
        v = rnd(38, n, 1, 1, L)
        bd, want_b = upload(v, dt), v.reshape(n, L)[:, np.arange(c) % L].reshape(n, 1, 1, c)
        kw["b_c"] = L
    print(f"binary {op} {act} {operand} dt{dt}", flush=True)
    sw.binary(upload(a, dt), bd, n, h, w, c, op, orc.ACT[act], dt, y, **kw)
    torch.cuda.synchronize()
    if operand == "scalar_first":
        want = so.act_np(act, so.binop_np(op, np.broadcast_to(want_b, a.shape), a))
    else:
        want = so.act_np(act, so.binop_np(op, a, want_b))
    # the reference's rounding of the 16-bit operands is part of the
    # comparison: round a and b to dt first for the 16-bit bars
    assert G.rel_err(download(y, (n, h, w, c), dt), want) <= BAR[dt]


@pytest.mark.parametrize("dt", [F32, F16, BF16], ids=["f32", "f16", "bf16"])
@pytest.mark.parametrize("parts", [[32, 12], [3, 5, 8], [4, 4], [2, 2, 2, 2, 2, 2, 2, 2], [13]],
                         ids=lambda p: "-".join(map(str, p)))
def test_concat_matches_oracle(parts, dt):
    n, h, w = 2, 9, 7
    xs = [rnd(40 + i, n, h, w, c) for i, c in enumerate(parts)]
    cout = sum(parts)
    y = G.poisoned(n * h * w * c4(cout), dt)
    sw.concat([(upload(x, dt), c, c4(c), 0) for x, c in zip(xs, parts)], n, h, w, dt, y)
    torch.cuda.synchronize()
    got = download(y, (n, h, w, cout), dt)
    assert G.rel_err(got, np.concatenate(xs, -1)) <= BAR[dt]
    # the padding lanes of the last vec4 are zero
    raw = G.host(y, dt).reshape(n * h * w, c4(cout))
    assert not raw[:, cout:].any()


# ---------------------------------------------------------------- models

@pytest.fixture(scope="module")
def segm():
    data = open(SEGM, "rb").read()
    return data, so.SwGraph(data)


def _op_inputs(op):
    ins = [op.get("in"), op.get("a"), op.get("res")]
    ins += [p["in"] for p in op.get("srcs", []) + op.get("parts", [])]
    b = op.get("b")
    if isinstance(b, dict) and len(b) == 1:
        (bk, bv), = b.items()
        if isinstance(bv, dict) and "tid" in bv:
            ins.append(bv["tid"])
    return sorted({t for t in ins if isinstance(t, int)})


SEGM_FUSED = [12, 15, 18, 21]  # first ops of the real model's inverted-residual blocks
SEGM_PAIRS = {33, 40}  # depthwise -> pointwise pairs a load may fuse (when the batch gives every CU a tile)
SEGM_RESIZE_CONCAT = [38]  # the 40x72 -> 80x144 resize folded into the concat after it


def _check_fused(m, fuse):
    """The model's fused launches: exactly the four inverted-residual blocks
    and the resize folded into the concat, plus depthwise -> pointwise pairs
    among SEGM_PAIRS only."""
    blocks = m.fused_blocks()
    if not fuse:
        assert blocks == []
        return []
    assert [f.first_op for f in blocks if f.kind == sw.FUSED_IR_BLOCK] == SEGM_FUSED
    assert [(f.first_op, f.n_ops) for f in blocks if f.kind == sw.FUSED_RESIZE_CONCAT] == [(k, 2) for k in
                                                                                            SEGM_RESIZE_CONCAT]
    pairs = [f.first_op for f in blocks if f.kind == sw.FUSED_DWPW]
    assert all(f.n_ops == 2 for f in blocks if f.kind == sw.FUSED_DWPW)
    assert set(pairs) <= SEGM_PAIRS, pairs
    assert len(blocks) == len(SEGM_FUSED) + len(SEGM_RESIZE_CONCAT) + len(pairs), [(f.first_op, f.kind) for f in blocks]
    return pairs


def _launch_steps(m, graph):
    """(first op, last op + 1) of each launch the model makes: one op, or a
    fused block's two, three or four."""
    firsts = {f.first_op: f.n_ops for f in m.fused_blocks()}
    k, out = 0, []
    while k < len(graph.g["ops"]):
        step = firsts.get(k, 1)
        out.append((k, k + step))
        k += step
    return out


def _stored(m, graph, name):
    """Tensors a fused model keeps (every one but a fused block's intermediates)."""
    internal = set()
    for f in m.fused_blocks():
        for k in range(f.first_op, f.first_op + f.n_ops - 1):
            internal.add(graph.T[graph.g["ops"][k]["out"]]["name"])
    return name not in internal


def _check_launches(m, graph, ref, bar):
    """Every launch fed the reference values of its inputs, its output against
    the reference's; the worst error."""
    T, ops = graph.T, graph.g["ops"]
    worst = 0.0
    for a, b in _launch_steps(m, graph):
        for k in range(a, b):
            for tid in _op_inputs(ops[k]):
                if any(ops[j]["out"] == tid for j in range(a, k)):
                    continue  # made inside the block
                m.write_tensor(T[tid]["name"], ref[T[tid]["name"]])
        m.infer_range(a, b)
        name = T[ops[b - 1]["out"]]["name"]
        e = G.rel_err(m.read_output(name), ref[name])
        worst = max(worst, e)
        assert e <= bar, (a, b, ops[b - 1]["kind"], name, e)
    return worst


@pytest.mark.parametrize("fuse", [True, False], ids=["fused", "unfused"])
@pytest.mark.parametrize("n", [1, 2])
def test_real_model_fp32_every_op_matches_oracle(segm, n, fuse):
    """Each of the 44 ops (each fused block as one launch), fed the oracle's
    values of its inputs, matches the oracle's output to 1e-4 (the per-op bar);
    the whole graph run end to end stays within 1e-3 of the oracle on every
    stored tensor (the per-op rounding differences accumulate through up to
    44 chained ops)."""
    data, graph = segm
    x = rnd(50 + n, n, 160, 288, 3)
    want = graph.run({"input_1": x}, n=n, keep_all=True)
    m = sw.SwModel(data, n=n, fuse=fuse)
    assert m.inputs == ["input_1"] and m.outputs == ["segment"]
    pairs = _check_fused(m, fuse)
    worst_op = _check_launches(m, graph, want, 1e-4)
    m.upload_input("input_1", x)
    m.infer()
    worst = max(G.rel_err(m.read_output(nm), w) for nm, w in want.items() if _stored(m, graph, nm))
    e_out = G.rel_err(m.read_output(), want["segment"])
    print(f"segm n={n} fuse={fuse} (pairs {pairs}): worst per-op {worst_op:.2e}, end to end: output {e_out:.2e}, "
          f"worst tensor {worst:.2e}", flush=True)
    assert worst <= 1e-3 and e_out <= 1e-3
    # a second frame through the device upload path reuses every buffer
    x2 = rnd(60 + n, n, 160, 288, 3)
    m.upload_input("input_1", torch.from_numpy(x2).cuda())
    m.infer()
    assert G.rel_err(m.read_output(), graph.run({"input_1": x2}, n=n)["segment"]) <= 1e-3
    m.close()


@pytest.mark.parametrize("fuse", [True, False], ids=["fused", "unfused"])
@pytest.mark.parametrize("dt", [F16, BF16], ids=["f16", "bf16"])
def test_real_model_16bit_every_op_matches_stored_dtype_oracle(segm, dt, fuse):
    """16-bit storage (weights converted at load): each op (each fused block
    as one launch), fed the values of the oracle run with the same storage
    rounding (weights, input and every op output rounded to dt), within 2e-2
    of that run's output. End to end, 44 ops of 16-bit rounding accumulate
    (bf16 keeps 8 mantissa bits): the segmentation mask (argmax of the two
    logits) agrees with the fp32 run on >= 99% of pixels, f16's logits stay
    within the ideal-storage distance + 5e-2 (measured 4.7e-2 against fp32);
    the distances are printed."""
    data, graph = segm
    n = 2
    x = rnd(70, n, 160, 288, 3)
    m = sw.SwModel(data, n=n, dt=conv.DType(dt), fuse=fuse)
    assert m.dt == dt
    blocks = m.fused_blocks()
    _check_fused(m, fuse)
    if fuse:
        print(f"segm dt{dt} fused blocks: " + ", ".join(f"ops {f.first_op}-{f.first_op + 2} {f.plan}" for f in blocks),
              flush=True)
    stored = so.SwGraph(data, round_dt=dt).run({"input_1": x}, n=n, keep_all=True)
    worst = _check_launches(m, graph, stored, 2e-2)
    m.upload_input("input_1", x)
    m.infer()
    got = m.read_output("segment")
    want32 = graph.run({"input_1": x}, n=n)["segment"]
    e_st = G.rel_err(got, stored["segment"])
    e32 = G.rel_err(got, want32)
    e_ideal = G.rel_err(stored["segment"], want32)  # ideal storage alone
    # what the model delivers: the per-pixel class (argmax of the 2 logits)
    agree = float(np.mean(got.argmax(-1) == want32.argmax(-1)))
    print(f"segm dt{dt} fuse={fuse}: worst per-op {worst:.2e}; end to end vs stored-dtype oracle {e_st:.2e}, "
          f"vs fp32 {e32:.2e} (ideal storage {e_ideal:.2e}), mask agreement {agree:.5f}", flush=True)
    assert agree >= 0.99
    if dt == F16:
        # measured: 4.7e-2 fused, 4.9e-2 unfused against fp32
        assert e32 <= e_ideal + 5e-2, (e32, e_ideal)


def _tile_batch(ref, reps):
    """A batch of `reps` copies of each reference tensor's images, in order
    (image i of the tiled batch is image i % n of the reference)."""
    return {k: np.concatenate([v] * reps) for k, v in ref.items()}


@pytest.mark.parametrize("dt", [F32, F16], ids=["f32", "f16"])
def test_real_model_batch64_every_launch(segm, dt):
    """The real model at batch 64 through aih_model_load, as the bench times
    it: fused as loaded by default -- also the depthwise -> pointwise pairs
    that batch 64 fuses (ops 33-34 and 40-41) and the resize folded into the
    concat (ops 38-39); 33 launches -- and every launch fed
    the oracle's values of its inputs against the oracle's output (fp32: 1e-4
    against the fp32 graph; f16: 2e-2 against the graph run with the same
    storage rounding). The batch is two oracle images repeated 32 times
    (images never interact), so all 64 are checked at the cost of two."""
    data, graph = segm
    n, base = 64, 2
    x2 = rnd(90, base, 160, 288, 3)
    x = np.concatenate([x2] * (n // base))
    m = sw.SwModel(data, n=n, dt=None if dt == F32 else conv.DType(dt))
    pairs = _check_fused(m, True)
    assert sorted(pairs) == sorted(SEGM_PAIRS) and m.info.n_launches == 33, (pairs, m.info.n_launches)
    for f in m.fused_blocks():
        if f.kind == sw.FUSED_DWPW:
            print(f"segm b64 dt{dt} pair ops {f.first_op}-{f.first_op + 1}: {f.dwpw}", flush=True)
    ref = graph if dt == F32 else so.SwGraph(data, round_dt=dt)
    want = _tile_batch(ref.run({"input_1": x2}, n=base, keep_all=True), n // base)
    worst = _check_launches(m, graph, want, 1e-4 if dt == F32 else 2e-2)
    m.upload_input("input_1", x)
    m.infer()
    e_out = G.rel_err(m.read_output(), want["segment"])
    print(f"segm b64 dt{dt}: {m.info.n_launches} launches, worst per launch {worst:.2e}, end to end {e_out:.2e}",
          flush=True)
    if dt == F32:
        assert e_out <= 1e-3
    m.close()


def test_tensor_storage_and_info(segm):
    data, graph = segm
    m = sw.SwModel(data, n=3)
    t = m.tensor("input_1")
    assert (t.n, t.h, t.w, t.c, t.stride_c, t.dt) == (3, 160, 288, 3, 4, 0)
    assert t.bytes == 3 * 160 * 288 * 4 * 4 and t.data
    seg = m.tensor("segment")  # an alias of the last resize's output
    assert (seg.h, seg.w, seg.c, seg.stride_c) == (160, 288, 2, 4)
    # four fused blocks, the resize folded into the concat (and at this batch fp32 depthwise -> pointwise
    # pairs): 44 ops in 35 launches less one per pair
    npairs = len(_check_fused(m, True))
    assert m.info.n_ops == 44 and m.info.n_fused == 5 + npairs and m.info.n_launches == 35 - npairs
    assert m.info.device_bytes > 0
    # a fused block's intermediates are never stored; ranges keep blocks whole
    inner = graph.T[graph.g["ops"][12]["out"]]["name"]
    for call in (lambda: m.read_output(inner), lambda: m.tensor(inner),
                 lambda: m.write_tensor(inner, np.zeros(3 * 10 * 18 * 96, np.float32))):
        with pytest.raises(conv.AihError, match="stays inside the fused block of ops 12..14"):
            call()
    for a, b in [(13, 15), (12, 13), (0, 14)]:
        with pytest.raises(conv.AihError, match="inside the fused block"):
            m.infer_range(a, b)
    # the resize folded into the concat after it: its output is never stored either
    rs = graph.T[graph.g["ops"][38]["out"]]["name"]
    with pytest.raises(conv.AihError, match="stays inside the fused block of ops 38..39"):
        m.read_output(rs)
    with pytest.raises(conv.AihError, match="inside the fused block"):
        m.infer_range(38, 39)
    m.infer_range(38, 40)  # the whole fold runs
    unfused = sw.SwModel(data, n=3, fuse=False)
    assert unfused.info.n_fused == 0 and unfused.info.n_launches == 44
    assert unfused.tensor(inner).c == 96
    assert unfused.info.device_bytes > m.info.device_bytes  # the intermediates are not allocated
    unfused.close()
    with pytest.raises(conv.AihError, match="no input named"):
        m.upload_input("nope", np.zeros(3, np.float32))
    with pytest.raises(conv.AihError, match="expected"):
        m.upload_input("input_1", np.zeros(7, np.float32))
    m.reset()
    m.close()


def test_synthetic_chain_through_the_native_loader(orc):
    from ai_engine_amd.workloads import Layer, _chain, make_weights

    layers = _chain([Layer("stem", 3, 32, k=3, s=2, act="relu"), Layer("e", 32, 128, act="relu"),
                     Layer("d", 128, 128, k=3, groups=128, act="relu"), Layer("p", 128, 32, res="stem"),
                     Layer("e2", 32, 128, act="relu6"), Layer("d2", 128, 128, k=3, s=2, groups=128, act="relu"),
                     Layer("p2", 128, 64), Layer("head", 64, 2)], 40, 72)
    wts = make_weights(layers, seed=9)
    data = sw.conv_graph_to_sw("chain", layers, wts, 40, 72, 3)
    n = 3
    x = rnd(80, n, 40, 72, 3)
    want = so.SwGraph(data).run({"input": x}, n=n)["head"]
    for fuse, blocks in [(True, [1, 4]), (False, [])]:
        m = sw.SwModel(data, n=n, fuse=fuse)
        assert [f.first_op for f in m.fused_blocks()] == blocks
        m.upload_input("input", x)
        m.infer()
        assert G.rel_err(m.read_output(), want) <= 1e-4
        m.close()


def test_depthwise_pointwise_pair_through_the_native_loader(orc):
    """An fp32 depthwise 3x3 whose output only the next 1x1 conv reads runs
    with it as one aih_conv_dwpw launch when the plan has a tile per CU
    (80x144 at batch 12), and not at batch 1 (180 tiles of 4x16 at most); the
    depthwise output is then never stored; results within 1e-4 of the
    oracle's graph run either way, each launch and end to end; a 16-bit load
    of the same file fuses the pair too, within the 16-bit per-launch bar."""
    from ai_engine_amd.workloads import Layer, _chain, make_weights

    layers = _chain([Layer("stem", 3, 32, k=3, s=2, act="relu"), Layer("d", 32, 32, k=3, groups=32, act="relu"),
                     Layer("p", 32, 24, act="relu"), Layer("head", 24, 2)], 160, 288)
    wts = make_weights(layers, seed=12)
    data = sw.conv_graph_to_sw("pair", layers, wts, 160, 288, 3)
    graph = so.SwGraph(data)
    for n, pairs in [(12, [(1, 2)]), (1, [])]:
        x = rnd(82 + n, n, 160, 288, 3)
        want = graph.run({"input": x}, n=n, keep_all=True)
        m = sw.SwModel(data, n=n)
        blocks = m.fused_blocks()
        assert [(f.first_op, f.n_ops) for f in blocks] == pairs
        if pairs:
            assert blocks[0].dwpw.tiles >= 256 and m.info.n_launches == 3
            with pytest.raises(conv.AihError, match="stays inside the fused block of ops 1..2"):
                m.read_output("d")
            with pytest.raises(conv.AihError, match="inside the fused block"):
                m.infer_range(2, 4)
        worst = _check_launches(m, graph, want, 1e-4)
        m.upload_input("input", x)
        m.infer()
        e = G.rel_err(m.read_output(), want["head"])
        print(f"dw->pw pair n={n} fused={bool(pairs)}: per launch {worst:.2e}, end to end {e:.2e}", flush=True)
        assert e <= 1e-4
        m.close()
    m16 = sw.SwModel(data, n=12, dt=conv.DType.F16)
    assert [(f.first_op, f.n_ops) for f in m16.fused_blocks()] == [(1, 2)]
    x = rnd(95, 12, 160, 288, 3)
    worst = _check_launches(m16, graph, so.SwGraph(data, round_dt=1).run({"input": x}, n=12, keep_all=True), 2e-2)
    print(f"dw->pw pair f16 n=12: per launch {worst:.2e}", flush=True)
    m16.close()


def test_fusion_needs_single_readers(orc):
    """An expand output that a second op also reads keeps its block unfused
    (the tensor must be stored); the next block still fuses. Results as the
    oracle's either way."""
    from ai_engine_amd.workloads import Layer, _chain, make_weights

    layers = _chain([Layer("stem", 3, 32, k=3, s=2, act="relu"), Layer("e", 32, 128, act="relu"),
                     Layer("d", 128, 128, k=3, groups=128, act="relu"), Layer("p", 128, 32, res="stem"),
                     Layer("side", 128, 32, src="e", res="p"),
                     Layer("e2", 32, 64, act="relu6"), Layer("d2", 64, 64, k=3, groups=64, act="relu6"),
                     Layer("p2", 64, 32, res="side"), Layer("head", 32, 2)], 24, 40)
    wts = make_weights(layers, seed=11)
    data = sw.conv_graph_to_sw("side", layers, wts, 24, 40, 3)
    n = 2
    x = rnd(81, n, 24, 40, 3)
    want = so.SwGraph(data).run({"input": x}, n=n)["head"]
    m = sw.SwModel(data, n=n)
    assert [f.first_op for f in m.fused_blocks()] == [5]
    assert m.tensor("e").c == 128  # stored: "side" reads it
    m.upload_input("input", x)
    m.infer()
    assert G.rel_err(m.read_output(), want) <= 1e-4
    m.close()


@pytest.mark.parametrize("dt", [F16, BF16], ids=["f16", "bf16"])
def test_encoder_through_the_native_loader_tuned(dt):
    """The headline encoder written as the converter's .sw and loaded by
    aih_model_load_ex with AIH_MODEL_TUNE (each fused block's launch options
    timed at load): all ten inverted-residual blocks fuse, the first one with
    the stem conv before it and the last one with the head after it where the
    timing picks that (the stem reading the staged fp32 upload either way),
    and the output equals bit for bit that of the op-level Model
    (ai_engine_amd.model) told to run the same kernels -- whose launches the
    oracle checks in test_gpu_workloads / test_gpu_ir_tiles / test_gpu_ir_stem
    / test_gpu_ir_head. Batch 8."""
    from ai_engine_amd import workloads as W
    from ai_engine_amd.model import Model

    n = 8
    layers, meta = W.mnv4_small_encoder_160x288(n)
    wts = W.make_weights(layers, seed=0)
    data = sw.conv_graph_to_sw("mnv4_small_encoder_160x288", layers, wts, meta["h"], meta["w"], 3)
    x = torch.from_numpy(rnd(91, n, meta["h"], meta["w"], 3)).cuda()
    m = sw.SwModel(data, n=n, dt=conv.DType(dt), tune=True)
    blocks = m.fused_blocks()
    ns = [f.n_ops for f in blocks]
    # 32 ops: the stem, ten blocks of three, the head; 12 launches, one less
    # for a joined stem (record from op 0) and for a joined head (from op 28)
    assert len(ns) == 10 and ns[1:-1] == [3] * 8 and ns[0] in (3, 4) and ns[-1] in (3, 4), ns
    assert blocks[0].first_op == (0 if ns[0] == 4 else 1) and blocks[-1].first_op == 28, blocks
    assert m.info.n_launches == 12 - (ns[0] - 3) - (ns[-1] - 3), (ns, m.info.n_launches)
    choices = {f"b{i}": (Model.STEM_PREFIX if f.n_ops == 4 and f.first_op == 0 else "")
               + Model.label_of(f.plan.kernel, f.plan.th, f.plan.tw, bool(f.plan.resident), f.plan.waves)
               + (Model.HEAD_SUFFIX if f.n_ops == 4 and f.first_op != 0 else "")
               for i, f in enumerate(blocks)}
    print(f"native tuned choices dt{dt}: {choices}", flush=True)
    m.upload_input("input", x)
    m.infer()
    got = np.ravel(m.read_output())
    ref = Model(layers, wts, n, meta["h"], meta["w"], 3, dt=conv.DType(dt), choices=choices)
    ref.upload_input(x)
    ref.infer()
    want = np.ravel(ref.read_output())
    assert np.array_equal(got, want), float(np.max(np.abs(got - want)))
    # the stored input slot, packed on demand, equals the op-level model's
    assert np.array_equal(np.ravel(m.read_output("input")), np.ravel(ref.read_output("input")))
    m.close()


def test_projection_reading_its_input_twice_stays_unfused(orc):
    """A projection whose residual is its own input (the depthwise output,
    cin == cout) reads that tensor through two slots: it counts as two
    readers, so neither the inverted-residual rule nor the depthwise ->
    pointwise rule may fuse it away (the residual would have no buffer).
    The graph loads unfused and matches the oracle."""
    from ai_engine_amd.workloads import Layer, _chain, make_weights

    layers = _chain([Layer("stem", 3, 32, k=3, s=2, act="relu"), Layer("e", 32, 128, act="relu"),
                     Layer("d", 128, 128, k=3, groups=128, act="relu"), Layer("p", 128, 128, res="d"),
                     Layer("head", 128, 2)], 48, 80)
    wts = make_weights(layers, seed=13)
    data = sw.conv_graph_to_sw("selfres", layers, wts, 48, 80, 3)
    n = 2
    x = rnd(84, n, 48, 80, 3)
    want = so.SwGraph(data).run({"input": x}, n=n)["head"]
    for dt in (None, conv.DType.F16):
        m = sw.SwModel(data, n=n, dt=dt)
        assert m.fused_blocks() == []
        assert m.tensor("d").c == 128
        m.upload_input("input", x)
        m.infer()
        e = G.rel_err(m.read_output(), want)
        print(f"self-residual projection dt={dt}: {e:.2e}", flush=True)
        assert e <= (1e-4 if dt is None else 5e-2)
        m.close()


def test_model_load_rejects_what_it_cannot_run(segm):
    """aih_model_load returns NULL with a message (no device work) for graphs
    it cannot run: an unsupported op kind, a weight reference outside the
    blob, a 16-bit file asked to widen, a zero batch."""
    from oracle import sw_oracle

    data, _ = segm
    g, blob = sw_oracle.read_container(data)
    bad = json_copy(g)
    bad["ops"].append({"kind": "maxpool", "in": 44, "out": 45, "kh": 2, "kw": 2, "sh": 2, "sw": 2, "pad": [0] * 4})
    with pytest.raises(conv.AihError, match="maxpool"):
        sw.SwModel(sw.write_container(bad, blob))
    bad = json_copy(g)
    bad["ops"][0]["w"]["off"] = len(blob)
    with pytest.raises(conv.AihError, match="outside the blob"):
        sw.SwModel(sw.write_container(bad, blob))
    bad = json_copy(g)
    bad["dt_default"] = "f16"
    for t in bad["tensors"]:
        t["dt"] = "f16"
    with pytest.raises(conv.AihError, match="fp32 file"):
        sw.SwModel(sw.write_container(bad, blob), dt=conv.DType.BF16)
    with pytest.raises(conv.AihError, match="n must be"):
        sw.SwModel(data, n=0)


def json_copy(g):
    import json

    return json.loads(json.dumps(g))

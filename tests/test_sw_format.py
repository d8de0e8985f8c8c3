"""CPU checks of the .sw path (no device): the container and graph readers --
the native one behind aih_sw_describe and the oracle's -- on the reference
converter's real output (tests/golden/segm_r11_160x288.sw), the reference's
own format tests (crates/ai-core/src/format/model.rs:321-401: round trip,
alias chains, bad magic / version, unknown fields ignored), and the weights:
unpacking each conv's weight reference reproduces the ONNX twin's
initializer bit for bit (golden hashes from tests/golden/make_segm_fixture.py),
and the product's packing functions rebuild the converter's bytes exactly.
"""
import hashlib
import json
import os
import struct

import numpy as np
import pytest

from ai_engine_amd import conv, sw

HERE = os.path.dirname(os.path.abspath(__file__))
SEGM = os.path.join(HERE, "golden", "segm_r11_160x288.sw")
ONNX_CONVS = os.path.join(HERE, "golden", "segm_r11_onnx_convs.json")


@pytest.fixture(scope="module")
def segm():
    return open(SEGM, "rb").read()


def test_native_reader_summarises_the_real_model(segm):
    d = sw.describe(segm)
    assert d["name"] == "segm-r11" and (d["h"], d["w"]) == (160, 288)
    assert d["dt_default"] == "f32" and d["dt_weights"] == "f32"
    assert (d["tensors"], d["aliases"], d["inputs"], d["outputs"]) == (46, 1, 1, 1)
    assert (d["ops"], d["conv"], d["resize"], d["binary"], d["gpool"], d["concat"]) == (44, 36, 4, 2, 1, 1)
    assert d["json_bytes"] == 11939
    assert d["blob_bytes"] == len(segm) - 12032  # JSON end 32 + 11939 rounded up to 256


def test_oracle_reader_agrees(orc, segm):
    from oracle import sw_oracle

    g, blob = sw_oracle.read_container(segm)
    assert len(g["ops"]) == 44 and len(g["tensors"]) == 46
    assert len(blob) == sw.describe(segm)["blob_bytes"]
    # op 0 is the stem: 160x288 3->32 k3 s2 ReLU, kg_pad 4, w.len = 9*4*8*64 (pack.rs:95)
    op0 = g["ops"][0]
    assert (op0["cin"], op0["cout"], op0["kh"], op0["sh"], op0["act"], op0["kg_pad"]) == (3, 32, 3, 2, "relu", 4)
    assert op0["w"]["len"] == 9 * 4 * 8 * 64
    # every weight reference is 256-aligned inside the blob (header.rs:19-22)
    for op in (o for o in g["ops"] if o["kind"] == "conv"):
        for key in ("w", "b"):
            if key in op:
                assert op[key]["off"] % 256 == 0 and op[key]["off"] + op[key]["len"] <= len(blob)


def test_unpacked_weights_match_the_onnx_twin(orc, segm):
    from oracle import sw_oracle

    golden = json.load(open(ONNX_CONVS))["convs"]
    g = sw_oracle.SwGraph.__new__(sw_oracle.SwGraph)
    g.g, g.blob = sw_oracle.read_container(segm)
    convs = [op for op in g.g["ops"] if op["kind"] == "conv"]
    assert len(convs) == len(golden) == 36
    for op, gd in zip(convs, golden):
        w, b = g.conv_weights(op)
        shape = tuple(gd["shape"])
        assert (op["cout"], op["cin"] // op["groups"], op["kh"], op["kw"]) == shape
        assert hashlib.sha256(np.ascontiguousarray(w.reshape(shape), np.float32).tobytes()).hexdigest() == \
            gd["weight_sha256"], gd["weight"]
        assert hashlib.sha256(np.ascontiguousarray(b, np.float32).tobytes()).hexdigest() == gd["bias_sha256"]
        assert list(op["pad"]) == gd["pads"] and [op["sh"], op["sw"]] == gd["strides"]
        assert op["groups"] == gd["group"]


def test_product_packing_rebuilds_the_converter_bytes(orc, segm):
    """pack(unpack(blob)) == blob for every conv: the product's packing
    functions write exactly what the reference's converter wrote."""
    from oracle import sw_oracle

    g = sw_oracle.SwGraph.__new__(sw_oracle.SwGraph)
    g.g, g.blob = sw_oracle.read_container(segm)
    for op in (o for o in g.g["ops"] if o["kind"] == "conv"):
        w, b = g.conv_weights(op)
        if op["groups"] > 1:
            wp = conv.pack_weights_dw(w, op["cout"], op["kh"], op["kw"])
        else:
            wp, kgp = conv.pack_weights_conv(w, op["cout"], op["cin"], op["kh"], op["kw"], 4)
            assert kgp == op["kg_pad"]
        bp = conv.pack_bias(b, op["cout"])
        assert wp.tobytes() == g.blob[op["w"]["off"]:op["w"]["off"] + op["w"]["len"]]
        assert bp.tobytes() == g.blob[op["b"]["off"]:op["b"]["off"] + op["b"]["len"]]


# ---- format/model.rs:321-401, restated on a tiny model ----

def tiny_graph():
    return dict(name="t", size=dict(h=4, w=4), dt_default="f32", dt_weights=None,
                tensors=[dict(name="x", h=4, w=4, c=3, dt="f32", alias=None, last_use=0),
                         dict(name="y", h=4, w=4, c=8, dt="f32", alias=None, last_use=1),
                         dict(name="y_view", h=4, w=4, c=4, dt="f32", alias=dict(of=1, cg_off=1), last_use=1)],
                inputs=[0], outputs=[2], states=[], consts=[],
                ops=[{"kind": "conv", "in": 0, "out": 1, "res": None, "cin": 3, "cout": 8, "kh": 1, "kw": 1,
                      "sh": 1, "sw": 1, "pad": [0, 0, 0, 0], "d": 1, "groups": 1, "act": "relu",
                      "w": dict(off=0, len=512), "b": dict(off=512, len=32), "kg_pad": 4}])


def test_container_roundtrip_and_blob_alignment():
    blob = bytes([7]) * 544
    data = sw.write_container(tiny_graph(), blob)
    g, b2 = sw.read_container(data)
    assert g == json.loads(json.dumps(tiny_graph())) and b2 == blob
    assert (len(data) - len(blob)) % 256 == 0
    d = sw.describe(data)
    assert (d["tensors"], d["aliases"], d["ops"], d["conv"], d["blob_bytes"]) == (3, 1, 1, 1, 544)


def test_alias_chain_resolution(orc):
    from oracle import sw_oracle

    g = sw_oracle.SwGraph.__new__(sw_oracle.SwGraph)
    g.g, g.blob = sw_oracle.read_container(sw.write_container(tiny_graph(), bytes(544)))
    g.T = g.g["tensors"]
    assert g.resolve(2) == (1, 1) and g.resolve(0) == (0, 0)


def test_rejects_bad_magic_version_and_truncation():
    data = bytearray(sw.write_container(tiny_graph(), bytes(544)))
    bad = bytearray(data)
    bad[0] = ord("X")
    with pytest.raises(conv.AihError, match="magic"):
        sw.describe(bytes(bad))
    bad = bytearray(data)
    bad[4] = 99
    with pytest.raises(conv.AihError, match="version 99"):
        sw.describe(bytes(bad))
    with pytest.raises(conv.AihError, match="truncated"):
        sw.describe(bytes(data[:20]))
    with pytest.raises(conv.AihError, match="truncated"):
        sw.describe(bytes(data[:200]))


def test_unknown_json_fields_are_ignored():
    g = tiny_graph()
    g["future_field"] = {"x": 1}
    g["ops"][0]["another"] = [1, 2, 3]
    d = sw.describe(sw.write_container(g, bytes(544)))
    assert d["ops"] == 1 and d["conv"] == 1


def test_unsupported_op_kind_and_bad_references_fail_with_a_message():
    g = tiny_graph()
    g["ops"].append({"kind": "maxpool", "in": 1, "out": 2, "kh": 2, "kw": 2, "sh": 2, "sw": 2, "pad": [0] * 4})
    with pytest.raises(conv.AihError, match="maxpool"):
        sw.describe(sw.write_container(g, bytes(544)))
    g = tiny_graph()
    g["ops"][0]["out"] = 9
    with pytest.raises(conv.AihError, match="tensor 9"):
        sw.describe(sw.write_container(g, bytes(544)))
    g = tiny_graph()
    g["tensors"][1]["alias"] = dict(of=2, cg_off=0)
    with pytest.raises(conv.AihError, match="cycle"):
        sw.describe(sw.write_container(g, bytes(544)))


def test_json_strings_with_escapes():
    g = tiny_graph()
    g["name"] = "tést \"q\" \\ 中"
    d = json.loads(json.dumps(sw.describe(sw.write_container(g, bytes(544)))))
    assert d["name"] == g["name"]


# ---------------------------------------------------------------- load-time geometry checks (no device)

def _edited(segm, edit):
    from oracle import sw_oracle

    g, blob = sw_oracle.read_container(segm)
    g = json.loads(json.dumps(g))
    edit(g)
    return sw.write_container(g, blob)


def _first(g, kind, pred=lambda o: True):
    return next(o for o in g["ops"] if o["kind"] == kind and pred(o))


@pytest.mark.parametrize("what,edit,fragment", [
    ("conv output height", lambda g: g["tensors"][g["ops"][0]["out"]].__setitem__("h", 81), "but the conv makes"),
    ("conv output channels", lambda g: g["tensors"][g["ops"][0]["out"]].__setitem__("c", 31), "but the conv makes"),
    ("conv input channels", lambda g: g["ops"][1].__setitem__("cin", g["ops"][1]["cin"] + 4), "cin"),
    ("weight length", lambda g: g["ops"][0]["w"].__setitem__("len", g["ops"][0]["w"]["len"] - 256),
     "packed layout needs"),
    ("bias length", lambda g: g["ops"][0]["b"].__setitem__("len", 64), "bias of 64 bytes"),
    ("kg_pad", lambda g: _first(g, "conv", lambda o: o["cin"] > 8 and o["groups"] == 1).__setitem__("kg_pad", 1),
     "kg_pad"),
    ("residual shape", lambda g: _first(g, "conv", lambda o: o.get("res") is not None).__setitem__("res", 0),
     "residual"),
    ("resize size", lambda g: _first(g, "resize").__setitem__("oh", 7), "resize to"),
    ("gpool output", lambda g: g["tensors"][_first(g, "gpool")["out"]].__setitem__("h", 2), "gpool"),
    ("binary operand", lambda g: _first(g, "binary", lambda o: "tensor" in o["b"])["b"]["tensor"]
     .__setitem__("tid", 0), "binary"),
    ("concat parts", lambda g: _first(g, "concat")["parts"][0].__setitem__("c", 1), "concat"),
    ("conv parts", lambda g: _first(g, "conv", lambda o: bool(o.get("srcs")))["srcs"][0].__setitem__("c", 40),
     "concat parts"),
])
def test_describe_rejects_inconsistent_geometry(segm, what, edit, fragment):
    """A file whose op fields disagree with its tensors or weight ranges is
    rejected at load (aih_sw_describe runs the same checks as aih_model_load
    before any device work), with a message naming the op."""
    bad = _edited(segm, edit)
    with pytest.raises(conv.AihError) as e:
        sw.describe(bad)
    assert fragment in str(e.value) and ".sw: op" in str(e.value), (what, str(e.value))


def test_describe_rejects_oversized_integers(segm):
    """A number beyond 2^64 where an unsigned integer is expected is a clean
    rejection (its conversion is checked before it happens)."""
    bad = _edited(segm, lambda g: g["ops"][0]["w"].__setitem__("len", 1e30))
    with pytest.raises(conv.AihError, match="expected an unsigned integer"):
        sw.describe(bad)

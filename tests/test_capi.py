"""CPU checks of the C ABI (no kernel launches): the library loads and exports
every function include/aih_conv.h declares, the host packing matches the
oracle's restatement of ai-core pack.rs byte for byte, the variant policy
behaves as specified, and invalid descriptors fail with -1 and a message
instead of crashing (the reference FFI's contract, crates/ai-ffi/src/lib.rs:45-52)."""
import ctypes as C
import os
import re

import numpy as np
import pytest

from ai_engine_amd import conv

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    names = set()
    for h in sorted(os.listdir(os.path.join(ROOT, "include"))):
        if not h.endswith(".h"):
            continue
        text = open(os.path.join(ROOT, "include", h)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names |= set(re.findall(r"\b(aih_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


def test_library_exports_every_declared_function():
    from ai_engine_amd import sw

    L = sw.lib()
    declared = header_functions()
    assert len(declared) >= 33
    for name in declared:
        assert hasattr(L, name), name
    assert set(conv.EXPORTS) | set(sw.EXPORTS) == set(declared)
    assert b"gfx950" in L.aih_version()


@pytest.mark.parametrize("dt", [0, 1, 2], ids=["f32", "f16", "bf16"])
def test_host_packing_matches_oracle(orc, dt):
    n, h, w, c = 2, 3, 5, 7
    x = orc.xs32_fill(1, n * h * w * c)
    assert np.array_equal(conv.pack_nhwc(x, n, h, w, c, conv.DType(dt)), orc.pack_nhwc(x, n, h, w, c, dt))
    packed = orc.pack_nhwc(x, n, h, w, c, dt)
    assert np.array_equal(conv.unpack_nhwc(packed, n, h, w, c, conv.DType(dt)),
                          orc.unpack_nhwc(packed, n, h, w, c, dt))
    for cout, cin, kh, kw in [(10, 6, 3, 3), (160, 960, 1, 1), (32, 3, 3, 3), (5, 7, 2, 1)]:
        wt = orc.xs32_fill(2, cout * cin * kh * kw)
        a, ka = conv.pack_weights_conv(wt, cout, cin, kh, kw, 4, conv.DType(dt))
        b, kb = orc.pack_weights_conv(wt, cout, cin, kh, kw, 4, dt)
        assert ka == kb and np.array_equal(a, b)
    wd = orc.xs32_fill(3, 13 * 9)
    assert np.array_equal(conv.pack_weights_dw(wd, 13, 3, 3, conv.DType(dt)), orc.pack_weights_dw(wd, 13, 3, 3, dt))
    b = orc.xs32_fill(4, 13)
    assert np.array_equal(conv.pack_bias(b, 13, conv.DType(dt)), orc.pack_bias(b, 13, dt))


def pw_plan(n, m, cin, cout, dt=0, splitk=0, variant=0):
    return conv.GemmPwSpec(m=m, kg=-(-cin // 4), ng=-(-cout // 4), dt=conv.DType(dt), n=n, splitk=splitk,
                           variant=conv.Variant(variant)).plan()


def test_pw_policy_splits_small_m_large_k():
    # skinny 960 -> 160 at 10x18: 2 pixel tiles cannot fill 256 CUs -> split-K,
    # on chip in one dispatch: 16x16 output blocks, K over 16 wavefronts, no
    # workspace
    p = pw_plan(1, 180, 960, 160)
    assert p.variant == conv.Variant.SPLITK and p.splitk == 16 and (p.bm, p.bn) == (16, 16)
    assert p.grid == 12 * 10 and p.ws_bytes == 0
    # 100 outputs are not whole 16-channel blocks: the tiled GEMM splits K
    # through a workspace, at most 8 chunks
    p = pw_plan(1, 180, 960, 100)
    assert p.variant == conv.Variant.SPLITK and 1 < p.splitk <= 8 and p.bm == 128
    assert p.ws_bytes == p.splitk * 180 * 100 * 4
    # same layer at batch 256: 360 tiles, forced whole -> one tile per
    # workgroup over the whole K (the policy splits it in four, see below)
    p = pw_plan(256, 180, 960, 160, variant=conv.Variant.TILE)
    assert p.variant == conv.Variant.TILE and p.splitk == 1 and p.ws_bytes == 0
    assert p.bn == 160 and p.grid == 360
    # 1x1 32 -> 64 at 80x144: short K (32) and 64 output channels, but 360
    # blocks of 32 pixels are fewer than four per CU: 16x16 output blocks, one
    # wavefront each (2880), K whole in each, no workspace
    p = pw_plan(1, 11520, 32, 64)
    assert p.variant == conv.Variant.DIRECT and p.splitk == 1 and (p.bm, p.bn) == (16, 16)
    assert p.grid == 720 * 4 and p.ws_bytes == 0
    # the same at batch 64: the direct kernel, 32 pixels a wavefront
    p = pw_plan(64, 11520, 32, 64)
    assert p.variant == conv.Variant.DIRECT and p.bm == 32 and p.bn == 64 and p.grid == 2048
    # the tiled GEMM forced: K is one stage, nothing to split; 90 pixel tiles
    # cannot fill 256 CUs, so the columns are cut into two 32-wide tiles
    p = pw_plan(1, 11520, 32, 64, variant=conv.Variant.TILE)
    assert p.variant == conv.Variant.TILE and p.bn == 32 and p.grid == 180
    # one output channel group: the one-pixel-per-thread kernel
    p = pw_plan(1, 11520, 128, 2)
    assert p.variant == conv.Variant.ROWS and p.ws_bytes == 0


def test_pw_policy_agrees_with_reference_on_its_splitk_kats(orc):
    # wherever the reference splits K (Splitk) or reduces K across a workgroup
    # (Gemv) on its own KAT shapes (gemm_pw.rs:337-354), the MI355X policy
    # splits K as well; where it picks Small/Tiled with a short K, it does not
    for m, kg, ng in [(144, 240, 40), (144, 40, 240), (144, 168, 28), (576, 30, 10), (2304, 18, 6), (1, 144, 36)]:
        assert orc.ref_pw_variant(m, kg, ng) in ("Splitk", "Gemv")
        p = conv.GemmPwSpec(m=m, kg=kg, ng=ng).plan()
        assert p.variant == conv.Variant.SPLITK, (m, kg, ng, p)
    for m, kg, ng in [(36864, 6, 4), (36864, 1, 4), (512, 8, 8)]:
        assert orc.ref_pw_variant(m, kg, ng) == "Small"
        p = conv.GemmPwSpec(m=m, kg=kg, ng=ng).plan()
        assert p.variant in (conv.Variant.TILE, conv.Variant.DIRECT) and p.splitk == 1, (m, kg, ng, p)


def test_pw_policy_long_k_fp32_many_pixels():
    """fp32, K >= 256 and at least 8 wavefront units per CU: the LDS-streamed
    GEMM over the whole K (960 -> 160 at 10x18, batch 256: 480 tiles of
    96 x 160, no workspace)."""
    p = pw_plan(256, 180, 960, 160)
    assert p.variant == conv.Variant.TILE and p.splitk == 1 and (p.bm, p.bn, p.grid, p.ws_bytes) == (96, 160, 480, 0)
    p = pw_plan(256, 180, 256, 160)
    assert p.splitk == 1 and p.bm == 96
    # at 16 bit (HBM-bound) the tiled GEMM keeps K whole
    p = conv.GemmPwSpec(m=180, kg=240, ng=40, n=256, dt=conv.DType.F16).plan()
    assert p.splitk == 1 and p.bm == 128
    # too few pixels for eight units per CU: the tiled GEMM's policy decides
    assert pw_plan(8, 180, 960, 160).bm != 96


def test_tiled_policy_splits_long_k_fp32_partial_second_round():
    """The tiled GEMM with fp32, long K and tiles between one and two per CU
    takes four K chunks: a 3x3 256 -> 160 conv at 10x18, batch 256 (360
    tiles of 128 x 160)."""
    op = conv.ConvOp(ih=10, iw=18, cin=256, cout=160, kh=3, kw=3, pad=(1, 1, 1, 1), n=256)
    p = op.plan()
    assert p.variant == conv.Variant.SPLITK and p.splitk == 4 and p.grid == 1440


def test_forced_splitk_factor_is_honoured():
    # AUTO with a forced factor: the one-dispatch kernel with that many K
    # chunks (a power of two up to 16) where the shape allows it
    for s in (1, 4, 8):
        p = pw_plan(1, 180, 960, 160, splitk=s)
        assert p.splitk == s and p.bm == 16 and p.ws_bytes == 0
        assert p.variant == (conv.Variant.SPLITK if s > 1 else conv.Variant.DIRECT)
    # other factors, or AIH_VAR_SPLITK: the tiled GEMM with a workspace
    p = pw_plan(1, 180, 960, 160, splitk=3)
    assert p.splitk == 3 and p.bm == 128 and p.ws_bytes == 3 * 180 * 160 * 4
    p = pw_plan(1, 180, 960, 160, splitk=4, variant=conv.Variant.SPLITK)
    assert p.splitk == 4 and p.bm == 128 and p.ws_bytes == 4 * 180 * 160 * 4
    p = pw_plan(1, 180, 960, 160, variant=conv.Variant.TILE)
    assert p.splitk == 1


def test_igemm_policy():
    big = conv.ConvIgemmSpec(ih=160, iw=288, cin=16, cout=32, k=3, s=2, pad=(1, 1, 1, 1), n=32)
    assert big.out_hw() == (80, 144)
    # 3x3 with <= 64 outputs: the direct kernel, eight wavefronts of 32-pixel
    # blocks per workgroup, one workgroup per CU
    p = big.plan()
    assert p.variant == conv.Variant.DIRECT and p.bm == 32 and p.bn == 32 and p.grid == 256 and p.ws_bytes == 0
    big.variant = conv.Variant.TILE
    p = big.plan()
    assert p.variant == conv.Variant.TILE and p.bn == 32 and p.grid == 32 * 80 * 144 // 128
    deep = conv.ConvIgemmSpec(ih=9, iw=16, cin=128, cout=128, k=3, pad=(1, 1, 1, 1))
    assert deep.plan().variant == conv.Variant.SPLITK


def test_igemm_direct_route_limits():
    """Shapes the direct route leaves to the tiled GEMM: an odd kg count per
    part at 16-bit storage, more than 64 outputs, a forced variant, a 5x5
    kernel, more than 10 MFMA steps per tap, weights beyond 160 KB of LDS,
    mixed storage."""
    V, D = conv.Variant, conv.DType

    def variant(**kw):
        base = dict(ih=16, iw=16, cin=32, cout=32, k=3, pad=(1, 1, 1, 1))
        base.update(kw)
        return conv.ConvIgemmSpec(**base).plan().variant

    assert variant() == V.DIRECT
    assert variant(cin=12) == V.DIRECT
    assert variant(cin=12, dt=D.F16) != V.DIRECT
    assert variant(cin=160, dt=D.F16) == V.DIRECT
    assert variant(cin=168, dt=D.F16) != V.DIRECT
    assert variant(cin=80) == V.DIRECT
    assert variant(cin=84) != V.DIRECT
    assert variant(cin=72, cout=64) != V.DIRECT  # 9 x 9 x 2 x 64 x 16 B of weights > 160 KB
    assert variant(cout=64) == V.DIRECT
    assert variant(cout=68) != V.DIRECT
    assert variant(variant=V.TILE) == V.TILE
    assert variant(splitk=2) == V.SPLITK
    assert variant(k=5, pad=(2, 2, 2, 2)) != V.DIRECT
    assert variant(wdt=D.F16) != V.DIRECT
    assert variant(cin=72, srcs=[conv.SrcView(c=48), conv.SrcView(c=24)], dt=D.F16) == V.DIRECT
    assert variant(cin=72, srcs=[conv.SrcView(c=48), conv.SrcView(c=24)]) == V.DIRECT  # 6 + 3 fp32 steps per tap
    # the stem route: <= 3 channels, 32 or 64 outputs (4 wavefronts of 32 pixels per workgroup)
    stem = conv.ConvIgemmSpec(ih=160, iw=288, cin=3, cout=32, k=3, s=2, pad=(1, 1, 1, 1), n=64).plan()
    assert stem.variant == V.DIRECT and stem.bn == 32 and stem.grid == 2048 and stem.ws_bytes == 0


def _expect_error(fn, fragment):
    with pytest.raises(conv.AihError) as e:
        fn()
    assert fragment in str(e.value)


def test_resize_rejects_bad_descriptors_before_the_device():
    """aih_resize / aih_resize_concat check the descriptor on the host; every
    call here passes no buffers at all, so none can reach a launch."""
    from ai_engine_amd import sw

    L = sw.lib()
    assert L.aih_resize_concat(None, None, None, None) == -1 and "null descriptor" in conv.last_error()
    assert L.aih_resize(None, None, None, None) == -1 and "null descriptor" in conv.last_error()

    def rc(**kw):
        f = dict(n=1, ih=4, iw=4, oh=8, ow=8, mode=0, dt=1, nparts=1, resized=1)
        f.update(kw)
        d = sw._ResizeConcat(f["n"], f["ih"], f["iw"], f["oh"], f["ow"], f["mode"], f["dt"], f["nparts"],
                             f["resized"], sw._srcs([(8, 8, 0)]))
        assert L.aih_resize_concat(C.byref(d), None, None, None) == -1
        return conv.last_error()

    assert "unknown dtype" in rc(dt=7)
    assert "zero-sized dimension" in rc(n=0)
    assert "below 2^24" in rc(ow=1 << 24)
    assert "unknown mode" in rc(mode=3)
    assert "null or misaligned output" in rc()
    d = sw._Resize(1, 4, 4, 8, 8, 0, 1, 1, sw._srcs([(8, 8, 0)]))
    assert L.aih_resize(C.byref(d), None, None, None) == -1 and "resize: null or misaligned output" in conv.last_error()


def test_invalid_descriptors_fail_cleanly():
    L = conv.lib()
    assert L.aih_conv_pw(None, None, None, None, None, None, None, 0, None) == -1
    assert "null descriptor" in conv.last_error()
    _expect_error(lambda: conv.GemmPwSpec(m=0, kg=1, ng=1).plan(), "must be > 0")
    _expect_error(lambda: conv.GemmPwSpec(m=4, kg=2, ng=1, kg_pad=1).plan(), "kg_pad")
    _expect_error(lambda: conv.GemmPwSpec(m=4, kg=2, ng=1, dt=conv.DType.F16, wdt=conv.DType.F32).plan(),
                  "unsupported (dt, wdt)")
    _expect_error(lambda: conv.GemmPwSpec(m=4, kg=2, ng=1, act=42).plan(), "activation")
    # null buffers are rejected before anything reaches the device
    _expect_error(lambda: conv.GemmPwSpec(m=4, kg=2, ng=1).run(None, None, None, None, None, stream=0), "null buffer")
    _expect_error(lambda: conv.GemmPwSpec(m=4, kg=2, ng=1, residual=True).run(16, 16, 16, None, 16, stream=0),
                  "res must be given")
    # lower_op's rejections (lowering.rs:136-140, conv_igemm.rs:80-83)
    op = conv.ConvOp(ih=8, iw=8, cin=4, cout=4, kh=1, kw=1, sh=2, sw=2)
    _expect_error(lambda: op.run(16, 16, 16, None, 16, stream=0), "1x1 conv with stride/pad")
    op = conv.ConvOp(ih=8, iw=8, cin=4, cout=4, kh=3, kw=1, pad=(1, 0, 1, 0))
    _expect_error(lambda: op.run(16, 16, 16, None, 16, stream=0), "square kernels")
    op = conv.ConvOp(ih=8, iw=8, cin=8, cout=16, kh=3, kw=3, groups=8)
    _expect_error(lambda: op.run(16, 16, 16, None, 16, stream=0), "depthwise")
    ig = conv.ConvIgemmSpec(ih=8, iw=8, cin=12, cout=8, k=3, pad=(1, 1, 1, 1),
                            srcs=[conv.SrcView(c=6), conv.SrcView(c=6)])
    _expect_error(lambda: ig.plan(), "only the last part")
    ig = conv.ConvIgemmSpec(ih=8, iw=8, cin=12, cout=8, k=3, pad=(1, 1, 1, 1),
                            srcs=[conv.SrcView(c=8), conv.SrcView(c=8)])
    _expect_error(lambda: ig.plan(), "do not add up")
    ig = conv.ConvIgemmSpec(ih=2, iw=2, cin=4, cout=4, k=5)
    _expect_error(lambda: ig.plan(), "larger than the padded input")
    # split-K without a workspace is an error, not a crash
    d = conv.GemmPwSpec(m=180, kg=240, ng=40, splitk=4, variant=conv.Variant.SPLITK).desc()
    assert L.aih_conv_pw(C.byref(d), 16, 16, 16, None, 16, None, 0, None) == -1
    assert "workspace" in conv.last_error()


# ---------------------------------------------------------------- fused inverted-residual block (plan only)

ENCODER_BLOCKS = [  # (n, ih, iw, cin, cexp, cout, s) of the 160x288 encoder's ten blocks, batch 64
    (64, 80, 144, 32, 128, 32, 1), (64, 80, 144, 32, 128, 32, 1), (64, 80, 144, 32, 128, 64, 2),
    (64, 40, 72, 64, 256, 64, 1), (64, 40, 72, 64, 256, 64, 1), (64, 40, 72, 64, 256, 96, 2),
    (64, 20, 36, 96, 384, 96, 1), (64, 20, 36, 96, 384, 96, 1), (64, 20, 36, 96, 384, 128, 2),
    (64, 10, 18, 128, 512, 128, 1),
]


@pytest.mark.parametrize("dt", [0, 1, 2], ids=["f32", "f16", "bf16"])
@pytest.mark.parametrize("blk", ENCODER_BLOCKS, ids=lambda b: "x".join(map(str, b)))
def test_ir_block_plan_covers_the_output_and_fits_lds(blk, dt):
    n, ih, iw, cin, cexp, cout, s = blk
    spec = conv.IrBlockSpec(ih=ih, iw=iw, cin=cin, cexp=cexp, cout=cout, s=s, n=n, dt=conv.DType(dt),
                            kernel=conv.IrKernel.TILE)
    p = spec.plan()
    assert p.kernel == conv.IrKernel.TILE
    oh, ow = spec.out_hw()
    tiles_y, tiles_x = -(-oh // p.th), -(-ow // p.tw)
    assert p.tiles == n * tiles_y * tiles_x
    assert 16 <= p.th * p.tw <= 256 and p.th <= oh and p.tw <= ow
    assert cexp % p.ec == 0 and p.ec % 32 == 0 and p.chunks == cexp // p.ec
    assert p.lds_bytes <= 160 * 1024 and p.occupancy >= 1
    assert 1 <= p.grid <= p.tiles
    # the LDS the kernel addresses: input tile with halo (rows padded by 16
    # bytes), expanded chunk, the packed expand / project / depthwise weights
    # and both biases of two chunks (or of all of E when they stay resident),
    # and the fp32 projection bias
    es = 4 if dt == 0 else 2
    wn = cexp if p.resident else 2 * p.ec
    halo = -(-(((p.th - 1) * s + 3) * ((p.tw - 1) * s + 3)) // 32) * 32
    need = halo * (cin * es + 16) + halo * (p.ec * es + 16) + wn * cin * es + wn * cout * es
    need += 11 * wn * es + cout * 4
    assert p.lds_bytes >= need


@pytest.mark.parametrize("dt", [1, 2], ids=["f16", "bf16"])
@pytest.mark.parametrize("blk", ENCODER_BLOCKS, ids=lambda b: "x".join(map(str, b)))
def test_ir_wave_plan_covers_the_output_and_fits_lds(blk, dt):
    """The wave kernel: tiles of at most 32 output pixels whose halo fits the
    instantiation's blocks, every tile covered, and the LDS it addresses --
    weight slots (all chunks or two), the fp32 projection bias, one expanded
    region of NPI x 32 pixels x 80 bytes per wavefront."""
    n, ih, iw, cin, cexp, cout, s = blk
    spec = conv.IrBlockSpec(ih=ih, iw=iw, cin=cin, cexp=cexp, cout=cout, s=s, n=n, dt=conv.DType(dt),
                            kernel=conv.IrKernel.WAVE)
    if not spec.fusable():
        _expect_error(spec.plan, "wave")
        return
    p = spec.plan()
    oh, ow = spec.out_hw()
    assert p.kernel == conv.IrKernel.WAVE and p.ec == 32 and p.chunks == cexp // 32
    assert p.th * p.tw <= 32 and p.th <= oh and p.tw <= ow
    assert p.tiles == n * -(-oh // p.th) * -(-ow // p.tw)
    halo = ((p.th - 1) * s + 3) * ((p.tw - 1) * s + 3)
    npi = 2 if halo <= 64 else 5
    assert halo <= npi * 32
    slot = 64 * cin + 64 * cout + 11 * 32 * 2
    weights = (cexp // 32 if p.resident else 2) * slot
    assert p.lds_bytes >= weights + cout * 4 + 2 * npi * 32 * 80 and p.lds_bytes <= 160 * 1024
    assert 1 <= p.grid <= p.tiles


def test_ir_block_rejects_unfusable_shapes():
    for kw in [dict(cin=12), dict(cexp=48), dict(cout=160), dict(cout=20), dict(s=3)]:
        base = dict(ih=8, iw=8, cin=32, cexp=128, cout=32, s=1, dt=conv.DType.F16)
        base.update(kw)
        spec = conv.IrBlockSpec(**base)
        assert not spec.fusable(), kw
        _expect_error(spec.plan, "ir_block")
    # fp32 needs cin % 8, 16-bit cin % 16
    assert conv.IrBlockSpec(ih=8, iw=8, cin=8, cexp=32, cout=32, dt=conv.DType.F32).fusable()
    assert not conv.IrBlockSpec(ih=8, iw=8, cin=8, cexp=32, cout=32, dt=conv.DType.F16).fusable()
    d = conv.IrBlockSpec(ih=8, iw=8, cin=32, cexp=128, cout=32, residual=True).desc()
    L = conv.lib()
    assert L.aih_ir_block(C.byref(d), 16, 16, 16, 16, 16, 16, 16, None, 16, None) == -1
    assert "res must be given" in conv.last_error()



def test_ir_block_head_plan_and_rejections():
    """The head joined to a block (aih_ir_block_head_plan): the block's split
    plan at the same tile and wavefronts plus the head's 8 KB of LDS (per
    16-pixel group and pixel, 16 lanes' four fp32 partial sums); what it
    does not take fails with the reason, and a null buffer fails before any
    launch."""
    import dataclasses
    F16 = conv.DType.F16
    blk = conv.IrBlockSpec(ih=10, iw=18, cin=128, cexp=512, cout=128, s=1, residual=True, dt=F16, n=64,
                           tile=(5, 6), waves=4, kernel=conv.IrKernel.SPLIT)
    head = conv.GemmPwSpec(m=180, kg=32, ng=1, dt=F16, n=64)
    assert head.plan().variant == conv.Variant.ROWS
    j, b = conv.IrBlockHeadSpec(blk, head).plan(), blk.plan()
    assert j.kernel == conv.IrKernel.SPLIT and (j.th, j.tw, j.waves, j.tiles) == (b.th, b.tw, b.waves, b.tiles)
    assert j.lds_bytes == b.lds_bytes + 2 * 16 * 16 * 16 and j.lds_bytes <= 160 * 1024
    # AUTO kernel: the head joins the split kernel
    a = conv.IrBlockHeadSpec(dataclasses.replace(blk, kernel=conv.IrKernel.AUTO, tile=(0, 0), waves=0), head).plan()
    assert a.kernel == conv.IrKernel.SPLIT
    bad = [
        (blk, dataclasses.replace(head, ng=2), "at most 4 outputs"),
        (blk, dataclasses.replace(head, kg=16), "kg = cout / 4"),
        (blk, dataclasses.replace(head, m=179), "same n and pixels"),
        (blk, dataclasses.replace(head, residual=True), "no residual"),
        (blk, dataclasses.replace(head, splitk=2), "narrow route"),
        (blk, dataclasses.replace(head, dt=conv.DType.BF16), "dt and wdt"),
        (dataclasses.replace(blk, kernel=conv.IrKernel.WAVE), head, "split kernel"),
        (dataclasses.replace(blk, cout=32, cin=32, cexp=128), dataclasses.replace(head, kg=8), "16 lanes"),
        (dataclasses.replace(blk, dt=conv.DType.F32), dataclasses.replace(head, dt=conv.DType.F32), "f16 or bf16"),
    ]
    for bb, hd, why in bad:
        _expect_error(conv.IrBlockHeadSpec(bb, hd).plan, why)
    L = conv.lib()
    assert L.aih_ir_block_head(C.byref(blk.desc()), C.byref(head.desc()), 16, 16, 16, 16, 16, 16, 16, 16, None,
                               16, 16, None, None) == -1
    assert "null buffer" in conv.last_error()

# ---------------------------------------------------------------- diagnostic overrides, forced placement

def _plan_in_subprocess(env: dict, code: str) -> str:
    """Runs `code` (printing its result) in a fresh interpreter with env set:
    the overrides are read once per process."""
    import os
    import subprocess
    import sys

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    e = dict(os.environ)
    e.update(env)
    r = subprocess.run([sys.executable, "-c", "import sys; sys.path.insert(0, %r)\n" % root + code],
                       capture_output=True, text=True, env=e, timeout=120)
    assert r.returncode == 0, r.stderr
    return r.stdout.strip()


PW_SPLITK_PROBE = (
    "from ai_engine_amd import conv\n"
    "p = conv.GemmPwSpec(m=180, kg=240, ng=40).plan()\n"
    "q = conv.GemmPwSpec(m=180, kg=240, ng=40, splitk=8).plan()\n"
    "print(p.splitk, q.splitk)\n")
IG_SPLIT_PROBE = (
    "from ai_engine_amd import conv\n"
    "s = conv.ConvIgemmSpec(ih=9, iw=16, cin=240, cout=96, k=3, pad=(1, 1, 1, 1))\n"
    "print(s.plan().splitk)\n")


def test_env_overrides_of_the_split_policy():
    # unset: the policy splits the skinny 960 -> 160 layer
    base = int(_plan_in_subprocess({"AIH_PW_SPLITK": ""}, PW_SPLITK_PROBE).split()[0])
    assert base > 1
    # AIH_PW_SPLITK forces the factor of AUTO calls; an explicit split still wins
    assert _plan_in_subprocess({"AIH_PW_SPLITK": "3"}, PW_SPLITK_PROBE).split() == ["3", "8"]
    assert _plan_in_subprocess({"AIH_PW_SPLITK": "1"}, PW_SPLITK_PROBE).split() == ["1", "8"]
    # malformed values are ignored
    assert int(_plan_in_subprocess({"AIH_PW_SPLITK": "x"}, PW_SPLITK_PROBE).split()[0]) == base
    # the override applies to every AUTO pointwise call, routed as a forced
    # split: a narrow head (one channel group) leaves its row kernel for the
    # tiled GEMM while it is set (the header documents this)
    narrow = ("from ai_engine_amd import conv\n"
              "p = conv.GemmPwSpec(m=180, kg=32, ng=1).plan()\n"
              "print(conv.Variant(p.variant).name, p.splitk)\n")
    assert _plan_in_subprocess({"AIH_PW_SPLITK": ""}, narrow).split()[0] == "ROWS"
    assert _plan_in_subprocess({"AIH_PW_SPLITK": "2"}, narrow).split() == ["SPLITK", "2"]
    # AIH_IGEMM_NO_SPLIT keeps a small-M, long-K 3x3 conv whole
    assert int(_plan_in_subprocess({"AIH_IGEMM_NO_SPLIT": ""}, IG_SPLIT_PROBE)) > 1
    assert int(_plan_in_subprocess({"AIH_IGEMM_NO_SPLIT": "1"}, IG_SPLIT_PROBE)) == 1


def test_ir_block_forced_weight_placement():
    base = dict(ih=40, iw=72, cin=64, cexp=256, cout=64, s=1, n=64, dt=conv.DType.F16)
    for tile in [(0, 0), (8, 8), (4, 16)]:
        r = conv.IrBlockSpec(tile=tile, weights=conv.IrWeights.RESIDENT, **base).plan()
        s = conv.IrBlockSpec(tile=tile, weights=conv.IrWeights.STREAMED, **base).plan()
        assert r.resident == 1 and s.resident == 0, tile
        if tile != (0, 0):
            assert (r.th, r.tw) == tile and (s.th, s.tw) == tile
        # streamed weights take two chunk slots; resident ones all of E
        assert r.lds_bytes > s.lds_bytes
    d = conv.IrBlockSpec(weights=7, **base).desc()
    p = conv.IrPlan()
    assert conv.lib().aih_ir_block_plan(C.byref(d), C.byref(p)) == -1
    assert "weight placement" in conv.last_error()


def test_ir_block_plan_depends_on_the_activations():
    """Clamp-type and other activations run different instantiations (with
    different register use): the plan cache keeps them apart."""
    A = conv.Activation
    base = dict(ih=40, iw=72, cin=64, cexp=256, cout=64, s=1, n=64, dt=conv.DType.F16)
    p1 = conv.IrBlockSpec(act_project=A.NONE, **base).plan()
    p2 = conv.IrBlockSpec(act_project=A.SIGMOID, **base).plan()
    p3 = conv.IrBlockSpec(act_project=A.NONE, **base).plan()
    assert (p1.th, p1.tw, p1.occupancy) == (p3.th, p3.tw, p3.occupancy)
    assert p1.occupancy >= 1 and p2.occupancy >= 1


def test_conv_plan_reports_the_route():
    A = conv.Activation
    pw = conv.ConvOp(ih=80, iw=144, cin=32, cout=64, act=A.RELU6, n=64)
    assert pw.plan().variant == conv.Variant.DIRECT
    assert conv.ConvOp(ih=10, iw=18, cin=960, cout=160).plan().variant == conv.Variant.SPLITK
    ig = conv.ConvOp(ih=40, iw=72, cin=32, cout=64, kh=3, kw=3, pad=(1, 1, 1, 1))
    assert ig.plan().variant == conv.Variant.DIRECT
    dw = conv.ConvOp(ih=40, iw=72, cin=32, cout=32, kh=3, kw=3, pad=(1, 1, 1, 1), groups=32)
    p = dw.plan()
    assert p.variant == conv.Variant.DIRECT and p.grid == 0 and p.ws_bytes == 0
    _expect_error(conv.ConvOp(ih=8, iw=8, cin=8, cout=8, sh=2, sw=2).plan, "stride/pad")


# ---------------------------------------------------------------- fused depthwise -> pointwise (host side)

@pytest.mark.parametrize("shape", [(40, 72, 256, 64, 1, 64), (80, 144, 44, 24, 1, 64), (20, 36, 96, 48, 2, 64),
                                   (7, 5, 20, 12, 1, 1), (19, 43, 52, 36, 2, 2)])
def test_dwpw_plan_covers_the_output_and_fits_lds(shape):
    """aih_conv_dwpw_plan's tiles cover the output, its LDS fits the CU, and
    the tile is a 16-column multiple of 2- or 4-row wavefronts (host only)."""
    ih, iw, c, cout, s, n = shape
    spec = conv.DwPwSpec(ih=ih, iw=iw, c=c, cout=cout, s=s, n=n)
    p = spec.plan()
    oh, ow = spec.out_hw()
    assert p.wave_rows in (2, 4) and p.tw % 16 == 0 and p.th % p.wave_rows == 0
    assert p.waves == (p.th // p.wave_rows) * (p.tw // 16) <= 8
    assert p.tiles == n * -(-oh // p.th) * -(-ow // p.tw) == p.grid
    assert p.chunks == -(-(-(-c // 4) * 4) // 16) and 0 < p.lds_bytes <= 160 * 1024


def test_dwpw_rejects_what_it_cannot_run():
    base = dict(ih=16, iw=16, c=32, cout=32)
    for kw, msg in [(dict(k=5), "3x3"), (dict(cout=80), "cout"),
                    (dict(s=3), "stride"), (dict(pad=(3, 1, 1, 1)), "padding"), (dict(kg_pad=4), "kg_pad"),
                    (dict(tile=(4, 48)), "forced tile"), (dict(tile=(6, 16)), "forced tile"),
                    (dict(rows=3), "forced tile")]:
        spec = conv.DwPwSpec(**{**base, **kw})
        assert not spec.fusable(), kw
        _expect_error(spec.plan, msg)
    d = conv.DwPwSpec(residual=True, **base).desc()
    assert conv.lib().aih_conv_dwpw(C.byref(d), 16, 16, 16, 16, 16, None, 16, None) == -1
    assert "res must be given" in conv.last_error()
    # 16-bit storage plans like fp32 (the same tiles and LDS bytes), with
    # 32-channel chunks
    for dt in (conv.DType.F16, conv.DType.BF16):
        p16, p32 = conv.DwPwSpec(dt=dt, **base).plan(), conv.DwPwSpec(**base).plan()
        assert (p16.th, p16.tw, p16.lds_bytes) == (p32.th, p32.tw, p32.lds_bytes)
        assert p16.chunks == 1 and p32.chunks == 2


def test_noalloc_rejects_workspace_beyond_scratch_on_the_host():
    # the size check of aih_conv_noalloc comes before any device call: on a
    # machine without a GPU the call still fails with the size in the message
    # (a 3x3 256 -> 160 fp32 conv at 10x18 batch 256: 118 MB of partial sums)
    L = conv.lib()
    op = conv.ConvOp(ih=10, iw=18, cin=256, cout=160, kh=3, kw=3, pad=(1, 1, 1, 1), n=256, dt=conv.DType.F32)
    need = op.workspace_bytes()
    assert need > 16 << 20, need
    d = op.desc()
    assert L.aih_conv_noalloc(C.byref(d), None, None, None, None, None, None) == -1
    assert str(need) in conv.last_error() and "scratch" in conv.last_error()

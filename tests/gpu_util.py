"""Helpers for the GPU parity tests: seeded inputs in the reference's stream
order, packing through the oracle (the converter's byte contract), NaN-poisoned
outputs, and the two error measures the reference uses."""
from __future__ import annotations

import numpy as np
import torch

from ai_engine_amd import conv
from oracle import oracle as orc

DEV = torch.device("cuda:0")
NP_DT = {0: np.float32, 1: np.uint16, 2: np.uint16}
POISON = {0: np.float32(np.nan).view(np.uint32), 1: 0x7E00, 2: 0x7FC0}


def stream(seed: int, *sizes: int) -> list[np.ndarray]:
    """XorShift32::new(seed) drawn in order into tensors of the given sizes."""
    flat = orc.xs32_fill(seed, int(sum(sizes)))
    out, o = [], 0
    for s in sizes:
        out.append(flat[o:o + s])
        o += s
    return out


def dev(a: np.ndarray) -> torch.Tensor:
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).to(DEV)
    return torch.from_numpy(a).to(DEV)


def poisoned(n_elems: int, dt: int) -> torch.Tensor:
    """Fresh output buffer filled with NaN (so unwritten elements cannot pass)."""
    if dt == 0:
        return torch.full((n_elems,), float("nan"), dtype=torch.float32, device=DEV)
    return torch.full((n_elems,), int(np.int16(np.uint16(POISON[dt]).view(np.int16))), dtype=torch.int16, device=DEV)


def host(t: torch.Tensor, dt: int) -> np.ndarray:
    a = t.detach().cpu().numpy()
    return a.view(np.uint16) if dt != 0 else a


def rel_err(got, want) -> float:
    """BASELINE metric (the reference's synthetic_e2e.rs:113-116 convention):
    max |gpu - cpu| / max(|cpu|, 1); NaN counts as infinite."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    if got.shape != want.shape:
        return float("inf")
    e = np.abs(got - want) / np.maximum(np.abs(want), 1.0)
    if np.isnan(e).any():
        return float("inf")
    return float(e.max(initial=0.0))


def testsuite_ok(got, want, atol, rtol) -> bool:
    """The reference GPU testsuite's compare (crates/ai-gpu/src/testsuite.rs:33-44)."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    return bool(np.all(np.abs(got - want) <= atol + rtol * np.abs(want)))


ACT = {name: conv.Activation(i) for name, i in orc.ACT.items()}


def rounded_ref(op, ih, iw, x, wts, b, r, dt, wdt, n=1):
    """fp32 reference on the inputs as stored in dt / wdt: separates the
    kernel's own error from the storage dtype's input quantisation."""
    return orc.conv2d_ref(op, ih, iw, orc.round_to(x, dt), orc.round_to(wts, wdt), orc.round_to(b, dt),
                          None if r is None else orc.round_to(r, dt), n=n)


def magnitude(op, ih, iw, x, wts, b, r, n=1):
    """sum |x||w| + |b| (+ |res|) per output: the scale of every rounding error
    that storing the inputs in a 16-bit dtype can introduce."""
    aop = orc.Conv2d.from_buffer_copy(op)
    aop.act = 0
    m = orc.conv2d_ref(aop, ih, iw, np.abs(x), np.abs(wts), np.abs(b), None, n=n)
    return m + (np.abs(r) if r is not None else 0.0)


class Result:
    def __init__(self, got, want, plan=None, want_r=None, mag=None):
        self.got, self.want, self.plan, self.want_r, self.mag = got, want, plan, want_r, mag

    def __iter__(self):  # (got, want, plan) unpacking
        return iter((self.got, self.want, self.plan))


def run_pw(h, w, cin, cout, act, residual, dt, seed, wdt=None, n=1, splitk=0, variant=0, xs=None, refs=True):
    """pw_case (testsuite.rs:325-371): returns Result(got, want, plan, want_r);
    refs=False skips the oracle (want, want_r, mag are None)."""
    wdt = dt if wdt is None else wdt
    if xs is None:
        x, wts, b, r = stream(seed, n * h * w * cin, cout * cin, cout, n * h * w * cout if residual else 0)
    else:
        x, wts, b, r = xs
    op = orc.conv2d(cin, cout, act=act)
    want = orc.conv2d_ref(op, h, w, x, wts, b, r if residual else None, n=n) if refs else None
    wp, kgp = orc.pack_weights_conv(wts, cout, cin, 1, 1, 4, wdt)
    xd = dev(orc.pack_nhwc(x, n, h, w, cin, dt))
    wd = dev(wp)
    bd = dev(orc.pack_bias(b, cout, dt))
    rd = dev(orc.pack_nhwc(r, n, h, w, cout, dt)) if residual else None
    ng = -(-cout // 4)
    yd = poisoned(n * h * w * ng * 4, dt)
    spec = conv.GemmPwSpec(m=h * w, kg=-(-cin // 4), ng=ng, act=ACT[act], residual=residual,
                           dt=conv.DType(dt), wdt=conv.DType(wdt), n=n, kg_pad=kgp,
                           variant=conv.Variant(variant), splitk=splitk)
    plan = spec.plan()
    spec.run(xd, wd, bd, rd, yd)
    torch.cuda.synchronize()
    got = orc.unpack_nhwc(host(yd, dt), n, h, w, cout, dt)
    if not refs:
        return Result(got, None, plan)
    rr = r if residual else None
    want_r = rounded_ref(op, h, w, x, wts, b, rr, dt, wdt, n) if (dt or wdt) else want
    mag = magnitude(op, h, w, x, wts, b, rr, n) if (dt or wdt) else None
    return Result(got, want, plan, want_r, mag)


def run_igemm(ih, iw, cin, cout, k, s, pad, act, residual, dt, seed, wdt=None, n=1, d=1, splitk=0, variant=0,
              parts=None, refs=True):
    """igemm_case / igemm_concat_case (testsuite.rs:588-720): returns Result
    (refs=False: no oracle)."""
    wdt = dt if wdt is None else wdt
    op = orc.conv2d(cin, cout, k=k, s=s, pad=list(pad), dil=d, act=act)
    oh, ow = orc.out_hw(op, ih, iw)
    if parts is None:
        x, wts, b, r = stream(seed, n * ih * iw * cin, cout * cin * k * k, cout,
                              n * oh * ow * cout if residual else 0)
        xin = x
        inputs = [dev(orc.pack_nhwc(x, n, ih, iw, cin, dt))]
        srcs = []
    else:
        assert n == 1
        sizes = [ih * iw * c for c in parts]
        vals = stream(seed, *sizes, cout * cin * k * k, cout, oh * ow * cout if residual else 0)
        pv, (wts, b, r) = vals[:len(parts)], vals[len(parts):]
        xin = np.concatenate([p.reshape(ih * iw, c) for p, c in zip(pv, parts)], axis=1).ravel()
        inputs = [dev(orc.pack_nhwc(p, 1, ih, iw, c, dt)) for p, c in zip(pv, parts)]
        srcs = [conv.SrcView(c=c) for c in parts]
    want = orc.conv2d_ref(op, ih, iw, xin, wts, b, r if residual else None, n=n) if refs else None
    wp, _ = orc.pack_weights_conv(wts, cout, cin, k, k, 4, wdt)
    wd = dev(wp)
    bd = dev(orc.pack_bias(b, cout, dt))
    rd = dev(orc.pack_nhwc(r, n, oh, ow, cout, dt)) if residual else None
    yd = poisoned(n * oh * ow * (-(-cout // 4)) * 4, dt)
    spec = conv.ConvIgemmSpec(ih=ih, iw=iw, cin=cin, cout=cout, k=k, s=s, d=d, pad=tuple(pad), act=ACT[act],
                              residual=residual, dt=conv.DType(dt), wdt=conv.DType(wdt), n=n,
                              variant=conv.Variant(variant), splitk=splitk, srcs=srcs)
    plan = spec.plan()
    spec.run(inputs, wd, bd, rd, yd)
    torch.cuda.synchronize()
    got = orc.unpack_nhwc(host(yd, dt), n, oh, ow, cout, dt)
    if not refs:
        return Result(got, None, plan)
    rr = r if residual else None
    want_r = rounded_ref(op, ih, iw, xin, wts, b, rr, dt, wdt, n) if (dt or wdt) else want
    mag = magnitude(op, ih, iw, xin, wts, b, rr, n) if (dt or wdt) else None
    return Result(got, want, plan, want_r, mag)


def run_dw(ih, iw, c, k, s, act, residual, dt, seed, pad=None, d=1, n=1, refs=True):
    """dw_case (testsuite.rs:416-464): returns Result (refs=False: no oracle)."""
    if pad is None:
        pad = [(k - 1) // 2] * 4
    op = orc.conv2d(c, c, k=k, s=s, pad=list(pad), dil=d, groups=c, act=act)
    oh, ow = orc.out_hw(op, ih, iw)
    x, wts, b, r = stream(seed, n * ih * iw * c, c * k * k, c, n * oh * ow * c if residual else 0)
    want = orc.conv2d_ref(op, ih, iw, x, wts, b, r if residual else None, n=n) if refs else None
    xd = dev(orc.pack_nhwc(x, n, ih, iw, c, dt))
    wd = dev(orc.pack_weights_dw(wts, c, k, k, dt))
    bd = dev(orc.pack_bias(b, c, dt))
    rd = dev(orc.pack_nhwc(r, n, oh, ow, c, dt)) if residual else None
    yd = poisoned(n * oh * ow * (-(-c // 4)) * 4, dt)
    spec = conv.ConvDwSpec(ih=ih, iw=iw, c=c, k=k, s=s, d=d, pad=tuple(pad), act=ACT[act], residual=residual,
                           dt=conv.DType(dt), n=n)
    spec.run(xd, wd, bd, rd, yd)
    torch.cuda.synchronize()
    got = orc.unpack_nhwc(host(yd, dt), n, oh, ow, c, dt)
    if not refs:
        return Result(got, None)
    rr = r if residual else None
    want_r = rounded_ref(op, ih, iw, x, wts, b, rr, dt, dt, n) if dt else want
    mag = magnitude(op, ih, iw, x, wts, b, rr, n) if dt else None
    return Result(got, want, None, want_r, mag)


class IrCase:
    """One fused inverted-residual block on seeded inputs: the host tensors,
    their packed device copies in `dt`, and the oracle's three-op chain
    (1x1 expand, depthwise 3x3, 1x1 project + residual, the ops the reference
    runs separately, crates/ai-gpu-runtime/src/lowering.rs:122-152) on the
    plain fp32 values (`want`) and with every stored tensor rounded to `dt`
    where the unfused path stores it (`want_stored`)."""

    def __init__(self, n, ih, iw, cin, cexp, cout, s, pad, residual, acts, dt, seed):
        self.n, self.ih, self.iw, self.cin, self.cexp, self.cout = n, ih, iw, cin, cexp, cout
        self.s, self.pad, self.residual, self.dt = s, tuple(pad), residual, dt
        self.act_e, self.act_d, self.act_p = acts
        op_e = orc.conv2d(cin, cexp, act=self.act_e)
        op_d = orc.conv2d(cexp, cexp, k=3, s=s, pad=list(pad), groups=cexp, act=self.act_d)
        op_p = orc.conv2d(cexp, cout, act=self.act_p)
        self.oh, self.ow = orc.out_hw(op_d, ih, iw)
        oh, ow = self.oh, self.ow
        x = orc.xs32_fill(seed, n * ih * iw * cin)
        we = orc.gauss_fill(seed + 1, 0.0, float(np.sqrt(2.0 / cin)), cexp * cin)
        be = orc.gauss_fill(seed + 2, 0.0, 0.01, cexp)
        wd = orc.gauss_fill(seed + 3, 0.0, float(np.sqrt(2.0 / 9)), cexp * 9)
        bd = orc.gauss_fill(seed + 4, 0.0, 0.01, cexp)
        wp = orc.gauss_fill(seed + 5, 0.0, float(np.sqrt(2.0 / cexp)), cout * cexp)
        bp = orc.gauss_fill(seed + 6, 0.0, 0.01, cout)
        r = orc.xs32_fill(seed + 7, n * oh * ow * cout) if residual else None

        def chain(rd):
            e = rd(orc.CpuConv(op_e, ih, iw, rd(we), rd(be)).run(rd(x), n, threads=8))
            d = rd(orc.CpuConv(op_d, ih, iw, rd(wd), rd(bd)).run(e, n, threads=8))
            y = orc.CpuConv(op_p, oh, ow, rd(wp), rd(bp), has_res=residual).run(
                d, n, rd(r) if residual else None, threads=8)
            return rd(y)

        self.want = chain(lambda v: v)
        self.want_stored = chain(lambda v: orc.round_to(v, dt))
        wep, _ = orc.pack_weights_conv(we, cexp, cin, 1, 1, 4, dt)
        wpp, _ = orc.pack_weights_conv(wp, cout, cexp, 1, 1, 4, dt)
        self.bufs = (dev(orc.pack_nhwc(x, n, ih, iw, cin, dt)), dev(wep), dev(orc.pack_bias(be, cexp, dt)),
                     dev(orc.pack_weights_dw(wd, cexp, 3, 3, dt)), dev(orc.pack_bias(bd, cexp, dt)), dev(wpp),
                     dev(orc.pack_bias(bp, cout, dt)),
                     dev(orc.pack_nhwc(r, n, oh, ow, cout, dt)) if residual else None)

    def spec(self, **kw):
        return conv.IrBlockSpec(ih=self.ih, iw=self.iw, cin=self.cin, cexp=self.cexp, cout=self.cout, s=self.s,
                                pad=self.pad, act_expand=ACT[self.act_e], act_dw=ACT[self.act_d],
                                act_project=ACT[self.act_p], residual=self.residual, dt=conv.DType(self.dt),
                                n=self.n, **kw)

    def run(self, spec) -> np.ndarray:
        """The fused launch of `spec` on this case's buffers, into a fresh
        NaN-filled output; the unpacked logical NHWC fp32 result."""
        yd = poisoned(self.n * self.oh * self.ow * (-(-self.cout // 4)) * 4, self.dt)
        spec.run(*self.bufs, yd)
        torch.cuda.synchronize()
        return orc.unpack_nhwc(host(yd, self.dt), self.n, self.oh, self.ow, self.cout, self.dt)

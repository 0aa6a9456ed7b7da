"""The int8 table-epilogue planner (host code of the HIP library, no GPU).

``qa_plan_epilogue_i8`` turns requantize -> activation table -> residual Add
-> rescaled copy into per-channel multiply-add constants and 256-entry
tables. The plan is evaluated here exactly the way the conv kernel evaluates
it and must equal the reference chain computed by the oracle on the same
int32 accumulators (random, int32 extremes, and values on both sides of every
rounding boundary), for every parameter family the executor produces.
Parameters outside the plan's exact range must be refused (the kernel then
runs the 128-bit epilogue)."""

import ctypes

import numpy as np
import pytest

from quantanything_amd.utils import quantize_multiplier

PLAN_E, PLAN_TC, PLAN_TR, PLAN_CH = 64, 64 + 1024, 64 + 2048, 64 + 3072


@pytest.fixture(scope="module")
def lib():
    from quantanything_amd import native

    if not native.available():
        pytest.skip(f"libqa_hip.so not loadable: {native.load_error()}")
    return native.library()


class _Desc:
    """The descriptor fields plan_epilogue reads."""

    def __init__(self, cout, **kw):
        self.Cout = cout
        self.zp = self.qmin = self.qmax = 0
        self.lut_offset = 0
        self.res = None
        self.res_first = self.res_so = 0
        self.za = self.ma = self.sa = self.zb = self.mb = self.sb = 0
        self.add_sign, self.add_zp, self.add_qmin, self.add_qmax = 1, 0, 0, 0
        self.y2 = None
        self.r2_zp_in = self.r2_m = self.r2_s = self.r2_zp_out = 0
        self.r2_qmin = self.r2_qmax = 0
        self.y_so = 0
        for k, v in kw.items():
            setattr(self, k, v)


def run_plan(plan, cout, acc, res_bytes=None):
    """The kernel's evaluation of a plan: acc [P, cout] int32 (wrapped
    accumulators), res_bytes [P, cout] stored residual bytes."""
    hd = plan[:16].view(np.int32)
    a, b, sh, flags = (int(v) for v in hd[:4])
    e_tab = plan[PLAN_E:PLAN_TC].view(np.int32)
    tc = plan[PLAN_TC:PLAN_TR].view(np.int32).astype(np.int64)
    tr = plan[PLAN_TR:PLAN_CH].view(np.int32).astype(np.int64)
    ch = plan[PLAN_CH:PLAN_CH + 16 * cout].view(np.int32).reshape(cout, 4)
    m = ch[:, 0].astype(np.int64)
    t = ch[:, 1].astype(np.int64)
    c = (ch[:, 3].astype(np.int64) << 32) | \
        (ch[:, 2].astype(np.int64) & 0xFFFFFFFF)
    r = acc.astype(np.int64) * m + c
    q0 = r >> t
    assert np.all((q0 >= -2**31) & (q0 < 2**31)), "plan range violated"
    i = np.clip(q0, a, b) - a
    if flags & 1:
        s = np.clip(tc[i] + tr[res_bytes.astype(np.uint8).astype(np.int64)],
                    0, sh)
        e = e_tab[s]
    else:
        e = e_tab[i]
    y = (e & 255).astype(np.uint8).view(np.int8)
    y2 = ((e >> 8) & 255).astype(np.uint8).view(np.int8)
    return y, y2


def reference_chain(ol, d, acc, mult, shift, pre, lut, res_bytes):
    """requantize -> lut -> Add -> rescale with the oracle's kernels."""
    p, cout = acc.shape
    q = ol.requantize(acc.astype(np.int32).reshape(p, cout, 1), p, cout, 1,
                      mult, shift, d.zp, d.qmin, d.qmax,
                      pre_bias=pre).reshape(p, cout)
    if lut is not None:
        q = ol.lut(q, lut, d.lut_offset)
    if d.res is not None:
        rq = res_bytes.astype(np.int8).astype(np.int32) + d.res_so
        first, second = (rq, q) if d.res_first else (q, rq)
        q = ol.add(first, second, d.za, d.ma, d.sa, d.zb, d.mb, d.sb,
                   d.add_zp, d.add_qmin, d.add_qmax, sign=d.add_sign)
    y = (q.astype(np.int64) - d.y_so).astype(np.int8)
    y2 = None
    if d.y2 is not None:
        q2 = ol.rescale(q, d.r2_zp_in, d.r2_m, d.r2_s, d.r2_zp_out,
                        d.r2_qmin, d.r2_qmax)
        y2 = (q2.astype(np.int64) - d.y_so).astype(np.int8)
    return y, y2


def accumulators(rng, mult, shift, pre, p_random=512):
    """Random int32 accumulators, the extremes, and for every channel values
    next to rounding boundaries of the requantization."""
    cout = len(mult)
    cols = [rng.integers(-2**31, 2**31, size=(p_random, cout),
                         dtype=np.int64),
            np.tile(np.array([[-2**31], [2**31 - 1], [0], [-1], [1]]),
                    (1, cout))]
    bnd = np.zeros((64, cout), np.int64)
    for c in range(cout):
        t = 31 + int(shift[c])
        m = int(mult[c]) or 1
        pb = int(pre[c]) if pre is not None else 0
        for k, half in enumerate(range(-16, 16)):
            # (w + pb) * m ~ (half + 1/2) * 2^t
            w = ((2 * half + 1) << (t - 1)) // m - pb
            bnd[2 * k, c] = w
            bnd[2 * k + 1, c] = w + 1
    cols.append(np.clip(bnd, -2**31, 2**31 - 1))
    return np.concatenate(cols).astype(np.int32)


def families(rng):
    """Parameter sets of the kinds the executor builds."""
    out = []
    for seed in range(6):
        r = np.random.default_rng(seed)
        cout = int(r.integers(1, 40))
        unsigned = bool(seed % 2)
        qmin, qmax = (0, 255) if unsigned else (-128, 127)
        zp = int(r.integers(qmin, qmax + 1))
        real = r.uniform(1e-5, 0.05, cout)
        pairs = [quantize_multiplier(v) for v in real]
        mult = np.array([m for m, _ in pairs], np.int64)
        shift = np.array([s for _, s in pairs], np.int64)
        pre = r.integers(-2**20, 2**20, cout) if seed % 3 else None
        kw = dict(zp=zp, qmin=qmin, qmax=qmax, y_so=128 if unsigned else 0)
        lut = None
        if seed in (1, 2, 4, 5):
            lut = r.integers(qmin, qmax + 1, 256).astype(np.int32)
            kw["lut_offset"] = qmin if seed != 4 else qmin + 17
            if seed == 5:
                lut = lut[:200]
        if seed in (2, 3, 5):
            ma, sa = quantize_multiplier(r.uniform(0.3, 2.0))
            mb, sb = quantize_multiplier(r.uniform(0.3, 2.0))
            kw.update(res=1, res_first=int(seed == 3), res_so=kw["y_so"],
                      za=int(r.integers(qmin, qmax)), ma=ma, sa=sa,
                      zb=int(r.integers(qmin, qmax)), mb=mb, sb=sb,
                      add_sign=-1 if seed == 5 else 1,
                      add_zp=int(r.integers(qmin, qmax)), add_qmin=qmin,
                      add_qmax=qmax)
        if seed in (1, 3, 4):
            m2, s2 = quantize_multiplier(r.uniform(0.5, 1.5))
            kw.update(y2=1, r2_zp_in=int(r.integers(qmin, qmax)), r2_m=m2,
                      r2_s=s2, r2_zp_out=int(r.integers(qmin, qmax)),
                      r2_qmin=qmin, r2_qmax=qmax)
        out.append((f"seed{seed}", _Desc(cout, **kw), mult, shift, pre, lut))
    return out


@pytest.mark.parametrize("case", range(6))
def test_plan_matches_reference_chain(lib, oracle_lib, case):
    from quantanything_amd.executor import plan_epilogue

    rng = np.random.default_rng(100 + case)
    name, d, mult, shift, pre, lut = families(rng)[case]
    plan = plan_epilogue(lib, d, mult, shift, pre, lut)
    assert plan is not None, name
    acc = accumulators(rng, mult, shift, pre)
    res_bytes = rng.integers(-128, 128, acc.shape).astype(np.int8)
    y, y2 = run_plan(plan, d.Cout, acc, res_bytes)
    ey, ey2 = reference_chain(oracle_lib, d, acc, mult, shift, pre, lut,
                              res_bytes)
    np.testing.assert_array_equal(y, ey)
    if ey2 is not None:
        np.testing.assert_array_equal(y2, ey2)


def test_plan_extreme_bias_and_multiplier(lib, oracle_lib):
    """|bias| up to 2^30 and multipliers near 2^31 with large shifts."""
    from quantanything_amd.executor import plan_epilogue

    mult = np.array([2**31 - 1, -(2**31 - 1), 2**30, 1, 12345], np.int64)
    shift = np.array([20, 25, 31, 0, -10], np.int64)
    pre = np.array([2**30, -(2**29), 123, -5, 2**30], np.int64)
    d = _Desc(5, zp=3, qmin=-128, qmax=127)
    plan = plan_epilogue(lib, d, mult, shift, pre)
    assert plan is not None
    rng = np.random.default_rng(7)
    acc = accumulators(rng, mult, shift, pre)
    y, _ = run_plan(plan, 5, acc)
    ey, _ = reference_chain(oracle_lib, d, acc, mult, shift, pre, None, None)
    np.testing.assert_array_equal(y, ey)


@pytest.mark.parametrize("mult,shift,what", [
    (1 << 31, 0, "multiplier beyond int32"),
    (1 << 30, -31, "left shift (31 + shift < 1)"),
    (1 << 30, 32, "shift beyond 62"),
    (1 << 30, -8, "shifted value beyond int32"),
])
def test_plan_refuses_out_of_range(lib, mult, shift, what):
    from quantanything_amd.executor import plan_epilogue

    d = _Desc(1, zp=0, qmin=-128, qmax=127)
    assert plan_epilogue(lib, d, [mult], [shift]) is None, what


def test_plan_refuses_wide_ranges_and_large_add_terms(lib):
    from quantanything_amd.executor import plan_epilogue

    d = _Desc(1, zp=0, qmin=-32768, qmax=32767)
    assert plan_epilogue(lib, d, [1 << 30], [0]) is None
    d = _Desc(1, zp=0, qmin=-128, qmax=127, res=1, za=0, ma=1 << 30, sa=-30,
              zb=0, mb=1 << 30, sb=0, add_qmin=-128, add_qmax=127)
    assert plan_epilogue(lib, d, [1 << 30], [0]) is None


def test_plan_bad_arguments(lib):
    from quantanything_amd.executor import EpiParams

    assert lib.qa_plan_epilogue_i8(None, None) == -1
    e = EpiParams()
    e.cout = 0
    buf = np.zeros(4096, np.uint8)
    assert lib.qa_plan_epilogue_i8(ctypes.byref(e), buf.ctypes.data) == -1
    assert lib.qa_epi_plan_bytes(3) == PLAN_CH + 48

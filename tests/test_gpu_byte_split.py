"""The byte-split 16-bit convolution through the C ABI (qa_d_conv with the
FP64 weights and the split planes), against a direct convolution in Python
integers with the reference's rounding (qa_kernels.cpp:188-205: round half
up of x m 2^-(31+shift), then + zp and the clip). The multipliers put many
sums exactly on a rounding tie (m = 2^30, shift 0: every odd sum), so the
epilogue's float64 form must hand those to its 128-bit form; every tile
code (byte split, FP64) gives the same result."""

import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _mbqm(x, m, s):
    ts = 31 + s
    p = x * m
    if ts > 0:
        ts = min(ts, 120)
        return (p + (1 << (ts - 1))) >> ts
    return p << min(-ts, 60)


def _direct(x, w, x_add, pre, mult, shift, zp, lo, hi):
    """x [N, H, W, C] stored int16, w [Cout, C, 3, 3]; pad 1, stride 1."""
    n, h, wd, c = x.shape
    cout = w.shape[0]
    xc = np.zeros((n, h + 2, wd + 2, c), np.int64)
    xc[:, 1:-1, 1:-1, :] = x.astype(np.int64) + x_add
    acc = np.zeros((n, h, wd, cout), np.int64)
    for ky in range(3):
        for kx in range(3):
            acc += np.einsum("nhwc,oc->nhwo", xc[:, ky:ky + h, kx:kx + wd, :],
                             w[:, :, ky, kx].astype(np.int64))
    y = np.empty_like(acc)
    for o in range(cout):
        v = acc[..., o] + pre[o]
        y[..., o] = np.array(
            [min(max(_mbqm(int(t), int(mult[o]), int(shift[o])) + zp, lo),
                 hi) for t in v.reshape(-1)], np.int64).reshape(v.shape)
    return y, acc


def _run_all_tiles(lib, xs, cin, w, x_add, pre, mult, shift, zp, lo, hi,
                   want):
    """qa_d_conv on stored int16 activations xs [N, H, W, Cs] with every
    byte-split and FP64 tile code; each result must equal ``want``."""
    import torch
    from quantanything_amd.executor import F64_TILES, ConvDesc

    n, h, w_, cs = xs.shape
    cout = w.shape[0]
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    ck, frows = ctypes.c_int64(0), ctypes.c_int64(0)
    nf = lib.qa_pack_weights_f64_size(cout, cin, 3, 3, 1, ctypes.byref(ck),
                                      ctypes.byref(frows))
    wf = np.empty(nf, np.int16)
    assert lib.qa_pack_weights_f64(w.ctypes.data, cout, cin, 3, 3, 1, 2,
                                   wf.ctypes.data) == 0
    kgp, rows = ctypes.c_int64(0), ctypes.c_int64(0)
    n8 = lib.qa_pack_weights_i8_size(cout, cin, 3, 3, 1, 0, ctypes.byref(kgp),
                                     ctypes.byref(rows))
    ws = np.empty(2 * n8, np.int8)
    wsum = np.empty(cout, np.int64)
    assert lib.qa_pack_weights_i16s(w.ctypes.data, cout, cin, 3, 3, 1,
                                    ws.ctypes.data, wsum.ctypes.data) == 0
    bufs = dict(x=dev(xs), wf=dev(wf), ws=dev(ws),
                wk=dev((128 + x_add) * wsum), pre=dev(pre), m=dev(mult),
                s=dev(shift),
                y=torch.zeros((n, h, w_, cout), dtype=torch.int16,
                              device="cuda"))
    d = ConvDesc()
    d.x, d.x_code = bufs["x"].data_ptr(), 2
    d.x_sn, d.x_sc, d.x_sp, d.x_add = h * w_ * cs, 1, cs, x_add
    (d.N, d.C, d.H, d.W, d.Cout, d.KH, d.KW, d.SH, d.SW, d.PH, d.PW, d.DH,
     d.DW, d.G, d.OH, d.OW) = (n, cin, h, w_, cout, 3, 3, 1, 1, 1, 1, 1, 1, 1,
                               h, w_)
    d.w, d.w_code, d.w_layout = bufs["wf"].data_ptr(), 8, 2
    d.w_kgp, d.w_rows, d.wide = ck.value, frows.value, 1
    d.pre_bias, d.mult, d.shift = (bufs["pre"].data_ptr(),
                                   bufs["m"].data_ptr(), bufs["s"].data_ptr())
    d.zp, d.qmin, d.qmax = zp, lo, hi
    d.y, d.y_code = bufs["y"].data_ptr(), 2
    d.y_sn, d.y_sc, d.y_sp, d.y_so = h * w_ * cout, 1, cout, 0
    d.wsplit, d.wsplit_k = bufs["ws"].data_ptr(), bufs["wk"].data_ptr()
    codes = [0] + [0x11000 | wm | tm << 4 for tm in (1, 2)
                   for wm in (1, 2, 4)] + [0x10000 | c for c in F64_TILES]
    s = torch.cuda.current_stream().cuda_stream
    for code in codes:
        d.tile = code
        bufs["y"].zero_()
        rc = lib.qa_d_conv(ctypes.byref(d), s)
        assert rc == 0, (hex(code), lib.qa_last_error())
        torch.cuda.synchronize()
        np.testing.assert_array_equal(bufs["y"].cpu().numpy().astype(np.int64),
                                      want, err_msg=f"tile {code:#x}")


@pytest.mark.parametrize("cin,cout", [(16, 16), (32, 48), (3, 16)])
def test_byte_split_ties_against_direct_sum(hip, cin, cout):
    lib = hip.require()
    rng = np.random.default_rng(cin * 100 + cout)
    n, h, w_ = 2, 7, 6
    cs = 4 if cin <= 4 else cin  # stored channels a pixel
    x = rng.integers(-40, 41, size=(n, h, w_, cin))
    xs = np.zeros((n, h, w_, cs), np.int16)
    xs[..., :cin] = x
    w = rng.integers(-3, 4, size=(cout, cin, 3, 3)).astype(np.int32)
    w[0, 0, 1, 1] = 32767  # an int16 extreme (its outputs saturate)
    x_add, zp, lo, hi = 5, 7, -32768, 32767
    pre = rng.integers(-50, 51, size=cout).astype(np.int64)
    mult = np.full(cout, 1 << 30, np.int64)  # odd sums: exact ties
    shift = np.zeros(cout, np.int64)
    mult[1::3], shift[1::3] = 3 << 28, -1     # ties at every fourth sum
    mult[2::3], shift[2::3] = 1518500250, 2   # an ordinary multiplier
    want, acc = _direct(xs[..., :cin], w, x_add, pre, mult, shift, zp, lo, hi)
    assert (acc % 2 == 1).any()
    _run_all_tiles(lib, xs, cin, w, x_add, pre, mult, shift, zp, lo, hi,
                   want)


def test_byte_split_full_int16_range(hip):
    """Activations over the whole int16 range (-32768 included) against
    weights at -32768 and 32767, 256 input channels (K = 2304): the high
    bytes reach -128 and 127, so the 65536 Hh and 256 (Hl + Lh) terms and
    the int32 headroom of each int8 MFMA sum (|xh wh| <= 2^14, K' < 2^16)
    are exercised. Multipliers of about 2^-27 keep most outputs inside the
    clip bounds."""
    lib = hip.require()
    rng = np.random.default_rng(2304)
    n, h, w_, cin, cout = 2, 5, 4, 256, 32
    xs = rng.integers(-32768, 32768, size=(n, h, w_, cin)).astype(np.int16)
    xs[0, :3, :3, :] = -32768  # a full window of the extremes
    xs[1, -3:, -3:, :] = 32767
    w = rng.integers(-32768, 32768, size=(cout, cin, 3, 3)).astype(np.int32)
    w[0] = -32768
    w[1] = 32767
    w[2, ::2] = -32768
    w[2, 1::2] = 32767
    x_add, zp, lo, hi = -3, 11, -32768, 32767
    pre = rng.integers(-(1 << 40), 1 << 40, size=cout).astype(np.int64)
    mult = rng.integers(1 << 30, 1 << 31, size=cout).astype(np.int64)
    shift = np.full(cout, 27, np.int64)
    shift[:3] = 33  # the extreme rows sum to about 2^41
    want, acc = _direct(xs, w, x_add, pre, mult, shift, zp, lo, hi)
    assert np.abs(acc).max() > 1 << 40
    assert ((want > lo) & (want < hi)).mean() > 0.5
    _run_all_tiles(lib, xs, cin, w, x_add, pre, mult, shift, zp, lo, hi,
                   want)

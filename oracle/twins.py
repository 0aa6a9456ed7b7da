"""NumPy / Python-integer restatements used as closed-form checks (test only).

* ``np_conv``   -- grouped, strided, dilated, padded convolution as a
                   sliding-window einsum (the form of the reference's own test
                   oracle, ``native.py:260-277`` used by
                   ``test_native.py:18-27``), evaluated in int64 / float64.
* ``mbqm_exact``-- ``round(x * m * 2^-(31+s))`` with Python integers and the
                   reference C++ clamps (``qa_kernels.cpp:196-205``).
* ``requantize_exact`` / ``rescale_exact`` / ``add_exact`` / ``mul_exact``
                -- element-by-element Python-integer versions of the fused
                   integer kernels (``qa_kernels.cpp:207-345``), for small
                   inputs.
"""

import numpy as np
from numpy.lib.stride_tricks import sliding_window_view


def np_conv(x, w, strides, pads, dilations, groups, dtype=np.int64):
    """y[N,Cout,OH,OW] by sliding windows; padding contributes zeros."""
    n, c, h, wd = x.shape
    cout, cg, kh, kw = w.shape
    sh, sw = strides
    dh, dw = dilations
    pt, pl, pb, pr = pads
    oh = (h + pt + pb - dh * (kh - 1) - 1) // sh + 1
    ow = (wd + pl + pr - dw * (kw - 1) - 1) // sw + 1
    xp = np.pad(x.astype(dtype), ((0, 0), (0, 0), (pt, pb), (pl, pr)))
    win = sliding_window_view(xp, (dh * (kh - 1) + 1, dw * (kw - 1) + 1),
                              axis=(2, 3))
    win = win[:, :, ::sh, ::sw, ::dh, ::dw][:, :, :oh, :ow]
    cog = cout // groups
    out = np.empty((n, cout, oh, ow), dtype=dtype)
    for g in range(groups):
        out[:, g * cog:(g + 1) * cog] = np.einsum(
            "nchwyx,ocyx->nohw", win[:, g * cg:(g + 1) * cg],
            w[g * cog:(g + 1) * cog].astype(dtype), optimize=True)
    return out


def mbqm_exact(x, m, s):
    p = int(x) * int(m)
    ts = 31 + int(s)
    if ts > 0:
        ts = min(ts, 120)
        return (p + (1 << (ts - 1))) >> ts
    return p << min(-ts, 60)


def _clip(v, lo, hi):
    return max(int(lo), min(int(hi), v))


def requantize_exact(acc, outer, C, inner, mult, shift, zp, qmin, qmax,
                     pre=None, post=None):
    a = np.asarray(acc).reshape(outer, C, inner)
    out = np.empty(a.shape, dtype=np.int64)
    for o in range(outer):
        for c in range(C):
            pb = int(pre[c]) if pre is not None else 0
            qb = (int(post[c]) if post is not None else 0) + int(zp)
            for i in range(inner):
                v = mbqm_exact(int(a[o, c, i]) + pb, mult[c], shift[c]) + qb
                out[o, c, i] = _clip(v, qmin, qmax)
    return out.reshape(np.shape(acc))


def rescale_exact(x, zp_in, m, s, zp_out, qmin, qmax):
    return np.array([_clip(mbqm_exact(int(v) - zp_in, m, s) + zp_out, qmin,
                           qmax) for v in np.ravel(x)], dtype=np.int64)


def add_exact(a, b, za, ma, sa, zb, mb, sb, zp_out, qmin, qmax, sign=1):
    return np.array([
        _clip(mbqm_exact(int(u) - za, ma, sa)
              + sign * mbqm_exact(int(v) - zb, mb, sb) + zp_out, qmin, qmax)
        for u, v in zip(np.ravel(a), np.ravel(b))], dtype=np.int64)


def mul_exact(a, b, za, zb, m, s, zp_out, qmin, qmax):
    return np.array([
        _clip(mbqm_exact((int(u) - za) * (int(v) - zb), m, s) + zp_out, qmin,
              qmax) for u, v in zip(np.ravel(a), np.ravel(b))],
        dtype=np.int64)

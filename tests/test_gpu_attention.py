"""Fused attention (qa_d_attention) against the three launches it replaces
(qa_d_matmul_act for q k^T, qa_d_softmax_lut, qa_d_matmul_act for . v) on
raw device buffers laid out as a QKV projection's output [B, T, 3, H, hd]
and an output in [B, T, H, hd]: bit for bit, for token counts that are not
multiples of 16 (up to the 256-column limit), head dims 16 to 128, and
operands stored at nonzero zero points. The unfused launches follow the
reference's MatMul / Softmax fallbacks (float_ops.py:181-186, :380-386)."""

import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _desc(MatmulDesc, a, b, y, shapes, qa_, qb_, qo):
    d = MatmulDesc()
    d.a, d.a_code, d.a_so, d.a_zp, d.a_scale = a[0], 1, qa_[1], qa_[1], \
        qa_[0]
    d.a_s0, d.a_s1, d.a_sm, d.a_sk = a[1]
    d.b, d.b_code, d.b_so, d.b_zp, d.b_scale = b[0], 1, qb_[1], qb_[1], \
        qb_[0]
    d.b_s0, d.b_s1, d.b_sn, d.b_sk = b[1]
    d.B0, d.B1, d.M, d.N, d.K = shapes
    d.y, d.y_code, d.y_so = y[0], 1, qo[4]
    d.y_s0, d.y_s1, d.y_sm, d.y_sn = y[1]
    d.out_scale, d.out_zp, d.qmin, d.qmax = qo[:4]
    return d


@pytest.mark.parametrize("B,H,T,hd", [(2, 3, 17, 32), (1, 2, 197, 64),
                                      (2, 1, 256, 64), (1, 1, 5, 16),
                                      (3, 2, 33, 128)])
def test_fused_attention_equals_three_launches(hip, B, H, T, hd):
    import torch

    from quantanything_amd.executor import AttentionDesc, MatmulDesc
    lib = hip.require()
    rng = np.random.default_rng(T * 7 + hd)
    qkv = rng.integers(-100, 101, size=(B, T, 3, H, hd), dtype=np.int8)
    dq = torch.from_numpy(qkv).cuda()
    base = dq.data_ptr()
    row = 3 * H * hd  # token stride
    s_b = T * row
    qs, ks, vs = (0.031, 3), (0.027, -5), (0.02, 2)  # scale, zp = so
    # the exact S and O ranges set their scales (some values clip)
    qf = (qkv[:, :, 0].astype(np.float64) - qs[1]) * qs[0]
    kf = (qkv[:, :, 1].astype(np.float64) - ks[1]) * ks[0]
    smax = np.abs(np.einsum("bthd,bshd->bhts", qf, kf)).max()
    S = (smax / 110.0, 4, -128, 127, 0)      # scale, zp, qmin, qmax, so
    P = (1.0 / 127.0, 0, -128, 127, 0)
    vmax = np.abs((qkv[:, :, 2].astype(np.float64) - vs[1]) * vs[0]).max()
    O = (vmax / 150.0, -3, -128, 127, -3)
    dS = torch.zeros((B, H, T, T), dtype=torch.int8, device="cuda")
    dP = torch.zeros_like(dS)
    dO1 = torch.zeros((B, T, H, hd), dtype=torch.int8, device="cuda")
    dO2 = torch.full((B, T, H, hd), 77, dtype=torch.int8, device="cuda")
    qk = _desc(MatmulDesc, (base, (s_b, hd, row, 1)),
               (base + H * hd, (s_b, hd, row, 1)),
               (dS.data_ptr(), (H * T * T, T * T, T, 1)), (B, H, T, T, hd),
               qs, ks, S)
    o_str = (T * H * hd, hd, H * hd, 1)
    av1 = _desc(MatmulDesc, (dP.data_ptr(), (H * T * T, T * T, T, 1)),
                (base + 2 * H * hd, (s_b, hd, 1, row)),
                (dO1.data_ptr(), o_str), (B, H, T, hd, T), (P[0], P[1]), vs,
                O)
    tab = torch.empty(65536, dtype=torch.float64, device="cuda")
    assert lib.qa_d_softmax_table(ctypes.c_double(S[0]), S[1], S[4],
                                  ctypes.c_void_p(tab.data_ptr()), None) == 0
    # the three launches
    assert lib.qa_d_matmul_act(ctypes.byref(qk), None) == 0
    assert lib.qa_d_softmax_lut(
        ctypes.c_void_p(dS.data_ptr()), B * H * T, T,
        ctypes.c_void_p(tab.data_ptr()), ctypes.c_void_p(dP.data_ptr()),
        ctypes.c_double(P[0]), P[1], P[2], P[3], P[4], None) == 0
    assert lib.qa_d_matmul_act(ctypes.byref(av1), None) == 0
    # fused
    ad = AttentionDesc()
    ad.qk = qk
    ad.av = _desc(MatmulDesc, (0, (0, 0, 0, 0)),
                  (base + 2 * H * hd, (s_b, hd, 1, row)),
                  (dO2.data_ptr(), o_str), (B, H, T, hd, T),
                  (P[0], P[1]), vs, O)
    ad.table = tab.data_ptr()
    ad.p_scale, ad.p_zp, ad.p_qmin, ad.p_qmax, ad.p_so = P
    assert lib.qa_attention_supported(ctypes.byref(ad)) == 1
    assert lib.qa_d_attention(ctypes.byref(ad), None) == 0
    torch.cuda.synchronize()
    o1, o2 = dO1.cpu().numpy(), dO2.cpu().numpy()
    assert np.unique(o1).size > 20  # a live result, not a constant
    np.testing.assert_array_equal(o2, o1)

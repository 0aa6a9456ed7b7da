"""Standalone device workloads of single integer layers.

* :class:`GemmWorkload` -- M=4096 K=576 N=64 uint8 x int8 GEMM with the
  per-column requantize fused into the epilogue (uint8 output, zero point
  128), run as one ``qa_d_conv`` launch in row-major (GEMM) mode.
* :class:`ConvWorkload` -- batch 32, 64->64, 3x3, stride 1, pad 1, 56x56
  NCHW uint8 conv with bias, requantize and the 256-entry SiLU table fused
  into the epilogue.

Inputs come from :mod:`quantanything_amd.synth`; both produce the quantized
output tensor that the reference computes with separate conv / GEMM,
requantize and LUT calls. Device storage is int8 holding ``q - 128``; the
conv's activations are channels-last on the device.
"""

import ctypes

import numpy as np
import torch

from quantanything_amd import native, synth
from quantanything_amd.executor import ConvDesc, _dev, _ok, plan_epilogue


class _Workload:
    def __init__(self):
        self.lib = native.require()

    def _pack(self, w_oihw, a_off):
        cout, cg, kh, kw = w_oihw.shape
        kgp, rows = ctypes.c_int64(0), ctypes.c_int64(0)
        size = self.lib.qa_pack_weights_i8_size(cout, cg, kh, kw, 1, 0,
                                                ctypes.byref(kgp),
                                                ctypes.byref(rows))
        wp = np.empty(size, np.int8)
        corr = np.empty(cout, np.int64)
        boff = np.empty(cout, np.int32)
        need = ctypes.c_int32(0)
        w32 = np.ascontiguousarray(w_oihw, dtype=np.int32)
        rc = self.lib.qa_pack_weights_i8(
            w32.ctypes.data, cout, cg, kh, kw, 1, a_off, 0, wp.ctypes.data,
            corr.ctypes.data, boff.ctypes.data, ctypes.byref(need))
        if rc != 0:
            raise RuntimeError("weights do not pack to int8")
        self.kgp, self.rows = kgp.value, rows.value
        self.wp = _dev(wp, np.int8)
        self.corr = _dev(corr, np.int64)
        self.boff = _dev(boff, np.int32)
        return kgp.value, rows.value, need.value

    def _plan(self, d, mult, shift, bias, lut=None):
        plan = plan_epilogue(self.lib, d, mult, shift, bias, lut)
        if plan is None:
            raise RuntimeError("workload parameters need the 128-bit "
                               "epilogue")
        self.plan = _dev(plan, np.uint8)
        d.epi_plan = self.plan.data_ptr()
        # the weights in fragment order too (the narrow-GEMM kernel's form)
        size = self.lib.qa_fragments_i8_size(d.w_rows, d.w_kgp)
        self.wfrag = torch.empty(max(size, 1), dtype=torch.int8,
                                 device="cuda")
        _ok(self.lib.qa_d_pack_fragments_i8(
            d.w, d.w_rows, d.w_kgp, self.wfrag.data_ptr(),
            torch.cuda.current_stream().cuda_stream),
            "qa_d_pack_fragments_i8")
        d.w_frag = self.wfrag.data_ptr()
        self.d = d

    def launch(self, stream=None):
        s = stream if stream is not None else \
            torch.cuda.current_stream().cuda_stream
        _ok(self.lib.qa_d_conv(ctypes.byref(self.d), s), "qa_d_conv")

    def output(self):
        """Quantized output ``q`` (int32, NumPy, NCHW / [M, N])."""
        torch.cuda.synchronize()
        q = self.y[:self.numel].to(torch.int32).cpu().numpy() + 128
        if len(self.out_shape) == 4:  # stored channels-last
            n, c, h, w = self.out_shape
            return q.reshape(n, h, w, c).transpose(0, 3, 1, 2)
        return q.reshape(self.out_shape)

    @property
    def arithmetic_intensity(self):
        return self.ops / self.bytes


class GemmWorkload(_Workload):
    """uint8 [M,K] x int8 [K,N] + bias -> requantize -> uint8 [M,N]
    (default: M=4096 K=576 N=64; ``vit_gemm_shapes`` lists the weight GEMMs
    of one ViT-S/16 block at batch 32)."""

    def __init__(self, seed=1, M=4096, K=576, N=64):
        super().__init__()
        g = synth.gemm_workload(seed, M=M, K=K, N=N)
        self.spec = g
        m, k, n = g["M"], g["K"], g["N"]
        self.x = _dev(g["a"].astype(np.int16) - 128, np.int8)
        a_off = 128 - g["zp_in"]
        kgp, rows, need = self._pack(
            g["w"].T.reshape(n, k, 1, 1).astype(np.int32), a_off)
        self.numel = m * n
        self.y = torch.empty(m * n, dtype=torch.int8, device="cuda")
        self.params = [_dev(g["bias"], np.int64), _dev(g["mult"], np.int64),
                       _dev(g["shift"], np.int64)]
        d = ConvDesc()
        d.x, d.x_code, d.x_sn, d.x_sc, d.x_sp, d.x_add = (
            self.x.data_ptr(), 1, k, 1, 0, a_off)
        (d.N, d.C, d.H, d.W, d.Cout, d.KH, d.KW, d.SH, d.SW, d.PH, d.PW,
         d.DH, d.DW, d.G, d.OH, d.OW) = (m, k, 1, 1, n, 1, 1, 1, 1, 0, 0, 1,
                                         1, 1, 1, 1)
        d.w, d.w_code, d.w_layout, d.w_kgp, d.w_rows = (
            self.wp.data_ptr(), 1, 0, kgp, rows)
        d.wide, d.needs_rowsum = 0, need
        d.corr, d.boff = self.corr.data_ptr(), self.boff.data_ptr()
        d.pre_bias, d.mult, d.shift = (p.data_ptr() for p in self.params)
        d.zp, d.qmin, d.qmax = g["zp_out"], g["qmin"], g["qmax"]
        d.y, d.y_code, d.y_sn, d.y_sc, d.y_sp, d.y_so = (
            self.y.data_ptr(), 1, n, 1, 0, 128)
        self._plan(d, g["mult"], g["shift"], g["bias"])
        self.out_shape = (m, n)
        self.ops = 2 * m * n * k
        self.bytes = m * k + k * n + m * n + n * 24
        self.name = f"qgemm M={m} K={k} N={n} u8xi8->u8 (+bias, requantize)"


class ConvWorkload(_Workload):
    """uint8 NCHW conv + bias -> requantize -> SiLU table -> uint8."""

    def __init__(self, seed=2, batch=32):
        super().__init__()
        c = synth.conv_workload(seed, batch=batch)
        self.spec = c
        x, w = c["x"], c["w"]
        n, cin, h, wd = x.shape
        cout, _, kh, kw = w.shape
        s, p = c["stride"], c["pad"]
        oh = (h + 2 * p - kh) // s + 1
        ow = (wd + 2 * p - kw) // s + 1
        # channels-last int8 activations (+64 bytes of load slack)
        xl = (x.astype(np.int16) - 128).transpose(0, 2, 3, 1).reshape(-1)
        self.x = _dev(np.concatenate([xl, np.zeros(64, np.int16)]), np.int8)
        a_off = 128 - c["zp_in"]
        kgp, rows, need = self._pack(w.astype(np.int32), a_off)
        self.numel = n * cout * oh * ow
        self.y = torch.empty(self.numel + 64, dtype=torch.int8,
                             device="cuda")
        self.params = [_dev(c["bias"], np.int64), _dev(c["mult"], np.int64),
                       _dev(c["shift"], np.int64), _dev(c["lut"], np.int32)]
        d = ConvDesc()
        d.x, d.x_code, d.x_sn, d.x_sc, d.x_sp, d.x_add = (
            self.x.data_ptr(), 1, h * wd * cin, 1, cin, a_off)
        (d.N, d.C, d.H, d.W, d.Cout, d.KH, d.KW, d.SH, d.SW, d.PH, d.PW,
         d.DH, d.DW, d.G, d.OH, d.OW) = (n, cin, h, wd, cout, kh, kw, s, s,
                                         p, p, 1, 1, 1, oh, ow)
        d.w, d.w_code, d.w_layout, d.w_kgp, d.w_rows = (
            self.wp.data_ptr(), 1, 0, kgp, rows)
        d.wide, d.needs_rowsum = 0, need
        d.corr, d.boff = self.corr.data_ptr(), self.boff.data_ptr()
        d.pre_bias, d.mult, d.shift = (p_.data_ptr() for p_ in self.params[:3])
        d.zp, d.qmin, d.qmax = c["zp_out"], c["qmin"], c["qmax"]
        d.lut, d.lut_offset, d.lut_len = (self.params[3].data_ptr(),
                                          c["lut_offset"], len(c["lut"]))
        d.y, d.y_code, d.y_sn, d.y_sc, d.y_sp, d.y_so = (
            self.y.data_ptr(), 1, oh * ow * cout, 1, cout, 128)
        self._plan(d, c["mult"], c["shift"], c["bias"], c["lut"])
        self.out_shape = (n, cout, oh, ow)
        self.ops = 2 * n * cout * oh * ow * cin * kh * kw
        self.bytes = x.size + w.size + n * cout * oh * ow + cout * 24 + 1024
        self.name = (f"qconv b{n} {cin}->{cout} {kh}x{kw} s{s} p{p} {h}x{wd} "
                     "u8 (+bias, requantize, SiLU table)")


class RequantizeWorkload(_Workload):
    """The standalone requantize of the conv workload's accumulators: int32
    NCHW [32, 64, 56, 56] (6.42 M values) + per-channel bias -> mbqm ->
    uint8 (int8 storage), one ``qa_d_requantize`` launch (the reference's
    separate ``qa_requantize_i32`` step, qa_kernels.cpp:207-228)."""

    def __init__(self, seed=2, batch=32):
        super().__init__()
        c = synth.conv_workload(seed, batch=batch)
        n, cout, hw = batch, c["w"].shape[0], c["x"].shape[2]
        st = synth.Stream(seed + 100)
        acc = st.integers(-(2**20), 2**20, (n, cout, hw * hw)).astype(
            np.int32)
        self.acc = _dev(acc, np.int32)
        self.numel = acc.size
        self.y = torch.empty(self.numel, dtype=torch.int8, device="cuda")
        self.params = [_dev(c[k], np.int64) for k in ("mult", "shift",
                                                      "bias")]
        self.args = (n, cout, hw * hw, c["zp_out"], c["qmin"], c["qmax"])
        self.ops = self.numel
        self.bytes = self.numel * (4 + 1) + cout * 24
        self.name = (f"requantize int32 [{n},{cout},{hw},{hw}] -> u8 "
                     "(per-channel bias, mbqm)")

    def launch(self, stream=None):
        s = stream if stream is not None else \
            torch.cuda.current_stream().cuda_stream
        outer, cc, inner, zp, qmin, qmax = self.args
        m, sh, b = (p.data_ptr() for p in self.params)
        _ok(self.lib.qa_d_requantize(self.acc.data_ptr(), 4,
                                     self.y.data_ptr(), 1, outer, cc, inner,
                                     m, sh, b, None, zp, qmin, qmax, 0, 128,
                                     s), "qa_d_requantize")


class LutWorkload(_Workload):
    """The standalone 256-entry SiLU table over the conv workload's uint8
    output (6.42 M values, int8 storage in and out), one ``qa_d_lut``
    launch (the reference's separate ``qa_lut`` step,
    qa_kernels.cpp:348-358)."""

    def __init__(self, seed=2, batch=32):
        super().__init__()
        c = synth.conv_workload(seed, batch=batch)
        n = batch * c["w"].shape[0] * c["x"].shape[2] * c["x"].shape[3]
        st = synth.Stream(seed + 200)
        self.x = _dev(st.integers(-128, 127, (n,)), np.int8)
        self.y = torch.empty(n, dtype=torch.int8, device="cuda")
        self.lut = _dev(c["lut"], np.int32)
        self.numel = n
        self.ops = n
        self.bytes = 2 * n + 4 * len(c["lut"])
        self.name = f"SiLU table u8 -> u8, {n} values"

    def launch(self, stream=None):
        s = stream if stream is not None else \
            torch.cuda.current_stream().cuda_stream
        n = self.numel
        _ok(self.lib.qa_d_lut(self.x.data_ptr(), 1, n, self.y.data_ptr(), 1,
                              n, 1, n, 0, self.lut.data_ptr(),
                              self.lut.numel(), 128, 128, s), "qa_d_lut")


def vit_gemm_shapes(batch=32, tokens=197, dim=384, mlp=1536):
    """``(name, M, K, N)`` of the weight GEMMs of one ViT block."""
    m = batch * tokens
    return [("qkv", m, dim, 3 * dim), ("proj", m, dim, dim),
            ("fc1", m, dim, mlp), ("fc2", m, mlp, dim)]

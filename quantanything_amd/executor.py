"""Device-resident integer executor.

Turns a calibrated container into a fixed sequence of GPU launches over
preallocated device buffers, so a whole inference pass runs without a host
round trip per node (the reference crosses Python -> C per node with host
NumPy arrays, ``quant_container.py:135-193``). The sequence can be captured
once into a HIP graph and replayed.

Storage: every quantized tensor lives on the device as int8 (types of at most
8 bits) or int16 (9-16 bits) holding ``q - so``, ``so`` = 0 for signed types
and 2^(bits-1) for unsigned ones. Layouts are NCHW; a tensor may be a view
(``offset`` into a buffer, ``nstride`` elements between images), which is how
``Split`` outputs are produced without a copy.

Fusion: a Conv / Gemm whose output feeds only a lookup-table activation runs
the table in its epilogue; if that result feeds only an Add whose other
operand already exists, the Add (rescale of both operands, sum, clip) runs in
the same epilogue. Every fused step applies the same integer operations, in
the same order, as the separate layers would.

torch is used for device memory, the stream and graph capture only; all
arithmetic is in ``libqa_hip.so``.
"""

import ctypes

import numpy as np
import torch

from quantanything_amd import native

_I64 = ctypes.c_int64
_P = ctypes.c_void_p
IDENTITY = (1 << 30, -1)  # multiplier exactly 1.0


class ConvDesc(ctypes.Structure):
    """``qa_conv_desc`` of ``include/qa_hip.h`` (all fields 8 bytes)."""

    _fields_ = (
        [("x", _P)] + [(n, _I64) for n in ("x_code", "x_nstride", "x_add",
                                          "rowmajor")]
        + [(n, _I64) for n in ("N", "C", "H", "W", "Cout", "KH", "KW", "SH",
                               "SW", "PH", "PW", "DH", "DW", "G", "OH", "OW")]
        + [("w", _P)] + [(n, _I64) for n in ("w_code", "w_kgp", "w_rows",
                                            "wide", "needs_rowsum")]
        + [(n, _P) for n in ("corr", "boff", "pre_bias", "mult", "shift")]
        + [(n, _I64) for n in ("zp", "qmin", "qmax")]
        + [("lut", _P), ("lut_offset", _I64), ("lut_len", _I64)]
        + [("res", _P)] + [(n, _I64) for n in ("res_nstride", "res_so",
                                              "res_first")]
        + [(n, _I64) for n in ("za", "ma", "sa", "zb", "mb", "sb", "add_sign",
                               "add_zp", "add_qmin", "add_qmax")]
        + [("y", _P)] + [(n, _I64) for n in ("y_code", "y_nstride", "y_so")])


def storage_of(quant_type_bits, signed):
    """``(code, torch dtype, storage offset)`` of a quantization type."""
    if quant_type_bits <= 8:
        return 1, torch.int8, 0 if signed else 128
    if quant_type_bits <= 16:
        return 2, torch.int16, 0 if signed else 32768
    raise NotImplementedError(
        f"{quant_type_bits}-bit tensors are not supported on the device")


class DeviceTensor:
    """A quantized tensor (or view) resident in device memory."""

    def __init__(self, buf, offset, shape, nstride, code, so, qp):
        self.buf, self.offset = buf, int(offset)
        self.shape, self.nstride = tuple(int(s) for s in shape), int(nstride)
        self.code, self.so, self.qp = code, int(so), qp

    @property
    def ptr(self):
        return self.buf.data_ptr() + self.offset * self.buf.element_size()

    @property
    def per_image(self):
        return int(np.prod(self.shape[1:], dtype=np.int64))

    @property
    def contiguous(self):
        return self.nstride == self.per_image

    def to_host(self):
        """Quantized values ``q`` as an int32 NumPy array."""
        n = self.shape[0]
        flat = self.buf[self.offset:self.offset + max(n - 1, 0) * self.nstride
                        + self.per_image]
        rows = [flat[i * self.nstride:i * self.nstride + self.per_image]
                for i in range(n)]
        data = torch.stack(rows) if rows else flat[:0]
        return (data.to(torch.int32).cpu().numpy().reshape(self.shape)
                + self.so)


def _dev(a, dtype):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=dtype)).cuda()


def _ok(rc, what):
    if rc != 0:
        err = native.library().qa_last_error()
        native.library().qa_clear_error()
        raise RuntimeError(f"{what} failed: {err.decode() if err else rc}")


class DeviceExecutor:
    """Plans and runs one integer inference pass for fixed input shapes."""

    def __init__(self, container, input_shapes):
        self.lib = native.require()
        self.c = container
        self.graph = container.graph
        bits, signed = container.layers[0].num_bits, \
            container.layers[0].signed
        self.code, self.dtype, self.so = storage_of(bits, signed)
        self.launches = []  # (name, fn(stream))
        self.keep = []  # host objects that launches point into
        self.tensors = {}
        self.inputs_f32 = {}
        self.outputs_f32 = {}
        self.cuda_graph = None
        self._plan(input_shapes)

    # -------------------------------------------------------------- utils --
    def _new(self, shape, qp):
        n = int(np.prod(shape, dtype=np.int64))
        buf = torch.empty(max(n, 1), dtype=self.dtype, device="cuda")
        per = int(np.prod(shape[1:], dtype=np.int64))
        return DeviceTensor(buf, 0, shape, per, self.code, self.so, qp)

    def _add(self, name, fn):
        self.launches.append((name, fn))

    def _params(self, layer):
        """Device copies of a layer's integer parameters (cached on it)."""
        if getattr(layer, "_dev_params", None) is None:
            layer._dev_params = {}
        return layer._dev_params

    # ------------------------------------------------------------ planning --
    def _plan(self, input_shapes):
        c, g = self.c, self.graph
        for name, shape in input_shapes.items():
            qp = c.qparams[name]
            xf = torch.empty(tuple(shape), dtype=torch.float32, device="cuda")
            t = self._new(tuple(shape), qp)
            self.inputs_f32[name] = xf
            self.tensors[name] = t
            n = xf.numel()
            self._add(f"quantize:{name}", lambda s, xf=xf, t=t, n=n, qp=qp:
                      _ok(self.lib.qa_d_quantize_f32(
                          xf.data_ptr(), t.ptr, t.code, n, qp.scale, qp.zp,
                          qp.qmin, qp.qmax, t.so, s), "quantize"))
        for name in c.const_names:
            qp = c.qparams[name]
            q = c.const_q[name]
            t = self._new(q.shape if q.ndim else (1,), qp)
            t.buf.copy_(torch.from_numpy(
                (q.astype(np.int64) - t.so).astype(
                    np.int8 if self.code == 1 else np.int16).reshape(-1)))
            self.tensors[name] = t

        layers = c.layers
        producer = g.producer_index()
        cons = {}
        for l in layers:
            for i in l.data_inputs:
                cons.setdefault(i, []).append(l)
        absorbed = set()
        for k, layer in enumerate(layers):
            if layer.name in absorbed:
                continue
            layer.check_ready()
            ins = [self.tensors[n] for n in layer.data_inputs]
            if layer.kind in ("conv", "gemm"):
                lut_layer = add_layer = None
                out_name = layer.node.outputs[0]
                users = cons.get(out_name, [])
                if out_name not in g.outputs and len(users) == 1 and \
                        users[0].kind == "lut":
                    lut_layer = users[0]
                    out_name = lut_layer.node.outputs[0]
                    users = cons.get(out_name, [])
                res = None
                if out_name not in g.outputs and len(users) == 1 and \
                        users[0].kind == "add" and \
                        len(users[0].data_inputs) == 2:
                    a = users[0]
                    others = [i for i in a.data_inputs if i != out_name]
                    if len(others) == 1 and others[0] in self.tensors and \
                            producer.get(others[0], -1) < \
                            producer.get(layer.node.outputs[0], 0):
                        add_layer = a
                        res = (others[0], a.data_inputs[0] == others[0])
                outs = self._plan_weighted(layer, ins[0], lut_layer,
                                           add_layer, res)
                final = add_layer or lut_layer or layer
                for l in (lut_layer, add_layer):
                    if l is not None:
                        absorbed.add(l.name)
                self.tensors[final.node.outputs[0]] = outs
                continue
            outs = getattr(self, "_plan_" + layer.kind)(layer, ins)
            for name, t in zip(layer.node.outputs, outs):
                self.tensors[name] = t
        for name in g.outputs:
            t = self.tensors[name]
            if not t.contiguous:
                raise NotImplementedError("graph output must be contiguous")
            yf = torch.empty(t.shape, dtype=torch.float32, device="cuda")
            self.outputs_f32[name] = yf
            n = yf.numel()
            self._add(f"dequantize:{name}", lambda s, t=t, yf=yf, n=n:
                      _ok(self.lib.qa_d_dequantize_f32(
                          t.ptr, t.code, yf.data_ptr(), n, t.qp.scale,
                          t.qp.zp, t.so, s), "dequantize"))

    def _weights_dev(self, layer, x, rowmajor):
        """Packs (once) the layer's weights for the MFMA or VALU path."""
        p = self._params(layer)
        a_off = x.so - layer.in_zp
        key = ("w", a_off, self.code)
        if key in p:
            return p[key]
        if layer.kind == "gemm":
            w = np.ascontiguousarray(layer.w_centered.T)  # [N, K]
            cout, cg, kh, kw, groups = w.shape[0], w.shape[1], 1, 1, 1
        else:
            w = layer.w_centered
            cout, cg, kh, kw = w.shape
            groups = layer.geometry(x.shape)[3]
        w32 = np.ascontiguousarray(w, dtype=np.int32)
        info = None
        if self.code == 1 and not layer.wide and cg * kh * kw < 131072:
            kgp, rows = _I64(0), _I64(0)
            size = self.lib.qa_pack_weights_i8_size(
                cout, cg, kh, kw, groups, ctypes.byref(kgp),
                ctypes.byref(rows))
            wp = np.empty(size, np.int8)
            corr = np.empty(cout, np.int64)
            boff = np.empty(cout, np.int32)
            need = ctypes.c_int32(0)
            rc = self.lib.qa_pack_weights_i8(
                w32.ctypes.data, cout, cg, kh, kw, groups, a_off,
                wp.ctypes.data, corr.ctypes.data, boff.ctypes.data,
                ctypes.byref(need))
            if rc == 0:
                info = dict(w=_dev(wp, np.int8), w_code=1, kgp=kgp.value,
                            rows=rows.value, corr=_dev(corr, np.int64),
                            boff=_dev(boff, np.int32), rowsum=need.value,
                            wide=0)
        if info is None:  # exact VALU path with int64 accumulation
            info = dict(w=_dev(w32.reshape(cout, cg, kh, kw), np.int32),
                        w_code=4, kgp=0, rows=0, corr=None, boff=None,
                        rowsum=0, wide=1)
        cout_all = cout
        info["mult"] = _dev(np.broadcast_to(layer.q_mult, (cout_all,)),
                            np.int64)
        info["shift"] = _dev(np.broadcast_to(layer.shift, (cout_all,)),
                             np.int64)
        info["pre"] = (None if layer.bias_int is None
                       else _dev(layer.bias_int, np.int64))
        p[key] = info
        return info

    def _plan_weighted(self, layer, x, lut_layer, add_layer, res):
        d = ConvDesc()
        if layer.kind == "conv":
            if len(x.shape) != 4:
                raise NotImplementedError("only 2-D convolution")
            strides, pads, dil, groups = layer.geometry(x.shape)
            n, cin, h, w = x.shape
            cout, cg, kh, kw = layer.w_centered.shape
            if cin != cg * groups or cout % groups:
                raise ValueError(f"conv shape mismatch: input C={cin}, "
                                 f"weight={layer.w_centered.shape}, "
                                 f"groups={groups}")
            oh = (h + pads[0] + pads[2] - dil[0] * (kh - 1) - 1) // \
                strides[0] + 1
            ow = (w + pads[1] + pads[3] - dil[1] * (kw - 1) - 1) // \
                strides[1] + 1
            out_shape = (n, cout, oh, ow)
            geo = (n, cin, h, w, cout, kh, kw, strides[0], strides[1],
                   pads[0], pads[1], dil[0], dil[1], groups, oh, ow)
            d.rowmajor = 0
            d.x_nstride = x.nstride
        else:
            k = layer.w_centered.shape[0]
            if x.shape[-1] != k:
                raise ValueError(f"gemm shape mismatch: {x.shape} x "
                                 f"{layer.w_centered.shape}")
            m = int(np.prod(x.shape[:-1]))
            if not (x.contiguous or len(x.shape) == 2):
                raise NotImplementedError("gemm input must be contiguous")
            ncol = layer.w_centered.shape[1]
            out_shape = layer.out_shape(x.shape)
            geo = (m, k, 1, 1, ncol, 1, 1, 1, 1, 0, 0, 1, 1, 1, 1, 1)
            d.rowmajor = 1
            d.x_nstride = x.nstride if len(x.shape) == 2 else k
        info = self._weights_dev(layer, x, d.rowmajor)
        (d.N, d.C, d.H, d.W, d.Cout, d.KH, d.KW, d.SH, d.SW, d.PH, d.PW,
         d.DH, d.DW, d.G, d.OH, d.OW) = geo
        d.x = x.ptr
        d.x_code = x.code
        d.x_add = x.so - layer.in_zp
        d.w = info["w"].data_ptr()
        d.w_code = info["w_code"]
        d.w_kgp = info["kgp"]
        d.w_rows = info["rows"]
        d.wide = info["wide"]
        d.needs_rowsum = info["rowsum"]
        d.corr = info["corr"].data_ptr() if info["corr"] is not None else None
        d.boff = info["boff"].data_ptr() if info["boff"] is not None else None
        d.pre_bias = info["pre"].data_ptr() if info["pre"] is not None \
            else None
        d.mult = info["mult"].data_ptr()
        d.shift = info["shift"].data_ptr()
        d.zp, d.qmin, d.qmax = layer.out_zp, layer.out_qmin, layer.out_qmax
        final_qp = layer.out_qp[0]
        if lut_layer is not None:
            p = self._params(lut_layer)
            if "lut" not in p:
                p["lut"] = _dev(lut_layer.lut, np.int32)
            d.lut = p["lut"].data_ptr()
            d.lut_offset = lut_layer.lut_offset
            d.lut_len = len(lut_layer.lut)
            final_qp = lut_layer.out_qp[0]
        y = self._new(out_shape, final_qp)
        if add_layer is not None:
            rname, first = res
            r = self.tensors[rname]
            if r.shape != tuple(out_shape) or r.code != self.code:
                raise NotImplementedError("residual shape mismatch")
            (ma, sa), (mb, sb) = add_layer.mults
            qa_, qb_ = add_layer.in_qp
            o = add_layer.out_qp[0]
            if layer.kind == "gemm" and not r.contiguous:
                raise NotImplementedError("strided Gemm residual")
            d.res = r.ptr
            d.res_nstride = r.nstride if layer.kind == "conv" else d.Cout
            d.res_so = r.so
            d.res_first = 1 if first else 0
            d.za, d.ma, d.sa = qa_.zp, ma, sa
            d.zb, d.mb, d.sb = qb_.zp, mb, sb
            d.add_sign = add_layer.sign
            d.add_zp, d.add_qmin, d.add_qmax = o.zp, o.qmin, o.qmax
            y.qp = o
        d.y = y.ptr
        d.y_code = y.code
        d.y_nstride = y.nstride if layer.kind == "conv" else d.Cout
        d.y_so = y.so
        self.keep.append(d)
        self._add(f"conv:{layer.name}", lambda s, d=d:
                  _ok(self.lib.qa_d_conv(ctypes.byref(d), s), "qa_d_conv"))
        return y

    def _plan_lut(self, layer, ins):
        x = ins[0]
        p = self._params(layer)
        if "lut" not in p:
            p["lut"] = _dev(layer.lut, np.int32)
        y = self._new(x.shape, layer.out_qp[0])
        lut = p["lut"]
        self._add(f"lut:{layer.name}", lambda s: _ok(self.lib.qa_d_lut(
            x.ptr, x.code, x.nstride, y.ptr, y.code, y.nstride, x.shape[0],
            x.per_image, layer.lut_offset, lut.data_ptr(), len(layer.lut),
            x.so, y.so, s), "qa_d_lut"))
        return [y]

    def _plan_add(self, layer, ins):
        a, b = ins
        if a.shape != b.shape:
            raise NotImplementedError("broadcasting Add on the device")
        (ma, sa), (mb, sb) = layer.mults
        qa_, qb_ = layer.in_qp
        o = layer.out_qp[0]
        y = self._new(a.shape, o)
        self._add(f"add:{layer.name}", lambda s: _ok(self.lib.qa_d_add(
            a.ptr, a.nstride, b.ptr, b.nstride, a.code, y.ptr, y.code,
            y.nstride, a.shape[0], a.per_image, qa_.zp, ma, sa, qb_.zp, mb,
            sb, layer.sign, o.zp, o.qmin, o.qmax, a.so, b.so, y.so, s),
            "qa_d_add"))
        return [y]

    def _plan_mul(self, layer, ins):
        a, b = ins
        if a.shape != b.shape:
            raise NotImplementedError("broadcasting Mul on the device")
        qa_, qb_ = layer.in_qp
        o = layer.out_qp[0]
        y = self._new(a.shape, o)
        self._add(f"mul:{layer.name}", lambda s: _ok(self.lib.qa_d_mul(
            a.ptr, a.nstride, b.ptr, b.nstride, a.code, y.ptr, y.code,
            y.nstride, a.shape[0], a.per_image, qa_.zp, qb_.zp, layer.mult,
            layer.shift, o.zp, o.qmin, o.qmax, a.so, b.so, y.so, s),
            "qa_d_mul"))
        return [y]

    def _plan_concat(self, layer, ins):
        axis = layer.node.attr("axis")
        nd = len(ins[0].shape)
        axis = axis + nd if axis < 0 else axis
        if axis != 1:
            raise NotImplementedError("Concat on the device needs axis 1")
        o = layer.out_qp[0]
        shape = list(ins[0].shape)
        shape[1] = sum(t.shape[1] for t in ins)
        y = self._new(tuple(shape), o)
        inner = int(np.prod(shape[2:], dtype=np.int64))
        off = 0
        for t, qp, (m, s_) in zip(ins, layer.in_qp, layer.mults):
            if qp.scale == o.scale and qp.zp == o.zp:
                m, s_ = IDENTITY
            dst = y.ptr + off * inner * y.buf.element_size()
            self._add(f"concat:{layer.name}", lambda st, t=t, qp=qp, m=m,
                      s_=s_, dst=dst: _ok(self.lib.qa_d_rescale(
                          t.ptr, t.code, t.nstride, dst, y.code, y.nstride,
                          t.shape[0], t.per_image, qp.zp, m, s_, o.zp, o.qmin,
                          o.qmax, t.so, y.so, st), "qa_d_rescale"))
            off += t.shape[1]
        return [y]

    def _plan_gap(self, layer, ins):
        x = ins[0]
        n, ch = x.shape[:2]
        area = int(np.prod(x.shape[2:], dtype=np.int64))
        mult, shift = layer.multiplier(area)
        o = layer.out_qp[0]
        y = self._new((n, ch) + (1,) * (len(x.shape) - 2), o)
        self._add(f"gap:{layer.name}", lambda s: _ok(self.lib.qa_d_gap(
            x.ptr, x.code, x.nstride, n, ch, area, layer.in_zp, x.so, mult,
            shift, o.zp, o.qmin, o.qmax, y.ptr, y.code, y.so, s), "qa_d_gap"))
        return [y]

    def _plan_bn(self, layer, ins):
        x = ins[0]
        if not x.contiguous:
            raise NotImplementedError("BatchNorm on a strided view")
        n, ch = x.shape[:2]
        inner = int(np.prod(x.shape[2:], dtype=np.int64))
        p = self._params(layer)
        if "mult" not in p:
            p["mult"] = _dev(layer.q_mult, np.int64)
            p["shift"] = _dev(layer.shift, np.int64)
            p["post"] = _dev(layer.q_B, np.int64)
        o = layer.out_qp[0]
        y = self._new(x.shape, o)
        self._add(f"bn:{layer.name}", lambda s: _ok(self.lib.qa_d_requantize(
            x.ptr, x.code, y.ptr, y.code, n, ch, inner, p["mult"].data_ptr(),
            p["shift"].data_ptr(), None, p["post"].data_ptr(), o.zp, o.qmin,
            o.qmax, layer.in_zp - x.so, y.so, s), "qa_d_requantize"))
        return [y]

    def _plan_shape(self, layer, ins):
        x = ins[0]
        op = layer.node.op_type
        if op == "Split":
            axis = layer.node.attr("axis", 0)
            axis = axis + len(x.shape) if axis < 0 else axis
            if axis != 1:
                raise NotImplementedError("Split on the device needs axis 1")
            node = layer.node
            if len(node.inputs) > 1 and node.inputs[1]:
                sizes = self.graph.initializers[node.inputs[1]].astype(
                    np.int64).tolist()
            else:
                sizes = node.attr("split") or \
                    [x.shape[1] // len(node.outputs)] * len(node.outputs)
            inner = int(np.prod(x.shape[2:], dtype=np.int64))
            outs, c0 = [], 0
            for sz in sizes:
                shape = (x.shape[0], sz) + x.shape[2:]
                outs.append(DeviceTensor(x.buf, x.offset + c0 * inner, shape,
                                         x.nstride, x.code, x.so, x.qp))
                c0 += sz
            return outs
        if op == "Flatten":
            axis = layer.node.attr("axis", 1)
            if axis != 1:
                raise NotImplementedError("Flatten on the device needs axis 1")
            return [DeviceTensor(x.buf, x.offset, (x.shape[0], x.per_image),
                                 x.nstride, x.code, x.so, x.qp)]
        raise NotImplementedError(f"{op} on the device")

    def _plan_fallback(self, layer, ins):
        op = layer.node.op_type
        x = ins[0]
        if op == "Softmax":
            ax = layer.node.attr("axis", -1 if self.graph.opset >= 13 else 1)
            ax = ax + len(x.shape) if ax < 0 else ax
            if ax != len(x.shape) - 1 or not x.contiguous:
                raise NotImplementedError("Softmax over a non-last axis")
            o = layer.out_qp[0]
            y = self._new(x.shape, o)
            cols = x.shape[-1]
            rows = int(np.prod(x.shape[:-1], dtype=np.int64))
            iq = layer.in_qp[0]
            self._add(f"softmax:{layer.name}", lambda s: _ok(
                self.lib.qa_d_softmax(x.ptr, x.code, rows, cols, iq.scale,
                                      iq.zp, x.so, y.ptr, y.code, o.scale,
                                      o.zp, o.qmin, o.qmax, y.so, s),
                "qa_d_softmax"))
            return [y]
        raise NotImplementedError(f"float fallback of {op} on the device")

    # ------------------------------------------------------------ running --
    def launch(self, stream=None):
        """Queues every launch on ``stream`` (default: torch's current)."""
        s = stream if stream is not None else \
            torch.cuda.current_stream().cuda_stream
        for _, fn in self.launches:
            fn(s)

    def capture(self):
        """Captures the launch sequence into a HIP graph (once)."""
        if self.cuda_graph is None:
            self.launch()  # warm-up outside capture
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                self.launch()
            self.cuda_graph = g
        return self.cuda_graph

    def replay(self):
        if self.cuda_graph is None:
            self.capture()
        self.cuda_graph.replay()

    def run(self, feeds, use_graph=False):
        """Copies float inputs in, runs the pass, returns float outputs."""
        for name, x in feeds.items():
            self.inputs_f32[name].copy_(torch.as_tensor(
                np.ascontiguousarray(x, dtype=np.float32)))
        if use_graph:
            self.replay()
        else:
            self.launch()
        torch.cuda.synchronize()
        return {k: v.cpu().numpy() for k, v in self.outputs_f32.items()}

    def integer_outputs(self):
        return {k: self.tensors[k].to_host() for k in self.graph.outputs}

// More float fallbacks of the integer pass (the reference's dequantize ->
// float operator -> quantize, quant_layers.py:195-205), for operators with
// no integer form:
//   Div / Max / Min of two activations (float32, float_ops.py:217-222) and
//   Pow (float64 cast to float32, :321-325), with broadcasting;
//   ReduceMean over any axes (:594-601);
//   Softmax / LogSoftmax over any axis (float64, :380-395);
//   AveragePool (window sums over the zero-padded input, :563-577).
// Inputs dequantize to the reference's float32 value (float)((q - zp) *
// scale); outputs quantize as qa_quantize_f32 does (double division, half
// to even). Sums run in float64 where the reference sums float32 values
// (ReduceMean, AveragePool) or float64 values in another order (Softmax):
// results agree within one output step. One thread per output element
// (per row for Softmax): these are fallbacks, not hot kernels.
#include <algorithm>

#include "../../include/qa_hip.h"
#include "qa_conv.h"

namespace qa {
namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ float deq(const void* p, int64_t code, int64_t i,
                                     int64_t so, int64_t zp, double scale) {
    return (float)((double)(load_any(p, (int)code, i) + so - zp) * scale);
}

__device__ __forceinline__ void put(void* p, int64_t code, int64_t i,
                                    int64_t so, float v, double scale,
                                    int64_t zp, int64_t qmin, int64_t qmax) {
    store_any(p, (int)code, i, qa_quantize_one(v, scale, zp, qmin, qmax) - so);
}

__global__ __launch_bounds__(kThreads) void k_fb_binary(qa_fb_binary d,
                                                        int64_t total) {
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * kThreads) {
        int64_t rem = i, ao = 0, bo = 0, yo = 0;
        for (int k = (int)d.ndim - 1; k >= 0; --k) {
            const int64_t c = rem % d.shape[k];
            rem /= d.shape[k];
            ao += c * d.as[k];
            bo += c * d.bs[k];
            yo += c * d.ys[k];
        }
        // code 0: a float32 constant operand
        const float a = d.a_code == 0
                            ? ((const float*)d.a)[ao]
                            : deq(d.a, d.a_code, ao, d.a_so, d.a_zp,
                                  d.a_scale);
        const float b = d.b_code == 0
                            ? ((const float*)d.b)[bo]
                            : deq(d.b, d.b_code, bo, d.b_so, d.b_zp,
                                  d.b_scale);
        float v;
        switch ((int)d.op) {
            case 0: v = a / b; break;
            case 1: v = fmaxf(a, b); break;
            case 2: v = fminf(a, b); break;
            default: v = (float)pow((double)a, (double)b);
        }
        // NumPy propagates NaN through maximum / minimum
        if (d.op == 1 || d.op == 2) {
            if (a != a) v = a;
            if (b != b) v = b;
        }
        put(d.y, d.y_code, yo, d.y_so, v, d.out_scale, d.out_zp, d.qmin,
            d.qmax);
    }
}

__global__ __launch_bounds__(kThreads) void k_fb_reduce_mean(qa_fb_reduce d,
                                                             int64_t nout,
                                                             int64_t nred) {
    for (int64_t o = (int64_t)blockIdx.x * kThreads + threadIdx.x; o < nout;
         o += (int64_t)gridDim.x * kThreads) {
        int64_t rem = o, xo = 0;
        for (int k = (int)d.nkeep - 1; k >= 0; --k) {
            const int64_t c = rem % d.keep[k];
            rem /= d.keep[k];
            xo += c * d.xks[k];
        }
        double sum = 0.0;
        for (int64_t r = 0; r < nred; ++r) {
            int64_t rr = r, off = xo;
            for (int k = (int)d.nred - 1; k >= 0; --k) {
                const int64_t c = rr % d.red[k];
                rr /= d.red[k];
                off += c * d.xrs[k];
            }
            sum += (double)deq(d.x, d.x_code, off, d.x_so, d.x_zp,
                               d.x_scale);
        }
        put(d.y, d.y_code, o, d.y_so, (float)(sum / (double)nred),
            d.out_scale, d.out_zp, d.qmin, d.qmax);
    }
}

__global__ __launch_bounds__(kThreads) void k_fb_softmax(qa_fb_softmax d) {
    const int64_t rows = d.outer * d.inner;
    for (int64_t r = (int64_t)blockIdx.x * kThreads + threadIdx.x; r < rows;
         r += (int64_t)gridDim.x * kThreads) {
        const int64_t o = r / d.inner, i = r - o * d.inner;
        const int64_t xb = o * d.xs_o + i * d.xs_i;
        const int64_t yb = o * d.ys_o + i * d.ys_i;
        auto x = [&](int64_t k) {
            return (double)deq(d.x, d.x_code, xb + k * d.xs_k, d.x_so,
                               d.x_zp, d.x_scale);
        };
        double mx = x(0);
        for (int64_t k = 1; k < d.len; ++k) mx = fmax(mx, x(k));
        double sum = 0.0;
        for (int64_t k = 0; k < d.len; ++k) sum += exp(x(k) - mx);
        const double lsum = log(sum);
        for (int64_t k = 0; k < d.len; ++k) {
            const double z = x(k) - mx;
            const float v = d.log ? (float)(z - lsum) : (float)(exp(z) / sum);
            put(d.y, d.y_code, yb + k * d.ys_k, d.y_so, v, d.out_scale,
                d.out_zp, d.qmin, d.qmax);
        }
    }
}

__global__ __launch_bounds__(kThreads) void k_fb_avgpool(qa_fb_avgpool d,
                                                         int64_t total) {
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * kThreads) {
        const int64_t c = i % d.C;
        int64_t r = i / d.C;
        const int64_t ox = r % d.OW;
        r /= d.OW;
        const int64_t oy = r % d.OH;
        const int64_t n = r / d.OH;
        double sum = 0.0;
        int64_t cnt = 0;
        for (int64_t ky = 0; ky < d.KH; ++ky) {
            const int64_t iy = oy * d.SH - d.PT + ky;
            for (int64_t kx = 0; kx < d.KW; ++kx) {
                const int64_t ix = ox * d.SW - d.PL + kx;
                if (iy < 0 || iy >= d.H || ix < 0 || ix >= d.W) continue;
                sum += (double)deq(d.x, d.x_code,
                                   n * d.x_sn + c * d.x_sc + iy * d.x_sh +
                                       ix * d.x_sw,
                                   d.x_so, d.x_zp, d.x_scale);
                ++cnt;
            }
        }
        const int64_t div = d.count_pad ? d.KH * d.KW : cnt;
        put(d.y, d.y_code,
            n * d.y_sn + c * d.y_sc + oy * d.y_sh + ox * d.y_sw, d.y_so,
            (float)(sum / (double)(div > 0 ? div : 1)), d.out_scale,
            d.out_zp, d.qmin, d.qmax);
    }
}

bool code_ok(int64_t c) { return c == 1 || c == 2 || c == 4; }

unsigned blocks_for(int64_t n) {
    return (unsigned)std::min<int64_t>(std::max<int64_t>(ceil_div(n, kThreads),
                                                         1),
                                       1 << 16);
}

bool launched(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_hip_error(what, e);
        return false;
    }
    return true;
}

}  // namespace
}  // namespace qa

using namespace qa;

QA_API int qa_d_fb_binary(const qa_fb_binary* d, void* stream) {
    if (!d || d->ndim < 1 || d->ndim > 6 ||
        !(d->a_code == 0 || code_ok(d->a_code)) ||
        !(d->b_code == 0 || code_ok(d->b_code)) || !code_ok(d->y_code) ||
        d->op < 0 ||
        d->op > 3) {
        set_error("qa_d_fb_binary", "bad descriptor");
        return -1;
    }
    int64_t total = 1;
    for (int k = 0; k < d->ndim; ++k) total *= std::max<int64_t>(d->shape[k],
                                                                 0);
    if (total == 0) return 0;
    if (!d->a || !d->b || !d->y) {
        set_error("qa_d_fb_binary", "null tensor");
        return -1;
    }
    k_fb_binary<<<blocks_for(total), kThreads, 0, (hipStream_t)stream>>>(
        *d, total);
    return launched("qa_d_fb_binary") ? 0 : -1;
}

QA_API int qa_d_fb_reduce_mean(const qa_fb_reduce* d, void* stream) {
    if (!d || d->nkeep < 0 || d->nkeep > 6 || d->nred < 1 || d->nred > 6 ||
        !code_ok(d->x_code) || !code_ok(d->y_code)) {
        set_error("qa_d_fb_reduce_mean", "bad descriptor");
        return -1;
    }
    int64_t nout = 1, nred = 1;
    for (int k = 0; k < d->nkeep; ++k) nout *= std::max<int64_t>(d->keep[k], 0);
    for (int k = 0; k < d->nred; ++k) nred *= std::max<int64_t>(d->red[k], 0);
    if (nout == 0) return 0;
    if (nred == 0 || !d->x || !d->y) {
        set_error("qa_d_fb_reduce_mean", "empty reduction or null tensor");
        return -1;
    }
    k_fb_reduce_mean<<<blocks_for(nout), kThreads, 0, (hipStream_t)stream>>>(
        *d, nout, nred);
    return launched("qa_d_fb_reduce_mean") ? 0 : -1;
}

QA_API int qa_d_fb_softmax(const qa_fb_softmax* d, void* stream) {
    if (!d || !code_ok(d->x_code) || !code_ok(d->y_code) || d->outer < 0 ||
        d->inner < 0 || d->len < 0) {
        set_error("qa_d_fb_softmax", "bad descriptor");
        return -1;
    }
    if (d->outer * d->inner == 0 || d->len == 0) return 0;
    if (!d->x || !d->y) {
        set_error("qa_d_fb_softmax", "null tensor");
        return -1;
    }
    k_fb_softmax<<<blocks_for(d->outer * d->inner), kThreads, 0,
                   (hipStream_t)stream>>>(*d);
    return launched("qa_d_fb_softmax") ? 0 : -1;
}

QA_API int qa_d_fb_avgpool(const qa_fb_avgpool* d, void* stream) {
    if (!d || !code_ok(d->x_code) || !code_ok(d->y_code) || d->KH < 1 ||
        d->KW < 1 || d->SH < 1 || d->SW < 1 || d->N < 0 || d->C < 0 ||
        d->OH < 0 || d->OW < 0) {
        set_error("qa_d_fb_avgpool", "bad descriptor");
        return -1;
    }
    const int64_t total = d->N * d->C * d->OH * d->OW;
    if (total == 0) return 0;
    if (!d->x || !d->y) {
        set_error("qa_d_fb_avgpool", "null tensor");
        return -1;
    }
    k_fb_avgpool<<<blocks_for(total), kThreads, 0, (hipStream_t)stream>>>(
        *d, total);
    return launched("qa_d_fb_avgpool") ? 0 : -1;
}

// Float fallbacks that move values to other positions, each value then
// requantized with the output parameters (the reference's dequantize ->
// float operator -> quantize, quant_layers.py:195-205):
//   Pad in reflect / edge mode or with a non-zero constant (float_ops.py:
//   499-513; the scale-preserving Pad is qa_d_pad_nd);
//   Gather with an index array (float_ops.py:490-496);
//   Cast to float16, bool and the integer types (float_ops.py:398-402).
// Inputs dequantize to the reference's float32 value (float)((q - zp) *
// scale). One thread per output element: these are fallbacks, not hot
// kernels.
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

// round_half_even(t / scale) + zp, clipped: utils.quantize on a float64
// array (the float32 entry divides the same double quotient).
__device__ __forceinline__ int64_t quantize_double(double t, double scale,
                                                   int64_t zp, int64_t qmin,
                                                   int64_t qmax) {
    double v = rint(t / scale) + (double)zp;
    if (v != v) return INT32_MIN;
    v = fmin(fmax(v, (double)qmin), (double)qmax);
    return (int64_t)v;
}

// NumPy's float32 -> int32 conversion on x86-64 (cvttss2si): truncation,
// and the "integer indefinite" INT32_MIN for values outside the range.
__device__ __forceinline__ int32_t trunc_i32(float v) {
    return (v >= -2147483648.0f && v < 2147483648.0f) ? (int32_t)v
                                                       : INT32_MIN;
}

__device__ __forceinline__ double cast_value(float v, int64_t to) {
    switch ((int)to) {
        case 10: return (double)(float)(_Float16)v;
        case 9: return v != 0.0f ? 1.0 : 0.0;
        case 6: return (double)trunc_i32(v);
        case 3: return (double)(int8_t)trunc_i32(v);
        case 2: return (double)(uint8_t)trunc_i32(v);
        case 5: return (double)(int16_t)trunc_i32(v);
        case 4: return (double)(uint16_t)trunc_i32(v);
        case 7:
            return (double)((v >= -9223372036854775808.0f &&
                             v < 9223372036854775808.0f)
                                ? (int64_t)v
                                : INT64_MIN);
        default: return (double)v;  // 1 float32, 11 float64
    }
}

// Source index along an axis of n elements for output coordinate c.
// Returns false (constant mode) when it lies in the padding.
__device__ __forceinline__ bool pad_source(int64_t c, int64_t lo, int64_t n,
                                           int64_t mode, int64_t* j) {
    int64_t s = c - lo;
    if (s >= 0 && s < n) {
        *j = s;
        return true;
    }
    if (mode == 0) return false;
    if (mode == 2 || n == 1) {
        *j = s < 0 ? 0 : n - 1;
        return true;
    }
    const int64_t period = 2 * (n - 1);
    s %= period;
    if (s < 0) s += period;
    *j = s < n ? s : period - s;
    return true;
}

__global__ __launch_bounds__(kThreads) void k_fb_pad(qa_fb_pad d,
                                                     int64_t total) {
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * kThreads) {
        int64_t rem = i, xo = 0, yo = 0;
        bool inside = true;
        for (int k = (int)d.ndim - 1; k >= 0; --k) {
            const int64_t c = rem % d.shape[k];
            rem /= d.shape[k];
            yo += c * d.ys[k];
            int64_t j = 0;
            inside = pad_source(c, d.lo[k], d.xshape[k], d.mode, &j) && inside;
            xo += j * d.xs[k];
        }
        const float v = inside ? deq(d.x, d.x_code, xo, d.x_so, d.x_zp,
                                     d.x_scale)
                               : (float)d.value;
        store_any(d.y, (int)d.y_code, yo,
                  qa_quantize_one(v, d.out_scale, d.out_zp, d.qmin, d.qmax) -
                      d.y_so);
    }
}

__global__ __launch_bounds__(kThreads) void k_fb_gather(qa_fb_gather d,
                                                        int64_t total) {
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * kThreads) {
        int64_t rem = i, xo = 0, yo = 0;
        for (int k = (int)d.ndim - 1; k >= 0; --k) {
            const int64_t c = rem % d.shape[k];
            rem /= d.shape[k];
            yo += c * d.ys[k];
            xo += (k == d.axis ? d.idx[c] : c) * d.xs[k];
        }
        const float v = deq(d.x, d.x_code, xo, d.x_so, d.x_zp, d.x_scale);
        store_any(d.y, (int)d.y_code, yo,
                  quantize_double(cast_value(v, d.cast_to), d.out_scale,
                                  d.out_zp, d.qmin, d.qmax) -
                      d.y_so);
    }
}

bool code_ok(int64_t c) { return c == 1 || c == 2 || c == 4; }

bool cast_ok(int64_t to) {
    switch ((int)to) {
        case 1: case 2: case 3: case 4: case 5: case 6: case 7: case 9:
        case 10: case 11:
            return true;
        default:
            return false;
    }
}

unsigned blocks_for(int64_t total) {
    return (unsigned)std::min<int64_t>(ceil_div(total, kThreads), 1 << 16);
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

QA_API int qa_d_fb_pad(const qa_fb_pad* d, void* stream) {
    if (!d || d->ndim < 1 || d->ndim > 6 || !code_ok(d->x_code) ||
        !code_ok(d->y_code) || d->mode < 0 || d->mode > 2) {
        set_error("qa_d_fb_pad", "bad descriptor");
        return -1;
    }
    int64_t total = 1;
    for (int k = 0; k < d->ndim; ++k) {
        if (d->shape[k] < 0 || d->xshape[k] < 0 || d->lo[k] < 0) {
            set_error("qa_d_fb_pad", "negative extent or padding");
            return -1;
        }
        // every output coordinate must map into the input in the copying
        // modes: an empty axis has nothing to copy
        if (d->mode != 0 && d->xshape[k] == 0 && d->shape[k] > 0) {
            set_error("qa_d_fb_pad", "reflect / edge padding of an empty axis");
            return -1;
        }
        total *= d->shape[k];
    }
    if (total == 0) return 0;
    if (!d->x || !d->y) {
        set_error("qa_d_fb_pad", "null tensor");
        return -1;
    }
    k_fb_pad<<<blocks_for(total), kThreads, 0, (hipStream_t)stream>>>(*d,
                                                                      total);
    return launched("qa_d_fb_pad") ? 0 : -1;
}

QA_API int qa_d_fb_gather(const qa_fb_gather* d, void* stream) {
    if (!d || d->ndim < 1 || d->ndim > 6 || !code_ok(d->x_code) ||
        !code_ok(d->y_code) || d->axis < -1 || d->axis >= d->ndim ||
        !cast_ok(d->cast_to)) {
        set_error("qa_d_fb_gather", "bad descriptor");
        return -1;
    }
    int64_t total = 1;
    for (int k = 0; k < d->ndim; ++k) {
        if (d->shape[k] < 0) {
            set_error("qa_d_fb_gather", "negative extent");
            return -1;
        }
        total *= d->shape[k];
    }
    if (d->axis >= 0 && (d->shape[d->axis] != d->nidx || !d->idx)) {
        set_error("qa_d_fb_gather", "index array does not match the axis");
        return -1;
    }
    if (total == 0) return 0;
    if (!d->x || !d->y) {
        set_error("qa_d_fb_gather", "null tensor");
        return -1;
    }
    k_fb_gather<<<blocks_for(total), kThreads, 0, (hipStream_t)stream>>>(
        *d, total);
    return launched("qa_d_fb_gather") ? 0 : -1;
}

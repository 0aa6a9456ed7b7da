// Whole-tensor operators of the quantized graph that are not element-wise:
// GlobalAveragePool (integer sum + requantize, quant_layers.py:563-590) and
// the float Softmax fallback (dequantize -> float64 softmax -> quantize,
// quant_layers.py:195-205 with float_ops.py:380-385).
#include "qa_common.h"

namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ int64_t load_s(const void* x, int code, int64_t i) {
    switch (code) {
        case 1: return ((const int8_t*)x)[i];
        case 2: return ((const int16_t*)x)[i];
        default: return ((const int32_t*)x)[i];
    }
}

__device__ __forceinline__ void store_s(void* y, int code, int64_t i,
                                        int64_t v) {
    switch (code) {
        case 1: ((int8_t*)y)[i] = (int8_t)v; break;
        case 2: ((int16_t*)y)[i] = (int16_t)v; break;
        default: ((int32_t*)y)[i] = (int32_t)v; break;
    }
}

__device__ __forceinline__ int64_t wave_sum(int64_t v) {
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

// One wave per (n, c) plane: acc = sum(q - zp_in) in int64, then
// out = clip(mbqm(acc, mult, shift) + zp_out) - out_so.
__global__ __launch_bounds__(kThreads) void k_gap(
    const void* __restrict__ x, int in_code, int64_t x_nstride, int64_t N,
    int64_t C, int64_t HW, int64_t zp_in, int64_t in_so, int64_t mult,
    int64_t shift, int64_t zp_out, int64_t qmin, int64_t qmax, void* out,
    int out_code, int64_t out_so) {
    const int64_t plane = (int64_t)blockIdx.x * (kThreads / 64) +
                          (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (plane >= N * C) return;
    const int64_t n = plane / C, c = plane - n * C;
    const int64_t base = n * x_nstride + c * HW;
    int64_t s = 0;
    for (int64_t i = lane; i < HW; i += 64) s += load_s(x, in_code, base + i);
    s = wave_sum(s);
    if (lane == 0) {
        const int64_t acc = s + HW * (in_so - zp_in);
        const int64_t q =
            qa_clip128(qa_mbqm(acc, mult, shift) + zp_out, qmin, qmax);
        store_s(out, out_code, plane, q - out_so);
    }
}

__device__ double block_reduce(double v, bool is_max, double* sh) {
    for (int off = 32; off > 0; off >>= 1) {
        const double o = __shfl_xor(v, off);
        v = is_max ? fmax(v, o) : v + o;
    }
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) sh[w] = v;
    __syncthreads();
    double r = sh[0];
    for (int i = 1; i < kThreads / 64; ++i) r = is_max ? fmax(r, sh[i]) : r + sh[i];
    return r;
}

// One work-group per row of `cols` values.
__global__ __launch_bounds__(kThreads) void k_softmax(
    const void* __restrict__ x, int in_code, int64_t rows, int64_t cols,
    double in_scale, int64_t in_zp, int64_t in_so, void* out, int out_code,
    double out_scale, int64_t out_zp, int64_t qmin, int64_t qmax,
    int64_t out_so) {
    __shared__ double sh[kThreads / 64];
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        const int64_t base = r * cols;
        double mx = -INFINITY;
        for (int64_t i = threadIdx.x; i < cols; i += kThreads) {
            const float xf = (float)((double)(load_s(x, in_code, base + i) +
                                              in_so - in_zp) * in_scale);
            mx = fmax(mx, (double)xf);
        }
        mx = block_reduce(mx, true, sh);
        double sum = 0.0;
        for (int64_t i = threadIdx.x; i < cols; i += kThreads) {
            const float xf = (float)((double)(load_s(x, in_code, base + i) +
                                              in_so - in_zp) * in_scale);
            sum += exp((double)xf - mx);
        }
        sum = block_reduce(sum, false, sh);
        for (int64_t i = threadIdx.x; i < cols; i += kThreads) {
            const float xf = (float)((double)(load_s(x, in_code, base + i) +
                                              in_so - in_zp) * in_scale);
            const float y = (float)(exp((double)xf - mx) / sum);
            store_s(out, out_code, base + i,
                    qa_quantize_one(y, out_scale, out_zp, qmin, qmax) - out_so);
        }
        __syncthreads();
    }
}

bool launched(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        qa::set_hip_error(what, e);
        return false;
    }
    return true;
}

}  // namespace

// GlobalAveragePool of device tensor x [N, C, HW] (image stride x_nstride)
// into out [N, C] with a scalar multiplier (in_scale / (out_scale * HW)).
QA_API int qa_d_gap(const void* x, int in_code, int64_t x_nstride, int64_t N,
                    int64_t C, int64_t HW, int64_t zp_in, int64_t in_so,
                    int64_t mult, int64_t shift, int64_t zp_out, int64_t qmin,
                    int64_t qmax, void* out, int out_code, int64_t out_so,
                    void* stream) {
    if (N * C <= 0) return 0;
    hipStream_t st = stream ? (hipStream_t)stream : qa::stream();
    const int64_t blocks = qa::ceil_div(N * C, kThreads / 64);
    k_gap<<<(unsigned)blocks, kThreads, 0, st>>>(
        x, in_code, x_nstride, N, C, HW, zp_in, in_so, mult, shift, zp_out,
        qmin, qmax, out, out_code, out_so);
    return launched("qa_d_gap") ? 0 : -1;
}

// Softmax over the last axis of a [rows, cols] device tensor through float:
// dequantize to float32, softmax in float64, cast to float32, quantize.
QA_API int qa_d_softmax(const void* x, int in_code, int64_t rows, int64_t cols,
                        double in_scale, int64_t in_zp, int64_t in_so,
                        void* out, int out_code, double out_scale,
                        int64_t out_zp, int64_t qmin, int64_t qmax,
                        int64_t out_so, void* stream) {
    if (rows <= 0 || cols <= 0) return 0;
    hipStream_t st = stream ? (hipStream_t)stream : qa::stream();
    const unsigned blocks = (unsigned)(rows < 65535 ? rows : 65535);
    k_softmax<<<blocks, kThreads, 0, st>>>(x, in_code, rows, cols, in_scale,
                                           in_zp, in_so, out, out_code,
                                           out_scale, out_zp, qmin, qmax,
                                           out_so);
    return launched("qa_d_softmax") ? 0 : -1;
}

// Whole-tensor operators of the quantized graph that are not element-wise:
// GlobalAveragePool (integer sum + requantize, quant_layers.py:563-590) and
// the float Softmax fallback (dequantize -> float64 softmax -> quantize,
// quant_layers.py:195-205 with float_ops.py:380-385). The exponentials are
// normalized by one reciprocal of their sum a row (the reference divides
// each: the float64 results differ by at most one unit in the last place,
// far below the float32 rounding that follows, and the outputs agree
// within one quantization step).
#include <algorithm>

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

// GlobalAveragePool: acc = sum over the HW pixels of (q - zp_in) in int64,
// out = clip(mbqm(acc, mult, shift) + zp_out) - out_so. Element (n, c, p) of
// x at x + n*x_sn + c*x_sc + p*x_sp. Channels-last inputs (x_sc == 1) use one
// thread per (n, c), so neighbouring threads read neighbouring bytes.
__global__ __launch_bounds__(kThreads) void k_gap_cl(
    const void* __restrict__ x, int in_code, int64_t x_sn, int64_t x_sp,
    int64_t N, int64_t C, int64_t HW, int64_t zp_in, int64_t in_so,
    int64_t mult, int64_t shift, int64_t zp_out, int64_t qmin, int64_t qmax,
    void* out, int out_code, int64_t out_sn, int64_t out_so) {
    const int64_t c = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    const int64_t n = blockIdx.y;
    if (c >= C) return;
    const int64_t base = n * x_sn + c;
    int64_t s = 0;
    for (int64_t p = 0; p < HW; ++p) s += load_s(x, in_code, base + p * x_sp);
    const int64_t acc = s + HW * (in_so - zp_in);
    const int64_t q =
        qa_clip128(qa_mbqm(acc, mult, shift) + zp_out, qmin, qmax);
    store_s(out, out_code, n * out_sn + c, q - out_so);
}

// Channels-last int8 input with C, the strides and the base multiples of 4:
// a thread sums 4 channels (one word per pixel) over a quarter of the
// pixels (the 4 waves of a work-group take pixels w, w+4, ...); the
// partial sums meet in LDS and wave 0 requantizes and stores.
__global__ __launch_bounds__(kThreads) void k_gap_cl4(
    const int8_t* __restrict__ x, int64_t x_sn, int64_t x_sp, int64_t C,
    int64_t HW, int64_t zp_in, int64_t in_so, int64_t mult, int64_t shift,
    int64_t zp_out, int64_t qmin, int64_t qmax, void* out, int out_code,
    int64_t out_sn, int64_t out_so) {
    __shared__ int part[3][4][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t c = ((int64_t)blockIdx.x * 64 + lane) * 4;
    const int64_t n = blockIdx.y;
    int s[4] = {0, 0, 0, 0};
    if (c < C) {
        const int8_t* p = x + n * x_sn + c;
#pragma unroll 4
        for (int64_t q = wave; q < HW; q += 4) {
            const uint32_t w = *(const uint32_t*)(p + q * x_sp);
#pragma unroll
            for (int r = 0; r < 4; ++r) s[r] += (int)(int8_t)(w >> (8 * r));
        }
    }
    if (wave > 0) {
#pragma unroll
        for (int r = 0; r < 4; ++r) part[wave - 1][r][lane] = s[r];
    }
    __syncthreads();
    if (wave > 0 || c >= C) return;
#pragma unroll
    for (int r = 0; r < 4; ++r)
        s[r] += part[0][r][lane] + part[1][r][lane] + part[2][r][lane];
    int64_t q[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int64_t acc = (int64_t)s[r] + HW * (in_so - zp_in);
        q[r] = qa_clip128(qa_mbqm(acc, mult, shift) + zp_out, qmin, qmax) -
               out_so;
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) store_s(out, out_code, n * out_sn + c + r, q[r]);
}

// Planar inputs: one wave per (n, c) plane.
__global__ __launch_bounds__(kThreads) void k_gap_planar(
    const void* __restrict__ x, int in_code, int64_t x_sn, int64_t x_sc,
    int64_t N, int64_t C, int64_t HW, int64_t zp_in, int64_t in_so,
    int64_t mult, int64_t shift, int64_t zp_out, int64_t qmin, int64_t qmax,
    void* out, int out_code, int64_t out_sn, int64_t out_so) {
    const int64_t plane = (int64_t)blockIdx.x * (kThreads / 64) +
                          (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (plane >= N * C) return;
    const int64_t n = plane / C, c = plane - n * C;
    const int64_t base = n * x_sn + c * x_sc;
    int64_t s = 0;
    for (int64_t i = lane; i < HW; i += 64) s += load_s(x, in_code, base + i);
    s = wave_sum(s);
    if (lane == 0) {
        const int64_t acc = s + HW * (in_so - zp_in);
        const int64_t q =
            qa_clip128(qa_mbqm(acc, mult, shift) + zp_out, qmin, qmax);
        store_s(out, out_code, n * out_sn + c, q - out_so);
    }
}

// Graph input, int8 storage with 4 bytes a pixel (C <= 4) and HW a
// multiple of 4: a thread quantizes 4 consecutive pixels (one 16-byte load
// per input plane, one 16-byte store), over a grid-strided range.
__global__ __launch_bounds__(kThreads) void k_quantize_cl4x4(
    const float* __restrict__ x, int64_t N, int64_t C, int64_t HW,
    int8_t* __restrict__ y, double scale, double inv, int64_t zp,
    int64_t qmin, int64_t qmax, int64_t so) {
    const int64_t groups = N * HW / 4;
    for (int64_t gi = (int64_t)blockIdx.x * kThreads + threadIdx.x;
         gi < groups; gi += (int64_t)gridDim.x * kThreads) {
        const int64_t i = gi * 4;  // first pixel
        const int64_t n = i / HW, p = i - n * HW;
        uint32_t w[4] = {0, 0, 0, 0};
        for (int64_t c = 0; c < C; ++c) {
            const float4 v = *(const float4*)(x + (n * C + c) * HW + p);
            const float f[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int k = 0; k < 4; ++k)
                w[k] |= (uint32_t)(uint8_t)(qa_quantize_one_fast(
                                                f[k], scale, inv, zp, qmin,
                                                qmax) -
                                            so)
                        << (8 * c);
        }
        *(uint4*)(y + i * 4) = make_uint4(w[0], w[1], w[2], w[3]);
    }
}

// Graph input: float32 NCHW -> int8 in the row order of a convolution
// whose stride is its kernel (KH x KW, no padding, H % KH == W % KW == 0):
// row (n, py, px) holds the patch's kernel rows ky = 0..KH-1 of KW pixels,
// 4 bytes a pixel (channel c in byte c, 0 above C), the bytes
// k_quantize_cl4x4 writes for that pixel. A thread quantizes 4 pixels of
// one image row (KW % 4 == 0: one patch) and stores their 16 bytes.
__global__ __launch_bounds__(kThreads) void k_quantize_patches(
    const float* __restrict__ x, int64_t N, int64_t C, int H, int W, int KH,
    int KW, int8_t* __restrict__ y, double scale, double inv, int64_t zp,
    int64_t qmin, int64_t qmax, int64_t so) {
    const int64_t HW = (int64_t)H * W;
    const int64_t groups = N * HW / 4;
    const int OH = H / KH, OW = W / KW;
    for (int64_t gi = (int64_t)blockIdx.x * kThreads + threadIdx.x;
         gi < groups; gi += (int64_t)gridDim.x * kThreads) {
        const int64_t i = gi * 4;  // first pixel
        const int64_t n = i / HW;
        const int p = (int)(i - n * HW);
        const int iy = p / W, ix = p - iy * W;
        const int py = iy / KH, ky = iy - py * KH;
        const int px = ix / KW, kx = ix - px * KW;
        uint32_t w[4] = {0, 0, 0, 0};
        for (int64_t c = 0; c < C; ++c) {
            const float4 v = *(const float4*)(x + (n * C + c) * HW + p);
            const float f[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int k = 0; k < 4; ++k)
                w[k] |= (uint32_t)(uint8_t)(qa_quantize_one_fast(
                                                f[k], scale, inv, zp, qmin,
                                                qmax) -
                                            so)
                        << (8 * c);
        }
        const int64_t row = (n * OH + py) * OW + px;
        *(uint4*)(y + ((row * KH + ky) * KW + kx) * 4) =
            make_uint4(w[0], w[1], w[2], w[3]);
    }
}

// Graph input: float32 NCHW -> quantized channels-last with pixel stride
// y_sp >= C (padding channels written as 0), one thread per pixel.
template <class TOut>
__global__ __launch_bounds__(kThreads) void k_quantize_cl(
    const float* __restrict__ x, int64_t N, int64_t C, int64_t HW,
    TOut* __restrict__ y, int64_t y_sp, double scale, double inv, int64_t zp,
    int64_t qmin, int64_t qmax, int64_t so, int word) {
    const int64_t total = N * HW;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * kThreads) {
        const int64_t n = i / HW, p = i - n * HW;
        TOut* dst = y + i * y_sp;
        if (word) {  // int8, 4 bytes a pixel, aligned: one word store
            uint32_t w = 0;
            for (int64_t c = 0; c < C; ++c)
                w |= (uint32_t)(uint8_t)(qa_quantize_one_fast(
                                             x[(n * C + c) * HW + p], scale,
                                             inv, zp, qmin, qmax) -
                                         so)
                     << (8 * c);
            *(uint32_t*)dst = w;
            continue;
        }
        for (int64_t c = 0; c < y_sp; ++c) {
            int64_t v = 0;
            if (c < C)
                v = qa_quantize_one_fast(x[(n * C + c) * HW + p], scale, inv,
                                         zp, qmin, qmax) - so;
            dst[c] = (TOut)v;
        }
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

// One work-group per row of `cols` values. Rows of at most kThreads * PER
// values are read once and their exponentials kept in registers; longer
// rows take three passes. Summation order is the same either way (thread
// t adds its values t, t + kThreads, ... in order, then the block
// reduction). outf (optional) receives the dequantized output,
// (q - out_zp) * out_scale, as qa_d_dequantize_f32 computes it.
constexpr int SOFTMAX_PER = 8;

__global__ __launch_bounds__(kThreads) void k_softmax(
    const void* __restrict__ x, int in_code, int64_t rows, int64_t cols,
    double in_scale, int64_t in_zp, int64_t in_so, void* out, int out_code,
    double out_scale, int64_t out_zp, int64_t qmin, int64_t qmax,
    int64_t out_so, float* __restrict__ outf) {
    __shared__ double sh[kThreads / 64];
    const bool held = cols <= (int64_t)kThreads * SOFTMAX_PER;
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        const int64_t base = r * cols;
        auto value = [&](int64_t i) {
            return (float)((double)(load_s(x, in_code, base + i) + in_so -
                                    in_zp) *
                           in_scale);
        };
        auto emit = [&](int64_t i, double e, double rsum) {
            const float y = (float)(e * rsum);
            const int64_t q = qa_quantize_one(y, out_scale, out_zp, qmin, qmax);
            store_s(out, out_code, base + i, q - out_so);
            if (outf)
                outf[base + i] =
                    (float)((double)(q - out_zp) * out_scale);
        };
        if (held) {
            float xf[SOFTMAX_PER];
            double mx = -INFINITY;
#pragma unroll
            for (int k = 0; k < SOFTMAX_PER; ++k) {
                const int64_t i = threadIdx.x + (int64_t)k * kThreads;
                xf[k] = i < cols ? value(i) : 0.0f;
                if (i < cols) mx = fmax(mx, (double)xf[k]);
            }
            mx = block_reduce(mx, true, sh);
            double e[SOFTMAX_PER], sum = 0.0;
#pragma unroll
            for (int k = 0; k < SOFTMAX_PER; ++k) {
                const int64_t i = threadIdx.x + (int64_t)k * kThreads;
                e[k] = i < cols ? exp((double)xf[k] - mx) : 0.0;
                sum += e[k];
            }
            sum = block_reduce(sum, false, sh);
            const double rsum = 1.0 / sum;
#pragma unroll
            for (int k = 0; k < SOFTMAX_PER; ++k) {
                const int64_t i = threadIdx.x + (int64_t)k * kThreads;
                if (i < cols) emit(i, e[k], rsum);
            }
        } else {
            double mx = -INFINITY;
            for (int64_t i = threadIdx.x; i < cols; i += kThreads)
                mx = fmax(mx, (double)value(i));
            mx = block_reduce(mx, true, sh);
            double sum = 0.0;
            for (int64_t i = threadIdx.x; i < cols; i += kThreads)
                sum += exp((double)value(i) - mx);
            sum = block_reduce(sum, false, sh);
            const double rsum = 1.0 / sum;
            for (int64_t i = threadIdx.x; i < cols; i += kThreads)
                emit(i, exp((double)value(i) - mx), rsum);
        }
        __syncthreads();
    }
}

// Rows of at most GS * PER values: GS lanes per row (64 / GS rows per
// wave, 4 waves per work-group), the row held in registers, reductions by
// lane shuffles within the lane group (no LDS, no barrier). Same float32
// inputs, float64 exponentials and sums and quantization as k_softmax; the
// maximum is taken over the float32 values (exact), and only the summation
// order differs.
template <int GS, int PER, class TI, class TO>
__global__ __launch_bounds__(kThreads) void k_softmax_rows(
    const TI* __restrict__ x, int64_t rows, int64_t cols, double in_scale,
    int64_t in_zp, int64_t in_so, TO* __restrict__ out, double out_scale,
    int64_t out_zp, int64_t qmin, int64_t qmax, int64_t out_so,
    float* __restrict__ outf) {
    constexpr int RPW = 64 / GS;  // rows per wave
    const int lane = threadIdx.x & 63;
    const int gl = lane % GS;
    const double inv = 1.0 / out_scale;
    const bool f32ok = qa_f32_form_ok(out_scale, out_zp, qmin, qmax);
    const float invf = (float)inv;
    const int64_t first = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * RPW +
                          lane / GS;
    for (int64_t r = first; r - lane / GS < rows;
         r += (int64_t)gridDim.x * 4 * RPW) {
        const bool live = r < rows;
        const int64_t base = (live ? r : 0) * cols;
        float xf[PER];
        float mx = -INFINITY;
#pragma unroll
        for (int k = 0; k < PER; ++k) {
            const int64_t i = gl + GS * k;
            xf[k] = live && i < cols
                        ? (float)((double)((int64_t)x[base + i] + in_so -
                                           in_zp) *
                                  in_scale)
                        : -INFINITY;
            mx = fmaxf(mx, xf[k]);
        }
#pragma unroll
        for (int o = GS / 2; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
        double e[PER], sum = 0.0;
#pragma unroll
        for (int k = 0; k < PER; ++k) {
            e[k] = gl + GS * k < cols ? exp((double)xf[k] - (double)mx) : 0.0;
            sum += e[k];
        }
#pragma unroll
        for (int o = GS / 2; o > 0; o >>= 1) sum += __shfl_xor(sum, o);
        const double rsum = 1.0 / sum;  // one division a row
        if (!live) continue;
#pragma unroll
        for (int k = 0; k < PER; ++k) {
            const int64_t i = gl + GS * k;
            if (i >= cols) continue;
            const float y = (float)(e[k] * rsum);
            const int64_t q = qa_quantize_mixed(y, f32ok, invf, out_scale, inv,
                                                out_zp, qmin, qmax);
            out[base + i] = (TO)(q - out_so);
            if (outf) outf[base + i] = (float)((double)(q - out_zp) * out_scale);
        }
    }
}

// int8 Softmax rows through a table of exponentials: t[256 m + s] =
// exp(F(s) - F(m)) in float64 for stored bytes s <= m (index byte + 128),
// F(b) = float32((b + in_so - in_zp) * in_scale), the values k_softmax_rows
// exponentiates (F is non-decreasing, so a row's maximum is F of its
// largest byte). Built once per layer.
__global__ __launch_bounds__(kThreads) void k_softmax_table(
    double in_scale, int64_t in_zp, int64_t in_so, double* __restrict__ t) {
    const int i = blockIdx.x * kThreads + threadIdx.x;
    if (i >= 65536) return;
    const int m = i >> 8, s = i & 255;
    const float fs = (float)((double)((int64_t)(s - 128) + in_so - in_zp) *
                             in_scale);
    const float fm = (float)((double)((int64_t)(m - 128) + in_so - in_zp) *
                             in_scale);
    t[i] = s <= m ? exp((double)fs - (double)fm) : 0.0;
}

// k_softmax_rows for int8 input and output with the exponentials read from
// k_softmax_table: the same float64 values, summed in the same order, so
// the results are those of k_softmax_rows. outf (optional): the dequantized
// output, as k_softmax_rows writes it.
// qa_quantize_one_fast out of line (the callers' rare near-tie values)
__device__ __noinline__ int softmax_quant_exact(float y, double scale,
                                                double inv, int64_t zp,
                                                int64_t qmin, int64_t qmax) {
    return (int)qa_quantize_one_fast(y, scale, inv, zp, qmin, qmax);
}

template <int GS, int PER>
__global__ __launch_bounds__(kThreads) void k_softmax_rows_lut(
    const int8_t* __restrict__ x, int64_t rows, int64_t cols,
    const double* __restrict__ t, int8_t* __restrict__ out, double out_scale,
    int64_t out_zp, int64_t qmin, int64_t qmax, int64_t out_so,
    float* __restrict__ outf) {
    constexpr int RPW = 64 / GS;  // rows per wave
    const int lane = threadIdx.x & 63;
    const int gl = lane % GS;
    const double inv = 1.0 / out_scale;
    const bool f32ok = qa_f32_form_ok(out_scale, out_zp, qmin, qmax);
    const float invf = (float)inv;
    const float tie = qa_f32_tie(out_zp, qmin, qmax);
    const int64_t first = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * RPW +
                          lane / GS;
    for (int64_t r = first; r - lane / GS < rows;
         r += (int64_t)gridDim.x * 4 * RPW) {
        const bool live = r < rows;
        const int64_t base = (live ? r : 0) * cols;
        int sv[PER];
        int mx = 0;
        // every load unconditional (clamped into the row), so that all of
        // them are in flight at once
#pragma unroll
        for (int k = 0; k < PER; ++k) {
            const int64_t i = gl + GS * k;
            const int v = (int)x[base + min(i, cols - 1)];
            sv[k] = live && i < cols ? v + 128 : -1;
            mx = max(mx, sv[k]);
        }
#pragma unroll
        for (int o = GS / 2; o > 0; o >>= 1) mx = max(mx, __shfl_xor(mx, o));
        const double* tr = t + 256 * mx;
        double e[PER], sum = 0.0;
#pragma unroll
        for (int k = 0; k < PER; ++k) {
            const double tv = tr[max(sv[k], 0)];
            e[k] = sv[k] >= 0 ? tv : 0.0;
            sum += e[k];
        }
#pragma unroll
        for (int o = GS / 2; o > 0; o >>= 1) sum += __shfl_xor(sum, o);
        const double rsum = 1.0 / sum;  // one division a row
        if (!live) continue;
        // the float32 form inline, the double form out of line for the
        // values whose tie test fails (few instructions a value: the
        // launch's code is fetched cold)
        float y[PER];
        int qv[PER];
        uint32_t slow = 0;
#pragma unroll
        for (int k = 0; k < PER; ++k) {
            y[k] = (float)(e[k] * rsum);
            bool sl = !f32ok;
            qv[k] = qa_quantize_f32(y[k], invf, tie, (int)out_zp, (int)qmin,
                                    (int)qmax, &sl);
            slow |= (uint32_t)sl << k;
        }
        if (__builtin_expect(slow != 0, 0)) {
            for (int k = 0; k < PER; ++k)
                if ((slow >> k) & 1)
                    qv[k] = softmax_quant_exact(y[k], out_scale, inv, out_zp,
                                                qmin, qmax);
        }
#pragma unroll
        for (int k = 0; k < PER; ++k) {
            const int64_t i = gl + GS * k;
            if (i >= cols) continue;
            out[base + i] = (int8_t)(qv[k] - out_so);
            if (outf)
                outf[base + i] = (float)((double)(qv[k] - out_zp) * out_scale);
        }
    }
}

// Rows of the table path: 16 lanes a row up to 256 columns, a wave a row up
// to 512 (8 values a lane) or 1024 (16 a lane).
bool softmax_lut_launch(const int8_t* x, int64_t rows, int64_t cols,
                        const double* t, int8_t* out, double out_scale,
                        int64_t out_zp, int64_t qmin, int64_t qmax,
                        int64_t out_so, float* outf, hipStream_t st) {
    if (cols <= 16 * 16) {
        const int64_t blocks = std::min<int64_t>((rows + 15) / 16, 65535);
        k_softmax_rows_lut<16, 16><<<(unsigned)blocks, kThreads, 0, st>>>(
            x, rows, cols, t, out, out_scale, out_zp, qmin, qmax, out_so,
            outf);
        return true;
    }
    const int64_t blocks = std::min<int64_t>((rows + 3) / 4, 65535);
    if (cols <= 64 * SOFTMAX_PER)
        k_softmax_rows_lut<64, SOFTMAX_PER><<<(unsigned)blocks, kThreads, 0,
                                              st>>>(
            x, rows, cols, t, out, out_scale, out_zp, qmin, qmax, out_so,
            outf);
    else if (cols <= 64 * 16)
        k_softmax_rows_lut<64, 16><<<(unsigned)blocks, kThreads, 0, st>>>(
            x, rows, cols, t, out, out_scale, out_zp, qmin, qmax, out_so,
            outf);
    else
        return false;
    return true;
}

bool softmax_launch(const void* x, int in_code, int64_t rows, int64_t cols,
                    double in_scale, int64_t in_zp, int64_t in_so, void* out,
                    int out_code, double out_scale, int64_t out_zp,
                    int64_t qmin, int64_t qmax, int64_t out_so, float* outf,
                    hipStream_t st) {
    auto rows_kernel = [&](auto ti, auto to) {
        typedef decltype(ti) TI;
        typedef decltype(to) TO;
        if (cols <= 16 * 16) {  // 16 lanes a row, 4 rows a wave
            const int64_t blocks = std::min<int64_t>((rows + 15) / 16, 65535);
            k_softmax_rows<16, 16, TI, TO><<<(unsigned)blocks, kThreads, 0,
                                             st>>>(
                (const TI*)x, rows, cols, in_scale, in_zp, in_so, (TO*)out,
                out_scale, out_zp, qmin, qmax, out_so, outf);
        } else if (cols <= 64 * SOFTMAX_PER) {  // a wave a row
            const int64_t blocks = std::min<int64_t>((rows + 3) / 4, 65535);
            k_softmax_rows<64, SOFTMAX_PER, TI, TO><<<(unsigned)blocks,
                                                      kThreads, 0, st>>>(
                (const TI*)x, rows, cols, in_scale, in_zp, in_so, (TO*)out,
                out_scale, out_zp, qmin, qmax, out_so, outf);
        } else {  // a wave a row, 16 values a lane
            const int64_t blocks = std::min<int64_t>((rows + 3) / 4, 65535);
            k_softmax_rows<64, 16, TI, TO><<<(unsigned)blocks, kThreads, 0,
                                             st>>>(
                (const TI*)x, rows, cols, in_scale, in_zp, in_so, (TO*)out,
                out_scale, out_zp, qmin, qmax, out_so, outf);
        }
    };
    // rows of at most 1024 values in registers (the table path,
    // qa_d_softmax_lut, sums its exponentials in the same order)
    const bool same = in_code == out_code && (in_code == 1 || in_code == 2);
    if (same && cols <= 64 * 16) {
        if (in_code == 1)
            rows_kernel(int8_t{}, int8_t{});
        else
            rows_kernel(int16_t{}, int16_t{});
    } else {
        const unsigned blocks = (unsigned)(rows < 65535 ? rows : 65535);
        k_softmax<<<blocks, kThreads, 0, st>>>(x, in_code, rows, cols,
                                               in_scale, in_zp, in_so, out,
                                               out_code, out_scale, out_zp,
                                               qmin, qmax, out_so, outf);
    }
    return true;
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

// GlobalAveragePool of x [N, C, HW] (strides x_sn, x_sc, x_sp) into out
// [N, C] (row stride out_sn) with a scalar multiplier.
QA_API int qa_d_gap(const void* x, int in_code, int64_t x_sn, int64_t x_sc,
                    int64_t x_sp, int64_t N, int64_t C, int64_t HW,
                    int64_t zp_in, int64_t in_so, int64_t mult, int64_t shift,
                    int64_t zp_out, int64_t qmin, int64_t qmax, void* out,
                    int out_code, int64_t out_sn, int64_t out_so,
                    void* stream) {
    if (N * C <= 0) return 0;
    hipStream_t st = (hipStream_t)stream;
    if (x_sc == 1 && in_code == 1 && C % 4 == 0 && x_sp % 4 == 0 &&
        x_sn % 4 == 0 && (uintptr_t)x % 4 == 0 && HW < (1 << 23)) {
        if (N > 65535) {
            qa::set_error("qa_d_gap", "N above 65535");
            return -1;
        }
        dim3 grid((unsigned)qa::ceil_div(C, 256), (unsigned)N);
        k_gap_cl4<<<grid, kThreads, 0, st>>>(
            (const int8_t*)x, x_sn, x_sp, C, HW, zp_in, in_so, mult, shift,
            zp_out, qmin, qmax, out, out_code, out_sn, out_so);
    } else if (x_sc == 1) {
        if (N > 65535) {
            qa::set_error("qa_d_gap", "N above 65535");
            return -1;
        }
        dim3 grid((unsigned)qa::ceil_div(C, kThreads), (unsigned)N);
        k_gap_cl<<<grid, kThreads, 0, st>>>(x, in_code, x_sn, x_sp, N, C, HW,
                                           zp_in, in_so, mult, shift, zp_out,
                                           qmin, qmax, out, out_code, out_sn,
                                           out_so);
    } else {
        if (x_sp != 1) {
            qa::set_error("qa_d_gap", "needs x_sc == 1 or x_sp == 1");
            return -1;
        }
        const int64_t blocks = qa::ceil_div(N * C, kThreads / 64);
        k_gap_planar<<<(unsigned)blocks, kThreads, 0, st>>>(
            x, in_code, x_sn, x_sc, N, C, HW, zp_in, in_so, mult, shift,
            zp_out, qmin, qmax, out, out_code, out_sn, out_so);
    }
    return launched("qa_d_gap") ? 0 : -1;
}

// Quantizes a float32 NCHW tensor into channels-last storage (int8 or int16)
// with pixel stride y_sp (>= C; padding channels are 0).
QA_API int qa_d_quantize_nhwc(const float* x, int64_t N, int64_t C,
                              int64_t HW, void* y, int y_code, int64_t y_sp,
                              double scale, int64_t zp, int64_t qmin,
                              int64_t qmax, int64_t so, void* stream) {
    if (N * HW <= 0) return 0;
    if (y_sp < C) {
        qa::set_error("qa_d_quantize_nhwc", "pixel stride below C");
        return -1;
    }
    hipStream_t st = (hipStream_t)stream;
    const unsigned g = qa::grid_1d(N * HW, kThreads, 1 << 20);
    const double inv = 1.0 / scale;
    const int word = y_code == 1 && y_sp == 4 && (uintptr_t)y % 4 == 0;
    if (word && C <= 4 && HW % 4 == 0 && (uintptr_t)y % 16 == 0 &&
        (uintptr_t)x % 16 == 0) {
        const unsigned g4 = qa::grid_1d(N * HW / 4, kThreads, 2048);
        k_quantize_cl4x4<<<g4, kThreads, 0, st>>>(
            x, N, C, HW, (int8_t*)y, scale, inv, zp, qmin, qmax, so);
    } else if (y_code == 1)
        k_quantize_cl<int8_t><<<g, kThreads, 0, st>>>(
            x, N, C, HW, (int8_t*)y, y_sp, scale, inv, zp, qmin, qmax, so,
            word);
    else if (y_code == 2)
        k_quantize_cl<int16_t><<<g, kThreads, 0, st>>>(
            x, N, C, HW, (int16_t*)y, y_sp, scale, inv, zp, qmin, qmax, so,
            0);
    else {
        qa::set_error("qa_d_quantize_nhwc", "storage must be int8 or int16");
        return -1;
    }
    return launched("qa_d_quantize_nhwc") ? 0 : -1;
}

QA_API int qa_d_quantize_patches(const float* x, int64_t N, int64_t C,
                                 int64_t H, int64_t W, int64_t KH, int64_t KW,
                                 void* y, double scale, int64_t zp,
                                 int64_t qmin, int64_t qmax, int64_t so,
                                 void* stream) {
    if (N <= 0) return 0;
    if (!x || !y || C < 1 || C > 4 || KH < 1 || KW < 4 || KW % 4 != 0 ||
        H < KH || W < KW || H % KH != 0 || W % KW != 0 ||
        H >= (1 << 15) || W >= (1 << 15) || (uintptr_t)x % 16 != 0 ||
        (uintptr_t)y % 16 != 0 || !(scale > 0.0)) {
        qa::set_error("qa_d_quantize_patches",
                      "needs 1-4 channels, KW a multiple of 4, H and W "
                      "multiples of the kernel (below 2^15), 16-byte aligned "
                      "buffers and a positive scale");
        return -1;
    }
    const unsigned g = qa::grid_1d(N * H * W / 4, kThreads, 2048);
    k_quantize_patches<<<g, kThreads, 0, (hipStream_t)stream>>>(
        x, N, C, (int)H, (int)W, (int)KH, (int)KW, (int8_t*)y, scale,
        1.0 / scale, zp, qmin, qmax, so);
    return launched("qa_d_quantize_patches") ? 0 : -1;
}

// Softmax over the last axis of a [rows, cols] device tensor through float:
// dequantize to float32, softmax in float64, cast to float32, quantize.
QA_API int qa_d_softmax(const void* x, int in_code, int64_t rows, int64_t cols,
                        double in_scale, int64_t in_zp, int64_t in_so,
                        void* out, int out_code, double out_scale,
                        int64_t out_zp, int64_t qmin, int64_t qmax,
                        int64_t out_so, void* stream) {
    if (rows <= 0 || cols <= 0) return 0;
    softmax_launch(x, in_code, rows, cols, in_scale, in_zp, in_so, out,
                   out_code, out_scale, out_zp, qmin, qmax, out_so, nullptr,
                   (hipStream_t)stream);
    return launched("qa_d_softmax") ? 0 : -1;
}

// Table of exponentials for qa_d_softmax_lut (65536 doubles).
QA_API int qa_d_softmax_table(double in_scale, int64_t in_zp, int64_t in_so,
                              double* table, void* stream) {
    if (!table || !(in_scale > 0.0)) {
        qa::set_error("qa_d_softmax_table", "needs a table and a positive scale");
        return -1;
    }
    k_softmax_table<<<65536 / kThreads, kThreads, 0, (hipStream_t)stream>>>(
        in_scale, in_zp, in_so, table);
    return launched("qa_d_softmax_table") ? 0 : -1;
}

// qa_d_softmax for int8 input and output reading the exponentials from a
// qa_d_softmax_table table of the same input quantization.
QA_API int qa_d_softmax_lut(const void* x, int64_t rows, int64_t cols,
                            const double* table, void* out, double out_scale,
                            int64_t out_zp, int64_t qmin, int64_t qmax,
                            int64_t out_so, void* stream) {
    if (rows <= 0 || cols <= 0) return 0;
    if (!table || !softmax_lut_launch((const int8_t*)x, rows, cols, table,
                                      (int8_t*)out, out_scale, out_zp, qmin,
                                      qmax, out_so, nullptr,
                                      (hipStream_t)stream)) {
        qa::set_error("qa_d_softmax_lut", "needs a table and at most 1024 "
                                          "columns");
        return -1;
    }
    return launched("qa_d_softmax_lut") ? 0 : -1;
}

// qa_d_softmax_lut that also writes the dequantized output (float32, same
// [rows, cols] layout) for a graph output.
QA_API int qa_d_softmax_lut_f32(const void* x, int64_t rows, int64_t cols,
                                const double* table, void* out,
                                double out_scale, int64_t out_zp,
                                int64_t qmin, int64_t qmax, int64_t out_so,
                                float* out_f32, void* stream) {
    if (rows <= 0 || cols <= 0) return 0;
    if (!table || !out_f32 ||
        !softmax_lut_launch((const int8_t*)x, rows, cols, table,
                            (int8_t*)out, out_scale, out_zp, qmin, qmax,
                            out_so, out_f32, (hipStream_t)stream)) {
        qa::set_error("qa_d_softmax_lut_f32", "needs a table, a float output "
                                              "and at most 1024 columns");
        return -1;
    }
    return launched("qa_d_softmax_lut_f32") ? 0 : -1;
}

// qa_d_softmax that also writes the dequantized output (float32, same
// [rows, cols] layout) for a graph output.
QA_API int qa_d_softmax_f32(const void* x, int in_code, int64_t rows,
                            int64_t cols, double in_scale, int64_t in_zp,
                            int64_t in_so, void* out, int out_code,
                            double out_scale, int64_t out_zp, int64_t qmin,
                            int64_t qmax, int64_t out_so, float* out_f32,
                            void* stream) {
    if (rows <= 0 || cols <= 0) return 0;
    if (!out_f32) {
        qa::set_error("qa_d_softmax_f32", "no float output");
        return -1;
    }
    softmax_launch(x, in_code, rows, cols, in_scale, in_zp, in_so, out,
                   out_code, out_scale, out_zp, qmin, qmax, out_so, out_f32,
                   (hipStream_t)stream);
    return launched("qa_d_softmax_f32") ? 0 : -1;
}

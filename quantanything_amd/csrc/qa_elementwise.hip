// Element-wise integer kernels: requantize, rescale, add, mul, LUT,
// float <-> integer conversion. HBM-bound; one element per thread per
// grid-stride step, 64-bit indices.
//
// Host-pointer exports replace the reference's (qa_kernels.cpp:287-386) with
// identical signatures and results; qa_d_* exports take device pointers, a
// stream, and the int8/int16 storage form used by the resident executor.
#include <algorithm>

#include "qa_common.h"

namespace {

constexpr int kThreads = 256;

// Element index -> channel of a [outer, C, inner] view.
__device__ __forceinline__ int64_t chan_of(int64_t i, int64_t C, int64_t inner,
                                           bool small) {
    if (small) return (int64_t)(((uint32_t)i / (uint32_t)inner) % (uint32_t)C);
    return (i / inner) % C;
}

// out = clip(mbqm(acc - sub + pre[c], m[c], s[c]) + post[c] + zp) - out_so
template <class TAcc, class TOut>
__global__ __launch_bounds__(kThreads) void k_requant(
    const TAcc* __restrict__ acc, TOut* __restrict__ out, int64_t n,
    int64_t C, int64_t inner, const int64_t* __restrict__ mult,
    const int64_t* __restrict__ shift, const int64_t* __restrict__ pre,
    const int64_t* __restrict__ post, int64_t zp, int64_t qmin, int64_t qmax,
    int64_t sub, int64_t out_so) {
    const bool small = n < (int64_t)0x7fffffff && inner < (int64_t)0x7fffffff;
    const int64_t step = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += step) {
        const int64_t c = chan_of(i, C, inner, small);
        const int64_t pb = pre ? pre[c] : 0;
        const int64_t qb = (post ? post[c] : 0) + zp;
        const qa_i128 v = qa_mbqm_fast((int64_t)acc[i] - sub + pb, mult[c],
                                       shift[c]) + qb;
        out[i] = (TOut)(qa_clip128(v, qmin, qmax) - out_so);
    }
}

// Requantize of int32 accumulators to int8 storage, [outer, C, inner]
// view with inner % 16 == 0: 16 consecutive accumulators (one row, so one
// channel) per thread, all four 16-byte loads issued before any arithmetic.
// With x = acc - sub + pre[c] in int32 and |m| < 2^31, 1 <= 31 + s <= 62,
// mbqm is one 64-bit multiply-add and an arithmetic shift:
// (x*m + 2^(t-1)) >> t, t = 31 + s (|x*m| < 2^62, no overflow); any other
// element takes the 128-bit form. Both clip in 64 bits.
__device__ __forceinline__ int64_t requant_elem(int64_t x, int64_t m,
                                                int64_t s, bool fast32,
                                                int64_t rnd, int64_t qb,
                                                int64_t lo, int64_t hi) {
    int64_t q;
    if (fast32 && x == (int64_t)(int32_t)x)
        q = ((int64_t)(int32_t)x * (int32_t)m + rnd) >> (31 + s);
    else
        q = qa_clip128(qa_mbqm_fast(x, m, s), -((int64_t)1 << 62),
                       (int64_t)1 << 62);
    q += qb;
    return q < lo ? lo : (q > hi ? hi : q);
}

__global__ __launch_bounds__(kThreads) void k_requant_v16_i32_i8(
    const int4* __restrict__ acc, int4* __restrict__ out, int64_t n16,
    uint32_t C, uint32_t inner16, const int64_t* __restrict__ mult,
    const int64_t* __restrict__ shift, const int64_t* __restrict__ pre,
    const int64_t* __restrict__ post, int64_t zp, int64_t qmin, int64_t qmax,
    int64_t sub, int64_t out_so) {
    const int64_t lo = qmin - out_so, hi = qmax - out_so;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n16;
         i += (int64_t)gridDim.x * kThreads) {
        int4 v[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) v[k] = acc[i * 4 + k];
        const uint32_t c = (uint32_t)((uint64_t)i / inner16) % C;
        const int64_t m = mult[c], s = shift[c];
        const int64_t pb = (pre ? pre[c] : 0) - sub;
        const int64_t qb = (post ? post[c] : 0) + zp - out_so;
        const int64_t am = m < 0 ? -m : m;
        const bool fast32 = am < ((int64_t)1 << 31) && s >= -30 && s <= 31;
        const int64_t rnd = fast32 ? (int64_t)1 << (30 + s) : 0;
        uint32_t w[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int a[4] = {v[k].x, v[k].y, v[k].z, v[k].w};
            uint32_t word = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j)
                word |= (uint32_t)(uint8_t)requant_elem(
                            (int64_t)a[j] + pb, m, s, fast32, rnd, qb, lo,
                            hi)
                        << (8 * j);
            w[k] = word;
        }
        out[i] = make_int4((int)w[0], (int)w[1], (int)w[2], (int)w[3]);
    }
}

// int8 storage in and out, contiguous: the table as 256 stored bytes in
// LDS (entry u = the output for stored input byte u), 64 bytes a thread
// whose loads are issued before the table is built.
__global__ __launch_bounds__(kThreads) void k_lut_i8_v64(
    const int4* __restrict__ x, int4* __restrict__ out, int64_t n16,
    int64_t offset, const int32_t* __restrict__ lut, int64_t len,
    int64_t in_so, int64_t out_so) {
    __shared__ uint8_t tab[256];
    const int64_t base = ((int64_t)blockIdx.x * kThreads) * 4;
    const int64_t stride = (int64_t)gridDim.x * kThreads * 4;
    int4 v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int64_t e = base + k * kThreads + threadIdx.x;
        if (e < n16) v[k] = x[e];
    }
    {
        const int u = threadIdx.x;  // stored byte, as int8
        int64_t idx = (int64_t)(int8_t)u + in_so - offset;
        idx = idx < 0 ? 0 : (idx >= len ? len - 1 : idx);
        tab[u] = (uint8_t)(int8_t)((int64_t)lut[idx] - out_so);
    }
    __syncthreads();
    for (int64_t b = base; b < n16; b += stride) {
        if (b != base) {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int64_t e = b + k * kThreads + threadIdx.x;
                if (e < n16) v[k] = x[e];
            }
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int64_t e = b + k * kThreads + threadIdx.x;
            if (e >= n16) continue;
            uint32_t w[4] = {(uint32_t)v[k].x, (uint32_t)v[k].y,
                             (uint32_t)v[k].z, (uint32_t)v[k].w};
#pragma unroll
            for (int q = 0; q < 4; ++q)
                w[q] = (uint32_t)tab[w[q] & 255] |
                       ((uint32_t)tab[(w[q] >> 8) & 255] << 8) |
                       ((uint32_t)tab[(w[q] >> 16) & 255] << 16) |
                       ((uint32_t)tab[w[q] >> 24] << 24);
            out[e] = make_int4((int)w[0], (int)w[1], (int)w[2], (int)w[3]);
        }
    }
}

// Whether the vector kernel takes a requantize: int32 accumulators to int8,
// rows of whole 16-value groups, 16-byte aligned operands.
bool requant_v16_ok(const void* acc, const void* out, int64_t n, int64_t C,
                    int64_t inner) {
    return inner % 16 == 0 && ((uintptr_t)acc & 15) == 0 &&
           ((uintptr_t)out & 15) == 0 && n / 16 < ((int64_t)1 << 32) &&
           C < ((int64_t)1 << 32);
}

void launch_requant_v16(const int32_t* acc, int8_t* out, int64_t n,
                        int64_t C, int64_t inner, const int64_t* mult,
                        const int64_t* shift, const int64_t* pre,
                        const int64_t* post, int64_t zp, int64_t qmin,
                        int64_t qmax, int64_t sub, int64_t out_so,
                        hipStream_t st) {
    const int64_t n16 = n / 16;
    k_requant_v16_i32_i8<<<qa::grid_1d(n16, kThreads, 1 << 16), kThreads, 0,
                           st>>>((const int4*)acc, (int4*)out, n16,
                                 (uint32_t)C, (uint32_t)(inner / 16), mult,
                                 shift, pre, post, zp, qmin, qmax, sub,
                                 out_so);
}

// Row-strided element-wise kernels: `rows` rows of `cols` elements, each
// operand with its own row stride (a channel slice of a channels-last tensor
// is rows = N*H*W pixels, cols = C_slice, stride = the buffer's channel
// count). One flat index per element, so narrow rows still fill the GPU.
#define QA_ROW_LOOP                                                         \
    const bool small_ = rows * cols < ((int64_t)1 << 32);                   \
    for (int64_t i_ = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;       \
         i_ < rows * cols; i_ += (int64_t)gridDim.x * blockDim.x)           \
        for (int64_t r = small_ ? (int64_t)((uint32_t)i_ / (uint32_t)cols)  \
                                : i_ / cols,                                \
                     i = i_ - r * cols, once_ = 1;                          \
             once_; once_ = 0)

template <class TIn, class TOut>
__global__ __launch_bounds__(kThreads) void k_rescale(
    const TIn* __restrict__ x, int64_t xs, TOut* __restrict__ out,
    int64_t os, int64_t rows, int64_t cols, int64_t zp_in, int64_t m,
    int64_t s, int64_t zp_out, int64_t qmin, int64_t qmax, int64_t in_so,
    int64_t out_so) {
    QA_ROW_LOOP {
        const qa_i128 v =
            qa_mbqm_fast((int64_t)x[r * xs + i] + in_so - zp_in, m, s) +
            zp_out;
        out[r * os + i] = (TOut)(qa_clip128(v, qmin, qmax) - out_so);
    }
}

template <class TIn, class TOut>
__global__ __launch_bounds__(kThreads) void k_add(
    const TIn* __restrict__ a, int64_t as, const TIn* __restrict__ b,
    int64_t bs, TOut* __restrict__ out, int64_t os, int64_t rows,
    int64_t cols, int64_t za, int64_t ma, int64_t sa, int64_t zb, int64_t mb,
    int64_t sb, int64_t sign, int64_t zp_out, int64_t qmin, int64_t qmax,
    int64_t a_so, int64_t b_so, int64_t out_so) {
    QA_ROW_LOOP {
        const qa_i128 v =
            qa_mbqm_fast((int64_t)a[r * as + i] + a_so - za, ma, sa) +
            (qa_i128)sign *
                qa_mbqm_fast((int64_t)b[r * bs + i] + b_so - zb, mb, sb) +
            zp_out;
        out[r * os + i] = (TOut)(qa_clip128(v, qmin, qmax) - out_so);
    }
}

// int8 -> int8 Add through two 256-entry tables built per work-group:
// each operand's rescaled term depends on its stored byte alone (RA[u] =
// mbqm(u + a_so - za, ma, sa), RB[u] = sign mbqm(u + b_so - zb, mb, sb), the
// exact 128-bit form, kept as int64), so the result is clip(RA[a] + RB[b] +
// zp_out), as k_add computes it. Four values a thread (word loads and
// stores) when W4, else one.
template <bool W4>
__global__ __launch_bounds__(kThreads) void k_add_i8_tab(
    const int8_t* __restrict__ a, int64_t as, const int8_t* __restrict__ b,
    int64_t bs, int8_t* __restrict__ out, int64_t os, int64_t rows,
    int64_t cols, int64_t za, int64_t ma, int64_t sa, int64_t zb, int64_t mb,
    int64_t sb, int64_t sign, int64_t zp_out, int64_t qmin, int64_t qmax,
    int64_t a_so, int64_t b_so, int64_t out_so) {
    __shared__ int64_t ta[256], tb[256];
    {
        const int u = threadIdx.x;  // kThreads == 256
        ta[u] = (int64_t)qa_clip128(
            qa_mbqm_fast((int64_t)(u - 128) + a_so - za, ma, sa),
            INT64_MIN / 4, INT64_MAX / 4);
        tb[u] = (int64_t)qa_clip128(
            (qa_i128)sign *
                qa_mbqm_fast((int64_t)(u - 128) + b_so - zb, mb, sb),
            INT64_MIN / 4, INT64_MAX / 4);
    }
    __syncthreads();
    auto one = [&](int av, int bv) {
        const int64_t v = ta[av + 128] + tb[bv + 128] + zp_out;
        return (int)((v < qmin ? qmin : (v > qmax ? qmax : v)) - out_so);
    };
    if (W4) {
        const int64_t cw = cols >> 2;  // words a row
        const bool small = rows * cw < ((int64_t)1 << 32);
        for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
             i < rows * cw; i += (int64_t)gridDim.x * kThreads) {
            const int64_t r =
                small ? (int64_t)((uint32_t)i / (uint32_t)cw) : i / cw;
            const int64_t c = (i - r * cw) * 4;
            const uint32_t wa = *(const uint32_t*)(a + r * as + c);
            const uint32_t wb = *(const uint32_t*)(b + r * bs + c);
            uint32_t w = 0;
#pragma unroll
            for (int k = 0; k < 4; ++k)
                w |= (uint32_t)(uint8_t)one((int8_t)(wa >> (8 * k)),
                                            (int8_t)(wb >> (8 * k)))
                     << (8 * k);
            *(uint32_t*)(out + r * os + c) = w;
        }
    } else {
        QA_ROW_LOOP {
            out[r * os + i] = (int8_t)one(a[r * as + i], b[r * bs + i]);
        }
    }
}

template <class TIn, class TOut>
__global__ __launch_bounds__(kThreads) void k_mul(
    const TIn* __restrict__ a, int64_t as, const TIn* __restrict__ b,
    int64_t bs, TOut* __restrict__ out, int64_t os, int64_t rows,
    int64_t cols, int64_t za, int64_t zb, int64_t m, int64_t s,
    int64_t zp_out, int64_t qmin, int64_t qmax, int64_t a_so, int64_t b_so,
    int64_t out_so) {
    QA_ROW_LOOP {
        const int64_t p = ((int64_t)a[r * as + i] + a_so - za) *
                          ((int64_t)b[r * bs + i] + b_so - zb);
        const qa_i128 v = qa_mbqm_fast(p, m, s) + zp_out;
        out[r * os + i] = (TOut)(qa_clip128(v, qmin, qmax) - out_so);
    }
}

template <class TIn, class TOut>
__global__ __launch_bounds__(kThreads) void k_lut(
    const TIn* __restrict__ x, int64_t xs, TOut* __restrict__ out,
    int64_t os, int64_t rows, int64_t cols, int64_t offset,
    const int32_t* __restrict__ lut, int64_t len, int64_t in_so,
    int64_t out_so) {
    QA_ROW_LOOP {
        int64_t idx = (int64_t)x[r * xs + i] + in_so - offset;
        idx = idx < 0 ? 0 : (idx >= len ? len - 1 : idx);
        out[r * os + i] = (TOut)((int64_t)lut[idx] - out_so);
    }
}

__device__ __forceinline__ int64_t quantize_one(float x, double scale,
                                                int64_t zp, int64_t qmin,
                                                int64_t qmax) {
    return qa_quantize_one(x, scale, zp, qmin, qmax);
}

template <class TOut>
__global__ __launch_bounds__(kThreads) void k_quantize(
    const float* __restrict__ x, TOut* __restrict__ q, int64_t n,
    double scale, int64_t zp, int64_t qmin, int64_t qmax, int64_t out_so) {
    const int64_t step = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += step)
        q[i] = (TOut)(quantize_one(x[i], scale, zp, qmin, qmax) - out_so);
}

// 16 float32 -> 16 int8 per thread (graph-input quantization).
__global__ __launch_bounds__(kThreads) void k_quantize_v16_i8(
    const float4* __restrict__ x, int4* __restrict__ q, int64_t n16,
    double scale, int64_t zp, int64_t qmin, int64_t qmax, int64_t out_so) {
    const int64_t step = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16;
         i += step) {
        uint32_t w[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float4 f = x[i * 4 + j];
            const uint32_t b0 = (uint8_t)(int8_t)(
                quantize_one(f.x, scale, zp, qmin, qmax) - out_so);
            const uint32_t b1 = (uint8_t)(int8_t)(
                quantize_one(f.y, scale, zp, qmin, qmax) - out_so);
            const uint32_t b2 = (uint8_t)(int8_t)(
                quantize_one(f.z, scale, zp, qmin, qmax) - out_so);
            const uint32_t b3 = (uint8_t)(int8_t)(
                quantize_one(f.w, scale, zp, qmin, qmax) - out_so);
            w[j] = b0 | (b1 << 8) | (b2 << 16) | (b3 << 24);
        }
        q[i] = make_int4((int)w[0], (int)w[1], (int)w[2], (int)w[3]);
    }
}

template <class TIn>
__global__ __launch_bounds__(kThreads) void k_dequantize(
    const TIn* __restrict__ q, float* __restrict__ x, int64_t n, double scale,
    int64_t zp, int64_t in_so) {
    const int64_t step = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += step)
        x[i] = (float)((double)((int64_t)q[i] + in_so - zp) * scale);
}

// Device entries launch on the caller's stream as given (NULL: the null
// stream, which is also what torch's default stream handle is).
hipStream_t pick(void* s) { return (hipStream_t)s; }

template <class T>
T* upload(int slot, const T* h, int64_t n, hipStream_t st) {
    T* d = (T*)qa::scratch(slot, (size_t)n * sizeof(T));
    if (!d) return nullptr;
    hipError_t e = hipMemcpyAsync(d, h, (size_t)n * sizeof(T),
                                  hipMemcpyDefault, st);
    if (e != hipSuccess) {
        qa::set_hip_error("hipMemcpyAsync(upload)", e);
        return nullptr;
    }
    return d;
}

bool download(void* h, const void* d, size_t bytes, hipStream_t st) {
    hipError_t e = hipMemcpyAsync(h, d, bytes, hipMemcpyDefault, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess) {
        qa::set_hip_error("download", e);
        return false;
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

template <class TAcc>
void requantize_abi(const TAcc* acc, int32_t* out, int64_t outer, int64_t C,
                    int64_t inner, const int64_t* mult, const int64_t* shift,
                    const int64_t* pre, const int64_t* post, int64_t zp,
                    int64_t qmin, int64_t qmax) {
    const int64_t n = outer * C * inner;
    if (n <= 0) return;
    qa::AbiCall call(out, (size_t)n * 4);
    hipStream_t st = qa::stream();
    if (!st) return;
    const TAcc* da = upload(0, acc, n, st);
    const int64_t* dm = upload(2, mult, C, st);
    const int64_t* ds = upload(3, shift, C, st);
    const int64_t* dpre = pre ? upload(4, pre, C, st) : nullptr;
    const int64_t* dpost = post ? upload(5, post, C, st) : nullptr;
    int32_t* dout = (int32_t*)qa::scratch(1, (size_t)n * 4);
    if (!da || !dm || !ds || !dout || (pre && !dpre) || (post && !dpost))
        return;
    k_requant<TAcc, int32_t><<<qa::grid_1d(n, kThreads), kThreads, 0, st>>>(
        da, dout, n, C, inner, dm, ds, dpre, dpost, zp, qmin, qmax, 0, 0);
    if (!launched("k_requant")) return;
    download(out, dout, (size_t)n * 4, st);
}

}  // namespace

// ===================================================== host-pointer ABI ===
// Every entry accepts host (or device) pointers, runs on the GPU and returns
// once the result is in `out`. Errors: see qa_last_error.

QA_API void qa_requantize_i32(const int32_t* acc, int32_t* out, int64_t outer,
                              int64_t C, int64_t inner, const int64_t* mult,
                              const int64_t* shift, const int64_t* pre_bias,
                              const int64_t* post_bias, int64_t zp,
                              int64_t qmin, int64_t qmax) {
    requantize_abi<int32_t>(acc, out, outer, C, inner, mult, shift, pre_bias,
                            post_bias, zp, qmin, qmax);
}

QA_API void qa_requantize_i64(const int64_t* acc, int32_t* out, int64_t outer,
                              int64_t C, int64_t inner, const int64_t* mult,
                              const int64_t* shift, const int64_t* pre_bias,
                              const int64_t* post_bias, int64_t zp,
                              int64_t qmin, int64_t qmax) {
    requantize_abi<int64_t>(acc, out, outer, C, inner, mult, shift, pre_bias,
                            post_bias, zp, qmin, qmax);
}

QA_API void qa_rescale(const int32_t* x, int32_t* out, int64_t n,
                       int64_t zp_in, int64_t m, int64_t s, int64_t zp_out,
                       int64_t qmin, int64_t qmax) {
    if (n <= 0) return;
    qa::AbiCall call(out, (size_t)n * 4);
    hipStream_t st = qa::stream();
    if (!st) return;
    const int32_t* dx = upload(0, x, n, st);
    int32_t* dy = (int32_t*)qa::scratch(1, (size_t)n * 4);
    if (!dx || !dy) return;
    k_rescale<int32_t, int32_t><<<qa::grid_1d(n, kThreads), kThreads, 0, st>>>(
        dx, n, dy, n, 1, n, zp_in, m, s, zp_out, qmin, qmax, 0, 0);
    if (!launched("k_rescale")) return;
    download(out, dy, (size_t)n * 4, st);
}

QA_API void qa_add(const int32_t* a, const int32_t* b, int32_t* out, int64_t n,
                   int64_t za, int64_t ma, int64_t sa, int64_t zb, int64_t mb,
                   int64_t sb, int64_t sign, int64_t zp_out, int64_t qmin,
                   int64_t qmax) {
    if (n <= 0) return;
    qa::AbiCall call(out, (size_t)n * 4);
    hipStream_t st = qa::stream();
    if (!st) return;
    const int32_t* da = upload(0, a, n, st);
    const int32_t* db = upload(2, b, n, st);
    int32_t* dy = (int32_t*)qa::scratch(1, (size_t)n * 4);
    if (!da || !db || !dy) return;
    k_add<int32_t, int32_t><<<qa::grid_1d(n, kThreads), kThreads, 0, st>>>(
        da, n, db, n, dy, n, 1, n, za, ma, sa, zb, mb, sb, sign, zp_out, qmin,
        qmax, 0, 0, 0);
    if (!launched("k_add")) return;
    download(out, dy, (size_t)n * 4, st);
}

QA_API void qa_mul(const int32_t* a, const int32_t* b, int32_t* out, int64_t n,
                   int64_t za, int64_t zb, int64_t m, int64_t s, int64_t zp_out,
                   int64_t qmin, int64_t qmax) {
    if (n <= 0) return;
    qa::AbiCall call(out, (size_t)n * 4);
    hipStream_t st = qa::stream();
    if (!st) return;
    const int32_t* da = upload(0, a, n, st);
    const int32_t* db = upload(2, b, n, st);
    int32_t* dy = (int32_t*)qa::scratch(1, (size_t)n * 4);
    if (!da || !db || !dy) return;
    k_mul<int32_t, int32_t><<<qa::grid_1d(n, kThreads), kThreads, 0, st>>>(
        da, n, db, n, dy, n, 1, n, za, zb, m, s, zp_out, qmin, qmax, 0, 0, 0);
    if (!launched("k_mul")) return;
    download(out, dy, (size_t)n * 4, st);
}

QA_API void qa_lut(const int32_t* x, int32_t* out, int64_t n, int64_t offset,
                   const int32_t* lut, int64_t lut_len) {
    if (n <= 0) return;
    qa::AbiCall call(out, (size_t)n * 4);
    if (lut_len <= 0) {
        qa::set_error("qa_lut", "empty table");
        return;
    }
    hipStream_t st = qa::stream();
    if (!st) return;
    const int32_t* dx = upload(0, x, n, st);
    const int32_t* dl = upload(2, lut, lut_len, st);
    int32_t* dy = (int32_t*)qa::scratch(1, (size_t)n * 4);
    if (!dx || !dl || !dy) return;
    k_lut<int32_t, int32_t><<<qa::grid_1d(n, kThreads), kThreads, 0, st>>>(
        dx, n, dy, n, 1, n, offset, dl, lut_len, 0, 0);
    if (!launched("k_lut")) return;
    download(out, dy, (size_t)n * 4, st);
}

QA_API void qa_quantize_f32(const float* x, int32_t* q, int64_t n,
                            double scale, int64_t zp, int64_t qmin,
                            int64_t qmax) {
    if (n <= 0) return;
    qa::AbiCall call(q, (size_t)n * 4);
    hipStream_t st = qa::stream();
    if (!st) return;
    const float* dx = upload(0, x, n, st);
    int32_t* dq = (int32_t*)qa::scratch(1, (size_t)n * 4);
    if (!dx || !dq) return;
    k_quantize<int32_t><<<qa::grid_1d(n, kThreads), kThreads, 0, st>>>(
        dx, dq, n, scale, zp, qmin, qmax, 0);
    if (!launched("k_quantize")) return;
    download(q, dq, (size_t)n * 4, st);
}

QA_API void qa_dequantize_f32(const int32_t* q, float* x, int64_t n,
                              double scale, int64_t zp) {
    if (n <= 0) return;
    qa::AbiCall call(x, (size_t)n * 4);
    hipStream_t st = qa::stream();
    if (!st) return;
    const int32_t* dq = upload(0, q, n, st);
    float* dx = (float*)qa::scratch(1, (size_t)n * 4);
    if (!dq || !dx) return;
    k_dequantize<int32_t><<<qa::grid_1d(n, kThreads), kThreads, 0, st>>>(
        dq, dx, n, scale, zp, 0);
    if (!launched("k_dequantize")) return;
    download(x, dx, (size_t)n * 4, st);
}

// =================================================== device-pointer API ===
// Storage codes: 1 = int8, 2 = int16, 4 = int32 (element size in bytes).
// `*_so` are storage offsets (q = stored + so). All calls are asynchronous
// on `stream` (NULL: the library stream) and return 0 on success.

#define QA_DISPATCH_STORAGE(code, T, ...)          \
    switch (code) {                                \
        case 1: { typedef int8_t T; __VA_ARGS__; break; }  \
        case 2: { typedef int16_t T; __VA_ARGS__; break; } \
        case 4: { typedef int32_t T; __VA_ARGS__; break; } \
        default: qa::set_error("storage", "unsupported storage code"); \
            return -1;                             \
    }

QA_API int qa_d_requantize(const void* acc, int acc_code, void* out,
                           int out_code, int64_t outer, int64_t C,
                           int64_t inner, const int64_t* mult,
                           const int64_t* shift, const int64_t* pre_bias,
                           const int64_t* post_bias, int64_t zp, int64_t qmin,
                           int64_t qmax, int64_t sub, int64_t out_so,
                           void* stream) {
    const int64_t n = outer * C * inner;
    if (n <= 0) return 0;
    hipStream_t st = pick(stream);
    if (acc_code == 4 && out_code == 1 &&
        requant_v16_ok(acc, out, n, C, inner)) {
        launch_requant_v16((const int32_t*)acc, (int8_t*)out, n, C, inner,
                           mult, shift, pre_bias, post_bias, zp, qmin, qmax,
                           sub, out_so, st);
        return launched("qa_d_requantize") ? 0 : -1;
    }
    const unsigned g = qa::grid_1d(n, kThreads, 1 << 20);
    if (acc_code == 8) {
        QA_DISPATCH_STORAGE(out_code, TO,
            k_requant<int64_t, TO><<<g, kThreads, 0, st>>>(
                (const int64_t*)acc, (TO*)out, n, C, inner, mult, shift,
                pre_bias, post_bias, zp, qmin, qmax, sub, out_so))
    } else {
        QA_DISPATCH_STORAGE(acc_code, TA,
            QA_DISPATCH_STORAGE(out_code, TO,
                k_requant<TA, TO><<<g, kThreads, 0, st>>>(
                    (const TA*)acc, (TO*)out, n, C, inner, mult, shift,
                    pre_bias, post_bias, zp, qmin, qmax, sub, out_so)))
    }
    return launched("qa_d_requantize") ? 0 : -1;
}

static dim3 grid_rows(int64_t rows, int64_t cols) {
    return dim3(qa::grid_1d(rows * cols, kThreads, 1 << 20));
}

QA_API int qa_d_rescale(const void* x, int in_code, int64_t x_rstride,
                        void* out, int out_code, int64_t out_rstride,
                        int64_t rows, int64_t cols, int64_t zp_in, int64_t m,
                        int64_t s, int64_t zp_out, int64_t qmin, int64_t qmax,
                        int64_t in_so, int64_t out_so, void* stream) {
    if (rows <= 0 || cols <= 0) return 0;
    hipStream_t st = pick(stream);
    const dim3 g = grid_rows(rows, cols);
    QA_DISPATCH_STORAGE(in_code, TI,
        QA_DISPATCH_STORAGE(out_code, TO,
            k_rescale<TI, TO><<<g, kThreads, 0, st>>>(
                (const TI*)x, x_rstride, (TO*)out, out_rstride, rows, cols,
                zp_in, m, s, zp_out, qmin, qmax, in_so, out_so)))
    return launched("qa_d_rescale") ? 0 : -1;
}

QA_API int qa_d_add(const void* a, int64_t a_rstride, const void* b,
                    int64_t b_rstride, int in_code, void* out, int out_code,
                    int64_t out_rstride, int64_t rows, int64_t cols,
                    int64_t za, int64_t ma, int64_t sa, int64_t zb,
                    int64_t mb, int64_t sb, int64_t sign, int64_t zp_out,
                    int64_t qmin, int64_t qmax, int64_t a_so, int64_t b_so,
                    int64_t out_so, void* stream) {
    if (rows <= 0 || cols <= 0) return 0;
    hipStream_t st = pick(stream);
    const dim3 g = grid_rows(rows, cols);
    // int8: the two operand tables, when every entry is an exact int64 far
    // from overflow (|m| < 2^31 and a right shift: |entry| < 2^41)
    auto small_mul = [](int64_t m, int64_t sh) {
        return m > -((int64_t)1 << 31) && m < ((int64_t)1 << 31) &&
               31 + sh >= 1 && 31 + sh <= 120;
    };
    if (in_code == 1 && out_code == 1 && qmin >= -(1 << 20) &&
        qmax <= (1 << 20) && (sign == 1 || sign == -1) &&
        small_mul(ma, sa) && small_mul(mb, sb) && za > -(1 << 20) &&
        za < (1 << 20) && zb > -(1 << 20) && zb < (1 << 20) &&
        a_so > -(1 << 20) && a_so < (1 << 20) && b_so > -(1 << 20) &&
        b_so < (1 << 20)) {
        const bool w4 = cols % 4 == 0 && a_rstride % 4 == 0 &&
                        b_rstride % 4 == 0 && out_rstride % 4 == 0 &&
                        (uintptr_t)a % 4 == 0 && (uintptr_t)b % 4 == 0 &&
                        (uintptr_t)out % 4 == 0;
        if (w4)
            k_add_i8_tab<true><<<grid_rows(rows, cols / 4), kThreads, 0, st>>>(
                (const int8_t*)a, a_rstride, (const int8_t*)b, b_rstride,
                (int8_t*)out, out_rstride, rows, cols, za, ma, sa, zb, mb, sb,
                sign, zp_out, qmin, qmax, a_so, b_so, out_so);
        else
            k_add_i8_tab<false><<<g, kThreads, 0, st>>>(
                (const int8_t*)a, a_rstride, (const int8_t*)b, b_rstride,
                (int8_t*)out, out_rstride, rows, cols, za, ma, sa, zb, mb, sb,
                sign, zp_out, qmin, qmax, a_so, b_so, out_so);
        return launched("qa_d_add") ? 0 : -1;
    }
    QA_DISPATCH_STORAGE(in_code, TI,
        QA_DISPATCH_STORAGE(out_code, TO,
            k_add<TI, TO><<<g, kThreads, 0, st>>>(
                (const TI*)a, a_rstride, (const TI*)b, b_rstride, (TO*)out,
                out_rstride, rows, cols, za, ma, sa, zb, mb, sb, sign, zp_out,
                qmin, qmax, a_so, b_so, out_so)))
    return launched("qa_d_add") ? 0 : -1;
}

QA_API int qa_d_mul(const void* a, int64_t a_rstride, const void* b,
                    int64_t b_rstride, int in_code, void* out, int out_code,
                    int64_t out_rstride, int64_t rows, int64_t cols,
                    int64_t za, int64_t zb, int64_t m, int64_t s,
                    int64_t zp_out, int64_t qmin, int64_t qmax, int64_t a_so,
                    int64_t b_so, int64_t out_so, void* stream) {
    if (rows <= 0 || cols <= 0) return 0;
    hipStream_t st = pick(stream);
    const dim3 g = grid_rows(rows, cols);
    QA_DISPATCH_STORAGE(in_code, TI,
        QA_DISPATCH_STORAGE(out_code, TO,
            k_mul<TI, TO><<<g, kThreads, 0, st>>>(
                (const TI*)a, a_rstride, (const TI*)b, b_rstride, (TO*)out,
                out_rstride, rows, cols, za, zb, m, s, zp_out, qmin, qmax,
                a_so, b_so, out_so)))
    return launched("qa_d_mul") ? 0 : -1;
}

QA_API int qa_d_lut(const void* x, int in_code, int64_t x_rstride, void* out,
                    int out_code, int64_t out_rstride, int64_t rows,
                    int64_t cols, int64_t offset, const int32_t* lut,
                    int64_t lut_len, int64_t in_so, int64_t out_so,
                    void* stream) {
    if (rows <= 0 || cols <= 0) return 0;
    hipStream_t st = pick(stream);
    const int64_t n = rows * cols;
    if (in_code == 1 && out_code == 1 && lut_len > 0 && n % 16 == 0 &&
        (rows == 1 || (x_rstride == cols && out_rstride == cols)) &&
        ((uintptr_t)x & 15) == 0 && ((uintptr_t)out & 15) == 0) {
        k_lut_i8_v64<<<qa::grid_1d(qa::ceil_div(n / 16, 4), kThreads,
                                   1 << 16),
                       kThreads, 0, st>>>((const int4*)x, (int4*)out, n / 16,
                                          offset, lut, lut_len, in_so,
                                          out_so);
        return launched("qa_d_lut") ? 0 : -1;
    }
    const dim3 g = grid_rows(rows, cols);
    QA_DISPATCH_STORAGE(in_code, TI,
        QA_DISPATCH_STORAGE(out_code, TO,
            k_lut<TI, TO><<<g, kThreads, 0, st>>>(
                (const TI*)x, x_rstride, (TO*)out, out_rstride, rows, cols,
                offset, lut, lut_len, in_so, out_so)))
    return launched("qa_d_lut") ? 0 : -1;
}

QA_API int qa_d_quantize_f32(const float* x, void* q, int out_code, int64_t n,
                             double scale, int64_t zp, int64_t qmin,
                             int64_t qmax, int64_t out_so, void* stream) {
    if (n <= 0) return 0;
    hipStream_t st = pick(stream);
    if (out_code == 1 && n % 16 == 0 && ((uintptr_t)x & 15) == 0 &&
        ((uintptr_t)q & 15) == 0) {
        const int64_t n16 = n / 16;
        k_quantize_v16_i8<<<qa::grid_1d(n16, kThreads, 1 << 20), kThreads, 0,
                            st>>>((const float4*)x, (int4*)q, n16, scale, zp,
                                  qmin, qmax, out_so);
        return launched("qa_d_quantize_f32") ? 0 : -1;
    }
    const unsigned g = qa::grid_1d(n, kThreads, 1 << 20);
    QA_DISPATCH_STORAGE(out_code, TO,
        k_quantize<TO><<<g, kThreads, 0, st>>>(x, (TO*)q, n, scale, zp, qmin,
                                               qmax, out_so))
    return launched("qa_d_quantize_f32") ? 0 : -1;
}

QA_API int qa_d_dequantize_f32(const void* q, int in_code, float* x,
                               int64_t n, double scale, int64_t zp,
                               int64_t in_so, void* stream) {
    if (n <= 0) return 0;
    hipStream_t st = pick(stream);
    const unsigned g = qa::grid_1d(n, kThreads, 1 << 20);
    QA_DISPATCH_STORAGE(in_code, TI,
        k_dequantize<TI><<<g, kThreads, 0, st>>>((const TI*)q, x, n, scale,
                                                 zp, in_so))
    return launched("qa_d_dequantize_f32") ? 0 : -1;
}

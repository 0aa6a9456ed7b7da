// Float fallbacks of the integer pass on device tensors, and the strided
// copy behind layout operators that are not views.
//
// The reference runs every operator without an integer implementation as
// dequantize -> float operator -> quantize (quant_layers.py:195-205):
//   LayerNorm  float_ops.py:336-347 (float64 statistics over the last axis,
//              then * gamma + beta, cast to float32),
//   MatMul     float_ops.py:181-186 (float32 matmul of two activations).
// Here the dequantized input is the reference's float32 value
// (float)((q - zp) * scale); LayerNorm follows the same float64 steps. The
// activation x activation MatMul sums the exact integer products
// sum (a - za)(b - zb) (int8: v_dot4_i32_i8) and scales the sum once,
// y = (float)(acc * sa * sb): the reference's float32 sums of float32
// products differ from it by a few float32 roundings, far below one output
// quantization step, so outputs agree within one step.
#include <algorithm>

#include "../../include/qa_hip.h"
#include "qa_conv.h"
#include "qa_stage.h"

namespace qa {
namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ float dequant_f32(int64_t q, int64_t zp,
                                             double scale) {
    return (float)((double)(q - zp) * scale);
}

// ------------------------------------------------------------ N-D copy --
// I32: the element count and every extent below 2^32, so that the index
// decode divides in 32 bits (a 64-bit division is a long software
// sequence per dimension and element).
template <bool I32>
__global__ __launch_bounds__(kThreads) void k_copy_nd(qa_nd_copy d,
                                                      int64_t total) {
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * kThreads) {
        int64_t xo = 0, yo = 0;
        if (I32) {
            uint32_t rem = (uint32_t)i;
            for (int k = (int)d.ndim - 1; k >= 0; --k) {
                const uint32_t n = (uint32_t)d.shape[k];
                const uint32_t q = rem / n;
                const int64_t c = (int64_t)(rem - q * n);
                rem = q;
                xo += c * d.xs[k];
                yo += c * d.ys[k];
            }
        } else {
            int64_t rem = i;
            for (int k = (int)d.ndim - 1; k >= 0; --k) {
                const int64_t c = rem % d.shape[k];
                rem /= d.shape[k];
                xo += c * d.xs[k];
                yo += c * d.ys[k];
            }
        }
        int64_t q = load_any(d.x, (int)d.x_code, xo) + d.x_so;
        if (d.mode == 1)
            q = qa_clip128(qa_mbqm_fast(q - d.zp_in, d.m, d.s) + d.zp_out,
                           d.qmin, d.qmax);
        else if (d.mode == 2)
            q = qa_quantize_one(dequant_f32(q, d.in_zp, d.in_scale),
                                d.out_scale, d.zp_out, d.qmin, d.qmax);
        store_any(d.y, (int)d.y_code, yo, q - d.y_so);
    }
}

// Plain copies (same storage on both sides, values unchanged) whose
// innermost axis is contiguous on both sides, in 16-byte chunks: chunk i is
// part i % cpr of inner row i / cpr, whose index decodes over the other
// axes in 32 bits (fewer than 2^32 chunks); strides in bytes.
__global__ __launch_bounds__(kThreads) void k_copy_nd16(
    const char* __restrict__ x, char* __restrict__ y, int ndim,
    int64_t cpr, int64_t chunks, qa_nd_copy d, int es) {
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
         i < chunks; i += (int64_t)gridDim.x * kThreads) {
        const uint32_t row = (uint32_t)i / (uint32_t)cpr;
        const uint32_t part = (uint32_t)i - row * (uint32_t)cpr;
        int64_t xo = (int64_t)part * 16, yo = xo;
        uint32_t rem = row;
        for (int k = ndim - 2; k >= 0; --k) {
            const uint32_t n = (uint32_t)d.shape[k];
            const uint32_t q = rem / n;
            const int64_t c = (int64_t)(rem - q * n);
            rem = q;
            xo += c * d.xs[k] * es;
            yo += c * d.ys[k] * es;
        }
        *(int4*)(y + yo) = *(const int4*)(x + xo);
    }
}

// Whether a copy descriptor is a plain copy k_copy_nd16 can do.
bool copy_nd16_applies(const qa_nd_copy& d, int64_t total) {
    const int es = (int)d.x_code;
    if (d.x_code != d.y_code || d.x_so != d.y_so || es > 4) return false;
    const int64_t lo = es == 1 ? -128 : es == 2 ? -32768 : INT32_MIN;
    const int64_t hi = es == 1 ? 127 : es == 2 ? 32767 : INT32_MAX;
    // mode 1 with the identity multiplier, equal zero points and a clip
    // range covering the storage changes no value
    const bool same =
        d.mode == 0 ||
        (d.mode == 1 && d.m == ((int64_t)1 << 30) && d.s == -1 &&
         d.zp_in == d.zp_out && d.qmin <= lo + d.x_so &&
         d.qmax >= hi + d.x_so);
    const int last = (int)d.ndim - 1;
    if (!same || d.xs[last] != 1 || d.ys[last] != 1 ||
        (d.shape[last] * es) % 16 != 0 || ((uintptr_t)d.x | (uintptr_t)d.y) % 16)
        return false;
    for (int k = 0; k < last; ++k)
        if ((d.xs[k] * es) % 16 || (d.ys[k] * es) % 16 ||
            d.shape[k] >= ((int64_t)1 << 32))
            return false;
    return total * es / 16 < ((int64_t)1 << 32);
}

// ----------------------------------------------------------- LayerNorm --
// GS lanes per row (64 / GS rows per wave): rows of at most GS * PER values
// are read once and held in registers; longer rows (GS = 64, PER = 0) are
// read again for each pass. The statistics are float64 sums in lane order
// then across the lane group (the reference sums in NumPy's order: results
// agree within one step).
template <int GS>
__device__ __forceinline__ double group_sum(double v) {
#pragma unroll
    for (int o = GS / 2; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

template <int GS, int PER, class TI, class TO>
__global__ __launch_bounds__(kThreads) void k_layernorm(
    const TI* __restrict__ x, int64_t x_rs, int64_t rows,
    int64_t cols, double in_scale, int64_t in_zp, int64_t x_so,
    const float* __restrict__ gamma, const float* __restrict__ beta,
    double eps, TO* __restrict__ y, int64_t y_rs, double out_scale,
    int64_t out_zp, int64_t qmin, int64_t qmax, int64_t y_so) {
    constexpr int RPW = 64 / GS;
    const int lane = threadIdx.x & 63;
    const int gl = lane % GS;
    const double inv = 1.0 / out_scale;
    const bool f32ok = qa_f32_form_ok(out_scale, out_zp, qmin, qmax);
    const float invf = (float)inv;
    const int64_t first =
        ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * RPW + lane / GS;
    for (int64_t r = first; r - lane / GS < rows;
         r += (int64_t)gridDim.x * 4 * RPW) {
        const bool live = r < rows;
        const int64_t rr = live ? r : 0;
        auto value = [&](int64_t i) {
            return (double)dequant_f32((int64_t)x[rr * x_rs + i] + x_so,
                                       in_zp, in_scale);
        };
        auto emit = [&](int64_t i, double v, double mean, double sd) {
            double t = (v - mean) / sd * (double)gamma[i];
            if (beta) t += (double)beta[i];
            const int64_t q = qa_quantize_mixed((float)t, f32ok, invf,
                                                out_scale, inv, out_zp, qmin,
                                                qmax);
            y[rr * y_rs + i] = (TO)(q - y_so);
        };
        if (PER > 0) {
            double v[PER > 0 ? PER : 1];
            double s = 0.0;
#pragma unroll
            for (int k = 0; k < PER; ++k) {
                const int64_t i = gl + GS * k;
                v[k] = i < cols ? value(i) : 0.0;
                s += v[k];
            }
            const double mean = group_sum<GS>(s) / (double)cols;
            double q2 = 0.0;
#pragma unroll
            for (int k = 0; k < PER; ++k) {
                const double t = v[k] - mean;
                if (gl + GS * k < cols) q2 += t * t;
            }
            const double sd = sqrt(group_sum<GS>(q2) / (double)cols + eps);
            if (!live) continue;
#pragma unroll
            for (int k = 0; k < PER; ++k)
                if (gl + GS * k < cols) emit(gl + GS * k, v[k], mean, sd);
            continue;
        }
        double s = 0.0;
        for (int64_t i = gl; i < cols; i += GS) s += value(i);
        const double mean = group_sum<GS>(s) / (double)cols;
        double q2 = 0.0;
        for (int64_t i = gl; i < cols; i += GS) {
            const double t = value(i) - mean;
            q2 += t * t;
        }
        const double sd = sqrt(group_sum<GS>(q2) / (double)cols + eps);
        if (!live) continue;
        for (int64_t i = gl; i < cols; i += GS) emit(i, value(i), mean, sd);
    }
}

// The output quantization of the word kernel below, biased by 128 - so so
// that a clipped value is its stored byte + 128: the float32 form of
// qa_quantize_mixed (tie = -1 where that form does not apply, so every
// value takes the double form), and wrap set where the clip range reaches
// past the int8 storage (whose bytes then wrap around).
struct LnQ {
    double scale, inv;
    float invf, tie, cb, lob, hib;
    int zp, qmin, qmax, so, wrap;
};

__device__ __noinline__ int ln_quant_exact(float y, double scale, double inv,
                                           int zp, int qmin, int qmax) {
    return (int)qa_quantize_one_fast(y, scale, inv, zp, qmin, qmax);
}

// int8 rows of at most 512 values, a multiple of 4 (transformer widths):
// 32 lanes a row (2 rows a wave), lane l holding the WPL 4-byte words
// l, l + 32, ... of its row (coalesced word loads and stores). The float64
// steps of k_layernorm (mean, mean square deviation, then (v - mean) / sd
// * gamma + beta, the division as one reciprocal a row) with per value:
// the dequantized value from a 256-entry table in LDS (the reference's
// float32 value of each stored byte, as a double), the affine step as one
// multiply and one fma, and the float32 form of the output quantization
// with v_cvt_pk_u8_f32 packing four values into their word (a word whose
// tie test fails in any lane is requantized by the double form). Every
// load of a row (its words, gamma and beta) is issued before the table is
// built, so their latencies overlap. NW waves a work-group (16: the grid
// is a quarter of the work-groups of 4-wave ones, which the dispatcher
// starts at a few nanoseconds each).
template <int WPL, int NW>
__global__ __launch_bounds__(64 * NW) void k_layernorm_w(
    const int8_t* __restrict__ x, int64_t x_rs, int64_t rows, int64_t cols,
    double in_scale, int64_t in_zp, int64_t x_so,
    const float* __restrict__ gamma, const float* __restrict__ beta,
    double eps, int8_t* __restrict__ y, int64_t y_rs, LnQ o) {
    __shared__ double s_dq[256];
    const int tid = threadIdx.x, lane = tid & 63;
    const int gl = lane & 31;
    const int words = (int)(cols >> 2);
    const int64_t first =
        ((int64_t)blockIdx.x * NW + (tid >> 6)) * 2 + (lane >> 5);
    const int64_t step = (int64_t)gridDim.x * 2 * NW;
    uint32_t u[WPL];
    float4 g4[WPL], b4[WPL];
    auto load_row = [&](int64_t r) __attribute__((always_inline)) {
        const uint32_t* xr = (const uint32_t*)(x + min(r, rows - 1) * x_rs);
#pragma unroll
        for (int k = 0; k < WPL; ++k) {
            const int w = min(gl + 32 * k, words - 1);
            u[k] = xr[w];
        }
    };
    load_row(first);
    // beta's loads read gamma when there is no beta (no branch between
    // the loads); its terms are then zero
    const float* bsrc = beta ? beta : gamma;
    const float bmul = beta ? 1.f : 0.f;
#pragma unroll
    for (int k = 0; k < WPL; ++k) {
        const int w = min(gl + 32 * k, words - 1);
        g4[k] = ((const float4*)gamma)[w];
        b4[k] = ((const float4*)bsrc)[w];
    }
    if (tid < 256)
        s_dq[tid] = (double)dequant_f32((int64_t)(tid - 128) + x_so, in_zp,
                                        in_scale);
    __syncthreads();
    const double inv_cols = 1.0 / (double)cols;
    for (int64_t r = first; r - (lane >> 5) < rows; r += step) {
        if (r != first) load_row(r);
        double v[WPL][4];
        double s = 0.0;
        // words past the row (a clamped re-read) count as zeros
#pragma unroll
        for (int k = 0; k < WPL; ++k)
#pragma unroll
            for (int b = 0; b < 4; ++b)
                v[k][b] = s_dq[((u[k] >> (8 * b)) & 255) ^ 128];
#pragma unroll
        for (int k = 0; k < WPL; ++k) {
            const bool live = gl + 32 * k < words;
#pragma unroll
            for (int b = 0; b < 4; ++b) s += live ? v[k][b] : 0.0;
        }
        const double mean = group_sum<32>(s) * inv_cols;
        double q2 = 0.0;
#pragma unroll
        for (int k = 0; k < WPL; ++k) {
            const bool live = gl + 32 * k < words;
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const double t = live ? v[k][b] - mean : 0.0;
                q2 = fma(t, t, q2);
            }
        }
        const double rsd =
            1.0 / sqrt(group_sum<32>(q2) * inv_cols + eps);
        if (r < rows) {
            uint32_t* yr = (uint32_t*)(y + r * y_rs);
#pragma unroll
            for (int k = 0; k < WPL; ++k) {
                const int w = gl + 32 * k;
                if (w >= words) continue;
                const float gg[4] = {g4[k].x, g4[k].y, g4[k].z, g4[k].w};
                const float bb[4] = {b4[k].x * bmul, b4[k].y * bmul,
                                     b4[k].z * bmul, b4[k].w * bmul};
                float t[4], q[4];
                bool slow = false;
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    t[b] = (float)fma((v[k][b] - mean) * rsd, (double)gg[b],
                                      (double)bb[b]);
                    const float rr = rintf(t[b] * o.invf);
                    const float dd = fmaf(t[b], o.invf, -rr);
                    slow |= !(fabsf(dd) < o.tie);
                    q[b] = __builtin_amdgcn_fmed3f(rr + o.cb, o.lob, o.hib);
                }
                if (__builtin_expect(slow, 0)) {
#pragma unroll
                    for (int b = 0; b < 4; ++b)
                        q[b] = (float)(ln_quant_exact(t[b], o.scale, o.inv,
                                                      o.zp, o.qmin, o.qmax) -
                                       o.so + 128);
                }
                if (__builtin_expect(o.wrap, 0)) {
#pragma unroll
                    for (int b = 0; b < 4; ++b)
                        q[b] = (float)((int)q[b] & 255);
                }
                uint32_t wv = __builtin_amdgcn_cvt_pk_u8_f32(q[0], 0, 0u);
                wv = __builtin_amdgcn_cvt_pk_u8_f32(q[1], 1, wv);
                wv = __builtin_amdgcn_cvt_pk_u8_f32(q[2], 2, wv);
                wv = __builtin_amdgcn_cvt_pk_u8_f32(q[3], 3, wv);
                yr[w] = wv ^ 0x80808080u;
            }
        }
    }
}

// ---------------------------------------------- activation x activation --
// C[b0, b1, m, n] = quantize(sa * sb * sum_k (A[.., m, k] - za) *
// (Bt[.., n, k] - zb)); A and Bt have unit stride along k. A work-group
// computes a 64 x 64 block of C, 4 x 4 per thread, K staged through LDS in
// chunks of 64. int8 storage: v_dot4_i32_i8 on the stored bytes, centred by
// row / column sums; int16: exact int64 products.
template <class T>
__global__ __launch_bounds__(kThreads) void k_matmul_act(qa_matmul_desc d) {
    constexpr int KC = 64;
    constexpr bool I8 = sizeof(T) == 1;
    constexpr int PAD = I8 ? 4 : 2;  // keeps 4-byte words aligned
    __shared__ T sa[64][KC + PAD];
    __shared__ T sb[64][KC + PAD];
    const int tid = threadIdx.x;
    const int tx = tid & 15, ty = tid >> 4;
    const int64_t bz = blockIdx.z;
    const int64_t b0 = bz / d.B1, b1 = bz - b0 * d.B1;
    const int64_t m0 = (int64_t)blockIdx.y * 64, n0 = (int64_t)blockIdx.x * 64;
    const T* A = (const T*)d.a + b0 * d.a_s0 + b1 * d.a_s1;
    const T* B = (const T*)d.b + b0 * d.b_s0 + b1 * d.b_s1;
    // centred = stored + add
    const int64_t a_add = d.a_so - d.a_zp, b_add = d.b_so - d.b_zp;
    int64_t acc[4][4] = {};
    int32_t acc32[4][4] = {};
    int32_t rs[4] = {0, 0, 0, 0}, cs[4] = {0, 0, 0, 0};  // stored sums
    for (int64_t k0 = 0; k0 < d.K; k0 += KC) {
        // stage: 64 rows x KC elements of each operand, zero past the ends;
        // consecutive threads walk the operand's unit-stride axis
        for (int e = tid; e < 64 * KC; e += kThreads) {
            int r = e / KC, c = e - r * KC;
            if (d.a_sk != 1) {
                c = e / 64;
                r = e - c * 64;
            }
            const int64_t m = m0 + r, k = k0 + c;
            sa[r][c] =
                (m < d.M && k < d.K) ? A[m * d.a_sm + k * d.a_sk] : (T)0;
        }
        for (int e = tid; e < 64 * KC; e += kThreads) {
            int r = e / KC, c = e - r * KC;
            if (d.b_sk != 1) {
                c = e / 64;
                r = e - c * 64;
            }
            const int64_t n = n0 + r, k = k0 + c;
            sb[r][c] =
                (n < d.N && k < d.K) ? B[n * d.b_sn + k * d.b_sk] : (T)0;
        }
        __syncthreads();
        if (I8) {
#pragma unroll 4
            for (int kk = 0; kk < KC; kk += 4) {
                int aw[4], bw[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    aw[i] = *(const int*)&sa[ty * 4 + i][kk];
                    bw[i] = *(const int*)&sb[tx * 4 + i][kk];
                }
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        acc32[i][j] = __builtin_amdgcn_sdot4(aw[i], bw[j],
                                                             acc32[i][j], false);
                if (a_add != 0 || b_add != 0) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        rs[i] = __builtin_amdgcn_sdot4(aw[i], 0x01010101, rs[i],
                                                       false);
                        cs[i] = __builtin_amdgcn_sdot4(bw[i], 0x01010101, cs[i],
                                                       false);
                    }
                }
            }
        } else {
            for (int kk = 0; kk < KC && k0 + kk < d.K; ++kk) {
                int64_t av[4], bv[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    av[i] = (int64_t)sa[ty * 4 + i][kk] + a_add;
                    bv[i] = (int64_t)sb[tx * 4 + i][kk] + b_add;
                }
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j) acc[i][j] += av[i] * bv[j];
            }
        }
        __syncthreads();
    }
    const double scale = d.a_scale * d.b_scale;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int64_t m = m0 + ty * 4 + i;
        if (m >= d.M) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t n = n0 + tx * 4 + j;
            if (n >= d.N) continue;
            int64_t v = acc[i][j];
            if (I8)  // (sa + a_add)(sb + b_add) summed over the K real terms
                v = (int64_t)acc32[i][j] + a_add * cs[j] + b_add * rs[i] +
                    d.K * a_add * b_add;
            const float yf = (float)((double)v * scale);
            const int64_t q =
                qa_quantize_one(yf, d.out_scale, d.out_zp, d.qmin, d.qmax);
            store_any(d.y, (int)d.y_code,
                      b0 * d.y_s0 + b1 * d.y_s1 + m * d.y_sm + n * d.y_sn,
                      q - d.y_so);
        }
    }
}

// int8 operands on the matrix cores. A work-group owns one (b0, b1) pair
// and 64 rows of C (16 per wave) and all N columns: it stages its A rows and
// all of Bt ([N, K]) in LDS, K zero-padded to a multiple of 64, then each
// wave runs v_mfma_i32_16x16x64_i8 over its 16 rows x every 16-column tile
// (lane l supplies row / column l % 16, bytes 16 (l / 16) .. + 15 of the
// 64-byte K-step; result register r of lane l is row 4 (l / 16) + r,
// column l % 16). Centring by row / column sums as k_matmul_act.
typedef int v4i_t __attribute__((ext_vector_type(4)));

template <bool SUMS, class TO>
__global__ __launch_bounds__(kThreads) void k_matmul_act_mfma(
    qa_matmul_desc d, int Kp, int Np) {
    extern __shared__ int4 lds4[];
    int8_t* lds = (int8_t*)lds4;
    const int RS = Kp + 16;  // LDS row stride (bytes)
    int8_t* sa = lds;                    // [64][RS]
    int8_t* sb = lds + 64 * RS;          // [Np][RS]
    int* ssum = (int*)(sb + Np * RS);    // [64 + Np] row / column sums
    const int tid = threadIdx.x;
    const int64_t bz = blockIdx.y;
    const int64_t b0 = bz / d.B1, b1 = bz - b0 * d.B1;
    const int64_t m0 = (int64_t)blockIdx.x * 64;
    const int8_t* A = (const int8_t*)d.a + b0 * d.a_s0 + b1 * d.a_s1;
    const int8_t* B = (const int8_t*)d.b + b0 * d.b_s0 + b1 * d.b_s1;
    auto stage = [&](int8_t* dst, const int8_t* src, int rows, int64_t r0,
                     int64_t rlim, int64_t rs, int64_t ks) {
        stage_i8_rows(dst, RS, src, rows, r0, rlim, rs, ks, d.K, Kp, tid);
    };
    stage(sa, A, 64, m0, d.M, d.a_sm, d.a_sk);
    stage(sb, B, Np, 0, d.N, d.b_sn, d.b_sk);
    __syncthreads();
    if (SUMS) {
        for (int r = tid; r < 64 + Np; r += kThreads) {
            const int8_t* row = r < 64 ? sa + r * RS : sb + (r - 64) * RS;
            int acc = 0;
            for (int c = 0; c < Kp; c += 4)
                acc = __builtin_amdgcn_sdot4(*(const int*)(row + c),
                                             0x01010101, acc, false);
            ssum[r] = acc;
        }
        __syncthreads();
    }
    const int lane = tid & 63, wave = tid >> 6;
    const int col = lane & 15, kg = lane >> 4;
    const int64_t a_add = d.a_so - d.a_zp, b_add = d.b_so - d.b_zp;
    const double scale = d.a_scale * d.b_scale;
    const double inv = 1.0 / d.out_scale;
    const bool f32ok = qa_f32_form_ok(d.out_scale, d.out_zp, d.qmin, d.qmax);
    const float invf = (float)inv;
    const int mr = wave * 16;  // the wave's 16 rows within the block
    if (m0 + mr >= d.M) return;
    const int ksteps = Kp / 64;
    // output row bases of the lane's 4 rows (hoisted out of the column
    // loop: four 64-bit products per element otherwise)
    TO* yrow[4];
#pragma unroll
    for (int r = 0; r < 4; ++r)
        yrow[r] = (TO*)d.y + b0 * d.y_s0 + b1 * d.y_s1 +
                  (m0 + mr + 4 * kg + r) * d.y_sm;
    // zero-point corrections: the row terms of the lane's 4 rows once per
    // wave, the column term once per column tile
    int64_t rterm[4] = {0, 0, 0, 0};
    if (SUMS) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
            rterm[r] = b_add * ssum[min(mr + 4 * kg + r, 63)] +
                       d.K * a_add * b_add;
    }
    for (int nt = 0; nt < Np; nt += 16) {
        v4i_t acc = {0, 0, 0, 0};
        for (int ks = 0; ks < ksteps; ++ks) {
            const int c = ks * 64 + kg * 16;
            const v4i_t fa = *(const v4i_t*)(sa + (mr + col) * RS + c);
            const v4i_t fb = *(const v4i_t*)(sb + (nt + col) * RS + c);
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa, fb, acc, 0, 0, 0);
        }
        const int64_t n = nt + col;
        if (n >= d.N) continue;
        const int64_t cterm = SUMS ? a_add * ssum[64 + n] : 0;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int ml = mr + 4 * kg + r;
            const int64_t m = m0 + ml;
            if (m >= d.M) continue;
            int64_t v = acc[r];
            if (SUMS) v += cterm + rterm[r];
            const float yf = (float)((double)v * scale);
            const int64_t q = qa_quantize_mixed(yf, f32ok, invf, d.out_scale,
                                                inv, d.out_zp, d.qmin, d.qmax);
            yrow[r][n * d.y_sn] = (TO)(q - d.y_so);
        }
    }
}

bool launched(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_hip_error(what, e);
        return false;
    }
    return true;
}

bool code_ok(int64_t c) { return c == 1 || c == 2 || c == 4; }

}  // namespace
}  // namespace qa

using namespace qa;

QA_API int qa_d_copy_nd(const qa_nd_copy* d, void* stream) {
    if (!d || d->ndim < 1 || d->ndim > 6 || !code_ok(d->x_code) ||
        !code_ok(d->y_code) || d->mode < 0 || d->mode > 2) {
        set_error("qa_d_copy_nd", "bad descriptor");
        return -1;
    }
    int64_t total = 1;
    for (int k = 0; k < d->ndim; ++k) {
        if (d->shape[k] < 0) {
            set_error("qa_d_copy_nd", "negative extent");
            return -1;
        }
        total *= d->shape[k];
    }
    if (total == 0) return 0;
    if (copy_nd16_applies(*d, total)) {
        const int es = (int)d->x_code;
        const int64_t cpr = d->shape[d->ndim - 1] * es / 16;
        const int64_t chunks = total * es / 16;
        const int64_t blocks =
            std::min<int64_t>(ceil_div(chunks, kThreads), 65535);
        k_copy_nd16<<<(unsigned)blocks, kThreads, 0, (hipStream_t)stream>>>(
            (const char*)d->x, (char*)d->y, (int)d->ndim, cpr, chunks, *d,
            es);
        return launched("qa_d_copy_nd") ? 0 : -1;
    }
    const int64_t blocks = std::min<int64_t>(ceil_div(total, kThreads), 65535);
    if (total < ((int64_t)1 << 32))  // every extent divides in 32 bits
        k_copy_nd<true><<<(unsigned)blocks, kThreads, 0,
                          (hipStream_t)stream>>>(*d, total);
    else
        k_copy_nd<false><<<(unsigned)blocks, kThreads, 0,
                           (hipStream_t)stream>>>(*d, total);
    return launched("qa_d_copy_nd") ? 0 : -1;
}

QA_API int qa_d_layernorm(const void* x, int x_code, int64_t x_rstride,
                          int64_t rows, int64_t cols, double in_scale,
                          int64_t in_zp, int64_t x_so, const float* gamma,
                          const float* beta, double eps, void* y, int y_code,
                          int64_t y_rstride, double out_scale, int64_t out_zp,
                          int64_t qmin, int64_t qmax, int64_t y_so,
                          void* stream) {
    if (rows <= 0 || cols <= 0) return 0;
    if (!x || !y || !gamma || !code_ok(x_code) || !code_ok(y_code)) {
        set_error("qa_d_layernorm", "bad arguments");
        return -1;
    }
    hipStream_t st = (hipStream_t)stream;
    // int8 rows of 4-byte words, at most 512 values: the word kernel
    if (x_code == 1 && y_code == 1 && cols % 4 == 0 && cols <= 512 &&
        x_rstride % 4 == 0 && y_rstride % 4 == 0 &&
        ((uintptr_t)x | (uintptr_t)y | (uintptr_t)gamma |
         (uintptr_t)(beta ? beta : gamma)) % 16 == 0) {
        constexpr int NW = 16;  // waves a work-group, 2 rows each
        const int64_t blocks =
            std::min<int64_t>(ceil_div(rows, 2 * NW), 65535);
        LnQ o;
        o.scale = out_scale;
        o.inv = 1.0 / out_scale;
        o.invf = (float)o.inv;
        o.tie = qa_f32_form_ok(out_scale, out_zp, qmin, qmax)
                    ? qa_f32_tie(out_zp, qmin, qmax)
                    : -1.0f;
        o.cb = (float)(out_zp - y_so + 128);
        o.lob = (float)(qmin - y_so + 128);
        o.hib = (float)(qmax - y_so + 128);
        o.zp = (int)out_zp;
        o.qmin = (int)qmin;
        o.qmax = (int)qmax;
        o.so = (int)y_so;
        o.wrap = qmin - y_so < -128 || qmax - y_so > 127;
        auto run = [&](auto kern) {
            kern<<<(unsigned)blocks, 64 * NW, 0, st>>>(
                (const int8_t*)x, x_rstride, rows, cols, in_scale, in_zp, x_so,
                gamma, beta, eps, (int8_t*)y, y_rstride, o);
        };
        const int wpl = (int)ceil_div(cols / 4, 32);
        if (wpl <= 1)
            run(k_layernorm_w<1, NW>);
        else if (wpl <= 2)
            run(k_layernorm_w<2, NW>);
        else if (wpl == 3)
            run(k_layernorm_w<3, NW>);
        else
            run(k_layernorm_w<4, NW>);
        return launched("qa_d_layernorm") ? 0 : -1;
    }
    auto go = [&](auto ti, auto to) {
        typedef decltype(ti) TI;
        typedef decltype(to) TO;
        if (cols <= 32 * 16) {  // 32 lanes a row, 2 rows a wave
            const int64_t blocks = std::min<int64_t>(ceil_div(rows, 8), 65535);
            k_layernorm<32, 16, TI, TO><<<(unsigned)blocks, kThreads, 0, st>>>(
                (const TI*)x, x_rstride, rows, cols, in_scale, in_zp, x_so,
                gamma, beta, eps, (TO*)y, y_rstride, out_scale, out_zp, qmin,
                qmax, y_so);
        } else {
            const int64_t blocks = std::min<int64_t>(ceil_div(rows, 4), 65535);
            k_layernorm<64, 0, TI, TO><<<(unsigned)blocks, kThreads, 0, st>>>(
                (const TI*)x, x_rstride, rows, cols, in_scale, in_zp, x_so,
                gamma, beta, eps, (TO*)y, y_rstride, out_scale, out_zp, qmin,
                qmax, y_so);
        }
    };
    if (x_code == 1 && y_code == 1)
        go(int8_t{}, int8_t{});
    else if (x_code == 2 && y_code == 2)
        go(int16_t{}, int16_t{});
    else {
        set_error("qa_d_layernorm", "input and output of one int8 / int16 "
                                    "storage");
        return -1;
    }
    return launched("qa_d_layernorm") ? 0 : -1;
}

QA_API int qa_d_matmul_act(const qa_matmul_desc* d, void* stream) {
    if (!d || d->a_code != d->b_code || (d->a_code != 1 && d->a_code != 2) ||
        !code_ok(d->y_code) || d->B0 < 0 || d->B1 <= 0 || d->M < 0 ||
        d->N < 0 || d->K < 0 || d->K >= (1 << 17)) {
        set_error("qa_d_matmul_act",
                  "needs int8 or int16 operands of one storage, K < 2^17");
        return -1;
    }
    if (d->B0 * d->B1 * d->M * d->N == 0) return 0;
    const int64_t gx = ceil_div(d->N, 64), gy = ceil_div(d->M, 64);
    const int64_t gz = d->B0 * d->B1;
    if (gx > 65535 || gy > 65535 || gz > 65535) {
        set_error("qa_d_matmul_act", "grid too large");
        return -1;
    }
    const dim3 grid((unsigned)gx, (unsigned)gy, (unsigned)gz);
    if (d->a_code == 1) {
        // matrix cores when the block's operands fit in LDS
        const int64_t Kp = round_up(std::max<int64_t>(d->K, 1), 64);
        const int64_t Np = round_up(d->N, 16);
        const int64_t bytes = (64 + Np) * (Kp + 16) + (64 + Np) * 4;
        if (bytes <= 64 * 1024 && ceil_div(d->M, 64) <= 65535 &&
            d->y_code == 1) {
            const dim3 g2((unsigned)ceil_div(d->M, 64), (unsigned)gz);
            const bool sums = d->a_so != d->a_zp || d->b_so != d->b_zp;
            if (sums)
                k_matmul_act_mfma<true, int8_t><<<g2, kThreads, bytes,
                                                  (hipStream_t)stream>>>(
                    *d, (int)Kp, (int)Np);
            else
                k_matmul_act_mfma<false, int8_t><<<g2, kThreads, bytes,
                                                   (hipStream_t)stream>>>(
                    *d, (int)Kp, (int)Np);
        } else {
            k_matmul_act<int8_t><<<grid, kThreads, 0, (hipStream_t)stream>>>(
                *d);
        }
    } else
        k_matmul_act<int16_t><<<grid, kThreads, 0, (hipStream_t)stream>>>(*d);
    return launched("qa_d_matmul_act") ? 0 : -1;
}

// VALU kernels: the exact integer convolution for operands that do not fit
// int8 after an offset (modulo-2^32 int32 or exact int64 accumulation, the
// 16-bit-model path), the ABI's VALU GEMM and the float32 conv / GEMM.
#include <algorithm>

#include "qa_conv.h"
#include "qa_valu.h"

namespace qa {
namespace {

constexpr int kThreads = 256;

// grid: x = pixel blocks of one image, y = output channels, z = images
// (y and z loop when Cout or N exceed the grid).
// Element (n, c, iy, ix) of x at x + n*x_sn + c*x_sc + (iy*W + ix)*x_sp.
template <bool WIDE>
__device__ __forceinline__ void conv_valu_one(const ConvArgs& a, int n, int co,
                                              int pix) {
    const int oy = pix / a.OW;
    const int ox = pix - oy * a.OW;
    const int g = co / a.Cog;
    const int64_t xb = (int64_t)n * a.x_sn + (int64_t)g * a.Cg * a.x_sc;
    const int64_t wb = (int64_t)co * a.Cg * a.KH * a.KW;
    uint32_t acc32 = 0;
    int64_t acc64 = 0;
    for (int ky = 0; ky < a.KH; ++ky) {
        const int iy = oy * a.SH - a.PH + ky * a.DH;
        if (iy < 0 || iy >= a.H) continue;
        for (int kx = 0; kx < a.KW; ++kx) {
            const int ix = ox * a.SW - a.PW + kx * a.DW;
            if (ix < 0 || ix >= a.W) continue;
            const int64_t pb = xb + ((int64_t)iy * a.W + ix) * a.x_sp;
            for (int c = 0; c < a.Cg; ++c) {
                int64_t xv = load_any(a.x, a.x_code, pb + c * a.x_sc) +
                             a.x_add;
                if (a.narrow16) xv = (int16_t)xv;
                const int64_t wv = load_any(
                    a.w, a.w_code, wb + ((int64_t)c * a.KH + ky) * a.KW + kx);
                if (WIDE)
                    acc64 += xv * wv;
                else
                    acc32 += (uint32_t)((int32_t)xv * (int32_t)wv);
            }
        }
    }
    const int64_t v = WIDE ? acc64 : (int64_t)(int32_t)acc32;
    const int64_t yi = (int64_t)n * a.y_sn + (int64_t)co * a.y_sc +
                       (int64_t)pix * a.y_sp;
    if (a.mode != EPI_QUANT) {
        store_any(a.y, a.y_code, yi, v);
        return;
    }
    int64_t rq = 0;
    if (a.res)
        rq = load_any(a.res, a.y_code, (int64_t)n * a.res_sn +
                                           (int64_t)co * a.res_sc +
                                           (int64_t)pix * a.res_sp) +
             a.res_so;
    const int64_t q = quant_one(a, v + (a.pre ? a.pre[co] : 0), a.mult[co],
                                a.shift[co], rq);
    store_any(a.y, a.y_code, yi, q - a.y_so);
    if (a.y2)
        store_any(a.y2, a.y_code,
                  (int64_t)n * a.y2_sn + (int64_t)co * a.y2_sc +
                      (int64_t)pix * a.y2_sp,
                  rescale2(a, q) - a.y_so);
}

template <bool WIDE>
__global__ __launch_bounds__(kThreads) void k_conv_valu(ConvArgs a) {
    const int pix = blockIdx.x * kThreads + threadIdx.x;
    if (pix >= a.OH * a.OW) return;
    for (int n = blockIdx.z; n < a.N; n += gridDim.z)
        for (int co = blockIdx.y; co < a.Cout; co += gridDim.y)
            conv_valu_one<WIDE>(a, n, co, pix);
}

template <bool WIDE>
__global__ __launch_bounds__(kThreads) void k_gemm_valu(
    const void* A, int a_code, const void* B, int b_code, void* C, int64_t M,
    int64_t N, int64_t K, const int32_t* gate, int32_t gate_on) {
    if (gate != nullptr && *gate != gate_on) return;
    const int64_t j = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (j >= N) return;
    for (int64_t i = blockIdx.y; i < M; i += gridDim.y) {
        uint32_t acc32 = 0;
        int64_t acc64 = 0;
        for (int64_t k = 0; k < K; ++k) {
            const int64_t x = load_any(A, a_code, i * K + k);
            const int64_t y = load_any(B, b_code, k * N + j);
            if (WIDE)
                acc64 += x * y;
            else
                acc32 += (uint32_t)((int32_t)x * (int32_t)y);
        }
        if (WIDE)
            ((int64_t*)C)[i * N + j] = acc64;
        else
            ((int32_t*)C)[i * N + j] = (int32_t)acc32;
    }
}

__global__ __launch_bounds__(kThreads) void k_conv_f32(const float* x,
                                                       const float* w,
                                                       float* y, ConvArgs a) {
    const int OHW = a.OH * a.OW;
    const int pix = blockIdx.x * kThreads + threadIdx.x;
    if (pix >= OHW) return;
    const int oy = pix / a.OW;
    const int ox = pix - oy * a.OW;
    const int64_t HW = (int64_t)a.H * a.W;
    for (int n = blockIdx.z; n < a.N; n += gridDim.z)
        for (int co = blockIdx.y; co < a.Cout; co += gridDim.y) {
            const int g = co / a.Cog;
            const float* xb = x + (int64_t)n * a.Cg * a.G * HW +
                              (int64_t)g * a.Cg * HW;
            const float* wb = w + (int64_t)co * a.Cg * a.KH * a.KW;
            float acc = 0.f;
            for (int ci = 0; ci < a.Cg; ++ci)
                for (int ky = 0; ky < a.KH; ++ky) {
                    const int iy = oy * a.SH - a.PH + ky * a.DH;
                    if (iy < 0 || iy >= a.H) continue;
                    for (int kx = 0; kx < a.KW; ++kx) {
                        const int ix = ox * a.SW - a.PW + kx * a.DW;
                        if (ix < 0 || ix >= a.W) continue;
                        acc = fmaf(wb[(ci * a.KH + ky) * a.KW + kx],
                                   xb[ci * HW + (int64_t)iy * a.W + ix], acc);
                    }
                }
            y[((int64_t)n * a.Cout + co) * OHW + pix] = acc;
        }
}

// 16x16 output tile per 256 threads, K staged through LDS in slices of 16.
__global__ __launch_bounds__(kThreads) void k_gemm_f32(const float* A,
                                                       const float* B,
                                                       float* C, int64_t M,
                                                       int64_t N, int64_t K) {
    __shared__ float sa[16][17];
    __shared__ float sb[16][17];
    const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
    const int64_t col = (int64_t)blockIdx.x * 16 + tx;
    for (int64_t rb = (int64_t)blockIdx.y * 16; rb < M;
         rb += (int64_t)gridDim.y * 16) {
        const int64_t row = rb + ty;
        float acc = 0.f;
        for (int64_t k0 = 0; k0 < K; k0 += 16) {
            sa[ty][tx] = (row < M && k0 + tx < K) ? A[row * K + k0 + tx] : 0.f;
            sb[ty][tx] =
                (k0 + ty < K && col < N) ? B[(k0 + ty) * N + col] : 0.f;
            __syncthreads();
#pragma unroll
            for (int k = 0; k < 16; ++k) acc = fmaf(sa[ty][k], sb[k][tx], acc);
            __syncthreads();
        }
        if (row < M && col < N) C[row * N + col] = acc;
    }
}

bool check(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_hip_error(what, e);
        return false;
    }
    return true;
}

}  // namespace

bool launch_conv_valu(const ConvArgs& a, hipStream_t st) {
    const int OHW = a.OH * a.OW;
    if (OHW <= 0 || a.N <= 0 || a.Cout <= 0) return true;
    dim3 grid((unsigned)ceil_div(OHW, kThreads),
              (unsigned)std::min<int64_t>(a.Cout, 65535),
              (unsigned)std::min<int64_t>(a.N, 65535));
    if (a.wide)
        k_conv_valu<true><<<grid, kThreads, 0, st>>>(a);
    else
        k_conv_valu<false><<<grid, kThreads, 0, st>>>(a);
    return check("k_conv_valu");
}

bool launch_gemm_valu(const void* A, int a_code, const void* B, int b_code,
                      void* C, int64_t M, int64_t N, int64_t K, bool wide,
                      hipStream_t st, const int32_t* gate, int32_t gate_on) {
    if (M <= 0 || N <= 0) return true;
    dim3 grid((unsigned)ceil_div(N, kThreads),
              (unsigned)std::min<int64_t>(M, 65535));
    if (wide)
        k_gemm_valu<true><<<grid, kThreads, 0, st>>>(A, a_code, B, b_code, C,
                                                     M, N, K, gate, gate_on);
    else
        k_gemm_valu<false><<<grid, kThreads, 0, st>>>(A, a_code, B, b_code,
                                                      C, M, N, K, gate,
                                                      gate_on);
    return check("k_gemm_valu");
}

// float32 convolution of one group as an implicit GEMM on the matrix cores
// (v_mfma_f32_16x16x4f32: lane i + 16 k holds A[i][k] and B[k][i], result
// register r of lane j + 16 g is C[4 g + r][j]). A work-group computes 64
// output pixels x 64 output channels of one image; each wave 16 pixels x
// the 64 channels (4 MFMA tiles). K = Cg KH KW runs in slices of 32: the
// im2col slice of the input (zero at the padding) and the weight slice go
// to LDS (rows of 80 floats, so that the 4 lane groups of a fragment read
// disjoint banks), double-buffered: slice s + 1's loads are in flight
// while slice s's MFMAs run. Products are float32, summed in float32 in
// another order than k_conv_f32 (agreement within float32 rounding).
constexpr int CF_K = 32, CF_RS = 80;
typedef float v4f __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(kThreads) void k_conv_f32_mfma(
    const float* __restrict__ x, const float* __restrict__ w,
    float* __restrict__ y, ConvArgs a, uint64_t mg_khw, uint64_t mg_kw) {
    __shared__ float sa[2][CF_K * CF_RS];  // [k][pixel]
    __shared__ float sb[2][CF_K * CF_RS];  // [k][channel]
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int OHW = a.OH * a.OW;
    const int m0 = blockIdx.x * 64, co0 = blockIdx.y * 64;
    const int n = blockIdx.z;
    const int KHW = a.KH * a.KW;
    const int K = a.Cg * KHW;
    const int64_t HW = (int64_t)a.H * a.W;
    const float* xn = x + (int64_t)n * a.Cg * HW;
    // this thread's staging: pixel tid % 64 of the A slice (k rows tid / 64
    // + 4 u), channel tid / 32 + 8 u of the B slice (k column tid % 32)
    const int ap = tid & 63, ak = tid >> 6;
    const int pix = m0 + ap;
    const bool pin = pix < OHW;
    const int oy = pin ? pix / a.OW : 0;
    const int ox = pin ? pix - oy * a.OW : 0;
    const int iy0 = oy * a.SH - a.PH, ix0 = ox * a.SW - a.PW;
    const int bk = tid & 31, bc = tid >> 5;
    float ra[8], rb[8];
    auto load = [&](int k0) {
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int k = k0 + ak + 4 * u;
            float v = 0.f;
            if (pin && k < K) {
                const int ci = (int)(((uint64_t)(uint32_t)k * mg_khw) >> 32);
                const int t = k - ci * KHW;
                const int ky = (int)(((uint64_t)(uint32_t)t * mg_kw) >> 32);
                const int kx = t - ky * a.KW;
                const int iy = iy0 + ky * a.DH, ix = ix0 + kx * a.DW;
                if ((unsigned)iy < (unsigned)a.H && (unsigned)ix < (unsigned)a.W)
                    v = xn[ci * HW + (int64_t)iy * a.W + ix];
            }
            ra[u] = v;
            const int co = co0 + bc + 8 * u, kb = k0 + bk;
            rb[u] = (co < a.Cout && kb < K) ? w[(int64_t)co * K + kb] : 0.f;
        }
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            sa[buf][(ak + 4 * u) * CF_RS + ap] = ra[u];
            sb[buf][bk * CF_RS + bc + 8 * u] = rb[u];
        }
    };
    v4f acc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] = v4f{0.f, 0.f, 0.f, 0.f};
    const int col = lane & 15, kg = lane >> 4;
    const int nsl = (K + CF_K - 1) / CF_K;
    load(0);
    store(0);
    __syncthreads();
    for (int s = 0; s < nsl; ++s) {
        const int buf = s & 1;
        if (s + 1 < nsl) load((s + 1) * CF_K);  // in flight during the MFMAs
#pragma unroll
        for (int kk = 0; kk < CF_K; kk += 4) {
            const float fa = sa[buf][(kk + kg) * CF_RS + wave * 16 + col];
#pragma unroll
            for (int j = 0; j < 4; ++j)
                acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(
                    fa, sb[buf][(kk + kg) * CF_RS + j * 16 + col], acc[j], 0,
                    0, 0);
        }
        if (s + 1 < nsl) store(buf ^ 1);  // the buffer last read at s - 1
        __syncthreads();
    }
    // lane j + 16 g holds pixels m0 + 16 wave + 4 g + r of channel 16 jt + j
    float* yn = y + (int64_t)n * a.Cout * OHW;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int co = co0 + j * 16 + col;
        if (co >= a.Cout) continue;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int p = m0 + wave * 16 + 4 * kg + r;
            if (p < OHW) yn[(int64_t)co * OHW + p] = acc[j][r];
        }
    }
}

bool launch_conv_f32(const float* x, const float* w, float* y,
                     const ConvArgs& a, hipStream_t st) {
    const int OHW = a.OH * a.OW;
    if (OHW <= 0 || a.N <= 0 || a.Cout <= 0) return true;
    const int64_t K = (int64_t)a.Cg * a.KH * a.KW;
    // (the multiply-shift divisions of k are exact for k < 2^16)
    if (a.G == 1 && K < 65536 && a.N <= 65535 &&
        ceil_div(a.Cout, 64) <= 65535) {
        const int khw = a.KH * a.KW;
        const uint64_t mg_khw = (((uint64_t)1 << 32) + khw - 1) / khw;
        const uint64_t mg_kw = (((uint64_t)1 << 32) + a.KW - 1) / a.KW;
        const dim3 grid((unsigned)ceil_div(OHW, 64),
                        (unsigned)ceil_div(a.Cout, 64), (unsigned)a.N);
        k_conv_f32_mfma<<<grid, kThreads, 0, st>>>(x, w, y, a, mg_khw, mg_kw);
        return check("k_conv_f32_mfma");
    }
    dim3 grid((unsigned)ceil_div(OHW, kThreads),
              (unsigned)std::min<int64_t>(a.Cout, 65535),
              (unsigned)std::min<int64_t>(a.N, 65535));
    k_conv_f32<<<grid, kThreads, 0, st>>>(x, w, y, a);
    return check("k_conv_f32");
}

bool launch_gemm_f32(const float* A, const float* B, float* C, int64_t M,
                     int64_t N, int64_t K, hipStream_t st) {
    if (M <= 0 || N <= 0) return true;
    dim3 grid((unsigned)ceil_div(N, 16),
              (unsigned)std::min<int64_t>(ceil_div(M, 16), 65535));
    k_gemm_f32<<<grid, kThreads, 0, st>>>(A, B, C, M, N, K);
    return check("k_gemm_f32");
}

}  // namespace qa

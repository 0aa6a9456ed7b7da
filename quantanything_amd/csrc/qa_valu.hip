// VALU conv / GEMM kernels (see qa_valu.h). One thread per output element;
// each work-group of 256 threads covers consecutive output pixels of one
// output channel, so the weight reads are wave-uniform (scalar-cached) and
// the activation reads of neighbouring lanes are neighbouring bytes.
#include "qa_epilogue.h"
#include "qa_valu.h"

namespace qa {
namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ int64_t load_x(const void* x, int code, int64_t i) {
    switch (code) {
        case 1: return ((const int8_t*)x)[i];
        case 2: return ((const int16_t*)x)[i];
        default: return ((const int32_t*)x)[i];
    }
}

__device__ __forceinline__ int64_t load_w(const void* w, int code, int64_t i) {
    return code == 2 ? (int64_t)((const int16_t*)w)[i]
                     : (int64_t)((const int32_t*)w)[i];
}

// grid: x = pixel blocks of one image plane, y = output channel, z = image
template <bool WIDE, int MODE>
__global__ __launch_bounds__(kThreads) void k_conv_valu(ValuConv c,
                                                        IgemmArgs e) {
    const int co = blockIdx.y;
    const int n = blockIdx.z;
    const int OHW = c.OH * c.OW;
    const int pix = blockIdx.x * kThreads + threadIdx.x;
    if (pix >= OHW) return;
    const int oy = pix / c.OW;
    const int ox = pix - oy * c.OW;
    const int Cg = c.C / c.G;
    const int Cog = c.Cout / c.G;
    const int g = co / Cog;
    const int64_t HW = (int64_t)c.H * c.W;
    const int64_t xbase = (int64_t)n * c.x_nstride + (int64_t)g * Cg * HW;
    const int64_t wbase = (int64_t)co * Cg * c.KH * c.KW;
    uint32_t acc32 = 0;
    int64_t acc64 = 0;
    for (int ci = 0; ci < Cg; ++ci) {
        for (int ky = 0; ky < c.KH; ++ky) {
            const int iy = oy * c.SH - c.PH + ky * c.DH;
            if (iy < 0 || iy >= c.H) continue;
            for (int kx = 0; kx < c.KW; ++kx) {
                const int ix = ox * c.SW - c.PW + kx * c.DW;
                if (ix < 0 || ix >= c.W) continue;
                int64_t xv = load_x(c.x, c.x_code,
                                    xbase + ci * HW + (int64_t)iy * c.W + ix) +
                             c.x_add;
                if (c.narrow16) xv = (int16_t)xv;
                const int64_t wv =
                    load_w(c.w, c.w_code, wbase + (ci * c.KH + ky) * c.KW + kx);
                if (WIDE)
                    acc64 += xv * wv;
                else
                    acc32 += (uint32_t)((int32_t)xv * (int32_t)wv);
            }
        }
    }
    const int64_t oidx =
        (int64_t)n * e.y_nstride + (e.y_choff + co) * (int64_t)OHW + pix;
    if (MODE == EPI_RAW64) {
        ((int64_t*)e.y)[oidx] = WIDE ? acc64 : (int64_t)(int32_t)acc32;
    } else if (MODE == EPI_RAW32) {
        ((int32_t*)e.y)[oidx] = WIDE ? (int32_t)acc64 : (int32_t)acc32;
    } else {
        const int64_t v = (WIDE ? acc64 : (int64_t)(int32_t)acc32) +
                          (e.pre ? e.pre[co] : 0);
        int64_t rq = 0;
        const bool has_res = e.res != nullptr;
        if (has_res) {
            const int64_t ridx = (int64_t)n * e.res_nstride +
                                 (e.res_choff + co) * (int64_t)OHW + pix;
            rq = (e.out_code == 1 ? (int64_t)((const int8_t*)e.res)[ridx]
                                  : (int64_t)((const int16_t*)e.res)[ridx]) +
                 e.res_so;
        }
        const int64_t q =
            quant_one(e, v, e.mult[co], e.shift[co], rq, has_res) - e.out_so;
        if (e.out_code == 1)
            ((int8_t*)e.y)[oidx] = (int8_t)q;
        else
            ((int16_t*)e.y)[oidx] = (int16_t)q;
    }
}

template <bool WIDE>
__global__ __launch_bounds__(kThreads) void k_gemm_valu(
    const void* A, int a_code, const void* B, int b_code, void* C, int64_t M,
    int64_t N, int64_t K) {
    const int64_t j = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    const int64_t i = blockIdx.y;
    if (j >= N) return;
    uint32_t acc32 = 0;
    int64_t acc64 = 0;
    for (int64_t k = 0; k < K; ++k) {
        const int64_t a = load_w(A, a_code, i * K + k);
        const int64_t b = load_w(B, b_code, k * N + j);
        if (WIDE)
            acc64 += a * b;
        else
            acc32 += (uint32_t)((int32_t)a * (int32_t)b);
    }
    if (WIDE)
        ((int64_t*)C)[i * N + j] = acc64;
    else
        ((int32_t*)C)[i * N + j] = (int32_t)acc32;
}

__global__ __launch_bounds__(kThreads) void k_conv_f32(const float* x,
                                                       const float* w,
                                                       float* y, ValuConv c) {
    const int co = blockIdx.y;
    const int n = blockIdx.z;
    const int OHW = c.OH * c.OW;
    const int pix = blockIdx.x * kThreads + threadIdx.x;
    if (pix >= OHW) return;
    const int oy = pix / c.OW;
    const int ox = pix - oy * c.OW;
    const int Cg = c.C / c.G;
    const int Cog = c.Cout / c.G;
    const int g = co / Cog;
    const int64_t HW = (int64_t)c.H * c.W;
    const float* xb = x + (int64_t)n * c.C * HW + (int64_t)g * Cg * HW;
    const float* wb = w + (int64_t)co * Cg * c.KH * c.KW;
    float acc = 0.f;
    for (int ci = 0; ci < Cg; ++ci)
        for (int ky = 0; ky < c.KH; ++ky) {
            const int iy = oy * c.SH - c.PH + ky * c.DH;
            if (iy < 0 || iy >= c.H) continue;
            for (int kx = 0; kx < c.KW; ++kx) {
                const int ix = ox * c.SW - c.PW + kx * c.DW;
                if (ix < 0 || ix >= c.W) continue;
                acc = fmaf(wb[(ci * c.KH + ky) * c.KW + kx],
                           xb[ci * HW + (int64_t)iy * c.W + ix], acc);
            }
        }
    y[((int64_t)n * c.Cout + co) * OHW + pix] = acc;
}

// 16x16 output tile per 256 threads, K staged through LDS in slices of 16.
__global__ __launch_bounds__(kThreads) void k_gemm_f32(const float* A,
                                                       const float* B,
                                                       float* C, int64_t M,
                                                       int64_t N, int64_t K) {
    __shared__ float sa[16][17];
    __shared__ float sb[16][17];
    const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
    const int64_t row = (int64_t)blockIdx.y * 16 + ty;
    const int64_t col = (int64_t)blockIdx.x * 16 + tx;
    float acc = 0.f;
    for (int64_t k0 = 0; k0 < K; k0 += 16) {
        sa[ty][tx] = (row < M && k0 + tx < K) ? A[row * K + k0 + tx] : 0.f;
        sb[ty][tx] = (k0 + ty < K && col < N) ? B[(k0 + ty) * N + col] : 0.f;
        __syncthreads();
#pragma unroll
        for (int k = 0; k < 16; ++k) acc = fmaf(sa[ty][k], sb[k][tx], acc);
        __syncthreads();
    }
    if (row < M && col < N) C[row * N + col] = acc;
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

bool launch_conv_valu(const ValuConv& c, const IgemmArgs& e, int mode,
                      hipStream_t st) {
    const int OHW = c.OH * c.OW;
    if (OHW <= 0 || c.N <= 0 || c.Cout <= 0) return true;
    dim3 grid((unsigned)ceil_div(OHW, kThreads), (unsigned)c.Cout,
              (unsigned)c.N);
    if (c.wide) {
        if (mode == EPI_RAW64)
            k_conv_valu<true, EPI_RAW64><<<grid, kThreads, 0, st>>>(c, e);
        else if (mode == EPI_RAW32)
            k_conv_valu<true, EPI_RAW32><<<grid, kThreads, 0, st>>>(c, e);
        else
            k_conv_valu<true, EPI_QUANT><<<grid, kThreads, 0, st>>>(c, e);
    } else {
        if (mode == EPI_RAW64)
            k_conv_valu<false, EPI_RAW64><<<grid, kThreads, 0, st>>>(c, e);
        else if (mode == EPI_RAW32)
            k_conv_valu<false, EPI_RAW32><<<grid, kThreads, 0, st>>>(c, e);
        else
            k_conv_valu<false, EPI_QUANT><<<grid, kThreads, 0, st>>>(c, e);
    }
    return check("k_conv_valu");
}

bool launch_gemm_valu(const void* A, int a_code, const void* B, int b_code,
                      void* C, int64_t M, int64_t N, int64_t K, bool wide,
                      hipStream_t st) {
    if (M <= 0 || N <= 0) return true;
    if (M > 65535) {
        set_error("launch_gemm_valu", "M above 65535");
        return false;
    }
    dim3 grid((unsigned)ceil_div(N, kThreads), (unsigned)M);
    if (wide)
        k_gemm_valu<true><<<grid, kThreads, 0, st>>>(A, a_code, B, b_code, C,
                                                     M, N, K);
    else
        k_gemm_valu<false><<<grid, kThreads, 0, st>>>(A, a_code, B, b_code,
                                                      C, M, N, K);
    return check("k_gemm_valu");
}

bool launch_conv_f32(const float* x, const float* w, float* y,
                     const ValuConv& c, hipStream_t st) {
    const int OHW = c.OH * c.OW;
    if (OHW <= 0 || c.N <= 0 || c.Cout <= 0) return true;
    dim3 grid((unsigned)ceil_div(OHW, kThreads), (unsigned)c.Cout,
              (unsigned)c.N);
    k_conv_f32<<<grid, kThreads, 0, st>>>(x, w, y, c);
    return check("k_conv_f32");
}

bool launch_gemm_f32(const float* A, const float* B, float* C, int64_t M,
                     int64_t N, int64_t K, hipStream_t st) {
    if (M <= 0 || N <= 0) return true;
    dim3 grid((unsigned)ceil_div(N, 16), (unsigned)ceil_div(M, 16));
    if (grid.y > 65535) {
        set_error("launch_gemm_f32", "M above 1048560");
        return false;
    }
    k_gemm_f32<<<grid, kThreads, 0, st>>>(A, B, C, M, N, K);
    return check("k_gemm_f32");
}

}  // namespace qa

// VALU convolution / GEMM kernels: the exact integer paths for operands that
// do not fit int8 after an offset (narrow: int16 products summed modulo
// 2^32; wide: int32 x int32 products summed in int64) and the float32 paths
// behind qa_conv_f32 / qa_gemm_f32.
#pragma once

#include "qa_igemm.h"

namespace qa {

struct ValuConv {
    const void* x;      // activations, NCHW
    int32_t x_code;     // 1 int8, 2 int16, 4 int32, 5 float32
    int64_t x_nstride;  // elements between images
    int64_t x_add;      // added to every activation (storage offset - zp)
    int32_t narrow16;   // 1: activations wrap to int16 before the product
    const void* w;      // weights OIHW (or [K][N] row-major for GEMM)
    int32_t w_code;     // 2 int16, 4 int32, 5 float32
    int32_t N, C, H, W, Cout, KH, KW, SH, SW, PH, PW, DH, DW, G, OH, OW;
    int32_t wide;       // 1: int64 accumulator, 0: modulo-2^32 accumulator
};

// Integer conv; `e` supplies the output and epilogue (mode EPI_RAW32 /
// EPI_RAW64 / EPI_QUANT with e.corr / e.boff unused).
bool launch_conv_valu(const ValuConv& c, const IgemmArgs& e, int mode,
                      hipStream_t st);

// y[M,N] = A[M,K] B[K,N] for int16/int32 operands (mode EPI_RAW32/RAW64).
bool launch_gemm_valu(const void* A, int a_code, const void* B, int b_code,
                      void* C, int64_t M, int64_t N, int64_t K, bool wide,
                      hipStream_t st);

bool launch_conv_f32(const float* x, const float* w, float* y,
                     const ValuConv& c, hipStream_t st);
bool launch_gemm_f32(const float* A, const float* B, float* C, int64_t M,
                     int64_t N, int64_t K, hipStream_t st);

}  // namespace qa

// VALU GEMM / float kernels used by the reference ABI entries.
#pragma once

#include "qa_conv.h"

namespace qa {

// C[M,N] = A[M,K] B[K,N] for int16/int32 operands (codes 2/4): products
// summed modulo 2^32 (int32 C) or in int64 (wide). With a gate, the kernel
// does nothing unless *gate == gate_on when it runs.
bool launch_gemm_valu(const void* A, int a_code, const void* B, int b_code,
                      void* C, int64_t M, int64_t N, int64_t K, bool wide,
                      hipStream_t st, const int32_t* gate = nullptr,
                      int32_t gate_on = 0);

// float32 NCHW conv (geometry from `a`; x/y/w pointers given separately).
bool launch_conv_f32(const float* x, const float* w, float* y,
                     const ConvArgs& a, hipStream_t st);
bool launch_gemm_f32(const float* A, const float* B, float* C, int64_t M,
                     int64_t N, int64_t K, hipStream_t st);

}  // namespace qa

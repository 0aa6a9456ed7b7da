// Implicit-GEMM convolution / GEMM on CDNA4 int8 MFMA.
//
// GEMM view: rows = output pixels (n, oy, ox) of one group, batch folded in
// (M = N*OH*OW); columns = output channels of the group; K = taps x input
// channels. K is laid out in "k-groups" of 16 bytes: k-group kg covers tap
// kg / CB and channels [16*(kg % CB), +16) of the group, CB = ceil(Cg/16).
// One MFMA (v_mfma_i32_16x16x64_i8) consumes 4 k-groups; lane l supplies row
// (l & 15) and k-group (l >> 4) of its 16x64 A fragment, and column (l & 15)
// and k-group (l >> 4) of its 64x16 B fragment. A and B use the same
// (lane, byte) -> k assignment, so the dot product is correct whatever order
// the hardware sums the 64 products in. Result lane l holds rows
// 4*(l >> 4) + i, i = 0..3, of column (l & 15).
//
// Operands are int8 after an offset: x = x_s + a_off (per tensor),
// w = w_s + b_off[co] (per output channel), so that
//   sum_k x w = MFMA(x_s, w_s) + a_off * colsum(w_s)[co]
//             + b_off[co] * (rowsum(x_s)[p] + K * a_off).
// Image padding is x = 0, i.e. x_s = -a_off ("pad value"); K-padding has
// w_s = 0 and is excluded from the row sums.
#pragma once

#include "qa_common.h"

namespace qa {

enum EpiMode {
    EPI_RAW32 = 0,  // int32 accumulator (wraps modulo 2^32), ABI narrow path
    EPI_RAW64 = 1,  // exact int64 accumulator, ABI wide path
    EPI_QUANT = 2,  // requantize (+LUT) (+residual add) -> int8/int16 storage
};

struct IgemmArgs {
    // ---- A operand (activations, int8 "x_s") ----
    const int8_t* x;
    int64_t x_nstride;  // elements between images (>= C*H*W)
    int64_t x_cstride;  // elements between channels (H*W for NCHW)
    int32_t rowmajor;   // 1: A is [M][lda] row-major (GEMM), 0: NCHW conv
    int64_t lda;
    int32_t C, H, W, Cg, G, Cog, KH, KW, SH, SW, PH, PW, DH, DW, OH, OW;
    int32_t CB, KG, KGp;  // channel blocks, k-groups, k-groups padded to 4
    int64_t M;            // rows per group = N*OH*OW
    int32_t pad_value;    // x_s of the (zero-point) padding
    int32_t Kreal;        // Cg*KH*KW
    // ---- B operand (packed weights) ----
    const int8_t* wp;     // [G][Cog_pad][KGp*16]
    int64_t wp_gstride;   // bytes between groups
    int64_t wp_rstride;   // bytes between rows (= KGp*16)
    // ---- corrections (indexed by global output channel) ----
    const int64_t* corr;  // a_off*colsum + K*a_off*b_off (NULL: 0)
    const int32_t* boff;  // b_off (only when rowsum is enabled)
    const int64_t* pre;   // bias added to the wrapped int32 accumulator
                          // before requantization (EPI_QUANT; NULL: 0)
    // ---- epilogue ----
    int32_t Cout;         // total output channels
    void* y;
    int64_t y_nstride;    // elements between output images
    int64_t y_choff;      // channel offset inside the output buffer
    int32_t out_code;     // storage of y for EPI_QUANT: 1 int8, 2 int16
    int64_t out_so;
    const int64_t* mult;
    const int64_t* shift;
    int64_t zp, qmin, qmax;
    const int32_t* lut;   // optional table applied after the clamp
    int64_t lut_off, lut_len;
    const void* res;      // optional residual add operand (same layout as y)
    int64_t res_nstride, res_choff, res_so;
    int64_t za, ma, sa, zb, mb, sb, add_sign, add_zp, add_qmin, add_qmax;
    int32_t res_first;    // 1: residual is the first Add operand
};

// Launches the MFMA kernel for `a` with epilogue `mode`; `rowsum` enables the
// per-row sums needed when any b_off != 0. Returns false on launch failure.
bool launch_igemm(const IgemmArgs& a, int mode, bool rowsum,
                  hipStream_t st);

}  // namespace qa

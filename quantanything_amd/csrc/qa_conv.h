// Convolution / GEMM on gfx950: shared argument block and epilogue.
//
// Activations are channels-last ("NHWC"): element (n, c, iy, ix) of the
// input lives at x + n*x_sn + (iy*W + ix)*x_sp + c*x_sc, with x_sc == 1 on
// the int8 MFMA path, so 16 consecutive input channels of one pixel are one
// aligned 16-byte load. A GEMM is the 1x1 case with H = W = 1 (row m is
// "image" m, x_sn = lda). Outputs use general strides: element (n, co, pix)
// (pix = oy*OW + ox) at y + n*y_sn + co*y_sc + pix*y_sp, so the same kernel
// writes NHWC tensors, NCHW ABI results or row-major GEMM results.
//
// int8 MFMA path (v_mfma_i32_16x16x64_i8): the GEMM is
//   C[Cout x P] = W[Cout x K] * X[K x P],  P = N*OH*OW pixels (batch folded)
// with K in 16-byte "k-groups": k-group kg covers tap kg / CB and input
// channels [16*(kg % CB), +16), CB = ceil(Cg/16) (layout 0). For inputs of at
// most 4 channels stored 4 bytes per pixel (layout 1, the 3-channel stem),
// k-group ky covers kernel row ky: bytes [4*kx + c] for kx < KW. Lane l
// supplies row / column (l & 15) and k-group (l >> 4) of its fragments; the
// accumulator lane l holds output channels 4*(l >> 4) + i, i = 0..3, of pixel
// (l & 15). Operands are int8 after offsets: x = x_s + a_off,
// w = w_s + b_off[co]:
//   sum x w = MFMA(w_s, x_s) + a_off*colsum(w_s)[co]
//           + b_off[co]*(pixsum(x_s)[p] + K*a_off)
// corr[co] holds the first and last terms; image padding is x = 0, so it is
// filled with x_s = -a_off ("pad_value"); K-padding has zero weights and is
// left out of pixsum.
#pragma once

#include "qa_common.h"

namespace qa {

constexpr int32_t TILE_VALID = 1 << 16;

enum EpiMode {
    EPI_RAW32 = 0,  // int32 accumulator (wraps modulo 2^32): ABI narrow path
    EPI_RAW64 = 1,  // exact int64 accumulator: ABI wide path
    EPI_QUANT = 2,  // requantize (+LUT) (+residual Add) -> int8/int16
};

struct ConvArgs {
    // ---- input ----
    const void* x;
    int32_t x_code;                 // 1 int8, 2 int16, 4 int32
    int64_t x_sn, x_sc, x_sp;       // strides (elements)
    int64_t x_add;                  // x_centred = stored + x_add
    int32_t narrow16;               // wrap activations to int16 (ABI narrow)
    // ---- geometry ----
    int32_t N, H, W, Cg, G, Cog, KH, KW, SH, SW, PH, PW, DH, DW, OH, OW;
    int32_t Cout;
    int64_t M;                      // N*OH*OW
    // ---- packed int8 weights (MFMA path) ----
    const int8_t* wp;
    const int8_t* wfrag;            // the same in fragment order, or NULL
    int32_t layout;                 // 0 tap-major 16-channel groups, 1 stem
    int32_t CB, KG, KGp, Kreal;
    uint64_t mg_cb, mg_kw;          // ceil(2^32 / CB), ceil(2^32 / KW)
    int32_t st_dn, st_doy, st_dox;  // a wave's pixel stride as (n, oy, ox)
    int32_t fastio;                 // y (res, y2): dense channels-last (the
                                    // int8 path: in 4-byte aligned 4-channel
                                    // words)
    int64_t y_pst, res_pst, y2_pst; // their pixel strides when fastio
    int32_t tile_hint;              // 0, or TILE_VALID | wm | split << 8 |
                                    // lds << 9 (MFMA tile choice)
    int64_t wp_gstride, wp_rstride; // bytes
    int32_t xcd_yfast;              // XCD order: channel blocks fastest
    int32_t pad_value;
    int32_t rowsum;                 // some b_off != 0
    const void* plan;               // table epilogue plan (int8 output)
    // ---- plain weights (VALU path): OIHW ----
    const void* w;
    int32_t w_code;                 // 2 int16, 4 int32
    int32_t wide;                   // int64 accumulation
    // ---- FP64 MFMA path weights (qa_pack_weights_f64) ----
    const void* wf;                 // [G][wf_rows][KH*KW][CK] int16 / int32
    int32_t CK, wf_rows;            // Cg rounded up to 32, Cog to 64
    int32_t wf_bytes;               // element size, 2 or 4
    // ---- the same weights split into two int8 planes (byte-split path,
    // qa_pack_weights_i16s): high bytes, then low bytes - 128, each in the
    // layout-0 form (CB, KG, KGp, wp_rstride, wp_gstride, mg_cb, mg_kw)
    const int8_t* ws;               // NULL: FP64 path only
    const int64_t* ws_k;            // per channel: (128 + x_add) * sum w
    // ---- per output channel ----
    const int64_t* corr;
    const int32_t* boff;
    const int64_t* pre;             // bias added after the int32 wrap
    const int64_t* mult;
    const int64_t* shift;
    // ---- epilogue ----
    int32_t mode;
    int64_t zp, qmin, qmax;
    const int32_t* lut;
    int64_t lut_off, lut_len;
    const void* res;
    int64_t res_sn, res_sc, res_sp, res_so;
    int32_t res_first;
    int64_t za, ma, sa, zb, mb, sb, add_sign, add_zp, add_qmin, add_qmax;
    void* y;
    int32_t y_code;                 // 1 int8, 2 int16, 4 int32, 8 int64
    int64_t y_sn, y_sc, y_sp, y_so;
    void* y2;                       // optional rescaled copy (same code)
    int64_t y2_sn, y2_sc, y2_sp;
    int64_t r2_zp_in, r2_m, r2_s, r2_zp_out, r2_qmin, r2_qmax;
    // ---- device-side path choice (NULL: always run) ----
    const int32_t* gate;            // the kernel runs only if *gate == gate_on
    int32_t gate_on;
};

// Table epilogue plan for int8 outputs (device buffer written by
// qa_plan_epilogue_i8). With per-channel constants m (int32), t (1..62) and
// c = pre_bias*m + 2^(t-1), the requantized value of the int32 accumulator w
// is q0 = (w*m + c) >> t, exact in int64 and within int32 (the planner checks
// both). Everything after it is a function of i = clip(q0, A, B) - A, at most
// 256 values, or, with a residual Add, of the stored residual byte u:
//   no residual: e = E[i]
//   residual:    e = E[clip(TC[i] + TR[u], 0, SH)]
// e holds the stored output byte in bits 0..7 and the stored byte of the
// rescaled second output in bits 8..15.
constexpr int PLAN_E = 64;             // int32 E[256]
constexpr int PLAN_TC = PLAN_E + 1024;  // int32 TC[256]
constexpr int PLAN_TR = PLAN_TC + 1024; // int32 TR[256]
constexpr int PLAN_CH = PLAN_TR + 1024; // int32x4 {m, t, c_lo, c_hi} per channel
// header (int32): [0] A, [1] B, [2] SH, [3] flags, [4] with PLAN_IDENT
// (no activation table, residual or second output: E[i] is the byte of
// A + i + D) the offset D = zp - y_so
constexpr int PLAN_RES = 1, PLAN_Y2 = 2, PLAN_IDENT = 4;

// The residual Add of a quantized value q and the residual's value res_q.
__device__ __forceinline__ int64_t quant_add(const ConvArgs& a, int64_t q,
                                             int64_t res_q) {
    const int64_t first = a.res_first ? res_q : q;
    const int64_t second = a.res_first ? q : res_q;
    const qa_i128 t = qa_mbqm_fast(first - a.za, a.ma, a.sa) +
                      (qa_i128)a.add_sign *
                          qa_mbqm_fast(second - a.zb, a.mb, a.sb) +
                      a.add_zp;
    return qa_clip128(t, a.add_qmin, a.add_qmax);
}

// The table index of a requantized value.
__device__ __forceinline__ int64_t lut_index(const ConvArgs& a, int64_t q) {
    const int64_t idx = q - a.lut_off;
    return idx < 0 ? 0 : (idx >= a.lut_len ? a.lut_len - 1 : idx);
}

// Requantize, table and residual Add of one accumulator (mode EPI_QUANT):
// returns the quantized value q (before the storage offset).
__device__ __forceinline__ int64_t quant_one(const ConvArgs& a, int64_t v,
                                             int64_t m, int64_t s,
                                             int64_t res_q) {
    int64_t q = qa_clip128(qa_mbqm_fast(v, m, s) + a.zp, a.qmin, a.qmax);
    if (a.lut) q = a.lut[lut_index(a, q)];
    if (a.res) q = quant_add(a, q, res_q);
    return q;
}

__device__ __forceinline__ int64_t rescale2(const ConvArgs& a, int64_t q) {
    return qa_clip128(qa_mbqm_fast(q - a.r2_zp_in, a.r2_m, a.r2_s) +
                          a.r2_zp_out,
                      a.r2_qmin, a.r2_qmax);
}

__device__ __forceinline__ int64_t load_any(const void* p, int code,
                                            int64_t i) {
    switch (code) {
        case 1: return ((const int8_t*)p)[i];
        case 2: return ((const int16_t*)p)[i];
        case 4: return ((const int32_t*)p)[i];
        default: return ((const int64_t*)p)[i];
    }
}

__device__ __forceinline__ void store_any(void* p, int code, int64_t i,
                                          int64_t v) {
    switch (code) {
        case 1: ((int8_t*)p)[i] = (int8_t)v; break;
        case 2: ((int16_t*)p)[i] = (int16_t)v; break;
        case 4: ((int32_t*)p)[i] = (int32_t)v; break;
        default: ((int64_t*)p)[i] = v; break;
    }
}

// Launchers; false on launch failure (recorded with set_error).
bool launch_conv_mfma(const ConvArgs& a, hipStream_t st);
// The int8 MFMA variants with weights staged in LDS / read from L2 (wm: 16
// channel groups per tile, 1/2/4/8; split: the 4 waves split K).
bool mfma_launch_lds(const ConvArgs& b, int wm, bool split, int epi,
                     hipStream_t st);
bool mfma_launch_l2(const ConvArgs& b, int wm, bool split, int epi,
                    hipStream_t st);
bool launch_conv_valu(const ConvArgs& a, hipStream_t st);
// Large GEMM descriptors (H = W = 1, K a multiple of 64) with the int8 table
// epilogue on 128 x 128 blocks (qa_gemm_big.hip); `epi` as chosen by
// launch_conv_mfma.
bool gemm_big_applies(const ConvArgs& b, int epi);
// stages 3 or 4: the K loop through that many LDS stages filled by direct
// loads; otherwise the register-staged two-buffer loop
bool launch_gemm_big(const ConvArgs& b, hipStream_t st, int stages = 0);
// Narrow GEMMs / pointwise convolutions (Cout 16, 32, 64 or blocks of 64,
// K a multiple of 64 up to 576, or 1280 with fragment-order weights, table
// plan without residual; a rescaled copy allowed): a 16 x 16 block a wave
// with its weight fragments in VGPRs (qa_gemm_narrow.hip).
bool gemm_narrow_applies(const ConvArgs& b, int epi);
// rtl: row tiles each wave computes (1..4) with the same weights
bool launch_gemm_narrow(const ConvArgs& b, hipStream_t st, int rtl);
// int8 convolutions over bands of output rows with the input band and the
// weights in LDS (qa_conv_band.hip); wm = 16-channel groups per work-group.
bool conv_band_applies(const ConvArgs& b, int epi, int wm);
bool launch_conv_band(const ConvArgs& b, int wm, hipStream_t st);
// Convolution with the work-group's weights held in VGPRs and the input
// bands in double-buffered LDS (qa_conv_wr.hip); wm = 16-channel groups per
// work-group (K <= 36 / wm K-steps of 64 bytes).
bool conv_wr_applies(const ConvArgs& b, int epi, int wm);
bool launch_conv_wr(const ConvArgs& b, int wm, hipStream_t st);
// Launch form of a descriptor's arguments (fastio, pixel strides, magic
// divisors); returns the epilogue variant (qa_conv_mfma.hip).
int fast_io_args(const ConvArgs& a, ConvArgs& b, int epi);
// Two chained 3x3 stride-1 convolutions (C -> C, C in {16, 32, 64, 128}) in one
// launch, the intermediate kept in LDS (qa_conv_pair.hip); arguments in
// launch form.
bool conv_pair_applies(const ConvArgs& b1, int epi1, const ConvArgs& b2,
                       int epi2);
bool conv_pair_tail_applies(const ConvArgs& b1, int epi1, const ConvArgs& b2,
                            int epi2, const ConvArgs& b3, int epi3);
// b3: the C2f block's cv2 run in the same launch (conv_pair_tail_applies)
bool launch_conv_pair(const ConvArgs& b1, const ConvArgs& b2, hipStream_t st,
                      const ConvArgs* b3 = nullptr);
// A convolution (weights-in-registers kernel, Cout 16, 32 or 64) whose
// output feeds only a 1x1 convolution of the same width: both in one
// launch, the intermediate kept per wave in LDS (qa_conv_wr.hip).
bool conv_chain_applies(const ConvArgs& b1, int epi1, const ConvArgs& b2,
                        int epi2);
bool launch_conv_chain(const ConvArgs& b1, const ConvArgs& b2, hipStream_t st);
// The same pair as two GEMMs over the same rows (qa_narrow_chain.hip): b1
// a 1x1 or k x k convolution of a multiple of 64 input channels and up to
// 256 output channels, b2 a 1x1 convolution of up to 256 reading its
// output, both with fragment-order weights; rtl row tiles of 16 a
// work-group.
bool narrow_chain_applies(const ConvArgs& b1, const ConvArgs& b2);
bool launch_narrow_chain(const ConvArgs& b1, const ConvArgs& b2, int rtl,
                         hipStream_t st);
// 16-bit operands on the FP64 matrix cores (qa_conv_f64.hip), exact.
bool launch_conv_f64(const ConvArgs& a, hipStream_t st);

// Input quantization fused into a layout-1 convolution (qa_conv_qin.hip):
// float32 NCHW graph input, quantized exactly like qa_d_quantize_nhwc.
struct QinArgs {
    const float* xf;
    double scale, inv;
    int64_t zp, qmin, qmax, so;
};
bool launch_conv_qin(const ConvArgs& a, const QinArgs& q, hipStream_t st);

// A convolution consumed only by a global average pool (qa_conv_pool.hip):
// pooled int8 output q = clip(mbqm(sum of stored bytes + base, mult, shift)
// + zp) - out_so per image and channel, base = HW * (so - zp_in).
struct PoolArgs {
    int64_t base, mult, shift, zp, qmin, qmax, out_so;
    int8_t* out;
    int64_t out_sn;
};
bool launch_conv_pool(const ConvArgs& a, const PoolArgs& p, hipStream_t st);
// Two 1x1 convolutions, the second's output pooled, in one launch
// (qa_conv_pw_pool.hip); arguments in launch form, b2 reading b1's output.
bool conv_pw_pool_applies(const ConvArgs& b1, const ConvArgs& b2);
// b1.wfrag / b2.wfrag: the weights in fragment order (required)
bool launch_conv_pw_pool(const ConvArgs& b1, const ConvArgs& b2,
                         const PoolArgs& p, hipStream_t st);
// Packed layout-0 weight rows (rows x kgp 16-byte chunks) in fragment
// order: the 1 KB MFMA fragment of each 16-row tile and 64-byte K-step
// contiguous, lane l's 16 bytes at 16 l (fragments_bytes bytes).
int64_t fragments_bytes(int64_t rows, int64_t kgp);
bool launch_pack_fragments(const int8_t* src, int64_t rows, int64_t kgp,
                           int8_t* dst, hipStream_t st);

}  // namespace qa

/*
 * qa_hip.h -- C ABI of libqa_hip.so, the MI355X (gfx950) integer inference
 * library for QuantAnything's quantized Conv / Gemm / MatMul path.
 *
 * Part 1 replaces, symbol for symbol, the C ABI that QuantAnything's loader
 * binds through ctypes (reference: quantization/native.py:104-128, selected
 * with QA_LIB at native.py:137). Signatures, argument meaning and results are
 * those of quantization/kernels/qa_kernels.cpp; results are bit-identical.
 * These entries take host (or device) pointers, run on the GPU and return
 * when the output is written. Like the reference they return void and are
 * re-entrant: each calling thread has its own stream and scratch buffers.
 * A failure (a geometry the reference would divide by zero on, a HIP error)
 * never aborts the process: the call fills its output with zeros, records
 * the message for qa_last_error() and prints it to stderr. Every call starts
 * afresh, so a later call computes its full result whether or not the caller
 * ever reads or clears the error (the reference's loader never does). Shapes
 * the reference accepts are all computed (no limit on N, Cout or M beyond
 * the 2^31 element bound of a dimension).
 *
 * Part 2 is additional surface the reference's loader ignores: backend
 * identification and errors, weight packing, and device-pointer entries used
 * by the device-resident executor (asynchronous on a caller stream).
 */
#ifndef QA_HIP_H
#define QA_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ===================== Part 1: the reference ABI (17 symbols) ========== */

/* qa_kernels.cpp:233-249. The GPU library reports the compute-unit count of
 * the current device, ignores set_num_threads and has no OpenMP. */
int qa_num_threads(void);
void qa_set_num_threads(int n);
int qa_has_openmp(void);

/* C[M,N] = A[M,K] B[K,N], row-major (qa_kernels.cpp:252-263). The narrow
 * integer form sums int16 products modulo 2^32 (an int32 accumulator), the
 * wide form int32 products in int64. */
void qa_gemm_f32(int64_t M, int64_t N, int64_t K, const float* A,
                 const float* B, float* C);
void qa_gemm_i16_i32(int64_t M, int64_t N, int64_t K, const int16_t* A,
                     const int16_t* B, int32_t* C);
void qa_gemm_i32_i64(int64_t M, int64_t N, int64_t K, const int32_t* A,
                     const int32_t* B, int64_t* C);

/* y[N,Cout,OH,OW] = conv(x[N,C,H,W], w[Cout,C/G,KH,KW]) with strides,
 * top/left pads, dilations and groups; taps outside the image contribute 0
 * (qa_kernels.cpp:273-284). The narrow form wraps activations to int16
 * before the product, like the reference's int16 im2col buffer. */
void qa_conv_f32(const float* x, const float* w, float* y, int64_t N,
                 int64_t C, int64_t H, int64_t W, int64_t Cout, int64_t KH,
                 int64_t KW, int64_t SH, int64_t SW, int64_t PH, int64_t PW,
                 int64_t DH, int64_t DW, int64_t G, int64_t OH, int64_t OW);
void qa_conv_i32_i16_i32(const int32_t* x, const int16_t* w, int32_t* y,
                         int64_t N, int64_t C, int64_t H, int64_t W,
                         int64_t Cout, int64_t KH, int64_t KW, int64_t SH,
                         int64_t SW, int64_t PH, int64_t PW, int64_t DH,
                         int64_t DW, int64_t G, int64_t OH, int64_t OW);
void qa_conv_i32_i32_i64(const int32_t* x, const int32_t* w, int64_t* y,
                         int64_t N, int64_t C, int64_t H, int64_t W,
                         int64_t Cout, int64_t KH, int64_t KW, int64_t SH,
                         int64_t SW, int64_t PH, int64_t PW, int64_t DH,
                         int64_t DW, int64_t G, int64_t OH, int64_t OW);

/* out[o,c,i] = clip(mbqm(acc + pre[c], mult[c], shift[c]) + post[c] + zp)
 * over the [outer, C, inner] view; pre/post may be NULL
 * (qa_kernels.cpp:287-302). mbqm(x,m,s) = round(x*m*2^-(31+s)) with a
 * 128-bit product, rounding half up. */
void qa_requantize_i32(const int32_t* acc, int32_t* out, int64_t outer,
                       int64_t C, int64_t inner, const int64_t* mult,
                       const int64_t* shift, const int64_t* pre_bias,
                       const int64_t* post_bias, int64_t zp, int64_t qmin,
                       int64_t qmax);
void qa_requantize_i64(const int64_t* acc, int32_t* out, int64_t outer,
                       int64_t C, int64_t inner, const int64_t* mult,
                       const int64_t* shift, const int64_t* pre_bias,
                       const int64_t* post_bias, int64_t zp, int64_t qmin,
                       int64_t qmax);

/* Element-wise integer kernels (qa_kernels.cpp:307-358). */
void qa_rescale(const int32_t* x, int32_t* out, int64_t n, int64_t zp_in,
                int64_t m, int64_t s, int64_t zp_out, int64_t qmin,
                int64_t qmax);
void qa_add(const int32_t* a, const int32_t* b, int32_t* out, int64_t n,
            int64_t za, int64_t ma, int64_t sa, int64_t zb, int64_t mb,
            int64_t sb, int64_t sign, int64_t zp_out, int64_t qmin,
            int64_t qmax);
void qa_mul(const int32_t* a, const int32_t* b, int32_t* out, int64_t n,
            int64_t za, int64_t zb, int64_t m, int64_t s, int64_t zp_out,
            int64_t qmin, int64_t qmax);
void qa_lut(const int32_t* x, int32_t* out, int64_t n, int64_t offset,
            const int32_t* lut, int64_t lut_len);

/* Per-tensor float <-> integer (qa_kernels.cpp:363-386): q = clip(
 * nearbyint(double(x)/scale) + zp), x = float(double(q - zp) * scale). */
void qa_quantize_f32(const float* x, int32_t* q, int64_t n, double scale,
                     int64_t zp, int64_t qmin, int64_t qmax);
void qa_dequantize_f32(const int32_t* q, float* x, int64_t n, double scale,
                       int64_t zp);

/* ===================== Part 2: additional surface ====================== */
/* No counterpart in the reference: its loader ignores these symbols. */

const char* qa_backend(void);       /* "hip-gfx950" */
const char* qa_last_error(void);    /* most recent failure of this thread
                                       since qa_clear_error, or NULL */
void qa_clear_error(void);
int qa_device_count(void);
int qa_device_arch(char* buf, int64_t len);
void* qa_stream(void);              /* the calling thread's library stream
                                       (hipStream_t) on the current device */
int qa_synchronize(void);

/* Storage codes of device tensors: 1 int8, 2 int16, 4 int32, 8 int64.
 * A quantized value q is stored as q - so (so: storage offset). */

/* Packs centred OIHW weights (w - w_zp, int32) for the int8 MFMA path.
 * Per output channel an offset b_off makes every value int8; K is laid out
 * in 16-byte groups padded to a multiple of 64 bytes, rows padded to a
 * multiple of 128 per group. layout 0: group kg = tap kg/CB, input channels
 * [16*(kg%CB), +16), CB = ceil(Cg/16). layout 1 (Cg <= 4, KW <= 16;
 * inputs stored 4 bytes per pixel): CB = ceil(KW/4) groups per kernel row,
 * group kg = kernel row kg / CB, byte 4*(kx - 4*(kg % CB)) + c. Writes wp
 * (qa_pack_weights_i8_size bytes), corr[c] = a_off*colsum_c +
 * K*a_off*b_off[c] and boff. Returns 0 on success, 1 when a channel spans
 * more than 255 values (use the VALU path), -1 on bad arguments;
 * *needs_rowsum is set when some b_off is non-zero. */
int64_t qa_pack_weights_i8_size(int64_t Cout, int64_t Cg, int64_t KH,
                                int64_t KW, int64_t G, int64_t layout,
                                int64_t* kgp, int64_t* rows_per_group);
int qa_pack_weights_i8(const int32_t* w, int64_t Cout, int64_t Cg, int64_t KH,
                       int64_t KW, int64_t G, int64_t a_off, int64_t layout,
                       int8_t* wp, int64_t* corr, int32_t* boff,
                       int32_t* needs_rowsum);

/* Packs centred OIHW weights (w - w_zp, int32) for the FP64 matrix-core
 * path of 16-bit models: elements of elem_bytes (2: int16, 4: int32) at
 * wp[g][r][tap][c], rows r padded to a multiple of 64 per group and input
 * channels c padded to a multiple of 32 (*ck), zero-filled; the kernel
 * converts them to double. Returns 0 on success, 1 when a value does not fit
 * the element (int16), |w| >= 2^17 or KH*KW*ck >= 2^19 (the sums would no
 * longer be exact in double: use the VALU path), -1 on bad arguments. The
 * size function returns the number of elements of wp. */
int64_t qa_pack_weights_f64_size(int64_t Cout, int64_t Cg, int64_t KH,
                                 int64_t KW, int64_t G, int64_t* ck,
                                 int64_t* rows_per_group);
int qa_pack_weights_f64(const int32_t* w, int64_t Cout, int64_t Cg,
                        int64_t KH, int64_t KW, int64_t G, int64_t elem_bytes,
                        void* wp);

/* Splits centred OIHW weights (w - w_zp, each in int16) for the byte-split
 * path of 16-bit models (int8 matrix cores): plane 0 the high bytes w >> 8,
 * plane 1 the low bytes (w & 255) - 128, each in the layout-0 form of
 * qa_pack_weights_i8 (qa_pack_weights_i8_size with layout 0 gives one
 * plane's bytes, kgp and rows; wp holds both planes, plane 1 right after
 * plane 0; positions without a weight hold w = 0), and wsum[co] the sum of
 * output channel co's weights. No counterpart in the reference: its 16-bit
 * convolution is qa_conv_i32_i32_i64 (qa_kernels.cpp:281-284). Returns 0,
 * 1 when a weight is outside int16, -1 on bad arguments. */
int qa_pack_weights_i16s(const int32_t* w, int64_t Cout, int64_t Cg,
                         int64_t KH, int64_t KW, int64_t G, int8_t* wp,
                         int64_t* wsum);

/* Fused integer convolution / GEMM on device tensors:
 *   acc = sum (x_stored + x_add) * w         (exact)
 *   q   = clip(mbqm(acc + pre_bias[c], mult[c], shift[c]) + zp)
 *   q   = lut[clip(q - lut_offset)]                        (if lut)
 *   q   = clip(mbqm(r - za) + sign*mbqm(q - zb) + add_zp)    (if res; the
 *         residual r is the first Add operand when res_first)
 *   y   = q - y_so;  y2 = clip(mbqm(q - r2_zp_in, r2_m, r2_s) + r2_zp_out)
 *         - y_so  (if y2: a rescaled copy, e.g. into a Concat buffer)
 * Input element (n, c, iy, ix) at x + n*x_sn + c*x_sc + (iy*W+ix)*x_sp;
 * output / residual / y2 element (n, c, pix) at p + n*sn + c*sc + pix*sp.
 * w_code 1: weights from qa_pack_weights_i8 (int8 MFMA; needs int8 input
 * with x_sc == 1 and 16-byte aligned channel groups, 4-byte for layout 1);
 * w_code 2/4: OIHW int16/int32 weights (VALU; int64 accumulation when wide);
 * w_code 8: weights from qa_pack_weights_f64 (w_layout = their element
 * bytes, w_kgp = ck, w_rows = rows per group; FP64 matrix cores, exact;
 * needs int16 input with x_sc == 1 and |x_add| <= 2^16; the sum wraps to
 * int32 unless wide).
 * A GEMM is the case H = W = KH = KW = 1 with row m as image m. */
typedef struct qa_conv_desc {
    const void* x;
    int64_t x_code, x_sn, x_sc, x_sp, x_add;
    int64_t N, C, H, W, Cout, KH, KW, SH, SW, PH, PW, DH, DW, G, OH, OW;
    const void* w;
    int64_t w_code, w_layout, w_kgp, w_rows, wide, needs_rowsum;
    const void* epi_plan;  /* device copy of a qa_plan_epilogue_i8 plan for
                              exactly these parameters, or NULL (MFMA path;
                              the 128-bit epilogue then runs) */
    const int64_t* corr;
    const int32_t* boff;
    const int64_t* pre_bias;
    const int64_t* mult;
    const int64_t* shift;
    int64_t zp, qmin, qmax;
    const int32_t* lut;
    int64_t lut_offset, lut_len;
    const void* res;
    int64_t res_sn, res_sc, res_sp, res_so, res_first;
    int64_t za, ma, sa, zb, mb, sb, add_sign, add_zp, add_qmin, add_qmax;
    void* y;
    int64_t y_code, y_sn, y_sc, y_sp, y_so;
    void* y2;
    int64_t y2_sn, y2_sc, y2_sp, r2_zp_in, r2_m, r2_s, r2_zp_out, r2_qmin,
        r2_qmax;
    int64_t tile;  /* 0: the library picks the MFMA tiling; otherwise
                      0x10000 | wm | split << 8 | lds << 9 with wm = 16-channel
                      groups per tile (1, 2, 4, 8), split = the 4 waves of a
                      work-group split K, lds = weights staged in LDS (a
                      caller's measured choice; ignored where it does not
                      apply); 0x10400: GEMM descriptors (H = W = 1, C a
                      multiple of 64) on 128 x 128 blocks (0x10403 /
                      0x10404: K through 3 / 4 LDS stages filled by direct
                      loads); 0x10800 | wm
                      (wm 1, 2, 4): bands of output rows with the input band
                      and the weights in LDS (layout 0, one group, a table
                      plan); 0x11000 | wm | R << 4 (wm 1, 2, 4): the weights
                      held in registers (at most 36 / wm K-steps of 64
                      bytes), bands of R output rows (R 0: the library's
                      choice) in LDS (layout 0, one group, a table plan,
                      int8 weights without a zero point); 0x12000 |
                      (T - 1) << 4 (T 1..4): 1x1 stride-1 convolutions and
                      GEMMs of 16, 32 or 64 output channels or a multiple
                      of 4 above 64 (in blocks of 64), C a multiple of 64
                      up to 576 (up to 1280 with Cout >= 64 and w_frag), a
                      table plan without residual (a rescaled copy
                      allowed): one 16 x 16 block a wave with its weight
                      fragments in registers, T row tiles of 16 a wave, the
                      activation rows staged in LDS (0x12001 is 0x12000).
                      FP64 path (w_code
                      8): 0x10000 | wm | tm << 4
                      | split << 8 with (wm, tm, split) one of (1,1,0),
                      (2,1,0), (1,4,0), (1,1,1), (2,1,1), (4,1,1); tm =
                      16-pixel tiles per wave; with wsplit, 0x11000 | wm |
                      tm << 4 ((wm, tm) in {1, 2, 4} x {1, 2}) runs the
                      byte-split form. Results do not depend on it. */
    const void* wsplit;        /* w_code 8 only, optional: the same weights
                                  from qa_pack_weights_i16s (both planes);
                                  the int16 input then runs on the int8
                                  matrix cores when it fits (C / G a
                                  multiple of 16, 16-byte aligned pixels,
                                  |x_add| <= 32767): x = 256 xh + xl + 128
                                  and w split alike, four int8 products and
                                  the pixel sums, exact in int64 */
    const int64_t* wsplit_k;   /* with wsplit: per output channel
                                  (128 + x_add) * wsum[co] */
    const void* w_frag;        /* w_code 1 only, optional: w in fragment
                                  order (qa_d_pack_fragments_i8 of w, w_rows,
                                  w_kgp); the narrow-GEMM kernel (tile
                                  0x12000 / 0x12001) then loads each weight
                                  fragment as one contiguous KB straight
                                  into registers, and qa_d_conv_pw_pool
                                  requires it. Results do not depend on it. */
} qa_conv_desc;

/* Host-side planner of the int8 table epilogue of qa_d_conv. From the
 * per-channel mult / shift / pre_bias and the clip, table, residual Add and
 * rescaled-copy parameters of a qa_conv_desc (host copies), writes a plan of
 * qa_epi_plan_bytes(cout) bytes; the caller copies it to the device and sets
 * epi_plan. Within it the requantization is one 32x32+64-bit multiply-add and
 * shift, and the table, residual Add and rescale are 256-entry lookups
 * computed here with the 128-bit arithmetic, so results equal the 128-bit
 * epilogue's. Returns 1 when planned, 0 when the parameters fall outside the
 * plan's exact range (|mult| < 2^31, 1 <= 31+shift <= 62, int64 headroom,
 * at most 256 output levels, residual terms below 2^28), -1 on bad
 * arguments. */
typedef struct qa_epi_params {
    int64_t cout;
    const int64_t* mult;
    const int64_t* shift;
    const int64_t* pre_bias;   /* NULL: 0 */
    int64_t zp, qmin, qmax;
    const int32_t* lut;        /* NULL: no table */
    int64_t lut_offset, lut_len;
    int64_t has_res, res_first, res_so;
    int64_t za, ma, sa, zb, mb, sb, add_sign, add_zp, add_qmin, add_qmax;
    int64_t has_y2, r2_zp_in, r2_m, r2_s, r2_zp_out, r2_qmin, r2_qmax;
    int64_t y_so;
} qa_epi_params;
int64_t qa_epi_plan_bytes(int64_t cout);
int qa_plan_epilogue_i8(const qa_epi_params* p, void* plan);

/* Float fallbacks on device tensors (the reference's dequantize -> float
 * operator -> quantize, quant_layers.py:195-205), and a strided copy. */

/* Element (i_0, .., i_{ndim-1}) of x at x + sum i_k * xs[k] goes to y +
 * sum i_k * ys[k] (ndim <= 6, element strides), as q = stored + x_so:
 * mode 0 unchanged, mode 1 q' = clip(mbqm(q - zp_in, m, s) + zp_out) (the
 * reference's rescale, qa_kernels.cpp:307-316), mode 2 the float fallback
 * q' = quantize((float)((q - in_zp) * in_scale), out_scale, zp_out) (e.g.
 * a Gather, float_ops.py:490-496); stored y = q' - y_so. Layout operators
 * that are not views (Transpose + Reshape) and Concat along any axis. */
typedef struct qa_nd_copy {
    const void* x;
    int64_t x_code, x_so;
    void* y;
    int64_t y_code, y_so;
    int64_t ndim, shape[6], xs[6], ys[6];
    int64_t mode, zp_in, m, s, zp_out, qmin, qmax;
    double in_scale;
    int64_t in_zp;
    double out_scale;
} qa_nd_copy;
int qa_d_copy_nd(const qa_nd_copy* d, void* stream);

/* Integer Pad with the zero point (the reference's ShapingQuantize on a
 * Pad node: float_ops.py:499-513 called with pad_value = input zero point,
 * quant_layers.py:642-650). Output element (i_0, .., i_{ndim-1}) of shape
 * `shape` (ndim <= 6) is x[i_k - lo_k] when every i_k - lo_k lies in
 * [0, xshape_k), else `fill` (the zero point as a stored value, zp - so);
 * element strides xs / ys; storage code 1, 2 or 4 for both. */
typedef struct qa_nd_pad {
    const void* x;
    int64_t code;
    void* y;
    int64_t ndim, shape[6], lo[6], xshape[6], xs[6], ys[6];
    int64_t fill;
} qa_nd_pad;
int qa_d_pad_nd(const qa_nd_pad* d, void* stream);

/* Integer MaxPool / GlobalMaxPool over stored values (float_ops.py:518-560
 * with pad_value = input qmin, quant_layers.py:642-650; GlobalMaxPool,
 * float_ops.py:586-589, is the window of the whole image). y[n, c, oy, ox]
 * = max over ky < KH, kx < KW of x[n, c, oy*SH - PT + ky*DH, ox*SW - PL +
 * kx*DW], a tap outside the image counting as `pad` (qmin - so). The caller
 * resolves auto_pad and ceil_mode into PT / PL and OH / OW. Element strides
 * of x and y per axis (n, c, h, w); storage code 1, 2 or 4 for both. */
typedef struct qa_maxpool_desc {
    const void* x;
    int64_t code;
    int64_t x_sn, x_sc, x_sh, x_sw;
    int64_t N, C, H, W, KH, KW, SH, SW, DH, DW, PT, PL, OH, OW;
    int64_t pad;
    void* y;
    int64_t y_sn, y_sc, y_sh, y_sw;
} qa_maxpool_desc;
int qa_d_maxpool(const qa_maxpool_desc* d, void* stream);

/* LayerNormalization over the last axis of [rows, cols] (row strides in
 * elements) as float_ops.py:336-347: x = (float)((q - in_zp) * in_scale),
 * float64 mean and variance, y = (x - mean) / sqrt(var + eps) * gamma
 * (+ beta), cast to float32, quantized with round-half-even. beta may be
 * NULL. x and y of one storage, int8 or int16 (codes 1 / 2). Results agree
 * with the reference within one quantization step (float64 summation
 * order). */
int qa_d_layernorm(const void* x, int x_code, int64_t x_rstride,
                   int64_t rows, int64_t cols, double in_scale, int64_t in_zp,
                   int64_t x_so, const float* gamma, const float* beta,
                   double eps, void* y, int y_code, int64_t y_rstride,
                   double out_scale, int64_t out_zp, int64_t qmin,
                   int64_t qmax, int64_t y_so, void* stream);

/* MatMul of two activations, the reference's float fallback
 * (float_ops.py:181-186): C[b0, b1, m, n] = quantize(sum_k A[b0, b1, m, k] *
 * B[b0, b1, k, n]) with A, B dequantized. B is passed transposed, as Bt[b0,
 * b1, n, k] at b + b0*b_s0 + b1*b_s1 + n*b_sn + k*b_sk; A at a + b0*a_s0
 * + b1*a_s1 + m*a_sm + k*a_sk. The exact integer
 * sum of (a - a_zp)(b - b_zp) is scaled once by a_scale * b_scale (float32
 * result), which agrees with the reference's float32 matmul within one
 * output quantization step. int8 or int16 storage (the same for A and B),
 * K < 2^17. a_sk / b_sk: the element strides along k (1 for the layouts
 * above; any value is accepted). */
typedef struct qa_matmul_desc {
    const void* a;
    int64_t a_code, a_so, a_zp;
    double a_scale;
    int64_t a_s0, a_s1, a_sm, a_sk;
    const void* b;
    int64_t b_code, b_so, b_zp;
    double b_scale;
    int64_t b_s0, b_s1, b_sn, b_sk;
    int64_t B0, B1, M, N, K;
    void* y;
    int64_t y_code, y_so, y_s0, y_s1, y_sm, y_sn;
    double out_scale;
    int64_t out_zp, qmin, qmax;
} qa_matmul_desc;
int qa_d_matmul_act(const qa_matmul_desc* d, void* stream);

/* Attention of one layer in one launch: S = MatMul(q, k^T) as
 * qa_d_matmul_act of `qk`, P = Softmax over S's rows as qa_d_softmax_lut
 * with `table` (qa_d_softmax_table of S's quantization and storage
 * offset), O = MatMul(P, v) as qa_d_matmul_act of `av`; S and P stay on
 * chip and are never written (qk.y and av.a are unused; qk.y_so / out_*
 * give S's storage offset and quantization, p_* and av.a_scale / a_zp /
 * a_so P's). The results equal those three launches bit for bit. No
 * counterpart in the reference, which runs the three operators one by one
 * (quant_layers.py:195-205, float_ops.py:181-186, :270-282). Conditions
 * (qa_attention_supported returns 1 when they hold): int8 operands and
 * output, operands stored at their zero points, S and O rows of at most
 * 256 columns, av.K == qk.N, av.M == qk.M, equal batch axes, the staged
 * operands within the LDS budget. */
typedef struct qa_attention_desc {
    qa_matmul_desc qk;
    const double* table;
    double p_scale;
    int64_t p_zp, p_qmin, p_qmax, p_so;
    qa_matmul_desc av;
} qa_attention_desc;
int qa_attention_supported(const qa_attention_desc* d);
int qa_d_attention(const qa_attention_desc* d, void* stream);

/* `stream` of every qa_d_* entry is the hipStream_t to launch on, used as
 * given (NULL: the null stream). The entries are asynchronous and return 0
 * on success, -1 on an error (see qa_last_error). */
int qa_d_conv(const qa_conv_desc* d, void* stream);

/* A convolution whose output only feeds a GlobalAveragePool, fused with
 * it: runs d as qa_d_conv would (int8 packed weights of layout 0, one
 * group, an epilogue plan, no residual or second output) but instead of
 * storing the output it pools it per image and channel,
 * q = clip(mbqm(sum_p (y_p - in_zp), mult, shift) + zp, qmin, qmax),
 * stored at out[n * out_sn + c] - out_so (int8); d->y is not written. The
 * reference runs the two layers separately (quant_layers.py:320-335, then
 * quant_layers.py:569-583); results are identical. d->tile: 0, or
 * 0x10000 | wm (64*wm output channels per work-group, wm 1 or 2). */
typedef struct qa_pool_params {
    int64_t in_zp;                        /* zero point of the conv output */
    int64_t mult, shift, zp, qmin, qmax;  /* the pool's requantization */
    void* out;
    int64_t out_sn, out_so;
} qa_pool_params;
int qa_d_conv_pool(const qa_conv_desc* d, const qa_pool_params* p,
                   void* stream);

/* Packed int8 weights (qa_pack_weights_i8, layout 0: rows of kgp 16-byte
 * K-groups, kgp a multiple of 4) rearranged in fragment order: the 1 KB
 * matrix-core fragment of each 16-row tile and 64-byte K-step stored
 * contiguously (chunk (j, s, l) at ((j * kgp / 4 + s) * 64 + l) * 16 is
 * K-group 4 s + l / 16 of row 16 j + l % 16; zero past the last row).
 * qa_fragments_i8_size gives the bytes (0 for invalid sizes);
 * qa_d_pack_fragments_i8 writes them from device memory to device memory.
 * No counterpart in the reference: the layout of qa_conv_desc.w_frag. */
int64_t qa_fragments_i8_size(int64_t rows, int64_t kgp);
int qa_d_pack_fragments_i8(const void* packed, int64_t rows, int64_t kgp,
                           void* out, void* stream);

/* qa_d_conv_pool with the convolution's producer in the same launch: d1
 * and d2 are int8 1x1 stride-1 convolutions (packed layout 0, one group,
 * table plans, no residual, rescaled copy or weight offsets), d2 reading
 * d1's output (d2->x == d1->y, d2->C == d1->Cout <= 256), images of at
 * most 64 pixels (d1->x dense channels-last, 16-byte aligned pixels), and
 * both with their weights in fragment order (d->w_frag). The pooled result
 * is what qa_d_conv(d1) then qa_d_conv_pool(d2, p) store; neither d1->y
 * nor d2->y is written. Returns -1, launching nothing, for any other pair.
 * The reference runs the three layers one after another
 * (quant_layers.py:320-335 twice, then quant_layers.py:569-583).
 * qa_conv_pw_pool_supported checks a pair without launching (1 or 0). */
int qa_conv_pw_pool_supported(const qa_conv_desc* d1, const qa_conv_desc* d2);
int qa_d_conv_pw_pool(const qa_conv_desc* d1, const qa_conv_desc* d2,
                      const qa_pool_params* p, void* stream);

/* Two chained convolutions in one launch (the bottleneck of a C2f block):
 * d1 and d2 are int8 3x3 stride-1 pad-1 convolutions C -> C (C = 16, 32,
 * 64 or 128; packed layout 0, one group, epilogue plans, dense channels-last
 * tensors), d1 without residual or rescaled copy, and d2 reads d1's output
 * (d2->x == d1->y). The result is what qa_d_conv(d1) then qa_d_conv(d2)
 * would store at d2->y (and d2->y2), with d2's residual Add; d1->y is not
 * written (the intermediate stays in LDS). Returns -1, launching nothing,
 * for any other pair. The reference runs the two convolutions and the Add
 * one after another (quant_layers.py:320-335 twice, quant_layers.py:493-
 * 513). qa_conv_pair_supported checks a pair without launching (1 or 0).
 * d2->tile: 0 (the library picks the band height), or 0x10000 | R for
 * bands of R output rows a work-group (ignored where they do not fit);
 * results do not depend on it. */
int qa_conv_pair_supported(const qa_conv_desc* d1, const qa_conv_desc* d2);
int qa_d_conv_pair(const qa_conv_desc* d1, const qa_conv_desc* d2,
                   void* stream);

/* qa_d_conv_pair (C = 16 or 32) with the C2f block's last 1x1
 * convolution d3 in the same launch: d3 reads the block's Concat, a dense
 * channels-last int8 tensor of at most 256 channels whose last C channels
 * are the pair's output or its rescaled copy (d2->y or d2->y2 == d3->x +
 * d3->C - C, the same pixel stride) and whose other channels earlier
 * launches have written; d3 has a table plan, no residual or rescaled copy
 * and at most 128 output channels (a multiple of 16). The results are what
 * qa_d_conv_pair then qa_d_conv(d3) store (d2->y and d2->y2 are still
 * written). Returns -1, launching nothing, for any
 * other triple; the reference runs the three convolutions one after another
 * (quant_layers.py:320-335 three times). qa_conv_pair_tail_supported
 * checks a triple without launching (1 or 0). */
int qa_conv_pair_tail_supported(const qa_conv_desc* d1,
                                const qa_conv_desc* d2,
                                const qa_conv_desc* d3);
int qa_d_conv_pair_tail(const qa_conv_desc* d1, const qa_conv_desc* d2,
                        const qa_conv_desc* d3, void* stream);

/* A convolution followed by a 1x1 convolution in one launch (the stride-2
 * conv feeding a C2f block's first 1x1 conv): d1 an int8 convolution of
 * C = 16, 32 or 64 output channels (packed layout 0, one group, a table
 * plan, no residual or rescaled copy, up to 9 K-steps of 64 bytes), d2 an
 * int8 1x1 stride-1 convolution C -> C with a table plan and no residual
 * (a rescaled copy d2->y2 is allowed), reading d1's output (d2->x ==
 * d1->y). The result is what qa_d_conv(d1) then qa_d_conv(d2) store at
 * d2->y (and d2->y2); d1->y is not
 * written. Returns -1, launching nothing, for any other pair; the
 * reference runs the two convolutions one after the other
 * (quant_layers.py:320-335 twice). A second form takes wider pairs when
 * both descriptors carry fragment-order weights (w_frag): d1 a 1x1 or
 * k x k convolution of a multiple of 64 input channels (K up to 1280
 * bytes, one group) and 16..256 output channels (a multiple of 16, no
 * rescaled copy), d2 a 1x1 convolution of 16..256 output channels reading
 * all of them; d1's stored bytes then pass through LDS only (the
 * late-stage C2f inputs of a classifier: Conv_126+Conv_134,
 * Conv_192+Conv_200 of YOLOv8n-cls). qa_conv_chain_supported checks a
 * pair without launching (1 or 0). d2->tile: 0, 0x10000 | R for bands of
 * R output rows a work-group (ignored where they do not fit), or
 * 0x12000 | (T - 1) << 4 for the second form with T row tiles of 16 a
 * work-group (T 1..4, fewer where LDS runs out). */
int qa_conv_chain_supported(const qa_conv_desc* d1, const qa_conv_desc* d2);
int qa_d_conv_chain(const qa_conv_desc* d1, const qa_conv_desc* d2,
                    void* stream);

/* Graph-input quantization fused into the first convolution: x is the
 * float32 NCHW input [N, C, H, W]; it is quantized exactly as
 * qa_d_quantize_nhwc would (scale, zp, clip; storage offset
 * d->x_add + in_zp) and convolved as qa_d_conv would convolve that int8
 * tensor, which is never written (d->x is not read). Requires the int8
 * weights of packed layout 1 (C <= 4, KH <= 4, KW <= 4, one group), an
 * epilogue plan, no residual and no rescaled copy, and a dense channels-last
 * output; anything else returns -1. d->tile: 0, or 0x10000 | R for R output
 * rows per work-group. The reference runs the two steps separately
 * (quant_container.py:150-155 quantizes the input, quant_layers.py:320-335
 * convolves it). */
int qa_d_quantize_conv(const qa_conv_desc* d, const float* x, double in_scale,
                       int64_t in_zp, int64_t in_qmin, int64_t in_qmax,
                       void* stream);

/* Element-wise device entries (storage codes as above, `*_so` storage
 * offsets). The row forms process `rows` rows of `cols` elements with one
 * row stride per operand (a channel slice of an NCHW tensor: rows = N,
 * cols = C_slice*H*W, stride = C*H*W). In qa_d_requantize, `sub` is
 * subtracted from the stored accumulator before the bias. */
int qa_d_requantize(const void* acc, int acc_code, void* out, int out_code,
                    int64_t outer, int64_t C, int64_t inner,
                    const int64_t* mult, const int64_t* shift,
                    const int64_t* pre_bias, const int64_t* post_bias,
                    int64_t zp, int64_t qmin, int64_t qmax, int64_t sub,
                    int64_t out_so, void* stream);
int qa_d_rescale(const void* x, int in_code, int64_t x_rstride, void* out,
                 int out_code, int64_t out_rstride, int64_t rows,
                 int64_t cols, int64_t zp_in, int64_t m, int64_t s,
                 int64_t zp_out, int64_t qmin, int64_t qmax, int64_t in_so,
                 int64_t out_so, void* stream);
int qa_d_add(const void* a, int64_t a_rstride, const void* b,
             int64_t b_rstride, int in_code, void* out, int out_code,
             int64_t out_rstride, int64_t rows, int64_t cols, int64_t za,
             int64_t ma, int64_t sa, int64_t zb, int64_t mb, int64_t sb,
             int64_t sign, int64_t zp_out, int64_t qmin, int64_t qmax,
             int64_t a_so, int64_t b_so, int64_t out_so, void* stream);
int qa_d_mul(const void* a, int64_t a_rstride, const void* b,
             int64_t b_rstride, int in_code, void* out, int out_code,
             int64_t out_rstride, int64_t rows, int64_t cols, int64_t za,
             int64_t zb, int64_t m, int64_t s, int64_t zp_out, int64_t qmin,
             int64_t qmax, int64_t a_so, int64_t b_so, int64_t out_so,
             void* stream);
int qa_d_lut(const void* x, int in_code, int64_t x_rstride, void* out,
             int out_code, int64_t out_rstride, int64_t rows, int64_t cols,
             int64_t offset, const int32_t* lut, int64_t lut_len,
             int64_t in_so, int64_t out_so, void* stream);
int qa_d_quantize_f32(const float* x, void* q, int out_code, int64_t n,
                      double scale, int64_t zp, int64_t qmin, int64_t qmax,
                      int64_t out_so, void* stream);
int qa_d_dequantize_f32(const void* q, int in_code, float* x, int64_t n,
                        double scale, int64_t zp, int64_t in_so,
                        void* stream);

/* GlobalAveragePool of x [N, C, HW] (element (n, c, p) at x + n*x_sn +
 * c*x_sc + p*x_sp; needs x_sc == 1 or x_sp == 1) into out [N, C] (row
 * stride out_sn): clip(mbqm(sum(q - zp_in), mult, shift) + zp_out)
 * (quant_layers.py:563-590). */
int qa_d_gap(const void* x, int in_code, int64_t x_sn, int64_t x_sc,
             int64_t x_sp, int64_t N, int64_t C, int64_t HW, int64_t zp_in,
             int64_t in_so, int64_t mult, int64_t shift, int64_t zp_out,
             int64_t qmin, int64_t qmax, void* out, int out_code,
             int64_t out_sn, int64_t out_so, void* stream);

/* Quantizes float32 NCHW input into channels-last int8/int16 storage with
 * pixel stride y_sp >= C (padding channels 0), half-to-even like
 * qa_quantize_f32. */
int qa_d_quantize_nhwc(const float* x, int64_t N, int64_t C, int64_t HW,
                       void* y, int y_code, int64_t y_sp, double scale,
                       int64_t zp, int64_t qmin, int64_t qmax, int64_t so,
                       void* stream);

/* Quantizes float32 NCHW input [N, C, H, W] (C <= 4) into the int8 rows of
 * a convolution whose stride equals its kernel KH x KW (no padding; KW a
 * multiple of 4, H and W multiples of the kernel; 16-byte aligned x and
 * y): row (n, py, px) of KH*KW*4 bytes holds the patch's pixels kernel row
 * by kernel row, 4 bytes a pixel, each the word qa_d_quantize_nhwc writes
 * with y_sp = 4 (channel c in byte c, 0 above C). The reference quantizes
 * the graph input (quant_container.py:150-155) and the convolution reads
 * its im2col columns (qa_kernels.cpp:107-137, 141-175); for such a
 * convolution those columns are these rows, so it runs as a 1x1
 * convolution over N*OH*OW one-pixel images of KH*KW*4 channels. */
int qa_d_quantize_patches(const float* x, int64_t N, int64_t C, int64_t H,
                          int64_t W, int64_t KH, int64_t KW, void* y,
                          double scale, int64_t zp, int64_t qmin,
                          int64_t qmax, int64_t so, void* stream);

/* Float fallback of Softmax over the last axis of [rows, cols]:
 * dequantize to float32, softmax in float64, float32, quantize
 * (quant_layers.py:195-205, float_ops.py:380-385). */
int qa_d_softmax(const void* x, int in_code, int64_t rows, int64_t cols,
                 double in_scale, int64_t in_zp, int64_t in_so, void* out,
                 int out_code, double out_scale, int64_t out_zp, int64_t qmin,
                 int64_t qmax, int64_t out_so, void* stream);

/* The int8 form of qa_d_softmax through a table of exponentials (results
 * identical to qa_d_softmax): qa_d_softmax_table fills table[65536] (device
 * float64) with exp(F(s) - F(m)) at 256 (m + 128) + s + 128 for stored
 * bytes s <= m, F(b) = float32((b + in_so - in_zp) * in_scale), once per
 * input quantization; qa_d_softmax_lut then reads a row's exponentials at
 * its largest byte (int8 input and output, cols <= 1024). The reference
 * computes exp per element (float_ops.py:380-385). qa_d_softmax_lut_f32
 * also writes the dequantized result to out_f32, as qa_d_softmax_f32. */
int qa_d_softmax_table(double in_scale, int64_t in_zp, int64_t in_so,
                       double* table, void* stream);
int qa_d_softmax_lut(const void* x, int64_t rows, int64_t cols,
                     const double* table, void* out, double out_scale,
                     int64_t out_zp, int64_t qmin, int64_t qmax,
                     int64_t out_so, void* stream);
int qa_d_softmax_lut_f32(const void* x, int64_t rows, int64_t cols,
                         const double* table, void* out, double out_scale,
                         int64_t out_zp, int64_t qmin, int64_t qmax,
                         int64_t out_so, float* out_f32, void* stream);

/* qa_d_softmax that also writes the dequantized result to out_f32
 * ([rows, cols] float32, (q - out_zp) * out_scale as qa_d_dequantize_f32
 * computes it) when the Softmax output is a graph output (the reference
 * dequantizes graph outputs after the pass, quant_container.py:186-192). */
int qa_d_softmax_f32(const void* x, int in_code, int64_t rows, int64_t cols,
                     double in_scale, int64_t in_zp, int64_t in_so, void* out,
                     int out_code, double out_scale, int64_t out_zp,
                     int64_t qmin, int64_t qmax, int64_t out_so,
                     float* out_f32, void* stream);

/* More float fallbacks (dequantize -> float op -> quantize, the reference's
 * quant_layers.py:195-205) for operators with no integer form. Operands
 * dequantize to (float)((q + so - zp) * scale); results quantize as
 * qa_quantize_f32 (double division, half to even) and are stored as q - so.
 * Element strides everywhere (a stride 0 broadcasts). */

/* Div (op 0), Max (1), Min (2) in float32 and Pow (3) in float64, of two
 * activations (float_ops.py:217-222, :321-325); output element
 * (i_0, .., i_{ndim-1}) of `shape` reads a at sum i_k as[k], b at
 * sum i_k bs[k], writes y at sum i_k ys[k]. An operand of code 0 is a
 * float32 constant, read as is. */
typedef struct qa_fb_binary {
    const void* a;
    int64_t a_code, a_so, a_zp;
    double a_scale;
    int64_t as[6];
    const void* b;
    int64_t b_code, b_so, b_zp;
    double b_scale;
    int64_t bs[6];
    void* y;
    int64_t y_code, y_so;
    int64_t ys[6];
    int64_t ndim, shape[6], op;
    double out_scale;
    int64_t out_zp, qmin, qmax;
} qa_fb_binary;
int qa_d_fb_binary(const qa_fb_binary* d, void* stream);

/* Integer Add / Sub (op 0) or Mul (op 1) with NumPy broadcasting
 * (quantization/native.py:465-500 broadcasts both operands, then calls
 * qa_add / qa_mul, qa_kernels.cpp:346-386). Element (i_0, .., i_{ndim-1})
 * of `shape` reads a at sum i_k as[k] and b at sum i_k bs[k] (stride 0 on a
 * broadcast axis) and writes y at sum i_k ys[k]:
 *   op 0: clip(mbqm(a - za, ma, sa) + sign * mbqm(b - zb, mb, sb) + zp_out)
 *   op 1: clip(mbqm((a - za) * (b - zb), ma, sa) + zp_out)
 * Values are stored as q - so (a_so, b_so, y_so) in storage codes 1, 2, 4. */
typedef struct qa_binary_nd {
    const void* a;
    const void* b;
    void* y;
    int64_t a_code, b_code, y_code, a_so, b_so, y_so;
    int64_t ndim, shape[6], as[6], bs[6], ys[6];
    int64_t op, za, ma, sa, zb, mb, sb, sign, zp_out, qmin, qmax;
} qa_binary_nd;
int qa_d_binary_nd(const qa_binary_nd* d, void* stream);

/* ReduceMean (float_ops.py:594-601): output element o (the kept dims,
 * written densely at y + o) = the mean over the reduced dims, summed in
 * float64. */
typedef struct qa_fb_reduce {
    const void* x;
    int64_t x_code, x_so, x_zp;
    double x_scale;
    int64_t nkeep, keep[6], xks[6];
    int64_t nred, red[6], xrs[6];
    void* y;
    int64_t y_code, y_so;
    double out_scale;
    int64_t out_zp, qmin, qmax;
} qa_fb_reduce;
int qa_d_fb_reduce_mean(const qa_fb_reduce* d, void* stream);

/* Softmax (log = 0) or LogSoftmax (log = 1) over one axis of length `len`
 * (float_ops.py:380-395, float64): row (o, i) of outer x inner rows, its
 * element k at o xs_o + k xs_k + i xs_i (likewise for y). */
typedef struct qa_fb_softmax {
    const void* x;
    int64_t x_code, x_so, x_zp;
    double x_scale;
    int64_t outer, len, inner, xs_o, xs_k, xs_i;
    void* y;
    int64_t y_code, y_so, ys_o, ys_k, ys_i;
    int64_t log;
    double out_scale;
    int64_t out_zp, qmin, qmax;
} qa_fb_softmax;
int qa_d_fb_softmax(const qa_fb_softmax* d, void* stream);

/* AveragePool (float_ops.py:563-577): the mean of the window's taps inside
 * the image (count_pad = 0) or their sum over KH*KW (count_pad = 1, the
 * zero padding counted); the caller resolves pads / auto_pad / ceil_mode
 * into PT, PL, OH, OW. Strides per axis (n, c, h, w). */
typedef struct qa_fb_avgpool {
    const void* x;
    int64_t x_code, x_so, x_zp;
    double x_scale;
    int64_t x_sn, x_sc, x_sh, x_sw;
    int64_t N, C, H, W, KH, KW, SH, SW, PT, PL, OH, OW, count_pad;
    void* y;
    int64_t y_code, y_so, y_sn, y_sc, y_sh, y_sw;
    double out_scale;
    int64_t out_zp, qmin, qmax;
} qa_fb_avgpool;
int qa_d_fb_avgpool(const qa_fb_avgpool* d, void* stream);

/* Pad that is not scale-preserving, so the reference runs it as a float
 * fallback (quant_layers.py:617-633 declines it; :195-205): reflect or edge
 * mode, or a non-zero constant (float_ops.py:499-513). Output element
 * (i_0, .., i_{ndim-1}) of `shape` reads x at source index j_k = i_k - lo_k
 * per axis: mode 0 (constant) takes `value` (the float32 pad value) when
 * some j_k lies outside [0, xshape_k); mode 1 (reflect) mirrors j_k about
 * the end elements without repeating them (period 2 (n - 1); n = 1 reads
 * element 0); mode 2 (edge) clamps j_k to the axis. The value is then
 * quantized with the output parameters. Element strides xs / ys. */
typedef struct qa_fb_pad {
    const void* x;
    int64_t x_code, x_so, x_zp;
    double x_scale;
    void* y;
    int64_t y_code, y_so;
    int64_t ndim, shape[6], lo[6], xshape[6], xs[6], ys[6];
    int64_t mode;
    double value;
    double out_scale;
    int64_t out_zp, qmin, qmax;
} qa_fb_pad;
int qa_d_fb_pad(const qa_fb_pad* d, void* stream);

/* Gather with an index array and Cast (float fallbacks, quant_layers.py:
 * 195-205 over float_ops.py:490-496 and :398-402). Output element
 * (i_0, .., i_{ndim-1}) of `shape` reads x at sum over k of c_k xs[k],
 * where c_k = i_k except on axis `axis` (-1: none), where c_k =
 * idx[i_k] (idx: nidx device int64 values in [0, extent), negative
 * indices already wrapped); a Gather's index dimensions arrive collapsed
 * into that one axis. The dequantized float32 value v is then cast to ONNX
 * element type `cast_to` (1 float32 and 11 float64: v; 10 float16: v
 * rounded to nearest even; 9 bool: v != 0; 6 int32 / 3 int8 / 2 uint8 /
 * 5 int16 / 4 uint16: truncated toward zero, INT32_MIN when outside the
 * int32 range, then wrapped to the width; 7 int64: truncated, INT64_MIN
 * outside the int64 range), as NumPy's astype does on x86-64, and
 * quantized: round_half_even((double)t / out_scale) + out_zp, clipped. */
typedef struct qa_fb_gather {
    const void* x;
    int64_t x_code, x_so, x_zp;
    double x_scale;
    const int64_t* idx;
    int64_t nidx, axis, cast_to;
    void* y;
    int64_t y_code, y_so;
    int64_t ndim, shape[6], xs[6], ys[6];
    double out_scale;
    int64_t out_zp, qmin, qmax;
} qa_fb_gather;
int qa_d_fb_gather(const qa_fb_gather* d, void* stream);

/* ---------------------------------------------- allocation-free GEMM --- */
/* No counterpart in the reference. For callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops, harnesses that forbid
 * hipMalloc): C[M,N] = A[M,K] B[K,N] with qa_gemm_i16_i32's semantics
 * (int16 operands, int32 sums modulo 2^32; results bit-identical to it), on
 * device-resident A, B, C, queued on `stream` (NULL: the null stream) with
 * no allocation and no host synchronisation. Its working memory (activation
 * range, int8-packed operands, correction terms, path flag) is one static
 * device array of qa_noalloc_scratch_bytes() bytes (32 MiB) per GPU, held
 * until the process ends; a problem needing more
 * (qa_gemm_i16_i32_noalloc_need) is rejected with -1 and an error message
 * before anything is queued. Every call on a GPU shares that array: calls
 * that overlap on one GPU (other streams, other threads) race. Returns 0
 * when queued, -1 on an error (see qa_last_error). */
int64_t qa_noalloc_scratch_bytes(void);
int64_t qa_gemm_i16_i32_noalloc_need(int64_t M, int64_t N, int64_t K);
int qa_gemm_i16_i32_noalloc(int64_t M, int64_t N, int64_t K, const int16_t* A,
                            const int16_t* B, int32_t* C, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* QA_HIP_H */

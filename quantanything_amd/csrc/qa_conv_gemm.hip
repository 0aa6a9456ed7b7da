// Convolution / GEMM entry points: the reference ABI (host pointers,
// qa_kernels.cpp:252-284) and the device-resident qa_d_conv.
//
// ABI integer path: operands are centred integers of any width. The library
// measures the activation range on the device and the per-channel weight
// ranges on the host; when every range spans at most 256 values it offsets
// both into int8, repacks the activations channels-last and runs the MFMA
// kernel with the exact correction terms (qa_conv.h); otherwise it runs the
// exact VALU kernel on the original data. Either way the result equals the
// reference's int32 (modulo 2^32) or int64 sums.
#include <string.h>

#include <algorithm>
#include <vector>

#include "../../include/qa_hip.h"
#include "qa_conv.h"
#include "qa_valu.h"

namespace qa {
namespace {

constexpr int kThreads = 256;
constexpr int64_t kRowPad = 128;  // packed weight rows per group: x128
constexpr int64_t kTail = 64;     // slack after packed activations

// ------------------------------------------------------------- kernels --
template <class T>
__global__ __launch_bounds__(kThreads) void k_range(const T* x, int64_t n,
                                                    int narrow16, int* mm) {
    int lo = INT32_MAX, hi = INT32_MIN;
    const int64_t step = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += step) {
        int v = (int)x[i];
        if (narrow16) v = (int16_t)v;
        lo = min(lo, v);
        hi = max(hi, v);
    }
    for (int off = 32; off > 0; off >>= 1) {
        lo = min(lo, __shfl_xor(lo, off));
        hi = max(hi, __shfl_xor(hi, off));
    }
    if ((threadIdx.x & 63) == 0) {
        atomicMin(&mm[0], lo);
        atomicMax(&mm[1], hi);
    }
}

// NCHW int32 -> channels-last int8 x_s = v - a_off with pixel stride Cs;
// padding channels are 0.
__global__ __launch_bounds__(kThreads) void k_pack_nhwc(
    const int32_t* x, int8_t* y, int64_t N, int64_t C, int64_t HW,
    int64_t Cs, int narrow16, int a_off) {
    const int64_t total = N * HW * Cs;
    const int64_t step = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
         i < total; i += step) {
        const int64_t c = i % Cs;
        const int64_t np = i / Cs;
        const int64_t n = np / HW, p = np - n * HW;
        int8_t v = 0;
        if (c < C) {
            int x0 = x[(n * C + c) * HW + p];
            if (narrow16) x0 = (int16_t)x0;
            v = (int8_t)(x0 - a_off);
        }
        y[i] = v;
    }
}

// Row-major A[M][K] -> int8 [M][Kp] with zero K-padding.
template <class T>
__global__ __launch_bounds__(kThreads) void k_pack_rows(
    const T* a, int8_t* y, int64_t M, int64_t K, int64_t Kp, int a_off) {
    const int64_t n = M * Kp;
    const int64_t step = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += step) {
        const int64_t m = i / Kp, k = i - m * Kp;
        y[i] = k < K ? (int8_t)((int)a[m * K + k] - a_off) : (int8_t)0;
    }
}

// ------------------------------------------------------------- helpers --
bool fits_i32(int64_t v) { return v >= 0 && v < ((int64_t)1 << 31); }

template <class T>
bool host_copy(const T* src, int64_t n, std::vector<T>& dst) {
    dst.resize((size_t)std::max<int64_t>(n, 1));
    if (n <= 0) return true;
    hipError_t e =
        hipMemcpy(dst.data(), src, (size_t)n * sizeof(T), hipMemcpyDefault);
    if (e != hipSuccess) {
        set_hip_error("hipMemcpy(host copy)", e);
        return false;
    }
    return true;
}

template <class T>
T* upload(int slot, const T* h, int64_t n, hipStream_t st) {
    T* d = (T*)scratch(slot, (size_t)std::max<int64_t>(n, 1) * sizeof(T));
    if (!d) return nullptr;
    if (n <= 0) return d;
    hipError_t e =
        hipMemcpyAsync(d, h, (size_t)n * sizeof(T), hipMemcpyDefault, st);
    if (e != hipSuccess) {
        set_hip_error("hipMemcpyAsync(upload)", e);
        return nullptr;
    }
    return d;
}

bool download(void* h, const void* d, size_t bytes, hipStream_t st) {
    hipError_t e = hipMemcpyAsync(h, d, bytes, hipMemcpyDefault, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess) {
        set_hip_error("download", e);
        return false;
    }
    return true;
}

template <class T>
bool device_range(const T* d, int64_t n, bool narrow16, hipStream_t st,
                  int* lo, int* hi) {
    int* mm = (int*)scratch(7, 2 * sizeof(int));
    if (!mm) return false;
    const int init[2] = {INT32_MAX, INT32_MIN};
    QA_HIP_RET(hipMemcpyAsync(mm, init, sizeof(init), hipMemcpyHostToDevice,
                              st), false);
    k_range<T><<<grid_1d(n, kThreads, 4096), kThreads, 0, st>>>(
        d, n, narrow16 ? 1 : 0, mm);
    QA_HIP_RET(hipGetLastError(), false);
    int out[2];
    if (!download(out, mm, sizeof(out), st)) return false;
    *lo = out[0];
    *hi = out[1];
    return true;
}

// Activation offset making [lo, hi] (0 included, for padding) int8.
bool activation_offset(int lo, int hi, int* a_off) {
    lo = std::min(lo, 0);
    hi = std::max(hi, 0);
    if ((int64_t)hi - lo > 255) return false;
    *a_off = (lo >= -128 && hi <= 127) ? 0 : lo + 128;
    return true;
}

void set_geometry(ConvArgs& a, int64_t N, int64_t C, int64_t H, int64_t W,
                  int64_t Cout, int64_t KH, int64_t KW, int64_t SH, int64_t SW,
                  int64_t PH, int64_t PW, int64_t DH, int64_t DW, int64_t G,
                  int64_t OH, int64_t OW) {
    a.N = (int32_t)N;
    a.H = (int32_t)H;
    a.W = (int32_t)W;
    a.Cg = (int32_t)(C / G);
    a.G = (int32_t)G;
    a.Cog = (int32_t)(Cout / G);
    a.Cout = (int32_t)Cout;
    a.KH = (int32_t)KH;
    a.KW = (int32_t)KW;
    a.SH = (int32_t)SH;
    a.SW = (int32_t)SW;
    a.PH = (int32_t)PH;
    a.PW = (int32_t)PW;
    a.DH = (int32_t)DH;
    a.DW = (int32_t)DW;
    a.OH = (int32_t)OH;
    a.OW = (int32_t)OW;
    a.M = N * OH * OW;
    a.Kreal = a.Cg * a.KH * a.KW;
}

// Packed-weight geometry of a layout (see qa_pack_weights_i8).
void pack_geometry(int64_t Cout, int64_t Cg, int64_t KH, int64_t KW,
                   int64_t G, int layout, int64_t* CB, int64_t* KG,
                   int64_t* KGp, int64_t* rows) {
    // layout 1: CB groups of 4 kernel columns per kernel row
    *CB = layout == 1 ? ceil_div(std::max<int64_t>(KW, 1), 4)
                      : ceil_div(Cg, 16);
    *KG = layout == 1 ? KH * *CB : KH * KW * *CB;
    *KGp = round_up(std::max<int64_t>(*KG, 1), 4);
    *rows = round_up(std::max<int64_t>(Cout / G, 1), kRowPad);
}

bool conv_shape_ok(int64_t N, int64_t C, int64_t H, int64_t W, int64_t Cout,
                   int64_t KH, int64_t KW, int64_t SH, int64_t SW, int64_t DH,
                   int64_t DW, int64_t G, int64_t OH, int64_t OW) {
    if (G <= 0 || C % G || Cout % G || SH <= 0 || SW <= 0 || DH <= 0 ||
        DW <= 0 || KH < 0 || KW < 0) {
        set_error("conv", "invalid geometry (groups, strides or dilations)");
        return false;
    }
    const int64_t dims[] = {N, C, H, W, Cout, KH, KW, OH, OW, N * OH * OW,
                            C * H * W};
    for (int64_t d : dims)
        if (!fits_i32(d)) {
            set_error("conv", "dimension outside [0, 2^31)");
            return false;
        }
    return true;
}

// Whether the int8 MFMA kernels' grids can hold the problem: work-group
// channel blocks of at least 16 channels on grid axis y, groups on axis z.
bool mfma_grid_ok(int64_t Cog, int64_t G) {
    return ceil_div(Cog, 16) <= 65535 && G <= 65535;
}

int pack_weights(const int32_t* w, int64_t Cout, int64_t Cg, int64_t KH,
                 int64_t KW, int64_t G, int64_t a_off, int layout, int8_t* wp,
                 int64_t* corr, int32_t* boff, int32_t* needs_rowsum) {
    if (G <= 0 || Cout % G || Cg < 0 || (layout == 1 && (Cg > 4 || KW > 16)))
        return -1;
    const int64_t Cog = Cout / G;
    int64_t CB, KG, KGp, rows;
    pack_geometry(Cout, Cg, KH, KW, G, layout, &CB, &KG, &KGp, &rows);
    const int64_t K = Cg * KH * KW;
    memset(wp, 0, (size_t)(G * rows * KGp * 16));
    int32_t any = 0;
    for (int64_t co = 0; co < Cout; ++co) {
        const int32_t* row = w + co * K;
        int lo = INT32_MAX, hi = INT32_MIN;
        for (int64_t k = 0; k < K; ++k) {
            lo = std::min(lo, row[k]);
            hi = std::max(hi, row[k]);
        }
        if (K == 0) lo = hi = 0;
        if ((int64_t)hi - lo > 255) return 1;
        const int b = (lo >= -128 && hi <= 127) ? 0 : lo + 128;
        if (b) any = 1;
        int64_t colsum = 0;
        const int64_t g = co / Cog, r = co % Cog;
        int8_t* dst = wp + (g * rows + r) * KGp * 16;
        for (int64_t c = 0; c < Cg; ++c)
            for (int64_t ky = 0; ky < KH; ++ky)
                for (int64_t kx = 0; kx < KW; ++kx) {
                    const int v = row[(c * KH + ky) * KW + kx] - b;
                    colsum += v;
                    const int64_t at =
                        layout == 1 ? (ky * CB + kx / 4) * 16 +
                                          kx % 4 * 4 + c
                                    : ((ky * KW + kx) * CB + c / 16) * 16 +
                                          c % 16;
                    dst[at] = (int8_t)v;
                }
        corr[co] = a_off * colsum + K * a_off * (int64_t)b;
        boff[co] = b;
    }
    *needs_rowsum = any;
    return 0;
}

// Packs host weights and uploads them; fills the weight part of `a`.
bool upload_weights(const std::vector<int32_t>& w32, int64_t Cout, int64_t Cg,
                    int64_t KH, int64_t KW, int64_t G, int a_off, int layout,
                    ConvArgs& a, hipStream_t st) {
    int64_t CB, KG, KGp, rows;
    pack_geometry(Cout, Cg, KH, KW, G, layout, &CB, &KG, &KGp, &rows);
    std::vector<int8_t> wp((size_t)(G * rows * KGp * 16));
    std::vector<int64_t> corr((size_t)std::max<int64_t>(Cout, 1));
    std::vector<int32_t> boff((size_t)std::max<int64_t>(Cout, 1));
    int32_t rowsum = 0;
    if (pack_weights(w32.data(), Cout, Cg, KH, KW, G, a_off, layout,
                     wp.data(), corr.data(), boff.data(), &rowsum) != 0)
        return false;
    a.wp = upload(2, wp.data(), (int64_t)wp.size(), st);
    a.corr = upload(3, corr.data(), Cout, st);
    a.boff = upload(4, boff.data(), Cout, st);
    if (!a.wp || !a.corr || !a.boff) return false;
    a.layout = layout;
    a.CB = (int32_t)CB;
    a.KG = (int32_t)KG;
    a.KGp = (int32_t)KGp;
    a.wp_rstride = KGp * 16;
    a.wp_gstride = rows * KGp * 16;
    a.rowsum = rowsum;
    a.pad_value = -a_off;
    return true;
}

// ------------------------------------------------------------ ABI conv --
template <bool WIDE, class TW>
void conv_abi(const int32_t* x, const TW* w, void* y, int64_t N, int64_t C,
              int64_t H, int64_t W, int64_t Cout, int64_t KH, int64_t KW,
              int64_t SH, int64_t SW, int64_t PH, int64_t PW, int64_t DH,
              int64_t DW, int64_t G, int64_t OH, int64_t OW) {
    const int64_t nout = N * Cout * OH * OW;
    if (nout <= 0) return;
    const size_t ybytes = (size_t)nout * (WIDE ? 8 : 4);
    AbiCall call(y, ybytes);
    if (!conv_shape_ok(N, C, H, W, Cout, KH, KW, SH, SW, DH, DW, G, OH, OW))
        return;
    hipStream_t st = stream();
    if (!st) return;
    void* dy = scratch(1, ybytes);
    if (!dy) return;
    const int64_t Cg = C / G;
    const int64_t K = Cg * KH * KW;
    const int64_t nx = N * C * H * W;
    if (K == 0 || nx == 0) {
        QA_HIP(hipMemsetAsync(dy, 0, ybytes, st));
        download(y, dy, ybytes, st);
        return;
    }
    const int32_t* dx = upload(0, x, nx, st);
    if (!dx) return;
    std::vector<TW> hw;
    if (!host_copy(w, Cout * K, hw)) return;
    std::vector<int32_t> w32(hw.begin(), hw.begin() + Cout * K);

    ConvArgs a;
    memset(&a, 0, sizeof(a));
    set_geometry(a, N, C, H, W, Cout, KH, KW, SH, SW, PH, PW, DH, DW, G, OH,
                 OW);
    a.mode = WIDE ? EPI_RAW64 : EPI_RAW32;
    a.y = dy;
    a.y_code = WIDE ? 8 : 4;
    a.y_sn = Cout * OH * OW;
    a.y_sc = OH * OW;
    a.y_sp = 1;

    int lo, hi, a_off = 0;
    if (!device_range(dx, nx, !WIDE, st, &lo, &hi)) return;
    const int layout = (G == 1 && Cg <= 4 && KW <= 16) ? 1 : 0;
    bool mfma = K < 131072 && activation_offset(lo, hi, &a_off) &&
                (layout == 1 || G == 1 || Cg % 16 == 0) &&
                mfma_grid_ok(Cout / G, G);
    if (mfma)
        mfma = upload_weights(w32, Cout, Cg, KH, KW, G, a_off, layout, a, st);
    if (!ok()) return;
    if (mfma) {
        const int64_t Cs = layout == 1 ? 4 : (G == 1 ? round_up(C, 16) : C);
        const int64_t HW = H * W;
        const int64_t nb = N * HW * Cs;
        int8_t* dxs = (int8_t*)scratch(6, (size_t)(nb + kTail));
        if (!dxs) return;
        k_pack_nhwc<<<grid_1d(nb, kThreads, 1 << 20), kThreads, 0, st>>>(
            dx, dxs, N, C, HW, Cs, WIDE ? 0 : 1, a_off);
        QA_HIP(hipGetLastError());
        a.x = dxs;
        a.x_code = 1;
        a.x_sn = HW * Cs;
        a.x_sc = 1;
        a.x_sp = Cs;
        if (!launch_conv_mfma(a, st)) return;
    } else {
        const TW* dw = upload(2, hw.data(), Cout * K, st);
        if (!dw) return;
        a.x = dx;
        a.x_code = 4;
        a.x_sn = C * H * W;
        a.x_sc = H * W;
        a.x_sp = 1;
        a.narrow16 = WIDE ? 0 : 1;
        a.w = dw;
        a.w_code = sizeof(TW);
        a.wide = WIDE ? 1 : 0;
        if (!launch_conv_valu(a, st)) return;
    }
    download(y, dy, ybytes, st);
}

// ------------------------------------------------------------ ABI GEMM --
template <bool WIDE, class T>
void gemm_abi(int64_t M, int64_t N, int64_t K, const T* A, const T* B,
              void* Cm) {
    if (M <= 0 || N <= 0) return;
    const size_t cbytes = (size_t)(M * N) * (WIDE ? 8 : 4);
    AbiCall call(Cm, cbytes);
    if (!fits_i32(M) || !fits_i32(N) || !fits_i32(K)) {
        set_error("gemm", "dimension outside [0, 2^31)");
        return;
    }
    hipStream_t st = stream();
    if (!st) return;
    void* dc = scratch(1, cbytes);
    if (!dc) return;
    if (K == 0) {
        QA_HIP(hipMemsetAsync(dc, 0, cbytes, st));
        download(Cm, dc, cbytes, st);
        return;
    }
    const T* da = upload(0, A, M * K, st);
    if (!da) return;
    std::vector<T> hb;
    if (!host_copy(B, K * N, hb)) return;
    int lo, hi, a_off = 0;
    if (!device_range(da, M * K, false, st, &lo, &hi)) return;
    bool mfma = K < 131072 && activation_offset(lo, hi, &a_off) &&
                mfma_grid_ok(N, 1);
    ConvArgs a;
    memset(&a, 0, sizeof(a));
    // A GEMM is a 1x1 convolution of M one-pixel "images" with K channels.
    set_geometry(a, M, K, 1, 1, N, 1, 1, 1, 1, 0, 0, 1, 1, 1, 1, 1);
    a.mode = WIDE ? EPI_RAW64 : EPI_RAW32;
    a.y = dc;
    a.y_code = WIDE ? 8 : 4;
    a.y_sn = N;
    a.y_sc = 1;
    a.y_sp = 0;
    if (mfma) {
        std::vector<int32_t> bt((size_t)(N * K));  // B^T: [N][K]
        for (int64_t k = 0; k < K; ++k)
            for (int64_t n = 0; n < N; ++n)
                bt[n * K + k] = (int32_t)hb[k * N + n];
        mfma = upload_weights(bt, N, K, 1, 1, 1, a_off, 0, a, st);
    }
    if (!ok()) return;
    if (mfma) {
        const int64_t Kp = round_up(K, 16);
        int8_t* das = (int8_t*)scratch(6, (size_t)(M * Kp + kTail));
        if (!das) return;
        k_pack_rows<T><<<grid_1d(M * Kp, kThreads, 1 << 20), kThreads, 0,
                         st>>>(da, das, M, K, Kp, a_off);
        QA_HIP(hipGetLastError());
        a.x = das;
        a.x_code = 1;
        a.x_sn = Kp;
        a.x_sc = 1;
        a.x_sp = 0;
        if (!launch_conv_mfma(a, st)) return;
    } else {
        const T* db = upload(2, hb.data(), K * N, st);
        if (!db) return;
        if (!launch_gemm_valu(da, sizeof(T), db, sizeof(T), dc, M, N, K, WIDE,
                              st))
            return;
    }
    download(Cm, dc, cbytes, st);
}

}  // namespace
}  // namespace qa

using namespace qa;

// ================================================== reference ABI exports ==
QA_API int qa_num_threads(void) {
    int d = 0, n = 0;
    if (hipGetDevice(&d) != hipSuccess) return 1;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, d) !=
        hipSuccess)
        return 1;
    return n;
}

QA_API void qa_set_num_threads(int n) { (void)n; }

QA_API int qa_has_openmp(void) { return 0; }

QA_API void qa_gemm_f32(int64_t M, int64_t N, int64_t K, const float* A,
                        const float* B, float* C) {
    if (M <= 0 || N <= 0) return;
    AbiCall call(C, (size_t)(M * N) * 4);
    hipStream_t st = stream();
    if (!st) return;
    const float* da = upload(0, A, M * K, st);
    const float* db = upload(2, B, K * N, st);
    float* dc = (float*)scratch(1, (size_t)(M * N) * 4);
    if (!da || !db || !dc) return;
    if (!launch_gemm_f32(da, db, dc, M, N, K, st)) return;
    download(C, dc, (size_t)(M * N) * 4, st);
}

QA_API void qa_gemm_i16_i32(int64_t M, int64_t N, int64_t K, const int16_t* A,
                            const int16_t* B, int32_t* C) {
    gemm_abi<false, int16_t>(M, N, K, A, B, C);
}

QA_API void qa_gemm_i32_i64(int64_t M, int64_t N, int64_t K, const int32_t* A,
                            const int32_t* B, int64_t* C) {
    gemm_abi<true, int32_t>(M, N, K, A, B, C);
}

#define QA_CONV_PARAMS                                                       \
    int64_t N, int64_t C, int64_t H, int64_t W, int64_t Cout, int64_t KH,    \
        int64_t KW, int64_t SH, int64_t SW, int64_t PH, int64_t PW,          \
        int64_t DH, int64_t DW, int64_t G, int64_t OH, int64_t OW
#define QA_CONV_FWD N, C, H, W, Cout, KH, KW, SH, SW, PH, PW, DH, DW, G, OH, OW

QA_API void qa_conv_f32(const float* x, const float* w, float* y,
                        QA_CONV_PARAMS) {
    const int64_t nout = N * Cout * OH * OW;
    if (nout <= 0) return;
    AbiCall call(y, (size_t)nout * 4);
    if (!conv_shape_ok(N, C, H, W, Cout, KH, KW, SH, SW, DH, DW, G, OH, OW))
        return;
    hipStream_t st = stream();
    if (!st) return;
    const float* dx = upload(0, x, N * C * H * W, st);
    const float* dw = upload(2, w, Cout * (C / G) * KH * KW, st);
    float* dy = (float*)scratch(1, (size_t)nout * 4);
    if (!dx || !dw || !dy) return;
    ConvArgs a;
    memset(&a, 0, sizeof(a));
    set_geometry(a, QA_CONV_FWD);
    if (!launch_conv_f32(dx, dw, dy, a, st)) return;
    download(y, dy, (size_t)nout * 4, st);
}

QA_API void qa_conv_i32_i16_i32(const int32_t* x, const int16_t* w,
                                int32_t* y, QA_CONV_PARAMS) {
    conv_abi<false, int16_t>(x, w, y, QA_CONV_FWD);
}

QA_API void qa_conv_i32_i32_i64(const int32_t* x, const int32_t* w,
                                int64_t* y, QA_CONV_PARAMS) {
    conv_abi<true, int32_t>(x, w, y, QA_CONV_FWD);
}

// ============================================== additional surface ==
QA_API int64_t qa_pack_weights_i8_size(int64_t Cout, int64_t Cg, int64_t KH,
                                       int64_t KW, int64_t G, int64_t layout,
                                       int64_t* kgp, int64_t* rows_per_group) {
    if (G <= 0 || Cout < 0 || Cout % G || layout < 0 || layout > 1) return -1;
    int64_t CB, KG, KGp, rows;
    pack_geometry(Cout, Cg, KH, KW, G, (int)layout, &CB, &KG, &KGp, &rows);
    if (kgp) *kgp = KGp;
    if (rows_per_group) *rows_per_group = rows;
    return G * rows * KGp * 16;
}

QA_API int qa_pack_weights_i8(const int32_t* w, int64_t Cout, int64_t Cg,
                              int64_t KH, int64_t KW, int64_t G, int64_t a_off,
                              int64_t layout, int8_t* wp, int64_t* corr,
                              int32_t* boff, int32_t* needs_rowsum) {
    return pack_weights(w, Cout, Cg, KH, KW, G, a_off, (int)layout, wp, corr,
                        boff, needs_rowsum);
}

QA_API int64_t qa_pack_weights_f64_size(int64_t Cout, int64_t Cg, int64_t KH,
                                        int64_t KW, int64_t G, int64_t* ck,
                                        int64_t* rows_per_group) {
    if (G <= 0 || Cout < 0 || Cout % G || Cg < 0 || KH < 0 || KW < 0)
        return -1;
    const int64_t CK = round_up(std::max<int64_t>(Cg, 1), 32);
    const int64_t rows = round_up(std::max<int64_t>(Cout / G, 1), 64);
    if (ck) *ck = CK;
    if (rows_per_group) *rows_per_group = rows;
    return G * rows * KH * KW * CK;
}

QA_API int qa_pack_weights_f64(const int32_t* w, int64_t Cout, int64_t Cg,
                               int64_t KH, int64_t KW, int64_t G,
                               int64_t elem_bytes, void* wp) {
    int64_t CK, rows;
    const int64_t n =
        qa_pack_weights_f64_size(Cout, Cg, KH, KW, G, &CK, &rows);
    if (n < 0 || !wp || (elem_bytes != 2 && elem_bytes != 4) ||
        (!w && Cout * Cg * KH * KW > 0))
        return -1;
    if (KH * KW * CK >= ((int64_t)1 << 19)) return 1;
    const int64_t lim = elem_bytes == 2 ? 32768 : (1 << 17);
    const int64_t K = Cg * KH * KW;
    for (int64_t i = 0; i < Cout * K; ++i)
        if (w[i] < -lim || w[i] >= lim) return 1;
    const int64_t Cog = Cout / G, taps = KH * KW;
    memset(wp, 0, (size_t)(n * elem_bytes));
    for (int64_t co = 0; co < Cout; ++co) {
        const int64_t g = co / Cog, r = co % Cog;
        const int64_t row = (g * rows + r) * taps * CK;
        for (int64_t c = 0; c < Cg; ++c)
            for (int64_t t = 0; t < taps; ++t) {
                const int32_t v = w[(co * Cg + c) * taps + t];
                if (elem_bytes == 2)
                    ((int16_t*)wp)[row + t * CK + c] = (int16_t)v;
                else
                    ((int32_t*)wp)[row + t * CK + c] = v;
            }
    }
    return 0;
}

QA_API int qa_pack_weights_i16s(const int32_t* w, int64_t Cout, int64_t Cg,
                                int64_t KH, int64_t KW, int64_t G, int8_t* wp,
                                int64_t* wsum) {
    if (G <= 0 || Cout < 0 || Cout % G || Cg < 0 || KH < 0 || KW < 0 ||
        !wp || !wsum || (!w && Cout * Cg * KH * KW > 0))
        return -1;
    int64_t CB, KG, KGp, rows;
    pack_geometry(Cout, Cg, KH, KW, G, 0, &CB, &KG, &KGp, &rows);
    const int64_t plane = G * rows * KGp * 16, K = Cg * KH * KW;
    for (int64_t i = 0; i < Cout * K; ++i)
        if (w[i] < -32768 || w[i] > 32767) return 1;
    // w = 0 where no weight sits: high byte 0, low byte 0 - 128
    memset(wp, 0, (size_t)plane);
    memset(wp + plane, 0x80, (size_t)plane);
    const int64_t Cog = Cout / G;
    for (int64_t co = 0; co < Cout; ++co) {
        const int32_t* row = w + co * K;
        const int64_t g = co / Cog, r = co % Cog;
        int8_t* hi = wp + (g * rows + r) * KGp * 16;
        int8_t* lo = hi + plane;
        int64_t sum = 0;
        for (int64_t c = 0; c < Cg; ++c)
            for (int64_t ky = 0; ky < KH; ++ky)
                for (int64_t kx = 0; kx < KW; ++kx) {
                    const int v = row[(c * KH + ky) * KW + kx];
                    const int64_t at =
                        ((ky * KW + kx) * CB + c / 16) * 16 + c % 16;
                    hi[at] = (int8_t)(v >> 8);
                    lo[at] = (int8_t)((v & 255) - 128);
                    sum += v;
                }
        wsum[co] = sum;
    }
    return 0;
}

namespace {

// Kernel arguments of a device descriptor: 1 for the int8 MFMA path, 0 for
// the VALU path, 3 for the FP64 MFMA path, 2 for an empty problem, -1 on
// error (recorded for `who`).
int desc_args(const qa_conv_desc* d, ConvArgs& a, const char* who) {
    if (!d) return -1;
    if (!conv_shape_ok(d->N, d->C, d->H, d->W, d->Cout, d->KH, d->KW, d->SH,
                       d->SW, d->DH, d->DW, d->G, d->OH, d->OW))
        return -1;
    if (d->N * d->Cout * d->OH * d->OW == 0) return 2;
    if (d->y_code != 1 && d->y_code != 2) {
        set_error(who, "output storage must be int8 or int16");
        return -1;
    }
    memset(&a, 0, sizeof(a));
    set_geometry(a, d->N, d->C, d->H, d->W, d->Cout, d->KH, d->KW, d->SH,
                 d->SW, d->PH, d->PW, d->DH, d->DW, d->G, d->OH, d->OW);
    a.x = d->x;
    a.x_code = (int32_t)d->x_code;
    a.x_sn = d->x_sn;
    a.x_sc = d->x_sc;
    a.x_sp = d->x_sp;
    a.x_add = d->x_add;
    a.corr = d->corr;
    a.boff = d->boff;
    a.pre = d->pre_bias;
    a.mult = d->mult;
    a.shift = d->shift;
    a.mode = EPI_QUANT;
    a.zp = d->zp;
    a.qmin = d->qmin;
    a.qmax = d->qmax;
    a.lut = d->lut;
    a.lut_off = d->lut_offset;
    a.lut_len = d->lut_len;
    a.res = d->res;
    a.res_sn = d->res_sn;
    a.res_sc = d->res_sc;
    a.res_sp = d->res_sp;
    a.res_so = d->res_so;
    a.res_first = (int32_t)d->res_first;
    a.za = d->za;
    a.ma = d->ma;
    a.sa = d->sa;
    a.zb = d->zb;
    a.mb = d->mb;
    a.sb = d->sb;
    a.add_sign = d->add_sign;
    a.add_zp = d->add_zp;
    a.add_qmin = d->add_qmin;
    a.add_qmax = d->add_qmax;
    a.y = d->y;
    a.y_code = (int32_t)d->y_code;
    a.y_sn = d->y_sn;
    a.y_sc = d->y_sc;
    a.y_sp = d->y_sp;
    a.y_so = d->y_so;
    a.y2 = d->y2;
    a.y2_sn = d->y2_sn;
    a.y2_sc = d->y2_sc;
    a.y2_sp = d->y2_sp;
    a.r2_zp_in = d->r2_zp_in;
    a.r2_m = d->r2_m;
    a.r2_s = d->r2_s;
    a.r2_zp_out = d->r2_zp_out;
    a.r2_qmin = d->r2_qmin;
    a.r2_qmax = d->r2_qmax;
    if (d->w_code == 1) {
        int64_t CB, KG, KGp, rows;
        pack_geometry(d->Cout, d->C / d->G, d->KH, d->KW, d->G,
                      (int)d->w_layout, &CB, &KG, &KGp, &rows);
        const uintptr_t xa = (uintptr_t)d->x;
        const bool aligned =
            d->w_layout == 1
                ? (d->x_sp % 4 == 0 && d->x_sn % 4 == 0 && xa % 4 == 0 &&
                   d->G == 1)
                : (xa % 16 == 0 && d->x_sn % 16 == 0 &&
                   (d->H * d->W == 1 || d->x_sp % 16 == 0) &&
                   (d->G == 1 || (d->C / d->G) % 16 == 0));
        if (d->x_code != 1 || d->x_sc != 1 || d->x_add < -127 ||
            d->x_add > 128 || d->w_kgp != KGp || d->w_rows != rows ||
            a.Kreal >= 131072 || !aligned) {
            set_error(who, "int8 MFMA path: operands do not match");
            return -1;
        }
        a.wp = (const int8_t*)d->w;
        a.wfrag = (const int8_t*)d->w_frag;
        a.layout = (int32_t)d->w_layout;
        a.CB = (int32_t)CB;
        a.KG = (int32_t)KG;
        a.KGp = (int32_t)KGp;
        a.wp_rstride = KGp * 16;
        a.wp_gstride = rows * KGp * 16;
        a.pad_value = (int32_t)(-d->x_add);
        a.rowsum = (int32_t)d->needs_rowsum;
        a.plan = d->epi_plan;
        a.tile_hint = (int32_t)d->tile;
        return 1;
    }
    if (d->w_code == 8) {
        int64_t CK, rows;
        qa_pack_weights_f64_size(d->Cout, d->C / d->G, d->KH, d->KW, d->G,
                                 &CK, &rows);
        if (d->x_code != 2 || d->x_sc != 1 || d->x_add < -65536 ||
            d->x_add > 65536 || d->w_kgp != CK || d->w_rows != rows ||
            (d->w_layout != 2 && d->w_layout != 4) ||
            d->KH * d->KW * CK >= ((int64_t)1 << 19)) {
            set_error(who, "FP64 MFMA path: operands do not match");
            return -1;
        }
        a.wf = d->w;
        a.wf_bytes = (int32_t)d->w_layout;
        a.CK = (int32_t)CK;
        a.wf_rows = (int32_t)rows;
        a.wide = (int32_t)d->wide;
        a.tile_hint = (int32_t)d->tile;
        if (d->wsplit && d->wsplit_k) {  // the byte-split planes
            int64_t CB, KG, KGp, prow;
            pack_geometry(d->Cout, d->C / d->G, d->KH, d->KW, d->G, 0, &CB,
                          &KG, &KGp, &prow);
            a.ws = (const int8_t*)d->wsplit;
            a.ws_k = d->wsplit_k;
            a.CB = (int32_t)CB;
            a.KG = (int32_t)KG;
            a.KGp = (int32_t)KGp;
            a.wp_rstride = KGp * 16;
            a.wp_gstride = prow * KGp * 16;
            a.mg_cb = (((uint64_t)1 << 32) + CB - 1) / (uint64_t)CB;
            a.mg_kw = (((uint64_t)1 << 32) + std::max<int64_t>(d->KW, 1) -
                       1) / (uint64_t)std::max<int64_t>(d->KW, 1);
        }
        return 3;
    }
    a.w = d->w;
    a.w_code = (int32_t)d->w_code;
    a.wide = (int32_t)d->wide;
    return 0;
}

}  // namespace

QA_API int qa_d_conv(const qa_conv_desc* d, void* stream_) {
    hipStream_t st = (hipStream_t)stream_;
    ConvArgs a;
    const int r = desc_args(d, a, "qa_d_conv");
    if (r < 0) return -1;
    if (r == 2) return 0;
    if (r == 1) return launch_conv_mfma(a, st) ? 0 : -1;
    if (r == 3) return launch_conv_f64(a, st) ? 0 : -1;
    return launch_conv_valu(a, st) ? 0 : -1;
}

// Launch forms of two chained convolution descriptors that the fused
// kernel takes, or false.
static bool pair_args(const qa_conv_desc* d1, const qa_conv_desc* d2,
                      ConvArgs& b1, ConvArgs& b2, const char* who) {
    ConvArgs a1, a2;
    if (desc_args(d1, a1, who) != 1 || desc_args(d2, a2, who) != 1)
        return false;
    const int e1 = fast_io_args(a1, b1, -1);  // Q8_TABLE or -1
    const int e2 = fast_io_args(a2, b2, -1);
    return conv_pair_applies(b1, e1, b2, e2);
}

QA_API int qa_conv_pair_supported(const qa_conv_desc* d1,
                                  const qa_conv_desc* d2) {
    ConvArgs b1, b2;
    return pair_args(d1, d2, b1, b2, "qa_conv_pair_supported") ? 1 : 0;
}

QA_API int qa_d_conv_pair(const qa_conv_desc* d1, const qa_conv_desc* d2,
                          void* stream_) {
    ConvArgs b1, b2;
    if (!pair_args(d1, d2, b1, b2, "qa_d_conv_pair")) {
        set_error("qa_d_conv_pair",
                  "needs two int8 3x3 stride-1 C -> C convolutions (C 16, "
                  "32, 64 or 128) with table plans, the second reading the "
                  "first's output");
        return -1;
    }
    return launch_conv_pair(b1, b2, (hipStream_t)stream_) ? 0 : -1;
}

static bool pair_tail_args(const qa_conv_desc* d1, const qa_conv_desc* d2,
                           const qa_conv_desc* d3, ConvArgs& b1, ConvArgs& b2,
                           ConvArgs& b3, const char* who) {
    ConvArgs a1, a2, a3;
    if (desc_args(d1, a1, who) != 1 || desc_args(d2, a2, who) != 1 ||
        desc_args(d3, a3, who) != 1)
        return false;
    const int e1 = fast_io_args(a1, b1, -1);  // Q8_TABLE or -1
    const int e2 = fast_io_args(a2, b2, -1);
    const int e3 = fast_io_args(a3, b3, -1);
    return conv_pair_tail_applies(b1, e1, b2, e2, b3, e3);
}

QA_API int qa_conv_pair_tail_supported(const qa_conv_desc* d1,
                                       const qa_conv_desc* d2,
                                       const qa_conv_desc* d3) {
    ConvArgs b1, b2, b3;
    return pair_tail_args(d1, d2, d3, b1, b2, b3,
                          "qa_conv_pair_tail_supported")
               ? 1
               : 0;
}

QA_API int qa_d_conv_pair_tail(const qa_conv_desc* d1,
                               const qa_conv_desc* d2,
                               const qa_conv_desc* d3, void* stream_) {
    ConvArgs b1, b2, b3;
    if (!pair_tail_args(d1, d2, d3, b1, b2, b3, "qa_d_conv_pair_tail")) {
        set_error("qa_d_conv_pair_tail",
                  "needs a fused pair (C 16 or 32) whose output is the "
                  "last channels of a 1x1 convolution's dense input (at most "
                  "256 input and 128 output channels, table plan, no "
                  "residual or second output)");
        return -1;
    }
    return launch_conv_pair(b1, b2, (hipStream_t)stream_, &b3) ? 0 : -1;
}

// 0: no chain kernel takes the pair; 1: the weights-in-registers chain
// (and maybe the narrow one); 2: the narrow chain only
static int chain_args(const qa_conv_desc* d1, const qa_conv_desc* d2,
                      ConvArgs& b1, ConvArgs& b2, const char* who) {
    ConvArgs a1, a2;
    if (desc_args(d1, a1, who) != 1 || desc_args(d2, a2, who) != 1)
        return 0;
    const int e1 = fast_io_args(a1, b1, -1);  // Q8_TABLE or -1
    const int e2 = fast_io_args(a2, b2, -1);
    if (conv_chain_applies(b1, e1, b2, e2)) return 1;
    return e1 != -1 && e2 != -1 && narrow_chain_applies(b1, b2) ? 2 : 0;
}

QA_API int qa_conv_chain_supported(const qa_conv_desc* d1,
                                   const qa_conv_desc* d2) {
    ConvArgs b1, b2;
    return chain_args(d1, d2, b1, b2, "qa_conv_chain_supported") ? 1 : 0;
}

QA_API int qa_d_conv_chain(const qa_conv_desc* d1, const qa_conv_desc* d2,
                           void* stream_) {
    ConvArgs b1, b2;
    const int k = chain_args(d1, d2, b1, b2, "qa_d_conv_chain");
    if (!k) {
        set_error("qa_d_conv_chain",
                  "needs an int8 convolution of 16, 32 or 64 output channels "
                  "(weights-in-registers form, no residual) and a 1x1 "
                  "convolution of the same width reading its output, both "
                  "with table plans; or, with the weights in fragment order, "
                  "a 1x1 or k x k convolution of a multiple of 64 input "
                  "channels and up to 256 output channels and a 1x1 "
                  "convolution of up to 256 reading its output");
        return -1;
    }
    // d2->tile 0x12000 | (T - 1) << 4: the narrow chain, T row tiles a
    // work-group; the narrow chain also where the other does not apply
    const int64_t t = d2->tile;
    const bool narrow_hint = (t & TILE_VALID) && ((t >> 13) & 1);
    if (k == 2 || (narrow_hint && narrow_chain_applies(b1, b2)))
        return launch_narrow_chain(b1, b2,
                                   narrow_hint ? 1 + (int)((t >> 4) & 3) : 1,
                                   (hipStream_t)stream_)
                   ? 0
                   : -1;
    return launch_conv_chain(b1, b2, (hipStream_t)stream_) ? 0 : -1;
}

QA_API int qa_d_conv_pool(const qa_conv_desc* d, const qa_pool_params* p,
                          void* stream_) {
    hipStream_t st = (hipStream_t)stream_;
    ConvArgs a;
    const int r = desc_args(d, a, "qa_d_conv_pool");
    if (r < 0) return -1;
    if (r == 2) return 0;
    if (r != 1 || !p || !p->out || d->y_code != 1) {
        set_error("qa_d_conv_pool",
                  "needs int8 packed weights, int8 storage and a pool");
        return -1;
    }
    PoolArgs pl;
    pl.base = d->OH * d->OW * (d->y_so - p->in_zp);
    pl.mult = p->mult;
    pl.shift = p->shift;
    pl.zp = p->zp;
    pl.qmin = p->qmin;
    pl.qmax = p->qmax;
    pl.out_so = p->out_so;
    pl.out = (int8_t*)p->out;
    pl.out_sn = p->out_sn;
    return launch_conv_pool(a, pl, st) ? 0 : -1;
}

static bool pw_pool_args(const qa_conv_desc* d1, const qa_conv_desc* d2,
                         ConvArgs& b1, ConvArgs& b2, const char* who) {
    ConvArgs a1, a2;
    if (desc_args(d1, a1, who) != 1 || desc_args(d2, a2, who) != 1)
        return false;
    fast_io_args(a1, b1, -1);
    fast_io_args(a2, b2, -1);
    return conv_pw_pool_applies(b1, b2);
}

QA_API int qa_conv_pw_pool_supported(const qa_conv_desc* d1,
                                     const qa_conv_desc* d2) {
    ConvArgs b1, b2;
    return pw_pool_args(d1, d2, b1, b2, "qa_conv_pw_pool_supported") ? 1 : 0;
}

QA_API int64_t qa_fragments_i8_size(int64_t rows, int64_t kgp) {
    return rows > 0 && kgp > 0 && kgp % 4 == 0 ? fragments_bytes(rows, kgp)
                                               : 0;
}

QA_API int qa_d_pack_fragments_i8(const void* packed, int64_t rows,
                                  int64_t kgp, void* out, void* stream_) {
    if (!packed || !out || qa_fragments_i8_size(rows, kgp) == 0) {
        set_error("qa_d_pack_fragments_i8",
                  "needs packed weights, rows > 0 and a multiple of 4 "
                  "K-groups");
        return -1;
    }
    return launch_pack_fragments((const int8_t*)packed, rows, kgp,
                                 (int8_t*)out, (hipStream_t)stream_)
               ? 0
               : -1;
}

QA_API int qa_d_conv_pw_pool(const qa_conv_desc* d1, const qa_conv_desc* d2,
                             const qa_pool_params* p, void* stream_) {
    ConvArgs b1, b2;
    if (!p || !p->out || !pw_pool_args(d1, d2, b1, b2, "qa_d_conv_pw_pool")) {
        set_error("qa_d_conv_pw_pool",
                  "needs two int8 1x1 convolutions with table plans (no "
                  "residual, second output or weight offsets), the second "
                  "reading the first's output, images of at most 64 pixels, "
                  "at most 256 channels between them, weights in fragment "
                  "order, and a pool");
        return -1;
    }
    PoolArgs pl;
    pl.base = d2->OH * d2->OW * (d2->y_so - p->in_zp);
    pl.mult = p->mult;
    pl.shift = p->shift;
    pl.zp = p->zp;
    pl.qmin = p->qmin;
    pl.qmax = p->qmax;
    pl.out_so = p->out_so;
    pl.out = (int8_t*)p->out;
    pl.out_sn = p->out_sn;
    return launch_conv_pw_pool(b1, b2, pl, (hipStream_t)stream_) ? 0 : -1;
}

QA_API int qa_d_quantize_conv(const qa_conv_desc* d, const float* x,
                              double in_scale, int64_t in_zp, int64_t in_qmin,
                              int64_t in_qmax, void* stream_) {
    hipStream_t st = (hipStream_t)stream_;
    ConvArgs a;
    const int r = desc_args(d, a, "qa_d_quantize_conv");
    if (r < 0) return -1;
    if (r == 2) return 0;
    if (r != 1 || !x || !(in_scale > 0.0)) {
        set_error("qa_d_quantize_conv",
                  "needs int8 packed weights, an input and a positive scale");
        return -1;
    }
    QinArgs q;
    q.xf = x;
    q.scale = in_scale;
    q.inv = 1.0 / in_scale;
    q.zp = in_zp;
    q.qmin = in_qmin;
    q.qmax = in_qmax;
    q.so = d->x_add + in_zp;  // stored = q - so, x_add = so - zp
    return launch_conv_qin(a, q, st) ? 0 : -1;
}

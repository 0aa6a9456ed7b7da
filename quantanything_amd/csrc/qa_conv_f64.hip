// Convolution / GEMM of 16-bit models on the FP64 matrix cores, exact.
//
// 16-bit models need sums of products wider than int32 (the reference's
// int32 x int32 -> int64 path, qa_kernels.cpp:281-284 and :260-263). Here
// the centred activations (|x| <= 2^17) and weights (|w| < 2^17) are
// converted to double: every product is an integer below 2^34 and every
// partial sum stays below 2^53 while K < 2^19, so each fused multiply-add of
// v_mfma_f64_16x16x4_f64 is exact in any order and the accumulator holds the
// exact integer sum, converted back to int64 for the 128-bit requantization
// epilogue. Results are identical to the int64 VALU form.
//
// A wave owns 16 output pixels (batch folded in; rows of the MFMA) x WM*16
// output channels (columns). K runs over the taps and, per tap, over chunks
// of 4V input channels: lane (pixel col, group q) loads the V consecutive
// channels 4V*cc + V*q .. + V-1 of its pixel as one vector, and MFMA j
// (j < V) sums channels {4V*cc + V*q + j : q = 0..3}. Channels past Cg meet
// zero weights (weights are packed as double rows [group][channel, padded
// to 64][tap][Cg padded to 32], zero-filled) and are loaded as 0, so every
// access stays inside the input. The MFMA's result register r of lane l is
// output row 4r + l/16, column l%16.
#include "qa_conv_mfma.h"

namespace qa {
namespace {

typedef double v4d __attribute__((ext_vector_type(4)));

template <int V>
struct VecI16;
template <>
struct VecI16<1> {
    typedef int16_t T;
    static __device__ __forceinline__ int get(T v, int) { return v; }
};
template <>
struct VecI16<2> {
    typedef int T;
    static __device__ __forceinline__ int get(T v, int j) {
        return (int)(int16_t)(v >> (16 * j));
    }
};
template <>
struct VecI16<4> {
    typedef int2 T;
    static __device__ __forceinline__ int get(T v, int j) {
        const int w = j < 2 ? v.x : v.y;
        return (int)(int16_t)(w >> (16 * (j & 1)));
    }
};
template <>
struct VecI16<8> {
    typedef int4 T;
    static __device__ __forceinline__ int get(T v, int j) {
        const int w = j < 2 ? v.x : (j < 4 ? v.y : (j < 6 ? v.z : v.w));
        return (int)(int16_t)(w >> (16 * (j & 1)));
    }
};

template <int WM, int V>
__global__ __launch_bounds__(256) void k_conv_f64(ConvArgs a) {
    typedef typename VecI16<V>::T VT;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int col = lane & 15, kgl = lane >> 4;
    const int g = blockIdx.z;
    const int co0 = blockIdx.y * WM * 16;
    const int64_t tile = (int64_t)blockIdx.x * 4 + wave;
    if (tile * 16 >= a.M) return;
    // this lane's fetch pixel (clamped into the tensor)
    const int64_t p = min(tile * 16 + col, a.M - 1);
    const PixPos pos = pix_decode(a, p);
    const int taps = a.KH * a.KW;
    const int nck = (a.Cg + 4 * V - 1) / (4 * V);
    const int16_t* xn = (const int16_t*)a.x + (int64_t)pos.n * a.x_sn +
                        (int64_t)g * a.Cg + V * kgl;
    const double* wrow =
        a.wf + ((int64_t)g * a.wf_rows + co0 + col) * taps * a.CK + V * kgl;
    const int64_t wblk = (int64_t)16 * taps * a.CK;  // the next 16 channels
    const double xadd = (double)a.x_add;
    v4d acc[WM];
#pragma unroll
    for (int i = 0; i < WM; ++i) acc[i] = v4d{0.0, 0.0, 0.0, 0.0};
    for (int ky = 0; ky < a.KH; ++ky) {
        const int iy = pos.oy * a.SH - a.PH + ky * a.DH;
        for (int kx = 0; kx < a.KW; ++kx) {
            const int ix = pos.ox * a.SW - a.PW + kx * a.DW;
            const bool in =
                (unsigned)iy < (unsigned)a.H && (unsigned)ix < (unsigned)a.W;
            const int16_t* px =
                xn + (in ? ((int64_t)iy * a.W + ix) * a.x_sp : 0);
            const double* wt = wrow + (int64_t)(ky * a.KW + kx) * a.CK;
            for (int cc = 0; cc < nck; ++cc) {
                // channels 4V*cc + V*kgl + j of the lane's pixel
                const bool live = in && 4 * V * cc + V * kgl < a.Cg;
                VT xv;
                if (live)
                    xv = *(const VT*)(px + 4 * V * cc);
                double av[V];
#pragma unroll
                for (int j = 0; j < V; ++j)
                    av[j] = live ? (double)VecI16<V>::get(xv, j) + xadd : 0.0;
#pragma unroll
                for (int i = 0; i < WM; ++i) {
                    const double* w = wt + i * wblk + 4 * V * cc;
                    double bw[V];
                    if (V == 1) {
                        bw[0] = w[0];
                    } else {
#pragma unroll
                        for (int j = 0; j < V; j += 2) {
                            const double2 t = *(const double2*)(w + j);
                            bw[j] = t.x;
                            bw[j + 1] = t.y;
                        }
                    }
#pragma unroll
                    for (int j = 0; j < V; ++j)
                        acc[i] = __builtin_amdgcn_mfma_f64_16x16x4f64(
                            av[j], bw[j], acc[i], 0, 0, 0);
                }
            }
        }
    }
    // epilogue: the exact sums of the lane's pixels 4r + kgl
#pragma unroll
    for (int i = 0; i < WM; ++i) {
        const int c = co0 + i * 16 + col;
        if (c >= a.Cog) continue;
        const int64_t co = (int64_t)g * a.Cog + c;
        const int64_t pre = a.pre ? a.pre[co] : 0;
        const int64_t m = a.mode == EPI_QUANT ? a.mult[co] : 0;
        const int64_t s = a.mode == EPI_QUANT ? a.shift[co] : 0;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t pp = tile * 16 + 4 * r + kgl;
            if (pp >= a.M) continue;
            const int64_t sum = (int64_t)acc[i][r];
            const int64_t v = a.wide ? sum : (int64_t)(int32_t)sum;
            const PixPos op = pix_decode(a, pp);
            const int64_t pix = (int64_t)op.oy * a.OW + op.ox;
            const int64_t yi = (int64_t)op.n * a.y_sn + co * a.y_sc +
                               pix * a.y_sp;
            if (a.mode != EPI_QUANT) {
                store_any(a.y, a.y_code, yi, v);
                continue;
            }
            int64_t rq = 0;
            if (a.res)
                rq = load_any(a.res, a.y_code,
                              (int64_t)op.n * a.res_sn + co * a.res_sc +
                                  pix * a.res_sp) +
                     a.res_so;
            const int64_t q = quant_one(a, v + pre, m, s, rq);
            store_any(a.y, a.y_code, yi, q - a.y_so);
            if (a.y2)
                store_any(a.y2, a.y_code,
                          (int64_t)op.n * a.y2_sn + co * a.y2_sc +
                              pix * a.y2_sp,
                          rescale2(a, q) - a.y_so);
        }
    }
}

template <int WM>
void launch_v(const ConvArgs& a, int v, dim3 grid, hipStream_t st) {
    switch (v) {
        case 8: k_conv_f64<WM, 8><<<grid, 256, 0, st>>>(a); break;
        case 4: k_conv_f64<WM, 4><<<grid, 256, 0, st>>>(a); break;
        case 2: k_conv_f64<WM, 2><<<grid, 256, 0, st>>>(a); break;
        default: k_conv_f64<WM, 1><<<grid, 256, 0, st>>>(a); break;
    }
}

}  // namespace

bool launch_conv_f64(const ConvArgs& a, hipStream_t st) {
    if (a.M <= 0 || a.Cog <= 0) return true;
    if (a.x_code != 2 || a.x_sc != 1 || a.narrow16 || a.M >= ((int64_t)1 << 31) ||
        a.CK != ((a.Cg + 31) & ~31) || a.wf_rows % 64 ||
        a.wf_rows < a.Cog || a.x_add < -65536 || a.x_add > 65536 ||
        (int64_t)a.KH * a.KW * a.CK >= ((int64_t)1 << 19) || a.G > 65535) {
        set_error("launch_conv_f64",
                  "needs int16 channels-last activations, weights packed by "
                  "qa_pack_weights_f64 and K below 2^19");
        return false;
    }
    // channels per lane vector: the widest that divides the channel count,
    // the strides and the address, without more K-padding than 4 channels
    const uintptr_t xa = (uintptr_t)a.x;
    const int64_t cg4 = (a.Cg + 3) & ~3;
    int v = 8;
    while (v > 1 &&
           (a.Cg % v || a.x_sn % v || a.x_sp % v || xa % (2 * v) ||
            ((a.Cg + 4 * v - 1) / (4 * v)) * 4 * v != cg4))
        v >>= 1;
    // channel block: as wide as keeps 4 waves per SIMD of every CU busy
    const int64_t ntiles = ceil_div(a.M, 16);
    const int64_t want = 16 * (int64_t)cu_count();
    int wm = a.Cog <= 16 ? 1 : (a.Cog <= 32 ? 2 : 4);
    if (a.tile_hint & TILE_VALID) {
        const int h = a.tile_hint & 0xff;
        if (h == 1 || h == 2 || h == 4) wm = h;
    } else {
        while (wm > 1 && ntiles * ceil_div(a.Cog, 16 * wm) * a.G < want)
            wm >>= 1;
    }
    const int64_t gx = ceil_div(ntiles, 4);
    const int64_t gy = ceil_div(a.Cog, 16 * wm);
    if (gx >= ((int64_t)1 << 31) || gy > 65535) {
        set_error("launch_conv_f64", "grid too large");
        return false;
    }
    const dim3 grid((unsigned)gx, (unsigned)gy, (unsigned)a.G);
    switch (wm) {
        case 1: launch_v<1>(a, v, grid, st); break;
        case 2: launch_v<2>(a, v, grid, st); break;
        default: launch_v<4>(a, v, grid, st); break;
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_hip_error("launch_conv_f64", e);
        return false;
    }
    return true;
}

}  // namespace qa

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
// A wave owns TM tiles of 16 output pixels (batch folded in; rows of the
// MFMA) x WM*16 output channels (columns), so each weight fragment it loads
// serves TM tiles and each activation fragment WM channel groups. K runs in
// steps of one tap x 4V input channels: lane (pixel col, group q) loads the V
// consecutive channels 4V*cc + V*q .. + V-1 of its pixel as one vector, and
// MFMA j (j < V) sums channels {4V*cc + V*q + j : q = 0..3}. The fragments
// of the next D steps are in flight while a step's MFMAs run. Channels past Cg
// meet zero weights (weights are packed as double rows [group][channel,
// padded to 64][tap][Cg padded to 32], zero-filled) and are loaded as 0, so
// every access stays inside the input. With KSPLIT the 4 waves of a
// work-group share their tiles and take every 4th K-step; the partial sums
// are added through LDS and each wave finishes a quarter of the outputs.
// The MFMA's result register r of lane l is output row 4r + l/16, column
// l%16.
#include <type_traits>

#include "qa_conv_mfma.h"

namespace qa {
namespace {

typedef double v4d __attribute__((ext_vector_type(4)));

// V consecutive int16 or int32 elements loaded as one fragment.
template <int V, class E>
struct Frag;
template <>
struct Frag<1, int16_t> {
    typedef int16_t T;
    static __device__ __forceinline__ int get(const T& v, int) { return v; }
};
template <>
struct Frag<4, int16_t> {
    typedef int2 T;
    static __device__ __forceinline__ int get(const T& v, int j) {
        const int w = j < 2 ? v.x : v.y;
        return (int)(int16_t)(w >> (16 * (j & 1)));
    }
};
template <>
struct Frag<8, int16_t> {
    typedef int4 T;
    static __device__ __forceinline__ int get(const T& v, int j) {
        const int w = j < 2 ? v.x : (j < 4 ? v.y : (j < 6 ? v.z : v.w));
        return (int)(int16_t)(w >> (16 * (j & 1)));
    }
};
template <>
struct Frag<1, int32_t> {
    typedef int T;
    static __device__ __forceinline__ int get(const T& v, int) { return v; }
};
template <>
struct Frag<4, int32_t> {
    typedef int4 T;
    static __device__ __forceinline__ int get(const T& v, int j) {
        return j == 0 ? v.x : (j == 1 ? v.y : (j == 2 ? v.z : v.w));
    }
};
struct I32x8 {
    int4 lo, hi;
};
template <>
struct Frag<8, int32_t> {
    typedef I32x8 T;
    static __device__ __forceinline__ int get(const T& v, int j) {
        return Frag<4, int32_t>::get(j < 4 ? v.lo : v.hi, j & 3);
    }
};

// Position of a K-step: tap (ky, kx) and channel chunk cc.
struct KPos {
    int ky, kx, cc;
};

// Advances by `by` (1 or 4) steps; branch-free, so that the load counters
// of the ring below stay countable.
template <int BY>
__device__ __forceinline__ void kpos_advance(const ConvArgs& a, int nck,
                                             KPos& k) {
    k.cc += BY;
#pragma unroll
    for (int r = 0; r < BY; ++r) {
        const bool wrap = k.cc >= nck;
        k.cc -= wrap ? nck : 0;
        const bool row = wrap && k.kx + 1 == a.KW;
        k.kx = row ? 0 : k.kx + (wrap ? 1 : 0);
        k.ky += row ? 1 : 0;
    }
}

// One output element of the exact sum `sum` (mode EPI_QUANT or raw).
__device__ __forceinline__ void f64_store(const ConvArgs& a, int64_t co,
                                          int64_t pp, int64_t sum,
                                          int64_t pre, int64_t m, int64_t s) {
    const int64_t v = a.wide ? sum : (int64_t)(int32_t)sum;
    // element indices of y, the residual and the copy: pixel * pixel stride
    // + channel when all are dense channels-last (fastio), else decoded
    int64_t yi, ri, y2i;
    if (a.fastio) {
        yi = pp * a.y_pst + co;
        ri = pp * a.res_pst + co;
        y2i = pp * a.y2_pst + co;
    } else {
        const PixPos op = pix_decode(a, pp);
        const int64_t pix = (int64_t)op.oy * a.OW + op.ox;
        yi = (int64_t)op.n * a.y_sn + co * a.y_sc + pix * a.y_sp;
        ri = (int64_t)op.n * a.res_sn + co * a.res_sc + pix * a.res_sp;
        y2i = (int64_t)op.n * a.y2_sn + co * a.y2_sc + pix * a.y2_sp;
    }
    if (a.mode != EPI_QUANT) {
        store_any(a.y, a.y_code, yi, v);
        return;
    }
    int64_t rq = 0;
    if (a.res) rq = load_any(a.res, a.y_code, ri) + a.res_so;
    const int64_t q = quant_one(a, v + pre, m, s, rq);
    store_any(a.y, a.y_code, yi, q - a.y_so);
    if (a.y2) store_any(a.y2, a.y_code, y2i, rescale2(a, q) - a.y_so);
}

// The 128-bit requantization of one value (out of line: the float64 form
// below hands it the rare values it cannot decide).
__device__ __noinline__ int64_t requant_exact(int64_t x, int64_t m, int64_t s,
                                              int64_t zp, int64_t lo,
                                              int64_t hi) {
    return qa_clip128(qa_mbqm_fast(x, m, s) + zp, lo, hi);
}

// Exact float64 forms of the fixed-point multiplies of the 16-bit epilogue
// (qa_mbqm: floor(x m 2^-ts + 1/2), ts = 31 + shift):
//  * requantize, |x| < 2^53, |m| < 2^31, 1 <= ts <= 120, clip bounds within
//    2^19: y = fma(x, m 2^-ts, 1/2 + zp) is one rounding of the exact value
//    (x and m 2^-ts are exact doubles), |error| <= 2^-52 |y|; below |y| =
//    2^20, floor(y) is the exact result unless frac(y) lies within 2^-30 of
//    0 or 1 (those values take requant_exact); above, the clip gives the
//    same bound either way.
//  * multiplies of a clipped value (|d| < 2^20) by |m| < 2^31 with 1 <= ts
//    <= 53 (the residual Add, the rescaled copy): d m is an exact double
//    below 2^51, and so is d m 2^-ts + 1/2, so floor gives the exact result.
struct MulD {
    double md;
    bool ok;
};
__device__ __forceinline__ MulD mul_d(int64_t m, int64_t shift, int64_t tmax) {
    const int64_t ts = 31 + shift;
    MulD r;
    r.ok = ts >= 1 && ts <= tmax && m > -((int64_t)1 << 31) &&
           m < ((int64_t)1 << 31);
    r.md = r.ok ? ldexp((double)m, -(int)ts) : 0.0;
    return r;
}
__device__ __forceinline__ double round_d(double d, double md) {
    return floor(fma(d, md, 0.5));
}
__device__ __forceinline__ double clamp_d(double v, int64_t lo, int64_t hi) {
    return fmin(fmax(v, (double)lo), (double)hi);
}

// The epilogue of NV exact sums v[j] of one output channel co at pixels
// pp[j] (skipped at or past M) for int16 outputs (mode EPI_QUANT, dense
// channels-last y / residual / copy): every value's table read and
// residual read is issued before the first of them is used and before the
// first store (one at a time they would each wait a memory round trip);
// the multiplies in their float64 forms where those apply. RES / Y2: a
// residual Add / a rescaled copy (compile-time, so that a launch without
// them holds none of their constants).
template <int NV, bool RES = true, bool Y2 = true>
__device__ __forceinline__ void epi16_batch(const ConvArgs& a, int64_t co,
                                            const int64_t (&pp)[NV],
                                            const int64_t (&v)[NV],
                                            int64_t pre, int64_t m,
                                            int64_t s) {
    constexpr int64_t B19 = (int64_t)1 << 19, B20 = (int64_t)1 << 20;
    const MulD rq = mul_d(m, s, 120);
    const bool fast = rq.ok && a.qmin > -B19 && a.qmax < B19;
    const double c0 = 0.5 + (double)a.zp;
    const MulD ra = mul_d(a.ma, a.sa, 53), rb = mul_d(a.mb, a.sb, 53);
    const bool rfast = ra.ok && rb.ok && (a.add_sign == 1 || a.add_sign == -1) &&
                       a.za > -B20 && a.za < B20 && a.zb > -B20 &&
                       a.zb < B20 && a.res_so > -B20 && a.res_so < B20 &&
                       a.qmin > -B19 && a.qmax < B19;
    const MulD r2 = mul_d(a.r2_m, a.r2_s, 53);
    const bool r2fast = r2.ok && a.r2_zp_in > -B20 && a.r2_zp_in < B20;
    int64_t q[NV];
    int32_t lv[NV];
    int32_t rv[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int64_t p = min(pp[j], a.M - 1);  // in bounds, unused past M
        const int64_t x = (a.wide ? v[j] : (int64_t)(int32_t)v[j]) + pre;
        bool slow = !fast || x >= ((int64_t)1 << 53) ||
                    x <= -((int64_t)1 << 53);
        const double y = fma((double)x, rq.md, c0);
        const double f = floor(y);
        const double fr = y - f;
        slow = slow || ((fr < 0x1p-30 || fr > 1.0 - 0x1p-30) &&
                        fabs(y) < 0x1p20);
        q[j] = slow ? requant_exact(x, m, s, a.zp, a.qmin, a.qmax)
                    : (int64_t)clamp_d(f, a.qmin, a.qmax);
        lv[j] = 0;
        rv[j] = 0;
        if (a.lut) lv[j] = a.lut[lut_index(a, q[j])];
        if (RES && a.res)
            rv[j] = ((const int16_t*)a.res)[p * a.res_pst + co];
    }
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        if (pp[j] >= a.M) continue;
        int64_t qq = a.lut ? (int64_t)lv[j] : q[j];
        if (RES && a.res) {
            const int64_t r = (int64_t)rv[j] + a.res_so;
            if (rfast && qq > -B19 && qq < B19) {
                const int64_t first = a.res_first ? r : qq;
                const int64_t second = a.res_first ? qq : r;
                const double t =
                    round_d((double)(first - a.za), ra.md) +
                    (double)a.add_sign *
                        round_d((double)(second - a.zb), rb.md) +
                    (double)a.add_zp;
                qq = (int64_t)clamp_d(t, a.add_qmin, a.add_qmax);
            } else {
                qq = quant_add(a, qq, r);
            }
        }
        ((int16_t*)a.y)[pp[j] * a.y_pst + co] = (int16_t)(qq - a.y_so);
        if (Y2 && a.y2) {
            const int64_t c =
                r2fast && qq > -B19 && qq < B19
                    ? (int64_t)clamp_d(round_d((double)(qq - a.r2_zp_in),
                                               r2.md) +
                                           (double)a.r2_zp_out,
                                       a.r2_qmin, a.r2_qmax)
                    : rescale2(a, qq);
            ((int16_t*)a.y2)[pp[j] * a.y2_pst + co] = (int16_t)(c - a.y_so);
        }
    }
}

template <int WM, int TM, int V, bool KSPLIT, class WE>
__global__ __launch_bounds__(256) void k_conv_f64(ConvArgs a) {
    typedef Frag<V, int16_t> XF;
    typedef Frag<V, WE> WF;
    typedef typename XF::T VT;
    typedef typename WF::T WT;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int col = lane & 15, kgl = lane >> 4;
    const int g = blockIdx.z;
    const int co0 = blockIdx.y * WM * 16;
    const int64_t tile0 =
        ((int64_t)blockIdx.x * (KSPLIT ? 1 : 4) + (KSPLIT ? 0 : wave)) * TM;
    if (tile0 * 16 >= a.M) return;  // uniform per work-group with KSPLIT
    const int taps = a.KH * a.KW;
    const int nck = (a.Cg + 4 * V - 1) / (4 * V);
    const int nsteps_all = taps * nck;
    // this wave's K-steps: all, or every 4th from `wave`
    const int kfirst = KSPLIT ? wave : 0;
    const int nsteps =
        KSPLIT ? (nsteps_all > wave ? (nsteps_all - wave + 3) / 4 : 0)
               : nsteps_all;
    // fetch side of the lane's TM pixels (clamped into the tensor)
    const int16_t* xb[TM];
    int iy0[TM], ix0[TM];
#pragma unroll
    for (int t = 0; t < TM; ++t) {
        const int64_t p = min((tile0 + t) * 16 + col, a.M - 1);
        const PixPos pos = pix_decode(a, p);
        xb[t] = (const int16_t*)a.x + (int64_t)pos.n * a.x_sn +
                (int64_t)g * a.Cg + V * kgl;
        iy0[t] = pos.oy * a.SH - a.PH;
        ix0[t] = pos.ox * a.SW - a.PW;
    }
    const WE* wrow = (const WE*)a.wf +
                     ((int64_t)g * a.wf_rows + co0 + col) * taps * a.CK +
                     V * kgl;
    const int64_t wblk = (int64_t)16 * taps * a.CK;  // the next 16 channels
    const double xadd = (double)a.x_add;

    // a ring of D K-steps in flight: slot d holds the fragments of step
    // n0 + d. Loads are issued for every lane (padding and channels past Cg
    // read the image's first element, a valid address, and are masked at
    // use), so the compiler can count them without branches.
    constexpr int D = V == 1 ? 4 : 2;
    VT xr[D][TM];
    bool lr[D][TM];
    WT wr[D][WM];
    KPos kf;  // the next step to fetch
    kf.ky = 0;
    kf.kx = 0;
    kf.cc = 0;
    for (int r = 0; r < kfirst; ++r) kpos_advance<1>(a, nck, kf);
    auto fetch = [&](VT (&xo)[TM], bool (&lo)[TM], WT (&bo)[WM]) {
        const bool chan = 4 * V * kf.cc + V * kgl < a.Cg;
#pragma unroll
        for (int t = 0; t < TM; ++t) {
            const int iy = iy0[t] + kf.ky * a.DH;
            const int ix = ix0[t] + kf.kx * a.DW;
            lo[t] = chan && (unsigned)iy < (unsigned)a.H &&
                    (unsigned)ix < (unsigned)a.W;
            const int64_t off =
                lo[t] ? ((int64_t)iy * a.W + ix) * a.x_sp + 4 * V * kf.cc
                      : -(int64_t)(V * kgl);
            xo[t] = *(const VT*)(xb[t] + off);
        }
        // steps past the end (ky == KH onwards) read tap 0: in bounds
        const int tap = kf.ky < a.KH ? kf.ky * a.KW + kf.kx : 0;
        const WE* wt = wrow + (int64_t)tap * a.CK + 4 * V * kf.cc;
#pragma unroll
        for (int i = 0; i < WM; ++i) bo[i] = *(const WT*)(wt + i * wblk);
        kpos_advance<KSPLIT ? 4 : 1>(a, nck, kf);
    };
    v4d acc[TM][WM];
#pragma unroll
    for (int t = 0; t < TM; ++t)
#pragma unroll
        for (int i = 0; i < WM; ++i) acc[t][i] = v4d{0.0, 0.0, 0.0, 0.0};
    auto compute = [&](const VT (&xv)[TM], const bool (&lv)[TM],
                       const WT (&bw)[WM]) {
#pragma unroll
        for (int t = 0; t < TM; ++t) {
            double av[V];
#pragma unroll
            for (int j = 0; j < V; ++j)
                av[j] = lv[t] ? (double)XF::get(xv[t], j) + xadd : 0.0;
#pragma unroll
            for (int j = 0; j < V; ++j)
#pragma unroll
                for (int i = 0; i < WM; ++i)
                    acc[t][i] = __builtin_amdgcn_mfma_f64_16x16x4f64(
                        av[j], (double)WF::get(bw[i], j), acc[t][i], 0, 0,
                        0);
        }
    };
    // every fetch is issued (steps past the end read in-bounds addresses
    // and are not used): no load sits behind a branch
#pragma unroll
    for (int d = 0; d < D; ++d) fetch(xr[d], lr[d], wr[d]);
    for (int n0 = 0; n0 < nsteps; n0 += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            if (n0 + d < nsteps) compute(xr[d], lr[d], wr[d]);
            fetch(xr[d], lr[d], wr[d]);
        }
    }

    if (KSPLIT) {
        // partial sums through LDS; wave w finishes row register r = w
        __shared__ double s_acc[4][WM][4][64];
#pragma unroll
        for (int i = 0; i < WM; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) s_acc[wave][i][r][lane] = acc[0][i][r];
        __syncthreads();
#pragma unroll
        for (int i = 0; i < WM; ++i) {
            const double sum = s_acc[0][i][wave][lane] +
                               s_acc[1][i][wave][lane] +
                               s_acc[2][i][wave][lane] +
                               s_acc[3][i][wave][lane];
            const int c = co0 + i * 16 + col;
            const int64_t pp = tile0 * 16 + 4 * wave + kgl;
            if (c >= a.Cog || pp >= a.M) continue;
            const int64_t co = (int64_t)g * a.Cog + c;
            const bool q = a.mode == EPI_QUANT;
            f64_store(a, co, pp, (int64_t)sum, a.pre ? a.pre[co] : 0,
                      q ? a.mult[co] : 0, q ? a.shift[co] : 0);
        }
        return;
    }
    // the exact sums of the lane's pixels 4r + kgl of each tile
#pragma unroll
    for (int i = 0; i < WM; ++i) {
        const int c = co0 + i * 16 + col;
        if (c >= a.Cog) continue;
        const int64_t co = (int64_t)g * a.Cog + c;
        const bool q = a.mode == EPI_QUANT;
        const int64_t pre = a.pre ? a.pre[co] : 0;
        const int64_t m = q ? a.mult[co] : 0;
        const int64_t s = q ? a.shift[co] : 0;
        if (q && a.fastio && a.y_code == 2) {
            int64_t pp[TM * 4], v[TM * 4];
#pragma unroll
            for (int t = 0; t < TM; ++t)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    pp[4 * t + r] = (tile0 + t) * 16 + 4 * r + kgl;
                    v[4 * t + r] = (int64_t)acc[t][i][r];
                }
            epi16_batch(a, co, pp, v, pre, m, s);
            continue;
        }
#pragma unroll
        for (int t = 0; t < TM; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t pp = (tile0 + t) * 16 + 4 * r + kgl;
                if (pp < a.M)
                    f64_store(a, co, pp, (int64_t)acc[t][i][r], pre, m, s);
            }
    }
}

// ---- the byte-split form: 16-bit convolution on the int8 matrix cores --
//
// A stored activation x (int16) is 256 xh + xl + 128 with xh = x >> 8 and
// xl = (x & 255) - 128, both int8, and a centred weight w = 256 wh + wl +
// 128 likewise (qa_pack_weights_i16s: planes of wh and wl, w = 0 where no
// weight sits). Over the K' positions one output sums (the 16 KGp bytes of
// a packed row; positions without a weight have w = 0, so whatever x they
// hold cancels):
//   sum (x + x_add) w = 65536 Hh + 256 (Hl + Lh) + Ll + 128 U
//                       + (128 + x_add) W
// with Hh = sum xh wh, Hl = sum xh wl, Lh = sum xl wh, Ll = sum xl wl (int8
// MFMA sums: |Hh| <= 2^14 K', |Hl + Lh| <= 2^15 K', exact in int32 for K' <
// 2^16), U = sum (256 xh + xl) (two MFMAs against all-ones columns, which
// leave each pixel's sum in the accumulator layout) and W = sum w (ws_k
// holds (128 + x_add) W). Image padding positions hold the stored zero
// point -x_add (x + x_add = 0). The exact int64 sum then takes the FP64
// path's epilogue. A wave owns TM tiles of 16 pixels (rows) x WM 16-channel
// blocks (columns); a lane's K-values of a step are the 16 channels of
// k-group 4 s + lane / 16 (32 bytes of int16, split with v_perm), loaded
// straight from memory with the next step's loads in flight. NARROW (at
// most 4 channels, stored 4 a pixel: the image stem): a lane loads its
// pixel's 8 bytes and the group's other 12 positions hold 0 (their weights
// are 0).
// EPI: 0 the general per-element epilogue (f64_store); else the int16 form
// (mode EPI_QUANT, dense channels-last y), bit 1 with a residual Add, bit 2
// with a rescaled copy.
template <int WM, int TM, bool NARROW, int EPI>
__global__ __launch_bounds__(256) void k_conv_bs(ConvArgs a) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int col = lane & 15, kgl = lane >> 4;
    const int g = blockIdx.z;
    const int co0 = blockIdx.y * WM * 16;
    const int64_t tile0 = ((int64_t)blockIdx.x * 4 + wave) * TM;
    // per k-group, built once per work-group: the element offset of its
    // 16 channels from the tap's input pixel (-1: no tap, the k-group pads
    // K) and the tap's displacement dy << 16 | dx (the host keeps both
    // below 2^31 and 2^15)
    extern __shared__ int2 s_kt[];
    for (int kg = threadIdx.x; kg < a.KGp; kg += 256) {
        int2 e = {-1, 0};
        if (kg < a.KG) {
            const int tap = kg / a.CB, cb = kg - tap * a.CB;
            const int ky = tap / a.KW, kx = tap - ky * a.KW;
            e.x = (ky * a.DH * a.W + kx * a.DW) * (int)a.x_sp + 16 * cb;
            e.y = (ky * a.DH) << 16 | (kx * a.DW);
        }
        s_kt[kg] = e;
    }
    __syncthreads();
    if (tile0 * 16 >= a.M) return;
    const int nsteps = a.KGp >> 2;
    const int16_t* xb[TM];
    int iy0[TM], ix0[TM], pb[TM];
#pragma unroll
    for (int t = 0; t < TM; ++t) {
        const int64_t p = min((tile0 + t) * 16 + col, a.M - 1);
        const PixPos pos = pix_decode(a, p);
        xb[t] = (const int16_t*)a.x + (int64_t)pos.n * a.x_sn +
                (int64_t)g * a.Cg;
        iy0[t] = pos.oy * a.SH - a.PH;
        ix0[t] = pos.ox * a.SW - a.PW;
        pb[t] = (iy0[t] * a.W + ix0[t]) * (int)a.x_sp;  // may be < 0
    }
    // the lane's weight row (channel co0 + 16 i + col) in the high plane;
    // the low plane G groups further
    const int8_t* wrow = a.ws + (int64_t)g * a.wp_gstride +
                         (int64_t)(co0 + col) * a.wp_rstride + 16 * kgl;
    const int64_t lo_off = (int64_t)a.G * a.wp_gstride;
    const int64_t wblk = 16 * a.wp_rstride;
    // the stored zero point's bytes, as four copies
    const int pz = (int)(-a.x_add);
    const int ph = (int)(((uint32_t)(pz >> 8) & 255u) * 0x01010101u);
    const int pl = (int)((((uint32_t)pz & 255u) ^ 0x80u) * 0x01010101u);
    const v4i ones = {0x01010101, 0x01010101, 0x01010101, 0x01010101};

    constexpr int D = 2;  // steps in flight
    int4 xr[D][TM][2];
    bool xin[D][TM];
    v4i whr[D][WM], wlr[D][WM];
    auto fetch = [&](int d, int s) {
        s = min(s, nsteps - 1);  // steps past the end: in bounds, unused
        const int2 e = s_kt[4 * s + kgl];
        const int dy = e.y >> 16, dx = e.y & 0xffff;
#pragma unroll
        for (int t = 0; t < TM; ++t) {
            const int iy = iy0[t] + dy, ix = ix0[t] + dx;
            const bool in = e.x >= 0 && (unsigned)iy < (unsigned)a.H &&
                            (unsigned)ix < (unsigned)a.W;
            // outside: the image's first pixel (in bounds, not used)
            const int off = in ? pb[t] + e.x : 0;
            if (NARROW) {
                const int2 u = *(const int2*)(xb[t] + off);
                xr[d][t][0] = int4{u.x, u.y, 0, 0};
                xr[d][t][1] = int4{0, 0, 0, 0};
            } else {
                xr[d][t][0] = *(const int4*)(xb[t] + off);
                xr[d][t][1] = *(const int4*)(xb[t] + off + 8);
            }
            xin[d][t] = in;
        }
#pragma unroll
        for (int i = 0; i < WM; ++i) {
            const int8_t* wp = wrow + i * wblk + 64 * s;
            whr[d][i] = *(const v4i*)wp;
            wlr[d][i] = *(const v4i*)(wp + lo_off);
        }
    };
    v4i hh[TM][WM], md[TM][WM], ll[TM][WM], sh[TM], sl[TM];
#pragma unroll
    for (int t = 0; t < TM; ++t) {
        sh[t] = sl[t] = v4i{0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < WM; ++i)
            hh[t][i] = md[t][i] = ll[t][i] = v4i{0, 0, 0, 0};
    }
    auto compute = [&](int d) {
#pragma unroll
        for (int t = 0; t < TM; ++t) {
            // int16 channels 2j (low half) and 2j + 1 of dword j: the high
            // bytes are bytes 1 and 3 of each dword, the low bytes 0 and 2
            const int4 u = xr[d][t][0], w = xr[d][t][1];
            v4i xh = {(int)__builtin_amdgcn_perm(u.y, u.x, 0x07050301u),
                      (int)__builtin_amdgcn_perm(u.w, u.z, 0x07050301u),
                      (int)__builtin_amdgcn_perm(w.y, w.x, 0x07050301u),
                      (int)__builtin_amdgcn_perm(w.w, w.z, 0x07050301u)};
            v4i xl = {(int)__builtin_amdgcn_perm(u.y, u.x, 0x06040200u),
                      (int)__builtin_amdgcn_perm(u.w, u.z, 0x06040200u),
                      (int)__builtin_amdgcn_perm(w.y, w.x, 0x06040200u),
                      (int)__builtin_amdgcn_perm(w.w, w.z, 0x06040200u)};
            xl ^= (int)0x80808080u;
            if (!xin[d][t]) {
                xh = v4i{ph, ph, ph, ph};
                xl = v4i{pl, pl, pl, pl};
            }
#pragma unroll
            for (int i = 0; i < WM; ++i) {
                hh[t][i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                    xh, whr[d][i], hh[t][i], 0, 0, 0);
                md[t][i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                    xh, wlr[d][i], md[t][i], 0, 0, 0);
                md[t][i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                    xl, whr[d][i], md[t][i], 0, 0, 0);
                ll[t][i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                    xl, wlr[d][i], ll[t][i], 0, 0, 0);
            }
            sh[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(xh, ones, sh[t], 0,
                                                          0, 0);
            sl[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(xl, ones, sl[t], 0,
                                                          0, 0);
        }
    };
#pragma unroll
    for (int d = 0; d < D; ++d) fetch(d, d);
    for (int n0 = 0; n0 < nsteps; n0 += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            if (n0 + d < nsteps) compute(d);
            fetch(d, n0 + d + D);
        }
    }
    // result register r of lane (col, kgl): pixel 4 kgl + r of the tile,
    // channel col of the block
#pragma unroll
    for (int i = 0; i < WM; ++i) {
        const int c = co0 + i * 16 + col;
        if (c >= a.Cog) continue;
        const int64_t co = (int64_t)g * a.Cog + c;
        const bool q = a.mode == EPI_QUANT;
        const int64_t pre = a.pre ? a.pre[co] : 0;
        const int64_t m = q ? a.mult[co] : 0;
        const int64_t sft = q ? a.shift[co] : 0;
        const int64_t kc = a.ws_k[co];
        int64_t pp[TM * 4], v[TM * 4];
#pragma unroll
        for (int t = 0; t < TM; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t u = (int64_t)sh[t][r] * 256 + sl[t][r];
                pp[4 * t + r] = (tile0 + t) * 16 + 4 * kgl + r;
                v[4 * t + r] = (int64_t)hh[t][i][r] * 65536 +
                               (int64_t)md[t][i][r] * 256 + ll[t][i][r] +
                               u * 128 + kc;
            }
        if constexpr (EPI != 0) {
            epi16_batch<TM * 4, (EPI & 2) != 0, (EPI & 4) != 0>(a, co, pp, v,
                                                              pre, m, sft);
        } else {
#pragma unroll
            for (int j = 0; j < TM * 4; ++j)
                if (pp[j] < a.M) f64_store(a, co, pp[j], v[j], pre, m, sft);
        }
    }
}

template <int WM, int TM, bool KS, class WE>
void launch_v(const ConvArgs& a, int v, dim3 grid, hipStream_t st) {
    switch (v) {
        case 8: k_conv_f64<WM, TM, 8, KS, WE><<<grid, 256, 0, st>>>(a); break;
        case 4: k_conv_f64<WM, TM, 4, KS, WE><<<grid, 256, 0, st>>>(a); break;
        default:
            k_conv_f64<WM, TM, 1, KS, WE><<<grid, 256, 0, st>>>(a);
            break;
    }
}

template <int WM, int TM, bool KS>
void launch_w(const ConvArgs& a, int v, dim3 grid, hipStream_t st) {
    if (a.wf_bytes == 2)
        launch_v<WM, TM, KS, int16_t>(a, v, grid, st);
    else
        launch_v<WM, TM, KS, int32_t>(a, v, grid, st);
}

struct F64Tile {
    int wm, tm;
    bool split;
};

// Tile code: wm | tm << 4 | split << 8 (also the low bits of a tile hint).
constexpr int f64_code(const F64Tile& t) {
    return t.wm | t.tm << 4 | (t.split ? 0x100 : 0);
}

constexpr F64Tile kF64Tiles[] = {
    {1, 1, false}, {2, 1, false}, {1, 4, false},
    {1, 1, true},  {2, 1, true},  {4, 1, true},
};

}  // namespace

bool launch_conv_f64(const ConvArgs& a, hipStream_t st) {
    if (a.M <= 0 || a.Cog <= 0) return true;
    if (a.x_code != 2 || a.x_sc != 1 || a.narrow16 || a.Cg < 1 ||
        a.M >= ((int64_t)1 << 31) || a.CK != ((a.Cg + 31) & ~31) ||
        a.wf_rows % 64 || a.wf_rows < a.Cog ||
        (a.wf_bytes != 2 && a.wf_bytes != 4) || a.x_add < -65536 ||
        a.x_add > 65536 ||
        (int64_t)a.KH * a.KW * a.CK >= ((int64_t)1 << 19) || a.G > 65535) {
        set_error("launch_conv_f64",
                  "needs int16 channels-last activations, weights packed by "
                  "qa_pack_weights_f64 and K below 2^19");
        return false;
    }
    // channels per lane vector: 8 or 4 when they divide the channel count,
    // the strides and the address without more K-padding than 4 channels
    const uintptr_t xa = (uintptr_t)a.x;
    const int64_t cg4 = (a.Cg + 3) & ~3;
    int v = 8;
    while (v > 1 &&
           (a.Cg % v || a.x_sn % v || a.x_sp % v || xa % (2 * v) ||
            ((a.Cg + 4 * v - 1) / (4 * v)) * 4 * v != cg4))
        v = v == 8 ? 4 : 1;
    ConvArgs b = a;
    {
        // dense channels-last y (residual, copy): element of pixel p and
        // channel c at p * pixel stride + c (a GEMM row is one pixel)
        const int64_t ohw = (int64_t)a.OH * a.OW;
        auto pst = [&](int64_t sn, int64_t sp) { return ohw == 1 ? sn : sp; };
        auto dense = [&](const void* p, int64_t sn, int64_t sc, int64_t sp) {
            return p == nullptr || (sc == 1 && (ohw == 1 || sn == ohw * sp));
        };
        b.fastio = dense(a.y, a.y_sn, a.y_sc, a.y_sp) &&
                   dense(a.res, a.res_sn, a.res_sc, a.res_sp) &&
                   dense(a.y2, a.y2_sn, a.y2_sc, a.y2_sp);
        b.y_pst = pst(a.y_sn, a.y_sp);
        b.res_pst = pst(a.res_sn, a.res_sp);
        b.y2_pst = pst(a.y2_sn, a.y2_sp);
    }
    const int64_t ntiles = ceil_div(a.M, 16);
    // the byte-split form on the int8 matrix cores: when the split planes
    // are given and the input fits it (16-byte aligned 16-channel groups,
    // K' = 16 KGp < 2^16, the stored zero point an int16); tile code 0x1000
    // | wm | tm << 4, by default the widest channel block, one tile a wave
    // narrow: at most 4 channels in 8-byte aligned 4-channel pixels
    const bool narrow = a.Cg <= 4 && a.G == 1 && a.x_sp % 4 == 0 &&
                        a.x_sn % 4 == 0 && xa % 8 == 0;
    if (a.ws && a.ws_k &&
        ((a.Cg % 16 == 0 && a.x_sp % 8 == 0 && a.x_sn % 8 == 0 &&
          xa % 16 == 0) ||
         narrow) &&
        a.KGp > 0 && a.KGp < 4096 && a.x_add >= -32767 &&
        a.x_add <= 32768 &&
        // the k-group table's int32 offsets, displacements below 2^15 and
        // every pixel base of the padded extent in int32
        (int64_t)(a.H + a.PH + a.KH * a.DH + a.SH) *
                (a.W + a.PW + a.KW * a.DW + a.SW) * a.x_sp +
                16 * (int64_t)a.CB < ((int64_t)1 << 31) &&
        (int64_t)(a.KH - 1) * a.DH < 32768 &&
        (int64_t)(a.KW - 1) * a.DW < 32768) {
        int code = 0x1010 | (a.Cog >= 64 ? 4 : a.Cog >= 32 ? 2 : 1);
        if (a.tile_hint & TILE_VALID) code = a.tile_hint & 0xffff;
        // the narrow form has one 16-channel block a wave
        const bool nform = narrow && a.Cg % 16 != 0;
        if (nform && (code & 0xff00) == 0x1000) code = (code & ~15) | 1;
        const int wm = code & 15, tm = (code >> 4) & 15;
        if ((code & 0xff00) == 0x1000 && (wm == 1 || wm == 2 || wm == 4) &&
            (tm == 1 || tm == 2)) {
            const int64_t gx = ceil_div(ntiles, 4 * tm);
            const int64_t gy = ceil_div(a.Cog, 16 * wm);
            if (gx >= ((int64_t)1 << 31) || gy > 65535) {
                set_error("launch_conv_f64", "grid too large");
                return false;
            }
            const dim3 grid((unsigned)gx, (unsigned)gy, (unsigned)a.G);
            // the epilogue's form: general, or int16 with / without the
            // residual Add and the rescaled copy
            const int epi = (b.mode == EPI_QUANT && b.fastio && b.y_code == 2)
                                ? 1 | (b.res ? 2 : 0) | (b.y2 ? 4 : 0)
                                : 0;
            using std::integral_constant;
            const size_t ktab = (size_t)a.KGp * sizeof(int2);  // k-groups
            auto tiles = [&](auto nr, auto ep) {
                constexpr bool NR = decltype(nr)::value;
                constexpr int EP = decltype(ep)::value;
                switch (code) {
                    case 0x1011: k_conv_bs<1, 1, NR, EP><<<grid, 256, ktab, st>>>(b); break;
                    case 0x1021: k_conv_bs<1, 2, NR, EP><<<grid, 256, ktab, st>>>(b); break;
                    default:
                        if constexpr (!NR) {
                            switch (code) {
                                case 0x1012: k_conv_bs<2, 1, false, EP><<<grid, 256, ktab, st>>>(b); break;
                                case 0x1014: k_conv_bs<4, 1, false, EP><<<grid, 256, ktab, st>>>(b); break;
                                case 0x1022: k_conv_bs<2, 2, false, EP><<<grid, 256, ktab, st>>>(b); break;
                                default: k_conv_bs<4, 2, false, EP><<<grid, 256, ktab, st>>>(b); break;
                            }
                        }
                        break;  // narrow: codes 0x1011 / 0x1021 only
                }
            };
            auto forms = [&](auto nr) {
                switch (epi) {
                    case 1: tiles(nr, integral_constant<int, 1>{}); break;
                    case 3: tiles(nr, integral_constant<int, 3>{}); break;
                    case 5: tiles(nr, integral_constant<int, 5>{}); break;
                    case 7: tiles(nr, integral_constant<int, 7>{}); break;
                    default: tiles(nr, integral_constant<int, 0>{}); break;
                }
            };
            if (nform)
                forms(std::true_type{});
            else
                forms(std::false_type{});
            const hipError_t e = hipGetLastError();
            if (e != hipSuccess) {
                set_hip_error("launch_conv_f64", e);
                return false;
            }
            return true;
        }
    }
    auto waves = [&](const F64Tile& t) {
        return ceil_div(ntiles, t.tm) * ceil_div(a.Cog, 16 * t.wm) * a.G *
               (t.split ? 4 : 1);
    };
    // tile: a caller's choice, else the first of these that gives every CU
    // 48 waves (a 64-cycle MFMA per wave needs many waves in flight to
    // cover the fragment loads), else K split over single channel groups
    F64Tile tile = {1, 1, true};
    bool chosen = false;
    if (a.tile_hint & TILE_VALID) {
        for (const F64Tile& t : kF64Tiles)
            if (f64_code(t) == (a.tile_hint & 0xffff)) {
                tile = t;
                chosen = true;
            }
    }
    if (!chosen) {
        const F64Tile order[] = {
            {2, 1, false}, {1, 1, false}, {2, 1, true}, {1, 1, true}};
        const int64_t want = 48 * (int64_t)cu_count();
        for (const F64Tile& t : order)
            if ((t.wm == 1 || a.Cog > 16) && waves(t) >= want) {
                tile = t;
                break;
            }
    }
    const int64_t gx = tile.split ? ceil_div(ntiles, tile.tm)
                                  : ceil_div(ntiles, 4 * tile.tm);
    const int64_t gy = ceil_div(a.Cog, 16 * tile.wm);
    if (gx >= ((int64_t)1 << 31) || gy > 65535) {
        set_error("launch_conv_f64", "grid too large");
        return false;
    }
    const dim3 grid((unsigned)gx, (unsigned)gy, (unsigned)a.G);
    switch (f64_code(tile)) {
        case 0x11: launch_w<1, 1, false>(b, v, grid, st); break;
        case 0x12: launch_w<2, 1, false>(b, v, grid, st); break;
        case 0x41: launch_w<1, 4, false>(b, v, grid, st); break;
        case 0x111: launch_w<1, 1, true>(b, v, grid, st); break;
        case 0x112: launch_w<2, 1, true>(b, v, grid, st); break;
        case 0x114: launch_w<4, 1, true>(b, v, grid, st); break;
        default:
            set_error("launch_conv_f64", "no kernel for this tile");
            return false;
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_hip_error("launch_conv_f64", e);
        return false;
    }
    return true;
}

}  // namespace qa

// int8 MFMA convolution / GEMM (data layout: qa_conv.h).
//
// Work-group = 4 wave64s, each owning the same WM*16 output channels and its
// own WN*16 consecutive output pixels (batch folded in), so every activation
// byte a wave loads is used only by that wave and the weight fragments are
// shared through L1/L2 by all waves and work-groups. Fragments are loaded
// straight from global memory into registers (16 contiguous bytes per lane),
// one K-step ahead of the MFMAs that consume them; there is no barrier in
// the main loop. The epilogue requantizes, applies the table (held in LDS),
// the residual Add and an optional rescaled second output, and stores 4
// consecutive output channels of a pixel as one 32-bit word.
//
// Epilogue variants (template EPI):
//   EPI_RAW32 / EPI_RAW64  accumulators for the reference ABI,
//   Q8_FAST   int64-only requantization, used when the host has checked
//             that every multiplier has |M| < 2^31, 1 <= 31+shift <= 62 and
//             every bias fits int32, so |acc + bias| <= 2^32 and the product
//             is exact in int64; then round(p * 2^-t) half up equals
//             (p >> t) + bit (t-1) of p, the reference's 128-bit result;
//   Q8_GENERAL the 128-bit form for any parameters.
#include "qa_conv.h"

namespace qa {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int Q8_FAST = 3;
constexpr int Q8_GENERAL = 4;

struct PixCtx {
    const int8_t* base;  // image base + group channel offset
    int iy0, ix0;
    int ok;
    uint32_t n, pix;
};

__device__ __forceinline__ int splat4(int b) {
    return (int)((uint32_t)(uint8_t)b * 0x01010101u);
}

// sum of the first nreal signed bytes of v (nreal in 1..16)
__device__ __forceinline__ int bytes_sum(v4i v, int nreal) {
    int s = 0;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        const int k = nreal - 4 * w;
        const int mask = k >= 4 ? 0x01010101
                                : (k <= 0 ? 0 : (int)((1u << (8 * k)) - 1) &
                                                     0x01010101);
        s = __builtin_amdgcn_sdot4(v[w], mask, s, false);
    }
    return s;
}

// B fragment: 16 bytes of K for one pixel.
template <int LAYOUT>
__device__ __forceinline__ v4i load_b(const ConvArgs& a, const PixCtx& P,
                                      bool kvalid, int ky, int kx, int cb,
                                      int kg, int* psum) {
    v4i v = {0, 0, 0, 0};
    if (!P.ok || !kvalid) return v;
    if (LAYOUT == 0) {
        const int iy = P.iy0 + ky * a.DH;
        const int ix = P.ix0 + kx * a.DW;
        if (iy < 0 || iy >= a.H || ix < 0 || ix >= a.W) {
            const int pv = splat4(a.pad_value);
            v = v4i{pv, pv, pv, pv};
            if (a.rowsum) *psum += min(16, a.Cg - cb * 16) * a.pad_value;
        } else {
            v = *(const v4i*)(P.base + ((int64_t)iy * a.W + ix) * a.x_sp +
                              cb * 16);
            if (a.rowsum) *psum += bytes_sum(v, min(16, a.Cg - cb * 16));
        }
        return v;
    }
    // LAYOUT 1: k-group kg = kernel row; 4 bytes (channels) per kx
    const int iy = P.iy0 + kg * a.DH;
    const bool row_ok = iy >= 0 && iy < a.H;
    const int mask = a.Cg >= 4 ? 0x01010101
                               : (int)((1u << (8 * a.Cg)) - 1) & 0x01010101;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        if (t < a.KW) {
            const int ix = P.ix0 + t * a.DW;
            int w;
            if (row_ok && ix >= 0 && ix < a.W) {
                w = *(const int*)(P.base + ((int64_t)iy * a.W + ix) * a.x_sp);
                if (a.rowsum) *psum = __builtin_amdgcn_sdot4(w, mask, *psum,
                                                             false);
            } else {
                w = splat4(a.pad_value);
                if (a.rowsum) *psum += a.Cg * a.pad_value;
            }
            v[t] = w;
        }
    }
    return v;
}

__device__ __forceinline__ uint32_t pack4(int64_t b0, int64_t b1, int64_t b2,
                                          int64_t b3) {
    return (uint32_t)(uint8_t)b0 | ((uint32_t)(uint8_t)b1 << 8) |
           ((uint32_t)(uint8_t)b2 << 16) | ((uint32_t)(uint8_t)b3 << 24);
}

// round(x * m * 2^-t) for 1 <= t <= 62 and an exact int64 product x*m
__device__ __forceinline__ int64_t mbqm64(int64_t x, int64_t m, int t) {
    const int64_t p = x * m;
    return (p >> t) + ((p >> (t - 1)) & 1);
}

__device__ __forceinline__ int64_t clamp64(int64_t v, int64_t lo,
                                           int64_t hi) {
    return v < lo ? lo : (v > hi ? hi : v);
}

template <int EPI>
__device__ __forceinline__ int64_t quant8(const ConvArgs& a,
                                          const int* __restrict__ s_lut,
                                          int64_t v, int64_t m, int t,
                                          int64_t res_q) {
    if (EPI == Q8_GENERAL) {
        int64_t q = qa_clip128(qa_mbqm(v, m, t - 31) + a.zp, a.qmin, a.qmax);
        if (a.lut) {
            int64_t idx = q - a.lut_off;
            idx = idx < 0 ? 0 : (idx >= a.lut_len ? a.lut_len - 1 : idx);
            q = s_lut ? s_lut[idx] : a.lut[idx];
        }
        if (a.res) {
            const int64_t f = a.res_first ? res_q : q;
            const int64_t s = a.res_first ? q : res_q;
            q = qa_clip128(qa_mbqm(f - a.za, a.ma, a.sa) +
                               (qa_i128)a.add_sign *
                                   qa_mbqm(s - a.zb, a.mb, a.sb) +
                               a.add_zp,
                           a.add_qmin, a.add_qmax);
        }
        return q;
    }
    int64_t q = clamp64(mbqm64(v, m, t) + a.zp, a.qmin, a.qmax);
    if (a.lut) {
        int64_t idx = q - a.lut_off;
        idx = idx < 0 ? 0 : (idx >= a.lut_len ? a.lut_len - 1 : idx);
        q = s_lut[idx];
    }
    if (a.res) {
        const int64_t f = a.res_first ? res_q : q;
        const int64_t s = a.res_first ? q : res_q;
        q = clamp64(mbqm64(f - a.za, a.ma, (int)(31 + a.sa)) +
                        a.add_sign *
                            mbqm64(s - a.zb, a.mb, (int)(31 + a.sb)) +
                        a.add_zp,
                    a.add_qmin, a.add_qmax);
    }
    return q;
}

template <int EPI>
__device__ __forceinline__ int64_t rescale8(const ConvArgs& a, int64_t q) {
    if (EPI == Q8_GENERAL) return rescale2(a, q);
    return clamp64(mbqm64(q - a.r2_zp_in, a.r2_m, (int)(31 + a.r2_s)) +
                       a.r2_zp_out,
                   a.r2_qmin, a.r2_qmax);
}

// KSPLIT: the 4 waves share the block's WN*16 pixels and split the K-steps
// (wave w takes steps w, w+4, ...); the partial accumulators are summed
// through LDS and wave 0 runs the epilogue. Used when the output has too
// few pixels to give every CU work otherwise.
template <int WM, int WN, int LAYOUT, int EPI, bool KSPLIT>
__global__ __launch_bounds__(256) void k_conv_mfma(ConvArgs a) {
    constexpr bool QUANT = EPI == Q8_FAST || EPI == Q8_GENERAL;
    constexpr int KSTRIDE = KSPLIT ? 4 : 1;
    __shared__ int s_lut[QUANT ? 256 : 1];
    __shared__ int s_red[KSPLIT ? 3 * WM * WN * 4 * 64 + 3 * WN * 64 : 1];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int g = blockIdx.z;
    const int co0 = blockIdx.y * (WM * 16);
    const int64_t pw0 =
        KSPLIT ? (int64_t)blockIdx.x * (WN * 16)
               : (int64_t)blockIdx.x * (4 * WN * 16) + (int64_t)wave * (WN * 16);
    const int kgl = lane >> 4;
    const int col = lane & 15;
    const uint32_t OHW = (uint32_t)(a.OH * a.OW);
    const bool lds_lut = QUANT && a.lut && a.lut_len <= 256;
    if (lds_lut) {
        for (int i = threadIdx.x; i < a.lut_len; i += 256) s_lut[i] = a.lut[i];
    }

    PixCtx px[WN];
#pragma unroll
    for (int j = 0; j < WN; ++j) {
        const int64_t p = pw0 + j * 16 + col;
        px[j].ok = p < a.M;
        const uint32_t pp = px[j].ok ? (uint32_t)p : 0u;
        const uint32_t n = pp / OHW;
        const uint32_t pix = pp - n * OHW;
        const int oy = (int)(pix / (uint32_t)a.OW);
        const int ox = (int)pix - oy * a.OW;
        px[j].n = n;
        px[j].pix = pix;
        px[j].iy0 = oy * a.SH - a.PH;
        px[j].ix0 = ox * a.SW - a.PW;
        px[j].base = (const int8_t*)a.x + (int64_t)n * a.x_sn +
                     (int64_t)g * a.Cg;
    }
    const int8_t* wrow[WM];
#pragma unroll
    for (int i = 0; i < WM; ++i)
        wrow[i] = a.wp + (int64_t)g * a.wp_gstride +
                  (int64_t)(co0 + i * 16 + col) * a.wp_rstride + kgl * 16;

    v4i acc[WM][WN];
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < WN; ++j) acc[i][j] = v4i{0, 0, 0, 0};
    int psum[WN];
#pragma unroll
    for (int j = 0; j < WN; ++j) psum[j] = 0;

    // k-group of this lane: kg = 4*ks + kgl -> (tap, cb), tap -> (ky, kx);
    // advanced incrementally by 4*KSTRIDE groups per step.
    const int ks0 = KSPLIT ? wave : 0;
    int cb = 4 * ks0 + kgl, ky = 0, kx = 0;
    if (LAYOUT == 0) {
        while (cb >= a.CB) {
            cb -= a.CB;
            if (++kx == a.KW) {
                kx = 0;
                ++ky;
            }
        }
    }
    const int KS = a.KGp >> 2;
    v4i af[WM], bf[WN];
    if (ks0 < KS) {
        const int kg = 4 * ks0 + kgl;
#pragma unroll
        for (int i = 0; i < WM; ++i) af[i] = *(const v4i*)(wrow[i] + ks0 * 64);
#pragma unroll
        for (int j = 0; j < WN; ++j)
            bf[j] = load_b<LAYOUT>(a, px[j], kg < a.KG, ky, kx, cb, kg,
                                   &psum[j]);
    }
    for (int ks = ks0; ks < KS; ks += KSTRIDE) {
        v4i an[WM], bn[WN];
        const bool more = ks + KSTRIDE < KS;
        if (more) {
            const int kg = 4 * (ks + KSTRIDE) + kgl;
            if (LAYOUT == 0) {
                cb += 4 * KSTRIDE;
                while (cb >= a.CB) {
                    cb -= a.CB;
                    if (++kx == a.KW) {
                        kx = 0;
                        ++ky;
                    }
                }
            }
#pragma unroll
            for (int i = 0; i < WM; ++i)
                an[i] = *(const v4i*)(wrow[i] + (ks + KSTRIDE) * 64);
#pragma unroll
            for (int j = 0; j < WN; ++j)
                bn[j] = load_b<LAYOUT>(a, px[j], kg < a.KG, ky, kx, cb, kg,
                                       &psum[j]);
        }
#pragma unroll
        for (int i = 0; i < WM; ++i)
#pragma unroll
            for (int j = 0; j < WN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                    af[i], bf[j], acc[i][j], 0, 0, 0);
        if (more) {
#pragma unroll
            for (int i = 0; i < WM; ++i) af[i] = an[i];
#pragma unroll
            for (int j = 0; j < WN; ++j) bf[j] = bn[j];
        }
    }

    if (KSPLIT) {  // sum the 4 waves' partial results into wave 0
        if (wave > 0) {
            int* dst = s_red + (wave - 1) * (WM * WN * 4 + WN) * 64;
#pragma unroll
            for (int i = 0; i < WM; ++i)
#pragma unroll
                for (int j = 0; j < WN; ++j)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        dst[((i * WN + j) * 4 + r) * 64 + lane] = acc[i][j][r];
#pragma unroll
            for (int j = 0; j < WN; ++j)
                dst[(WM * WN * 4 + j) * 64 + lane] = psum[j];
        }
        __syncthreads();
        if (wave > 0) return;
#pragma unroll
        for (int w = 0; w < 3; ++w) {
            const int* src = s_red + w * (WM * WN * 4 + WN) * 64;
#pragma unroll
            for (int i = 0; i < WM; ++i)
#pragma unroll
                for (int j = 0; j < WN; ++j)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        acc[i][j][r] += src[((i * WN + j) * 4 + r) * 64 + lane];
#pragma unroll
            for (int j = 0; j < WN; ++j)
                psum[j] += src[(WM * WN * 4 + j) * 64 + lane];
        }
    }

    if (a.rowsum) {  // lanes col, col+16, col+32, col+48 hold partial sums
#pragma unroll
        for (int j = 0; j < WN; ++j) {
            int s = psum[j];
            s += __shfl_xor(s, 16);
            s += __shfl_xor(s, 32);
            psum[j] = s;
        }
    }
    if (lds_lut && !KSPLIT) __syncthreads();  // KSPLIT synced above
    const int* lut = lds_lut ? s_lut : nullptr;

    // ---- epilogue ----
#pragma unroll
    for (int i = 0; i < WM; ++i) {
        const int cl = co0 + i * 16 + kgl * 4;  // first of 4 channels
        const int64_t cg0 = (int64_t)g * a.Cog + cl;
        int64_t corr[4], pre[4], mlt[4];
        int bo[4], tsh[4];
        bool cv[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            cv[r] = cl + r < a.Cog;
            const int64_t co = cv[r] ? cg0 + r : cg0 - cl;
            corr[r] = a.corr ? a.corr[co] : 0;
            bo[r] = a.rowsum ? a.boff[co] : 0;
            pre[r] = (QUANT && a.pre) ? a.pre[co] : 0;
            mlt[r] = QUANT ? a.mult[co] : 0;
            tsh[r] = QUANT ? (int)(31 + a.shift[co]) : 0;
        }
        const bool all4 = cv[0] && cv[1] && cv[2] && cv[3];
#pragma unroll
        for (int j = 0; j < WN; ++j) {
            if (!px[j].ok) continue;
            const int64_t rs = psum[j];
            const int64_t ybase = (int64_t)px[j].n * a.y_sn +
                                  (int64_t)px[j].pix * a.y_sp;
            if (!QUANT) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    if (!cv[r]) continue;
                    const int64_t o = ybase + (cg0 + r) * a.y_sc;
                    if (EPI == EPI_RAW64)
                        ((int64_t*)a.y)[o] = (int64_t)acc[i][j][r] + corr[r] +
                                             (int64_t)bo[r] * rs;
                    else
                        ((int32_t*)a.y)[o] =
                            (int32_t)((uint32_t)acc[i][j][r] +
                                      (uint32_t)corr[r] +
                                      (uint32_t)bo[r] * (uint32_t)rs);
                }
                continue;
            }
            int64_t rq[4] = {0, 0, 0, 0};
            if (a.res) {
                const int64_t rb = (int64_t)px[j].n * a.res_sn +
                                   (int64_t)px[j].pix * a.res_sp + cg0;
                if (all4 && a.res_sc == 1 && (rb & 3) == 0) {
                    const uint32_t w = *(const uint32_t*)((const int8_t*)a.res +
                                                          rb);
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        rq[r] = (int64_t)(int8_t)(w >> (8 * r)) + a.res_so;
                } else {
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (cv[r])
                            rq[r] = (int64_t)((const int8_t*)
                                                  a.res)[rb + r * a.res_sc] +
                                    a.res_so;
                }
            }
            int64_t q[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                // the reference adds the bias to the int32 accumulator
                const int64_t v =
                    (int64_t)(int32_t)((uint32_t)acc[i][j][r] +
                                       (uint32_t)corr[r] +
                                       (uint32_t)bo[r] * (uint32_t)rs) +
                    pre[r];
                q[r] = quant8<EPI>(a, lut, v, mlt[r], tsh[r], rq[r]);
            }
            const int64_t yo = ybase + cg0;
            if (all4 && a.y_sc == 1 && (yo & 3) == 0) {
                *(uint32_t*)((int8_t*)a.y + yo) =
                    pack4(q[0] - a.y_so, q[1] - a.y_so, q[2] - a.y_so,
                          q[3] - a.y_so);
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (cv[r])
                        ((int8_t*)a.y)[ybase + (cg0 + r) * a.y_sc] =
                            (int8_t)(q[r] - a.y_so);
            }
            if (a.y2) {
                const int64_t b2 = (int64_t)px[j].n * a.y2_sn +
                                   (int64_t)px[j].pix * a.y2_sp;
                int64_t q2[4];
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    q2[r] = rescale8<EPI>(a, q[r]) - a.y_so;
                const int64_t o2 = b2 + cg0;
                if (all4 && a.y2_sc == 1 && (o2 & 3) == 0) {
                    *(uint32_t*)((int8_t*)a.y2 + o2) =
                        pack4(q2[0], q2[1], q2[2], q2[3]);
                } else {
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (cv[r])
                            ((int8_t*)a.y2)[b2 + (cg0 + r) * a.y2_sc] =
                                (int8_t)q2[r];
                }
            }
        }
    }
}

template <int WM, int WN, int LAYOUT, bool KSPLIT>
bool launch_cfg(const ConvArgs& a, int epi, hipStream_t st) {
    dim3 grid((unsigned)ceil_div(a.M, (KSPLIT ? 1 : 4) * WN * 16),
              (unsigned)ceil_div(a.Cog, WM * 16), (unsigned)a.G);
    switch (epi) {
        case EPI_RAW32:
            k_conv_mfma<WM, WN, LAYOUT, EPI_RAW32, KSPLIT>
                <<<grid, 256, 0, st>>>(a);
            break;
        case EPI_RAW64:
            k_conv_mfma<WM, WN, LAYOUT, EPI_RAW64, KSPLIT>
                <<<grid, 256, 0, st>>>(a);
            break;
        case Q8_FAST:
            k_conv_mfma<WM, WN, LAYOUT, Q8_FAST, KSPLIT>
                <<<grid, 256, 0, st>>>(a);
            break;
        default:
            k_conv_mfma<WM, WN, LAYOUT, Q8_GENERAL, KSPLIT>
                <<<grid, 256, 0, st>>>(a);
            break;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_hip_error("k_conv_mfma launch", e);
        return false;
    }
    return true;
}

// Tile choice: the widest pixel tile that still gives >= 2 work-groups per
// CU; when even 64-pixel tiles do not, the waves split K instead.
template <int WM, int LAYOUT>
bool launch_wm(const ConvArgs& a, int epi, hipStream_t st) {
    constexpr int WN_WIDE = WM <= 4 ? 4 : 2;
    const int64_t cblocks = ceil_div(a.Cog, WM * 16) * (int64_t)a.G;
    if (LAYOUT == 1 || ceil_div(a.M, 4 * WN_WIDE * 16) * cblocks >= 512)
        return launch_cfg<WM, WN_WIDE, LAYOUT, false>(a, epi, st);
    if (ceil_div(a.M, 4 * 16) * cblocks >= 512 || a.KGp < 16)
        return launch_cfg<WM, 1, LAYOUT, false>(a, epi, st);
    return launch_cfg<WM, 1, LAYOUT, true>(a, epi, st);
}

// True when a multiplier allows the int64 epilogue.
bool fast_ok(int64_t m, int64_t shift) {
    const int64_t am = m < 0 ? -m : m;
    return am < ((int64_t)1 << 31) && 31 + shift >= 1 && 31 + shift <= 62;
}

}  // namespace

bool launch_conv_mfma(const ConvArgs& a, hipStream_t st) {
    if (a.M <= 0 || a.Cog <= 0 || a.G <= 0) return true;
    if (a.M >= ((int64_t)1 << 31) || a.KGp < 4 || (a.KGp & 3)) {
        set_error("launch_conv_mfma", "unsupported problem size");
        return false;
    }
    int epi = a.mode;
    if (a.mode == EPI_QUANT) {
        if (a.y_code != 1) {
            set_error("launch_conv_mfma", "int8 output expected");
            return false;
        }
        // parameters are read back from the host-visible descriptor copies
        bool fast = a.fast_hint != 0;
        if (a.res) fast = fast && fast_ok(a.ma, a.sa) && fast_ok(a.mb, a.sb);
        if (a.y2) fast = fast && fast_ok(a.r2_m, a.r2_s);
        epi = fast ? Q8_FAST : Q8_GENERAL;
    }
    if (a.layout == 1) {
        if (a.Cog <= 16) return launch_wm<1, 1>(a, epi, st);
        if (a.Cog <= 32) return launch_wm<2, 1>(a, epi, st);
        if (a.Cog <= 64) return launch_wm<4, 1>(a, epi, st);
        return launch_wm<8, 1>(a, epi, st);
    }
    if (a.Cog <= 16) return launch_wm<1, 0>(a, epi, st);
    if (a.Cog <= 32) return launch_wm<2, 0>(a, epi, st);
    if (a.Cog <= 64) return launch_wm<4, 0>(a, epi, st);
    return launch_wm<8, 0>(a, epi, st);
}

}  // namespace qa

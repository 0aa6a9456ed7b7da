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
//   Q8_TABLE  int8 output through a host-built plan (qa_conv.h): one int64
//             multiply-add and shift per element, then 256-entry LDS tables
//             for clip, activation table, residual Add and rescaled copy,
//   Q8_GENERAL the 128-bit form for any parameters.
#include "qa_conv.h"

namespace qa {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int Q8_TABLE = 3;
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

// The 128-bit epilogue of one accumulator (Q8_GENERAL).
__device__ __forceinline__ int64_t quant_general(const ConvArgs& a,
                                                 const int* __restrict__ s_lut,
                                                 int64_t v, int64_t m,
                                                 int64_t shift, int64_t res_q) {
    int64_t q = qa_clip128(qa_mbqm(v, m, shift) + a.zp, a.qmin, a.qmax);
    if (a.lut) {
        int64_t idx = q - a.lut_off;
        idx = idx < 0 ? 0 : (idx >= a.lut_len ? a.lut_len - 1 : idx);
        q = s_lut ? s_lut[idx] : a.lut[idx];
    }
    if (a.res) {
        const int64_t f = a.res_first ? res_q : q;
        const int64_t s = a.res_first ? q : res_q;
        q = qa_clip128(qa_mbqm(f - a.za, a.ma, a.sa) +
                           (qa_i128)a.add_sign * qa_mbqm(s - a.zb, a.mb, a.sb) +
                           a.add_zp,
                       a.add_qmin, a.add_qmax);
    }
    return q;
}

// Low bytes of four table entries packed into one word (byte = 0), or their
// second bytes (byte = 1).
__device__ __forceinline__ uint32_t pack_entries(const int e[4], int byte) {
    const uint32_t sel_lo = byte ? 0x0c0c0501u : 0x0c0c0400u;
    const uint32_t lo = __builtin_amdgcn_perm((uint32_t)e[1], (uint32_t)e[0],
                                              sel_lo);
    const uint32_t hi = __builtin_amdgcn_perm((uint32_t)e[3], (uint32_t)e[2],
                                              sel_lo);
    return __builtin_amdgcn_perm(hi, lo, 0x05040100u);
}

// KSPLIT: the 4 waves share the block's WN*16 pixels and split the K-steps
// (wave w takes steps w, w+4, ...); the partial accumulators are summed
// through LDS and wave 0 runs the epilogue. Used when the output has too
// few pixels to give every CU work otherwise.
template <int WM, int WN, int LAYOUT, int EPI, bool KSPLIT>
__global__ __launch_bounds__(256) void k_conv_mfma(ConvArgs a) {
    constexpr bool QUANT = EPI == Q8_TABLE || EPI == Q8_GENERAL;
    constexpr bool TABLE = EPI == Q8_TABLE;
    constexpr int KSTRIDE = KSPLIT ? 4 : 1;
    // Q8_GENERAL: activation table; Q8_TABLE: E, TC, TR of the plan
    __shared__ int s_tab[TABLE ? 768 : (QUANT ? 256 : 1)];
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
    const bool lds_tab =
        TABLE || (QUANT && a.lut && a.lut_len <= 256);
    if (TABLE) {
        const int* tab = (const int*)((const char*)a.plan + PLAN_E);
        const int n = (((const int*)a.plan)[3] & PLAN_RES) ? 768 : 256;
        for (int i = threadIdx.x; i < n; i += 256) s_tab[i] = tab[i];
    } else if (lds_tab) {
        for (int i = threadIdx.x; i < a.lut_len; i += 256) s_tab[i] = a.lut[i];
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
    if (lds_tab && !KSPLIT) __syncthreads();  // KSPLIT synced above

    // ---- epilogue ----
    if (TABLE) {
        const int* hd = (const int*)a.plan;
        const int A = hd[0], B = hd[1], SH = hd[2];
        const bool res = a.res != nullptr, two = a.y2 != nullptr;
        const int4* pch = (const int4*)((const char*)a.plan + PLAN_CH);
#pragma unroll
        for (int i = 0; i < WM; ++i) {
            const int cl = co0 + i * 16 + kgl * 4;  // first of 4 channels
            const int64_t cg0 = (int64_t)g * a.Cog + cl;
            uint32_t corr[4], bo[4];
            int mlt[4], tsh[4];
            int64_t cst[4];
            bool cv[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                cv[r] = cl + r < a.Cog;
                const int64_t co = cv[r] ? cg0 + r : cg0 - cl;
                const int4 pc = pch[co];
                mlt[r] = pc.x;
                tsh[r] = pc.y;
                cst[r] = (int64_t)(((uint64_t)(uint32_t)pc.w << 32) |
                                   (uint32_t)pc.z);
                corr[r] = a.corr ? (uint32_t)a.corr[co] : 0u;
                bo[r] = a.rowsum ? (uint32_t)a.boff[co] : 0u;
            }
            const bool all4 = cv[0] && cv[1] && cv[2] && cv[3];
#pragma unroll
            for (int j = 0; j < WN; ++j) {
                if (!px[j].ok) continue;
                const uint32_t rs = (uint32_t)psum[j];
                int e[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    // int32 accumulator (wraps like the reference's)
                    const int w = (int)((uint32_t)acc[i][j][r] + corr[r] +
                                        bo[r] * rs);
                    const int q0 =
                        (int)(((int64_t)w * mlt[r] + cst[r]) >> tsh[r]);
                    e[r] = min(max(q0, A), B) - A;
                }
                if (res) {
                    const int64_t rb = (int64_t)px[j].n * a.res_sn +
                                       (int64_t)px[j].pix * a.res_sp + cg0;
                    uint32_t u[4];
                    if (all4 && a.res_sc == 1 && (rb & 3) == 0) {
                        const uint32_t wv =
                            *(const uint32_t*)((const int8_t*)a.res + rb);
#pragma unroll
                        for (int r = 0; r < 4; ++r) u[r] = (wv >> (8 * r)) & 255u;
                    } else {
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            u[r] = cv[r] ? ((const uint8_t*)
                                                a.res)[rb + r * a.res_sc]
                                         : 0u;
                    }
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int t = s_tab[256 + e[r]] + s_tab[512 + u[r]];
                        e[r] = min(max(t, 0), SH);
                    }
                }
#pragma unroll
                for (int r = 0; r < 4; ++r) e[r] = s_tab[e[r]];
                const int64_t ybase = (int64_t)px[j].n * a.y_sn +
                                      (int64_t)px[j].pix * a.y_sp;
                const int64_t yo = ybase + cg0;
                if (all4 && a.y_sc == 1 && (yo & 3) == 0) {
                    *(uint32_t*)((int8_t*)a.y + yo) = pack_entries(e, 0);
                } else {
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (cv[r])
                            ((int8_t*)a.y)[ybase + (cg0 + r) * a.y_sc] =
                                (int8_t)e[r];
                }
                if (two) {
                    const int64_t b2 = (int64_t)px[j].n * a.y2_sn +
                                       (int64_t)px[j].pix * a.y2_sp;
                    const int64_t o2 = b2 + cg0;
                    if (all4 && a.y2_sc == 1 && (o2 & 3) == 0) {
                        *(uint32_t*)((int8_t*)a.y2 + o2) = pack_entries(e, 1);
                    } else {
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            if (cv[r])
                                ((int8_t*)a.y2)[b2 + (cg0 + r) * a.y2_sc] =
                                    (int8_t)(e[r] >> 8);
                    }
                }
            }
        }
        return;
    }
    const int* lut = lds_tab ? s_tab : nullptr;
#pragma unroll
    for (int i = 0; i < WM; ++i) {
        const int cl = co0 + i * 16 + kgl * 4;  // first of 4 channels
        const int64_t cg0 = (int64_t)g * a.Cog + cl;
        int64_t corr[4], pre[4], mlt[4], shf[4];
        int bo[4];
        bool cv[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            cv[r] = cl + r < a.Cog;
            const int64_t co = cv[r] ? cg0 + r : cg0 - cl;
            corr[r] = a.corr ? a.corr[co] : 0;
            bo[r] = a.rowsum ? a.boff[co] : 0;
            pre[r] = (QUANT && a.pre) ? a.pre[co] : 0;
            mlt[r] = QUANT ? a.mult[co] : 0;
            shf[r] = QUANT ? a.shift[co] : 0;
        }
#pragma unroll
        for (int j = 0; j < WN; ++j) {
            if (!px[j].ok) continue;
            const int64_t rs = psum[j];
            const int64_t ybase = (int64_t)px[j].n * a.y_sn +
                                  (int64_t)px[j].pix * a.y_sp;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                if (!cv[r]) continue;
                const int64_t o = ybase + (cg0 + r) * a.y_sc;
                if (EPI == EPI_RAW64) {
                    ((int64_t*)a.y)[o] = (int64_t)acc[i][j][r] + corr[r] +
                                         (int64_t)bo[r] * rs;
                    continue;
                }
                const int32_t w = (int32_t)((uint32_t)acc[i][j][r] +
                                            (uint32_t)corr[r] +
                                            (uint32_t)bo[r] * (uint32_t)rs);
                if (EPI == EPI_RAW32) {
                    ((int32_t*)a.y)[o] = w;
                    continue;
                }
                int64_t rq = 0;
                if (a.res)
                    rq = (int64_t)((const int8_t*)a.res)
                             [(int64_t)px[j].n * a.res_sn +
                              (int64_t)px[j].pix * a.res_sp +
                              (cg0 + r) * a.res_sc] +
                         a.res_so;
                // the reference adds the bias to the int32 accumulator
                const int64_t q =
                    quant_general(a, lut, (int64_t)w + pre[r], mlt[r], shf[r],
                                  rq);
                ((int8_t*)a.y)[o] = (int8_t)(q - a.y_so);
                if (a.y2)
                    ((int8_t*)a.y2)[(int64_t)px[j].n * a.y2_sn +
                                    (int64_t)px[j].pix * a.y2_sp +
                                    (cg0 + r) * a.y2_sc] =
                        (int8_t)(rescale2(a, q) - a.y_so);
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
        case Q8_TABLE:
            k_conv_mfma<WM, WN, LAYOUT, Q8_TABLE, KSPLIT>
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
        epi = a.plan ? Q8_TABLE : Q8_GENERAL;
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

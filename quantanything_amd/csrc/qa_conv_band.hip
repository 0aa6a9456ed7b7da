// int8 convolution over bands of output rows, operands in LDS.
//
// A work-group owns R output rows of one image (the band) and WM*16 output
// channels. It stages the band's input rows, halo and image padding
// included (padding holds the pad value, so the K loop has no bounds
// checks), and its weight rows in LDS once; every tap of every pixel then
// reads its fragment from LDS. Each wave computes TM = 4 tiles of 16 band
// pixels in lockstep, so each weight fragment feeds TM MFMAs and each
// activation fragment WM (v_mfma_i32_16x16x64_i8; a K-step is four 16-byte
// k-groups of the packed layout-0 weights: tap kg / CB, channels
// 16 (kg % CB) ..). The epilogue is the int8 table plan of qa_conv.h.
//
// LDS: band [BR][BW] pixels of PS bytes (PS = Cg, plus 16 when Cg / 16 is
// even, so that the 16 pixels of a fragment read hit distinct banks);
// weights [WM*16][KGp*16 + 16]; the k-group table [KGp] (LDS offset of the
// k-group's pixel and channel block, -1 past the real K).
#include "qa_conv_mfma.h"

namespace qa {
namespace {

constexpr int BAND_TM = 4;

struct BandGeom {
    int R, BR, BW, PS, RSW, nbands;
    int lds;  // bytes
};

template <int WM>
__global__ __launch_bounds__(256) void k_conv_band(ConvArgs a, BandGeom bg) {
    extern __shared__ int4 lds4[];
    int8_t* s_x = (int8_t*)lds4;                              // band
    int8_t* s_w = s_x + bg.BR * bg.BW * bg.PS;                // weights
    int* s_kt = (int*)(s_w + WM * 16 * bg.RSW);               // k-groups
    __shared__ int s_tab[768];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int col = lane & 15, kgl = lane >> 4;
    // the channel blocks of a band read the same band: one XCD runs them
    const XcdBlock blk = xcd_block(true);
    const int n = (int)blk.x / bg.nbands;
    const int oy0 = ((int)blk.x - n * bg.nbands) * bg.R;
    const int co0 = (int)blk.y * WM * 16;
    const int rows = min(bg.R, a.OH - oy0);     // output rows of the band
    const int npix = rows * a.OW;
    const int KGp = a.KGp;
    const int KS = KGp >> 2;

    // ---- stage: band (pad value outside the image), weights, tables ----
    {
        const int cpp = a.Cg >> 4;  // 16-byte chunks per pixel
        const int nch = bg.BR * bg.BW * cpp;
        const int iy0 = oy0 * a.SH - a.PH;
        const int pv = splat4(a.pad_value);
        const int8_t* xn = (const int8_t*)a.x + (int64_t)n * a.x_sn;
        // four loads in flight per thread before their LDS stores, held in
        // named vector registers (arrays or struct selects here would live
        // in scratch); unconditional loads (padding and chunks past the end read the
        // image's first chunk, in bounds) selected by value afterwards
        const v4i pad4 = {pv, pv, pv, pv};
        auto band_ld = [&](int e, int& at) -> v4i {
            const bool live = e < nch;
            const int pix = live ? e / cpp : 0, ch = live ? e - pix * cpp : 0;
            const int br = pix / bg.BW, bc = pix - br * bg.BW;
            const int iy = iy0 + br, ix = bc - a.PW;
            at = live ? pix * bg.PS + ch * 16 : -1;
            const bool in = live && (unsigned)iy < (unsigned)a.H &&
                            (unsigned)ix < (unsigned)a.W;
            const v4i l = *(const v4i*)(
                xn + (in ? ((int64_t)iy * a.W + ix) * a.x_sp + ch * 16 : 0));
            return in ? l : pad4;
        };
        for (int e0 = tid; e0 < nch; e0 += 4 * 256) {
            int a0, a1, a2, a3;
            const v4i v0 = band_ld(e0, a0), v1 = band_ld(e0 + 256, a1);
            const v4i v2 = band_ld(e0 + 512, a2), v3 = band_ld(e0 + 768, a3);
            if (a0 >= 0) *(v4i*)(s_x + a0) = v0;
            if (a1 >= 0) *(v4i*)(s_x + a1) = v1;
            if (a2 >= 0) *(v4i*)(s_x + a2) = v2;
            if (a3 >= 0) *(v4i*)(s_x + a3) = v3;
        }
        const int wch = WM * 16 * KGp;
        auto w_ld = [&](int e, int& at) -> v4i {
            const bool live = e < wch;
            const int r = live ? e / KGp : 0, k = live ? e - r * KGp : 0;
            at = live ? r * bg.RSW + k * 16 : -1;
            return *(const v4i*)(a.wp + (int64_t)(co0 + r) * a.wp_rstride +
                                 k * 16);
        };
        for (int e0 = tid; e0 < wch; e0 += 4 * 256) {
            int a0, a1, a2, a3;
            const v4i v0 = w_ld(e0, a0), v1 = w_ld(e0 + 256, a1);
            const v4i v2 = w_ld(e0 + 512, a2), v3 = w_ld(e0 + 768, a3);
            if (a0 >= 0) *(v4i*)(s_w + a0) = v0;
            if (a1 >= 0) *(v4i*)(s_w + a1) = v1;
            if (a2 >= 0) *(v4i*)(s_w + a2) = v2;
            if (a3 >= 0) *(v4i*)(s_w + a3) = v3;
        }
        for (int kg = tid; kg < KGp; kg += 256) {
            int off = -1;
            if (kg < a.KG) {
                const int tap = kg / a.CB, cb = kg - tap * a.CB;
                const int ky = tap / a.KW, kx = tap - ky * a.KW;
                off = (ky * a.DH * bg.BW + kx * a.DW) * bg.PS + cb * 16;
            }
            s_kt[kg] = off;
        }
        for (int i = tid; i < 768; i += 256)
            s_tab[i] = ((const int*)((const char*)a.plan + PLAN_E))[i];
    }
    const int4 hdr = *(const int4*)a.plan;
    int cm[WM], ct[WM];
    int64_t cc[WM];
    uint32_t ccorr[WM], cbo[WM];
#pragma unroll
    for (int i = 0; i < WM; ++i) {
        const int c = min(co0 + 16 * i + col, a.Cout - 1);
        const int4 pc = ((const int4*)((const char*)a.plan + PLAN_CH))[c];
        cm[i] = pc.x;
        ct[i] = pc.y;
        cc[i] = (int64_t)(((uint64_t)(uint32_t)pc.w << 32) | (uint32_t)pc.z);
        ccorr[i] = a.corr ? (uint32_t)a.corr[c] : 0u;
        cbo[i] = a.rowsum ? (uint32_t)a.boff[c] : 0u;
    }
    __syncthreads();

    // ---- the wave's TM tiles: lane pixel bases in the band ----
    int base[BAND_TM];
#pragma unroll
    for (int j = 0; j < BAND_TM; ++j) {
        const int q = min(16 * (wave + 4 * j) + col, npix - 1);
        const int r = q / a.OW, ox = q - r * a.OW;
        base[j] = (r * a.SH * bg.BW + ox * a.SW) * bg.PS;
    }
    v4i acc[BAND_TM][WM];
#pragma unroll
    for (int j = 0; j < BAND_TM; ++j)
#pragma unroll
        for (int i = 0; i < WM; ++i) acc[j][i] = v4i{0, 0, 0, 0};
    int psum[BAND_TM] = {0, 0, 0, 0};
    const v4i zero = {0, 0, 0, 0};
    for (int s = 0; s < KS; ++s) {
        const int off = s_kt[4 * s + kgl];
        v4i fa[BAND_TM], fb[WM];
#pragma unroll
        for (int j = 0; j < BAND_TM; ++j)
            fa[j] = off >= 0 ? *(const v4i*)(s_x + base[j] + off) : zero;
#pragma unroll
        for (int i = 0; i < WM; ++i)
            fb[i] = *(const v4i*)(s_w + (16 * i + col) * bg.RSW + 64 * s +
                                  16 * kgl);
#pragma unroll
        for (int j = 0; j < BAND_TM; ++j) {
            if (16 * (wave + 4 * j) >= npix) continue;  // past the band
#pragma unroll
            for (int i = 0; i < WM; ++i)
                acc[j][i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                    fa[j], fb[i], acc[j][i], 0, 0, 0);
        }
        if (a.rowsum) {
#pragma unroll
            for (int j = 0; j < BAND_TM; ++j)
                psum[j] += bytes_sum(fa[j], off >= 0 ? 16 : 0);
        }
    }

    // ---- epilogue (table plan): lane holds pixels 4 kgl + r of a tile ----
    const int pA = hdr.x, pB = hdr.y, pSH = hdr.z;
    const bool res = a.res != nullptr;
    const int64_t pimg = (int64_t)n * a.OH * a.OW + (int64_t)oy0 * a.OW;
#pragma unroll
    for (int j = 0; j < BAND_TM; ++j) {
        int ps[4] = {0, 0, 0, 0};
        if (a.rowsum) {
            int sj = psum[j];
            sj += __shfl_xor(sj, 16);
            sj += __shfl_xor(sj, 32);
#pragma unroll
            for (int r = 0; r < 4; ++r) ps[r] = __shfl(sj, 4 * kgl + r);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int q = 16 * (wave + 4 * j) + 4 * kgl + r;
            if (q >= npix) continue;
            const int64_t p = pimg + q;
#pragma unroll
            for (int i = 0; i < WM; ++i) {
                const int c = co0 + 16 * i + col;
                if (c >= a.Cout) continue;
                uint32_t wu = (uint32_t)acc[j][i][r] + ccorr[i];
                if (a.rowsum) wu += cbo[i] * (uint32_t)ps[r];
                const int q0 =
                    (int)(((int64_t)(int)wu * cm[i] + cc[i]) >> ct[i]);
                int e = min(max(q0, pA), pB) - pA;
                if (res) {
                    const int u =
                        (uint8_t)((const int8_t*)a.res)[p * a.res_pst + c];
                    e = min(max(s_tab[256 + e] + s_tab[512 + u], 0), pSH);
                }
                const int ev = s_tab[e];
                ((int8_t*)a.y)[p * a.y_pst + c] = (int8_t)(ev & 255);
                if (a.y2)
                    ((int8_t*)a.y2)[p * a.y2_pst + c] =
                        (int8_t)((ev >> 8) & 255);
            }
        }
    }
}

// Band geometry for `R` output rows; lds = 0 when it does not fit.
BandGeom band_geom(const ConvArgs& b, int wm, int R) {
    BandGeom g;
    g.R = R;
    g.BR = (R - 1) * b.SH + (b.KH - 1) * b.DH + 1;
    g.BW = (b.OW - 1) * b.SW + (b.KW - 1) * b.DW + 1;
    g.PS = b.Cg + (((b.Cg >> 4) & 1) ? 0 : 16);
    g.RSW = b.KGp * 16 + 16;
    g.nbands = (b.OH + R - 1) / R;
    const int64_t bytes = (int64_t)g.BR * g.BW * g.PS +
                          (int64_t)wm * 16 * g.RSW + (int64_t)b.KGp * 4;
    // gfx950 gives a work-group up to 160 KB; two work-groups a CU
    g.lds = bytes <= 76 * 1024 ? (int)bytes : 0;
    return g;
}

}  // namespace

bool conv_band_applies(const ConvArgs& b, int epi, int wm) {
    const uintptr_t xa = (uintptr_t)b.x;
    if (!(epi == Q8_TABLE && b.mode == EPI_QUANT && b.fastio && b.plan &&
          b.G == 1 && b.layout == 0 && b.x_code == 1 && b.x_sc == 1 &&
          b.Cg % 16 == 0 && b.Cg > 0 && xa % 16 == 0 && b.x_sp % 16 == 0 &&
          b.x_sn % 16 == 0 && b.y_code == 1 && b.OW <= 16 * 4 * BAND_TM &&
          b.M < ((int64_t)1 << 31) && b.N * (int64_t)b.OH < (1 << 30)))
        return false;
    return band_geom(b, wm, 1).lds > 0;
}

bool launch_conv_band(const ConvArgs& b, int wm, hipStream_t st) {
    if (wm != 1 && wm != 2 && wm != 4) wm = 4;
    // the most rows whose pixels fill at most the 4 waves x TM tiles and
    // whose band fits in LDS
    int R = 1;
    while (R < b.OH && (R + 1) * b.OW <= 16 * 4 * BAND_TM &&
           band_geom(b, wm, R + 1).lds > 0)
        ++R;
    const BandGeom g = band_geom(b, wm, R);
    if (g.lds == 0) {
        set_error("launch_conv_band", "band does not fit in LDS");
        return false;
    }
    const int64_t gx = (int64_t)b.N * g.nbands;
    const int64_t gy = ceil_div(b.Cout, 16 * wm);
    if (gx >= ((int64_t)1 << 31) || gy > 65535) {
        set_error("launch_conv_band", "grid too large");
        return false;
    }
    const dim3 grid((unsigned)gx, (unsigned)gy);
    switch (wm) {
        case 1: k_conv_band<1><<<grid, 256, g.lds, st>>>(b, g); break;
        case 2: k_conv_band<2><<<grid, 256, g.lds, st>>>(b, g); break;
        default: k_conv_band<4><<<grid, 256, g.lds, st>>>(b, g); break;
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_hip_error("launch_conv_band", e);
        return false;
    }
    return true;
}

}  // namespace qa

// Two chained 3x3 convolutions in one launch: y = f2(f1(x)) (+ residual),
// the bottleneck of a C2f block (3x3 stride-1 conv, SiLU, 3x3 conv, SiLU,
// Add of the block input), each conv C -> C channels with C in {16, 32, 64}
// (and 128: k_conv_pair_cs below).
//
// A work-group owns R output rows of one image and all C channels. It
// stages in LDS, with every load of a thread in flight before its stores:
// the input rows oy0 - 2 .. oy0 + R + 1 (the image padding holds conv 1's
// pad value), and both convs' packed weight rows. Phase 1 computes conv 1
// over the intermediate rows oy0 - 1 .. oy0 + R that lie inside the image
// (halo rows are recomputed by the neighbouring bands) and writes its
// stored bytes (table epilogue) into a second LDS band whose image padding
// holds conv 2's pad value; the intermediate tensor never goes to HBM.
// Phase 2 computes conv 2 from that band with the full table epilogue
// (residual Add from HBM, rescaled copy) and stores the output words.
// Each phase holds its conv's weight fragments in VGPRs (C/16 channel tiles
// x KS K-steps) and reads only the activation fragment from LDS per K-step;
// v_mfma_i32_16x16x64_i8 with 16 pixels as rows and 16 channels as
// columns, the k-group layout of the packed layout-0 weights (tap kg / CB,
// channels 16 (kg % CB) ..), one k-group offset table for both bands (same
// width and pixel stride).
//
// TAIL (C 16/32): the C2f block's last 1x1 convolution (cv2) runs in the
// same launch. Its input is the block's Concat, whose last C channels are
// this pair's output or its rescaled second output, and whose other
// channels (the prefix) earlier launches wrote. The band's output pixels' prefix channels are staged in LDS with
// everything else; per phase-2 tile conv 2's output words also go to a
// per-wave LDS tile (16 pixels x C bytes), and cv2's MFMAs read their
// fragments from those two, with cv2's weights staged in LDS; cv2's table
// epilogue stores its output. cv2 is a separate launch otherwise, and for
// C = 64, where the pair's weights leave too little LDS for cv2's weights
// and bands of more than two rows (every extra band stages all weights
// again: slower than the two launches).
#include "qa_conv_mfma.h"

namespace qa {
namespace {

constexpr int CP_NW = 8;           // waves per work-group
constexpr int CP_NT = 64 * CP_NW;  // threads per work-group
constexpr int CP_SB = 8;           // band chunks (16 bytes) a thread stages
constexpr int CP_SW = 5;           // weight chunks a thread stages per conv

struct PairGeom {
    int R;                 // output rows per band
    int BW, PS;            // band width (pixels) and pixel bytes in LDS
    int bpi, nbands;       // bands per image, in all
    int xb_bytes;          // input band (R + 4 rows)
    int mb_bytes;          // intermediate band (R + 2 rows)
    int RSW;               // LDS row stride of the staged weights
    int lds;               // dynamic LDS bytes (0: does not fit)
    uint32_t m_w, m_bw, m_kgp;  // ceil(2^32 / d), d >= 2
    // TAIL: cv2's weights (T3 16-channel blocks, rows of RSW3 bytes, KS3
    // K-steps), the per-wave tiles (16 rows of RT bytes) and the band's
    // prefix channels (rows of RP bytes a pixel) in LDS, at these offsets;
    // the pair's output (t_y2: its second output) is Concat channels off_d ..
    int t_w3, t_tile, t_pre, RSW3, KS3, T3, RT, RP, off_d, Ctot, t_y2;
    uint32_t m_kgp3;
};

__device__ __forceinline__ int cp_div(int n, uint32_t m) {
    return (int)__umulhi((uint32_t)n, m);
}

// WM <= 2: at most 128 VGPRs, so that two work-groups share a CU
template <int WM, bool RES, bool TAIL>
__global__ __launch_bounds__(CP_NT)
__attribute__((amdgpu_waves_per_eu(WM <= 2 ? 4 : 1))) void k_conv_pair(
    ConvArgs a1, ConvArgs a2, PairGeom g, ConvArgs a3) {
    constexpr int C = 16 * WM;          // channels of every tensor
    constexpr int KS = (9 * WM + 3) / 4;  // K-steps: KGp = round_up(9 WM, 4)
    constexpr int LCPP = WM == 1 ? 0 : WM == 2 ? 1 : 2;  // log2 chunks/pixel
    extern __shared__ int4 lds4[];
    int8_t* s_x = (int8_t*)lds4;         // input band
    int8_t* s_m = s_x + g.xb_bytes;      // intermediate band
    int8_t* s_w1 = s_m + g.mb_bytes;     // conv 1 weights: C rows x RSW
    int8_t* s_w2 = s_w1 + C * g.RSW;     // conv 2 weights
    int* s_kt = (int*)(s_w2 + C * g.RSW);  // 4 KS k-group offsets
    __shared__ int s_tab1[256];
    __shared__ int s_tab2[768];
    __shared__ int4 s_pc[2][C];
    __shared__ uint32_t s_corr[2][C];
    __shared__ int s_tab3[TAIL ? 256 : 1];
    __shared__ int4 s_pc3[TAIL ? 128 : 1];
    int8_t* s_w3 = (int8_t*)lds4 + g.t_w3;    // TAIL: cv2's weights
    int8_t* s_t = (int8_t*)lds4 + g.t_tile;   // TAIL: per-wave tiles
    int8_t* s_pre = (int8_t*)lds4 + g.t_pre;  // TAIL: the band's prefix
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 15, kgl = lane >> 4;
    const int KGp = 4 * KS;
    const int W = a1.W, OW = a2.OW, OH = a2.OH;
    const int band = blockIdx.x;
    const int n = band / g.bpi;
    const int oy0 = (band - n * g.bpi) * g.R;
    const int R = min(g.R, OH - oy0);   // output rows of this band
    const int iy0 = oy0 - 2;            // image row of input band row 0
    const int BR = R + 4;               // input band rows
    const int MR = R + 2;               // intermediate band rows
    const int pv1 = splat4(a1.pad_value), pv2 = splat4(a2.pad_value);
    const v4i pad1 = {pv1, pv1, pv1, pv1}, pad2 = {pv2, pv2, pv2, pv2};

    // ---- staging: input rows inside the image as one run of pixels from
    // row iy0 + r_lo (chunk e: pixel e / C16, part e % C16, at band row
    // r_lo + p / W, column 1 + p % W), then the weight rows of both convs
    // (chunk e: row e / KGp, part e % KGp); all loads before the stores
    const int r_lo = max(0, -iy0), r_hi = min(BR, a1.H - iy0);
    const int nreal = max(r_hi - r_lo, 0) * W * WM;
    const int wch = C * KGp;
    {
        v4i vx[CP_SB], w1[CP_SW], w2[CP_SW];
        int ax[CP_SB], aw[CP_SW];
        {
            const int xsp = (int)a1.x_sp;
            const int8_t* xrow = (const int8_t*)a1.x + (int64_t)n * a1.x_sn +
                                 (int64_t)(iy0 + r_lo) * W * a1.x_sp;
            const int ch = tid & (WM - 1);  // the same part for every u
#pragma unroll
            for (int u = 0; u < CP_SB; ++u) {
                const int e = tid + u * CP_NT;
                const int p = e >> LCPP;
                const int row = cp_div(p, g.m_w), ix = p - row * W;
                const bool ok = e < nreal;
                ax[u] = ok ? ((r_lo + row) * g.BW + ix + 1) * g.PS + ch * 16
                           : -1;
                vx[u] = *(const v4i*)(xrow + (ok ? p * xsp + ch * 16 : 0));
            }
        }
        {
            const int rs1 = (int)a1.wp_rstride, rs2 = (int)a2.wp_rstride;
#pragma unroll
            for (int u = 0; u < CP_SW; ++u) {
                const int e = tid + u * CP_NT;
                const int r = cp_div(e, g.m_kgp), k = e - r * KGp;
                const bool ok = e < wch;
                aw[u] = ok ? r * g.RSW + k * 16 : -1;
                w1[u] = *(const v4i*)(a1.wp + (ok ? r * rs1 + k * 16 : 0));
                w2[u] = *(const v4i*)(a2.wp + (ok ? r * rs2 + k * 16 : 0));
            }
        }
        // TAIL: the first round of cv2's weight rows and of the band's
        // prefix channels, cv2's table entry and constants, requested with
        // the loads above (each later round would be one more memory
        // round trip before the first MFMA); NE chunks a thread a round
        // (C 32: one, to keep the registers within 4 waves a SIMD)
        constexpr bool EARLY = TAIL && WM <= 2;
        constexpr int NE = WM == 1 ? 4 : 1;
        const int kgp3 = TAIL ? 4 * g.KS3 : 0;
        const int n3 = TAIL ? 16 * g.T3 * kgp3 : 0;
        const int cpp3 = TAIL ? g.off_d >> 4 : 1;
        const int np3 = TAIL ? R * OW * cpp3 : 0;
        const int8_t* xp3 =
            TAIL ? (const int8_t*)a3.x + ((int64_t)n * OH + oy0) * OW * a3.x_sp
                 : nullptr;
        v4i w3[NE], pv3[NE];
        int a3w[NE], ap3[NE];
        int tv3 = 0;
        int4 pc3v = int4{0, 0, 0, 0};
        uint32_t corr3v = 0;
        auto load_w3 = [&](int e0) __attribute__((always_inline)) {
            const int rs3 = (int)a3.wp_rstride;
#pragma unroll
            for (int u = 0; u < NE; ++u) {
                const int e = e0 + u * CP_NT;
                const int r = cp_div(e, g.m_kgp3), k = e - r * kgp3;
                const bool ok = e < n3;
                a3w[u] = ok ? r * g.RSW3 + k * 16 : -1;
                w3[u] = *(const v4i*)(a3.wp + (ok ? r * rs3 + k * 16 : 0));
            }
        };
        auto load_pre = [&](int e0) __attribute__((always_inline)) {
#pragma unroll
            for (int u = 0; u < NE; ++u) {
                const int e = e0 + u * CP_NT;
                const bool ok = e < np3;
                const int px = ok ? e / cpp3 : 0, c = ok ? e - px * cpp3 : 0;
                ap3[u] = ok ? px * g.RP + c * 16 : -1;
                pv3[u] = *(const v4i*)(xp3 + (int64_t)px * a3.x_sp + c * 16);
            }
        };
        if constexpr (EARLY) {
            load_w3(tid);
            load_pre(tid);
            tv3 = ((const int*)((const char*)a3.plan + PLAN_E))[tid & 255];
            const int cl = min(tid, a3.Cout - 1);
            pc3v = ((const int4*)((const char*)a3.plan + PLAN_CH))[cl];
            corr3v = a3.corr ? (uint32_t)a3.corr[cl] : 0u;
        }
        // pad values: input band rows outside the image and its two pad
        // columns; intermediate rows outside the image and its pad columns
        for (int e = tid; e < BR * g.BW * WM; e += CP_NT) {
            const int p = e >> LCPP, ch = e & (WM - 1);
            const int row = cp_div(p, g.m_bw), c = p - row * g.BW;
            if (row < r_lo || row >= r_hi || c == 0 || c == g.BW - 1)
                *(v4i*)(s_x + p * g.PS + ch * 16) = pad1;
        }
        for (int e = tid; e < MR * g.BW * WM; e += CP_NT) {
            const int p = e >> LCPP, ch = e & (WM - 1);
            const int row = cp_div(p, g.m_bw), c = p - row * g.BW;
            const int my = oy0 - 1 + row;
            if ((unsigned)my >= (unsigned)OH || c == 0 || c == g.BW - 1)
                *(v4i*)(s_m + p * g.PS + ch * 16) = pad2;
        }
        for (int kg = tid; kg < KGp; kg += CP_NT) {
            int off = 0;  // padding k-groups: any in-band address
            if (kg < 9 * WM) {
                const int tap = kg / WM, cb = kg - tap * WM;
                const int ky = tap / 3, kx = tap - ky * 3;
                off = (ky * g.BW + kx) * g.PS + cb * 16;
            }
            s_kt[kg] = off;
        }
        for (int i = tid; i < 256; i += CP_NT)
            s_tab1[i] = ((const int*)((const char*)a1.plan + PLAN_E))[i];
        for (int i = tid; i < 768; i += CP_NT)
            s_tab2[i] = ((const int*)((const char*)a2.plan + PLAN_E))[i];
        if (tid < C) {
            s_pc[0][tid] = ((const int4*)((const char*)a1.plan + PLAN_CH))[tid];
            s_corr[0][tid] = a1.corr ? (uint32_t)a1.corr[tid] : 0u;
        } else if (tid < 2 * C) {
            const int c = tid - C;
            s_pc[1][c] = ((const int4*)((const char*)a2.plan + PLAN_CH))[c];
            s_corr[1][c] = a2.corr ? (uint32_t)a2.corr[c] : 0u;
        }
#pragma unroll
        for (int u = 0; u < CP_SB; ++u)
            if (ax[u] >= 0) *(v4i*)(s_x + ax[u]) = vx[u];
#pragma unroll
        for (int u = 0; u < CP_SW; ++u)
            if (aw[u] >= 0) {
                *(v4i*)(s_w1 + aw[u]) = w1[u];
                *(v4i*)(s_w2 + aw[u]) = w2[u];
            }
        if constexpr (TAIL) {  // cv2's weights, table, constants
            for (int e0 = tid; e0 < n3; e0 += NE * CP_NT) {
                if (!EARLY || e0 != tid) load_w3(e0);
#pragma unroll
                for (int u = 0; u < NE; ++u)
                    if (a3w[u] >= 0) *(v4i*)(s_w3 + a3w[u]) = w3[u];
            }
            // the prefix channels of the band's output pixels
            for (int e0 = tid; e0 < np3; e0 += NE * CP_NT) {
                if (!EARLY || e0 != tid) load_pre(e0);
#pragma unroll
                for (int u = 0; u < NE; ++u)
                    if (ap3[u] >= 0) *(v4i*)(s_pre + ap3[u]) = pv3[u];
            }
            if (!EARLY) {
                tv3 = ((const int*)((const char*)a3.plan + PLAN_E))[tid & 255];
                const int cl = min(tid, a3.Cout - 1);
                pc3v = ((const int4*)((const char*)a3.plan + PLAN_CH))[cl];
                corr3v = a3.corr ? (uint32_t)a3.corr[cl] : 0u;
            }
            if (tid < 256) s_tab3[tid] = tv3;
            if (tid < 16 * g.T3) {  // the correction folded in (plan_q0)
                const uint64_t cf = (uint64_t)plan_fold(
                    (int64_t)(((uint64_t)(uint32_t)pc3v.w << 32) |
                              (uint32_t)pc3v.z),
                    corr3v, pc3v.x);
                s_pc3[tid] = int4{pc3v.x, pc3v.y, (int)(uint32_t)cf,
                                  (int)(uint32_t)(cf >> 32)};
            }
        }
    }
    __syncthreads();

    const int q = lane & 3;
    const uint32_t sel1 = q < 2 ? 0x05040100u : 0x03020706u;
    const uint32_t sel2 = (q & 1) ? 0x03070105u : 0x06020400u;
    const int cq = col & ~3;
    int kt[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) kt[s] = s_kt[4 * s + kgl];
    v4i wb[KS][WM];
    int cm[WM], ct[WM];
    int64_t cc[WM];  // the plan constant with the correction folded in
    auto load_conv = [&](const int8_t* s_w, int which) {
#pragma unroll
        for (int s = 0; s < KS; ++s)
#pragma unroll
            for (int i = 0; i < WM; ++i)
                wb[s][i] = *(const v4i*)(s_w + (16 * i + col) * g.RSW +
                                         64 * s + 16 * kgl);
#pragma unroll
        for (int i = 0; i < WM; ++i) {
            const int4 pc = s_pc[which][16 * i + col];
            cm[i] = pc.x;
            ct[i] = pc.y;
            cc[i] = plan_fold((int64_t)(((uint64_t)(uint32_t)pc.w << 32) |
                                        (uint32_t)pc.z),
                              s_corr[which][16 * i + col], pc.x);
            // opaque, so that each value is one 32x32 -> 64 multiply-add
            // instead of a re-associated 64-bit product
            asm volatile("" : "+v"(cc[i]));
        }
    };
    // accumulators of the 16 pixels whose band base offsets are xb
    auto tile_mfma = [&](const int8_t* xb, v4i (&acc)[WM]) {
#pragma unroll
        for (int i = 0; i < WM; ++i) acc[i] = v4i{0, 0, 0, 0};
        v4i fa[KS];
#pragma unroll
        for (int s = 0; s < KS; ++s) fa[s] = *(const v4i*)(xb + kt[s]);
#pragma unroll
        for (int s = 0; s < KS; ++s)
#pragma unroll
            for (int i = 0; i < WM; ++i)
                acc[i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                    fa[s], wb[s][i], acc[i], 0, 0, 0);
    };

    // ---- phase 1: conv 1 over the intermediate rows inside the image ----
    load_conv(s_w1, 0);
    {
        const int4 h1 = *(const int4*)a1.plan;
        const int mr_lo = max(0, 1 - oy0), mr_hi = min(MR, OH + 1 - oy0);
        const int npix = (mr_hi - mr_lo) * OW;
        const int ntile = (npix + 15) >> 4;
        for (int t = wave; t < ntile; t += CP_NW) {
            const int qp = mr_lo * OW + min(16 * t + col, npix - 1);
            const int mr = cp_div(qp, g.m_w), mc = qp - mr * OW;
            v4i acc[WM];
            tile_mfma(s_x + (mr * g.BW + mc) * g.PS, acc);
            // lane q stores pixel 16 t + 4 kgl + q, channels 16 i + cq ..
            const int pq = 16 * t + 4 * kgl + q;
            const bool pok = pq < npix;
            const int sq = mr_lo * OW + min(pq, npix - 1);
            const int sr = cp_div(sq, g.m_w), sc = sq - sr * OW;
            int8_t* dst = s_m + (sr * g.BW + sc + 1) * g.PS + cq;
#pragma unroll
            for (int i = 0; i < WM; ++i) {
                int e[4];
#pragma unroll
                for (int rr = 0; rr < 4; ++rr)
                    e[rr] = s_tab1[med3_i32(plan_q0(acc[i][rr], cm[i], cc[i],
                                                    ct[i]),
                                            h1.x, h1.y) -
                                   h1.x];
                const uint32_t wy =
                    quad_transpose(pack_entries(e, 0), sel1, sel2);
                if (pok) *(uint32_t*)(dst + 16 * i) = wy;
            }
        }
    }
    __syncthreads();

    // ---- phase 2: conv 2 over the band's output rows ----
    load_conv(s_w2, 1);
    {
        const int4 h2 = *(const int4*)a2.plan;
        const int pA = h2.x, pB = h2.y, pSH = h2.z;
        const int npix = R * OW;
        const int ntile = (npix + 15) >> 4;
        const int64_t pimg = ((int64_t)n * OH + oy0) * OW;
        for (int t = wave; t < ntile; t += CP_NW) {
            const int pq = 16 * t + 4 * kgl + q;  // pixel this lane stores
            const bool pok = pq < npix;
            const int64_t p = pimg + min(pq, npix - 1);
            uint32_t rw[WM];
            if (RES) {
                const int8_t* pr = (const int8_t*)a2.res + p * a2.res_pst;
#pragma unroll
                for (int i = 0; i < WM; ++i)
                    rw[i] = *(const uint32_t*)(pr + 16 * i + cq);
            }
            const int qp = min(16 * t + col, npix - 1);
            const int r = cp_div(qp, g.m_w), ox = qp - r * OW;
            v4i acc[WM];
            tile_mfma(s_m + (r * g.BW + ox) * g.PS, acc);
            int8_t* tw = s_t + wave * 16 * g.RT;  // TAIL: the wave's tile
#pragma unroll
            for (int i = 0; i < WM; ++i) {
                int e[4];
#pragma unroll
                for (int rr = 0; rr < 4; ++rr)
                    e[rr] = med3_i32(plan_q0(acc[i][rr], cm[i], cc[i], ct[i]),
                                     pA, pB) -
                            pA;
                if (RES) {
                    const uint32_t rv = quad_transpose(rw[i], sel1, sel2);
#pragma unroll
                    for (int rr = 0; rr < 4; ++rr) {
                        const int v = s_tab2[256 + e[rr]] +
                                      s_tab2[512 + ((rv >> (8 * rr)) & 255)];
                        e[rr] = med3_i32(v, 0, pSH);
                    }
                }
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) e[rr] = s_tab2[e[rr]];
                const int c0 = 16 * i + cq;
                const uint32_t wy =
                    quad_transpose(pack_entries(e, 0), sel1, sel2);
                if (pok) *(uint32_t*)((int8_t*)a2.y + p * a2.y_pst + c0) = wy;
                uint32_t w2 = 0;
                if (a2.y2) {
                    w2 = quad_transpose(pack_entries(e, 1), sel1, sel2);
                    if (pok)
                        *(uint32_t*)((int8_t*)a2.y2 + p * a2.y2_pst + c0) = w2;
                }
                if (TAIL)
                    *(uint32_t*)(tw + (4 * kgl + q) * g.RT + c0) =
                        g.t_y2 ? w2 : wy;
            }
            if (TAIL) {
                // the wave's tile words before its reads of them
                __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
                const int4 h3 = *(const int4*)a3.plan;
                constexpr int TJ = 4;  // cv2's channel blocks at a time
                for (int j0 = 0; j0 < g.T3; j0 += TJ) {
                    v4i acc3[TJ];
#pragma unroll
                    for (int j = 0; j < TJ; ++j) acc3[j] = v4i{0, 0, 0, 0};
#pragma unroll
                    for (int s3 = 0; s3 < 4; ++s3) {
                        if (s3 >= g.KS3) continue;
                        // row col of the tile: pixel qp of the band; past
                        // the Concat's channels the weights are zero and
                        // any bytes do (the tile's last chunk is read)
                        const int c16 = (4 * s3 + kgl) * 16;
                        const int8_t* src3 =
                            c16 < g.off_d
                                ? s_pre + qp * g.RP + c16
                                : tw + col * g.RT +
                                      min(c16, g.Ctot - 16) - g.off_d;
                        const v4i fa3 = *(const v4i*)src3;
#pragma unroll
                        for (int j = 0; j < TJ; ++j)
                            if (j0 + j < g.T3)
                                acc3[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                                    fa3,
                                    *(const v4i*)(s_w3 +
                                                  (16 * (j0 + j) + col) *
                                                      g.RSW3 +
                                                  64 * s3 + 16 * kgl),
                                    acc3[j], 0, 0, 0);
                    }
#pragma unroll
                    for (int j = 0; j < TJ; ++j) {
                        const int c3 = 16 * (j0 + j) + cq;
                        if (j0 + j >= g.T3) continue;
                        const int4 pc3 = s_pc3[16 * (j0 + j) + col];
                        const int64_t cc3 =
                            (int64_t)(((uint64_t)(uint32_t)pc3.w << 32) |
                                      (uint32_t)pc3.z);
                        int e3[4];
#pragma unroll
                        for (int rr = 0; rr < 4; ++rr)
                            e3[rr] = s_tab3[med3_i32(
                                             plan_q0(acc3[j][rr], pc3.x, cc3,
                                                     pc3.y),
                                             h3.x, h3.y) -
                                             h3.x];
                        const uint32_t wy3 =
                            quad_transpose(pack_entries(e3, 0), sel1, sel2);
                        if (pok && c3 < a3.Cout)
                            *(uint32_t*)((int8_t*)a3.y + p * a3.y_pst + c3) =
                                wy3;
                    }
                }
                // this tile's reads before the next tile's words
                __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
            }
        }
    }
}

// The 128-channel form (8 channel tiles): both weight sets (2 x 150 KB)
// exceed LDS, so the 8 waves split the channels instead of the tiles: wave
// w owns channels 16 w .. 16 w + 15 of both convs, loads its weight
// fragments of conv 1 (18 K-steps) straight from L2 into VGPRs while the
// band is staged and those of conv 2 during phase 1, and walks every tile
// of the band in both phases (all waves read the same activation
// fragments from LDS). Staging, bands, tables and epilogues as above.
template <bool RES>
__global__ __launch_bounds__(CP_NT) void k_conv_pair_cs(ConvArgs a1,
                                                        ConvArgs a2,
                                                        PairGeom g,
                                                        ConvArgs) {
    constexpr int WM = 8, C = 128, KS = 18, LCPP = 3;
    extern __shared__ int4 lds4[];
    int8_t* s_x = (int8_t*)lds4;         // input band
    int8_t* s_m = s_x + g.xb_bytes;      // intermediate band
    int* s_kt = (int*)(s_m + g.mb_bytes);  // 4 KS k-group offsets
    __shared__ int s_tab1[256];
    __shared__ int s_tab2[768];
    __shared__ int4 s_pc[2][C];
    __shared__ uint32_t s_corr[2][C];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 15, kgl = lane >> 4;
    const int KGp = 4 * KS;
    const int W = a1.W, OW = a2.OW, OH = a2.OH;
    const int band = blockIdx.x;
    const int n = band / g.bpi;
    const int oy0 = (band - n * g.bpi) * g.R;
    const int R = min(g.R, OH - oy0);
    const int iy0 = oy0 - 2;
    const int BR = R + 4, MR = R + 2;
    const int pv1 = splat4(a1.pad_value), pv2 = splat4(a2.pad_value);
    const v4i pad1 = {pv1, pv1, pv1, pv1}, pad2 = {pv2, pv2, pv2, pv2};
    const int co = 16 * wave + col;  // this lane's weight row (both convs)
    // conv 1's weight fragments, in flight with the band's loads
    // a weight fragment: one contiguous KB a wave load from the
    // fragment-order copy (ConvArgs.wfrag; the wave's tile, K-step s at
    // 1 KB s), else 16 rows x 64 bytes of the packed rows (half lines:
    // their loads arrive about 2.5x slower)
    auto wfrag = [&](const ConvArgs& a, int& st) {
        st = a.wfrag ? 1024 : 64;
        return a.wfrag ? a.wfrag + (int64_t)wave * KS * 1024 + 16 * lane
                       : a.wp + (int64_t)co * a.wp_rstride + 16 * kgl;
    };
    int wst1;
    const int8_t* wp1 = wfrag(a1, wst1);
    v4i wb[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) wb[s] = *(const v4i*)(wp1 + wst1 * s);
    const int r_lo = max(0, -iy0), r_hi = min(BR, a1.H - iy0);
    const int nreal = max(r_hi - r_lo, 0) * W * WM;
    {
        v4i vx[CP_SB];
        int ax[CP_SB];
        const int xsp = (int)a1.x_sp;
        const int8_t* xrow = (const int8_t*)a1.x + (int64_t)n * a1.x_sn +
                             (int64_t)(iy0 + r_lo) * W * a1.x_sp;
        const int ch = tid & (WM - 1);
#pragma unroll
        for (int u = 0; u < CP_SB; ++u) {
            const int e = tid + u * CP_NT;
            const int p = e >> LCPP;
            const int row = cp_div(p, g.m_w), ix = p - row * W;
            const bool ok = e < nreal;
            ax[u] = ok ? ((r_lo + row) * g.BW + ix + 1) * g.PS + ch * 16 : -1;
            vx[u] = *(const v4i*)(xrow + (ok ? p * xsp + ch * 16 : 0));
        }
        for (int e = tid; e < BR * g.BW * WM; e += CP_NT) {
            const int p = e >> LCPP, c = e & (WM - 1);
            const int row = cp_div(p, g.m_bw), cc = p - row * g.BW;
            if (row < r_lo || row >= r_hi || cc == 0 || cc == g.BW - 1)
                *(v4i*)(s_x + p * g.PS + c * 16) = pad1;
        }
        for (int e = tid; e < MR * g.BW * WM; e += CP_NT) {
            const int p = e >> LCPP, c = e & (WM - 1);
            const int row = cp_div(p, g.m_bw), cc = p - row * g.BW;
            const int my = oy0 - 1 + row;
            if ((unsigned)my >= (unsigned)OH || cc == 0 || cc == g.BW - 1)
                *(v4i*)(s_m + p * g.PS + c * 16) = pad2;
        }
        for (int kg = tid; kg < KGp; kg += CP_NT) {
            const int tap = kg / WM, cb = kg - tap * WM;  // 72 = 9 x 8 real
            const int ky = tap / 3, kx = tap - ky * 3;
            s_kt[kg] = (ky * g.BW + kx) * g.PS + cb * 16;
        }
        for (int i = tid; i < 256; i += CP_NT)
            s_tab1[i] = ((const int*)((const char*)a1.plan + PLAN_E))[i];
        for (int i = tid; i < 768; i += CP_NT)
            s_tab2[i] = ((const int*)((const char*)a2.plan + PLAN_E))[i];
        if (tid < C) {
            s_pc[0][tid] = ((const int4*)((const char*)a1.plan + PLAN_CH))[tid];
            s_corr[0][tid] = a1.corr ? (uint32_t)a1.corr[tid] : 0u;
        } else if (tid < 2 * C) {
            const int c = tid - C;
            s_pc[1][c] = ((const int4*)((const char*)a2.plan + PLAN_CH))[c];
            s_corr[1][c] = a2.corr ? (uint32_t)a2.corr[c] : 0u;
        }
#pragma unroll
        for (int u = 0; u < CP_SB; ++u)
            if (ax[u] >= 0) *(v4i*)(s_x + ax[u]) = vx[u];
    }
    __syncthreads();

    const int q = lane & 3;
    const uint32_t sel1 = q < 2 ? 0x05040100u : 0x03020706u;
    const uint32_t sel2 = (q & 1) ? 0x03070105u : 0x06020400u;
    const int cq = col & ~3;
    int kt[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) kt[s] = s_kt[4 * s + kgl];
    auto consts = [&](int which, int& cm, int& ct, int64_t& cc,
                      uint32_t& cr) {
        const int4 pc = s_pc[which][co];
        cm = pc.x;
        ct = pc.y;
        cr = s_corr[which][co];
        // the correction folded into the constant (plan_q0)
        cc = plan_fold(
            (int64_t)(((uint64_t)(uint32_t)pc.w << 32) | (uint32_t)pc.z), cr,
            pc.x);
        asm volatile("" : "+v"(cc));  // one multiply-add a value (above)
    };
    auto tile_acc = [&](const int8_t* xb, const v4i (&w)[KS]) {
        v4i fa[KS];
#pragma unroll
        for (int s = 0; s < KS; ++s) fa[s] = *(const v4i*)(xb + kt[s]);
        v4i acc = {0, 0, 0, 0};
#pragma unroll
        for (int s = 0; s < KS; ++s)
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[s], w[s], acc, 0,
                                                        0, 0);
        return acc;
    };

    // ---- phase 1 (conv 2's weights in flight) ----
    int wst2;
    const int8_t* wp2 = wfrag(a2, wst2);
    v4i wb2[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) wb2[s] = *(const v4i*)(wp2 + wst2 * s);
    {
        int cm, ct;
        int64_t cc;
        uint32_t cr;
        consts(0, cm, ct, cc, cr);
        const int4 h1 = *(const int4*)a1.plan;
        const int mr_lo = max(0, 1 - oy0), mr_hi = min(MR, OH + 1 - oy0);
        const int npix = (mr_hi - mr_lo) * OW;
        const int ntile = (npix + 15) >> 4;
        for (int t = 0; t < ntile; ++t) {
            const int qp = mr_lo * OW + min(16 * t + col, npix - 1);
            const int mr = cp_div(qp, g.m_w), mc = qp - mr * OW;
            const v4i acc = tile_acc(s_x + (mr * g.BW + mc) * g.PS, wb);
            const int pq = 16 * t + 4 * kgl + q;
            const int sq = mr_lo * OW + min(pq, npix - 1);
            const int sr = cp_div(sq, g.m_w), sc = sq - sr * OW;
            int e[4];
#pragma unroll
            for (int rr = 0; rr < 4; ++rr)
                e[rr] = s_tab1[med3_i32(plan_q0(acc[rr], cm, cc, ct), h1.x,
                                        h1.y) -
                               h1.x];
            const uint32_t wy = quad_transpose(pack_entries(e, 0), sel1, sel2);
            if (pq < npix)
                *(uint32_t*)(s_m + (sr * g.BW + sc + 1) * g.PS + 16 * wave +
                             cq) = wy;
        }
    }
    __syncthreads();

    // ---- phase 2 ----
    {
        int cm, ct;
        int64_t cc;
        uint32_t cr;
        consts(1, cm, ct, cc, cr);
        const int4 h2 = *(const int4*)a2.plan;
        const int pA = h2.x, pB = h2.y, pSH = h2.z;
        const int npix = R * OW;
        const int ntile = (npix + 15) >> 4;
        const int64_t pimg = ((int64_t)n * OH + oy0) * OW;
        const int c0 = 16 * wave + cq;
        for (int t = 0; t < ntile; ++t) {
            const int pq = 16 * t + 4 * kgl + q;
            const bool pok = pq < npix;
            const int64_t p = pimg + min(pq, npix - 1);
            uint32_t rw = 0;
            if (RES)
                rw = *(const uint32_t*)((const int8_t*)a2.res +
                                        p * a2.res_pst + c0);
            const int qp = min(16 * t + col, npix - 1);
            const int r = cp_div(qp, g.m_w), ox = qp - r * OW;
            const v4i acc = tile_acc(s_m + (r * g.BW + ox) * g.PS, wb2);
            int e[4];
#pragma unroll
            for (int rr = 0; rr < 4; ++rr)
                e[rr] = med3_i32(plan_q0(acc[rr], cm, cc, ct), pA, pB) - pA;
            if (RES) {
                const uint32_t rv = quad_transpose(rw, sel1, sel2);
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) {
                    const int v = s_tab2[256 + e[rr]] +
                                  s_tab2[512 + ((rv >> (8 * rr)) & 255)];
                    e[rr] = med3_i32(v, 0, pSH);
                }
            }
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) e[rr] = s_tab2[e[rr]];
            const uint32_t wy = quad_transpose(pack_entries(e, 0), sel1, sel2);
            if (pok) *(uint32_t*)((int8_t*)a2.y + p * a2.y_pst + c0) = wy;
            if (a2.y2) {
                const uint32_t w2 =
                    quad_transpose(pack_entries(e, 1), sel1, sel2);
                if (pok) *(uint32_t*)((int8_t*)a2.y2 + p * a2.y2_pst + c0) = w2;
            }
        }
    }
}

uint32_t cp_magic(int64_t d) {
    return (uint32_t)((((uint64_t)1 << 32) + (uint64_t)d - 1) /
                      (uint64_t)std::max<int64_t>(d, 2));
}

// Geometry for bands of R output rows (with b3: and cv2's tail); lds = 0
// when it does not fit or the staging exceeds what the threads hold.
PairGeom pair_geom(const ConvArgs& b, int R, const ConvArgs* b3 = nullptr) {
    const int C = b.Cg, wm = C / 16;
    PairGeom g;
    g.R = R;
    g.BW = b.W + 2;
    g.PS = C + ((wm & 1) ? 0 : 16);
    g.bpi = (b.OH + R - 1) / R;
    g.nbands = b.N * g.bpi;
    g.RSW = b.KGp * 16 + 16;
    const int64_t xb = (int64_t)(R + 4) * g.BW * g.PS;
    const int64_t mb = (int64_t)(R + 2) * g.BW * g.PS;
    g.xb_bytes = (int)std::min<int64_t>(xb, 1 << 30);
    g.mb_bytes = (int)std::min<int64_t>(mb, 1 << 30);
    // 128 channels: the weights go straight to VGPRs, not through LDS
    const int64_t wbytes = C == 128 ? 0 : 2 * (int64_t)C * g.RSW;
    int64_t bytes = xb + mb + wbytes + b.KGp * 4;
    g.t_w3 = g.t_tile = g.t_pre = g.RSW3 = g.KS3 = g.T3 = g.RT = g.RP = 0;
    g.off_d = g.Ctot = g.t_y2 = 0;
    g.m_kgp3 = 2;
    if (b3) {
        bytes = (bytes + 15) / 16 * 16;
        g.Ctot = b3->Cg;
        g.off_d = b3->Cg - C;
        g.KS3 = b3->KGp / 4;
        g.T3 = (b3->Cout + 15) / 16;
        g.RSW3 = b3->KGp * 16 + 16;
        g.RT = C + 16;
        g.t_w3 = (int)bytes;
        bytes += (int64_t)16 * g.T3 * g.RSW3;
        g.t_tile = (int)bytes;
        bytes += (int64_t)CP_NW * 16 * g.RT;
        g.RP = g.off_d + 16;
        g.t_pre = (int)bytes;
        bytes += (int64_t)R * b.OW * g.RP;
        g.m_kgp3 = cp_magic(b3->KGp);
    }
    const int64_t bchunks = (int64_t)(R + 4) * b.W * wm;
    const int64_t wchunks = C == 128 ? 0 : (int64_t)C * b.KGp;
    g.lds = bytes <= 140 * 1024 && bchunks <= (int64_t)CP_SB * CP_NT &&
                    wchunks <= (int64_t)CP_SW * CP_NT &&
                    (int64_t)(R + 4) * g.BW * wm < (1 << 16)
                ? (int)bytes
                : 0;
    g.m_w = cp_magic(b.W);
    g.m_bw = cp_magic(g.BW);
    g.m_kgp = cp_magic(b.KGp);
    return g;
}

using PairKern = void (*)(ConvArgs, ConvArgs, PairGeom, ConvArgs);

PairKern pair_kernel(int wm, bool res, bool tail) {
    if (tail) {
        switch (wm * 2 + (res ? 1 : 0)) {
            case 2: return &k_conv_pair<1, false, true>;
            case 3: return &k_conv_pair<1, true, true>;
            case 4: return &k_conv_pair<2, false, true>;
            case 5: return &k_conv_pair<2, true, true>;
            default: return nullptr;
        }
    }
    switch (wm * 2 + (res ? 1 : 0)) {
        case 16: return &k_conv_pair_cs<false>;
        case 17: return &k_conv_pair_cs<true>;
        case 2: return &k_conv_pair<1, false, false>;
        case 3: return &k_conv_pair<1, true, false>;
        case 4: return &k_conv_pair<2, false, false>;
        case 5: return &k_conv_pair<2, true, false>;
        case 8: return &k_conv_pair<4, false, false>;
        case 9: return &k_conv_pair<4, true, false>;
        default: return nullptr;
    }
}

bool conv_3x3_same(const ConvArgs& b) {
    return b.G == 1 && b.layout == 0 && b.KH == 3 && b.KW == 3 &&
           b.SH == 1 && b.SW == 1 && b.PH == 1 && b.PW == 1 && b.DH == 1 &&
           b.DW == 1 && b.OH == b.H && b.OW == b.W && b.Cg == b.Cout;
}

}  // namespace

bool conv_pair_applies(const ConvArgs& b1, int epi1, const ConvArgs& b2,
                       int epi2) {
    const int C = b1.Cout;
    if (!(C == 16 || C == 32 || C == 64 || C == 128)) return false;
    if (!(epi1 == Q8_TABLE && epi2 == Q8_TABLE && b1.mode == EPI_QUANT &&
          b2.mode == EPI_QUANT && b1.fastio && b2.fastio && b1.plan &&
          b2.plan && conv_3x3_same(b1) && conv_3x3_same(b2) &&
          b2.Cout == C && b1.N == b2.N && b2.H == b1.OH && b2.W == b1.OW &&
          b1.KGp == 4 * ((9 * C / 16 + 3) / 4) && b2.KGp == b1.KGp &&
          b1.x_code == 1 && b1.x_sc == 1 && b2.x_code == 1 &&
          b2.x_sc == 1 && b1.rowsum == 0 && b2.rowsum == 0 &&
          b1.res == nullptr && b1.y2 == nullptr && b2.x == b1.y &&
          b2.y_code == 1 && b1.W >= 2 &&
          (uintptr_t)b1.x % 16 == 0 && b1.x_sp % 16 == 0 &&
          b1.x_sn % 16 == 0 &&
          (int64_t)b1.H * b1.W * b1.x_sp < ((int64_t)1 << 31) &&
          (int64_t)(C + 128) * b1.wp_rstride < ((int64_t)1 << 31) &&
          (int64_t)(C + 128) * b2.wp_rstride < ((int64_t)1 << 31) &&
          b2.M < ((int64_t)1 << 31) && b1.N * (int64_t)b1.OH < (1 << 30)))
        return false;
    return pair_geom(b1, 1).lds > 0;
}

// cv2 of a C2f block after the pair whose output is the last C channels
// of its input (the block's Concat): a 1x1 stride-1 int8 conv with a table
// plan, no residual, second output or row sums, dense channels-last input
// and output, at most 256 input and 128 output channels.
bool conv_pair_tail_applies(const ConvArgs& b1, int epi1, const ConvArgs& b2,
                            int epi2, const ConvArgs& b3, int epi3) {
    const int C = b1.Cout;
    if (C > 32 || !conv_pair_applies(b1, epi1, b2, epi2)) return false;
    if (!(epi3 == Q8_TABLE && b3.mode == EPI_QUANT && b3.fastio && b3.plan &&
          b3.G == 1 && b3.layout == 0 && b3.KH == 1 && b3.KW == 1 &&
          b3.SH == 1 && b3.SW == 1 && b3.PH == 0 && b3.PW == 0 &&
          b3.H == b2.OH && b3.W == b2.OW && b3.OH == b3.H && b3.OW == b3.W &&
          b3.N == b2.N && b3.x_code == 1 && b3.x_sc == 1 && b3.rowsum == 0 &&
          b3.res == nullptr && b3.y2 == nullptr && b3.y_code == 1 &&
          b3.Cg % 16 == 0 && b3.Cg <= 256 && b3.Cg >= C &&
          b3.KGp == 4 * ((b3.Cg / 16 + 3) / 4) && b3.Cout % 16 == 0 &&
          b3.Cout <= 128 && (uintptr_t)b3.x % 16 == 0 &&
          b3.x_sp % 16 == 0 &&
          b3.x_sn == (int64_t)b3.H * b3.W * b3.x_sp &&
          (((const int8_t*)b2.y == (const int8_t*)b3.x + (b3.Cg - C) &&
            b2.y_pst == b3.x_sp) ||
           (b2.y2 != nullptr &&
            (const int8_t*)b2.y2 == (const int8_t*)b3.x + (b3.Cg - C) &&
            b2.y2_pst == b3.x_sp)) &&
          (int64_t)b3.Cout * b3.wp_rstride < ((int64_t)1 << 31) &&
          b3.M < ((int64_t)1 << 31)))
        return false;
    return pair_geom(b1, 1, &b3).lds > 0;
}

bool launch_conv_pair(const ConvArgs& b1, const ConvArgs& b2,
                      hipStream_t st, const ConvArgs* b3) {
    const int wm = b1.Cout / 16;
    const PairKern kern = pair_kernel(wm, b2.res != nullptr, b3 != nullptr);
    if (!kern) {
        set_error("launch_conv_pair", "unsupported channel count");
        return false;
    }
    // R: the least (rounds of resident work-groups) x (staging, counted as
    // 4 tile rounds, + tile rounds of both phases)
    const int cus = cu_count();
    int bestR = 1;
    int64_t best = -1;
    for (int R = 1; R <= b1.OH; ++R) {
        const PairGeom g = pair_geom(b1, R, b3);
        if (g.lds == 0) break;
        const int res = resident_blocks((const void*)kern, CP_NT, g.lds);
        const int64_t rounds = ceil_div(g.nbands, (int64_t)res * cus);
        const int64_t split = wm == 8 ? 1 : CP_NW;  // waves sharing tiles
        const int64_t t1 = ceil_div(ceil_div((int64_t)(R + 2) * b1.OW, 16),
                                    split);
        const int64_t t2 = ceil_div(ceil_div((int64_t)R * b1.OW, 16), split);
        const int64_t cost = rounds * (4 + t1 + t2);
        if (best < 0 || cost < best) {
            best = cost;
            bestR = R;
        }
    }
    // a caller's measured band height (tile code 0x10000 | R on the second
    // descriptor), where the band fits
    if (b2.tile_hint & TILE_VALID) {
        const int rh = b2.tile_hint & 0xffff;
        if (rh >= 1 && rh <= b1.OH && pair_geom(b1, rh, b3).lds > 0)
            bestR = rh;
    }
    PairGeom g = pair_geom(b1, bestR, b3);
    // which of the pair's outputs is the Concat's slice
    if (b3)
        g.t_y2 = (const int8_t*)b2.y == (const int8_t*)b3->x + g.off_d ? 0 : 1;
    if (g.lds == 0 || g.nbands >= ((int64_t)1 << 31)) {
        set_error("launch_conv_pair", "band does not fit");
        return false;
    }
    hipLaunchKernelGGL(kern, dim3((unsigned)g.nbands), dim3(CP_NT),
                       (size_t)g.lds, st, b1, b2, g, b3 ? *b3 : b2);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_hip_error("launch_conv_pair", e);
        return false;
    }
    return true;
}

}  // namespace qa

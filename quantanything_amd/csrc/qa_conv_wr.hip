// int8 convolution with the weights held in registers, one band of output
// rows per work-group, operands staged in LDS with every load in flight.
//
// For convolutions with few output channels per work-group (Cout <= 64 for
// 3x3 taps of 64 channels: K <= 576 bytes with 4 channel tiles), a wave
// can hold every weight fragment it needs in VGPRs: WM channel tiles x KS
// K-steps x 4 registers (144 VGPRs at the largest). The K loop then reads
// only the activation fragment from LDS (one 16-byte read a lane per
// K-step, feeding WM MFMAs), which keeps the LDS traffic at 16 bytes per
// lane and MFMA group instead of 16 (WM + 1).
//
// A work-group owns R output rows of one image (the band) and WM*16 output
// channels; R is chosen so that the grid is about one work-group per CU.
// Staging is latency-bound on this memory system unless many loads are in
// flight, so each thread issues all of its chunks of the band's input rows
// and of the weight rows (up to WR_SB + WR_SW 16-byte chunks) before it
// stores any to LDS (image padding: the pad value, stored separately);
// one barrier, then the weights go from LDS to registers and the
// waves split the band's 16-pixel tiles (tile t goes to wave t % WR_NW). MFMA:
// v_mfma_i32_16x16x64_i8 with the 16 pixels as rows and 16 output channels
// as columns; a K-step is four 16-byte k-groups of the packed layout-0
// weights (tap kg / CB, channels 16 (kg % CB) ..), whose band offsets come
// from a k-group table in LDS (k-groups past the real K point at offset 0:
// their weights are zero).
//
// Epilogue: the int8 table plan of qa_conv.h (per-channel multiply-add and
// shift with the zero-point correction folded into the constant, one med3
// clip, 256-entry clip / activation / residual / copy tables), 4 channels
// of a pixel stored as one word after a 4x4 byte transpose within each
// lane quad, residual words fetched before the tile's MFMAs.
#include "qa_conv_mfma.h"

namespace qa {
namespace {

constexpr int WR_NW = 8;          // waves per work-group
constexpr int WR_NT = 64 * WR_NW;  // threads per work-group
constexpr int WR_SB = 8;          // band chunks (16 bytes) a thread stages
constexpr int WR_SW = 8;          // weight chunks a thread stages
constexpr int WR_HB = 2;          // band rounds held through phase 0

// K-step counts the kernel is instantiated for (a layer runs the smallest
// one >= its K-steps); WM channel tiles hold at most 36 / WM steps (144
// weight VGPRs)
constexpr int WR_STEPS[] = {1, 2, 3, 5, 9, 18, 36};

int wr_steps(int wm, int ks) {
    for (int v : WR_STEPS)
        if (v >= ks && v <= 36 / wm) return v;
    return 0;
}

struct WrGeom {
    int R, BR, BW, PS;    // rows per band, band rows / columns, pixel bytes
    int nbands, bpi;      // bands in all, bands per image
    int band_bytes;       // the LDS band
    int RSW;              // LDS row stride of the staged weights
    int lds;              // dynamic LDS bytes (0: does not fit)
    int KSR;              // K-steps the kernel runs (>= KGp / 4, zero-padded)
    int ost;              // output staged through a per-wave LDS tile
    // ceil(2^32 / d) for d = band columns, KGp, OW, W (all >= 2) and the
    // 16-byte chunks of a pixel (used when >= 2):
    // floor(n / d) = (n * m) >> 32 for the n < 2^16 used here
    uint32_t m_bw, m_kgp, m_ow, m_w, m_cpp;
};

__device__ __forceinline__ int wr_div(int n, uint32_t m) {
    return (int)__umulhi((uint32_t)n, m);
}

// KS: K-steps of 64 bytes, a compile-time count (the packed K rounded up
// to one of the instantiated counts; the extra steps have zero weights).
// RES: a residual Add is fused (its words are fetched one tile ahead; the
// variant without it has no loads in the tile loop, so no wait there on
// the counter that the output stores share).
// CH: a 1x1 convolution a2 (WM*16 -> WM*16 channels, stride 1, no
// residual; its rescaled copy y2 allowed) consumes the output, which then
// never leaves the work-group:
// each tile's stored bytes go to a per-wave LDS tile (16 pixels x 80
// bytes), are read back as the 1x1 conv's activation fragment (one K-step)
// and a2's table epilogue stores a2's output (a covers every channel:
// one channel block).
template <int WM, int KS, bool RES, bool CH>
__global__ __launch_bounds__(WR_NT) void k_conv_wr(ConvArgs a, WrGeom bg,
                                                   ConvArgs a2) {
    constexpr int NW = WR_NW, NT = WR_NT;
    constexpr int SB = WR_SB, SW = WR_SW, HB = WR_HB;
    extern __shared__ int4 lds4[];
    int8_t* s_band = (int8_t*)lds4;                          // band
    int8_t* s_w = s_band + bg.band_bytes;                    // weights
    int* s_kt = (int*)(s_w + WM * 16 * bg.RSW);              // k-groups
    // CH: a2's weights (WM*16 rows of 64 + 16 bytes), the wave tiles
    int8_t* s_w2 = (int8_t*)(s_kt + 4 * KS);
    int8_t* s_t = s_w2 + (CH ? WM * 16 * 80 : 0);
    __shared__ int s_tab[768];
    __shared__ int4 s_pc[WM * 16];
    __shared__ uint32_t s_corr[WM * 16];
    __shared__ int s_tab2[CH ? 256 : 1];
    __shared__ int4 s_pc2[CH ? WM * 16 : 1];
    __shared__ uint32_t s_corr2[CH ? WM * 16 : 1];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 15, kgl = lane >> 4;
    // the channel blocks of a band read the same band: one XCD runs them
    const XcdBlock blk = xcd_block(true);
    const int co0 = (int)blk.y * WM * 16;
    const int KGp = a.KGp;
    const int cpp = a.Cg >> 4;  // 16-byte chunks per input pixel
    const int nch = bg.BR * bg.BW * cpp;
    const int pv = splat4(a.pad_value);
    const v4i pad4 = {pv, pv, pv, pv};

    const int band = (int)blk.x;
    const int n = band / bg.bpi;
    const int oy0 = (band - n * bg.bpi) * bg.R;
    const int iy0 = oy0 * a.SH - a.PH;
    const int8_t* xn = (const int8_t*)a.x + (int64_t)n * a.x_sn;
    const int wch = WM * 16 * KGp;

    // ---- staging. The band's rows inside the image are one run of
    // pixels p = 0 .. (r_hi - r_lo) W - 1 from image row iy0 + r_lo; chunk
    // e < nreal is pixel e / cpp, 16-byte part e % cpp, at band row
    // r_lo + p / W, column PW + p % W (columns past the band's width are
    // loaded and dropped); weight chunk e is row e / KGp, part e % KGp.
    // Every load of the thread (band and weight chunks, in rounds of NT
    // chunks; rounds past the data are skipped) is issued before its
    // stores, from straight-line code with few instructions a chunk (it
    // runs once, from a cold instruction cache); the pad value fills the
    // band's other positions. The band's rounds are stored in two phases:
    // all but the last nh <= HB rounds before the first barrier, the
    // held ones after the tiles that need only the earlier rows (phase 0)
    // have been computed, so that the later loads' latency overlaps phase
    // 0's MFMAs.
    const int r_lo = max(0, -iy0);
    const int r_hi = max(min(bg.BR, a.H - iy0), r_lo);
    const int nreal = (r_hi - r_lo) * a.W * cpp;
    const int nr = (nreal + NT - 1) / NT;  // rounds of band chunks
    const int nh = min(HB, max(nr - 1, 0));  // the last rounds, held
    const int h = nr - nh;                       // rounds stored first
    v4i vx[SB], vh[HB];
    int ax[SB], axh[HB];
    const int xsp = (int)a.x_sp;
    const int8_t* xrow = xn + (int64_t)(iy0 + r_lo) * a.W * a.x_sp;
    const int colmax = bg.BW - a.PW;  // real columns kept
    auto load_round = [&](int u, v4i& v, int& at) {
        const int e = tid + u * NT;
        const int p = cpp == 1 ? e : wr_div(e, bg.m_cpp);
        const int ch = e - p * cpp;
        const int row = wr_div(p, bg.m_w), ix = p - row * a.W;
        const bool ok = e < nreal && ix < colmax;
        at = ok ? ((r_lo + row) * bg.BW + ix + a.PW) * bg.PS + ch * 16 : -1;
        v = *(const v4i*)(xrow + (e < nreal ? p * xsp + ch * 16 : 0));
    };
    // weights, tables and per-channel constants: loaded first and stored
    // behind their own barrier, so that the weights' copy into registers
    // overlaps the band's loads (the loads complete in issue order)
    {
        v4i vw[SW];
        int aw[SW];
        {
            const int wrs = (int)a.wp_rstride;
            const int8_t* wrow = a.wp + (int64_t)co0 * a.wp_rstride;
#pragma unroll
            for (int u = 0; u < SW; ++u) {
                aw[u] = -1;
                if (u * NT < wch) {
                    const int e = tid + u * NT;
                    const int r = wr_div(e, bg.m_kgp), k = e - r * KGp;
                    const bool ok = e < wch;
                    aw[u] = ok ? r * bg.RSW + k * 16 : -1;
                    vw[u] = *(const v4i*)(wrow + (ok ? r * wrs + k * 16 : 0));
                }
            }
        }
        constexpr int NTV = (768 + NT - 1) / NT;
        int tv[NTV];
#pragma unroll
        for (int j = 0; j < NTV; ++j)
            tv[j] = tid + j * NT < 768
                        ? ((const int*)((const char*)a.plan +
                                        PLAN_E))[tid + j * NT]
                        : 0;
        int4 pcv = int4{0, 0, 0, 0};
        uint32_t corrv = 0;
        if (tid < WM * 16) {
            const int c = min(co0 + tid, a.Cout - 1);
            pcv = ((const int4*)((const char*)a.plan + PLAN_CH))[c];
            corrv = a.corr ? (uint32_t)a.corr[c] : 0u;
        }
        // a2's weight rows (4 chunks each, K = one 64-byte step), table
        // and constants
        v4i w2v = v4i{0, 0, 0, 0};
        int t2v = 0;
        int4 pc2v = int4{0, 0, 0, 0};
        uint32_t corr2v = 0;
        if (CH) {
            if (tid < WM * 16 * 4)
                w2v = *(const v4i*)(a2.wp + (int64_t)(tid >> 2) * a2.wp_rstride +
                                    (tid & 3) * 16);
            if (tid < 256)
                t2v = ((const int*)((const char*)a2.plan + PLAN_E))[tid];
            if (tid < WM * 16) {
                pc2v = ((const int4*)((const char*)a2.plan + PLAN_CH))[tid];
                corr2v = a2.corr ? (uint32_t)a2.corr[tid] : 0u;
            }
        }
        // the band: rounds stored after the first barrier, then the held
        // ones (issued last)
#pragma unroll
        for (int u = 0; u < SB; ++u) {
            ax[u] = -1;
            if (u < h) load_round(u, vx[u], ax[u]);
        }
#pragma unroll
        for (int j = 0; j < HB; ++j) {
            axh[j] = -1;
            if (j < nh) load_round(h + j, vh[j], axh[j]);
        }
        // pad value: band rows outside the image (all columns), then the
        // columns left and right of the image on the other rows
        {
            const int rowc = bg.BW * cpp;  // chunks of a band row
            const int nprow = r_lo + (bg.BR - r_hi);
            for (int e = tid; e < nprow * rowc; e += NT) {
                const int rr = e / rowc, c = e - rr * rowc;
                const int row = rr < r_lo ? rr : r_hi + (rr - r_lo);
                *(v4i*)(s_band + row * bg.BW * bg.PS + (c / cpp) * bg.PS +
                        (c % cpp) * 16) = pad4;
            }
            const int rpad = max(bg.BW - a.PW - a.W, 0);  // right columns
            const int pc = (a.PW + rpad) * cpp;           // chunks a row
            for (int e = tid; e < (r_hi - r_lo) * pc; e += NT) {
                const int rr = e / pc, c = e - rr * pc;
                const int j = c / cpp, ch = c - j * cpp;
                const int col = j < a.PW ? j : a.W + j;
                *(v4i*)(s_band + ((r_lo + rr) * bg.BW + col) * bg.PS +
                        ch * 16) = pad4;
            }
        }
        for (int kg = tid; kg < 4 * KS; kg += NT) {
            int off = 0;  // padding k-groups: any in-band address
            if (kg < a.KG) {
                const int tap = kg / a.CB, cb = kg - tap * a.CB;
                const int ky = tap / a.KW, kx = tap - ky * a.KW;
                off = (ky * a.DH * bg.BW + kx * a.DW) * bg.PS + cb * 16;
            }
            s_kt[kg] = off;
        }
        // weight rows past KGp chunks up to the instantiated K-steps: zero
        if (4 * KS > KGp) {
            const int tail = 4 * KS - KGp;
            for (int e = tid; e < WM * 16 * tail; e += NT) {
                const int r = e / tail;
                *(v4i*)(s_w + r * bg.RSW + (KGp + e - r * tail) * 16) =
                    v4i{0, 0, 0, 0};
            }
        }
#pragma unroll
        for (int u = 0; u < SW; ++u)
            if (aw[u] >= 0) *(v4i*)(s_w + aw[u]) = vw[u];
#pragma unroll
        for (int j = 0; j < NTV; ++j)
            if (tid + j * NT < 768) s_tab[tid + j * NT] = tv[j];
        if (tid < WM * 16) {
            s_pc[tid] = pcv;
            s_corr[tid] = corrv;
        }
        if (CH) {
            if (tid < WM * 16 * 4)
                *(v4i*)(s_w2 + (tid >> 2) * 80 + (tid & 3) * 16) = w2v;
            if (tid < 256) s_tab2[tid] = t2v;
            if (tid < WM * 16) {
                s_pc2[tid] = pc2v;
                s_corr2[tid] = corr2v;
            }
        }
    }
    __syncthreads();

    // weights of the lane: channel tile i, K-step s: row co0 + 16 i + col,
    // bytes 64 s + 16 kgl (steps past KGp / 4 hold zeros); band offsets of
    // its k-groups
    v4i wb[KS][WM];
    int kt[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) {
        kt[s] = s_kt[4 * s + kgl];
#pragma unroll
        for (int i = 0; i < WM; ++i)
            wb[s][i] = *(const v4i*)(s_w + (16 * i + col) * bg.RSW + 64 * s +
                                     16 * kgl);
    }
    // per-channel plan constants, the correction term folded in (plan_q0;
    // K <= 36 K-steps: |w| + |corr| < 2^27)
    int cm[WM], ct[WM];
    int64_t cc[WM];
#pragma unroll
    for (int i = 0; i < WM; ++i) {
        const int4 pc = s_pc[16 * i + col];
        cm[i] = pc.x;
        ct[i] = pc.y;
        cc[i] = plan_fold(
            (int64_t)(((uint64_t)(uint32_t)pc.w << 32) | (uint32_t)pc.z),
            s_corr[16 * i + col], pc.x);
    }
    const int4 hdr = *(const int4*)a.plan;
    const int pA = hdr.x, pB = hdr.y, pSH = hdr.z;
    const int* tabE = s_tab - pA;  // tabE[v] = E[v - pA] for v in [pA, pB]
    const int* tabC = s_tab + 256 - pA;
    // CH: a2's weight fragments (one K-step) and per-channel constants
    v4i wb2[CH ? WM : 1];
    int cm2[CH ? WM : 1], ct2[CH ? WM : 1];
    int64_t cc2[CH ? WM : 1];
    int4 hdr2 = int4{0, 0, 0, 0};
    if (CH) {
#pragma unroll
        for (int i = 0; i < WM; ++i) {
            wb2[i] = *(const v4i*)(s_w2 + (16 * i + col) * 80 + 16 * kgl);
            const int4 pc = s_pc2[16 * i + col];
            cm2[i] = pc.x;
            ct2[i] = pc.y;
            cc2[i] = plan_fold((int64_t)(((uint64_t)(uint32_t)pc.w << 32) |
                                         (uint32_t)pc.z),
                               s_corr2[16 * i + col], pc.x);
        }
        hdr2 = *(const int4*)a2.plan;
    }
    const int* tabE2 = s_tab2 - hdr2.x;
    // the band's first rounds (the loads have had the weights' copy to
    // arrive)
#pragma unroll
    for (int u = 0; u < SB; ++u)
        if (ax[u] >= 0) *(v4i*)(s_band + ax[u]) = vx[u];
    __syncthreads();
    int8_t* s_tw = s_t + wave * (16 * 80);  // this wave's tile (CH)
    const int q = lane & 3;
    const uint32_t sel1 = q < 2 ? 0x05040100u : 0x03020706u;
    const uint32_t sel2 = (q & 1) ? 0x03070105u : 0x06020400u;
    const int cq = col & ~3;

    {
        const int npix = min(bg.R, a.OH - oy0) * a.OW;
        const int ntile = (npix + 15) >> 4;
        const int64_t pimg = (int64_t)n * a.OH * a.OW + (int64_t)oy0 * a.OW;
        const int8_t* sb = s_band;
        // residual words (4 channels of the pixel this lane stores) of
        // tile t: 0 past the band or the channels
        auto load_res = [&](int t, uint32_t (&rw)[WM]) {
            const int pq = 16 * t + 4 * kgl + q;
            const bool ok = pq < npix;
            const int8_t* pr = (const int8_t*)a.res + (pimg + pq) * a.res_pst;
#pragma unroll
            for (int i = 0; i < WM; ++i) {
                const int c0 = co0 + 16 * i + cq;
                rw[i] = ok && c0 < a.Cout ? *(const uint32_t*)(pr + c0) : 0u;
            }
        };
        // activation fragments of tile t: the lane's pixel (rows of the
        // MFMA) in the band buffer, one 16-byte read per K-step (tiles past
        // the band read its last pixel)
        auto frags = [&](v4i (&f)[KS], int t) {
            const int qp = min(16 * t + col, npix - 1);
            const int r = wr_div(qp, bg.m_ow), ox = qp - r * a.OW;
            const int8_t* xb = sb + (r * a.SH * bg.BW + ox * a.SW) * bg.PS;
#pragma unroll
            for (int s = 0; s < KS; ++s) f[s] = *(const v4i*)(xb + kt[s]);
        };
        auto mfmas = [&](const v4i (&f)[KS], v4i (&c)[WM]) {
#pragma unroll
            for (int i = 0; i < WM; ++i) c[i] = v4i{0, 0, 0, 0};
#pragma unroll
            for (int s = 0; s < KS; ++s)
#pragma unroll
                for (int i = 0; i < WM; ++i)
                    c[i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                        f[s], wb[s][i], c[i], 0, 0, 0);
        };
        // epilogue, branch-free part: lane holds pixels 4 kgl + r, channel
        // co0 + 16 i + col. Per value: multiply-add, shift, one med3 clip
        // and one table read whose address folds in the clip's lower
        // bound; every table read of the tile is issued before the first
        // use. e4 gets the entries (bits 0..7 the stored byte of y, 8..15
        // that of y2).
        auto epi_math = [&](const v4i (&c)[WM], const uint32_t (&rw)[WM],
                            int (&e4)[WM][4]) {
#pragma unroll
            for (int i = 0; i < WM; ++i)
#pragma unroll
                for (int rr = 0; rr < 4; ++rr)
                    e4[i][rr] = med3_i32(
                        plan_q0(c[i][rr], cm[i], cc[i], ct[i]), pA, pB);
#pragma unroll
            for (int i = 0; i < WM; ++i) {
                if (RES) {
                    const uint32_t rv = quad_transpose(rw[i], sel1, sel2);
#pragma unroll
                    for (int rr = 0; rr < 4; ++rr)
                        e4[i][rr] = tabC[e4[i][rr]] +
                                    s_tab[512 + ((rv >> (8 * rr)) & 255)];
#pragma unroll
                    for (int rr = 0; rr < 4; ++rr)
                        e4[i][rr] = s_tab[med3_i32(e4[i][rr], 0, pSH)];
                } else {
#pragma unroll
                    for (int rr = 0; rr < 4; ++rr) e4[i][rr] = tabE[e4[i][rr]];
                }
            }
        };
        // the stores of tile t: 4 channels of a pixel as one word (CH: the
        // wave's LDS tile)
        auto epi_store = [&](int t, const int (&e4)[WM][4], bool tok) {
            const int pq = 16 * t + 4 * kgl + q;  // pixel within the band
            const bool pok = tok && pq < npix;
            const int64_t p = pimg + pq;
#pragma unroll
            for (int i = 0; i < WM; ++i) {
                const int c0 = co0 + 16 * i + cq;  // Cout % 4 == 0
                const bool sok = pok && c0 < a.Cout;
                const uint32_t wy =
                    quad_transpose(pack_entries(e4[i], 0), sel1, sel2);
                if (CH) {  // pixel 4 kgl + q of the tile, channels c0 ..
                    *(uint32_t*)(s_tw + (4 * kgl + q) * 80 + c0) = wy;
                    continue;
                }
                if (sok) *(uint32_t*)((int8_t*)a.y + p * a.y_pst + c0) = wy;
                if (a.y2) {
                    const uint32_t w2 =
                        quad_transpose(pack_entries(e4[i], 1), sel1, sel2);
                    if (sok)
                        *(uint32_t*)((int8_t*)a.y2 + p * a.y2_pst + c0) = w2;
                }
            }
        };
        // ost (no residual or chained conv; 16-byte aligned outputs, Cout
        // a multiple of 16): the tile's stored bytes go to the wave's LDS
        // tile (16 pixels x OS bytes; byte writes at immediate offsets,
        // no packing or lane exchange), then each lane stores 16 channels
        // of one pixel: pixel lp of the tile, channels co0 + 16 lc ..
        constexpr int OS = 16 * WM + 16;
        int8_t* const s_ow = s_t + wave * (16 * OS);
        const int lp = lane / WM, lc = lane % WM;
        const bool lact = lane < 16 * WM && co0 + 16 * lc < a.Cout;
        const int ypst = (int)a.y_pst, y2pst = (int)a.y2_pst;
        int8_t* const yb = (int8_t*)a.y + pimg * a.y_pst + co0 + 16 * lc;
        int8_t* const y2b =
            a.y2 ? (int8_t*)a.y2 + pimg * a.y2_pst + co0 + 16 * lc : nullptr;
        auto epi_store_staged = [&](int t, const int (&e4)[WM][4]) {
            const int pq = 16 * t + lp;
            const bool sok = lact && pq < npix;
            int8_t* const wbyte = s_ow + 4 * kgl * OS + col;
#pragma unroll
            for (int i = 0; i < WM; ++i)
#pragma unroll
                for (int rr = 0; rr < 4; ++rr)
                    wbyte[rr * OS + 16 * i] = (int8_t)e4[i][rr];
            // the wave's byte writes before its reads of them by other
            // lanes (LDS instructions of a wave complete in order; the
            // wait also keeps the compiler from moving them)
            __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
            __builtin_amdgcn_wave_barrier();
            const v4i v = *(const v4i*)(s_ow + lp * OS + 16 * lc);
            __builtin_amdgcn_wave_barrier();
            if (sok) *(v4i*)(yb + pq * ypst) = v;
            if (a.y2) {  // the rescaled copy: the entries' second bytes
#pragma unroll
                for (int i = 0; i < WM; ++i)
#pragma unroll
                    for (int rr = 0; rr < 4; ++rr)
                        wbyte[rr * OS + 16 * i] = (int8_t)(e4[i][rr] >> 8);
                __builtin_amdgcn_s_waitcnt(0xc07f);
                __builtin_amdgcn_wave_barrier();
                const v4i v2 = *(const v4i*)(s_ow + lp * OS + 16 * lc);
                __builtin_amdgcn_wave_barrier();
                if (sok) *(v4i*)(y2b + pq * y2pst) = v2;
            }
        };
        // phase 0: the tiles whose input rows are all among the band rows
        // of the first h rounds (the rows above the image count as staged)
        int T0 = ntile;
        if (h < nr) {
            const int rows = r_lo + (h * NT) / (a.W * cpp);
            const int need = (a.KH - 1) * a.DH + 1;  // band rows a row uses
            const int orows = rows >= need ? (rows - need) / a.SH + 1 : 0;
            T0 = min(orows * a.OW, npix) >> 4;
        }
#pragma unroll 1
        for (int ph = 0; ph < 2; ++ph) {
          if (ph == 1) {
#pragma unroll
              for (int j = 0; j < HB; ++j)
                  if (axh[j] >= 0) *(v4i*)(s_band + axh[j]) = vh[j];
              __syncthreads();
          }
          const int tb = ph == 0 ? 0 : T0, te = ph == 0 ? T0 : ntile;
          uint32_t rwn[WM];
          if (RES && tb + wave < te) load_res(tb + wave, rwn);
          for (int t = tb + wave; t < te; t += NW) {
            const int pq = 16 * t + 4 * kgl + q;  // pixel within the band
            const bool pok = pq < npix;
            const int64_t p = pimg + pq;
            uint32_t rw[WM];
            if (RES) {
#pragma unroll
                for (int i = 0; i < WM; ++i) rw[i] = rwn[i];
                if (t + NW < te) load_res(t + NW, rwn);
            }
            v4i fa[KS], acc[WM];
            frags(fa, t);
            mfmas(fa, acc);
            {
                int e4[WM][4];
                epi_math(acc, rw, e4);
                if (!CH && !RES && bg.ost)
                    epi_store_staged(t, e4);
                else
                    epi_store(t, e4, true);
            }
            if (CH) {
                // the wave's own LDS writes above, read back by other lanes
                // of the same wave (LDS instructions of a wave complete in
                // order; the wait also keeps the compiler from moving them)
                __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
                __builtin_amdgcn_wave_barrier();
                // 1x1 conv: pixel col of the tile, channels 16 kgl .. (the
                // k-groups past WM*16 channels have zero weights)
                const v4i fa2 = *(const v4i*)(s_tw + col * 80 + 16 * kgl);
                v4i acc2[WM];
#pragma unroll
                for (int i = 0; i < WM; ++i)
                    acc2[i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                        fa2, wb2[i], v4i{0, 0, 0, 0}, 0, 0, 0);
                __builtin_amdgcn_wave_barrier();
#pragma unroll
                for (int i = 0; i < WM; ++i) {
                    int e[4];
#pragma unroll
                    for (int rr = 0; rr < 4; ++rr)
                        e[rr] = tabE2[med3_i32(
                            plan_q0(acc2[i][rr], cm2[i], cc2[i], ct2[i]),
                            hdr2.x, hdr2.y)];
                    const int c0 = 16 * i + cq;
                    const uint32_t wy =
                        quad_transpose(pack_entries(e, 0), sel1, sel2);
                    if (pok)
                        *(uint32_t*)((int8_t*)a2.y + p * a2.y_pst + c0) = wy;
                    if (a2.y2) {  // a2's rescaled copy (a Concat input)
                        const uint32_t w2 =
                            quad_transpose(pack_entries(e, 1), sel1, sel2);
                        if (pok)
                            *(uint32_t*)((int8_t*)a2.y2 + p * a2.y2_pst +
                                         c0) = w2;
                    }
                }
            }
          }
        }
    }
}

// Geometry for bands of R output rows; lds = 0 when it does not fit in LDS
// or the band and weight chunks exceed what the threads stage.
WrGeom wr_geom(const ConvArgs& b, int wm, int R, bool ch = false) {
    WrGeom g;
    g.R = R;
    g.BR = (R - 1) * b.SH + (b.KH - 1) * b.DH + 1;
    g.BW = (b.OW - 1) * b.SW + (b.KW - 1) * b.DW + 1;
    g.PS = b.Cg + (((b.Cg >> 4) & 1) ? 0 : 16);
    g.bpi = (b.OH + R - 1) / R;
    g.nbands = b.N * g.bpi;
    g.KSR = wr_steps(wm, b.KGp / 4);
    // weight rows hold the instantiated K-steps (the tail chunks zeroed)
    g.RSW = std::max<int>(4 * g.KSR, b.KGp) * 16 + 16;
    const int64_t band = (int64_t)g.BR * g.BW * g.PS;
    const int64_t bchunks = (int64_t)g.BR * b.W * (b.Cg >> 4);
    const int64_t wchunks = (int64_t)wm * 16 * b.KGp;
    g.band_bytes = (int)std::min<int64_t>(band, 1 << 30);
    auto magic = [](int64_t d) {
        return (uint32_t)((((uint64_t)1 << 32) + (uint64_t)d - 1) /
                          (uint64_t)std::max<int64_t>(d, 2));
    };
    g.m_bw = magic(g.BW);
    g.m_kgp = magic(b.KGp);
    g.m_ow = magic(b.OW);
    g.m_w = magic(b.W);
    g.m_cpp = magic(b.Cg >> 4);
    int64_t bytes =
        band + (int64_t)wm * 16 * g.RSW + (int64_t)g.KSR * 16 +
        (ch ? (int64_t)wm * 16 * 80 + WR_NW * 16 * 80 : 0);
    // the output staged through LDS (16-byte stores of whole 16-channel
    // blocks, never the pixel's padding channels) when it fits
    const int64_t otile = (int64_t)WR_NW * 16 * (16 * wm + 16);
    g.ost = !ch && b.res == nullptr && b.Cout % 16 == 0 &&
            (uintptr_t)b.y % 16 == 0 && b.y_pst % 16 == 0 &&
            (b.y2 == nullptr ||
             ((uintptr_t)b.y2 % 16 == 0 && b.y2_pst % 16 == 0)) &&
            (int64_t)R * b.OW * std::max(b.y_pst, b.y2_pst) <
                ((int64_t)1 << 31) &&
            bytes + otile <= 150 * 1024;
    if (g.ost) bytes += otile;
    // gfx950 gives a work-group up to 160 KB of LDS
    g.lds = bytes <= 150 * 1024 && bchunks <= (int64_t)WR_SB * WR_NT &&
                    wchunks <= (int64_t)WR_SW * WR_NT &&
                    (int64_t)g.BR * g.BW * (b.Cg >> 4) < (1 << 16)
                ? (int)bytes
                : 0;
    return g;
}

using WrKern = void (*)(ConvArgs, WrGeom, ConvArgs);

template <int WM, bool RES, bool CH>
WrKern wr_kernel(int ks) {
    switch (ks) {
        case 1: return &k_conv_wr<WM, 1, RES, CH>;
        case 2: return &k_conv_wr<WM, 2, RES, CH>;
        case 3: return &k_conv_wr<WM, 3, RES, CH>;
        case 5: return &k_conv_wr<WM, 5, RES, CH>;
        case 9:  // with the chained conv, 4 channel tiles would spill
            if constexpr (!(CH && WM == 4)) return &k_conv_wr<WM, 9, RES, CH>;
            break;
        case 18:
            if constexpr (WM <= 2 && !CH) return &k_conv_wr<WM, 18, RES, CH>;
            break;
        case 36:
            if constexpr (WM == 1 && !CH) return &k_conv_wr<WM, 36, RES, CH>;
            break;
        default: break;
    }
    return nullptr;
}

template <bool RES, bool CH>
WrKern wr_kernel_wm(int wm, int ks) {
    return wm == 1   ? wr_kernel<1, RES, CH>(ks)
           : wm == 2 ? wr_kernel<2, RES, CH>(ks)
           : wm == 4 ? wr_kernel<4, RES, CH>(ks)
                     : nullptr;
}

// ch: with a chained 1x1 convolution (no residual variant)
WrKern wr_kernel_rt(int wm, int ks, bool res, bool ch = false) {
    if (ch) return res ? nullptr : wr_kernel_wm<false, true>(wm, ks);
    return res ? wr_kernel_wm<true, false>(wm, ks)
               : wr_kernel_wm<false, false>(wm, ks);
}

// Work-groups of a kernel resident per CU with `lds` dynamic bytes.
int wr_resident(WrKern k, int lds) {
    return resident_blocks((const void*)k, WR_NT, lds);
}

}  // namespace

bool conv_wr_applies(const ConvArgs& b, int epi, int wm) {
    const uintptr_t xa = (uintptr_t)b.x, ya = (uintptr_t)b.y;
    if (wm != 1 && wm != 2 && wm != 4) return false;
    if (!(epi == Q8_TABLE && b.mode == EPI_QUANT && b.fastio && b.plan &&
          b.G == 1 && b.layout == 0 && b.x_code == 1 && b.x_sc == 1 &&
          b.rowsum == 0 && b.Cg % 16 == 0 && b.Cg > 0 &&
          b.W >= 2 &&
          b.Cout % 4 == 0 &&
          b.OW >= 2 &&
          b.KGp % 4 == 0 && wr_steps(wm, b.KGp / 4) > 0 && xa % 16 == 0 &&
          b.x_sp % 16 == 0 && b.x_sn % 16 == 0 && b.y_code == 1 &&
          ya % 4 == 0 && b.y_pst % 4 == 0 &&
          (b.res == nullptr ||
           ((uintptr_t)b.res % 4 == 0 && b.res_pst % 4 == 0)) &&
          (b.y2 == nullptr ||
           ((uintptr_t)b.y2 % 4 == 0 && b.y2_pst % 4 == 0)) &&
          b.M < ((int64_t)1 << 31) && b.N * (int64_t)b.OH < (1 << 30) &&
          (int64_t)b.H * b.W * b.x_sp < ((int64_t)1 << 31) &&
          (int64_t)(b.Cout + 128) * b.wp_rstride < ((int64_t)1 << 31)))
        return false;
    return wr_geom(b, wm, 1).lds > 0;
}

namespace {

// Shared launcher: b alone (ch false, b2 unused) or b with the chained 1x1
// convolution b2.
bool wr_launch(const ConvArgs& b, int wm, bool ch, const ConvArgs& b2,
               hipStream_t st) {
    // R: the least (rounds of resident work-groups) x (staging, counted as
    // 4 tiles, + tiles per wave)
    const int cus = cu_count();
    const int64_t cblocks = ceil_div(b.Cout, 16 * wm);
    const bool res = b.res != nullptr;
    int bestR = 1;
    int64_t best = -1;
    for (int R = 1; R <= b.OH; ++R) {
        const WrGeom g = wr_geom(b, wm, R, ch);
        if (g.lds == 0) break;
        const int nres = wr_resident(wr_kernel_rt(wm, g.KSR, res, ch), g.lds);
        const int64_t rounds =
            ceil_div(g.nbands * cblocks, (int64_t)nres * cus);
        const int64_t cost =
            rounds * (4 + ceil_div(ceil_div((int64_t)R * b.OW, 16), WR_NW));
        if (best < 0 || cost < best) {
            best = cost;
            bestR = R;
        }
    }
    // a caller's measured band height: tile code 0x11000 | wm | R << 4 of
    // the convolution, or 0x10000 | R of the chained 1x1 convolution
    int rh = 0;
    if (ch) {
        if (b2.tile_hint & TILE_VALID) rh = b2.tile_hint & 0xffff;
    } else if ((b.tile_hint & TILE_VALID) && ((b.tile_hint >> 12) & 1)) {
        rh = (b.tile_hint >> 4) & 15;
    }
    if (rh >= 1 && rh <= b.OH && wr_geom(b, wm, rh, ch).lds > 0) bestR = rh;
    const WrGeom g = wr_geom(b, wm, bestR, ch);
    const int64_t gx = g.nbands;
    if (g.lds == 0 || cblocks > 65535 || gx >= ((int64_t)1 << 31)) {
        set_error("launch_conv_wr", "band or grid does not fit");
        return false;
    }
    const dim3 grid((unsigned)gx, (unsigned)cblocks);
    const WrKern kern = wr_kernel_rt(wm, g.KSR, res, ch);
    if (!kern) {
        set_error("launch_conv_wr", "no kernel for the K-steps");
        return false;
    }
    hipLaunchKernelGGL(kern, grid, dim3(WR_NT), (size_t)g.lds, st, b, g, b2);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_hip_error("launch_conv_wr", e);
        return false;
    }
    return true;
}

}  // namespace

bool launch_conv_wr(const ConvArgs& b, int wm, hipStream_t st) {
    if (!conv_wr_applies(b, Q8_TABLE, wm)) {
        set_error("launch_conv_wr", "convolution outside the kernel's scope");
        return false;
    }
    return wr_launch(b, wm, false, b, st);
}

bool conv_chain_applies(const ConvArgs& b1, int epi1, const ConvArgs& b2,
                        int epi2) {
    const int wm = b1.Cout / 16;
    if (!((wm == 1 || wm == 2 || wm == 4) && b1.Cout == 16 * wm &&
          conv_wr_applies(b1, epi1, wm) && b1.res == nullptr &&
          b1.y2 == nullptr && wr_steps(wm, b1.KGp / 4) <= (wm == 4 ? 5 : 9)))
        return false;
    return epi2 == Q8_TABLE && b2.mode == EPI_QUANT && b2.fastio && b2.plan &&
           b2.G == 1 && b2.layout == 0 && b2.KH == 1 && b2.KW == 1 &&
           b2.SH == 1 && b2.SW == 1 && b2.PH == 0 && b2.PW == 0 &&
           b2.Cg == b1.Cout && b2.Cout == b1.Cout && b2.KGp == 4 &&
           b2.x == b1.y && b2.N == b1.N && b2.H == b1.OH && b2.W == b1.OW &&
           b2.OH == b2.H && b2.OW == b2.W && b2.res == nullptr &&
           (b2.y2 == nullptr ||
            ((uintptr_t)b2.y2 % 4 == 0 && b2.y2_pst % 4 == 0)) &&
           b2.rowsum == 0 && b2.y_code == 1 &&
           (uintptr_t)b2.y % 4 == 0 && b2.y_pst % 4 == 0 &&
           wr_geom(b1, wm, 1, true).lds > 0;
}

bool launch_conv_chain(const ConvArgs& b1, const ConvArgs& b2,
                       hipStream_t st) {
    return wr_launch(b1, b1.Cout / 16, true, b2, st);
}

}  // namespace qa

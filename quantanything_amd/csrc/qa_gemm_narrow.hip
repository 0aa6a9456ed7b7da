// Narrow int8 GEMMs and pointwise convolutions with the table epilogue:
// 16, 32 or 64 output channels, or any multiple of 4 in blocks of 64; K a
// multiple of 64 up to 576 (1280 in 64-channel blocks with the weights in
// fragment order); any number of rows M (the standalone 4096 x 576 x 64
// GEMM, the 1x1 convolutions of a classifier's late stages, its
// 1280 -> 1000 head).
//
// Such a launch moves a few MB and does well under a microsecond of matrix
// work, so its time is its chain of dependent steps, not arithmetic. The
// kernel is built so that the chain is one memory round trip: the few
// arguments it reads arrive in one scalar load round (a compact argument
// block instead of the 700-byte convolution block), then every load of a
// lane is issued unconditionally (table entry, weights, activations,
// header, per-channel constants, correction), one wait, the table to LDS,
// one barrier, the MFMAs and the epilogue.
//
// A work-group of 4 waves covers 16 rows x 64 channels (Cout 64), 32 x 32
// or 64 x 16; wave w owns one 16 x 16 block. With the weights in fragment
// order (ConvArgs.wfrag) each wave loads its 16 x K block's fragments
// straight into VGPRs, one contiguous KB a load. The activation rows (and
// otherwise the weight rows, K bytes each) go to
// LDS by direct global -> LDS loads in which each group of 4 lanes reads one
// 64-byte K-step of one row: adjacent lanes, adjacent bytes, so a load
// instruction is 16 requests of 64 bytes (a lane per row, as the MFMA
// fragment layout would have it, makes 64 requests of 16 bytes, and the
// 4096 x 576 x 64 GEMM took 3.2 instead of 2.95 us). In LDS the 64-byte
// segment of (K-step s, row r) sits at (s R + r) 64 (R rows of the
// operand), its 16-byte chunk k at position k ^ ((r >> 2) & 3), so that
// the 16 lanes of a fragment read (rows 16 j .. 16 j + 15, one chunk) fall
// in distinct bank groups. The MFMA takes the weights as its first
// operand, so its result lane l holds channels 4 (l >> 4) + i of row
// (l & 15): four consecutive bytes of one output row, stored as one word,
// with no exchange between lanes. Epilogue per value: the plan's 64-bit
// multiply-add and shift with the zero-point correction folded into its
// constant, one med3 clip, then the table entry or, for an identity plan
// (plain requantize), the byte offset.
#include "qa_conv_mfma.h"

namespace qa {
namespace {

constexpr int GN_KMAX = 20;  // K-steps of 64 bytes (K up to 1280)

// The kernel's arguments, read in one scalar round; the ones its first
// loads need also go as leading scalar arguments, which the dispatch
// preloads into SGPRs (no scalar load before the first vector load).
struct GnArgs {
    const int8_t* x;       // activation rows, xpst bytes apart
    const int8_t* wp;      // packed weight rows, 16 * KGp bytes apart
    const int8_t* wf;      // the same in fragment order (WF)
    const char* plan;      // table epilogue plan
    const int64_t* corr;   // per-channel correction (NULL: none)
    const int32_t* boff;   // per-channel weight offsets (RS)
    int8_t* y;             // output rows, ypst bytes apart
    int8_t* y2;            // the rescaled copy (NULL: none), y2pst apart
    int64_t xpst, ypst, y2pst, M;
    int32_t KGp, Cout, RTL, pad;
    // CV (a k x k convolution, Cg a multiple of 64): the image geometry;
    // row p is output pixel p of the batch, K-step s covers tap s / CBK,
    // input channels 64 (s % CBK) ..; x_sn / xpst: image / pixel strides
    int64_t x_sn;
    int32_t H, W, OH, OW, SH, SW, PH, PW, DH, DW, KW, CBK, padv, pad2;
};

// NB: 16-channel blocks (1, 2 or 4) a work-group; blockIdx.y selects the
// work-group's block of 16 NB channels (NB = 4 past 64 output channels).
// Its 4 waves cover 4 / NB row tiles of 16 at a time, RTL times (each
// wave's weight fragments stay in VGPRs over its RTL row tiles, which
// the work-group stages together). RS: pixel sums (weights with an
// offset). WF: the weights in fragment order, each wave's fragments loaded
// straight into VGPRs (one contiguous KB a load); otherwise staged in LDS
// like the activations. KM: K-steps held (9; 20 with NB = 4 and WF).
// Dynamic LDS: the activation rows (16 (4 / NB) RTL of them), then (not
// WF) the weight rows.
// CV: the activation rows are the im2col rows of a convolution (each
// 64-byte K-step one tap's 64 channels of one input pixel, loaded like a
// GEMM row's); a tap outside the image loads pixel (0, 0) and then has
// its LDS bytes overwritten with the pad value.
#define GN_ARGS(g) \
    (g).x, (g).wf, (g).plan, (g).xpst, (g).M, (g).KGp, (g).RTL, (g)
template <int NB, bool RS, bool WF, int KM, bool CV = false>
__global__ __launch_bounds__(256) void k_gemm_narrow(
    const int8_t* x, const int8_t* wf, const char* plan, int64_t xpst,
    int64_t M, int32_t KGp, int32_t RTL, GnArgs a) {
    constexpr int RT = 4 / NB;
    constexpr int RW = 16 * NB;  // weight rows
    extern __shared__ int4 gn_dyn[];
    __shared__ int s_tab[256];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 15, kg = lane >> 4;
    const int nks = KGp >> 2;  // 64-byte K-steps, 1..KM
    const int RX = 16 * RT * RTL;               // the work-group's rows
    int8_t* const s_x = (int8_t*)gn_dyn;
    int8_t* const s_w = s_x + RX * nks * 64;
    const int cw = (int)blockIdx.y * RW;          // the work-group's channels
    const int c0 = cw + (wave % NB) * 16;         // this wave's
    const int64_t px = (int64_t)blockIdx.x * RX;  // the work-group's rows

    // every request first: the table entry, then the direct loads of both
    // operands (instruction i of an operand: segments 16 i .. 16 i + 15 in
    // (K-step, row) order, row fastest; lane l: segment 16 i + l / 4,
    // position l % 4), then the constants
    const int tv = ((const int*)(plan + PLAN_E))[tid];
    const int g = lane >> 2, q = lane & 3;
    auto dloads = [&](const int8_t* base, int64_t rs, int R, int64_t rmax,
                      int8_t* dst) __attribute__((always_inline)) {
        const int n = R * nks / 16;  // instructions (R a multiple of 16)
        for (int i = wave; i < n; i += 4) {
            const int sg = 16 * i + g, st = sg / R, r = sg - st * R;
            const int64_t row = min((int64_t)r, rmax);
            __builtin_amdgcn_global_load_lds(
                base + row * rs + 64 * st + 16 * (q ^ ((r >> 2) & 3)),
                dst + 1024 * i, 16, 0, 0);
        }
    };
    v4i fwr[KM];
    if (WF) {  // fragment (tile c0 / 16, K-step s) at 1024 (tile nks + s)
        const int8_t* wr = wf + (int64_t)(c0 >> 4) * nks * 1024 + 16 * lane;
#pragma unroll
        for (int s = 0; s < KM; ++s)
            fwr[s] = *(const v4i*)(wr + 1024 * min(s, nks - 1));
    }
    uint32_t fix = 0;  // CV: this lane's padding chunks (instruction bits)
    if (CV) {
        const int n = RX * nks / 16;
        const int ohw = a.OH * a.OW;
        int k = 0;
        for (int i = wave; i < n; i += 4, ++k) {
            const int sg = 16 * i + g, st = sg / RX, r = sg - st * RX;
            const int64_t p = min(px + r, M - 1);
            const int nimg = (int)(p / ohw);
            const int rem = (int)(p - (int64_t)nimg * ohw);
            const int oy = rem / a.OW, ox = rem - oy * a.OW;
            const int tap = st / a.CBK, cpart = st - tap * a.CBK;
            const int ky = tap / a.KW, kx = tap - ky * a.KW;
            const int iy = oy * a.SH - a.PH + ky * a.DH;
            const int ix = ox * a.SW - a.PW + kx * a.DW;
            const bool in = iy >= 0 && iy < a.H && ix >= 0 && ix < a.W;
            fix |= (in ? 0u : 1u) << k;
            __builtin_amdgcn_global_load_lds(
                x + (int64_t)nimg * a.x_sn +
                    ((int64_t)(in ? iy : 0) * a.W + (in ? ix : 0)) * xpst +
                    64 * cpart + 16 * (q ^ ((r >> 2) & 3)),
                s_x + 1024 * i, 16, 0, 0);
        }
    } else {
        dloads(x + px * xpst, xpst, RX, M - 1 - px, s_x);
    }
    if (!WF)  // weight rows cw .. cw + RW - 1 (packed rows padded to 128)
        dloads(a.wp + (int64_t)cw * 16 * KGp, 16 * KGp, RW, RW - 1, s_w);
    const int4 hdr = *(const int4*)plan;
    const int pD = ((const int*)plan)[4];
    int4 pc[4];
    uint32_t crr[4], cbo[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int c = min(c0 + 4 * kg + r, a.Cout - 1);
        pc[r] = ((const int4*)(plan + PLAN_CH))[c];
        crr[r] = a.corr ? (uint32_t)a.corr[c] : 0u;
        cbo[r] = RS ? (uint32_t)a.boff[c] : 0u;
    }
    // every load done (the direct ones among them), the table to LDS, then
    // one bare barrier (the empty asm keeps LDS accesses on their side)
    __builtin_amdgcn_s_waitcnt(0x0f70);
    s_tab[tid] = tv;
    if (CV && fix) {  // padding taps: the pad value over what was loaded
        const int pv = (int)((uint32_t)(uint8_t)a.padv * 0x01010101u);
        const int n = RX * nks / 16;
        int k = 0;
        for (int i = wave; i < n; i += 4, ++k)
            if ((fix >> k) & 1)
                *(v4i*)(s_x + 1024 * i + 16 * lane) = v4i{pv, pv, pv, pv};
    }
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (!WF) {
        const int8_t* fw0 =
            s_w + (c0 - cw + col) * 64 + 16 * (kg ^ ((col >> 2) & 3));
#pragma unroll
        for (int s = 0; s < KM; ++s)
            fwr[s] = *(const v4i*)(fw0 + min(s, nks - 1) * RW * 64);
    }
    int64_t cc[4];
#pragma unroll
    for (int r = 0; r < 4; ++r)
        cc[r] = plan_fold((int64_t)(((uint64_t)(uint32_t)pc[r].w << 32) |
                                    (uint32_t)pc[r].z),
                          crr[r], pc[r].x);
    const int pA = hdr.x, pB = hdr.y;
    const bool idt = hdr.w & PLAN_IDENT;
    const int cs = c0 + 4 * kg;  // the lane's 4 channels (Cout % 4 == 0)
    // row tile j = wave / NB + RT t of the work-group: rows 16 j + col,
    // chunk kg of K-step s
    for (int t = 0; t < RTL; ++t) {
        const int j = wave / NB + RT * t;
        const int8_t* fx0 =
            s_x + (16 * j + col) * 64 + 16 * (kg ^ ((col >> 2) & 3));
        v4i acc = v4i{0, 0, 0, 0};
        int psum = 0;
#pragma unroll
        for (int s = 0; s < KM; ++s) {
            if (s < nks) {
                const v4i fx = *(const v4i*)(fx0 + s * RX * 64);
                acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(fwr[s], fx, acc,
                                                           0, 0, 0);
                if (RS) psum += bytes_sum(fx, 16);
            }
        }
        if (RS) {  // the row's byte sum over its 4 k-group lanes
            psum += __shfl_xor(psum, 16);
            psum += __shfl_xor(psum, 32);
        }
        int e[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            int w = acc[r];
            if (RS) w += (int)(cbo[r] * (uint32_t)psum);
            const int v = med3_i32(plan_q0(w, pc[r].x, cc[r], pc[r].y), pA,
                                   pB);
            e[r] = idt ? v + pD : s_tab[v - pA];
        }
        const int64_t p = px + 16 * j + col;
        if (p < M && cs < a.Cout) {
            *(uint32_t*)(a.y + p * a.ypst + cs) = pack_entries(e, 0);
            if (a.y2)
                *(uint32_t*)(a.y2 + p * a.y2pst + cs) = pack_entries(e, 1);
        }
    }
}

}  // namespace

// A k x k convolution the narrow kernel takes as a GEMM over im2col rows
// (tile codes with the weights in fragment order).
bool narrow_conv_applies(const ConvArgs& b, int epi) {
    const uintptr_t xa = (uintptr_t)b.x;
    return epi == Q8_TABLE && b.mode == EPI_QUANT && b.fastio && b.plan &&
           !b.res && b.G == 1 && b.layout == 0 && b.wfrag &&
           (b.KH > 1 || b.KW > 1 || b.SH > 1 || b.SW > 1 || b.PH > 0 ||
            b.PW > 0 || b.OH != b.H || b.OW != b.W) &&
           b.x_code == 1 && b.x_sc == 1 && b.Cg % 64 == 0 &&
           b.x_sp % 16 == 0 && b.x_sn % 16 == 0 && xa % 16 == 0 &&
           b.KGp * 16 == b.Cg * b.KH * b.KW &&
           b.Cout >= 16 && b.Cout % 4 == 0 &&
           (b.Cout <= 64 ? b.Cout % 16 == 0 : b.Cout <= 64 * 65535) &&
           (b.KGp <= 36 || (b.KGp <= 4 * GN_KMAX && b.Cout >= 64)) &&
           b.wp_rstride == (int64_t)b.KGp * 16 && b.y_code == 1 &&
           b.M < ((int64_t)1 << 31) &&
           (int64_t)b.OH * b.OW < ((int64_t)1 << 31) &&
           (int64_t)b.H * b.W * b.x_sp < ((int64_t)1 << 31);
}

bool gemm_narrow_applies(const ConvArgs& b, int epi) {
    if (narrow_conv_applies(b, epi)) return true;
    const uintptr_t xa = (uintptr_t)b.x;
    const int64_t hw = (int64_t)b.H * b.W;
    // a row's stride: the GEMM's row stride, or the pixel stride of a
    // dense channels-last tensor
    const int64_t xpst = hw == 1 ? b.x_sn : b.x_sp;
    return epi == Q8_TABLE && b.mode == EPI_QUANT && b.fastio && b.plan &&
           !b.res && b.G == 1 && b.layout == 0 && b.KH == 1 &&
           b.KW == 1 && b.SH == 1 && b.SW == 1 && b.PH == 0 && b.PW == 0 &&
           b.OH == b.H && b.OW == b.W && (hw == 1 || b.x_sn == hw * b.x_sp) &&
           b.x_code == 1 && b.x_sc == 1 && xpst % 16 == 0 && xa % 16 == 0 &&
           b.Cout >= 16 && b.Cout % 4 == 0 &&
           (b.Cout <= 64 ? b.Cout % 16 == 0 : b.Cout <= 64 * 65535) &&
           b.Cg % 64 == 0 && b.KGp * 16 == b.Cg &&
           (b.KGp <= 36 ||
            (b.KGp <= 4 * GN_KMAX && b.Cout >= 64 && b.wfrag)) &&
           b.wp_rstride == (int64_t)b.KGp * 16 && b.y_code == 1 &&
           b.M < ((int64_t)1 << 31);
}

bool launch_gemm_narrow(const ConvArgs& b, hipStream_t st, int rtl) {
    // Cout 16 / 32 / 64: one channel block of Cout; beyond, blocks of 64
    const int nb = b.Cout <= 64 ? b.Cout / 16 : 4;
    // row tiles a wave: 1..4, fewer where the rows would not fit in 64 KB
    // of LDS (results do not depend on it)
    const int64_t per = (int64_t)(b.KGp / 4) * 64 * 16 * (4 / nb);
    const int64_t wrows = b.wfrag ? 0 : (int64_t)(b.KGp / 4) * 64 * 16 * nb;
    rtl = std::max(1, std::min(rtl, 4));
    while (rtl > 1 && per * rtl + wrows > 64 * 1024) --rtl;
    const int rx = 16 * (4 / nb) * rtl;  // rows a work-group
    const int64_t blocks = ceil_div(b.M, rx);
    const int64_t cblocks = ceil_div(b.Cout, 16 * nb);
    if (blocks >= ((int64_t)1 << 31) || cblocks > 65535) {
        set_error("launch_gemm_narrow", "grid too large");
        return false;
    }
    GnArgs g;
    g.x = (const int8_t*)b.x;
    g.wp = b.wp;
    g.wf = b.wfrag;
    g.plan = (const char*)b.plan;
    g.corr = b.corr;
    g.boff = b.boff;
    g.y = (int8_t*)b.y;
    g.y2 = (int8_t*)b.y2;
    g.xpst = (int64_t)b.H * b.W == 1 ? b.x_sn : b.x_sp;
    g.ypst = b.y_pst;
    g.y2pst = b.y2_pst;
    g.M = b.M;
    g.KGp = b.KGp;
    g.Cout = b.Cout;
    g.RTL = rtl;
    g.pad = 0;
    const bool cv = narrow_conv_applies(b, Q8_TABLE);
    if (cv) {
        g.xpst = b.x_sp;
        g.x_sn = b.x_sn;
        g.H = b.H;
        g.W = b.W;
        g.OH = b.OH;
        g.OW = b.OW;
        g.SH = b.SH;
        g.SW = b.SW;
        g.PH = b.PH;
        g.PW = b.PW;
        g.DH = b.DH;
        g.DW = b.DW;
        g.KW = b.KW;
        g.CBK = b.Cg / 64;
        g.padv = b.pad_value;
    }
    const dim3 grid((unsigned)blocks, (unsigned)cblocks);
    // activation rows, then (without fragment order) the weight rows
    const size_t lds = (size_t)(b.KGp / 4) * 64 *
                       (rx + (b.wfrag ? 0 : 16 * nb));
    if (lds > 64 * 1024) {
        set_error("launch_gemm_narrow", "rows do not fit in LDS");
        return false;
    }
    if (cv) {  // im2col rows, fragment-order weights
        const int kcase = (b.KGp > 36 ? 0 : nb) * 2 + (b.rowsum ? 1 : 0);
        switch (kcase) {
#define QA_GN_CV(NB, RS, KM)                                                  \
    case (KM == 9 ? NB : 0) * 2 + RS:                                        \
        k_gemm_narrow<NB, RS != 0, true, KM, true><<<grid, 256, lds, st>>>(GN_ARGS(g)); \
        break;
            QA_GN_CV(1, 0, 9) QA_GN_CV(1, 1, 9) QA_GN_CV(2, 0, 9)
            QA_GN_CV(2, 1, 9) QA_GN_CV(4, 0, 9) QA_GN_CV(4, 1, 9)
            QA_GN_CV(4, 0, GN_KMAX) QA_GN_CV(4, 1, GN_KMAX)
#undef QA_GN_CV
        }
    } else if (b.KGp > 36) {  // 10..20 K-steps: 64-channel blocks
        if (nb != 4 || !b.wfrag) {
            set_error("launch_gemm_narrow", "K past 576 needs 64-channel "
                                            "blocks and fragment-order "
                                            "weights");
            return false;
        }
        if (b.rowsum)
            k_gemm_narrow<4, true, true, GN_KMAX><<<grid, 256, lds, st>>>(GN_ARGS(g));
        else
            k_gemm_narrow<4, false, true, GN_KMAX><<<grid, 256, lds, st>>>(GN_ARGS(g));
    } else {
        switch (nb * 4 + (b.rowsum ? 2 : 0) + (b.wfrag ? 1 : 0)) {
#define QA_GN_CASE(NB, RS, WF)                                            \
    case NB * 4 + RS * 2 + WF:                                            \
        k_gemm_narrow<NB, RS != 0, WF != 0, 9><<<grid, 256, lds, st>>>(GN_ARGS(g)); \
        break;
            QA_GN_CASE(1, 0, 0) QA_GN_CASE(1, 1, 0) QA_GN_CASE(2, 0, 0)
            QA_GN_CASE(2, 1, 0) QA_GN_CASE(4, 0, 0) QA_GN_CASE(4, 1, 0)
            QA_GN_CASE(1, 0, 1) QA_GN_CASE(1, 1, 1) QA_GN_CASE(2, 0, 1)
            QA_GN_CASE(2, 1, 1) QA_GN_CASE(4, 0, 1) QA_GN_CASE(4, 1, 1)
#undef QA_GN_CASE
        }
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_hip_error("launch_gemm_narrow", e);
        return false;
    }
    return true;
}

}  // namespace qa

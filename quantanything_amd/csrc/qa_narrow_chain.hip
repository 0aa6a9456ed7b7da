// A convolution and the 1x1 convolution that alone reads its output, in
// one launch, as two GEMMs over the same rows: conv 1 (1x1, or k x k over
// its im2col rows, C1 <= 256 output channels) writes its stored bytes into
// an LDS tile of the work-group's rows, and conv 2 (1x1, C1 -> C2 <= 256)
// reads them from there; conv 1's output never goes to HBM. The late-stage
// pairs of a classifier backbone (the stride-2 3x3 conv into a C2f block
// and the block's first 1x1 conv) are this shape.
//
// A work-group of 8 waves owns 16 RTL rows (output pixels) and every
// channel of both convolutions. Every load is issued before the first use:
// conv 1's rows go to LDS by direct global -> LDS loads (each group of 4
// lanes one 64-byte K-step of one row: one tap's 64 channels of one input
// pixel; taps outside the image get the pad value afterwards), conv 1's
// weight fragments (fragment order, one contiguous KB a load) go straight
// into the VGPRs of the wave that owns their channel tile (tile j to wave
// j % 8), requested last so that its MFMAs start as they arrive; conv 2's
// whole weight set, both tables and every channel's plan constants go to
// LDS by direct loads. MFMA v_mfma_i32_16x16x64_i8 with the weights as the first operand,
// so the result lane l holds channels 4 (l >> 4) + r of row (l & 15): the
// 4 stored bytes are one word, into the LDS tile (conv 1) or to HBM (conv
// 2, with the rescaled copy of a Concat). Epilogues: the table plan of
// qa_conv.h (multiply-add and shift with the correction folded into the
// constant, one med3 clip, one table read).
#include "qa_conv_mfma.h"

namespace qa {
namespace {

constexpr int NC_NW = 8;           // waves a work-group
constexpr int NC_NT = 64 * NC_NW;  // threads
constexpr int NC_CMAX = 256;       // channels of either convolution

struct NcArgs {
    // conv 1: rows of the GEMM (CV: im2col rows of the image)
    const int8_t* x;
    int64_t xpst, x_sn;  // row (pixel) and image strides
    const int8_t* wf1;   // fragment-order weights
    const char* plan1;
    const int64_t* corr1;
    // conv 2
    const int8_t* wf2;
    const char* plan2;
    const int64_t* corr2;
    int8_t* y;
    int8_t* y2;
    int64_t ypst, y2pst, M;
    int32_t ks1, ks2, C1, C2, RTL, RSM;
    int32_t H, W, OH, OW, SH, SW, PH, PW, DH, DW, KW, CBK, padv, lds_m,
        lds_w2;
};

// KM1: K-steps of conv 1 (exactly: its MFMA sequence has no branches,
// so each MFMA waits for its own weight fragment only); CT1 / CT2: channel
// tiles a wave owns at most in each conv; CV1: conv 1 is a k x k
// convolution.
// NW2: conv 2's fragment loads a wave (2 or 8; a fixed count, so that the
// waits for conv 1's weights, requested before them, count exactly).
// s_waitcnt vmcnt(n) for a count known after unrolling (n < 64)
__device__ __forceinline__ void wait_vm(int n) {
#define QA_VM(N) \
    case N:      \
        __builtin_amdgcn_s_waitcnt(0x0f70 | ((N) & 15) | (((N) >> 4) << 14)); \
        break;
#define QA_VM4(N) QA_VM(N) QA_VM(N + 1) QA_VM(N + 2) QA_VM(N + 3)
#define QA_VM16(N) QA_VM4(N) QA_VM4(N + 4) QA_VM4(N + 8) QA_VM4(N + 12)
    switch (n) {
        QA_VM16(0) QA_VM16(16) QA_VM16(32) QA_VM16(48)
        default: __builtin_amdgcn_s_waitcnt(0x0f70); break;
    }
#undef QA_VM16
#undef QA_VM4
#undef QA_VM
}

template <int KM1, int CT1, int CT2, bool CV1, int NW2>
__global__ __launch_bounds__(NC_NT) void k_narrow_chain(NcArgs a) {
    extern __shared__ int4 nc_dyn[];
    int8_t* const s_x = (int8_t*)nc_dyn;   // conv 1's rows
    int8_t* const s_m = s_x + a.lds_m;     // conv 1's output tile
    int8_t* const s_w2 = s_x + a.lds_w2;   // conv 2's weights
    __shared__ __attribute__((aligned(16))) int s_tab1[256], s_tab2[256];
    __shared__ int4 s_pc[2][NC_CMAX];
    __shared__ __attribute__((aligned(16))) int64_t s_cr[2][NC_CMAX];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 15, kg = lane >> 4;
    const int g = lane >> 2, q = lane & 3;
    const int RX = 16 * a.RTL;
    const int64_t px = (int64_t)blockIdx.x * RX;
    constexpr int ks1 = KM1;
    const int ks2 = a.ks2;
    const int T1 = a.C1 >> 4, T2 = a.C2 >> 4;

    const int4 hdr1 = *(const int4*)a.plan1;
    const int4 hdr2 = *(const int4*)a.plan2;

    // ---- every request first: the tables, the plans' per-channel
    // constants and the corrections by direct global -> LDS loads (16
    // bytes a lane; channels past the last read the last one), the waves
    // taking turns
    {
        const int n1 = (a.C1 + 63) >> 6, n2 = (a.C2 + 63) >> 6;
        const int m1 = a.corr1 ? (a.C1 + 127) >> 7 : 0;
        const int m2 = a.corr2 ? (a.C2 + 127) >> 7 : 0;
        const int items = 2 + n1 + n2 + m1 + m2;
        for (int it = wave; it < items; it += NC_NW) {
            const int8_t* src;
            int8_t* dst;
            if (it < 2) {
                src = (const int8_t*)(it ? a.plan2 : a.plan1) + PLAN_E +
                      16 * lane;
                dst = (int8_t*)(it ? s_tab2 : s_tab1);
            } else if (it < 2 + n1 + n2) {
                const int h = it >= 2 + n1, i = it - 2 - (h ? n1 : 0);
                const int c = min(64 * i + lane, (h ? a.C2 : a.C1) - 1);
                src = (const int8_t*)(h ? a.plan2 : a.plan1) + PLAN_CH +
                      16 * c;
                dst = (int8_t*)&s_pc[h][64 * i];
            } else {
                const int h = it >= 2 + n1 + n2 + m1;
                const int i = it - 2 - n1 - n2 - (h ? m1 : 0);
                const int c = min(128 * i + 2 * lane, (h ? a.C2 : a.C1) - 2);
                src = (const int8_t*)((h ? a.corr2 : a.corr1) + c);
                dst = (int8_t*)&s_cr[h][128 * i];
            }
            __builtin_amdgcn_global_load_lds(src, dst, 16, 0, 0);
        }
    }
    // conv 1's rows: instruction i covers segments 16 i .. 16 i + 15 in
    // (K-step, row) order, row fastest; lane l: segment 16 i + l / 4,
    // position l % 4 holding chunk (l % 4) ^ ((row >> 2) & 3)
    uint32_t fix = 0;  // CV1: this lane's padding chunks (instruction bits)
    {
        const int n = RX * ks1 / 16;
        const int ohw = a.OH * a.OW;
        int k = 0;
        for (int i = wave; i < n; i += NC_NW, ++k) {
            const int sg = 16 * i + g, st = sg / RX, r = sg - st * RX;
            const int64_t p = min(px + r, a.M - 1);
            const int sw = 16 * (q ^ ((r >> 2) & 3));
            const int8_t* src;
            if (CV1) {
                const int nimg = (int)(p / ohw);
                const int rem = (int)(p - (int64_t)nimg * ohw);
                const int oy = rem / a.OW, ox = rem - oy * a.OW;
                const int tap = st / a.CBK, cpart = st - tap * a.CBK;
                const int ky = tap / a.KW, kx = tap - ky * a.KW;
                const int iy = oy * a.SH - a.PH + ky * a.DH;
                const int ix = ox * a.SW - a.PW + kx * a.DW;
                const bool in = iy >= 0 && iy < a.H && ix >= 0 && ix < a.W;
                fix |= (in ? 0u : 1u) << k;
                src = a.x + (int64_t)nimg * a.x_sn +
                      ((int64_t)(in ? iy : 0) * a.W + (in ? ix : 0)) *
                          a.xpst +
                      64 * cpart + sw;
            } else {
                src = a.x + p * a.xpst + 64 * st + sw;
            }
            __builtin_amdgcn_global_load_lds(src, s_x + 1024 * i, 16, 0, 0);
        }
    }
    asm volatile("" ::: "memory");  // the weights' loads stay after these
    // conv 1's weight fragments of the wave's tiles (a tile past the last
    // reads the last one and is not stored), requested last: the barrier
    // below waits for everything before them only, and conv 1's MFMAs
    // start as its fragments arrive
    v4i w1[CT1][KM1];
    const int8_t* wr[CT1];
#pragma unroll
    for (int i = 0; i < CT1; ++i)
        wr[i] = a.wf1 + (int64_t)min(wave + NC_NW * i, T1 - 1) * ks1 * 1024 +
                16 * lane;
#pragma unroll
    for (int s = 0; s < KM1; ++s) {  // in the order the MFMAs use them
#pragma unroll
        for (int i = 0; i < CT1; ++i)
            w1[i][s] = *(const v4i*)(wr[i] + 1024 * s);
        asm volatile("" ::: "memory");  // (kept in that order)
    }
    // conv 2's weights, fragment order, to LDS (needed after conv 1 only);
    // slots past the last fragment load the last one again into its own
    // place (the same bytes)
#pragma unroll
    for (int k = 0; k < NW2; ++k) {
        const int i = min(wave + NC_NW * k, T2 * ks2 - 1);
        __builtin_amdgcn_global_load_lds(a.wf2 + 1024 * i + 16 * lane,
                                         s_w2 + 1024 * i, 16, 0, 0);
    }

    // the tables, constants and rows landed (loads complete in issue
    // order: conv 1's weights and conv 2's follow them); the padding taps'
    // pad value; one bare barrier
    constexpr int NW = CT1 * KM1 + NW2;  // loads after the rows (<= 44)
    __builtin_amdgcn_s_waitcnt(0x0f70 | (NW & 15) | ((NW >> 4) << 14));
    if (CV1 && fix) {
        const int pv = (int)((uint32_t)(uint8_t)a.padv * 0x01010101u);
        const int n = RX * ks1 / 16;
        int k = 0;
        for (int i = wave; i < n; i += NC_NW, ++k)
            if ((fix >> k) & 1)
                *(v4i*)(s_x + 1024 * i + 16 * lane) = v4i{pv, pv, pv, pv};
    }
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");

    // the table epilogue of one accumulator: channels c + r of conv h
    auto epi = [&](int h, const v4i& acc, int c, const int4& hdr,
                   const int* tab, int (&e)[4])
                   __attribute__((always_inline)) {
        const int* tabE = tab - hdr.x;
        const bool corr = h ? a.corr2 != nullptr : a.corr1 != nullptr;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int4 pc = s_pc[h][c + r];
            const int64_t cc = plan_fold(
                (int64_t)(((uint64_t)(uint32_t)pc.w << 32) | (uint32_t)pc.z),
                corr ? (uint32_t)s_cr[h][c + r] : 0u, pc.x);
            e[r] = tabE[med3_i32(plan_q0(acc[r], pc.x, cc, pc.y), hdr.x,
                                 hdr.y)];
        }
    };
    const int sw = 16 * (kg ^ ((col >> 2) & 3));
    // ---- conv 1: row tiles t, the wave's channel tiles; stored bytes to
    // the LDS tile (rows of RSM bytes). The first row tile is peeled off
    // the loop, so that its MFMAs wait for each weight fragment in turn
    // (a loop over them would wait for all of them first).
    auto conv1_tile = [&](int t, auto first) __attribute__((always_inline)) {
        constexpr bool FIRST = decltype(first)::value;
        const int8_t* fx0 = s_x + (16 * t + col) * 64 + sw;
        v4i acc[CT1];
#pragma unroll
        for (int i = 0; i < CT1; ++i) acc[i] = v4i{0, 0, 0, 0};
#pragma unroll
        for (int s = 0; s < KM1; ++s) {
            if (FIRST) wait_vm(NW - CT1 * (s + 1));
            const v4i fx = *(const v4i*)(fx0 + s * RX * 64);
#pragma unroll
            for (int i = 0; i < CT1; ++i)
                acc[i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                    w1[i][s], fx, acc[i], 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < CT1; ++i) {
            const int j = wave + NC_NW * i;
            if (j < T1) {
                int e[4];
                epi(0, acc[i], 16 * j + 4 * kg, hdr1, s_tab1, e);
                *(uint32_t*)(s_m + (16 * t + col) * a.RSM + 16 * j + 4 * kg) =
                    pack_entries(e, 0);
            }
        }
    };
    conv1_tile(0, std::true_type{});
    for (int t = 1; t < a.RTL; ++t) conv1_tile(t, std::false_type{});
    // conv 2's weights landed too; the tile written
    __builtin_amdgcn_s_waitcnt(0x0f70);
    __syncthreads();

    // ---- conv 2 over the LDS tile: the wave's channel tiles j2, stored
    // words (and the rescaled copy)
    for (int t = 0; t < a.RTL; ++t) {
        const int8_t* fm = s_m + (16 * t + col) * a.RSM + 16 * kg;
        v4i acc[CT2];
#pragma unroll
        for (int i = 0; i < CT2; ++i) acc[i] = v4i{0, 0, 0, 0};
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            if (s < ks2) {
                const v4i fx = *(const v4i*)(fm + 64 * s);
#pragma unroll
                for (int i = 0; i < CT2; ++i) {
                    const int j2 = min(wave + NC_NW * i, T2 - 1);
                    const v4i wv = *(const v4i*)(s_w2 + (j2 * ks2 + s) * 1024 +
                                                 16 * lane);
                    acc[i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wv, fx,
                                                                  acc[i], 0,
                                                                  0, 0);
                }
            }
        }
        const int64_t p = px + 16 * t + col;
#pragma unroll
        for (int i = 0; i < CT2; ++i) {
            const int j2 = wave + NC_NW * i;
            if (j2 < T2 && p < a.M) {
                int e[4];
                const int c = 16 * j2 + 4 * kg;
                epi(1, acc[i], c, hdr2, s_tab2, e);
                *(uint32_t*)(a.y + p * a.ypst + c) = pack_entries(e, 0);
                if (a.y2)
                    *(uint32_t*)(a.y2 + p * a.y2pst + c) = pack_entries(e, 1);
            }
        }
    }
}

using NcKern = void (*)(NcArgs);

template <int KM1, bool CV1>
NcKern nc_kernel_ct(int ct1, int ct2, int nw2) {
    if (nw2 <= 2) {
        if (ct1 == 1)
            return ct2 == 1 ? &k_narrow_chain<KM1, 1, 1, CV1, 2>
                            : &k_narrow_chain<KM1, 1, 2, CV1, 2>;
        return ct2 == 1 ? &k_narrow_chain<KM1, 2, 1, CV1, 2>
                        : &k_narrow_chain<KM1, 2, 2, CV1, 2>;
    }
    if (ct1 == 1)
        return ct2 == 1 ? &k_narrow_chain<KM1, 1, 1, CV1, 8>
                        : &k_narrow_chain<KM1, 1, 2, CV1, 8>;
    return ct2 == 1 ? &k_narrow_chain<KM1, 2, 1, CV1, 8>
                    : &k_narrow_chain<KM1, 2, 2, CV1, 8>;
}

// The instantiated K-step counts of conv 1: 2 and 4 (1x1 over 128 or 256
// channels), 9 (3x3 over 64, or 1x1 over 576), 18 (3x3 over 128).
NcKern nc_kernel(bool cv, int ks1, int ct1, int ct2, int nw2) {
    if (cv) {
        switch (ks1) {
            case 9: return nc_kernel_ct<9, true>(ct1, ct2, nw2);
            case 18: return nc_kernel_ct<18, true>(ct1, ct2, nw2);
            default: return nullptr;
        }
    }
    switch (ks1) {
        case 2: return nc_kernel_ct<2, false>(ct1, ct2, nw2);
        case 4: return nc_kernel_ct<4, false>(ct1, ct2, nw2);
        case 9: return nc_kernel_ct<9, false>(ct1, ct2, nw2);
        default: return nullptr;
    }
}

// conv 1 as rows of a GEMM (1x1, stride 1, no padding) or not
bool nc_gemm_rows(const ConvArgs& b) {
    return b.KH == 1 && b.KW == 1 && b.SH == 1 && b.SW == 1 && b.PH == 0 &&
           b.PW == 0 && b.OH == b.H && b.OW == b.W;
}

// LDS layout for RTL row tiles: conv 1's rows, the output tile, conv 2's
// weights; 0 when it does not fit
int nc_lds(const ConvArgs& b1, const ConvArgs& b2, int rtl, int* off_m,
           int* off_w2, int* rsm) {
    const int rx = 16 * rtl;
    const int64_t xb = (int64_t)rx * (b1.KGp / 4) * 64;
    *rsm = b1.Cout + 16;
    const int64_t mb = (int64_t)rx * *rsm;
    const int64_t wb = (int64_t)(b2.Cout / 16) * (b2.KGp / 4) * 1024;
    *off_m = (int)xb;
    *off_w2 = (int)(xb + mb);
    const int64_t tot = xb + mb + wb;
    return tot <= 128 * 1024 ? (int)tot : 0;
}

}  // namespace

bool narrow_chain_applies(const ConvArgs& b1, const ConvArgs& b2) {
    const uintptr_t xa = (uintptr_t)b1.x;
    const bool rows1 = nc_gemm_rows(b1);
    const int64_t hw = (int64_t)b1.H * b1.W;
    auto table = [](const ConvArgs& b) {
        return b.mode == EPI_QUANT && b.fastio && b.plan && b.G == 1 &&
               b.layout == 0 && b.wfrag && b.rowsum == 0 && !b.res &&
               b.y_code == 1 && b.gate == nullptr;
    };
    int om, ow, rs;
    return table(b1) && table(b2) && !b1.y2 && b1.x_code == 1 &&
           b1.x_sc == 1 && b1.Cg % 64 == 0 &&
           b1.KGp * 16 == b1.Cg * b1.KH * b1.KW && b1.KGp <= 80 &&
           b1.Cout % 16 == 0 && b1.Cout >= 16 && b1.Cout <= NC_CMAX &&
           xa % 16 == 0 && b1.x_sp % 16 == 0 && b1.x_sn % 16 == 0 &&
           (rows1 ? (hw == 1 || b1.x_sn == hw * b1.x_sp) : true) &&
           b2.KH == 1 && b2.KW == 1 && b2.SH == 1 && b2.SW == 1 &&
           b2.PH == 0 && b2.PW == 0 && b2.x == b1.y && b2.N == b1.N &&
           b2.H == b1.OH && b2.W == b1.OW && b2.OH == b2.H &&
           b2.OW == b2.W && b2.Cg == b1.Cout && b2.KGp * 16 == b2.Cg &&
           b2.Cout % 16 == 0 && b2.Cout >= 16 && b2.Cout <= NC_CMAX &&
           b2.y_pst % 4 == 0 && (uintptr_t)b2.y % 4 == 0 &&
           (b2.y2 == nullptr ||
            ((uintptr_t)b2.y2 % 4 == 0 && b2.y2_pst % 4 == 0)) &&
           b1.M < ((int64_t)1 << 31) &&
           (int64_t)b1.H * b1.W * b1.x_sp < ((int64_t)1 << 31) &&
           nc_kernel(!rows1, b1.KGp / 4, 1, 1, 1) != nullptr &&
           (b2.Cout / 16) * (b2.KGp / 4) <= 8 * NC_NW &&
           nc_lds(b1, b2, 1, &om, &ow, &rs) > 0;
}

// rtl: row tiles of 16 a work-group (1..4; fewer where LDS runs out)
bool launch_narrow_chain(const ConvArgs& b1, const ConvArgs& b2, int rtl,
                         hipStream_t st) {
    if (!narrow_chain_applies(b1, b2)) {
        set_error("launch_narrow_chain", "convolutions outside the kernel's "
                                         "scope");
        return false;
    }
    rtl = std::max(1, std::min(rtl, 4));
    int om = 0, ow = 0, rsm = 0;
    while (rtl > 1 && nc_lds(b1, b2, rtl, &om, &ow, &rsm) == 0) --rtl;
    const int lds = nc_lds(b1, b2, rtl, &om, &ow, &rsm);
    const int T1 = b1.Cout / 16, T2 = b2.Cout / 16;
    const int ct1 = T1 > NC_NW ? 2 : 1, ct2 = T2 > NC_NW ? 2 : 1;
    const bool cv = !nc_gemm_rows(b1);
    // conv 2's fragment loads a wave
    const int nw2 = (int)ceil_div((int64_t)T2 * (b2.KGp / 4), NC_NW);
    const NcKern k = nc_kernel(cv, b1.KGp / 4, ct1, ct2, nw2);
    NcArgs a;
    a.x = (const int8_t*)b1.x;
    a.xpst = (int64_t)b1.H * b1.W == 1 && !cv ? b1.x_sn : b1.x_sp;
    a.x_sn = b1.x_sn;
    a.wf1 = b1.wfrag;
    a.plan1 = (const char*)b1.plan;
    a.corr1 = b1.corr;
    a.wf2 = b2.wfrag;
    a.plan2 = (const char*)b2.plan;
    a.corr2 = b2.corr;
    a.y = (int8_t*)b2.y;
    a.y2 = (int8_t*)b2.y2;
    a.ypst = b2.y_pst;
    a.y2pst = b2.y2_pst;
    a.M = b1.M;
    a.ks1 = b1.KGp / 4;
    a.ks2 = b2.KGp / 4;
    a.C1 = b1.Cout;
    a.C2 = b2.Cout;
    a.RTL = rtl;
    a.RSM = rsm;
    a.H = b1.H;
    a.W = b1.W;
    a.OH = b1.OH;
    a.OW = b1.OW;
    a.SH = b1.SH;
    a.SW = b1.SW;
    a.PH = b1.PH;
    a.PW = b1.PW;
    a.DH = b1.DH;
    a.DW = b1.DW;
    a.KW = b1.KW;
    a.CBK = b1.Cg / 64;
    a.padv = b1.pad_value;
    a.lds_m = om;
    a.lds_w2 = ow;
    const int64_t blocks = ceil_div(b1.M, 16 * rtl);
    hipLaunchKernelGGL(k, dim3((unsigned)blocks), dim3(NC_NT), (size_t)lds, st,
                       a);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_hip_error("launch_narrow_chain", e);
        return false;
    }
    return true;
}

}  // namespace qa

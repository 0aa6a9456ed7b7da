// Two pointwise convolutions and a global average pool in one launch: a
// 1x1 convolution C0 -> C1 whose output only feeds a 1x1 convolution
// C1 -> C2 whose output only feeds the pool (the head of a classification
// network: the last C2f block's 1x1 conv, then the 1x1 conv to the head's
// width, pooled). Neither convolution's output is written; the pooled
// int8 values are, as qa_d_conv_pool stores them.
//
// A work-group of 8 waves owns one image (at most 64 pixels) and a block
// of C2 output channels. It runs the whole first convolution of its image
// (the work-groups of one image each compute it again: its weights are
// tens of KB, the image a few thousand MACs per channel) into an LDS image
// of stored bytes, then its block of the second convolution, summing the
// stored bytes of each channel over the image's pixels. A wave holds the
// weight fragments of every channel tile it owns, for all K-steps, in
// VGPRs, loaded straight from global memory: every load of the launch
// (tables, the image's pixels, per-channel constants, both weight sets) is
// issued before the first use, so the work-group waits about one memory
// round trip. The weights come in fragment order (ConvArgs.wfrag:
// the 1 KB MFMA fragment of a 16-channel tile and K-step contiguous, lane
// l's 16 bytes at 16 l), so each wave load is one contiguous KB, whole
// cache lines; read from the packed rows (16 rows x 64 bytes a load, half
// lines) the same bytes took 2.5x as long to arrive.
//
// Channel tiles of 16 go to the waves round robin (tile j to wave j % 8);
// MFMA v_mfma_i32_16x16x64_i8 with 16 pixels as rows and 16 channels as
// columns, so a lane holds one channel and 4 pixels. Epilogues: the table
// plan of qa_conv.h (multiply-add and shift with the correction folded
// into the constant, one med3 clip, one table read) for both; the first
// stores the byte in the LDS image, the second adds the sign-extended
// stored byte of the valid pixels; the pool's requantization is that of
// qa_d_conv_pool.
#include "qa_conv_mfma.h"

namespace qa {
namespace {

constexpr int PP_NW = 8;            // waves per work-group
constexpr int PP_NT = 64 * PP_NW;   // threads
constexpr int PP_PMAX = 64;         // pixels of an image
constexpr int PP_XU = 4;            // image chunks a thread loads (16 bytes)

struct PwPoolGeom {
    int P;       // pixels of an image (OH * OW <= 64)
    int RS1;     // LDS row stride of the input image, 16-byte units
    int RS2;     // of the intermediate image
    int cblk;    // second-convolution channels per work-group
    int nt1;     // 16-channel tiles of the first convolution
    int cr1;     // 16-byte chunks of an input pixel's real channels
    int lds;     // dynamic LDS bytes
};

// KS1 / KS2: K-steps (64 bytes) of the two convolutions; CT1 / CT2: channel
// tiles a wave owns at most (tiles j, j + 8, ...).
// w1f / w2f: the two weight sets in fragment order.
template <int KS1, int CT1, int KS2, int CT2>
__global__ __launch_bounds__(PP_NT) void k_conv_pw_pool(
    ConvArgs a1, ConvArgs a2, PoolArgs pl, PwPoolGeom g,
    const int8_t* __restrict__ w1f, const int8_t* __restrict__ w2f) {
    extern __shared__ int4 pp_lds[];
    int8_t* s_x = (int8_t*)pp_lds;                     // P x RS1 units
    int8_t* s_y = s_x + g.P * g.RS1 * 16;              // 64 x RS2 units
    __shared__ int s_tab1[256], s_tab2[256];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 15, kgl = lane >> 4;
    // the channel blocks of one image run on one XCD (they read the same
    // pixels)
    const XcdBlock blk = xcd_block(true);
    const int n = (int)blk.x;
    const int cb0 = (int)blk.y * g.cblk;
    const int nt2 = min(g.cblk, a2.Cout - cb0) >> 4;
    const int P = g.P;

    // ---- every request first: the tables, the image, the constants, the
    // weights (loads complete in issue order, so the stores below wait for
    // the first ones only)
    const int tv = tid < 256 ? ((const int*)((const char*)a1.plan + PLAN_E))[tid]
                             : ((const int*)((const char*)a2.plan +
                                             PLAN_E))[tid - 256];
    const int8_t* xn = (const int8_t*)a1.x + (int64_t)n * a1.x_sn;
    const int nx = P * g.cr1;  // real chunks of the image
    v4i xv[PP_XU];
    int xat[PP_XU];
#pragma unroll
    for (int j = 0; j < PP_XU; ++j) {
        const int u = tid + j * PP_NT;
        const int p = u / g.cr1, k = u - p * g.cr1;
        const bool ok = u < nx;
        xat[j] = ok ? (p * g.RS1 + k) * 16 : -1;
        xv[j] = *(const v4i*)(xn + (ok ? p * a1.x_sp + k * 16 : 0));
    }
    int4 pc1[CT1], pc2[CT2];
    uint32_t cr1[CT1], cr2[CT2];
#pragma unroll
    for (int i = 0; i < CT1; ++i) {
        const int c = min(16 * (wave + PP_NW * i) + col, a1.Cout - 1);
        pc1[i] = ((const int4*)((const char*)a1.plan + PLAN_CH))[c];
        cr1[i] = a1.corr ? (uint32_t)a1.corr[c] : 0u;
    }
#pragma unroll
    for (int i = 0; i < CT2; ++i) {
        const int c = min(cb0 + 16 * (wave + PP_NW * i) + col, a2.Cout - 1);
        pc2[i] = ((const int4*)((const char*)a2.plan + PLAN_CH))[c];
        cr2[i] = a2.corr ? (uint32_t)a2.corr[c] : 0u;
    }
    // fragment (tile j, K-step s) at 1024 (j KS + s), this lane's 16 bytes
    // at 16 lane; tiles past the last read the last one
    v4i w1[CT1][KS1], w2[CT2][KS2];
#pragma unroll
    for (int i = 0; i < CT1; ++i) {
        const int j = min(wave + PP_NW * i, g.nt1 - 1);
        const int8_t* wr = w1f + (int64_t)j * KS1 * 1024 + 16 * lane;
#pragma unroll
        for (int s = 0; s < KS1; ++s) w1[i][s] = *(const v4i*)(wr + 1024 * s);
    }
#pragma unroll
    for (int i = 0; i < CT2; ++i) {
        const int j = (cb0 >> 4) + min(wave + PP_NW * i, nt2 - 1);
        const int8_t* wr = w2f + (int64_t)j * KS2 * 1024 + 16 * lane;
#pragma unroll
        for (int s = 0; s < KS2; ++s) w2[i][s] = *(const v4i*)(wr + 1024 * s);
    }
    const int4 hdr1 = *(const int4*)a1.plan;
    const int4 hdr2 = *(const int4*)a2.plan;

    // tables (the second's entries as sign-extended stored bytes) and the
    // image to LDS; chunks past the real channels stay unwritten (their
    // weights are zero)
    if (tid < 256)
        s_tab1[tid] = tv;
    else
        s_tab2[tid - 256] = (int)(int8_t)(tv & 255);
#pragma unroll
    for (int j = 0; j < PP_XU; ++j)
        if (xat[j] >= 0) *(v4i*)(s_x + xat[j]) = xv[j];
    __syncthreads();

    const int TP = (P + 15) >> 4;  // pixel tiles
    // ---- the first convolution: the lane's channel 16 (wave + 8 i) + col,
    // pixels 16 t + 4 kgl + r, its stored byte into the LDS image
    {
        int cm[CT1], ct[CT1];
        int64_t cc[CT1];
#pragma unroll
        for (int i = 0; i < CT1; ++i) {
            cm[i] = pc1[i].x;
            ct[i] = pc1[i].y;
            cc[i] = plan_fold((int64_t)(((uint64_t)(uint32_t)pc1[i].w << 32) |
                                        (uint32_t)pc1[i].z),
                              cr1[i], pc1[i].x);
        }
        const int* tabE = s_tab1 - hdr1.x;
        for (int t = 0; t < TP; ++t) {
            const int8_t* xr =
                s_x + (min(16 * t + col, P - 1) * g.RS1 + kgl) * 16;
            v4i f[KS1];
#pragma unroll
            for (int s = 0; s < KS1; ++s) f[s] = *(const v4i*)(xr + 64 * s);
            // every tile of the wave (a tile past the last computes the
            // last one again and is not stored): the tiles' MFMA chains and
            // table reads interleave
            v4i acc[CT1];
#pragma unroll
            for (int i = 0; i < CT1; ++i) acc[i] = v4i{0, 0, 0, 0};
#pragma unroll
            for (int s = 0; s < KS1; ++s)
#pragma unroll
                for (int i = 0; i < CT1; ++i)
                    acc[i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                        f[s], w1[i][s], acc[i], 0, 0, 0);
            int e[CT1][4];
#pragma unroll
            for (int i = 0; i < CT1; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    e[i][r] = tabE[med3_i32(
                        plan_q0(acc[i][r], cm[i], cc[i], ct[i]), hdr1.x,
                        hdr1.y)];
            int8_t* yb = s_y + (16 * t + 4 * kgl) * g.RS2 * 16 + col;
#pragma unroll
            for (int i = 0; i < CT1; ++i) {
                const int tile = wave + PP_NW * i;
                if (tile < g.nt1) {
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        yb[r * g.RS2 * 16 + 16 * tile] = (int8_t)e[i][r];
                }
            }
        }
    }
    __syncthreads();

    // ---- the second convolution over the LDS image, pooled: the lane's
    // channel cb0 + 16 (wave + 8 i) + col
    int cm[CT2], ct[CT2], csum[CT2];
    int64_t cc[CT2];
#pragma unroll
    for (int i = 0; i < CT2; ++i) {
        cm[i] = pc2[i].x;
        ct[i] = pc2[i].y;
        cc[i] = plan_fold((int64_t)(((uint64_t)(uint32_t)pc2[i].w << 32) |
                                    (uint32_t)pc2[i].z),
                          cr2[i], pc2[i].x);
        csum[i] = 0;
    }
    const int* tabE2 = s_tab2 - hdr2.x;
    for (int t = 0; t < TP; ++t) {
        const int8_t* xr = s_y + (min(16 * t + col, P - 1) * g.RS2 + kgl) * 16;
        v4i f[KS2];
#pragma unroll
        for (int s = 0; s < KS2; ++s) f[s] = *(const v4i*)(xr + 64 * s);
        const int nv = P - (16 * t + 4 * kgl);  // the lane's real pixels
        v4i acc[CT2];
#pragma unroll
        for (int i = 0; i < CT2; ++i) acc[i] = v4i{0, 0, 0, 0};
#pragma unroll
        for (int s = 0; s < KS2; ++s)
#pragma unroll
            for (int i = 0; i < CT2; ++i)
                acc[i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(f[s], w2[i][s],
                                                              acc[i], 0, 0, 0);
#pragma unroll
        for (int i = 0; i < CT2; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int e = tabE2[med3_i32(
                    plan_q0(acc[i][r], cm[i], cc[i], ct[i]), hdr2.x, hdr2.y)];
                csum[i] += r < nv ? e : 0;
            }
    }
    // the 4 lane groups' sums; lanes 0..15 hold their channels' pools
#pragma unroll
    for (int i = 0; i < CT2; ++i) {
        if (wave + PP_NW * i >= nt2) break;
        int s = csum[i];
        s += __shfl_xor(s, 16);
        s += __shfl_xor(s, 32);
        const int c = cb0 + 16 * (wave + PP_NW * i) + col;
        if (kgl == 0) {
            const int64_t q =
                qa_clip128(qa_mbqm((int64_t)s + pl.base, pl.mult, pl.shift) +
                               pl.zp,
                           pl.qmin, pl.qmax);
            pl.out[(int64_t)n * pl.out_sn + c] = (int8_t)(q - pl.out_so);
        }
    }
}

using PpKern = void (*)(ConvArgs, ConvArgs, PoolArgs, PwPoolGeom,
                       const int8_t*, const int8_t*);

// Fragment order of packed layout-0 weights: 16-byte chunk (tile j,
// K-step s, lane l) of the output at ((j KS + s) 64 + l) 16 is chunk
// 4 s + (l >> 4) of row 16 j + (l & 15) of the packed rows (zero past the
// last row).
__global__ __launch_bounds__(256) void k_pack_fragments(
    const int8_t* __restrict__ src, int64_t rows, int64_t kgp,
    int8_t* __restrict__ dst, int64_t chunks) {
    const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (q >= chunks) return;
    const int64_t ks = kgp >> 2;
    const int l = (int)(q & 63);
    const int64_t js = q >> 6, j = js / ks, s = js - j * ks;
    const int64_t row = 16 * j + (l & 15);
    v4i v = v4i{0, 0, 0, 0};
    if (row < rows)
        v = *(const v4i*)(src + (row * kgp + 4 * s + (l >> 4)) * 16);
    *(v4i*)(dst + q * 16) = v;
}

// The instantiated K-step pairs (first, second), with 2 and 3 channel
// tiles a wave at most (256 first-convolution channels, 384 second ones a
// work-group).
template <int KS1>
PpKern pp_kernel2(int ks2) {
    switch (ks2) {
        case 1: return &k_conv_pw_pool<KS1, 2, 1, 3>;
        case 2: return &k_conv_pw_pool<KS1, 2, 2, 3>;
        case 4: return &k_conv_pw_pool<KS1, 2, 4, 3>;
        default: return nullptr;
    }
}

PpKern pp_kernel(int ks1, int ks2) {
    switch (ks1) {
        case 1: return pp_kernel2<1>(ks2);
        case 2: return pp_kernel2<2>(ks2);
        case 4: return pp_kernel2<4>(ks2);
        case 6: return pp_kernel2<6>(ks2);
        case 8: return pp_kernel2<8>(ks2);
        default: return nullptr;
    }
}

bool pointwise(const ConvArgs& b) {
    return b.G == 1 && b.layout == 0 && b.KH == 1 && b.KW == 1 &&
           b.SH == 1 && b.SW == 1 && b.PH == 0 && b.PW == 0 &&
           b.OH == b.H && b.OW == b.W && b.plan && b.mode == EPI_QUANT &&
           b.y_code == 1 && !b.res && !b.y2 && b.rowsum == 0 &&
           b.x_code == 1 && b.x_sc == 1 && b.Cg % 16 == 0 &&
           b.KGp % 4 == 0 && b.Cout % 16 == 0 && b.gate == nullptr;
}

// Geometry of a pair the kernel takes (lds 0: it does not).
PwPoolGeom pp_geom(const ConvArgs& b1, const ConvArgs& b2, int cblk) {
    PwPoolGeom g{};
    g.P = b1.OH * b1.OW;
    g.RS1 = b1.KGp + 1;
    g.RS2 = b2.KGp + 1;
    g.cblk = cblk;
    g.nt1 = b1.Cout / 16;
    g.cr1 = b1.Cg / 16;
    const bool ok =
        pointwise(b1) && pointwise(b2) && b2.x == b1.y &&
        b2.Cg == b1.Cout && b2.N == b1.N && b2.H == b1.OH &&
        b2.W == b1.OW && g.P >= 1 && g.P <= PP_PMAX &&
        g.P * g.cr1 <= PP_XU * PP_NT && g.nt1 <= 2 * PP_NW &&
        cblk % 16 == 0 && cblk <= 3 * 16 * PP_NW && cblk >= 16 &&
        (uintptr_t)b1.x % 16 == 0 && b1.x_sp % 16 == 0 &&
        b1.x_sn % 16 == 0 && (int64_t)g.P * b1.x_sp < ((int64_t)1 << 31) &&
        b1.N <= 65535 && pp_kernel(b1.KGp / 4, b2.KGp / 4) != nullptr;
    const int64_t lds = (int64_t)g.P * g.RS1 * 16 + PP_PMAX * g.RS2 * 16;
    g.lds = ok && lds <= 96 * 1024 ? (int)lds : 0;
    return g;
}

// Channels of the second convolution per work-group: 320 for the 1280 of a
// classifier head (4 blocks, one work-group per image and block fills the
// CUs at batch 64), else the largest multiple of 16 up to 384 dividing
// Cout into about 4 blocks.
int pp_cblk(const ConvArgs& b2) {
    const int tiles = b2.Cout / 16;
    const int per = std::min(3 * PP_NW, (tiles + 3) / 4);
    return 16 * std::max(per, 1);
}

}  // namespace

bool conv_pw_pool_applies(const ConvArgs& b1, const ConvArgs& b2) {
    return pp_geom(b1, b2, pp_cblk(b2)).lds > 0;
}

int64_t fragments_bytes(int64_t rows, int64_t kgp) {
    return ceil_div(rows, 16) * (kgp / 4) * 1024;
}

bool launch_pack_fragments(const int8_t* src, int64_t rows, int64_t kgp,
                           int8_t* dst, hipStream_t st) {
    const int64_t chunks = fragments_bytes(rows, kgp) / 16;
    if (chunks == 0) return true;
    if (ceil_div(chunks, 256) >= ((int64_t)1 << 31)) {
        set_error("qa_d_pack_fragments_i8", "weights too large");
        return false;
    }
    hipLaunchKernelGGL(k_pack_fragments, dim3((unsigned)ceil_div(chunks, 256)),
                       dim3(256), 0, st, src, rows, kgp, dst, chunks);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_hip_error("qa_d_pack_fragments_i8", e);
        return false;
    }
    return true;
}

bool launch_conv_pw_pool(const ConvArgs& b1, const ConvArgs& b2,
                         const PoolArgs& pl, hipStream_t st) {
    const int cblk = pp_cblk(b2);
    const PwPoolGeom g = pp_geom(b1, b2, cblk);
    const PpKern k = pp_kernel(b1.KGp / 4, b2.KGp / 4);
    if (g.lds == 0 || !k || !pl.out || !b1.wfrag || !b2.wfrag) {
        set_error("launch_conv_pw_pool", "convolutions outside the kernel's "
                                         "scope, or weights not in fragment "
                                         "order");
        return false;
    }
    const dim3 grid((unsigned)b1.N, (unsigned)ceil_div(b2.Cout, cblk));
    hipLaunchKernelGGL(k, grid, dim3(PP_NT), (size_t)g.lds, st, b1, b2, pl, g,
                       b1.wfrag, b2.wfrag);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_hip_error("launch_conv_pw_pool", e);
        return false;
    }
    return true;
}

}  // namespace qa

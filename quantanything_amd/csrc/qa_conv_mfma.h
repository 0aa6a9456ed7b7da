// int8 MFMA convolution / GEMM kernel templates (data layout: qa_conv.h).
// Included by the two translation units that instantiate them (weights
// staged in LDS / read from L2), so that the builds run in parallel.
//
// Persistent tiles. A tile is 16 consecutive output pixels (batch folded
// in) times the WM*16 output channels of the work-group's channel block
// (the grid's y after xcd_block). Each wave64 walks its own sequence of tiles (tile, tile +
// stride, ...); with KSPLIT the 4 waves of a work-group share each tile and
// split its K-steps. Fragments come straight from global memory into
// registers (16 contiguous bytes per lane) through a ring of D K-steps that
// runs across tile boundaries, so the loads of the next tile are in flight
// while the current tile's MFMAs and epilogue execute; there is no barrier
// in the main loop (KSPLIT: two per tile, for the reduction).
//
// Everything the epilogue needs besides the accumulators is ready before
// the loop: the tables and the block's per-channel records sit in LDS, and
// the residual words of the next tile are fetched one tile ahead.
//
// Epilogue variants (template EPI):
//   EPI_RAW32 / EPI_RAW64  accumulators for the reference ABI,
//   Q8_TABLE  int8 output through a host-built plan (qa_conv.h): one int64
//             multiply-add and shift per element, then 256-entry LDS tables
//             for clip, activation table, residual Add and rescaled copy;
//             4 consecutive channels of a pixel are stored as one word,
//   Q8_GENERAL the 128-bit form for any parameters.
#pragma once

#include <map>
#include <mutex>
#include <tuple>
#include <type_traits>

#include "qa_conv.h"

namespace qa {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int Q8_TABLE = 3;
constexpr int Q8_GENERAL = 4;

// Output pixel of one lane, walked through the tiles by a constant stride
// (st_dn, st_doy, st_dox) with one carry per coordinate instead of a
// division per tile.
struct PixPos {
    int n, oy, ox;
};

__device__ __forceinline__ PixPos pix_decode(const ConvArgs& a, int64_t p) {
    const uint32_t pp = (uint32_t)p;  // < 2^31
    const uint32_t ohw = (uint32_t)(a.OH * a.OW);
    PixPos q;
    q.n = (int)(pp / ohw);
    const uint32_t pix = pp - (uint32_t)q.n * ohw;
    q.oy = (int)(pix / (uint32_t)a.OW);
    q.ox = (int)pix - q.oy * a.OW;
    return q;
}

__device__ __forceinline__ void pix_step(const ConvArgs& a, PixPos& q) {
    q.ox += a.st_dox;
    const int cx = q.ox >= a.OW;
    q.ox -= cx ? a.OW : 0;
    q.oy += a.st_doy + cx;
    const int cy = q.oy >= a.OH;
    q.oy -= cy ? a.OH : 0;
    q.n += a.st_dn + cy;
}

// Fetch side of one lane's pixel: image base (+ group channel offset) and
// the top-left input coordinate of its receptive field.
struct FetchPix {
    const int8_t* base;  // image base (+ group channel offset)
    const int8_t* org;   // base + offset of input position (iy0, ix0)
    int iy0, ix0;
};

__device__ __forceinline__ FetchPix fetch_pix(const ConvArgs& a, PixPos q,
                                              int g) {
    FetchPix f;
    const int n = q.n < a.N ? q.n : 0;  // past the end: read image 0
    f.iy0 = q.oy * a.SH - a.PH;
    f.ix0 = q.ox * a.SW - a.PW;
    f.base = (const int8_t*)a.x + (int64_t)n * a.x_sn + (int64_t)g * a.Cg;
    f.org = f.base + ((int64_t)f.iy0 * a.W + f.ix0) * a.x_sp;
    return f;
}

// floor(n / d) for n < 2^16 with m = ceil(2^32 / d) (d < 2^16): the error
// of m*d - 2^32 < d stays below one step for such n.
__device__ __forceinline__ int div_magic(int n, uint64_t m) {
    return (int)(((uint64_t)(uint32_t)n * m) >> 32);
}

__device__ __forceinline__ int splat4(int b) {
    return (int)((uint32_t)(uint8_t)b * 0x01010101u);
}

// The work-group's (x, y, z) block after an XCD-aware reordering of the
// grid. Work-groups are dealt to the 8 XCDs (each with its own L2)
// round-robin in flattened-id order, x fastest: work-group f runs on XCD
// f % 8 as that XCD's (f / 8)-th. XCD i takes the i-th contiguous range of
// a linear order of the grid (XCD i holds q + (i < r) work-groups for
// q = total / 8, r = total % 8) in which y varies fastest (yfast: the
// channel blocks of one pixel block, which read the same activations, run
// on one XCD) or x does (the pixel blocks of one channel block, which read
// the same weights). Wave-uniform scalar arithmetic, once per work-group.
struct XcdBlock {
    uint32_t x, y, z;
};
__device__ __forceinline__ XcdBlock xcd_block(bool yfast) {
    const uint32_t gx = gridDim.x, gy = gridDim.y;
    const uint32_t gxy = gx * gy, total = gxy * gridDim.z;
    const uint32_t f = (blockIdx.z * gy + blockIdx.y) * gx + blockIdx.x;
    const uint32_t xcd = f & 7, q = total >> 3, r = total & 7;
    const uint32_t lid = xcd * q + min(xcd, r) + (f >> 3);
    const uint32_t z = lid / gxy, rem = lid - z * gxy;
    XcdBlock b;
    b.z = z;
    if (yfast) {
        b.x = rem / gy;
        b.y = rem - b.x * gy;
    } else {
        b.y = rem / gx;
        b.x = rem - b.y * gx;
    }
    return b;
}

// sum of the first nreal signed bytes of v (nreal in 0..16)
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

// sum of the real bytes of a layout-1 fragment; nreal = bytes per word
// (the channels) | real words << 8: the first bytes of the first words
__device__ __forceinline__ int bytes_sum_l1(v4i v, int nreal) {
    const int nb = nreal & 0xff, nw = nreal >> 8;
    const int mask = nb >= 4 ? 0x01010101
                             : (int)((1u << (8 * nb)) - 1) & 0x01010101;
    int s = 0;
#pragma unroll
    for (int w = 0; w < 4; ++w)
        if (w < nw) s = __builtin_amdgcn_sdot4(v[w], mask, s, false);
    return s;
}


// Where k-group kg of one lane reads (layout 0: tap kg / CB, channel block
// kg % CB; layout 1: kernel row kg / CB, kernel columns 4 (kg % CB) ..
// + 3): input offsets (dy, dx) from the pixel's receptive-field origin and
// the byte offset of that position.
struct KTap {
    int dy, dx;
    int64_t off;
    int nreal;  // real bytes: layout 0 of the 16; layout 1: of each word,
                // | real words (kernel columns) << 8
};

// Tap table entry of k-group kg (layout 0), built in LDS by each
// work-group: the K loop reads one entry a step instead of decoding the
// tap with divisions.
struct KTabE {
    int64_t off;   // byte offset from the receptive-field origin
    int32_t dydx;  // dy | dx << 16
    int32_t nreal;
};

template <int LAYOUT>
__device__ __forceinline__ KTap ktap(const ConvArgs& a, int kg) {
    KTap t;
    if (LAYOUT == 0) {
        const int tap = div_magic(kg, a.mg_cb);
        const int cb = kg - tap * a.CB;
        const int ky = div_magic(tap, a.mg_kw);
        const int kx = tap - ky * a.KW;
        t.dy = ky * a.DH;
        t.dx = kx * a.DW;
        t.off = ((int64_t)t.dy * a.W + t.dx) * a.x_sp + cb * 16;
        t.nreal = kg < a.KG ? min(16, a.Cg - cb * 16) : 0;
    } else {
        int ky = kg, part = 0;
        if (a.CB > 1) {  // kernels wider than 4 columns
            ky = kg / a.CB;
            part = kg - ky * a.CB;
        }
        t.dy = ky * a.DH;
        t.dx = 4 * part * a.DW;
        t.off = ((int64_t)t.dy * a.W + t.dx) * a.x_sp;
        t.nreal = kg < a.KG ? (a.Cg | min(4, a.KW - 4 * part) << 8) : 0;
    }
    return t;
}

// B fragment of one pixel, loaded from an address that is always inside
// the input (image padding and pixels past the end read the image origin);
// *pad receives the lanes that must read pad_value instead (layout 0: a
// flag; layout 1: one bit per kx word), applied when the fragment is used.
template <int LAYOUT>
__device__ __forceinline__ v4i load_b(const ConvArgs& a, const FetchPix& P,
                                      const KTap& t, int* pad) {
    const int iy = P.iy0 + t.dy;
    const bool row_ok = (unsigned)iy < (unsigned)a.H;
    if (LAYOUT == 0) {
        const int ix = P.ix0 + t.dx;
        const bool in = row_ok && (unsigned)ix < (unsigned)a.W;
        *pad = !in;
        return *(const v4i*)(in ? P.org + t.off : P.base);
    }
    v4i v;
    int m = 0;
    const int nw = t.nreal >> 8;  // words inside the kernel
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int ix = P.ix0 + t.dx + k * a.DW;
        const bool in =
            row_ok && (unsigned)ix < (unsigned)a.W && k < nw;
        if (!in) m |= 1 << k;
        v[k] = *(const int*)(in ? P.org + t.off + (int64_t)k * a.DW * a.x_sp
                                : P.base);
    }
    *pad = m;
    return v;
}

// The fragment as the MFMA consumes it: pad_value where the image is padded.
template <int LAYOUT>
__device__ __forceinline__ v4i apply_pad(v4i v, int pad, int pv) {
    if (LAYOUT == 0) {
        if (pad) v = v4i{pv, pv, pv, pv};
        return v;
    }
#pragma unroll
    for (int k = 0; k < 4; ++k)
        if (pad & (1 << k)) v[k] = pv;
    return v;
}

// The 128-bit epilogue of one accumulator (Q8_GENERAL).
__device__ __forceinline__ int64_t quant_general(const ConvArgs& a,
                                                 int64_t v, int64_t m,
                                                 int64_t shift, int64_t res_q) {
    int64_t q = qa_clip128(qa_mbqm(v, m, shift) + a.zp, a.qmin, a.qmax);
    if (a.lut) {
        int64_t idx = q - a.lut_off;
        idx = idx < 0 ? 0 : (idx >= a.lut_len ? a.lut_len - 1 : idx);
        q = a.lut[idx];
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

// med3(x, lo, hi) = clip(x, lo, hi) for lo <= hi, as one VALU instruction
// (the compiler otherwise emits a max and a min).
__device__ __forceinline__ int med3_i32(int x, int lo, int hi) {
    int r;
    asm("v_med3_i32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "v"(lo), "v"(hi));
    return r;
}

// q0 = (w*m + c) >> t for a table-plan constant c that has the channel's
// correction term folded in: c = c_plan + corr*m (mod 2^64). w is the raw
// MFMA sum and w + corr the corrected int32 accumulator, exact when
// |w| + |corr| < 2^31 (8-bit operands, K < 2^16); the sum w*m + c equals
// (w + corr)*m + c_plan, which the planner keeps within int64, so the
// modular arithmetic gives it exactly.
__device__ __forceinline__ int plan_q0(int w, int m, int64_t c, int t) {
    return (int)((int64_t)((uint64_t)((int64_t)w * m) + (uint64_t)c) >> t);
}

// The table-plan constant with the correction term folded in (see plan_q0).
__device__ __forceinline__ int64_t plan_fold(int64_t c, uint32_t corr, int m) {
    return (int64_t)((uint64_t)c + (uint64_t)((int64_t)(int)corr * m));
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


// One output element on the general path: the ABI results (raw int32 /
// int64 sums in any layout) and the 128-bit requantization for parameters
// or layouts outside the table epilogue (rare: its loops stay rolled).
template <int EPI>
__device__ __forceinline__ void store_general(
    const ConvArgs& a, int accv, int64_t p, int64_t co,
    int rs) {
    const PixPos op = pix_decode(a, p);
    const int64_t pixo = op.oy * a.OW + op.ox;
    const int64_t corr = a.corr ? a.corr[co] : 0;
    const int64_t bo = a.rowsum ? a.boff[co] : 0;
    const int64_t o = (int64_t)op.n * a.y_sn + pixo * a.y_sp + co * a.y_sc;
    if (EPI == EPI_RAW64) {
        ((int64_t*)a.y)[o] = (int64_t)accv + corr + bo * rs;
        return;
    }
    const int32_t w = (int32_t)((uint32_t)accv + (uint32_t)corr +
                                (uint32_t)bo * (uint32_t)rs);
    if (EPI == EPI_RAW32) {
        ((int32_t*)a.y)[o] = w;
        return;
    }
    int64_t rq = 0;
    if (a.res)
        rq = (int64_t)((const int8_t*)a.res)[(int64_t)op.n * a.res_sn +
                                             pixo * a.res_sp + co * a.res_sc] +
             a.res_so;
    // the reference adds the bias to the int32 sum
    const int64_t qv = quant_general(a, (int64_t)w + (a.pre ? a.pre[co] : 0),
                                     a.mult[co], a.shift[co], rq);
    ((int8_t*)a.y)[o] = (int8_t)(qv - a.y_so);
    if (a.y2)
        ((int8_t*)a.y2)[(int64_t)op.n * a.y2_sn + pixo * a.y2_sp +
                        co * a.y2_sc] = (int8_t)(rescale2(a, qv) - a.y_so);
}

// 4x4 byte transpose across the 4 lanes of a quad (q = lane & 3): lane q
// holds bytes (x[q][0], .., x[q][3]) and ends with (x[0][q], .., x[3][q]).
// s1/s2 are the lane's byte selectors (quad_selectors).
__device__ __forceinline__ uint32_t quad_transpose(uint32_t w, uint32_t s1,
                                                   uint32_t s2) {
    // partner lane q ^ 2 (quad_perm 2,3,0,1), then q ^ 1 (1,0,3,2)
    uint32_t p = (uint32_t)__builtin_amdgcn_mov_dpp((int)w, 0x4E, 0xF, 0xF,
                                                    true);
    const uint32_t t = __builtin_amdgcn_perm(p, w, s1);
    p = (uint32_t)__builtin_amdgcn_mov_dpp((int)t, 0xB1, 0xF, 0xF, true);
    return __builtin_amdgcn_perm(p, t, s2);
}

// Waves per SIMD the register allocation must allow (occupancy target).
template <int WM>
constexpr int waves_per_simd() {
    return WM >= 8 ? 2 : 3;
}

// Weight chunks (16 bytes) a work-group can stage in LDS: 48 KB.
constexpr int ALDS_CHUNKS = 3072;

// K-steps in flight per wave (ring of fragment registers), within the
// register budget of the tile: 8 when the ring holds only the activation
// fragments (weights in LDS), fewer when it also holds WM weight fragments.
template <int WM, bool ALDS>
constexpr int ring_depth() {
    return ALDS ? 8 : (WM <= 1 ? 8 : (WM <= 2 ? 4 : (WM <= 4 ? 3 : 2)));
}

// ALDS: the work-group's weight rows (WM*16 rows of KGp*16 bytes, row
// stride KGp*16 + 16 so that 16-byte reads of 16 consecutive rows hit
// distinct banks) are copied to LDS once and read from there; otherwise
// every wave reads them from global memory (L2) each K-step.
template <int WM, int LAYOUT, int EPI, bool KSPLIT, bool ALDS>
__global__ __launch_bounds__(256)
__attribute__((amdgpu_waves_per_eu(waves_per_simd<WM>(), 8))) void k_conv_mfma(
    ConvArgs a) {
    // a path chosen on the device (work-group-uniform, before any barrier)
    if (a.gate != nullptr && *a.gate != a.gate_on) return;
    constexpr bool QUANT = EPI == Q8_TABLE || EPI == Q8_GENERAL;
    constexpr bool TABLE = EPI == Q8_TABLE;
    constexpr int KSTRIDE = KSPLIT ? 4 : 1;
    constexpr int D = ring_depth<WM, ALDS>();
    extern __shared__ v4i s_w[];  // ALDS weights, 16-byte units
    // Q8_TABLE: E, TC, TR of the plan
    __shared__ int s_tab[TABLE ? 768 : 1];
    __shared__ int s_red[KSPLIT ? 3 * (WM * 4 + 1) * 64 : 1];
    const int lane = threadIdx.x & 63;
    // wave index in a scalar register: the tile walk below is wave-uniform
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // (pixel block, channel block, group) of the work-group
    const XcdBlock blk = xcd_block(a.xcd_yfast != 0);
    const int g = (int)blk.z;
    const int kgl = lane >> 4;
    const int col = lane & 15;
    const int co0 = (int)blk.y * (WM * 16);
    const bool res = TABLE && a.res != nullptr;
    // the epilogue tables first: their loads overlap everything below
    const int ntab = res ? 768 : 256;
    int tabv[TABLE ? 3 : 1];
    if (TABLE) {
        const int* tab = (const int*)((const char*)a.plan + PLAN_E);
#pragma unroll
        for (int j = 0; j < 3; ++j) {
            const int i = threadIdx.x + 256 * j;
            tabv[j] = i < ntab ? tab[i] : 0;
        }
    }

    // Tiles of 16 consecutive output pixels; the pixel blocks that run on
    // one XCD form contiguous ranges (xcd_block). A wave's tiles are tile,
    // tile + tstride, ...
    const uint32_t nb = gridDim.x;
    const uint32_t bx = blk.x;
    const int64_t ntiles = (a.M + 15) >> 4;
    const int64_t tstride = KSPLIT ? (int64_t)nb : (int64_t)nb * 4;
    int64_t tile = KSPLIT ? (int64_t)bx : (int64_t)bx * 4 + wave;
    const bool has_tile = tile < ntiles;  // uniform within a KSPLIT group

    const int KS = a.KGp >> 2;                   // K-steps of 64 bytes
    const int L = KSPLIT ? (KS + 3) >> 2 : KS;   // steps per wave and tile
    const int st0 = KSPLIT ? wave : 0;

    const int8_t* wrow = a.wp + (int64_t)g * a.wp_gstride +
                         (int64_t)(co0 + col) * a.wp_rstride + kgl * 16;
    const int64_t wstep = 16 * a.wp_rstride;  // next 16 rows

    // ---- fetch side: (ftile, fi) is the next K-step to load; the stream
    // of (tile, step) runs through the D ring slots without gaps ----
    int64_t ftile = tile;
    int fi = 0;
    PixPos fpos = pix_decode(a, tile * 16 + col);
    FetchPix fp = fetch_pix(a, fpos, g);
    constexpr int AS = ALDS ? 1 : D;  // ring slots holding weights
    v4i af[AS][WM], bf[D];
    int pd[D];  // pad flags of the slot's activation fragment
    int nr[D];  // real bytes of the slot's activation fragment (row sums)
    // layout 0: the work-group's tap table (after its ALDS weights)
    KTabE* s_kt = (KTabE*)(s_w + (ALDS ? WM * 16 * (a.KGp + 1) : 0));
    // tab: the table is ready (after the first barrier)
    auto fetch = [&](auto tab, v4i* fa, v4i& fb, int& pds, int& nrs)
                     __attribute__((always_inline)) {
        const int step = st0 + fi * KSTRIDE;
        if (ftile < ntiles && step < KS) {
            KTap t;
            if (decltype(tab)::value && LAYOUT == 0) {
                const KTabE e = s_kt[4 * step + kgl];
                t.off = e.off;
                t.dy = e.dydx & 0xffff;
                t.dx = e.dydx >> 16;
                t.nreal = e.nreal;
            } else {
                t = ktap<LAYOUT>(a, 4 * step + kgl);
            }
            if (!ALDS) {
#pragma unroll
                for (int i = 0; i < WM; ++i)
                    fa[i] = *(const v4i*)(wrow + i * wstep + step * 64);
            }
            fb = load_b<LAYOUT>(a, fp, t, &pds);
            nrs = t.nreal;
        }
        if (ftile < ntiles) {
            if (++fi == L) {
                fi = 0;
                ftile += tstride;
                pix_step(a, fpos);
                fp = fetch_pix(a, fpos, g);
            }
        }
    };
    // plan header: clip bounds of the requantized value, residual range
    int pA = 0, pB = 0, pSH = 0;
    if (TABLE) {
        const int4 h = *(const int4*)a.plan;
        pA = h.x;
        pB = h.y;
        pSH = h.z;
    }
    // ---- the block's per-channel constants, loaded once per work-group
    // (thread t < WM*16: channel co0 + t) and read from LDS after the
    // barrier into the lane's registers (channels co0 + i*16 + col)
    __shared__ int4 s_pc[TABLE ? WM * 16 : 1];
    __shared__ uint2 s_cb[TABLE ? WM * 16 : 1];
    int4 cst_pc = int4{0, 0, 0, 0};
    uint2 cst_cb = uint2{0u, 0u};
    if (TABLE && threadIdx.x < WM * 16) {
        const int c = min(co0 + (int)threadIdx.x, a.Cog - 1);
        const int64_t co = (int64_t)g * a.Cog + c;
        cst_pc = ((const int4*)((const char*)a.plan + PLAN_CH))[co];
        cst_cb.x = a.corr ? (uint32_t)a.corr[co] : 0u;
        cst_cb.y = a.rowsum ? (uint32_t)a.boff[co] : 0u;
    }
    int cm[TABLE ? WM : 1], ct[TABLE ? WM : 1];
    int64_t cc[TABLE ? WM : 1];
    uint32_t ccorr[TABLE ? WM : 1], cbo[TABLE ? WM : 1];
    const int q = lane & 3;  // lane within its quad
    const uint32_t sel1 = q < 2 ? 0x05040100u : 0x03020706u;
    const uint32_t sel2 = (q & 1) ? 0x03070105u : 0x06020400u;
    // channel-quad of this lane: channels co0 + i*16 + (col & ~3) .. +3
    const int cq = col & ~3;

    // ---- residual words, one tile ahead (fast layout): lane q loads the 4
    // channels of pixel 4*kgl + q of its channel quad, transposed on use
    const bool res_wave = res && (!KSPLIT || wave == 0);
    constexpr int RM = TABLE ? WM : 1;
    uint32_t rwn[RM], rwc[RM];
    auto load_res = [&](int64_t t) __attribute__((always_inline)) {
        const int64_t p = t * 16 + 4 * kgl + q;
        const bool ok = p < a.M;
#pragma unroll
        for (int i = 0; i < RM; ++i) {
            const int c0 = co0 + i * 16 + cq;
            uint32_t w = 0;
            if (ok && a.fastio) {
                const int64_t rb = p * a.res_pst + (int64_t)g * a.Cog + c0;
                if (c0 + 3 < a.Cog) {
                    w = *(const uint32_t*)((const int8_t*)a.res + rb);
                } else {
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (c0 + r < a.Cog)
                            w |= (uint32_t)((const uint8_t*)a.res)[rb + r]
                                 << (8 * r);
                }
            }
            rwn[i] = w;
        }
    };
    if (res_wave && has_tile) {
        load_res(tile);
#pragma unroll
        for (int i = 0; i < RM; ++i) rwc[i] = rwn[i];
        if (tile + tstride < ntiles) load_res(tile + tstride);
    }

    // weight rows of the channel block, bound for LDS: loaded here (all in
    // flight with the ring's first loads), stored after them
    const int RS = a.KGp + 1;  // LDS row stride (16-byte units)
    constexpr int MAXC = ALDS ? ALDS_CHUNKS / 256 : 1;
    v4i wtmp[MAXC];
    const int nchunk = WM * 16 * a.KGp;
    if (ALDS) {
        const int8_t* wsrc = a.wp + (int64_t)g * a.wp_gstride +
                             (int64_t)co0 * a.wp_rstride;
#pragma unroll
        for (int k = 0; k < MAXC; ++k) {
            const int c = threadIdx.x + 256 * k;
            if (c < nchunk) {
                const int row = c / a.KGp, kc = c - row * a.KGp;
                wtmp[k] = *(const v4i*)(wsrc + (int64_t)row * a.wp_rstride +
                                        kc * 16);
            }
        }
    }
    // first loads of the ring (in flight with the weight and table loads)
    if (has_tile) {
#pragma unroll
        for (int s = 0; s < D; ++s)
            fetch(std::false_type(), af[ALDS ? 0 : s], bf[s], pd[s], nr[s]);
    }
    if (LAYOUT == 0) {  // the tap table, read after the barrier
        for (int kg = threadIdx.x; kg < a.KGp; kg += 256) {
            const KTap t = ktap<0>(a, kg);
            KTabE e;
            e.off = t.off;
            e.dydx = t.dy | (t.dx << 16);
            e.nreal = t.nreal;
            s_kt[kg] = e;
        }
    }
    if (ALDS) {
#pragma unroll
        for (int k = 0; k < MAXC; ++k) {
            const int c = threadIdx.x + 256 * k;
            if (c < nchunk) {
                const int row = c / a.KGp, kc = c - row * a.KGp;
                s_w[row * RS + kc] = wtmp[k];
            }
        }
    }
    if (TABLE) {
#pragma unroll
        for (int j = 0; j < 3; ++j) {
            const int i = threadIdx.x + 256 * j;
            if (i < ntab) s_tab[i] = tabv[j];
        }
        if (threadIdx.x < WM * 16) {
            s_pc[threadIdx.x] = cst_pc;
            s_cb[threadIdx.x] = cst_cb;
        }
    }
    __syncthreads();
    if (TABLE) {
#pragma unroll
        for (int i = 0; i < WM; ++i) {
            const int4 pc = s_pc[i * 16 + col];
            const uint2 cb = s_cb[i * 16 + col];
            cm[i] = pc.x;
            ct[i] = pc.y;
            cc[i] = (int64_t)(((uint64_t)(uint32_t)pc.w << 32) |
                              (uint32_t)pc.z);
            ccorr[i] = cb.x;
            cbo[i] = cb.y;
        }
    }
    if (!has_tile) return;
    const int pv = splat4(a.pad_value);

    v4i acc[WM];
#pragma unroll
    for (int i = 0; i < WM; ++i) acc[i] = v4i{0, 0, 0, 0};
    int psum = 0;

    // Epilogue of the finished tile, then move to the next one. The lane
    // holds, per channel group i, output channel co0 + i*16 + col for the
    // 4 pixels 4*kgl + r of the tile.
    auto finish_tile = [&]() __attribute__((always_inline)) {
        bool store = true;
        if (KSPLIT) {  // sum the 4 waves' partial results into wave 0
            if (wave > 0) {
                int* dst = s_red + (wave - 1) * (WM * 4 + 1) * 64;
#pragma unroll
                for (int i = 0; i < WM; ++i)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        dst[(i * 4 + r) * 64 + lane] = acc[i][r];
                dst[WM * 4 * 64 + lane] = psum;
            }
            __syncthreads();
            if (wave == 0) {
#pragma unroll
                for (int w = 0; w < 3; ++w) {
                    const int* src = s_red + w * (WM * 4 + 1) * 64;
#pragma unroll
                    for (int i = 0; i < WM; ++i)
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            acc[i][r] += src[(i * 4 + r) * 64 + lane];
                    psum += src[WM * 4 * 64 + lane];
                }
            }
            __syncthreads();
            store = wave == 0;
        }
        if (store) {
            // row sums of the lane's 4 pixels (held by lanes 4*kgl + r)
            int ps[4] = {0, 0, 0, 0};
            if (a.rowsum) {
                psum += __shfl_xor(psum, 16);
                psum += __shfl_xor(psum, 32);
#pragma unroll
                for (int r = 0; r < 4; ++r) ps[r] = __shfl(psum, 4 * kgl + r);
            }
            const int64_t p0 = tile * 16 + 4 * kgl;  // first of the 4 pixels
            if (TABLE) {  // launched only with the fast output layout
                const int64_t pq = p0 + q;  // pixel this lane stores
                const bool pok = pq < a.M;
#pragma unroll
                for (int i = 0; i < WM; ++i) {
                    int e[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        // int32 accumulator (wraps like the reference's)
                        uint32_t wu = (uint32_t)acc[i][r] + ccorr[i];
                        if (a.rowsum) wu += cbo[i] * (uint32_t)ps[r];
                        const int q0 = (int)(((int64_t)(int)wu * cm[i] +
                                              cc[i]) >> ct[i]);
                        e[r] = min(max(q0, pA), pB) - pA;
                    }
                    if (res) {
                        const uint32_t rv =
                            quad_transpose(rwc[i], sel1, sel2);
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const int t = s_tab[256 + e[r]] +
                                          s_tab[512 + ((rv >> (8 * r)) & 255)];
                            e[r] = min(max(t, 0), pSH);
                        }
                    }
#pragma unroll
                    for (int r = 0; r < 4; ++r) e[r] = s_tab[e[r]];
                    const int c0 = co0 + i * 16 + cq;
                    const int64_t cofs = (int64_t)g * a.Cog + c0;
                    const uint32_t wy =
                        quad_transpose(pack_entries(e, 0), sel1, sel2);
                    if (pok) {
                        int8_t* py = (int8_t*)a.y + pq * a.y_pst + cofs;
                        if (c0 + 3 < a.Cog) {
                            *(uint32_t*)py = wy;
                        } else {
#pragma unroll
                            for (int r = 0; r < 4; ++r)
                                if (c0 + r < a.Cog) py[r] = (int8_t)(wy >> (8 * r));
                        }
                    }
                    if (a.y2) {
                        const uint32_t w2 =
                            quad_transpose(pack_entries(e, 1), sel1, sel2);
                        if (pok) {
                            int8_t* p2 = (int8_t*)a.y2 + pq * a.y2_pst + cofs;
                            if (c0 + 3 < a.Cog) {
                                *(uint32_t*)p2 = w2;
                            } else {
#pragma unroll
                                for (int r = 0; r < 4; ++r)
                                    if (c0 + r < a.Cog)
                                        p2[r] = (int8_t)(w2 >> (8 * r));
                            }
                        }
                    }
                }
            } else {
                // general layouts: one element at a time
#pragma unroll 1
                for (int r = 0; r < 4; ++r) {
                    const int64_t p = p0 + r;
                    if (p >= a.M) continue;
#pragma unroll 1
                    for (int i = 0; i < WM; ++i) {
                        const int c = co0 + i * 16 + col;
                        if (c < a.Cog)
                            store_general<EPI>(a, acc[i][r], p,
                                               (int64_t)g * a.Cog + c, ps[r]);
                    }
                }
            }
        }
        // next tile
        tile += tstride;
        if (res_wave) {
#pragma unroll
            for (int i = 0; i < RM; ++i) rwc[i] = rwn[i];
            if (tile + tstride < ntiles) load_res(tile + tstride);
        }
#pragma unroll
        for (int i = 0; i < WM; ++i) acc[i] = v4i{0, 0, 0, 0};
        psum = 0;
    };

    // ---- main loop: one ring slot per step; a tile ends at any slot ----
    int ci = 0;  // consumer's step within the tile
    while (true) {
#pragma unroll
        for (int s = 0; s < D; ++s) {
            const int cstep = st0 + ci * KSTRIDE;
            if (cstep < KS) {
                const v4i b = apply_pad<LAYOUT>(bf[s], pd[s], pv);
                // rows = the 16 pixels, columns = 16 output channels
#pragma unroll
                for (int i = 0; i < WM; ++i) {
                    const v4i wf =
                        ALDS ? s_w[(i * 16 + col) * RS + 4 * cstep + kgl]
                             : af[ALDS ? 0 : s][i];
                    acc[i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                        b, wf, acc[i], 0, 0, 0);
                }
                if (a.rowsum)
                    psum += LAYOUT == 0 ? bytes_sum(b, nr[s])
                                        : bytes_sum_l1(b, nr[s]);
            }
            fetch(std::true_type(), af[ALDS ? 0 : s], bf[s], pd[s], nr[s]);
            if (++ci == L) {
                ci = 0;
                finish_tile();
                if (tile >= ntiles) return;
            }
        }
    }
}

// Work-groups of `block` threads of kernel k resident per CU with `lds`
// dynamic LDS bytes on the current device, cached per (kernel, block, lds,
// device): the band launchers ask for every candidate band height at every
// launch.
inline int resident_blocks(const void* k, int block, int lds) {
    static std::mutex mu;
    static std::map<std::tuple<const void*, int, int, int>, int> cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) dev = -1;
    const auto key = std::make_tuple(k, block, lds, dev);
    {
        std::lock_guard<std::mutex> g(mu);
        const auto it = cache.find(key);
        if (it != cache.end()) return it->second;
    }
    int nbk = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nbk, k, block,
                                                     (size_t)lds) !=
            hipSuccess ||
        nbk <= 0)
        nbk = 1;
    std::lock_guard<std::mutex> g(mu);
    cache[key] = nbk;
    return nbk;
}

// Compute units of the current device (cached per device).
int cu_count() {
    static int cus[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cus[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount,
                                  dev) != hipSuccess ||
            n <= 0)
            n = 256;
        cus[dev] = n;
    }
    return cus[dev];
}

// Launches one instantiation with a persistent grid: as many work-groups as
// are resident at once (occupancy of this kernel), at most one per 4 tiles.
// Weight bytes an ALDS work-group stages in LDS.
inline int64_t alds_bytes(int wm, int64_t kgp) { return wm * 16 * (kgp * 16 + 16); }

// LDS per CU of the current device (cached).
int64_t lds_per_cu() {
    static int64_t v = 0;
    if (v == 0) {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(
                &n, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, dev) !=
                hipSuccess ||
            n <= 0)
            n = 65536;
        v = n;
    }
    return v;
}

template <int WM, int LAYOUT, int EPI, bool KSPLIT, bool ALDS>
bool launch_kernel(const ConvArgs& a0, hipStream_t st) {
    auto* kern = &k_conv_mfma<WM, LAYOUT, EPI, KSPLIT, ALDS>;
    static int resident = 0;  // work-groups per CU without dynamic LDS
    static int64_t static_lds = 0;
    if (resident == 0) {
        int nbk = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
                &nbk, (const void*)kern, 256, 0) != hipSuccess ||
            nbk <= 0)
            nbk = 1;
        hipFuncAttributes fa;
        if (hipFuncGetAttributes(&fa, (const void*)kern) == hipSuccess)
            static_lds = (int64_t)fa.sharedSizeBytes;
        resident = nbk;
    }
    const size_t dyn = (ALDS ? (size_t)alds_bytes(WM, a0.KGp) : 0) +
                       (LAYOUT == 0 ? (size_t)a0.KGp * sizeof(KTabE) : 0);
    int res_blocks = resident;
    if (dyn) {  // LDS limit with the staged weights
        const int64_t by_lds = lds_per_cu() / (static_lds + (int64_t)dyn);
        if (by_lds < res_blocks) res_blocks = (int)(by_lds < 1 ? 1 : by_lds);
    }
    const int64_t cblocks = ceil_div(a0.Cog, WM * 16);
    const int64_t ntiles = ceil_div(a0.M, 16);
    const int64_t need = KSPLIT ? ntiles : ceil_div(ntiles, 4);
    int64_t cap = (int64_t)res_blocks * cu_count() / (cblocks * a0.G);
    if (cap < 1) cap = 1;
    const int64_t gx = need < cap ? need : cap;
    // a wave's pixel stride (16 pixels per tile) as (n, oy, ox) offsets
    ConvArgs a = a0;
    const int64_t stride = 16 * gx * (KSPLIT ? 1 : 4);
    const int64_t ohw = (int64_t)a.OH * a.OW;
    a.st_dn = (int32_t)(stride / ohw);
    a.st_doy = (int32_t)((stride % ohw) / a.OW);
    a.st_dox = (int32_t)((stride % ohw) % a.OW);
    // the channel blocks of a pixel block on one XCD when the activations
    // outweigh the weights (each XCD then reads all weights once), else
    // the pixel blocks of a channel block (each XCD reads all activations)
    const int64_t in_bytes = (int64_t)a.N * a.H * a.W * a.Cg * a.G;
    const int64_t w_bytes = (int64_t)a.Cout * a.KGp * 16;
    a.xcd_yfast = in_bytes >= w_bytes ? 1 : 0;
    dim3 grid((unsigned)gx, (unsigned)cblocks, (unsigned)a.G);
    kern<<<grid, 256, dyn, st>>>(a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_hip_error("k_conv_mfma launch", e);
        return false;
    }
    return true;
}

template <int WM, int LAYOUT, bool KSPLIT, bool ALDS>
bool launch_epi(const ConvArgs& a, int epi, hipStream_t st) {
    switch (epi) {
        case EPI_RAW32:
            return launch_kernel<WM, LAYOUT, EPI_RAW32, KSPLIT, ALDS>(a, st);
        case EPI_RAW64:
            return launch_kernel<WM, LAYOUT, EPI_RAW64, KSPLIT, ALDS>(a, st);
        case Q8_TABLE:
            return launch_kernel<WM, LAYOUT, Q8_TABLE, KSPLIT, ALDS>(a, st);
        default:
            return launch_kernel<WM, LAYOUT, Q8_GENERAL, KSPLIT, ALDS>(a, st);
    }
}

template <int LAYOUT, bool KSPLIT, bool ALDS>
bool launch_wm(const ConvArgs& a, int wm, int epi, hipStream_t st) {
    switch (wm) {
        case 1: return launch_epi<1, LAYOUT, KSPLIT, ALDS>(a, epi, st);
        case 2: return launch_epi<2, LAYOUT, KSPLIT, ALDS>(a, epi, st);
        case 4: return launch_epi<4, LAYOUT, KSPLIT, ALDS>(a, epi, st);
        default: return launch_epi<8, LAYOUT, KSPLIT, ALDS>(a, epi, st);
    }
}

template <bool ALDS>
bool launch_variant(const ConvArgs& b, int wm, bool split, int epi,
                    hipStream_t st) {
    if (b.layout == 1) return launch_wm<1, false, ALDS>(b, wm, epi, st);
    return split ? launch_wm<0, true, ALDS>(b, wm, epi, st)
                 : launch_wm<0, false, ALDS>(b, wm, epi, st);
}

}  // namespace
}  // namespace qa

// Graph-input quantization fused into a layout-1 convolution (inputs of at
// most 4 channels, the image stem): float32 NCHW -> int8 -> conv -> int8
// table epilogue in one launch, so the int8 input tensor never goes through
// HBM (it would be written once and read back by the conv).
//
// A work-group owns a band of R output rows of one image. Phase 1 reads the
// band's input rows (R-1)*SH + (KH-1)*DH + 1 of all channels as float4
// (coalesced rows of each plane), quantizes them exactly like
// qa_d_quantize_nhwc (qa_quantize_one_fast) and writes them to LDS as one
// 4-byte word per pixel, channels in bytes 0..C-1 (0 above), with image
// padding pre-filled with the zero point's stored byte on every side, so
// phase 2 needs no bounds checks. Phase 2: the 4 waves take 16-pixel tiles
// of the band in turn; a lane's fragment (pixel col, kernel row kgl) is the
// 4 words at kernel taps kx = 0..3 of its LDS row, the same bytes the
// unfused kernel loads from the int8 tensor, then one MFMA per 16 output
// channels and the table epilogue of k_conv_mfma (Q8_TABLE).
#include "qa_conv_mfma.h"

namespace qa {
namespace {

constexpr int QIN_THREADS = 256;
constexpr int QIN_U = 2;  // input items a thread loads per round

struct QinGeom {
    int R;           // output rows per band
    int IR, RW;      // LDS rows and row width (words) of a band
    int c0;          // LDS column of input column 0 (>= PW; 4-aligned: VEC)
    int bands;       // ceil(OH / R)
    int CBK;         // 16-channel output blocks
    int f32;         // the float32 quantization form applies
    uint64_t mg_ow;  // ceil(2^32 / OW)
    uint64_t mg_pw;  // ceil(2^32 / pad columns per row)
    uint64_t mg_gw;  // ceil(2^32 / items per input row)
    int s64y, s64x;  // 64 output pixels as rows and columns (s64x < OW)
};

// The float32 quantization form (qa_quantize_f32) with the rounding and
// the conversion to an integer done by additions of M = 1.5 * 2^23:
// t = fma(x, invf, M) is M plus the integer nearest to x * invf when
// |x * invf| < 2^22 (the floats in [2^23, 2^24) are the integers there),
// r = t - M is that integer exactly and d = fma(x, invf, -r) the residual
// that qa_quantize_f32 tests (*slow unless |d| < tie; NaN fails the test).
// t + zp clipped to [M + qmin, M + qmax] is the quantized value plus M, an
// integer float in [2^23, 2^24], so its low mantissa byte is the value's
// low two's-complement byte (2^22 is a multiple of 256); the result is
// those float bits. For |x * invf| >= 2^22 the clip gives qmax or qmin
// (qmax - zp and zp - qmin < 2^19, and the additions round monotonically),
// as the exact form does. qa_f32_form_ok bounds qmin, qmax and zp.
struct QinF32 {
    float invf, tie, zpf, lo, hi;
};
constexpr float QIN_M = 12582912.0f;  // 1.5 * 2^23

__device__ __forceinline__ uint32_t quant_bits(float x, const QinF32& k,
                                               bool* slow) {
    const float t = fmaf(x, k.invf, QIN_M);
    const float r = t - QIN_M;
    const float d = fmaf(x, k.invf, -r);
    *slow |= !(fabsf(d) < k.tie);
    return __float_as_uint(__builtin_amdgcn_fmed3f(t + k.zpf, k.lo, k.hi));
}

// Quantized word of one pixel: channel c in byte c (storage offset so
// subtracted), bytes above CIN zero. The float32 form; *slow is set when a
// value is near a rounding tie, NaN, or the scales are outside that form
// (f32 false), and then the word must be recomputed by pixel_word_exact.
template <int CIN>
__device__ __forceinline__ uint32_t pixel_word_f32(const float (&f)[CIN],
                                                   const QinF32& k, bool f32,
                                                   bool* slow) {
    *slow |= !f32;
    uint32_t b[CIN];
#pragma unroll
    for (int c = 0; c < CIN; ++c) b[c] = quant_bits(f[c], k, slow);
    // low bytes gathered (v_perm: selector bytes 0-3 pick the second
    // operand's bytes, 4-7 the first's, 0x0c a zero)
    if (CIN == 1) return b[0] & 0xffu;
    const uint32_t lo2 =
        __builtin_amdgcn_perm(b[CIN > 1 ? 1 : 0], b[0], 0x0c0c0400u);
    if (CIN == 2) return lo2;
    if (CIN == 3) return __builtin_amdgcn_perm(b[2], lo2, 0x0c040100u);
    const uint32_t hi2 = __builtin_amdgcn_perm(b[CIN > 3 ? 3 : 0],
                                               b[CIN > 2 ? 2 : 0], 0x0c0c0400u);
    return __builtin_amdgcn_perm(hi2, lo2, 0x05040100u);
}

// The same word exactly as qa_quantize_one per value (double division).
template <int CIN>
__device__ __forceinline__ uint32_t pixel_word_exact(const float* src, int HW,
                                                  const QinArgs& q) {
    uint32_t w = 0;
    for (int c = 0; c < CIN; ++c)
        w |= (uint32_t)(uint8_t)(qa_quantize_one_fast(src[(int64_t)c * HW],
                                                      q.scale, q.inv, q.zp,
                                                      q.qmin, q.qmax) -
                                 q.so)
             << (8 * c);
    return w;
}

template <int CIN, bool VEC>
__global__ __launch_bounds__(QIN_THREADS) void k_conv_qin(ConvArgs a,
                                                          QinArgs q,
                                                          QinGeom g) {
    extern __shared__ int s_raw[];  // IR x RW words
    __shared__ int s_tab[256];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // consecutive bands of an image on one XCD (blocks are dealt to the 8
    // XCDs round-robin): their halo rows meet in that XCD's L2
    const uint32_t nb = gridDim.x, xcd = blockIdx.x & 7;
    const uint32_t q8 = nb >> 3, r8 = nb & 7;
    const uint32_t bid = xcd * q8 + min(xcd, r8) + (blockIdx.x >> 3);
    const int n = (int)(bid / (uint32_t)g.bands);
    const int band = (int)bid - n * g.bands;
    const int oy0 = band * g.R;
    const int iy_base = oy0 * a.SH - a.PH;
    const int pv = splat4(a.pad_value);

    // ---- phase 1: input rows -> LDS (quantized words, padding filled) --
    for (int i = tid; i < 256; i += QIN_THREADS)
        s_tab[i] = ((const int*)((const char*)a.plan + PLAN_E))[i];
    const int HW = a.H * a.W;
    const float* xn = q.xf + (int64_t)n * CIN * HW;
    QinF32 qk;
    {
        const int so = (int)q.so;
        const int zp = (int)q.zp - so;
        qk.invf = (float)q.inv;
        qk.tie = qa_f32_tie(zp, q.qmin - so, q.qmax - so);
        qk.zpf = (float)zp;
        qk.lo = QIN_M + (float)((int)q.qmin - so);
        qk.hi = QIN_M + (float)((int)q.qmax - so);
    }
    const bool f32 = g.f32;
    constexpr int PX = VEC ? 4 : 1;  // pixels per item
    const int GW = a.W / PX;          // items per input row
    // items (PX pixels of one input row, all CIN planes) i = tid + 256 k:
    // row i / GW, item i % GW; QIN_U items a thread, all their loads in
    // flight before the first quantization (one memory round trip a
    // round)
    const int items = g.IR * GW;
    for (int i0 = tid; i0 < items; i0 += QIN_THREADS * QIN_U) {
        float v[QIN_U][CIN][PX];
        int dsto[QIN_U];
        bool in[QIN_U];
#pragma unroll
        for (int k = 0; k < QIN_U; ++k) {
            const int i = i0 + k * QIN_THREADS;
            const bool ok = i < items;
            const int r = ok ? div_magic(i, g.mg_gw) : 0;
            const int u = ok ? i - r * GW : 0;
            const int iy = iy_base + r;
            in[k] = ok && (unsigned)iy < (unsigned)a.H;
            dsto[k] = ok ? r * g.RW + g.c0 + PX * u : -1;
            const float* src = xn + (in[k] ? iy : 0) * a.W + PX * u;
#pragma unroll
            for (int c = 0; c < CIN; ++c) {
                if (VEC) {
                    const float4 t = *(const float4*)(src + c * HW);
                    v[k][c][0] = t.x;
                    v[k][c][PX > 1 ? 1 : 0] = t.y;
                    v[k][c][PX > 2 ? 2 : 0] = t.z;
                    v[k][c][PX > 3 ? 3 : 0] = t.w;
                } else {
                    v[k][c][0] = src[c * HW];
                }
            }
        }
        uint32_t slowbits = 0;  // bit k * PX + p: recompute exactly
#pragma unroll
        for (int k = 0; k < QIN_U; ++k) {
            if (dsto[k] < 0) continue;
            uint32_t w[PX];
#pragma unroll
            for (int p = 0; p < PX; ++p) {
                float f[CIN];
#pragma unroll
                for (int c = 0; c < CIN; ++c) f[c] = v[k][c][p];
                bool slow = false;
                w[p] = pixel_word_f32<CIN>(f, qk, f32, &slow);
                if (!in[k]) w[p] = (uint32_t)pv;
                if (slow && in[k]) slowbits |= 1u << (k * PX + p);
            }
            int* dst = s_raw + dsto[k];
            if (VEC)
                *(uint4*)dst = make_uint4(w[0], w[PX > 1 ? 1 : 0],
                                          w[PX > 2 ? 2 : 0],
                                          w[PX > 3 ? 3 : 0]);
            else
                *dst = (int)w[0];
        }
        // rare: values near a rounding tie (or scales outside the float32
        // form) take the exact double-division path, one pixel at a time
        while (slowbits) {
            const int b = __builtin_ctz(slowbits);
            slowbits &= slowbits - 1;
            const int k = b / PX, p = b - k * PX;
            const int i = i0 + k * QIN_THREADS;
            const int r = div_magic(i, g.mg_gw), u = i - r * GW;
            const float* src = xn + (iy_base + r) * a.W + PX * u + p;
            s_raw[r * g.RW + g.c0 + PX * u + p] =
                (int)pixel_word_exact<CIN>(src, HW, q);
        }
    }
    {  // pad columns: c0 - PW .. c0 - 1 and c0 + W .. RW - 1
        const int lo = g.c0 - a.PW, PC = g.RW - lo - a.W;
        for (int i = tid; i < g.IR * PC; i += QIN_THREADS) {
            const int r = div_magic(i, g.mg_pw);
            const int k = i - r * PC;
            s_raw[r * g.RW + lo + (k < a.PW ? k : a.W + k)] = pv;
        }
    }
    __syncthreads();

    // ---- phase 2: 16-pixel tiles of the band, one MFMA per 16 channels --
    const int col = lane & 15, kgl = lane >> 4, qd = lane & 3;
    const int Rv = min(g.R, a.OH - oy0);  // valid rows of this band
    const int bpix = Rv * a.OW;
    const int ntile = (bpix + 15) >> 4;
    const int64_t pix0 = ((int64_t)n * a.OH + oy0) * a.OW;  // band's first
    const uint32_t sel1 = qd < 2 ? 0x05040100u : 0x03020706u;
    const uint32_t sel2 = (qd & 1) ? 0x03070105u : 0x06020400u;
    const int cq = col & ~3;
    // k-group kgl is kernel row kgl; past the kernel rows the weights are
    // zero: those lanes read row KH - 1 (any bytes do), left out of the
    // row sums
    const int kbase = min(kgl, a.KH - 1) * a.DH * g.RW + g.c0 - a.PW;
    const int shrw = a.SH * g.RW;
    const int nreal = kgl < a.KH ? (a.Cg | a.KW << 8) : 0;
    const int4 hdr = *(const int4*)a.plan;
    const int* tabE = s_tab - hdr.x;  // tabE[v] = E[v - A] for v in [A, B]
    // LDS word of band pixel p's receptive field (this lane's kernel row);
    // increasing in p, so pixels past the band clamp to the last one's
    auto fbase = [&](int p) {
        const int oyl = div_magic(p, g.mg_ow);
        return __mul24(oyl, shrw) + kbase + __mul24(p - oyl * a.OW, a.SW);
    };
    const int bmax = fbase(bpix - 1);
    // a wave's next tile is 64 pixels on: s64y rows and s64x < OW columns,
    // plus one carry into the next row
    const int dstep = __mul24(g.s64y, shrw) + __mul24(g.s64x, a.SW);
    const int dcarry = shrw - __mul24(a.OW, a.SW);
    int8_t* const yb = (int8_t*)a.y + pix0 * a.y_pst;  // the band's output
    const int ypst = (int)a.y_pst;  // bpix * y_pst < 2^31 (host)
    const bool whole = (a.Cout & 3) == 0;  // every 4-channel word stored
    auto tiles = [&](auto RS) {
        constexpr bool ROWSUM = decltype(RS)::value;
        for (int cb = 0; cb < g.CBK; ++cb) {
            const int co0 = cb * 16;
            const v4i wf = *(const v4i*)(a.wp +
                                         (int64_t)(co0 + col) * a.wp_rstride +
                                         kgl * 16);
            const int c = min(co0 + col, a.Cout - 1);
            const int4 pc = ((const int4*)((const char*)a.plan + PLAN_CH))[c];
            // the correction folded into the plan constant (plan_q0; K is
            // one 64-byte step: |w| + |corr| + |boff * rowsum| < 2^26); kept
            // opaque so that the tile loop is one 32x32->64 multiply-add a
            // value rather than a re-associated 64x64 product
            int64_t cc = plan_fold(
                (int64_t)(((uint64_t)(uint32_t)pc.w << 32) | (uint32_t)pc.z),
                a.corr ? (uint32_t)a.corr[c] : 0u, pc.x);
            asm volatile("" : "+v"(cc));
            const uint32_t cbo = ROWSUM ? (uint32_t)a.boff[c] : 0u;
            // this lane's fetch pixel walks the band 64 pixels a step
            const int fp0 = wave * 16 + col;
            int ox = fp0 - div_magic(fp0, g.mg_ow) * a.OW;
            int base = fbase(fp0);
            for (int t = wave; t < ntile; t += 4) {
                const int bs = min(base, bmax);
                v4i b;
#pragma unroll
                for (int k = 0; k < 4; ++k) b[k] = s_raw[bs + k * a.DW];
                ox += g.s64x;
                base += dstep;
                const bool carry = ox >= a.OW;
                ox -= carry ? a.OW : 0;
                base += carry ? dcarry : 0;
                const v4i acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                    b, wf, v4i{0, 0, 0, 0}, 0, 0, 0);
                int ps[4] = {0, 0, 0, 0};
                if (ROWSUM) {
                    int psum = bytes_sum_l1(b, nreal);
                    psum += __shfl_xor(psum, 16);
                    psum += __shfl_xor(psum, 32);
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        ps[r] = __shfl(psum, 4 * kgl + r);
                }
                int e[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    int w = acc[r];
                    if (ROWSUM) w += (int)(cbo * (uint32_t)ps[r]);
                    e[r] = tabE[med3_i32(plan_q0(w, pc.x, cc, pc.y), hdr.x,
                                         hdr.y)];
                }
                const uint32_t wy =
                    quad_transpose(pack_entries(e, 0), sel1, sel2);
                const int pq = t * 16 + 4 * kgl + qd;  // pixel this lane stores
                const int c0 = co0 + cq;
                if (pq < bpix && c0 < a.Cout) {
                    int8_t* py = yb + (pq * ypst + c0);
                    if (whole || c0 + 3 < a.Cout) {
                        *(uint32_t*)py = wy;
                    } else {
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            if (c0 + r < a.Cout)
                                py[r] = (int8_t)(wy >> (8 * r));
                    }
                }
            }
        }
    };
    if (a.rowsum)
        tiles(std::true_type());
    else
        tiles(std::false_type());
}

uint64_t magic(int d) { return (((uint64_t)1 << 32) + d - 1) / (uint64_t)d; }

}  // namespace

bool launch_conv_qin(const ConvArgs& a0, const QinArgs& q, hipStream_t st) {
    ConvArgs a = a0;
    const int64_t ohw = (int64_t)a.OH * a.OW;
    const bool dense = a.y_sc == 1 && (a.N == 1 || a.y_sn == ohw * a.y_sp) &&
                       a.y_sp % 4 == 0 && (uintptr_t)a.y % 4 == 0;
    if (a.layout != 1 || a.G != 1 || a.KGp != 4 || a.KH < 1 || a.KH > 4 ||
        a.KW < 1 || a.KW > 4 ||
        a.Cg < 1 || a.Cg > 4 || !a.plan || a.mode != EPI_QUANT || a.y_code != 1 ||
        a.res || a.y2 || !dense || a.M >= ((int64_t)1 << 31)) {
        set_error("qa_d_quantize_conv",
                  "needs layout-1 int8 weights (C, KH, KW <= 4, one group), "
                  "an epilogue plan, no residual or second output and a "
                  "dense channels-last int8 output");
        return false;
    }
    a.y_pst = a.y_sp;
    QinGeom g;
    const bool vec = a.W % 4 == 0 && (uintptr_t)q.xf % 16 == 0;
    // LDS row: input columns -PW .. (OW-1)*SW - PW + 3*DW (taps kx <= 3)
    // and the whole image row, column ix at c0 + ix
    g.c0 = vec ? (a.PW + 3) / 4 * 4 : a.PW;
    {
        const int last = std::max(g.c0 - a.PW + (a.OW - 1) * a.SW + 3 * a.DW,
                                  g.c0 + a.W - 1);
        g.RW = (last + 1 + 3) / 4 * 4;
    }
    g.CBK = (a.Cout + 15) / 16;
    // the float32 form on stored values (q - so)
    g.f32 = qa_f32_form_ok(q.scale, q.zp - q.so, q.qmin - q.so, q.qmax - q.so);
    auto in_rows = [&](int R) { return (R - 1) * a.SH + (a.KH - 1) * a.DH + 1; };
    auto lds = [&](int R) { return (int64_t)in_rows(R) * g.RW * 4; };
    int R = 0;
    const int hint = a.tile_hint & TILE_VALID ? (a.tile_hint & 0xffff) : 0;
    if (hint >= 1 && hint <= a.OH && lds(hint) <= 60 * 1024) R = hint;
    if (R == 0) {  // the most rows that still give 4 work-groups per CU
        const int64_t want = 4 * (int64_t)cu_count();
        for (int r : {16, 8, 4, 2, 1}) {
            if (r > a.OH || lds(r) > 32 * 1024) continue;
            R = r;
            if ((int64_t)a.N * ((a.OH + r - 1) / r) >= want) break;
        }
        if (R == 0) R = 1;
    }
    g.R = R;
    g.IR = in_rows(R);
    g.bands = (a.OH + R - 1) / R;
    const int64_t shm = lds(R);
    const int64_t blocks = (int64_t)a.N * g.bands;
    if (shm > 60 * 1024 || (int64_t)R * a.OW >= (1 << 16) ||
        (int64_t)R * a.OW * a.y_pst + a.Cout >= ((int64_t)1 << 31) ||
        (int64_t)g.IR * g.RW >= (1 << 16) || blocks >= ((int64_t)1 << 31)) {
        set_error("qa_d_quantize_conv", "image rows too wide for one band");
        return false;
    }
    g.mg_ow = magic(a.OW);
    g.s64y = 64 / a.OW;
    g.s64x = 64 % a.OW;
    g.mg_pw = magic(std::max(g.RW - (g.c0 - a.PW) - a.W, 1));
    g.mg_gw = magic(std::max(vec ? a.W / 4 : a.W, 1));
    auto go = [&](auto kern) {
        kern<<<(unsigned)blocks, QIN_THREADS, shm, st>>>(a, q, g);
    };
    switch (a.Cg * 2 + (vec ? 1 : 0)) {
        case 2: go(k_conv_qin<1, false>); break;
        case 3: go(k_conv_qin<1, true>); break;
        case 4: go(k_conv_qin<2, false>); break;
        case 5: go(k_conv_qin<2, true>); break;
        case 6: go(k_conv_qin<3, false>); break;
        case 7: go(k_conv_qin<3, true>); break;
        case 8: go(k_conv_qin<4, false>); break;
        default: go(k_conv_qin<4, true>); break;
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_hip_error("qa_d_quantize_conv", e);
        return false;
    }
    return true;
}

}  // namespace qa

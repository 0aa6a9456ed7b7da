// A convolution whose only consumer is a global average pool, fused: the
// int8 table epilogue's output bytes are summed over each image's pixels
// and the pool is requantized in the same launch, so the convolution's
// output (4 MB for the YOLOv8n-cls head at batch 64) is never written and
// the pool needs no launch of its own.
//
// A work-group owns one image and 4*WM*16 output channels, whose weight
// rows it stages in LDS once; each of its 4 waves owns WM*16 of those
// channels and walks all of the image's 16-pixel tiles (fragments from
// HBM/L2 like k_conv_mfma, the next K-step's load in flight, one MFMA per
// 16 channels and K-step), adding the stored bytes of the valid pixels per
// channel, then requantizes its channels' pools,
// q = clip(mbqm(sum + HW*(so - zp_in), mult, shift) + zp_out), as the pool
// kernel does.
#include "qa_conv_mfma.h"

namespace qa {
namespace {

template <int WM>
__global__ __launch_bounds__(256) void k_conv_pool(ConvArgs a, PoolArgs pl) {
    extern __shared__ v4i s_w[];  // 4*WM*16 weight rows, RS units apart
    __shared__ int s_tab[256];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n = blockIdx.x;
    const int cb0 = blockIdx.y * (4 * WM * 16);  // the work-group's channels
    const int co0 = cb0 + wave * WM * 16;        // this wave's
    const int col = lane & 15, kgl = lane >> 4;
    const int P = a.OH * a.OW;
    const int TPI = (P + 15) >> 4;
    const int KS = a.KGp >> 2;
    const int RS = a.KGp + 1;  // LDS row stride (16-byte units)
    const int pv = splat4(a.pad_value);
    // weight rows of the work-group (rows are padded to 128 in the packed
    // layout, so whole blocks are always in bounds) and the table
    {
        const int8_t* src = a.wp + (int64_t)cb0 * a.wp_rstride;
        const int units = 4 * WM * 16 * a.KGp;
        // eight loads in flight per thread before their stores (a loop of
        // load-then-store would wait one memory round trip per unit)
        for (int u0 = threadIdx.x; u0 < units; u0 += 8 * 256) {
            v4i w[8];
            int at[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int u = u0 + j * 256;
                const bool ok = u < units;
                const int row = ok ? u / a.KGp : 0;
                const int kc = ok ? u - row * a.KGp : 0;
                at[j] = ok ? row * RS + kc : -1;
                w[j] = *(const v4i*)(src + (int64_t)row * a.wp_rstride +
                                     kc * 16);
            }
#pragma unroll
            for (int j = 0; j < 8; ++j)
                if (at[j] >= 0) s_w[at[j]] = w[j];
        }
        s_tab[threadIdx.x] = ((const int*)((const char*)a.plan + PLAN_E))[threadIdx.x];
    }
    const int4 hdr = *(const int4*)a.plan;
    // this lane's channels co0 + i*16 + col and their constants
    int cm[WM], ct[WM];
    int64_t cc[WM];
    uint32_t ccorr[WM], cbo[WM];
#pragma unroll
    for (int i = 0; i < WM; ++i) {
        const int c = min(co0 + i * 16 + col, a.Cout - 1);
        const int4 pc = ((const int4*)((const char*)a.plan + PLAN_CH))[c];
        cm[i] = pc.x;
        ct[i] = pc.y;
        cc[i] = (int64_t)(((uint64_t)(uint32_t)pc.w << 32) | (uint32_t)pc.z);
        ccorr[i] = a.corr ? (uint32_t)a.corr[c] : 0u;
        cbo[i] = a.rowsum ? (uint32_t)a.boff[c] : 0u;
    }
    __syncthreads();
    if (co0 >= a.Cout) return;  // a wave past the last channel block
    const v4i* wl = s_w + (wave * WM * 16 + col) * RS + kgl;
    int csum[WM];
#pragma unroll
    for (int i = 0; i < WM; ++i) csum[i] = 0;
    for (int t = 0; t < TPI; ++t) {
        // this lane's pixel (clamped into the image) as a fetch position
        const int p = min(t * 16 + col, P - 1);
        const FetchPix fp = fetch_pix(a, pix_decode(a, (int64_t)n * P + p), 0);
        v4i acc[WM];
#pragma unroll
        for (int i = 0; i < WM; ++i) acc[i] = v4i{0, 0, 0, 0};
        int psum = 0;
        // K-steps with the next one's fragment in flight
        KTap tp = ktap<0>(a, kgl);
        int padn;
        v4i bn = load_b<0>(a, fp, tp, &padn);
        int nrn = tp.nreal;
        for (int ks = 0; ks < KS; ++ks) {
            const v4i b = apply_pad<0>(bn, padn, pv);
            const int nr = nrn;
            if (ks + 1 < KS) {
                tp = ktap<0>(a, 4 * (ks + 1) + kgl);
                bn = load_b<0>(a, fp, tp, &padn);
                nrn = tp.nreal;
            }
#pragma unroll
            for (int i = 0; i < WM; ++i)
                acc[i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                    b, wl[i * 16 * RS + 4 * ks], acc[i], 0, 0, 0);
            if (a.rowsum) psum += bytes_sum(b, nr);
        }
        int ps[4] = {0, 0, 0, 0};
        if (a.rowsum) {
            psum += __shfl_xor(psum, 16);
            psum += __shfl_xor(psum, 32);
#pragma unroll
            for (int r = 0; r < 4; ++r) ps[r] = __shfl(psum, 4 * kgl + r);
        }
        const int p0 = t * 16 + 4 * kgl;  // the lane's 4 pixels p0 + r
#pragma unroll
        for (int i = 0; i < WM; ++i) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                uint32_t wu = (uint32_t)acc[i][r] + ccorr[i];
                if (a.rowsum) wu += cbo[i] * (uint32_t)ps[r];
                const int q0 =
                    (int)(((int64_t)(int)wu * cm[i] + cc[i]) >> ct[i]);
                const int e = s_tab[min(max(q0, hdr.x), hdr.y) - hdr.x];
                if (p0 + r < P) csum[i] += (int)(int8_t)(e & 255);
            }
        }
    }
    // add the 4 lane groups; lanes 0..15 then hold their channels' sums
#pragma unroll
    for (int i = 0; i < WM; ++i) {
        int s = csum[i];
        s += __shfl_xor(s, 16);
        s += __shfl_xor(s, 32);
        const int c = co0 + i * 16 + col;
        if (kgl == 0 && c < a.Cout) {
            const int64_t q =
                qa_clip128(qa_mbqm((int64_t)s + pl.base, pl.mult, pl.shift) +
                               pl.zp,
                           pl.qmin, pl.qmax);
            pl.out[(int64_t)n * pl.out_sn + c] = (int8_t)(q - pl.out_so);
        }
    }
}

// The pointwise form (1x1 kernel, stride 1, no padding, dense channels-last
// input with 16-byte aligned pixels): the work-group stages its image's
// activations (P pixels of KGp*16 bytes, zero past the Cg channels) in LDS
// beside the weight rows, behind the same barrier, so the tile loop reads
// LDS only. The epilogue is the plan form with the zero-point correction
// folded into the 64-bit constant (plan_q0; KGp <= 1024 keeps
// |w| + |corr| + |boff * rowsum| below 2^30, so the int32 sum of the
// general kernel never wraps) and one med3 clip; the table in LDS holds
// the stored bytes sign-extended.
template <int WM, bool ROWSUM>
__global__ __launch_bounds__(256) void k_conv_pool_pw(ConvArgs a,
                                                      PoolArgs pl) {
    extern __shared__ v4i s_w[];  // weight rows, then the image's pixels
    __shared__ int s_tab[256];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n = blockIdx.x;
    const int cb0 = blockIdx.y * (4 * WM * 16);  // the work-group's channels
    const int co0 = cb0 + wave * WM * 16;        // this wave's
    const int col = lane & 15, kgl = lane >> 4;
    const int P = a.OH * a.OW;
    const int TPI = (P + 15) >> 4;
    const int KGp = a.KGp;
    const int KS = KGp >> 2;
    const int RS = KGp + 1;  // LDS row stride of weights and pixels (units)
    v4i* s_x = s_w + 4 * WM * 16 * RS;
    {
        // weight units, then pixel units: eight loads in flight per
        // thread before their stores
        const int8_t* wsrc = a.wp + (int64_t)cb0 * a.wp_rstride;
        const int8_t* xsrc = (const int8_t*)a.x + (int64_t)n * a.x_sn;
        const int wunits = 4 * WM * 16 * KGp;
        const int units = wunits + P * KGp;
        const int creal = a.Cg >> 4;  // 16-byte units of real channels
        for (int u0 = threadIdx.x; u0 < units; u0 += 8 * 256) {
            v4i w[8];
            int at[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int u = u0 + j * 256;
                const bool wt = u < wunits;
                const int v = wt ? u : u - wunits;
                const int row = u < units ? v / KGp : 0;
                const int kc = u < units ? v - row * KGp : 0;
                at[j] = u < units ? (wt ? 0 : 4 * WM * 16 * RS) + row * RS + kc
                                  : -1;
                w[j] = v4i{0, 0, 0, 0};
                if (wt)
                    w[j] = *(const v4i*)(wsrc + (int64_t)row * a.wp_rstride +
                                         kc * 16);
                else if (u < units && kc < creal)
                    w[j] = *(const v4i*)(xsrc + (int64_t)row * a.x_sp + kc * 16);
            }
#pragma unroll
            for (int j = 0; j < 8; ++j)
                if (at[j] >= 0) s_w[at[j]] = w[j];
        }
        s_tab[threadIdx.x] = (int)(int8_t)(
            ((const int*)((const char*)a.plan + PLAN_E))[threadIdx.x] & 255);
    }
    const int4 hdr = *(const int4*)a.plan;
    const int* tabE = s_tab - hdr.x;  // tabE[v] = E[v - A] for v in [A, B]
    // this lane's channels co0 + i*16 + col and their constants
    int cm[WM], ct[WM];
    int64_t cc[WM];
    uint32_t cbo[WM];
#pragma unroll
    for (int i = 0; i < WM; ++i) {
        const int c = min(co0 + i * 16 + col, a.Cout - 1);
        const int4 pc = ((const int4*)((const char*)a.plan + PLAN_CH))[c];
        cm[i] = pc.x;
        ct[i] = pc.y;
        cc[i] = plan_fold(
            (int64_t)(((uint64_t)(uint32_t)pc.w << 32) | (uint32_t)pc.z),
            a.corr ? (uint32_t)a.corr[c] : 0u, pc.x);
        cbo[i] = ROWSUM ? (uint32_t)a.boff[c] : 0u;
    }
    __syncthreads();
    if (co0 >= a.Cout) return;  // a wave past the last channel block
    const v4i* wl = s_w + (wave * WM * 16 + col) * RS + kgl;
    int csum[WM];
#pragma unroll
    for (int i = 0; i < WM; ++i) csum[i] = 0;
    for (int t = 0; t < TPI; ++t) {
        // this lane's pixel, clamped into the image
        const v4i* xr = s_x + min(t * 16 + col, P - 1) * RS + kgl;
        v4i acc[WM];
#pragma unroll
        for (int i = 0; i < WM; ++i) acc[i] = v4i{0, 0, 0, 0};
        int psum = 0;
        for (int ks = 0; ks < KS; ++ks) {
            const v4i b = xr[4 * ks];
#pragma unroll
            for (int i = 0; i < WM; ++i)
                acc[i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                    b, wl[i * 16 * RS + 4 * ks], acc[i], 0, 0, 0);
            if (ROWSUM) psum += bytes_sum(b, 16);  // zero past the channels
        }
        int ps[4] = {0, 0, 0, 0};
        if (ROWSUM) {
            psum += __shfl_xor(psum, 16);
            psum += __shfl_xor(psum, 32);
#pragma unroll
            for (int r = 0; r < 4; ++r) ps[r] = __shfl(psum, 4 * kgl + r);
        }
        const int p0 = t * 16 + 4 * kgl;  // the lane's 4 pixels p0 + r
        const int nv = P - p0;            // of which the first nv are real
#pragma unroll
        for (int i = 0; i < WM; ++i) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                int w = acc[i][r];
                if (ROWSUM) w += (int)(cbo[i] * (uint32_t)ps[r]);
                const int e =
                    tabE[med3_i32(plan_q0(w, cm[i], cc[i], ct[i]), hdr.x,
                                  hdr.y)];
                csum[i] += r < nv ? e : 0;
            }
        }
    }
    // add the 4 lane groups; lanes 0..15 then hold their channels' sums
#pragma unroll
    for (int i = 0; i < WM; ++i) {
        int s = csum[i];
        s += __shfl_xor(s, 16);
        s += __shfl_xor(s, 32);
        const int c = co0 + i * 16 + col;
        if (kgl == 0 && c < a.Cout) {
            const int64_t q =
                qa_clip128(qa_mbqm((int64_t)s + pl.base, pl.mult, pl.shift) +
                               pl.zp,
                           pl.qmin, pl.qmax);
            pl.out[(int64_t)n * pl.out_sn + c] = (int8_t)(q - pl.out_so);
        }
    }
}

}  // namespace

bool launch_conv_pool(const ConvArgs& a0, const PoolArgs& pl, hipStream_t st) {
    ConvArgs a = a0;
    if (a.G != 1 || a.layout != 0 || !a.plan || a.mode != EPI_QUANT ||
        a.y_code != 1 || a.res || a.y2 || !pl.out ||
        a.M >= ((int64_t)1 << 31) || a.N > 65535 || a.KGp >= (1 << 12)) {
        set_error("qa_d_conv_pool",
                  "needs one group, packed layout 0, an epilogue plan, no "
                  "residual or second output, and an int8 pooled output");
        return false;
    }
    a.mg_cb = (((uint64_t)1 << 32) + a.CB - 1) / (uint64_t)a.CB;
    a.mg_kw = (((uint64_t)1 << 32) + a.KW - 1) / (uint64_t)a.KW;
    // a work-group stages 4*wm*16 weight rows; rows are padded to 128 in
    // the packed layout, so wm <= 2 keeps every staged row in bounds
    auto lds = [&](int w) { return (size_t)4 * w * 16 * (a.KGp + 1) * 16; };
    const int wm_max = a.Cout <= 64 ? 1 : 2;
    int wm = 0;
    if (a.tile_hint & TILE_VALID) {
        const int h = a.tile_hint & 0xff;
        if ((h == 1 || h == 2) && h <= wm_max) wm = h;
    }
    if (wm == 0) wm = wm_max;
    while (wm > 1 && lds(wm) > 64 * 1024) wm >>= 1;
    if (lds(wm) > 64 * 1024) {
        set_error("qa_d_conv_pool", "weight rows too long for LDS");
        return false;
    }
    const dim3 grid((unsigned)a.N, (unsigned)ceil_div(a.Cout, 4 * 16 * wm));
    // pointwise: the image's pixels staged too (rows of KGp + 1 units)
    const size_t pw_lds =
        lds(wm) + (size_t)a.OH * a.OW * (a.KGp + 1) * 16;
    const bool pw = a.KH == 1 && a.KW == 1 && a.SH == 1 && a.SW == 1 &&
                    a.PH == 0 && a.PW == 0 && a.OH == a.H && a.OW == a.W &&
                    a.Cg % 16 == 0 && a.x_sc == 1 && a.x_sp % 16 == 0 &&
                    a.x_sn % 16 == 0 && (uintptr_t)a.x % 16 == 0 &&
                    a.x_code == 1 && a.KGp <= 1024 && pw_lds <= 96 * 1024;
    if (pw) {
        auto go = [&](auto kern) { kern<<<grid, 256, pw_lds, st>>>(a, pl); };
        if (wm == 1)
            a.rowsum ? go(k_conv_pool_pw<1, true>) : go(k_conv_pool_pw<1, false>);
        else
            a.rowsum ? go(k_conv_pool_pw<2, true>) : go(k_conv_pool_pw<2, false>);
    } else if (wm == 1)
        k_conv_pool<1><<<grid, 256, lds(1), st>>>(a, pl);
    else
        k_conv_pool<2><<<grid, 256, lds(2), st>>>(a, pl);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_hip_error("qa_d_conv_pool", e);
        return false;
    }
    return true;
}

}  // namespace qa

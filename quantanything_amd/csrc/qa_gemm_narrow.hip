// Narrow int8 GEMMs and pointwise convolutions with the table epilogue:
// 16, 32 or 64 output channels, K a multiple of 64 up to 576, any number of
// rows M (the standalone 4096 x 576 x 64 GEMM, the 1x1 convolutions of 16 -
// 64 channels over 64 to 576 input channels).
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
// or 64 x 16; wave w owns one 16 x 16 block and holds all of its K-steps'
// weight fragments in VGPRs. The MFMA takes the weights as its first
// operand, so its result lane l holds channels 4 (l >> 4) + i of row
// (l & 15): four consecutive bytes of one output row, stored as one word,
// with no exchange between lanes. With ALDS (Cout 64: one row tile) the
// work-group's 16 activation rows go once to LDS by direct global -> LDS
// loads, a quarter of the L1 reads of loading them per wave; a direct load
// of 64 lanes fills 1 KB of LDS in lane order, lane l taking row l & 15,
// k-group l >> 4 of its K-step, which is the MFMA fragment layout, so each
// fragment read is one contiguous KB. Epilogue per value: the plan's 64-bit
// multiply-add and shift with the zero-point correction folded into its
// constant, one med3 clip, then the table entry or, for an identity plan
// (plain requantize), the byte offset.
#include "qa_conv_mfma.h"

namespace qa {
namespace {

constexpr int GN_KMAX = 9;  // K-steps of 64 bytes held in registers
constexpr int GN_DEVICES = 16;

// The kernel's arguments, read in one scalar round.
struct GnArgs {
    const int8_t* x;       // activation rows, xpst bytes apart
    const int8_t* wp;      // packed weight rows, 16 * KGp bytes apart
    const char* plan;      // table epilogue plan
    const int64_t* corr;   // per-channel correction (zeros when none)
    const int32_t* boff;   // per-channel weight offsets (RS)
    int8_t* y;             // output rows, ypst bytes apart
    int64_t xpst, ypst, M;
    int32_t KGp, pad;
};

// The correction read by plans without one (zero-initialized; read only).
__device__ int64_t gn_zero_corr[64];

// NB: 16-channel blocks (1, 2 or 4); the work-group's 4 waves cover 4 / NB
// row tiles of 16. RS: pixel sums (weights with an offset). ALDS: the
// activation rows staged once in LDS (NB = 4).
template <int NB, bool RS, bool ALDS>
__global__ __launch_bounds__(256) void k_gemm_narrow(GnArgs a) {
    static_assert(!ALDS || NB == 4, "one row tile per work-group");
    constexpr int RT = 4 / NB;
    __shared__ int s_tab[256];
    // ALDS: K-step s of row r, k-group g at 16 (64 s + 16 g + r). (A size
    // that depends on ALDS makes hipcc's host pass drop the launch stubs
    // when the direct-load builtin writes the array; unused, it takes no
    // LDS.)
    __shared__ __attribute__((aligned(16))) int8_t s_x[16 * 64 * GN_KMAX];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 15, kg = lane >> 4;
    const int c0 = (wave % NB) * 16;
    const int64_t p0 = ((int64_t)blockIdx.x * RT + wave / NB) * 16;
    const int nks = a.KGp >> 2;  // 64-byte K-steps, 1..GN_KMAX
    const int8_t* xr = a.x + min(p0 + col, a.M - 1) * a.xpst + 16 * kg;
    const int8_t* wr = a.wp + (c0 + col) * (16 * a.KGp) + 16 * kg;

    // every request first, unconditionally
    const int tv = ((const int*)(a.plan + PLAN_E))[tid];
    v4i fw[GN_KMAX], fx[GN_KMAX];
#pragma unroll
    for (int s = 0; s < GN_KMAX; ++s) {
        const int o = min(s, nks - 1) * 64;  // past the last: re-read it
        fw[s] = *(const v4i*)(wr + o);
        if (!ALDS) fx[s] = *(const v4i*)(xr + o);
    }
    if (ALDS) {
        // wave w: K-steps w, w + 4, ... (each LDS KB written once: the
        // compiler would order two direct loads to one address by a wait)
        auto dload = [&](int t) __attribute__((always_inline)) {
            __builtin_amdgcn_global_load_lds(xr + t * 64, s_x + 1024 * t, 16,
                                             0, 0);
        };
#pragma unroll
        for (int s = 0; s < GN_KMAX; s += 4)
            if (s + wave < nks) dload(s + wave);
    }
    const int4 hdr = *(const int4*)a.plan;
    const int pD = ((const int*)a.plan)[4];
    int4 pc[4];
    uint32_t crr[4], cbo[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int c = c0 + 4 * kg + r;
        pc[r] = ((const int4*)(a.plan + PLAN_CH))[c];
        crr[r] = (uint32_t)a.corr[c];
        cbo[r] = RS ? (uint32_t)a.boff[c] : 0u;
    }
    // every load done (the direct ones among them), the table to LDS, then
    // one bare barrier (the empty asm keeps LDS accesses on their side)
    __builtin_amdgcn_s_waitcnt(0x0f70);
    s_tab[tid] = tv;
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (ALDS) {
#pragma unroll
        for (int s = 0; s < GN_KMAX; ++s)
            fx[s] = *(const v4i*)(s_x + 1024 * min(s, nks - 1) + 16 * lane);
    }

    v4i acc = v4i{0, 0, 0, 0};
    int psum = 0;
#pragma unroll
    for (int s = 0; s < GN_KMAX; ++s) {
        if (s < nks) {
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(fw[s], fx[s], acc, 0,
                                                        0, 0);
            if (RS) psum += bytes_sum(fx[s], 16);
        }
    }
    if (RS) {  // the row's byte sum over its 4 k-group lanes
        psum += __shfl_xor(psum, 16);
        psum += __shfl_xor(psum, 32);
    }

    const int pA = hdr.x, pB = hdr.y;
    const bool idt = hdr.w & PLAN_IDENT;
    int e[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        int w = acc[r];
        if (RS) w += (int)(cbo[r] * (uint32_t)psum);
        const int64_t cc = plan_fold(
            (int64_t)(((uint64_t)(uint32_t)pc[r].w << 32) |
                      (uint32_t)pc[r].z),
            crr[r], pc[r].x);
        const int v = med3_i32(plan_q0(w, pc[r].x, cc, pc[r].y), pA, pB);
        e[r] = idt ? v + pD : s_tab[v - pA];
    }
    const int64_t p = p0 + col;
    if (p < a.M)
        *(uint32_t*)(a.y + p * a.ypst + c0 + 4 * kg) = pack_entries(e, 0);
}

}  // namespace

bool gemm_narrow_applies(const ConvArgs& b, int epi) {
    const uintptr_t xa = (uintptr_t)b.x;
    const int64_t hw = (int64_t)b.H * b.W;
    // a row's stride: the GEMM's row stride, or the pixel stride of a
    // dense channels-last tensor
    const int64_t xpst = hw == 1 ? b.x_sn : b.x_sp;
    return epi == Q8_TABLE && b.mode == EPI_QUANT && b.fastio && b.plan &&
           !b.res && !b.y2 && b.G == 1 && b.layout == 0 && b.KH == 1 &&
           b.KW == 1 && b.SH == 1 && b.SW == 1 && b.PH == 0 && b.PW == 0 &&
           b.OH == b.H && b.OW == b.W && (hw == 1 || b.x_sn == hw * b.x_sp) &&
           b.x_code == 1 && b.x_sc == 1 && xpst % 16 == 0 && xa % 16 == 0 &&
           (b.Cout == 16 || b.Cout == 32 || b.Cout == 64) &&
           b.Cg % 64 == 0 && b.KGp * 16 == b.Cg && b.KGp <= 4 * GN_KMAX &&
           b.wp_rstride == (int64_t)b.KGp * 16 && b.y_code == 1 &&
           b.M < ((int64_t)1 << 31);
}

bool launch_gemm_narrow(const ConvArgs& b, hipStream_t st, bool alds) {
    const int nb = b.Cout / 16;
    const int64_t blocks = ceil_div(b.M, 16 * (4 / nb));
    if (blocks >= ((int64_t)1 << 31)) {
        set_error("launch_gemm_narrow", "grid too large");
        return false;
    }
    const int64_t* corr = b.corr;
    if (!corr) {  // gn_zero_corr's address on the current device
        static int64_t* zeros[GN_DEVICES] = {};
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess || dev < 0 ||
            dev >= GN_DEVICES ||
            (!zeros[dev] &&
             hipGetSymbolAddress((void**)&zeros[dev],
                                 HIP_SYMBOL(gn_zero_corr)) != hipSuccess)) {
            set_error("launch_gemm_narrow", "no zero correction array");
            return false;
        }
        corr = zeros[dev];
    }
    GnArgs g;
    g.x = (const int8_t*)b.x;
    g.wp = b.wp;
    g.plan = (const char*)b.plan;
    g.corr = corr;
    g.boff = b.boff;
    g.y = (int8_t*)b.y;
    g.xpst = (int64_t)b.H * b.W == 1 ? b.x_sn : b.x_sp;
    g.ypst = b.y_pst;
    g.M = b.M;
    g.KGp = b.KGp;
    g.pad = 0;
    const dim3 grid((unsigned)blocks);
    if (nb == 4 && alds) {
        if (b.rowsum)
            k_gemm_narrow<4, true, true><<<grid, 256, 0, st>>>(g);
        else
            k_gemm_narrow<4, false, true><<<grid, 256, 0, st>>>(g);
    } else {
        switch (nb * 2 + (b.rowsum ? 1 : 0)) {
#define QA_GN_CASE(NB, RS)                                          \
    case NB * 2 + RS:                                               \
        k_gemm_narrow<NB, RS != 0, false><<<grid, 256, 0, st>>>(g); \
        break;
            QA_GN_CASE(1, 0) QA_GN_CASE(1, 1) QA_GN_CASE(2, 0)
            QA_GN_CASE(2, 1) QA_GN_CASE(4, 0) QA_GN_CASE(4, 1)
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

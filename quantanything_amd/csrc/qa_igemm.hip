// MFMA implicit-GEMM kernel (see qa_igemm.h for the data layout).
//
// Work-group: 256 threads = 4 wave64s arranged WAVES_M x WAVES_N; each wave
// owns a (WM*16) x (WN*16) block of the output tile and keeps WM*WN
// 16x16 int32 accumulators. Per K-step (64 bytes of K) the work-group
// gathers its A tile (BM rows x 4 k-groups, 16 bytes each) from HBM into LDS
// -- the NCHW gather transposes activations so that K becomes contiguous --
// and every wave reads its B fragments (packed weights, 16 contiguous bytes
// per lane) straight from global memory, where they stay L2-resident.
#include "qa_epilogue.h"

namespace qa {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t pack4(int b0, int b1, int b2, int b3) {
    return (uint32_t)(uint8_t)b0 | ((uint32_t)(uint8_t)b1 << 8) |
           ((uint32_t)(uint8_t)b2 << 16) | ((uint32_t)(uint8_t)b3 << 24);
}

__device__ __forceinline__ int bsum4(uint32_t w) {
    return (int)(int8_t)(w & 0xff) + (int)(int8_t)((w >> 8) & 0xff) +
           (int)(int8_t)((w >> 16) & 0xff) + (int)(int8_t)(w >> 24);
}

// One 16-byte (row, k-group) unit of the A tile. Accumulates the row sum of
// the real (non K-padding) values into *rs when ROWSUM.
template <bool ROWSUM>
__device__ __forceinline__ int4 load_unit(const IgemmArgs& a,
                                          const int8_t* __restrict__ xrow,
                                          bool prow, int iy0, int ix0,
                                          int64_t p, int kgi, int* rs) {
    int v[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) v[j] = 0;
    if (prow && kgi < a.KG) {
        if (a.rowmajor) {
            const int k0 = kgi * 16;
            const int nch = min(16, a.Kreal - k0);
            const int8_t* src = a.x + p * a.lda + k0;
            if (nch == 16 && (((uintptr_t)src) & 15) == 0) {
                const int4 w = *(const int4*)src;
                if (ROWSUM)
                    *rs += bsum4((uint32_t)w.x) + bsum4((uint32_t)w.y) +
                           bsum4((uint32_t)w.z) + bsum4((uint32_t)w.w);
                return w;
            }
#pragma unroll
            for (int j = 0; j < 16; ++j)
                if (j < nch) v[j] = src[j];
        } else {
            const int tap = kgi / a.CB;
            const int cb = kgi - tap * a.CB;
            const int ky = tap / a.KW;
            const int kx = tap - ky * a.KW;
            const int iy = iy0 + ky * a.DH;
            const int ix = ix0 + kx * a.DW;
            const int nch = min(16, a.Cg - cb * 16);
            if (iy < 0 || iy >= a.H || ix < 0 || ix >= a.W) {
#pragma unroll
                for (int j = 0; j < 16; ++j)
                    if (j < nch) v[j] = a.pad_value;
            } else {
                const int8_t* src = xrow + (int64_t)(cb * 16) * a.x_cstride +
                                    (int64_t)iy * a.W + ix;
#pragma unroll
                for (int j = 0; j < 16; ++j)
                    if (j < nch) v[j] = src[(int64_t)j * a.x_cstride];
            }
        }
        if (ROWSUM) {
            int s = 0;
#pragma unroll
            for (int j = 0; j < 16; ++j) s += v[j];
            *rs += s;
        }
    }
    int4 r;
    r.x = (int)pack4(v[0], v[1], v[2], v[3]);
    r.y = (int)pack4(v[4], v[5], v[6], v[7]);
    r.z = (int)pack4(v[8], v[9], v[10], v[11]);
    r.w = (int)pack4(v[12], v[13], v[14], v[15]);
    return r;
}

template <int WAVES_M, int WAVES_N, int WM, int WN, int MODE, bool ROWSUM>
__global__ __launch_bounds__(256) void k_igemm(IgemmArgs a) {
    constexpr int BM = WAVES_M * WM * 16;
    constexpr int BN = WAVES_N * WN * 16;
    constexpr int UPT = BM * 4 / 256;  // A units per thread per K-step
    static_assert(256 % BM == 0 || BM == 256, "BM must divide 256");
    __shared__ int4 sA[4 * BM];
    __shared__ int sRow[ROWSUM ? BM : 1];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wave_m = wave % WAVES_M;
    const int wave_n = wave / WAVES_M;
    const int g = blockIdx.z;
    const int64_t m0 = (int64_t)blockIdx.x * BM;
    const int n0 = blockIdx.y * BN;
    const uint32_t OHW = (uint32_t)(a.OH * a.OW);

    // ---- loader row of this thread (fixed over the K loop) ----
    const int lrow = tid % BM;
    const int64_t p = m0 + lrow;
    const bool prow = p < a.M;
    int iy0 = 0, ix0 = 0;
    const int8_t* xrow = a.x;
    if (prow && !a.rowmajor) {
        const uint32_t n_img = (uint32_t)p / OHW;
        const uint32_t pix = (uint32_t)p - n_img * OHW;
        const int oy = (int)(pix / (uint32_t)a.OW);
        const int ox = (int)pix - oy * a.OW;
        iy0 = oy * a.SH - a.PH;
        ix0 = ox * a.SW - a.PW;
        xrow = a.x + (int64_t)n_img * a.x_nstride +
               (int64_t)g * a.Cg * a.x_cstride;
    }
    int rs = 0;
    if (ROWSUM) {
        if (tid < BM) sRow[tid] = 0;
    }

    v4i acc[WM][WN];
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < WN; ++j) acc[i][j] = v4i{0, 0, 0, 0};

    const int8_t* wg = a.wp + (int64_t)g * a.wp_gstride;
    const int KS = a.KGp >> 2;
    for (int ks = 0; ks < KS; ++ks) {
        int4 u[UPT];
#pragma unroll
        for (int j = 0; j < UPT; ++j) {
            const int kgl = (tid + 256 * j) / BM;
            u[j] = load_unit<ROWSUM>(a, xrow, prow, iy0, ix0, p, ks * 4 + kgl,
                                     &rs);
        }
        v4i bf[WN];
#pragma unroll
        for (int wn = 0; wn < WN; ++wn) {
            const int col = n0 + wave_n * WN * 16 + wn * 16 + (lane & 15);
            bf[wn] = *(const v4i*)(wg + (int64_t)col * a.wp_rstride +
                                   (ks * 4 + (lane >> 4)) * 16);
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < UPT; ++j) {
            const int kgl = (tid + 256 * j) / BM;
            sA[kgl * BM + lrow] = u[j];
        }
        __syncthreads();
        v4i af[WM];
#pragma unroll
        for (int wm = 0; wm < WM; ++wm)
            af[wm] = *(const v4i*)&sA[(lane >> 4) * BM + wave_m * WM * 16 +
                                      wm * 16 + (lane & 15)];
#pragma unroll
        for (int wm = 0; wm < WM; ++wm)
#pragma unroll
            for (int wn = 0; wn < WN; ++wn)
                acc[wm][wn] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                    af[wm], bf[wn], acc[wm][wn], 0, 0, 0);
    }

    if (ROWSUM) {
        atomicAdd(&sRow[lrow], rs);
        __syncthreads();
    }

    // ---- epilogue ----
#pragma unroll
    for (int wn = 0; wn < WN; ++wn) {
        const int col = n0 + wave_n * WN * 16 + wn * 16 + (lane & 15);
        if (col >= a.Cog) continue;
        const int co = g * a.Cog + col;
        const int64_t corr = a.corr ? a.corr[co] : 0;
        const int64_t boff = ROWSUM ? (int64_t)a.boff[co] : 0;
        int64_t pre = 0, mult = 0, shift = 0;
        if (MODE == EPI_QUANT) {
            pre = a.pre ? a.pre[co] : 0;
            mult = a.mult[co];
            shift = a.shift[co];
        }
#pragma unroll
        for (int wm = 0; wm < WM; ++wm) {
            const int rbase = wave_m * WM * 16 + wm * 16 + (lane >> 4) * 4;
            const int64_t pb = m0 + rbase;
            if (pb >= a.M) continue;
            int64_t val[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int64_t rsum = ROWSUM ? (int64_t)sRow[rbase + i] : 0;
                if (MODE == EPI_RAW64) {
                    val[i] = (int64_t)acc[wm][wn][i] + corr + boff * rsum;
                } else {
                    const uint32_t w32 = (uint32_t)acc[wm][wn][i] +
                                         (uint32_t)corr +
                                         (uint32_t)boff * (uint32_t)rsum;
                    val[i] = (int64_t)(int32_t)w32;
                }
            }
            if (MODE == EPI_QUANT) {
                const bool has_res = a.res != nullptr;
                const bool vec4 = a.out_code == 1 && (OHW & 3) == 0 &&
                                  pb + 3 < a.M && (a.y_nstride & 3) == 0 &&
                                  (((uintptr_t)a.y) & 3) == 0;
                int64_t q[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    q[i] = 0;
                    if (pb + i < a.M) {
                        const uint32_t pp = (uint32_t)(pb + i);
                        const uint32_t ni = pp / OHW;
                        const uint32_t px = pp - ni * OHW;
                        int64_t rq = 0;
                        if (has_res) {
                            const int64_t ridx =
                                (int64_t)ni * a.res_nstride +
                                (a.res_choff + co) * (int64_t)OHW + px;
                            rq = (a.out_code == 1
                                      ? (int64_t)((const int8_t*)a.res)[ridx]
                                      : (int64_t)((const int16_t*)a.res)[ridx]) +
                                 a.res_so;
                        }
                        q[i] = quant_one(a, val[i] + pre, mult, shift, rq,
                                         has_res) -
                               a.out_so;
                        if (!vec4) {
                            const int64_t oidx =
                                (int64_t)ni * a.y_nstride +
                                (a.y_choff + co) * (int64_t)OHW + px;
                            if (a.out_code == 1)
                                ((int8_t*)a.y)[oidx] = (int8_t)q[i];
                            else
                                ((int16_t*)a.y)[oidx] = (int16_t)q[i];
                        }
                    }
                }
                if (vec4) {
                    // 4 consecutive pixels of one plane, 4-byte aligned
                    const uint32_t ni = (uint32_t)pb / OHW;
                    const uint32_t px = (uint32_t)pb - ni * OHW;
                    const int64_t oidx = (int64_t)ni * a.y_nstride +
                                         (a.y_choff + co) * (int64_t)OHW + px;
                    *(uint32_t*)((int8_t*)a.y + oidx) =
                        pack4((int)q[0], (int)q[1], (int)q[2], (int)q[3]);
                }
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    if (pb + i < a.M) {
                        const uint32_t pp = (uint32_t)(pb + i);
                        const uint32_t ni = pp / OHW;
                        const uint32_t px = pp - ni * OHW;
                        const int64_t oidx = (int64_t)ni * a.y_nstride +
                                             (a.y_choff + co) * (int64_t)OHW +
                                             px;
                        if (MODE == EPI_RAW64)
                            ((int64_t*)a.y)[oidx] = val[i];
                        else
                            ((int32_t*)a.y)[oidx] = (int32_t)val[i];
                    }
                }
            }
        }
    }
}

template <int WAVES_M, int WAVES_N, int WM, int WN>
bool launch_cfg(const IgemmArgs& a, int mode, bool rowsum, hipStream_t st) {
    constexpr int BM = WAVES_M * WM * 16;
    constexpr int BN = WAVES_N * WN * 16;
    dim3 grid((unsigned)ceil_div(a.M, BM), (unsigned)ceil_div(a.Cog, BN),
              (unsigned)a.G);
#define QA_LAUNCH(MODE, RS) \
    k_igemm<WAVES_M, WAVES_N, WM, WN, MODE, RS><<<grid, 256, 0, st>>>(a)
    if (rowsum) {
        if (mode == EPI_RAW32) QA_LAUNCH(EPI_RAW32, true);
        else if (mode == EPI_RAW64) QA_LAUNCH(EPI_RAW64, true);
        else QA_LAUNCH(EPI_QUANT, true);
    } else {
        if (mode == EPI_RAW32) QA_LAUNCH(EPI_RAW32, false);
        else if (mode == EPI_RAW64) QA_LAUNCH(EPI_RAW64, false);
        else QA_LAUNCH(EPI_QUANT, false);
    }
#undef QA_LAUNCH
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_hip_error("k_igemm launch", e);
        return false;
    }
    return true;
}

}  // namespace

bool launch_igemm(const IgemmArgs& a, int mode, bool rowsum, hipStream_t st) {
    if (a.M <= 0 || a.Cog <= 0 || a.G <= 0) return true;
    if (a.M >= ((int64_t)1 << 31)) {
        set_error("launch_igemm", "more than 2^31 output rows per group");
        return false;
    }
    if (a.Cog <= 16) return launch_cfg<4, 1, 4, 1>(a, mode, rowsum, st);
    if (a.Cog <= 32) return launch_cfg<4, 1, 4, 2>(a, mode, rowsum, st);
    if (a.Cog <= 64) return launch_cfg<2, 2, 4, 2>(a, mode, rowsum, st);
    return launch_cfg<2, 2, 4, 4>(a, mode, rowsum, st);
}

}  // namespace qa

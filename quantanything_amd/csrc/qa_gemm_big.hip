// Large int8 GEMMs with the table epilogue (the weight MatMuls of
// transformers: M = batch x tokens rows, K and N in the hundreds or more).
//
// The convolution kernel computes 16-row tiles and reuses each weight
// fragment once per tile; for GEMMs of thousands of rows that leaves the
// matrix cores waiting on the memory pipe. Here a work-group computes a
// 128 x 128 block of C: its 4 waves (2 x 2) own 64 x 64 each, i.e. 4 x 4
// MFMA tiles of v_mfma_i32_16x16x64_i8, so every A fragment feeds 4 MFMAs
// and every B fragment 4. K runs in 64- or 128-byte steps through two LDS
// buffers (global -> registers for the next step while a step's MFMAs run,
// one barrier a step), or (S > 0) in 64-byte steps through S LDS stages
// filled straight from global memory (global_load_lds_dwordx4: no
// registers hold loads in flight, so S - 1 steps are requested ahead). The epilogue is the int8 table plan of qa_conv.h
// (per-channel multiply-add and shift, 256-entry clip / activation /
// residual / copy tables), identical in results to the convolution
// kernel's; residual, copy and pixel sums are template flags, full tiles
// skip the bounds tests, and each lane stores 4 channels of a row as one
// word (4x4 byte transpose across a lane quad).
//
// Operands: A row p (one pixel of a GEMM descriptor, H = W = 1) at
// x + p * x_sn, K = Cg bytes; B = the packed weight rows (layout 0, one
// group), K bytes each, rows padded to 128.
#include <type_traits>

#include "qa_conv_mfma.h"

namespace qa {
namespace {

constexpr int GB_M = 128, GB_N = 128;

// BK: K bytes a step (64 or 128: one or two MFMA K-depths per barrier);
// P: steps whose global loads are in flight (a ring of P register slots:
// step k's operands are requested when step k - P is stored to LDS, so the
// memory latency is covered by P steps of MFMAs; with K <= P * BK every
// load is issued before the first MFMA).
// RES / Y2 / RS: residual Add, rescaled second output, pixel sums of the
// activations (weights with an offset) in the epilogue.
// S > 0 (BK 64, P unused): stage s holds A (128 rows x 64 bytes) and B
// (128 x 64) at dynamic LDS bytes 16384 s and 16384 s + 8192; row r's
// 16-byte chunk c sits at position c ^ ((r >> 1) & 3) of the row, so that
// the 8 rows one fragment read serves at a time fall in distinct banks
// without padding (a 64-lane direct load fills 1 KB contiguously: 16 rows
// of 4 positions, lane l at row l / 4, position l % 4).
constexpr int GB_STAGE = 16384;

// vmcnt(n) for n a multiple of 4 up to 12 (expcnt and lgkmcnt not waited)
__device__ __forceinline__ void wait_vm(int n) {
    switch (n) {
        case 0: __builtin_amdgcn_s_waitcnt(0x0f70); break;
        case 4: __builtin_amdgcn_s_waitcnt(0x0f74); break;
        case 8: __builtin_amdgcn_s_waitcnt(0x0f78); break;
        default: __builtin_amdgcn_s_waitcnt(0x0f7c); break;
    }
}
template <int P, int BK, bool RES, bool Y2, bool RS, int S>
__global__ __launch_bounds__(256) void k_gemm_big(ConvArgs a) {
    static_assert(S == 0 || (BK == 64 && S >= 2 && S <= 5), "stages");
    constexpr int GB_K = BK;
    constexpr int GB_RS = BK + 16;  // LDS row stride (bytes)
    constexpr int CPR = BK / 16;    // 16-byte chunks per row
    constexpr int CH = GB_M * CPR / 256;  // chunks per thread and operand
    // the two register-path buffers (S > 0: the dynamic stages instead)
    constexpr int SAB = S > 0 ? 16 : GB_M * GB_RS;
    __shared__ __attribute__((aligned(16))) int8_t sA[2][SAB];
    __shared__ __attribute__((aligned(16))) int8_t sB[2][SAB];
    extern __shared__ int4 gb_dyn[];
    __shared__ int s_tab[768];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int col = lane & 15, kg = lane >> 4;
    // tile of this work-group: consecutive work-groups go to different
    // XCDs (round robin), so the linear index is remapped to make the
    // tiles of each XCD consecutive; consecutive tiles share their A rows
    // (column blocks fastest), which then stay in that XCD's L2
    const int nb = (a.Cout + GB_N - 1) / GB_N;
    const int ntile = gridDim.x;
    const int per = (ntile + 7) / 8;
    const int bid = blockIdx.x;
    const int xcd = bid & 7, idx = bid >> 3;
    // XCDs 0..rem-1 hold per tiles, the others per - 1 (when ntile % 8)
    const int rem = ntile - 8 * (per - 1);
    const int t = xcd < rem ? xcd * per + idx
                            : rem * per + (xcd - rem) * (per - 1) + idx;
    const int64_t m0 = (int64_t)(t / nb) * GB_M;
    const int n0 = (t % nb) * GB_N;
    const int K = a.KGp * 16;
    const int nk = K / GB_K;
    const int8_t* xa = (const int8_t*)a.x;

    // global -> registers: per operand and step, CH chunks of 16 bytes per
    // thread (chunk tid + 256 j: row (tid / CPR) + j * 256 / CPR, bytes
    // 16 (tid % CPR)); loads past the last step re-read it (in bounds,
    // unused)
    constexpr int RSTEP = 256 / CPR;  // rows between a thread's chunks
    const int lr = tid / CPR, lk = (tid % CPR) * 16;
    typedef int vch __attribute__((ext_vector_type(4 * CH)));
    vch ra[S > 0 ? 1 : P], rb[S > 0 ? 1 : P];
    auto gload = [&](vch& va, vch& vb, int ks) __attribute__((always_inline)) {
        const int o = min(ks, nk - 1) * GB_K + lk;
#pragma unroll
        for (int j = 0; j < CH; ++j) {
            const int r = lr + j * RSTEP;
            const int4 x = *(const int4*)(xa + min(m0 + r, a.M - 1) * a.x_sn +
                                          o);
            const int4 w =
                *(const int4*)(a.wp + (int64_t)(n0 + r) * a.wp_rstride + o);
            va[4 * j] = x.x;
            va[4 * j + 1] = x.y;
            va[4 * j + 2] = x.z;
            va[4 * j + 3] = x.w;
            vb[4 * j] = w.x;
            vb[4 * j + 1] = w.y;
            vb[4 * j + 2] = w.z;
            vb[4 * j + 3] = w.w;
        }
    };
    auto sstore = [&](const vch& va, const vch& vb, int buf)
                      __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < CH; ++j) {
            const int r = lr + j * RSTEP;
            *(int4*)&sA[buf][r * GB_RS + lk] =
                int4{va[4 * j], va[4 * j + 1], va[4 * j + 2], va[4 * j + 3]};
            *(int4*)&sB[buf][r * GB_RS + lk] =
                int4{vb[4 * j], vb[4 * j + 1], vb[4 * j + 2], vb[4 * j + 3]};
        }
    };
    // S > 0: this lane's direct loads: rows 32 wave + lane / 4 (+ 16) of
    // A and B, the global chunk stored at position lane % 4 of its row
    int8_t* const stg = (int8_t*)gb_dyn;
    const int lrow = 32 * wave + (lane >> 2);
    const int gch = 16 * ((lane & 3) ^ ((lrow >> 1) & 3));
    const int8_t* const ga0 =
        xa + min(m0 + lrow, a.M - 1) * a.x_sn + gch;
    const int8_t* const ga1 =
        xa + min(m0 + lrow + 16, a.M - 1) * a.x_sn + gch;
    const int8_t* const gb0 = a.wp + (int64_t)(n0 + lrow) * a.wp_rstride + gch;
    const int8_t* const gb1 = gb0 + 16 * a.wp_rstride;
    // step ks of 64 bytes into stage ks % S (4 direct loads a lane)
    auto dload = [&](int ks) __attribute__((always_inline)) {
        int8_t* const sb = stg + (ks % S) * GB_STAGE + 32 * 64 * wave;
        const int ko = ks * 64;
        __builtin_amdgcn_global_load_lds(ga0 + ko, sb, 16, 0, 0);
        __builtin_amdgcn_global_load_lds(ga1 + ko, sb + 16 * 64, 16, 0, 0);
        __builtin_amdgcn_global_load_lds(gb0 + ko, sb + 8192, 16, 0, 0);
        __builtin_amdgcn_global_load_lds(gb1 + ko, sb + 8192 + 16 * 64, 16,
                                         0, 0);
    };
    // the plan's tables (768 entries, 3 a thread) requested before the
    // operands, so that storing them waits for them alone (loads complete
    // in issue order)
    int tv[3];
#pragma unroll
    for (int j = 0; j < 3; ++j)
        tv[j] = ((const int*)((const char*)a.plan + PLAN_E))[tid + 256 * j];
    if constexpr (S > 0) {
        // the first S - 1 steps in flight: they overlap the set-up below
#pragma unroll
        for (int sl = 0; sl < S - 1; ++sl)
            if (sl < nk) dload(sl);
    } else {
        // every slot's loads first: they overlap the table set-up below
#pragma unroll
        for (int sl = 0; sl < P; ++sl) gload(ra[sl], rb[sl], sl);
    }

    // tables of the plan (S > 0: stored after the K loop, since an LDS
    // store here would wait for the direct loads in flight) and the lane's
    // 4 channels' constants
    if constexpr (S == 0) {
#pragma unroll
        for (int j = 0; j < 3; ++j) s_tab[tid + 256 * j] = tv[j];
    }
    const int4 hdr = *(const int4*)a.plan;
    // the lane's 4 channels' constants, the zero-point correction folded
    // into the plan constant (plan_q0; K <= 16384 keeps |w| + |corr| +
    // |boff * rowsum| below 2^31, so the int32 sum never wraps)
    int cm[4], ct[4];
    int64_t cc[4];
    uint32_t cbo[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int c = min(n0 + 64 * wn + 16 * j + col, a.Cout - 1);
        const int4 pc = ((const int4*)((const char*)a.plan + PLAN_CH))[c];
        cm[j] = pc.x;
        ct[j] = pc.y;
        cc[j] = plan_fold(
            (int64_t)(((uint64_t)(uint32_t)pc.w << 32) | (uint32_t)pc.z),
            a.corr ? (uint32_t)a.corr[c] : 0u, pc.x);
        cbo[j] = RS ? (uint32_t)a.boff[c] : 0u;
    }

    v4i acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = v4i{0, 0, 0, 0};
    int psum[4] = {0, 0, 0, 0};  // stored-byte sums of the lane's A rows
    // one K-step (BK / 64 MFMA depths) from LDS buffer buf
    auto mfma_step = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int h = 0; h < BK / 64; ++h) {
            v4i fa[4], fb[4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
                fa[i] = *(const v4i*)&sA[buf][(64 * wm + 16 * i + col) *
                                                  GB_RS + 64 * h + 16 * kg];
#pragma unroll
            for (int j = 0; j < 4; ++j)
                fb[j] = *(const v4i*)&sB[buf][(64 * wn + 16 * j + col) *
                                                  GB_RS + 64 * h + 16 * kg];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                        fa[i], fb[j], acc[i][j], 0, 0, 0);
            if (RS) {
#pragma unroll
                for (int i = 0; i < 4; ++i) psum[i] += bytes_sum(fa[i], 16);
            }
        }
    };
    // S > 0: a lane's fragment of rows 16 i + col, chunk kg, at position
    // kg ^ ((col >> 1) & 3) of the row (the tile's row bases are multiples
    // of 16)
    const int foff = col * 64 + 16 * (kg ^ ((col >> 1) & 3));
    auto mfma_stage = [&](const int8_t* sb) __attribute__((always_inline)) {
        v4i fa[4], fb[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
            fa[i] = *(const v4i*)(sb + (64 * wm + 16 * i) * 64 + foff);
#pragma unroll
        for (int j = 0; j < 4; ++j)
            fb[j] = *(const v4i*)(sb + 8192 + (64 * wn + 16 * j) * 64 + foff);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                    fa[i], fb[j], acc[i][j], 0, 0, 0);
        if (RS) {
#pragma unroll
            for (int i = 0; i < 4; ++i) psum[i] += bytes_sum(fa[i], 16);
        }
    };
    if constexpr (S > 0) {
        // step ks: this wave's loads of it done (those of the next
        // min(S - 2, nk - 1 - ks) steps may still be in flight), barrier
        // (every wave's part landed, and every wave is past step ks - 1,
        // whose stage the refill below overwrites), request step
        // ks + S - 1, MFMAs
        for (int ks = 0; ks < nk; ++ks) {
            wait_vm(4 * min(S - 2, nk - 1 - ks));
            // a bare barrier: the explicit wait above is the only one the
            // direct loads need (a fenced barrier would wait for all of
            // them); the empty asm keeps LDS accesses on their side of it
            asm volatile("" ::: "memory");
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
            if (ks + S - 1 < nk) dload(ks + S - 1);
            mfma_stage(stg + (ks % S) * GB_STAGE);
        }
#pragma unroll
        for (int j = 0; j < 3; ++j) s_tab[tid + 256 * j] = tv[j];
        __syncthreads();
    } else
    // step ks from slot sl: to LDS buffer ks & 1 (last read two steps ago,
    // before the previous step's barrier), refill the slot with step
    // ks + P, barrier, MFMAs
    for (int k0 = 0; k0 < nk; k0 += P) {
#pragma unroll
        for (int sl = 0; sl < P; ++sl) {
            const int ks = k0 + sl;
            if (ks < nk) {
                sstore(ra[sl], rb[sl], ks & 1);
                if (ks + P < nk) gload(ra[sl], rb[sl], ks + P);
                __syncthreads();
                mfma_step(ks & 1);
            }
        }
    }

    // epilogue: lane holds rows 16 i + 4 kg + r, column 16 j + col; the
    // quad's 4 channels of one row go out as one word (lane q of a quad
    // stores row 16 i + 4 kg + q, channels cq .. cq + 3). Per value: the
    // plan's multiply-add and shift, one med3 clip and one table read whose
    // LDS address folds in the clip's lower bound.
    const int pA = hdr.x, pB = hdr.y, pSH = hdr.z;
    // identity table (a plain requantize): the byte of clip(q0) + D
    const bool ident = !RES && !Y2 && (hdr.w & PLAN_IDENT);
    const int pD = ((const int*)a.plan)[4];
    const int* tabE = s_tab - pA;  // tabE[v] = E[v - pA] for v in [pA, pB]
    const int q = lane & 3;
    const uint32_t sel1 = q < 2 ? 0x05040100u : 0x03020706u;
    const uint32_t sel2 = (q & 1) ? 0x03070105u : 0x06020400u;
    const int cq = col & ~3;
    // the tile's rows and columns all inside the output: no bounds tests
    const bool full = m0 + GB_M <= a.M && n0 + GB_N <= a.Cout;
    auto epilogue = [&](auto checked, auto identity)
                        __attribute__((always_inline)) {
        constexpr bool CHK = decltype(checked)::value;
        constexpr bool IDT = decltype(identity)::value;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            int ps[4] = {0, 0, 0, 0};
            if (RS) {
                int sm = psum[i];
                sm += __shfl_xor(sm, 16);
                sm += __shfl_xor(sm, 32);
#pragma unroll
                for (int r = 0; r < 4; ++r) ps[r] = __shfl(sm, 4 * kg + r);
            }
            const int64_t pq = m0 + 64 * wm + 16 * i + 4 * kg + q;
            const bool pok = !CHK || pq < a.M;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int c0 = n0 + 64 * wn + 16 * j + cq;
                const bool cfull = !CHK || c0 + 3 < a.Cout;
                uint32_t rv = 0;
                if (RES) {
                    uint32_t w = 0;
                    const int8_t* pr =
                        (const int8_t*)a.res + pq * a.res_pst + c0;
                    if (!CHK) {
                        w = *(const uint32_t*)pr;
                    } else if (pok) {
                        if (cfull) {
                            w = *(const uint32_t*)pr;
                        } else {
#pragma unroll
                            for (int r = 0; r < 4; ++r)
                                if (c0 + r < a.Cout)
                                    w |= (uint32_t)(uint8_t)pr[r] << (8 * r);
                        }
                    }
                    rv = quad_transpose(w, sel1, sel2);
                }
                int e[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    int w = acc[i][j][r];
                    if (RS) w += (int)(cbo[j] * (uint32_t)ps[r]);
                    const int v =
                        med3_i32(plan_q0(w, cm[j], cc[j], ct[j]), pA, pB);
                    if (RES) {
                        const int tsum = s_tab[256 - pA + v] +
                                         s_tab[512 + ((rv >> (8 * r)) & 255)];
                        e[r] = s_tab[med3_i32(tsum, 0, pSH)];
                    } else if (IDT) {
                        e[r] = v + pD;
                    } else {
                        e[r] = tabE[v];
                    }
                }
                const uint32_t wy =
                    quad_transpose(pack_entries(e, 0), sel1, sel2);
                const uint32_t w2 =
                    Y2 ? quad_transpose(pack_entries(e, 1), sel1, sel2) : 0u;
                int8_t* py = (int8_t*)a.y + pq * a.y_pst + c0;
                int8_t* p2 = Y2 ? (int8_t*)a.y2 + pq * a.y2_pst + c0
                                : nullptr;
                if (!CHK || (pok && cfull)) {
                    *(uint32_t*)py = wy;
                    if (Y2) *(uint32_t*)p2 = w2;
                } else if (pok) {
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (c0 + r < a.Cout) {
                            py[r] = (int8_t)(wy >> (8 * r));
                            if (Y2) p2[r] = (int8_t)(w2 >> (8 * r));
                        }
                }
            }
        }
    };
    if (ident) {
        if (full)
            epilogue(std::false_type{}, std::true_type{});
        else
            epilogue(std::true_type{}, std::true_type{});
    } else if (full) {
        epilogue(std::false_type{}, std::false_type{});
    } else {
        epilogue(std::true_type{}, std::false_type{});
    }
}

}  // namespace

bool gemm_big_applies(const ConvArgs& b, int epi) {
    const uintptr_t xa = (uintptr_t)b.x;
    return epi == Q8_TABLE && b.mode == EPI_QUANT && b.fastio && b.plan &&
           b.G == 1 && b.layout == 0 && b.KH == 1 && b.KW == 1 &&
           b.H == 1 && b.W == 1 && b.OH == 1 && b.OW == 1 && b.x_code == 1 &&
           b.x_sc == 1 && b.Cg % 64 == 0 && b.Cg <= 16384 &&
           b.KGp * 16 == b.Cg &&
           b.wp_rstride == (int64_t)b.KGp * 16 && b.x_sn % 16 == 0 &&
           xa % 16 == 0 && b.y_code == 1 && b.M < ((int64_t)1 << 31);
}

bool launch_gemm_big(const ConvArgs& b, hipStream_t st, int stages) {
    const int64_t tiles = ceil_div(b.M, GB_M) * ceil_div(b.Cout, GB_N);
    if (tiles >= ((int64_t)1 << 31)) {
        set_error("launch_gemm_big", "grid too large");
        return false;
    }
    const int K = b.KGp * 16;
    const dim3 grid((unsigned)tiles);
    const int flags = (b.res ? 1 : 0) | (b.y2 ? 2 : 0) | (b.rowsum ? 4 : 0);
    auto go = [&](auto kp, auto kbk, auto ks) {
        constexpr int KP = decltype(kp)::value, KBK = decltype(kbk)::value;
        constexpr int KS = decltype(ks)::value;
        const size_t lds = (size_t)KS * GB_STAGE;
        switch (flags) {
#define QA_GB_CASE(F)                                                    \
    case F:                                                              \
        k_gemm_big<KP, KBK, (F & 1) != 0, (F & 2) != 0, (F & 4) != 0, KS> \
            <<<grid, 256, lds, st>>>(b);                                 \
        break;
            QA_GB_CASE(0) QA_GB_CASE(1) QA_GB_CASE(2) QA_GB_CASE(3)
            QA_GB_CASE(4) QA_GB_CASE(5) QA_GB_CASE(6) QA_GB_CASE(7)
#undef QA_GB_CASE
        }
    };
    // 128-byte steps when K allows, else 64-byte steps, the next step's
    // loads in flight (measured on the ViT-S GEMMs: deeper rings, which
    // cost VGPRs and so occupancy, were not faster in the pass)
    // or (stages 3 / 4) the direct-to-LDS pipeline of 64-byte steps
    using I1 = std::integral_constant<int, 1>;
    using I0 = std::integral_constant<int, 0>;
    using B64 = std::integral_constant<int, 64>;
    if (stages == 3)
        go(I1{}, B64{}, std::integral_constant<int, 3>{});
    else if (stages == 4)
        go(I1{}, B64{}, std::integral_constant<int, 4>{});
    else if (K % 128 == 0)
        go(I1{}, std::integral_constant<int, 128>{}, I0{});
    else
        go(I1{}, B64{}, I0{});
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_hip_error("launch_gemm_big", e);
        return false;
    }
    return true;
}

}  // namespace qa

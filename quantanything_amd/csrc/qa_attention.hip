// Attention fused into one launch: S = q k^T, P = Softmax over S's rows,
// O = P v, int8 operands on the matrix cores (v_mfma_i32_16x16x64_i8), S
// and P never leave the work-group. Each value is the one the three
// separate launches produce (k_matmul_act_mfma, k_softmax_rows_lut,
// k_matmul_act_mfma):
//   S: the exact integer dot product scaled once in float64, cast to
//      float32 and quantized (qa_quantize_mixed) with S's parameters;
//   P: exponentials from the qa_d_softmax_table table of S's quantization,
//      summed per lane in column order (columns col + 16 nt of a row sit in
//      lane col, nt = 0, 1, .., exactly the 16-lanes-a-row layout of
//      k_softmax_rows_lut<16, 16>), then across the row's 16 lanes by xor
//      shuffles 8, 4, 2, 1, one float64 reciprocal a row;
//   O: as S, from P and v.
//
// A work-group owns one (b0, b1) pair and 4 tiles of 16 query rows, one a
// wave. It stages k (rows of depth K) and v^T (rows of depth N_S) in LDS,
// zero-padded to the MFMA depth. S = q k^T leaves lane (col, kg) holding
// rows 4 kg + r, column 16 nt + col of every 16-column block nt, so one
// load of the exponential table serves 4 rows of the tile (4 table rows a
// wave-wide gather: about half the address-unit time of 16). P's bytes go
// to the wave's LDS tile row by row and come back as 16-byte fragments of
// O^T = v^T P^T, whose lane holds 4 consecutive features of one row (one
// word store).
//
// Per value: the float32 quantization (multiply, round, one fma for the
// tie test, one med3 clip) and v_cvt_pk_u8_f32, which converts the clipped
// value biased by 128 - so to its byte; a group of four whose tie test
// fails in any lane is requantized by the double form. Every loop over the
// 16-column blocks is branch-free (blocks past the launch's repeat the
// last block's k rows and count as columns past N_S), so each phase has
// all of its loads in flight at once.
#include "../../include/qa_hip.h"
#include "qa_conv_mfma.h"

namespace qa {
namespace {

typedef int v4a __attribute__((ext_vector_type(4)));

constexpr int QA_ATT_KSQ = 2;  // q / k depth up to 128 bytes

struct AttnGeom {
    int NpS;       // S columns rounded up to 16 (at most 256)
    int KpQ;       // q / k depth rounded up to 64
    int KpV;       // S columns (the depth of P v) rounded up to 64
    int NV;        // O columns rounded up to 16
    int RSK, RSV;  // LDS row strides (bytes) of depth KpQ / KpV rows
    int tiles;     // 16-row tiles of S and O per (b0, b1)
    int tpw;       // tiles per work-group (one a wave)
};

// One quantization's constants: qa_quantize_mixed's arguments and the
// float32 form's threshold (-1 where that form does not apply), and the
// clip bounds and zero point biased by 128 - so (the stored byte + 128).
// wrap: the clip range reaches past the int8 storage, whose bytes then
// wrap around (the stored byte is q - so modulo 256).
struct AttnQ {
    double scale, inv;
    float invf, tie, cb, lob, hib;
    int zp, qmin, qmax, so, wrap;
};

// The fused launch's operands and constants, compacted on the host.
struct AttnArgs {
    const int8_t *q, *k, *v;
    int8_t* y;
    int64_t q_s0, q_s1, q_sm, q_sk;
    int64_t k_s0, k_s1, k_sn, k_sk;
    int64_t v_s0, v_s1, v_sn, v_sk;
    int64_t y_s0, y_s1, y_sm, y_sn;
    const double* table;
    int B1, M, Ns, Kq, No;
    int oword;      // O rows stored a word (4 features) at a time
    double sS, sO;  // a_scale * b_scale of q k^T and of P v
    AttnQ S, P, O;
};

// qa_quantize_mixed's double form, out of line so that its registers stay
// out of the callers' loops.
__device__ __noinline__ int quant_exact(float y, double scale, double inv,
                                        int zp, int qmin, int qmax) {
    return (int)qa_quantize_one_fast(y, scale, inv, zp, qmin, qmax);
}

// quantize(y) + 128 - so by the float32 form (qa_quantize_f32, its clip on
// the biased bounds); sets slow where that form does not decide.
__device__ __forceinline__ float qb_fast(float y, const AttnQ& c, bool& slow) {
    const float r = rintf(y * c.invf);
    const float dd = fmaf(y, c.invf, -r);
    slow |= !(fabsf(dd) < c.tie);
    return __builtin_amdgcn_fmed3f(r + c.cb, c.lob, c.hib);
}

__device__ __forceinline__ float qb_exact(float y, const AttnQ& c) {
    return (float)(quant_exact(y, c.scale, c.inv, c.zp, c.qmin, c.qmax) -
                   c.so + 128);
}

// biased values of a storage that wraps, taken modulo 256 (a branch that
// is uniform: the flag is a kernel argument)
__device__ __forceinline__ void wrap_u8(float (&b)[4], const AttnQ& c) {
    if (c.wrap) {
#pragma unroll
        for (int r = 0; r < 4; ++r) b[r] = (float)((int)b[r] & 255);
    }
}

// four biased values (integers in [0, 255]) as the bytes of one word
__device__ __forceinline__ uint32_t pack_u8(const float (&b)[4]) {
    uint32_t w = __builtin_amdgcn_cvt_pk_u8_f32(b[0], 0, 0u);
    w = __builtin_amdgcn_cvt_pk_u8_f32(b[1], 1, w);
    w = __builtin_amdgcn_cvt_pk_u8_f32(b[2], 2, w);
    return __builtin_amdgcn_cvt_pk_u8_f32(b[3], 3, w);
}

// the 4 x 4 byte transpose of words a, b, c, d (rows) into o[0..3]
// (columns): o[j] = a.j | b.j << 8 | c.j << 16 | d.j << 24
__device__ __forceinline__ void transpose4(uint32_t a, uint32_t b, uint32_t c,
                                           uint32_t d, uint32_t* o) {
    const uint32_t ab0 = __builtin_amdgcn_perm(b, a, 0x05010400u);
    const uint32_t ab1 = __builtin_amdgcn_perm(b, a, 0x07030602u);
    const uint32_t cd0 = __builtin_amdgcn_perm(d, c, 0x05010400u);
    const uint32_t cd1 = __builtin_amdgcn_perm(d, c, 0x07030602u);
    o[0] = __builtin_amdgcn_perm(cd0, ab0, 0x05040100u);
    o[1] = __builtin_amdgcn_perm(cd0, ab0, 0x07060302u);
    o[2] = __builtin_amdgcn_perm(cd1, ab1, 0x05040100u);
    o[3] = __builtin_amdgcn_perm(cd1, ab1, 0x07060302u);
}

// NTS: 16-column blocks of S the kernel holds (>= the launch's NpS / 16);
// KSQ: 64-byte K-steps of q k^T (>= KpQ / 64).
template <int NTS, int KSQ>
__global__ __launch_bounds__(256, 3) void k_attention(AttnArgs d, AttnGeom g) {
    extern __shared__ int4 lds4[];
    int8_t* sk = (int8_t*)lds4;       // [NpS][RSK]  k rows
    int8_t* sv = sk + g.NpS * g.RSK;  // [NV][RSV]   v^T rows
    int8_t* sp = sv + g.NV * g.RSV;   // [4][16][RSV] P tiles
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 15, kg = lane >> 4;
    // the work-groups of one (b0, b1) pair read the same k and v: one XCD
    // runs them (xcd_block, x fastest)
    const XcdBlock blk = xcd_block(false);
    const int64_t bz = blk.y;
    const int64_t b0 = bz / d.B1, b1 = bz - b0 * d.B1;
    const int rt = (int)blk.x * g.tpw + wave;  // the wave's tile
    const int64_t m0 = (int64_t)rt * 16;

    // the lane's q fragments (row m0 + col, clamped; bytes past K are
    // zero), requested before the staging
    v4a fq[KSQ];
    {
        const int8_t* qr = d.q + b0 * d.q_s0 + b1 * d.q_s1 +
                           min(m0 + col, (int64_t)d.M - 1) * d.q_sm;
#pragma unroll
        for (int ks = 0; ks < KSQ; ++ks) {
            const int c = ks * 64 + kg * 16;
            fq[ks] = v4a{0, 0, 0, 0};
            if (c < d.Kq) fq[ks] = *(const v4a*)(qr + c);
        }
    }

    // ---- staging: k rows as 16-byte chunks; v^T 16 words a thread (4
    // keys x 16 features, transposed in registers), keys past N_S zero;
    // a round's loads all in flight before its stores ----
    {
        const int8_t* kb = d.k + b0 * d.k_s0 + b1 * d.k_s1;
        const int8_t* vb = d.v + b0 * d.v_s0 + b1 * d.v_s1;
        const int cpr = g.KpQ >> 4;        // k chunks per row
        const int nk = g.NpS * cpr;        // k chunks
        const int nq = g.KpV >> 2;         // key quads
        const int nvj = nq * (g.NV >> 4);  // v^T jobs (key quad, 16 features)
        for (int e0 = tid, j = tid; e0 < nk || j < nvj;
             e0 += 4 * 256, j += 256) {
            v4a kc[4], vc[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int e = e0 + u * 256;
                kc[u] = v4a{0, 0, 0, 0};
                if (e < nk) {
                    const int r = e / cpr, c = (e - r * cpr) * 16;
                    if (r < d.Ns && c < d.Kq)
                        kc[u] = *(const v4a*)(kb + (int64_t)r * d.k_sn + c);
                }
            }
            const int n16 = j / nq, c4 = j - n16 * nq;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int key = 4 * c4 + i;
                vc[i] = v4a{0, 0, 0, 0};
                if (j < nvj && key < d.Ns)
                    vc[i] = *(const v4a*)(vb + (int64_t)key * d.v_sk +
                                          16 * n16);
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int e = e0 + u * 256;
                if (e < nk) {
                    const int r = e / cpr, c = (e - r * cpr) * 16;
                    *(v4a*)(sk + r * g.RSK + c) = kc[u];
                }
            }
            if (j < nvj) {
                int8_t* dst = sv + 16 * n16 * g.RSV + 4 * c4;
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    uint32_t o[4];
                    transpose4((uint32_t)vc[0][w], (uint32_t)vc[1][w],
                               (uint32_t)vc[2][w], (uint32_t)vc[3][w], o);
#pragma unroll
                    for (int b = 0; b < 4; ++b)
                        *(uint32_t*)(dst + (4 * w + b) * g.RSV) = o[b];
                }
            }
        }
    }
    __syncthreads();
    if (rt >= g.tiles) return;  // a wave past the last tile

    const int nts = g.NpS >> 4;
    const int ksq = g.KpQ >> 6;
    // ---- S's scores: rows 4 kg + r, column 16 nt + col in sacc[nt][r] ----
    v4a sacc[NTS];
#pragma unroll
    for (int nt = 0; nt < NTS; ++nt) {
        const int8_t* kr =
            sk + (min(nt, nts - 1) * 16 + col) * g.RSK + kg * 16;
        sacc[nt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
            fq[0], *(const v4a*)kr, v4a{0, 0, 0, 0}, 0, 0, 0);
        if (KSQ > 1 && ksq > 1)
            sacc[nt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                fq[KSQ - 1], *(const v4a*)(kr + 64), sacc[nt], 0, 0, 0);
    }
    // The rows' maxima first: S's quantization is non-decreasing in the
    // integer score (the float64 scaling, the float32 cast, the rounding
    // and the clip all are; a storage that wraps is not supported here),
    // so a row's largest byte is the quantization of its largest score
    // over the columns before N_S. Then each block's bytes, whose table
    // reads go out at once: they overlap the next blocks' quantization.
    int amx[4] = {INT_MIN, INT_MIN, INT_MIN, INT_MIN};
#pragma unroll
    for (int nt = 0; nt < NTS; ++nt) {
        const bool live = 16 * nt + 16 <= d.Ns || 16 * nt + col < d.Ns;
#pragma unroll
        for (int r = 0; r < 4; ++r)
            amx[r] = max(amx[r], live ? sacc[nt][r] : INT_MIN);
    }
    uint32_t row[4];  // table offset of the row's maximum (a 16-bit index:
                      // the loads take the table as a scalar base)
    {
        float bm[4];
        bool slow = false;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
#pragma unroll
            for (int o = 8; o > 0; o >>= 1)
                amx[r] = max(amx[r], __shfl_xor(amx[r], o));
            bm[r] = qb_fast((float)((double)amx[r] * d.sS), d.S, slow);
        }
        if (slow) {
#pragma unroll
            for (int r = 0; r < 4; ++r)
                bm[r] = qb_exact((float)((double)amx[r] * d.sS), d.S);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) row[r] = ((uint32_t)bm[r] & 255u) << 8;
    }

    // ---- the Softmax of rows 4 kg + r ----
    uint32_t sw[NTS];
    double e[NTS][4];
#pragma unroll
    for (int nt = 0; nt < NTS; ++nt) {
        float b[4];
        bool slow = false;
#pragma unroll
        for (int r = 0; r < 4; ++r)
            b[r] = qb_fast((float)((double)sacc[nt][r] * d.sS), d.S, slow);
        if (slow) {
#pragma unroll
            for (int r = 0; r < 4; ++r)
                b[r] = qb_exact((float)((double)sacc[nt][r] * d.sS), d.S);
        }
        sw[nt] = pack_u8(b);
#pragma unroll
        for (int r = 0; r < 4; ++r)
            e[nt][r] = d.table[row[r] | ((sw[nt] >> (8 * r)) & 255u)];
    }
    // phase boundaries for the scheduler: each phase's values die in it
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int nt = 0; nt < NTS; ++nt)
        if (16 * nt + 16 > d.Ns && 16 * nt + col >= d.Ns) {
#pragma unroll
            for (int r = 0; r < 4; ++r) e[nt][r] = 0.0;
        }
    double rs[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        double t = 0.0;
#pragma unroll
        for (int nt = 0; nt < NTS; ++nt) t += e[nt][r];
#pragma unroll
        for (int o = 8; o > 0; o >>= 1) t += __shfl_xor(t, o);
        rs[r] = 1.0 / t;  // one division a row
    }
    __builtin_amdgcn_sched_barrier(0);
    // P's stored bytes to the wave's tile, rows of RSV bytes (columns past
    // N_S meet v^T's zero rows)
    int8_t* pw = sp + wave * 16 * g.RSV;
#pragma unroll
    for (int nt = 0; nt < NTS; ++nt) {
        float b[4];
        bool slow = false;
#pragma unroll
        for (int r = 0; r < 4; ++r)
            b[r] = qb_fast((float)(e[nt][r] * rs[r]), d.P, slow);
        if (slow) {
#pragma unroll
            for (int r = 0; r < 4; ++r)
                b[r] = qb_exact((float)(e[nt][r] * rs[r]), d.P);
        }
        wrap_u8(b, d.P);
        const uint32_t w = pack_u8(b) ^ 0x80808080u;
#pragma unroll
        for (int r = 0; r < 4; ++r)
            pw[(4 * kg + r) * g.RSV + 16 * nt + col] = (int8_t)(w >> (8 * r));
    }
    // the wave's P bytes before its reads of them
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    __builtin_amdgcn_sched_barrier(0);

    // ---- O^T = v^T P^T, 4 blocks of 16 features at a time: lane (col,
    // kg) holds row m0 + col, features 16 dt + 4 kg + r ----
    constexpr int KSV = (NTS + 3) / 4;  // K-steps of P v
    const int dts = g.NV >> 4, ksv = g.KpV >> 6;
    v4a pf[KSV];  // the lane's P fragments: row col, bytes 64 ks + 16 kg
#pragma unroll
    for (int ks = 0; ks < KSV; ++ks)
        pf[ks] = ks < ksv ? *(const v4a*)(pw + col * g.RSV + ks * 64 + kg * 16)
                          : v4a{0, 0, 0, 0};
    const int64_t m = m0 + col;
    int8_t* const yr = d.y + b0 * d.y_s0 + b1 * d.y_s1 + m * d.y_sm;
    for (int dt0 = 0; dt0 < dts; dt0 += 4) {
        v4a acc[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            acc[u] = v4a{0, 0, 0, 0};
            if (dt0 + u >= dts) continue;
            // K-steps past KpV repeat the last one against zero fragments
#pragma unroll
            for (int ks = 0; ks < KSV; ++ks)
                acc[u] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                    *(const v4a*)(sv + ((dt0 + u) * 16 + col) * g.RSV +
                                  min(ks, ksv - 1) * 64 + kg * 16),
                    pf[ks], acc[u], 0, 0, 0);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            if (dt0 + u >= dts) continue;
            float b[4];
            bool slow = false;
#pragma unroll
            for (int r = 0; r < 4; ++r)
                b[r] = qb_fast((float)((double)acc[u][r] * d.sO), d.O, slow);
            if (slow) {
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    b[r] = qb_exact((float)((double)acc[u][r] * d.sO), d.O);
            }
            wrap_u8(b, d.O);
            if (m >= d.M) continue;
            const int n = (dt0 + u) * 16 + 4 * kg;  // features n .. n + 3
            const uint32_t w = pack_u8(b) ^ 0x80808080u;
            if (d.oword) {
                *(uint32_t*)(yr + n) = w;
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    yr[(int64_t)(n + r) * d.y_sn] = (int8_t)(w >> (8 * r));
            }
        }
    }
}

// Geometry and LDS bytes of a fused launch; false (with the reason) when
// the descriptor is outside the fused kernel's conditions.
bool attn_geom(const qa_attention_desc* d, AttnGeom* g, int64_t* lds,
               const char** why) {
    const qa_matmul_desc& qk = d->qk;
    const qa_matmul_desc& av = d->av;
    *why = nullptr;
    if (qk.a_code != 1 || qk.b_code != 1 || av.b_code != 1 ||
        av.y_code != 1) {
        *why = "needs int8 operands and output";
    } else if (qk.a_so != qk.a_zp || qk.b_so != qk.b_zp ||
               av.b_so != av.b_zp || d->p_so != d->p_zp) {
        *why = "needs operands stored at their zero points";
    } else if (!d->table || !(d->p_scale > 0) || !(qk.out_scale > 0) ||
               !(av.out_scale > 0)) {
        *why = "needs the exponential table and positive scales";
    } else if (qk.a_sk != 1 || qk.K % 16 != 0 || qk.a_sm % 16 != 0 ||
               qk.a_s0 % 16 != 0 || qk.a_s1 % 16 != 0 ||
               (uintptr_t)qk.a % 16 != 0 || qk.b_sk != 1 ||
               qk.b_sn % 16 != 0 || qk.b_s0 % 16 != 0 ||
               qk.b_s1 % 16 != 0 || (uintptr_t)qk.b % 16 != 0 ||
               av.b_sn != 1 || av.b_sk % 16 != 0 || av.b_s0 % 16 != 0 ||
               av.b_s1 % 16 != 0 || (uintptr_t)av.b % 16 != 0 ||
               av.N % 16 != 0) {
        *why = "needs q and k rows and v columns of 16-byte aligned, "
               "contiguous bytes";
    } else if (qk.B0 < 1 || qk.B1 < 1 || qk.M < 1 || qk.N < 1 ||
               qk.N > 256 || qk.K < 1 || qk.K > 64 * QA_ATT_KSQ || av.N < 1 ||
               av.N > 256 || av.K != qk.N || av.M != qk.M ||
               av.B0 != qk.B0 || av.B1 != qk.B1 ||
               qk.B0 * qk.B1 > 65535 || qk.M >= ((int64_t)1 << 24)) {
        *why = "needs S rows of at most 256 columns, O of at most 256, and "
               "matching shapes";
    } else if (std::max({std::llabs(qk.qmin), std::llabs(qk.qmax),
                         std::llabs(d->p_qmin), std::llabs(d->p_qmax),
                         std::llabs(av.qmin), std::llabs(av.qmax)}) > 32768) {
        *why = "needs 8- or 16-bit clip bounds";
    } else if (av.a_scale != d->p_scale || av.a_zp != d->p_zp ||
               av.a_so != d->p_so) {
        *why = "P's quantization differs between the Softmax and P v";
    } else if (qk.qmin - qk.y_so < -128 || qk.qmax - qk.y_so > 127) {
        *why = "needs S's clip range within its int8 storage";
    }
    if (*why) return false;
    g->NpS = (int)round_up(qk.N, 16);
    g->KpQ = (int)round_up(qk.K, 64);
    g->KpV = (int)round_up(qk.N, 64);
    g->NV = (int)round_up(av.N, 16);
    g->RSK = g->KpQ + 16;
    g->RSV = g->KpV + 16;
    g->tiles = (int)ceil_div(qk.M, 16);
    g->tpw = 4;  // one 16-row tile per wave
    // k rows and v^T rows once per work-group, a P tile per wave
    *lds = (int64_t)g->NpS * g->RSK + (int64_t)g->NV * g->RSV +
           4LL * 16 * g->RSV;
    if (*lds > 96 * 1024) {
        *why = "operands exceed the LDS budget";
        return false;
    }
    return true;
}

}  // namespace
}  // namespace qa

using namespace qa;

QA_API int qa_attention_supported(const qa_attention_desc* d) {
    if (!d) return 0;
    AttnGeom g;
    int64_t lds;
    const char* why;
    return attn_geom(d, &g, &lds, &why) ? 1 : 0;
}

QA_API int qa_d_attention(const qa_attention_desc* d, void* stream) {
    if (!d) {
        set_error("qa_d_attention", "null descriptor");
        return -1;
    }
    AttnGeom g;
    int64_t lds;
    const char* why;
    if (!attn_geom(d, &g, &lds, &why)) {
        set_error("qa_d_attention", why);
        return -1;
    }
    const qa_matmul_desc& qk = d->qk;
    const qa_matmul_desc& av = d->av;
    auto qc = [](double scale, int64_t zp, int64_t qmin, int64_t qmax,
                 int64_t so) {
        AttnQ c;
        c.scale = scale;
        c.inv = 1.0 / scale;
        c.invf = (float)c.inv;
        c.zp = (int)zp;
        c.qmin = (int)qmin;
        c.qmax = (int)qmax;
        c.so = (int)so;
        // -1: every value takes the double form
        c.tie = qa_f32_form_ok(scale, zp, qmin, qmax)
                    ? qa_f32_tie(zp, qmin, qmax)
                    : -1.0f;
        c.cb = (float)(zp - so + 128);
        c.lob = (float)(qmin - so + 128);
        c.hib = (float)(qmax - so + 128);
        c.wrap = qmin - so < -128 || qmax - so > 127;
        return c;
    };
    AttnArgs a;
    a.q = (const int8_t*)qk.a;
    a.k = (const int8_t*)qk.b;
    a.v = (const int8_t*)av.b;
    a.y = (int8_t*)av.y;
    a.q_s0 = qk.a_s0, a.q_s1 = qk.a_s1, a.q_sm = qk.a_sm, a.q_sk = qk.a_sk;
    a.k_s0 = qk.b_s0, a.k_s1 = qk.b_s1, a.k_sn = qk.b_sn, a.k_sk = qk.b_sk;
    a.v_s0 = av.b_s0, a.v_s1 = av.b_s1, a.v_sn = av.b_sn, a.v_sk = av.b_sk;
    a.y_s0 = av.y_s0, a.y_s1 = av.y_s1, a.y_sm = av.y_sm, a.y_sn = av.y_sn;
    a.table = d->table;
    a.B1 = (int)qk.B1;
    a.M = (int)qk.M;
    a.Ns = (int)qk.N;
    a.Kq = (int)qk.K;
    a.No = (int)av.N;
    a.oword = av.y_sn == 1 && av.y_sm % 4 == 0 && av.y_s0 % 4 == 0 &&
              av.y_s1 % 4 == 0 && (uintptr_t)av.y % 4 == 0;
    a.sS = qk.a_scale * qk.b_scale;
    a.sO = av.a_scale * av.b_scale;
    a.S = qc(qk.out_scale, qk.out_zp, qk.qmin, qk.qmax, qk.y_so);
    a.P = qc(d->p_scale, d->p_zp, d->p_qmin, d->p_qmax, d->p_so);
    a.O = qc(av.out_scale, av.out_zp, av.qmin, av.qmax, av.y_so);
    const dim3 grid((unsigned)ceil_div(g.tiles, g.tpw),
                    (unsigned)(qk.B0 * qk.B1));
    const int nts = g.NpS / 16, ksq = g.KpQ / 64;
    hipStream_t st = (hipStream_t)stream;
    auto go = [&](auto kern) {
        kern<<<grid, 256, (size_t)lds, st>>>(a, g);
    };
    // the smallest instantiated block count >= nts
    if (ksq == 1) {
        if (nts <= 4) go(k_attention<4, 1>);
        else if (nts <= 8) go(k_attention<8, 1>);
        else if (nts <= 13) go(k_attention<13, 1>);
        else go(k_attention<16, 1>);
    } else {
        if (nts <= 4) go(k_attention<4, 2>);
        else if (nts <= 8) go(k_attention<8, 2>);
        else if (nts <= 13) go(k_attention<13, 2>);
        else go(k_attention<16, 2>);
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_hip_error("qa_d_attention", e);
        return -1;
    }
    return 0;
}

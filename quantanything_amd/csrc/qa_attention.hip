// Attention fused into one launch: S = q k^T, P = Softmax over S's rows,
// O = P v, int8 operands on the matrix cores (v_mfma_i32_16x16x64_i8), S
// and P never leave the work-group. Each value is the one the three
// separate launches produce (k_matmul_act_mfma, k_softmax_rows_lut,
// k_matmul_act_mfma):
//   S: the exact integer dot product scaled once in float64, cast to
//      float32 and quantized (qa_quantize_mixed) with S's parameters;
//   P: exponentials from the qa_d_softmax_table table of S's quantization,
//      summed per lane in column order (columns col + 16 nt of a row sit in
//      lane col, nt = 0..15, exactly the 16-lanes-a-row layout of
//      k_softmax_rows_lut<16, 16>), then across the row's 16 lanes by xor
//      shuffles 8, 4, 2, 1, one float64 reciprocal a row;
//   O: as S, from P and v.
//
// A work-group owns one (b0, b1) pair and a run of 16-row tiles of S / O:
// it stages k (S's columns, as rows of depth K), v^T (O's columns, as rows
// of depth N_S) and its q rows in LDS, zero-padded to the MFMA depth; each
// wave takes tiles in turn. Per tile: S's 16 x N_S accumulators in
// registers (MFMA C layout: lane col + 16 kg holds rows 4 kg + r, column
// col + 16 nt), S quantized and the Softmax row by row in registers, P's
// bytes to the wave's LDS tile (rows of N_S rounded up to 64, zero past
// N_S), read back as the A operand of O = P v.
#include "../../include/qa_hip.h"
#include "qa_conv_mfma.h"

namespace qa {
namespace {

typedef int v4a __attribute__((ext_vector_type(4)));

constexpr int QA_ATT_KSQ = 2;  // q / k depth up to 128 bytes
constexpr int QA_ATT_U = 8;    // staging chunks a thread has in flight

struct AttnGeom {
    int NpS;       // S columns rounded up to 16 (at most 256)
    int KpQ;       // q / k depth rounded up to 64
    int KpV;       // S columns (the depth of P v) rounded up to 64
    int NV;        // O columns rounded up to 16
    int RSK, RSV;  // LDS row strides (bytes) of depth KpQ / KpV rows
    int tiles;     // 16-row tiles of S and O per (b0, b1)
    int tpw;       // tiles per work-group
};

// One quantization's constants: qa_quantize_mixed's arguments and the
// float32 form's threshold and bounds (qa_quantize_f32), precomputed.
struct AttnQ {
    double scale, inv;
    float invf, tie, zpf, qminf, qmaxf;
    int zp, qmin, qmax, so, f32;
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
    double sS, sO;  // a_scale * b_scale of q k^T and of P v
    AttnQ S, P, O;
};

// qa_quantize_mixed with the constants precomputed, split: quant_fast is
// the float32 form (qa_quantize_f32) and sets *slow where that form does not
// decide (near-ties, NaN, or the scales outside the form); those values are
// recomputed by quant_exact, the double form, called out of line so that
// its registers stay out of the callers' loops. Together they return
// qa_quantize_mixed's value.
__device__ __noinline__ int quant_exact(float y, double scale, double inv,
                                        int zp, int qmin, int qmax) {
    return (int)qa_quantize_one_fast(y, scale, inv, zp, qmin, qmax);
}

__device__ __forceinline__ int quant_fast(float y, const AttnQ& c,
                                          bool* slow) {
    const float r = rintf(y * c.invf);
    const float dd = fmaf(y, c.invf, -r);
    *slow = !(c.f32 && fabsf(dd) < c.tie);
    return (int)__builtin_amdgcn_fmed3f(r + c.zpf, c.qminf, c.qmaxf);
}

__device__ __forceinline__ int quant_slow(float y, const AttnQ& c) {
    return quant_exact(y, c.scale, c.inv, c.zp, c.qmin, c.qmax);
}

__global__ __launch_bounds__(256) void k_attention(AttnArgs d, AttnGeom g) {
    extern __shared__ int4 lds4[];
    int8_t* sk = (int8_t*)lds4;              // [NpS][RSK]  k rows
    int8_t* sv = sk + g.NpS * g.RSK;          // [NV][RSV]   v^T rows
    int8_t* sp = sv + g.NV * g.RSV;           // [4][16][RSV] S / P tiles
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 15, kg = lane >> 4;
    // the work-groups of one (b0, b1) pair read the same k and v: one XCD
    // runs them (xcd_block, x fastest)
    const XcdBlock blk = xcd_block(false);
    const int64_t bz = blk.y;
    const int64_t b0 = bz / d.B1, b1 = bz - b0 * d.B1;
    const int rt0 = (int)blk.x * g.tpw;
    const int rt1 = min(rt0 + g.tpw, g.tiles);

    // the wave's q fragments of tile rt (rows past M read row M - 1,
    // bytes past K are zero); the first tile's are requested before the
    // staging below
    const int8_t* qb = d.q + b0 * d.q_s0 + b1 * d.q_s1;
    const int ksq = g.KpQ >> 6;
    v4a fa[QA_ATT_KSQ];
    auto load_q = [&](int rt) {
        const int8_t* qr =
            qb + min((int64_t)rt * 16 + col, (int64_t)d.M - 1) * d.q_sm;
#pragma unroll
        for (int ks = 0; ks < QA_ATT_KSQ; ++ks) {
            const int c = ks * 64 + kg * 16;
            fa[ks] = v4a{0, 0, 0, 0};
            if (ks < ksq && c < d.Kq) fa[ks] = *(const v4a*)(qr + c);
        }
    };
    load_q(rt0 + wave);

    // ---- staging: k rows (16-byte chunks along the depth) and v^T rows
    // (16 consecutive v columns of one row per chunk, scattered to 16 LDS
    // rows), zero past N_S and the depth; every load of the thread in
    // flight before the first store ----
    {
        const int8_t* kb = d.k + b0 * d.k_s0 + b1 * d.k_s1;
        const int8_t* vb = d.v + b0 * d.v_s0 + b1 * d.v_s1;
        const int cpr = g.KpQ >> 4;        // k chunks per row
        const int nk = g.NpS * cpr;        // k chunks
        const int nvr = g.NV >> 4;         // v^T row groups
        const int nch = nk + nvr * g.KpV;  // all chunks
        for (int e0 = tid; e0 < nch; e0 += QA_ATT_U * 256) {
            v4a ch[QA_ATT_U];
#pragma unroll
            for (int u = 0; u < QA_ATT_U; ++u) {
                const int e = e0 + u * 256;
                ch[u] = v4a{0, 0, 0, 0};
                if (e < nk) {
                    const int r = e / cpr, c = (e - r * cpr) * 16;
                    if (r < d.Ns && c < d.Kq)
                        ch[u] = *(const v4a*)(kb + (int64_t)r * d.k_sn + c);
                } else if (e < nch) {
                    const int f = e - nk;
                    const int c = f / nvr, n = (f - c * nvr) * 16;
                    if (c < d.Ns)
                        ch[u] = *(const v4a*)(vb + (int64_t)c * d.v_sk + n);
                }
            }
#pragma unroll
            for (int u = 0; u < QA_ATT_U; ++u) {
                const int e = e0 + u * 256;
                if (e < nk) {
                    const int r = e / cpr, c = (e - r * cpr) * 16;
                    *(v4a*)(sk + r * g.RSK + c) = ch[u];
                } else if (e < nch) {
                    const int f = e - nk;
                    const int c = f / nvr, n = (f - c * nvr) * 16;
                    const int8_t* bt = (const int8_t*)&ch[u];
#pragma unroll
                    for (int j = 0; j < 16; ++j)
                        sv[(n + j) * g.RSV + c] = bt[j];
                }
            }
        }
    }
    __syncthreads();

    // the wave's tile: S as columns of 16 row bytes (column n at 16 n, so a
    // lane's 4 rows 4 kg + r of a column are one word), then P over it as
    // rows of RSV bytes (P's columns past N_S meet v^T's zero rows)
    int8_t* pw = sp + wave * 16 * g.RSV;
    const int nts = g.NpS >> 4;
    const int ksv = g.KpV >> 6, dts = g.NV >> 4;
    int8_t* const yb = d.y + b0 * d.y_s0 + b1 * d.y_s1;

    for (int rt = rt0 + wave; rt < rt1; rt += 4) {
        const int64_t m0 = (int64_t)rt * 16;  // the tile's first row
        if (rt != rt0 + wave) load_q(rt);  // a later tile of the wave
        // ---- S quantized a 16 x 16 block at a time: the stored bytes +
        // 128 of the lane's 4 rows, one word a column ----
        for (int nt0 = 0; nt0 < nts; nt0 += 4) {  // 4 blocks at a time
            v4a acc[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                acc[u] = v4a{0, 0, 0, 0};
                const int nt = min(nt0 + u, nts - 1);
#pragma unroll
                for (int ks = 0; ks < QA_ATT_KSQ; ++ks)
                    if (ks < ksq)
                        acc[u] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                            fa[ks],
                            *(const v4a*)(sk + (nt * 16 + col) * g.RSK +
                                          ks * 64 + kg * 16),
                            acc[u], 0, 0, 0);
            }
            float yf[4][4];
            int qv[4][4];
            uint32_t slow = 0;  // bit 4 u + r: the double form
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    bool sl;
                    yf[u][r] = (float)((double)acc[u][r] * d.sS);
                    qv[u][r] = quant_fast(yf[u][r], d.S, &sl);
                    slow |= (uint32_t)sl << (4 * u + r);
                }
            if (slow) {
#pragma unroll
                for (int u = 0; u < 4; ++u)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if ((slow >> (4 * u + r)) & 1)
                            qv[u][r] = quant_slow(yf[u][r], d.S);
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int n = (nt0 + u) * 16 + col;
                if (nt0 + u < nts && n < d.Ns) {
                    uint32_t w = 0;
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        w |= (uint32_t)((qv[u][r] - d.S.so + 128) & 255)
                             << (8 * r);
                    *(uint32_t*)(pw + n * 16 + 4 * kg) = w;
                }
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        uint32_t sw[16];  // S words of the lane's columns (0: past N_S)
        int mx[4] = {0, 0, 0, 0};
#pragma unroll
        for (int nt = 0; nt < 16; ++nt) {
            const bool live = nt < nts && nt * 16 + col < d.Ns;
            sw[nt] = live ? *(const uint32_t*)(pw + (nt * 16 + col) * 16 +
                                               4 * kg)
                          : 0u;
#pragma unroll
            for (int r = 0; r < 4; ++r)
                if (live) mx[r] = max(mx[r], (int)((sw[nt] >> (8 * r)) & 255));
        }
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int o = 8; o > 0; o >>= 1)
                mx[r] = max(mx[r], __shfl_xor(mx[r], o));
        // ---- the Softmax, two rows at a time (their table reads in
        // flight together); P over the tile ----
#pragma unroll 1
        for (int r0 = 0; r0 < 4; r0 += 2) {
            double e[2][16], sum[2] = {0.0, 0.0};
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int m = r0 + h == 0 ? mx[0] : r0 + h == 1 ? mx[1]
                            : r0 + h == 2 ? mx[2] : mx[3];
                const double* tr = d.table + 256 * m;
#pragma unroll
                for (int nt = 0; nt < 16; ++nt) {
                    const bool live = nt < nts && nt * 16 + col < d.Ns;
                    e[h][nt] = live ? tr[(sw[nt] >> (8 * (r0 + h))) & 255]
                                    : 0.0;
                }
            }
#pragma unroll
            for (int h = 0; h < 2; ++h) {
#pragma unroll
                for (int nt = 0; nt < 16; ++nt) sum[h] += e[h][nt];
#pragma unroll
                for (int o = 8; o > 0; o >>= 1)
                    sum[h] += __shfl_xor(sum[h], o);
                const double rsum = 1.0 / sum[h];  // one division a row
                int8_t* prow = pw + (4 * kg + r0 + h) * g.RSV;
                float yp[16];
                int qp[16];
                uint32_t slow = 0;
#pragma unroll
                for (int nt = 0; nt < 16; ++nt) {
                    bool sl;
                    yp[nt] = (float)(e[h][nt] * rsum);
                    qp[nt] = quant_fast(yp[nt], d.P, &sl);
                    slow |= (uint32_t)sl << nt;
                }
                if (slow) {
#pragma unroll
                    for (int nt = 0; nt < 16; ++nt)
                        if ((slow >> nt) & 1) qp[nt] = quant_slow(yp[nt], d.P);
                }
#pragma unroll
                for (int nt = 0; nt < 16; ++nt)
                    if (nt < nts && nt * 16 + col < d.Ns)
                        prow[nt * 16 + col] = (int8_t)(qp[nt] - d.P.so);
            }
        }
        // the wave's P bytes before its reads of them
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        // ---- O = P v: 16 rows x NV columns, 4 blocks at a time ----
        for (int dt0 = 0; dt0 < dts; dt0 += 4) {
            v4a acc2[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                acc2[u] = v4a{0, 0, 0, 0};
                const int dt = min(dt0 + u, dts - 1);
                for (int ks = 0; ks < ksv; ++ks) {
                    const int c = ks * 64 + kg * 16;
                    acc2[u] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                        *(const v4a*)(pw + col * g.RSV + c),
                        *(const v4a*)(sv + (dt * 16 + col) * g.RSV + c),
                        acc2[u], 0, 0, 0);
                }
            }
            float yo[4][4];
            int qo[4][4];
            uint32_t slow = 0;
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    bool sl;
                    yo[u][r] = (float)((double)acc2[u][r] * d.sO);
                    qo[u][r] = quant_fast(yo[u][r], d.O, &sl);
                    slow |= (uint32_t)sl << (4 * u + r);
                }
            if (slow) {
#pragma unroll
                for (int u = 0; u < 4; ++u)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if ((slow >> (4 * u + r)) & 1)
                            qo[u][r] = quant_slow(yo[u][r], d.O);
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int n = (dt0 + u) * 16 + col;
                if (dt0 + u >= dts || n >= d.No) continue;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int64_t m = m0 + 4 * kg + r;
                    if (m < d.M)
                        yb[m * d.y_sm + n * d.y_sn] =
                            (int8_t)(qo[u][r] - d.O.so);
                }
            }
        }
        // this tile's reads of P before the next tile's S words
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
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
    }
    if (*why) return false;
    g->NpS = (int)round_up(qk.N, 16);
    g->KpQ = (int)round_up(qk.K, 64);
    g->KpV = (int)round_up(qk.N, 64);
    g->NV = (int)round_up(av.N, 16);
    g->RSK = g->KpQ + 16;
    g->RSV = g->KpV + 16;
    g->tiles = (int)ceil_div(qk.M, 16);
    // one 16-row tile per wave
    g->tpw = 4;
    // k rows and v^T rows once per work-group, an S / P tile per wave (S
    // as NpS columns of 16 bytes, or P as 16 rows of RSV bytes)
    *lds = (int64_t)g->NpS * g->RSK + (int64_t)g->NV * g->RSV +
           4LL * std::max(16 * g->RSV, 16 * g->NpS);
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
        c.f32 = qa_f32_form_ok(scale, zp, qmin, qmax) ? 1 : 0;
        c.tie = qa_f32_tie(zp, qmin, qmax);
        c.zpf = (float)zp;
        c.qminf = (float)qmin;
        c.qmaxf = (float)qmax;
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
    a.sS = qk.a_scale * qk.b_scale;
    a.sO = av.a_scale * av.b_scale;
    a.S = qc(qk.out_scale, qk.out_zp, qk.qmin, qk.qmax, qk.y_so);
    a.P = qc(d->p_scale, d->p_zp, d->p_qmin, d->p_qmax, d->p_so);
    a.O = qc(av.out_scale, av.out_zp, av.qmin, av.qmax, av.y_so);
    const dim3 grid((unsigned)ceil_div(g.tiles, g.tpw),
                    (unsigned)(qk.B0 * qk.B1));
    k_attention<<<grid, 256, (size_t)lds, (hipStream_t)stream>>>(a, g);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_hip_error("qa_d_attention", e);
        return -1;
    }
    return 0;
}

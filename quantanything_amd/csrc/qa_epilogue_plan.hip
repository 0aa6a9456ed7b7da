// Host-side planner of the int8 table epilogue (plan layout: qa_conv.h).
//
// The fused conv epilogue of the reference chain
//   q = clip(mbqm(acc + bias, M, shift) + zp, qmin, qmax)     requantize
//   q = lut[clip(q - offset, 0, len-1)]                         activation
//   q = clip(mbqm(a - za) + sign*mbqm(b - zb) + zp_add, ...)   residual Add
// (quantization/kernels/qa_kernels.cpp:188-230, :348-361, :319-332) is a
// 128-bit computation per element. For int8 outputs only the first step
// depends on the accumulator: it becomes one int64 multiply-add and shift
// with per-channel constants, and every later step is a function of at most
// 256 values, tabulated here with the same 128-bit arithmetic.
#include <string.h>

#include "../../include/qa_hip.h"
#include "qa_conv.h"

namespace {

using qa::PLAN_CH;
using qa::PLAN_E;
using qa::PLAN_TC;
using qa::PLAN_TR;

constexpr int64_t TERM_LIMIT = (int64_t)1 << 28;

inline int64_t rescale_q(const qa_epi_params* p, int64_t q) {
    return qa_clip128(qa_mbqm(q - p->r2_zp_in, p->r2_m, p->r2_s) +
                          p->r2_zp_out,
                      p->r2_qmin, p->r2_qmax);
}

// stored output byte (bits 0..7) and stored rescaled-copy byte (8..15)
inline int32_t entry(const qa_epi_params* p, int64_t q) {
    uint32_t e = (uint8_t)(int8_t)(q - p->y_so);
    if (p->has_y2) e |= (uint32_t)(uint8_t)(int8_t)(rescale_q(p, q) - p->y_so)
                        << 8;
    return (int32_t)e;
}

// One Add operand term: mbqm(v - z, m, s), times `sign` for the second one.
inline bool add_term(qa_i128 t, int64_t* out) {
    if (t > TERM_LIMIT || t < -TERM_LIMIT) return false;
    *out = (int64_t)t;
    return true;
}

}  // namespace

QA_API int64_t qa_epi_plan_bytes(int64_t cout) {
    return cout < 0 ? -1 : PLAN_CH + 16 * cout;
}

QA_API int qa_plan_epilogue_i8(const qa_epi_params* p, void* plan_) {
    if (!p || !plan_ || p->cout <= 0 || !p->mult || !p->shift) return -1;
    if (p->lut && p->lut_len <= 0) return -1;
    if (p->qmin > p->qmax || p->qmax - p->qmin > 255) return 0;
    const int64_t A = p->qmin - p->zp, B = p->qmax - p->zp;
    if (A < INT32_MIN || B > INT32_MAX) return 0;
    uint8_t* plan = (uint8_t*)plan_;
    memset(plan, 0, (size_t)qa_epi_plan_bytes(p->cout));
    int32_t* hd = (int32_t*)plan;
    int32_t* E = (int32_t*)(plan + PLAN_E);
    int32_t* TC = (int32_t*)(plan + PLAN_TC);
    int32_t* TR = (int32_t*)(plan + PLAN_TR);
    int32_t* ch = (int32_t*)(plan + PLAN_CH);

    // ---- per channel: q0 = (w*m + c) >> t for every int32 w -------------
    const qa_i128 w_max = (qa_i128)1 << 31;  // |w| <= 2^31
    for (int64_t c = 0; c < p->cout; ++c) {
        const int64_t m = p->mult[c];
        const int64_t t = 31 + p->shift[c];
        if (t < 1 || t > 62 || m < INT32_MIN || m > INT32_MAX) return 0;
        const int64_t pre = p->pre_bias ? p->pre_bias[c] : 0;
        const qa_i128 cc = (qa_i128)pre * m + ((qa_i128)1 << (t - 1));
        const qa_i128 am = m < 0 ? -(qa_i128)m : (qa_i128)m;
        const qa_i128 bound = w_max * am + (cc < 0 ? -cc : cc);
        // the multiply-add stays in int64 and the shifted value in int32
        if (bound >= ((qa_i128)1 << 63) || bound >= ((qa_i128)1 << (31 + t)))
            return 0;
        const uint64_t cu = (uint64_t)(int64_t)cc;
        ch[4 * c + 0] = (int32_t)m;
        ch[4 * c + 1] = (int32_t)t;
        ch[4 * c + 2] = (int32_t)(uint32_t)cu;
        ch[4 * c + 3] = (int32_t)(uint32_t)(cu >> 32);
    }

    // ---- tables over i = q - qmin -----------------------------------------
    const int64_t levels = p->qmax - p->qmin + 1;
    int64_t sh = 0;
    if (p->has_res) {
        if (p->add_qmin > p->add_qmax || p->add_qmax - p->add_qmin > 255)
            return 0;
        sh = p->add_qmax - p->add_qmin;
    }
    for (int64_t i = 0; i < levels; ++i) {
        int64_t q = p->qmin + i;
        if (p->lut) {
            int64_t k = q - p->lut_offset;
            k = k < 0 ? 0 : (k >= p->lut_len ? p->lut_len - 1 : k);
            q = p->lut[k];
        }
        if (!p->has_res) {
            E[i] = entry(p, q);
            continue;
        }
        const qa_i128 t =
            p->res_first ? (qa_i128)p->add_sign * qa_mbqm(q - p->zb, p->mb,
                                                          p->sb)
                         : qa_mbqm(q - p->za, p->ma, p->sa);
        int64_t v;
        if (!add_term(t + p->add_zp - p->add_qmin, &v)) return 0;
        TC[i] = (int32_t)v;
    }
    if (p->has_res) {
        for (int u = 0; u < 256; ++u) {  // stored residual byte u
            const int64_t r = (int64_t)(int8_t)(uint8_t)u + p->res_so;
            const qa_i128 t =
                p->res_first ? qa_mbqm(r - p->za, p->ma, p->sa)
                             : (qa_i128)p->add_sign *
                                   qa_mbqm(r - p->zb, p->mb, p->sb);
            int64_t v;
            if (!add_term(t, &v)) return 0;
            TR[u] = (int32_t)v;
        }
        for (int64_t s = 0; s <= sh; ++s) E[s] = entry(p, p->add_qmin + s);
    }
    hd[0] = (int32_t)A;
    hd[1] = (int32_t)B;
    hd[2] = (int32_t)sh;
    hd[3] = (p->has_res ? qa::PLAN_RES : 0) | (p->has_y2 ? qa::PLAN_Y2 : 0);
    if (!p->has_res && !p->has_y2 && !p->lut) {
        hd[3] |= qa::PLAN_IDENT;
        hd[4] = (int32_t)(p->zp - p->y_so);
    }
    return 1;
}

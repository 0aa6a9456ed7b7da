// Shared epilogue of the conv / GEMM kernels: requantize, optional lookup
// table, optional residual Add, all exact (qa_common.h).
#pragma once

#include "qa_igemm.h"

namespace qa {

// Requantize + LUT + residual add of one accumulator (EPI_QUANT).
__device__ __forceinline__ int64_t quant_one(const IgemmArgs& a, int64_t v,
                                             int64_t m, int64_t s,
                                             int64_t res_q, bool has_res) {
    int64_t q = qa_clip128(qa_mbqm_fast(v, m, s) + a.zp, a.qmin, a.qmax);
    if (a.lut) {
        int64_t idx = q - a.lut_off;
        idx = idx < 0 ? 0 : (idx >= a.lut_len ? a.lut_len - 1 : idx);
        q = a.lut[idx];
    }
    if (has_res) {
        const int64_t first = a.res_first ? res_q : q;
        const int64_t second = a.res_first ? q : res_q;
        const qa_i128 t = qa_mbqm_fast(first - a.za, a.ma, a.sa) +
                          (qa_i128)a.add_sign *
                              qa_mbqm_fast(second - a.zb, a.mb, a.sb) +
                          a.add_zp;
        q = qa_clip128(t, a.add_qmin, a.add_qmax);
    }
    return q;
}

}  // namespace qa

// Integer Add / Sub / Mul with NumPy broadcasting over up to six axes, for
// operand shapes that the row kernels of qa_elementwise.hip (equal shapes,
// or one operand of batch 1) do not cover: a per-channel or per-column
// constant, [N, C, H, W] against [N, C, 1, 1], strided views. The reference
// broadcasts both operands to the output shape, then runs qa_add / qa_mul
// element by element (quantization/native.py:465-500, qa_kernels.cpp:346-386);
// the arithmetic here is the same per element:
//   add: clip(mbqm(a - za, ma, sa) + sign * mbqm(b - zb, mb, sb) + zp)
//   mul: clip(mbqm((a - za) * (b - zb), m, s) + zp)
// Operands and output are stored values (q - so) of any storage code; a
// broadcast axis has stride 0. One thread per output element.
#include <algorithm>

#include "../../include/qa_hip.h"
#include "qa_conv.h"

namespace qa {
namespace {

constexpr int kThreads = 256;

template <int OP>
__global__ __launch_bounds__(kThreads) void k_binary_nd(qa_binary_nd d,
                                                        int64_t total) {
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * kThreads) {
        int64_t rem = i, ao = 0, bo = 0, yo = 0;
        for (int k = (int)d.ndim - 1; k >= 0; --k) {
            const int64_t c = rem % d.shape[k];
            rem /= d.shape[k];
            ao += c * d.as[k];
            bo += c * d.bs[k];
            yo += c * d.ys[k];
        }
        const int64_t a = load_any(d.a, (int)d.a_code, ao) + d.a_so - d.za;
        const int64_t b = load_any(d.b, (int)d.b_code, bo) + d.b_so - d.zb;
        qa_i128 v;
        if (OP == 0)
            v = qa_mbqm_fast(a, d.ma, d.sa) +
                (qa_i128)d.sign * qa_mbqm_fast(b, d.mb, d.sb) + d.zp_out;
        else
            v = qa_mbqm_fast(a * b, d.ma, d.sa) + d.zp_out;
        store_any(d.y, (int)d.y_code, yo,
                  qa_clip128(v, d.qmin, d.qmax) - d.y_so);
    }
}

bool code_ok(int64_t c) { return c == 1 || c == 2 || c == 4; }

}  // namespace
}  // namespace qa

using namespace qa;

QA_API int qa_d_binary_nd(const qa_binary_nd* d, void* stream) {
    if (!d || d->ndim < 1 || d->ndim > 6 || !code_ok(d->a_code) ||
        !code_ok(d->b_code) || !code_ok(d->y_code) || d->op < 0 ||
        d->op > 1) {
        set_error("qa_d_binary_nd", "bad descriptor");
        return -1;
    }
    int64_t total = 1;
    for (int k = 0; k < d->ndim; ++k) {
        if (d->shape[k] < 0) {
            set_error("qa_d_binary_nd", "negative extent");
            return -1;
        }
        total *= d->shape[k];
    }
    if (total == 0) return 0;
    if (!d->a || !d->b || !d->y) {
        set_error("qa_d_binary_nd", "null tensor");
        return -1;
    }
    const unsigned g = (unsigned)std::min<int64_t>(ceil_div(total, kThreads),
                                                   1 << 16);
    hipStream_t st = (hipStream_t)stream;
    if (d->op == 0)
        k_binary_nd<0><<<g, kThreads, 0, st>>>(*d, total);
    else
        k_binary_nd<1><<<g, kThreads, 0, st>>>(*d, total);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_hip_error("qa_d_binary_nd", e);
        return -1;
    }
    return 0;
}

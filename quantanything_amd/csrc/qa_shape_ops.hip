// Integer shaping operators whose output parameters are the input's, so they
// move stored values without arithmetic (quant_layers.py:593-650):
//   Pad with the zero point           (float_ops.py:499-513, pad_value = zp)
//   MaxPool with qmin as padding      (float_ops.py:518-560, pad_value = qmin)
//   GlobalMaxPool                     (float_ops.py:586-589)
// Stored values (q - so) of any storage code; the padding value arrives as a
// stored value too.
#include <algorithm>

#include "../../include/qa_hip.h"
#include "qa_common.h"

namespace qa {
namespace {

constexpr int kThreads = 256;

template <class T>
__global__ __launch_bounds__(kThreads) void k_pad_nd(qa_nd_pad d,
                                                     int64_t total) {
    const T fill = (T)d.fill;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * kThreads) {
        int64_t rem = i, xo = 0, yo = 0;
        bool inside = true;
        for (int k = (int)d.ndim - 1; k >= 0; --k) {
            const int64_t c = rem % d.shape[k];
            rem /= d.shape[k];
            yo += c * d.ys[k];
            const int64_t src = c - d.lo[k];
            inside = inside && src >= 0 && src < d.xshape[k];
            xo += src * d.xs[k];
        }
        ((T*)d.y)[yo] = inside ? ((const T*)d.x)[xo] : fill;
    }
}

// One output element per thread, channels fastest (coalesced on
// channels-last tensors). A window tap outside the image contributes the
// padding value, as the reference's padded array does.
template <class T>
__global__ __launch_bounds__(kThreads) void k_maxpool(qa_maxpool_desc d,
                                                      int64_t total) {
    const T* x = (const T*)d.x;
    T* y = (T*)d.y;
    const int pad = (int)d.pad;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * kThreads) {
        const int64_t c = i % d.C;
        int64_t r = i / d.C;
        const int64_t ox = r % d.OW;
        r /= d.OW;
        const int64_t oy = r % d.OH;
        const int64_t n = r / d.OH;
        const T* xb = x + n * d.x_sn + c * d.x_sc;
        int acc = INT32_MIN;
        for (int64_t ky = 0; ky < d.KH; ++ky) {
            const int64_t iy = oy * d.SH - d.PT + ky * d.DH;
            const bool row_in = iy >= 0 && iy < d.H;
            for (int64_t kx = 0; kx < d.KW; ++kx) {
                const int64_t ix = ox * d.SW - d.PL + kx * d.DW;
                const int v = (row_in && ix >= 0 && ix < d.W)
                                  ? (int)xb[iy * d.x_sh + ix * d.x_sw]
                                  : pad;
                acc = max(acc, v);
            }
        }
        y[n * d.y_sn + c * d.y_sc + oy * d.y_sh + ox * d.y_sw] = (T)acc;
    }
}

bool code_ok(int64_t c) { return c == 1 || c == 2 || c == 4; }

unsigned blocks_for(int64_t total) {
    return (unsigned)std::min<int64_t>(ceil_div(total, kThreads), 1 << 16);
}

bool launched(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_hip_error(what, e);
        return false;
    }
    return true;
}

}  // namespace
}  // namespace qa

using namespace qa;

QA_API int qa_d_pad_nd(const qa_nd_pad* d, void* stream) {
    if (!d || d->ndim < 1 || d->ndim > 6 || !code_ok(d->code)) {
        set_error("qa_d_pad_nd", "bad descriptor");
        return -1;
    }
    int64_t total = 1;
    for (int k = 0; k < d->ndim; ++k) {
        if (d->shape[k] < 0 || d->xshape[k] < 0 || d->lo[k] < 0) {
            set_error("qa_d_pad_nd", "negative extent or padding");
            return -1;
        }
        total *= d->shape[k];
    }
    if (total == 0) return 0;
    if (!d->x || !d->y) {
        set_error("qa_d_pad_nd", "null tensor");
        return -1;
    }
    hipStream_t st = (hipStream_t)stream;
    const unsigned nb = blocks_for(total);
    switch (d->code) {
        case 1: k_pad_nd<int8_t><<<nb, kThreads, 0, st>>>(*d, total); break;
        case 2: k_pad_nd<int16_t><<<nb, kThreads, 0, st>>>(*d, total); break;
        default: k_pad_nd<int32_t><<<nb, kThreads, 0, st>>>(*d, total);
    }
    return launched("qa_d_pad_nd") ? 0 : -1;
}

QA_API int qa_d_maxpool(const qa_maxpool_desc* d, void* stream) {
    if (!d || !code_ok(d->code) || d->N < 0 || d->C < 0 || d->H < 0 ||
        d->W < 0 || d->OH < 0 || d->OW < 0 || d->KH < 1 || d->KW < 1 ||
        d->SH < 1 || d->SW < 1 || d->DH < 1 || d->DW < 1) {
        set_error("qa_d_maxpool", "bad descriptor");
        return -1;
    }
    const int64_t total = d->N * d->C * d->OH * d->OW;
    if (total == 0) return 0;
    if (!d->x || !d->y) {
        set_error("qa_d_maxpool", "null tensor");
        return -1;
    }
    hipStream_t st = (hipStream_t)stream;
    const unsigned nb = blocks_for(total);
    switch (d->code) {
        case 1: k_maxpool<int8_t><<<nb, kThreads, 0, st>>>(*d, total); break;
        case 2: k_maxpool<int16_t><<<nb, kThreads, 0, st>>>(*d, total); break;
        default: k_maxpool<int32_t><<<nb, kThreads, 0, st>>>(*d, total);
    }
    return launched("qa_d_maxpool") ? 0 : -1;
}

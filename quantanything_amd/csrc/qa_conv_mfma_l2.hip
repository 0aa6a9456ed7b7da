// int8 MFMA convolution / GEMM: the variants that read weights from L2
// (kernel templates: qa_conv_mfma.h; tile choice: qa_conv_mfma.hip).
#include "qa_conv_mfma.h"

namespace qa {

bool mfma_launch_l2(const ConvArgs& b, int wm, bool split, int epi,
                    hipStream_t st) {
    return launch_variant<false>(b, wm, split, epi, st);
}

}  // namespace qa

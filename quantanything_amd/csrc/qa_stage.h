// Staging of int8 operand rows into LDS for the activation-MatMul kernels
// (one 256-thread work-group cooperating).
#pragma once

#include "qa_common.h"

namespace qa {

constexpr int QA_STAGE_THREADS = 256;

// Rows [r0, r0 + rows) of an operand, element (r, c) at src[r * rs + c * ks]
// for c < K, to dst[r * RS + c] for c < Kp (Kp a multiple of 16), zero past
// rlim rows and K columns: 16-byte loads along a unit-stride axis when it is
// aligned, else byte loads, several in flight per thread.
__device__ inline void stage_i8_rows(int8_t* dst, int RS, const int8_t* src,
                                     int rows, int64_t r0, int64_t rlim,
                                     int64_t rs, int64_t ks, int64_t K, int Kp,
                                     int tid) {
    const bool al = ((uintptr_t)src & 15) == 0;
    constexpr int U = 4;  // loads in flight per thread
    if (ks == 1 && al && rs % 16 == 0 && K % 16 == 0) {
        const int cpr = Kp / 16;  // 16-byte chunks per row
        const int n16 = rows * cpr;
        for (int e0 = tid; e0 < n16; e0 += U * QA_STAGE_THREADS) {
            int4 v[U];
            int at[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int e = e0 + u * QA_STAGE_THREADS;
                const int r = e / cpr, c = (e - r * cpr) * 16;
                const int64_t rr = r0 + r;
                v[u] = int4{0, 0, 0, 0};
                at[u] = e < n16 ? r * RS + c : -1;
                if (e < n16 && rr < rlim && c < K)
                    v[u] = *(const int4*)(src + rr * rs + c);
            }
#pragma unroll
            for (int u = 0; u < U; ++u)
                if (at[u] >= 0) *(int4*)(dst + at[u]) = v[u];
        }
        return;
    }
    if (rs == 1 && al && ks % 16 == 0 && rows % 16 == 0 &&
        (r0 + rows <= rlim || rlim % 16 == 0)) {
        // 16 consecutive rows of one column per load, scattered to LDS
        const int rpc = rows / 16;
        const int n16 = rpc * Kp;
        for (int e0 = tid; e0 < n16; e0 += U * QA_STAGE_THREADS) {
            int4 v[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int e = e0 + u * QA_STAGE_THREADS;
                const int c = e / rpc, r = (e - c * rpc) * 16;
                const int64_t rr = r0 + r;
                v[u] = int4{0, 0, 0, 0};
                if (e < n16 && rr < rlim && c < K)
                    v[u] = *(const int4*)(src + rr + (int64_t)c * ks);
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int e = e0 + u * QA_STAGE_THREADS;
                if (e >= n16) continue;
                const int c = e / rpc, r = (e - c * rpc) * 16;
                const int8_t* b = (const int8_t*)&v[u];
#pragma unroll
                for (int j = 0; j < 16; ++j) dst[(r + j) * RS + c] = b[j];
            }
        }
        return;
    }
    const int n = rows * Kp;
    for (int e0 = tid; e0 < n; e0 += 8 * QA_STAGE_THREADS) {
        int8_t v[8];
        int at[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int e = e0 + j * QA_STAGE_THREADS;
            int r = e / Kp, c = e - r * Kp;
            if (ks != 1) {
                c = e / rows;
                r = e - c * rows;
            }
            const int64_t rr = r0 + r;
            at[j] = e < n ? r * RS + c : -1;
            v[j] = (e < n && rr < rlim && c < K)
                       ? src[rr * rs + (int64_t)c * ks]
                       : 0;
        }
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (at[j] >= 0) dst[at[j]] = v[j];
    }
}

}  // namespace qa

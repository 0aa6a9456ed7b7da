// Allocation-free variant of the narrow integer GEMM (qa_gemm_i16_i32):
// qa_gemm_i16_i32_noalloc. The caller passes device-resident A, B and C and
// a stream; every buffer the computation needs beyond them (the activation
// range, the int8-packed operands, the per-column correction terms and the
// path flag) lives in one file-scope device array of fixed size, so the call
// makes no hipMalloc / hipFree and no host synchronisation: it can run inside
// HIP graph capture or a serving loop that must not allocate.
//
// The path (int8 MFMA with zero-point correction terms, or the exact VALU
// GEMM when an operand's range spans more than 256 values) is decided on the
// device from the data: both kernels are launched and each returns at once
// unless the flag in the scratch header selects it.
//
// The array is shared by every call on a GPU and keeps the last call's
// contents: each call re-initialises the header it reads. Calls that
// overlap on one GPU (two streams, two threads) race on it.
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <mutex>

#include "../../include/qa_hip.h"
#include "qa_conv.h"
#include "qa_valu.h"

namespace {

constexpr size_t kNoAllocBytes = (size_t)32 << 20;

}  // namespace

// One per GPU, held from module load until the process ends.
static __device__ __align__(256) unsigned char scratch[kNoAllocBytes];

namespace qa {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxDevices = 16;
constexpr int64_t kHeader = 256;  // int32 header: lo, hi, use_valu, a_off
constexpr int64_t kTail = 64;     // slack after the packed activations
constexpr int64_t kRowPad = 128;  // packed weight rows: multiple of 128

std::once_flag g_once[kMaxDevices];
void* g_ptr[kMaxDevices];
hipError_t g_err[kMaxDevices];

// Device address of `scratch` on the current device (looked up once per
// device; the array's host-side name is not a device address).
void* scratch_base() {
    int d = 0;
    if (hipGetDevice(&d) != hipSuccess || d < 0 || d >= kMaxDevices) {
        set_error("qa_gemm_i16_i32_noalloc", "no current device");
        return nullptr;
    }
    std::call_once(g_once[d], [d] {
        void* p = nullptr;
        g_err[d] = hipGetSymbolAddress(&p, HIP_SYMBOL(::scratch));
        g_ptr[d] = g_err[d] == hipSuccess ? p : nullptr;
    });
    if (!g_ptr[d]) {
        set_hip_error("hipGetSymbolAddress(scratch)", g_err[d]);
        return nullptr;
    }
    return g_ptr[d];
}

// Header: [0] lo, [1] hi of A, [2] use_valu, [3] a_off. force_valu sets the
// flag from the start (problems outside the MFMA path's limits).
__global__ void k_na_begin(int32_t* hdr, int32_t force_valu) {
    if (threadIdx.x == 0) {
        hdr[0] = INT32_MAX;
        hdr[1] = INT32_MIN;
        hdr[2] = force_valu;
        hdr[3] = 0;
    }
}

__global__ __launch_bounds__(kThreads) void k_na_range(const int16_t* x,
                                                       int64_t n,
                                                       int32_t* hdr) {
    int lo = INT32_MAX, hi = INT32_MIN;
    const int64_t step = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += step) {
        const int v = x[i];
        lo = min(lo, v);
        hi = max(hi, v);
    }
    for (int off = 32; off > 0; off >>= 1) {
        lo = min(lo, __shfl_xor(lo, off));
        hi = max(hi, __shfl_xor(hi, off));
    }
    if ((threadIdx.x & 63) == 0) {
        atomicMin(&hdr[0], lo);
        atomicMax(&hdr[1], hi);
    }
}

// Work-group sum / min / max over 256 threads (4 waves).
template <class T, class Op>
__device__ T block_reduce(T v, Op op, T* red) {
    for (int off = 32; off > 0; off >>= 1) v = op(v, __shfl_xor(v, off));
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return op(op(red[0], red[1]), op(red[2], red[3]));
}

// One work-group per packed weight row r (= output column of B): the
// column's offset b (so that B[:, r] - b fits int8), its int8 row
// [k-groups of 16 bytes, zero past K] and the sum of the offset values.
// Rows past N are zero. A column whose values span more than 256 sets the
// VALU flag.
__global__ __launch_bounds__(kThreads) void k_na_pack_b(
    const int16_t* B, int64_t K, int64_t N, int64_t rowbytes, int8_t* wp,
    int32_t* boff, int64_t* colsum, int32_t* hdr) {
    __shared__ int s_i[4];
    __shared__ long long s_l[4];
    const int64_t r = blockIdx.x;
    int8_t* dst = wp + r * rowbytes;
    if (r >= N) {
        for (int64_t j = threadIdx.x; j < rowbytes; j += kThreads) dst[j] = 0;
        return;
    }
    int lo = INT32_MAX, hi = INT32_MIN;
    for (int64_t k = threadIdx.x; k < K; k += kThreads) {
        const int v = B[k * N + r];
        lo = min(lo, v);
        hi = max(hi, v);
    }
    auto mn = [](int a, int b) { return min(a, b); };
    auto mx = [](int a, int b) { return max(a, b); };
    lo = block_reduce(lo, mn, s_i);
    hi = block_reduce(hi, mx, s_i);
    if (K == 0) lo = hi = 0;
    const bool fits = (int64_t)hi - lo <= 255;
    const int b = (lo >= -128 && hi <= 127) ? 0 : lo + 128;
    if (!fits && threadIdx.x == 0) atomicOr(&hdr[2], 1);
    long long s = 0;
    for (int64_t j = threadIdx.x; j < rowbytes; j += kThreads) {
        const int v = j < K ? (int)B[j * N + r] - b : 0;
        dst[j] = (int8_t)v;
        s += v;
    }
    auto add = [](long long a, long long c) { return a + c; };
    s = block_reduce(s, add, s_l);
    if (threadIdx.x == 0) {
        boff[r] = b;
        colsum[r] = s;
    }
}

// The activation offset from A's range (0 included) and the per-column
// correction corr = a_off * colsum + K * a_off * b_off, in place over colsum.
__global__ __launch_bounds__(kThreads) void k_na_finish(int64_t* corr,
                                                        const int32_t* boff,
                                                        int64_t N, int64_t K,
                                                        int32_t* hdr) {
    const int lo = min(hdr[0], 0), hi = max(hdr[1], 0);
    const bool fits = (int64_t)hi - lo <= 255;
    const int a_off = !fits ? 0 : (lo >= -128 && hi <= 127) ? 0 : lo + 128;
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        hdr[3] = a_off;
        if (!fits) atomicOr(&hdr[2], 1);
    }
    const int64_t n = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (n < N) corr[n] = a_off * corr[n] + K * a_off * (int64_t)boff[n];
}

// A[M][K] -> int8 [M][Kp] (A - a_off, zero past K) plus a zero tail; skipped
// on the VALU path.
__global__ __launch_bounds__(kThreads) void k_na_pack_a(const int16_t* A,
                                                        int8_t* y, int64_t M,
                                                        int64_t K, int64_t Kp,
                                                        const int32_t* hdr) {
    if (hdr[2] != 0) return;
    const int a_off = hdr[3];
    const int64_t n = M * Kp + kTail;
    const int64_t step = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += step) {
        const int64_t m = i / Kp, k = i - m * Kp;
        y[i] = (m < M && k < K) ? (int8_t)((int)A[m * K + k] - a_off)
                                : (int8_t)0;
    }
}

__global__ __launch_bounds__(kThreads) void k_na_zero(int32_t* c, int64_t n) {
    const int64_t step = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += step)
        c[i] = 0;
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

QA_API int64_t qa_noalloc_scratch_bytes(void) { return (int64_t)kNoAllocBytes; }

// Whether the int8 MFMA path can take the problem: exact int32 sums
// (K < 2^17) and a channel-block grid within 65535.
static bool na_mfma_ok(int64_t N, int64_t K) {
    return K < 131072 && ceil_div(N, 16) <= 65535;
}

QA_API int64_t qa_gemm_i16_i32_noalloc_need(int64_t M, int64_t N, int64_t K) {
    if (M < 0 || N < 0 || K < 0) return -1;
    if (!na_mfma_ok(N, K)) return kHeader;  // VALU path: the header only
    const int64_t KGp = round_up(std::max<int64_t>(ceil_div(K, 16), 1), 4);
    const int64_t rows = round_up(std::max<int64_t>(N, 1), kRowPad);
    const int64_t Kp = round_up(K, 16);
    return kHeader + round_up(N * 8, 256) + round_up(N * 4, 256) +
           round_up(rows * KGp * 16, 256) + M * Kp + kTail;
}

QA_API int qa_gemm_i16_i32_noalloc(int64_t M, int64_t N, int64_t K,
                                   const int16_t* A, const int16_t* B,
                                   int32_t* C, void* stream_) {
    const char* who = "qa_gemm_i16_i32_noalloc";
    hipStream_t st = (hipStream_t)stream_;
    (void)hipGetLastError();
    const int64_t lim = (int64_t)1 << 31;
    if (M < 0 || N < 0 || K < 0 || M >= lim || N >= lim || K >= lim) {
        set_error(who, "dimension outside [0, 2^31)");
        return -1;
    }
    if (M == 0 || N == 0) return 0;
    if (!C || (K > 0 && (!A || !B))) {
        set_error(who, "null operand");
        return -1;
    }
    if (K == 0) {
        k_na_zero<<<grid_1d(M * N, kThreads, 1 << 16), kThreads, 0, st>>>(
            C, M * N);
        return launched("k_na_zero") ? 0 : -1;
    }
    const int64_t need = qa_gemm_i16_i32_noalloc_need(M, N, K);
    if (need > (int64_t)kNoAllocBytes) {
        char msg[160];
        snprintf(msg, sizeof(msg),
                 "problem needs %lld bytes of scratch; the maximum is %lld",
                 (long long)need, (long long)kNoAllocBytes);
        set_error(who, msg);
        return -1;
    }
    char* base = (char*)scratch_base();
    if (!base) return -1;
    const int64_t KG = ceil_div(K, 16);
    const int64_t KGp = round_up(KG, 4);
    const int64_t rows = round_up(N, kRowPad);
    const int64_t Kp = round_up(K, 16);
    int32_t* hdr = (int32_t*)base;
    int64_t* corr = (int64_t*)(base + kHeader);
    int32_t* boff = (int32_t*)(base + kHeader + round_up(N * 8, 256));
    int8_t* wp = (int8_t*)((char*)boff + round_up(N * 4, 256));
    int8_t* xa = wp + round_up(rows * KGp * 16, 256);

    const bool mfma_ok = na_mfma_ok(N, K);
    k_na_begin<<<1, 64, 0, st>>>(hdr, mfma_ok ? 0 : 1);
    if (!launched("k_na_begin")) return -1;
    k_na_range<<<grid_1d(M * K, kThreads, 4096), kThreads, 0, st>>>(A, M * K,
                                                                    hdr);
    if (!launched("k_na_range")) return -1;
    if (mfma_ok) {
        k_na_pack_b<<<(unsigned)rows, kThreads, 0, st>>>(
            B, K, N, KGp * 16, wp, boff, corr, hdr);
        if (!launched("k_na_pack_b")) return -1;
        k_na_finish<<<(unsigned)ceil_div(N, kThreads), kThreads, 0, st>>>(
            corr, boff, N, K, hdr);
        if (!launched("k_na_finish")) return -1;
        k_na_pack_a<<<grid_1d(M * Kp + kTail, kThreads, 1 << 16), kThreads,
                      0, st>>>(A, xa, M, K, Kp, hdr);
        if (!launched("k_na_pack_a")) return -1;

        ConvArgs a;
        memset(&a, 0, sizeof(a));
        // a GEMM is a 1x1 convolution of M one-pixel images with K channels
        a.N = (int32_t)M;
        a.H = a.W = 1;
        a.Cg = (int32_t)K;
        a.G = 1;
        a.Cog = a.Cout = (int32_t)N;
        a.KH = a.KW = a.SH = a.SW = a.DH = a.DW = a.OH = a.OW = 1;
        a.M = M;
        a.Kreal = (int32_t)K;
        a.x = xa;
        a.x_code = 1;
        a.x_sn = Kp;
        a.x_sc = 1;
        a.x_sp = 0;
        a.wp = wp;
        a.layout = 0;
        a.CB = (int32_t)KG;
        a.KG = (int32_t)KG;
        a.KGp = (int32_t)KGp;
        a.wp_rstride = KGp * 16;
        a.wp_gstride = rows * KGp * 16;
        a.rowsum = 1;  // the column offsets are known on the device only
        a.corr = corr;
        a.boff = boff;
        a.mode = EPI_RAW32;
        a.y = C;
        a.y_code = 4;
        a.y_sn = N;
        a.y_sc = 1;
        a.y_sp = 0;
        a.gate = hdr + 2;
        a.gate_on = 0;
        // the persistent k_conv_mfma (which honours the gate), widest block
        const int wm = N >= 128 ? 8 : N >= 64 ? 4 : N >= 32 ? 2 : 1;
        a.tile_hint = TILE_VALID | wm | (1 << 9);
        if (!launch_conv_mfma(a, st)) return -1;
    }
    if (!launch_gemm_valu(A, 2, B, 2, C, M, N, K, false, st, hdr + 2, 1))
        return -1;
    return 0;
}

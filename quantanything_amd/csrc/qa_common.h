// Shared definitions of the MI355X (gfx950) integer inference library.
//
// Conventions used by every kernel:
//  * NCHW activations, OIHW weights, row-major GEMM operands (the layouts of
//    the reference ABI, quantization/kernels/qa_kernels.cpp:51-185).
//  * Device-resident quantized tensors are stored as int8 (types of <= 8
//    bits) or int16 (9..16 bits) holding  stored = q - storage_offset,
//    storage_offset = 0 for signed types and 2^(bits-1) for unsigned ones
//    (uint8 q in [0,255] is stored as q-128 in [-128,127]).
//  * Every fixed-point multiply is the reference's exact one: a 128-bit
//    product rounded half up, right shifts clamped to 120 and left shifts to
//    60, clamps applied to the 128-bit value (qa_kernels.cpp:188-205).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef __int128 qa_i128;

#define QA_API extern "C" __attribute__((visibility("default")))

// ---------------------------------------------------------------- mbqm ----
// round(x * mult * 2^-(31+shift)) with a wrapping 128-bit product.
__host__ __device__ __forceinline__ qa_i128 qa_mbqm(int64_t x, int64_t mult,
                                                   int64_t shift) {
    const qa_i128 p = (qa_i128)x * (qa_i128)mult;
    int64_t ts = 31 + shift;
    if (ts > 0) {
        if (ts > 120) ts = 120;
        return (p + ((qa_i128)1 << (ts - 1))) >> ts;
    }
    int64_t ls = -ts;
    if (ls > 60) ls = 60;
    return p * ((qa_i128)1 << ls);
}

// Fast path of qa_mbqm for |x| < 2^32 and |mult| < 2^31 (the product is
// exact in int64), which covers every 8-bit-model accumulator; falls back to
// the 128-bit form otherwise. Bit-identical to qa_mbqm for all inputs:
// floor((p + 2^(t-1)) / 2^t) == (p >> t) + bit (t-1) of p, with no overflow,
// and for t >= 64 the rounded value of |p| < 2^63 is 0.
//
// A second path covers |x| < 2^62 with |mult| < 2^31 and 1 <= 31+shift <=
// 94 (16-bit-model accumulators): the product is formed from two 32x32-bit
// products, x*m = (x_hi*m) * 2^32 + x_lo*m with x_lo = x mod 2^32 unsigned,
// each exact in int64, instead of a full 128-bit multiply.
__host__ __device__ __forceinline__ qa_i128 qa_mbqm_fast(int64_t x,
                                                        int64_t mult,
                                                        int64_t shift) {
    const uint64_t ax = x < 0 ? 0ull - (uint64_t)x : (uint64_t)x;
    const uint64_t am = mult < 0 ? 0ull - (uint64_t)mult : (uint64_t)mult;
    const int64_t ts = 31 + shift;
    if ((am >> 31) == 0 && ts > 0) {
        if ((ax >> 32) == 0) {
            if (ts >= 64) return 0;
            const int64_t p = x * mult;
            return (qa_i128)((p >> ts) + ((p >> (ts - 1)) & 1));
        }
        if ((ax >> 62) == 0 && ts <= 94) {
            const int32_t m = (int32_t)mult;
            const int64_t p_hi = (x >> 32) * (int64_t)m;  // |.| < 2^61
            const uint32_t xl = (uint32_t)x;
            // xl * m as a signed 64-bit value (|.| < 2^63)
            uint64_t u = (uint64_t)xl * (uint64_t)(uint32_t)m;
            if (m < 0) u -= (uint64_t)xl << 32;
            const qa_i128 p = ((qa_i128)p_hi << 32) + (qa_i128)(int64_t)u;
            return (p + ((qa_i128)1 << (ts - 1))) >> ts;
        }
    }
    return qa_mbqm(x, mult, shift);
}

__host__ __device__ __forceinline__ int64_t qa_clip128(qa_i128 v, int64_t lo,
                                                      int64_t hi) {
    if (v < (qa_i128)lo) return lo;
    if (v > (qa_i128)hi) return hi;
    return (int64_t)v;
}

// q = clip(nearbyint(double(x) / scale) + zp) with IEEE double division and
// round-half-even; NaN -> INT32_MIN, which is what the reference's
// double -> int32 conversion yields on x86-64 (qa_kernels.cpp:363-376).
__device__ __forceinline__ int64_t qa_quantize_one(float x, double scale,
                                                   int64_t zp, int64_t qmin,
                                                   int64_t qmax) {
    double v = rint((double)x / scale) + (double)zp;
    if (v != v) return INT32_MIN;
    if (v < (double)qmin) v = (double)qmin;
    if (v > (double)qmax) v = (double)qmax;
    return (int64_t)(int32_t)v;
}

// qa_quantize_one with a multiplication by inv = 1/scale (double) instead
// of the division. The product is within 2^-51 relative of the correctly
// rounded quotient, so both round to the same integer unless the product
// lies within 2^-48 * |y| of a half-integer (or is huge, infinite or NaN);
// those take the division. Bit-identical to qa_quantize_one.
__device__ __forceinline__ int64_t qa_quantize_one_fast(float x, double scale,
                                                        double inv, int64_t zp,
                                                        int64_t qmin,
                                                        int64_t qmax) {
    const double y = (double)x * inv;
    const double r = rint(y);
    const double ay = fabs(y);
    if (!(ay < 2147483648.0) ||
        fabs(fabs(y - r) - 0.5) <= ay * 0x1p-48)
        return qa_quantize_one(x, scale, zp, qmin, qmax);
    double v = r + (double)zp;
    if (v < (double)qmin) v = (double)qmin;
    if (v > (double)qmax) v = (double)qmax;
    return (int64_t)(int32_t)v;
}

// float32 form of qa_quantize_one for scales in [2^-60, 2^60] and clip
// bounds within [-2^22, 2^22] whose width B = 2 max(qmax - zp, zp - qmin) + 2
// is at most 2^20, with invf = float(1 / scale) and tie = 0.5 - B 2^-22
// (qa_f32_tie). r = rint(x * invf) in float32 and d = x * invf - r by one
// fused multiply-add. invf is within 2^-24 of 1 / scale relatively and the
// reference's double quotient y* within 2^-53 of x / scale, so for |y*| <= B
// the distance of y* from r is below |d| + 2^-25 + (B + 1) 2^-24, under 1/2
// when |d| < tie: y* rounds to r. Beyond B, r + zp lies past qmin or qmax
// whichever way r rounds, and the clip decides. r + zp is exact while
// |r| < 2^23, and past the clip bounds beyond. A near-tie (|d| >= tie),
// NaN or an infinity sets *slow, and the caller must use
// qa_quantize_one_fast.
__device__ __forceinline__ int qa_quantize_f32(float x, float invf, float tie,
                                               int zp, int qmin, int qmax,
                                               bool* slow) {
    const float r = rintf(x * invf);
    const float d = fmaf(x, invf, -r);
    *slow |= !(fabsf(d) < tie);  // also for NaN (inf - inf included)
    // one med3 clip; for a NaN x the result is not used (*slow is set)
    return (int)__builtin_amdgcn_fmed3f(r + (float)zp, (float)qmin,
                                        (float)qmax);
}

// qa_quantize_f32's threshold for a clip range (exact in float32).
__host__ __device__ __forceinline__ float qa_f32_tie(int64_t zp, int64_t qmin,
                                                    int64_t qmax) {
    const int64_t w = qmax - zp > zp - qmin ? qmax - zp : zp - qmin;
    return (float)(0.5 - (double)(2 * w + 2) * 0x1p-22);
}

// Whether qa_quantize_f32 applies to a quantization (scale in [2^-60,
// 2^60], clip bounds within +-2^22 and less than 2^19 from the zero point,
// which lies inside them).
__host__ __device__ __forceinline__ bool qa_f32_form_ok(double scale,
                                                       int64_t zp,
                                                       int64_t qmin,
                                                       int64_t qmax) {
    return scale >= 0x1p-60 && scale <= 0x1p60 && qmin >= -(1 << 22) &&
           qmax <= (1 << 22) && zp >= qmin && zp <= qmax &&
           qmax - zp < (1 << 19) && zp - qmin < (1 << 19);
}

// qa_quantize_one_fast's result through the float32 form where that form
// decides (f32ok from qa_f32_form_ok, invf = float(1 / scale)), the double
// form otherwise (near-ties, NaN): a few float instructions per value
// instead of the double ones.
__device__ __forceinline__ int64_t qa_quantize_mixed(float x, bool f32ok,
                                                     float invf, double scale,
                                                     double inv, int64_t zp,
                                                     int64_t qmin,
                                                     int64_t qmax) {
    if (f32ok) {
        bool slow = false;
        const int q = qa_quantize_f32(x, invf, qa_f32_tie(zp, qmin, qmax),
                                      (int)zp, (int)qmin, (int)qmax, &slow);
        if (!slow) return q;
    }
    return qa_quantize_one_fast(x, scale, inv, zp, qmin, qmax);
}

// --------------------------------------------------------------- errors ---
namespace qa {

// Records a failure of the calling thread: it marks the current host-pointer
// ABI call as failed (see AbiCall), makes the message the one qa_last_error
// returns, and prints it to stderr (the first 16 failures of a thread), so a
// caller that never checks still sees it.
void set_error(const char* where, const char* what);
void set_hip_error(const char* where, hipError_t e);
// False once the current ABI call (since its AbiCall was constructed) failed.
bool ok();

#define QA_HIP(call)                                        \
    do {                                                    \
        hipError_t qa_e_ = (call);                          \
        if (qa_e_ != hipSuccess) {                          \
            ::qa::set_hip_error(#call, qa_e_);              \
            return;                                         \
        }                                                   \
    } while (0)

#define QA_HIP_RET(call, ret)                               \
    do {                                                    \
        hipError_t qa_e_ = (call);                          \
        if (qa_e_ != hipSuccess) {                          \
            ::qa::set_hip_error(#call, qa_e_);              \
            return ret;                                     \
        }                                                   \
    } while (0)

// Stream of the calling thread on the current device (default priority,
// non-blocking). Each thread has its own, so host-pointer ABI calls from
// several threads run concurrently, like the reference's re-entrant kernels.
hipStream_t stream();

// A device scratch buffer of at least `bytes`, owned by the calling thread
// (one set of slots per thread and device), reused across its ABI calls.
void* scratch(int slot, size_t bytes);

// Scope of one host-pointer ABI call. Construction starts a new call: the
// per-call failure flag is cleared (an earlier failure on this thread never
// makes a later call skip its work) and so is HIP's last-error state.
// Destruction, when the call failed, fills the caller's output with zeros
// (out may be a host or a device pointer), so no call returns with its
// output unwritten.
struct AbiCall {
    AbiCall(void* out, size_t out_bytes);
    ~AbiCall();
    AbiCall(const AbiCall&) = delete;
    AbiCall& operator=(const AbiCall&) = delete;

  private:
    void* out_;
    size_t bytes_;
};

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline int64_t round_up(int64_t a, int64_t b) { return ceil_div(a, b) * b; }

inline unsigned grid_1d(int64_t n, int threads, int64_t cap = 1 << 16) {
    int64_t g = ceil_div(n, threads);
    if (g < 1) g = 1;
    if (g > cap) g = cap;
    return (unsigned)g;
}

}  // namespace qa

// Library runtime: error reporting, the per-device stream, scratch buffers
// and the diagnostic exports (qa_backend, qa_last_error, ...).
#include <stdio.h>
#include <string.h>
#include <sys/syscall.h>
#include <sys/types.h>
#include <unistd.h>

#include "qa_common.h"

namespace qa {

namespace {

constexpr int kMaxDevices = 16;
constexpr int kSlots = 8;
constexpr int kMaxPrinted = 16;

// One thread's stream and scratch buffers on one device.
struct DeviceState {
    hipStream_t stream = nullptr;
    void* buf[kSlots] = {};
    size_t cap[kSlots] = {};
};

// A thread's state on every device. The destructor runs at thread exit
// (for the main thread: at exit(), before static destructors and so while
// the HIP runtime is still up); it drains the thread's streams and releases
// its buffers.
struct ThreadState {
    DeviceState dev[kMaxDevices];
    // A thread that ends while the process runs returns its stream and
    // buffers. The main thread's state is destroyed only inside exit(),
    // after which the HIP runtime (and a profiler attached to it) may
    // already be torn down: there nothing is released, the driver reclaims
    // the process's streams and memory.
    ~ThreadState() {
        if ((pid_t)syscall(SYS_gettid) == getpid()) return;
        for (int d = 0; d < kMaxDevices; ++d) {
            DeviceState& s = dev[d];
            if (!s.stream) continue;
            if (hipSetDevice(d) != hipSuccess) continue;
            hipStreamSynchronize(s.stream);
            for (int k = 0; k < kSlots; ++k)
                if (s.buf[k]) hipFree(s.buf[k]);
            hipStreamDestroy(s.stream);
        }
    }
};

thread_local ThreadState t_state;
thread_local char t_error[512] = {0};
thread_local bool t_failed = false;       // since the last qa_clear_error
thread_local bool t_call_failed = false;  // in the current ABI call
thread_local int t_printed = 0;

int current_device() {
    int d = 0;
    if (hipGetDevice(&d) != hipSuccess || d < 0 || d >= kMaxDevices) d = 0;
    return d;
}

}  // namespace

void set_error(const char* where, const char* what) {
    snprintf(t_error, sizeof(t_error), "%s: %s", where, what);
    if (t_printed < kMaxPrinted) {
        fprintf(stderr, "[qa_hip] error: %s%s\n", t_error,
                t_printed + 1 == kMaxPrinted
                    ? " (further errors of this thread are not printed)"
                    : "");
        ++t_printed;
    }
    t_failed = true;
    t_call_failed = true;
}

void set_hip_error(const char* where, hipError_t e) {
    set_error(where, hipGetErrorString(e));
}

bool ok() { return !t_call_failed; }

hipStream_t stream() {
    DeviceState& s = t_state.dev[current_device()];
    if (!s.stream) {
        hipStream_t st = nullptr;
        // Default priority on purpose: streams of different priorities
        // are not used anywhere in this library.
        hipError_t e = hipStreamCreateWithFlags(&st, hipStreamNonBlocking);
        if (e != hipSuccess) {
            set_hip_error("hipStreamCreateWithFlags", e);
            return nullptr;
        }
        s.stream = st;
    }
    return s.stream;
}

void* scratch(int slot, size_t bytes) {
    DeviceState& s = t_state.dev[current_device()];
    if (bytes == 0) bytes = 256;
    if (s.cap[slot] < bytes) {
        if (s.buf[slot]) {
            // Freed only once the stream has drained (the buffer may still be
            // read by the previous call's kernels).
            if (s.stream) hipStreamSynchronize(s.stream);
            hipFree(s.buf[slot]);
            s.buf[slot] = nullptr;
            s.cap[slot] = 0;
        }
        size_t want = bytes + bytes / 4;
        want = (want + 4095) & ~(size_t)4095;
        void* p = nullptr;
        hipError_t e = hipMalloc(&p, want);
        if (e != hipSuccess) {
            set_hip_error("hipMalloc(scratch)", e);
            return nullptr;
        }
        s.buf[slot] = p;
        s.cap[slot] = want;
    }
    return s.buf[slot];
}

AbiCall::AbiCall(void* out, size_t out_bytes) : out_(out), bytes_(out_bytes) {
    t_call_failed = false;
    (void)hipGetLastError();
}

AbiCall::~AbiCall() {
    if (!t_call_failed || !out_ || bytes_ == 0) return;
    // Device (or managed) memory is cleared through HIP; anything else is
    // host memory the caller allocated.
    hipPointerAttribute_t at;
    bool device = false;
    if (hipPointerGetAttributes(&at, out_) == hipSuccess)
        device = at.type == hipMemoryTypeDevice ||
                 at.type == hipMemoryTypeManaged;
    (void)hipGetLastError();  // an unknown host pointer reports an error
    if (device) {
        if (hipMemset(out_, 0, bytes_) != hipSuccess) (void)hipGetLastError();
    } else {
        memset(out_, 0, bytes_);
    }
}

}  // namespace qa

// ------------------------------------------------------------ exports ---

// Identifies the backend so a caller can assert that the GPU library (and
// not a CPU build) is the one loaded.
QA_API const char* qa_backend(void) { return "hip-gfx950"; }

// Message of the most recent failure on the calling thread, or NULL when no
// call of this thread failed since the last qa_clear_error. Host-pointer ABI
// entries return void like the reference's, so this is how a caller learns
// that a call failed; a failed call leaves zeros in its output, and the next
// call runs normally whether or not the error was cleared.
QA_API const char* qa_last_error(void) {
    return qa::t_failed ? qa::t_error : nullptr;
}

QA_API void qa_clear_error(void) {
    qa::t_failed = false;
    qa::t_error[0] = 0;
}

// Number of visible GPUs (0 when the HIP runtime finds none).
QA_API int qa_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

// gfx architecture name of the current device into `buf` (NUL-terminated);
// returns 0 on success.
QA_API int qa_device_arch(char* buf, int64_t len) {
    hipDeviceProp_t prop;
    int d = 0;
    if (hipGetDevice(&d) != hipSuccess) return -1;
    if (hipGetDeviceProperties(&prop, d) != hipSuccess) return -1;
    if (len > 0) {
        strncpy(buf, prop.gcnArchName, (size_t)len - 1);
        buf[len - 1] = 0;
    }
    return 0;
}

// The calling thread's library stream on the current device (hipStream_t as
// a pointer).
QA_API void* qa_stream(void) { return (void*)qa::stream(); }

// Waits for all work the calling thread queued through the library on the
// current device.
QA_API int qa_synchronize(void) {
    hipError_t e = hipStreamSynchronize(qa::stream());
    if (e != hipSuccess) {
        qa::set_hip_error("hipStreamSynchronize", e);
        return -1;
    }
    return 0;
}

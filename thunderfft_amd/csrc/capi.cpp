// capi.cpp -- the C ABI of include/thunderfft/thunderfft.h: argument checks,
// the per-(device, precision) twiddle cache and kernel dispatch.
//
// Check order and error kinds follow the reference host wrapper
// (include/thunderfft/detail/thunderfft_impl_kernel.cuh:13-21) and cache
// (include/thunderfft/detail/thunderfft_impl_twiddle.cuh:279-327,358-378):
// invalid arguments are reported before any HIP call, HIP failures as
// "[ThunderFFT] <context>: <hip error string>".
#include <hip/hip_runtime.h>

#include <climits>
#include <cmath>
#include <cstdint>
#include <atomic>
#include <mutex>
#include <string>
#include <vector>

#include "launch.hpp"
#include "thunderfft/thunderfft.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const std::string& message) {
    g_last_error = message;
    return code;
}

int fail_hip(hipError_t err, const char* context) {
    return fail(THFF_EIO, std::string("[ThunderFFT] ") + context + ": " + hipGetErrorString(err));
}

bool supported_length(int n) {
    return n == 64 || n == 128 || n == 256 || n == 512 || n == 1024 || n == 2048 || n == 4096;
}

bool supported_precision(int p) { return p == THFF_FLOAT || p == THFF_HALF; }

const char* precision_name(int p) { return p == THFF_FLOAT ? "float" : "half"; }

// Twiddle registry: one table per (precision, device) is current, as in the
// reference cache (thunderfft_impl_twiddle.cuh:26-36,310-326).  Transforms
// read it without a lock: `current` names the live length and `table[s]`
// the table of length 64 << s, both published with release stores after the
// table is filled.  Initialize with a new length makes that length current
// and keeps the replaced table allocated (it is freed by Finalize), so a
// transform that another thread has just enqueued never reads freed memory;
// Initialize and Finalize are serialised per precision by g_mutex, like the
// reference's per-T mutex.  At most the seven tables of one precision stay
// allocated per device (8128 values, 65 KB).  Finalize while a transform that
// uses the table is still in flight on another thread is the caller's race,
// as in the reference.
constexpr int kMaxDevices = 64;
constexpr int kLengths = 7;  // 64 << s, s < 7

struct DeviceTables {
    std::atomic<int> current{0};  // live length, 0 when released
    std::atomic<int> num_cus{0};
    std::atomic<float2*> table[kLengths] = {};
};
DeviceTables g_tables[2][kMaxDevices];
std::mutex g_mutex[2];

// Workspace of the allocation-free 2-D convolution (thff_conv2d_noalloc):
// one fp32 spectrum of the largest image the multi-pass form takes,
// 1024 x 1024 (8 MiB), in a device array of this library's code object, so
// that each GPU the library runs on holds its own copy until the process
// ends.  In host code `scratch` names the symbol, not a device address: the
// address of the current device's copy is resolved once per device with
// hipGetSymbolAddress (in ThunderFFTInitialize, which every convolution
// requires first, or at the first call) and kept in g_scratch.  Every
// allocation-free call on a GPU shares that GPU's copy: calls that overlap on
// one GPU race.  Nothing in it needs clearing: the filter pass writes every
// value before the column pass reads it.
constexpr long long kScratchValues = 1024LL * 1024LL;
__device__ __align__(256) float2 scratch[kScratchValues];
std::atomic<float2*> g_scratch[kMaxDevices] = {};
std::mutex g_scratch_mutex;

// This device's copy of `scratch` (device: the current device).
int scratch_address(int device, float2** out) {
    float2* p = g_scratch[device].load(std::memory_order_acquire);
    if (!p) {
        std::lock_guard<std::mutex> lock(g_scratch_mutex);
        p = g_scratch[device].load(std::memory_order_relaxed);
        if (!p) {
            void* address = nullptr;
            const hipError_t err = hipGetSymbolAddress(&address, HIP_SYMBOL(scratch));
            if (err != hipSuccess) return fail_hip(err, "hipGetSymbolAddress (conv2d workspace)");
            p = static_cast<float2*>(address);
            g_scratch[device].store(p, std::memory_order_release);
        }
    }
    *out = p;
    return THFF_OK;
}

int length_slot(int n) {
    int s = 0;
    while ((64 << s) < n) ++s;
    return s;
}

// The current device's registry entry, or null with the error recorded.
DeviceTables* device_tables(int precision, const char* who, int* device_out) {
    int device = 0;
    const hipError_t err = hipGetDevice(&device);
    if (err != hipSuccess) {
        fail_hip(err, who);
        return nullptr;
    }
    if (device < 0 || device >= kMaxDevices) {
        fail(THFF_EIO, std::string("[ThunderFFT] ") + who + ": device " + std::to_string(device) +
                           " is beyond the " + std::to_string(kMaxDevices) +
                           " devices this build supports");
        return nullptr;
    }
    if (device_out) *device_out = device;
    return &g_tables[precision][device];
}

// W[m] = (cos, sin)(2*pi*m/N) in fp64, rounded once to fp32; the quarter
// points are exact so that W[0] = 1 + 0i bit for bit.
std::vector<float2> build_table(int n) {
    std::vector<float2> h(n);
    const double tau = 6.283185307179586476925286766559;
    for (int m = 0; m < n; ++m) {
        const double a = tau * static_cast<double>(m) / static_cast<double>(n);
        h[m] = make_float2(static_cast<float>(std::cos(a)), static_cast<float>(std::sin(a)));
    }
    h[0] = make_float2(1.f, 0.f);
    h[n / 4] = make_float2(0.f, 1.f);
    h[n / 2] = make_float2(-1.f, 0.f);
    h[3 * n / 4] = make_float2(0.f, -1.f);
    return h;
}

hipError_t dispatch(int n, int precision, bool forward, bool aligned, const void* in, void* out,
                    int batch, const float2* tw, int cus, hipStream_t s) {
#define THFF_C2C_CASE(L) \
    case L: return thff::launch_c2c<L>(precision, forward, aligned, in, out, batch, tw, cus, s)
    switch (n) {
        THFF_C2C_CASE(64);
        THFF_C2C_CASE(128);
        THFF_C2C_CASE(256);
        THFF_C2C_CASE(512);
        THFF_C2C_CASE(1024);
        THFF_C2C_CASE(2048);
        THFF_C2C_CASE(4096);
    default: return hipErrorInvalidValue;
    }
#undef THFF_C2C_CASE
}

hipError_t dispatch_conv1d(int n, int precision, bool per_signal, const void* x, const void* h,
                           void* y, int batch, const float2* tw, int cus, hipStream_t s) {
    switch (n) {
    case 64: return thff::launch_conv1d<64>(precision, per_signal, x, h, y, batch, tw, cus, s);
    case 128: return thff::launch_conv1d<128>(precision, per_signal, x, h, y, batch, tw, cus, s);
    case 256: return thff::launch_conv1d<256>(precision, per_signal, x, h, y, batch, tw, cus, s);
    case 512: return thff::launch_conv1d<512>(precision, per_signal, x, h, y, batch, tw, cus, s);
    case 1024: return thff::launch_conv1d<1024>(precision, per_signal, x, h, y, batch, tw, cus, s);
    case 2048: return thff::launch_conv1d<2048>(precision, per_signal, x, h, y, batch, tw, cus, s);
    case 4096: return thff::launch_conv1d<4096>(precision, per_signal, x, h, y, batch, tw, cus, s);
    default: return hipErrorInvalidValue;
    }
}

hipError_t dispatch_conv1d_real_filter(int n, const float* h, float2* spectrum, int channels,
                                       float scale, const float2* tw, hipStream_t s) {
    switch (n) {
    case 64: return thff::launch_conv1d_real_filter<64>(h, spectrum, channels, scale, tw, s);
    case 128: return thff::launch_conv1d_real_filter<128>(h, spectrum, channels, scale, tw, s);
    case 256: return thff::launch_conv1d_real_filter<256>(h, spectrum, channels, scale, tw, s);
    case 512: return thff::launch_conv1d_real_filter<512>(h, spectrum, channels, scale, tw, s);
    case 1024: return thff::launch_conv1d_real_filter<1024>(h, spectrum, channels, scale, tw, s);
    case 2048: return thff::launch_conv1d_real_filter<2048>(h, spectrum, channels, scale, tw, s);
    case 4096: return thff::launch_conv1d_real_filter<4096>(h, spectrum, channels, scale, tw, s);
    default: return hipErrorInvalidValue;
    }
}

hipError_t dispatch_conv1d_real(int n, int precision, const void* x, const float2* spectrum,
                                void* y, int batch, int channels, const float2* tw, int cus,
                                hipStream_t s) {
#define THFF_REAL_CASE(L)                                                                     \
    case L:                                                                                   \
        return thff::launch_conv1d_real<L>(precision, x, spectrum, y, batch, channels, tw, cus, s)
    switch (n) {
        THFF_REAL_CASE(64);
        THFF_REAL_CASE(128);
        THFF_REAL_CASE(256);
        THFF_REAL_CASE(512);
        THFF_REAL_CASE(1024);
        THFF_REAL_CASE(2048);
        THFF_REAL_CASE(4096);
    default: return hipErrorInvalidValue;
    }
#undef THFF_REAL_CASE
}

// The current device's table for (precision, n) and its CU count, or an
// error naming the missing ThunderFFTInitialize call.  Lock-free: two
// acquire loads of the registry (see DeviceTables).
int cached_table(int precision, int n, const char* who, const float2** table, int* cus) {
    int device = 0;
    DeviceTables* d = device_tables(precision, who, &device);
    if (!d) return THFF_EIO;
    if (d->current.load(std::memory_order_acquire) == n) {
        const float2* t = d->table[length_slot(n)].load(std::memory_order_acquire);
        if (t) {
            *table = t;
            *cus = d->num_cus.load(std::memory_order_relaxed);
            return THFF_OK;
        }
    }
    return fail(THFF_EIO, std::string("[ThunderFFT] ") + who + ": no twiddle table for N=" +
                              std::to_string(n) + " on device " + std::to_string(device) +
                              "; call ThunderFFTInitialize<" + precision_name(precision) + ">(" +
                              std::to_string(n) + ") first");
}

// The kernels move 16-byte vectors: every buffer must start on a 16-byte
// boundary (any hipMalloc'd pointer, and any offset of whole transforms).
bool aligned16(const void* p) { return (reinterpret_cast<std::uintptr_t>(p) & 15) == 0; }

int conv1d_impl(int precision, int n, const void* x, const void* h, void* y, int batch,
                int per_signal_filter, void* stream, bool synchronize) {
    if (!supported_precision(precision))
        return fail(THFF_EINVAL, "ThunderFFT_conv1d supports float and half only");
    if (!supported_length(n)) return fail(THFF_EINVAL, "Unsupported ThunderFFT length");
    if (batch < 0) return fail(THFF_EINVAL, "ThunderFFT batch must be nonnegative");
    if (batch == 0) return THFF_OK;
    if (!x || !h || !y)
        return fail(THFF_EINVAL, "ThunderFFT_conv1d requires non-null signal, filter and output");
    if (y == x || y == h)
        return fail(THFF_EINVAL, "ThunderFFT_conv1d output must not alias its inputs");
    if (!aligned16(x) || !aligned16(h) || !aligned16(y))
        return fail(THFF_EINVAL, "ThunderFFT_conv1d requires 16-byte aligned buffers");
    const long long fpb = thff::c2c_transforms_per_block(n);
    if ((static_cast<long long>(batch) + fpb - 1) / fpb * 256 > static_cast<long long>(UINT32_MAX))
        return fail(THFF_EINVAL, "ThunderFFT batch exceeds one launch for this length");
    const float2* table = nullptr;
    int cus = 0;
    const int rc = cached_table(precision, n, "ThunderFFT_conv1d", &table, &cus);
    if (rc != THFF_OK) return rc;
    auto s = static_cast<hipStream_t>(stream);
    hipError_t err = dispatch_conv1d(n, precision, per_signal_filter != 0, x, h, y, batch, table,
                                     cus, s);
    if (err != hipSuccess) return fail_hip(err, "ThunderFFT_conv1d launch");
    if (synchronize) {
        err = hipStreamSynchronize(s);
        if (err != hipSuccess) return fail_hip(err, "ThunderFFT_conv1d synchronize");
    }
    return THFF_OK;
}

int finish(hipStream_t s, bool synchronize, const char* who) {
    if (!synchronize) return THFF_OK;
    const hipError_t err = hipStreamSynchronize(s);
    return err == hipSuccess ? THFF_OK : fail_hip(err, who);
}

int conv1d_real_filter_impl(int precision, int n, const void* h, void* spectrum, int channels,
                            float scale, void* stream, bool synchronize) {
    if (!supported_precision(precision))
        return fail(THFF_EINVAL, "ThunderFFT_conv1d_real_filter supports float and half only");
    if (!supported_length(n)) return fail(THFF_EINVAL, "Unsupported ThunderFFT length");
    if (channels < 0) return fail(THFF_EINVAL, "ThunderFFT channels must be nonnegative");
    if (channels == 0) return THFF_OK;
    if (!h || !spectrum)
        return fail(THFF_EINVAL, "ThunderFFT_conv1d_real_filter requires non-null filter and spectrum");
    if (spectrum == h)
        return fail(THFF_EINVAL, "ThunderFFT_conv1d_real_filter spectrum must not alias the filter");
    const float2* table = nullptr;
    int cus = 0;
    const int rc = cached_table(precision, n, "ThunderFFT_conv1d_real_filter", &table, &cus);
    if (rc != THFF_OK) return rc;
    auto s = static_cast<hipStream_t>(stream);
    const hipError_t err = dispatch_conv1d_real_filter(
        n, static_cast<const float*>(h), static_cast<float2*>(spectrum), channels, scale, table, s);
    if (err != hipSuccess) return fail_hip(err, "ThunderFFT_conv1d_real_filter launch");
    return finish(s, synchronize, "ThunderFFT_conv1d_real_filter synchronize");
}

int conv1d_real_impl(int precision, int n, const void* x, const void* spectrum, void* y,
                     int batch, int channels, void* stream, bool synchronize) {
    if (!supported_precision(precision))
        return fail(THFF_EINVAL, "ThunderFFT_conv1d_real supports float and half only");
    if (!supported_length(n)) return fail(THFF_EINVAL, "Unsupported ThunderFFT length");
    if (batch < 0) return fail(THFF_EINVAL, "ThunderFFT batch must be nonnegative");
    if (batch == 0) return THFF_OK;
    if (channels <= 0) return fail(THFF_EINVAL, "ThunderFFT channels must be positive");
    if (!x || !spectrum || !y)
        return fail(THFF_EINVAL, "ThunderFFT_conv1d_real requires non-null signal, spectrum and output");
    if (y == x || y == spectrum)
        return fail(THFF_EINVAL, "ThunderFFT_conv1d_real output must not alias its inputs");
    if (!aligned16(x) || !aligned16(y))
        return fail(THFF_EINVAL, "ThunderFFT_conv1d_real requires 16-byte aligned signal and output");
    // Complex transforms: one per pair of signals of a channel.
    const long long transforms = (static_cast<long long>(batch) + 1) / 2 * channels;
    const long long fpb = thff::c2c_transforms_per_block(n);
    if ((transforms + fpb - 1) / fpb * 256 > static_cast<long long>(UINT32_MAX))
        return fail(THFF_EINVAL, "ThunderFFT batch exceeds one launch for this length");
    const float2* table = nullptr;
    int cus = 0;
    const int rc = cached_table(precision, n, "ThunderFFT_conv1d_real", &table, &cus);
    if (rc != THFF_OK) return rc;
    auto s = static_cast<hipStream_t>(stream);
    const hipError_t err = dispatch_conv1d_real(n, precision, x, static_cast<const float2*>(spectrum),
                                                y, batch, channels, table, cus, s);
    if (err != hipSuccess) return fail_hip(err, "ThunderFFT_conv1d_real launch");
    return finish(s, synchronize, "ThunderFFT_conv1d_real synchronize");
}

int conv1d_valid_impl(int precision, const void* x, long long input_len, const void* taps,
                      int filter_len, void* y, int batch, void* stream, bool synchronize) {
    if (!supported_precision(precision))
        return fail(THFF_EINVAL, "ThunderFFT_conv1d_valid supports float and half only");
    // The reference sample's two argument checks (sample/conv1d/main.cu:223-230).
    if (filter_len < 1 || filter_len > 64)
        return fail(THFF_EINVAL, "ThunderFFT_conv1d_valid: filter_len must be in [1, 64]");
    if (input_len < filter_len)
        return fail(THFF_EINVAL, "ThunderFFT_conv1d_valid: input_len must be >= filter_len");
    if (batch < 0) return fail(THFF_EINVAL, "ThunderFFT batch must be nonnegative");
    if (batch == 0) return THFF_OK;
    if (!x || !taps || !y)
        return fail(THFF_EINVAL, "ThunderFFT_conv1d_valid requires non-null input, filter and output");
    if (y == x || y == taps)
        return fail(THFF_EINVAL, "ThunderFFT_conv1d_valid output must not alias its inputs");
    const std::uintptr_t elem = precision == THFF_FLOAT ? 8 : 4;
    if ((reinterpret_cast<std::uintptr_t>(x) | reinterpret_cast<std::uintptr_t>(y)) % elem ||
        reinterpret_cast<std::uintptr_t>(taps) % 8)
        return fail(THFF_EINVAL, "ThunderFFT_conv1d_valid: misaligned pointer");
    // Window groups of one launch (fp32: 64 windows of 64 points per group;
    // fp16: 16 windows of 256 points), counted in 32 bits by the kernels'
    // grid walk.
    const long long window = precision == THFF_FLOAT ? 64 : 256;
    const long long per_group = precision == THFF_FLOAT ? 64 : 16;
    const long long valid = window + 1 - filter_len;
    const long long windows = (input_len - filter_len + 1 + valid - 1) / valid;
    if ((windows + per_group - 1) / per_group * batch * 256 > static_cast<long long>(UINT32_MAX))
        return fail(THFF_EINVAL, "ThunderFFT batch exceeds one launch for this length");
    const float2* table = nullptr;
    int cus = 0;
    const int rc = cached_table(precision, 64, "ThunderFFT_conv1d_valid", &table, &cus);
    if (rc != THFF_OK) return rc;
    auto s = static_cast<hipStream_t>(stream);
    const hipError_t err = thff::launch_conv1d_valid(precision, x, input_len,
                                                     static_cast<const float2*>(taps), filter_len,
                                                     y, batch, table, cus, s);
    if (err != hipSuccess) return fail_hip(err, "ThunderFFT_conv1d_valid launch");
    return finish(s, synchronize, "ThunderFFT_conv1d_valid synchronize");
}

// 2-D convolution sizes: rows = cols = 64 and 128 run one fused kernel per
// image (the image stays on chip); 1024 runs the multi-pass form of the
// reference's built sample (sample/conv2d/thunder.cu:70-207): the filter's
// spectrum into a stream-ordered workspace, then row FFTs (the C2C kernel),
// a column pass doing FFT x H x IFFT, and inverse row FFTs, in place in y.
int conv2d_impl(int precision, int rows, int cols, const void* x, const void* h, void* y,
                int batch, void* stream, bool synchronize, bool allocate = true) {
    if (!supported_precision(precision))
        return fail(THFF_EINVAL, "ThunderFFT_conv2d supports float and half only");
    if (rows != cols || (rows != 64 && rows != 128 && rows != 1024))
        return fail(THFF_EINVAL,
                    "ThunderFFT_conv2d supports 64 x 64, 128 x 128 and 1024 x 1024 images only");
    if (batch < 0) return fail(THFF_EINVAL, "ThunderFFT batch must be nonnegative");
    if (batch == 0) return THFF_OK;
    if (!x || !h || !y)
        return fail(THFF_EINVAL, "ThunderFFT_conv2d requires non-null images, filter and output");
    if (y == x || y == h)
        return fail(THFF_EINVAL, "ThunderFFT_conv2d output must not alias its inputs");
    if (!aligned16(x) || !aligned16(h) || !aligned16(y))
        return fail(THFF_EINVAL, "ThunderFFT_conv2d requires 16-byte aligned buffers");
    if (batch > (rows == 1024 ? (1 << 16) : (1 << 24)))
        return fail(THFF_EINVAL, "ThunderFFT batch exceeds one launch");
    if (!allocate && static_cast<long long>(rows) * cols > kScratchValues)
        return fail(THFF_EINVAL,
                    "ThunderFFT_conv2d_noalloc: the image exceeds the allocation-free workspace "
                    "(one 1024 x 1024 spectrum)");
    const float2* table = nullptr;
    int cus = 0;
    const int rc = cached_table(precision, rows, "ThunderFFT_conv2d", &table, &cus);
    if (rc != THFF_OK) return rc;
    auto s = static_cast<hipStream_t>(stream);
    hipError_t err = hipSuccess;
    if (rows == 64) {
        err = thff::launch_conv2d64(precision, x, h, y, batch, table, cus, s);
    } else if (rows == 128) {
        err = thff::launch_conv2d128(precision, x, h, y, batch, table, cus, s);
    } else {
        constexpr int kN = 1024;
        const size_t spectrum_bytes = sizeof(float2) * kN * kN;
        void* spectrum = nullptr;
        if (allocate) {
            err = hipMallocAsync(&spectrum, spectrum_bytes, s);
            if (err != hipSuccess) return fail_hip(err, "ThunderFFT_conv2d workspace");
        } else {
            int device = 0;
            err = hipGetDevice(&device);
            if (err != hipSuccess) return fail_hip(err, "hipGetDevice (conv2d)");
            float2* p = nullptr;
            const int src = scratch_address(device, &p);
            if (src != THFF_OK) return src;
            spectrum = p;
        }
        auto* H = static_cast<float2*>(spectrum);
        const int row_signals = batch * kN;
        // H = FFT2(h) / (rows * cols): columns (scaled, into fp32), then rows in place
        err = thff::launch_conv2d_cols(precision, false, h, H, nullptr, kN, 1,
                                       1.0f / (static_cast<float>(kN) * kN), table, cus, s);
        if (err == hipSuccess)
            err = thff::launch_c2c<kN>(THFF_FLOAT, true, true, H, H, kN, table, cus, s);
        if (err == hipSuccess)
            err = thff::launch_c2c<kN>(precision, true, true, x, y, row_signals, table, cus, s);
        if (err == hipSuccess)
            err = thff::launch_conv2d_cols(precision, true, y, y, H, kN, batch, 0.0f, table,
                                           cus, s);
        if (err == hipSuccess)
            err = thff::launch_c2c<kN>(precision, false, true, y, y, row_signals, table, cus, s);
        if (allocate) {
            const hipError_t ferr = hipFreeAsync(spectrum, s);
            if (err == hipSuccess) err = ferr;
        }
    }
    if (err != hipSuccess) return fail_hip(err, "ThunderFFT_conv2d launch");
    if (synchronize) {
        err = hipStreamSynchronize(s);
        if (err != hipSuccess) return fail_hip(err, "ThunderFFT_conv2d synchronize");
    }
    return THFF_OK;
}

int global_impl(int precision, int n, int forward, const void* d_input, void* d_output, int batch,
                void* stream, bool synchronize) {
    if (!supported_precision(precision))
        return fail(THFF_EINVAL, "ThunderFFT_global supports float and half only");
    if (!supported_length(n)) return fail(THFF_EINVAL, "Unsupported ThunderFFT length");
    if (batch < 0) return fail(THFF_EINVAL, "ThunderFFT batch must be nonnegative");
    if (batch == 0) return THFF_OK;
    if (!d_input || !d_output || d_input == d_output)
        return fail(THFF_EINVAL, "ThunderFFT requires separate non-null input/output buffers");
    // Any vec2_t<T> buffer (the reference contract) is accepted: element
    // alignment is required, 16-byte alignment selects the staged kernels.
    const std::uintptr_t elem = precision == THFF_FLOAT ? 8 : 4;
    const std::uintptr_t addr_bits = reinterpret_cast<std::uintptr_t>(d_input) |
                                     reinterpret_cast<std::uintptr_t>(d_output);
    if (addr_bits % elem != 0)
        return fail(THFF_EINVAL, precision == THFF_FLOAT
                                     ? "ThunderFFT requires 8-byte aligned float2 buffers"
                                     : "ThunderFFT requires 4-byte aligned half2 buffers");
    const bool aligned = addr_bits % 16 == 0;
    // The dispatch grid counts work-items in 32 bits.
    const long long fpb = thff::c2c_transforms_per_block(n);
    const long long items = (static_cast<long long>(batch) + fpb - 1) / fpb * 256;
    if (items > static_cast<long long>(UINT32_MAX))
        return fail(THFF_EINVAL, "ThunderFFT batch exceeds one launch for this length");

    const float2* table = nullptr;
    int cus = 0;
    const int rc = cached_table(precision, n, "ThunderFFT_global", &table, &cus);
    if (rc != THFF_OK) return rc;
    auto s = static_cast<hipStream_t>(stream);
    hipError_t err = dispatch(n, precision, forward != 0, aligned, d_input, d_output, batch, table,
                              cus, s);
    if (err != hipSuccess) return fail_hip(err, "ThunderFFT_global launch");
    return finish(s, synchronize, "ThunderFFT_global synchronize");
}

}  // namespace

namespace thff {
int c2c_transforms_per_block(int n) { return 256 * 16 / n; }
}  // namespace thff

extern "C" {

int thff_version(void) { return 100; }

const char* thff_last_error(void) { return g_last_error.c_str(); }

int thff_initialize(int precision, int n) {
    if (!supported_precision(precision))
        return fail(THFF_EINVAL, "ThunderFFTInitialize<T>: supported T are float and half only");
    if (!supported_length(n))
        return fail(THFF_EINVAL, "ThunderFFTInitialize<T>: unsupported FFT size");
    std::lock_guard<std::mutex> lock(g_mutex[precision]);
    int device = 0;
    DeviceTables* d = device_tables(precision, "hipGetDevice (initialize)", &device);
    if (!d) return THFF_EIO;
    float2* workspace = nullptr;  // the allocation-free conv2d's, resolved once per device
    const int wrc = scratch_address(device, &workspace);
    if (wrc != THFF_OK) return wrc;
    if (d->current.load(std::memory_order_relaxed) == n) return THFF_OK;
    std::atomic<float2*>& slot = d->table[length_slot(n)];
    if (!slot.load(std::memory_order_relaxed)) {
        int cus = 0;
        hipError_t err = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device);
        if (err != hipSuccess) return fail_hip(err, "hipDeviceGetAttribute (initialize)");
        const std::vector<float2> host = build_table(n);
        float2* table = nullptr;
        err = hipMalloc(reinterpret_cast<void**>(&table), sizeof(float2) * n);
        if (err != hipSuccess) return fail_hip(err, "hipMalloc twiddle table");
        err = hipMemcpy(table, host.data(), sizeof(float2) * n, hipMemcpyHostToDevice);
        if (err != hipSuccess) {
            (void)hipFree(table);
            return fail_hip(err, "hipMemcpy twiddle table");
        }
        d->num_cus.store(cus, std::memory_order_relaxed);
        slot.store(table, std::memory_order_release);
    }
    d->current.store(n, std::memory_order_release);
    return THFF_OK;
}

int thff_finalize(int precision) {
    if (!supported_precision(precision))
        return fail(THFF_EINVAL, "ThunderFFTFinalize<T>: supported T are float and half only");
    std::lock_guard<std::mutex> lock(g_mutex[precision]);
    DeviceTables* d = device_tables(precision, "hipGetDevice (finalize)", nullptr);
    if (!d) return THFF_EIO;
    d->current.store(0, std::memory_order_release);
    hipError_t first = hipSuccess;
    for (auto& slot : d->table) {
        float2* table = slot.exchange(nullptr, std::memory_order_acq_rel);
        if (!table) continue;
        const hipError_t err = hipFree(table);
        if (first == hipSuccess) first = err;
    }
    return first == hipSuccess ? THFF_OK : fail_hip(first, "hipFree cached twiddle (finalize)");
}

int thff_global(int precision, int n, int forward, const void* d_input, void* d_output, int batch,
                void* stream) {
    return global_impl(precision, n, forward, d_input, d_output, batch, stream, true);
}

int thff_global_async(int precision, int n, int forward, const void* d_input, void* d_output,
                      int batch, void* stream) {
    return global_impl(precision, n, forward, d_input, d_output, batch, stream, false);
}

int thff_conv1d(int precision, int n, const void* d_x, const void* d_h, void* d_y, int batch,
                int per_signal_filter, void* stream) {
    return conv1d_impl(precision, n, d_x, d_h, d_y, batch, per_signal_filter, stream, true);
}

int thff_conv1d_async(int precision, int n, const void* d_x, const void* d_h, void* d_y,
                      int batch, int per_signal_filter, void* stream) {
    return conv1d_impl(precision, n, d_x, d_h, d_y, batch, per_signal_filter, stream, false);
}

int thff_conv1d_real_filter(int precision, int n, const void* d_h, void* d_spectrum,
                            int channels, float scale, void* stream) {
    return conv1d_real_filter_impl(precision, n, d_h, d_spectrum, channels, scale, stream, true);
}

int thff_conv1d_real_filter_async(int precision, int n, const void* d_h, void* d_spectrum,
                                  int channels, float scale, void* stream) {
    return conv1d_real_filter_impl(precision, n, d_h, d_spectrum, channels, scale, stream, false);
}

int thff_conv1d_real(int precision, int n, const void* d_x, const void* d_spectrum, void* d_y,
                     int batch, int channels, void* stream) {
    return conv1d_real_impl(precision, n, d_x, d_spectrum, d_y, batch, channels, stream, true);
}

int thff_conv1d_real_async(int precision, int n, const void* d_x, const void* d_spectrum,
                           void* d_y, int batch, int channels, void* stream) {
    return conv1d_real_impl(precision, n, d_x, d_spectrum, d_y, batch, channels, stream, false);
}

int thff_conv1d_valid(int precision, const void* d_x, long long input_len, const void* d_taps,
                      int filter_len, void* d_y, int batch, void* stream) {
    return conv1d_valid_impl(precision, d_x, input_len, d_taps, filter_len, d_y, batch, stream,
                             true);
}

int thff_conv1d_valid_async(int precision, const void* d_x, long long input_len,
                            const void* d_taps, int filter_len, void* d_y, int batch,
                            void* stream) {
    return conv1d_valid_impl(precision, d_x, input_len, d_taps, filter_len, d_y, batch, stream,
                             false);
}

int thff_conv2d(int precision, int rows, int cols, const void* d_x, const void* d_h, void* d_y,
                int batch, void* stream) {
    return conv2d_impl(precision, rows, cols, d_x, d_h, d_y, batch, stream, true);
}

int thff_conv2d_async(int precision, int rows, int cols, const void* d_x, const void* d_h,
                      void* d_y, int batch, void* stream) {
    return conv2d_impl(precision, rows, cols, d_x, d_h, d_y, batch, stream, false);
}

int thff_conv2d_noalloc(int precision, int rows, int cols, const void* d_x, const void* d_h,
                        void* d_y, int batch, void* stream) {
    return conv2d_impl(precision, rows, cols, d_x, d_h, d_y, batch, stream, false, false);
}

int thff_twiddle_info(int precision, const void** d_table, int* n) {
    if (!supported_precision(precision)) return fail(THFF_EINVAL, "unsupported precision");
    if (!d_table || !n) return fail(THFF_EINVAL, "thff_twiddle_info: null output pointer");
    std::lock_guard<std::mutex> lock(g_mutex[precision]);
    DeviceTables* d = device_tables(precision, "hipGetDevice (twiddle info)", nullptr);
    if (!d) return THFF_EIO;
    const int live = d->current.load(std::memory_order_acquire);
    *n = live;
    *d_table = live ? d->table[length_slot(live)].load(std::memory_order_acquire) : nullptr;
    return THFF_OK;
}

int thff_fill_uniform(int precision, void* d_out, long long count, unsigned long long seed,
                      long long first_element, void* stream) {
    if (!supported_precision(precision)) return fail(THFF_EINVAL, "unsupported precision");
    if (count < 0 || first_element < 0) return fail(THFF_EINVAL, "negative count or offset");
    if (count == 0) return THFF_OK;
    if (!d_out) return fail(THFF_EINVAL, "thff_fill_uniform: null output");
    const hipError_t err = thff::launch_fill_uniform(precision, d_out, count, seed, first_element,
                                                     static_cast<hipStream_t>(stream));
    if (err != hipSuccess) return fail_hip(err, "thff_fill_uniform launch");
    return THFF_OK;
}

int thff_copy_nt(void* d_dst, const void* d_src, long long bytes, void* stream) {
    if (bytes < 0 || bytes % 16 != 0)
        return fail(THFF_EINVAL, "thff_copy_nt: bytes must be a non-negative multiple of 16");
    if (bytes == 0) return THFF_OK;
    if (!d_dst || !d_src) return fail(THFF_EINVAL, "thff_copy_nt: null pointer");
    const auto d = reinterpret_cast<unsigned long long>(d_dst);
    const auto s = reinterpret_cast<unsigned long long>(d_src);
    if ((d | s) & 15) return fail(THFF_EINVAL, "thff_copy_nt: buffers must be 16-byte aligned");
    const auto ub = static_cast<unsigned long long>(bytes);
    if (d < s + ub && s < d + ub) return fail(THFF_EINVAL, "thff_copy_nt: buffers overlap");
    const hipError_t err = thff::launch_copy_nt(d_dst, d_src, bytes, static_cast<hipStream_t>(stream));
    if (err != hipSuccess) return fail_hip(err, "thff_copy_nt launch");
    return THFF_OK;
}

}  // extern "C"

// Host runtime of libheadshot_hip: error reporting, device queries and the
// stream-ordered row copy (GpuContext::copy_rows, engine/tensor.rs:146-160).
#include <stdarg.h>
#include <stdio.h>

#include <atomic>

#include "hs_common.hpp"

namespace hs {

namespace {
thread_local char g_last_error[512] = "";

constexpr int kMaxDevices = 64;
std::atomic<int> g_cus[kMaxDevices];
}  // namespace

hs_status fail(hs_status code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof g_last_error, fmt, ap);
    va_end(ap);
    return code;
}

hs_status check_launch(const char* what) {
    hipError_t err = hipGetLastError();
    if (err != hipSuccess)
        return fail(HS_EHIP, "%s: kernel launch failed: %s", what, hipGetErrorString(err));
    return HS_OK;
}

int num_cus() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 256;
    int n = g_cus[dev].load(std::memory_order_relaxed);
    if (n > 0) return n;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
        n = 256;
    g_cus[dev].store(n, std::memory_order_relaxed);
    return n;
}

}  // namespace hs

extern "C" {

int32_t hs_abi_version(void) { return HS_ABI_VERSION; }

const char* hs_status_string(hs_status status) {
    switch (status) {
        case HS_OK: return "HS_OK";
        case HS_EINVAL: return "HS_EINVAL";
        case HS_EHIP: return "HS_EHIP";
        case HS_EUNSUPPORTED: return "HS_EUNSUPPORTED";
        default: return "HS_UNKNOWN";
    }
}

const char* hs_last_error(void) { return hs::g_last_error; }

hs_status hs_copy_rows(hs_stream_t stream, const void* src, int64_t src_row, void* dst,
                       int64_t dst_row, int64_t n_rows, int64_t row_bytes) {
    if (n_rows < 0 || row_bytes < 0 || src_row < 0 || dst_row < 0)
        return hs::fail(HS_EINVAL, "copy_rows: negative row index, count or width");
    if (n_rows == 0 || row_bytes == 0) return HS_OK;
    // every byte offset below stays under 2^50
    const int64_t lim = (int64_t{1} << 49) / row_bytes;
    if (n_rows > lim || src_row > lim || dst_row > lim)
        return hs::fail(HS_EINVAL, "copy_rows: rows or width too large");
    if (!src || !dst) return hs::fail(HS_EINVAL, "copy_rows: null buffer");
    const int64_t bytes = n_rows * row_bytes;
    const char* s = static_cast<const char*>(src) + src_row * row_bytes;
    char* d = static_cast<char*>(dst) + dst_row * row_bytes;
    if (hs::overlaps(s, bytes, d, bytes))
        return hs::fail(HS_EINVAL, "copy_rows: source and destination rows overlap");
    hipError_t err = hipMemcpyAsync(d, s, static_cast<size_t>(bytes), hipMemcpyDeviceToDevice,
                                    static_cast<hipStream_t>(stream));
    if (err != hipSuccess)
        return hs::fail(HS_EHIP, "copy_rows: hipMemcpyAsync failed: %s", hipGetErrorString(err));
    return HS_OK;
}

}  // extern "C"

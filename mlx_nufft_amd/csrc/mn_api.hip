// Library-wide state and small entry points: error messages, version,
// geometry validation and the zero-fill kernel.
#include <mutex>

#include "mn_common.h"

namespace mn {

static thread_local std::string g_last_error;

void set_error(const std::string &msg) { g_last_error = msg; }
void clear_error() { g_last_error.clear(); }

int check_bins(const mn_bins *g) {
    MN_REQUIRE(g != nullptr, "bin geometry is NULL");
    MN_REQUIRE(g->dim >= 1 && g->dim <= 3, "dim must be 1, 2 or 3");
    MN_REQUIRE(g->w >= 2 && g->w <= kMaxW, "kernel width w must be in [2, 16]");
    int64_t total = 1;
    for (int d = 0; d < g->dim; ++d) {
        MN_REQUIRE(g->n[d] >= 1 && g->n[d] < (int64_t(1) << 30), "grid size out of range");
        // tile wrap arithmetic covers [-n, 3n), which needs n >= w
        MN_REQUIRE(g->n[d] >= g->w, "grid size must be >= the kernel width w");
        MN_REQUIRE(g->m[d] >= 1 && g->m[d] <= g->n[d], "bin size must be in [1, n]");
        MN_REQUIRE(g->nb[d] == (g->n[d] + g->m[d] - 1) / g->m[d], "nb must equal ceil(n/m)");
        total *= g->nb[d];
    }
    MN_REQUIRE(total < (int64_t(1) << 31), "too many bins");
    return MN_OK;
}

int max_lds_per_block() {
    static int cached[64];
    static std::once_flag once[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 65536;
    std::call_once(once[dev], [dev]() {
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess ||
            v <= 0)
            v = 65536;
        cached[dev] = v;
    });
    return cached[dev];
}

__global__ void k_fill_zero16(uint4 *__restrict__ p, int64_t n16) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (; i < n16; i += stride) p[i] = make_uint4(0u, 0u, 0u, 0u);
}

__global__ void k_fill_zero1(unsigned char *__restrict__ p, int64_t n) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0;
}

int fill_zero(void *ptr, int64_t bytes, hipStream_t s) {
    if (bytes <= 0) return MN_OK;
    MN_REQUIRE(ptr != nullptr, "fill_zero: NULL pointer");
    uintptr_t a = reinterpret_cast<uintptr_t>(ptr);
    int64_t head = (int64_t)((16 - (a & 15)) & 15);
    if (head > bytes) head = bytes;
    if (head) {
        k_fill_zero1<<<1, 64, 0, s>>>(static_cast<unsigned char *>(ptr), head);
        MN_LAUNCH_CHECK("fill_zero");
    }
    int64_t body = (bytes - head) / 16;
    if (body) {
        int64_t blocks = (body + 255) / 256;
        if (blocks > 65536) blocks = 65536;
        k_fill_zero16<<<(unsigned)blocks, 256, 0, s>>>(
            reinterpret_cast<uint4 *>(static_cast<unsigned char *>(ptr) + head), body);
        MN_LAUNCH_CHECK("fill_zero");
    }
    int64_t tail = bytes - head - body * 16;
    if (tail) {
        k_fill_zero1<<<1, 64, 0, s>>>(static_cast<unsigned char *>(ptr) + head + body * 16, tail);
        MN_LAUNCH_CHECK("fill_zero");
    }
    return MN_OK;
}

}  // namespace mn

extern "C" {

const char *mn_last_error(void) { return mn::g_last_error.c_str(); }

int mn_version(void) { return 100; }

int mn_device_lds_bytes(void) {
    mn::clear_error();
    return mn::max_lds_per_block();
}

int mn_fill_zero(void *ptr, int64_t bytes, mn_stream_t stream) {
    mn::clear_error();
    MN_REQUIRE(bytes >= 0, "fill_zero: negative size");
    return mn::fill_zero(ptr, bytes, mn::as_stream(stream));
}

}  // extern "C"

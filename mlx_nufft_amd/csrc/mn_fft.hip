// Fine-grid FFT through rocFFT: in-place complex64 (or complex128) transforms
// with a plan cache keyed by (device, dim, lengths, batch, direction,
// precision). Each cached plan
// owns its execution info and work buffer; execution is asynchronous on the
// caller's stream. The cache is the only mutable library state, guarded by
// a mutex.
// ref: vkfft_bridge/vkfft_bridge.cpp:25-71 (plan cache + in-place execute),
// gpu_t3.py:94-148 and nd.py:374-383 (the FFT stage it serves).
#include <rocfft/rocfft.h>

#include <map>
#include <mutex>
#include <tuple>

#include "mn_common.h"

namespace mn {
namespace {

struct FftKey {
    int dev, dim;
    int64_t n0, n1, n2, batch;
    int dir;
    int f64;  // 1: complex128 (double precision)
    bool operator<(const FftKey &o) const {
        return std::tie(dev, dim, n0, n1, n2, batch, dir, f64) <
               std::tie(o.dev, o.dim, o.n0, o.n1, o.n2, o.batch, o.dir, o.f64);
    }
};

struct FftPlan {
    rocfft_plan plan = nullptr;
    rocfft_execution_info info = nullptr;
    void *work = nullptr;
    size_t work_bytes = 0;
};

std::mutex g_mu;
std::map<FftKey, FftPlan> g_plans;
bool g_setup = false;

#define MN_FFT_CHECK(expr)                                                              \
    do {                                                                                \
        rocfft_status _s = (expr);                                                      \
        if (_s != rocfft_status_success) {                                              \
            ::mn::set_error(std::string(#expr) + " failed, rocfft status " + std::to_string((int)_s)); \
            return MN_ERUNTIME;                                                         \
        }                                                                               \
    } while (0)

void destroy_plan(FftPlan &p) {
    if (p.info) rocfft_execution_info_destroy(p.info);
    if (p.plan) rocfft_plan_destroy(p.plan);
    if (p.work) (void)hipFree(p.work);
    p = FftPlan{};
}

int make_plan(const FftKey &k, FftPlan *out) {
    size_t lengths[3];
    const int64_t n[3] = {k.n0, k.n1, k.n2};
    for (int d = 0; d < k.dim; ++d) lengths[d] = (size_t)n[k.dim - 1 - d];  // fastest first
    FftPlan p;
    rocfft_status st = rocfft_plan_create(
        &p.plan, rocfft_placement_inplace,
        k.dir > 0 ? rocfft_transform_type_complex_inverse : rocfft_transform_type_complex_forward,
        k.f64 ? rocfft_precision_double : rocfft_precision_single, (size_t)k.dim, lengths,
        (size_t)k.batch, nullptr);
    if (st != rocfft_status_success) {
        set_error("rocfft_plan_create failed, status " + std::to_string((int)st));
        return MN_ERUNTIME;
    }
    st = rocfft_plan_get_work_buffer_size(p.plan, &p.work_bytes);
    if (st != rocfft_status_success) {
        destroy_plan(p);
        set_error("rocfft_plan_get_work_buffer_size failed");
        return MN_ERUNTIME;
    }
    st = rocfft_execution_info_create(&p.info);
    if (st != rocfft_status_success) {
        destroy_plan(p);
        set_error("rocfft_execution_info_create failed");
        return MN_ERUNTIME;
    }
    if (p.work_bytes) {
        hipError_t e = hipMalloc(&p.work, p.work_bytes);
        if (e != hipSuccess) {
            p.work = nullptr;
            destroy_plan(p);
            set_error(std::string("FFT work buffer: ") + hipGetErrorString(e));
            return MN_ERUNTIME;
        }
        st = rocfft_execution_info_set_work_buffer(p.info, p.work, p.work_bytes);
        if (st != rocfft_status_success) {
            destroy_plan(p);
            set_error("rocfft_execution_info_set_work_buffer failed");
            return MN_ERUNTIME;
        }
    }
    *out = p;
    return MN_OK;
}

}  // namespace
}  // namespace mn

namespace mn {
namespace {

// Look up (or create) the cached plan and execute it in place on the stream.
int fft_exec(int dim, const int64_t n[3], int64_t batch, int isign, void *data, int f64,
             mn_stream_t stream) {
    MN_REQUIRE(dim >= 1 && dim <= 3, "fft: dim must be 1, 2 or 3");
    MN_REQUIRE(batch >= 1, "fft: batch must be >= 1");
    MN_REQUIRE(data != nullptr, "fft: NULL data");
    FftKey k{};
    MN_HIP_CHECK(hipGetDevice(&k.dev));
    k.dim = dim;
    int64_t nn[3] = {1, 1, 1};
    for (int d = 0; d < dim; ++d) {
        MN_REQUIRE(n[d] >= 1, "fft: lengths must be >= 1");
        nn[d] = n[d];
    }
    k.n0 = nn[0];
    k.n1 = nn[1];
    k.n2 = nn[2];
    k.batch = batch;
    k.dir = isign >= 0 ? 1 : -1;
    k.f64 = f64 ? 1 : 0;
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_setup) {
        MN_FFT_CHECK(rocfft_setup());
        g_setup = true;
    }
    auto it = g_plans.find(k);
    if (it == g_plans.end()) {
        FftPlan p;
        int rc = make_plan(k, &p);
        if (rc) return rc;
        it = g_plans.emplace(k, p).first;
    }
    FftPlan &p = it->second;
    MN_FFT_CHECK(rocfft_execution_info_set_stream(p.info, as_stream(stream)));
    void *buf[1] = {data};
    MN_FFT_CHECK(rocfft_execute(p.plan, buf, nullptr, p.info));
    return MN_OK;
}

}  // namespace
}  // namespace mn

using namespace mn;

extern "C" {

int mn_fft_exec(int dim, const int64_t n[3], int64_t batch, int isign, void *data,
                mn_stream_t stream) {
    clear_error();
    return fft_exec(dim, n, batch, isign, data, 0, stream);
}

int mn_fft_exec_f64(int dim, const int64_t n[3], int64_t batch, int isign, void *data,
                    mn_stream_t stream) {
    clear_error();
    return fft_exec(dim, n, batch, isign, data, 1, stream);
}

int mn_fft_cache_clear(void) {
    clear_error();
    std::lock_guard<std::mutex> lock(g_mu);
    for (auto &kv : g_plans) destroy_plan(kv.second);
    g_plans.clear();
    fftl_cache_clear();
    return MN_OK;
}

}  // extern "C"

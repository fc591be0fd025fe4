// expi: e^{i*isign*phi} for large-magnitude fp64 phases on the GPU.
// The components are summed in native fp64 (left to right) and the fp64
// sincos does the reduction mod 2pi, so there is no magnitude ceiling; the
// result is rounded to complex64. Non-finite phases give NaN per element.
// ref: dfmath.py:29-54 (df64 kernel), dfmath.py:57-134 (expi).
#include "mn_common.h"

namespace mn {
namespace {

constexpr int kMaxComp = 8;
struct Comps { const double *p[kMaxComp]; };

__global__ void k_expi(Comps cs, int ncomp, int64_t n, double sgn, float2 *__restrict__ out) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (; i < n; i += stride) {
        double ph = cs.p[0][i];
        for (int k = 1; k < ncomp; ++k) ph = ph + cs.p[k][i];
        double s, c;
        sincos(sgn * ph, &s, &c);
        out[i] = make_float2((float)c, (float)s);
    }
}

}  // namespace
}  // namespace mn

using namespace mn;

extern "C" {

int mn_expi(int ncomp, const double *const *comps, int64_t n, int isign, void *out,
            mn_stream_t stream) {
    clear_error();
    MN_REQUIRE(ncomp >= 1 && ncomp <= kMaxComp, "expi: ncomp must be in [1, 8]");
    MN_REQUIRE(comps != nullptr && out != nullptr, "expi: NULL pointer");
    MN_REQUIRE(n >= 0, "expi: negative length");
    if (n == 0) return MN_OK;
    Comps c{};
    for (int k = 0; k < ncomp; ++k) {
        MN_REQUIRE(comps[k] != nullptr, "expi: NULL component");
        c.p[k] = comps[k];
    }
    int64_t blocks = (n + 255) / 256;
    if (blocks > 262144) blocks = 262144;
    k_expi<<<(unsigned)blocks, 256, 0, as_stream(stream)>>>(c, ncomp, n, isign >= 0 ? 1.0 : -1.0,
                                                            static_cast<float2 *>(out));
    MN_LAUNCH_CHECK("expi");
    return MN_OK;
}

}  // extern "C"

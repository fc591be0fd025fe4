// Mode shuffle + deconvolution between the FFT-ordered fine grid and the
// modeord=0 mode box, one thread per output element, batched over grids.
//   crop (type 1): fk[m] = grid[(m - N/2) mod n] * prod_d dec_d[m_d]
//                  (ref: nd.py:416-435)
//   pad  (type 2, type-3 inner grid): grid[r] = fk[m] * prod_d dec_d[m_d] in
//                  band, 0 elsewhere (ref: nd.py:878-906, gpu_t3.py:630-651)
// Shapes are right-aligned into 3 slots (unused leading dims have size 1),
// so the last dim is the fastest in memory in both arrays.
#include "mn_common.h"

namespace mn {
namespace {

struct Dec3 { const float *p[3]; };
struct Dec3d { const double *p[3]; };

__global__ void k_crop(int64_t total, int N0, int N1, int N2, int n0, int n1, int n2, Dec3 dec,
                       const float2 *__restrict__ grid, float2 *__restrict__ fk) {
    int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const int64_t gsz = (int64_t)n0 * n1 * n2;
    for (; idx < total; idx += stride) {
        int64_t t = idx;
        const int m2 = (int)(t % N2);
        t /= N2;
        const int m1 = (int)(t % N1);
        t /= N1;
        const int m0 = (int)(t % N0);
        const int64_t bt = t / N0;
        int r0 = m0 - N0 / 2, r1 = m1 - N1 / 2, r2 = m2 - N2 / 2;
        r0 += r0 < 0 ? n0 : 0;
        r1 += r1 < 0 ? n1 : 0;
        r2 += r2 < 0 ? n2 : 0;
        float d = dec.p[0] ? dec.p[0][m0] : 1.0f;
        if (dec.p[1]) d = d * dec.p[1][m1];
        if (dec.p[2]) d = d * dec.p[2][m2];
        const float2 v = grid[bt * gsz + ((int64_t)r0 * n1 + r1) * n2 + r2];
        fk[idx] = make_float2(v.x * d, v.y * d);
    }
}

__global__ void k_pad(int64_t total, int N0, int N1, int N2, int n0, int n1, int n2, Dec3 dec,
                      const float2 *__restrict__ fk, float2 *__restrict__ grid) {
    int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const int64_t fsz = (int64_t)N0 * N1 * N2;
    for (; idx < total; idx += stride) {
        int64_t t = idx;
        const int r2 = (int)(t % n2);
        t /= n2;
        const int r1 = (int)(t % n1);
        t /= n1;
        const int r0 = (int)(t % n0);
        const int64_t bt = t / n0;
        const int q0 = r0 - ((r0 >= n0 - N0 / 2) ? n0 : 0);
        const int q1 = r1 - ((r1 >= n1 - N1 / 2) ? n1 : 0);
        const int q2 = r2 - ((r2 >= n2 - N2 / 2) ? n2 : 0);
        const bool inband = q0 >= -(N0 / 2) && q0 < N0 - N0 / 2 && q1 >= -(N1 / 2) &&
                            q1 < N1 - N1 / 2 && q2 >= -(N2 / 2) && q2 < N2 - N2 / 2;
        float2 out = make_float2(0.0f, 0.0f);
        if (inband) {
            const int m0 = q0 + N0 / 2, m1 = q1 + N1 / 2, m2 = q2 + N2 / 2;
            float d = dec.p[0] ? dec.p[0][m0] : 1.0f;
            if (dec.p[1]) d = d * dec.p[1][m1];
            if (dec.p[2]) d = d * dec.p[2][m2];
            const float2 v = fk[bt * fsz + ((int64_t)m0 * N1 + m1) * N2 + m2];
            out = make_float2(v.x * d, v.y * d);
        }
        grid[idx] = out;
    }
}

// k_pad in double precision: complex128 modes times fp64 factors into a
// complex128 grid (the type-3 inner grid ahead of an fp64 FFT).
__global__ void k_pad_c128(int64_t total, int N0, int N1, int N2, int n0, int n1, int n2,
                           Dec3d dec, const double2 *__restrict__ fk, double2 *__restrict__ grid) {
    int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const int64_t fsz = (int64_t)N0 * N1 * N2;
    for (; idx < total; idx += stride) {
        int64_t t = idx;
        const int r2 = (int)(t % n2);
        t /= n2;
        const int r1 = (int)(t % n1);
        t /= n1;
        const int r0 = (int)(t % n0);
        const int64_t bt = t / n0;
        const int q0 = r0 - ((r0 >= n0 - N0 / 2) ? n0 : 0);
        const int q1 = r1 - ((r1 >= n1 - N1 / 2) ? n1 : 0);
        const int q2 = r2 - ((r2 >= n2 - N2 / 2) ? n2 : 0);
        const bool inband = q0 >= -(N0 / 2) && q0 < N0 - N0 / 2 && q1 >= -(N1 / 2) &&
                            q1 < N1 - N1 / 2 && q2 >= -(N2 / 2) && q2 < N2 - N2 / 2;
        double2 out = make_double2(0.0, 0.0);
        if (inband) {
            const int m0 = q0 + N0 / 2, m1 = q1 + N1 / 2, m2 = q2 + N2 / 2;
            double d = dec.p[0] ? dec.p[0][m0] : 1.0;
            if (dec.p[1]) d = d * dec.p[1][m1];
            if (dec.p[2]) d = d * dec.p[2][m2];
            const double2 v = fk[bt * fsz + ((int64_t)m0 * N1 + m1) * N2 + m2];
            out = make_double2(v.x * d, v.y * d);
        }
        grid[idx] = out;
    }
}

__global__ void k_round_c64(int64_t n, const double2 *__restrict__ in, float2 *__restrict__ out) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (; i < n; i += stride) {
        const double2 v = in[i];
        out[i] = make_float2((float)v.x, (float)v.y);
    }
}

// Right-align dim-sized shapes into 3 slots; dec pointers follow the dims.
int align3(int dim, const int64_t *a, const int64_t *b, const float *const dec[3], int A[3],
           int Bv[3], Dec3 *D) {
    MN_REQUIRE(dim >= 1 && dim <= 3, "dim must be 1, 2 or 3");
    const int off = 3 - dim;
    *D = Dec3{};
    for (int s = 0; s < 3; ++s) {
        A[s] = 1;
        Bv[s] = 1;
    }
    for (int d = 0; d < dim; ++d) {
        MN_REQUIRE(a[d] >= 1 && a[d] < (int64_t(1) << 30), "grid size out of range");
        MN_REQUIRE(b[d] >= 1 && b[d] <= a[d], "mode count must be in [1, n_up]");
        A[off + d] = (int)a[d];
        Bv[off + d] = (int)b[d];
        D->p[off + d] = dec ? dec[d] : nullptr;
    }
    return MN_OK;
}

unsigned grid_blocks(int64_t total) {
    int64_t b = (total + 255) / 256;
    return (unsigned)(b > 262144 ? 262144 : (b < 1 ? 1 : b));
}

}  // namespace
}  // namespace mn

using namespace mn;

extern "C" {

int mn_crop_deconv(int dim, const int64_t n_up[3], const int64_t N[3], int64_t batch,
                   const void *grid, const float *const dec[3], void *fk, mn_stream_t stream) {
    clear_error();
    int n[3], m[3];
    Dec3 D;
    int rc = align3(dim, n_up, N, dec, n, m, &D);
    if (rc) return rc;
    MN_REQUIRE(batch >= 1, "crop: batch must be >= 1");
    MN_REQUIRE(grid && fk, "crop: NULL grid or output");
    const int64_t total = batch * (int64_t)m[0] * m[1] * m[2];
    k_crop<<<grid_blocks(total), 256, 0, as_stream(stream)>>>(
        total, m[0], m[1], m[2], n[0], n[1], n[2], D, static_cast<const float2 *>(grid),
        static_cast<float2 *>(fk));
    MN_LAUNCH_CHECK("crop_deconv");
    return MN_OK;
}

int mn_pad_deconv(int dim, const int64_t n_up[3], const int64_t N[3], int64_t batch,
                  const void *fk, const float *const dec[3], void *grid, mn_stream_t stream) {
    clear_error();
    int n[3], m[3];
    Dec3 D;
    int rc = align3(dim, n_up, N, dec, n, m, &D);
    if (rc) return rc;
    MN_REQUIRE(batch >= 1, "pad: batch must be >= 1");
    MN_REQUIRE(grid && fk, "pad: NULL input or grid");
    const int64_t total = batch * (int64_t)n[0] * n[1] * n[2];
    k_pad<<<grid_blocks(total), 256, 0, as_stream(stream)>>>(
        total, m[0], m[1], m[2], n[0], n[1], n[2], D, static_cast<const float2 *>(fk),
        static_cast<float2 *>(grid));
    MN_LAUNCH_CHECK("pad_deconv");
    return MN_OK;
}

int mn_pad_deconv_c128(int dim, const int64_t n_up[3], const int64_t N[3], int64_t batch,
                       const void *fk, const double *const dec[3], void *grid,
                       mn_stream_t stream) {
    clear_error();
    int n[3], m[3];
    Dec3 D;
    int rc = align3(dim, n_up, N, nullptr, n, m, &D);
    if (rc) return rc;
    MN_REQUIRE(batch >= 1, "pad: batch must be >= 1");
    MN_REQUIRE(grid && fk, "pad: NULL input or grid");
    Dec3d Dd{};
    for (int d = 0; d < dim; ++d) Dd.p[3 - dim + d] = dec ? dec[d] : nullptr;
    const int64_t total = batch * (int64_t)n[0] * n[1] * n[2];
    k_pad_c128<<<grid_blocks(total), 256, 0, as_stream(stream)>>>(
        total, m[0], m[1], m[2], n[0], n[1], n[2], Dd, static_cast<const double2 *>(fk),
        static_cast<double2 *>(grid));
    MN_LAUNCH_CHECK("pad_deconv_c128");
    return MN_OK;
}

int mn_round_c64(int64_t n, const void *in, void *out, mn_stream_t stream) {
    clear_error();
    MN_REQUIRE(n >= 1, "round_c64: n must be >= 1");
    MN_REQUIRE(in && out, "round_c64: NULL input or output");
    k_round_c64<<<grid_blocks(n), 256, 0, as_stream(stream)>>>(
        n, static_cast<const double2 *>(in), static_cast<float2 *>(out));
    MN_LAUNCH_CHECK("round_c64");
    return MN_OK;
}

}  // extern "C"

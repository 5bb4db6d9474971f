// WignerDBasis: per-edge Wigner-D basis matrices in closed form.
//
// The reference computes D = matrix_exp(theta * (a0 G0 + a1 G1)) per edge
// (wigner.py:144-240) with axis a = (-d_y, d_x, 0)/|.| and theta = acos(d_z),
// d = v/(|v| + eps), then returns M = D[:, perm] (wigner.py:358-367).
//
// The generators obey [G0,G1] = G2 (cyclic) and G2 is m-diagonal: it couples
// only the (+m, -m) pair of every irrep.  Writing a = rho (cos phi, sin phi),
//     exp(theta rho (cos phi G0 + sin phi G1)) = Z(phi) V Z(theta rho) V^T Z(-phi)
// with Z(x) = exp(x G2) (2x2 rotations by m x on each pair) and the constant
// V = exp(pi/2 G1) (host-built in float64 per irrep).  Each thread produces
// one column j of M, i.e. column perm[j] of D, by applying the five factors
// to a unit vector: O(n^2) work per column, no matrix exponential.
//
// Plan layout per irrep (lvals order), n = 2l+1 doubles blocks:
//   V (n*n, row-major) | z (n): signed m coupling of each row | partner (n)
#include "feq_internal.h"

#include <cfloat>
#include <cmath>

namespace feq {
namespace {

constexpr int kMaxN = 2 * (FEQ_MAX_BLOCKS - 1) + 1;  // 33

struct WignerArgs {
    int32_t nirr;
    int32_t dim;
    int32_t lvals[FEQ_MAX_IRREPS];
    int32_t off[FEQ_MAX_IRREPS];       // component offset of every irrep
    int32_t plan_off[FEQ_MAX_IRREPS];  // offset of every irrep's plan block (doubles)
};

__device__ __forceinline__ float sanitize(double v) {
    // nan_to_num(x, 0.0): NaN -> 0, +-inf -> +-FLT_MAX
    if (v != v) return 0.0f;
    if (v > static_cast<double>(FLT_MAX)) return FLT_MAX;
    if (v < -static_cast<double>(FLT_MAX)) return -FLT_MAX;
    return static_cast<float>(v);
}

__global__ void __launch_bounds__(256)
k_wigner(WignerArgs A, const double* __restrict__ plan, const int32_t* __restrict__ perm,
         int64_t E, const float* __restrict__ dirs, float* __restrict__ out) {
    const int64_t g = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
    const int dim = A.dim;
    if (g >= E * dim) return;
    const int64_t e = g / dim;
    const int j = static_cast<int>(g % dim);
    const int c0 = perm[j];
    int k = 0;
    while (k + 1 < A.nirr && c0 >= A.off[k + 1]) ++k;
    const int l = A.lvals[k], n = 2 * l + 1, base = A.off[k];
    const int c = c0 - base;
    float* col = out + e * dim * dim + j;  // element (row r) at col[r * dim]

    // ---- edge frame, float32 like rot_to_ez -----------------------------------
    const float eps = 1e-8f;
    const float vx = dirs[3 * e], vy = dirs[3 * e + 1], vz = dirs[3 * e + 2];
    const float nv = sqrtf(vx * vx + vy * vy + vz * vz) + eps;
    const float dx = vx / nv, dy = vy / nv, dz = vz / nv;
    const float a0r = -dy, a1r = dx;
    const float na = sqrtf(a0r * a0r + a1r * a1r) + eps;
    const float a0 = a0r / na, a1 = a1r / na;
    const float theta = acosf(fminf(fmaxf(dz, -1.0f), 1.0f));

    double y[kMaxN];
    const double* V = plan + A.plan_off[k];
    const double* z = V + n * n;
    const double* pr = z + n;
    const double rho = sqrt(static_cast<double>(a0) * a0 + static_cast<double>(a1) * a1);
    if (l == 0) {
        y[0] = 1.0;
    } else if (rho == 0.0) {
        for (int r = 0; r < n; ++r) y[r] = r == c ? 1.0 : 0.0;
    } else {
        const double phi = atan2(static_cast<double>(a1), static_cast<double>(a0));
        const double ang = static_cast<double>(theta) * rho;
        // cos/sin of k*phi and k*ang, k = 0..l, by the angle-addition recurrence
        double cp[FEQ_MAX_BLOCKS], sp[FEQ_MAX_BLOCKS], ca[FEQ_MAX_BLOCKS], sa[FEQ_MAX_BLOCKS];
        cp[0] = 1.0; sp[0] = 0.0; ca[0] = 1.0; sa[0] = 0.0;
        double c1p, s1p, c1a, s1a;
        sincos(phi, &s1p, &c1p);
        sincos(ang, &s1a, &c1a);
        for (int q = 1; q <= l; ++q) {
            cp[q] = cp[q - 1] * c1p - sp[q - 1] * s1p;
            sp[q] = sp[q - 1] * c1p + cp[q - 1] * s1p;
            ca[q] = ca[q - 1] * c1a - sa[q - 1] * s1a;
            sa[q] = sa[q - 1] * c1a + ca[q - 1] * s1a;
        }
        // sin/cos of (zr * x) with zr a signed integer
        auto zc = [&](int r, const double* cc) { int m = static_cast<int>(z[r]); return cc[m < 0 ? -m : m]; };
        auto zs = [&](int r, const double* ss) { int m = static_cast<int>(z[r]); double v = ss[m < 0 ? -m : m]; return m < 0 ? -v : v; };
        // v1 = Z(-phi) e_c: entries at c and its partner p
        const int p = static_cast<int>(pr[c]);
        const double v_c = zc(c, cp);
        const double v_p = p != c ? -zs(p, sp) : 0.0;
        // w = V^T v1
        double w[kMaxN], u[kMaxN];
        for (int q = 0; q < n; ++q) w[q] = V[c * n + q] * v_c + (p != c ? V[p * n + q] * v_p : 0.0);
        // u = Z(ang) w
        for (int r = 0; r < n; ++r) {
            const int pr_r = static_cast<int>(pr[r]);
            u[r] = zc(r, ca) * w[r] + (pr_r != r ? zs(r, sa) * w[pr_r] : 0.0);
        }
        // x = V u  (reuse w)
        for (int r = 0; r < n; ++r) {
            double acc = 0.0;
            for (int q = 0; q < n; ++q) acc += V[r * n + q] * u[q];
            w[r] = acc;
        }
        // y = Z(phi) x
        for (int r = 0; r < n; ++r) {
            const int pr_r = static_cast<int>(pr[r]);
            y[r] = zc(r, cp) * w[r] + (pr_r != r ? zs(r, sp) * w[pr_r] : 0.0);
        }
    }
    for (int r = 0; r < dim; ++r) {
        float v = 0.0f;
        if (r >= base && r < base + n) v = sanitize(y[r - base]);
        col[static_cast<int64_t>(r) * dim] = v;
    }
}

}  // namespace
}  // namespace feq

using namespace feq;

extern "C" size_t feq_wigner_plan_doubles(const int32_t* lvals, int32_t n) {
    size_t s = 0;
    for (int i = 0; i < n; ++i) {
        const size_t d = 2 * static_cast<size_t>(lvals[i]) + 1;
        s += d * d + 2 * d;
    }
    return s;
}

extern "C" int feq_wigner_basis(const int32_t* lvals, int32_t n, const double* plan,
                                const int32_t* perm, int64_t E, const float* dirs, float* out,
                                feq_stream_t stream) {
    if (!lvals || n < 1) return fail(FEQ_ERR_INVALID, "lvals must be non-empty");
    if (n > FEQ_MAX_IRREPS) return fail(FEQ_ERR_UNSUPPORTED, "more than %d irreps", FEQ_MAX_IRREPS);
    if (E < 0) return fail(FEQ_ERR_INVALID, "negative edge count");
    WignerArgs A{};
    A.nirr = n;
    int dim = 0;
    size_t po = 0;
    for (int i = 0; i < n; ++i) {
        if (lvals[i] < 0 || lvals[i] >= FEQ_MAX_BLOCKS)
            return fail(FEQ_ERR_UNSUPPORTED, "degree %d outside [0, %d]", lvals[i], FEQ_MAX_BLOCKS - 1);
        A.lvals[i] = lvals[i];
        A.off[i] = dim;
        A.plan_off[i] = static_cast<int32_t>(po);
        const int d = 2 * lvals[i] + 1;
        dim += d;
        po += static_cast<size_t>(d) * d + 2 * d;
    }
    A.dim = dim;
    if (E == 0) return FEQ_OK;
    if (!plan || !perm || !dirs || !out) return fail(FEQ_ERR_INVALID, "NULL pointer");
    const int64_t total = E * dim;
    FEQ_LAUNCH("k_wigner", k_wigner, dim3(ceil_div(total, 256)), dim3(256), 0, stream_of(stream), A,
                       plan, perm, E, dirs, out);
    return FEQ_OK;
}

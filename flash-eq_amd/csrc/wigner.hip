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

// Column c of D for an irrep of degree L (n = 2L + 1) and edge angles (phi,
// ang = theta rho): D = Z(phi) V Z(ang) V^T Z(-phi), where Z(x) rotates the
// (r, 2L - r) pair by (L - r) x -- the structure of the m-diagonal generator,
// which the host checks when it builds V.  All indices are compile-time, so
// the vectors live in registers.
template <int L>
__device__ __forceinline__ void wigner_column(const double* __restrict__ V, int c, double phi,
                                              double ang, double (&y)[2 * L + 1]) {
    constexpr int n = 2 * L + 1;
    double cp[L + 1], sp[L + 1], ca[L + 1], sa[L + 1];
    cp[0] = 1.0;
    sp[0] = 0.0;
    ca[0] = 1.0;
    sa[0] = 0.0;
    double c1p, s1p, c1a, s1a;
    sincos(phi, &s1p, &c1p);
    sincos(ang, &s1a, &c1a);
#pragma unroll
    for (int q = 1; q <= L; ++q) {
        cp[q] = cp[q - 1] * c1p - sp[q - 1] * s1p;
        sp[q] = sp[q - 1] * c1p + cp[q - 1] * s1p;
        ca[q] = ca[q - 1] * c1a - sa[q - 1] * s1a;
        sa[q] = sa[q - 1] * c1a + ca[q - 1] * s1a;
    }
    // v1 = Z(-phi) e_c: entries at c (cos) and its partner n-1-c (sin of the
    // partner's coupling), then w = V^T v1
    const int pc = n - 1 - c;
    const int mc = L - c;                         // coupling of row c
    const int amc = mc < 0 ? -mc : mc;
    double cphi = 1.0, sphi = 0.0;
#pragma unroll
    for (int q = 0; q <= L; ++q)
        if (q == amc) {
            cphi = cp[q];
            sphi = sp[q];
        }
    const double v_c = cphi;
    const double v_p = pc != c ? (mc < 0 ? -sphi : sphi) : 0.0;
    double w[n], u[n];
#pragma unroll
    for (int q = 0; q < n; ++q) w[q] = V[c * n + q] * v_c + V[pc * n + q] * v_p;
    // u = Z(ang) w
#pragma unroll
    for (int r = 0; r < n; ++r) {
        const int m = L - r, am = m < 0 ? -m : m;
        u[r] = ca[am] * w[r] + (r != L ? (m < 0 ? -sa[am] : sa[am]) * w[n - 1 - r] : 0.0);
    }
    // x = V u, y = Z(phi) x
    double xv[n];
#pragma unroll
    for (int r = 0; r < n; ++r) {
        double acc = 0.0;
#pragma unroll
        for (int q = 0; q < n; ++q) acc += V[r * n + q] * u[q];
        xv[r] = acc;
    }
#pragma unroll
    for (int r = 0; r < n; ++r) {
        const int m = L - r, am = m < 0 ? -m : m;
        y[r] = cp[am] * xv[r] + (r != L ? (m < 0 ? -sp[am] : sp[am]) * xv[n - 1 - r] : 0.0);
    }
}

template <int L>
__device__ __forceinline__ void column_into(const double* V, int c, double phi, double ang,
                                            bool ident, float* dst, int stride) {
    constexpr int n = 2 * L + 1;
    double y[n];
    if (L == 0) {
        y[0] = 1.0;
    } else if (ident) {
#pragma unroll
        for (int r = 0; r < n; ++r) y[r] = r == c ? 1.0 : 0.0;
    } else {
        wigner_column<L>(V, c, phi, ang, y);
    }
#pragma unroll
    for (int r = 0; r < n; ++r) dst[r * stride] = sanitize(y[r]);
}

struct EdgeFrame {
    double phi, ang;
    int ident;   // axis of zero length: D = I
};

// Workgroup: a tile of EPB edges; thread t computes standard column c0 = t % dim
// of edge t / dim into an LDS tile of the edges' M = D[:, perm] matrices, which
// is then written with coalesced stores.
__global__ void __launch_bounds__(256)
k_wigner(WignerArgs A, int epb, const double* __restrict__ plan, const int32_t* __restrict__ perm,
         int64_t E, const float* __restrict__ dirs, float* __restrict__ out) {
    extern __shared__ float sM[];                      // epb x dim x dim
    __shared__ EdgeFrame sFr[256];
    __shared__ int sInv[FEQ_MAX_SLOTS];
    const int dim = A.dim, dd = dim * dim;
    const int64_t e0 = static_cast<int64_t>(blockIdx.x) * epb;
    const int ne = static_cast<int>(E - e0 < epb ? E - e0 : epb);
    for (int q = threadIdx.x; q < epb * dd; q += blockDim.x) sM[q] = 0.0f;
    for (int j = threadIdx.x; j < dim; j += blockDim.x) sInv[perm[j]] = j;
    if (threadIdx.x < ne) {
        // edge frame in float32 like rot_to_ez: d = v/(|v|+eps), axis = (-d_y, d_x, 0)/(|.|+eps),
        // theta = acos(clamp(d_z, -1, 1)); a = rho (cos phi, sin phi)
        const int64_t e = e0 + threadIdx.x;
        const float eps = 1e-8f;
        const float vx = dirs[3 * e], vy = dirs[3 * e + 1], vz = dirs[3 * e + 2];
        const float nv = sqrtf(vx * vx + vy * vy + vz * vz) + eps;
        const float dx = vx / nv, dy = vy / nv, dz = vz / nv;
        const float a0r = -dy, a1r = dx;
        const float na = sqrtf(a0r * a0r + a1r * a1r) + eps;
        const float a0 = a0r / na, a1 = a1r / na;
        const float theta = acosf(fminf(fmaxf(dz, -1.0f), 1.0f));
        const double rho = sqrt(static_cast<double>(a0) * a0 + static_cast<double>(a1) * a1);
        EdgeFrame f;
        f.ident = rho == 0.0;
        f.phi = f.ident ? 0.0 : atan2(static_cast<double>(a1), static_cast<double>(a0));
        f.ang = static_cast<double>(theta) * rho;
        sFr[threadIdx.x] = f;
    }
    __syncthreads();
    const int el = threadIdx.x / dim;
    if (el < ne) {
        const int c0 = threadIdx.x % dim;
        int k = 0;
        while (k + 1 < A.nirr && c0 >= A.off[k + 1]) ++k;
        const int l = A.lvals[k], base = A.off[k], c = c0 - base;
        const double* V = plan + A.plan_off[k];
        const EdgeFrame f = sFr[el];
        float* dst = sM + el * dd + base * dim + sInv[c0];   // rows base.., column j
        switch (l) {
#define FEQ_WCASE(LL) \
    case LL: column_into<LL>(V, c, f.phi, f.ang, f.ident, dst, dim); break;
            FEQ_WCASE(0) FEQ_WCASE(1) FEQ_WCASE(2) FEQ_WCASE(3) FEQ_WCASE(4) FEQ_WCASE(5)
            FEQ_WCASE(6) FEQ_WCASE(7) FEQ_WCASE(8) FEQ_WCASE(9) FEQ_WCASE(10) FEQ_WCASE(11)
            FEQ_WCASE(12) FEQ_WCASE(13) FEQ_WCASE(14) FEQ_WCASE(15) FEQ_WCASE(16)
#undef FEQ_WCASE
            default: break;
        }
    }
    __syncthreads();
    float* o = out + e0 * dd;
    for (int q = threadIdx.x; q < ne * dd; q += blockDim.x) o[q] = sM[q];
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
    // one thread per (edge, column); the edges' matrices are staged in LDS
    const int epb = 256 / dim;
    const size_t lds = sizeof(float) * static_cast<size_t>(epb) * dim * dim;
    if (lds > 64 * 1024) return fail(FEQ_ERR_UNSUPPORTED, "representation dimension %d too large", dim);
    FEQ_LAUNCH("k_wigner", k_wigner, dim3(ceil_div(E, epb)), dim3(256), lds, stream_of(stream), A,
               epb, plan, perm, E, dirs, out);
    return FEQ_OK;
}

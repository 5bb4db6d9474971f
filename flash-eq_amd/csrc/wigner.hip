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
#include <type_traits>

namespace feq {
namespace {

struct WignerArgs {
    int32_t nirr;
    int32_t dim;
    int32_t lvals[FEQ_MAX_IRREPS];
    int32_t off[FEQ_MAX_IRREPS];       // component offset of every irrep
    int32_t plan_off[FEQ_MAX_IRREPS];  // offset of every irrep's plan block (doubles)
};

// nan_to_num(x, 0.0) in the output type: NaN -> 0, +-inf -> +-max
template <class T>
__device__ __forceinline__ T sanitize(double v) {
    if (v != v) return T(0);
    if constexpr (std::is_same_v<T, float>) {
        if (v > static_cast<double>(FLT_MAX)) return FLT_MAX;
        if (v < -static_cast<double>(FLT_MAX)) return -FLT_MAX;
        return static_cast<float>(v);
    } else {
        if (v > DBL_MAX) return DBL_MAX;
        if (v < -DBL_MAX) return -DBL_MAX;
        return v;
    }
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

template <int L, class T>
__device__ __forceinline__ void column_into(const double* V, int c, double phi, double ang,
                                            bool ident, T* dst, int stride) {
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
    for (int r = 0; r < n; ++r) dst[r * stride] = sanitize<T>(y[r]);
}

struct EdgeFrame {
    double phi, ang;
    int ident;   // axis of zero length: D = I
};

// Workgroup: a tile of EPB edges; thread t computes standard column c0 = t % dim
// of edge t / dim into an LDS tile of the edges' M = D[:, perm] matrices, which
// is then written with coalesced stores.
// LMAX: the largest degree the launch handles (the register footprint of the
// per-column vectors grows with it, so small representations get a small kernel).
// T = float: the frame in float32, as the reference's float32 rot_to_ez (whose
// clamp bounds +-(1 - eps) round to +-1); T = double: the frame in float64 with
// the clamp as written (a float64 module runs rot_to_ez in float64).
template <int LMAX, class T>
__global__ void __launch_bounds__(256)
k_wigner(WignerArgs A, int epb, const double* __restrict__ plan, const int32_t* __restrict__ perm,
         int64_t E, const T* __restrict__ dirs, T* __restrict__ out) {
    extern __shared__ __align__(16) char sMraw[];
    T* sM = reinterpret_cast<T*>(sMraw);              // epb x dim x dim
    __shared__ EdgeFrame sFr[256];
    __shared__ int sInv[FEQ_MAX_SLOTS];
    const int dim = A.dim, dd = dim * dim;
    const int64_t e0 = static_cast<int64_t>(blockIdx.x) * epb;
    const int ne = static_cast<int>(E - e0 < epb ? E - e0 : epb);
    for (int q = threadIdx.x; q < epb * dd; q += blockDim.x) sM[q] = T(0);
    for (int j = threadIdx.x; j < dim; j += blockDim.x) sInv[perm[j]] = j;
    if (threadIdx.x < ne) {
        // edge frame in float32 like rot_to_ez: d = v/(|v|+eps), axis = (-d_y, d_x, 0)/(|.|+eps),
        // theta = acos(clamp(d_z, -1, 1)); a = rho (cos phi, sin phi)
        const int64_t e = e0 + threadIdx.x;
        const T eps = T(1e-8);
        const T vx = dirs[3 * e], vy = dirs[3 * e + 1], vz = dirs[3 * e + 2];
        const T nv = sqrt(vx * vx + vy * vy + vz * vz) + eps;
        const T dx = vx / nv, dy = vy / nv, dz = vz / nv;
        const T a0r = -dy, a1r = dx;
        const T na = sqrt(a0r * a0r + a1r * a1r) + eps;
        const T a0 = a0r / na, a1 = a1r / na;
        const T theta = acos(fmin(fmax(dz, T(-1) + eps), T(1) - eps));
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
        T* dst = sM + el * dd + base * dim + sInv[c0];   // rows base.., column j
        switch (l) {
#define FEQ_WCASE(LL) \
    case LL:                                                                             \
        if constexpr (LL <= LMAX) column_into<LL>(V, c, f.phi, f.ang, f.ident, dst, dim); \
        break;
            FEQ_WCASE(0) FEQ_WCASE(1) FEQ_WCASE(2) FEQ_WCASE(3) FEQ_WCASE(4) FEQ_WCASE(5)
            FEQ_WCASE(6) FEQ_WCASE(7) FEQ_WCASE(8) FEQ_WCASE(9) FEQ_WCASE(10) FEQ_WCASE(11)
            FEQ_WCASE(12) FEQ_WCASE(13) FEQ_WCASE(14) FEQ_WCASE(15) FEQ_WCASE(16)
#undef FEQ_WCASE
            default: break;
        }
    }
    __syncthreads();
    T* o = out + e0 * dd;
    for (int q = threadIdx.x; q < ne * dd; q += blockDim.x) o[q] = sM[q];
}

// ---- backward: gradient with respect to the edge directions --------------------------
//
// With X(phi) = cos(phi) G0 + sin(phi) G1 = Z(phi) V G2 V^T Z(-phi) and the
// exponent theta (a0 G0 + a1 G1) = ang X(phi) (a = rho (cos phi, sin phi),
// ang = theta rho), the derivatives of D = exp(ang X(phi)) are exact and cheap:
//     dD/dang = X D,        dD/dphi = G2 D - D G2
// (phi enters as a conjugation by the z-rotation Z(phi) = exp(phi G2)).  Each
// thread takes one column c of an irrep block of D and adds, with G = dL/dD
// (the columns of dL/dM moved back through perm):
//     <G[:,c], X D[:,c]>                                 to dL/dang,
//     <G[:,c], G2 D[:,c]> - z_c <G[:,pc], D[:,c]>        to dL/dphi
// (z_c = L - c: G2's coupling of row c to its partner row pc = n-1-c).  At
// rho = 0 (the forward's D = I) the exponent is theta (a0 G0 + a1 G1) at a = 0,
// whose derivative is dD/da_k = theta G_k: the threads add <G[:,c], G_k e_c>.
// One thread per edge then chains (phi, ang) -- or (a0, a1) -- back through
// a = a_raw/(|a_raw|+eps), a_raw = (-d_y, d_x), theta = acos(d_z) and
// d = v/(|v|+eps), the operations of rot_to_ez (wigner.py:220-238), with
// torch's conventions (the norm's gradient is 0 at 0).

// out = X(phi) y for one irrep: Z(phi) V G2 V^T Z(-phi) y, with cos(q phi),
// sin(q phi) for q = 0..L in cpm, spm.
template <int L>
__device__ __forceinline__ void apply_axis_generator(const double* __restrict__ V,
                                                     const double (&cpm)[L + 1],
                                                     const double (&spm)[L + 1],
                                                     const double (&y)[2 * L + 1],
                                                     double (&out)[2 * L + 1]) {
    constexpr int n = 2 * L + 1;
    double u[n], w[n], x[n];
    // u = Z(-phi) y
#pragma unroll
    for (int r = 0; r < n; ++r) {
        const int m = L - r, am = m < 0 ? -m : m;
        u[r] = cpm[am] * y[r] - (r != L ? (m < 0 ? -spm[am] : spm[am]) * y[n - 1 - r] : 0.0);
    }
    // w = V^T u
#pragma unroll
    for (int q = 0; q < n; ++q) {
        double acc = 0.0;
#pragma unroll
        for (int r = 0; r < n; ++r) acc += V[r * n + q] * u[r];
        w[q] = acc;
    }
    // w <- G2 w: (G2 w)[r] = (L - r) w[n-1-r]
#pragma unroll
    for (int r = 0; r < n; ++r) u[r] = static_cast<double>(L - r) * w[n - 1 - r];
    // x = V u
#pragma unroll
    for (int r = 0; r < n; ++r) {
        double acc = 0.0;
#pragma unroll
        for (int q = 0; q < n; ++q) acc += V[r * n + q] * u[q];
        x[r] = acc;
    }
    // out = Z(phi) x
#pragma unroll
    for (int r = 0; r < n; ++r) {
        const int m = L - r, am = m < 0 ? -m : m;
        out[r] = cpm[am] * x[r] + (r != L ? (m < 0 ? -spm[am] : spm[am]) * x[n - 1 - r] : 0.0);
    }
}

template <int L>
__device__ __forceinline__ void multiples(double ang, double (&c)[L + 1], double (&s)[L + 1]) {
    c[0] = 1.0;
    s[0] = 0.0;
    if (L == 0) return;
    double s1, c1;
    sincos(ang, &s1, &c1);
#pragma unroll
    for (int q = 1; q <= L; ++q) {
        c[q] = c[q - 1] * c1 - s[q - 1] * s1;
        s[q] = s[q - 1] * c1 + c[q - 1] * s1;
    }
}

// Contributions of column c of one irrep block.  gcol / gpar: columns c and
// n-1-c of dL/dD restricted to the block's rows.  t0/t1: (dL/dang, dL/dphi), or
// at rho = 0 (ident) (dL/da0, dL/da1) without the factor theta.
template <int L, class T>
__device__ __forceinline__ void column_grad(const double* V, int c, double phi, double ang,
                                            bool ident, const T* gcol, const T* gpar,
                                            int stride, double& t0, double& t1) {
    constexpr int n = 2 * L + 1;
    t0 = 0.0;
    t1 = 0.0;
    if (L == 0) return;                       // D = 1 is constant
    double g[n], gp[n], y[n], xy[n];
#pragma unroll
    for (int r = 0; r < n; ++r) {
        g[r] = gcol[r * stride];
        gp[r] = gpar[r * stride];
    }
    if (ident) {
        double cz[L + 1], sz[L + 1], c9[L + 1], s9[L + 1];
        multiples<L>(0.0, cz, sz);
        multiples<L>(0.5 * M_PI, c9, s9);
#pragma unroll
        for (int r = 0; r < n; ++r) y[r] = r == c ? 1.0 : 0.0;
        apply_axis_generator<L>(V, cz, sz, y, xy);      // G0 e_c
#pragma unroll
        for (int r = 0; r < n; ++r) t0 += g[r] * xy[r];
        apply_axis_generator<L>(V, c9, s9, y, xy);      // G1 e_c
#pragma unroll
        for (int r = 0; r < n; ++r) t1 += g[r] * xy[r];
        return;
    }
    wigner_column<L>(V, c, phi, ang, y);
    double cp[L + 1], sp[L + 1];
    multiples<L>(phi, cp, sp);
    apply_axis_generator<L>(V, cp, sp, y, xy);
#pragma unroll
    for (int r = 0; r < n; ++r) {
        t0 += g[r] * xy[r];
        t1 += g[r] * static_cast<double>(L - r) * y[n - 1 - r] - static_cast<double>(L - c) * gp[r] * y[r];
    }
}

template <int LMAX, class T>
__global__ void __launch_bounds__(256)
k_wigner_bwd(WignerArgs A, int epb, const double* __restrict__ plan, const int32_t* __restrict__ perm,
             int64_t E, const T* __restrict__ dirs, const T* __restrict__ gM,
             T* __restrict__ gdirs) {
    extern __shared__ __align__(16) char sGraw[];
    T* sG = reinterpret_cast<T*>(sGraw);              // epb x dim x dim (dL/dM tile)
    __shared__ EdgeFrame sFr[256];
    __shared__ int sInv[FEQ_MAX_SLOTS];
    __shared__ double sT0[256], sT1[256];
    const int dim = A.dim, dd = dim * dim;
    const int64_t e0 = static_cast<int64_t>(blockIdx.x) * epb;
    const int ne = static_cast<int>(E - e0 < epb ? E - e0 : epb);
    const T* gsrc = gM + e0 * dd;
    for (int q = threadIdx.x; q < ne * dd; q += blockDim.x) sG[q] = gsrc[q];
    for (int j = threadIdx.x; j < dim; j += blockDim.x) sInv[perm[j]] = j;
    // The frame in double from the float32 directions: near the poles (|d_z| -> 1)
    // d theta / d d_z = -1/sqrt(1 - d_z^2) amplifies the float32 rounding of d_z
    // (1 - |d_z| = 3e-6 loses 2% to it), while the forward's matrices are
    // insensitive to it; the gradient is therefore formed from an exact frame.
    double dxv = 0.0, dyv = 0.0, dzv = 0.0, nvv = 0.0, nav = 0.0, a0v = 0.0, a1v = 0.0, thv = 0.0;
    const double eps = 1e-8;
    if (threadIdx.x < ne) {
        const int64_t e = e0 + threadIdx.x;
        const double vx = dirs[3 * e], vy = dirs[3 * e + 1], vz = dirs[3 * e + 2];
        nvv = sqrt(vx * vx + vy * vy + vz * vz);
        const double nv = nvv + eps;
        dxv = vx / nv;
        dyv = vy / nv;
        dzv = vz / nv;
        const double a0r = -dyv, a1r = dxv;
        nav = sqrt(a0r * a0r + a1r * a1r);
        const double na = nav + eps;
        a0v = a0r / na;
        a1v = a1r / na;
        // the reference's clamp to [-1 + eps, 1 - eps] (wigner.py:235), which
        // binds in float64 (within ~1.4e-4 rad of the poles; in float32 its
        // bounds round to +-1, as the forward's float32 frame has them)
        thv = acos(fmin(fmax(dzv, -1.0 + eps), 1.0 - eps));
        const double rho = sqrt(a0v * a0v + a1v * a1v);
        EdgeFrame f;
        f.ident = rho == 0.0;
        f.phi = f.ident ? 0.0 : atan2(a1v, a0v);
        f.ang = thv * rho;
        sFr[threadIdx.x] = f;
    }
    __syncthreads();
    const int el = threadIdx.x / dim;
    double t0 = 0.0, t1 = 0.0;
    if (el < ne) {
        const int c0 = threadIdx.x % dim;
        int k = 0;
        while (k + 1 < A.nirr && c0 >= A.off[k + 1]) ++k;
        const int l = A.lvals[k], base = A.off[k], c = c0 - base, n = 2 * l + 1;
        const double* V = plan + A.plan_off[k];
        const EdgeFrame f = sFr[el];
        // column c of dL/dD is column sInv[c] of dL/dM; rows base.. of the block
        const T* gcol = sG + el * dd + base * dim + sInv[c0];
        const T* gpar = sG + el * dd + base * dim + sInv[base + n - 1 - c];
        switch (l) {
#define FEQ_WCASE(LL)                                                                    \
    case LL:                                                                             \
        if constexpr (LL <= LMAX)                                                        \
            column_grad<LL>(V, c, f.phi, f.ang, f.ident, gcol, gpar, dim, t0, t1);       \
        break;
            FEQ_WCASE(0) FEQ_WCASE(1) FEQ_WCASE(2) FEQ_WCASE(3) FEQ_WCASE(4) FEQ_WCASE(5)
            FEQ_WCASE(6) FEQ_WCASE(7) FEQ_WCASE(8) FEQ_WCASE(9) FEQ_WCASE(10) FEQ_WCASE(11)
            FEQ_WCASE(12) FEQ_WCASE(13) FEQ_WCASE(14) FEQ_WCASE(15) FEQ_WCASE(16)
#undef FEQ_WCASE
            default: break;
        }
    }
    sT0[threadIdx.x] = t0;
    sT1[threadIdx.x] = t1;
    __syncthreads();
    if (threadIdx.x >= ne) return;
    // per edge: sum the columns in a fixed order, then the chain rule
    double s0 = 0.0, s1 = 0.0;
    for (int q = 0; q < dim; ++q) {
        s0 += sT0[threadIdx.x * dim + q];
        s1 += sT1[threadIdx.x * dim + q];
    }
    const EdgeFrame f = sFr[threadIdx.x];
    const double th = thv, a0 = a0v, a1 = a1v;
    double ga0, ga1, gth;
    if (f.ident) {
        ga0 = th * s0;
        ga1 = th * s1;
        gth = 0.0;                            // the exponent theta * (a . G) vanishes with a
    } else {
        const double rho = sqrt(a0 * a0 + a1 * a1);
        const double cph = a0 / rho, sph = a1 / rho;
        const double grho = th * s0;          // ang = theta rho
        gth = rho * s0;
        ga0 = cph * grho - sph / rho * s1;
        ga1 = sph * grho + cph / rho * s1;
    }
    // a = a_raw / (|a_raw| + eps), a_raw = (-d_y, d_x)
    const double ar0 = -dyv, ar1 = dxv, na = nav, ta = na + eps;
    double gr0 = ga0 / ta, gr1 = ga1 / ta;
    if (na > 0.0) {
        const double dotp = (ga0 * ar0 + ga1 * ar1) / (na * ta * ta);
        gr0 -= dotp * ar0;
        gr1 -= dotp * ar1;
    }
    double gd0 = gr1, gd1 = -gr0, gd2 = 0.0;
    // theta = acos(clamp(d_z, -1 + eps, 1 - eps)): -1/sqrt(1 - d_z^2) where the
    // clamp passes d_z, 0 where it binds (torch's clamp gradient), so the
    // directions along +-e_z get finite gradients, the float64 values of the
    // reference's formula (its float32 autograd has 0 * -inf = NaN there)
    const double dz = dzv;
    if (gth != 0.0 && dz >= -1.0 + eps && dz <= 1.0 - eps) gd2 = -gth / sqrt(1.0 - dz * dz);
    // d = v / (|v| + eps)
    const int64_t e = e0 + threadIdx.x;
    const double vx = dirs[3 * e], vy = dirs[3 * e + 1], vz = dirs[3 * e + 2];
    const double nv = nvv, tv = nv + eps;
    double gv0 = gd0 / tv, gv1 = gd1 / tv, gv2 = gd2 / tv;
    if (nv > 0.0) {
        const double dotv = (gd0 * vx + gd1 * vy + gd2 * vz) / (nv * tv * tv);
        gv0 -= dotv * vx;
        gv1 -= dotv * vy;
        gv2 -= dotv * vz;
    }
    gdirs[3 * e] = static_cast<T>(gv0);
    gdirs[3 * e + 1] = static_cast<T>(gv1);
    gdirs[3 * e + 2] = static_cast<T>(gv2);
}

// Calls f with std::integral_constant<int, LMAX> for the smallest compiled LMAX
// that covers every degree of A.
template <class Fn>
int with_lmax(const WignerArgs& A, Fn&& f) {
    int lmax = 0;
    for (int i = 0; i < A.nirr; ++i) lmax = A.lvals[i] > lmax ? A.lvals[i] : lmax;
    if (lmax <= 2) return f(std::integral_constant<int, 2>{});
    if (lmax <= 4) return f(std::integral_constant<int, 4>{});
    if (lmax <= 6) return f(std::integral_constant<int, 6>{});
    if (lmax <= 10) return f(std::integral_constant<int, 10>{});
    return f(std::integral_constant<int, 16>{});
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

namespace {
int wigner_args(const int32_t* lvals, int32_t n, WignerArgs& A) {
    if (!lvals || n < 1) return fail(FEQ_ERR_INVALID, "lvals must be non-empty");
    if (n > FEQ_MAX_IRREPS) return fail(FEQ_ERR_UNSUPPORTED, "more than %d irreps", FEQ_MAX_IRREPS);
    A = WignerArgs{};
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
    return FEQ_OK;
}

// Edges per workgroup: one thread per (edge, column), the edges' matrices
// (dim x dim values of T) staged in at most 64 KB of LDS.
template <class T>
int wigner_epb(int dim, int* epb, size_t* lds) {
    int e = 256 / dim;
    const int cap = static_cast<int>((64 * 1024) / (sizeof(T) * static_cast<size_t>(dim) * dim));
    e = e < cap ? e : cap;
    if (e < 1) return fail(FEQ_ERR_UNSUPPORTED, "representation dimension %d too large", dim);
    *epb = e;
    *lds = sizeof(T) * static_cast<size_t>(e) * dim * dim;
    return FEQ_OK;
}

template <class T>
int wigner_fwd(const int32_t* lvals, int32_t n, const double* plan, const int32_t* perm, int64_t E,
               const T* dirs, T* out, feq_stream_t stream) {
    WignerArgs A;
    if (int rc = wigner_args(lvals, n, A)) return rc;
    if (E < 0) return fail(FEQ_ERR_INVALID, "negative edge count");
    if (E == 0) return FEQ_OK;
    if (!plan || !perm || !dirs || !out) return fail(FEQ_ERR_INVALID, "NULL pointer");
    int epb;
    size_t lds;
    if (int rc = wigner_epb<T>(A.dim, &epb, &lds)) return rc;
    return with_lmax(A, [&](auto LL) -> int {
        auto kern = k_wigner<decltype(LL)::value, T>;
        FEQ_LAUNCH("k_wigner", kern, dim3(ceil_div(E, epb)), dim3(256), lds, stream_of(stream), A,
                   epb, plan, perm, E, dirs, out);
        return FEQ_OK;
    });
}

template <class T>
int wigner_bwd(const int32_t* lvals, int32_t n, const double* plan, const int32_t* perm, int64_t E,
               const T* dirs, const T* grad_out, T* grad_dirs, feq_stream_t stream) {
    WignerArgs A;
    if (int rc = wigner_args(lvals, n, A)) return rc;
    if (E < 0) return fail(FEQ_ERR_INVALID, "negative edge count");
    if (E == 0) return FEQ_OK;
    if (!plan || !perm || !dirs || !grad_out || !grad_dirs) return fail(FEQ_ERR_INVALID, "NULL pointer");
    int epb;
    size_t lds;
    if (int rc = wigner_epb<T>(A.dim, &epb, &lds)) return rc;
    return with_lmax(A, [&](auto LL) -> int {
        auto kern = k_wigner_bwd<decltype(LL)::value, T>;
        FEQ_LAUNCH("k_wigner_bwd", kern, dim3(ceil_div(E, epb)), dim3(256), lds, stream_of(stream), A,
                   epb, plan, perm, E, dirs, grad_out, grad_dirs);
        return FEQ_OK;
    });
}
}  // namespace

extern "C" int feq_wigner_basis(const int32_t* lvals, int32_t n, const double* plan,
                                const int32_t* perm, int64_t E, const float* dirs, float* out,
                                feq_stream_t stream) {
    return wigner_fwd<float>(lvals, n, plan, perm, E, dirs, out, stream);
}

extern "C" int feq_wigner_basis_f64(const int32_t* lvals, int32_t n, const double* plan,
                                    const int32_t* perm, int64_t E, const double* dirs, double* out,
                                    feq_stream_t stream) {
    return wigner_fwd<double>(lvals, n, plan, perm, E, dirs, out, stream);
}

extern "C" int feq_wigner_basis_bwd(const int32_t* lvals, int32_t n, const double* plan,
                                    const int32_t* perm, int64_t E, const float* dirs,
                                    const float* grad_out, float* grad_dirs, feq_stream_t stream) {
    return wigner_bwd<float>(lvals, n, plan, perm, E, dirs, grad_out, grad_dirs, stream);
}

extern "C" int feq_wigner_basis_bwd_f64(const int32_t* lvals, int32_t n, const double* plan,
                                        const int32_t* perm, int64_t E, const double* dirs,
                                        const double* grad_out, double* grad_dirs, feq_stream_t stream) {
    return wigner_bwd<double>(lvals, n, plan, perm, E, dirs, grad_out, grad_dirs, stream);
}

// Node-side neighbours of the edge path: the separable equivariant layer norm,
// the equivariant layer norm and the norm gating of the transformer block,
// forward and backward, on node tables x (N, mult, dim) of float32.
//
// Norm kernels run one wave per node: lane l owns channels l, l + 64, ...;
// statistics over channels are wave reductions (__shfl_xor, the same order on
// every lane), so results do not depend on the grid.  Parameter gradients are
// per-wave partials over a fixed grid, summed by reduce_partials in a fixed
// order (deterministic, no atomics).  The gating's Linear stays a library GEMM;
// its kernels run one thread per (node, channel) row.
//
// Formulas: SeparableEquivariantLayerNorm norm.py:177-246 (_ChannelLayerNorm
// :89-93, _EquivariantRMSNorm :109-112), EquivariantLayerNorm norm.py:148-174,
// RepNorm norm.py:19-55, EquivariantGating gating.py:54-76.
#include "feq_internal.h"

#include <algorithm>

namespace feq {
namespace {

constexpr int kWaves = 4;                          // nodes per workgroup, one per wave
constexpr int kMaxS = FEQ_NODE_MAX_SCALARS;
constexpr int kBwdGroups = 1536;                   // workgroups of the backward norm kernels (6 per CU: whole rounds at 2 or 3 resident)
constexpr int kStageRow = 1152;                    // node rows (mult * dim floats) staged in LDS
constexpr int kRowThreads = 256;

struct NodeL {
    int mult, dim, nreps;
    int vec;  // node rows move with 16-byte accesses (mult % 4 == 0, tables 16-byte aligned)
    int ns;   // scalar (l = 0) irreps
    int nhc;  // l > 0 components per channel
    int off[FEQ_MAX_IRREPS + 1];
    int deg[FEQ_MAX_IRREPS];
    int spos[kMaxS];  // component offset of each scalar irrep, in order
};

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }  // NULL passes

int make_nodel(const int32_t* lvals, int32_t nreps, int32_t mult, NodeL* L) {
    if (!lvals || nreps < 1 || nreps > FEQ_MAX_IRREPS)
        return fail(FEQ_ERR_INVALID, "node layout: 1..%d irreps required", FEQ_MAX_IRREPS);
    if (mult < 1 || mult > FEQ_NODE_MAX_MULT)
        return fail(FEQ_ERR_UNSUPPORTED, "node kernels take 1..%d channels (got %d)",
                    FEQ_NODE_MAX_MULT, mult);
    *L = NodeL{};
    L->mult = mult;
    L->vec = mult % 4 == 0;   // and the caller ANDs in its tables' alignment
    L->nreps = nreps;
    int o = 0;
    for (int k = 0; k < nreps; ++k) {
        const int l = lvals[k];
        if (l < 0 || l > 16) return fail(FEQ_ERR_INVALID, "node layout: degree %d out of range", l);
        L->off[k] = o;
        L->deg[k] = l;
        if (l == 0) {
            if (L->ns < kMaxS) L->spos[L->ns] = o;
            ++L->ns;
        } else {
            L->nhc += 2 * l + 1;
        }
        o += 2 * l + 1;
    }
    L->off[nreps] = o;
    L->dim = o;
    return FEQ_OK;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

// The per-node statistics of the norms (means, variances, their gradient
// sums) are formed in float64: a LayerNorm output near zero is v - mu, and a
// float32 mu leaves it with an absolute error of ~1e-7, which the next norm's
// 1/|v| (an EquivariantLayerNorm of a scalar irrep) turns into relative errors
// of 1e-4 and more downstream.  The elements stay float32 in memory.
__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

// Orders a wave's LDS writes before its other lanes' reads.
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Coalesced copy of one node row by a wave: 16-byte accesses with vec (the row
// a multiple of 4 floats, both ends 16-byte aligned), else 4-byte.
__device__ __forceinline__ void row_copy(float* __restrict__ d, const float* __restrict__ s, int64_t n,
                                         int lane, bool vec) {
    if (vec) {
        const int64_t n4 = n >> 2;
        for (int64_t i = lane; i < n4; i += 64)
            reinterpret_cast<float4*>(d)[i] = reinterpret_cast<const float4*>(s)[i];
    } else {
        for (int64_t i = lane; i < n; i += 64) d[i] = s[i];
    }
}

__device__ __forceinline__ void put4(float* v, const float4 a) {
    v[0] = a.x;
    v[1] = a.y;
    v[2] = a.z;
    v[3] = a.w;
}
__device__ __forceinline__ float4 get4(const float* v) { return make_float4(v[0], v[1], v[2], v[3]); }

// A component-major row (dim, N, mult) of node n into a node-major LDS row
// (c dim + d), and back: 16-byte runs of 4 channels with vec.
__device__ __forceinline__ void cm_to_row(float* __restrict__ srow, const float* __restrict__ t, int64_t N,
                                          int64_t n, int mult, int dim, int lane, bool vec) {
    if (vec) {
        const int m4 = mult >> 2;
        for (int q = lane; q < dim * m4; q += 64) {
            const int d = q / m4, c = 4 * (q - d * m4);
            const float4 v = reinterpret_cast<const float4*>(t + (d * N + n) * mult)[c >> 2];
            srow[c * dim + d] = v.x;
            srow[(c + 1) * dim + d] = v.y;
            srow[(c + 2) * dim + d] = v.z;
            srow[(c + 3) * dim + d] = v.w;
        }
    } else {
        for (int d = 0; d < dim; ++d)
            for (int c = lane; c < mult; c += 64) srow[c * dim + d] = t[(d * N + n) * mult + c];
    }
}
__device__ __forceinline__ void row_to_cm(float* __restrict__ t, const float* __restrict__ srow, int64_t N,
                                          int64_t n, int mult, int dim, int lane, bool vec, float scale = 1.0f) {
    if (vec) {
        const int m4 = mult >> 2;
        for (int q = lane; q < dim * m4; q += 64) {
            const int d = q / m4, c = 4 * (q - d * m4);
            reinterpret_cast<float4*>(t + (d * N + n) * mult)[c >> 2] =
                make_float4(scale * srow[c * dim + d], scale * srow[(c + 1) * dim + d],
                            scale * srow[(c + 2) * dim + d], scale * srow[(c + 3) * dim + d]);
        }
    } else {
        for (int d = 0; d < dim; ++d)
            for (int c = lane; c < mult; c += 64) t[(d * N + n) * mult + c] = scale * srow[c * dim + d];
    }
}

// Each lane's share of one node's x and gy rows, held in registers: the
// backward kernels load the next node's rows while the current node is
// computed, then move them into LDS.  With vec, lane l holds the float4s l,
// l + 64, ... of the row; else the floats l, l + 64, ....  With gy
// component-major (the _cm forms), gy is read as the row's runs of channels
// per component and staged at the node-major positions.
constexpr int kRowPer = kStageRow / 64;
constexpr int kRowPer4 = (kStageRow / 4 + 63) / 64;
struct RowPrefetch {
    float x[4 * kRowPer4], g[4 * kRowPer4];
    __device__ __forceinline__ void load(const float* __restrict__ xs, const float* __restrict__ gs,
                                         int64_t n, int64_t N, int64_t row, int lane, bool vec) {
        if (n >= N) return;
        if (vec) {
            const float4* x4 = reinterpret_cast<const float4*>(xs + n * row);
            const float4* g4 = reinterpret_cast<const float4*>(gs + n * row);
#pragma unroll
            for (int i = 0; i < kRowPer4; ++i) {
                const int64_t q = lane + 64 * i;
                if (4 * q < row) {
                    put4(x + 4 * i, x4[q]);
                    put4(g + 4 * i, g4[q]);
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < kRowPer; ++i) {
                const int64_t idx = lane + 64 * i;
                if (idx < row) {
                    x[i] = xs[n * row + idx];
                    g[i] = gs[n * row + idx];
                }
            }
        }
    }
    __device__ __forceinline__ void store(float* sx, float* sg, int64_t row, int lane, bool vec) const {
        if (vec) {
#pragma unroll
            for (int i = 0; i < kRowPer4; ++i) {
                const int64_t q = lane + 64 * i;
                if (4 * q < row) {
                    reinterpret_cast<float4*>(sx)[q] = get4(x + 4 * i);
                    reinterpret_cast<float4*>(sg)[q] = get4(g + 4 * i);
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < kRowPer; ++i) {
                const int64_t idx = lane + 64 * i;
                if (idx < row) {
                    sx[idx] = x[i];
                    sg[idx] = g[i];
                }
            }
        }
    }
    // gy component-major (dim, N, mult): element (d, c) of node n sits at
    // (d N + n) mult + c; the lane's share is the same positions of the row in
    // component-major order (d mult + c), so each component is a contiguous run.
    __device__ __forceinline__ void load_cm(const float* __restrict__ xs, const float* __restrict__ gs,
                                            int64_t n, int64_t N, int64_t row, int mult, int lane, bool vec) {
        if (n >= N) return;
        if (vec) {
            const float4* x4 = reinterpret_cast<const float4*>(xs + n * row);
            const int m4 = mult >> 2;
#pragma unroll
            for (int i = 0; i < kRowPer4; ++i) {
                const int q = lane + 64 * i;
                if (4 * q < row) {
                    const int d = q / m4, c4 = q - d * m4;
                    put4(x + 4 * i, x4[q]);
                    put4(g + 4 * i, reinterpret_cast<const float4*>(gs + (d * N + n) * mult)[c4]);
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < kRowPer; ++i) {
                const int64_t idx = lane + 64 * i;
                if (idx < row) {
                    const int d = static_cast<int>(idx) / mult, c = static_cast<int>(idx) - d * mult;
                    x[i] = xs[n * row + idx];
                    g[i] = gs[(d * N + n) * mult + c];
                }
            }
        }
    }
    __device__ __forceinline__ void store_cm(float* sx, float* sg, int64_t row, int mult, int dim,
                                             int lane, bool vec) const {
        if (vec) {
            const int m4 = mult >> 2;
#pragma unroll
            for (int i = 0; i < kRowPer4; ++i) {
                const int q = lane + 64 * i;
                if (4 * q < row) {
                    const int d = q / m4, c = 4 * (q - d * m4);
                    reinterpret_cast<float4*>(sx)[q] = get4(x + 4 * i);
#pragma unroll
                    for (int j = 0; j < 4; ++j) sg[(c + j) * dim + d] = g[4 * i + j];
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < kRowPer; ++i) {
                const int64_t idx = lane + 64 * i;
                if (idx < row) {
                    const int d = static_cast<int>(idx) / mult, c = static_cast<int>(idx) - d * mult;
                    sx[idx] = x[i];
                    sg[c * dim + d] = g[i];
                }
            }
        }
    }
};

// Workgroups per CU the norm backward kernels are compiled for: three (at
// most 168 VGPRs) where one channel per lane and the staged rows fit without
// spilling, so that more nodes' rows are in flight; otherwise no bound (the
// compiler's choice).  `heavy`: the forms that do not fit 168 (the
// component-major gradient read with 4-byte accesses, and the separable
// norm's component-major form with an addend).
constexpr int norm_bwd_blocks(int cpl, bool stage, bool heavy) { return cpl == 1 && stage && !heavy ? 3 : 1; }

// The rows of an addend to the input gradient (a second branch's gradient of
// the same input, summed here instead of in a separate pass): loaded when a
// node's computation starts, in flight during it, and added as the node's
// gradient row is written.  Lane mapping as RowPrefetch.
struct RowAddend {
    float a[4 * kRowPer4];
    template <bool VEC>
    __device__ __forceinline__ void load(const float* __restrict__ ga, int64_t n, int64_t row, int lane) {
        if constexpr (VEC) {
            const float4* a4 = reinterpret_cast<const float4*>(ga + n * row);
#pragma unroll
            for (int i = 0; i < kRowPer4; ++i) {
                const int64_t q = lane + 64 * i;
                if (4 * q < row) put4(a + 4 * i, a4[q]);
            }
        } else {
#pragma unroll
            for (int i = 0; i < kRowPer; ++i) {
                const int64_t idx = lane + 64 * i;
                if (idx < row) a[i] = ga[n * row + idx];
            }
        }
    }
    template <bool VEC>
    __device__ __forceinline__ void store_sum(float* __restrict__ gx, const float* sg, int64_t n, int64_t row,
                                              int lane) const {
        if constexpr (VEC) {
            float4* g4 = reinterpret_cast<float4*>(gx + n * row);
#pragma unroll
            for (int i = 0; i < kRowPer4; ++i) {
                const int64_t q = lane + 64 * i;
                if (4 * q < row) {
                    const float4 v = reinterpret_cast<const float4*>(sg)[q];
                    g4[q] = make_float4(v.x + a[4 * i], v.y + a[4 * i + 1], v.z + a[4 * i + 2], v.w + a[4 * i + 3]);
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < kRowPer; ++i) {
                const int64_t idx = lane + 64 * i;
                if (idx < row) gx[n * row + idx] = sg[idx] + a[i];
            }
        }
    }
};

__device__ __forceinline__ float sigmoidf(float v) { return 1.0f / (1.0f + expf(-v)); }

// ---- separable layer norm ---------------------------------------------------
// scalars: (v - mu) / (sd + eps) * w_s[c, j] + b_s[c, j], mu and sd (biased)
// over the channels; l > 0 components: v * w_h[c] / sqrt(mean(v^2) + eps), the
// mean over every channel and l > 0 component of the node.

// STAGE: the node row moves through LDS (coalesced), computed in place.
// CMO (with STAGE): y is component-major (dim, N, mult), the layout the
// channel-mixing maps after the norm take, written as contiguous channel runs.
template <int CPL, bool STAGE, bool CMO = false, bool VEC = false>
__global__ void __launch_bounds__(64 * kWaves)
k_sepnorm_fwd(NodeL L, int64_t N, const float* __restrict__ x, const float* __restrict__ ws,
              const float* __restrict__ bs, const float* __restrict__ wh, float eps,
              float* __restrict__ y) {
    static_assert(STAGE || !CMO, "component-major output goes through the LDS stage");
    __shared__ __align__(16) float lds[STAGE ? kWaves * kStageRow : 1];
    const int lane = threadIdx.x & 63;
    const int64_t n = static_cast<int64_t>(blockIdx.x) * kWaves + (threadIdx.x >> 6);
    if (n >= N) return;
    const int64_t row = static_cast<int64_t>(L.mult) * L.dim;
    float* sx = lds + (threadIdx.x >> 6) * kStageRow;
    if (STAGE) {
        row_copy(sx, x + n * row, row, lane, VEC);
        wave_sync();
    }
    const float* xn = STAGE ? sx : x + n * row;
    float* yn = STAGE ? sx : y + n * row;
    const float fm = static_cast<float>(L.mult);
#pragma unroll
    for (int j = 0; j < kMaxS; ++j) {
        if (j >= L.ns) break;
        const int d = L.spos[j];
        double v[CPL];
        double s = 0.0;
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            const int c = lane + 64 * i;
            v[i] = c < L.mult ? xn[c * L.dim + d] : 0.0f;
            s += v[i];
        }
        const double mu = wave_sum(s) / fm;
        double q = 0.0;
#pragma unroll
        for (int i = 0; i < CPL; ++i)
            if (lane + 64 * i < L.mult) q += (v[i] - mu) * (v[i] - mu);
        const double den = sqrt(wave_sum(q) / fm) + eps;
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            const int c = lane + 64 * i;
            if (c < L.mult)
                yn[c * L.dim + d] = static_cast<float>((v[i] - mu) / den * ws[c * L.ns + j] +
                                                       bs[c * L.ns + j]);
        }
    }
    if (L.nhc > 0) {  // w_h is NULL without l > 0 irreps
        double h = 0.0;
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            const int c = lane + 64 * i;
            if (c >= L.mult) continue;
            for (int k = 0; k < L.nreps; ++k) {
                if (L.deg[k] == 0) continue;
                for (int d = L.off[k]; d < L.off[k + 1]; ++d) {
                    const double v = xn[c * L.dim + d];
                    h += v * v;
                }
            }
        }
        const double rms = sqrt(wave_sum(h) / (fm * L.nhc) + eps);
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            const int c = lane + 64 * i;
            if (c >= L.mult) continue;
            const float f = static_cast<float>(wh[c] / rms);
            for (int k = 0; k < L.nreps; ++k) {
                if (L.deg[k] == 0) continue;
                for (int d = L.off[k]; d < L.off[k + 1]; ++d) yn[c * L.dim + d] = xn[c * L.dim + d] * f;
            }
        }
    }
    if (STAGE) {
        wave_sync();
        if constexpr (CMO) {
            row_to_cm(y, sx, N, n, L.mult, L.dim, lane, VEC);
        } else {
            row_copy(y + n * row, sx, row, lane, VEC);
        }
    }
}

// Backward.  Scalars, with gp = gy w_s and den = sd + eps:
//   gx = (gp - mean(gp)) / den - sum(gp (v - mu)) (v - mu) / (mult sd den^2);
// l > 0, with S = sum over the node of gy v w_h[c]:
//   gx = gy w_h[c] / rms - S v / (count rms^3).
// Per-wave partials: pS, pB (mult, ns) of gy (v - mu) / den and gy; pH (mult) of
// sum_d gy v / rms.
// CMG (with STAGE): gy is component-major (dim, N, mult); x and gx node-major.
// ADD (with STAGE): gx = the norm's input gradient + ga (node-major).  NSM:
// the most scalar irreps the instance handles (1, the common case, keeps the
// per-wave parameter partials to two registers per channel).
template <int CPL, bool STAGE, bool CMG = false, bool VEC = false, bool ADD = false, int NSM = kMaxS>
__global__ void __launch_bounds__(64 * kWaves, norm_bwd_blocks(CPL, STAGE, CMG && ((ADD && NSM > 1) || !VEC)))
k_sepnorm_bwd(NodeL L, int64_t N, const float* __restrict__ gy, const float* __restrict__ x,
              const float* __restrict__ ws, const float* __restrict__ wh, float eps,
              float* __restrict__ gx, float* __restrict__ pS, float* __restrict__ pB,
              float* __restrict__ pH, const float* __restrict__ ga) {
    static_assert(STAGE || !CMG, "component-major gradients go through the LDS stage");
    static_assert(STAGE || !ADD, "the gradient addend goes through the LDS stage");
    const int lane = threadIdx.x & 63;
    const int64_t wave = static_cast<int64_t>(blockIdx.x) * kWaves + (threadIdx.x >> 6);
    const int64_t nw = static_cast<int64_t>(gridDim.x) * kWaves;
    const int64_t row = static_cast<int64_t>(L.mult) * L.dim;
    const float fm = static_cast<float>(L.mult);
    const float cnt = fm * L.nhc;
    float aS[CPL][NSM], aB[CPL][NSM], aH[CPL];
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
        aH[i] = 0.0f;
#pragma unroll
        for (int j = 0; j < NSM; ++j) aS[i][j] = aB[i][j] = 0.0f;
    }
    __shared__ __align__(16) float lds[STAGE ? 2 * kWaves * kStageRow : 1];
    float* sx = lds + (threadIdx.x >> 6) * 2 * kStageRow;
    float* sg = sx + kStageRow;
    RowPrefetch pf;
    RowAddend ad;
    if (STAGE) {
        if constexpr (CMG) pf.load_cm(x, gy, wave, N, row, L.mult, lane, VEC);
        else pf.load(x, gy, wave, N, row, lane, VEC);
    }
    for (int64_t n = wave; n < N; n += nw) {
        if (STAGE) {
            wave_sync();  // the previous node's stores have read sg
            if constexpr (CMG) {
                pf.store_cm(sx, sg, row, L.mult, L.dim, lane, VEC);
                pf.load_cm(x, gy, n + nw, N, row, L.mult, lane, VEC);   // in flight during this node
            } else {
                pf.store(sx, sg, row, lane, VEC);
                pf.load(x, gy, n + nw, N, row, lane, VEC);
            }
            if constexpr (ADD) ad.template load<VEC>(ga, n, row, lane);
            wave_sync();
        }
        const float* xn = STAGE ? sx : x + n * row;
        const float* gn = STAGE ? sg : gy + n * row;
        float* on = STAGE ? sg : gx + n * row;
#pragma unroll
        for (int j = 0; j < NSM; ++j) {
            if (j >= L.ns) break;
            const int d = L.spos[j];
            double v[CPL], gp[CPL];
            float g[CPL];
            double s = 0.0;
#pragma unroll
            for (int i = 0; i < CPL; ++i) {
                const int c = lane + 64 * i;
                const bool ok = c < L.mult;
                v[i] = ok ? xn[c * L.dim + d] : 0.0f;
                g[i] = ok ? gn[c * L.dim + d] : 0.0f;
                gp[i] = ok ? static_cast<double>(g[i]) * ws[c * L.ns + j] : 0.0;
                s += v[i];
            }
            const double mu = wave_sum(s) / fm;
            double q = 0.0, sg = 0.0, sgv = 0.0;
#pragma unroll
            for (int i = 0; i < CPL; ++i) {
                if (lane + 64 * i >= L.mult) continue;
                const double t = v[i] - mu;
                q += t * t;
                sg += gp[i];
                sgv += gp[i] * t;
            }
            const double sd = sqrt(wave_sum(q) / fm);
            const double mg = wave_sum(sg) / fm;
            sgv = wave_sum(sgv);
            const double den = sd + eps;
            const double coef = sd > 0.0 ? sgv / (fm * sd * den * den) : 0.0;
#pragma unroll
            for (int i = 0; i < CPL; ++i) {
                const int c = lane + 64 * i;
                if (c >= L.mult) continue;
                const double t = v[i] - mu;
                on[c * L.dim + d] = static_cast<float>((gp[i] - mg) / den - coef * t);
                aS[i][j] += g[i] * static_cast<float>(t / den);
                aB[i][j] += g[i];
            }
        }
        if (L.nhc > 0) {  // w_h is NULL without l > 0 irreps
            double h = 0.0, S = 0.0;
#pragma unroll
            for (int i = 0; i < CPL; ++i) {
                const int c = lane + 64 * i;
                if (c >= L.mult) continue;
                double t = 0.0;
                for (int k = 0; k < L.nreps; ++k) {
                    if (L.deg[k] == 0) continue;
                    for (int d = L.off[k]; d < L.off[k + 1]; ++d) {
                        const double v = xn[c * L.dim + d];
                        h += v * v;
                        t += gn[c * L.dim + d] * v;
                    }
                }
                S += t * wh[c];
            }
            const double rms_d = sqrt(wave_sum(h) / cnt + eps);
            const float rms = static_cast<float>(rms_d);
            const float k2 = static_cast<float>(wave_sum(S) / (cnt * rms_d * rms_d * rms_d));
#pragma unroll
            for (int i = 0; i < CPL; ++i) {
                const int c = lane + 64 * i;
                if (c >= L.mult) continue;
                const float a = static_cast<float>(wh[c] / rms_d);
                float t = 0.0f;
                for (int k = 0; k < L.nreps; ++k) {
                    if (L.deg[k] == 0) continue;
                    for (int d = L.off[k]; d < L.off[k + 1]; ++d) {
                        const float v = xn[c * L.dim + d];
                        const float g = gn[c * L.dim + d];
                        on[c * L.dim + d] = g * a - k2 * v;
                        t += g * v;
                    }
                }
                aH[i] += t / rms;
            }
        }
        if (STAGE) {
            wave_sync();
            if constexpr (ADD) ad.template store_sum<VEC>(gx, sg, n, row, lane);
            else row_copy(gx + n * row, sg, row, lane, VEC);
        }
    }
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
        const int c = lane + 64 * i;
        if (c >= L.mult) continue;
        if (pH) pH[wave * L.mult + c] = aH[i];
#pragma unroll
        for (int j = 0; j < NSM; ++j) {
            if (j >= L.ns) break;
            pS[(wave * L.mult + c) * L.ns + j] = aS[i][j];
            pB[(wave * L.mult + c) * L.ns + j] = aB[i][j];
        }
    }
}

// ---- residual connection with a component-major branch -------------------------
// out (N, mult, dim) = x (N, mult, dim) + scale[0] y with y component-major
// (dim, N, mult): the block's MLP output joins the residual stream without a
// separate transpose.  A wave per node stages y's component runs in LDS, then
// writes the node row.  Fixed grid (kResGroups workgroups, nodes grid-stride).
constexpr int kResGroups = 1024;

__global__ void __launch_bounds__(64 * kWaves)
k_scale_add_cm(int64_t N, int mult, int dim, int vec, const float* __restrict__ x, const float* __restrict__ y,
               const float* __restrict__ scale, float* __restrict__ out) {
    __shared__ __align__(16) float lds[kWaves * kStageRow];
    const int lane = threadIdx.x & 63;
    float* sy = lds + (threadIdx.x >> 6) * kStageRow;
    const float sc = scale[0];
    const int64_t row = static_cast<int64_t>(mult) * dim;
    const int64_t nw = static_cast<int64_t>(gridDim.x) * kWaves;
    for (int64_t n = static_cast<int64_t>(blockIdx.x) * kWaves + (threadIdx.x >> 6); n < N; n += nw) {
        cm_to_row(sy, y, N, n, mult, dim, lane, vec);
        wave_sync();
        if (vec) {
            const float4* x4 = reinterpret_cast<const float4*>(x + n * row);
            float4* o4 = reinterpret_cast<float4*>(out + n * row);
            for (int64_t i = lane; i < row / 4; i += 64) {
                const float4 a = x4[i], b = reinterpret_cast<const float4*>(sy)[i];
                o4[i] = make_float4(a.x + sc * b.x, a.y + sc * b.y, a.z + sc * b.z, a.w + sc * b.w);
            }
        } else {
            for (int64_t i = lane; i < row; i += 64) out[n * row + i] = x[n * row + i] + sc * sy[i];
        }
        wave_sync();   // this node's reads of sy are done before the next node's writes
    }
}

// Its backward for grad_out g (node-major): grad_y (component-major) =
// scale[0] g (NULL: not formed) and per-workgroup float64 partials of sum g y.
__global__ void __launch_bounds__(64 * kWaves)
k_scale_add_cm_bwd(int64_t N, int mult, int dim, int vec, const float* __restrict__ g,
                   const float* __restrict__ y, const float* __restrict__ scale, float* __restrict__ gy,
                   double* __restrict__ part) {
    __shared__ __align__(16) float lds[kWaves * kStageRow];
    __shared__ double red[kWaves];
    const int lane = threadIdx.x & 63;
    float* sg = lds + (threadIdx.x >> 6) * kStageRow;
    const float sc = scale[0];
    const int64_t row = static_cast<int64_t>(mult) * dim;
    const int64_t nw = static_cast<int64_t>(gridDim.x) * kWaves;
    double acc = 0.0;
    for (int64_t n = static_cast<int64_t>(blockIdx.x) * kWaves + (threadIdx.x >> 6); n < N; n += nw) {
        row_copy(sg, g + n * row, row, lane, vec);
        wave_sync();
        if (vec) {
            const int m4 = mult >> 2;
            for (int q = lane; q < dim * m4; q += 64) {
                const int d = q / m4, c = 4 * (q - d * m4);
                const float4 v = make_float4(sg[c * dim + d], sg[(c + 1) * dim + d], sg[(c + 2) * dim + d],
                                             sg[(c + 3) * dim + d]);
                const int64_t o4 = ((d * N + n) * mult + c) >> 2;
                if (gy) reinterpret_cast<float4*>(gy)[o4] = make_float4(sc * v.x, sc * v.y, sc * v.z, sc * v.w);
                const float4 w = reinterpret_cast<const float4*>(y)[o4];
                acc += (static_cast<double>(v.x) * w.x + static_cast<double>(v.y) * w.y) +
                       (static_cast<double>(v.z) * w.z + static_cast<double>(v.w) * w.w);
            }
        } else {
            for (int d = 0; d < dim; ++d)
                for (int c = lane; c < mult; c += 64) {
                    const float v = sg[c * dim + d];
                    const int64_t o = (d * N + n) * mult + c;
                    if (gy) gy[o] = sc * v;
                    acc += static_cast<double>(v) * y[o];
                }
        }
        wave_sync();
    }
    acc = wave_sum(acc);
    if (lane == 0) red[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) part[blockIdx.x] = (red[0] + red[1]) + (red[2] + red[3]);
}

// out[0] = (float) sum of part[0 .. n) by one workgroup in a fixed order.
__global__ void __launch_bounds__(64 * kWaves)
k_sum_f64(const double* __restrict__ part, int n, float* __restrict__ out) {
    __shared__ double red[kWaves];
    double acc = 0.0;
    for (int i = threadIdx.x; i < n; i += 64 * kWaves) acc += part[i];
    acc = wave_sum(acc);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) out[0] = static_cast<float>((red[0] + red[1]) + (red[2] + red[3]));
}

// ---- equivariant layer norm ---------------------------------------------------
// Per irrep k: norm n_c = sqrt(sum_d x^2 + eps); with weights, a LayerNorm over
// the channels ln_c = (n_c - mu) rstd w_c + b_c (rstd = 1 / sqrt(var + ln_eps));
// y = x ln_c / (n_c + eps), or x / (n_c + eps) without weights (one channel).

// CMO (with STAGE): y component-major (dim, N, mult), as the separable norm's.
template <int CPL, bool STAGE, bool CMO = false, bool VEC = false>
__global__ void __launch_bounds__(64 * kWaves)
k_eqnorm_fwd(NodeL L, int64_t N, const float* __restrict__ x, const float* __restrict__ w,
             const float* __restrict__ b, float eps, float ln_eps, float* __restrict__ y) {
    static_assert(STAGE || !CMO, "component-major output goes through the LDS stage");
    __shared__ __align__(16) float lds[STAGE ? kWaves * kStageRow : 1];
    const int lane = threadIdx.x & 63;
    const int64_t n = static_cast<int64_t>(blockIdx.x) * kWaves + (threadIdx.x >> 6);
    if (n >= N) return;
    const int64_t row = static_cast<int64_t>(L.mult) * L.dim;
    float* sx = lds + (threadIdx.x >> 6) * kStageRow;
    if (STAGE) {
        row_copy(sx, x + n * row, row, lane, VEC);
        wave_sync();
    }
    const float* xn = STAGE ? sx : x + n * row;
    float* yn = STAGE ? sx : y + n * row;
    const float fm = static_cast<float>(L.mult);
    for (int k = 0; k < L.nreps; ++k) {
        const int d0 = L.off[k], d1 = L.off[k + 1];
        double nr[CPL];
        double s = 0.0;
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            const int c = lane + 64 * i;
            double q = 0.0;
            if (c < L.mult)
                for (int d = d0; d < d1; ++d) {
                    const double v = xn[c * L.dim + d];
                    q += v * v;
                }
            nr[i] = sqrt(q + eps);
            if (c < L.mult) s += nr[i];
        }
        double mu = 0.0, rstd = 0.0;
        if (w) {
            mu = wave_sum(s) / fm;
            double q = 0.0;
#pragma unroll
            for (int i = 0; i < CPL; ++i)
                if (lane + 64 * i < L.mult) q += (nr[i] - mu) * (nr[i] - mu);
            rstd = 1.0 / sqrt(wave_sum(q) / fm + ln_eps);
        }
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            const int c = lane + 64 * i;
            if (c >= L.mult) continue;
            const float f = static_cast<float>(w ? ((nr[i] - mu) * rstd * w[c] + b[c]) / (nr[i] + eps)
                                                 : 1.0 / (nr[i] + eps));
            for (int d = d0; d < d1; ++d) yn[c * L.dim + d] = xn[c * L.dim + d] * f;
        }
    }
    if (STAGE) {
        wave_sync();
        if constexpr (CMO) {
            row_to_cm(y, sx, N, n, L.mult, L.dim, lane, VEC);
        } else {
            row_copy(y + n * row, sx, row, lane, VEC);
        }
    }
}

// Backward per irrep: dfac = sum_d gy x; with weights dln = dfac / (n + eps),
// dn = -dfac ln / (n + eps)^2 + rstd (dnh - mean(dnh) - nh mean(dnh nh)) with
// dnh = dln w, nh = (n - mu) rstd; gx = gy fac + x dn / n.
// Per-wave partials of sum dln nh (pW) and sum dln (pB), per channel.
// CMG (with STAGE): gy component-major (dim, N, mult); x and gx node-major.
// ADD (with STAGE): gx = the norm's input gradient + ga (node-major).
template <int CPL, bool STAGE, bool CMG = false, bool VEC = false, bool ADD = false>
__global__ void __launch_bounds__(64 * kWaves, norm_bwd_blocks(CPL, STAGE, CMG && !VEC))
k_eqnorm_bwd(NodeL L, int64_t N, const float* __restrict__ gy, const float* __restrict__ x,
             const float* __restrict__ w, const float* __restrict__ b, float eps, float ln_eps,
             float* __restrict__ gx, float* __restrict__ pW, float* __restrict__ pB,
             const float* __restrict__ ga) {
    static_assert(STAGE || !ADD, "the gradient addend goes through the LDS stage");
    static_assert(STAGE || !CMG, "component-major gradients go through the LDS stage");
    const int lane = threadIdx.x & 63;
    const int64_t wave = static_cast<int64_t>(blockIdx.x) * kWaves + (threadIdx.x >> 6);
    const int64_t nw = static_cast<int64_t>(gridDim.x) * kWaves;
    const int64_t row = static_cast<int64_t>(L.mult) * L.dim;
    const float fm = static_cast<float>(L.mult);
    float aW[CPL], aB[CPL];
#pragma unroll
    for (int i = 0; i < CPL; ++i) aW[i] = aB[i] = 0.0f;
    __shared__ __align__(16) float lds[STAGE ? 2 * kWaves * kStageRow : 1];
    float* sx = lds + (threadIdx.x >> 6) * 2 * kStageRow;
    float* sg = sx + kStageRow;
    RowPrefetch pf;
    RowAddend ad;
    if (STAGE) {
        if constexpr (CMG) pf.load_cm(x, gy, wave, N, row, L.mult, lane, VEC);
        else pf.load(x, gy, wave, N, row, lane, VEC);
    }
    for (int64_t n = wave; n < N; n += nw) {
        if (STAGE) {
            wave_sync();  // the previous node's stores have read sg
            if constexpr (CMG) {
                pf.store_cm(sx, sg, row, L.mult, L.dim, lane, VEC);
                pf.load_cm(x, gy, n + nw, N, row, L.mult, lane, VEC);   // in flight during this node
            } else {
                pf.store(sx, sg, row, lane, VEC);
                pf.load(x, gy, n + nw, N, row, lane, VEC);
            }
            if constexpr (ADD) ad.template load<VEC>(ga, n, row, lane);
            wave_sync();
        }
        const float* xn = STAGE ? sx : x + n * row;
        const float* gn = STAGE ? sg : gy + n * row;
        float* on = STAGE ? sg : gx + n * row;
        for (int k = 0; k < L.nreps; ++k) {
            const int d0 = L.off[k], d1 = L.off[k + 1];
            double nr[CPL], df[CPL];
            double s = 0.0;
#pragma unroll
            for (int i = 0; i < CPL; ++i) {
                const int c = lane + 64 * i;
                double q = 0.0, t = 0.0;
                if (c < L.mult)
                    for (int d = d0; d < d1; ++d) {
                        const double v = xn[c * L.dim + d];
                        q += v * v;
                        t += gn[c * L.dim + d] * v;
                    }
                nr[i] = sqrt(q + eps);
                df[i] = t;
                if (c < L.mult) s += nr[i];
            }
            float fac[CPL];
            double dn[CPL];
            if (w) {
                const double mu = wave_sum(s) / fm;
                double q = 0.0;
#pragma unroll
                for (int i = 0; i < CPL; ++i)
                    if (lane + 64 * i < L.mult) q += (nr[i] - mu) * (nr[i] - mu);
                const double rstd = 1.0 / sqrt(wave_sum(q) / fm + ln_eps);
                double nh[CPL], dnh[CPL], dln[CPL];
                double m1 = 0.0, m2 = 0.0;
#pragma unroll
                for (int i = 0; i < CPL; ++i) {
                    const int c = lane + 64 * i;
                    const bool ok = c < L.mult;
                    const double den = nr[i] + eps;
                    nh[i] = (nr[i] - mu) * rstd;
                    const double ln = ok ? nh[i] * w[c] + b[c] : 0.0;
                    fac[i] = static_cast<float>(ln / den);
                    dln[i] = df[i] / den;
                    dnh[i] = ok ? dln[i] * w[c] : 0.0;
                    dn[i] = -df[i] * ln / (den * den);
                    if (ok) {
                        m1 += dnh[i];
                        m2 += dnh[i] * nh[i];
                    }
                }
                m1 = wave_sum(m1) / fm;
                m2 = wave_sum(m2) / fm;
#pragma unroll
                for (int i = 0; i < CPL; ++i) {
                    dn[i] += rstd * (dnh[i] - m1 - nh[i] * m2);
                    if (lane + 64 * i < L.mult) {
                        aW[i] += static_cast<float>(dln[i] * nh[i]);
                        aB[i] += static_cast<float>(dln[i]);
                    }
                }
            } else {
#pragma unroll
                for (int i = 0; i < CPL; ++i) {
                    const double den = nr[i] + eps;
                    fac[i] = static_cast<float>(1.0 / den);
                    dn[i] = -df[i] / (den * den);
                }
            }
#pragma unroll
            for (int i = 0; i < CPL; ++i) {
                const int c = lane + 64 * i;
                if (c >= L.mult) continue;
                const float r = static_cast<float>(dn[i] / nr[i]);
                for (int d = d0; d < d1; ++d)
                    on[c * L.dim + d] = gn[c * L.dim + d] * fac[i] + xn[c * L.dim + d] * r;
            }
        }
        if (STAGE) {
            wave_sync();
            if constexpr (ADD) ad.template store_sum<VEC>(gx, sg, n, row, lane);
            else row_copy(gx + n * row, sg, row, lane, VEC);
        }
    }
    if (!pW) return;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
        const int c = lane + 64 * i;
        if (c >= L.mult) continue;
        pW[wave * L.mult + c] = aW[i];
        pB[wave * L.mult + c] = aB[i];
    }
}

// ---- gating ---------------------------------------------------------------------
// A workgroup takes a tile of consecutive (node, channel) rows: the tile's
// components move between HBM and LDS with coalesced loads and stores, and
// thread t works on row t of the tile in LDS (odd row strides such as 9 floats
// are free of bank conflicts).

constexpr int kTileFloats = 2560;  // LDS floats per staged tensor (10 KB: 256 rows of up to 10 components)

__device__ __forceinline__ int tile_rows(const NodeL& L) {
    return min(kRowThreads, kTileFloats / L.dim);
}

__device__ __forceinline__ void tile_load(float* __restrict__ s, const float* __restrict__ g, int64_t n) {
    for (int64_t i = threadIdx.x; i < n; i += kRowThreads) s[i] = g[i];
}

__device__ __forceinline__ void tile_store(float* __restrict__ g, const float* __restrict__ s, int64_t n) {
    for (int64_t i = threadIdx.x; i < n; i += kRowThreads) g[i] = s[i];
}

__global__ void __launch_bounds__(kRowThreads)
k_gate_norms(NodeL L, int64_t rows, const float* __restrict__ x, float eps, float* __restrict__ nrm) {
    __shared__ float sx[kTileFloats];
    const int R = tile_rows(L);
    const int64_t r0 = static_cast<int64_t>(blockIdx.x) * R;
    const int nr = static_cast<int>(min<int64_t>(R, rows - r0));
    tile_load(sx, x + r0 * L.dim, int64_t(nr) * L.dim);
    __syncthreads();
    const int t = threadIdx.x;
    if (t >= nr) return;
    for (int k = 0; k < L.nreps; ++k) {
        float q = 0.0f;
        for (int d = L.off[k]; d < L.off[k + 1]; ++d) q += sx[t * L.dim + d] * sx[t * L.dim + d];
        nrm[(r0 + t) * L.nreps + k] = sqrtf(q + eps);
    }
}

__global__ void __launch_bounds__(kRowThreads)
k_gate_apply(NodeL L, int64_t rows, const float* __restrict__ x, const float* __restrict__ lin,
             float* __restrict__ y) {
    __shared__ float sx[kTileFloats];
    const int R = tile_rows(L);
    const int64_t r0 = static_cast<int64_t>(blockIdx.x) * R;
    const int nr = static_cast<int>(min<int64_t>(R, rows - r0));
    const int64_t n = int64_t(nr) * L.dim;
    tile_load(sx, x + r0 * L.dim, n);
    __syncthreads();
    const int t = threadIdx.x;
    if (t < nr)
        for (int k = 0; k < L.nreps; ++k) {
            const float g = sigmoidf(lin[(r0 + t) * L.nreps + k]);
            for (int d = L.off[k]; d < L.off[k + 1]; ++d) sx[t * L.dim + d] *= g;
        }
    __syncthreads();
    tile_store(y + r0 * L.dim, sx, n);
}

__global__ void __launch_bounds__(kRowThreads)
k_gate_bwd_lin(NodeL L, int64_t rows, const float* __restrict__ gy, const float* __restrict__ x,
               const float* __restrict__ lin, float* __restrict__ dlin) {
    __shared__ float sx[kTileFloats];
    __shared__ float sg[kTileFloats];
    const int R = tile_rows(L);
    const int64_t r0 = static_cast<int64_t>(blockIdx.x) * R;
    const int nr = static_cast<int>(min<int64_t>(R, rows - r0));
    const int64_t n = int64_t(nr) * L.dim;
    tile_load(sx, x + r0 * L.dim, n);
    tile_load(sg, gy + r0 * L.dim, n);
    __syncthreads();
    const int t = threadIdx.x;
    if (t >= nr) return;
    for (int k = 0; k < L.nreps; ++k) {
        float q = 0.0f;
        for (int d = L.off[k]; d < L.off[k + 1]; ++d) q += sg[t * L.dim + d] * sx[t * L.dim + d];
        const float g = sigmoidf(lin[(r0 + t) * L.nreps + k]);
        dlin[(r0 + t) * L.nreps + k] = q * (g * (1.0f - g));
    }
}

__global__ void __launch_bounds__(kRowThreads)
k_gate_bwd_x(NodeL L, int64_t rows, const float* __restrict__ gy, const float* __restrict__ x,
             const float* __restrict__ lin, const float* __restrict__ nrm,
             const float* __restrict__ dnrm, float* __restrict__ gx) {
    __shared__ float sx[kTileFloats];
    __shared__ float sg[kTileFloats];
    const int R = tile_rows(L);
    const int64_t r0 = static_cast<int64_t>(blockIdx.x) * R;
    const int nr = static_cast<int>(min<int64_t>(R, rows - r0));
    const int64_t n = int64_t(nr) * L.dim;
    tile_load(sx, x + r0 * L.dim, n);
    tile_load(sg, gy + r0 * L.dim, n);
    __syncthreads();
    const int t = threadIdx.x;
    if (t < nr)
        for (int k = 0; k < L.nreps; ++k) {
            const int64_t i = (r0 + t) * L.nreps + k;
            const float g = sigmoidf(lin[i]);
            const float q = dnrm[i] / nrm[i];
            for (int d = L.off[k]; d < L.off[k + 1]; ++d)
                sg[t * L.dim + d] = sg[t * L.dim + d] * g + sx[t * L.dim + d] * q;
        }
    __syncthreads();
    tile_store(gx + r0 * L.dim, sg, n);
}

// Component-major tables (dim, N, mult): element (p, d) of pair p = (node,
// channel) sits at d * P + p, so consecutive threads read consecutive floats.
// The per-pair values (norms, gate inputs and their gradients) are (P, nreps).
// W = 4 (with NR = nreps): each thread takes four consecutive pairs with
// 16-byte accesses (P a multiple of 4, the tables 16-byte aligned), its 4 NR
// per-pair values as NR float4s, four independent sums per load.  W = 1: one
// pair per thread, any nreps (NR = 0: read from L).

template <int W>
__device__ __forceinline__ void ld_w(const float* __restrict__ s, float (&v)[W]) {
    if constexpr (W == 4) {
        const float4 f = *reinterpret_cast<const float4*>(s);
        v[0] = f.x;
        v[1] = f.y;
        v[2] = f.z;
        v[3] = f.w;
    } else {
        v[0] = *s;
    }
}
template <int W>
__device__ __forceinline__ void st_w(float* __restrict__ d, const float (&v)[W]) {
    if constexpr (W == 4) *reinterpret_cast<float4*>(d) = make_float4(v[0], v[1], v[2], v[3]);
    else *d = v[0];
}
// the W * nr per-pair values of the thread's pairs p .. p + W - 1 (contiguous)
template <int W, int NRS>
__device__ __forceinline__ void ld_pairs(const float* __restrict__ s, int64_t p, int nr, float (&v)[W * NRS]) {
    if constexpr (W == 4) {
#pragma unroll
        for (int q = 0; q < NRS; ++q) {
            float t[4];
            ld_w<4>(s + p * NRS + 4 * q, t);
#pragma unroll
            for (int j = 0; j < 4; ++j) v[4 * q + j] = t[j];
        }
    } else {
#pragma unroll
        for (int k = 0; k < NRS; ++k) v[k] = k < nr ? s[p * nr + k] : 0.0f;
    }
}
template <int W, int NRS>
__device__ __forceinline__ void st_pairs(float* __restrict__ d, int64_t p, int nr, const float (&v)[W * NRS]) {
    if constexpr (W == 4) {
#pragma unroll
        for (int q = 0; q < NRS; ++q) {
            const float t[4] = {v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]};
            st_w<4>(d + p * NRS + 4 * q, t);
        }
    } else {
#pragma unroll
        for (int k = 0; k < NRS; ++k)
            if (k < nr) d[p * nr + k] = v[k];
    }
}
// per-pair value of pair w, irrep k
template <int W, int NRS>
__device__ __forceinline__ int pv(int w, int k) { return W == 4 ? w * NRS + k : k; }

// NRS: the per-pair register rows (NR, or FEQ_MAX_IRREPS for W = 1)
#define FEQ_GATE_CM_HEAD                                                                   \
    constexpr int NRS = W == 4 ? NR : FEQ_MAX_IRREPS;                                       \
    const int nr = W == 4 ? NR : L.nreps;                                                   \
    const int64_t p = (static_cast<int64_t>(blockIdx.x) * kRowThreads + threadIdx.x) * W;  \
    if (p >= P) return;

template <int W, int NR>
__global__ void __launch_bounds__(kRowThreads)
k_gate_norms_cm(NodeL L, int64_t P, const float* __restrict__ x, float eps, float* __restrict__ nrm) {
    FEQ_GATE_CM_HEAD
    float out[W * NRS];
#pragma unroll
    for (int k = 0; k < NRS; ++k) {
        if (k >= nr) break;
        float q[W] = {};
        for (int d = L.off[k]; d < L.off[k + 1]; ++d) {
            float v[W];
            ld_w<W>(x + d * P + p, v);
#pragma unroll
            for (int w = 0; w < W; ++w) q[w] += v[w] * v[w];
        }
#pragma unroll
        for (int w = 0; w < W; ++w) out[pv<W, NRS>(w, k)] = sqrtf(q[w] + eps);
    }
    st_pairs<W, NRS>(nrm, p, nr, out);
}

template <int W, int NR>
__global__ void __launch_bounds__(kRowThreads)
k_gate_apply_cm(NodeL L, int64_t P, const float* __restrict__ x, const float* __restrict__ lin,
                float* __restrict__ y) {
    FEQ_GATE_CM_HEAD
    float lv[W * NRS];
    ld_pairs<W, NRS>(lin, p, nr, lv);
#pragma unroll
    for (int k = 0; k < NRS; ++k) {
        if (k >= nr) break;
        float g[W];
#pragma unroll
        for (int w = 0; w < W; ++w) g[w] = sigmoidf(lv[pv<W, NRS>(w, k)]);
        for (int d = L.off[k]; d < L.off[k + 1]; ++d) {
            float v[W];
            ld_w<W>(x + d * P + p, v);
#pragma unroll
            for (int w = 0; w < W; ++w) v[w] *= g[w];
            st_w<W>(y + d * P + p, v);
        }
    }
}

template <int W, int NR>
__global__ void __launch_bounds__(kRowThreads)
k_gate_bwd_lin_cm(NodeL L, int64_t P, const float* __restrict__ gy, const float* __restrict__ x,
                  const float* __restrict__ lin, float* __restrict__ dlin) {
    FEQ_GATE_CM_HEAD
    float lv[W * NRS];
    ld_pairs<W, NRS>(lin, p, nr, lv);
#pragma unroll
    for (int k = 0; k < NRS; ++k) {
        if (k >= nr) break;
        float q[W] = {};
        for (int d = L.off[k]; d < L.off[k + 1]; ++d) {
            float a[W], v[W];
            ld_w<W>(gy + d * P + p, a);
            ld_w<W>(x + d * P + p, v);
#pragma unroll
            for (int w = 0; w < W; ++w) q[w] += a[w] * v[w];
        }
#pragma unroll
        for (int w = 0; w < W; ++w) {
            const float g = sigmoidf(lv[pv<W, NRS>(w, k)]);
            lv[pv<W, NRS>(w, k)] = q[w] * (g * (1.0f - g));
        }
    }
    st_pairs<W, NRS>(dlin, p, nr, lv);
}

template <int W, int NR>
__global__ void __launch_bounds__(kRowThreads)
k_gate_bwd_x_cm(NodeL L, int64_t P, const float* __restrict__ gy, const float* __restrict__ x,
                const float* __restrict__ lin, const float* __restrict__ nrm,
                const float* __restrict__ dnrm, float* __restrict__ gx) {
    FEQ_GATE_CM_HEAD
    float lv[W * NRS], nv[W * NRS], dv[W * NRS];
    ld_pairs<W, NRS>(lin, p, nr, lv);
    ld_pairs<W, NRS>(nrm, p, nr, nv);
    ld_pairs<W, NRS>(dnrm, p, nr, dv);
#pragma unroll
    for (int k = 0; k < NRS; ++k) {
        if (k >= nr) break;
        float g[W], q[W];
#pragma unroll
        for (int w = 0; w < W; ++w) {
            const int i = pv<W, NRS>(w, k);
            g[w] = sigmoidf(lv[i]);
            q[w] = dv[i] / nv[i];
        }
        for (int d = L.off[k]; d < L.off[k + 1]; ++d) {
            float a[W], v[W];
            ld_w<W>(gy + d * P + p, a);
            ld_w<W>(x + d * P + p, v);
#pragma unroll
            for (int w = 0; w < W; ++w) a[w] = a[w] * g[w] + v[w] * q[w];
            st_w<W>(gx + d * P + p, a);
        }
    }
}
#undef FEQ_GATE_CM_HEAD

// ---- host ---------------------------------------------------------------------

int cpl_of(int mult) { return mult <= 64 ? 1 : mult <= 128 ? 2 : 4; }

int64_t bwd_waves(int64_t N) {
    return std::min<int64_t>(ceil_div(N, kWaves), kBwdGroups) * kWaves;
}

// partials of n floats per wave, and reduce_partials' temporary
size_t partial_floats(int64_t waves, int64_t n) {
    return align_up(static_cast<size_t>(waves * n), 64) + align_up(static_cast<size_t>(ceil_div(waves, 32) * n), 64);
}

int check_rows(int64_t N, const void* a, const void* b, const void* c) {
    if (N < 0) return fail(FEQ_ERR_INVALID, "negative node count");
    if (N > 0 && (!a || !b || !c)) return fail(FEQ_ERR_INVALID, "NULL tensor pointer");
    return FEQ_OK;
}

}  // namespace
}  // namespace feq

using namespace feq;

#define FEQ_NODE_DISPATCH_S(CPL_, ...)                         \
    switch (CPL_) {                                            \
        case 1: { constexpr int cpl = 1; __VA_ARGS__; } break; \
        case 2: { constexpr int cpl = 2; __VA_ARGS__; } break; \
        default: { constexpr int cpl = 4; __VA_ARGS__; } break; \
    }
// whether node rows move with 16-byte accesses
#define FEQ_VEC_DISPATCH(COND_, ...)                           \
    if (COND_) {                                               \
        constexpr bool vec = true;                             \
        __VA_ARGS__;                                           \
    } else {                                                   \
        constexpr bool vec = false;                            \
        __VA_ARGS__;                                           \
    }
// whether the input gradient takes an addend
#define FEQ_ADD_DISPATCH(COND_, ...)                           \
    if (COND_) {                                               \
        constexpr bool add = true;                             \
        __VA_ARGS__;                                           \
    } else {                                                   \
        constexpr bool add = false;                            \
        __VA_ARGS__;                                           \
    }
// channels per lane and whether a node row is staged in LDS
#define FEQ_NODE_DISPATCH(L_, ...)                                                        \
    if (int64_t(L_.mult) * L_.dim <= kStageRow) {                                         \
        constexpr bool stage = true;                                                      \
        FEQ_NODE_DISPATCH_S(cpl_of(L_.mult), __VA_ARGS__)                                 \
    } else {                                                                              \
        constexpr bool stage = false;                                                     \
        FEQ_NODE_DISPATCH_S(cpl_of(L_.mult), __VA_ARGS__)                                 \
    }

namespace {
int sepnorm_fwd(const int32_t* lvals, int32_t nreps, int32_t mult, int64_t N, const float* x,
                const float* w_s, const float* b_s, const float* w_h, float eps, float* y, bool cm,
                feq_stream_t stream) {
    NodeL L;
    if (int rc = make_nodel(lvals, nreps, mult, &L)) return rc;
    if (L.ns > kMaxS) return fail(FEQ_ERR_UNSUPPORTED, "at most %d scalar irreps", kMaxS);
    if (int rc = check_rows(N, x, y, x)) return rc;
    if ((L.ns && (!w_s || !b_s)) || (L.nhc && !w_h)) return fail(FEQ_ERR_INVALID, "NULL norm weight");
    L.vec = L.vec && al16(x) && al16(y);
    if (cm && int64_t(L.mult) * L.dim > kStageRow)
        return fail(FEQ_ERR_UNSUPPORTED, "component-major norm output: at most %d floats per node", kStageRow);
    if (N == 0) return FEQ_OK;
    hipStream_t s = stream_of(stream);
    const dim3 grid(static_cast<unsigned>(ceil_div(N, kWaves)));
    if (cm) {
        FEQ_VEC_DISPATCH(L.vec, FEQ_NODE_DISPATCH_S(cpl_of(L.mult), {
            auto k = k_sepnorm_fwd<cpl, true, true, vec>;
            FEQ_LAUNCH("k_sepnorm_fwd", k, grid, dim3(64 * kWaves), 0, s, L, N, x, w_s, b_s, w_h, eps, y);
        }))
        return FEQ_OK;
    }
    FEQ_VEC_DISPATCH(L.vec, FEQ_NODE_DISPATCH(L, {
        auto k = k_sepnorm_fwd<cpl, stage, false, stage && vec>;
        FEQ_LAUNCH("k_sepnorm_fwd", k, grid, dim3(64 * kWaves), 0, s, L, N, x, w_s, b_s, w_h, eps, y);
    }))
    return FEQ_OK;
}
}  // namespace

extern "C" int feq_sepnorm_fwd(const int32_t* lvals, int32_t nreps, int32_t mult, int64_t N,
                               const float* x, const float* w_s, const float* b_s,
                               const float* w_h, float eps, float* y, feq_stream_t stream) {
    return sepnorm_fwd(lvals, nreps, mult, N, x, w_s, b_s, w_h, eps, y, false, stream);
}

extern "C" int feq_sepnorm_fwd_cm(const int32_t* lvals, int32_t nreps, int32_t mult, int64_t N,
                                  const float* x, const float* w_s, const float* b_s,
                                  const float* w_h, float eps, float* y, feq_stream_t stream) {
    return sepnorm_fwd(lvals, nreps, mult, N, x, w_s, b_s, w_h, eps, y, true, stream);
}

extern "C" size_t feq_sepnorm_workspace(const int32_t* lvals, int32_t nreps, int32_t mult, int64_t N) {
    NodeL L;
    if (make_nodel(lvals, nreps, mult, &L) || N <= 0) return 0;
    const int64_t w = bwd_waves(N);
    return sizeof(float) * (2 * partial_floats(w, int64_t(mult) * L.ns) + partial_floats(w, mult)) + 256;
}

namespace {
int sepnorm_bwd(const int32_t* lvals, int32_t nreps, int32_t mult, int64_t N, const float* gy,
                const float* x, const float* w_s, const float* w_h, float eps, const float* ga, float* gx,
                float* gw_s, float* gb_s, float* gw_h, void* ws, size_t ws_bytes, bool cm,
                feq_stream_t stream) {
    NodeL L;
    if (int rc = make_nodel(lvals, nreps, mult, &L)) return rc;
    if (cm && int64_t(L.mult) * L.dim > kStageRow)
        return fail(FEQ_ERR_UNSUPPORTED, "component-major norm gradient: at most %d floats per node", kStageRow);
    if (ga && int64_t(L.mult) * L.dim > kStageRow)
        return fail(FEQ_ERR_UNSUPPORTED, "norm gradient with an addend: at most %d floats per node", kStageRow);
    if (L.ns > kMaxS) return fail(FEQ_ERR_UNSUPPORTED, "at most %d scalar irreps", kMaxS);
    if (int rc = check_rows(N, gy, x, gx)) return rc;
    if ((L.ns && (!w_s || !gw_s || !gb_s)) || (L.nhc && (!w_h || !gw_h)))
        return fail(FEQ_ERR_INVALID, "NULL norm weight or gradient");
    L.vec = L.vec && al16(gy) && al16(x) && al16(gx) && al16(ga);
    hipStream_t s = stream_of(stream);
    const int64_t nsc = int64_t(mult) * L.ns;
    if (N == 0) {
        if (L.ns) {
            if (int rc = fill_zero(gw_s, nsc, s)) return rc;
            if (int rc = fill_zero(gb_s, nsc, s)) return rc;
        }
        if (L.nhc) return fill_zero(gw_h, mult, s);
        return FEQ_OK;
    }
    if (!ws || ws_bytes < feq_sepnorm_workspace(lvals, nreps, mult, N))
        return fail(FEQ_ERR_WORKSPACE, "separable norm workspace too small");
    const int64_t w = bwd_waves(N);
    float* base = static_cast<float*>(ws);
    float* pS = base;
    float* pB = pS + partial_floats(w, nsc);
    float* pH = pB + partial_floats(w, nsc);
    if (cm) {
        FEQ_ADD_DISPATCH(ga != nullptr, FEQ_VEC_DISPATCH(L.vec, FEQ_NODE_DISPATCH_S(cpl_of(L.mult), {
            auto k = L.ns <= 1 ? k_sepnorm_bwd<cpl, true, true, vec, add, 1> : k_sepnorm_bwd<cpl, true, true, vec, add>;
            FEQ_LAUNCH("k_sepnorm_bwd", k, dim3(static_cast<unsigned>(w / kWaves)), dim3(64 * kWaves), 0,
                       s, L, N, gy, x, w_s, w_h, eps, gx, pS, pB, L.nhc ? pH : nullptr, ga);
        })))
    } else {
        FEQ_ADD_DISPATCH(ga != nullptr, FEQ_VEC_DISPATCH(L.vec, FEQ_NODE_DISPATCH(L, {
            auto k = L.ns <= 1 ? k_sepnorm_bwd<cpl, stage, false, stage && vec, stage && add, 1>
                               : k_sepnorm_bwd<cpl, stage, false, stage && vec, stage && add>;
            FEQ_LAUNCH("k_sepnorm_bwd", k, dim3(static_cast<unsigned>(w / kWaves)), dim3(64 * kWaves), 0,
                       s, L, N, gy, x, w_s, w_h, eps, gx, pS, pB, L.nhc ? pH : nullptr, ga);
        })))
    }
    PartialJob jobs[3];
    int nj = 0;
    if (L.ns) {
        jobs[nj++] = PartialJob{pS, int(w), nsc, gw_s, pS + w * nsc};
        jobs[nj++] = PartialJob{pB, int(w), nsc, gb_s, pB + w * nsc};
    }
    if (L.nhc) jobs[nj++] = PartialJob{pH, int(w), mult, gw_h, pH + w * mult};
    return reduce_partials_multi(jobs, nj, s);
}
}  // namespace

extern "C" int feq_sepnorm_bwd(const int32_t* lvals, int32_t nreps, int32_t mult, int64_t N,
                               const float* gy, const float* x, const float* w_s, const float* w_h,
                               float eps, float* gx, float* gw_s, float* gb_s, float* gw_h,
                               void* ws, size_t ws_bytes, feq_stream_t stream) {
    return sepnorm_bwd(lvals, nreps, mult, N, gy, x, w_s, w_h, eps, nullptr, gx, gw_s, gb_s, gw_h, ws, ws_bytes,
                       false, stream);
}

extern "C" int feq_sepnorm_bwd_cm(const int32_t* lvals, int32_t nreps, int32_t mult, int64_t N,
                                  const float* gy, const float* x, const float* w_s, const float* w_h,
                                  float eps, float* gx, float* gw_s, float* gb_s, float* gw_h,
                                  void* ws, size_t ws_bytes, feq_stream_t stream) {
    return sepnorm_bwd(lvals, nreps, mult, N, gy, x, w_s, w_h, eps, nullptr, gx, gw_s, gb_s, gw_h, ws, ws_bytes,
                       true, stream);
}

extern "C" int feq_sepnorm_bwd_add(const int32_t* lvals, int32_t nreps, int32_t mult, int64_t N,
                                   const float* gy, const float* x, const float* w_s, const float* w_h,
                                   float eps, const float* gx_add, float* gx, float* gw_s, float* gb_s,
                                   float* gw_h, void* ws, size_t ws_bytes, int32_t cm, feq_stream_t stream) {
    if (N > 0 && !gx_add) return fail(FEQ_ERR_INVALID, "NULL gradient addend");
    return sepnorm_bwd(lvals, nreps, mult, N, gy, x, w_s, w_h, eps, gx_add, gx, gw_s, gb_s, gw_h, ws, ws_bytes,
                       cm != 0, stream);
}

namespace {
int eqnorm_fwd(const int32_t* lvals, int32_t nreps, int32_t mult, int64_t N, const float* x,
               const float* w_ln, const float* b_ln, float eps, float ln_eps, float* y, bool cm,
               feq_stream_t stream) {
    NodeL L;
    if (int rc = make_nodel(lvals, nreps, mult, &L)) return rc;
    if (int rc = check_rows(N, x, y, x)) return rc;
    if (!w_ln != !b_ln) return fail(FEQ_ERR_INVALID, "LayerNorm weight and bias go together");
    L.vec = L.vec && al16(x) && al16(y);
    if (cm && int64_t(L.mult) * L.dim > kStageRow)
        return fail(FEQ_ERR_UNSUPPORTED, "component-major norm output: at most %d floats per node", kStageRow);
    if (N == 0) return FEQ_OK;
    hipStream_t s = stream_of(stream);
    const dim3 grid(static_cast<unsigned>(ceil_div(N, kWaves)));
    if (cm) {
        FEQ_VEC_DISPATCH(L.vec, FEQ_NODE_DISPATCH_S(cpl_of(L.mult), {
            auto k = k_eqnorm_fwd<cpl, true, true, vec>;
            FEQ_LAUNCH("k_eqnorm_fwd", k, grid, dim3(64 * kWaves), 0, s, L, N, x, w_ln, b_ln, eps, ln_eps, y);
        }))
        return FEQ_OK;
    }
    FEQ_VEC_DISPATCH(L.vec, FEQ_NODE_DISPATCH(L, {
        auto k = k_eqnorm_fwd<cpl, stage, false, stage && vec>;
        FEQ_LAUNCH("k_eqnorm_fwd", k, grid, dim3(64 * kWaves), 0, s, L, N, x, w_ln, b_ln, eps, ln_eps, y);
    }))
    return FEQ_OK;
}
}  // namespace

extern "C" int feq_eqnorm_fwd(const int32_t* lvals, int32_t nreps, int32_t mult, int64_t N,
                              const float* x, const float* w_ln, const float* b_ln, float eps,
                              float ln_eps, float* y, feq_stream_t stream) {
    return eqnorm_fwd(lvals, nreps, mult, N, x, w_ln, b_ln, eps, ln_eps, y, false, stream);
}

extern "C" int feq_eqnorm_fwd_cm(const int32_t* lvals, int32_t nreps, int32_t mult, int64_t N,
                                 const float* x, const float* w_ln, const float* b_ln, float eps,
                                 float ln_eps, float* y, feq_stream_t stream) {
    return eqnorm_fwd(lvals, nreps, mult, N, x, w_ln, b_ln, eps, ln_eps, y, true, stream);
}

extern "C" size_t feq_eqnorm_workspace(const int32_t* lvals, int32_t nreps, int32_t mult, int64_t N) {
    NodeL L;
    if (make_nodel(lvals, nreps, mult, &L) || N <= 0) return 0;
    return sizeof(float) * 2 * partial_floats(bwd_waves(N), mult) + 256;
}

namespace {
int eqnorm_bwd(const int32_t* lvals, int32_t nreps, int32_t mult, int64_t N, const float* gy,
               const float* x, const float* w_ln, const float* b_ln, float eps, float ln_eps, const float* ga,
               float* gx, float* gw_ln, float* gb_ln, void* ws, size_t ws_bytes, bool cm,
               feq_stream_t stream) {
    NodeL L;
    if (int rc = make_nodel(lvals, nreps, mult, &L)) return rc;
    if (cm && int64_t(L.mult) * L.dim > kStageRow)
        return fail(FEQ_ERR_UNSUPPORTED, "component-major norm gradient: at most %d floats per node", kStageRow);
    if (ga && int64_t(L.mult) * L.dim > kStageRow)
        return fail(FEQ_ERR_UNSUPPORTED, "norm gradient with an addend: at most %d floats per node", kStageRow);
    if (int rc = check_rows(N, gy, x, gx)) return rc;
    if (!w_ln != !b_ln) return fail(FEQ_ERR_INVALID, "LayerNorm weight and bias go together");
    L.vec = L.vec && al16(gy) && al16(x) && al16(gx) && al16(ga);
    if (w_ln && (!gw_ln || !gb_ln)) return fail(FEQ_ERR_INVALID, "NULL LayerNorm gradient");
    hipStream_t s = stream_of(stream);
    if (N == 0) {
        if (!w_ln) return FEQ_OK;
        if (int rc = fill_zero(gw_ln, mult, s)) return rc;
        return fill_zero(gb_ln, mult, s);
    }
    if (w_ln && (!ws || ws_bytes < feq_eqnorm_workspace(lvals, nreps, mult, N)))
        return fail(FEQ_ERR_WORKSPACE, "equivariant norm workspace too small");
    const int64_t w = bwd_waves(N);
    float* pW = w_ln ? static_cast<float*>(ws) : nullptr;
    float* pB = w_ln ? pW + partial_floats(w, mult) : nullptr;
    if (cm) {
        FEQ_ADD_DISPATCH(ga != nullptr, FEQ_VEC_DISPATCH(L.vec, FEQ_NODE_DISPATCH_S(cpl_of(L.mult), {
            auto k = k_eqnorm_bwd<cpl, true, true, vec, add>;
            FEQ_LAUNCH("k_eqnorm_bwd", k, dim3(static_cast<unsigned>(w / kWaves)), dim3(64 * kWaves), 0,
                       s, L, N, gy, x, w_ln, b_ln, eps, ln_eps, gx, pW, pB, ga);
        })))
    } else {
        FEQ_ADD_DISPATCH(ga != nullptr, FEQ_VEC_DISPATCH(L.vec, FEQ_NODE_DISPATCH(L, {
            auto k = k_eqnorm_bwd<cpl, stage, false, stage && vec, stage && add>;
            FEQ_LAUNCH("k_eqnorm_bwd", k, dim3(static_cast<unsigned>(w / kWaves)), dim3(64 * kWaves), 0,
                       s, L, N, gy, x, w_ln, b_ln, eps, ln_eps, gx, pW, pB, ga);
        })))
    }
    if (!w_ln) return FEQ_OK;
    const PartialJob jobs[2] = {PartialJob{pW, int(w), mult, gw_ln, pW + w * mult},
                                PartialJob{pB, int(w), mult, gb_ln, pB + w * mult}};
    return reduce_partials_multi(jobs, 2, s);
}
}  // namespace

extern "C" int feq_eqnorm_bwd(const int32_t* lvals, int32_t nreps, int32_t mult, int64_t N,
                              const float* gy, const float* x, const float* w_ln, const float* b_ln,
                              float eps, float ln_eps, float* gx, float* gw_ln, float* gb_ln,
                              void* ws, size_t ws_bytes, feq_stream_t stream) {
    return eqnorm_bwd(lvals, nreps, mult, N, gy, x, w_ln, b_ln, eps, ln_eps, nullptr, gx, gw_ln, gb_ln, ws,
                      ws_bytes, false, stream);
}

extern "C" int feq_eqnorm_bwd_cm(const int32_t* lvals, int32_t nreps, int32_t mult, int64_t N,
                                 const float* gy, const float* x, const float* w_ln, const float* b_ln,
                                 float eps, float ln_eps, float* gx, float* gw_ln, float* gb_ln,
                                 void* ws, size_t ws_bytes, feq_stream_t stream) {
    return eqnorm_bwd(lvals, nreps, mult, N, gy, x, w_ln, b_ln, eps, ln_eps, nullptr, gx, gw_ln, gb_ln, ws,
                      ws_bytes, true, stream);
}

extern "C" int feq_eqnorm_bwd_add(const int32_t* lvals, int32_t nreps, int32_t mult, int64_t N,
                                  const float* gy, const float* x, const float* w_ln, const float* b_ln,
                                  float eps, float ln_eps, const float* gx_add, float* gx, float* gw_ln,
                                  float* gb_ln, void* ws, size_t ws_bytes, int32_t cm, feq_stream_t stream) {
    if (N > 0 && !gx_add) return fail(FEQ_ERR_INVALID, "NULL gradient addend");
    return eqnorm_bwd(lvals, nreps, mult, N, gy, x, w_ln, b_ln, eps, ln_eps, gx_add, gx, gw_ln, gb_ln, ws,
                      ws_bytes, cm != 0, stream);
}

// v4: the component-major kernels' 16-byte form (four pairs per thread)
#define FEQ_GATE_PRELUDE(a, b, c, d)                                                      \
    NodeL L;                                                                              \
    if (int rc = make_nodel(lvals, nreps, mult, &L)) return rc;                           \
    if (int rc = check_rows(N, a, b, c)) return rc;                                       \
    if (N == 0) return FEQ_OK;                                                            \
    const int64_t rows = N * mult;                                                        \
    const bool v4 = cm && mult % 4 == 0 && nreps <= 4 && al16(a) && al16(b) && al16(c) && al16(d);  \
    const dim3 grid(static_cast<unsigned>(                                                \
        ceil_div(rows, cm ? kRowThreads * (v4 ? 4 : 1) : std::min(kRowThreads, kTileFloats / L.dim))));  \
    hipStream_t s = stream_of(stream);

extern "C" int feq_gate_norms(const int32_t* lvals, int32_t nreps, int32_t mult, int64_t N,
                              int32_t cm, const float* x, float eps, float* norms,
                              feq_stream_t stream) {
    FEQ_GATE_PRELUDE(x, norms, x, x)
    if (cm) {
        auto k = !v4 ? k_gate_norms_cm<1, 0> : nreps == 1 ? k_gate_norms_cm<4, 1> : nreps == 2 ? k_gate_norms_cm<4, 2>
                 : nreps == 3 ? k_gate_norms_cm<4, 3> : k_gate_norms_cm<4, 4>;
        FEQ_LAUNCH("k_gate_norms", k, grid, dim3(kRowThreads), 0, s, L, rows, x, eps, norms);
    } else
        FEQ_LAUNCH("k_gate_norms", k_gate_norms, grid, dim3(kRowThreads), 0, s, L, rows, x, eps, norms);
    return FEQ_OK;
}

extern "C" int feq_gate_apply(const int32_t* lvals, int32_t nreps, int32_t mult, int64_t N,
                              int32_t cm, const float* x, const float* lin, float* y,
                              feq_stream_t stream) {
    FEQ_GATE_PRELUDE(x, lin, y, y)
    if (cm) {
        auto k = !v4 ? k_gate_apply_cm<1, 0> : nreps == 1 ? k_gate_apply_cm<4, 1> : nreps == 2 ? k_gate_apply_cm<4, 2>
                 : nreps == 3 ? k_gate_apply_cm<4, 3> : k_gate_apply_cm<4, 4>;
        FEQ_LAUNCH("k_gate_apply", k, grid, dim3(kRowThreads), 0, s, L, rows, x, lin, y);
    } else
        FEQ_LAUNCH("k_gate_apply", k_gate_apply, grid, dim3(kRowThreads), 0, s, L, rows, x, lin, y);
    return FEQ_OK;
}

extern "C" int feq_gate_bwd_lin(const int32_t* lvals, int32_t nreps, int32_t mult, int64_t N,
                                int32_t cm, const float* gy, const float* x, const float* lin,
                                float* grad_lin, feq_stream_t stream) {
    FEQ_GATE_PRELUDE(gy, x, lin, grad_lin)
    if (!grad_lin) return fail(FEQ_ERR_INVALID, "NULL tensor pointer");
    if (cm) {
        auto k = !v4 ? k_gate_bwd_lin_cm<1, 0> : nreps == 1 ? k_gate_bwd_lin_cm<4, 1> : nreps == 2 ? k_gate_bwd_lin_cm<4, 2>
                 : nreps == 3 ? k_gate_bwd_lin_cm<4, 3> : k_gate_bwd_lin_cm<4, 4>;
        FEQ_LAUNCH("k_gate_bwd_lin", k, grid, dim3(kRowThreads), 0, s, L, rows, gy, x, lin, grad_lin);
    } else
        FEQ_LAUNCH("k_gate_bwd_lin", k_gate_bwd_lin, grid, dim3(kRowThreads), 0, s, L, rows, gy, x,
                   lin, grad_lin);
    return FEQ_OK;
}

extern "C" int feq_gate_bwd_x(const int32_t* lvals, int32_t nreps, int32_t mult, int64_t N,
                              int32_t cm, const float* gy, const float* x, const float* lin,
                              const float* norms, const float* grad_norms, float* gx,
                              feq_stream_t stream) {
    FEQ_GATE_PRELUDE(gy, x, lin, gx)
    if (!norms || !grad_norms || !gx) return fail(FEQ_ERR_INVALID, "NULL tensor pointer");
    if (cm) {
        auto k = !v4 ? k_gate_bwd_x_cm<1, 0> : nreps == 1 ? k_gate_bwd_x_cm<4, 1> : nreps == 2 ? k_gate_bwd_x_cm<4, 2>
                 : nreps == 3 ? k_gate_bwd_x_cm<4, 3> : k_gate_bwd_x_cm<4, 4>;
        FEQ_LAUNCH("k_gate_bwd_x", k, grid, dim3(kRowThreads), 0, s, L, rows, gy, x, lin, norms, grad_norms,
                   gx);
    } else
        FEQ_LAUNCH("k_gate_bwd_x", k_gate_bwd_x, grid, dim3(kRowThreads), 0, s, L, rows, gy, x, lin,
                   norms, grad_norms, gx);
    return FEQ_OK;
}

extern "C" size_t feq_scale_add_cm_workspace(void) { return sizeof(double) * kResGroups; }

extern "C" int feq_scale_add_cm(const float* x, const float* y, const float* scale, int64_t N, int32_t mult,
                                int32_t dim, float* out, feq_stream_t stream) {
    if (N < 0 || mult < 1 || dim < 1) return fail(FEQ_ERR_INVALID, "invalid sizes");
    if (int64_t(mult) * dim > kStageRow)
        return fail(FEQ_ERR_UNSUPPORTED, "component-major residual: at most %d floats per node", kStageRow);
    if (N == 0) return FEQ_OK;
    if (!x || !y || !scale || !out) return fail(FEQ_ERR_INVALID, "NULL pointer");
    const int64_t g = ceil_div(N, kWaves);
    const int vec = mult % 4 == 0 && al16(x) && al16(y) && al16(out);
    FEQ_LAUNCH("k_scale_add_cm", k_scale_add_cm, dim3(static_cast<unsigned>(g < kResGroups ? g : kResGroups)),
               dim3(64 * kWaves), 0, stream_of(stream), N, int(mult), int(dim), vec, x, y, scale, out);
    return FEQ_OK;
}

extern "C" int feq_scale_add_cm_bwd(const float* grad_out, const float* y, const float* scale, int64_t N,
                                    int32_t mult, int32_t dim, float* grad_y, float* grad_scale, void* ws,
                                    size_t ws_bytes, feq_stream_t stream) {
    if (N < 0 || mult < 1 || dim < 1) return fail(FEQ_ERR_INVALID, "invalid sizes");
    if (int64_t(mult) * dim > kStageRow)
        return fail(FEQ_ERR_UNSUPPORTED, "component-major residual: at most %d floats per node", kStageRow);
    if (!grad_scale && !grad_y) return FEQ_OK;
    if (!scale || (N > 0 && (!grad_out || !y))) return fail(FEQ_ERR_INVALID, "NULL pointer");
    if (!ws || ws_bytes < feq_scale_add_cm_workspace())
        return fail(FEQ_ERR_WORKSPACE, "residual workspace too small");
    hipStream_t s = stream_of(stream);
    double* part = static_cast<double*>(ws);
    const int vec = mult % 4 == 0 && al16(grad_out) && al16(y) && al16(grad_y);
    FEQ_LAUNCH("k_scale_add_cm_bwd", k_scale_add_cm_bwd, dim3(kResGroups), dim3(64 * kWaves), 0, s, N, int(mult),
               int(dim), vec, grad_out, y, scale, grad_y, part);
    if (grad_scale) FEQ_LAUNCH("k_sum_f64", k_sum_f64, dim3(1), dim3(64 * kWaves), 0, s, part, kResGroups, grad_scale);
    return FEQ_OK;
}

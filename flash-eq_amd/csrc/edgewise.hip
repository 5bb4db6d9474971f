// Fused EquivariantEdgewiseLinear: y = Q-rotate( Lambda(r) (x P) ).
//
// Reference pipeline (flash_eq/layers/linear.py:100-160): f = bmm(x, P);
// out = block_diagonal_cuda(f, rw(), r, ...); y = bmm(out, Q^T), where the
// table rw() = einsum('koi,bkw->boiw', C, F) is the SeparableRadialNet output
// (radial.py:259-275).  Because the table has rank K in the channel pair,
//   lerp_t(T)[co,ci,w] = sum_k C[k,co,ci] F_e[k,w],   F_e = (1-t) F[lo] + t F[lo+1],
// so the per-edge mix factorises as
//   Z_k[ci, o] = sum_i F_e[k, w(o,i)] fs[ci, i]      (cheap, per edge)
//   yd[co, o]  = sum_k sum_ci C[k,co,ci] Z_k[ci, o]  (the GEMM-shaped part)
// with fs = s^l (x P) and the 2x2 [[a,b],[-b,a]] structure on (+m,-m) pairs.
// The table (num_bins+1, Cout, Cin, Wdim) is never formed.
//
// Backward (H_k = C_k^T gd, gd = s^l (gy Q)):
//   dfs[ci,i] = sum_k sum_o F_e[k,w(o,i)] H_k[ci,o]     -> dx = s^l dfs P^T
//   dF_e[k,w(o,i)] = sum_ci fs[ci,i] H_k[ci,o]         -> dF[lo] += (1-t) dF_e, dF[hi] += t dF_e
//   dC[k,co,ci] = sum_e sum_o gd[co,o] Z_k[ci,o]
//   dr = dt/dr sum_{k,w} (F[hi]-F[lo]) dF_e + sigma/(r(r+sigma)) sum_{k,w} (l_i+l_o) F_e dF_e
// which equals the reference's grad_distances (block_diagonal.cu:990-1036,
// 1113-1160) for a table of this form, including NaN at r = 0.
#include "feq_internal.h"

#include <mutex>

namespace feq {
namespace {

// Threads per workgroup of the shape-generic kernels: 256, 512 or 1024, the
// smallest that gives a CU at least 16 waves at the layout's LDS (pick_threads;
// measured at lvals 0..6 x 32 channels: the backward at 89 KB of LDS, one
// workgroup per CU, 28.2 / 17.2 / 11.5 ms per published step with 256 / 512 /
// 1024 threads; lvals 0..4 (48 KB, three workgroups) 7.6 / 5.1 / 6.3 ms).
constexpr int kMaxThreads = 1024;
constexpr int kBwdGroups = 1024;  // workgroups of the backward pass

struct Blk {
    int m, ni, no, in_off, out_off, w_off;
};

__device__ __forceinline__ Blk get_blk(const feq_layout& L, int k) {
    return {L.blk[k][0], L.blk[k][1], L.blk[k][2], L.blk[k][3], L.blk[k][4], L.blk[k][5]};
}

// Block / index / component of an m-first output slot (blk = -1: not mixed).
__device__ __forceinline__ int out_block(const feq_layout& L, int slot, int& o, int& c) {
    for (int k = 0; k < L.nblocks; ++k) {
        const int w = L.blk[k][0] == 0 ? 1 : 2;
        const int off = L.blk[k][4];
        if (slot >= off && slot < off + w * L.blk[k][2]) {
            o = (slot - off) / w;
            c = (slot - off) % w;
            return k;
        }
    }
    return -1;
}

__device__ __forceinline__ int in_block(const feq_layout& L, int slot, int& i, int& c) {
    for (int k = 0; k < L.nblocks; ++k) {
        const int w = L.blk[k][0] == 0 ? 1 : 2;
        const int off = L.blk[k][3];
        if (slot >= off && slot < off + w * L.blk[k][1]) {
            i = (slot - off) / w;
            c = (slot - off) % w;
            return k;
        }
    }
    return -1;
}

// Z[ci, slot] = sum_i F_e[w(o,i)] fs[ci, i] for one rank component (sFk = F_e[k, :]).
__device__ __forceinline__ float z_entry(const feq_layout& L, const float* sFk, const float* sf,
                                         int ci, int slot) {
    int o, c;
    const int kb = out_block(L, slot, o, c);
    if (kb < 0) return 0.0f;
    const Blk b = get_blk(L, kb);
    const float* f = sf + ci * L.din + b.in_off;
    float acc = 0.0f;
    if (b.m == 0) {
        const float* w = sFk + b.w_off + o * b.ni;
        for (int i = 0; i < b.ni; ++i) acc += w[i] * f[i];
    } else {
        const float* w = sFk + b.w_off + 2 * o * b.ni;
        for (int i = 0; i < b.ni; ++i) {
            const float a = w[2 * i], bb = w[2 * i + 1];
            const float fr = f[2 * i], fi = f[2 * i + 1];
            acc += c == 0 ? (a * fr + bb * fi) : (a * fi - bb * fr);
        }
    }
    return acc;
}

// dfs[ci, slot] contribution of one rank component: sum_o F_e[w(o,i)] H[ci, o] (transposed 2x2).
__device__ __forceinline__ float dz_entry(const feq_layout& L, const float* sFk, const float* sH,
                                          int ci, int slot) {
    int i, c;
    const int kb = in_block(L, slot, i, c);
    if (kb < 0) return 0.0f;
    const Blk b = get_blk(L, kb);
    const float* h = sH + ci * L.dout + b.out_off;
    float acc = 0.0f;
    if (b.m == 0) {
        for (int o = 0; o < b.no; ++o) acc += sFk[b.w_off + o * b.ni + i] * h[o];
    } else {
        for (int o = 0; o < b.no; ++o) {
            const float a = sFk[b.w_off + 2 * (o * b.ni + i)];
            const float bb = sFk[b.w_off + 2 * (o * b.ni + i) + 1];
            const float hr = h[2 * o], hi = h[2 * o + 1];
            acc += c == 0 ? (a * hr - bb * hi) : (bb * hr + a * hi);
        }
    }
    return acc;
}

// Weight w -> (block, o, i, component) and its degree sum l_i + l_o.
__device__ __forceinline__ int weight_info(const feq_layout& L, int w, Blk& b, int& o, int& i,
                                           int& comp) {
    int k = L.nblocks - 1;
    while (k > 0 && w < L.blk[k][5]) --k;
    b = get_blk(L, k);
    const int rel = w - b.w_off;
    if (b.m == 0) {
        o = rel / b.ni;
        i = rel % b.ni;
        comp = 0;
        return L.lslot_in[b.in_off + i] + L.lslot_out[b.out_off + o];
    }
    comp = rel & 1;
    o = (rel >> 1) / b.ni;
    i = (rel >> 1) % b.ni;
    return L.lslot_in[b.in_off + 2 * i] + L.lslot_out[b.out_off + 2 * o];
}

template <int NT>
__device__ __forceinline__ float block_sum(float v, float* red) {
    for (int off = 32; off > 0; off >>= 1) v += __shfl_down(v, off, 64);
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[wid] = v;
    __syncthreads();
    float s = 0.0f;
    for (int w = 0; w < NT / 64; ++w) s += red[w];
    __syncthreads();
    return s;
}

struct EwDims {
    int K;
    int nbins;
};

// ---------------------------------------------------------------------------
// SC: the channel patterns C (K, Cout, Cin) staged in LDS (read in the
// innermost GEMM loops; from global memory each read exposed the L2 latency),
// where they fit beside the edge's rows.
template <int kThreads, bool SC>
__global__ void __launch_bounds__(kThreads)
k_ew_fwd(feq_layout L, feq_binning B, EwDims D, const float* __restrict__ x,
         const float* __restrict__ P, const float* __restrict__ Q, const float* __restrict__ dist,
         const float* __restrict__ C, const float* __restrict__ F, float* __restrict__ y) {
    extern __shared__ float sm[];
    const int cin = L.cin, cout = L.cout, din = L.din, dout = L.dout, wd = L.wdim, K = D.K;
    float* sx = sm;                 // cin*din
    float* sP = sx + cin * din;     // din*din
    float* sQ = sP + din * din;     // dout*dout
    float* sf = sQ + dout * dout;   // cin*din
    float* sF = sf + cin * din;     // K*wd
    float* sZ = sF + K * wd;        // cin*dout
    float* sy = sZ + cin * dout;    // cout*dout
    float* sC = sy + cout * dout;   // K*cout*cin (SC)
    const int64_t e = blockIdx.x;
    const int tid = threadIdx.x;
    if constexpr (SC)
        for (int q = tid; q < K * cout * cin; q += kThreads) sC[q] = C[q];
    for (int q = tid; q < cin * din; q += kThreads) sx[q] = x[e * cin * din + q];
    for (int q = tid; q < din * din; q += kThreads) sP[q] = P[e * din * din + q];
    for (int q = tid; q < dout * dout; q += kThreads) sQ[q] = Q[e * dout * dout + q];
    const float r = dist[e];
    const EdgeBin eb = edge_bin(r, B);
    const float sw = r / (r + B.sh_scale);
    {
        const float* flo = F + static_cast<int64_t>(eb.lo) * K * wd;
        const float* fhi = flo + K * wd;
        for (int q = tid; q < K * wd; q += kThreads) sF[q] = lerp_bins(flo[q], fhi[q], eb.t);
    }
    for (int q = tid; q < cout * dout; q += kThreads) sy[q] = 0.0f;
    __syncthreads();
    for (int q = tid; q < cin * din; q += kThreads) {
        const int ci = q / din, j = q % din;
        float acc = 0.0f;
        for (int d = 0; d < din; ++d) acc += sx[ci * din + d] * sP[d * din + j];
        sf[q] = acc * ipowf(sw, L.lslot_in[j]);
    }
    __syncthreads();
    for (int k = 0; k < K; ++k) {
        for (int q = tid; q < cin * dout; q += kThreads)
            sZ[q] = z_entry(L, sF + k * wd, sf, q / dout, q % dout);
        __syncthreads();
        const float* Ck = (SC ? sC : C) + static_cast<int64_t>(k) * cout * cin;
        for (int q = tid; q < cout * dout; q += kThreads) {
            const int co = q / dout, slot = q % dout;
            float acc = 0.0f;
            for (int ci = 0; ci < cin; ++ci) acc += Ck[co * cin + ci] * sZ[ci * dout + slot];
            sy[q] += acc;
        }
        __syncthreads();
    }
    for (int q = tid; q < cout * dout; q += kThreads) sy[q] *= ipowf(sw, L.lslot_out[q % dout]);
    __syncthreads();
    for (int q = tid; q < cout * dout; q += kThreads) {
        const int co = q / dout, d = q % dout;
        float acc = 0.0f;
        for (int j = 0; j < dout; ++j) acc += sy[co * dout + j] * sQ[d * dout + j];
        y[e * cout * dout + q] = acc;
    }
}

// ---------------------------------------------------------------------------
// Each workgroup walks a contiguous edge range; dC is accumulated per
// workgroup in LDS and written as a partial, and the per-edge radial-function
// gradient dF_e is written per edge; the shared tail bins dF_e and sums the
// partials in a fixed order (deterministic, no atomics).
template <int kThreads, bool SC>
__global__ void __launch_bounds__(kThreads)
k_ew_bwd(feq_layout L, feq_binning B, EwDims D, int64_t E, const float* __restrict__ gy,
         const float* __restrict__ x, const float* __restrict__ P, const float* __restrict__ Q,
         const float* __restrict__ dist, const float* __restrict__ C,
         const float* __restrict__ F, float* __restrict__ gx, float* __restrict__ dFe,
         float* __restrict__ gdist, float* __restrict__ gP, float* __restrict__ gQ,
         float* __restrict__ dC_part) {
    extern __shared__ float sm[];
    __shared__ float red[kThreads / 64];
    const int cin = L.cin, cout = L.cout, din = L.din, dout = L.dout, wd = L.wdim, K = D.K;
    float* sx = sm;                 // cin*din
    float* sP = sx + cin * din;     // din*din
    float* sQ = sP + din * din;     // dout*dout
    float* sg = sQ + dout * dout;   // cout*dout : gy, then gd
    float* sgd = sg + cout * dout;  // cout*dout
    float* sf = sgd + cout * dout;  // cin*din
    float* sdf = sf + cin * din;    // cin*din
    float* sF = sdf + cin * din;    // K*wd
    float* sZ = sF + K * wd;        // cin*dout
    float* sH = sZ + cin * dout;    // cin*dout
    float* sy = sH + cin * dout;    // cout*dout (only with gQ)
    float* sdC = sy + cout * dout;  // K*cout*cin
    float* sC = sdC + K * cout * cin;   // K*cout*cin (SC)
    const int tid = threadIdx.x;
    if constexpr (SC)
        for (int q = tid; q < K * cout * cin; q += kThreads) sC[q] = C[q];   // read after the first barrier
    const int64_t per = (E + gridDim.x - 1) / gridDim.x;
    const int64_t e0 = blockIdx.x * per;
    const int64_t e1 = e0 + per < E ? e0 + per : E;
    const int ncc = K * cout * cin;
    for (int q = tid; q < ncc; q += kThreads) sdC[q] = 0.0f;
    for (int64_t e = e0; e < e1; ++e) {
        __syncthreads();
        for (int q = tid; q < cin * din; q += kThreads) sx[q] = x[e * cin * din + q];
        for (int q = tid; q < din * din; q += kThreads) sP[q] = P[e * din * din + q];
        for (int q = tid; q < dout * dout; q += kThreads) sQ[q] = Q[e * dout * dout + q];
        for (int q = tid; q < cout * dout; q += kThreads) sg[q] = gy[e * cout * dout + q];
        const float r = dist[e];
        const EdgeBin eb = edge_bin(r, B);
        const float sigma = B.sh_scale;
        const float sw = r / (r + sigma);
        const float* flo = F + static_cast<int64_t>(eb.lo) * K * wd;
        const float* fhi = flo + K * wd;
        for (int q = tid; q < K * wd; q += kThreads) sF[q] = lerp_bins(flo[q], fhi[q], eb.t);
        for (int q = tid; q < cin * din; q += kThreads) sdf[q] = 0.0f;
        if (gQ)
            for (int q = tid; q < cout * dout; q += kThreads) sy[q] = 0.0f;
        __syncthreads();
        for (int q = tid; q < cin * din; q += kThreads) {
            const int ci = q / din, j = q % din;
            float acc = 0.0f;
            for (int d = 0; d < din; ++d) acc += sx[ci * din + d] * sP[d * din + j];
            sf[q] = acc * ipowf(sw, L.lslot_in[j]);
        }
        for (int q = tid; q < cout * dout; q += kThreads) {
            const int co = q / dout, j = q % dout;
            float acc = 0.0f;
            for (int d = 0; d < dout; ++d) acc += sg[co * dout + d] * sQ[d * dout + j];
            sgd[q] = acc * ipowf(sw, L.lslot_out[j]);
        }
        __syncthreads();
        float acc_t = 0.0f, acc_s = 0.0f;
        for (int k = 0; k < K; ++k) {
            const float* Ck = (SC ? sC : C) + static_cast<int64_t>(k) * cout * cin;
            for (int q = tid; q < cin * dout; q += kThreads) {
                const int ci = q / dout, slot = q % dout;
                float acc = 0.0f;
                for (int co = 0; co < cout; ++co) acc += Ck[co * cin + ci] * sgd[co * dout + slot];
                sH[q] = acc;
                sZ[q] = z_entry(L, sF + k * wd, sf, ci, slot);
            }
            __syncthreads();
            // dC[k] += gd Z^T
            for (int q = tid; q < cout * cin; q += kThreads) {
                const int co = q / cin, ci = q % cin;
                float acc = 0.0f;
                for (int s = 0; s < dout; ++s) acc += sgd[co * dout + s] * sZ[ci * dout + s];
                sdC[k * cout * cin + q] += acc;
            }
            // dfs += F_e^T H
            for (int q = tid; q < cin * din; q += kThreads)
                sdf[q] += dz_entry(L, sF + k * wd, sH, q / din, q % din);
            // recomputed forward output (only for grad_Q)
            if (gQ)
                for (int q = tid; q < cout * dout; q += kThreads) {
                    const int co = q / dout, slot = q % dout;
                    float acc = 0.0f;
                    for (int ci = 0; ci < cin; ++ci) acc += Ck[co * cin + ci] * sZ[ci * dout + slot];
                    sy[q] += acc;
                }
            // dF_e[k, w] and the distance-gradient partial sums
            for (int w = tid; w < wd; w += kThreads) {
                Blk b;
                int o, i, comp;
                const int Lsum = weight_info(L, w, b, o, i, comp);
                float g = 0.0f;
                for (int ci = 0; ci < cin; ++ci) {
                    const float* f = sf + ci * din + b.in_off;
                    const float* h = sH + ci * dout + b.out_off;
                    if (b.m == 0) {
                        g += f[i] * h[o];
                    } else {
                        const float fr = f[2 * i], fi = f[2 * i + 1];
                        const float hr = h[2 * o], hi = h[2 * o + 1];
                        g += comp == 0 ? (fr * hr + fi * hi) : (fi * hr - fr * hi);
                    }
                }
                const int64_t fo = static_cast<int64_t>(k) * wd + w;
                dFe[e * K * wd + fo] = g;    // binned afterwards in a fixed order (ew_tail)
                acc_t += (fhi[fo] - flo[fo]) * g;
                acc_s += static_cast<float>(Lsum) * sF[fo] * g;
            }
            __syncthreads();
        }
        if (gdist) {
            const float st = block_sum<kThreads>(acc_t, red);
            const float ss = block_sum<kThreads>(acc_s, red);
            if (tid == 0) {
                float v = st * eb.dtdr;
                if (L.has_lpos) v += ss * (sigma / (r * (r + sigma)));
                gdist[e] = v;
            }
        }
        // dx = s^l dfs P^T ; dP = x^T (s^l dfs)
        for (int q = tid; q < cin * din; q += kThreads) sdf[q] *= ipowf(sw, L.lslot_in[q % din]);
        if (gQ)
            for (int q = tid; q < cout * dout; q += kThreads) sy[q] *= ipowf(sw, L.lslot_out[q % dout]);
        __syncthreads();
        if (gx)
            for (int q = tid; q < cin * din; q += kThreads) {
                const int ci = q / din, d = q % din;
                float acc = 0.0f;
                for (int j = 0; j < din; ++j) acc += sdf[ci * din + j] * sP[d * din + j];
                gx[e * cin * din + q] = acc;
            }
        if (gP)
            for (int q = tid; q < din * din; q += kThreads) {
                const int d = q / din, j = q % din;
                float acc = 0.0f;
                for (int ci = 0; ci < cin; ++ci) acc += sx[ci * din + d] * sdf[ci * din + j];
                gP[e * din * din + q] = acc;
            }
        if (gQ)
            for (int q = tid; q < dout * dout; q += kThreads) {
                const int d = q / dout, j = q % dout;
                float acc = 0.0f;
                for (int co = 0; co < cout; ++co) acc += sg[co * dout + d] * sy[co * dout + j];
                gQ[e * dout * dout + q] = acc;
            }
    }
    __syncthreads();
    for (int q = tid; q < ncc; q += kThreads) dC_part[static_cast<int64_t>(blockIdx.x) * ncc + q] = sdC[q];
}

size_t fwd_lds(const feq_layout& L, int K) {
    return sizeof(float) * (2 * L.cin * L.din + L.din * L.din + L.dout * L.dout + K * L.wdim +
                            L.cin * L.dout + L.cout * L.dout);
}

size_t bwd_lds(const feq_layout& L, int K) {
    return sizeof(float) * (2 * L.cin * L.din + L.din * L.din + L.dout * L.dout +
                            3 * L.cout * L.dout + L.cin * L.din + K * L.wdim +
                            2 * L.cin * L.dout + static_cast<size_t>(K) * L.cout * L.cin);
}

// Bytes of the staged channel patterns (the SC kernels), 0 where they would not
// fit beside the kernel's other LDS.
size_t c_lds(const feq_layout& L, int K, size_t base) {
    const size_t c = sizeof(float) * static_cast<size_t>(K) * L.cout * L.cin;
    return base + c <= 160 * 1024 ? c : 0;
}

int ensure_lds(const void* fn, size_t bytes) {
    if (bytes > 160 * 1024) return fail(FEQ_ERR_UNSUPPORTED, "needs %zu bytes of LDS", bytes);
    if (bytes > 64 * 1024)
        FEQ_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                    static_cast<int>(bytes)));
    return FEQ_OK;
}

int groups_for(int64_t E) { return static_cast<int>(E < kBwdGroups ? (E > 0 ? E : 1) : kBwdGroups); }

// Threads per workgroup for a kernel needing `lds` bytes: the smallest of 256,
// 512 and 1024 with which the workgroups that fit a CU's 160 KB of LDS give it
// at least 16 waves (more threads per edge when LDS keeps occupancy low).
int pick_threads(size_t lds) {
    const int groups = static_cast<int>((160 * 1024) / (lds > 0 ? lds : 1));
    for (int nt = 256; nt < kMaxThreads; nt *= 2)
        if (groups * (nt / 64) >= 16) return nt;
    return kMaxThreads;
}


}  // namespace
}  // namespace feq

using namespace feq;

extern "C" size_t feq_edgewise_workspace(const feq_layout* L, const feq_binning* b, int32_t rank,
                                         int64_t E) {
    if (!L || rank < 1) return 0;
    const int64_t ncc = static_cast<int64_t>(rank) * L->cout * L->cin, kw = static_cast<int64_t>(rank) * L->wdim;
    // dC partials, the per-edge radial-function gradient dF_e and the tail's buffers
    const size_t generic = b ? sizeof(float) * (static_cast<size_t>(groups_for(E)) * ncc + 64 +
                                                static_cast<size_t>(E) * kw + 64 +
                                                ew_tail_floats(*b, static_cast<int>(kw), E, groups_for(E), ncc)) + 256
                             : 0;
    const size_t split = b ? ew_split_bwd_workspace(*L, *b, rank, E, false) : 0;
    return generic > split ? generic : split;
}

extern "C" size_t feq_edgewise_fwd_workspace(const feq_layout* L, const feq_binning*, int32_t rank,
                                             int64_t) {
    if (!L || rank < 1) return 0;
    return ew_split_workspace(*L, rank) + 256;
}

extern "C" int feq_edgewise_fwd(const feq_layout* L, const feq_binning* b, int32_t rank,
                                int64_t E, const float* x, const float* P, const float* Q,
                                const float* dist, const float* C, const float* F, float* y,
                                void* ws, size_t ws_bytes, feq_stream_t stream) {
    if (int rc = check_layout(L)) return rc;
    if (int rc = check_binning(b)) return rc;
    if (rank < 1) return fail(FEQ_ERR_INVALID, "rank must be positive");
    if (E < 0) return fail(FEQ_ERR_INVALID, "negative edge count");
    if (E == 0) return FEQ_OK;
    if (E > 0x7fffffffLL) return fail(FEQ_ERR_UNSUPPORTED, "more than 2^31-1 edges");
    if (!x || !P || !Q || !dist || !C || !F || !y) return fail(FEQ_ERR_INVALID, "NULL pointer");
    const int path = ew_path();
    if (path == kPathSplit) {
        const int rc = ew_split_fwd(*L, *b, rank, E, x, nullptr, 0, P, Q, dist, C, F, y, ws,
                                    ws_bytes, false, stream_of(stream));
        if (rc != -1) return rc;
    }
    const size_t clds = c_lds(*L, rank, fwd_lds(*L, rank)), lds = fwd_lds(*L, rank) + clds;
    const int nt = pick_threads(lds);
    auto kern = clds ? (nt == 256 ? k_ew_fwd<256, true> : nt == 512 ? k_ew_fwd<512, true> : k_ew_fwd<1024, true>)
                     : (nt == 256 ? k_ew_fwd<256, false> : nt == 512 ? k_ew_fwd<512, false> : k_ew_fwd<1024, false>);
    if (int rc = ensure_lds(reinterpret_cast<const void*>(kern), lds)) return rc;
    EwDims D{rank, b->num_bins};
    FEQ_LAUNCH("k_ew_fwd", kern, dim3(E), dim3(nt), lds, stream_of(stream), *L, *b, D, x, P, Q, dist, C,
               F, y);
    return FEQ_OK;
}

extern "C" int feq_edgewise_bwd(const feq_layout* L, const feq_binning* b, int32_t rank,
                                int64_t E, const float* gy, const float* x, const float* P,
                                const float* Q, const float* dist, const float* C, const float* F,
                                float* gx, float* gC, float* gF, float* gdist, float* gP,
                                float* gQ, void* ws, size_t ws_bytes, feq_stream_t stream) {
    if (int rc = check_layout(L)) return rc;
    if (int rc = check_binning(b)) return rc;
    if (rank < 1) return fail(FEQ_ERR_INVALID, "rank must be positive");
    if (E < 0) return fail(FEQ_ERR_INVALID, "negative edge count");
    if (E > 0x7fffffffLL) return fail(FEQ_ERR_UNSUPPORTED, "more than 2^31-1 edges");
    if (!gC || !gF) return fail(FEQ_ERR_INVALID, "grad_C and grad_F are required");
    hipStream_t s = stream_of(stream);
    const int64_t ncc = static_cast<int64_t>(rank) * L->cout * L->cin;
    const int64_t nF = static_cast<int64_t>(b->num_bins + 1) * rank * L->wdim;
    if (E == 0) {
        if (int rc = fill_zero(gF, nF, s)) return rc;
        return fill_zero(gC, ncc, s);
    }
    if (!gy || !x || !P || !Q || !dist || !C || !F) return fail(FEQ_ERR_INVALID, "NULL pointer");
    if (!ws || ws_bytes < feq_edgewise_workspace(L, b, rank, E))
        return fail(FEQ_ERR_WORKSPACE, "edgewise workspace too small");
    const int path = ew_path();
    if (path == kPathSplit && !gP && !gQ) {
        const int rc = ew_split_bwd(*L, *b, rank, E, gy, x, nullptr, 0, P, Q, dist, C, F, gx, gC, gF,
                                    gdist, nullptr, ws, ws_bytes, false, s);
        if (rc != -1) return rc;
    }
    // generic kernel: per-workgroup dC partials and the per-edge dF_e, then the
    // fixed-order binning and partial sums of the shared tail (no atomics)
    const int kw = rank * L->wdim;
    if (!ew_tail_supported(*b, kw))
        return fail(FEQ_ERR_UNSUPPORTED, "empty radial-function rows");
    const size_t clds = c_lds(*L, rank, bwd_lds(*L, rank)), lds = bwd_lds(*L, rank) + clds;
    const int nt = pick_threads(lds);
    auto kern = clds ? (nt == 256 ? k_ew_bwd<256, true> : nt == 512 ? k_ew_bwd<512, true> : k_ew_bwd<1024, true>)
                     : (nt == 256 ? k_ew_bwd<256, false> : nt == 512 ? k_ew_bwd<512, false> : k_ew_bwd<1024, false>);
    if (int rc = ensure_lds(reinterpret_cast<const void*>(kern), lds)) return rc;
    const int G = groups_for(E);
    float* part = static_cast<float*>(ws);
    float* dFe = part + align_up(static_cast<size_t>(G) * ncc, 64);
    float* tail = dFe + align_up(static_cast<size_t>(E) * kw, 64);
    EwDims D{rank, b->num_bins};
    FEQ_LAUNCH("k_ew_bwd", kern, dim3(G), dim3(nt), lds, s, *L, *b, D, E, gy, x, P, Q, dist,
                       C, F, gx, dFe, gdist, gP, gQ, part);
    return ew_tail(*L, *b, rank, E, dist, F, dFe, part, G, ncc, gC, gF, nullptr, tail, s);
}

extern "C" int feq_edgewise_fused_supported(const feq_layout* L, const feq_binning* b, int32_t rank) {
    if (!L || !b || rank < 1 || check_layout(L) || check_binning(b)) return 0;
    if (ew_path() == kPathSplit && ew_split_supported(*L, *b, rank, false)) return 1;
    return fwd_lds(*L, rank) <= 160 * 1024 && bwd_lds(*L, rank) <= 160 * 1024 &&
           ew_tail_supported(*b, rank * L->wdim);
}

// ---- message-passing form: x is a node table, edge e reads row src[e] -----------
extern "C" int feq_edgewise_src_supported(const feq_layout* L, const feq_binning* b, int32_t rank) {
    if (!L || !b || check_layout(L) || check_binning(b)) return 0;
    if (ew_path() != kPathSplit) return 0;
    return ew_split_supported(*L, *b, rank, false) && ew_split_supported(*L, *b, rank, true);
}

// ---- allocation-free message-passing forward ---------------------------------------
// The forward's only scratch is the fp16-split copy of the channel patterns
// (written by k_ews_prep on every call).  This variant keeps it in a
// file-scope device array, so it needs no caller workspace and allocates
// nothing; every device holds its own copy of the array, at its own address.
static __device__ __align__(256) unsigned char scratch[FEQ_NOALLOC_SCRATCH_BYTES];

namespace {
std::mutex g_scratch_mu;
void* g_scratch_ptr[FEQ_MAX_DEVICES] = {};

// Device address of `scratch` on the device of stream s (the current device
// for the null stream), looked up once per device with that device current
// (the array's host-side name is not a device address; each device holds its
// own copy at its own address).
int scratch_ptr(hipStream_t s, void** out) {
    int dev = -1;
    if (s) {
        hipDevice_t d = -1;
        const hipError_t err = hipStreamGetDevice(s, &d);
        if (err != hipSuccess) return fail(FEQ_ERR_HIP, "hipStreamGetDevice: %s", hipGetErrorString(err));
        dev = static_cast<int>(d);
    } else if (hipGetDevice(&dev) != hipSuccess) {
        return fail(FEQ_ERR_HIP, "no current HIP device");
    }
    if (dev < 0 || dev >= FEQ_MAX_DEVICES)
        return fail(FEQ_ERR_HIP, "device id %d beyond %d", dev, FEQ_MAX_DEVICES);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        int cur = -1;
        if (hipGetDevice(&cur) != hipSuccess) return fail(FEQ_ERR_HIP, "no current HIP device");
        if (cur != dev && hipSetDevice(dev) != hipSuccess) return fail(FEQ_ERR_HIP, "hipSetDevice(%d)", dev);
        void* p = nullptr;
        const hipError_t err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (cur != dev) (void)hipSetDevice(cur);
        if (err != hipSuccess || !p)
            return fail(FEQ_ERR_HIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(err));
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return FEQ_OK;
}
}  // namespace

extern "C" int feq_edgewise_fwd_src_noalloc(const feq_layout* L, const feq_binning* b,
                                            int32_t rank, int64_t E, const float* x,
                                            int64_t num_src, const int64_t* src, const float* P,
                                            const float* Q, const float* dist, const float* C,
                                            const float* F, float* y, feq_stream_t stream) {
    if (int rc = check_layout(L)) return rc;
    if (int rc = check_binning(b)) return rc;
    if (rank < 1) return fail(FEQ_ERR_INVALID, "rank must be positive");
    const size_t need = feq_edgewise_fwd_workspace(L, b, rank, E);
    if (need > FEQ_NOALLOC_SCRATCH_BYTES)
        return fail(FEQ_ERR_UNSUPPORTED, "layout needs %zu bytes of scratch, the static array holds %d",
                    need, FEQ_NOALLOC_SCRATCH_BYTES);
    void* ws = nullptr;
    if (int rc = scratch_ptr(stream_of(stream), &ws)) return rc;
    return feq_edgewise_fwd_src(L, b, rank, E, x, num_src, src, P, Q, dist, C, F, y, ws,
                                FEQ_NOALLOC_SCRATCH_BYTES, stream);
}

extern "C" int feq_edgewise_fwd_src(const feq_layout* L, const feq_binning* b, int32_t rank,
                                    int64_t E, const float* x, int64_t num_src, const int64_t* src,
                                    const float* P, const float* Q, const float* dist,
                                    const float* C, const float* F, float* y, void* ws,
                                    size_t ws_bytes, feq_stream_t stream) {
    return feq_edgewise_fwd_src_ex(L, b, rank, E, x, num_src, src, P, Q, dist, C, F, y, 0, ws,
                                   ws_bytes, stream);
}

extern "C" int feq_edgewise_fwd_src_ex(const feq_layout* L, const feq_binning* b, int32_t rank,
                                       int64_t E, const float* x, int64_t num_src, const int64_t* src,
                                       const float* P, const float* Q, const float* dist,
                                       const float* C, const float* F, float* y, int32_t flags,
                                       void* ws, size_t ws_bytes, feq_stream_t stream) {
    if (int rc = check_layout(L)) return rc;
    if (flags & ~FEQ_EW_HALF_ACCURACY) return fail(FEQ_ERR_INVALID, "unknown flags 0x%x", flags);
    if (int rc = check_binning(b)) return rc;
    if (rank < 1) return fail(FEQ_ERR_INVALID, "rank must be positive");
    if (E < 0 || num_src < 0) return fail(FEQ_ERR_INVALID, "negative edge or node count");
    if (E == 0) return FEQ_OK;
    if (E > 0x7fffffffLL) return fail(FEQ_ERR_UNSUPPORTED, "more than 2^31-1 edges");
    if (!x || !src || !P || !Q || !dist || !C || !F || !y) return fail(FEQ_ERR_INVALID, "NULL pointer");
    if (!feq_edgewise_src_supported(L, b, rank))
        return fail(FEQ_ERR_UNSUPPORTED, "no message-passing kernels for this layout");
    const int rc = ew_split_fwd(*L, *b, rank, E, x, src, num_src, P, Q, dist, C, F, y, ws, ws_bytes,
                                (flags & FEQ_EW_HALF_ACCURACY) != 0, stream_of(stream));
    return rc == -1 ? fail(FEQ_ERR_UNSUPPORTED, "tensors must be 16-byte aligned") : rc;
}

extern "C" int feq_edgewise_bwd_src(const feq_layout* L, const feq_binning* b, int32_t rank,
                                    int64_t E, const float* gy, const float* x, int64_t num_src,
                                    const int64_t* src, const float* P, const float* Q,
                                    const float* dist, const float* C, const float* F,
                                    float* gx_edges, float* gC, float* gF, float* gdist, void* ws,
                                    size_t ws_bytes, feq_stream_t stream) {
    if (int rc = check_layout(L)) return rc;
    if (int rc = check_binning(b)) return rc;
    if (rank < 1) return fail(FEQ_ERR_INVALID, "rank must be positive");
    if (E < 0 || num_src < 0) return fail(FEQ_ERR_INVALID, "negative edge or node count");
    if (E > 0x7fffffffLL) return fail(FEQ_ERR_UNSUPPORTED, "more than 2^31-1 edges");
    if (!gC || !gF || !gx_edges) return fail(FEQ_ERR_INVALID, "grad_x_edges, grad_C and grad_F are required");
    hipStream_t s = stream_of(stream);
    if (E == 0) {
        if (int rc = fill_zero(gF, static_cast<int64_t>(b->num_bins + 1) * rank * L->wdim, s)) return rc;
        return fill_zero(gC, static_cast<int64_t>(rank) * L->cout * L->cin, s);
    }
    if (!gy || !x || !src || !P || !Q || !dist || !C || !F) return fail(FEQ_ERR_INVALID, "NULL pointer");
    if (!feq_edgewise_src_supported(L, b, rank))
        return fail(FEQ_ERR_UNSUPPORTED, "no message-passing kernels for this layout");
    if (!ws || ws_bytes < feq_edgewise_workspace(L, b, rank, E))
        return fail(FEQ_ERR_WORKSPACE, "edgewise workspace too small");
    const int rc = ew_split_bwd(*L, *b, rank, E, gy, x, src, num_src, P, Q, dist, C, F, gx_edges, gC,
                                gF, gdist, nullptr, ws, ws_bytes, false, s);
    return rc == -1 ? fail(FEQ_ERR_UNSUPPORTED, "tensors must be 16-byte aligned") : rc;
}

extern "C" size_t feq_edgewise_bwd_src_nodes_workspace(const feq_layout* L, const feq_binning* b,
                                                       int32_t rank, int64_t E) {
    if (!L || !b || rank < 1 || E < 0) return 0;
    return ew_split_bwd_workspace(*L, *b, rank, E, true) + 256;
}

extern "C" int feq_edgewise_bwd_src_nodes(const feq_layout* L, const feq_binning* b, int32_t rank,
                                          int64_t E, const float* gy, const float* x, int64_t num_src,
                                          const int64_t* src, const int32_t* perm_src,
                                          const int32_t* offsets_src, const float* P, const float* Q,
                                          const float* dist, const float* C, const float* F,
                                          float* gx_nodes, float* gC, float* gF, float* gdist,
                                          void* ws, size_t ws_bytes, feq_stream_t stream) {
    return feq_edgewise_bwd_src_nodes_ex(L, b, rank, E, gy, x, num_src, src, perm_src, offsets_src, P,
                                         Q, dist, C, F, gx_nodes, gC, gF, gdist, 0, ws, ws_bytes,
                                         stream);
}

extern "C" int feq_edgewise_bwd_src_nodes_ex(const feq_layout* L, const feq_binning* b, int32_t rank,
                                             int64_t E, const float* gy, const float* x,
                                             int64_t num_src, const int64_t* src,
                                             const int32_t* perm_src, const int32_t* offsets_src,
                                             const float* P, const float* Q, const float* dist,
                                             const float* C, const float* F, float* gx_nodes,
                                             float* gC, float* gF, float* gdist, int32_t flags,
                                             void* ws, size_t ws_bytes, feq_stream_t stream) {
    if (int rc = check_layout(L)) return rc;
    if (flags & ~FEQ_EW_HALF_ACCURACY) return fail(FEQ_ERR_INVALID, "unknown flags 0x%x", flags);
    if (int rc = check_binning(b)) return rc;
    if (rank < 1) return fail(FEQ_ERR_INVALID, "rank must be positive");
    if (E < 0 || num_src < 0) return fail(FEQ_ERR_INVALID, "negative edge or node count");
    if (E > 0x7fffffffLL || num_src > 0x7fffffffLL)
        return fail(FEQ_ERR_UNSUPPORTED, "more than 2^31-1 edges or nodes");
    if (!gC || !gF || (num_src > 0 && !gx_nodes))
        return fail(FEQ_ERR_INVALID, "grad_x_nodes, grad_C and grad_F are required");
    hipStream_t s = stream_of(stream);
    if (E == 0) {
        if (int rc = fill_zero(gF, static_cast<int64_t>(b->num_bins + 1) * rank * L->wdim, s)) return rc;
        if (int rc = fill_zero(gx_nodes, num_src * L->cin * L->din, s)) return rc;
        return fill_zero(gC, static_cast<int64_t>(rank) * L->cout * L->cin, s);
    }
    if (!gy || !x || !src || !perm_src || !offsets_src || !P || !Q || !dist || !C || !F)
        return fail(FEQ_ERR_INVALID, "NULL pointer");
    if (!feq_edgewise_src_supported(L, b, rank))
        return fail(FEQ_ERR_UNSUPPORTED, "no message-passing kernels for this layout");
    if (!ws || ws_bytes < feq_edgewise_bwd_src_nodes_workspace(L, b, rank, E))
        return fail(FEQ_ERR_WORKSPACE, "edgewise workspace too small");
    const NodeScatter ns{perm_src, offsets_src, gx_nodes, nullptr};
    const int rc = ew_split_bwd(*L, *b, rank, E, gy, x, src, num_src, P, Q, dist, C, F, nullptr, gC,
                                gF, gdist, &ns, ws, ws_bytes, (flags & FEQ_EW_HALF_ACCURACY) != 0, s);
    return rc == -1 ? fail(FEQ_ERR_UNSUPPORTED, "tensors must be 16-byte aligned") : rc;
}

// ---- gradients for the bases on the split kernels --------------------------------------
extern "C" int feq_edgewise_pq_supported(const feq_layout* L, const feq_binning* b, int32_t rank) {
    if (!L || !b || check_layout(L) || check_binning(b)) return 0;
    if (ew_path() != kPathSplit) return 0;
    return ew_split_pq_supported(*L, *b, rank);
}

extern "C" int feq_edgewise_fwd_ym(const feq_layout* L, const feq_binning* b, int32_t rank, int64_t E,
                                   const float* x, int64_t num_src, const int64_t* src, const float* P,
                                   const float* Q, const float* dist, const float* C, const float* F,
                                   float* y, float* ym, int32_t flags, void* ws, size_t ws_bytes,
                                   feq_stream_t stream) {
    if (int rc = check_layout(L)) return rc;
    if (flags & ~FEQ_EW_HALF_ACCURACY) return fail(FEQ_ERR_INVALID, "unknown flags 0x%x", flags);
    if (int rc = check_binning(b)) return rc;
    if (rank < 1) return fail(FEQ_ERR_INVALID, "rank must be positive");
    if (E < 0 || num_src < 0) return fail(FEQ_ERR_INVALID, "negative edge or node count");
    if (E == 0) return FEQ_OK;
    if (E > 0x7fffffffLL) return fail(FEQ_ERR_UNSUPPORTED, "more than 2^31-1 edges");
    if (!x || !P || !Q || !dist || !C || !F || !y || !ym) return fail(FEQ_ERR_INVALID, "NULL pointer");
    if (!feq_edgewise_pq_supported(L, b, rank))
        return fail(FEQ_ERR_UNSUPPORTED, "no kernels forming the bases' gradients for this layout");
    const BasisGrads bg{ym, nullptr, nullptr, nullptr};
    const int rc = ew_split_fwd(*L, *b, rank, E, x, src, src ? num_src : 0, P, Q, dist, C, F, y, ws,
                                ws_bytes, src && (flags & FEQ_EW_HALF_ACCURACY) != 0, stream_of(stream),
                                nullptr, &bg);
    return rc == -1 ? fail(FEQ_ERR_UNSUPPORTED, "tensors must be 16-byte aligned") : rc;
}

extern "C" int feq_edgewise_bwd_pq(const feq_layout* L, const feq_binning* b, int32_t rank, int64_t E,
                                   const float* gy, const float* x, int64_t num_src, const int64_t* src,
                                   const int32_t* perm_src, const int32_t* offsets_src, const float* P,
                                   const float* Q, const float* dist, const float* C, const float* F,
                                   const float* ym, float* gx, float* gC, float* gF, float* gdist,
                                   float* gP, float* gQ, int32_t flags, void* ws, size_t ws_bytes,
                                   feq_stream_t stream) {
    if (int rc = check_layout(L)) return rc;
    if (flags & ~FEQ_EW_HALF_ACCURACY) return fail(FEQ_ERR_INVALID, "unknown flags 0x%x", flags);
    if (int rc = check_binning(b)) return rc;
    if (rank < 1) return fail(FEQ_ERR_INVALID, "rank must be positive");
    if (E < 0 || num_src < 0) return fail(FEQ_ERR_INVALID, "negative edge or node count");
    if (E > 0x7fffffffLL || num_src > 0x7fffffffLL)
        return fail(FEQ_ERR_UNSUPPORTED, "more than 2^31-1 edges or nodes");
    const bool nodes = src != nullptr;
    if (!gC || !gF || !gx) return fail(FEQ_ERR_INVALID, "grad_x, grad_C and grad_F are required");
    hipStream_t s = stream_of(stream);
    if (E == 0) {
        if (int rc = fill_zero(gF, static_cast<int64_t>(b->num_bins + 1) * rank * L->wdim, s)) return rc;
        if (nodes)
            if (int rc = fill_zero(gx, num_src * L->cin * L->din, s)) return rc;
        return fill_zero(gC, static_cast<int64_t>(rank) * L->cout * L->cin, s);
    }
    if (!gy || !x || !P || !Q || !dist || !C || !F || (nodes && (!perm_src || !offsets_src)))
        return fail(FEQ_ERR_INVALID, "NULL pointer");
    if (gQ && !ym) return fail(FEQ_ERR_INVALID, "grad_Q needs ym, the rows before the rotation");
    if (!feq_edgewise_pq_supported(L, b, rank))
        return fail(FEQ_ERR_UNSUPPORTED, "no kernels forming the bases' gradients for this layout");
    const size_t need = nodes ? feq_edgewise_bwd_src_nodes_workspace(L, b, rank, E)
                              : feq_edgewise_workspace(L, b, rank, E);
    if (!ws || ws_bytes < need) return fail(FEQ_ERR_WORKSPACE, "edgewise workspace too small");
    const BasisGrads bg{nullptr, ym, gP, gQ};
    const NodeScatter ns{perm_src, offsets_src, gx, nullptr};
    const int rc = ew_split_bwd(*L, *b, rank, E, gy, x, src, nodes ? num_src : 0, P, Q, dist, C, F,
                                nodes ? nullptr : gx, gC, gF, gdist, nodes ? &ns : nullptr, ws, ws_bytes,
                                nodes && (flags & FEQ_EW_HALF_ACCURACY) != 0, s, nullptr, &bg);
    return rc == -1 ? fail(FEQ_ERR_UNSUPPORTED, "tensors must be 16-byte aligned") : rc;
}

// ---- message-passing form fused with the attention's head weighting and sum pooling ----
namespace {
int check_pool_args(const feq_layout* L, int32_t heads, int32_t chan_per_head) {
    if (heads < 1 || heads > kPoolMaxHeads)
        return fail(FEQ_ERR_UNSUPPORTED, "pooled form: heads must be in [1, %d], got %d", kPoolMaxHeads, heads);
    if (chan_per_head < 4 || chan_per_head % 4 || static_cast<int64_t>(chan_per_head) * heads > L->cout)
        return fail(FEQ_ERR_UNSUPPORTED,
                    "pooled form: channels per head must be a positive multiple of 4 with "
                    "heads * channels per head <= Cout, got %d x %d for Cout %d",
                    heads, chan_per_head, L->cout);
    return FEQ_OK;
}
}  // namespace

extern "C" int feq_edgewise_pool_supported(const feq_layout* L, const feq_binning* b, int32_t rank) {
    if (!L || !b || check_layout(L) || check_binning(b)) return 0;
    if (ew_path() != kPathSplit) return 0;
    return ew_pool_supported(*L, *b, rank);
}

extern "C" size_t feq_edgewise_fwd_src_pool_workspace(const feq_layout* L, const feq_binning*,
                                                      int32_t rank, int64_t E) {
    if (!L || rank < 1 || E < 0) return 0;
    return ew_pool_fwd_workspace(*L, rank, E) + 256;
}

namespace {
int fwd_src_pool(const feq_layout* L, const feq_binning* b, int32_t rank, int64_t E, const float* x,
                 int64_t num_src, const int64_t* src, const float* P, const float* Q, const float* dist,
                 const float* C, const float* F, const float* attn, int32_t heads, int32_t chan_per_head,
                 const int64_t* dst, const int32_t* perm_dst, const int32_t* offsets_dst, int64_t num_dst,
                 float* out, float* y_pos, float* ym, int32_t flags, void* ws, size_t ws_bytes,
                 feq_stream_t stream) {
    if (int rc = check_layout(L)) return rc;
    if (flags & ~FEQ_EW_HALF_ACCURACY) return fail(FEQ_ERR_INVALID, "unknown flags 0x%x", flags);
    if (int rc = check_binning(b)) return rc;
    if (rank < 1) return fail(FEQ_ERR_INVALID, "rank must be positive");
    if (E < 0 || num_src < 0 || num_dst < 0) return fail(FEQ_ERR_INVALID, "negative edge or node count");
    if (E > 0x7fffffffLL || num_dst > 0x7fffffffLL)
        return fail(FEQ_ERR_UNSUPPORTED, "more than 2^31-1 edges or nodes");
    if (int rc = check_pool_args(L, heads, chan_per_head)) return rc;
    if (!feq_edgewise_pool_supported(L, b, rank))
        return fail(FEQ_ERR_UNSUPPORTED, "no pooled message-passing kernels for this layout");
    hipStream_t s = stream_of(stream);
    if (num_dst > 0 && !out) return fail(FEQ_ERR_INVALID, "NULL out");
    if (E == 0) return fill_zero(out, num_dst * L->cout * L->dout, s);
    // no edge has a destination: nothing to sum (and the backward's grad_Q is zero
    // without reading ym)
    if (num_dst == 0) return FEQ_OK;
    if (ym && !feq_edgewise_pq_supported(L, b, rank))
        return fail(FEQ_ERR_UNSUPPORTED, "no kernels forming the bases' gradients for this layout");
    if (!x || !src || !P || !Q || !dist || !C || !F || !attn || !dst || !perm_dst || !offsets_dst)
        return fail(FEQ_ERR_INVALID, "NULL pointer");
    if (!ws || ws_bytes < feq_edgewise_fwd_src_pool_workspace(L, b, rank, E))
        return fail(FEQ_ERR_WORKSPACE, "edgewise workspace too small");
    const DstPool dp{perm_dst, offsets_dst, dst, attn, num_dst, heads, chan_per_head, out, nullptr};
    const BasisGrads bg{ym, nullptr, nullptr, nullptr};
    const int rc = ew_split_fwd(*L, *b, rank, E, x, src, num_src, P, Q, dist, C, F, y_pos, ws, ws_bytes,
                                (flags & FEQ_EW_HALF_ACCURACY) != 0, s, &dp, ym ? &bg : nullptr);
    return rc == -1 ? fail(FEQ_ERR_UNSUPPORTED, "tensors must be 16-byte aligned") : rc;
}
}  // namespace

extern "C" int feq_edgewise_fwd_src_pool(const feq_layout* L, const feq_binning* b, int32_t rank,
                                         int64_t E, const float* x, int64_t num_src,
                                         const int64_t* src, const float* P, const float* Q,
                                         const float* dist, const float* C, const float* F,
                                         const float* attn, int32_t heads, int32_t chan_per_head,
                                         const int64_t* dst, const int32_t* perm_dst,
                                         const int32_t* offsets_dst, int64_t num_dst, float* out,
                                         float* y_pos, int32_t flags, void* ws, size_t ws_bytes,
                                         feq_stream_t stream) {
    return fwd_src_pool(L, b, rank, E, x, num_src, src, P, Q, dist, C, F, attn, heads, chan_per_head, dst,
                        perm_dst, offsets_dst, num_dst, out, y_pos, nullptr, flags, ws, ws_bytes, stream);
}

extern "C" int feq_edgewise_fwd_src_pool_ym(const feq_layout* L, const feq_binning* b, int32_t rank,
                                            int64_t E, const float* x, int64_t num_src,
                                            const int64_t* src, const float* P, const float* Q,
                                            const float* dist, const float* C, const float* F,
                                            const float* attn, int32_t heads, int32_t chan_per_head,
                                            const int64_t* dst, const int32_t* perm_dst,
                                            const int32_t* offsets_dst, int64_t num_dst, float* out,
                                            float* y_pos, float* ym, int32_t flags, void* ws,
                                            size_t ws_bytes, feq_stream_t stream) {
    if (!ym) return fail(FEQ_ERR_INVALID, "NULL ym");
    return fwd_src_pool(L, b, rank, E, x, num_src, src, P, Q, dist, C, F, attn, heads, chan_per_head, dst,
                        perm_dst, offsets_dst, num_dst, out, y_pos, ym, flags, ws, ws_bytes, stream);
}

namespace {
int bwd_src_pool(const feq_layout* L, const feq_binning* b, int32_t rank, int64_t E, const float* grad_out,
                 const float* attn, int32_t heads, int32_t chan_per_head, const int64_t* dst,
                 int64_t num_dst, const float* x, int64_t num_src, const int64_t* src,
                 const int32_t* perm_src, const int32_t* offsets_src, const float* P, const float* Q,
                 const float* dist, const float* C, const float* F, const float* ym, float* gx_nodes,
                 float* gC, float* gF, float* gdist, float* gP, float* gQ, int32_t flags, void* ws,
                 size_t ws_bytes, feq_stream_t stream) {
    if (int rc = check_layout(L)) return rc;
    if (flags & ~FEQ_EW_HALF_ACCURACY) return fail(FEQ_ERR_INVALID, "unknown flags 0x%x", flags);
    if (int rc = check_binning(b)) return rc;
    if (rank < 1) return fail(FEQ_ERR_INVALID, "rank must be positive");
    if (E < 0 || num_src < 0 || num_dst < 0) return fail(FEQ_ERR_INVALID, "negative edge or node count");
    if (E > 0x7fffffffLL || num_src > 0x7fffffffLL || num_dst > 0x7fffffffLL)
        return fail(FEQ_ERR_UNSUPPORTED, "more than 2^31-1 edges or nodes");
    if (int rc = check_pool_args(L, heads, chan_per_head)) return rc;
    if (!gC || !gF || (num_src > 0 && !gx_nodes))
        return fail(FEQ_ERR_INVALID, "grad_x_nodes, grad_C and grad_F are required");
    if (!feq_edgewise_pool_supported(L, b, rank))
        return fail(FEQ_ERR_UNSUPPORTED, "no pooled message-passing kernels for this layout");
    hipStream_t s = stream_of(stream);
    if ((gP || gQ) && !feq_edgewise_pq_supported(L, b, rank))
        return fail(FEQ_ERR_UNSUPPORTED, "no kernels forming the bases' gradients for this layout");
    if (gQ && E > 0 && num_dst > 0 && !ym)
        return fail(FEQ_ERR_INVALID, "grad_Q needs ym, the rows before the rotation");
    if (E == 0 || num_dst == 0) {
        // no edge reaches the pooled output: every gradient is zero
        if (int rc = fill_zero(gF, static_cast<int64_t>(b->num_bins + 1) * rank * L->wdim, s)) return rc;
        if (int rc = fill_zero(gx_nodes, num_src * L->cin * L->din, s)) return rc;
        if (gdist)
            if (int rc = fill_zero(gdist, E, s)) return rc;
        if (gP)
            if (int rc = fill_zero(gP, E * L->din * L->din, s)) return rc;
        if (gQ)
            if (int rc = fill_zero(gQ, E * L->dout * L->dout, s)) return rc;
        return fill_zero(gC, static_cast<int64_t>(rank) * L->cout * L->cin, s);
    }
    if (!grad_out || !attn || !dst || !x || !src || !perm_src || !offsets_src || !P || !Q || !dist ||
        !C || !F)
        return fail(FEQ_ERR_INVALID, "NULL pointer");
    if (!ws || ws_bytes < feq_edgewise_bwd_src_nodes_workspace(L, b, rank, E))
        return fail(FEQ_ERR_WORKSPACE, "edgewise workspace too small");
    const NodeScatter ns{perm_src, offsets_src, gx_nodes, nullptr};
    const DstPool dp{nullptr, nullptr, dst, attn, num_dst, heads, chan_per_head, nullptr, nullptr};
    const BasisGrads bg{nullptr, ym, gP, gQ};
    const int rc = ew_split_bwd(*L, *b, rank, E, grad_out, x, src, num_src, P, Q, dist, C, F, nullptr,
                                gC, gF, gdist, &ns, ws, ws_bytes, (flags & FEQ_EW_HALF_ACCURACY) != 0, s,
                                &dp, (gP || gQ) ? &bg : nullptr);
    return rc == -1 ? fail(FEQ_ERR_UNSUPPORTED, "tensors must be 16-byte aligned") : rc;
}
}  // namespace

extern "C" int feq_edgewise_bwd_src_pool(const feq_layout* L, const feq_binning* b, int32_t rank,
                                         int64_t E, const float* grad_out, const float* attn,
                                         int32_t heads, int32_t chan_per_head, const int64_t* dst,
                                         int64_t num_dst, const float* x, int64_t num_src,
                                         const int64_t* src, const int32_t* perm_src,
                                         const int32_t* offsets_src, const float* P, const float* Q,
                                         const float* dist, const float* C, const float* F,
                                         float* gx_nodes, float* gC, float* gF, float* gdist,
                                         int32_t flags, void* ws, size_t ws_bytes,
                                         feq_stream_t stream) {
    return bwd_src_pool(L, b, rank, E, grad_out, attn, heads, chan_per_head, dst, num_dst, x, num_src, src,
                        perm_src, offsets_src, P, Q, dist, C, F, nullptr, gx_nodes, gC, gF, gdist, nullptr,
                        nullptr, flags, ws, ws_bytes, stream);
}

extern "C" int feq_edgewise_bwd_src_pool_pq(const feq_layout* L, const feq_binning* b, int32_t rank,
                                            int64_t E, const float* grad_out, const float* attn,
                                            int32_t heads, int32_t chan_per_head, const int64_t* dst,
                                            int64_t num_dst, const float* x, int64_t num_src,
                                            const int64_t* src, const int32_t* perm_src,
                                            const int32_t* offsets_src, const float* P, const float* Q,
                                            const float* dist, const float* C, const float* F,
                                            const float* ym, float* gx_nodes, float* gC, float* gF,
                                            float* gdist, float* gP, float* gQ, int32_t flags, void* ws,
                                            size_t ws_bytes, feq_stream_t stream) {
    return bwd_src_pool(L, b, rank, E, grad_out, attn, heads, chan_per_head, dst, num_dst, x, num_src, src,
                        perm_src, offsets_src, P, Q, dist, C, F, ym, gx_nodes, gC, gF, gdist, gP, gQ, flags,
                        ws, ws_bytes, stream);
}

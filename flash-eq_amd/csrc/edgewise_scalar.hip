// EquivariantEdgewiseLinear with scalar outputs (lvals_out = [0]): the last
// projection of a transformer whose output representation is [0]xC, e.g. the
// value projection of its final block.
//
// With lvals_out = [0] only the m = 0 block of the mixing matrix exists: output
// slot 0 takes the m = 0 input slots j = l (l = 0 .. Lin, the first Lin + 1
// columns of the m-first basis), weight w = l, solid-harmonic factor s^l
// (linear.py:100-160, block_diagonal.cu:1220-1258 for the m-block layout):
//   fs0[c, l] = sum_d x[c, d] P[d, l]                 (the m = 0 columns of x P)
//   z[c, k]   = sum_l F_e[k, l] s^l fs0[c, l]
//   y[co]     = Q[0, 0] sum_k sum_c C_k[co, c] z[c, k]
// A few hundred FMAs per edge against the full layer's ~30 thousand, so the
// kernels are plain VALU code with a wave per edge and a lane per input
// channel (Cin = 64): the row x[src[e]] is one coalesced read, the basis
// columns, radial functions and Q[0, 0] are wave-uniform, C_k[:, c] sits in the
// lane's registers for the whole launch, and the Cout output sums are wave
// reductions that halve the values per lane at each exchange.
//
// Backward, per edge (gq = Q[0, 0] gy):
//   gz[c, k]   = sum_co C_k[co, c] gq[co]
//   dx[c, d]   = sum_l P[d, l] s^l sum_k F_e[k, l] gz[c, k]
//   dF_e[k, l] = s^l sum_c gz[c, k] fs0[c, l]        (binned by the shared tail)
//   dC_k[co,c] += gq[co] z[c, k]                     (lane registers, per-workgroup partials)
// A wave walks 16-edge tiles; in the message-passing form the tiles follow the
// CSR by source, dx is summed per source node in tile order and nodes whose
// edges cross a tile boundary leave partial rows (NodeScatter), as in the
// split family, so the node sums are deterministic.
#include "ew_canon.h"
#include "feq_internal.h"

namespace feq {
namespace {

constexpr int kCin = 64;      // a lane per input channel
constexpr int kWaves = 4;     // waves per workgroup
constexpr int kTile = 16;     // edges per backward tile (the NodeScatter tile)

__device__ __forceinline__ int64_t ceil_div_d(int64_t a, int64_t b) { return (a + b - 1) / b; }

int sc_cus() {
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) == hipSuccess) {
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
            cus = v;
    }
    return cus;
}

// Sums over the 64 lanes of N per-lane values (N a power of two <= 64): each
// exchange halves the values a lane keeps (lanes with the exchanged lane bit
// set keep the upper half), then the single value is summed over the
// remaining lane bits.  Lane l returns value l / (64 / N).  The exchanges over
// lane bits 5 and 4 are v_permlane32_swap / v_permlane16_swap (one swap and
// one add per pair, no select); the later ones add both halves and select the
// result (a select between two loaded array elements would be turned into an
// indexed access of the whole array).
template <int N>
__device__ __forceinline__ float wave_sums(const float (&v)[N]) {
    static_assert(N >= 1 && N <= 64 && (N & (N - 1)) == 0, "power of two");
    const int lane = threadIdx.x & 63;
    float w[N];
#pragma unroll
    for (int i = 0; i < N; ++i) w[i] = v[i];
    if constexpr (N >= 2) {
#pragma unroll
        for (int i = 0; i < N / 2; ++i) {
            const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(w[i]), __float_as_uint(w[i + N / 2]),
                                                            false, false);
            w[i] = __uint_as_float(p[0]) + __uint_as_float(p[1]);
        }
    }
    if constexpr (N >= 4) {
#pragma unroll
        for (int i = 0; i < N / 4; ++i) {
            const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(w[i]), __float_as_uint(w[i + N / 4]),
                                                            false, false);
            w[i] = __uint_as_float(p[0]) + __uint_as_float(p[1]);
        }
    }
    int bit = 8;
#pragma unroll
    for (int m = N / 8; m >= 1; m >>= 1) {
        const bool upper = (lane & bit) != 0;
#pragma unroll
        for (int i = 0; i < m; ++i) {
            const float a = w[i] + __shfl_xor(w[i], bit, 64);
            const float b = w[i + m] + __shfl_xor(w[i + m], bit, 64);
            w[i] = upper ? b : a;
        }
        bit >>= 1;
    }
    float s = w[0];
    for (int off = N >= 4 ? bit : (N == 2 ? 16 : 32); off >= 1; off >>= 1) s += __shfl_xor(s, off, 64);
    return s;
}

// The radial-function table F (num_bins + 1, K, Lin + 1) in LDS: a few KB,
// read by every edge.
__device__ __forceinline__ void stage_table(float* sF, const float* __restrict__ F, int n) {
    for (int q = threadIdx.x; q < n; q += blockDim.x) sF[q] = F[q];
    __syncthreads();
}

// Per-edge constants of a group of NB edges; every load of the group is
// issued before the first use (indices clamped in range, then masked), so one
// memory latency covers the group.  The edge index is wave-uniform: the row
// index, distance, basis columns and Q[0, 0] are scalar loads.  The bin, the
// interpolation weight and s = r / (r + sigma) of edge i are computed by lane i
// and broadcast, not by every lane.
template <int LIN, int NB>
struct Group0 {
    static constexpr int DIN = (LIN + 1) * (LIN + 1), NL = LIN + 1;
    static_assert(NB <= 64, "a lane per edge of the group");
    float xr[NB][DIN];
    float pc[NB][DIN][NL];
    float r[NB], q[NB], t[NB], sh[NB];
    int lo[NB];
    int64_t row[NB];

    __device__ __forceinline__ void load(int64_t e0, int64_t E, const float* __restrict__ x,
                                         const int64_t* __restrict__ src, int64_t nsrc,
                                         const int32_t* __restrict__ perm, const float* __restrict__ P,
                                         const float* __restrict__ Q, const float* __restrict__ dist,
                                         int64_t (&e)[NB], int lane, const feq_binning& B) {
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            const int64_t p = e0 + i < E ? e0 + i : E - 1;
            e[i] = perm ? perm[p] : p;
        }
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            int64_t rw = e[i];
            if (src) {
                rw = src[e[i]];
                rw = rw >= 0 && rw < nsrc ? rw : -1;
            }
            row[i] = e0 + i < E ? rw : -1;
            r[i] = dist[e[i]];
            q[i] = Q[e[i]];
        }
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            const float* xs = x + ((row[i] >= 0 ? row[i] : 0) * kCin + lane) * DIN;
            const uint32_t mk = row[i] >= 0 ? ~0u : 0u;
#pragma unroll
            for (int d = 0; d < DIN; ++d) xr[i][d] = __uint_as_float(__float_as_uint(xs[d]) & mk);
        }
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            const float* pe = P + e[i] * DIN * DIN;
#pragma unroll
            for (int d = 0; d < DIN; ++d)
#pragma unroll
                for (int l = 0; l < NL; ++l) pc[i][d][l] = pe[d * DIN + l];
        }
        float rl = r[0];
#pragma unroll
        for (int i = 1; i < NB; ++i) rl = lane == i ? r[i] : rl;
        const EdgeBin eb = edge_bin(rl, B);
        const float sl = rl / (rl + B.sh_scale);
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            lo[i] = __builtin_amdgcn_readlane(eb.lo, i);
            t[i] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(eb.t), i));
            sh[i] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sl), i));
        }
    }

    // The group's positions j0 .. j0 + NB - 1 of a tile whose per-position
    // values sit one per lane (lane j: position j; positions past np repeat the
    // last): edge, row (-1: none), bin, weight, s, Q[0, 0] come by readlane, and
    // only the rows x[row] and P[e] are loaded here.
    __device__ __forceinline__ void load_known(int j0, int np, int el, int rl, int lol, float tl, float shl,
                                               float ql, const float* __restrict__ x,
                                               const float* __restrict__ P, int64_t (&e)[NB], int lane) {
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            const int j = j0 + i < np ? j0 + i : np - 1;
            e[i] = __builtin_amdgcn_readlane(el, j);
            const int rw = __builtin_amdgcn_readlane(rl, j);
            row[i] = j0 + i < np ? rw : -1;
            lo[i] = __builtin_amdgcn_readlane(lol, j);
            t[i] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(tl), j));
            sh[i] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(shl), j));
            q[i] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ql), j));
        }
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            const float* xs = x + ((row[i] >= 0 ? row[i] : 0) * kCin + lane) * DIN;
            const uint32_t mk = row[i] >= 0 ? ~0u : 0u;
#pragma unroll
            for (int d = 0; d < DIN; ++d) xr[i][d] = __uint_as_float(__float_as_uint(xs[d]) & mk);
        }
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            const float* pe = P + e[i] * DIN * DIN;
#pragma unroll
            for (int d = 0; d < DIN; ++d)
#pragma unroll
                for (int l = 0; l < NL; ++l) pc[i][d][l] = pe[d * DIN + l];
        }
    }

    // fs0[l] = sum_d x[d] P[d, l]; fe[k][l] = F_e[k, l] s^l from the LDS table
    template <int K>
    __device__ __forceinline__ void edge(int i, const float* sF, float (&fs0)[NL], float (&fe)[K][NL],
                                         float (&pw)[NL]) const {
#pragma unroll
        for (int l = 0; l < NL; ++l) {
            float a = 0.0f;
#pragma unroll
            for (int d = 0; d < DIN; ++d) a += xr[i][d] * pc[i][d][l];
            fs0[l] = a;
        }
        float p = 1.0f;
#pragma unroll
        for (int l = 0; l < NL; ++l) {
            pw[l] = p;
            p *= sh[i];
        }
        const float* flo = sF + lo[i] * K * NL;
#pragma unroll
        for (int k = 0; k < K; ++k)
#pragma unroll
            for (int l = 0; l < NL; ++l) fe[k][l] = lerp_bins(flo[k * NL + l], flo[K * NL + k * NL + l], t[i]) * pw[l];
    }
};

constexpr int kGroup = 4;   // edges loaded together (forward)
constexpr int kGroupB = 2;  // edges loaded together (backward: more state per edge)

// Forward: waves walk groups of kGroup consecutive edges (grid-stride).
// YM: also writes m = y / Q[0, 0] (the rows before the rotation) to ym.
template <int LIN, int COUT, int K, bool YM = false>
__global__ void __launch_bounds__(64 * kWaves)
k_ew0_fwd(feq_binning B, int64_t E, const float* __restrict__ x, const int64_t* __restrict__ src,
          int64_t nsrc, const float* __restrict__ P, const float* __restrict__ Q,
          const float* __restrict__ dist, const float* __restrict__ C, const float* __restrict__ F,
          float* __restrict__ y, float* __restrict__ ym) {
    using G = Group0<LIN, kGroup>;
    constexpr int NL = G::NL;
    extern __shared__ float sF[];
    stage_table(sF, F, (B.num_bins + 1) * K * NL);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    float cw[K][COUT];   // C_k[co, lane]
#pragma unroll
    for (int k = 0; k < K; ++k)
#pragma unroll
        for (int co = 0; co < COUT; ++co) cw[k][co] = C[(k * COUT + co) * kCin + lane];
    const int64_t ng = ceil_div_d(E, kGroup);
    const int64_t w0 = static_cast<int64_t>(blockIdx.x) * kWaves + wave;
    const int64_t nw = static_cast<int64_t>(gridDim.x) * kWaves;
    for (int64_t gi = w0; gi < ng; gi += nw) {
        const int64_t e0 = gi * kGroup;
        G g;
        int64_t e[kGroup];
        g.load(e0, E, x, src, nsrc, nullptr, P, Q, dist, e, lane, B);
#pragma unroll
        for (int i = 0; i < kGroup; ++i) {
            if (e0 + i >= E) break;
            float fs0[NL], fe[K][NL], pw[NL];
            g.template edge<K>(i, sF, fs0, fe, pw);
            float v[COUT];
#pragma unroll
            for (int co = 0; co < COUT; ++co) v[co] = 0.0f;
#pragma unroll
            for (int k = 0; k < K; ++k) {
                float z = 0.0f;
#pragma unroll
                for (int l = 0; l < NL; ++l) z += fe[k][l] * fs0[l];
#pragma unroll
                for (int co = 0; co < COUT; ++co) v[co] += cw[k][co] * z;
            }
            const float sum = wave_sums<COUT>(v);
            constexpr int GROUP = 64 / COUT;   // lanes that hold one output
            if (lane % GROUP == 0) {
                y[(e0 + i) * COUT + lane / GROUP] = sum * g.q[i];
                if constexpr (YM) ym[(e0 + i) * COUT + lane / GROUP] = sum;
            }
        }
    }
}

// Backward: a wave per 16-edge tile (grid-stride over tiles), its positions in
// groups of kGroupB.  perm: NULL for the identity order; without NS.perm the
// per-edge dx rows go to gx.
// GPQ: also the gradients for the bases (either pointer may be NULL):
//   gP[e][d, l] = sum_c x[c, d] dL/dfs0[c, l] for the m = 0 columns l <= Lin
//                 (zero in the other columns: y does not read them),
//   gQ[e]       = sum_co gy[co] ym[co]  (ym: the forward's rows before Q).
// The gP sums ride in the same wave reduction as the dF_e row.
template <int LIN, int COUT, int K, bool GPQ = false>
__global__ void __launch_bounds__(64 * kWaves)
k_ew0_bwd(feq_binning B, int64_t E, int64_t ntiles, const float* __restrict__ gy,
          const float* __restrict__ x, const int64_t* __restrict__ src, int64_t nsrc,
          const float* __restrict__ P, const float* __restrict__ Q, const float* __restrict__ dist,
          const float* __restrict__ C, const float* __restrict__ F, float* __restrict__ gx,
          float* __restrict__ dFe, float* __restrict__ dCp, NodeScatter NS,
          const float* __restrict__ ym, float* __restrict__ gPo, float* __restrict__ gQo) {
    using G = Group0<LIN, kGroupB>;
    constexpr int DIN = G::DIN, NL = G::NL, KW = K * NL;
    constexpr int NS0 = GPQ ? KW + DIN * NL : KW;   // wave sums per edge
    constexpr int NV = NS0 <= 1 ? 1 : (NS0 <= 2 ? 2 : (NS0 <= 4 ? 4 : (NS0 <= 8 ? 8 : (NS0 <= 16 ? 16 : (NS0 <= 32 ? 32 : 64)))));
    static_assert(NS0 <= 64, "at most 64 sums per edge");
    static_assert(!GPQ || DIN * DIN <= 128, "two gP entries per lane");
    static_assert(kTile % kGroupB == 0, "whole groups per tile");
    extern __shared__ float sF[];
    __shared__ float sdc[kWaves][K * COUT][64];
    stage_table(sF, F, (B.num_bins + 1) * K * NL);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const bool nodes = NS.perm != nullptr;
    float cw[K][COUT], acc[K][COUT];
#pragma unroll
    for (int k = 0; k < K; ++k)
#pragma unroll
        for (int co = 0; co < COUT; ++co) {
            cw[k][co] = C[(k * COUT + co) * kCin + lane];
            acc[k][co] = 0.0f;
        }
    const int64_t w0 = static_cast<int64_t>(blockIdx.x) * kWaves + wave;
    const int64_t nw = static_cast<int64_t>(gridDim.x) * kWaves;
    for (int64_t tile = w0; tile < ntiles; tile += nw) {
        const int64_t p0 = tile * kTile;
        const int np = static_cast<int>(E - p0 < kTile ? E - p0 : kTile);
        float run[DIN];   // the current source node's dx sum (node form)
#pragma unroll
        for (int d = 0; d < DIN; ++d) run[d] = 0.0f;
        int js = 0;
        int64_t nnext = -2;   // source of the position after the current group
        // the tile's per-position values, lane j for position j, in one round of
        // dependent loads (CSR position -> edge -> source row, distance, Q, gy)
        const int jl = lane < np ? lane : np - 1;
        const int64_t el = nodes ? static_cast<int64_t>(NS.perm[p0 + jl]) : p0 + jl;
        int64_t rl = el;
        if (src) {
            rl = src[el];
            rl = rl >= 0 && rl < nsrc ? rl : -1;
        }
        const float dl = dist[el], ql = Q[el];
        const EdgeBin ebl = edge_bin(dl, B);
        const float shl = dl / (dl + B.sh_scale);
        float gql[COUT];   // Q[0, 0] gy of position lane
#pragma unroll
        for (int co = 0; co < COUT; ++co) gql[co] = gy[el * COUT + co] * ql;
        for (int j0 = 0; j0 < np; j0 += kGroupB) {
            G g;
            int64_t e[kGroupB];
            g.load_known(j0, np, static_cast<int>(el), static_cast<int>(rl), ebl.lo, ebl.t, shl, ql, x, P, e,
                         lane);
            float gq[kGroupB][COUT];
#pragma unroll
            for (int i = 0; i < kGroupB; ++i) {
                const int j = j0 + i < np ? j0 + i : np - 1;
#pragma unroll
                for (int co = 0; co < COUT; ++co)
                    gq[i][co] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(gql[co]), j));
            }
            if (nodes) {
                const int jn = j0 + kGroupB;
                nnext = jn < np ? __builtin_amdgcn_readlane(static_cast<int>(rl), jn) : -2;
            }
#pragma unroll
            for (int i = 0; i < kGroupB; ++i) {
                const int j = j0 + i;
                if (j >= np) break;
                float fs0[NL], fe[K][NL], pw[NL];
                g.template edge<K>(i, sF, fs0, fe, pw);
                float gz[K];
#pragma unroll
                for (int k = 0; k < K; ++k) {
                    float z = 0.0f, gk = 0.0f;
#pragma unroll
                    for (int l = 0; l < NL; ++l) z += fe[k][l] * fs0[l];
#pragma unroll
                    for (int co = 0; co < COUT; ++co) {
                        gk += cw[k][co] * gq[i][co];
                        acc[k][co] += gq[i][co] * z;
                    }
                    gz[k] = gk;
                }
                float gfs[NL];
#pragma unroll
                for (int l = 0; l < NL; ++l) {
                    float a = 0.0f;
#pragma unroll
                    for (int k = 0; k < K; ++k) a += fe[k][l] * gz[k];
                    gfs[l] = a;
                }
                float dx[DIN];
#pragma unroll
                for (int d = 0; d < DIN; ++d) {
                    float a = 0.0f;
#pragma unroll
                    for (int l = 0; l < NL; ++l) a += g.pc[i][d][l] * gfs[l];
                    dx[d] = a;
                }
                // dF_e[k, l] = s^l sum_c gz[c, k] fs0[c, l]  (then gP's sums)
                float dv[NV];
#pragma unroll
                for (int q = 0; q < NV; ++q) {
                    float v = 0.0f;
                    if (q < KW)
                        v = gz[q / NL] * fs0[q % NL] * pw[q % NL];
                    else if (q < NS0)
                        v = g.xr[i][(q - KW) / NL] * gfs[(q - KW) % NL];
                    dv[q] = v;
                }
                const float ds = wave_sums<NV>(dv);
                constexpr int GROUP = 64 / NV;
                if (lane % GROUP == 0 && lane / GROUP < KW) dFe[e[i] * KW + lane / GROUP] = ds;
                if constexpr (GPQ) {
                    // lane q GROUP holds sum q; entry n = d DIN + l of gP reads sum
                    // KW + d NL + l when l < NL
                    if (gPo) {
#pragma unroll
                        for (int h = 0; h < 2; ++h) {
                            const int n = lane + 64 * h;
                            const int d = n / DIN, l = n % DIN;
                            const bool m0 = l < NL && n < DIN * DIN;
                            const float v = __shfl(ds, m0 ? (KW + d * NL + l) * GROUP : 0, 64);
                            if (n < DIN * DIN) gPo[e[i] * DIN * DIN + n] = m0 ? v : 0.0f;
                        }
                    }
                    if (gQo) {
                        float a = 0.0f;
#pragma unroll
                        for (int co = 0; co < COUT; ++co) a += gy[e[i] * COUT + co] * ym[e[i] * COUT + co];
                        if (lane == 0) gQo[e[i]] = a;
                    }
                }
                if (!nodes) {
                    float* gr = gx + (e[i] * kCin + lane) * DIN;
#pragma unroll
                    for (int d = 0; d < DIN; ++d) gr[d] = dx[d];
                    continue;
                }
                // per-node sums in tile order (edges without a valid source are dropped)
#pragma unroll
                for (int d = 0; d < DIN; ++d) run[d] += dx[d];
                const int64_t n = g.row[i];
                const int64_t nn = i + 1 < kGroupB ? (j + 1 < np ? g.row[i + 1] : -2) : nnext;
                if (nn == n) continue;
                if (n >= 0) {
                    float* dst;
                    const int b = NS.offsets[n], en = NS.offsets[n + 1];
                    if (b / kTile != (en - 1) / kTile)
                        dst = NS.part + ((2 * tile + (js == 0 ? 0 : 1)) * kCin + lane) * DIN;
                    else
                        dst = NS.out + (n * kCin + lane) * DIN;
#pragma unroll
                    for (int d = 0; d < DIN; ++d) dst[d] = run[d];
                }
#pragma unroll
                for (int d = 0; d < DIN; ++d) run[d] = 0.0f;
                js = j + 1;
            }
        }
    }
    // dC partial of the workgroup: the waves' lane accumulators summed in wave order
    constexpr int NQ = K * COUT;
#pragma unroll
    for (int q = 0; q < NQ; ++q) sdc[wave][q][lane] = acc[q / COUT][q % COUT];
    __syncthreads();
    float* part = dCp + static_cast<int64_t>(blockIdx.x) * NQ * kCin;
    for (int q = threadIdx.x; q < NQ * kCin; q += 64 * kWaves) {
        float a = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) a += sdc[w][q / kCin][q % kCin];
        part[q] = a;   // layout (k, co, c): the (K, Cout, Cin) order of C
    }
}

// Shapes with scalar-output kernels: (Lin, Cout), Cin = 64, rank 4.
#define FEQ_EW0_SHAPES(X) \
    X(2, 8)               \
    X(2, 1)

constexpr int kRank0 = 4;

bool canonical0(const feq_layout& L, int lin) {
    int32_t li[FEQ_MAX_BLOCKS], lo[1] = {0};
    for (int i = 0; i <= lin; ++i) li[i] = i;
    feq_layout ref;
    if (feq_layout_init(&ref, li, lin + 1, lo, 1, L.cin, L.cout) != FEQ_OK) return false;
    if (ref.din != L.din || ref.dout != L.dout || ref.wdim != L.wdim || ref.nblocks != L.nblocks)
        return false;
    for (int k = 0; k < L.nblocks; ++k)
        for (int c = 0; c < 6; ++c)
            if (ref.blk[k][c] != L.blk[k][c]) return false;
    for (int s = 0; s < L.din; ++s)
        if (ref.lslot_in[s] != L.lslot_in[s]) return false;
    return ref.lslot_out[0] == L.lslot_out[0];
}

// The radial table's LDS (dynamic); beyond 64 KB the kernel's limit is raised.
int table_lds(const void* kern, size_t lds) {
    if (lds > 96 * 1024) return fail(FEQ_ERR_UNSUPPORTED, "radial table of %zu B does not fit LDS", lds);
    if (lds > 64 * 1024)
        FEQ_HIP(hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)));
    return FEQ_OK;
}

int groups0(int64_t ntiles) {
    const int64_t g = static_cast<int64_t>(sc_cus()) * 4;
    const int64_t w = ceil_div(ntiles, kWaves);
    return static_cast<int>(w < g ? (w > 0 ? w : 1) : g);
}

}  // namespace

bool ew0_supported(const feq_layout& L, int rank) {
    if (rank != kRank0 || L.cin != kCin) return false;
#define FEQ_SUP(li, co) \
    if (L.cout == co && canonical0(L, li)) return true;
    FEQ_EW0_SHAPES(FEQ_SUP)
#undef FEQ_SUP
    return false;
}

size_t ew0_bwd_workspace(const feq_layout& L, const feq_binning& B, int rank, int64_t E, bool nodes) {
    if (!ew0_supported(L, rank)) return 0;
    const int64_t ntiles = ceil_div(E, kTile);
    const int G = groups0(ntiles);
    const int64_t kw = static_cast<int64_t>(rank) * L.wdim, ncc = static_cast<int64_t>(rank) * L.cout * L.cin;
    Carver cv(nullptr);
    cv.take<float>(E * kw);
    cv.take<float>(static_cast<size_t>(G) * ncc);
    cv.take<float>(ew_tail_floats(B, static_cast<int>(kw), E, G, ncc));
    if (nodes) cv.take<float>(static_cast<size_t>(ntiles) * 2 * L.cin * L.din);
    return cv.used + 256;
}

int ew0_fwd(const feq_layout& L, const feq_binning& B, int rank, int64_t E, const float* x,
            const int64_t* src, int64_t nsrc, const float* P, const float* Q, const float* dist,
            const float* C, const float* F, float* y, float* ym, hipStream_t s) {
    const int64_t g = static_cast<int64_t>(sc_cus()) * 8, need = ceil_div(ceil_div(E, kGroup), kWaves);
    const unsigned grid = static_cast<unsigned>(need < g ? need : g);
    const size_t lds = 4 * static_cast<size_t>(B.num_bins + 1) * rank * L.wdim;
#define FEQ_FWD(li, co)                                                                      \
    if (L.cout == co && canonical0(L, li)) {                                                 \
        auto kern = ym ? k_ew0_fwd<li, co, kRank0, true> : k_ew0_fwd<li, co, kRank0>;        \
        if (int rc = table_lds(reinterpret_cast<const void*>(kern), lds)) return rc;         \
        FEQ_LAUNCH("k_ew0_fwd", kern, dim3(grid), dim3(64 * kWaves), lds, s, B, E, x, src, nsrc, P, \
                   Q, dist, C, F, y, ym);                                                    \
        return FEQ_OK;                                                                       \
    }
    if (rank == kRank0 && L.cin == kCin) {
        FEQ_EW0_SHAPES(FEQ_FWD)
    }
#undef FEQ_FWD
    return fail(FEQ_ERR_UNSUPPORTED, "no scalar-output kernels for this layout");
}

int ew0_bwd(const feq_layout& L, const feq_binning& B, int rank, int64_t E, const float* gy,
            const float* x, const int64_t* src, int64_t nsrc, const float* P, const float* Q,
            const float* dist, const float* C, const float* F, float* gx, float* gC, float* gF,
            float* gdist, const NodeScatter* ns, void* ws, size_t ws_bytes, hipStream_t s,
            const float* ym, float* gP, float* gQ) {
    if (gQ && !ym) return fail(FEQ_ERR_INVALID, "grad_Q needs the rows before the rotation");
    if (ws_bytes < ew0_bwd_workspace(L, B, rank, E, ns != nullptr))
        return fail(FEQ_ERR_WORKSPACE, "edgewise workspace too small");
    const int64_t ntiles = ceil_div(E, kTile);
    const int G = groups0(ntiles);
    const int kw = rank * L.wdim;
    const int64_t ncc = static_cast<int64_t>(rank) * L.cout * L.cin;
    Carver cv(ws);
    float* dFe = cv.take<float>(E * kw);
    float* dCp = cv.take<float>(static_cast<size_t>(G) * ncc);
    float* tail = cv.take<float>(ew_tail_floats(B, kw, E, G, ncc));
    NodeScatter NS{};
    if (ns) {
        NS = *ns;
        NS.part = cv.take<float>(static_cast<size_t>(ntiles) * 2 * L.cin * L.din);
    }
    const size_t lds = 4 * static_cast<size_t>(B.num_bins + 1) * rank * L.wdim;
#define FEQ_BWD(li, co)                                                                          \
    if (L.cout == co && canonical0(L, li)) {                                                     \
        auto kern = (gP || gQ) ? k_ew0_bwd<li, co, kRank0, true> : k_ew0_bwd<li, co, kRank0>;   \
        if (int rc = table_lds(reinterpret_cast<const void*>(kern), lds)) return rc;             \
        FEQ_LAUNCH("k_ew0_bwd", kern, dim3(G), dim3(64 * kWaves), lds, s, B, E, ntiles, gy, x, src, \
                   nsrc, P, Q, dist, C, F, gx, dFe, dCp, NS, ym, gP, gQ);                       \
        if (ns)                                                                                  \
            if (int rc = node_fix(NS, nsrc, static_cast<int64_t>(L.cin) * L.din / 4, s)) return rc; \
        return ew_tail(L, B, rank, E, dist, F, dFe, dCp, G, ncc, gC, gF, gdist, tail, s);        \
    }
    if (rank == kRank0 && L.cin == kCin) {
        FEQ_EW0_SHAPES(FEQ_BWD)
    }
#undef FEQ_BWD
    return fail(FEQ_ERR_UNSUPPORTED, "no scalar-output kernels for this layout");
}

}  // namespace feq

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
// exchange halves the values a lane keeps, then the single value is summed
// over the remaining lane groups.  Lane l returns value (l >> (6 - log2 N)).
template <int N>
__device__ __forceinline__ float wave_sums(float (&v)[N]) {
    static_assert(N >= 1 && N <= 64 && (N & (N - 1)) == 0, "power of two");
    const int lane = threadIdx.x & 63;
    int n = N, half_lanes = 32;
    float w[N];
#pragma unroll
    for (int i = 0; i < N; ++i) w[i] = v[i];
#pragma unroll
    for (int step = 0; (1 << step) < N; ++step) {
        // lanes with bit `half_lanes` set keep the upper half of the values
        const bool upper = (lane & half_lanes) != 0;
        n >>= 1;
#pragma unroll
        for (int i = 0; i < N / 2; ++i) {
            if (i < n) {
                const float send = upper ? w[i] : w[i + n];
                const float keep = upper ? w[i + n] : w[i];
                w[i] = keep + __shfl_xor(send, half_lanes, 64);
            }
        }
        half_lanes >>= 1;
    }
    float s = w[0];
    for (int off = half_lanes; off >= 1; off >>= 1) s += __shfl_xor(s, off, 64);
    return s;
}

struct SRows {
    const float* x;
    const int64_t* src;   // NULL: edge e reads row e
    int64_t nsrc;
};

__device__ __forceinline__ int64_t s_row(const SRows& X, int64_t e) {
    if (!X.src) return e;
    const int64_t r = X.src[e];
    return r >= 0 && r < X.nsrc ? r : -1;
}

// Per-edge state shared by both directions: fs0 of this lane's channel, the
// scaled radial functions F_e[k, l] s^l, Q[0, 0].
template <int LIN, int K>
struct Edge0 {
    static constexpr int DIN = (LIN + 1) * (LIN + 1), NL = LIN + 1;
    float xr[DIN];
    float fs0[NL];
    float fe[K][NL];
    float pw[NL];
    float q00;
    float pcol[DIN][NL];

    __device__ __forceinline__ void load(const feq_binning& B, const SRows& X, int64_t e,
                                         const float* __restrict__ P, const float* __restrict__ Q,
                                         const float* __restrict__ dist, const float* __restrict__ F,
                                         int lane) {
        const int64_t row = s_row(X, e);
        const float* xs = X.x + ((row >= 0 ? row : 0) * kCin + lane) * DIN;
#pragma unroll
        for (int d = 0; d < DIN; ++d) xr[d] = row >= 0 ? xs[d] : 0.0f;
        const float* pe = P + e * DIN * DIN;
#pragma unroll
        for (int d = 0; d < DIN; ++d)
#pragma unroll
            for (int l = 0; l < NL; ++l) pcol[d][l] = pe[d * DIN + l];
        q00 = Q[e];
        const float r = dist[e];
        const EdgeBin eb = edge_bin(r, B);
        const float s = r / (r + B.sh_scale);
        float p = 1.0f;
#pragma unroll
        for (int l = 0; l < NL; ++l) {
            pw[l] = p;
            p *= s;
        }
        const float* flo = F + static_cast<int64_t>(eb.lo) * K * NL;
#pragma unroll
        for (int k = 0; k < K; ++k)
#pragma unroll
            for (int l = 0; l < NL; ++l)
                fe[k][l] = lerp_bins(flo[k * NL + l], flo[K * NL + k * NL + l], eb.t) * pw[l];
#pragma unroll
        for (int l = 0; l < NL; ++l) {
            float a = 0.0f;
#pragma unroll
            for (int d = 0; d < DIN; ++d) a += xr[d] * pcol[d][l];
            fs0[l] = a;
        }
    }
};

// Forward: waves walk the edges (grid-stride), one edge at a time.
template <int LIN, int COUT, int K>
__global__ void __launch_bounds__(64 * kWaves)
k_ew0_fwd(feq_binning B, int64_t E, SRows X, const float* __restrict__ P, const float* __restrict__ Q,
          const float* __restrict__ dist, const float* __restrict__ C, const float* __restrict__ F,
          float* __restrict__ y) {
    using ED = Edge0<LIN, K>;
    const int lane = threadIdx.x & 63;
    float cw[K][COUT];   // C_k[co, lane]
#pragma unroll
    for (int k = 0; k < K; ++k)
#pragma unroll
        for (int co = 0; co < COUT; ++co) cw[k][co] = C[(k * COUT + co) * kCin + lane];
    const int64_t w0 = static_cast<int64_t>(blockIdx.x) * kWaves + (threadIdx.x >> 6);
    const int64_t nw = static_cast<int64_t>(gridDim.x) * kWaves;
    for (int64_t e = w0; e < E; e += nw) {
        ED ed;
        ed.load(B, X, e, P, Q, dist, F, lane);
        float z[K];
#pragma unroll
        for (int k = 0; k < K; ++k) {
            float a = 0.0f;
#pragma unroll
            for (int l = 0; l < ED::NL; ++l) a += ed.fe[k][l] * ed.fs0[l];
            z[k] = a;
        }
        float v[COUT];
#pragma unroll
        for (int co = 0; co < COUT; ++co) {
            float a = 0.0f;
#pragma unroll
            for (int k = 0; k < K; ++k) a += cw[k][co] * z[k];
            v[co] = a;
        }
        const float sum = wave_sums<COUT>(v);
        constexpr int GROUP = 64 / COUT;   // lanes that hold one output
        if (lane % GROUP == 0) y[e * COUT + lane / GROUP] = sum * ed.q00;
    }
}

// Backward: a wave per 16-edge tile (grid-stride over tiles).  perm: NULL for
// the identity order; ns: NULL for per-edge dx rows into gx.
template <int LIN, int COUT, int K>
__global__ void __launch_bounds__(64 * kWaves)
k_ew0_bwd(feq_binning B, int64_t E, int64_t ntiles, const float* __restrict__ gy, SRows X,
          const float* __restrict__ P, const float* __restrict__ Q, const float* __restrict__ dist,
          const float* __restrict__ C, const float* __restrict__ F, float* __restrict__ gx,
          float* __restrict__ dFe, float* __restrict__ dCp, NodeScatter NS) {
    using ED = Edge0<LIN, K>;
    constexpr int DIN = ED::DIN, NL = ED::NL, KW = K * NL;
    constexpr int NV = KW <= 1 ? 1 : (KW <= 2 ? 2 : (KW <= 4 ? 4 : (KW <= 8 ? 8 : (KW <= 16 ? 16 : 32))));
    static_assert(KW <= 32, "radial row of at most 32 values");
    __shared__ float sdc[kWaves][K * COUT * kCin / 64][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
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
        for (int j = 0; j < np; ++j) {
            const int64_t e = nodes ? NS.perm[p0 + j] : p0 + j;
            ED ed;
            ed.load(B, X, e, P, Q, dist, F, lane);
            float gq[COUT];
#pragma unroll
            for (int co = 0; co < COUT; ++co) gq[co] = gy[e * COUT + co] * ed.q00;
            float z[K], gz[K];
#pragma unroll
            for (int k = 0; k < K; ++k) {
                float a = 0.0f, g = 0.0f;
#pragma unroll
                for (int l = 0; l < NL; ++l) a += ed.fe[k][l] * ed.fs0[l];
#pragma unroll
                for (int co = 0; co < COUT; ++co) g += cw[k][co] * gq[co];
                z[k] = a;
                gz[k] = g;
            }
#pragma unroll
            for (int k = 0; k < K; ++k)
#pragma unroll
                for (int co = 0; co < COUT; ++co) acc[k][co] += gq[co] * z[k];
            // dx of this edge and channel
            float gfs[NL];
#pragma unroll
            for (int l = 0; l < NL; ++l) {
                float a = 0.0f;
#pragma unroll
                for (int k = 0; k < K; ++k) a += ed.fe[k][l] * gz[k];
                gfs[l] = a;
            }
            float dx[DIN];
#pragma unroll
            for (int d = 0; d < DIN; ++d) {
                float a = 0.0f;
#pragma unroll
                for (int l = 0; l < NL; ++l) a += ed.pcol[d][l] * gfs[l];
                dx[d] = a;
            }
            // dF_e[k, l] = s^l sum_c gz[c, k] fs0[c, l]
            float dv[NV];
#pragma unroll
            for (int q = 0; q < NV; ++q) dv[q] = q < KW ? gz[q / NL] * ed.fs0[q % NL] * ed.pw[q % NL] : 0.0f;
            const float ds = wave_sums<NV>(dv);
            constexpr int GROUP = 64 / NV;
            if (lane % GROUP == 0 && lane / GROUP < KW) dFe[e * KW + lane / GROUP] = ds;
            if (!nodes) {
                float* g = gx + (e * kCin + lane) * DIN;
#pragma unroll
                for (int d = 0; d < DIN; ++d) g[d] = dx[d];
                continue;
            }
            // per-node sums in tile order (rows of edges with no valid source are dropped)
#pragma unroll
            for (int d = 0; d < DIN; ++d) run[d] += dx[d];
            const int64_t n = s_row(X, e);
            if (j + 1 < np && s_row(X, NS.perm[p0 + j + 1]) == n) continue;
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
            const float* C, const float* F, float* y, hipStream_t s) {
    const SRows X{x, src, nsrc};
    const int64_t g = static_cast<int64_t>(sc_cus()) * 8, need = ceil_div(E, kWaves);
    const unsigned grid = static_cast<unsigned>(need < g ? need : g);
#define FEQ_FWD(li, co)                                                                      \
    if (L.cout == co && canonical0(L, li)) {                                                 \
        auto kern = k_ew0_fwd<li, co, kRank0>;                                               \
        FEQ_LAUNCH("k_ew0_fwd", kern, dim3(grid), dim3(64 * kWaves), 0, s, B, E, X, P, Q, dist, C, \
                   F, y);                                                                    \
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
            float* gdist, const NodeScatter* ns, void* ws, size_t ws_bytes, hipStream_t s) {
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
    const SRows X{x, src, nsrc};
#define FEQ_BWD(li, co)                                                                          \
    if (L.cout == co && canonical0(L, li)) {                                                     \
        auto kern = k_ew0_bwd<li, co, kRank0>;                                                   \
        FEQ_LAUNCH("k_ew0_bwd", kern, dim3(G), dim3(64 * kWaves), 0, s, B, E, ntiles, gy, X, P, Q, \
                   dist, C, F, gx, dFe, dCp, NS);                                                \
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

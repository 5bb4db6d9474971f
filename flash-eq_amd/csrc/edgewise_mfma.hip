// Fused EquivariantEdgewiseLinear on the fp32 matrix cores of gfx950.
//
// Same mathematics as edgewise.hip (see the derivation there); this file is
// the fast path for canonical representations lvals = [0, 1, ..., L] and
// channel counts known at compile time.  Per edge e the interpolated radial
// functions define a sparse mixing matrix in the m-first basis,
//     M_e[o][i] = sign(t) F_e[k, w(t)]     for every term t = (o, i, w, sign),
// fixed by the m-block layout (2x2 [[a, b], [-b, a]] blocks for m > 0), so
//     yd[co, e, o] = sum_k sum_i M_ek[o][i] G_k[co, e, i],  G_k = C_k fs.
// A workgroup (4 waves) owns a tile of 16 edges.  GEMM columns are ordered
// slot-major (column = 16 * slot + e): MFMA lane l then holds every slot of
// edge e = l % 16 for its rows, so all contractions with M_e run in registers.
//
//   forward   G_k = C_k fs                  M = Cout, N = 16 Din, K = Cin
//             (one B fragment of fs feeds all K rank components)
//   backward  H_k = C_k^T gd                M = Cin,  N = 16 Dout, K = Cout
//             dfs = sum_k M_ek^T H_k, dF_e[k, w] = sum_ci fs H_k (register
//             partials, two lane shuffles, one LDS pass over the 4 waves)
//             dC_k += U_k fs^T, U_k = M_ek^T gd   M = Cout, N = Cin, K = 16 Din
//
// MFMA v_mfma_f32_16x16x4f32: lane l supplies A[l%16][l/16] and B[l/16][l%16]
// and holds D[4*(l/16)+r][l%16] in register r (checked on the device).  LDS
// rows use odd strides, so the column-wise stores of the builders and the MFMA
// fragment loads are bank-conflict free.
#include "feq_internal.h"
#include "ew_canon.h"

#include <algorithm>
#include <array>
#include <type_traits>

namespace feq {
namespace {

typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kNE = 16;       // edges per tile
constexpr int kThreads = 256;

__device__ __forceinline__ v4f mfma(float a, float b, v4f c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

struct TileEdge {
    int lo;
    float t;
    float s;
    int valid;
};

// ---- register prefetch of a tile's raw inputs ------------------------------
// While the matrix cores work on tile t, every thread already holds its share
// of tile t + gridDim.x in registers: its (edge, channel) rows of x (or gy),
// its slice of the tile's P and Q blocks and (threads < kNE) one distance.
// Rows past the last edge read as zero, so a prefetch beyond the last tile
// touches no memory.

// Rows (e, c) of a (E, CH, D) tensor; thread t holds rows q = t + kThreads j.
template <int CH, int D>
struct RowRegs {
    static constexpr int NR = kNE * CH / kThreads;
    static_assert(kNE * CH % kThreads == 0, "rows must split evenly over the workgroup");
    float v[NR][D];
    __device__ __forceinline__ void load(const float* __restrict__ src, int64_t e0, int64_t E) {
#pragma unroll
        for (int j = 0; j < NR; ++j) {
            const int q = threadIdx.x + kThreads * j;
            const int e = q / CH, c = q % CH;
            if (e0 + e < E) {
                const float* p = src + ((e0 + e) * CH + c) * D;
#pragma unroll
                for (int d = 0; d < D; ++d) v[j][d] = p[d];
            } else {
#pragma unroll
                for (int d = 0; d < D; ++d) v[j][d] = 0.0f;
            }
        }
    }
};

// x rows in the MFMA accumulator layout: lane (le, lg) of wave w holds rows
// (e0 + le, c = 16 (w + 4 j) + 4 lg + r), r < 4.
template <int CH, int D>
struct LaneRows {
    static constexpr int RPW = CH / 64;
    static_assert(CH % 64 == 0, "lane rows need whole 64-channel groups");
    float v[RPW][4][D];
    __device__ __forceinline__ void load(const float* __restrict__ src, int64_t e0, int64_t E) {
        const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
        const int le = lane & 15, lg = lane >> 4;
        const bool ok = e0 + le < E;
#pragma unroll
        for (int j = 0; j < RPW; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                if (ok) {
                    const float* p = src + ((e0 + le) * CH + 16 * (wave + 4 * j) + 4 * lg + r) * D;
#pragma unroll
                    for (int d = 0; d < D; ++d) v[j][r][d] = p[d];
                } else {
#pragma unroll
                    for (int d = 0; d < D; ++d) v[j][r][d] = 0.0f;
                }
            }
    }
};

// N consecutive floats starting at element `base` (a tile's P or Q block).
template <int N>
struct BlockRegs {
    static constexpr int NR = (N + kThreads - 1) / kThreads;
    float v[NR];
    __device__ __forceinline__ void load(const float* __restrict__ src, int64_t base, int64_t end) {
#pragma unroll
        for (int j = 0; j < NR; ++j) {
            const int q = threadIdx.x + kThreads * j;
            v[j] = (q < N && base + q < end) ? src[base + q] : 0.0f;
        }
    }
    __device__ __forceinline__ void store(float* dst) const {
#pragma unroll
        for (int j = 0; j < NR; ++j) {
            const int q = threadIdx.x + kThreads * j;
            if (q < N) dst[q] = v[j];
        }
    }
};

// Edge state of a tile from the prefetched distances (threads < kNE).
template <int LIN, int LOUT>
__device__ __forceinline__ void commit_edges(const feq_binning& B, int64_t E, int64_t e0, float r,
                                             TileEdge* sE, float* sSin, float* sSout) {
    constexpr int DIN = (LIN + 1) * (LIN + 1), DOUT = (LOUT + 1) * (LOUT + 1);
    const int tid = threadIdx.x;
    if (tid < kNE) {
        TileEdge te;
        te.valid = (e0 + tid) < E;
        if (!te.valid) r = 1.0f;
        const EdgeBin eb = edge_bin(r, B);
        te.lo = eb.lo;
        te.t = eb.t;
        te.s = r / (r + B.sh_scale);
        sE[tid] = te;
#pragma unroll
        for (int j = 0; j < DIN; ++j) sSin[tid * DIN + j] = ipowf(te.s, SlotL<LIN>::l[j]);
#pragma unroll
        for (int j = 0; j < DOUT; ++j) sSout[tid * DOUT + j] = ipowf(te.s, SlotL<LOUT>::l[j]);
    }
}

// F_e = (1-t) F[lo] + t F[lo+1] for the tile's edges; Ft is the radial-function
// table (num_bins+1, KW), in LDS or in global memory.
template <int KW>
__device__ __forceinline__ void interp_tile(const TileEdge* sE, const float* Ft, float* sFe) {
    for (int q = threadIdx.x; q < kNE * KW; q += kThreads) {
        const int e = q / KW, rest = q % KW;
        const TileEdge te = sE[e];
        const float* flo = Ft + te.lo * KW;
        sFe[q] = lerp_bins(flo[rest], flo[KW + rest], te.t);
    }
}

// Rows F[lo] and F[lo + 1] of the radial-function table for a tile's edges;
// thread t holds elements q = t + kThreads j of the (kNE, KW) tile.  `sLo`
// holds the tile's lower bins (in range even for padding edges).
template <int KW>
struct FRowRegs {
    static constexpr int NR = (kNE * KW + kThreads - 1) / kThreads;
    float lo[NR], hi[NR];
    __device__ __forceinline__ void load(const float* __restrict__ F, const int* sLo) {
#pragma unroll
        for (int j = 0; j < NR; ++j) {
            const int q = threadIdx.x + kThreads * j;
            if (q < kNE * KW) {
                const float* f = F + sLo[q / KW] * KW + q % KW;
                lo[j] = f[0];
                hi[j] = f[KW];
            }
        }
    }
    __device__ __forceinline__ void commit(const TileEdge* sE, float* sFe) const {
#pragma unroll
        for (int j = 0; j < NR; ++j) {
            const int q = threadIdx.x + kThreads * j;
            if (q < kNE * KW) sFe[q] = lerp_bins(lo[j], hi[j], sE[q / KW].t);
        }
    }
};

// dst[c * stride + 16 i + e] = s^l_i sum_d rows(e, c)[d] R_e[d, i]  (x P or gy Q)
template <int CH, int D>
__device__ __forceinline__ void rotate_regs(const RowRegs<CH, D>& rr, const float* sR,
                                            const float* sS, float* dst, int stride) {
#pragma unroll
    for (int j = 0; j < RowRegs<CH, D>::NR; ++j) {
        const int q = threadIdx.x + kThreads * j;
        const int e = q / CH, c = q % CH;
        const float* re = sR + e * D * D;
#pragma unroll
        for (int i = 0; i < D; ++i) {
            float acc = 0.0f;
#pragma unroll
            for (int d = 0; d < D; ++d) acc += rr.v[j][d] * re[d * D + i];
            dst[c * stride + 16 * i + e] = acc * sS[e * D + i];
        }
    }
}

// ---------------------------------------------------------------------------
// A fragments of C_k (or C_k^T) staged in LDS in fragment order:
// frag[((k * NRB + rb) * NS + s) * 64 + lane] = A[16 rb + lane%16][4 s + lane/16],
// so each wave reads one contiguous, conflict-free 256-byte row per fragment.
template <int K, int NRB, int NS, bool TRANS>
__device__ void stage_frags(const float* __restrict__ C, int cout, int cin, float* frag) {
    for (int q = threadIdx.x; q < K * NRB * NS * 64; q += kThreads) {
        const int lane = q & 63, s = (q >> 6) % NS, rb = ((q >> 6) / NS) % NRB, k = (q >> 6) / (NS * NRB);
        const int row = 16 * rb + (lane & 15), col = 4 * s + (lane >> 4);
        // A = C_k (rows co, cols ci) or A = C_k^T (rows ci, cols co)
        frag[q] = TRANS ? C[(static_cast<int64_t>(k) * cout + col) * cin + row]
                        : C[(static_cast<int64_t>(k) * cout + row) * cin + col];
    }
}

// x rows of a tile rotated into the m-first frame: fs[ci][16 i + e] =
// s^l_i sum_d x[e, ci, d] P_e[d, i] (thread t handles rows q = t + kThreads j).
template <int CIN, int DIN>
__device__ __forceinline__ void rotate_rows(const float* __restrict__ x, int64_t e0, int64_t E,
                                            const float* sP, const float* sSin, float* sf,
                                            int fs) {
    RowRegs<CIN, DIN> rr;
    rr.load(x, e0, E);
    rotate_regs<CIN, DIN>(rr, sP, sSin, sf, fs);
}

// A fragments held in registers for the whole launch.  Lane (le, lg) of wave w
// keeps A[16 (w + 4 j) + le][lg * NS + s] of every rank component k, with
// A = C_k (rows co, cols ci) or A = C_k^T (rows ci, cols co).  The reduction
// index of every product is ordered c = lg * NS + s: any order is valid as long
// as the B fragments use the same one.
template <int RPW, int K, int NS>
struct AFrags {
    float v[RPW][K][NS];
    __device__ __forceinline__ void load(const float* __restrict__ C, int cout, int cin,
                                         bool trans) {
        const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
        const int le = lane & 15, lg = lane >> 4;
#pragma unroll
        for (int j = 0; j < RPW; ++j)
#pragma unroll
            for (int k = 0; k < K; ++k)
#pragma unroll
                for (int s = 0; s < NS; ++s) {
                    const int row = 16 * (wave + 4 * j) + le, col = lg * NS + s;
                    v[j][k][s] = trans ? C[(static_cast<int64_t>(k) * cout + col) * cin + row]
                                       : C[(static_cast<int64_t>(k) * cout + row) * cin + col];
                }
    }
};

// Forward: G_k = C_k fs on the matrix cores, y = Q-rotate(s^l sum_k M_ek G_k).
// Two workgroups share a CU (C_k lives in registers, not LDS), so one
// workgroup's rotations, contractions and memory traffic overlap the other's
// matrix-core loop.  The rank components run in two passes to halve the live
// accumulators.
template <int CIN, int COUT, int LIN, int LOUT, int K>
__global__ void __launch_bounds__(kThreads, 2)
k_ewc_fwd(feq_binning B, int64_t E, int64_t ntiles, const float* __restrict__ x,
          const float* __restrict__ P, const float* __restrict__ Q,
          const float* __restrict__ dist, const float* __restrict__ C,
          const float* __restrict__ F, float* __restrict__ y) {
    using T = Canon<LIN, LOUT>;
    constexpr int DIN = T::DIN, DOUT = T::DOUT, WD = T::WD, KW = K * WD;
    constexpr int FS = 16 * DIN + 1;
    constexpr int YS = COUT * DOUT + 1;
    constexpr int RPW = COUT / 64, NS = CIN / 4, KH = 1;
    constexpr int BIG = CIN * FS > kNE * YS ? CIN * FS : kNE * YS;
    static_assert(COUT % 64 == 0 && CIN % 16 == 0, "unsupported channel counts");
    extern __shared__ float4 smem4[];
    float* sf = reinterpret_cast<float*>(smem4);   // fs tile, later the y staging tile
    float* sP = sf + BIG;
    float* sQ = sP + kNE * DIN * DIN;
    float* sSin = sQ + kNE * DOUT * DOUT;
    float* sSout = sSin + kNE * DIN;
    float* sFe = sSout + kNE * DOUT;
    TileEdge* sE = reinterpret_cast<TileEdge*>(sFe + kNE * KW);

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int le = lane & 15, lg = lane >> 4;
    AFrags<RPW, K, NS> A;
    A.load(C, COUT, CIN, false);

    for (int64_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
        const int64_t e0 = tile * kNE;
        __syncthreads();   // the previous tile's readers of the LDS tiles are done
        {
            BlockRegs<kNE * DIN * DIN> pr;
            BlockRegs<kNE * DOUT * DOUT> qr;
            pr.load(P, e0 * DIN * DIN, E * DIN * DIN);
            qr.load(Q, e0 * DOUT * DOUT, E * DOUT * DOUT);
            const float r = (tid < kNE && e0 + tid < E) ? dist[e0 + tid] : 1.0f;
            pr.store(sP);
            qr.store(sQ);
            commit_edges<LIN, LOUT>(B, E, e0, r, sE, sSin, sSout);
        }
        __syncthreads();
        interp_tile<KW>(sE, F, sFe);
        rotate_rows<CIN, DIN>(x, e0, E, sP, sSin, sf, FS);
        __syncthreads();

        // lane (edge le, rows co = 16 (wave + 4 j) + 4 lg + r)
        float yv[RPW][DOUT][4];
#pragma unroll
        for (int j = 0; j < RPW; ++j)
#pragma unroll
            for (int o = 0; o < DOUT; ++o)
#pragma unroll
                for (int r = 0; r < 4; ++r) yv[j][o][r] = 0.0f;
#pragma unroll
        for (int k0 = 0; k0 < K; k0 += KH) {
            v4f acc[RPW][KH][DIN];
#pragma unroll
            for (int j = 0; j < RPW; ++j)
#pragma unroll
                for (int kk = 0; kk < KH; ++kk)
#pragma unroll
                    for (int i = 0; i < DIN; ++i) acc[j][kk][i] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
            // B fragments are loaded one step ahead; the scheduling fence after
            // each step keeps the compiler from hoisting every step's loads.
            float b[2][DIN];
#pragma unroll
            for (int i = 0; i < DIN; ++i) b[0][i] = sf[lg * NS * FS + le + 16 * i];
#pragma unroll
            for (int s = 0; s < NS; ++s) {
                if (s + 1 < NS) {
                    const float* row = sf + (lg * NS + s + 1) * FS + le;
#pragma unroll
                    for (int i = 0; i < DIN; ++i) b[(s + 1) & 1][i] = row[16 * i];
                }
#pragma unroll
                for (int j = 0; j < RPW; ++j)
#pragma unroll
                    for (int kk = 0; kk < KH; ++kk)
#pragma unroll
                        for (int i = 0; i < DIN; ++i)
                            acc[j][kk][i] = mfma(A.v[j][k0 + kk][s], b[s & 1][i], acc[j][kk][i]);
                __builtin_amdgcn_sched_barrier(0);
            }
#pragma unroll
            for (int kk = 0; kk < KH; ++kk) {
                float fk[WD];
#pragma unroll
                for (int w = 0; w < WD; ++w) fk[w] = sFe[le * KW + (k0 + kk) * WD + w];
#pragma unroll
                for (int t = 0; t < T::NT; ++t) {
                    const Term tm = T::terms[t];
                    const float c = tm.neg ? -fk[tm.w] : fk[tm.w];
#pragma unroll
                    for (int j = 0; j < RPW; ++j)
#pragma unroll
                        for (int r = 0; r < 4; ++r) yv[j][tm.o][r] += c * acc[j][kk][tm.i][r];
                }
            }
        }
#pragma unroll
        for (int o = 0; o < DOUT; ++o) {
            const float sc = sSout[le * DOUT + o];
#pragma unroll
            for (int j = 0; j < RPW; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r) yv[j][o][r] *= sc;
        }
        __syncthreads();   // every wave is done reading fs: the tile becomes the y stage
        const float* qe = sQ + le * DOUT * DOUT;
#pragma unroll
        for (int d = 0; d < DOUT; ++d) {
            float qrow[DOUT];
#pragma unroll
            for (int o = 0; o < DOUT; ++o) qrow[o] = qe[d * DOUT + o];
#pragma unroll
            for (int j = 0; j < RPW; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    float acc_d = 0.0f;
#pragma unroll
                    for (int o = 0; o < DOUT; ++o) acc_d += yv[j][o][r] * qrow[o];
                    sf[le * YS + (16 * (wave + 4 * j) + 4 * lg + r) * DOUT + d] = acc_d;
                }
        }
        __syncthreads();
        float* yt = y + e0 * COUT * DOUT;
        if (E - e0 >= kNE) {
#pragma unroll
            for (int m = 0; m < kNE * COUT * DOUT / kThreads; ++m) {
                const int q = tid + kThreads * m;
                yt[q] = sf[(q / (COUT * DOUT)) * YS + q % (COUT * DOUT)];
            }
        } else {
            for (int q = tid; q < (E - e0) * COUT * DOUT; q += kThreads)
                yt[q] = sf[(q / (COUT * DOUT)) * YS + q % (COUT * DOUT)];
        }
    }
}

// Register pipeline of the backward kernels.  At the top of the iteration for
// tile t the registers hold tile t's x and gy rows, P and Q blocks and F rows,
// and the distances of tiles t and t + G (G = gridDim.x); `next()` issues the
// loads for tile t + G (whose bins are known one tile ahead) and the distance
// of tile t + 2G, so every global load has a whole tile of work to arrive.
template <int CIN, int COUT, int LIN, int LOUT, int K, bool XLANE>
struct BwdPipe {
    using T = Canon<LIN, LOUT>;
    static constexpr int DIN = T::DIN, DOUT = T::DOUT, KW = K * T::WD;
    // x rows: one (edge, channel) row per thread and pass (XLANE false, for an
    // fs tile in LDS) or in the accumulator layout (XLANE true, fs in registers)
    typename std::conditional<XLANE, LaneRows<CIN, DIN>, RowRegs<CIN, DIN>>::type xr;
    RowRegs<COUT, DOUT> gr;
    BlockRegs<kNE * DIN * DIN> pr;
    BlockRegs<kNE * DOUT * DOUT> qr;
    FRowRegs<KW> fr;
    float r_cur = 1.0f, r_next = 1.0f;

    __device__ __forceinline__ float load_dist(const float* __restrict__ dist, int64_t t,
                                               int64_t E) const {
        const int64_t e = t * kNE + threadIdx.x;
        return (threadIdx.x < kNE && e < E) ? dist[e] : 1.0f;
    }
    __device__ __forceinline__ void load_rows(int64_t t, int64_t E, const float* __restrict__ x,
                                              const float* __restrict__ gy,
                                              const float* __restrict__ P,
                                              const float* __restrict__ Q) {
        const int64_t p0 = t * kNE;
        xr.load(x, p0, E);
        gr.load(gy, p0, E);
        pr.load(P, p0 * DIN * DIN, E * DIN * DIN);
        qr.load(Q, p0 * DOUT * DOUT, E * DOUT * DOUT);
    }
    // Before the loop: tile t0's rows, bins and F rows; tile t0 + G's distance.
    __device__ void prologue(const feq_binning& B, int64_t t0, int64_t G, int64_t E,
                             const float* x, const float* gy, const float* P, const float* Q,
                             const float* dist, const float* F, int* sLo) {
        r_cur = load_dist(dist, t0, E);
        if (threadIdx.x < kNE) sLo[threadIdx.x] = edge_bin(r_cur, B).lo;
        r_next = load_dist(dist, t0 + G, E);
        load_rows(t0, E, x, gy, P, Q);
        __syncthreads();
        fr.load(F, sLo);
    }
    // Tile top (after a barrier): P/Q blocks and edge state to LDS, and the
    // next tile's bins for the F-row prefetch.
    __device__ __forceinline__ void commit(const feq_binning& B, int64_t E, int64_t e0, float* sP,
                                           float* sQ, TileEdge* sE, float* sSin, float* sSout,
                                           int* sLo) {
        pr.store(sP);
        qr.store(sQ);
        commit_edges<LIN, LOUT>(B, E, e0, r_cur, sE, sSin, sSout);
        if (threadIdx.x < kNE) sLo[threadIdx.x] = edge_bin(r_next, B).lo;
    }
    // After the next barrier: F_e, gd = s^l (gy Q) and (row layout) fs =
    // s^l (x P) to LDS.
    __device__ __forceinline__ void rotate(const TileEdge* sE, float* sFe, const float* sP,
                                           const float* sQ, const float* sSin,
                                           const float* sSout, float* sf, int fs, float* sG,
                                           int gs) const {
        fr.commit(sE, sFe);
        if constexpr (!XLANE) rotate_regs<CIN, DIN>(xr, sP, sSin, sf, fs);
        rotate_regs<COUT, DOUT>(gr, sQ, sSout, sG, gs);
    }
    // Accumulator layout only: fsr[j][r][i] = s^l_i sum_d x[d] P_e[d, i] for
    // the lane's rows of edge le.
    template <int RPW>
    __device__ __forceinline__ void lane_fs(const float* sP, const float* sSin,
                                            float (&fsr)[RPW][4][DIN]) const {
        const int le = threadIdx.x & 15;
        const float* pe = sP + le * DIN * DIN;
#pragma unroll
        for (int j = 0; j < RPW; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int i = 0; i < DIN; ++i) {
                    float acc = 0.0f;
#pragma unroll
                    for (int d = 0; d < DIN; ++d) acc += xr.v[j][r][d] * pe[d * DIN + i];
                    fsr[j][r][i] = acc * sSin[le * DIN + i];
                }
    }
    // Once the tile's register data is in LDS (after a barrier): loads for tile t + G.
    __device__ __forceinline__ void next(int64_t t, int64_t G, int64_t E, const float* x,
                                         const float* gy, const float* P, const float* Q,
                                         const float* dist, const float* F, const int* sLo) {
        load_rows(t + G, E, x, gy, P, Q);
        fr.load(F, sLo);
        r_cur = r_next;
        r_next = load_dist(dist, t + 2 * G, E);
    }
};

// A fragments of C_k^T for one rank component: lane (le, lg) of wave w holds
// C_k[lg * NS + s][16 (w + 4 j) + le] for every s (read from L2 per pass).
template <int RPW, int NS>
__device__ __forceinline__ void load_ct_frags(const float* __restrict__ C, int k, int cout,
                                              int cin, float (&a)[RPW][NS]) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int le = lane & 15, lg = lane >> 4;
#pragma unroll
    for (int j = 0; j < RPW; ++j)
#pragma unroll
        for (int s = 0; s < NS; ++s)
            a[j][s] = C[(static_cast<int64_t>(k) * cout + lg * NS + s) * cin + 16 * (wave + 4 * j) + le];
}

// s^l of every m-first slot of a canonical representation with lmax L, from s.
template <int L>
__device__ __forceinline__ void slot_powers(float s, float (&pw)[(L + 1) * (L + 1)]) {
    float p[L + 1];
    p[0] = 1.0f;
#pragma unroll
    for (int l = 1; l <= L; ++l) p[l] = p[l - 1] * s;
#pragma unroll
    for (int j = 0; j < (L + 1) * (L + 1); ++j) pw[j] = p[SlotL<L>::l[j]];
}

// Rows (e, c) of a tile rotated into the m-first frame with per-edge matrices
// read by wave-uniform (scalar) loads; thread t owns rows q = t + kThreads j,
// whose edge e = q / CH is the same for the whole wave (CH % 64 == 0).
// out[j][i] = s_e^l_i sum_d rows(e, c)[d] R_e[d, i]; padding edges give zeros.
template <int CH, int L>
__device__ __forceinline__ void rotate_rows_uniform(const float* __restrict__ src,
                                                    const float* __restrict__ R, int64_t e0,
                                                    int64_t E, const TileEdge* sE,
                                                    float (&out)[kNE * CH / kThreads][(L + 1) * (L + 1)]) {
    constexpr int D = (L + 1) * (L + 1), NR = kNE * CH / kThreads;
    static_assert(CH % 64 == 0, "one edge per wave and row");
    const int wv = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int j = 0; j < NR; ++j) {
        const int q = wv * 64 + lane + kThreads * j;
        const int e = (wv * 64 + kThreads * j) / CH, c = q % CH;
        if (e0 + e < E) {
            const float* row = src + ((e0 + e) * CH + c) * D;
            const float* re = R + (e0 + e) * D * D;
            float v[D], pw[D];
#pragma unroll
            for (int d = 0; d < D; ++d) v[d] = row[d];
            slot_powers<L>(sE[e].s, pw);
#pragma unroll
            for (int i = 0; i < D; ++i) {
                float acc = 0.0f;
#pragma unroll
                for (int d = 0; d < D; ++d) acc += v[d] * re[d * D + i];
                out[j][i] = acc * pw[i];
            }
        } else {
#pragma unroll
            for (int i = 0; i < D; ++i) out[j][i] = 0.0f;
        }
    }
}

// Backward, part 1: H_k = C_k^T gd on the matrix cores, one rank component per
// pass; in registers dfs = sum_k M_ek^T H_k and the per-edge radial gradient
// dF_e[k, w] = sum_ci fs H_k; then dx = s^l dfs P^T.  Two workgroups share a
// CU: C_k^T streams from L2 (the next component is prefetched during the
// current pass), Q is read with wave-uniform loads, fs is built directly in
// the accumulator layout, and LDS holds the gd tile, P and the dF partials.
template <int CIN, int COUT, int LIN, int LOUT, int K>
__global__ void __launch_bounds__(kThreads, 2)
k_ewc_bwd_x(feq_binning B, int64_t E, int64_t ntiles, const float* __restrict__ gy,
            const float* __restrict__ x, const float* __restrict__ P, const float* __restrict__ Q,
            const float* __restrict__ dist, const float* __restrict__ C,
            const float* __restrict__ F, float* __restrict__ gx, float* __restrict__ dFe) {
    using T = Canon<LIN, LOUT>;
    constexpr int DIN = T::DIN, DOUT = T::DOUT, WD = T::WD, KW = K * WD;
    constexpr int GS = 16 * DOUT + 1;     // gd rows
    constexpr int XS = CIN * DIN + 1;     // dx staging per edge
    constexpr int RPW = CIN / 64, NS = COUT / 4, NRG = kNE * COUT / kThreads;
    constexpr int GBIG = COUT * GS > kNE * XS ? COUT * GS : kNE * XS;
    static_assert(CIN % 64 == 0 && COUT % 64 == 0, "unsupported channel counts");
    extern __shared__ float4 smem4[];
    float* sG = reinterpret_cast<float*>(smem4);   // gd tile, later dx staging
    float* sDF = sG + GBIG;                        // dF_e partials per wave
    float* sP = sDF + 4 * K * kNE * WD;
    float* sFe = sP + kNE * DIN * DIN;
    TileEdge* sE = reinterpret_cast<TileEdge*>(sFe + kNE * KW);

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int le = lane & 15, lg = lane >> 4;
    const int wv = __builtin_amdgcn_readfirstlane(wave);

    for (int64_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
        const int64_t e0 = tile * kNE;
        __syncthreads();   // the previous tile's readers of the LDS tiles are done
        {
            BlockRegs<kNE * DIN * DIN> pr;
            pr.load(P, e0 * DIN * DIN, E * DIN * DIN);
            pr.store(sP);
        }
        if (tid < kNE) {
            TileEdge te;
            te.valid = (e0 + tid) < E;
            const float r = te.valid ? dist[e0 + tid] : 1.0f;
            const EdgeBin eb = edge_bin(r, B);
            te.lo = eb.lo;
            te.t = eb.t;
            te.s = r / (r + B.sh_scale);
            sE[tid] = te;
        }
        __syncthreads();
        interp_tile<KW>(sE, F, sFe);
        {
            float gdr[NRG][DOUT];
            rotate_rows_uniform<COUT, LOUT>(gy, Q, e0, E, sE, gdr);
#pragma unroll
            for (int j = 0; j < NRG; ++j) {
                const int e = (wv * 64 + kThreads * j) / COUT;
                const int co = (wv * 64 + lane + kThreads * j) % COUT;
#pragma unroll
                for (int o = 0; o < DOUT; ++o) sG[co * GS + 16 * o + e] = gdr[j][o];
            }
        }
        float pin[DIN];
        slot_powers<LIN>(sE[le].s, pin);
        float fsr[RPW][4][DIN];
        {
            LaneRows<CIN, DIN> xr;
            xr.load(x, e0, E);
            const float* pe = sP + le * DIN * DIN;
#pragma unroll
            for (int j = 0; j < RPW; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r)
#pragma unroll
                    for (int i = 0; i < DIN; ++i) {
                        float acc = 0.0f;
#pragma unroll
                        for (int d = 0; d < DIN; ++d) acc += xr.v[j][r][d] * pe[d * DIN + i];
                        fsr[j][r][i] = acc * pin[i];
                    }
        }
        float a_cur[RPW][NS];
        __syncthreads();   // gd tile complete

        float dfs[RPW][4][DIN];
#pragma unroll
        for (int j = 0; j < RPW; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int i = 0; i < DIN; ++i) dfs[j][r][i] = 0.0f;
#pragma unroll 1
        for (int k = 0; k < K; ++k) {
            load_ct_frags<RPW, NS>(C, k, COUT, CIN, a_cur);
            v4f accH[RPW][DOUT];
#pragma unroll
            for (int j = 0; j < RPW; ++j)
#pragma unroll
                for (int o = 0; o < DOUT; ++o) accH[j][o] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
            float b[2][DOUT];
#pragma unroll
            for (int o = 0; o < DOUT; ++o) b[0][o] = sG[lg * NS * GS + le + 16 * o];
#pragma unroll
            for (int s = 0; s < NS; ++s) {
                if (s + 1 < NS) {
                    const float* row = sG + (lg * NS + s + 1) * GS + le;
#pragma unroll
                    for (int o = 0; o < DOUT; ++o) b[(s + 1) & 1][o] = row[16 * o];
                }
#pragma unroll
                for (int j = 0; j < RPW; ++j)
#pragma unroll
                    for (int o = 0; o < DOUT; ++o)
                        accH[j][o] = mfma(a_cur[j][s], b[s & 1][o], accH[j][o]);
                __builtin_amdgcn_sched_barrier(0);
            }
            float fk[WD], pf[WD];
#pragma unroll
            for (int w = 0; w < WD; ++w) {
                fk[w] = sFe[le * KW + k * WD + w];
                pf[w] = 0.0f;
            }
#pragma unroll
            for (int j = 0; j < RPW; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r)
#pragma unroll
                    for (int t = 0; t < T::NT; ++t) {
                        const Term tm = T::terms[t];
                        const float h = accH[j][tm.o][r];
                        const float c = tm.neg ? -fk[tm.w] : fk[tm.w];
                        dfs[j][r][tm.i] += c * h;
                        pf[tm.w] += (tm.neg ? -fsr[j][r][tm.i] : fsr[j][r][tm.i]) * h;
                    }
            // sum over the 4 lane groups: the wave's rows of this edge
#pragma unroll
            for (int w = 0; w < WD; ++w) {
                float v = pf[w];
                v += __shfl_xor(v, 16, 64);
                v += __shfl_xor(v, 32, 64);
                if (lg == 0) sDF[((wave * K + k) * kNE + le) * WD + w] = v;
            }
        }
        __syncthreads();   // dF partials complete; gd no longer needed
        const int64_t nval = E - e0 < kNE ? E - e0 : kNE;
        for (int q = tid; q < nval * KW; q += kThreads) {
            const int e = q / KW, kw = q % KW, k = kw / WD, w = kw % WD;
            float acc = 0.0f;
#pragma unroll
            for (int v = 0; v < 4; ++v) acc += sDF[((v * K + k) * kNE + e) * WD + w];
            dFe[(e0 + e) * KW + kw] = acc;
        }
        // dx = s^l dfs P^T, staged through LDS for coalesced stores
        {
            const float* pe = sP + le * DIN * DIN;
#pragma unroll
            for (int j = 0; j < RPW; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int ci = 16 * (wave + 4 * j) + 4 * lg + r;
                    float ds[DIN];
#pragma unroll
                    for (int i = 0; i < DIN; ++i) ds[i] = dfs[j][r][i] * pin[i];
#pragma unroll
                    for (int d = 0; d < DIN; ++d) {
                        float acc = 0.0f;
#pragma unroll
                        for (int i = 0; i < DIN; ++i) acc += ds[i] * pe[d * DIN + i];
                        sG[le * XS + ci * DIN + d] = acc;
                    }
                }
        }
        __syncthreads();
        float* xt = gx + e0 * CIN * DIN;
        if (nval == kNE) {
#pragma unroll
            for (int m = 0; m < kNE * CIN * DIN / kThreads; ++m) {
                const int q = tid + kThreads * m;
                xt[q] = sG[(q / (CIN * DIN)) * XS + q % (CIN * DIN)];
            }
        } else {
            for (int q = tid; q < nval * CIN * DIN; q += kThreads)
                xt[q] = sG[(q / (CIN * DIN)) * XS + q % (CIN * DIN)];
        }
    }
}

// Backward, part 2: dC_k += U_k fs^T with U_k[co][16 i + e] = (M_ek^T gd)[co][i]
// for rank component k; one partial per workgroup.  Two workgroups share a
// CU: P and Q are read with wave-uniform loads, gd stays in the registers of
// the threads that build U_k, and LDS holds only the fs tile and one U_k tile
// (row stride 16 Din + 4 floats, so each 16-lane quarter of a 128-bit operand
// read covers all 64 banks once).  The reduction index is ordered c = KL lg +
// s: lane group lg covers KL = 4 Din consecutive columns, read four at a time.
template <int CIN, int COUT, int LIN, int LOUT, int K>
__global__ void __launch_bounds__(kThreads, 2)
k_ewc_bwd_c(feq_binning B, int64_t E, int64_t ntiles, const float* __restrict__ gy,
            const float* __restrict__ x, const float* __restrict__ P, const float* __restrict__ Q,
            const float* __restrict__ dist, const float* __restrict__ F,
            float* __restrict__ dC_part) {
    using T = Canon<LIN, LOUT>;
    constexpr int DIN = T::DIN, DOUT = T::DOUT, WD = T::WD, KW = K * WD;
    constexpr int RS = 16 * DIN + 4;
    constexpr int KL = 4 * DIN, NG = DIN;       // columns per lane group, float4 groups
    constexpr int CT = (COUT / 16) * (CIN / 16);
    constexpr int CTPW = CT / 4;
    constexpr int NRX = kNE * CIN / kThreads, NRG = kNE * COUT / kThreads;
    static_assert(CT % 4 == 0 && CIN % 64 == 0 && COUT % 64 == 0, "unsupported channel counts");
    extern __shared__ float4 smem4[];
    float* sf = reinterpret_cast<float*>(smem4);   // CIN x RS, fs[ci][16 i + e]
    float* sU = sf + CIN * RS;                     // COUT x RS, U_k[co][16 i + e]
    float* sFe = sU + COUT * RS;
    TileEdge* sE = reinterpret_cast<TileEdge*>(sFe + kNE * KW);

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int le = lane & 15, lg = lane >> 4;
    const int wv = __builtin_amdgcn_readfirstlane(wave);
    v4f accC[K][CTPW];
#pragma unroll
    for (int k = 0; k < K; ++k)
#pragma unroll
        for (int j = 0; j < CTPW; ++j) accC[k][j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};

    for (int64_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
        const int64_t e0 = tile * kNE;
        __syncthreads();   // the previous tile's readers of the LDS tiles are done
        if (tid < kNE) {
            TileEdge te;
            te.valid = (e0 + tid) < E;
            const float r = te.valid ? dist[e0 + tid] : 1.0f;
            const EdgeBin eb = edge_bin(r, B);
            te.lo = eb.lo;
            te.t = eb.t;
            te.s = r / (r + B.sh_scale);
            sE[tid] = te;
        }
        __syncthreads();
        interp_tile<KW>(sE, F, sFe);
        {
            float fsr[NRX][DIN];
            rotate_rows_uniform<CIN, LIN>(x, P, e0, E, sE, fsr);
#pragma unroll
            for (int j = 0; j < NRX; ++j) {
                const int e = (wv * 64 + kThreads * j) / CIN, c = (wv * 64 + lane + kThreads * j) % CIN;
#pragma unroll
                for (int i = 0; i < DIN; ++i) sf[c * RS + 16 * i + e] = fsr[j][i];
            }
        }
        float gdr[NRG][DOUT];
        rotate_rows_uniform<COUT, LOUT>(gy, Q, e0, E, sE, gdr);
#pragma unroll
        for (int k = 0; k < K; ++k) {
            if (k > 0) __syncthreads();   // the previous U_k is no longer read
#pragma unroll
            for (int j = 0; j < NRG; ++j) {
                const int e = (wv * 64 + kThreads * j) / COUT, co = (wv * 64 + lane + kThreads * j) % COUT;
                const float* fe = sFe + e * KW + k * WD;
                float u[DIN];
#pragma unroll
                for (int i = 0; i < DIN; ++i) u[i] = 0.0f;
#pragma unroll
                for (int t = 0; t < T::NT; ++t) {
                    const Term tm = T::terms[t];
                    const float c = tm.neg ? -fe[tm.w] : fe[tm.w];
                    u[tm.i] += c * gdr[j][tm.o];
                }
#pragma unroll
                for (int i = 0; i < DIN; ++i) sU[co * RS + 16 * i + e] = u[i];
            }
            __syncthreads();   // U_k (and at k = 0 the fs tile) complete
#pragma unroll
            for (int g = 0; g < NG; ++g) {
#pragma unroll
                for (int j = 0; j < CTPW; ++j) {
                    const int tt = wave + 4 * j;
                    const int rbA = tt / (CIN / 16), cbB = tt % (CIN / 16);
                    const float4 aq = *reinterpret_cast<const float4*>(
                        sU + (16 * rbA + le) * RS + KL * lg + 4 * g);
                    const float4 bq = *reinterpret_cast<const float4*>(
                        sf + (16 * cbB + le) * RS + KL * lg + 4 * g);
                    accC[k][j] = mfma(aq.x, bq.x, accC[k][j]);
                    accC[k][j] = mfma(aq.y, bq.y, accC[k][j]);
                    accC[k][j] = mfma(aq.z, bq.z, accC[k][j]);
                    accC[k][j] = mfma(aq.w, bq.w, accC[k][j]);
                }
            }
        }
    }
    float* part = dC_part + static_cast<int64_t>(blockIdx.x) * K * COUT * CIN;
#pragma unroll
    for (int k = 0; k < K; ++k)
#pragma unroll
        for (int j = 0; j < CTPW; ++j) {
            const int tt = wave + 4 * j;
            const int rbA = tt / (CIN / 16), cbB = tt % (CIN / 16);
#pragma unroll
            for (int r = 0; r < 4; ++r)
                part[(k * COUT + 16 * rbA + 4 * lg + r) * CIN + 16 * cbB + le] = accC[k][j][r];
        }
}

int device_cus() {
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) == hipSuccess) {
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
            cus = v;
    }
    return cus;
}

int grid_for(int64_t ntiles, int per_cu) {
    const int64_t g = static_cast<int64_t>(device_cus()) * per_cu;
    return static_cast<int>(ntiles < g ? ntiles : g);
}

int set_lds(const void* kern, size_t lds) {
    if (lds > 160 * 1024) return fail(FEQ_ERR_UNSUPPORTED, "kernel needs %zu B of LDS", lds);
    if (lds > 64 * 1024)
        FEQ_HIP(hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                    static_cast<int>(lds)));
    return FEQ_OK;
}

template <int CIN, int COUT, int LIN, int LOUT, int K>
constexpr size_t fwd_lds() {
    using T = Canon<LIN, LOUT>;
    constexpr size_t FS = 16 * T::DIN + 1, YS = COUT * T::DOUT + 1;
    constexpr size_t BIG = CIN * FS > kNE * YS ? CIN * FS : kNE * YS;
    return 4 * (BIG + kNE * T::DIN * T::DIN + kNE * T::DOUT * T::DOUT + kNE * T::DIN +
                kNE * T::DOUT + kNE * K * T::WD) +
           kNE * sizeof(TileEdge);
}

template <int CIN, int COUT, int LIN, int LOUT, int K>
constexpr size_t bwd_x_lds() {
    using T = Canon<LIN, LOUT>;
    constexpr size_t GS = 16 * T::DOUT + 1, XS = CIN * T::DIN + 1;
    constexpr size_t GBIG = COUT * GS > kNE * XS ? COUT * GS : kNE * XS;
    return 4 * (GBIG + 4 * K * kNE * T::WD + kNE * T::DIN * T::DIN + kNE * K * T::WD) +
           kNE * sizeof(TileEdge);
}

template <int CIN, int COUT, int LIN, int LOUT, int K>
constexpr size_t bwd_c_lds() {
    using T = Canon<LIN, LOUT>;
    constexpr size_t RS = 16 * T::DIN + 4;
    return 4 * (CIN * RS + COUT * RS + kNE * K * T::WD) + kNE * sizeof(TileEdge);
}

template <int CIN, int COUT, int LIN, int LOUT, int K>
int launch_fwd(const feq_binning& B, int64_t E, const float* x, const float* P, const float* Q,
               const float* dist, const float* C, const float* F, float* y, hipStream_t s) {
    constexpr size_t lds = fwd_lds<CIN, COUT, LIN, LOUT, K>();
    static_assert(lds <= 80 * 1024, "two forward workgroups must fit one CU's LDS");
    auto kern = k_ewc_fwd<CIN, COUT, LIN, LOUT, K>;
    if (int rc = set_lds(reinterpret_cast<const void*>(kern), lds)) return rc;
    const int64_t ntiles = ceil_div(E, kNE);
    FEQ_LAUNCH("k_ewc_fwd", kern, dim3(grid_for(ntiles, 2)), dim3(kThreads), lds, s, B, E, ntiles,
               x, P, Q, dist, C, F, y);
    return FEQ_OK;
}

template <int CIN, int COUT, int LIN, int LOUT, int K>
size_t bwd_ws(const feq_binning& B, int64_t E) {
    using T = Canon<LIN, LOUT>;
    const int G = grid_for(ceil_div(E, kNE), 2);
    const int64_t kw = static_cast<int64_t>(K) * T::WD, ncc = static_cast<int64_t>(K) * COUT * CIN;
    return align_up(4 * E * kw, 256) + align_up(4 * static_cast<size_t>(G) * ncc, 256) +
           4 * ew_tail_floats(B, static_cast<int>(kw), E, G, ncc) + 1024;
}

// Backward launches: input gradient and dF_e, channel-pattern partials, then
// the shared tail (binned radial-function gradient, distance gradient, sums).
template <int CIN, int COUT, int LIN, int LOUT, int K>
int launch_bwd(const feq_layout& L, const feq_binning& B, int64_t E, const float* gy,
               const float* x, const float* P, const float* Q, const float* dist, const float* C,
               const float* F, float* gx, float* gC, float* gF, float* gdist, char* ws,
               size_t ws_bytes, hipStream_t s) {
    using T = Canon<LIN, LOUT>;
    constexpr size_t xlds = bwd_x_lds<CIN, COUT, LIN, LOUT, K>();
    constexpr size_t clds = bwd_c_lds<CIN, COUT, LIN, LOUT, K>();
    const int kw = K * T::WD;
    if (!ew_tail_supported(B, kw)) return -1;
    auto kx = k_ewc_bwd_x<CIN, COUT, LIN, LOUT, K>;
    auto kc = k_ewc_bwd_c<CIN, COUT, LIN, LOUT, K>;
    const int64_t ntiles = ceil_div(E, kNE);
    const int Gx = grid_for(ntiles, xlds <= 80 * 1024 ? 2 : 1);
    const int G = grid_for(ntiles, clds <= 80 * 1024 ? 2 : 1);
    const int64_t ncc = static_cast<int64_t>(K) * COUT * CIN;
    Carver cv(ws);
    float* dFe = cv.take<float>(E * kw);
    float* dCp = cv.take<float>(static_cast<size_t>(G) * ncc);
    float* tail = cv.take<float>(ew_tail_floats(B, kw, E, G, ncc));
    if (cv.used > ws_bytes) return fail(FEQ_ERR_WORKSPACE, "edgewise workspace too small");
    if (int rc = set_lds(reinterpret_cast<const void*>(kx), xlds)) return rc;
    FEQ_LAUNCH("k_ewc_bwd_x", kx, dim3(Gx), dim3(kThreads), xlds, s, B, E, ntiles, gy, x, P, Q,
               dist, C, F, gx, dFe);
    if (int rc = set_lds(reinterpret_cast<const void*>(kc), clds)) return rc;
    FEQ_LAUNCH("k_ewc_bwd_c", kc, dim3(G), dim3(kThreads), clds, s, B, E, ntiles, gy, x, P, Q,
               dist, F, dCp);
    return ew_tail(L, B, K, E, dist, F, dFe, dCp, G, ncc, gC, gF, gdist, tail, s);
}

// The layout is the canonical (0..lin) x (0..lout) pair the kernels are built for.
bool is_canonical(const feq_layout& L, int lin, int lout) {
    int32_t li[FEQ_MAX_BLOCKS], lo[FEQ_MAX_BLOCKS];
    for (int i = 0; i <= lin; ++i) li[i] = i;
    for (int i = 0; i <= lout; ++i) lo[i] = i;
    feq_layout ref;
    if (feq_layout_init(&ref, li, lin + 1, lo, lout + 1, L.cin, L.cout) != FEQ_OK) return false;
    if (ref.din != L.din || ref.dout != L.dout || ref.wdim != L.wdim || ref.nblocks != L.nblocks)
        return false;
    for (int k = 0; k < L.nblocks; ++k)
        for (int c = 0; c < 6; ++c)
            if (ref.blk[k][c] != L.blk[k][c]) return false;
    for (int s = 0; s < L.din; ++s)
        if (ref.lslot_in[s] != L.lslot_in[s]) return false;
    for (int s = 0; s < L.dout; ++s)
        if (ref.lslot_out[s] != L.lslot_out[s]) return false;
    return true;
}

}  // namespace

// Shapes with a compiled fast path: (Cin, Cout, Lin, Lout), rank 4.
#define FEQ_EW_SHAPES(X) \
    X(64, 64, 2, 2)      \
    X(32, 64, 1, 2)

size_t ew_mfma_bwd_workspace(const feq_layout& L, const feq_binning& B, int rank, int64_t E) {
    if (rank != 4) return 0;
#define FEQ_WS(ci, co, li, lo)                                                   \
    if (L.cin == ci && L.cout == co && is_canonical(L, li, lo) && (ci) % 64 == 0) \
        return bwd_ws<ci, co, li, lo, 4>(B, E);
    FEQ_EW_SHAPES(FEQ_WS)
#undef FEQ_WS
    return 0;
}

int ew_mfma_fwd(const feq_layout& L, const feq_binning& B, int rank, int64_t E, const float* x,
                const float* P, const float* Q, const float* dist, const float* C, const float* F,
                float* y, hipStream_t s) {
    if (rank != 4) return -1;
#define FEQ_FWD(ci, co, li, lo)                                \
    if (L.cin == ci && L.cout == co && is_canonical(L, li, lo)) \
        return launch_fwd<ci, co, li, lo, 4>(B, E, x, P, Q, dist, C, F, y, s);
    FEQ_EW_SHAPES(FEQ_FWD)
#undef FEQ_FWD
    return -1;
}

int ew_mfma_bwd(const feq_layout& L, const feq_binning& B, int rank, int64_t E, const float* gy,
                const float* x, const float* P, const float* Q, const float* dist, const float* C,
                const float* F, float* gx, float* gC, float* gF, float* gdist, void* ws,
                size_t ws_bytes, hipStream_t s) {
    if (rank != 4 || !gx) return -1;
    char* w = static_cast<char*>(ws);
#define FEQ_BWD(ci, co, li, lo)                                                                  \
    if constexpr ((ci) % 64 == 0) {                                                              \
        if (L.cin == ci && L.cout == co && is_canonical(L, li, lo))                              \
            return launch_bwd<ci, co, li, lo, 4>(L, B, E, gy, x, P, Q, dist, C, F, gx, gC, gF,   \
                                                 gdist, w, ws_bytes, s);                         \
    }
    FEQ_EW_SHAPES(FEQ_BWD)
#undef FEQ_BWD
    return -1;
}

}  // namespace feq

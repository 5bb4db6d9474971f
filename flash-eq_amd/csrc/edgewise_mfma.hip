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

#include <array>

namespace feq {
namespace {

typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kNE = 16;       // edges per tile
constexpr int kThreads = 256;

__device__ __forceinline__ v4f mfma(float a, float b, v4f c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// ---- compile-time m-first layout of a canonical (lvals = 0..L) pair --------
struct Term {
    int o, i, w, neg;
};

template <int LIN, int LOUT>
struct Canon {
    static constexpr int DIN = (LIN + 1) * (LIN + 1);
    static constexpr int DOUT = (LOUT + 1) * (LOUT + 1);
    static constexpr int MMIN = LIN < LOUT ? LIN : LOUT;
    static constexpr int nin(int m) { return LIN - m + 1; }
    static constexpr int nout(int m) { return LOUT - m + 1; }
    static constexpr int in_off(int m) {
        int o = 0;
        for (int q = 0; q < m; ++q) o += (q ? 2 : 1) * nin(q);
        return o;
    }
    static constexpr int out_off(int m) {
        int o = 0;
        for (int q = 0; q < m; ++q) o += (q ? 2 : 1) * nout(q);
        return o;
    }
    static constexpr int w_off(int m) {
        int o = 0;
        for (int q = 0; q < m; ++q) o += (q ? 2 : 1) * nin(q) * nout(q);
        return o;
    }
    static constexpr int WD = w_off(MMIN + 1);
    static constexpr int count() {
        int n = 0;
        for (int m = 0; m <= MMIN; ++m) n += (m ? 4 : 1) * nin(m) * nout(m);
        return n;
    }
    static constexpr int NT = count();
    static constexpr std::array<Term, NT> make_terms() {
        std::array<Term, NT> t{};
        int n = 0;
        for (int m = 0; m <= MMIN; ++m) {
            const int ni = nin(m), no = nout(m), io = in_off(m), oo = out_off(m), wo = w_off(m);
            for (int o = 0; o < no; ++o)
                for (int i = 0; i < ni; ++i) {
                    if (m == 0) {
                        t[n++] = Term{oo + o, io + i, wo + o * ni + i, 0};
                    } else {
                        const int wa = wo + 2 * (o * ni + i);
                        const int ro = oo + 2 * o, im_o = ro + 1, ri = io + 2 * i, im_i = ri + 1;
                        t[n++] = Term{ro, ri, wa, 0};          // re += a f_re
                        t[n++] = Term{ro, im_i, wa + 1, 0};    // re += b f_im
                        t[n++] = Term{im_o, im_i, wa, 0};      // im += a f_im
                        t[n++] = Term{im_o, ri, wa + 1, 1};    // im -= b f_re
                    }
                }
        }
        return t;
    }
    static constexpr std::array<Term, NT> terms = make_terms();
};

// l of every m-first component of a canonical representation with lmax L
template <int L>
struct SlotL {
    static constexpr std::array<int, (L + 1) * (L + 1)> make() {
        std::array<int, (L + 1) * (L + 1)> v{};
        int s = 0;
        for (int l = 0; l <= L; ++l) v[s++] = l;
        for (int m = 1; m <= L; ++m)
            for (int l = m; l <= L; ++l) {
                v[s++] = l;
                v[s++] = l;
            }
        return v;
    }
    static constexpr std::array<int, (L + 1) * (L + 1)> l = make();
};

struct TileEdge {
    int lo;
    float t;
    float s;
    int valid;
};

// Per-edge bins, solid-harmonic powers and F_e of one tile; P, Q tiles.
template <int LIN, int LOUT, int K>
__device__ void stage_tile(const feq_binning& B, int64_t E, int64_t e0,
                           const float* __restrict__ P, const float* __restrict__ Q,
                           const float* __restrict__ dist, const float* __restrict__ F,
                           float* sP, float* sQ, TileEdge* sE, float* sSin, float* sSout,
                           float* sFe) {
    using T = Canon<LIN, LOUT>;
    constexpr int DIN = T::DIN, DOUT = T::DOUT, KW = K * T::WD;
    const int tid = threadIdx.x;
    for (int q = tid; q < kNE * DIN * DIN; q += kThreads)
        sP[q] = (e0 + q / (DIN * DIN) < E) ? P[e0 * DIN * DIN + q] : 0.0f;
    for (int q = tid; q < kNE * DOUT * DOUT; q += kThreads)
        sQ[q] = (e0 + q / (DOUT * DOUT) < E) ? Q[e0 * DOUT * DOUT + q] : 0.0f;
    if (tid < kNE) {
        TileEdge te;
        te.valid = (e0 + tid) < E;
        const float r = te.valid ? dist[e0 + tid] : 1.0f;
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
    __syncthreads();
    for (int q = tid; q < kNE * KW; q += kThreads) {
        const int e = q / KW, rest = q % KW;
        const TileEdge te = sE[e];
        const float* flo = F + static_cast<int64_t>(te.lo) * KW;
        sFe[q] = lerp_bins(flo[rest], flo[KW + rest], te.t);
    }
}

// fs[ci][16 i + e] = s^l_i sum_d x[e, ci, d] P[e, d, i]
template <int CIN, int DIN>
__device__ void rotate_in(int64_t E, int64_t e0, const float* __restrict__ x, const float* sP,
                          const float* sSin, float* sf, int fs) {
    for (int q = threadIdx.x; q < kNE * CIN; q += kThreads) {
        const int e = q / CIN, ci = q % CIN;
        float xv[DIN];
        if (e0 + e < E) {
            const float* xr = x + ((e0 + e) * CIN + ci) * DIN;
#pragma unroll
            for (int d = 0; d < DIN; ++d) xv[d] = xr[d];
        } else {
#pragma unroll
            for (int d = 0; d < DIN; ++d) xv[d] = 0.0f;
        }
        const float* pe = sP + e * DIN * DIN;
#pragma unroll
        for (int i = 0; i < DIN; ++i) {
            float acc = 0.0f;
#pragma unroll
            for (int d = 0; d < DIN; ++d) acc += xv[d] * pe[d * DIN + i];
            sf[ci * fs + 16 * i + e] = acc * sSin[e * DIN + i];
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

template <int CIN, int COUT, int LIN, int LOUT, int K>
__global__ void __launch_bounds__(kThreads)
k_ewc_fwd(feq_binning B, int64_t E, int64_t ntiles, const float* __restrict__ x,
          const float* __restrict__ P, const float* __restrict__ Q,
          const float* __restrict__ dist, const float* __restrict__ C,
          const float* __restrict__ F, float* __restrict__ y) {
    using T = Canon<LIN, LOUT>;
    constexpr int DIN = T::DIN, DOUT = T::DOUT, WD = T::WD, KW = K * WD;
    constexpr int FS = 16 * DIN + 1;
    constexpr int YS = COUT * DOUT + 1;
    constexpr int RB = COUT / 16, RPW = RB / 4, NS = CIN / 4;
    constexpr int BIG = CIN * FS > kNE * YS ? CIN * FS : kNE * YS;
    static_assert(COUT % 64 == 0 && CIN % 16 == 0, "unsupported channel counts");
    extern __shared__ float4 smem4[];
    float* sCf = reinterpret_cast<float*>(smem4);  // K x RB x NS x 64 A fragments
    float* sf = sCf + K * RB * NS * 64;            // fs tile, later the y staging tile
    float* sP = sf + BIG;
    float* sQ = sP + kNE * DIN * DIN;
    float* sSin = sQ + kNE * DOUT * DOUT;
    float* sSout = sSin + kNE * DIN;
    float* sFe = sSout + kNE * DOUT;
    TileEdge* sE = reinterpret_cast<TileEdge*>(sFe + kNE * KW);

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int le = lane & 15, lg = lane >> 4;
    stage_frags<K, RB, NS, false>(C, COUT, CIN, sCf);

    for (int64_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
        const int64_t e0 = tile * kNE;
        __syncthreads();
        stage_tile<LIN, LOUT, K>(B, E, e0, P, Q, dist, F, sP, sQ, sE, sSin, sSout, sFe);
        __syncthreads();
        rotate_in<CIN, DIN>(E, e0, x, sP, sSin, sf, FS);
        __syncthreads();

        v4f acc[RPW][K][DIN];
#pragma unroll
        for (int j = 0; j < RPW; ++j)
#pragma unroll
            for (int k = 0; k < K; ++k)
#pragma unroll
                for (int i = 0; i < DIN; ++i) acc[j][k][i] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 2
        for (int s = 0; s < NS; ++s) {
            float b[DIN];
            const float* row = sf + (4 * s + lg) * FS + le;
#pragma unroll
            for (int i = 0; i < DIN; ++i) b[i] = row[16 * i];
#pragma unroll
            for (int j = 0; j < RPW; ++j)
#pragma unroll
                for (int k = 0; k < K; ++k) {
                    const float a = sCf[((k * RB + wave + 4 * j) * NS + s) * 64 + lane];
#pragma unroll
                    for (int i = 0; i < DIN; ++i) acc[j][k][i] = mfma(a, b[i], acc[j][k][i]);
                }
        }
        // epilogue: lane (edge le, rows 16(wave+4j) + 4 lg + r)
        float yv[RPW][DOUT][4];
#pragma unroll
        for (int j = 0; j < RPW; ++j)
#pragma unroll
            for (int o = 0; o < DOUT; ++o)
#pragma unroll
                for (int r = 0; r < 4; ++r) yv[j][o][r] = 0.0f;
#pragma unroll
        for (int k = 0; k < K; ++k) {
            float fk[WD];
#pragma unroll
            for (int w = 0; w < WD; ++w) fk[w] = sFe[le * KW + k * WD + w];
#pragma unroll
            for (int t = 0; t < T::NT; ++t) {
                const Term tm = T::terms[t];
                const float c = tm.neg ? -fk[tm.w] : fk[tm.w];
#pragma unroll
                for (int j = 0; j < RPW; ++j)
#pragma unroll
                    for (int r = 0; r < 4; ++r) yv[j][tm.o][r] += c * acc[j][k][tm.i][r];
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
                    float a = 0.0f;
#pragma unroll
                    for (int o = 0; o < DOUT; ++o) a += yv[j][o][r] * qrow[o];
                    sf[le * YS + (16 * (wave + 4 * j) + 4 * lg + r) * DOUT + d] = a;
                }
        }
        __syncthreads();
        const int64_t nval = E - e0 < kNE ? E - e0 : kNE;
        float* yt = y + e0 * COUT * DOUT;
        for (int q = tid; q < nval * COUT * DOUT; q += kThreads) {
            const int e = q / (COUT * DOUT), rest = q % (COUT * DOUT);
            yt[q] = sf[e * YS + rest];
        }
    }
}

// ---------------------------------------------------------------------------
// gd[co][16 o + e] = s^l_o sum_d gy[e, co, d] Q[e, d, o]
template <int COUT, int DOUT>
__device__ void rotate_grad(int64_t E, int64_t e0, const float* __restrict__ gy, const float* sQ,
                            const float* sSout, float* sG, int gs) {
    for (int q = threadIdx.x; q < kNE * COUT; q += kThreads) {
        const int e = q / COUT, co = q % COUT;
        float gv[DOUT];
        if (e0 + e < E) {
            const float* gr = gy + ((e0 + e) * COUT + co) * DOUT;
#pragma unroll
            for (int d = 0; d < DOUT; ++d) gv[d] = gr[d];
        } else {
#pragma unroll
            for (int d = 0; d < DOUT; ++d) gv[d] = 0.0f;
        }
        const float* qe = sQ + e * DOUT * DOUT;
#pragma unroll
        for (int o = 0; o < DOUT; ++o) {
            float a = 0.0f;
#pragma unroll
            for (int d = 0; d < DOUT; ++d) a += gv[d] * qe[d * DOUT + o];
            sG[co * gs + 16 * o + e] = a * sSout[e * DOUT + o];
        }
    }
}

// Backward, part 1: H_k = C_k^T gd (MFMA), dfs = sum_k M_ek^T H_k and
// dF_e[k, w] = sum_ci fs H_k in registers, dx = s^l dfs P^T.
template <int CIN, int COUT, int LIN, int LOUT, int K>
__global__ void __launch_bounds__(kThreads)
k_ewc_bwd_x(feq_binning B, int64_t E, int64_t ntiles, const float* __restrict__ gy,
            const float* __restrict__ x, const float* __restrict__ P, const float* __restrict__ Q,
            const float* __restrict__ dist, const float* __restrict__ C,
            const float* __restrict__ F, float* __restrict__ gx, float* __restrict__ dFe) {
    using T = Canon<LIN, LOUT>;
    constexpr int DIN = T::DIN, DOUT = T::DOUT, WD = T::WD, KW = K * WD;
    constexpr int FS = 16 * DIN + 1;      // fs rows
    constexpr int GS = 16 * DOUT + 1;     // gd rows
    constexpr int XS = CIN * DIN + 1;     // dx staging per edge
    constexpr int HRB = CIN / 16, RPW = HRB / 4, NS = COUT / 4;
    constexpr int GBIG = COUT * GS > kNE * XS ? COUT * GS : kNE * XS;
    constexpr int DFN = 4 * K * kNE * WD;
    static_assert(CIN % 64 == 0 && COUT % 4 == 0, "unsupported channel counts");
    static_assert(DFN <= GBIG, "dF partials must fit the gd tile");
    extern __shared__ float4 smem4[];
    float* sCf = reinterpret_cast<float*>(smem4);  // K x HRB x NS x 64 fragments of C_k^T
    float* sf = sCf + K * HRB * NS * 64;           // CIN x FS
    float* sG = sf + CIN * FS;                     // gd tile; later dF partials and dx staging
    float* sP = sG + GBIG;
    float* sQ = sP + kNE * DIN * DIN;
    float* sSin = sQ + kNE * DOUT * DOUT;
    float* sSout = sSin + kNE * DIN;
    float* sFe = sSout + kNE * DOUT;
    TileEdge* sE = reinterpret_cast<TileEdge*>(sFe + kNE * KW);

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int le = lane & 15, lg = lane >> 4;
    stage_frags<K, HRB, NS, true>(C, COUT, CIN, sCf);

    for (int64_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
        const int64_t e0 = tile * kNE;
        __syncthreads();
        stage_tile<LIN, LOUT, K>(B, E, e0, P, Q, dist, F, sP, sQ, sE, sSin, sSout, sFe);
        __syncthreads();
        rotate_in<CIN, DIN>(E, e0, x, sP, sSin, sf, FS);
        rotate_grad<COUT, DOUT>(E, e0, gy, sQ, sSout, sG, GS);
        __syncthreads();
        v4f accH[RPW][K][DOUT];
#pragma unroll
        for (int j = 0; j < RPW; ++j)
#pragma unroll
            for (int k = 0; k < K; ++k)
#pragma unroll
                for (int o = 0; o < DOUT; ++o) accH[j][k][o] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 2
        for (int s = 0; s < NS; ++s) {
            float b[DOUT];
            const float* row = sG + (4 * s + lg) * GS + le;
#pragma unroll
            for (int o = 0; o < DOUT; ++o) b[o] = row[16 * o];
#pragma unroll
            for (int j = 0; j < RPW; ++j)
#pragma unroll
                for (int k = 0; k < K; ++k) {
                    const float a = sCf[((k * HRB + wave + 4 * j) * NS + s) * 64 + lane];
#pragma unroll
                    for (int o = 0; o < DOUT; ++o) accH[j][k][o] = mfma(a, b[o], accH[j][k][o]);
                }
        }
        __syncthreads();   // gd no longer needed: its tile holds the dF partials, then dx
        float dfs[RPW][DIN][4];
#pragma unroll
        for (int j = 0; j < RPW; ++j)
#pragma unroll
            for (int i = 0; i < DIN; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r) dfs[j][i][r] = 0.0f;
#pragma unroll
        for (int k = 0; k < K; ++k) {
            float fk[WD], pf[WD];
#pragma unroll
            for (int w = 0; w < WD; ++w) {
                fk[w] = sFe[le * KW + k * WD + w];
                pf[w] = 0.0f;
            }
#pragma unroll
            for (int j = 0; j < RPW; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float* frow = sf + (16 * (wave + 4 * j) + 4 * lg + r) * FS + le;
                    float fv[DIN];
#pragma unroll
                    for (int i = 0; i < DIN; ++i) fv[i] = frow[16 * i];
#pragma unroll
                    for (int t = 0; t < T::NT; ++t) {
                        const Term tm = T::terms[t];
                        const float h = accH[j][k][tm.o][r];
                        const float c = tm.neg ? -fk[tm.w] : fk[tm.w];
                        dfs[j][tm.i][r] += c * h;
                        pf[tm.w] += (tm.neg ? -fv[tm.i] : fv[tm.i]) * h;
                    }
                }
            // sum over the 4 lane groups: the wave's 16 ci rows of this edge
#pragma unroll
            for (int w = 0; w < WD; ++w) {
                float v = pf[w];
                v += __shfl_xor(v, 16, 64);
                v += __shfl_xor(v, 32, 64);
                pf[w] = v;
            }
            if (lg == 0) {
#pragma unroll
                for (int w = 0; w < WD; ++w) sG[((wave * K + k) * kNE + le) * WD + w] = pf[w];
            }
        }
        __syncthreads();
        const int64_t nval = E - e0 < kNE ? E - e0 : kNE;
        for (int q = tid; q < nval * KW; q += kThreads) {
            const int e = q / KW, kw = q % KW, k = kw / WD, w = kw % WD;
            float a = 0.0f;
#pragma unroll
            for (int v = 0; v < 4; ++v) a += sG[((v * K + k) * kNE + e) * WD + w];
            dFe[(e0 + e) * KW + kw] = a;
        }
        __syncthreads();
        // dx = s^l dfs P^T, staged through LDS for coalesced stores
        {
            const float* pe = sP + le * DIN * DIN;
            float si[DIN];
#pragma unroll
            for (int i = 0; i < DIN; ++i) si[i] = sSin[le * DIN + i];
#pragma unroll
            for (int j = 0; j < RPW; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int ci = 16 * (wave + 4 * j) + 4 * lg + r;
#pragma unroll
                    for (int d = 0; d < DIN; ++d) {
                        float a = 0.0f;
#pragma unroll
                        for (int i = 0; i < DIN; ++i) a += dfs[j][i][r] * si[i] * pe[d * DIN + i];
                        sG[le * XS + ci * DIN + d] = a;
                    }
                }
        }
        __syncthreads();
        float* xt = gx + e0 * CIN * DIN;
        for (int q = tid; q < nval * CIN * DIN; q += kThreads) {
            const int e = q / (CIN * DIN), rest = q % (CIN * DIN);
            xt[q] = sG[e * XS + rest];
        }
    }
}

// Backward, part 2: dC_k += U_k fs^T, U_k[co][16 i + e] = sum_t sign F_e[k, w] gd[co][16 o + e],
// accumulated over the workgroup's tiles; one partial per workgroup.
template <int CIN, int COUT, int LIN, int LOUT, int K>
__global__ void __launch_bounds__(kThreads)
k_ewc_bwd_c(feq_binning B, int64_t E, int64_t ntiles, const float* __restrict__ gy,
            const float* __restrict__ x, const float* __restrict__ P, const float* __restrict__ Q,
            const float* __restrict__ dist, const float* __restrict__ F,
            float* __restrict__ dC_part) {
    using T = Canon<LIN, LOUT>;
    constexpr int DIN = T::DIN, DOUT = T::DOUT, WD = T::WD, KW = K * WD;
    constexpr int FS = 16 * DIN + 1, GS = 16 * DOUT + 1;
    constexpr int CT = (COUT / 16) * (CIN / 16);
    constexpr int CTPW = CT / 4;
    static_assert(CT % 4 == 0, "dC tiles must split over 4 waves");
    extern __shared__ float4 smem4[];
    float* sf = reinterpret_cast<float*>(smem4);   // CIN x FS
    float* sG = sf + CIN * FS;                     // COUT x GS
    float* sU = sG + COUT * GS;                    // COUT x FS
    float* sP = sU + COUT * FS;
    float* sQ = sP + kNE * DIN * DIN;
    float* sSin = sQ + kNE * DOUT * DOUT;
    float* sSout = sSin + kNE * DIN;
    float* sFe = sSout + kNE * DOUT;
    TileEdge* sE = reinterpret_cast<TileEdge*>(sFe + kNE * KW);

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int le = lane & 15, lg = lane >> 4;
    v4f accC[K][CTPW];
#pragma unroll
    for (int k = 0; k < K; ++k)
#pragma unroll
        for (int j = 0; j < CTPW; ++j) accC[k][j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};

    for (int64_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
        const int64_t e0 = tile * kNE;
        __syncthreads();
        stage_tile<LIN, LOUT, K>(B, E, e0, P, Q, dist, F, sP, sQ, sE, sSin, sSout, sFe);
        __syncthreads();
        rotate_in<CIN, DIN>(E, e0, x, sP, sSin, sf, FS);
        rotate_grad<COUT, DOUT>(E, e0, gy, sQ, sSout, sG, GS);
#pragma unroll
        for (int k = 0; k < K; ++k) {
            __syncthreads();   // gd ready; previous readers of sU are done
            for (int q = tid; q < kNE * COUT; q += kThreads) {
                const int e = q / COUT, co = q % COUT;
                float g[DOUT], u[DIN];
#pragma unroll
                for (int o = 0; o < DOUT; ++o) g[o] = sG[co * GS + 16 * o + e];
#pragma unroll
                for (int i = 0; i < DIN; ++i) u[i] = 0.0f;
                const float* fe = sFe + e * KW + k * WD;
#pragma unroll
                for (int t = 0; t < T::NT; ++t) {
                    const Term tm = T::terms[t];
                    const float c = tm.neg ? -fe[tm.w] : fe[tm.w];
                    u[tm.i] += c * g[tm.o];
                }
#pragma unroll
                for (int i = 0; i < DIN; ++i) sU[co * FS + 16 * i + e] = u[i];
            }
            __syncthreads();
#pragma unroll
            for (int j = 0; j < CTPW; ++j) {
                const int tt = wave + 4 * j;
                const int rbA = tt / (CIN / 16), cbB = tt % (CIN / 16);
                const float* arow = sU + (16 * rbA + le) * FS + lg;
                const float* brow = sf + (16 * cbB + le) * FS + lg;
#pragma unroll 4
                for (int s = 0; s < 4 * DIN; ++s) accC[k][j] = mfma(arow[4 * s], brow[4 * s], accC[k][j]);
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

// Binned radial-function gradient and distance gradient from dF_e.
// Each workgroup owns a contiguous edge chunk; wave v keeps its own
// histogram hist_v[bin][k*wdim + w] in LDS and walks its edges in order,
// so every sum has a fixed order.  dr_e = dt/dr sum (F[hi]-F[lo]) dF_e
// + [l>0 pairs] sigma/(r(r+sigma)) sum (l_i+l_o) F_e dF_e.
__global__ void __launch_bounds__(kThreads)
k_ewm_bins(feq_layout L, feq_binning B, int K, int64_t E, int64_t chunk,
           const float* __restrict__ dist, const float* __restrict__ F,
           const float* __restrict__ dFe, float* __restrict__ gdist, float* __restrict__ hist_part) {
    extern __shared__ float sh[];
    const int kw = K * L.wdim;
    const int nb1 = B.num_bins + 1;
    const int hsz = nb1 * kw;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int* fl = reinterpret_cast<int*>(sh + 4 * hsz);  // l_in + l_out per weight
    if (threadIdx.x == 0) {
        for (int k = 0; k < L.nblocks; ++k) {
            const int m = L.blk[k][0], ni = L.blk[k][1], no = L.blk[k][2];
            const int ioff = L.blk[k][3], ooff = L.blk[k][4], woff = L.blk[k][5];
            for (int o = 0; o < no; ++o)
                for (int i = 0; i < ni; ++i) {
                    if (m == 0) {
                        fl[woff + o * ni + i] = L.lslot_in[ioff + i] + L.lslot_out[ooff + o];
                    } else {
                        const int lsum = L.lslot_in[ioff + 2 * i] + L.lslot_out[ooff + 2 * o];
                        fl[woff + 2 * (o * ni + i)] = lsum;
                        fl[woff + 2 * (o * ni + i) + 1] = lsum;
                    }
                }
        }
    }
    for (int q = threadIdx.x; q < 4 * hsz; q += kThreads) sh[q] = 0.0f;
    __syncthreads();
    float* hist = sh + wave * hsz;
    const int64_t e_begin = blockIdx.x * chunk;
    const int64_t e_end = e_begin + chunk < E ? e_begin + chunk : E;
    const float sigma = B.sh_scale;
    for (int64_t e = e_begin + wave; e < e_end; e += 4) {
        const float r = dist[e];
        const EdgeBin eb = edge_bin(r, B);
        const float* flo = F + static_cast<int64_t>(eb.lo) * kw;
        const float* g = dFe + e * kw;
        float st = 0.0f, ss = 0.0f;
        for (int q = lane; q < kw; q += 64) {
            const float gv = g[q];
            const float lo = flo[q], hi = flo[kw + q];
            hist[eb.lo * kw + q] += (1.0f - eb.t) * gv;
            hist[(eb.lo + 1) * kw + q] += eb.t * gv;
            st += (hi - lo) * gv;
            ss += static_cast<float>(fl[q % L.wdim]) * lerp_bins(lo, hi, eb.t) * gv;
        }
        if (gdist) {
            for (int off = 32; off > 0; off >>= 1) {
                st += __shfl_xor(st, off, 64);
                ss += __shfl_xor(ss, off, 64);
            }
            if (lane == 0) {
                float v = st * eb.dtdr;
                if (L.has_lpos) v += ss * (sigma / (r * (r + sigma)));
                gdist[e] = v;
            }
        }
    }
    __syncthreads();
    float* out = hist_part + static_cast<int64_t>(blockIdx.x) * hsz;
    for (int q = threadIdx.x; q < hsz; q += kThreads)
        out[q] = ((sh[q] + sh[hsz + q]) + sh[2 * hsz + q]) + sh[3 * hsz + q];
}

__global__ void k_sum_partials(const float* __restrict__ part, int groups, int64_t n,
                               float* __restrict__ out) {
    const int64_t q = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
    if (q >= n) return;
    float acc = 0.0f;
    for (int g = 0; g < groups; ++g) acc += part[static_cast<int64_t>(g) * n + q];
    out[q] = acc;
}

int reduce_partials(const float* part, int groups, int64_t n, float* out, hipStream_t s) {
    FEQ_LAUNCH("k_sum_partials", k_sum_partials, dim3(ceil_div(n, 256)), dim3(256), 0, s, part, groups, n, out);
    return FEQ_OK;
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
    return 4 * (static_cast<size_t>(K) * COUT * CIN + BIG + kNE * T::DIN * T::DIN +
                kNE * T::DOUT * T::DOUT + kNE * T::DIN + kNE * T::DOUT + kNE * K * T::WD) +
           kNE * sizeof(TileEdge);
}

template <int CIN, int COUT, int LIN, int LOUT, int K>
constexpr size_t bwd_x_lds() {
    using T = Canon<LIN, LOUT>;
    constexpr size_t FS = 16 * T::DIN + 1, GS = 16 * T::DOUT + 1, XS = CIN * T::DIN + 1;
    constexpr size_t GBIG = COUT * GS > kNE * XS ? COUT * GS : kNE * XS;
    return 4 * (static_cast<size_t>(K) * COUT * CIN + CIN * FS + GBIG + kNE * T::DIN * T::DIN +
                kNE * T::DOUT * T::DOUT + kNE * T::DIN + kNE * T::DOUT + kNE * K * T::WD) +
           kNE * sizeof(TileEdge);
}

template <int CIN, int COUT, int LIN, int LOUT, int K>
constexpr size_t bwd_c_lds() {
    using T = Canon<LIN, LOUT>;
    constexpr size_t FS = 16 * T::DIN + 1, GS = 16 * T::DOUT + 1;
    return 4 * (CIN * FS + COUT * GS + COUT * FS + kNE * T::DIN * T::DIN + kNE * T::DOUT * T::DOUT +
                kNE * T::DIN + kNE * T::DOUT + kNE * K * T::WD) +
           kNE * sizeof(TileEdge);
}

constexpr int64_t kBinChunk = 1024;

size_t bins_lds_bytes(const feq_layout& L, const feq_binning& B, int K) {
    return 4 * static_cast<size_t>(4) * (B.num_bins + 1) * K * L.wdim + 4 * L.wdim + 16;
}

template <int CIN, int COUT, int LIN, int LOUT, int K>
int launch_fwd(const feq_binning& B, int64_t E, const float* x, const float* P, const float* Q,
               const float* dist, const float* C, const float* F, float* y, hipStream_t s) {
    constexpr size_t lds = fwd_lds<CIN, COUT, LIN, LOUT, K>();
    auto kern = k_ewc_fwd<CIN, COUT, LIN, LOUT, K>;
    if (int rc = set_lds(reinterpret_cast<const void*>(kern), lds)) return rc;
    const int64_t ntiles = ceil_div(E, kNE);
    FEQ_LAUNCH("k_ewc_fwd", kern, dim3(grid_for(ntiles, lds <= 80 * 1024 ? 2 : 1)), dim3(kThreads), lds,
                       s, B, E, ntiles, x, P, Q, dist, C, F, y);
    return FEQ_OK;
}

template <int CIN, int COUT, int LIN, int LOUT, int K>
size_t bwd_ws(const feq_binning& B, int64_t E) {
    using T = Canon<LIN, LOUT>;
    const int64_t G = grid_for(ceil_div(E, kNE), 2);
    const int64_t kw = static_cast<int64_t>(K) * T::WD;
    return align_up(4 * E * kw, 256) + align_up(4 * G * K * COUT * CIN, 256) +
           align_up(4 * ceil_div(E, kBinChunk) * (B.num_bins + 1) * kw, 256) + 1024;
}

template <int CIN, int COUT, int LIN, int LOUT, int K>
int launch_bwd(const feq_layout& L, const feq_binning& B, int64_t E, const float* gy,
               const float* x, const float* P, const float* Q, const float* dist, const float* C,
               const float* F, float* gx, float* gC, float* gF, float* gdist, char* ws,
               size_t ws_bytes, hipStream_t s) {
    using T = Canon<LIN, LOUT>;
    constexpr size_t xlds = bwd_x_lds<CIN, COUT, LIN, LOUT, K>();
    constexpr size_t clds = bwd_c_lds<CIN, COUT, LIN, LOUT, K>();
    const size_t blds = bins_lds_bytes(L, B, K);
    if (blds > 160 * 1024 || xlds > 160 * 1024 || clds > 160 * 1024) return -1;
    auto kx = k_ewc_bwd_x<CIN, COUT, LIN, LOUT, K>;
    auto kc = k_ewc_bwd_c<CIN, COUT, LIN, LOUT, K>;
    const int64_t ntiles = ceil_div(E, kNE);
    const int Gx = grid_for(ntiles, xlds <= 80 * 1024 ? 2 : 1);
    const int G = grid_for(ntiles, clds <= 80 * 1024 ? 2 : 1);
    const int64_t nchunks = ceil_div(E, kBinChunk);
    const int64_t kw = static_cast<int64_t>(K) * T::WD;
    const int64_t hsz = (B.num_bins + 1) * kw;
    Carver cv(ws);
    float* dFe = cv.take<float>(E * kw);
    float* dCp = cv.take<float>(static_cast<size_t>(G) * K * COUT * CIN);
    float* hp = cv.take<float>(nchunks * hsz);
    if (cv.used > ws_bytes) return fail(FEQ_ERR_WORKSPACE, "edgewise workspace too small");
    if (int rc = set_lds(reinterpret_cast<const void*>(kx), xlds)) return rc;
    FEQ_LAUNCH("k_ewc_bwd_x", kx, dim3(Gx), dim3(kThreads), xlds, s, B, E, ntiles, gy, x, P, Q, dist, C, F,
                       gx, dFe);
    if (int rc = set_lds(reinterpret_cast<const void*>(kc), clds)) return rc;
    FEQ_LAUNCH("k_ewc_bwd_c", kc, dim3(G), dim3(kThreads), clds, s, B, E, ntiles, gy, x, P, Q, dist, F,
                       dCp);
    if (int rc = set_lds(reinterpret_cast<const void*>(&k_ewm_bins), blds)) return rc;
    FEQ_LAUNCH("k_ewm_bins", k_ewm_bins, dim3(nchunks), dim3(kThreads), blds, s, L, B, K, E, kBinChunk,
                       dist, F, dFe, gdist, hp);
    if (int rc = reduce_partials(dCp, G, static_cast<int64_t>(K) * COUT * CIN, gC, s)) return rc;
    return reduce_partials(hp, static_cast<int>(nchunks), hsz, gF, s);
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

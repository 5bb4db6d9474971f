// Fused EquivariantEdgewiseLinear with its GEMMs on the fp16 matrix cores of
// gfx950, at fp32 accuracy.
//
// Same mathematics as edgewise.hip and edgewise_mfma.hip: with the separable
// radial table T[b,o,i,w] = sum_k C[k,o,i] F[b,k,w] the per-edge mix of a
// 16-edge tile is one GEMM shared by all edges, G_k = C_k fs (M = Cout,
// N = 16 Din, K = Cin), followed by a per-edge contraction with the
// interpolated radial functions F_e (the sparse mixing matrix M_ek of the
// m-block layout, 2x2 [[a, b], [-b, a]] blocks for m > 0).
//
// gfx950 has no fp32-input matrix instruction faster than v_mfma_f32_16x16x4
// (157 TFLOP/s); v_mfma_f32_16x16x32_f16 is 16x faster.  Every fp32 operand
// is therefore split into two fp16 parts after an exact power-of-two scaling,
//     a = 2^-e (a_hi + a_lo),  a_hi = fp16(2^e a),  a_lo = fp16(2^e a - a_hi),
// and a product is a_hi b_hi + a_hi b_lo + a_lo b_hi (three MFMAs, fp32
// accumulation).  The scaling puts the largest magnitude of each scaled block
// in [2^14, 2^15), so nothing overflows fp16 and every element within 2^-29 of
// that maximum keeps an 11-bit hi and 11-bit lo part: the dropped terms
// (a_lo b_lo and the residuals below a_lo, b_lo) are ~2^-22 of each product,
// the accuracy of an fp32 GEMM.  Scales:
//   C_k      one per rank component (every workgroup derives the same value);
//   fs       one per edge (a GEMM column block), reduced over the 16 lanes that
//            produce the edge's rows.
// Both are undone for free: 1/scale_k is folded into the interpolated radial
// functions of the contraction and 1/scale_e into the s^l_out output scaling.
//
// Operand layout of v_mfma_f32_16x16x32_f16: lane l supplies eight consecutive
// reduction indices of row l % 16 of A and of column l % 16 of B (which eight,
// as a function of l / 16, only has to agree between A and B), and holds
// D[4 (l / 16) + r][l % 16] in register r.  GEMM columns are slot-major
// (column = 16 slot + edge), so lane l holds every slot of edge l % 16 for its
// rows and the per-edge contraction runs in registers.
#include "ew_canon.h"
#include "feq_internal.h"

namespace feq {
namespace {

typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));

constexpr int kNE = 16;        // edges per tile
constexpr int kThreads = 256;  // 4 waves

__device__ __forceinline__ v4f mfma_h(h8 a, h8 b, v4f c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Exponent e of the power-of-two scale for a block whose largest magnitude is
// m: m 2^e lies in [2^14, 2^15) for normal m; e is clamped to [-113, 126] so
// that 2^e and 2^-e are normal floats (zero or subnormal m gives 2^126).
__device__ __forceinline__ int scale_exp(float m) {
    const int ex = static_cast<int>((__float_as_uint(m) >> 23) & 0xffu);
    int e = 141 - ex;
    e = e < -113 ? -113 : e;
    return e > 126 ? 126 : e;
}

__device__ __forceinline__ float exp2i(int e) {
    return __uint_as_float(static_cast<unsigned>(e + 127) << 23);
}

__device__ __forceinline__ void split_f16(float a, _Float16& hi, _Float16& lo) {
    hi = static_cast<_Float16>(a);
    lo = static_cast<_Float16>(a - static_cast<float>(hi));
}

// Byte offset of lane slot (g, e) = lane 16 g + e inside a 1 KB fragment chunk
// (64 lanes x 8 halves).  The XOR swizzle keeps the fragment reads (a
// permutation of the chunk per 16 lanes) and the producers' 8-byte writes
// (4 edges x 16 channel quads per wave) free of bank conflicts.
__device__ __forceinline__ int bslot(int g, int e) { return (16 * g + (e ^ (4 * g))) * 16; }

struct EdgeState {
    int lo;
    float t;
    float s;
    int valid;
};

// s^l of every m-first slot of a canonical representation with lmax L.
template <int L>
__device__ __forceinline__ void slot_pow(float s, float (&pw)[(L + 1) * (L + 1)]) {
    float p[L + 1];
    p[0] = 1.0f;
#pragma unroll
    for (int l = 1; l <= L; ++l) p[l] = p[l - 1] * s;
#pragma unroll
    for (int j = 0; j < (L + 1) * (L + 1); ++j) pw[j] = p[SlotL<L>::l[j]];
}

// Split fragments of the constant GEMM operand, written once per call by
// k_ews_prep: C_k (forward, rows co) or C_k^T (input gradient, rows ci),
// scaled by one power of two per rank component k (largest magnitude in
// [2^14, 2^15)) and split into fp16 hi and lo parts.  Fragment (k, rb, ks) of
// lane l (row 16 rb + l % 16, reduction indices 32 ks + 8 (l / 16) + 0..7)
// occupies 32 bytes at ((k * NRB + rb) * NKS + ks) * 64 + l: eight hi halves,
// then eight lo halves.  inv[k] receives 2^-e_k.
template <int K, int NROW, int NRED, bool TRANS>
__global__ void __launch_bounds__(kThreads)
k_ews_prep(const float* __restrict__ C, h8* __restrict__ frag, float* __restrict__ inv) {
    // one workgroup per (k, rb): the rank's scale, then its NKS * 64 fragments
    constexpr int NCH = NROW * NRED, NRB = NROW / 16, NKS = NRED / 32;
    static_assert(NKS * 64 <= kThreads, "one fragment per thread");
    __shared__ float red[kThreads / 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int k = blockIdx.x / NRB, rb = blockIdx.x % NRB;
    const float* Ck = C + static_cast<int64_t>(k) * NCH;
    float v = 0.0f;
    for (int q = tid; q < NCH; q += kThreads) v = fmaxf(v, fabsf(Ck[q]));
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float m = red[0];
#pragma unroll
    for (int w = 1; w < kThreads / 64; ++w) m = fmaxf(m, red[w]);
    const int e = scale_exp(m);
    const float sc = exp2i(e);
    if (rb == 0 && tid == 0) inv[k] = exp2i(-e);
    if (tid < NKS * 64) {
        const int l = tid & 63, ks = tid >> 6;
        const int row = 16 * rb + (l & 15), c0 = 32 * ks + 8 * (l >> 4);
        h8 hi, lo;
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) {
            // A = C_k (row co, reduction ci) or C_k^T (row ci, reduction co); C is (K, Cout, Cin)
            const float a = TRANS ? Ck[(c0 + jj) * NROW + row] : Ck[row * NRED + c0 + jj];
            _Float16 h, lw;
            split_f16(a * sc, h, lw);
            hi[jj] = h;
            lo[jj] = lw;
        }
        const int q = ((k * NRB + rb) * NKS + ks) * 64 + l;
        frag[2 * q] = hi;
        frag[2 * q + 1] = lo;
    }
}

// The (kNE, N) block of a (E, N) tensor that starts at edge e0, as float4s:
// thread t holds float4 q = t + kThreads n of the block.  A full tile is read
// with 16-byte loads (the block starts at a multiple of 16 edges, so it is
// 16-byte aligned); the last, partial tile element by element, zero-padded.
template <int N, int NV>
__device__ __forceinline__ void load_tile4(const float* __restrict__ src, int64_t e0, int64_t E,
                                           float4 (&v)[NV]) {
    constexpr int NQ = kNE * N / 4;
    const int tid = threadIdx.x;
    if (e0 + kNE <= E) {
        const float4* s4 = reinterpret_cast<const float4*>(src + e0 * N);
#pragma unroll
        for (int n = 0; n < NV; ++n) {
            const int q = tid + kThreads * n;
            v[n] = q < NQ ? s4[q] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
    } else {
        const int64_t lim = (E - e0) * N;
#pragma unroll
        for (int n = 0; n < NV; ++n) {
            const int q = tid + kThreads * n;
            float f[4];
#pragma unroll
            for (int c = 0; c < 4; ++c) f[c] = (q < NQ && 4 * q + c < lim) ? src[e0 * N + 4 * q + c] : 0.0f;
            v[n] = make_float4(f[0], f[1], f[2], f[3]);
        }
    }
}

// Stores a block read by load_tile4 into LDS with a row stride of S floats per edge.
template <int N, int NV, int S>
__device__ __forceinline__ void store_tile4(const float4 (&v)[NV], float* dst) {
    constexpr int NQ = kNE * N / 4;
    const int tid = threadIdx.x;
#pragma unroll
    for (int n = 0; n < NV; ++n) {
        const int q = tid + kThreads * n;
        if (q < NQ) {
            const float f[4] = {v[n].x, v[n].y, v[n].z, v[n].w};
#pragma unroll
            for (int c = 0; c < 4; ++c) dst[((4 * q + c) / N) * S + (4 * q + c) % N] = f[c];
        }
    }
}

// ---------------------------------------------------------------------------
// Forward: y = Q-rotate(s^l_out sum_k M_ek G_k), G_k = C_k fs, fs = s^l_in (x P).
// A workgroup owns one 16-edge tile at a time; wave w owns output rows
// co = 16 (w + 4 j) + ..., j < Cout / 64.  Per tile: (1) global loads of x,
// P, Q and distances; (2) P/Q to LDS; (3) fs rows are rotated by threads that
// own 4 channels of one edge, scaled per edge, split and written as fp16
// fragments; (4) per slot i the waves run the 3-term MFMA products for all
// rank components and contract them into y (registers); (5) Q rotation and
// direct 16-byte stores (each lane owns 4 consecutive channels of one edge).
template <int CIN, int COUT, int LIN, int LOUT, int K>
__global__ void __launch_bounds__(kThreads, 2)
k_ews_fwd(feq_binning B, int64_t E, int64_t ntiles, const float* __restrict__ x,
          const float* __restrict__ P, const float* __restrict__ Q,
          const float* __restrict__ dist, const h8* __restrict__ Cfrag,
          const float* __restrict__ Cinv, const float* __restrict__ F, float* __restrict__ y) {
    using T = Canon<LIN, LOUT>;
    constexpr int DIN = T::DIN, DOUT = T::DOUT, WD = T::WD, KW = K * WD;
    constexpr int PS = (DIN * DIN + 3) / 4 * 4, QS = (DOUT * DOUT + 3) / 4 * 4;
    constexpr int RPW = COUT / 64, NKS = CIN / 32, NC4 = CIN / 4;
    constexpr int CHUNK = 1024;                                  // bytes per fragment chunk
    constexpr int NPR = (kNE * NC4 + kThreads - 1) / kThreads;   // producer passes
    constexpr int NPL = (kNE * DIN * DIN / 4 + kThreads - 1) / kThreads;
    constexpr int NQL = (kNE * DOUT * DOUT / 4 + kThreads - 1) / kThreads;
    static_assert(COUT % 64 == 0 && CIN % 32 == 0 && NC4 <= 64, "unsupported channel counts");
    static_assert((kNE * NC4) % kThreads == 0 || kNE * NC4 < kThreads, "producer split");

    extern __shared__ float4 smem4[];
    char* sB = reinterpret_cast<char*>(smem4);                   // [2][DIN][NKS] chunks
    float* sP = reinterpret_cast<float*>(sB + 2 * DIN * NKS * CHUNK);
    float* sQ = sP + kNE * PS;
    float* sFe = sQ + kNE * QS;
    float* sSout = sFe + kNE * KW;
    float* sInvK = sSout + kNE * DOUT;
    EdgeState* sE = reinterpret_cast<EdgeState*>(sInvK + K);

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int le = lane & 15, lg = lane >> 4;

    if (tid < K) sInvK[tid] = Cinv[tid];   // read after the first tile barrier

    for (int64_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
        const int64_t e0 = tile * kNE;
        // (1) global loads for this tile
        float xr[NPR][4 * DIN];
#pragma unroll
        for (int p = 0; p < NPR; ++p) {
            const int q = tid + kThreads * p;
            const int e = q / NC4, c4 = q % NC4;
            if (q < kNE * NC4 && e0 + e < E) {
                const float4* src = reinterpret_cast<const float4*>(x + ((e0 + e) * CIN + 4 * c4) * DIN);
#pragma unroll
                for (int v = 0; v < DIN; ++v) {
                    const float4 f = src[v];
                    xr[p][4 * v] = f.x;
                    xr[p][4 * v + 1] = f.y;
                    xr[p][4 * v + 2] = f.z;
                    xr[p][4 * v + 3] = f.w;
                }
            } else {
#pragma unroll
                for (int v = 0; v < 4 * DIN; ++v) xr[p][v] = 0.0f;
            }
        }
        float4 pr[NPL], qr[NQL];
        load_tile4<DIN * DIN, NPL>(P, e0, E, pr);
        load_tile4<DOUT * DOUT, NQL>(Q, e0, E, qr);
        const float rd = (tid < kNE && e0 + tid < E) ? dist[e0 + tid] : 1.0f;

        __syncthreads();   // the previous tile's readers of every LDS buffer are done
        // (2) P, Q and edge state to LDS
        store_tile4<DIN * DIN, NPL, PS>(pr, sP);
        store_tile4<DOUT * DOUT, NQL, QS>(qr, sQ);
        if (tid < kNE) {
            EdgeState es;
            es.valid = e0 + tid < E;
            const EdgeBin eb = edge_bin(rd, B);
            es.lo = eb.lo;
            es.t = eb.t;
            es.s = rd / (rd + B.sh_scale);
            sE[tid] = es;
        }
        __syncthreads();

        // (3) radial functions of the tile (with 1/scale_k folded in)
        for (int q = tid; q < kNE * KW; q += kThreads) {
            const int e = q / KW, rest = q % KW;
            const EdgeState es = sE[e];
            const float* flo = F + static_cast<int64_t>(es.lo) * KW + rest;
            sFe[q] = lerp_bins(flo[0], flo[KW], es.t) * sInvK[rest / WD];
        }
        // fs rows: thread (e, c4) owns channels 4 c4 .. 4 c4 + 3 of edge e
#pragma unroll
        for (int p = 0; p < NPR; ++p) {
            const int q = tid + kThreads * p;
            const int e = q / NC4, c4 = q % NC4;
            const bool act = q < kNE * NC4;
            const int ee = act ? e : 0;
            float pw[DIN];
            slot_pow<LIN>(sE[ee].s, pw);
            float fs[4][DIN];
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int i = 0; i < DIN; ++i) fs[r][i] = 0.0f;
            const float* pe = sP + ee * PS;
#pragma unroll
            for (int d = 0; d < DIN; ++d)
#pragma unroll
                for (int i = 0; i < DIN; ++i) {
                    const float pv = pe[d * DIN + i];
#pragma unroll
                    for (int r = 0; r < 4; ++r) fs[r][i] += xr[p][r * DIN + d] * pv;
                }
            float m = 0.0f;
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int i = 0; i < DIN; ++i) {
                    fs[r][i] *= pw[i];
                    m = fmaxf(m, fabsf(fs[r][i]));
                }
#pragma unroll
            for (int off = NC4 / 2; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
            const int ex = scale_exp(m);
            const float sc = exp2i(ex);
            if (act && c4 == 0) {
                float po[DOUT];
                slot_pow<LOUT>(sE[e].s, po);
                const float inv = exp2i(-ex);
#pragma unroll
                for (int o = 0; o < DOUT; ++o) sSout[e * DOUT + o] = po[o] * inv;
            }
            if (act) {
                const int ks = c4 / 8, g = (c4 / 2) % 4, half = c4 % 2;
                char* base = sB + ks * CHUNK + bslot(g, e) + 8 * half;
#pragma unroll
                for (int i = 0; i < DIN; ++i) {
                    h4 hv, lv;
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        _Float16 h, l;
                        split_f16(fs[r][i] * sc, h, l);
                        hv[r] = h;
                        lv[r] = l;
                    }
                    *reinterpret_cast<h4*>(base + (i * NKS) * CHUNK) = hv;
                    *reinterpret_cast<h4*>(base + ((DIN + i) * NKS) * CHUNK) = lv;
                }
            }
        }
        // A fragments of this wave's rows (L2-resident), in flight across the
        // barrier.  The empty asm makes the pointer opaque per tile, so the
        // loads are not hoisted out of the tile loop (their registers would
        // then stay live through the producer phase).
        const h8* cfr = Cfrag;
        asm volatile("" : "+s"(cfr));
        h8 ahi[RPW][K][NKS], alo[RPW][K][NKS];
#pragma unroll
        for (int j = 0; j < RPW; ++j)
#pragma unroll
            for (int k = 0; k < K; ++k)
#pragma unroll
                for (int ks = 0; ks < NKS; ++ks) {
                    const h8* src = cfr + 2 * (((k * (COUT / 16) + wave + 4 * j) * NKS + ks) * 64 + lane);
                    ahi[j][k][ks] = src[0];
                    alo[j][k][ks] = src[1];
                }
        __syncthreads();

        // (4) GEMM per input slot and contraction into y (m-first output slots)
        using TG = TermGroups<LIN, LOUT, false>;
        float yv[RPW][DOUT][4];
#pragma unroll
        for (int j = 0; j < RPW; ++j)
#pragma unroll
            for (int o = 0; o < DOUT; ++o)
#pragma unroll
                for (int r = 0; r < 4; ++r) yv[j][o][r] = 0.0f;
        const float* fe = sFe + le * KW;
        const int myslot = bslot(lg, le);
        // B fragments are double-buffered one slot ahead; the scheduling fence
        // at the end of each slot keeps the compiler from hoisting every
        // slot's loads (which would not fit the register budget).
        h8 bh[2][NKS], bl[2][NKS];
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) {
            bh[0][ks] = *reinterpret_cast<const h8*>(sB + ks * CHUNK + myslot);
            bl[0][ks] = *reinterpret_cast<const h8*>(sB + (DIN * NKS + ks) * CHUNK + myslot);
        }
        static_for<DIN>([&](auto I) {
            constexpr int i = decltype(I)::value;
            constexpr int cur = i & 1;
            if constexpr (i + 1 < DIN) {
#pragma unroll
                for (int ks = 0; ks < NKS; ++ks) {
                    bh[cur ^ 1][ks] = *reinterpret_cast<const h8*>(sB + ((i + 1) * NKS + ks) * CHUNK + myslot);
                    bl[cur ^ 1][ks] =
                        *reinterpret_cast<const h8*>(sB + ((DIN + i + 1) * NKS + ks) * CHUNK + myslot);
                }
            }
            v4f acc[RPW][K];
#pragma unroll
            for (int j = 0; j < RPW; ++j)
#pragma unroll
                for (int k = 0; k < K; ++k) acc[j][k] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
                for (int j = 0; j < RPW; ++j)
#pragma unroll
                    for (int k = 0; k < K; ++k) {
                        acc[j][k] = mfma_h(alo[j][k][ks], bh[cur][ks], acc[j][k]);
                        acc[j][k] = mfma_h(ahi[j][k][ks], bl[cur][ks], acc[j][k]);
                        acc[j][k] = mfma_h(ahi[j][k][ks], bh[cur][ks], acc[j][k]);
                    }
            static_for<TG::count(i)>([&](auto TT) {
                constexpr Term tm = TG::sorted[TG::start[i] + decltype(TT)::value];
#pragma unroll
                for (int k = 0; k < K; ++k) {
                    const float c = tm.neg ? -fe[k * WD + tm.w] : fe[k * WD + tm.w];
#pragma unroll
                    for (int j = 0; j < RPW; ++j)
#pragma unroll
                        for (int r = 0; r < 4; ++r) yv[j][tm.o][r] += c * acc[j][k][r];
                }
            });
            __builtin_amdgcn_sched_barrier(0);
        });
        // Uses of every y register here keep the compiler from sinking the
        // contractions into the store branch below (which would keep all
        // MFMA results live until then).
#pragma unroll
        for (int j = 0; j < RPW; ++j)
#pragma unroll
            for (int o = 0; o < DOUT; ++o)
#pragma unroll
                for (int r = 0; r < 4; ++r) asm volatile("" ::"v"(yv[j][o][r]));

        // (5) output scaling, Q rotation and stores
        {
            const float* so = sSout + le * DOUT;
            const float* qe = sQ + le * QS;
#pragma unroll
            for (int o = 0; o < DOUT; ++o) {
                const float sc = so[o];
#pragma unroll
                for (int j = 0; j < RPW; ++j)
#pragma unroll
                    for (int r = 0; r < 4; ++r) yv[j][o][r] *= sc;
            }
#pragma unroll
            for (int j = 0; j < RPW; ++j) {
                float out[4 * DOUT];
#pragma unroll
                for (int d = 0; d < DOUT; ++d) {
                    float qrow[DOUT];
#pragma unroll
                    for (int o = 0; o < DOUT; ++o) qrow[o] = qe[d * DOUT + o];
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        float a = 0.0f;
#pragma unroll
                        for (int o = 0; o < DOUT; ++o) a += yv[j][o][r] * qrow[o];
                        out[r * DOUT + d] = a;
                    }
                }
                if (e0 + le < E) {
                    float4* dst = reinterpret_cast<float4*>(
                        y + ((e0 + le) * COUT + 16 * (wave + 4 * j) + 4 * lg) * DOUT);
#pragma unroll
                    for (int v = 0; v < DOUT; ++v)
                        dst[v] = make_float4(out[4 * v], out[4 * v + 1], out[4 * v + 2], out[4 * v + 3]);
                }
            }
        }
    }
}

template <int CIN, int COUT, int LIN, int LOUT, int K>
constexpr size_t ews_fwd_lds() {
    using T = Canon<LIN, LOUT>;
    constexpr size_t PS = (T::DIN * T::DIN + 3) / 4 * 4, QS = (T::DOUT * T::DOUT + 3) / 4 * 4;
    return 2 * T::DIN * (CIN / 32) * 1024 +
           4 * (kNE * PS + kNE * QS + kNE * K * T::WD + kNE * T::DOUT + K) +
           kNE * sizeof(EdgeState);
}

int ews_cus() {
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) == hipSuccess) {
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
            cus = v;
    }
    return cus;
}

int ews_set_lds(const void* kern, size_t lds) {
    if (lds > 160 * 1024) return fail(FEQ_ERR_UNSUPPORTED, "kernel needs %zu B of LDS", lds);
    if (lds > 64 * 1024)
        FEQ_HIP(hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                    static_cast<int>(lds)));
    return FEQ_OK;
}

// Workspace of the split forward: C fragments and the rank scales.
template <int CIN, int COUT, int K>
constexpr size_t ews_cfrag_bytes() {
    return align_up(static_cast<size_t>(K) * COUT * CIN * 2 * sizeof(_Float16), 256) + 256;
}

template <int CIN, int COUT, int LIN, int LOUT, int K>
int launch_ews_fwd(const feq_binning& B, int64_t E, const float* x, const float* P, const float* Q,
                   const float* dist, const float* C, const float* F, float* y, void* ws,
                   size_t ws_bytes, hipStream_t s) {
    constexpr size_t lds = ews_fwd_lds<CIN, COUT, LIN, LOUT, K>();
    static_assert(lds <= 80 * 1024, "two forward workgroups must fit one CU's LDS");
    if (!ws || ws_bytes < ews_cfrag_bytes<CIN, COUT, K>())
        return fail(FEQ_ERR_WORKSPACE, "edgewise forward workspace too small");
    Carver cv(ws);
    h8* frag = cv.take<h8>(static_cast<size_t>(K) * COUT * CIN / 4);
    float* inv = cv.take<float>(K);
    auto prep = k_ews_prep<K, COUT, CIN, false>;
    FEQ_LAUNCH("k_ews_prep", prep, dim3(K * COUT / 16), dim3(kThreads), 0, s, C, frag, inv);
    auto kern = k_ews_fwd<CIN, COUT, LIN, LOUT, K>;
    if (int rc = ews_set_lds(reinterpret_cast<const void*>(kern), lds)) return rc;
    const int64_t ntiles = ceil_div(E, kNE);
    const int64_t g = static_cast<int64_t>(ews_cus()) * 2;
    const int grid = static_cast<int>(ntiles < g ? ntiles : g);
    FEQ_LAUNCH("k_ews_fwd", kern, dim3(grid), dim3(kThreads), lds, s, B, E, ntiles, x, P, Q, dist,
               frag, inv, F, y);
    return FEQ_OK;
}

// The layout is the canonical (0..lin) x (0..lout) pair of the instantiation.
bool canonical(const feq_layout& L, int lin, int lout) {
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

// Shapes with a split-fp16 fast path: (Cin, Cout, Lin, Lout), rank 4.
#define FEQ_EWS_SHAPES(X) \
    X(64, 64, 2, 2)       \
    X(32, 64, 1, 2)

size_t ew_split_workspace(const feq_layout& L, int rank) {
    if (rank != 4) return 0;
#define FEQ_WS(ci, co, li, lo) \
    if (L.cin == ci && L.cout == co && canonical(L, li, lo)) return ews_cfrag_bytes<ci, co, 4>();
    FEQ_EWS_SHAPES(FEQ_WS)
#undef FEQ_WS
    return 0;
}

// The split kernels read and write x, P, Q and y with 16-byte accesses.
static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int ew_split_fwd(const feq_layout& L, const feq_binning& B, int rank, int64_t E, const float* x,
                 const float* P, const float* Q, const float* dist, const float* C, const float* F,
                 float* y, void* ws, size_t ws_bytes, hipStream_t s) {
    if (rank != 4 || !aligned16(x) || !aligned16(P) || !aligned16(Q) || !aligned16(y)) return -1;
#define FEQ_FWD(ci, co, li, lo)                                \
    if (L.cin == ci && L.cout == co && canonical(L, li, lo))   \
        return launch_ews_fwd<ci, co, li, lo, 4>(B, E, x, P, Q, dist, C, F, y, ws, ws_bytes, s);
    FEQ_EWS_SHAPES(FEQ_FWD)
#undef FEQ_FWD
    return -1;
}

}  // namespace feq

// EquivariantEdgewiseLinear at high degree (canonical lvals 0..L in and out,
// L = 6: dim 49, 13x13 Wigner blocks) for bfloat16 features, on the bf16
// matrix cores of gfx950 with float32 accumulation.
//
// Same mathematics as edgewise.hip: with the separable radial table
// T[b,o,i,w] = sum_k C[k,o,i] F[b,k,w] (SeparableRadialNet, radial.py:259-275)
//   y = Q-rotate( s^l_out sum_k M_ek (C_k fs) ),   fs = s^l_in (x P),
// where M_ek is the per-edge mixing matrix of the interpolated radial
// functions F_e (2x2 [[a, b], [-b, a]] blocks on (+m, -m) pairs, block
// diagonal over m).  At dim 49 an edge's slots no longer fit the registers of
// the lanes that own it, so the layer runs in stages:
//   k_hl_rot_in   fs^T[e, j, c] = s^l(j) sum_d x[e, c, d] P[e, d, j]  (bf16, slot-major),
//                 one (C x D) x (D x D) bf16 MFMA product per edge; the same
//                 kernel forms gd^T = s^l (gy Q) in the backward;
//   k_hl_mix      per edge, G_k^T = fs^T C_k^T, the contraction with F_e and
//                 the rotation back y = (s^l ym) Q^T as three chained bf16
//                 MFMA products (each product's accumulators are the next
//                 one's B operand, split into hi and lo bf16 halves where the
//                 precision needs it; below at k_hl_mixr); with C_k^T, M_ek^T
//                 and P it forms dx from gd^T (k_hl_mix_t);
//   k_hl_dfe      dF_e[k, w] = sum over the terms (o, i, w) of sign <gd_o, C_k fs_i>,
//                 G_k = C_k fs and Z_k = gd^T G_k as two chained bf16 MFMA
//                 products per edge (below at k_hl_dfer);
//   k_hl_dc       dC_k = sum over (e, i) of U_k fs^T with U_k = gd M_ek, both as
//                 chained bf16 MFMA products per edge whose B operands are read
//                 transposed from LDS (below at k_hl_dcc); per-workgroup
//                 partials summed in a fixed order.
// The binned radial-function and distance gradients reuse the tail of the
// other fused families (edgewise_tail.hip).

#include "ew_canon.h"
#include "feq_internal.h"

namespace feq {
namespace {

typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 bf8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

constexpr int kT = 256;   // threads per workgroup
constexpr int kNE = 16;   // edges per MFMA tile (the B columns)

__device__ __forceinline__ v4f mfma_bf(bf8 a, bf8 b, v4f c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

template <int L>
struct HL {
    using Cn = Canon<L, L>;
    static constexpr int D = Cn::DIN;
    static constexpr int WD = Cn::WD;
    static constexpr int NG = L + 1;                      // m-groups
    static constexpr int goff(int m) { return Cn::in_off(m); }
    static constexpr int gsize(int m) { return (m ? 2 : 1) * (L - m + 1); }
    static constexpr int group_of(int s) {
        int m = 0;
        while (m + 1 < NG && goff(m + 1) <= s) ++m;
        return m;
    }
    static constexpr int GMAX = gsize(1) > gsize(0) ? gsize(1) : gsize(0);
    static constexpr int wsize(int m) { return Cn::w_off(m + 1) - Cn::w_off(m); }
    static constexpr int WGMAX = [] {
        int w = 0;
        for (int m = 0; m < NG; ++m) w = wsize(m) > w ? wsize(m) : w;
        return w;
    }();
    // degree of component d in the standard (l, m) order
    static constexpr int deg(int d) {
        int l = 0;
        while ((l + 1) * (l + 1) <= d) ++l;
        return l;
    }
};

// s^l for 0 <= l <= 7 from s, s^2 and s^4, without a loop
__device__ __forceinline__ float pow_sel(float s1, float s2, float s4, int l) {
    return ((l & 1) ? s1 : 1.0f) * ((l & 2) ? s2 : 1.0f) * ((l & 4) ? s4 : 1.0f);
}

__device__ __forceinline__ float ipowf_small(float s, int l) {
    float p = 1.0f;
    for (int i = 0; i < l; ++i) p *= s;
    return p;
}

// ---- rotations ------------------------------------------------------------------
// Basis rows d are in the standard (l, m) order, columns j in the m-first order
// (the WignerDBasis layout); the kernels take any basis, block-diagonal or not.

// out[e, j, c] = s_e^{l(j)} sum_d in[e, c, d] R[e, d, j]   (fs^T = s^l (x P), gd^T = s^l (gy Q))
//
// On the bf16 matrix cores: a wave takes one edge at a time and forms the
// (C x D) x (D x D) product as (C / 16) x ceil(D / 16) tiles of
// v_mfma_f32_16x16x32_bf16, the reduction over d padded to whole 32-steps with
// zeros.  Inputs are bf16 already, so the products are exact and only the
// fp32 accumulation order differs from a scalar loop; a dense basis costs the
// same as a block-diagonal one (64 MFMAs per edge at D = 49, C = 128).
//   A (rows c, reduction d): the edge's (C, D) row copied to LDS with 16-byte
//     moves; a lane's eight consecutive d of channel c start at element
//     c D + d0, which is 2-byte aligned only, so each fragment is five dword
//     reads shifted by v_alignbyte.
//   B (reduction d, columns j): eight d of basis column j, strided by D in
//     memory, read from global memory as 16-bit loads (the basis is read once).
//   D (rows c, columns j): lane holds four consecutive channels of one slot;
//     staged as [j][c] rows (stride C + 8 against bank conflicts) over the A
//     copy, then written with 16-byte stores in the slot-major output order.
template <int L, int C>
struct RotIn {
    static constexpr int D = (L + 1) * (L + 1), ROW = C * D;
    static constexpr int NCB = C / 16, NJB = (D + 15) / 16, KS = (D + 31) / 32;
    static constexpr int SST = C + 8;                                   // stage row stride
    static constexpr int BYTES_A = 2 * ROW + 16;                        // + the last fragment's over-read
    static constexpr int BYTES_S = 2 * D * SST;
    static constexpr int REG = ((BYTES_A > BYTES_S ? BYTES_A : BYTES_S) + 15) / 16 * 16;
    static constexpr int EPW = 4;                                       // edges per wave
};

template <int L, int C>
__global__ void __launch_bounds__(kT, 2)
k_hl_rot_in(int64_t E, const __bf16* __restrict__ in, const __bf16* __restrict__ R,
            const float* __restrict__ dist, float sigma, __bf16* __restrict__ out) {
    using RI = RotIn<L, C>;
    constexpr int D = RI::D, ROW = RI::ROW, NCB = RI::NCB, NJB = RI::NJB, KS = RI::KS;
    constexpr int SST = RI::SST, REG = RI::REG;
    static_assert(C % 16 == 0 && (2 * ROW) % 16 == 0 && (2 * SST) % 16 == 0, "tile shapes");
    __shared__ uint4 smem[4 * REG / 16];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int le = lane & 15, lg = lane >> 4;
    char* reg = reinterpret_cast<char*>(smem) + wave * REG;
    const uint32_t* rw = reinterpret_cast<const uint32_t*>(reg);
    __bf16* stage = reinterpret_cast<__bf16*>(reg);
    int lj[NJB];
#pragma unroll
    for (int jb = 0; jb < NJB; ++jb) {
        const int j = 16 * jb + le;
        lj[jb] = j < D ? SlotL<L>::l[j] : 0;
    }
    const int64_t w0 = (static_cast<int64_t>(blockIdx.x) * 4 + wave) * RI::EPW;
#pragma unroll 1
    for (int i = 0; i < RI::EPW; ++i) {
        const int64_t e = w0 + i;
        if (e >= E) break;
        // the edge's input row to LDS, every load issued before the first
        // write (the previous edge's stage reads are done: a wave's LDS
        // operations complete in issue order)
        const uint4* src = reinterpret_cast<const uint4*>(in + e * ROW);
        constexpr int NQ = (ROW / 8 + 63) / 64;
        uint4 xv[NQ];
#pragma unroll
        for (int n = 0; n < NQ; ++n) xv[n] = src[lane + 64 * n < ROW / 8 ? lane + 64 * n : ROW / 8 - 1];
#pragma unroll
        for (int n = 0; n < NQ; ++n)
            if (lane + 64 * n < ROW / 8) reinterpret_cast<uint4*>(reg)[lane + 64 * n] = xv[n];
        // B fragments: basis column j, rows d0 .. d0 + 7
        const unsigned short* Rs = reinterpret_cast<const unsigned short*>(R) + e * D * D;
        bf8 b[NJB][KS];
#pragma unroll
        for (int jb = 0; jb < NJB; ++jb)
#pragma unroll
            for (int s = 0; s < KS; ++s) {
                const int j = 16 * jb + le, d0 = 32 * s + 8 * lg;
                u16x8 v;
#pragma unroll
                for (int t = 0; t < 8; ++t)
                    v[t] = (j < D && d0 + t < D) ? Rs[(d0 + t) * D + j] : static_cast<unsigned short>(0);
                b[jb][s] = __builtin_bit_cast(bf8, v);
            }
        const float r = dist[e];
        const float sv = r / (r + sigma);
        asm volatile("" ::: "memory");
        const float s2 = sv * sv, s4 = s2 * s2;
        float pw[NJB];
#pragma unroll
        for (int jb = 0; jb < NJB; ++jb) pw[jb] = pow_sel(sv, s2, s4, lj[jb]);
        // A fragments: channel c, elements d0 .. d0 + 7 (zero past D)
        auto frag_a = [&](int cb, int s) -> bf8 {
            const int d0 = 32 * s + 8 * lg;
            uint32_t o[4] = {0u, 0u, 0u, 0u};
            if (d0 < D) {
                const int f0 = (16 * cb + le) * D + d0;
                const uint32_t* w = rw + (f0 >> 1);
                const uint32_t sh = static_cast<uint32_t>(f0 & 1) * 2u;
                uint32_t wv[5];
#pragma unroll
                for (int k = 0; k < 5; ++k) wv[k] = w[k];
#pragma unroll
                for (int k = 0; k < 4; ++k) o[k] = __builtin_amdgcn_alignbyte(wv[k + 1], wv[k], sh);
                if (32 * s + 32 > D) {   // the step that crosses D: zero elements d >= D
                    const int nv = D - d0;
#pragma unroll
                    for (int k = 0; k < 4; ++k)
                        o[k] &= (2 * k < nv ? 0x0000ffffu : 0u) | (2 * k + 1 < nv ? 0xffff0000u : 0u);
                }
            }
            return __builtin_bit_cast(bf8, (u32x4{o[0], o[1], o[2], o[3]}));
        };
        bf8 a[NCB][KS];
#pragma unroll
        for (int cb = 0; cb < NCB; ++cb)
#pragma unroll
            for (int s = 0; s < KS; ++s) a[cb][s] = frag_a(cb, s);
        asm volatile("" ::: "memory");
#pragma unroll
        for (int cb = 0; cb < NCB; ++cb)
#pragma unroll
            for (int jb = 0; jb < NJB; ++jb) {
                v4f acc = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int s = 0; s < KS; ++s) acc = mfma_bf(a[cb][s], b[jb][s], acc);
                const int j = 16 * jb + le;
                if (j < D) {
                    bf4 v;
#pragma unroll
                    for (int q = 0; q < 4; ++q) v[q] = static_cast<__bf16>(acc[q] * pw[jb]);
                    *reinterpret_cast<bf4*>(stage + j * SST + 16 * cb + 4 * lg) = v;
                }
            }
        asm volatile("" ::: "memory");
        uint4* dst = reinterpret_cast<uint4*>(out + e * ROW);
#pragma unroll
        for (int n = 0; n < NQ; ++n) {
            const int q = lane + 64 * n;
            if (q < ROW / 8) {
                const int j = q / (C / 8), c8 = q - j * (C / 8);
                dst[q] = *reinterpret_cast<const uint4*>(stage + j * SST + 8 * c8);
            }
        }
        asm volatile("" ::: "memory");
    }
}

// out[e, c, d] = sum_j R[e, d, j] s_e^{l(j)} in[e, j, c]   (y = (s^l ym) Q^T, dx = (s^l dfs) P^T)
//
// On the bf16 matrix cores, one edge per wave at a time: D[c][d] =
// sum_j v[j][c] R[d][j] with v = s^l in (float32) split into bf16 hi and lo
// parts (two products per step, 16 significant bits: far below the bf16
// rounding of the output) and the basis rows exact in bf16.
//   A (rows c, reduction j): eight j of channel c, strided by C floats in
//     memory, read as float32 and split;
//   B (reduction j, columns d): eight consecutive j of basis row d (2-byte
//     aligned), dword reads shifted by v_alignbyte;
//   D: lane holds slot d of four channels, staged in LDS as the output's
//     [c][d] rows and written with 16-byte stores.
// ---- constant GEMM operand --------------------------------------------------------
// bf16 A-operand fragments of C_k (TRANS = false: rows co, reduction ci) or C_k^T
// (rows ci, reduction co); C is (K, Cout, Cin).  Fragment (k, rb, ks) of lane l
// (row 16 rb + l % 16, reduction indices 32 ks + 8 (l / 16) + 0..7) at
// ((k * NRB + rb) * NKS + ks) * 64 + l.
template <bool TRANS>
__global__ void k_hl_prep(const float* __restrict__ C, int K, int cout, int cin,
                          bf8* __restrict__ frag) {
    const int nrow = TRANS ? cin : cout, nred = TRANS ? cout : cin;
    const int nrb = nrow / 16, nks = nred / 32;
    const int64_t q = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
    if (q >= static_cast<int64_t>(K) * nrb * nks * 64) return;
    const int l = static_cast<int>(q % 64), ks = static_cast<int>((q / 64) % nks);
    const int rb = static_cast<int>((q / 64 / nks) % nrb), k = static_cast<int>(q / 64 / nks / nrb);
    const int row = 16 * rb + (l & 15), c0 = 32 * ks + 8 * (l >> 4);
    const float* Ck = C + static_cast<int64_t>(k) * cout * cin;
    bf8 v;
#pragma unroll
    for (int j = 0; j < 8; ++j)
        v[j] = static_cast<__bf16>(TRANS ? Ck[(c0 + j) * cin + row] : Ck[row * cin + c0 + j]);
    frag[q] = v;
}

// Interpolated radial functions of a 16-edge tile: sF[(k WD + w) 16 + e]
// (zero for edges past the last), and the tile's bins.
template <int KW, int NT>
__device__ __forceinline__ void fill_tile_F(const feq_binning& B, int64_t E, int64_t e0,
                                            const float* __restrict__ dist,
                                            const float* __restrict__ F, float* sF, int* slo,
                                            float* st) {
    const int tid = threadIdx.x;
    if (tid < kNE) {
        const int64_t e = e0 + tid;
        const bool valid = e < E;
        const EdgeBin eb = edge_bin(valid ? dist[e] : 0.0f, B);
        slo[tid] = valid ? eb.lo : -1;
        st[tid] = eb.t;
    }
    __syncthreads();
    for (int q = tid; q < KW * kNE; q += NT) {
        const int ed = q % kNE, kw = q / kNE;
        const int lo = slo[ed];
        sF[q] = lo >= 0 ? lerp_bins(F[static_cast<int64_t>(lo) * KW + kw],
                                    F[static_cast<int64_t>(lo + 1) * KW + kw], st[ed])
                        : 0.0f;
    }
    __syncthreads();
}

// ---- the mix and the output rotation as chained matrix-core products ---------------
// The per-edge contraction with the radial functions (~13k VALU cycles per edge
// at C = 128 when done in registers) runs on the matrix cores, fed straight
// from the accumulators of the product before it:
//   stage 1  G^T[j, c] = sum_ci fs^T[j, ci] C_k^T[ci, c]   (16 slot rows x 16 channels
//            per v_mfma_f32_16x16x32_bf16; A: the edge's staged slot rows, B: the
//            C_k fragments of k_hl_prep held for the launch)
//   stage 2  ym^T[o, c] = sum_k sum_i M_ek[o, i] G_k^T[i, c]
//   stage 3  out[c, d] = sum_j R[d, j] s^l(j) ym[j, c]
// The accumulator layout of a 16 x 16 product (lane l holds rows 4 (l / 16) + r
// of column l % 16) is exactly the B-operand layout of the next product's
// reduction over those rows, so stages 2 and 3 take their B operands from the
// previous accumulators: stage 2 G rounded to bf16, two ranks per 32-step;
// stage 3 s^l ym split into bf16 hi and lo halves that share one 32-step (its
// A operand repeats its four values).  (G split into hi and lo as well measured
// 3.57 against 3.13 ms per forward at config 5 and moved the output's error
// against float64 from 5.2e-3 to 4.4e-3 of its largest entry, with a 2e-2
// bar.)  The slots are grouped into 16-row blocks that each hold whole m-groups
// (HLB), so M_ek -- block diagonal over m -- has only diagonal block tiles.  The
// A operands of stages 2 and 3 (the interpolated radial functions with the
// m-block signs, and the basis gathered at the block's slots) are built once
// per edge in LDS and read by every wave.  A workgroup of C / 16 waves takes
// one edge at a time (wave w owns the channels 16 w .. 16 w + 15).
// TRANS = false: fs^T -> y with C_k and Q (forward); TRANS = true: gd^T -> dx
// with C_k^T, M_ek^T and P (input gradient).
template <int L>
struct HLB {
    static constexpr int D = (L + 1) * (L + 1), NG = L + 1, MAXB = 8;
    struct Plan {
        int nb;
        int slot[MAXB][16];           // m-first slot of row r of block b, -1 for padding
        int deg[MAXB][16];            // its degree (0 for padding)
        short coef[MAXB][16][16];     // 2 w + neg of M_e[o row, i row] (-1: zero)
    };
    static constexpr Plan make() {
        Plan p{};
        for (int b = 0; b < MAXB; ++b)
            for (int r = 0; r < 16; ++r) {
                p.slot[b][r] = -1;
                p.deg[b][r] = 0;
                for (int c = 0; c < 16; ++c) p.coef[b][r][c] = -1;
            }
        int order[NG] = {}, size[NG] = {};
        for (int m = 0; m < NG; ++m) {
            order[m] = m;
            size[m] = (m ? 2 : 1) * (L - m + 1);
        }
        for (int a = 0; a < NG; ++a)                 // by size, largest first (stable)
            for (int c = a + 1; c < NG; ++c)
                if (size[order[c]] > size[order[a]]) {
                    const int t = order[a];
                    order[a] = order[c];
                    order[c] = t;
                }
        int fill[MAXB] = {}, blk[D] = {}, row[D] = {};
        p.nb = 0;
        for (int q = 0; q < NG; ++q) {               // first fit
            const int m = order[q];
            int b = 0;
            while (b < p.nb && fill[b] + size[m] > 16) ++b;
            if (b == p.nb) ++p.nb;
            for (int u = 0; u < size[m]; ++u) {
                const int s = Canon<L, L>::in_off(m) + u;
                p.slot[b][fill[b]] = s;
                p.deg[b][fill[b]] = SlotL<L>::l[s];
                blk[s] = b;
                row[s] = fill[b]++;
            }
        }
        for (int t = 0; t < Canon<L, L>::NT; ++t) {
            const Term tm = Canon<L, L>::terms[t];
            p.coef[blk[tm.o]][row[tm.o]][row[tm.i]] = static_cast<short>(2 * tm.w + tm.neg);
        }
        return p;
    }
    static constexpr Plan P = make();
    static constexpr int NB = P.nb;
};

__device__ __forceinline__ void split_bf(float v, __bf16& h, __bf16& l) {
    h = static_cast<__bf16>(v);
    l = static_cast<__bf16>(v - static_cast<float>(h));
}

template <int L, int C, int K, bool TRANS>
__global__ void __launch_bounds__(4 * C, 1)
k_hl_mixr(feq_binning B, int64_t E, const __bf16* __restrict__ src, const float* __restrict__ dist,
          const float* __restrict__ F, const bf8* __restrict__ frag, const __bf16* __restrict__ R,
          __bf16* __restrict__ out) {
    using HB = HLB<L>;
    constexpr int D = HB::D, NB = HB::NB, WD = HL<L>::WD, KW = K * WD;
    constexpr int NT = 4 * C, NW = C / 16, NKS = C / 32, NDB = (D + 15) / 16;
    constexpr int RS = 2 * C + 16;                              // LDS row stride in bytes (odd 16-byte units)
    constexpr int NQ = (D * C / 8 + NT - 1) / NT;               // 16-byte row chunks per thread
    constexpr int NF = (KW + NT - 1) / NT;                      // radial functions per thread
    constexpr int NRF = NDB * NB * 64, NCF = NB * K * 64;        // fragments per edge
    constexpr int NRI = (NRF + NT - 1) / NT;                    // basis fragments per thread
    constexpr int NCI = (NCF + NT - 1) / NT;                    // coefficient fragments per thread
    static_assert(C % 32 == 0 && NB <= HB::MAXB && D <= 16 * NDB, "shapes");
    __shared__ __align__(16) char sRows[2][(D + 1) * RS];   // + a zero row for padding
    __shared__ float sPow[2][8];                             // s^l, l <= 7
    __shared__ __align__(16) float sFe[2][KW];
    __shared__ __align__(16) u32x4 sCo[2][NCF];   // A fragments, four values repeated
    __shared__ __align__(16) u32x4 sR[2][NRF];
    __shared__ __align__(16) __bf16 sOut[NW][16 * D];

    const int tid = threadIdx.x, lane = tid & 63, le = lane & 15, lg = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

    // the rank fragments of this wave's 16 channels, for the launch
    bf8 Bk[K][NKS];
#pragma unroll
    for (int k = 0; k < K; ++k)
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) Bk[k][ks] = frag[((k * NW + wave) * NKS + ks) * 64 + lane];
    // per-lane rows of every block: the stage-1 A row (slot of row le) and the
    // degrees of the accumulator rows 4 lg + r
    // (padding rows read the zero row D; every per-lane choice below is an
    // address or a mask, never a condition, so that the compiler keeps no
    // launch-long lane masks in scalar registers)
    int arow[NB], adeg[NB][4];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        const int sl = HB::P.slot[b][le];
        arow[b] = (sl >= 0 ? sl : D) * RS;
#pragma unroll
        for (int r = 0; r < 4; ++r) adeg[b][r] = HB::P.deg[b][4 * lg + r];
    }
    // Table lookups of this thread's fragment items, once per launch, as 16-bit
    // fields two per register: the basis element offsets d D + j (0 where the
    // entry is zero, cleared by rmask), and for the coefficients the element k
    // WD + w of the radial functions (bits 0-13), its sign (bit 14) and
    // whether it is non-zero (bit 15)
    static_assert(D * D < 0x10000 && KW < 0x4000, "16-bit table fields");
    unsigned roff[NRI][2], rmask[NRI][2], ccode[NCI][2];
#pragma unroll
    for (int n = 0; n < NRI; ++n) {
        const int q = tid + NT * n;
        const int fl = q & 63, b = (q >> 6) % NB, db = (q >> 6) / NB;
        const int d = 16 * db + (fl & 15);
        unsigned v[4], m[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int j = q < NRF ? HB::P.slot[b][4 * (fl >> 4) + t] : -1;
            const bool ok = d < D && j >= 0;
            v[t] = ok ? static_cast<unsigned>(d * D + j) : 0u;
            m[t] = ok ? 0xffffu : 0u;
        }
        roff[n][0] = v[0] | (v[1] << 16);
        roff[n][1] = v[2] | (v[3] << 16);
        rmask[n][0] = m[0] | (m[1] << 16);
        rmask[n][1] = m[2] | (m[3] << 16);
    }
#pragma unroll
    for (int n = 0; n < NCI; ++n) {
        const int q = tid + NT * n;
        const int fl = q & 63, k = (q >> 6) % K, b = (q >> 6) / K;
        unsigned v[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int c = q >= NCF ? -1
                          : TRANS ? HB::P.coef[b][4 * (fl >> 4) + t][fl & 15]
                                  : HB::P.coef[b][fl & 15][4 * (fl >> 4) + t];
            v[t] = c < 0 ? 0u : static_cast<unsigned>(k * WD + (c >> 1)) | ((c & 1u) << 14) | 0x8000u;
        }
        ccode[n][0] = v[0] | (v[1] << 16);
        ccode[n][1] = v[2] | (v[3] << 16);
    }
    auto field = [](const unsigned (&w)[2], int t) -> unsigned { return (w[t >> 1] >> (16 * (t & 1))) & 0xffffu; };

    // Edge i of this workgroup is e_i = blockIdx.x + i gridDim.x.  Iteration i
    // computes e_i from LDS buffers i % 2 and, around that, prepares the
    // edges after it: it writes the slot rows and basis fragments of e_{i+1}
    // and the interpolated radial functions of e_{i+2} (loaded into
    // registers during iteration i - 1), builds the coefficient fragments of
    // e_{i+1} from the radial functions written during iteration i - 1, and
    // issues the loads of e_{i+2}'s rows and basis and of e_{i+3}'s radial
    // functions (whose bin needs e_{i+3}'s distance, loaded one iteration
    // earlier still).  One barrier per edge; the waves of a SIMD overlap one
    // edge's products with another's preparation.  Every load is unconditional
    // (indices clamped; what is loaded for edges past the last is not used).
    const int64_t stride = gridDim.x;
    auto edge = [&](int64_t i) -> int64_t {
        const int64_t e = blockIdx.x + i * stride;
        return e < E ? e : E - 1;
    };
    u32x4 pq[NQ];
    unsigned short pr[NRI][4];
    float pflo[NF], pfhi[NF], pt = 0.0f;
    auto load_rows = [&](int64_t e) {
        const u32x4* s4 = reinterpret_cast<const u32x4*>(src + e * D * C);
#pragma unroll
        for (int n = 0; n < NQ; ++n) {
            const int q = tid + NT * n;
            pq[n] = s4[q < D * C / 8 ? q : 0];
        }
        const unsigned short* Rb = reinterpret_cast<const unsigned short*>(R + e * D * D);
#pragma unroll
        for (int n = 0; n < NRI; ++n)
#pragma unroll
            for (int t = 0; t < 4; ++t) pr[n][t] = Rb[field(roff[n], t)];
    };
    auto load_radial = [&](float rd) {   // the two bin rows of an edge at distance rd
        const EdgeBin eb = edge_bin(rd, B);
        pt = eb.t;
        const float* flo = F + static_cast<int64_t>(eb.lo) * KW;
#pragma unroll
        for (int n = 0; n < NF; ++n) {
            const int q = tid + NT * n < KW ? tid + NT * n : 0;
            pflo[n] = flo[q];
            pfhi[n] = flo[q + KW];
        }
    };
    auto write_rows = [&](int buf) {
#pragma unroll
        for (int n = 0; n < NQ; ++n) {
            const int q = tid + NT * n;
            if ((D * C / 8) % NT == 0 || q < D * C / 8)
                *reinterpret_cast<u32x4*>(sRows[buf] + (q / (C / 8)) * RS + (q % (C / 8)) * 16) = pq[n];
        }
#pragma unroll
        for (int n = 0; n < NRI; ++n) {
            const int q = tid + NT * n;
            const unsigned lo = (pr[n][0] | (static_cast<unsigned>(pr[n][1]) << 16)) & rmask[n][0];
            const unsigned hi = (pr[n][2] | (static_cast<unsigned>(pr[n][3]) << 16)) & rmask[n][1];
            if (NRF % NT == 0 || q < NRF) sR[buf][q] = u32x4{lo, hi, lo, hi};
        }
    };
    auto write_radial = [&](int buf) {
#pragma unroll
        for (int n = 0; n < NF; ++n) {
            const int q = tid + NT * n;
            if (KW % NT == 0 || q < KW) sFe[buf][q] = lerp_bins(pflo[n], pfhi[n], pt);
        }
    };
    // stage-2 A fragments: M_ek (rows o = le, columns i = 4 lg + t) or M_ek^T
    auto build_coef = [&](int buf) {
#pragma unroll
        for (int n = 0; n < NCI; ++n) {
            const int q = tid + NT * n;
            if (NCF % NT == 0 || q < NCF) {
                unsigned v[4];
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const unsigned code = field(ccode[n], t);
                    unsigned u = __float_as_uint(sFe[buf][code & 0x3fffu]);
                    u = (u ^ ((code & 0x4000u) << 17)) & (0u - (code >> 15));
                    v[t] = __builtin_bit_cast(unsigned short, static_cast<__bf16>(__uint_as_float(u)));
                }
                const unsigned lo = v[0] | (v[1] << 16), hi = v[2] | (v[3] << 16);
                sCo[buf][q] = u32x4{lo, hi, lo, hi};
            }
        }
    };
    auto s_of = [&](float rd) { return rd / (rd + B.sh_scale); };

    // prologue: e_0's rows, basis, radial functions and coefficients, e_1's
    // radial functions in LDS; e_1's rows and basis and e_2's bin rows in
    // registers; the distances of e_2 and e_3 known
    float d0 = dist[edge(0)], d1 = dist[edge(1)];
    float s_cur = s_of(d0), s_n1 = s_of(d1);
    load_rows(edge(0));
    load_radial(d0);
    for (int q = tid; q < 2 * (RS / 16); q += NT)   // the zero rows
        *reinterpret_cast<u32x4*>(sRows[q / (RS / 16)] + D * RS + (q % (RS / 16)) * 16) = u32x4{0u, 0u, 0u, 0u};
    if (tid < 8) sPow[0][tid] = ipowf_small(s_cur, tid);
    write_rows(0);
    write_radial(0);
    load_radial(d1);
    write_radial(1);
    __syncthreads();
    build_coef(0);
    float d2 = dist[edge(2)];
    float s_n2 = s_of(d2);
    float dq = dist[edge(3)];
    load_rows(edge(1));
    load_radial(d2);

    // two iterations per trip, so that the buffer of each is a compile-time
    // constant (LDS addresses then fold into instruction offsets)
    auto iteration = [&](int64_t i, auto CB) __attribute__((always_inline)) {
        const int64_t e = blockIdx.x + i * stride;
        constexpr int cb = decltype(CB)::value, nb = cb ^ 1;
        __syncthreads();
        write_rows(nb);               // e_{i+1}
        write_radial(cb);             // e_{i+2}
        build_coef(nb);               // e_{i+1}, from its radial functions written last iteration
        if (tid < 8) sPow[nb][tid] = ipowf_small(s_n1, tid);
        s_cur = s_n1;
        s_n1 = s_n2;
        s_n2 = s_of(dq);
        load_rows(edge(i + 2));
        load_radial(dq);              // e_{i+3}
        dq = dist[edge(i + 4)];

        // stages 1 and 2 over the blocks, software-pipelined: the next block's
        // stage-1 products are issued before this block's splits and stage-2
        // products, which wait on the previous accumulators
        const char* rows = sRows[cb];
        const u32x4* coef = sCo[cb];
        const u32x4* rfr = sR[cb];
        bf8 ym[NB];   // s^l ym rows 4 lg + r of each block: hi in [0, 4), lo in [4, 8)
        v4f gacc[2][K];
        auto stage1 = [&](int b, v4f (&g)[K]) __attribute__((always_inline)) {
            bf8 a[NKS];
#pragma unroll
            for (int ks = 0; ks < NKS; ++ks)
                a[ks] = *reinterpret_cast<const bf8*>(rows + arow[b] + (32 * ks + 8 * lg) * 2);
#pragma unroll
            for (int k = 0; k < K; ++k) g[k] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
                for (int k = 0; k < K; ++k) g[k] = mfma_bf(a[ks], Bk[k][ks], g[k]);
        };
        const float* pw = sPow[cb];
        stage1(0, gacc[0]);
        static_for<NB>([&](auto BB) __attribute__((always_inline)) {
            constexpr int b = decltype(BB)::value, cur = b & 1;
            if constexpr (b + 1 < NB) stage1(b + 1, gacc[cur ^ 1]);
            v4f y = v4f{0.0f, 0.0f, 0.0f, 0.0f};
            // G rounded to bf16, two ranks per 32-step
#pragma unroll
            for (int k = 0; k < K; k += 2) {
                bf8 gb;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    gb[r] = static_cast<__bf16>(gacc[cur][k][r]);
                    gb[4 + r] = static_cast<__bf16>(gacc[cur][k + 1][r]);
                }
                const u32x4 c0 = coef[(b * K + k) * 64 + lane], c1 = coef[(b * K + k + 1) * 64 + lane];
                y = mfma_bf(__builtin_bit_cast(bf8, (u32x4{c0.x, c0.y, c1.x, c1.y})), gb, y);
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                __bf16 h, l;
                split_bf(y[r] * pw[adeg[b][r]], h, l);
                ym[b][r] = h;
                ym[b][4 + r] = l;
            }
        });
        // stage 3: out^T[d, c] for the 16-row blocks of d (independent
        // accumulators, one per d block), staged per wave and stored
        v4f o[NDB];
#pragma unroll
        for (int db = 0; db < NDB; ++db) o[db] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int db = 0; db < NDB; ++db)
                o[db] = mfma_bf(__builtin_bit_cast(bf8, rfr[(db * NB + b) * 64 + lane]), ym[b], o[db]);
        __bf16* so = sOut[wave];
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int d = 16 * db + 4 * lg + r;
                if (d < D) so[le * D + d] = static_cast<__bf16>(o[db][r]);
            }
        // the wave's 16 channel rows are contiguous in out: 16-byte stores
        asm volatile("" ::: "memory");
        constexpr int NCH = 16 * D * 2 / 16;
        uint4* dst = reinterpret_cast<uint4*>(out + (e * C + 16 * wave) * D);
        const uint4* s4o = reinterpret_cast<const uint4*>(so);
#pragma unroll
        for (int n = 0; n < (NCH + 63) / 64; ++n) {
            const int q = lane + 64 * n;
            if (q < NCH) dst[q] = s4o[q];
        }
        asm volatile("" ::: "memory");
    };
    for (int64_t i = 0; blockIdx.x + i * stride < E; i += 2) {
        iteration(i, std::integral_constant<int, 0>{});
        if (blockIdx.x + (i + 1) * stride >= E) break;
        iteration(i + 1, std::integral_constant<int, 1>{});
    }
}

// Sums of four per-lane values over the wave's four 16-lane rows: lane (row g,
// column c) returns the sum over rows of v[g] at column c (gfx950 lane swaps).
__device__ __forceinline__ float quad_row_sums(float v0, float v1, float v2, float v3) {
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v0), __float_as_uint(v1), false, false);
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v2), __float_as_uint(v3), false, false);
    const float s = __uint_as_float(p[0]) + __uint_as_float(p[1]);
    const float t = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    const auto z = __builtin_amdgcn_permlane32_swap(__float_as_uint(s), __float_as_uint(t), false, false);
    return __uint_as_float(z[0]) + __uint_as_float(z[1]);
}

// ---- per-edge radial-function gradient as chained matrix-core products ----------
// dF_e[k, w] = sum over the terms (o, i, w) of sign Z_k[o, i], with
//   Z_k[o, i] = sum_co gd^T[o, co] G_k[co, i],   G_k = C_k fs,
// where (o, i) ranges over the diagonal blocks of HLB (every term couples two
// slots of one m-group).  Stage 1 forms G_k for 16 channels x 16 slots per
// v_mfma_f32_16x16x32_bf16 (A: the C_k fragments held for the launch, B: the
// edge's staged fs^T slot rows); its accumulators (lane l: channels 4 (l / 16)
// + r of slot l % 16) are the B operand of stage 2's reduction over those
// channels, split into bf16 hi and lo halves that share one 32-step, with the
// edge's gd^T rows as the A operand.  Wave w owns rank k = w / H and the
// channels 64 h .. 64 h + 63, h = w % H (H = C / 64 waves per rank): the H
// partial Z_k of an edge go to LDS and are summed, and mapped to
// the radial functions' terms, in the next iteration, after its barrier.  The
// edge loop is pipelined as in k_hl_mixr: one barrier per edge, the next
// edge's rows loaded into registers while the current one is computed.
template <int L>
struct HLTerms {   // the (at most two) Z entries of every radial function w
    static constexpr int WD = Canon<L, L>::WD;
    struct Tab {
        int n[WD];
        int b[WD][2], ro[WD][2], ri[WD][2], neg[WD][2];
    };
    static constexpr Tab make() {
        Tab t{};
        using HB = HLB<L>;
        int blk[HB::D] = {}, row[HB::D] = {};
        for (int b = 0; b < HB::NB; ++b)
            for (int r = 0; r < 16; ++r)
                if (HB::P.slot[b][r] >= 0) {
                    blk[HB::P.slot[b][r]] = b;
                    row[HB::P.slot[b][r]] = r;
                }
        for (int q = 0; q < Canon<L, L>::NT; ++q) {
            const Term tm = Canon<L, L>::terms[q];
            const int j = t.n[tm.w]++;
            t.b[tm.w][j] = blk[tm.o];
            t.ro[tm.w][j] = row[tm.o];
            t.ri[tm.w][j] = row[tm.i];
            t.neg[tm.w][j] = tm.neg;
        }
        return t;
    }
    static constexpr Tab T = make();
};

template <int L, int C, int K>
__global__ void __launch_bounds__(4 * C, 1)
k_hl_dfer(int64_t E, const __bf16* __restrict__ fsT, const __bf16* __restrict__ gdT,
          const bf8* __restrict__ frag, float* __restrict__ dFe) {
    using HB = HLB<L>;
    using HT = HLTerms<L>;
    constexpr int D = HB::D, NB = HB::NB, WD = HL<L>::WD, KW = K * WD;
    constexpr int NT = 4 * C, NRB = C / 16, NKS = C / 32, H = C / 64;
    constexpr int RS = 2 * C + 16;                              // LDS row stride in bytes
    constexpr int NQ = (D * C / 8 + NT - 1) / NT;               // 16-byte row chunks per thread and operand
    constexpr int NI = (KW + NT - 1) / NT;                      // radial functions per thread
    constexpr int ZT = NB * 64;                                 // u32x4 of one wave's Z tiles
    static_assert(C % 64 == 0 && NT / 64 == K * H, "one wave per rank and 64 channels");
    static_assert(D * D < 0x10000, "16-bit table fields");
    __shared__ __align__(16) char sFs[2][(D + 1) * RS];          // + a zero row for padding
    __shared__ __align__(16) char sGd[2][(D + 1) * RS];
    __shared__ __align__(16) u32x4 sZ[2][K * H * ZT];

    const int tid = threadIdx.x, lane = tid & 63, le = lane & 15, lg = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wk = wave / H, wh = wave % H;

    // C_k rows of this wave's four 16-channel blocks, for the launch
    bf8 Ak[4][NKS];
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) Ak[c][ks] = frag[((wk * NRB + 4 * wh + c) * NKS + ks) * 64 + lane];
    int arow[NB];   // byte offset of the slot row of lane row le in each block (zero row for padding)
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        const int sl = HB::P.slot[b][le];
        arow[b] = (sl >= 0 ? sl : D) * RS;
    }
    // the Z entries of this thread's radial functions (k, w): LDS element
    // offsets (u32 units) within one buffer and their weights (the sign; 0
    // for the unused second entry of an m = 0 function)
    unsigned zoff[NI][2];
    float zw[NI][2];
#pragma unroll
    for (int n = 0; n < NI; ++n) {
        const int q = (tid + NT * n) % KW, k = q / WD, w = q % WD;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int jj = j < HT::T.n[w] ? j : 0;
            const int b = HT::T.b[w][jj], ro = HT::T.ro[w][jj], ri = HT::T.ri[w][jj];
            // Z[ro][ri] sits in lane 16 (ro / 4) + ri, component ro % 4, of tile (k, h, b)
            zoff[n][j] = static_cast<unsigned>(((k * H) * NB + b) * 64 * 4 + (16 * (ro / 4) + ri) * 4 + ro % 4);
            zw[n][j] = j < HT::T.n[w] ? (HT::T.neg[w][jj] ? -1.0f : 1.0f) : 0.0f;
        }
    }

    const int64_t stride = gridDim.x;
    auto edge = [&](int64_t i) -> int64_t {
        const int64_t e = blockIdx.x + i * stride;
        return e < E ? e : E - 1;
    };
    u32x4 pf[NQ], pg[NQ];
    auto load_rows = [&](int64_t e) {
        const u32x4* f4 = reinterpret_cast<const u32x4*>(fsT + e * D * C);
        const u32x4* g4 = reinterpret_cast<const u32x4*>(gdT + e * D * C);
#pragma unroll
        for (int n = 0; n < NQ; ++n) {
            const int q = tid + NT * n < D * C / 8 ? tid + NT * n : 0;
            pf[n] = f4[q];
            pg[n] = g4[q];
        }
    };
    auto write_rows = [&](int buf) {
#pragma unroll
        for (int n = 0; n < NQ; ++n) {
            const int q = tid + NT * n;
            if ((D * C / 8) % NT == 0 || q < D * C / 8) {
                const int off = (q / (C / 8)) * RS + (q % (C / 8)) * 16;
                *reinterpret_cast<u32x4*>(sFs[buf] + off) = pf[n];
                *reinterpret_cast<u32x4*>(sGd[buf] + off) = pg[n];
            }
        }
    };
    // dF_e of an edge from its Z partials (summed over the channel halves)
    auto emit = [&](int buf, int64_t e) {
        const unsigned* z = reinterpret_cast<const unsigned*>(sZ[buf]);
#pragma unroll
        for (int n = 0; n < NI; ++n) {
            const int q = tid + NT * n;
            float acc = 0.0f;
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int h = 0; h < H; ++h) acc = fmaf(zw[n][j], __uint_as_float(z[zoff[n][j] + h * ZT * 4]), acc);
            if (KW % NT == 0 || q < KW) dFe[e * KW + q] = acc;
        }
    };

    for (int q = tid; q < 2 * (RS / 16); q += NT) {   // the zero rows
        *reinterpret_cast<u32x4*>(sFs[q / (RS / 16)] + D * RS + (q % (RS / 16)) * 16) = u32x4{0u, 0u, 0u, 0u};
        *reinterpret_cast<u32x4*>(sGd[q / (RS / 16)] + D * RS + (q % (RS / 16)) * 16) = u32x4{0u, 0u, 0u, 0u};
    }
    load_rows(edge(0));
    write_rows(0);
    load_rows(edge(1));

    auto iteration = [&](int64_t i, auto CB) __attribute__((always_inline)) {
        constexpr int cb = decltype(CB)::value, nb = cb ^ 1;
        __syncthreads();
        write_rows(nb);                                  // e_{i+1}
        if (i > 0) emit(nb, blockIdx.x + (i - 1) * stride);   // e_{i-1}
        load_rows(edge(i + 2));
        const char* fr = sFs[cb];
        const char* gr = sGd[cb];
        u32x4* zo = sZ[cb] + (wk * H + wh) * ZT;
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            bf8 bfs[NKS];
#pragma unroll
            for (int ks = 0; ks < NKS; ++ks)
                bfs[ks] = *reinterpret_cast<const bf8*>(fr + arow[b] + (32 * ks + 8 * lg) * 2);
            v4f g[4];
#pragma unroll
            for (int c = 0; c < 4; ++c) g[c] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
                for (int c = 0; c < 4; ++c) g[c] = mfma_bf(Ak[c][ks], bfs[ks], g[c]);
            v4f z = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                // gd^T[o = slot(b, le)][channels 16 (4 h + c) + 4 lg .. + 3], twice (hi, lo)
                const uint2 a2 = *reinterpret_cast<const uint2*>(gr + arow[b] + (16 * (4 * wh + c) + 4 * lg) * 2);
                bf8 gb;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    __bf16 hh, ll;
                    split_bf(g[c][r], hh, ll);
                    gb[r] = hh;
                    gb[4 + r] = ll;
                }
                z = mfma_bf(__builtin_bit_cast(bf8, (u32x4{a2.x, a2.y, a2.x, a2.y})), gb, z);
            }
            zo[b * 64 + lane] = __builtin_bit_cast(u32x4, z);
        }
    };
    int64_t i = 0;
    for (; blockIdx.x + i * stride < E; i += 2) {
        iteration(i, std::integral_constant<int, 0>{});
        if (blockIdx.x + (i + 1) * stride >= E) {
            i += 1;
            break;
        }
        iteration(i + 1, std::integral_constant<int, 1>{});
    }
    // the last edge's Z (written into buffer (i - 1) % 2)
    __syncthreads();
    if (i > 0) emit(static_cast<int>((i - 1) & 1), blockIdx.x + (i - 1) * stride);
}

// ---- channel-pattern gradient as chained matrix-core products --------------------
// dC_k[co][ci] = sum over the edges e and slots i of U_k[co][i] fs[ci][i], with
// U_k = gd M_ek (U_k^T[i][co] = sum_o M_ek[o][i] gd^T[o][co], the transposed
// mixing of block_diagonal.cu:483-503), per edge in two chained bf16 products:
//   stage 1  U_k^T for the 16 slot rows of one HLB block (B: the edge's gd^T
//            rows of the block, k = the block's 16 o rows, the other 16 zero;
//            A: the per-edge M_ek^T fragment of the block, built in LDS);
//   stage 2  dC_k += U_k fs^T over the slots of two blocks per 32-step: the two
//            stage-1 accumulators (lane l: rows 4 (l / 16) + r of column co =
//            l % 16) rounded to bf16 are the A operand (rows co, reduction
//            (block, row)), the edge's fs^T rows of the same (block, row) pairs
//            the B operand.
// Both B operands read slot rows transposed straight from LDS with
// ds_read_b64_tr_b16: within a 16-lane group, lane s points at row s / 4 and
// 4-column chunk s % 4 of its read and receives 4 rows of one column (lane t:
// element j of row j, column t), so the rows may sit anywhere (the HLB block
// order is a per-lane address; padding rows point at a zero row).  A workgroup
// of C / 16 waves takes one edge at a time; wave w owns the output rows
// 16 w .. 16 w + 15 of every rank, its dC accumulators live for the launch,
// and each workgroup writes one partial dC.  The edge loop is pipelined as in
// k_hl_mixr: one barrier per edge, the rows of the next edge and the radial
// functions of the one after it loaded into registers during the current one.
typedef short v4s __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4s lds_v4s;

__device__ __forceinline__ bf8 tr_pair(const char* lo, const char* hi) {
    const v4s a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(lo));
    const v4s b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(hi));
    typedef short v8s __attribute__((ext_vector_type(8)));
    const v8s v = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
    return __builtin_bit_cast(bf8, v);
}

template <int C>
constexpr int dc_threads() { return 4 * C; }

template <int L, int C, int K>
__global__ void __launch_bounds__(dc_threads<C>(), 1)
k_hl_dcc(feq_binning B, int64_t E, const __bf16* __restrict__ gdT, const __bf16* __restrict__ fsT,
         const float* __restrict__ dist, const float* __restrict__ F, float* __restrict__ dCp) {
    using HB = HLB<L>;
    constexpr int D = HB::D, NB = HB::NB, WD = HL<L>::WD, KW = K * WD;
    constexpr int NT = dc_threads<C>(), NCB = C / 16, NPAIR = (NB + 1) / 2;
    constexpr int RS = 2 * C + 32;                  // row stride (bytes): consecutive rows 8 banks apart
    constexpr int NQ = (D * C / 8 + NT - 1) / NT;   // 16-byte row chunks per thread and tensor
    constexpr int NF = (KW + NT - 1) / NT;          // radial functions per thread
    constexpr int NCF = NB * K * 32;                // coefficient fragments (lane groups 0 and 1) per edge
    constexpr int NCI = (NCF + NT - 1) / NT;
    static_assert(K == 4 && C % 64 == 0 && NT <= 1024, "four ranks; 64 or 128 channels");
    static_assert(KW < 0x4000 && RS % 8 == 0, "16-bit coefficient codes; 8-byte transposed reads");
    __shared__ __align__(16) char sFs[2][(D + 1) * RS];   // + a zero row for padding
    __shared__ __align__(16) char sGd[2][(D + 1) * RS];
    __shared__ __align__(16) float sFe[2][KW];
    __shared__ __align__(16) u32x4 sCo[2][NCF];

    const int tid = threadIdx.x, lane = tid & 63, le = lane & 15, lg = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rsel = le >> 2, csel = le & 3;        // the row and 4-column chunk this lane points at
    const unsigned amask = lg < 2 ? 0xffffffffu : 0u;   // stage-1 A: reduction rows 16 .. 31 are zero

    // per-lane byte offsets of the transposed reads: stage-1 B (gd rows of
    // block b, rows 8 lg + 4 h + rsel; lane groups 2 and 3 read the zero row)
    // and stage-2 B (fs rows of pair p, block 2 p + h, rows 4 lg + rsel)
    int gdo[NB][2], fso[NPAIR][2];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int sl = lg < 2 ? HB::P.slot[b][8 * lg + 4 * h + rsel] : -1;
            gdo[b][h] = (sl >= 0 ? sl : D) * RS + 32 * wave + 8 * csel;
        }
#pragma unroll
    for (int p = 0; p < NPAIR; ++p)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int b = 2 * p + h;
            const int sl = b < NB ? HB::P.slot[b][4 * lg + rsel] : -1;
            fso[p][h] = (sl >= 0 ? sl : D) * RS + 8 * csel;
        }
    // this thread's coefficient fragment items: lane fl (groups 0, 1) of
    // fragment (b, k) holds M_ek^T[row fl % 16][row 8 (fl / 16) + t] of block
    // b, t < 8: the element k WD + w of the radial functions (bits 0-13), its
    // sign (bit 14), whether it is non-zero (bit 15); two per register
    unsigned ccode[NCI][4];
#pragma unroll
    for (int n = 0; n < NCI; ++n) {
        const int q = tid + NT * n;
        const int fl = q & 31, k = (q >> 5) % K, b = (q >> 5) / K;
        unsigned v[8];
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const int c = q < NCF ? HB::P.coef[b][8 * (fl >> 4) + t][fl & 15] : -1;
            v[t] = c < 0 ? 0u : static_cast<unsigned>(k * WD + (c >> 1)) | ((c & 1u) << 14) | 0x8000u;
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) ccode[n][t] = v[2 * t] | (v[2 * t + 1] << 16);
    }

    v4f acc[K][NCB];
#pragma unroll
    for (int k = 0; k < K; ++k)
#pragma unroll
        for (int cb = 0; cb < NCB; ++cb) acc[k][cb] = v4f{0.0f, 0.0f, 0.0f, 0.0f};

    // Edge i of this workgroup is e_i = blockIdx.x + i gridDim.x.  Iteration i
    // computes e_i from LDS buffers i % 2; around that it writes the rows of
    // e_{i+1} and the interpolated radial functions of e_{i+2} (loaded during
    // iteration i - 1), builds e_{i+1}'s coefficient fragments from its radial
    // functions (written during iteration i - 1), and loads e_{i+2}'s rows and
    // e_{i+3}'s bin rows.  Loads are unconditional (indices clamped).
    const int64_t stride = gridDim.x;
    auto edge = [&](int64_t i) -> int64_t {
        const int64_t e = blockIdx.x + i * stride;
        return e < E ? e : E - 1;
    };
    u32x4 pf[NQ], pg[NQ];
    float pflo[NF], pfhi[NF], pt = 0.0f;
    auto load_rows = [&](int64_t e) {
        const u32x4* f4 = reinterpret_cast<const u32x4*>(fsT + e * D * C);
        const u32x4* g4 = reinterpret_cast<const u32x4*>(gdT + e * D * C);
#pragma unroll
        for (int n = 0; n < NQ; ++n) {
            const int q = tid + NT * n;
            const int qq = q < D * C / 8 ? q : 0;
            pf[n] = f4[qq];
            pg[n] = g4[qq];
        }
    };
    auto load_radial = [&](float rd) {
        const EdgeBin eb = edge_bin(rd, B);
        pt = eb.t;
        const float* flo = F + static_cast<int64_t>(eb.lo) * KW;
#pragma unroll
        for (int n = 0; n < NF; ++n) {
            const int q = tid + NT * n < KW ? tid + NT * n : 0;
            pflo[n] = flo[q];
            pfhi[n] = flo[q + KW];
        }
    };
    auto write_rows = [&](int buf) {
#pragma unroll
        for (int n = 0; n < NQ; ++n) {
            const int q = tid + NT * n;
            if ((D * C / 8) % NT == 0 || q < D * C / 8) {
                const int off = (q / (C / 8)) * RS + (q % (C / 8)) * 16;
                *reinterpret_cast<u32x4*>(sFs[buf] + off) = pf[n];
                *reinterpret_cast<u32x4*>(sGd[buf] + off) = pg[n];
            }
        }
    };
    auto write_radial = [&](int buf) {
#pragma unroll
        for (int n = 0; n < NF; ++n) {
            const int q = tid + NT * n;
            if (KW % NT == 0 || q < KW) sFe[buf][q] = lerp_bins(pflo[n], pfhi[n], pt);
        }
    };
    auto build_coef = [&](int buf) {
#pragma unroll
        for (int n = 0; n < NCI; ++n) {
            const int q = tid + NT * n;
            if (NCF % NT == 0 || q < NCF) {
                unsigned w[4];
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    unsigned h2[2];
#pragma unroll
                    for (int u = 0; u < 2; ++u) {
                        const unsigned code = (ccode[n][t] >> (16 * u)) & 0xffffu;
                        unsigned x = __float_as_uint(sFe[buf][code & 0x3fffu]);
                        x = (x ^ ((code & 0x4000u) << 17)) & (0u - (code >> 15));
                        h2[u] = __builtin_bit_cast(unsigned short, static_cast<__bf16>(__uint_as_float(x)));
                    }
                    w[t] = h2[0] | (h2[1] << 16);
                }
                sCo[buf][q] = u32x4{w[0], w[1], w[2], w[3]};
            }
        }
    };

    // prologue: e_0's rows, radial functions and coefficients, e_1's radial
    // functions in LDS; e_1's rows and e_2's bin rows in registers
    float d0 = dist[edge(0)], d1 = dist[edge(1)];
    load_rows(edge(0));
    load_radial(d0);
    for (int q = tid; q < 2 * (RS / 16); q += NT) {   // the zero rows
        const int buf = q / (RS / 16), c = q % (RS / 16);
        *reinterpret_cast<u32x4*>(sFs[buf] + D * RS + c * 16) = u32x4{0u, 0u, 0u, 0u};
        *reinterpret_cast<u32x4*>(sGd[buf] + D * RS + c * 16) = u32x4{0u, 0u, 0u, 0u};
    }
    write_rows(0);
    write_radial(0);
    load_radial(d1);
    write_radial(1);
    __syncthreads();
    build_coef(0);
    float dq = dist[edge(3)];
    load_rows(edge(1));
    load_radial(dist[edge(2)]);

    auto iteration = [&](int64_t i, auto CB) __attribute__((always_inline)) {
        constexpr int cb = decltype(CB)::value, nb = cb ^ 1;
        __syncthreads();
        write_rows(nb);               // e_{i+1}
        write_radial(cb);             // e_{i+2}
        build_coef(nb);               // e_{i+1}, from its radial functions written last iteration
        load_rows(edge(i + 2));
        load_radial(dq);              // e_{i+3}
        dq = dist[edge(i + 4)];

        const char* fs = sFs[cb];
        const char* gd = sGd[cb];
        const u32x4* co = sCo[cb];
        const int cl = lane & 31;
#pragma unroll
        for (int p = 0; p < NPAIR; ++p) {
            // stage 1 for the pair's blocks, rounded into the stage-2 A operands
            bf8 a2[K];
#pragma unroll
            for (int k = 0; k < K; ++k) {
                v4f u[2] = {v4f{0.0f, 0.0f, 0.0f, 0.0f}, v4f{0.0f, 0.0f, 0.0f, 0.0f}};
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int b = 2 * p + h;
                    if (b < NB) {
                        u32x4 c = co[(b * K + k) * 32 + cl];
                        c &= amask;
                        const bf8 bg = tr_pair(gd + gdo[b][0], gd + gdo[b][1]);
                        u[h] = mfma_bf(__builtin_bit_cast(bf8, c), bg, u[h]);
                    }
                }
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    a2[k][r] = static_cast<__bf16>(u[0][r]);
                    a2[k][4 + r] = static_cast<__bf16>(u[1][r]);
                }
            }
            // stage 2: one fs fragment per column block serves the four ranks
#pragma unroll
            for (int c = 0; c < NCB; ++c) {
                const bf8 bf = tr_pair(fs + fso[p][0] + 32 * c, fs + fso[p][1] + 32 * c);
#pragma unroll
                for (int k = 0; k < K; ++k) acc[k][c] = mfma_bf(a2[k], bf, acc[k][c]);
            }
        }
    };
    for (int64_t i = 0; blockIdx.x + i * stride < E; i += 2) {
        iteration(i, std::integral_constant<int, 0>{});
        if (blockIdx.x + (i + 1) * stride >= E) break;
        iteration(i + 1, std::integral_constant<int, 1>{});
    }
    // partial dC of this workgroup: lane holds rows 4 lg + r of each 16-row block
    float* part = dCp + static_cast<int64_t>(blockIdx.x) * K * C * C;
#pragma unroll
    for (int k = 0; k < K; ++k)
#pragma unroll
        for (int c = 0; c < NCB; ++c)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int orow = 16 * wave + 4 * lg + r;
                part[(k * C + orow) * C + 16 * c + le] = acc[k][c][r];
            }
}

// ---- host side ----------------------------------------------------------------------------
constexpr int kRank = 4;
int grid_tiles(int64_t ntiles) {
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        cus = 256;
    return static_cast<int>(ntiles < cus ? ntiles : cus);
}

struct HLWs {
    bf8* cfrag;      // A fragments (C_k or C_k^T)
    __bf16* fsT;     // (E, D, Cin)
    __bf16* gdT;     // (E, D, Cout)               backward
    float* dFe;      // (E, K WD)                  backward
    float* dCp;      // (groups, K Cout, Cin)      backward: per-workgroup dC partials
    float* tail;     // ew_tail workspace          backward
};

// Workgroups of the channel-pattern gradient: one per CU (one edge at a time).
int dc_groups(int64_t E) { return grid_tiles(E); }

template <int L>
size_t hl_layout(const feq_binning& B, int C, int64_t E, bool backward, HLWs* w, void* base) {
    constexpr int D = HL<L>::D, KW = kRank * HL<L>::WD;
    const size_t nfrag = static_cast<size_t>(kRank) * C * C / 8;   // bf8 fragments
    size_t off = 0;
    char* p = static_cast<char*>(base);
    auto take = [&](size_t bytes) -> void* {
        void* r = p ? p + off : nullptr;
        off += align_up(bytes, 256);
        return r;
    };
    HLWs t{};
    t.cfrag = static_cast<bf8*>(take(nfrag * sizeof(bf8)));
    t.fsT = static_cast<__bf16*>(take(2 * static_cast<size_t>(E) * D * C));
    if (backward) {
        const int groups = dc_groups(E);
        t.gdT = static_cast<__bf16*>(take(2 * static_cast<size_t>(E) * D * C));
        t.dFe = static_cast<float*>(take(4 * static_cast<size_t>(E) * KW));
        t.dCp = static_cast<float*>(take(4 * static_cast<size_t>(groups) * kRank * C * C));
        t.tail = static_cast<float*>(take(4 * ew_tail_floats(B, KW, E, groups,
                                                             static_cast<int64_t>(kRank) * C * C)));
    }
    if (w) *w = t;
    return off + 256;
}

template <int L, int C>
int hl_rot_in(int64_t E, const __bf16* in, const __bf16* R, const float* dist, float sigma,
              __bf16* out, hipStream_t s) {
    auto kern = k_hl_rot_in<L, C>;
    FEQ_LAUNCH("k_hl_rot_in", kern, dim3(ceil_div(E, 4 * RotIn<L, C>::EPW)), dim3(kT), 0, s, E, in, R,
               dist, sigma, out);
    return FEQ_OK;
}

template <bool TRANS>
int hl_prep(const float* C, int K, int cout, int cin, bf8* frag, hipStream_t s) {
    const int64_t n = static_cast<int64_t>(K) * cout * cin / 8;
    auto kern = k_hl_prep<TRANS>;
    FEQ_LAUNCH("k_hl_prep", kern, dim3(ceil_div(n, 256)), dim3(256), 0, s, C, K, cout, cin, frag);
    return FEQ_OK;
}

template <int L, int CH>
int hl_fwd(const feq_binning& B, int64_t E, const __bf16* x, const __bf16* P, const __bf16* Q,
           const float* dist, const float* C, const float* F, __bf16* y, __bf16* fs_out, void* ws,
           size_t ws_bytes, hipStream_t s) {
    HLWs w;
    if (ws_bytes < hl_layout<L>(B, CH, E, false, &w, ws)) return fail(FEQ_ERR_WORKSPACE, "high-degree workspace too small");
    __bf16* fs = fs_out ? fs_out : w.fsT;
    if (int rc = hl_prep<false>(C, kRank, CH, CH, w.cfrag, s)) return rc;
    if (int rc = hl_rot_in<L, CH>(E, x, P, dist, B.sh_scale, fs, s)) return rc;
    auto mix = k_hl_mixr<L, CH, kRank, false>;
    FEQ_LAUNCH("k_hl_mix", mix, dim3(grid_tiles(E)), dim3(4 * CH), 0, s, B, E, fs, dist, F, w.cfrag, Q, y);
    return FEQ_OK;
}

template <int L, int CH>
int hl_bwd(const feq_layout& Lay, const feq_binning& B, int64_t E, const __bf16* gy, const __bf16* x,
           const __bf16* P, const __bf16* Q, const float* dist, const float* C, const float* F,
           __bf16* gx, float* gC, float* gF, float* gdist, const __bf16* fs_in, void* ws,
           size_t ws_bytes, hipStream_t s) {
    HLWs w;
    if (ws_bytes < hl_layout<L>(B, CH, E, true, &w, ws)) return fail(FEQ_ERR_WORKSPACE, "high-degree workspace too small");
    // gd = s^l_out (gy Q), fs = s^l_in (x P)
    if (int rc = hl_rot_in<L, CH>(E, gy, Q, dist, B.sh_scale, w.gdT, s)) return rc;
    const __bf16* fs = fs_in;
    if (!fs) {
        if (int rc = hl_rot_in<L, CH>(E, x, P, dist, B.sh_scale, w.fsT, s)) return rc;
        fs = w.fsT;
    }
    // dF_e from <gd, C_k fs>
    if (int rc = hl_prep<false>(C, kRank, CH, CH, w.cfrag, s)) return rc;
    auto kd = k_hl_dfer<L, CH, kRank>;
    FEQ_LAUNCH("k_hl_dfe", kd, dim3(grid_tiles(E)), dim3(4 * CH), 0, s, E, fs, w.gdT, w.cfrag, w.dFe);
    // dfs = sum_k M_ek^T C_k^T gd, dx = (s^l_in dfs) P^T
    if (gx) {
        if (int rc = hl_prep<true>(C, kRank, CH, CH, w.cfrag, s)) return rc;
        auto km = k_hl_mixr<L, CH, kRank, true>;
        FEQ_LAUNCH("k_hl_mix_t", km, dim3(grid_tiles(E)), dim3(4 * CH), 0, s, B, E, w.gdT, dist, F, w.cfrag,
                   P, gx);
    }
    // dC = sum over (e, i) of (M_ek^T gd) fs^T, per-workgroup partials; the
    // shared tail sums them in a fixed order with the binned radial-function
    // gradient and the distance gradient
    const int groups = dc_groups(E);
    auto kc = k_hl_dcc<L, CH, kRank>;
    FEQ_LAUNCH("k_hl_dc", kc, dim3(groups), dim3(dc_threads<CH>()), 0, s, B, E, w.gdT, fs, dist, F, w.dCp);
    return ew_tail(Lay, B, kRank, E, dist, F, w.dFe, w.dCp, groups, static_cast<int64_t>(kRank) * CH * CH,
                   gC, gF, gdist, w.tail, s);
}

bool canonical_pair(const feq_layout& L, int lmax) {
    int32_t lv[FEQ_MAX_BLOCKS];
    for (int i = 0; i <= lmax; ++i) lv[i] = i;
    feq_layout ref;
    if (feq_layout_init(&ref, lv, lmax + 1, lv, lmax + 1, L.cin, L.cout) != FEQ_OK) return false;
    if (ref.din != L.din || ref.dout != L.dout || ref.wdim != L.wdim || ref.nblocks != L.nblocks)
        return false;
    for (int k = 0; k < L.nblocks; ++k)
        for (int c = 0; c < 6; ++c)
            if (ref.blk[k][c] != L.blk[k][c]) return false;
    for (int q = 0; q < L.din; ++q)
        if (ref.lslot_in[q] != L.lslot_in[q] || ref.lslot_out[q] != L.lslot_out[q]) return false;
    return true;
}

// Shapes with a high-degree path: lvals 0..L in and out, Cin = Cout = CH, rank 4.
#define FEQ_HL_SHAPES(X) \
    X(6, 128)            \
    X(6, 64)

bool hl_supported(const feq_layout& L, const feq_binning& B, int rank) {
    if (rank != kRank || L.cin != L.cout) return false;
#define FEQ_SUP(l, ch) \
    if (L.cin == ch && canonical_pair(L, l)) return ew_tail_supported(B, kRank * HL<l>::WD);
    FEQ_HL_SHAPES(FEQ_SUP)
#undef FEQ_SUP
    return false;
}

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }  // NULL passes

}  // namespace
}  // namespace feq

using namespace feq;

extern "C" int feq_edgewise_hl_supported(const feq_layout* L, const feq_binning* b, int32_t rank) {
    if (!L || !b) return 0;
    return hl_supported(*L, *b, rank) ? 1 : 0;
}

extern "C" size_t feq_edgewise_hl_workspace(const feq_layout* L, const feq_binning* b, int32_t rank,
                                            int64_t E, int32_t backward) {
    if (!L || !b || !hl_supported(*L, *b, rank) || E < 0) return 0;
#define FEQ_WS(l, ch) \
    if (L->cin == ch && canonical_pair(*L, l)) return hl_layout<l>(*b, ch, E, backward != 0, nullptr, nullptr);
    FEQ_HL_SHAPES(FEQ_WS)
#undef FEQ_WS
    return 0;
}

extern "C" int feq_edgewise_hl_fwd(const feq_layout* L, const feq_binning* b, int32_t rank,
                                   int64_t E, const void* x, const void* P, const void* Q,
                                   const float* dist, const float* C, const float* F, void* y,
                                   void* fs_out, void* ws, size_t ws_bytes, feq_stream_t stream) {
    if (!L || !b) return fail(FEQ_ERR_INVALID, "NULL layout or binning");
    if (!hl_supported(*L, *b, rank)) return fail(FEQ_ERR_UNSUPPORTED, "no high-degree kernels for this layout");
    if (E < 0) return fail(FEQ_ERR_INVALID, "negative edge count");
    if (E == 0) return FEQ_OK;
    if (E > 0x7fffffffLL) return fail(FEQ_ERR_UNSUPPORTED, "more than 2^31-1 edges");
    if (!x || !P || !Q || !dist || !C || !F || !y || !ws) return fail(FEQ_ERR_INVALID, "NULL pointer");
    if (!al16(x) || !al16(y) || !al16(ws) || !al16(fs_out))
        return fail(FEQ_ERR_INVALID, "x, y, fs_out and the workspace must be 16-byte aligned");
    hipStream_t s = stream_of(stream);
    const auto* xb = static_cast<const __bf16*>(x);
    const auto* Pb = static_cast<const __bf16*>(P);
    const auto* Qb = static_cast<const __bf16*>(Q);
#define FEQ_FWD(l, ch) \
    if (L->cin == ch && canonical_pair(*L, l)) \
        return hl_fwd<l, ch>(*b, E, xb, Pb, Qb, dist, C, F, static_cast<__bf16*>(y), \
                             static_cast<__bf16*>(fs_out), ws, ws_bytes, s);
    FEQ_HL_SHAPES(FEQ_FWD)
#undef FEQ_FWD
    return fail(FEQ_ERR_UNSUPPORTED, "no high-degree kernels for this layout");
}

extern "C" int feq_edgewise_hl_bwd(const feq_layout* L, const feq_binning* b, int32_t rank,
                                   int64_t E, const void* gy, const void* x, const void* P,
                                   const void* Q, const float* dist, const float* C, const float* F,
                                   void* gx, float* gC, float* gF, float* gdist,
                                   const void* fs_in, void* ws, size_t ws_bytes,
                                   feq_stream_t stream) {
    if (!L || !b) return fail(FEQ_ERR_INVALID, "NULL layout or binning");
    if (!hl_supported(*L, *b, rank)) return fail(FEQ_ERR_UNSUPPORTED, "no high-degree kernels for this layout");
    if (E < 0) return fail(FEQ_ERR_INVALID, "negative edge count");
    if (E > 0x7fffffffLL) return fail(FEQ_ERR_UNSUPPORTED, "more than 2^31-1 edges");
    if (!gC || !gF) return fail(FEQ_ERR_INVALID, "grad_C and grad_F are required");
    hipStream_t s = stream_of(stream);
    if (E == 0) {
        if (int rc = fill_zero(gF, static_cast<int64_t>(b->num_bins + 1) * rank * L->wdim, s)) return rc;
        return fill_zero(gC, static_cast<int64_t>(rank) * L->cout * L->cin, s);
    }
    if (!gy || !x || !P || !Q || !dist || !C || !F || !ws) return fail(FEQ_ERR_INVALID, "NULL pointer");
    if (!al16(gy) || !al16(x) || !al16(gx) || !al16(ws) || !al16(fs_in))
        return fail(FEQ_ERR_INVALID, "gy, x, gx, fs_in and the workspace must be 16-byte aligned");
    const auto* gyb = static_cast<const __bf16*>(gy);
    const auto* xb = static_cast<const __bf16*>(x);
    const auto* Pb = static_cast<const __bf16*>(P);
    const auto* Qb = static_cast<const __bf16*>(Q);
#define FEQ_BWD(l, ch) \
    if (L->cin == ch && canonical_pair(*L, l)) \
        return hl_bwd<l, ch>(*L, *b, E, gyb, xb, Pb, Qb, dist, C, F, static_cast<__bf16*>(gx), gC, gF, \
                             gdist, static_cast<const __bf16*>(fs_in), ws, ws_bytes, s);
    FEQ_HL_SHAPES(FEQ_BWD)
#undef FEQ_BWD
    return fail(FEQ_ERR_UNSUPPORTED, "no high-degree kernels for this layout");
}

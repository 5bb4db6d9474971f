// Fused EquivariantEdgewiseLinear with its GEMMs on the fp16 matrix cores of
// gfx950, at fp32 accuracy.
//
// Same mathematics as edgewise.hip: with the separable
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

// split_f16(a * sc) with both halves formed by fused multiply-adds with a
// half-precision result (v_fma_mix): hi = fp16(a sc), lo = fp16(a sc - hi),
// where a sc - hi is exact inside the fma.  sc is a power of two, so a sc is
// exact and the halves equal split_f16's.
__device__ __forceinline__ void split_f16s(float a, float sc, _Float16& hi, _Float16& lo) {
    hi = static_cast<_Float16>(__builtin_fmaf(a, sc, 0.0f));
    lo = static_cast<_Float16>(__builtin_fmaf(a, sc, -static_cast<float>(hi)));
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
    // the thread's eight fragment values are requested before the rank's
    // maximum (they do not depend on its scale): one memory latency, not two
    const int l = tid & 63, ks = tid >> 6;
    const int row = 16 * rb + (l & 15), c0 = 32 * ks + 8 * (l >> 4);
    float av[8];
    if (tid < NKS * 64) {
#pragma unroll
        for (int jj = 0; jj < 8; ++jj)
            // A = C_k (row co, reduction ci) or C_k^T (row ci, reduction co); C is (K, Cout, Cin)
            av[jj] = TRANS ? Ck[(c0 + jj) * NROW + row] : Ck[row * NRED + c0 + jj];
    }
    static_assert(NCH % kThreads == 0, "whole rows of the rank per thread");
    float v = 0.0f;
#pragma unroll
    for (int r = 0; r < NCH / kThreads; ++r) v = fmaxf(v, fabsf(Ck[tid + r * kThreads]));
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
        h8 hi, lo;
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) {
            _Float16 h, lw;
            split_f16s(av[jj], sc, h, lw);
            hi[jj] = h;
            lo[jj] = lw;
        }
        const int q = ((k * NRB + rb) * NKS + ks) * 64 + l;
        frag[2 * q] = hi;
        frag[2 * q + 1] = lo;
    }
}

// Rows of the layer input: row e of x, or, in the message-passing form, row
// src[e] of a node table of nsrc rows (the gather x[src] done inside the
// kernels).  x_row returns the row an edge reads, or -1 for an index outside
// [0, nsrc), which reads as a zero row.
struct XRows {
    const float* x;
    const int64_t* src;
    int64_t nsrc;
};

template <bool GATHER>
__device__ __forceinline__ int64_t x_row(const XRows& X, int64_t e) {
    if constexpr (!GATHER) {
        return e;
    } else {
        const int64_t r = X.src[e];
        return r >= 0 && r < X.nsrc ? r : -1;
    }
}

__device__ __forceinline__ bool node_crosses_tiles(int b, int e) { return b / kNE != (e - 1) / kNE; }

// Rows e0 + j (j < kNE) of a (E, N) tensor, or rows perm[e0 + j] (PERM):
// thread t reads elements t % 16 + 16 k of row t / 16 (one index lookup per
// thread; a row of N floats need not be 16-byte aligned), zeros past the last
// edge.  (Fewer registers in flight than 16-byte loads of the tile's block.)
template <int N>
constexpr int rows_per_thread() { return (N + 15) / 16; }

template <int N, bool PERM>
__device__ __forceinline__ void load_rows(const float* __restrict__ src, int64_t e0, int64_t E,
                                          const int32_t* __restrict__ perm,
                                          float (&v)[rows_per_thread<N>()]) {
    static_assert(kThreads == 16 * kNE, "16 threads per edge row");
    const int j = threadIdx.x >> 4, c = threadIdx.x & 15;
    const bool ok = e0 + j < E;
    int64_t r = 0;
    if (ok) {
        if constexpr (PERM) r = perm[e0 + j]; else r = e0 + j;
    }
    const float* row = src + r * N;
#pragma unroll
    for (int k = 0; k < rows_per_thread<N>(); ++k) {
        const int idx = c + 16 * k;
        v[k] = (ok && idx < N) ? row[idx] : 0.0f;
    }
}

// load_rows for a row index already known (row r, ok = the position is in range).
template <int N>
__device__ __forceinline__ void load_row_at(const float* __restrict__ src, int64_t r, bool ok,
                                            float (&v)[rows_per_thread<N>()]) {
    const int c = threadIdx.x & 15;
    const float* row = src + (ok ? r : 0) * N;
#pragma unroll
    for (int k = 0; k < rows_per_thread<N>(); ++k) {
        const int idx = c + 16 * k;
        v[k] = (ok && idx < N) ? row[idx] : 0.0f;
    }
}

// Stores rows read by load_rows into LDS with a row stride of S floats.
template <int N, int S>
__device__ __forceinline__ void store_rows(const float (&v)[rows_per_thread<N>()], float* dst) {
    const int j = threadIdx.x >> 4, c = threadIdx.x & 15;
#pragma unroll
    for (int k = 0; k < rows_per_thread<N>(); ++k) {
        const int idx = c + 16 * k;
        if (idx < N) dst[j * S + idx] = v[k];
    }
}

// Row stride (floats) of a tile of kNE rows of n floats staged in LDS: a
// multiple of 4 (16-byte rows) with an odd number of 16-byte units, so 16-byte
// accesses of consecutive rows hit distinct banks.
constexpr int stage_stride(int n) { return ((n + 3) / 4 | 1) * 4; }

// Writes this lane's 4 rows x D floats (rows c0 .. c0 + 3 of edge le, contiguous
// in global memory) into the staging tile, whose edge rows hold CH * D floats.
template <int CH, int D>
__device__ __forceinline__ void stage_rows(float* stage, int le, int c0, const float (&out)[4 * D]) {
    float4* dst = reinterpret_cast<float4*>(stage + le * stage_stride(CH * D) + c0 * D);
#pragma unroll
    for (int v = 0; v < D; ++v) dst[v] = make_float4(out[4 * v], out[4 * v + 1], out[4 * v + 2], out[4 * v + 3]);
}

// Copies the staged tile (nval edges) to its contiguous global rows with
// fully coalesced 16-byte stores.
template <int CH, int D>
__device__ __forceinline__ void flush_stage(const float* stage, float* __restrict__ g, int nval) {
    constexpr int ROW4 = CH * D / 4, SS4 = stage_stride(CH * D) / 4;
    static_assert((CH * D) % 4 == 0, "rows of whole float4s");
    const float4* s4 = reinterpret_cast<const float4*>(stage);
    float4* g4 = reinterpret_cast<float4*>(g);
    if (nval == kNE) {
#pragma unroll
        for (int n = 0; n < kNE * ROW4 / kThreads; ++n) {
            const int q = threadIdx.x + kThreads * n;
            g4[q] = s4[(q / ROW4) * SS4 + q % ROW4];
        }
        if constexpr ((kNE * ROW4) % kThreads != 0) {
            const int q = threadIdx.x + kThreads * (kNE * ROW4 / kThreads);
            if (q < kNE * ROW4) g4[q] = s4[(q / ROW4) * SS4 + q % ROW4];
        }
    } else {
        for (int q = threadIdx.x; q < nval * ROW4; q += kThreads) g4[q] = s4[(q / ROW4) * SS4 + q % ROW4];
    }
}

// flush_stage with the rows scattered: staged row j goes to global row rows[j].
template <int CH, int D>
__device__ __forceinline__ void flush_stage_rows(const float* stage, float* __restrict__ g,
                                                 const int32_t* __restrict__ rows, int nval) {
    constexpr int ROW4 = CH * D / 4, SS4 = stage_stride(CH * D) / 4;
    static_assert((CH * D) % 4 == 0, "rows of whole float4s");
    const float4* s4 = reinterpret_cast<const float4*>(stage);
    float4* g4 = reinterpret_cast<float4*>(g);
    for (int q = threadIdx.x; q < nval * ROW4; q += kThreads) {
        const int j = q / ROW4, c = q % ROW4;
        g4[static_cast<int64_t>(rows[j]) * ROW4 + c] = s4[j * SS4 + c];
    }
}

// The staged tile's rows (nval edges, source nodes node[j], -1 for none) summed
// per node in tile order: a node within the tile gets its row, a node that
// crosses a tile boundary a partial row (NodeScatter).  node[kNE] and
// node[kNE + 1] are the nodes of the positions just before and just after the
// tile (-1 for none): a run crosses a boundary when it starts the tile and
// continues the previous position's node, or ends the tile and the next
// position continues it (the CSR offsets give the same answer, at the price of
// dependent global loads in the epilogue).
template <int CH, int D>
__device__ __forceinline__ void scatter_stage(const float* stage, const int* node, const NodeScatter& NS,
                                              int64_t tile, int nval) {
    constexpr int ROW4 = CH * D / 4, SS4 = stage_stride(CH * D) / 4;
    static_assert((CH * D) % 4 == 0, "rows of whole float4s");
    const float4* s4 = reinterpret_cast<const float4*>(stage);
    float4* out4 = reinterpret_cast<float4*>(NS.out);
    float4* part4 = reinterpret_cast<float4*>(NS.part);
    for (int q = threadIdx.x; q < ROW4; q += kThreads) {
        float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        int js = 0;   // first position of the current node's run
        for (int j = 0; j < nval; ++j) {
            const float4 v = s4[j * SS4 + q];
            acc.x += v.x;
            acc.y += v.y;
            acc.z += v.z;
            acc.w += v.w;
            const int n = node[j];
            if (j + 1 < nval && node[j + 1] == n) continue;
            if (n >= 0) {
                if ((js == 0 && n == node[kNE]) || (j + 1 == kNE && n == node[kNE + 1]))
                    part4[(2 * tile + (js == 0 ? 0 : 1)) * ROW4 + q] = acc;
                else
                    out4[static_cast<int64_t>(n) * ROW4 + q] = acc;
            }
            acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            js = j + 1;
        }
    }
}

// scatter_stage for the pooled forward: row j of the staged tile weighted by
// w[j][head] (w: kPoolMaxHeads floats per position) before the per-node sums
// by destination.  A float4 of a row lies within one head (hc * D % 4 == 0,
// checked by the host).
template <int CH, int D>
__device__ __forceinline__ void scatter_stage_w(const float* stage, const int* node, const float* w,
                                                const DstPool& DP, int64_t tile, int nval) {
    constexpr int ROW4 = CH * D / 4, SS4 = stage_stride(CH * D) / 4;
    static_assert((CH * D) % 4 == 0, "rows of whole float4s");
    const float4* s4 = reinterpret_cast<const float4*>(stage);
    float4* out4 = reinterpret_cast<float4*>(DP.out);
    float4* part4 = reinterpret_cast<float4*>(DP.part);
    for (int q = threadIdx.x; q < ROW4; q += kThreads) {
        const int hq = (4 * q) / (DP.hc * D);
        const int h = hq < DP.heads ? hq : DP.heads - 1;
        float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        int js = 0;   // first position of the current node's run
        for (int j = 0; j < nval; ++j) {
            const float4 v = s4[j * SS4 + q];
            const float a = w[j * kPoolMaxHeads + h];
            acc.x += a * v.x;
            acc.y += a * v.y;
            acc.z += a * v.z;
            acc.w += a * v.w;
            const int n = node[j];
            if (j + 1 < nval && node[j + 1] == n) continue;
            if (n >= 0) {
                if ((js == 0 && n == node[kNE]) || (j + 1 == kNE && n == node[kNE + 1]))
                    part4[(2 * tile + (js == 0 ? 0 : 1)) * ROW4 + q] = acc;
                else
                    out4[static_cast<int64_t>(n) * ROW4 + q] = acc;
            }
            acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            js = j + 1;
        }
    }
}

// Destination node of an edge of the pooled form, -1 outside [0, ndst).
__device__ __forceinline__ int64_t pool_node(const DstPool& DP, int64_t e) {
    const int64_t n = DP.dst[e];
    return n >= 0 && n < DP.ndst ? n : -1;
}

// Head of output channel c in the pooled form.
__device__ __forceinline__ int pool_head(const DstPool& DP, int c) {
    const int h = c / DP.hc;
    return h < DP.heads ? h : DP.heads - 1;
}

// Rows of the nodes that scatter_stage did not write: the sums of the partial
// rows of a node that crosses tile boundaries (in tile order), zeros for a node
// without edges.  One 64-lane workgroup per node.
__global__ void __launch_bounds__(64)
k_ews_node_fix(NodeScatter NS, int64_t row4) {
    const int64_t n = blockIdx.x;
    const int b = NS.offsets[n], e = NS.offsets[n + 1];
    if (b < e && !node_crosses_tiles(b, e)) return;
    const float4* part4 = reinterpret_cast<const float4*>(NS.part);
    float4* out4 = reinterpret_cast<float4*>(NS.out);
    for (int64_t q = threadIdx.x; q < row4; q += 64) {
        float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (b < e) {
            const int t0 = b / kNE, t1 = (e - 1) / kNE;
            for (int t = t0; t <= t1; ++t) {
                const int slot = (t == t0 && b % kNE != 0) ? 1 : 0;
                const float4 v = part4[(2 * static_cast<int64_t>(t) + slot) * row4 + q];
                acc.x += v.x;
                acc.y += v.y;
                acc.z += v.z;
                acc.w += v.w;
            }
        }
        out4[n * row4 + q] = acc;
    }
}

// Degree of m-first slot j of a canonical representation (4-bit packed table).
template <int L>
struct SlotDegPacked {
    static constexpr int D = (L + 1) * (L + 1), NW = (D + 15) / 16;
    static constexpr std::array<unsigned long long, NW> make() {
        std::array<unsigned long long, NW> w{};
        for (int j = 0; j < D; ++j)
            w[j / 16] |= static_cast<unsigned long long>(SlotL<L>::l[j]) << (4 * (j % 16));
        return w;
    }
    static constexpr std::array<unsigned long long, NW> words = make();
};

template <int L>
__device__ __forceinline__ int slot_degree(int j) {
    using S = SlotDegPacked<L>;
    unsigned long long w = S::words[0];
#pragma unroll
    for (int n = 1; n < S::NW; ++n) w = (j >> 4) == n ? S::words[n] : w;
    return static_cast<int>((w >> (4 * (j & 15))) & 15u);
}

__device__ __forceinline__ int std_degree(int d, int L) {
    int l = 0;
    for (int k = 1; k <= L; ++k) l += d >= k * k;
    return l;
}

// Bit k set when element t % 16 + 16 k of a (D, D) basis row (this thread's
// share, as read by load_rows) lies outside the degree blocks.  The positions
// are the same for every tile, so this runs once per launch.
template <int L>
__device__ __forceinline__ unsigned off_block_bits_rows() {
    constexpr int D = (L + 1) * (L + 1), N = D * D;
    static_assert(rows_per_thread<N>() <= 32, "one bit per element");
    unsigned bits = 0;
#pragma unroll
    for (int k = 0; k < rows_per_thread<N>(); ++k) {
        const int pos = (threadIdx.x & 15) + 16 * k;
        const bool off = pos < N && std_degree(pos / D, L) != slot_degree<L>(pos % D);
        bits |= static_cast<unsigned>(off) << k;
    }
    return bits;
}

// 1 when an element of this share that lies outside the degree blocks (bits
// from off_block_bits_rows) is non-zero (-0 counts as zero).
template <int NR>
__device__ __forceinline__ int off_block_nonzero_rows(const float (&v)[NR], unsigned bits) {
    unsigned acc = 0;
#pragma unroll
    for (int k = 0; k < NR; ++k) acc |= ((bits >> k) & 1u) ? __float_as_uint(v[k]) : 0u;
    return (acc & 0x7fffffffu) != 0;
}

// Sums of four per-lane values over the wave's four 16-lane rows: lane
// (row g, column c) returns sum over rows of v[g] at column c.  Two
// v_permlane16_swap (odd rows of the first operand <-> even rows of the second)
// and one v_permlane32_swap (upper half of the first <-> lower half of the
// second) instead of eight cross-lane shuffles.
// Sum over the 16 lanes of a row (every lane receives it): lane swaps within
// quads, then the half-row and row mirrors (DPP).
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp_f<0xB1>(v);    // quad_perm [1, 0, 3, 2]
    v += dpp_f<0x4E>(v);    // quad_perm [2, 3, 0, 1]
    v += dpp_f<0x141>(v);   // row_half_mirror: quads 0 <-> 1, 2 <-> 3
    v += dpp_f<0x140>(v);   // row_mirror: half-rows 0 <-> 1
    return v;
}

__device__ __forceinline__ float quad_lane_sums(const float (&v)[4]) {
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v[0]), __float_as_uint(v[1]), false, false);
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v[2]), __float_as_uint(v[3]), false, false);
    // rows of s: v0 (0+1), v1 (0+1), v0 (2+3), v1 (2+3); of t likewise for v2, v3
    const float s = __uint_as_float(p[0]) + __uint_as_float(p[1]);
    const float t = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    const auto z = __builtin_amdgcn_permlane32_swap(__float_as_uint(s), __float_as_uint(t), false, false);
    return __uint_as_float(z[0]) + __uint_as_float(z[1]);
}

// out[r][j] = sum_d x[r][d] R[d][j] for NR rows (x P, gy Q).  SPARSE sums only
// the degree block of column j.
template <int L, bool SPARSE, int NR>
__device__ __forceinline__ void rotate_cols(const float* __restrict__ x, const float* re,
                                            float (&out)[NR][(L + 1) * (L + 1)]) {
    constexpr int D = (L + 1) * (L + 1);
#pragma unroll
    for (int r = 0; r < NR; ++r)
#pragma unroll
        for (int j = 0; j < D; ++j) out[r][j] = 0.0f;
    if constexpr (SPARSE) {
        static_for<D>([&](auto JJ) {
            constexpr int j = decltype(JJ)::value, l = SlotL<L>::l[j];
#pragma unroll
            for (int d = l * l; d < (l + 1) * (l + 1); ++d) {
                const float rv = re[d * D + j];
#pragma unroll
                for (int r = 0; r < NR; ++r) out[r][j] += x[r * D + d] * rv;
            }
        });
    } else {
#pragma unroll
        for (int d = 0; d < D; ++d)
#pragma unroll
            for (int j = 0; j < D; ++j) {
                const float rv = re[d * D + j];
#pragma unroll
                for (int r = 0; r < NR; ++r) out[r][j] += x[r * D + d] * rv;
            }
    }
}

// out[r][d] = sum_j R[d][j] v(r, j) for 4 rows (y = v Q^T, dx = v P^T);
// v(r, j) = vin[j][r].  SPARSE sums only the degree block of row d.
template <int L, bool SPARSE>
__device__ __forceinline__ void rotate_rows(const float (&vin)[(L + 1) * (L + 1)][4], const float* re,
                                            float (&out)[4 * (L + 1) * (L + 1)]) {
    constexpr int D = (L + 1) * (L + 1);
    using DB = DegreeBlocks<L>;
    static_for<D>([&](auto DD) {
        constexpr int d = decltype(DD)::value, l = DB::deg(d);
        float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if constexpr (SPARSE) {
#pragma unroll
            for (int n = l * l; n < (l + 1) * (l + 1); ++n) {
                const int j = DB::slots[n];
                const float rv = re[d * D + j];
#pragma unroll
                for (int r = 0; r < 4; ++r) a[r] += vin[j][r] * rv;
            }
        } else {
#pragma unroll
            for (int j = 0; j < D; ++j) {
                const float rv = re[d * D + j];
#pragma unroll
                for (int r = 0; r < 4; ++r) a[r] += vin[j][r] * rv;
            }
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) out[r * D + d] = a[r];
    });
}

// Solid-harmonic factors.  Every term (i -> o, w) of the mixing matrix joins
// degrees l_in(w) and l_out(w), so the forward and input-gradient kernels fold
// the factors s^l_in of the input slots and s^l_out of the output slots into
// the per-edge radial functions, F'_e[k, w] = F_e[k, w] s_e^(l_in(w) + l_out(w)),
// and use the rotated rows unscaled (the channel-pattern kernel scales its rows:
// measured faster there, its register allocation being tighter).  The powers s_e^l, l <= LIN + LOUT, of a tile's edges sit in
// LDS; the threads filling F' serve one fixed (k, w) each (so the degree sum
// of a thread is fixed for the launch) and the edges t / KW, t / KW + G, ...
__device__ __forceinline__ void edge_powers(float s, int n, float* out) {
    float p = 1.0f;
    for (int l = 0; l < n; ++l) {
        out[l] = p;
        p *= s;
    }
}

// ---------------------------------------------------------------------------
// Forward: y = Q-rotate(s^l_out sum_k M_ek G_k), G_k = C_k fs, fs = s^l_in (x P).
// A workgroup owns one 16-edge tile at a time; wave w owns output rows
// co = 16 (w + 4 j) + ..., j < Cout / 64.  Per tile: (1) P, Q and edge state
// to LDS, and a test whether every off-block entry of the tile's P and Q is
// zero (then the rotations sum over the degree blocks only); (2) fs rows are
// rotated by threads that own 4 channels of one edge, scaled per edge, split
// and written as fp16 fragments; (3) one pass over the slots with the A
// fragments of every rank component in registers: per slot i the 3-term MFMA
// products are contracted into y (registers); (4) the next tile's global loads
// are issued, then the Q rotation, staged in LDS and stored with coalesced
// 16-byte stores.  Row strides of the per-edge LDS blocks are odd, so the 16
// edges of a wave's lanes hit distinct banks.
//
// POOL (message-passing form only): tile positions walk the CSR by destination
// (DP.perm), and the staged tile is summed per destination node with the
// attention weights (scatter_stage_w) instead of stored per edge; y, when not
// NULL, receives the unweighted rows in that position order.
template <int CIN, int COUT, int LIN, int LOUT, int K, int OCC, bool GATHER, bool LP, bool POOL,
          bool YM = false>
__global__ void __launch_bounds__(kThreads, OCC)
k_ews_fwd(feq_binning B, int64_t E, int64_t ntiles, XRows X,
          const float* __restrict__ P, const float* __restrict__ Q,
          const float* __restrict__ dist, const h8* __restrict__ Cfrag,
          const float* __restrict__ Cinv, const float* __restrict__ F, float* __restrict__ y,
          DstPool DP, float* __restrict__ ym) {
    static_assert(GATHER || !POOL, "the pooled form is a message-passing form");
    using T = Canon<LIN, LOUT>;
    using TG = TermGroups<LIN, LOUT, false>;
    constexpr int DIN = T::DIN, DOUT = T::DOUT, WD = T::WD, KW = K * WD;
    constexpr int PS = DIN * DIN | 1, QS = DOUT * DOUT | 1, KWS = KW | 1;
    constexpr int NSP = LIN + LOUT + 1, FG = kThreads / KW;
    static_assert(KW <= kThreads, "one radial (k, w) per fill thread");
    constexpr int RPW = COUT / 64, NKS = CIN / 32, NC4 = CIN / 4;
    constexpr int KP = K;                                        // rank components per pass
    constexpr int CHUNK = 1024;                                  // bytes per fragment chunk
    constexpr int NPR = (kNE * NC4 + kThreads - 1) / kThreads;   // producer passes
    static_assert(COUT % 64 == 0 && CIN % 32 == 0 && NC4 <= 64, "unsupported channel counts");
    static_assert((kNE * NC4) % kThreads == 0 || kNE * NC4 < kThreads, "producer split");

    constexpr int BREG = 2 * DIN * NKS * CHUNK > 4 * kNE * stage_stride(COUT * DOUT)
                             ? 2 * DIN * NKS * CHUNK : 4 * kNE * stage_stride(COUT * DOUT);
    extern __shared__ float4 smem4[];
    char* sB = reinterpret_cast<char*>(smem4);                   // [2][DIN][NKS] chunks, then the y stage
    float* sP = reinterpret_cast<float*>(sB + BREG);
    float* sQ = sP + kNE * PS;
    float* sFe = sQ + kNE * QS;
    float* sSout = sFe + kNE * KWS;                              // 1 / scale_e
    float* sSp = sSout + kNE;                                    // s_e^l, l < NSP
    float* sInvK = sSp + kNE * NSP;
    EdgeState* sE = reinterpret_cast<EdgeState*>(sInvK + K);
    int* sNode = reinterpret_cast<int*>(sE + kNE);               // destination per position, + 2 neighbours (POOL)
    float* sW = reinterpret_cast<float*>(sNode + kNE + 4);       // [kNE][kPoolMaxHeads] weights (POOL)

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform (scalar)
    const int le = lane & 15, lg = lane >> 4;
    const unsigned pbits = off_block_bits_rows<LIN>(), qbits = off_block_bits_rows<LOUT>();
    const int fkw = tid % KW, fe0 = tid / KW, fl = T::wl_of(fkw % WD);   // radial fill: fixed (k, w)

    if (tid < K) sInvK[tid] = Cinv[tid];   // read after the first tile barrier

    // global loads of one tile (zeros past the last edge)
    float xr[NPR][4 * DIN];
    float pr[rows_per_thread<DIN * DIN>()], qr[rows_per_thread<DOUT * DOUT>()];
    float rd;
    int nd = -1;       // POOL: destination of position tid (tid < kNE; kNE, kNE + 1: the neighbours)
    float wt = 0.0f;   // POOL: weight (position tid / kPoolMaxHeads, head tid % kPoolMaxHeads)
    static_assert(kNE * kPoolMaxHeads <= kThreads, "one weight per thread");
    auto load_tile = [&](int64_t t) {
        const int64_t f0 = t * kNE;
        // Every index first (the source rows, the CSR permutation for the P, Q
        // and attention rows, the positions' destinations and distances): the
        // in-order memory counter then waits once for all of them before the
        // rows they point to are requested.  Without POOL the P and Q rows are
        // the tile's own and only the source rows are indexed.
        int64_t xrow[NPR];
#pragma unroll
        for (int p = 0; p < NPR; ++p) {
            const int q = tid + kThreads * p;
            const int e = q / NC4;
            xrow[p] = q < kNE * NC4 && f0 + e < E ? x_row<GATHER>(X, f0 + e) : -1;
        }
        const int rj = tid >> 4;                     // the P / Q / attention row of this thread
        const bool rok = f0 + rj < E;
        int64_t re = f0 + rj;
        if constexpr (POOL) {
            re = rok ? DP.perm[f0 + rj] : 0;
            // positions f0 .. f0 + kNE - 1, then f0 - 1 and f0 + kNE (the neighbours)
            const int64_t pn = tid < kNE ? f0 + tid : tid == kNE ? f0 - 1 : f0 + kNE;
            nd = (tid < kNE + 2 && pn >= 0 && pn < E) ? DP.node_pos[pn] : -1;
            rd = (tid < kNE && f0 + tid < E) ? DP.dist_pos[f0 + tid] : 1.0f;
        } else {
            rd = (tid < kNE && f0 + tid < E) ? dist[f0 + tid] : 1.0f;
        }
#pragma unroll
        for (int p = 0; p < NPR; ++p) {
            const int q = tid + kThreads * p;
            const int c4 = q % NC4;
            if (xrow[p] >= 0) {
                const float4* src = reinterpret_cast<const float4*>(X.x + (xrow[p] * CIN + 4 * c4) * DIN);
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
        load_row_at<DIN * DIN>(P, re, rok, pr);
        load_row_at<DOUT * DOUT>(Q, re, rok, qr);
        if constexpr (POOL) {
            const int wh = tid % kPoolMaxHeads;       // weight (position rj, head wh)
            static_assert(kPoolMaxHeads == 16, "the weight row of a thread is its P / Q row");
            wt = (rok && wh < DP.heads) ? DP.attn[re * DP.heads + wh] : 0.0f;
        }
    };

    // fs rows of this thread: rotation, per-edge scale, split, fragment writes
    auto produce = [&](auto sparse) {
        constexpr bool SP = decltype(sparse)::value;
#pragma unroll
        for (int p = 0; p < NPR; ++p) {
            const int q = tid + kThreads * p;
            const int e = q / NC4, c4 = q % NC4;
            const bool act = q < kNE * NC4;
            const int ee = act ? e : 0;
            float fs[4][DIN];
            rotate_cols<LIN, SP, 4>(xr[p], sP + ee * PS, fs);
            float m = 0.0f;
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int i = 0; i < DIN; ++i) m = fmaxf(m, fabsf(fs[r][i]));
#pragma unroll
            for (int off = NC4 / 2; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
            const int ex = scale_exp(m);
            const float sc = exp2i(ex);
            if (act && c4 == 0) sSout[e] = exp2i(-ex);
            if (act) {
                const int ks = c4 / 8, g = (c4 / 2) % 4, half = c4 % 2;
                char* base = sB + ks * CHUNK + bslot(g, e) + 8 * half;
#pragma unroll
                for (int i = 0; i < DIN; ++i) {
                    h4 hv, lv;
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        _Float16 h, l;
                        if constexpr (LP) {
                            h = static_cast<_Float16>(fs[r][i] * sc);
                        } else {
                            split_f16s(fs[r][i], sc, h, l);
                            lv[r] = l;
                        }
                        hv[r] = h;
                    }
                    *reinterpret_cast<h4*>(base + (i * NKS) * CHUNK) = hv;
                    if constexpr (!LP) *reinterpret_cast<h4*>(base + ((DIN + i) * NKS) * CHUNK) = lv;
                }
            }
        }
    };

    load_tile(blockIdx.x);
    for (int64_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
        const int64_t e0 = tile * kNE;
        __syncthreads();   // the previous tile's readers of every LDS buffer are done
        // (1) P, Q and edge state to LDS; block-structure test of the tile
        store_rows<DIN * DIN, PS>(pr, sP);
        store_rows<DOUT * DOUT, QS>(qr, sQ);
        if (tid < kNE) {
            EdgeState es;
            es.valid = e0 + tid < E;
            const EdgeBin eb = edge_bin(rd, B);
            es.lo = eb.lo;
            es.t = eb.t;
            es.s = rd / (rd + B.sh_scale);
            sE[tid] = es;
            edge_powers(es.s, NSP, sSp + tid * NSP);
        }
        if constexpr (POOL) {
            if (tid < kNE + 2) sNode[tid] = nd;
            sW[tid] = wt;
        }
        const bool dense =
            __syncthreads_or(off_block_nonzero_rows(pr, pbits) | off_block_nonzero_rows(qr, qbits)) != 0;

        // (2) radial functions of the tile (1/scale_k folded in) and fs fragments
        if (fe0 < FG) {
            const float ik = sInvK[fkw / WD];
            for (int e = fe0; e < kNE; e += FG) {
                const EdgeState es = sE[e];
                const float* flo = F + static_cast<int64_t>(es.lo) * KW + fkw;
                sFe[e * KWS + fkw] = lerp_bins(flo[0], flo[KW], es.t) * ik * sSp[e * NSP + fl];
            }
        }
        if (dense)
            produce(std::false_type{});
        else
            produce(std::true_type{});
        __syncthreads();

        // (3) GEMM per input slot, all rank components (KP = K) in one pass
        float yv[RPW][DOUT][4];
#pragma unroll
        for (int j = 0; j < RPW; ++j)
#pragma unroll
            for (int o = 0; o < DOUT; ++o)
#pragma unroll
                for (int r = 0; r < 4; ++r) yv[j][o][r] = 0.0f;
        const float* fe = sFe + le * KWS;
        const int myslot = bslot(lg, le);
        static_for<K / KP>([&](auto PP) {
            constexpr int k0 = decltype(PP)::value * KP;
            // A fragments of this pass (L2-resident); the opaque pointer keeps
            // the loads inside the tile loop
            const h8* cfr = Cfrag;
            asm volatile("" : "+s"(cfr));
            h8 ahi[RPW][KP][NKS], alo[RPW][KP][NKS];
#pragma unroll
            for (int j = 0; j < RPW; ++j)
#pragma unroll
                for (int kk = 0; kk < KP; ++kk)
#pragma unroll
                    for (int ks = 0; ks < NKS; ++ks) {
                        const h8* src =
                            cfr + 2 * ((((k0 + kk) * (COUT / 16) + wave + 4 * j) * NKS + ks) * 64 + lane);
                        ahi[j][kk][ks] = src[0];
                        if constexpr (!LP) alo[j][kk][ks] = src[1];
                    }
            // Software pipeline over the slots: iteration i issues the MFMAs of
            // slot i + 1 (B fragments loaded one iteration earlier) and the
            // fragment loads of slot i + 2, then contracts slot i, so matrix and
            // vector work of one wave overlap.  The fence at the end of each
            // iteration keeps the compiler from hoisting later slots' loads.
            h8 bh[2][NKS], bl[2][NKS];
            v4f acc[2][RPW][KP];
            auto load_b = [&](int slot, int buf) {
#pragma unroll
                for (int ks = 0; ks < NKS; ++ks) {
                    bh[buf][ks] = *reinterpret_cast<const h8*>(sB + (slot * NKS + ks) * CHUNK + myslot);
                    if constexpr (!LP)
                        bl[buf][ks] = *reinterpret_cast<const h8*>(sB + ((DIN + slot) * NKS + ks) * CHUNK + myslot);
                }
            };
            auto mfma_slot = [&](int buf, int ab) {
#pragma unroll
                for (int j = 0; j < RPW; ++j)
#pragma unroll
                    for (int kk = 0; kk < KP; ++kk) acc[ab][j][kk] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
                    for (int j = 0; j < RPW; ++j)
#pragma unroll
                        for (int kk = 0; kk < KP; ++kk) {
                            if constexpr (!LP) {
                                acc[ab][j][kk] = mfma_h(alo[j][kk][ks], bh[buf][ks], acc[ab][j][kk]);
                                acc[ab][j][kk] = mfma_h(ahi[j][kk][ks], bl[buf][ks], acc[ab][j][kk]);
                            }
                            acc[ab][j][kk] = mfma_h(ahi[j][kk][ks], bh[buf][ks], acc[ab][j][kk]);
                        }
            };
            load_b(0, 0);
            if constexpr (DIN > 1) load_b(1, 1);
            mfma_slot(0, 0);
            static_for<DIN>([&](auto I) {
                constexpr int i = decltype(I)::value;
                constexpr int cur = i & 1;
                if constexpr (i + 1 < DIN) mfma_slot(cur ^ 1, cur ^ 1);
                if constexpr (i + 2 < DIN) load_b(i + 2, cur);
                static_for<TG::count(i)>([&](auto TT) {
                    constexpr Term tm = TG::sorted[TG::start[i] + decltype(TT)::value];
#pragma unroll
                    for (int kk = 0; kk < KP; ++kk) {
                        const float f = fe[(k0 + kk) * WD + tm.w];
                        const float c = tm.neg ? -f : f;
#pragma unroll
                        for (int j = 0; j < RPW; ++j)
#pragma unroll
                            for (int r = 0; r < 4; ++r) yv[j][tm.o][r] += c * acc[cur][j][kk][r];
                    }
                });
                // Pin the contraction to this iteration: without these (empty)
                // read-modify-write uses the compiler defers it past later
                // slots' MFMAs and keeps their results live.
#pragma unroll
                for (int j = 0; j < RPW; ++j)
#pragma unroll
                    for (int o = 0; o < DOUT; ++o)
#pragma unroll
                        for (int r = 0; r < 4; ++r) asm volatile("" : "+v"(yv[j][o][r]));
                __builtin_amdgcn_sched_barrier(0);
            });
        });

        // (4) next tile's global loads, then output scaling, Q rotation and stores
        load_tile(tile + gridDim.x);
        const float* qe = sQ + le * QS;
        {
            const float sc = sSout[le];
#pragma unroll
            for (int o = 0; o < DOUT; ++o)
#pragma unroll
                for (int j = 0; j < RPW; ++j)
#pragma unroll
                    for (int r = 0; r < 4; ++r) yv[j][o][r] *= sc;
        }
        __syncthreads();   // every wave is done with the fragments: the buffer becomes the y stage
#pragma unroll
        for (int j = 0; j < RPW; ++j) {
            float out[4 * DOUT];
            if (dense)
                rotate_rows<LOUT, false>(yv[j], qe, out);
            else
                rotate_rows<LOUT, true>(yv[j], qe, out);
            stage_rows<COUT, DOUT>(reinterpret_cast<float*>(sB), le, 16 * (wave + 4 * j) + 4 * lg, out);
        }
        __syncthreads();
        const int nval = static_cast<int>(E - e0 < kNE ? E - e0 : kNE);
        if (!POOL || y) flush_stage<COUT, DOUT>(reinterpret_cast<const float*>(sB), y + e0 * COUT * DOUT, nval);
        if constexpr (POOL)
            scatter_stage_w<COUT, DOUT>(reinterpret_cast<const float*>(sB), sNode, sW, DP, tile, nval);
        if constexpr (YM) {
            // the rows before the rotation (the block-diagonal output m, y = m
            // Q^T), kept for the gradient of Q: staged and stored like y
            __syncthreads();   // the y stage is read
#pragma unroll
            for (int j = 0; j < RPW; ++j) {
                float out[4 * DOUT];
#pragma unroll
                for (int o = 0; o < DOUT; ++o)
#pragma unroll
                    for (int r = 0; r < 4; ++r) out[r * DOUT + o] = yv[j][o][r];
                stage_rows<COUT, DOUT>(reinterpret_cast<float*>(sB), le, 16 * (wave + 4 * j) + 4 * lg, out);
            }
            __syncthreads();
            if constexpr (POOL)   // rows in edge order: tile row e is edge DP.perm[e0 + e]
                flush_stage_rows<COUT, DOUT>(reinterpret_cast<const float*>(sB), ym, DP.perm + e0, nval);
            else
                flush_stage<COUT, DOUT>(reinterpret_cast<const float*>(sB), ym + e0 * COUT * DOUT, nval);
        }
    }
}

// ---------------------------------------------------------------------------
// Input gradient: H_k = C_k^T gd (M = Cin, N = 16 Dout, K = Cout) with
// gd = s^l_out (gy Q), then in registers
//   dfs[ci, i] = sum_k sum_o M_ek[o][i] H_k[ci, o]      dx = s^l_in dfs P^T
//   dF_e[k, w] = sum_ci sum_{terms (o, i, w)} sign fs[ci, i] H_k[ci, o]
// (the per-edge radial-function gradient, binned afterwards), where
// fs = s^l_in (x P) is built directly in the accumulator layout: lane
// (le, lg) of wave w holds rows ci = 16 (w + 4 j) + 4 lg + r of edge le.
// gd is scaled per edge and split into fp16 fragments like fs in the forward;
// C_k^T comes pre-split from k_ews_prep (same per-rank scale as C_k), one pass
// of KP rank components at a time.  At the end of a pass its dF_e partials are
// summed over the wave's four lane groups with lane swaps (four values per
// register), unscaled, and summed over the four waves in LDS.  Rotations use the degree blocks when the tile's P
// and Q have no entry off them; dx is staged in LDS and stored coalesced.
//
// GP (pooled form): gy is the pooled output's gradient (ndst rows) and edge e
// reads attn[e, head(c)] gy[dst[e], c, :] (DstPool).
template <int CIN, int COUT, int LIN, int LOUT, int K, bool GATHER, bool SCATTER, bool LP, bool GP,
          bool GPQ = false>
__global__ void __launch_bounds__(kThreads, 2)
k_ews_bwd_x(feq_binning B, int64_t E, int64_t ntiles, const float* __restrict__ gy,
            XRows X, const float* __restrict__ P,
            const float* __restrict__ Q, const float* __restrict__ dist,
            const h8* __restrict__ Cfrag, const float* __restrict__ Cinv,
            const float* __restrict__ F, float* __restrict__ gx, float* __restrict__ dFe,
            NodeScatter NS, DstPool DP, const float* __restrict__ ym, float* __restrict__ gPo,
            float* __restrict__ gQo) {
    static_assert(GATHER || !SCATTER, "the per-node sums need the message-passing form");
    static_assert(SCATTER || !GP, "the pooled form sums the input gradient per source node");
    using T = Canon<LIN, LOUT>;
    using TG = TermGroups<LIN, LOUT, true>;
    constexpr int DIN = T::DIN, DOUT = T::DOUT, WD = T::WD, KW = K * WD;
    constexpr int PS = DIN * DIN | 1, QS = DOUT * DOUT | 1, KWS = KW | 1;
    constexpr int NSP = LIN + LOUT + 1, FG = kThreads / KW;
    static_assert(KW <= kThreads, "one radial (k, w) per fill thread");
    // One rank component per GEMM pass: measured on MI355X at 160k edges, 432 us
    // against 457 us with passes of two (whose extra A fragments and
    // accumulators spill at two workgroups per CU) and 567 us for one pass at
    // one workgroup per CU.
    constexpr int KP = 1;
    constexpr int RPW = CIN / 64, NKS = COUT / 32, NC4 = COUT / 4;
    constexpr int CHUNK = 1024;
    constexpr int NPR = (kNE * NC4 + kThreads - 1) / kThreads;
    constexpr int BREG = 2 * DOUT * NKS * CHUNK > 4 * kNE * stage_stride(CIN * DIN)
                             ? 2 * DOUT * NKS * CHUNK : 4 * kNE * stage_stride(CIN * DIN);
    static_assert(CIN % 64 == 0 && COUT % 32 == 0 && NC4 <= 64, "unsupported channel counts");
    static_assert((kNE * NC4) % kThreads == 0 || kNE * NC4 < kThreads, "producer split");

    extern __shared__ float4 smem4[];
    char* sB = reinterpret_cast<char*>(smem4);                   // gd fragments, then the dx stage
    float* sP = reinterpret_cast<float*>(sB + BREG);
    float* sQ = sP + kNE * PS;
    float* sFe = sQ + kNE * QS;
    float* sDF = sFe + kNE * KWS;                                 // [4 waves][kNE][KW]
    float* sSp = sDF + 4 * kNE * KW;                              // s_e^l, l < NSP
    float* sEinv = sSp + kNE * NSP;                               // 1 / scale_e
    float* sInvK = sEinv + kNE;
    EdgeState* sE = reinterpret_cast<EdgeState*>(sInvK + K);
    int* sNode = reinterpret_cast<int*>(sE + kNE);                // source node per position, + 2 neighbours (SCATTER)
    int* sEid = sNode + kNE + 4;                                  // edge per position (SCATTER)

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform (scalar)
    const int le = lane & 15, lg = lane >> 4;
    const unsigned pbits = off_block_bits_rows<LIN>(), qbits = off_block_bits_rows<LOUT>();
    const int fkw = tid % KW, fe0 = tid / KW, fl = T::wl_of(fkw % WD);   // radial fill: fixed (k, w)
    if (tid < K) sInvK[tid] = Cinv[tid];

    // global loads of one tile: gy rows of the producer threads, x rows of the
    // lane layout, P, Q, distances (zeros past the last edge)
    float gr[NPR][4 * DOUT];
    float gw[NPR];   // GP: attention weight of the producer's channels (0 without a destination)
    int64_t gqe[NPR];   // GPQ: the producer's edge (-1: none)
    float xl[RPW][4 * DIN];
    // P and Q of the prefetched tile: each thread's share of one edge row
    float prs[rows_per_thread<DIN * DIN>()], qrs[rows_per_thread<DOUT * DOUT>()];
    float rd;
    int nd = -1, eid = 0;   // SCATTER: source node of position tid (and neighbours), edge of position tid
    auto load_tile = [&](int64_t t) {
        const int64_t f0 = t * kNE;
        // Every index first (position-ordered arrays with SCATTER, see the
        // forward), then the rows they point to.
        int64_t grow[NPR];   // row of gy each producer reads (-1: none)
        int64_t gedge[NPR];  // GP: the producer's edge (its attention weights)
#pragma unroll
        for (int p = 0; p < NPR; ++p) {
            const int q = tid + kThreads * p;
            const int e = q / NC4;
            const bool valid = q < kNE * NC4 && f0 + e < E;
            gedge[p] = 0;
            if constexpr (GP) {
                grow[p] = valid ? NS.dnode_pos[f0 + e] : -1;
                gedge[p] = valid ? NS.perm[f0 + e] : 0;
            } else if constexpr (SCATTER) {
                grow[p] = valid ? NS.perm[f0 + e] : -1;
            } else {
                grow[p] = valid ? f0 + e : -1;
            }
            // GPQ: the producer's edge (with GP the gy row is its destination's)
            if constexpr (GPQ) gqe[p] = GP ? (valid ? gedge[p] : -1) : grow[p];
        }
        int64_t xrow[RPW];
#pragma unroll
        for (int j = 0; j < RPW; ++j) {
            if constexpr (SCATTER)
                xrow[j] = f0 + le < E ? NS.src_pos[f0 + le] : -1;
            else
                xrow[j] = f0 + le < E ? x_row<GATHER>(X, f0 + le) : -1;
        }
        const int rj = tid >> 4;                     // the P / Q row of this thread
        const bool rok = f0 + rj < E;
        int64_t re = f0 + rj;
        if constexpr (SCATTER) {
            re = rok ? NS.perm[f0 + rj] : 0;
            // positions f0 .. f0 + kNE - 1, then f0 - 1 and f0 + kNE (the neighbours)
            const int64_t pn = tid < kNE ? f0 + tid : tid == kNE ? f0 - 1 : f0 + kNE;
            nd = (tid < kNE + 2 && pn >= 0 && pn < E) ? NS.src_pos[pn] : -1;
            eid = (tid < kNE && f0 + tid < E) ? NS.perm[f0 + tid] : 0;
            rd = (tid < kNE && f0 + tid < E) ? NS.dist_pos[f0 + tid] : 1.0f;
        } else {
            rd = (tid < kNE && f0 + tid < E) ? dist[f0 + tid] : 1.0f;
        }
#pragma unroll
        for (int p = 0; p < NPR; ++p) {
            const int q = tid + kThreads * p;
            const int c4 = q % NC4;
            gw[p] = 1.0f;
            if constexpr (GP) gw[p] = grow[p] >= 0 ? DP.attn[gedge[p] * DP.heads + pool_head(DP, 4 * c4)] : 0.0f;
            if (grow[p] >= 0) {
                const float4* src = reinterpret_cast<const float4*>(gy + (grow[p] * COUT + 4 * c4) * DOUT);
#pragma unroll
                for (int v = 0; v < DOUT; ++v) {
                    const float4 f = src[v];
                    gr[p][4 * v] = f.x;
                    gr[p][4 * v + 1] = f.y;
                    gr[p][4 * v + 2] = f.z;
                    gr[p][4 * v + 3] = f.w;
                }
            } else {
#pragma unroll
                for (int v = 0; v < 4 * DOUT; ++v) gr[p][v] = 0.0f;
            }
        }
#pragma unroll
        for (int j = 0; j < RPW; ++j) {
            if (xrow[j] >= 0) {
                const float4* src = reinterpret_cast<const float4*>(
                    X.x + (xrow[j] * CIN + 16 * (wave + 4 * j) + 4 * lg) * DIN);
#pragma unroll
                for (int v = 0; v < DIN; ++v) {
                    const float4 f = src[v];
                    xl[j][4 * v] = f.x;
                    xl[j][4 * v + 1] = f.y;
                    xl[j][4 * v + 2] = f.z;
                    xl[j][4 * v + 3] = f.w;
                }
            } else {
#pragma unroll
                for (int v = 0; v < 4 * DIN; ++v) xl[j][v] = 0.0f;
            }
        }
        load_row_at<DIN * DIN>(P, re, rok, prs);
        load_row_at<DOUT * DOUT>(Q, re, rok, qrs);
    };

    // gd fragments (producer threads) and fs in the lane layout
    float fsr[RPW][4][DIN];
    auto produce = [&](auto sparse) {
        constexpr bool SP = decltype(sparse)::value;
#pragma unroll
        for (int p = 0; p < NPR; ++p) {
            const int q = tid + kThreads * p;
            const int e = q / NC4, c4 = q % NC4;
            const bool act = q < kNE * NC4;
            const int ee = act ? e : 0;
            float gd[4][DOUT];
            rotate_cols<LOUT, SP, 4>(gr[p], sQ + ee * QS, gd);
            if constexpr (GP) {
#pragma unroll
                for (int r = 0; r < 4; ++r)
#pragma unroll
                    for (int o = 0; o < DOUT; ++o) gd[r][o] *= gw[p];
            }
            float m = 0.0f;
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int o = 0; o < DOUT; ++o) m = fmaxf(m, fabsf(gd[r][o]));
#pragma unroll
            for (int off = NC4 / 2; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
            const int ex = scale_exp(m);
            const float sc = exp2i(ex);
            if (act && c4 == 0) sEinv[e] = exp2i(-ex);
            if (act) {
                const int ks = c4 / 8, g = (c4 / 2) % 4, half = c4 % 2;
                char* base = sB + ks * CHUNK + bslot(g, e) + 8 * half;
#pragma unroll
                for (int o = 0; o < DOUT; ++o) {
                    h4 hv, lv;
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        _Float16 h, l;
                        if constexpr (LP) {
                            h = static_cast<_Float16>(gd[r][o] * sc);
                        } else {
                            split_f16s(gd[r][o], sc, h, l);
                            lv[r] = l;
                        }
                        hv[r] = h;
                    }
                    *reinterpret_cast<h4*>(base + (o * NKS) * CHUNK) = hv;
                    if constexpr (!LP) *reinterpret_cast<h4*>(base + ((DOUT + o) * NKS) * CHUNK) = lv;
                }
            }
        }
#pragma unroll
        for (int j = 0; j < RPW; ++j) rotate_cols<LIN, SP, 4>(xl[j], sP + le * PS, fsr[j]);
    };

    load_tile(blockIdx.x);
    for (int64_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
        const int64_t e0 = tile * kNE;
        __syncthreads();   // the previous tile's readers of every LDS buffer are done
        store_rows<DIN * DIN, PS>(prs, sP);
        store_rows<DOUT * DOUT, QS>(qrs, sQ);
        if (tid < kNE) {
            EdgeState es;
            es.valid = e0 + tid < E;
            const EdgeBin eb = edge_bin(rd, B);
            es.lo = eb.lo;
            es.t = eb.t;
            es.s = rd / (rd + B.sh_scale);
            sE[tid] = es;
            edge_powers(es.s, NSP, sSp + tid * NSP);
        }
        if constexpr (SCATTER) {
            if (tid < kNE + 2) sNode[tid] = nd;
            if (tid < kNE) sEid[tid] = eid;
        }
        const bool dense =
            __syncthreads_or(off_block_nonzero_rows(prs, pbits) | off_block_nonzero_rows(qrs, qbits)) != 0;

        // radial functions (1/scale_k folded in), gd fragments, fs in lane layout
        if (fe0 < FG) {
            const float ik = sInvK[fkw / WD];
            for (int e = fe0; e < kNE; e += FG) {
                const EdgeState es = sE[e];
                const float* flo = F + static_cast<int64_t>(es.lo) * KW + fkw;
                sFe[e * KWS + fkw] = lerp_bins(flo[0], flo[KW], es.t) * ik * sSp[e * NSP + fl];
            }
        }
        if (dense)
            produce(std::false_type{});
        else
            produce(std::true_type{});
        if constexpr (GPQ) {
            // gQ[e][d][o] = sum over the edge's channels c of gy[c][d] m[c][o]:
            // each producer's four channels, then the sum over the 16 producers
            // of the edge (one 16-lane row), stored by the row's first lane
            static_assert(NC4 == 16 && NPR == 1, "one edge per 16-lane row of producers");
            if (gQo) {
                const int c4 = tid % NC4;
#pragma unroll
                for (int p = 0; p < NPR; ++p) {
                    // the producer's rows of m (y = m Q^T), loaded here rather
                    // than with the tile's prefetch, whose registers stay live
                    // through the previous tile's epilogue
                    float yk[4 * DOUT];
                    if (gqe[p] >= 0) {
                        const float4* src = reinterpret_cast<const float4*>(ym + (gqe[p] * COUT + 4 * c4) * DOUT);
#pragma unroll
                        for (int v = 0; v < DOUT; ++v) {
                            const float4 f = src[v];
                            yk[4 * v] = f.x;
                            yk[4 * v + 1] = f.y;
                            yk[4 * v + 2] = f.z;
                            yk[4 * v + 3] = f.w;
                        }
                    } else {
#pragma unroll
                        for (int v = 0; v < 4 * DOUT; ++v) yk[v] = 0.0f;
                    }
                    float* dst = gQo + (gqe[p] >= 0 ? gqe[p] : 0) * DOUT * DOUT;
#pragma unroll
                    for (int d = 0; d < DOUT; ++d)
#pragma unroll
                        for (int o = 0; o < DOUT; ++o) {
                            float a = 0.0f;
#pragma unroll
                            for (int r = 0; r < 4; ++r) a += gr[p][r * DOUT + d] * yk[r * DOUT + o];
                            if constexpr (GP) a *= gw[p];   // gy_e = attn[e, head] gout[dst[e]]
                            a = row16_sum(a);
                            if (c4 == 0 && gqe[p] >= 0) dst[d * DOUT + o] = a;
                        }
                }
            }
        }
        __syncthreads();

        // GEMM per output slot o, rank components in passes of KP; contractions
        // into dfs and the dF_e partials
        float dfs[RPW][4][DIN];
#pragma unroll
        for (int j = 0; j < RPW; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int i = 0; i < DIN; ++i) dfs[j][r][i] = 0.0f;
        const float* fe = sFe + le * KWS;
        const float einv = sEinv[le];
        const int myslot = bslot(lg, le);
        static_for<K / KP>([&](auto PP) {
            constexpr int k0 = decltype(PP)::value * KP;
            const h8* cfr = Cfrag;
            asm volatile("" : "+s"(cfr));
            h8 ahi[RPW][KP][NKS], alo[RPW][KP][NKS];
#pragma unroll
            for (int j = 0; j < RPW; ++j)
#pragma unroll
                for (int kk = 0; kk < KP; ++kk)
#pragma unroll
                    for (int ks = 0; ks < NKS; ++ks) {
                        const h8* src =
                            cfr + 2 * ((((k0 + kk) * (CIN / 16) + wave + 4 * j) * NKS + ks) * 64 + lane);
                        ahi[j][kk][ks] = src[0];
                        if constexpr (!LP) alo[j][kk][ks] = src[1];
                    }
            float pf[KP][WD];
#pragma unroll
            for (int kk = 0; kk < KP; ++kk)
#pragma unroll
                for (int w = 0; w < WD; ++w) pf[kk][w] = 0.0f;
            // software pipeline over the output slots: slot o + 1's MFMAs are
            // issued before slot o is contracted, slot o + 2's fragments loaded
            h8 bh[2][NKS], bl[2][NKS];
            v4f acc2[2][RPW][KP];
            auto load_b = [&](int slot, int buf) {
#pragma unroll
                for (int ks = 0; ks < NKS; ++ks) {
                    bh[buf][ks] = *reinterpret_cast<const h8*>(sB + (slot * NKS + ks) * CHUNK + myslot);
                    if constexpr (!LP)
                        bl[buf][ks] = *reinterpret_cast<const h8*>(sB + ((DOUT + slot) * NKS + ks) * CHUNK + myslot);
                }
            };
            auto mfma_slot = [&](int buf, int ab) {
#pragma unroll
                for (int j = 0; j < RPW; ++j)
#pragma unroll
                    for (int kk = 0; kk < KP; ++kk) acc2[ab][j][kk] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
                    for (int j = 0; j < RPW; ++j)
#pragma unroll
                        for (int kk = 0; kk < KP; ++kk) {
                            if constexpr (!LP) {
                                acc2[ab][j][kk] = mfma_h(alo[j][kk][ks], bh[buf][ks], acc2[ab][j][kk]);
                                acc2[ab][j][kk] = mfma_h(ahi[j][kk][ks], bl[buf][ks], acc2[ab][j][kk]);
                            }
                            acc2[ab][j][kk] = mfma_h(ahi[j][kk][ks], bh[buf][ks], acc2[ab][j][kk]);
                        }
            };
            load_b(0, 0);
            if constexpr (DOUT > 1) load_b(1, 1);
            mfma_slot(0, 0);
            static_for<DOUT>([&](auto OO) {
                constexpr int o = decltype(OO)::value;
                constexpr int cur = o & 1;
                if constexpr (o + 1 < DOUT) mfma_slot(cur ^ 1, cur ^ 1);
                if constexpr (o + 2 < DOUT) load_b(o + 2, cur);
                auto& acc = acc2[cur];
                static_for<TG::count(o)>([&](auto TT) {
                    constexpr Term tm = TG::sorted[TG::start[o] + decltype(TT)::value];
#pragma unroll
                    for (int kk = 0; kk < KP; ++kk) {
                        const float f = fe[(k0 + kk) * WD + tm.w];
                        const float c = tm.neg ? -f : f;
                        float part = 0.0f;
#pragma unroll
                        for (int j = 0; j < RPW; ++j)
#pragma unroll
                            for (int r = 0; r < 4; ++r) {
                                dfs[j][r][tm.i] += c * acc[j][kk][r];
                                part += fsr[j][r][tm.i] * acc[j][kk][r];
                            }
                        pf[kk][tm.w] += tm.neg ? -part : part;
                    }
                });
                // Pin the contraction to this slot: without these (empty)
                // read-modify-write uses the compiler defers it past later
                // slots' MFMAs and keeps their results live.
#pragma unroll
                for (int j = 0; j < RPW; ++j)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
#pragma unroll
                        for (int i = 0; i < DIN; ++i) asm volatile("" : "+v"(dfs[j][r][i]));
                __builtin_amdgcn_sched_barrier(0);
            });
            // the pass's dF_e partials, value n = KP w + kk: sums over the four
            // lane groups, four values per register (lane group g keeps value
            // 4 q + g of quad q), unscaled and stored by every lane
            constexpr int NV = KP * WD, NQ = (NV + 3) / 4;
            const float sck = sInvK[k0 + lg % KP] * einv;   // 4 q + lg = lg (mod KP)
            float* dst = sDF + (wave * kNE + le) * KW + k0 * WD;
            static_for<NQ>([&](auto QQ) {
                constexpr int q = decltype(QQ)::value;
                float v[4];
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int n = 4 * q + g;
                    v[g] = n < NV ? pf[n % KP][n / KP] : 0.0f;
                }
                const float u = quad_lane_sums(v);
                const int n = 4 * q + lg;
                if (4 * q + 3 < NV || n < NV) dst[(n % KP) * WD + n / KP] = u * sck;
            });
        });

        // next tile's global loads, then dx = dfs P^T / scale_e (s^l_in is in
        // the radial functions) staged in LDS, and the dF_e sums over the waves
        constexpr int kGPQuads = (DIN * DIN + 3) / 4;
        float gpl[GPQ ? kGPQuads : 1];   // GPQ: gP partials, lane group g holds value 4 q + g
        if constexpr (GPQ) {
            // gP[e][d][i] = sum over the channels c of x[c][d] (dL/df)[c][i]
            // with dL/df = dfs / scale_e: this lane's rows (x reloaded; before
            // the next tile's prefetch, so that its registers are free), then
            // the sum over the wave's four lane groups; the four waves are
            // summed after the tile's stores
            if (gPo) {
                const float sc = sEinv[le];
                int64_t xr0;
                if constexpr (SCATTER)
                    xr0 = e0 + le < E ? NS.src_pos[e0 + le] : -1;
                else
                    xr0 = e0 + le < E ? x_row<GATHER>(X, e0 + le) : -1;
                float xg[RPW][4 * DIN];
#pragma unroll
                for (int j = 0; j < RPW; ++j) {
                    if (xr0 >= 0) {
                        const float4* src = reinterpret_cast<const float4*>(
                            X.x + (xr0 * CIN + 16 * (wave + 4 * j) + 4 * lg) * DIN);
#pragma unroll
                        for (int v = 0; v < DIN; ++v) {
                            const float4 f = src[v];
                            xg[j][4 * v] = f.x;
                            xg[j][4 * v + 1] = f.y;
                            xg[j][4 * v + 2] = f.z;
                            xg[j][4 * v + 3] = f.w;
                        }
                    } else {
#pragma unroll
                        for (int v = 0; v < 4 * DIN; ++v) xg[j][v] = 0.0f;
                    }
                }
                static_for<kGPQuads>([&](auto QQ) {
                    constexpr int q = decltype(QQ)::value;
                    float v[4];
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        const int n = 4 * q + g, d = n / DIN, i = n % DIN;
                        float a = 0.0f;
                        if (n < DIN * DIN)
#pragma unroll
                            for (int j = 0; j < RPW; ++j)
#pragma unroll
                                for (int r = 0; r < 4; ++r) a += xg[j][r * DIN + d] * dfs[j][r][i];
                        v[g] = a;
                    }
                    gpl[q] = quad_lane_sums(v) * sc;
                });
            }
        }
        load_tile(tile + gridDim.x);
        __syncthreads();   // fragments consumed, dF_e partials complete
        {
            const float* pe = sP + le * PS;
            asm volatile("" : "+v"(pe));   // no reuse of the P values loaded for fs
            const float sc = sEinv[le];
#pragma unroll
            for (int i = 0; i < DIN; ++i)
#pragma unroll
                for (int j = 0; j < RPW; ++j)
#pragma unroll
                    for (int r = 0; r < 4; ++r) dfs[j][r][i] *= sc;
#pragma unroll
            for (int j = 0; j < RPW; ++j) {
                float vin[DIN][4], out[4 * DIN];
#pragma unroll
                for (int i = 0; i < DIN; ++i)
#pragma unroll
                    for (int r = 0; r < 4; ++r) vin[i][r] = dfs[j][r][i];
                if (dense)
                    rotate_rows<LIN, false>(vin, pe, out);
                else
                    rotate_rows<LIN, true>(vin, pe, out);
                stage_rows<CIN, DIN>(reinterpret_cast<float*>(sB), le, 16 * (wave + 4 * j) + 4 * lg, out);
            }
        }
        const int nval = static_cast<int>(E - e0 < kNE ? E - e0 : kNE);
        // dF_e of the unscaled rows times s^(l_in(w) + l_out(w))
        if (fe0 < FG) {
            for (int e = fe0; e < nval; e += FG) {
                const int q = e * KW + fkw;
                float a = sDF[q];
#pragma unroll
                for (int v = 1; v < 4; ++v) a += sDF[v * kNE * KW + q];
                const int64_t ed = SCATTER ? static_cast<int64_t>(sEid[e]) : e0 + e;
                dFe[ed * KW + fkw] = a * sSp[e * NSP + fl];
            }
        }
        __syncthreads();
        if constexpr (SCATTER)
            scatter_stage<CIN, DIN>(reinterpret_cast<const float*>(sB), sNode, NS, tile, nval);
        else
            flush_stage<CIN, DIN>(reinterpret_cast<const float*>(sB), gx + e0 * CIN * DIN, nval);
        if constexpr (GPQ) {
            if (gPo) {
                // the four waves' partials through the (now read) stage buffer
                constexpr int GS = 4 * kGPQuads;
                float* sG = reinterpret_cast<float*>(sB);   // [wave][edge][GS]
                static_assert(4 * kNE * GS * sizeof(float) <= BREG, "gP partials fit the stage");
                __syncthreads();
#pragma unroll
                for (int q = 0; q < kGPQuads; ++q) sG[(wave * kNE + le) * GS + 4 * q + lg] = gpl[q];
                __syncthreads();
                for (int idx = tid; idx < nval * DIN * DIN; idx += kThreads) {
                    const int e = idx / (DIN * DIN), n = idx % (DIN * DIN);
                    const float a = sG[e * GS + n] + sG[(kNE + e) * GS + n] + sG[(2 * kNE + e) * GS + n] +
                                    sG[(3 * kNE + e) * GS + n];
                    const int64_t ed = SCATTER ? static_cast<int64_t>(sEid[e]) : e0 + e;
                    gPo[ed * DIN * DIN + n] = a;
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Channel-pattern gradient: per 16-edge tile, for every rank component k,
//   dC_k[co][ci] += sum over (slot i, edge e) of U_k[co][(i, e)] fs[ci][(i, e)],
//   U_k[co][e][i] = sum_{terms (o, i, w)} sign F_e[k, w] gd[co][e][o]   (M_ek^T gd)
// with gd = s^l_out (gy Q), fs = s^l_in (x P): a GEMM with M = Cout, N = Cin
// and a reduction over the 16 Din (slot, edge) pairs of the tile (slot-major,
// padded to whole 32-steps with zero fragments).  Producers own one channel
// of four edges (threads 4 c .. 4 c + 3 share channel c), so each U_k row and
// fs column gets its own power-of-two scale from a lane-quad maximum (no
// extra barrier); each rank's tile product is unscaled row by column into a
// float32 accumulator that lives for the whole launch.  fs fragments stay in
// LDS for the tile; the U_k fragments of one rank at a time share their
// buffer with the tile's P and Q.  Wave w owns output rows 16 w .. 16 w + 15,
// whose U_k rows its own lanes produce, so only the fs fragments are shared
// between waves.  One partial dC per workgroup.
//
// GP (pooled form): edge e reads attn[e, head(c)] gy[dst[e], c, :] (DstPool).
template <int CIN, int COUT, int LIN, int LOUT, int K, bool GATHER, bool LP, bool GP>
__global__ void __launch_bounds__(kThreads, 2)
k_ews_bwd_c(feq_binning B, int64_t E, int64_t ntiles, const float* __restrict__ gy,
            XRows X, const float* __restrict__ P,
            const float* __restrict__ Q, const float* __restrict__ dist,
            const float* __restrict__ F, float* __restrict__ dC_part, DstPool DP) {
    static_assert(GATHER || !GP, "the pooled form is a message-passing form");
    using T = Canon<LIN, LOUT>;
    constexpr int DIN = T::DIN, DOUT = T::DOUT, WD = T::WD, KW = K * WD;
    constexpr int PS = DIN * DIN | 1, QS = DOUT * DOUT | 1;
    constexpr int WDP = (WD + 3) / 4 * 4;                        // radial row of one (k, edge), float4s
    constexpr int RB = COUT / 16, CB = CIN / 16;                 // 16-row / 16-column blocks
    constexpr int NKG = 2 * DIN;                                 // 8-edge groups of the reduction
    constexpr int NKS = (NKG + 3) / 4;                           // 32-steps
    constexpr int ARR = NKG * 256;                               // bytes per (split, block) array
    static_assert(RB == kThreads / 64 && 4 * CIN <= kThreads && 4 * COUT == kThreads,
                  "unsupported channel counts");
    static_assert(4 * (kNE * PS + kNE * QS) <= 2 * RB * ARR, "P and Q must fit the U buffer");

    extern __shared__ float4 smem4[];
    char* sF = reinterpret_cast<char*>(smem4);                   // fs fragments [2][CB][NKG][16][16 B]
    char* sU = sF + 2 * CB * ARR;                                // U_k fragments [2][RB][NKG][16][16 B]
    float* sP = reinterpret_cast<float*>(sU);                    // P, Q of the tile (producer phase only)
    float* sQ = sP + kNE * PS;
    float* sFe = reinterpret_cast<float*>(sU + 2 * RB * ARR);   // [K][kNE][WDP], 0 past the last edge
    float* sInvF = sFe + K * kNE * WDP;                          // 1 / scale of fs column ci
    float* sInvU = sInvF + CIN;                                  // 1 / scale of U_k row co
    EdgeState* sE = reinterpret_cast<EdgeState*>(sInvU + COUT);

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int le = lane & 15, lg = lane >> 4;
    const unsigned pbits = off_block_bits_rows<LIN>(), qbits = off_block_bits_rows<LOUT>();
    const int pc = tid >> 2, pq = tid & 3;                        // producer: channel, edge quad

    v4f acc_tot[K][CB];
#pragma unroll
    for (int k = 0; k < K; ++k)
#pragma unroll
        for (int b = 0; b < CB; ++b) acc_tot[k][b] = v4f{0.0f, 0.0f, 0.0f, 0.0f};

    for (int64_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
        const int64_t e0 = tile * kNE;
        // global loads: four edges' rows of one input channel / one output channel.
        // Unconditional: edges past the last (and channels past Cin / Cout) read
        // the last one's rows; their radial functions are zero, so their U_k rows
        // are zero and they add nothing to dC.  The row indices (sources; with
        // GP, destinations) are all requested before the rows they point to.
        float xr[4][DIN], gr[4][DOUT], gw[4];
        const int pci = pc < CIN ? pc : CIN - 1, pco = pc < COUT ? pc : COUT - 1;
        int64_t xi[4], gi[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int64_t e = e0 + 4 * pq + q < E ? e0 + 4 * pq + q : E - 1;
            xi[q] = x_row<GATHER>(X, e);
            if constexpr (GP) gi[q] = pool_node(DP, e); else gi[q] = e;
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int64_t e = e0 + 4 * pq + q < E ? e0 + 4 * pq + q : E - 1;
            // an index outside the node table (message-passing form) reads row 0;
            // the edge is then marked invalid, so it adds nothing either
            const float* xs = X.x + ((xi[q] >= 0 ? xi[q] : 0) * CIN + pci) * DIN;
            gw[q] = 1.0f;
            // pooled form: a destination outside [0, ndst) reads row 0 with weight 0
            if constexpr (GP) gw[q] = gi[q] >= 0 ? DP.attn[e * DP.heads + pool_head(DP, pco)] : 0.0f;
            const float* gs = gy + ((gi[q] >= 0 ? gi[q] : 0) * COUT + pco) * DOUT;
#pragma unroll
            for (int d = 0; d < DIN; ++d) xr[q][d] = xs[d];
#pragma unroll
            for (int d = 0; d < DOUT; ++d) gr[q][d] = gs[d];
        }
        float pr[rows_per_thread<DIN * DIN>()], qr[rows_per_thread<DOUT * DOUT>()];
        load_rows<DIN * DIN, false>(P, e0, E, nullptr, pr);
        load_rows<DOUT * DOUT, false>(Q, e0, E, nullptr, qr);
        const float rd = (tid < kNE && e0 + tid < E) ? dist[e0 + tid] : 1.0f;

        __syncthreads();   // the previous tile's readers of every LDS buffer are done
        store_rows<DIN * DIN, PS>(pr, sP);
        store_rows<DOUT * DOUT, QS>(qr, sQ);
        if (tid < kNE) {
            EdgeState es;
            es.valid = e0 + tid < E && x_row<GATHER>(X, e0 + tid) >= 0;
            const EdgeBin eb = edge_bin(rd, B);
            es.lo = eb.lo;
            es.t = eb.t;
            es.s = rd / (rd + B.sh_scale);
            sE[tid] = es;
        }
        const bool dense =
            __syncthreads_or(off_block_nonzero_rows(pr, pbits) | off_block_nonzero_rows(qr, qbits)) != 0;

        for (int q = tid; q < kNE * KW; q += kThreads) {
            const int e = q / KW, rest = q % KW;
            const EdgeState es = sE[e];
            const float* flo = F + static_cast<int64_t>(es.lo) * KW + rest;
            sFe[((rest / WD) * kNE + e) * WDP + rest % WD] = es.valid ? lerp_bins(flo[0], flo[KW], es.t) : 0.0f;
        }
        // fs (input channel pc of edges 4 pq .. 4 pq + 3) and gd (output channel pc)
        float gd[4][DOUT];
        {
            float fs[4][DIN];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int e = 4 * pq + q;
                float pi[DIN], po[DOUT], t1[1][DIN], t2[1][DOUT];
                slot_pow<LIN>(sE[e].s, pi);
                slot_pow<LOUT>(sE[e].s, po);
                if (dense) {
                    rotate_cols<LIN, false, 1>(xr[q], sP + e * PS, t1);
                    rotate_cols<LOUT, false, 1>(gr[q], sQ + e * QS, t2);
                } else {
                    rotate_cols<LIN, true, 1>(xr[q], sP + e * PS, t1);
                    rotate_cols<LOUT, true, 1>(gr[q], sQ + e * QS, t2);
                }
#pragma unroll
                for (int i = 0; i < DIN; ++i) fs[q][i] = t1[0][i] * pi[i];
#pragma unroll
                for (int o = 0; o < DOUT; ++o) gd[q][o] = t2[0][o] * po[o] * gw[q];
            }
            float m = 0.0f;
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int i = 0; i < DIN; ++i) m = fmaxf(m, fabsf(fs[q][i]));
            m = fmaxf(m, __shfl_xor(m, 1, 64));
            m = fmaxf(m, __shfl_xor(m, 2, 64));
            const int ex = scale_exp(m);
            const float sc = exp2i(ex);
            if (pc < CIN) {
                if (pq == 0) sInvF[pc] = exp2i(-ex);
                char* arr = sF + (pc / 16) * ARR;
#pragma unroll
                for (int i = 0; i < DIN; ++i) {
                    h4 hv, lv;
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        _Float16 h, l;
                        if constexpr (LP) {
                            h = static_cast<_Float16>(fs[q][i] * sc);
                        } else {
                            split_f16s(fs[q][i], sc, h, l);
                            lv[q] = l;
                        }
                        hv[q] = h;
                    }
                    const int off = ((2 * i + (pq >> 1)) * 16 + pc % 16) * 16 + 8 * (pq & 1);
                    *reinterpret_cast<h4*>(arr + off) = hv;
                    if constexpr (!LP) *reinterpret_cast<h4*>(arr + CB * ARR + off) = lv;
                }
            }
        }
        __syncthreads();   // fs fragments complete; P and Q no longer read

        // Wave w owns output rows co = 16 w + ..., the channels its own producer
        // lanes hold gd for: its U_k fragments are written and read by the wave
        // alone (a wave's LDS operations execute in issue order), so the rank
        // components need no workgroup barrier.
        const int nbase = lane;   // fragment reads: lane (g, n) at 16-byte slot 16 g + n of an 8-edge group row
        char* uarr = sU + wave * ARR;
        static_for<K>([&](auto KK) {
            constexpr int k = decltype(KK)::value;
            // U_k row pc of edges 4 pq .. 4 pq + 3, scaled per row, to fragments
            {
                float u[4][DIN];
#pragma unroll
                for (int q = 0; q < 4; ++q)
#pragma unroll
                    for (int i = 0; i < DIN; ++i) u[q][i] = 0.0f;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float4* fe4 = reinterpret_cast<const float4*>(sFe + (k * kNE + 4 * pq + q) * WDP);
                    float fe[WDP];
#pragma unroll
                    for (int v = 0; v < WDP / 4; ++v) {
                        const float4 f = fe4[v];
                        fe[4 * v] = f.x;
                        fe[4 * v + 1] = f.y;
                        fe[4 * v + 2] = f.z;
                        fe[4 * v + 3] = f.w;
                    }
#pragma unroll
                    for (int t = 0; t < T::NT; ++t) {
                        const Term tm = T::terms[t];
                        const float c = tm.neg ? -fe[tm.w] : fe[tm.w];
                        u[q][tm.i] += c * gd[q][tm.o];
                    }
                }
                float m = 0.0f;
#pragma unroll
                for (int q = 0; q < 4; ++q)
#pragma unroll
                    for (int i = 0; i < DIN; ++i) m = fmaxf(m, fabsf(u[q][i]));
                m = fmaxf(m, __shfl_xor(m, 1, 64));
                m = fmaxf(m, __shfl_xor(m, 2, 64));
                const int ex = scale_exp(m);
                const float sc = exp2i(ex);
                if (pq == 0) sInvU[pc] = exp2i(-ex);
#pragma unroll
                for (int i = 0; i < DIN; ++i) {
                    h4 hv, lv;
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        _Float16 h, l;
                        if constexpr (LP) {
                            h = static_cast<_Float16>(u[q][i] * sc);
                        } else {
                            split_f16s(u[q][i], sc, h, l);
                            lv[q] = l;
                        }
                        hv[q] = h;
                    }
                    const int off = ((2 * i + (pq >> 1)) * 16 + pc % 16) * 16 + 8 * (pq & 1);
                    *reinterpret_cast<h4*>(uarr + off) = hv;
                    if constexpr (!LP) *reinterpret_cast<h4*>(uarr + RB * ARR + off) = lv;
                }
            }

            v4f acc[CB];
#pragma unroll
            for (int b = 0; b < CB; ++b) acc[b] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int ks = 0; ks < NKS; ++ks) {
                const int kg = 4 * ks + lg;
                const bool live = kg < NKG;   // the last step's upper lane groups pad with zeros
                const h8 z = h8{0, 0, 0, 0, 0, 0, 0, 0};
                // all fragments of the step first, then the three products of
                // the CB blocks interleaved (CB independent accumulation chains)
                const char* ua = uarr + (16 * ks * 4 + nbase) * 16;
                const h8 ah = live ? *reinterpret_cast<const h8*>(ua) : z;
                h8 al = z, bh[CB], bl[CB];
                if constexpr (!LP) al = live ? *reinterpret_cast<const h8*>(ua + RB * ARR) : z;
#pragma unroll
                for (int b = 0; b < CB; ++b) {
                    const char* arr = sF + b * ARR + (16 * ks * 4 + nbase) * 16;
                    bh[b] = live ? *reinterpret_cast<const h8*>(arr) : z;
                    if constexpr (!LP) bl[b] = live ? *reinterpret_cast<const h8*>(arr + CB * ARR) : z;
                }
                if constexpr (!LP) {
#pragma unroll
                    for (int b = 0; b < CB; ++b) acc[b] = mfma_h(al, bh[b], acc[b]);
#pragma unroll
                    for (int b = 0; b < CB; ++b) acc[b] = mfma_h(ah, bl[b], acc[b]);
                }
#pragma unroll
                for (int b = 0; b < CB; ++b) acc[b] = mfma_h(ah, bh[b], acc[b]);
            }
            // unscale row (co) by column (ci) into the launch accumulator
            float ru[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) ru[r] = sInvU[16 * wave + 4 * lg + r];
#pragma unroll
            for (int b = 0; b < CB; ++b) {
                const float cf = sInvF[16 * b + le];
#pragma unroll
                for (int r = 0; r < 4; ++r) acc_tot[k][b][r] += acc[b][r] * (ru[r] * cf);
            }
        });
    }
    float* part = dC_part + static_cast<int64_t>(blockIdx.x) * K * COUT * CIN;
#pragma unroll
    for (int k = 0; k < K; ++k)
#pragma unroll
        for (int b = 0; b < CB; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                part[(k * COUT + 16 * wave + 4 * lg + r) * CIN + 16 * b + le] = acc_tot[k][b][r];
}

template <int CIN, int COUT, int LIN, int LOUT, int K>
constexpr size_t ews_bwd_c_lds() {
    using T = Canon<LIN, LOUT>;
    constexpr size_t ARR = 2 * T::DIN * 256, WDP = (T::WD + 3) / 4 * 4;
    return 2 * (CIN / 16) * ARR + 2 * (COUT / 16) * ARR + 4 * (K * kNE * WDP + CIN + COUT) +
           kNE * sizeof(EdgeState);
}

template <int CIN, int COUT, int LIN, int LOUT, int K>
constexpr size_t ews_bwd_x_lds() {
    using T = Canon<LIN, LOUT>;
    constexpr size_t PS = T::DIN * T::DIN | 1, QS = T::DOUT * T::DOUT | 1;
    constexpr size_t KW = K * T::WD, KWS = KW | 1;
    constexpr size_t FR = 2 * T::DOUT * (COUT / 32) * 1024, ST = 4 * kNE * stage_stride(CIN * T::DIN);
    return (FR > ST ? FR : ST) +
           4 * (kNE * PS + kNE * QS + kNE * KWS + 4 * kNE * KW + kNE * (LIN + LOUT + 1) + kNE + K) +
           kNE * sizeof(EdgeState) + (2 * kNE + 4) * sizeof(int);
}

template <int CIN, int COUT, int LIN, int LOUT, int K>
constexpr size_t ews_fwd_lds() {
    using T = Canon<LIN, LOUT>;
    constexpr size_t PS = T::DIN * T::DIN | 1, QS = T::DOUT * T::DOUT | 1, KWS = K * T::WD | 1;
    constexpr size_t FR = 2 * T::DIN * (CIN / 32) * 1024, ST = 4 * kNE * stage_stride(COUT * T::DOUT);
    return (FR > ST ? FR : ST) +
           4 * (kNE * PS + kNE * QS + kNE * KWS + kNE + kNE * (LIN + LOUT + 1) + K) +
           kNE * sizeof(EdgeState) + (kNE + 4) * sizeof(int) + 4 * kNE * kPoolMaxHeads;
}

// Workgroups per CU of the forward.  Two, measured on MI355X at 160k edges
// with all rank components in one GEMM pass: 253 us, against 261 us with two
// passes and 306 us at three workgroups per CU, where the 168-register budget
// forces spills.
template <int CIN, int COUT, int LIN, int LOUT, int K>
constexpr int ews_fwd_occ() {
    static_assert(2 * ews_fwd_lds<CIN, COUT, LIN, LOUT, K>() <= 160 * 1024, "forward LDS");
    return 2;
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

// Workspace of the pooled forward: the C fragments, two partial rows per tile,
// the sources and destinations in CSR position order.
template <int CIN, int COUT, int LIN, int LOUT, int K>
size_t ews_pool_fwd_ws(int64_t E) {
    using T = Canon<LIN, LOUT>;
    return ews_cfrag_bytes<CIN, COUT, K>() +
           align_up(4 * static_cast<size_t>(ceil_div(E, kNE)) * 2 * COUT * T::DOUT, 256) +
           align_up(8 * static_cast<size_t>(E), 256) + 2 * align_up(4 * static_cast<size_t>(E), 256) + 512;
}

// Source, destination and distance of every CSR position p (edge perm[p]) of
// the pooled forward, so that its tile loads index them directly.
__global__ void k_pool_order(int64_t E, const int32_t* __restrict__ perm, const int64_t* __restrict__ src,
                             const int64_t* __restrict__ dst, const float* __restrict__ dist, int64_t ndst,
                             int64_t* __restrict__ src_pos, int32_t* __restrict__ node_pos,
                             float* __restrict__ dist_pos) {
    const int64_t p = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
    if (p >= E) return;
    const int64_t e = perm[p];
    src_pos[p] = src[e];
    dist_pos[p] = dist[e];
    const int64_t n = dst[e];
    node_pos[p] = n >= 0 && n < ndst ? static_cast<int32_t>(n) : -1;
}

// lp: one fp16 product per operand pair (message-passing form only).
// dp: the pooled form (message-passing form only).
template <int CIN, int COUT, int LIN, int LOUT, int K, bool GATHER>
int launch_ews_fwd(const feq_binning& B, int64_t E, XRows x, const float* P, const float* Q,
                   const float* dist, const float* C, const float* F, float* y, void* ws,
                   size_t ws_bytes, bool lp, const DstPool* dp, hipStream_t s, float* ym) {
    using T = Canon<LIN, LOUT>;
    constexpr size_t lds = ews_fwd_lds<CIN, COUT, LIN, LOUT, K>();
    constexpr int occ = ews_fwd_occ<CIN, COUT, LIN, LOUT, K>();
    static_assert(lds <= 80 * 1024, "two forward workgroups must fit one CU's LDS");
    const size_t need = dp ? ews_pool_fwd_ws<CIN, COUT, LIN, LOUT, K>(E) : ews_cfrag_bytes<CIN, COUT, K>();
    if (!ws || ws_bytes < need) return fail(FEQ_ERR_WORKSPACE, "edgewise forward workspace too small");
    const int64_t ntiles = ceil_div(E, kNE);
    Carver cv(ws);
    h8* frag = cv.take<h8>(static_cast<size_t>(K) * COUT * CIN / 4);
    float* inv = cv.take<float>(K);
    DstPool DP{};
    XRows X = x;
    if (dp) {
        DP = *dp;
        DP.part = cv.take<float>(static_cast<size_t>(ntiles) * 2 * COUT * T::DOUT);
        int64_t* src_pos = cv.take<int64_t>(E);
        int32_t* node_pos = cv.take<int32_t>(E);
        float* dist_pos = cv.take<float>(E);
        FEQ_LAUNCH("k_pool_order", k_pool_order, dim3(static_cast<unsigned>(ceil_div(E, kThreads))),
                   dim3(kThreads), 0, s, E, DP.perm, x.src, DP.dst, dist, DP.ndst, src_pos, node_pos,
                   dist_pos);
        DP.src_pos = src_pos;
        DP.node_pos = node_pos;
        DP.dist_pos = dist_pos;
        X.src = src_pos;
    }
    auto prep = k_ews_prep<K, COUT, CIN, false>;
    FEQ_LAUNCH("k_ews_prep", prep, dim3(K * COUT / 16), dim3(kThreads), 0, s, C, frag, inv);
    auto kern = k_ews_fwd<CIN, COUT, LIN, LOUT, K, occ, GATHER, false, false>;
    if constexpr (GATHER) {
        if (dp)
            kern = lp ? k_ews_fwd<CIN, COUT, LIN, LOUT, K, occ, true, true, true>
                      : k_ews_fwd<CIN, COUT, LIN, LOUT, K, occ, true, false, true>;
        else if (lp)
            kern = k_ews_fwd<CIN, COUT, LIN, LOUT, K, occ, true, true, false>;
    } else {
        if (dp) return fail(FEQ_ERR_INVALID, "the pooled form needs the message-passing form");
    }
    if (ym) {
        // (one fp16 product per pair only in the message-passing form)
        if (dp)
            kern = lp ? k_ews_fwd<CIN, COUT, LIN, LOUT, K, occ, GATHER, GATHER, GATHER, true>
                      : k_ews_fwd<CIN, COUT, LIN, LOUT, K, occ, GATHER, false, GATHER, true>;
        else
            kern = lp ? k_ews_fwd<CIN, COUT, LIN, LOUT, K, occ, GATHER, GATHER, false, true>
                      : k_ews_fwd<CIN, COUT, LIN, LOUT, K, occ, GATHER, false, false, true>;
    }
    if (int rc = ews_set_lds(reinterpret_cast<const void*>(kern), lds)) return rc;
    const int64_t g = static_cast<int64_t>(ews_cus()) * occ;
    const int grid = static_cast<int>(ntiles < g ? ntiles : g);
    FEQ_LAUNCH("k_ews_fwd", kern, dim3(grid), dim3(kThreads), lds, s, B, E, ntiles, X, P, Q, dist,
               frag, inv, F, y, DP, ym);
    if (dp) {
        const NodeScatter NS{DP.perm, DP.offsets, DP.out, DP.part};
        if (int rc = node_fix(NS, DP.ndst, static_cast<int64_t>(COUT * T::DOUT / 4), s)) return rc;
    }
    return FEQ_OK;
}

// Workspace of the split backward: dF_e (E, K Wdim), the per-workgroup dC
// partials, the tail's histogram partials and sums, the C^T fragments; with
// the per-node sums, two partial rows per tile.
template <int CIN, int COUT, int LIN, int LOUT, int K>
size_t ews_bwd_ws(const feq_binning& B, int64_t E, bool nodes) {
    using T = Canon<LIN, LOUT>;
    const int64_t ntiles = ceil_div(E, kNE), g = static_cast<int64_t>(ews_cus()) * 2;
    const int G = static_cast<int>(ntiles < g ? ntiles : g);
    const int64_t kw = static_cast<int64_t>(K) * T::WD, ncc = static_cast<int64_t>(K) * COUT * CIN;
    const size_t part = nodes ? align_up(4 * static_cast<size_t>(ntiles) * 2 * CIN * T::DIN, 256) +
                                    3 * align_up(4 * static_cast<size_t>(E), 256)
                              : 0;
    return align_up(4 * E * kw, 256) + align_up(4 * static_cast<size_t>(G) * ncc, 256) +
           align_up(4 * ew_tail_floats(B, static_cast<int>(kw), E, G, ncc), 256) +
           ews_cfrag_bytes<CIN, COUT, K>() + part + 1024;
}

// Source row, distance and (pooled form) destination of every CSR-by-source
// position p (edge perm[p]) of the input-gradient kernel's tile walk.
__global__ void k_scatter_order(int64_t E, const int32_t* __restrict__ perm, const int64_t* __restrict__ src,
                                int64_t nsrc, const float* __restrict__ dist, const int64_t* __restrict__ dst,
                                int64_t ndst, int32_t* __restrict__ src_pos, float* __restrict__ dist_pos,
                                int32_t* __restrict__ dnode_pos) {
    const int64_t p = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
    if (p >= E) return;
    const int64_t e = perm[p];
    const int64_t r = src[e];
    src_pos[p] = r >= 0 && r < nsrc ? static_cast<int32_t>(r) : -1;
    dist_pos[p] = dist[e];
    if (dst) {
        const int64_t n = dst[e];
        dnode_pos[p] = n >= 0 && n < ndst ? static_cast<int32_t>(n) : -1;
    }
}

// ns: NULL for the per-edge input gradient gx; else the per-node sums into
// ns->out (gx unused; ns->part is carved from the workspace here).
template <int CIN, int COUT, int LIN, int LOUT, int K, bool GATHER>
int launch_ews_bwd(const feq_layout& L, const feq_binning& B, int64_t E, const float* gy,
                   XRows x, const float* P, const float* Q, const float* dist,
                   const float* C, const float* F, float* gx, float* gC, float* gF, float* gdist,
                   const NodeScatter* ns, void* ws, size_t ws_bytes, bool lp, const DstPool* dp,
                   hipStream_t s, const BasisGrads* bg) {
    using T = Canon<LIN, LOUT>;
    constexpr size_t xlds = ews_bwd_x_lds<CIN, COUT, LIN, LOUT, K>();
    constexpr size_t clds = ews_bwd_c_lds<CIN, COUT, LIN, LOUT, K>();
    static_assert(xlds <= 80 * 1024, "two input-gradient workgroups must fit one CU's LDS");
    static_assert(clds <= 80 * 1024, "two channel-gradient workgroups must fit one CU's LDS");
    const int kw = K * T::WD;
    if (!ew_tail_supported(B, kw)) return -1;
    const int64_t ntiles = ceil_div(E, kNE), g = static_cast<int64_t>(ews_cus()) * 2;
    const int G = static_cast<int>(ntiles < g ? ntiles : g);
    const int64_t ncc = static_cast<int64_t>(K) * COUT * CIN;
    Carver cv(ws);
    float* dFe = cv.take<float>(E * kw);
    float* dCp = cv.take<float>(static_cast<size_t>(G) * ncc);
    float* tail = cv.take<float>(ew_tail_floats(B, kw, E, G, ncc));
    h8* frag = cv.take<h8>(static_cast<size_t>(K) * COUT * CIN / 4);
    float* inv = cv.take<float>(K);
    NodeScatter NS{};
    if (ns) {
        NS = *ns;
        NS.part = cv.take<float>(static_cast<size_t>(ntiles) * 2 * CIN * T::DIN);
        NS.src_pos = cv.take<int32_t>(E);
        NS.dist_pos = cv.take<float>(E);
        NS.dnode_pos = cv.take<int32_t>(E);
    }
    if (!ws || cv.used > ws_bytes) return fail(FEQ_ERR_WORKSPACE, "edgewise workspace too small");
    if (dp && !ns) return fail(FEQ_ERR_INVALID, "the pooled form needs the per-node input gradient");
    const bool gpq = bg && (bg->gP || bg->gQ);
    if (bg && bg->gQ && !bg->ym) return fail(FEQ_ERR_INVALID, "grad_Q needs the rows before the rotation");
    const float* bym = bg ? bg->ym : nullptr;
    float* bgP = bg ? bg->gP : nullptr;
    float* bgQ = bg ? bg->gQ : nullptr;
    const DstPool DP = dp ? *dp : DstPool{};
    if (ns) {
        if (!x.src) return fail(FEQ_ERR_INVALID, "per-node sums need the message-passing form");
        FEQ_LAUNCH("k_scatter_order", k_scatter_order, dim3(static_cast<unsigned>(ceil_div(E, kThreads))),
                   dim3(kThreads), 0, s, E, NS.perm, x.src, x.nsrc, dist, dp ? DP.dst : nullptr, DP.ndst,
                   const_cast<int32_t*>(NS.src_pos), const_cast<float*>(NS.dist_pos),
                   const_cast<int32_t*>(NS.dnode_pos));
    }
    auto prep = k_ews_prep<K, CIN, COUT, true>;
    FEQ_LAUNCH("k_ews_prep", prep, dim3(K * CIN / 16), dim3(kThreads), 0, s, C, frag, inv);
    auto kc = k_ews_bwd_c<CIN, COUT, LIN, LOUT, K, GATHER, false, false>;
    if constexpr (GATHER) {
        if (ns) {
            auto kx = lp ? k_ews_bwd_x<CIN, COUT, LIN, LOUT, K, true, true, true, false>
                         : k_ews_bwd_x<CIN, COUT, LIN, LOUT, K, true, true, false, false>;
            if (dp && gpq)
                kx = lp ? k_ews_bwd_x<CIN, COUT, LIN, LOUT, K, true, true, true, true, true>
                        : k_ews_bwd_x<CIN, COUT, LIN, LOUT, K, true, true, false, true, true>;
            else if (dp)
                kx = lp ? k_ews_bwd_x<CIN, COUT, LIN, LOUT, K, true, true, true, true>
                        : k_ews_bwd_x<CIN, COUT, LIN, LOUT, K, true, true, false, true>;
            else if (gpq)
                kx = lp ? k_ews_bwd_x<CIN, COUT, LIN, LOUT, K, true, true, true, false, true>
                        : k_ews_bwd_x<CIN, COUT, LIN, LOUT, K, true, true, false, false, true>;
            if (int rc = ews_set_lds(reinterpret_cast<const void*>(kx), xlds)) return rc;
            FEQ_LAUNCH("k_ews_bwd_x", kx, dim3(G), dim3(kThreads), xlds, s, B, E, ntiles, gy, x, P, Q,
                       dist, frag, inv, F, nullptr, dFe, NS, DP, bym, bgP, bgQ);
            if (int rc = node_fix(NS, x.nsrc, static_cast<int64_t>(CIN * T::DIN / 4), s)) return rc;
        }
        if (dp)
            kc = lp ? k_ews_bwd_c<CIN, COUT, LIN, LOUT, K, true, true, true>
                    : k_ews_bwd_c<CIN, COUT, LIN, LOUT, K, true, false, true>;
        else if (lp)
            kc = k_ews_bwd_c<CIN, COUT, LIN, LOUT, K, true, true, false>;
    } else {
        if (ns) return fail(FEQ_ERR_INVALID, "per-node sums need the message-passing form");
    }
    if (!ns) {
        auto kx = gpq ? k_ews_bwd_x<CIN, COUT, LIN, LOUT, K, GATHER, false, false, false, true>
                      : k_ews_bwd_x<CIN, COUT, LIN, LOUT, K, GATHER, false, false, false>;
        if (int rc = ews_set_lds(reinterpret_cast<const void*>(kx), xlds)) return rc;
        FEQ_LAUNCH("k_ews_bwd_x", kx, dim3(G), dim3(kThreads), xlds, s, B, E, ntiles, gy, x, P, Q,
                   dist, frag, inv, F, gx, dFe, NS, DP, bym, bgP, bgQ);
    }
    if (int rc = ews_set_lds(reinterpret_cast<const void*>(kc), clds)) return rc;
    FEQ_LAUNCH("k_ews_bwd_c", kc, dim3(G), dim3(kThreads), clds, s, B, E, ntiles, gy, x, P, Q,
               dist, F, dCp, DP);
    return ew_tail(L, B, K, E, dist, F, dFe, dCp, G, ncc, gC, gF, gdist, tail, s);
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

int node_fix(const NodeScatter& ns, int64_t nsrc, int64_t row4, hipStream_t s) {
    if (nsrc > 0)
        FEQ_LAUNCH("k_ews_node_fix", k_ews_node_fix, dim3(static_cast<unsigned>(nsrc)), dim3(64), 0, s,
                   ns, row4);
    return FEQ_OK;
}

// Shapes with a split-fp16 fast path: (Cin, Cout, Lin, Lout), rank 4.
#define FEQ_EWS_SHAPES(X) \
    X(64, 64, 2, 2)       \
    X(64, 64, 1, 2)       \
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

size_t ew_split_bwd_workspace(const feq_layout& L, const feq_binning& B, int rank, int64_t E,
                              bool nodes) {
    if (rank != 4) return 0;
    if (ew0_supported(L, rank)) return ew0_bwd_workspace(L, B, rank, E, nodes);
#define FEQ_WS(ci, co, li, lo)                                                                 \
    if constexpr ((ci) % 64 == 0) {                                                            \
        if (L.cin == ci && L.cout == co && canonical(L, li, lo))                               \
            return ews_bwd_ws<ci, co, li, lo, 4>(B, E, nodes);                                 \
    }
    FEQ_EWS_SHAPES(FEQ_WS)
#undef FEQ_WS
    return 0;
}

int ew_split_bwd(const feq_layout& L, const feq_binning& B, int rank, int64_t E, const float* gy,
                 const float* x, const int64_t* src, int64_t nsrc, const float* P, const float* Q,
                 const float* dist, const float* C, const float* F, float* gx, float* gC, float* gF,
                 float* gdist, const NodeScatter* ns, void* ws, size_t ws_bytes, bool lp, hipStream_t s,
                 const DstPool* dp, const BasisGrads* bg) {
    float* gout = ns ? ns->out : gx;
    if (rank != 4 || !gout || !aligned16(gy) || !aligned16(x) || !aligned16(P) || !aligned16(Q) ||
        !aligned16(gout) || (ns && !src))
        return -1;
    if (ew0_supported(L, rank)) {
        if (dp) return fail(FEQ_ERR_UNSUPPORTED, "no pooled form for scalar-output layouts");
        return ew0_bwd(L, B, rank, E, gy, x, src, nsrc, P, Q, dist, C, F, gx, gC, gF, gdist, ns, ws,
                       ws_bytes, s, bg ? bg->ym : nullptr, bg ? bg->gP : nullptr, bg ? bg->gQ : nullptr);
    }
    if (dp && !src) return fail(FEQ_ERR_INVALID, "the pooled form needs the message-passing form");
    const XRows X{x, src, nsrc};
#define FEQ_BWD(ci, co, li, lo)                                                                   \
    if constexpr ((ci) % 64 == 0) {                                                               \
        if (L.cin == ci && L.cout == co && canonical(L, li, lo))                                  \
            return src ? launch_ews_bwd<ci, co, li, lo, 4, true>(L, B, E, gy, X, P, Q, dist, C, F, \
                                                                 gx, gC, gF, gdist, ns, ws, ws_bytes, lp, dp, s, bg) \
                       : launch_ews_bwd<ci, co, li, lo, 4, false>(L, B, E, gy, X, P, Q, dist, C, F, \
                                                                  gx, gC, gF, gdist, ns, ws, ws_bytes, lp, dp, s, bg); \
    }
    FEQ_EWS_SHAPES(FEQ_BWD)
#undef FEQ_BWD
    return -1;
}

int ew_split_fwd(const feq_layout& L, const feq_binning& B, int rank, int64_t E, const float* x,
                 const int64_t* src, int64_t nsrc, const float* P, const float* Q, const float* dist,
                 const float* C, const float* F, float* y, void* ws, size_t ws_bytes, bool lp,
                 hipStream_t s, const DstPool* dp, const BasisGrads* bg) {
    if (rank != 4) return -1;
    float* ym = bg ? bg->ym_out : nullptr;
    if (ew0_supported(L, rank)) {
        if (dp) return fail(FEQ_ERR_UNSUPPORTED, "no pooled form for scalar-output layouts");
        return ew0_fwd(L, B, rank, E, x, src, nsrc, P, Q, dist, C, F, y, ym, s);
    }
    if (!aligned16(x) || !aligned16(P) || !aligned16(Q) || !aligned16(y) || (dp && !aligned16(dp->out)) ||
        (ym && !aligned16(ym)))
        return -1;
    if (dp && !src) return fail(FEQ_ERR_INVALID, "the pooled form needs the message-passing form");
    const XRows X{x, src, nsrc};
#define FEQ_FWD(ci, co, li, lo)                                                                  \
    if (L.cin == ci && L.cout == co && canonical(L, li, lo))                                     \
        return src ? launch_ews_fwd<ci, co, li, lo, 4, true>(B, E, X, P, Q, dist, C, F, y, ws,    \
                                                             ws_bytes, lp, dp, s, ym)             \
                   : launch_ews_fwd<ci, co, li, lo, 4, false>(B, E, X, P, Q, dist, C, F, y, ws,   \
                                                              ws_bytes, lp, dp, s, ym);
    FEQ_EWS_SHAPES(FEQ_FWD)
#undef FEQ_FWD
    return -1;
}

// Shapes the split kernels (and so the message-passing entry points) serve.
bool ew_split_supported(const feq_layout& L, const feq_binning& B, int rank, bool backward) {
    if (rank != 4) return false;
    if (ew0_supported(L, rank)) return true;
    bool ok = false;
#define FEQ_SUP(ci, co, li, lo)                                                          \
    if (L.cin == ci && L.cout == co && canonical(L, li, lo))                             \
        ok = backward ? ((ci) % 64 == 0 && ew_tail_supported(B, 4 * L.wdim)) : true;
    FEQ_EWS_SHAPES(FEQ_SUP)
#undef FEQ_SUP
    return ok;
}

bool ew_split_pq_supported(const feq_layout& L, const feq_binning& B, int rank) {
    return rank == 4 && ew_split_supported(L, B, rank, true);
}

bool ew_pool_supported(const feq_layout& L, const feq_binning& B, int rank) {
    return rank == 4 && !ew0_supported(L, rank) && ew_split_supported(L, B, rank, true);
}

size_t ew_pool_fwd_workspace(const feq_layout& L, int rank, int64_t E) {
    if (rank != 4) return 0;
#define FEQ_WS(ci, co, li, lo) \
    if (L.cin == ci && L.cout == co && canonical(L, li, lo)) return ews_pool_fwd_ws<ci, co, li, lo, 4>(E);
    FEQ_EWS_SHAPES(FEQ_WS)
#undef FEQ_WS
    return 0;
}

}  // namespace feq

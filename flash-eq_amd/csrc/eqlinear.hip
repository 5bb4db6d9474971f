// EquivariantLinear on component-major node tables (linear.py:242-268 of the
// reference mixes the channels of each degree with its own weight and adds the
// bias to the scalar degrees): for every component d of the representation,
//   out[d] = in[d] B_k(d) (+ bias[:, j] when d is the j-th scalar irrep with a bias),
// in (D, rows, K), out (D, rows, NOUT), B_k the (K, NOUT) matrix of irrep k.
// The forward takes B_k = W_k^T (K = Cin, NOUT = Cout), the input gradient
// B_k = W_k (K = Cout, NOUT = Cin) and no bias.
//
// The rows are tall and the matrices narrow (K, NOUT of 32..128): float32
// library GEMMs run these at a third of either the HBM or the fp32 matrix-core
// bound.  Here every product runs on the fp16 matrix cores with split operands
// (v = hi + lo, both fp16, of v scaled by a power of two): hi B_hi + hi B_lo +
// lo B_hi carries ~22 bits per product, float32 accumulation, so the result
// matches a float32 GEMM to within its own rounding, and the matrix work is 5x
// below the bytes: the kernel streams in and out at HBM speed.
//
// One launch covers every component: waves walk contiguous runs of 16-row
// blocks of the (d, row) space (two workgroups of four waves per CU); a wave holds the
// B_k fragments (split once per call by k_eql_prep) of its output columns --
// all of them for most layouts -- in registers while the component's irrep
// stays the same.  Lane l
// reads row l % 16 of the block, columns 8 (l / 16) .. + 7 of each 32-step
// (two 16-byte loads), which is the A layout of v_mfma_f32_16x16x32_f16; each
// row gets its own scale from its largest magnitude (four lanes hold a row),
// undone on the accumulators with the column's B scale.  The next two
// blocks' rows are in flight during a block's products.
#include "feq_internal.h"

#include <type_traits>

namespace feq {
namespace {

typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));

constexpr int kEqlMaxComps = 64;   // components (dim) of one representation
constexpr int kEqlMaxReps = 16;    // irreps

// Per-component irrep index and bias column (-1: none), passed by value.
struct EqlMap {
    int8_t irrep[kEqlMaxComps];
    int8_t bcol[kEqlMaxComps];
};

__device__ __forceinline__ v4f mfma16(h8 a, h8 b, v4f c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Power-of-two scale exponent e for a block whose largest magnitude is m:
// m 2^e in [2^14, 2^15); clamped so that 2^e and 2^-e are normal floats.
__device__ __forceinline__ int eql_scale_exp(float m) {
    const int ex = static_cast<int>((__float_as_uint(m) >> 23) & 0xffu);
    int e = 141 - ex;
    e = e < -113 ? -113 : e;
    return e > 126 ? 126 : e;
}

__device__ __forceinline__ float eql_exp2i(int e) {
    return __uint_as_float(static_cast<unsigned>(e + 127) << 23);
}

// hi = fp16(a sc), lo = fp16(a sc - hi) (sc a power of two: a sc is exact)
__device__ __forceinline__ void eql_split(float a, float sc, _Float16& hi, _Float16& lo) {
    hi = static_cast<_Float16>(__builtin_fmaf(a, sc, 0.0f));
    lo = static_cast<_Float16>(__builtin_fmaf(a, sc, -static_cast<float>(hi)));
}

// B fragments of every irrep: for irrep k, 32-step s and column block c, lane
// l holds column 16 c + l % 16, rows 32 s + 8 (l / 16) + j (j = 0..7) of B_k
// as fp16 hi and lo (two h8 per lane, hi first), each column scaled by its own
// power of two (binv[k NOUT + n] = 1 / scale).  One wave per (irrep, column
// block): its four lane groups hold a column's rows, so the column maximum is
// two lane exchanges.
// trans = 0: B_k[kk][n] = W[(k NOUT + n) K + kk] (W_k^T of W (nreps NOUT, K));
// trans = 1: B_k[kk][n] = W[(k K + kk) NOUT + n] (W_k of W (nreps K, NOUT)).
template <int K, int NOUT>
__global__ void __launch_bounds__(64)
k_eql_prep(const float* __restrict__ W, int trans, h8* __restrict__ frag, float* __restrict__ binv) {
    constexpr int NS = K / 32, NC = NOUT / 16;
    const int k = blockIdx.x / NC, c = blockIdx.x % NC;
    const int lane = threadIdx.x, lr = lane & 15, lg = lane >> 4;
    const int n = 16 * c + lr;
    const float* Wk = W + static_cast<int64_t>(k) * K * NOUT;
    float b[NS][8];
    float m = 0.0f;
#pragma unroll
    for (int s = 0; s < NS; ++s)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int kk = 32 * s + 8 * lg + j;
            b[s][j] = trans ? Wk[kk * NOUT + n] : Wk[n * K + kk];
            m = fmaxf(m, fabsf(b[s][j]));
        }
    m = fmaxf(m, __shfl_xor(m, 16, 64));
    m = fmaxf(m, __shfl_xor(m, 32, 64));
    const int e = eql_scale_exp(m);
    const float sc = eql_exp2i(e);
    if (lg == 0) binv[k * NOUT + n] = eql_exp2i(-e);
    h8* fk = frag + static_cast<int64_t>(k) * NS * NC * 64 * 2;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
        h8 hi, lo;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            _Float16 h, l;
            eql_split(b[s][j], sc, h, l);
            hi[j] = h;
            lo[j] = l;
        }
        const int q = (s * NC + c) * 64 + lane;
        fk[2 * q] = hi;
        fk[2 * q + 1] = lo;
    }
}

// Waves per 16-row block: the fewest (1, 2 or 4) for which a wave's share of
// the B_k fragments (8 VGPRs per 32-step and column block), its two row
// buffers and the split rows (24 VGPRs per 32-step) stay within 200 VGPRs, so
// that most layouts give each wave rows of its own and all output columns.
template <int K, int NOUT>
constexpr int eql_wpb() {
    constexpr int NS = K / 32, NC = NOUT / 16;
    return NS * NC * 8 + NS * 24 <= 200 ? 1 : NS * (NC / 2) * 8 + NS * 24 <= 200 ? 2 : 4;
}

// Blocks in flight per wave.
template <int K, int NOUT>
constexpr int eql_depth() { return 2; }

// out[d] = in[d] B_k(d) (+ bias) for in (D, rows, K), out (D, rows, NOUT).
// Workgroups of four waves; WPB waves share a 16-row block (each with NCB of
// its column blocks), so a workgroup works on 4 / WPB blocks at a time.  Each
// wave takes a contiguous run of blocks (so its irrep, and with it the B
// fragments in its registers, rarely changes) and keeps the rows of its next
// PD blocks in flight.  The finished block goes through LDS, so that it
// leaves as 16-byte row segments (a few wide stores rather than one 4-byte
// store per accumulator: vector-memory waits count stores too); each wave
// stages and stores only its own columns, so no barrier spans waves.
template <int K, int NOUT>
__global__ void __launch_bounds__(256, 2)
k_eql_mm(const float* __restrict__ in, int64_t rows, int D, EqlMap map, const h8* __restrict__ frag,
         const float* __restrict__ binv, const float* __restrict__ bias, int nbias,
         float* __restrict__ out) {
    constexpr int WPB = eql_wpb<K, NOUT>();
    constexpr int NCB = NOUT / 16 / WPB;                 // column blocks per wave
    constexpr int NS = K / 32;                           // 32-steps
    constexpr int SLOTS = 4 / WPB;                       // row blocks per workgroup at a time
    constexpr int PD = eql_depth<K, NOUT>();             // blocks in flight per wave
    constexpr int OS = NOUT + 4;                         // LDS row stride of the output stage (floats)
    static_assert(K % 32 == 0 && NOUT % 16 == 0 && NCB * WPB * 16 == NOUT, "unsupported sizes");
    __shared__ __align__(16) float sOut[SLOTS][16 * OS];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int slot = wave / WPB, cg = wave % WPB;       // row-block slot, column group
    const int lr = lane & 15, lg = lane >> 4;
    const uint32_t nb = static_cast<uint32_t>((rows + 15) / 16);
    const uint32_t total = nb * static_cast<uint32_t>(D);
    // this slot's contiguous run of blocks
    const uint32_t nslot = gridDim.x * SLOTS, sid = blockIdx.x * SLOTS + slot;
    const uint32_t per = total / nslot, extra = total % nslot;
    const uint32_t bbeg = sid * per + (sid < extra ? sid : extra);
    const uint32_t bend = bbeg + per + (sid < extra ? 1 : 0);

    h8 bh[NS][NCB], bl[NS][NCB];
    float cinv[NCB];   // 1 / scale of this lane's column in each of the wave's column blocks
    int kcur = -1;

    auto load = [&](uint32_t blk, float (&a)[NS][8]) {
        const uint32_t d = blk / nb;
        const int64_t r = static_cast<int64_t>(blk - d * nb) * 16 + lr;
        const bool ok = r < rows;
        const float* src = in + ((static_cast<int64_t>(d) * rows + (ok ? r : 0)) * K + 8 * lg);
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const float4 u = *reinterpret_cast<const float4*>(src + 32 * s);
            const float4 v = *reinterpret_cast<const float4*>(src + 32 * s + 4);
            a[s][0] = ok ? u.x : 0.0f;
            a[s][1] = ok ? u.y : 0.0f;
            a[s][2] = ok ? u.z : 0.0f;
            a[s][3] = ok ? u.w : 0.0f;
            a[s][4] = ok ? v.x : 0.0f;
            a[s][5] = ok ? v.y : 0.0f;
            a[s][6] = ok ? v.z : 0.0f;
            a[s][7] = ok ? v.w : 0.0f;
        }
    };

    auto block = [&](uint32_t blk, const float (&a)[NS][8]) {
        const uint32_t d = blk / nb;
        const int64_t r0 = static_cast<int64_t>(blk - d * nb) * 16;
        const int k = map.irrep[d];
        if (k != kcur) {   // wave-uniform: the fragments of this irrep's columns
            const h8* fk = frag + static_cast<int64_t>(k) * NS * (NOUT / 16) * 64 * 2;
#pragma unroll
            for (int s = 0; s < NS; ++s)
#pragma unroll
                for (int c = 0; c < NCB; ++c) {
                    const int q = (s * (NOUT / 16) + cg * NCB + c) * 64 + lane;
                    bh[s][c] = fk[2 * q];
                    bl[s][c] = fk[2 * q + 1];
                }
#pragma unroll
            for (int c = 0; c < NCB; ++c) cinv[c] = binv[k * NOUT + 16 * (cg * NCB + c) + lr];
            kcur = k;
        }
        // this row's scale: its largest magnitude over the four lanes holding it
        float m = 0.0f;
#pragma unroll
        for (int s = 0; s < NS; ++s)
#pragma unroll
            for (int j = 0; j < 8; ++j) m = fmaxf(m, fabsf(a[s][j]));
        m = fmaxf(m, __shfl_xor(m, 16, 64));
        m = fmaxf(m, __shfl_xor(m, 32, 64));
        const int e = eql_scale_exp(m);
        const float sc = eql_exp2i(e);
        const float rinv = eql_exp2i(-e);
        h8 ah[NS], al[NS];
#pragma unroll
        for (int s = 0; s < NS; ++s)
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                _Float16 h, l;
                eql_split(a[s][j], sc, h, l);
                ah[s][j] = h;
                al[s][j] = l;
            }
        // accumulator rows 4 lg + i: their scales from the lanes holding those rows
        float ri[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) ri[i] = __shfl(rinv, 4 * lg + i, 64);
        const int bc = map.bcol[d];
        float* so = sOut[slot];
#pragma unroll
        for (int c = 0; c < NCB; ++c) {
            v4f acc = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int s = 0; s < NS; ++s) {
                acc = mfma16(al[s], bh[s][c], acc);
                acc = mfma16(ah[s], bl[s][c], acc);
                acc = mfma16(ah[s], bh[s][c], acc);
            }
            const int n = 16 * (cg * NCB + c) + lr;
            const float bv = bc >= 0 ? bias[static_cast<int64_t>(n) * nbias + bc] : 0.0f;
#pragma unroll
            for (int i = 0; i < 4; ++i) so[(4 * lg + i) * OS + n] = acc[i] * (ri[i] * cinv[c]) + bv;
        }
        // the wave's own columns of the 16 rows leave as 16-byte segments (each
        // wave reads back only what it staged: no barrier between waves)
        __builtin_amdgcn_wave_barrier();
        constexpr int C4 = NCB * 4;                     // float4s per row and wave
        float* dst = out + (static_cast<int64_t>(d) * rows + r0) * NOUT + 16 * cg * NCB;
        const float* src = so + 16 * cg * NCB;
#pragma unroll
        for (int q = lane; q < 16 * C4; q += 64) {
            const int row = q / C4, c4 = q % C4;
            if (r0 + row < rows)
                *reinterpret_cast<float4*>(dst + static_cast<int64_t>(row) * NOUT + 4 * c4) =
                    *reinterpret_cast<const float4*>(src + row * OS + 4 * c4);
        }
        __builtin_amdgcn_wave_barrier();
    };

    // PD blocks in flight: the buffers rotate with static indices (unrolled)
    float a[PD][NS][8];
#pragma unroll
    for (int p = 0; p < PD; ++p)
        if (bbeg + p < bend) load(bbeg + p, a[p]);
    for (uint32_t blk = bbeg; blk < bend; blk += PD) {
#pragma unroll
        for (int p = 0; p < PD; ++p) {
            if (blk + p < bend) {
                block(blk + p, a[p]);
                if (blk + p + PD < bend) load(blk + p + PD, a[p]);
            }
        }
    }
}

// ---- weight and bias gradients ---------------------------------------------------
// gW_k = sum over the rows of irrep k of gy^T x (CO x CI), gb_k = sum over those
// rows of gy (scalar irreps with a bias); an irrep's rows are contiguous in the
// component-major tables ((2l+1) rows per node).  A workgroup sums CPW chunks
// of 64 (or 32) rows of one irrep into one partial; k_eql_wsum adds the partials of
// each irrep in a fixed order (deterministic, no atomics).
//
// Per chunk the workgroup stages gy and x as fp16 hi / lo in LDS, row-major,
// each column scaled by its own power of two over the chunk (a column's
// largest magnitude: per-thread maxima, lane exchanges, the four waves through
// LDS), and reads the operands with ds_read_b64_tr_b16: a lane of a 16-lane
// group points at row s / 4, 4-column chunk s % 4 and receives 4 rows of one
// column, which for two reads is the A / B layout of v_mfma_f32_16x16x32_f16
// with the chunk's rows as the reduction.  The waves form a 2 x 2 grid over
// the (CO / 16) x (CI / 16) output blocks; each 32-row step's products are
// unscaled (row and column scales) into the launch-long accumulators.  The
// next chunk's rows are loaded during the products.
struct EqlWg {
    int64_t row0[kEqlMaxReps];    // first table row of the irrep
    int64_t nrows[kEqlMaxReps];   // its rows ((2l+1) rows per node)
    int32_t wg0[kEqlMaxReps + 1]; // its first workgroup
    int32_t nreps, cpw;           // irreps; chunks per workgroup
};

typedef short v4s __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4s lds_v4s;

// Two transposing reads: rows 0..3 of one column from a, rows 4..7 from b.
__device__ __forceinline__ h8 tr_h8(const _Float16* a, const _Float16* b) {
    const v4s x = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(a));
    const v4s y = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(b));
    typedef short v8s __attribute__((ext_vector_type(8)));
    const v8s v = {x[0], x[1], x[2], x[3], y[0], y[1], y[2], y[3]};
    return __builtin_bit_cast(h8, v);
}

// Rows per staged chunk: 64, or 32 where the staged rows of both tables would
// not fit the registers beside the accumulators (128 x 128).
constexpr int eql_chunk_rows(int CO, int CI) { return CO + CI > 192 ? 32 : 64; }

template <int CO, int CI>
__global__ void __launch_bounds__(256, 2)
k_eql_wgrad(const float* __restrict__ G, const float* __restrict__ X, EqlWg T, float* __restrict__ pw,
            float* __restrict__ pb) {
    constexpr int RC = eql_chunk_rows(CO, CI);               // rows per chunk
    constexpr int GS = CO + 8, XS = CI + 8;                  // LDS row strides (halves)
    constexpr int QG = CO / 4, PG = 256 / QG, NG = RC / PG;  // gy staging: column quads, row phases, rows
    constexpr int QX = CI / 4, PX = 256 / QX, NX = RC / PX;
    constexpr int RPW = CO / 32, CPW = CI / 32;              // row / column blocks per wave (2 x 2 waves)
    static_assert(CO % 32 == 0 && CI % 32 == 0 && QG <= 64 && QX <= 64, "unsupported sizes");
    __shared__ __align__(16) _Float16 sG[2][RC * GS];
    __shared__ __align__(16) _Float16 sX[2][RC * XS];
    __shared__ float sMax[4][CO + CI];
    __shared__ float sSum[4][CO];
    __shared__ float sInv[CO + CI];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    int k = 0;
    while (k + 1 < T.nreps && static_cast<int>(blockIdx.x) >= T.wg0[k + 1]) ++k;
    const int64_t nrows = T.nrows[k];
    const int64_t nch = (nrows + RC - 1) / RC;
    const int64_t cbeg = static_cast<int64_t>(blockIdx.x - T.wg0[k]) * T.cpw;
    const int64_t cend = cbeg + T.cpw < nch ? cbeg + T.cpw : nch;
    const float* Gk = G + T.row0[k] * CO;
    const float* Xk = X + T.row0[k] * CI;

    const int qg = tid % QG, pg = tid / QG, qx = tid % QX, px = tid / QX;
    float gv[NG][4], xv[NX][4];
    auto load = [&](int64_t c) {
        const int64_t r0 = c * RC;
#pragma unroll
        for (int i = 0; i < NG; ++i) {
            const int64_t r = r0 + pg + PG * i;
            float4 u = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (r < nrows) u = *reinterpret_cast<const float4*>(Gk + r * CO + 4 * qg);
            gv[i][0] = u.x; gv[i][1] = u.y; gv[i][2] = u.z; gv[i][3] = u.w;
        }
#pragma unroll
        for (int i = 0; i < NX; ++i) {
            const int64_t r = r0 + px + PX * i;
            float4 u = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (r < nrows) u = *reinterpret_cast<const float4*>(Xk + r * CI + 4 * qx);
            xv[i][0] = u.x; xv[i][1] = u.y; xv[i][2] = u.z; xv[i][3] = u.w;
        }
    };

    const int wr = wave >> 1, wc = wave & 1;
    const int lg = lane >> 4, ls = lane & 15;
    v4f acc[RPW][CPW];
#pragma unroll
    for (int i = 0; i < RPW; ++i)
#pragma unroll
        for (int j = 0; j < CPW; ++j) acc[i][j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    float bacc = 0.0f;   // thread t < CO: the bias gradient partial of column t

    if (cbeg < cend) load(cbeg);
    for (int64_t c = cbeg; c < cend; ++c) {
        // column maxima (and gy column sums) over this thread's rows, then over
        // the row phases of the wave
        float mg[4], sg[4], mx[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            mg[q] = 0.0f;
            sg[q] = 0.0f;
            mx[q] = 0.0f;
#pragma unroll
            for (int i = 0; i < NG; ++i) {
                mg[q] = fmaxf(mg[q], fabsf(gv[i][q]));
                sg[q] += gv[i][q];
            }
#pragma unroll
            for (int i = 0; i < NX; ++i) mx[q] = fmaxf(mx[q], fabsf(xv[i][q]));
        }
#pragma unroll
        for (int off = QG; off < 64; off <<= 1)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                mg[q] = fmaxf(mg[q], __shfl_xor(mg[q], off, 64));
                sg[q] += __shfl_xor(sg[q], off, 64);
            }
#pragma unroll
        for (int off = QX; off < 64; off <<= 1)
#pragma unroll
            for (int q = 0; q < 4; ++q) mx[q] = fmaxf(mx[q], __shfl_xor(mx[q], off, 64));
        if (lane < QG)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                sMax[wave][4 * qg + q] = mg[q];
                sSum[wave][4 * qg + q] = sg[q];
            }
        if (lane < QX)
#pragma unroll
            for (int q = 0; q < 4; ++q) sMax[wave][CO + 4 * qx + q] = mx[q];
        __syncthreads();
        // scale, split and stage this thread's rows
        {
            float m[4];
#pragma unroll
            for (int q = 0; q < 4; ++q)
                m[q] = fmaxf(fmaxf(sMax[0][4 * qg + q], sMax[1][4 * qg + q]),
                             fmaxf(sMax[2][4 * qg + q], sMax[3][4 * qg + q]));
            float sc[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int e = eql_scale_exp(m[q]);
                sc[q] = eql_exp2i(e);
                if (pg == 0) sInv[4 * qg + q] = eql_exp2i(-e);
            }
#pragma unroll
            for (int i = 0; i < NG; ++i) {
                h4 hv, lv;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    _Float16 h, l;
                    eql_split(gv[i][q], sc[q], h, l);
                    hv[q] = h;
                    lv[q] = l;
                }
                *reinterpret_cast<h4*>(&sG[0][(pg + PG * i) * GS + 4 * qg]) = hv;
                *reinterpret_cast<h4*>(&sG[1][(pg + PG * i) * GS + 4 * qg]) = lv;
            }
#pragma unroll
            for (int q = 0; q < 4; ++q)
                m[q] = fmaxf(fmaxf(sMax[0][CO + 4 * qx + q], sMax[1][CO + 4 * qx + q]),
                             fmaxf(sMax[2][CO + 4 * qx + q], sMax[3][CO + 4 * qx + q]));
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int e = eql_scale_exp(m[q]);
                sc[q] = eql_exp2i(e);
                if (px == 0) sInv[CO + 4 * qx + q] = eql_exp2i(-e);
            }
#pragma unroll
            for (int i = 0; i < NX; ++i) {
                h4 hv, lv;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    _Float16 h, l;
                    eql_split(xv[i][q], sc[q], h, l);
                    hv[q] = h;
                    lv[q] = l;
                }
                *reinterpret_cast<h4*>(&sX[0][(px + PX * i) * XS + 4 * qx]) = hv;
                *reinterpret_cast<h4*>(&sX[1][(px + PX * i) * XS + 4 * qx]) = lv;
            }
            if (tid < CO) bacc += (sSum[0][tid] + sSum[1][tid]) + (sSum[2][tid] + sSum[3][tid]);
        }
        if (c + 1 < cend) load(c + 1);
        __syncthreads();
        // the column scales of this wave's blocks (output row co = 16 mb + 4 lg + r
        // is a gy column, output column ci = 16 nb + ls an x column)
        float ix[CPW];
#pragma unroll
        for (int j = 0; j < CPW; ++j) ix[j] = sInv[CO + 16 * (wc * CPW + j) + ls];
#pragma unroll
        for (int ks = 0; ks < RC / 32; ++ks) {
            const int ra = 32 * ks + 8 * lg + (ls >> 2), ca = 4 * (ls & 3);
            h8 bh[CPW], bl[CPW];
#pragma unroll
            for (int j = 0; j < CPW; ++j) {
                const int col = 16 * (wc * CPW + j) + ca;
                bh[j] = tr_h8(&sX[0][ra * XS + col], &sX[0][(ra + 4) * XS + col]);
                bl[j] = tr_h8(&sX[1][ra * XS + col], &sX[1][(ra + 4) * XS + col]);
            }
#pragma unroll
            for (int i = 0; i < RPW; ++i) {
                const int col = 16 * (wr * RPW + i) + ca;
                const h8 ah = tr_h8(&sG[0][ra * GS + col], &sG[0][(ra + 4) * GS + col]);
                const h8 al = tr_h8(&sG[1][ra * GS + col], &sG[1][(ra + 4) * GS + col]);
                float ig[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) ig[r] = sInv[16 * (wr * RPW + i) + 4 * lg + r];
#pragma unroll
                for (int j = 0; j < CPW; ++j) {
                    v4f t = v4f{0.0f, 0.0f, 0.0f, 0.0f};
                    t = mfma16(al, bh[j], t);
                    t = mfma16(ah, bl[j], t);
                    t = mfma16(ah, bh[j], t);
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc[i][j][r] += t[r] * (ig[r] * ix[j]);
                }
            }
        }
        __syncthreads();   // every wave is done with this chunk's LDS
    }
    float* pwk = pw + static_cast<int64_t>(blockIdx.x) * CO * CI;
#pragma unroll
    for (int i = 0; i < RPW; ++i)
#pragma unroll
        for (int j = 0; j < CPW; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                pwk[(16 * (wr * RPW + i) + 4 * lg + r) * CI + 16 * (wc * CPW + j) + ls] = acc[i][j][r];
    if (tid < CO) pb[static_cast<int64_t>(blockIdx.x) * CO + tid] = bacc;
}

// Sum of the partials p[w0 .. w1) at stride st by the eight lanes j = lane % 8
// of an aligned lane octet: lane j adds partials w0 + j, w0 + j + 8, ... (two
// chains, so that two loads are in flight), then the octet combines its eight
// sums over lane bits 0, 1, 2: a fixed order.
__device__ __forceinline__ float eql_octet_sum(const float* __restrict__ p, int w0, int w1, int64_t st,
                                               int j) {
    float a0 = 0.0f, a1 = 0.0f;
    int w = w0 + j;
    for (; w + 8 < w1; w += 16) {
        a0 += p[static_cast<int64_t>(w) * st];
        a1 += p[static_cast<int64_t>(w + 8) * st];
    }
    if (w < w1) a0 += p[static_cast<int64_t>(w) * st];
    float v = a0 + a1;
    v += __shfl_xor(v, 1, 64);
    v += __shfl_xor(v, 2, 64);
    v += __shfl_xor(v, 4, 64);
    return v;
}

// gW[k] = sum of irrep k's partials (a fixed order); gb[co][bcol[k]] likewise
// for the scalar irreps with a bias column.  Eight lanes per output element.
__global__ void __launch_bounds__(256)
k_eql_wsum(const float* __restrict__ pw, const float* __restrict__ pb, EqlWg T, EqlMap bmap, int CO,
           int CI, int nbias, float* __restrict__ gw, float* __restrict__ gb) {
    const int64_t nw = static_cast<int64_t>(T.nreps) * CO * CI;
    const int64_t i = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) >> 3;
    const int j = threadIdx.x & 7;
    // every lane of an octet takes the same branch (i is per octet)
    if (i < nw) {
        const int k = static_cast<int>(i / (static_cast<int64_t>(CO) * CI));
        const int64_t e = i - static_cast<int64_t>(k) * CO * CI;
        const float v = eql_octet_sum(pw + e, T.wg0[k], T.wg0[k + 1], static_cast<int64_t>(CO) * CI, j);
        if (j == 0) gw[i] = v;
    } else if (gb && i < nw + static_cast<int64_t>(T.nreps) * CO) {
        const int64_t q = i - nw;
        const int k = static_cast<int>(q / CO), co = static_cast<int>(q % CO);
        const int bc = bmap.bcol[k];
        if (bc >= 0) {
            const float v = eql_octet_sum(pb + co, T.wg0[k], T.wg0[k + 1], CO, j);
            if (j == 0) gb[static_cast<int64_t>(co) * nbias + bc] = v;
        }
    }
}

bool eql_map(const int32_t* lvals, int32_t nreps, const int32_t* bias_cols, EqlMap& m, int& D) {
    if (!lvals || nreps < 1 || nreps > kEqlMaxReps) return false;
    D = 0;
    for (int k = 0; k < nreps; ++k) {
        if (lvals[k] < 0) return false;
        const int n = 2 * lvals[k] + 1;
        if (D + n > kEqlMaxComps) return false;
        for (int i = 0; i < n; ++i) {
            m.irrep[D + i] = static_cast<int8_t>(k);
            const int bc = bias_cols ? bias_cols[k] : -1;
            m.bcol[D + i] = static_cast<int8_t>(lvals[k] == 0 && bc >= 0 ? bc : -1);
        }
        D += n;
    }
    return true;
}

int eql_cus() {
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) == hipSuccess) {
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
            cus = v;
    }
    return cus;
}

bool eql_sizes_ok(int K, int NOUT) {
    return (K == 32 || K == 64 || K == 128) && (NOUT == 32 || NOUT == 64 || NOUT == 128);
}

template <typename Fn>
int with_sizes(int K, int NOUT, Fn&& fn) {
#define FEQ_EQL_CASE(k, n) \
    if (K == k && NOUT == n) return fn(std::integral_constant<int, k>{}, std::integral_constant<int, n>{});
    FEQ_EQL_CASE(32, 32) FEQ_EQL_CASE(32, 64) FEQ_EQL_CASE(32, 128)
    FEQ_EQL_CASE(64, 32) FEQ_EQL_CASE(64, 64) FEQ_EQL_CASE(64, 128)
    FEQ_EQL_CASE(128, 32) FEQ_EQL_CASE(128, 64) FEQ_EQL_CASE(128, 128)
#undef FEQ_EQL_CASE
    return fail(FEQ_ERR_UNSUPPORTED, "equivariant linear: no kernel for %d -> %d channels", K, NOUT);
}

size_t eql_frag_bytes(int32_t nreps, int K, int NOUT) {
    return static_cast<size_t>(nreps) * (K / 32) * (NOUT / 16) * 64 * 2 * sizeof(h8);
}

int eql_run(const int32_t* lvals, int32_t nreps, int64_t rows, int K, int NOUT, int trans,
            const float* in, const float* W, const float* bias, int32_t nbias, const int32_t* bias_cols,
            float* out, void* ws, size_t ws_bytes, hipStream_t s) {
    EqlMap map{};
    int D = 0;
    if (!eql_map(lvals, nreps, bias ? bias_cols : nullptr, map, D))
        return fail(FEQ_ERR_INVALID, "equivariant linear: invalid lvals (at most %d irreps, %d components)",
                    kEqlMaxReps, kEqlMaxComps);
    if (rows < 0) return fail(FEQ_ERR_INVALID, "negative row count");
    if (bias && nbias < 1) return fail(FEQ_ERR_INVALID, "bias needs at least one column");
    if (bias)
        for (int k = 0; k < nreps; ++k)
            if (bias_cols[k] >= nbias) return fail(FEQ_ERR_INVALID, "bias column out of range");
    const size_t fb = eql_frag_bytes(nreps, K, NOUT);
    const size_t need = fb + 256 + sizeof(float) * kEqlMaxReps * NOUT;
    return with_sizes(K, NOUT, [&](auto KK, auto NN) -> int {
        constexpr int Kc = decltype(KK)::value, Nc = decltype(NN)::value;
        if (rows == 0) return FEQ_OK;
        if (!in || !W || !out || !ws) return fail(FEQ_ERR_INVALID, "NULL pointer");
        if ((reinterpret_cast<uintptr_t>(in) | reinterpret_cast<uintptr_t>(ws)) & 15)
            return fail(FEQ_ERR_INVALID, "input and workspace must be 16-byte aligned");
        if (ws_bytes < need) return fail(FEQ_ERR_WORKSPACE, "equivariant linear workspace too small");
        h8* frag = static_cast<h8*>(ws);
        float* binv = reinterpret_cast<float*>(static_cast<char*>(ws) + ((fb + 255) / 256) * 256);
        FEQ_LAUNCH("k_eql_prep", (k_eql_prep<Kc, Nc>), dim3(nreps * (Nc / 16)), dim3(64), 0, s, W, trans, frag,
                   binv);
        constexpr int SLOTS = 4 / eql_wpb<Kc, Nc>();
        const int64_t blocks = (rows + 15) / 16 * D;
        if (blocks > 0x7fffffffLL) return fail(FEQ_ERR_UNSUPPORTED, "equivariant linear: too many rows");
        const int64_t wgs = (blocks + SLOTS - 1) / SLOTS;
        const int64_t cap = static_cast<int64_t>(eql_cus()) * 2;   // one resident wave of workgroups
        const unsigned grid = static_cast<unsigned>(wgs < cap ? wgs : cap);
        FEQ_LAUNCH("k_eql_mm", (k_eql_mm<Kc, Nc>), dim3(grid), dim3(256), 0, s, in, rows, D, map, frag,
                   binv, bias, nbias, out);
        return FEQ_OK;
    });
}

// The workgroups of the weight gradient: chunks of rc rows per irrep, about
// two workgroups per CU in all.
EqlWg eql_wg_table(const int32_t* lvals, int32_t nreps, int64_t rows, int rc) {
    EqlWg T{};
    T.nreps = nreps;
    int64_t total = 0, row = 0;
    for (int k = 0; k < nreps; ++k) {
        T.row0[k] = row;
        T.nrows[k] = (2 * static_cast<int64_t>(lvals[k]) + 1) * rows;
        row += T.nrows[k];
        total += (T.nrows[k] + rc - 1) / rc;
    }
    const int64_t target = static_cast<int64_t>(eql_cus()) * 2;
    int64_t cpw = (total + target - 1) / target;
    T.cpw = static_cast<int32_t>(cpw < 1 ? 1 : cpw);
    int32_t w = 0;
    for (int k = 0; k < nreps; ++k) {
        T.wg0[k] = w;
        w += static_cast<int32_t>(((T.nrows[k] + rc - 1) / rc + T.cpw - 1) / T.cpw);
    }
    T.wg0[nreps] = w;
    return T;
}

size_t eql_wg_bytes(int32_t nwg, int CO, int CI) {
    return (static_cast<size_t>(nwg) * CO * CI + static_cast<size_t>(nwg) * CO) * sizeof(float) + 256;
}

}  // namespace

extern "C" size_t feq_eqlinear_bwd_w_workspace(const int32_t* lvals, int32_t nreps, int64_t rows,
                                               int32_t cin, int32_t cout) {
    EqlMap m{};
    int D = 0;
    if (rows < 0 || !eql_map(lvals, nreps, nullptr, m, D)) return 0;
    const EqlWg T = eql_wg_table(lvals, nreps, rows, eql_chunk_rows(cout, cin));
    return eql_wg_bytes(T.wg0[nreps], cout, cin);
}

extern "C" int feq_eqlinear_bwd_w(const int32_t* lvals, int32_t nreps, int64_t rows, int32_t cin,
                                  int32_t cout, const float* grad_y, const float* x, int32_t nbias,
                                  const int32_t* bias_cols, float* grad_w, float* grad_b, void* ws,
                                  size_t ws_bytes, feq_stream_t stream) {
    EqlMap map{};
    int D = 0;
    if (!eql_map(lvals, nreps, grad_b ? bias_cols : nullptr, map, D))
        return fail(FEQ_ERR_INVALID, "equivariant linear: invalid lvals (at most %d irreps, %d components)",
                    kEqlMaxReps, kEqlMaxComps);
    if (rows < 0) return fail(FEQ_ERR_INVALID, "negative row count");
    if (grad_b && (!bias_cols || nbias < 1)) return fail(FEQ_ERR_INVALID, "bias gradient needs bias columns");
    if (grad_b)
        for (int k = 0; k < nreps; ++k)
            if (bias_cols[k] >= nbias) return fail(FEQ_ERR_INVALID, "bias column out of range");
    if (!eql_sizes_ok(cout, cin))
        return fail(FEQ_ERR_UNSUPPORTED, "equivariant linear: no kernel for %d -> %d channels", cin, cout);
    if (!grad_w) return fail(FEQ_ERR_INVALID, "NULL grad_w");
    hipStream_t s = stream_of(stream);
    // per-irrep bias column of the scalar irreps (the sum kernel reads it by irrep)
    EqlMap bmap{};
    for (int k = 0; k < nreps; ++k)
        bmap.bcol[k] = static_cast<int8_t>(grad_b && lvals[k] == 0 && bias_cols[k] >= 0 ? bias_cols[k] : -1);
    const EqlWg T = eql_wg_table(lvals, nreps, rows, eql_chunk_rows(cout, cin));
    const int32_t nwg = T.wg0[nreps];
    if (nwg > 0) {
        if (!grad_y || !x || !ws) return fail(FEQ_ERR_INVALID, "NULL pointer");
        if ((reinterpret_cast<uintptr_t>(grad_y) | reinterpret_cast<uintptr_t>(x) |
             reinterpret_cast<uintptr_t>(ws)) & 15)
            return fail(FEQ_ERR_INVALID, "tables and workspace must be 16-byte aligned");
        if (ws_bytes < eql_wg_bytes(nwg, cout, cin))
            return fail(FEQ_ERR_WORKSPACE, "equivariant linear workspace too small");
    }
    float* pw = static_cast<float*>(ws);
    float* pb = pw + static_cast<size_t>(nwg) * cout * cin;
    if (nwg > 0) {
        const int rc = with_sizes(cout, cin, [&](auto CC, auto II) -> int {
            constexpr int CO = decltype(CC)::value, CI = decltype(II)::value;
            FEQ_LAUNCH("k_eql_wgrad", (k_eql_wgrad<CO, CI>), dim3(nwg), dim3(256), 0, s, grad_y, x, T, pw, pb);
            return FEQ_OK;
        });
        if (rc) return rc;
    }
    const int64_t n = static_cast<int64_t>(nreps) * cout * cin + static_cast<int64_t>(nreps) * cout;
    FEQ_LAUNCH("k_eql_wsum", k_eql_wsum, dim3(static_cast<unsigned>((8 * n + 255) / 256)), dim3(256), 0, s, pw,
               pb, T, bmap, static_cast<int>(cout), static_cast<int>(cin), nbias, grad_w, grad_b);
    return FEQ_OK;
}

extern "C" size_t feq_eqlinear_workspace(int32_t nreps, int32_t cin, int32_t cout) {
    if (nreps < 1 || cin < 32 || cout < 32) return 0;
    const size_t f = eql_frag_bytes(nreps, cin, cout), b = eql_frag_bytes(nreps, cout, cin);
    const size_t n = static_cast<size_t>(cin > cout ? cin : cout);
    return (f > b ? f : b) + 256 + sizeof(float) * kEqlMaxReps * n;
}

extern "C" int feq_eqlinear_supported(int32_t cin, int32_t cout) {
    return eql_sizes_ok(cin, cout) && eql_sizes_ok(cout, cin);
}

extern "C" int feq_eqlinear_fwd(const int32_t* lvals, int32_t nreps, int64_t rows, int32_t cin,
                                int32_t cout, const float* x, const float* weight, const float* bias,
                                int32_t nbias, const int32_t* bias_cols, float* y, void* ws,
                                size_t ws_bytes, feq_stream_t stream) {
    if (bias && !bias_cols) return fail(FEQ_ERR_INVALID, "bias needs bias_cols");
    return eql_run(lvals, nreps, rows, cin, cout, 0, x, weight, bias, nbias, bias_cols, y, ws, ws_bytes,
                   stream_of(stream));
}

extern "C" int feq_eqlinear_bwd_x(const int32_t* lvals, int32_t nreps, int64_t rows, int32_t cin,
                                  int32_t cout, const float* grad_y, const float* weight, float* grad_x,
                                  void* ws, size_t ws_bytes, feq_stream_t stream) {
    return eql_run(lvals, nreps, rows, cout, cin, 1, grad_y, weight, nullptr, 0, nullptr, grad_x, ws,
                   ws_bytes, stream_of(stream));
}

}  // namespace feq

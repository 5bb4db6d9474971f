// Dense helpers of the node-side layers: tiled transposes between node-major
// (rows, c, dim) and component-major (dim, rows, c) tables, deterministic
// column sums (bias gradients), and float32 dot products accumulated in
// float64 (gradients of scalar parameters).  All are single passes at HBM
// speed, deterministic, and free of memsets (safe to record into HIP graphs).
#include "feq_internal.h"

#include <type_traits>

namespace feq {
namespace {

constexpr int kTileElems = 4096;   // elements of one transpose tile

// q = n / d for n, d < 2^16 with m = ceil(2^32 / d) (2^32 itself for d = 1):
// n * m / 2^32 exceeds n / d by less than n * d / (d * 2^32) < 1 / d, so the
// floor is exact.
__device__ inline uint32_t div16(uint32_t n, uint64_t m) {
    return static_cast<uint32_t>((static_cast<uint64_t>(n) * m) >> 32);
}

inline uint64_t div16_magic(uint32_t d) { return ((uint64_t{1} << 32) + d - 1) / d; }

// out[b][j][i] = in[b][i][j] for in (batch, M, N).  A workgroup moves one
// TM x TN tile through LDS: the reads walk the tile's input rows, the writes its
// output rows, both in consecutive addresses.  With TN = N (narrow input) the
// tile's reads are one contiguous run, with TM = M (narrow output) its writes.
// The LDS row stride is odd so neither phase has bank conflicts.
template <typename T>
__global__ void __launch_bounds__(256)
k_transpose(const T* __restrict__ in, int64_t M, int64_t N, int TM, int TN, int S, uint64_t mag_tn,
            uint64_t mag_tm, int64_t tiles_n, T* __restrict__ out) {
    extern __shared__ __align__(16) unsigned char lds_raw[];
    T* s = reinterpret_cast<T*>(lds_raw);
    const int64_t tile = blockIdx.x;
    const int64_t tm = tile / tiles_n, tn = tile - tm * tiles_n;
    const int64_t m0 = tm * TM, n0 = tn * TN;
    const int h = static_cast<int>(M - m0 < TM ? M - m0 : TM);
    const int w = static_cast<int>(N - n0 < TN ? N - n0 : TN);
    const int64_t boff = static_cast<int64_t>(blockIdx.y) * M * N;
    const T* src = in + boff;
    T* dst = out + boff;
    const uint32_t total = static_cast<uint32_t>(TM) * TN;
    for (uint32_t i = threadIdx.x; i < total; i += 256) {
        const int r = static_cast<int>(div16(i, mag_tn));
        const int c = static_cast<int>(i) - r * TN;
        if (r < h && c < w) s[c * S + r] = src[(m0 + r) * N + n0 + c];
    }
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < total; i += 256) {
        const int c = static_cast<int>(div16(i, mag_tm));
        const int r = static_cast<int>(i) - c * TM;
        if (r < h && c < w) dst[(n0 + c) * M + m0 + r] = s[c * S + r];
    }
}

// The narrow transposes of float tables (in (batch, M, N) with N <= 32 or
// M <= 32: node-major <-> component-major moves) with 16-byte accesses on both
// sides.  NARROW_N: a tile is TM whole input rows, one contiguous run of TM N
// floats, and N output rows of TM floats; LDS holds it as the output rows
// (stride S = TM + 4, 16-byte aligned rows).  Otherwise (M <= 32) a tile is TN
// columns of the M input rows and one contiguous output run of TN M floats,
// held densely in LDS in output order.  The host takes this form when every
// row start is 16-byte aligned (M % 4 == 0, resp. N % 4 == 0, aligned bases).
template <bool NARROW_N>
__global__ void __launch_bounds__(256)
k_transpose4(const float* __restrict__ in, int64_t M, int64_t N, int TM, int TN, int S, uint64_t mag,
             int64_t tiles_n, float* __restrict__ out) {
    extern __shared__ float4 lds4[];
    float* s = reinterpret_cast<float*>(lds4);
    const int64_t tile = blockIdx.x;
    const int64_t tm = tile / tiles_n, tn = tile - tm * tiles_n;
    const int64_t m0 = tm * TM, n0 = tn * TN;
    const int h = static_cast<int>(M - m0 < TM ? M - m0 : TM);
    const int w = static_cast<int>(N - n0 < TN ? N - n0 : TN);
    const int64_t boff = static_cast<int64_t>(blockIdx.y) * M * N;
    const float* src = in + boff;
    float* dst = out + boff;
    const int tid = threadIdx.x;
    if constexpr (NARROW_N) {
        // read: the run of h rows x N, element i -> (r = i / N, c = i % N) -> s[c S + r]
        const float4* r4 = reinterpret_cast<const float4*>(src + m0 * N);
        const int run4 = h * static_cast<int>(N) / 4;
        for (int q = tid; q < run4; q += 256) {
            const float4 v = r4[q];
            const float e[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t i = 4 * q + j;
                const int r = static_cast<int>(div16(i, mag));
                const int c = static_cast<int>(i) - r * static_cast<int>(N);
                s[c * S + r] = e[j];
            }
        }
        __syncthreads();
        // write: N output rows of h floats at dst + c M + m0
        const int h4 = h / 4;
        for (int q = tid; q < static_cast<int>(N) * h4; q += 256) {
            const int c = q / h4, r = 4 * (q - c * h4);
            *reinterpret_cast<float4*>(dst + c * M + m0 + r) = *reinterpret_cast<const float4*>(s + c * S + r);
        }
    } else {
        // read: M input rows of w floats at src + r N + n0 -> s[c M + r] (output order)
        const int w4 = w / 4;
        for (int q = tid; q < static_cast<int>(M) * w4; q += 256) {
            const int r = q / w4, c = 4 * (q - r * w4);
            const float4 v = *reinterpret_cast<const float4*>(src + r * N + n0 + c);
            s[c * M + r] = v.x;
            s[(c + 1) * M + r] = v.y;
            s[(c + 2) * M + r] = v.z;
            s[(c + 3) * M + r] = v.w;
        }
        __syncthreads();
        // write: one contiguous run of w M floats at dst + n0 M
        float4* d4 = reinterpret_cast<float4*>(dst + n0 * M);
        const float4* s4 = reinterpret_cast<const float4*>(s);
        for (int q = tid; q < w * static_cast<int>(M) / 4; q += 256) d4[q] = s4[q];
    }
}

struct TransposePlan {
    int TM, TN, S;
    int64_t tiles_m, tiles_n;
};

TransposePlan transpose_plan(int64_t M, int64_t N) {
    TransposePlan p{};
    if (N <= 32) {
        p.TN = static_cast<int>(N);
        p.TM = kTileElems / p.TN / 64 * 64;
    } else if (M <= 32) {
        p.TM = static_cast<int>(M);
        p.TN = kTileElems / p.TM / 64 * 64;
    } else {
        p.TM = 64;
        p.TN = 64;
    }
    p.S = p.TM | 1;
    p.tiles_m = ceil_div(M, p.TM);
    p.tiles_n = ceil_div(N, p.TN);
    return p;
}

bool al16p(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

template <typename T>
int transpose(const T* in, int64_t batch, int64_t M, int64_t N, T* out, hipStream_t s) {
    const TransposePlan p = transpose_plan(M, N);
    if constexpr (std::is_same<T, float>::value) {
        const bool narrow_n = N <= 32 && M > 32 && M % 4 == 0;
        const bool narrow_m = M <= 32 && N > 32 && N % 4 == 0;
        if ((narrow_n || narrow_m) && al16p(in) && al16p(out)) {
            const int64_t tiles = p.tiles_m * p.tiles_n;
            if (tiles > 0x7fffffff || batch > 65535)
                return fail(FEQ_ERR_UNSUPPORTED, "transpose: %lld tiles x %lld matrices exceeds the grid",
                            static_cast<long long>(tiles), static_cast<long long>(batch));
            const dim3 grid(static_cast<unsigned>(tiles), static_cast<unsigned>(batch));
            if (narrow_n) {
                const int S = p.TM + 4;
                const size_t lds = sizeof(float) * static_cast<size_t>(S) * p.TN;
                FEQ_LAUNCH("k_transpose", k_transpose4<true>, grid, dim3(256), lds, s, in, M, N, p.TM, p.TN,
                           S, div16_magic(static_cast<uint32_t>(N)), p.tiles_n, out);
            } else {
                const size_t lds = sizeof(float) * static_cast<size_t>(p.TM) * p.TN;
                FEQ_LAUNCH("k_transpose", k_transpose4<false>, grid, dim3(256), lds, s, in, M, N, p.TM,
                           p.TN, 0, uint64_t{0}, p.tiles_n, out);
            }
            return FEQ_OK;
        }
    }
    const int64_t tiles = p.tiles_m * p.tiles_n;
    if (tiles > 0x7fffffff || batch > 65535)
        return fail(FEQ_ERR_UNSUPPORTED, "transpose: %lld tiles x %lld matrices exceeds the grid",
                    static_cast<long long>(tiles), static_cast<long long>(batch));
    const size_t lds = sizeof(T) * static_cast<size_t>(p.S) * p.TN;
    auto kern = k_transpose<T>;
    FEQ_LAUNCH("k_transpose", kern, dim3(static_cast<unsigned>(tiles), static_cast<unsigned>(batch)),
               dim3(256), lds, s, in, M, N, p.TM, p.TN, p.S, div16_magic(p.TN),
               div16_magic(p.TM), p.tiles_n, out);
    return FEQ_OK;
}

// ---- column sums ---------------------------------------------------------------
// out[k][j] = sum of in[i][j] over the rows i of chunk k.  A workgroup covers a
// tile of TPR * VEC columns (TPR threads across, VEC columns per thread) and one
// chunk of rows; its 256 / TPR thread rows take interleaved input rows, and
// their partials are combined by a fixed tree in LDS.
template <typename T, int VEC>
__global__ void __launch_bounds__(256)
k_colsum(const T* __restrict__ in, int64_t rows, int64_t cols, int tpr_log2, int64_t rows_per_chunk,
         T* __restrict__ out) {
    __shared__ T s[256 * VEC];
    const int tpr = 1 << tpr_log2;
    const int rpp = 256 >> tpr_log2;
    const int lc = threadIdx.x & (tpr - 1);
    const int rg = threadIdx.x >> tpr_log2;
    const int64_t col = static_cast<int64_t>(blockIdx.x) * tpr * VEC + lc * VEC;
    const int64_t r0 = static_cast<int64_t>(blockIdx.y) * rows_per_chunk;
    const int64_t r1 = r0 + rows_per_chunk < rows ? r0 + rows_per_chunk : rows;
    T acc[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) acc[v] = T(0);
    if (col + VEC <= cols) {
        for (int64_t r = r0 + rg; r < r1; r += rpp) {
            const T* p = in + r * cols + col;
            if constexpr (VEC == 4) {
                const float4 q = *reinterpret_cast<const float4*>(p);
                acc[0] += q.x; acc[1] += q.y; acc[2] += q.z; acc[3] += q.w;
            } else if constexpr (VEC == 2) {
                const double2 q = *reinterpret_cast<const double2*>(p);
                acc[0] += q.x; acc[1] += q.y;
            } else {
                acc[0] += p[0];
            }
        }
    } else {
        for (int64_t r = r0 + rg; r < r1; r += rpp)
#pragma unroll
            for (int v = 0; v < VEC; ++v)
                if (col + v < cols) acc[v] += in[r * cols + col + v];
    }
    const int width = tpr * VEC;
#pragma unroll
    for (int v = 0; v < VEC; ++v) s[rg * width + lc * VEC + v] = acc[v];
    __syncthreads();
    for (int half = rpp >> 1; half > 0; half >>= 1) {
        if (rg < half)
#pragma unroll
            for (int v = 0; v < VEC; ++v)
                s[rg * width + lc * VEC + v] += s[(rg + half) * width + lc * VEC + v];
        __syncthreads();
    }
    if (rg == 0)
#pragma unroll
        for (int v = 0; v < VEC; ++v)
            if (col + v < cols) out[static_cast<int64_t>(blockIdx.y) * cols + col + v] = s[lc * VEC + v];
}

constexpr int64_t kColsumGroups = 2048;   // target workgroups per pass

struct ColsumPass {
    int64_t rows, chunks, rows_per_chunk;
    int vec, tpr_log2;
    int64_t ctiles;
};

ColsumPass colsum_pass(int64_t rows, int64_t cols, int vec) {
    ColsumPass p{};
    p.rows = rows;
    p.vec = vec;
    const int64_t lanes = ceil_div(cols, vec);
    int t = 0;
    while ((int64_t{1} << t) < lanes && t < 6) ++t;
    p.tpr_log2 = t;
    p.ctiles = ceil_div(cols, (int64_t{1} << t) * vec);
    const int64_t rpp = 256 >> t;
    int64_t chunks = ceil_div(kColsumGroups, p.ctiles);
    const int64_t most = ceil_div(rows, rpp * 8);     // at least eight rows per thread
    if (chunks > most) chunks = most;
    // few rows (the chunked weight gradients' partial products): one pass, so
    // one launch, however few workgroups it has
    if (chunks < 1 || rows <= 256) chunks = 1;
    p.rows_per_chunk = ceil_div(rows, chunks);
    p.chunks = p.rows_per_chunk > 0 ? ceil_div(rows, p.rows_per_chunk) : 1;
    return p;
}

// The passes of one column sum: the first reads the input with vector width
// first_vec, the later ones read the previous pass's partial table (256-byte
// aligned) with later_vec; the last pass writes the output.
template <typename Fn>
void colsum_passes(int64_t rows, int64_t cols, int first_vec, int later_vec, Fn fn) {
    int v = first_vec;
    for (int k = 0;; ++k) {
        const ColsumPass p = colsum_pass(rows, cols, v);
        fn(k, p);
        if (p.chunks == 1) return;
        rows = p.chunks;
        v = later_vec;
    }
}

// Bytes of the two partial tables (even passes, odd passes), the larger of
// the two first-pass vector widths, so the layout does not depend on alignment.
template <typename T>
void colsum_tables(int64_t rows, int64_t cols, size_t* even, size_t* odd) {
    constexpr int kVec = sizeof(T) == 4 ? 4 : 2;
    const int later = cols % kVec == 0 ? kVec : 1;
    *even = *odd = 0;
    for (int first : {1, later})
        colsum_passes(rows, cols, first, later, [&](int k, const ColsumPass& p) {
            if (p.chunks == 1) return;
            size_t& slot = (k & 1) ? *odd : *even;
            const size_t need = align_up(static_cast<size_t>(p.chunks * cols) * sizeof(T), 256);
            if (need > slot) slot = need;
        });
}

template <typename T>
size_t colsum_ws_bytes(int64_t rows, int64_t cols) {
    size_t even, odd;
    colsum_tables<T>(rows, cols, &even, &odd);
    return even + odd;
}

template <typename T, int V>
int colsum_launch(const ColsumPass& p, const T* in, int64_t cols, T* out, hipStream_t s) {
    if (p.ctiles > 0x7fffffff || p.chunks > 65535)
        return fail(FEQ_ERR_UNSUPPORTED, "column sums: grid too large");
    auto kern = k_colsum<T, V>;
    FEQ_LAUNCH("k_colsum", kern, dim3(static_cast<unsigned>(p.ctiles), static_cast<unsigned>(p.chunks)),
               dim3(256), 0, s, in, p.rows, cols, p.tpr_log2, p.rows_per_chunk, out);
    return FEQ_OK;
}

template <typename T>
int column_sums(const T* in, int64_t rows, int64_t cols, T* out, void* ws, size_t ws_bytes,
                hipStream_t s) {
    constexpr int kVec = sizeof(T) == 4 ? 4 : 2;
    size_t even, odd;
    colsum_tables<T>(rows, cols, &even, &odd);
    if (even + odd > 0 && (!ws || ws_bytes < even + odd))
        return fail(FEQ_ERR_WORKSPACE, "column-sum workspace too small");
    const int later = cols % kVec == 0 ? kVec : 1;
    const int first = later == kVec && (reinterpret_cast<uintptr_t>(in) & 15u) == 0 ? kVec : 1;
    unsigned char* w = static_cast<unsigned char*>(ws);
    const T* src = in;
    int rc = FEQ_OK;
    colsum_passes(rows, cols, first, later, [&](int k, const ColsumPass& p) {
        if (rc) return;
        T* dst = p.chunks == 1 ? out : reinterpret_cast<T*>(w + ((k & 1) ? even : 0));
        rc = p.vec == kVec ? colsum_launch<T, kVec>(p, src, cols, dst, s)
                           : colsum_launch<T, 1>(p, src, cols, dst, s);
        src = dst;
    });
    return rc;
}

// ---- dot products accumulated in float64 -----------------------------------------
constexpr int kDotGroups = 1024;

__device__ inline double wave_sum_d(double v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

__global__ void __launch_bounds__(256)
k_dot_f64(const float* __restrict__ a, const float* __restrict__ b, int64_t n,
          double* __restrict__ part, const float* __restrict__ scale, float* __restrict__ sa) {
    // sa (may be NULL): sa[i] = scale[0] a[i], written in the same pass
    __shared__ double s[4];
    double acc = 0.0;
    const float sc = sa ? scale[0] : 0.0f;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
    const int64_t t0 = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b) |
          reinterpret_cast<uintptr_t>(sa)) & 15u) == 0) {
        const float4* a4 = reinterpret_cast<const float4*>(a);
        const float4* b4 = reinterpret_cast<const float4*>(b);
        const int64_t n4 = n / 4;
        for (int64_t i = t0; i < n4; i += stride) {
            const float4 x = a4[i], y = b4[i];
            acc += (static_cast<double>(x.x) * y.x + static_cast<double>(x.y) * y.y) +
                   (static_cast<double>(x.z) * y.z + static_cast<double>(x.w) * y.w);
            if (sa) reinterpret_cast<float4*>(sa)[i] = make_float4(sc * x.x, sc * x.y, sc * x.z, sc * x.w);
        }
        for (int64_t i = 4 * n4 + t0; i < n; i += stride) {
            acc += static_cast<double>(a[i]) * b[i];
            if (sa) sa[i] = sc * a[i];
        }
    } else {
        for (int64_t i = t0; i < n; i += stride) {
            acc += static_cast<double>(a[i]) * b[i];
            if (sa) sa[i] = sc * a[i];
        }
    }
    acc = wave_sum_d(acc);
    if ((threadIdx.x & 63) == 0) s[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) part[blockIdx.x] = (s[0] + s[1]) + (s[2] + s[3]);
}

// out = x + scale[0] y (a residual connection with a scalar layer scale);
// x NULL: out = scale[0] y.
template <bool X>
__global__ void __launch_bounds__(256)
k_scale_add(const float* __restrict__ x, const float* __restrict__ y, const float* __restrict__ scale,
            int64_t n, float* __restrict__ out) {
    const float sc = scale[0];
    const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
    const int64_t t0 = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y) |
          reinterpret_cast<uintptr_t>(out)) & 15u) == 0) {
        const int64_t n4 = n / 4;
        for (int64_t i = t0; i < n4; i += stride) {
            const float4 b = reinterpret_cast<const float4*>(y)[i];
            float4 r = make_float4(sc * b.x, sc * b.y, sc * b.z, sc * b.w);
            if constexpr (X) {
                const float4 a = reinterpret_cast<const float4*>(x)[i];
                r = make_float4(a.x + r.x, a.y + r.y, a.z + r.z, a.w + r.w);
            }
            reinterpret_cast<float4*>(out)[i] = r;
        }
        for (int64_t i = 4 * n4 + t0; i < n; i += stride) out[i] = (X ? x[i] : 0.0f) + sc * y[i];
    } else {
        for (int64_t i = t0; i < n; i += stride) out[i] = (X ? x[i] : 0.0f) + sc * y[i];
    }
}

// out = tables[0] + tables[1] + ... (in that order) over n floats: the
// gradients of a tensor that several consumers read, summed in one pass.
constexpr int kMaxTables = 16;
struct Tables {
    const float* p[kMaxTables];
};

__global__ void __launch_bounds__(256)
k_sum_tables(Tables T, int nt, int64_t n, int vec, float* __restrict__ out) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
    const int64_t t0 = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (vec) {
        const int64_t n4 = n / 4;
        for (int64_t i = t0; i < n4; i += stride) {
            float4 a = reinterpret_cast<const float4*>(T.p[0])[i];
            for (int j = 1; j < nt; ++j) {
                const float4 b = reinterpret_cast<const float4*>(T.p[j])[i];
                a = make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
            }
            reinterpret_cast<float4*>(out)[i] = a;
        }
        for (int64_t i = 4 * n4 + t0; i < n; i += stride) {
            float a = T.p[0][i];
            for (int j = 1; j < nt; ++j) a += T.p[j][i];
            out[i] = a;
        }
    } else {
        for (int64_t i = t0; i < n; i += stride) {
            float a = T.p[0][i];
            for (int j = 1; j < nt; ++j) a += T.p[j][i];
            out[i] = a;
        }
    }
}

unsigned stream_grid(int64_t n) {
    const int64_t g = (n / 4 + 255) / 256;
    return static_cast<unsigned>(g < 4096 ? (g < 1 ? 1 : g) : 4096);
}

// out[0] = (float) sum of part[0..groups) by one workgroup in a fixed order.
__global__ void __launch_bounds__(256)
k_dot_finish(const double* __restrict__ part, int groups, float* __restrict__ out) {
    __shared__ double s[4];
    double acc = 0.0;
    for (int i = threadIdx.x; i < groups; i += 256) acc += part[i];
    acc = wave_sum_d(acc);
    if ((threadIdx.x & 63) == 0) s[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) out[0] = static_cast<float>((s[0] + s[1]) + (s[2] + s[3]));
}

}  // namespace
}  // namespace feq

using namespace feq;

extern "C" int feq_transpose(const void* in, int64_t batch, int64_t rows, int64_t cols,
                             int32_t elem_bytes, void* out, feq_stream_t stream) {
    if (batch < 0 || rows < 0 || cols < 0) return fail(FEQ_ERR_INVALID, "negative size");
    if (batch == 0 || rows == 0 || cols == 0) return FEQ_OK;
    if (!in || !out) return fail(FEQ_ERR_INVALID, "NULL pointer");
    if (in == out) return fail(FEQ_ERR_INVALID, "transpose: in-place is not supported");
    hipStream_t s = stream_of(stream);
    switch (elem_bytes) {
        case 2: return transpose(static_cast<const uint16_t*>(in), batch, rows, cols,
                                 static_cast<uint16_t*>(out), s);
        case 4: return transpose(static_cast<const float*>(in), batch, rows, cols,
                                 static_cast<float*>(out), s);
        case 8: return transpose(static_cast<const double*>(in), batch, rows, cols,
                                 static_cast<double*>(out), s);
        default: return fail(FEQ_ERR_UNSUPPORTED, "transpose: element size %d", elem_bytes);
    }
}

extern "C" size_t feq_column_sums_workspace(int64_t rows, int64_t cols, int32_t elem_bytes) {
    if (rows <= 0 || cols <= 0) return 0;
    return elem_bytes == 8 ? colsum_ws_bytes<double>(rows, cols) : colsum_ws_bytes<float>(rows, cols);
}

extern "C" int feq_column_sums(const void* in, int64_t rows, int64_t cols, int32_t elem_bytes,
                               void* out, void* ws, size_t ws_bytes, feq_stream_t stream) {
    if (rows < 0 || cols < 0) return fail(FEQ_ERR_INVALID, "negative size");
    if (cols == 0) return FEQ_OK;
    if (!out || (rows > 0 && !in)) return fail(FEQ_ERR_INVALID, "NULL pointer");
    hipStream_t s = stream_of(stream);
    switch (elem_bytes) {
        case 4: return column_sums(static_cast<const float*>(in), rows, cols,
                                   static_cast<float*>(out), ws, ws_bytes, s);
        case 8: return column_sums(static_cast<const double*>(in), rows, cols,
                                   static_cast<double*>(out), ws, ws_bytes, s);
        default: return fail(FEQ_ERR_UNSUPPORTED, "column sums: element size %d", elem_bytes);
    }
}

extern "C" size_t feq_dot_f64_workspace(void) { return sizeof(double) * kDotGroups; }

extern "C" int feq_dot_f64(const float* a, const float* b, int64_t n, float* out, void* ws,
                           size_t ws_bytes, feq_stream_t stream) {
    if (n < 0) return fail(FEQ_ERR_INVALID, "negative length");
    if (!out || (n > 0 && (!a || !b))) return fail(FEQ_ERR_INVALID, "NULL pointer");
    if (!ws || ws_bytes < feq_dot_f64_workspace())
        return fail(FEQ_ERR_WORKSPACE, "dot workspace too small");
    hipStream_t s = stream_of(stream);
    double* part = static_cast<double*>(ws);
    FEQ_LAUNCH("k_dot_f64", k_dot_f64, dim3(kDotGroups), dim3(256), 0, s, a, b, n, part,
               static_cast<const float*>(nullptr), static_cast<float*>(nullptr));
    FEQ_LAUNCH("k_dot_finish", k_dot_finish, dim3(1), dim3(256), 0, s, part, kDotGroups, out);
    return FEQ_OK;
}

extern "C" int feq_scale_add(const float* x, const float* y, const float* scale, int64_t n, float* out,
                             feq_stream_t stream) {
    if (n < 0) return fail(FEQ_ERR_INVALID, "negative length");
    if (n == 0) return FEQ_OK;
    if (!x || !y || !scale || !out) return fail(FEQ_ERR_INVALID, "NULL pointer");
    FEQ_LAUNCH("k_scale_add", k_scale_add<true>, dim3(stream_grid(n)), dim3(256), 0, stream_of(stream), x, y,
               scale, n, out);
    return FEQ_OK;
}

extern "C" int feq_sum_tables(const float* const* tables, int32_t num_tables, int64_t n, float* out,
                              feq_stream_t stream) {
    if (n < 0 || num_tables < 1 || num_tables > kMaxTables)
        return fail(FEQ_ERR_INVALID, "sum of tables: 1 to %d tables of n >= 0 floats", kMaxTables);
    if (n == 0) return FEQ_OK;
    if (!tables || !out) return fail(FEQ_ERR_INVALID, "NULL pointer");
    Tables T{};
    bool vec = (reinterpret_cast<uintptr_t>(out) & 15u) == 0;
    for (int j = 0; j < num_tables; ++j) {
        if (!tables[j]) return fail(FEQ_ERR_INVALID, "NULL table");
        T.p[j] = tables[j];
        vec = vec && (reinterpret_cast<uintptr_t>(tables[j]) & 15u) == 0;
    }
    FEQ_LAUNCH("k_sum_tables", k_sum_tables, dim3(stream_grid(n)), dim3(256), 0, stream_of(stream), T,
               int(num_tables), n, int(vec), out);
    return FEQ_OK;
}

extern "C" int feq_scale_add_bwd(const float* grad_out, const float* y, const float* scale, int64_t n,
                                 float* grad_y, float* grad_scale, void* ws, size_t ws_bytes,
                                 feq_stream_t stream) {
    if (n < 0) return fail(FEQ_ERR_INVALID, "negative length");
    if (!grad_scale && !grad_y) return FEQ_OK;
    if (!scale || (n > 0 && (!grad_out || !y))) return fail(FEQ_ERR_INVALID, "NULL pointer");
    hipStream_t s = stream_of(stream);
    if (!grad_scale) {   // grad_y alone: the scaled copy
        if (n == 0) return FEQ_OK;
        FEQ_LAUNCH("k_scale_add", k_scale_add<false>, dim3(stream_grid(n)), dim3(256), 0, s,
                   static_cast<const float*>(nullptr), grad_out, scale, n, grad_y);
        return FEQ_OK;
    }
    if (!ws || ws_bytes < feq_dot_f64_workspace()) return fail(FEQ_ERR_WORKSPACE, "dot workspace too small");
    double* part = static_cast<double*>(ws);
    FEQ_LAUNCH("k_dot_f64", k_dot_f64, dim3(kDotGroups), dim3(256), 0, s, grad_out, y, n, part, scale, grad_y);
    FEQ_LAUNCH("k_dot_finish", k_dot_finish, dim3(1), dim3(256), 0, s, part, kDotGroups, grad_scale);
    return FEQ_OK;
}

// Graph-side kernels: CSR grouping of the edges by destination (or source),
// row gathers and segmented sums.  The attention kernels are in attention.hip.
//
// All edge->node reductions walk each node's edge segment in CSR order, one
// workgroup per node, so results are deterministic and need no atomics
// (the reference scatters with atomics: pooling.py:21-30, attention.py:124-141).
#include "feq_internal.h"

#include <rocprim/device/device_radix_sort.hpp>

namespace feq {
namespace {

constexpr int kThreads = 256;

__global__ void k_csr_keys(const int64_t* __restrict__ dst, int64_t E, int64_t N,
                           int32_t* __restrict__ keys, int32_t* __restrict__ vals) {
    const int64_t e = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
    if (e >= E) return;
    const int64_t d = dst[e];
    // edges whose destination is out of range are sorted past the last node
    keys[e] = (d >= 0 && d < N) ? static_cast<int32_t>(d) : static_cast<int32_t>(N);
    vals[e] = static_cast<int32_t>(e);
}

__global__ void k_csr_offsets(const int32_t* __restrict__ keys, int64_t E, int64_t N,
                              int32_t* __restrict__ offsets) {
    const int64_t n = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
    if (n > N) return;
    // first index with key >= n
    int64_t lo = 0, hi = E;
    while (lo < hi) {
        const int64_t mid = (lo + hi) >> 1;
        if (keys[mid] < n) lo = mid + 1; else hi = mid;
    }
    offsets[n] = static_cast<int32_t>(lo);
}

__global__ void __launch_bounds__(kThreads)
k_segment_sum(const float* __restrict__ x, int64_t row, const int32_t* __restrict__ perm,
              const int32_t* __restrict__ offsets, float* __restrict__ out) {
    const int64_t n = blockIdx.x;
    const int b = offsets[n], e_end = offsets[n + 1];
    for (int64_t c = threadIdx.x; c < row; c += kThreads) {
        float acc = 0.0f;
        for (int i = b; i < e_end; ++i) acc += x[static_cast<int64_t>(perm[i]) * row + c];
        out[n * row + c] = acc;
    }
}

// Short rows (coordinates: 3 floats), one node per thread, the same
// summation order.
constexpr int64_t kShortSegRow = 16;
__global__ void __launch_bounds__(256)
k_segment_sum_short(const float* __restrict__ x, int64_t row, const int32_t* __restrict__ perm,
                    const int32_t* __restrict__ offsets, int64_t N, float* __restrict__ out) {
    const int64_t n = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (n >= N) return;
    const int b = offsets[n], e_end = offsets[n + 1];
    float acc[kShortSegRow];
#pragma unroll
    for (int c = 0; c < kShortSegRow; ++c) acc[c] = 0.0f;
    for (int i = b; i < e_end; ++i) {
        const float* xr = x + static_cast<int64_t>(perm[i]) * row;
#pragma unroll
        for (int c = 0; c < kShortSegRow; ++c)
            if (c < row) acc[c] += xr[c];
    }
#pragma unroll
    for (int c = 0; c < kShortSegRow; ++c)
        if (c < row) out[n * row + c] = acc[c];
}

// 16-byte variants for rows of whole float4s (row4 = row / 4): one thread per
// float4 of the output (gather) or per float4 column of a node (segment sum).
__global__ void k_segment_sum4(const float4* __restrict__ x, int64_t row4,
                               const int32_t* __restrict__ perm, const int32_t* __restrict__ offsets,
                               float4* __restrict__ out) {
    const int64_t n = blockIdx.y;
    const int64_t c = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
    if (c >= row4) return;
    const int b = offsets[n], e_end = offsets[n + 1];
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    // loads of eight edges at a time in flight, summed in segment order
    constexpr int U = 8;
    int i = b;
    for (; i + U <= e_end; i += U) {
        float4 v[U];
#pragma unroll
        for (int j = 0; j < U; ++j) v[j] = x[static_cast<int64_t>(perm[i + j]) * row4 + c];
#pragma unroll
        for (int j = 0; j < U; ++j) {
            acc.x += v[j].x;
            acc.y += v[j].y;
            acc.z += v[j].z;
            acc.w += v[j].w;
        }
    }
    for (; i < e_end; ++i) {
        const float4 v = x[static_cast<int64_t>(perm[i]) * row4 + c];
        acc.x += v.x;
        acc.y += v.y;
        acc.z += v.z;
        acc.w += v.w;
    }
    out[n * row4 + c] = acc;
}

// One row per wave (the row index is wave-uniform), lanes across its float4s.
__global__ void __launch_bounds__(256)
k_gather_rows4(const float4* __restrict__ src, int64_t row4, const int64_t* __restrict__ idx,
               int64_t nrows, int64_t nsrc, float4* __restrict__ out) {
    const int64_t r = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (r >= nrows) return;
    const int lane = threadIdx.x & 63;
    const int64_t s = idx[r];
    const bool ok = s >= 0 && s < nsrc;
    const float4* in = src + (ok ? s : 0) * row4;
    float4* o = out + r * row4;
    for (int64_t c = lane; c < row4; c += 64) o[c] = ok ? in[c] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
}

__global__ void k_gather_rows(const float* __restrict__ src, int64_t row,
                              const int64_t* __restrict__ idx, int64_t nrows, int64_t nsrc,
                              float* __restrict__ out) {
    const int64_t r = blockIdx.x;
    const int64_t s = idx[r];
    const bool ok = s >= 0 && s < nsrc;
    for (int64_t c = threadIdx.x; c < row; c += blockDim.x)
        out[r * row + c] = ok ? src[s * row + c] : 0.0f;
}

// Short rows (coordinates: 3 floats), one row per thread.
constexpr int64_t kShortRow = 16;
__global__ void __launch_bounds__(256)
k_gather_rows_short(const float* __restrict__ src, int64_t row, const int64_t* __restrict__ idx, int64_t nrows,
                    int64_t nsrc, float* __restrict__ out) {
    const int64_t r = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (r >= nrows) return;
    const int64_t s = idx[r];
    const bool ok = s >= 0 && s < nsrc;
    for (int64_t c = 0; c < row; ++c) out[r * row + c] = ok ? src[s * row + c] : 0.0f;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace feq

using namespace feq;

// The stable key sort is rocPRIM's radix sort held to its block-sort + merge
// form at every size.  Above 2^20 items rocPRIM would otherwise switch to its
// onesweep form, which clears its look-back states with hipMemsetAsync and
// resets a block-id counter from the host on every call; recorded into a HIP
// graph, those nodes are not redone correctly on replays, the stale states and
// block ids give scatter positions out of range and the replay faults.  The
// merge form launches kernels only, so a captured CSR build replays like the
// eager one.  Both forms are stable.
using CsrSortConfig = rocprim::radix_sort_config<rocprim::default_config, rocprim::default_config,
                                                 rocprim::default_config, size_t(1) << 31>;

static size_t radix_temp_bytes(int64_t E) {
    size_t bytes = 0;
    (void)rocprim::radix_sort_pairs<CsrSortConfig>(nullptr, bytes, static_cast<const int32_t*>(nullptr),
                                                   static_cast<int32_t*>(nullptr),
                                                   static_cast<const int32_t*>(nullptr),
                                                   static_cast<int32_t*>(nullptr), static_cast<int>(E), 0, 32);
    return bytes;
}

extern "C" size_t feq_csr_workspace(int64_t E, int64_t) {
    if (E <= 0) return 0;
    // keys in, keys out, values in, radix temp
    return 3 * align_up(sizeof(int32_t) * E, 256) + align_up(radix_temp_bytes(E), 256) + 256;
}

extern "C" int feq_csr_by_dst(const int64_t* dst, int64_t E, int64_t N, int32_t* perm,
                              int32_t* offsets, void* ws, size_t ws_bytes, feq_stream_t stream) {
    if (E < 0 || N < 1) return fail(FEQ_ERR_INVALID, "invalid graph sizes");
    if (E >= 0x7fffffffLL || N >= 0x7fffffffLL)
        return fail(FEQ_ERR_UNSUPPORTED, "graphs above 2^31-1 edges or nodes");
    if (!offsets) return fail(FEQ_ERR_INVALID, "NULL offsets");
    hipStream_t s = stream_of(stream);
    if (E == 0) {
        FEQ_LAUNCH("k_csr_offsets", k_csr_offsets, dim3(ceil_div(N + 1, 256)), dim3(256), 0, s,
                           static_cast<const int32_t*>(nullptr), int64_t(0), N, offsets);
        return FEQ_OK;
    }
    if (!dst || !perm) return fail(FEQ_ERR_INVALID, "NULL pointer");
    if (!ws || ws_bytes < feq_csr_workspace(E, N))
        return fail(FEQ_ERR_WORKSPACE, "CSR workspace too small");
    Carver cv(ws);
    int32_t* keys_in = cv.take<int32_t>(E);
    int32_t* keys_out = cv.take<int32_t>(E);
    int32_t* vals_in = cv.take<int32_t>(E);
    size_t tb = radix_temp_bytes(E);
    void* temp = cv.take<char>(tb);
    FEQ_LAUNCH("k_csr_keys", k_csr_keys, dim3(ceil_div(E, 256)), dim3(256), 0, s, dst, E, N, keys_in,
                       vals_in);
    int end_bit = 1;
    while ((int64_t(1) << end_bit) <= N) ++end_bit;  // keys lie in [0, N]
    FEQ_HIP(rocprim::radix_sort_pairs<CsrSortConfig>(temp, tb, keys_in, keys_out, vals_in, perm,
                                                     static_cast<int>(E), 0, end_bit, s));
    FEQ_LAUNCH("k_csr_offsets", k_csr_offsets, dim3(ceil_div(N + 1, 256)), dim3(256), 0, s, keys_out, E, N,
                       offsets);
    return FEQ_OK;
}

extern "C" int feq_segment_sum(const float* x, int64_t row, const int32_t* perm,
                               const int32_t* offsets, int64_t N, float* out,
                               feq_stream_t stream) {
    if (row < 0 || N < 0) return fail(FEQ_ERR_INVALID, "invalid sizes");
    if (N == 0 || row == 0) return FEQ_OK;
    if (!offsets || !out) return fail(FEQ_ERR_INVALID, "NULL pointer");
    if (row % 4 == 0 && aligned16(x) && aligned16(out)) {
        const int64_t row4 = row / 4;
        const unsigned bx = static_cast<unsigned>(ceil_div(row4, 64));
        FEQ_LAUNCH("k_segment_sum", k_segment_sum4, dim3(bx, static_cast<unsigned>(N)), dim3(64), 0,
                   stream_of(stream), reinterpret_cast<const float4*>(x), row4, perm, offsets,
                   reinterpret_cast<float4*>(out));
        return FEQ_OK;
    }
    if (row <= kShortSegRow) {
        FEQ_LAUNCH("k_segment_sum", k_segment_sum_short, dim3(static_cast<unsigned>(ceil_div(N, 256))), dim3(256),
                   0, stream_of(stream), x, row, perm, offsets, N, out);
        return FEQ_OK;
    }
    FEQ_LAUNCH("k_segment_sum", k_segment_sum, dim3(N), dim3(kThreads), 0, stream_of(stream), x, row, perm,
                       offsets, out);
    return FEQ_OK;
}

extern "C" int feq_gather_rows(const float* src, int64_t nsrc, int64_t row, const int64_t* idx,
                               int64_t nrows, float* out, feq_stream_t stream) {
    if (row < 0 || nrows < 0 || nsrc < 0) return fail(FEQ_ERR_INVALID, "invalid sizes");
    if (nrows == 0 || row == 0) return FEQ_OK;
    if (!src || !idx || !out) return fail(FEQ_ERR_INVALID, "NULL pointer");
    if (row % 4 == 0 && aligned16(src) && aligned16(out)) {
        FEQ_LAUNCH("k_gather_rows", k_gather_rows4, dim3(static_cast<unsigned>(ceil_div(nrows, 4))),
                   dim3(256), 0, stream_of(stream), reinterpret_cast<const float4*>(src), row / 4,
                   idx, nrows, nsrc, reinterpret_cast<float4*>(out));
        return FEQ_OK;
    }
    if (row <= kShortRow) {
        FEQ_LAUNCH("k_gather_rows", k_gather_rows_short, dim3(static_cast<unsigned>(ceil_div(nrows, 256))),
                   dim3(256), 0, stream_of(stream), src, row, idx, nrows, nsrc, out);
        return FEQ_OK;
    }
    FEQ_LAUNCH("k_gather_rows", k_gather_rows, dim3(nrows), dim3(row < 256 ? 64 : 256), 0,
                       stream_of(stream), src, row, idx, nrows, nsrc, out);
    return FEQ_OK;
}

// ---- sum of squares (the benchmarks' training loss sum(y^2)) -----------------
// A fixed grid of kSsqGroups workgroups each sums a contiguous share of y^2 into
// one partial; the partials are summed in a fixed order.  Deterministic, and
// no memset: safe to record into a HIP graph.
namespace feq {
namespace {
constexpr int kSsqGroups = 1024;

__device__ inline float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ inline float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ inline int64_t ceil_div_i(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Sum of y^2 of float32 (BF16 = false) or bfloat16 (BF16 = true) values, each
// squared and summed in float32: 16-byte loads (4 floats or 8 bf16) when y is
// aligned.
template <bool BF16>
__global__ void __launch_bounds__(256)
k_sum_squares(const void* __restrict__ yv, int64_t n, float* __restrict__ part) {
    __shared__ float s[4];
    constexpr int PER = BF16 ? 8 : 4;     // values per 16-byte load
    float acc = 0.0f;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
    const int64_t t0 = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    auto sq = [](uint4 v) {
        if constexpr (BF16) {
            float a = 0.0f;
            const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float lo = bf16_lo(w[j]), hi = bf16_hi(w[j]);
                a += lo * lo + hi * hi;
            }
            return a;
        } else {
            const float a = __uint_as_float(v.x), b = __uint_as_float(v.y);
            const float c = __uint_as_float(v.z), d = __uint_as_float(v.w);
            return a * a + b * b + c * c + d * d;
        }
    };
    auto scalar = [&](int64_t i) {
        if constexpr (BF16) {
            const uint16_t h = static_cast<const uint16_t*>(yv)[i];
            const float f = __uint_as_float(static_cast<uint32_t>(h) << 16);
            return f * f;
        } else {
            const float f = static_cast<const float*>(yv)[i];
            return f * f;
        }
    };
    int64_t tail0 = 0;
    if ((reinterpret_cast<uintptr_t>(yv) & 15u) == 0) {
        // each workgroup walks a contiguous chunk of whole 1024-load steps: eight
        // (then four) coalesced loads in flight per thread, streamed past the
        // caches, four partial sums combined in a fixed order
        const uint4* y4 = static_cast<const uint4*>(yv);
        const int64_t n4 = n / PER;
        const int64_t steps = ceil_div_i(n4, 1024);
        const int64_t per_wg = ceil_div_i(steps, gridDim.x);
        const int64_t b0 = static_cast<int64_t>(blockIdx.x) * per_wg * 1024;
        const int64_t b1 = b0 + per_wg * 1024 < n4 ? b0 + per_wg * 1024 : n4;
        float a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
        int64_t i = b0 + threadIdx.x;
        for (; i + 1792 < b1; i += 2048) {
            typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
            const u32x4* yn = reinterpret_cast<const u32x4*>(y4 + i);
            uint4 v[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const u32x4 w = __builtin_nontemporal_load(yn + 256 * k);
                v[k] = make_uint4(w.x, w.y, w.z, w.w);
            }
            acc += sq(v[0]) + sq(v[4]);
            a1 += sq(v[1]) + sq(v[5]);
            a2 += sq(v[2]) + sq(v[6]);
            a3 += sq(v[3]) + sq(v[7]);
        }
        for (; i + 768 < b1; i += 1024) {
            const uint4 v0 = y4[i], v1 = y4[i + 256], v2 = y4[i + 512], v3 = y4[i + 768];
            acc += sq(v0);
            a1 += sq(v1);
            a2 += sq(v2);
            a3 += sq(v3);
        }
        for (; i < b1; i += 256) acc += sq(y4[i]);
        acc = (acc + a1) + (a2 + a3);
        tail0 = PER * n4;
    }
    for (int64_t i = tail0 + t0; i < n; i += stride) acc += scalar(i);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o);
    if ((threadIdx.x & 63) == 0) s[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) part[blockIdx.x] = (s[0] + s[1]) + (s[2] + s[3]);
}
}  // namespace
}  // namespace feq

extern "C" size_t feq_sum_squares_workspace(void) {
    return sizeof(float) * (kSsqGroups + kSsqGroups / 32) + 256;
}

extern "C" int feq_sum_squares(const float* y, int64_t n, float* out, void* ws, size_t ws_bytes,
                               feq_stream_t stream) {
    if (n < 0) return fail(FEQ_ERR_INVALID, "negative length");
    if (!out || (n > 0 && !y)) return fail(FEQ_ERR_INVALID, "NULL pointer");
    if (!ws || ws_bytes < feq_sum_squares_workspace())
        return fail(FEQ_ERR_WORKSPACE, "sum-of-squares workspace too small");
    hipStream_t s = stream_of(stream);
    float* part = static_cast<float*>(ws);
    auto kern = k_sum_squares<false>;
    FEQ_LAUNCH("k_sum_squares", kern, dim3(kSsqGroups), dim3(256), 0, s, y, n, part);
    return reduce_partials(part, kSsqGroups, 1, out, part + kSsqGroups, s);
}

extern "C" int feq_sum_squares_bf16(const void* y, int64_t n, float* out, void* ws, size_t ws_bytes,
                                    feq_stream_t stream) {
    if (n < 0) return fail(FEQ_ERR_INVALID, "negative length");
    if (!out || (n > 0 && !y)) return fail(FEQ_ERR_INVALID, "NULL pointer");
    if (!ws || ws_bytes < feq_sum_squares_workspace())
        return fail(FEQ_ERR_WORKSPACE, "sum-of-squares workspace too small");
    hipStream_t s = stream_of(stream);
    float* part = static_cast<float*>(ws);
    auto kern = k_sum_squares<true>;
    FEQ_LAUNCH("k_sum_squares", kern, dim3(kSsqGroups), dim3(256), 0, s, y, n, part);
    return reduce_partials(part, kSsqGroups, 1, out, part + kSsqGroups, s);
}

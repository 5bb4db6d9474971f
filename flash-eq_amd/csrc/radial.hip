// The radial network of SeparableRadialNet (radial.py:200-275) evaluated at the
// bin edges: F = head(silu(W2 silu(W1 basis + b1) + b2)) + b3, the trunk's two
// Linear + SiLU layers and the head Linear, for the (num_bins + 1) rows of the
// sinusoidal basis.  The rows are independent, so the forward and the
// per-row part of the backward give each row a workgroup (its activations in
// LDS, weights read through the cache); the weight gradients, sums over the
// rows, are one thread per weight summing the rows in order.  Three launches
// in place of the library's dozen small GEMM, activation and reduction
// launches; deterministic.
#include "feq_internal.h"

namespace feq {
namespace {

constexpr int kRadThreads = 256;

__device__ __forceinline__ float sigm(float z) { return 1.0f / (1.0f + expf(-z)); }
__device__ __forceinline__ float dsilu(float z) {
    const float s = sigm(z);
    return s * (1.0f + z * (1.0f - s));
}

// dst[j] = bias[j] + sum_i W[j][i] src[i], j < J (W row-major J x I); four
// partial sums per thread.
__device__ __forceinline__ void row_dense(const float* __restrict__ W, const float* __restrict__ bias,
                                          const float* src, int I, int J, float* dst) {
    for (int j = threadIdx.x; j < J; j += kRadThreads) {
        const float* w = W + static_cast<int64_t>(j) * I;
        float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
        int i = 0;
#pragma unroll 4
        for (; i + 3 < I; i += 4) {
            a0 += w[i] * src[i];
            a1 += w[i + 1] * src[i + 1];
            a2 += w[i + 2] * src[i + 2];
            a3 += w[i + 3] * src[i + 3];
        }
        for (; i < I; ++i) a0 += w[i] * src[i];
        dst[j] = bias[j] + ((a0 + a1) + (a2 + a3));
    }
}

// One workgroup per row b: the trunk's pre-activations z1, z2 and activations
// h1, h2 into acts[b] = [z1 | z2 | h1 | h2] (4 H floats) and F[b].
__global__ void __launch_bounds__(kRadThreads)
k_radial_fwd(const float* __restrict__ basis, const float* __restrict__ W1, const float* __restrict__ b1,
             const float* __restrict__ W2, const float* __restrict__ b2, const float* __restrict__ W3,
             const float* __restrict__ b3, int I, int H, int O, float* __restrict__ F,
             float* __restrict__ acts) {
    extern __shared__ float lds[];
    float* x = lds;
    float* z = x + I;        // z1 | z2 | h1 | h2
    const int64_t b = blockIdx.x;
    for (int i = threadIdx.x; i < I; i += kRadThreads) x[i] = basis[b * I + i];
    __syncthreads();
    row_dense(W1, b1, x, I, H, z);
    __syncthreads();
    for (int j = threadIdx.x; j < H; j += kRadThreads) z[2 * H + j] = z[j] * sigm(z[j]);
    __syncthreads();
    row_dense(W2, b2, z + 2 * H, H, H, z + H);
    __syncthreads();
    for (int j = threadIdx.x; j < H; j += kRadThreads) z[3 * H + j] = z[H + j] * sigm(z[H + j]);
    __syncthreads();
    row_dense(W3, b3, z + 3 * H, H, O, F + b * O);
    for (int q = threadIdx.x; q < 4 * H; q += kRadThreads) acts[b * 4 * H + q] = z[q];
}

// Backward, per row b: gz2 = (gF[b] W3) silu'(z2), gz1 = (gz2 W2) silu'(z1)
// into grows[b] = [gz2 | gz1].
__global__ void __launch_bounds__(kRadThreads)
k_radial_bwd_rows(const float* __restrict__ W2, const float* __restrict__ W3, const float* __restrict__ gF,
                  const float* __restrict__ acts, int H, int O, float* __restrict__ grows) {
    extern __shared__ float lds[];
    float* gf = lds;          // O
    float* g2 = gf + O;       // H
    const int64_t b = blockIdx.x;
    const float* a = acts + b * 4 * H;
    for (int o = threadIdx.x; o < O; o += kRadThreads) gf[o] = gF[b * O + o];
    __syncthreads();
    for (int i = threadIdx.x; i < H; i += kRadThreads) {
        float s0 = 0.0f, s1 = 0.0f;
        int o = 0;
#pragma unroll 8
        for (; o + 1 < O; o += 2) {
            s0 += gf[o] * W3[static_cast<int64_t>(o) * H + i];
            s1 += gf[o + 1] * W3[static_cast<int64_t>(o + 1) * H + i];
        }
        if (o < O) s0 += gf[o] * W3[static_cast<int64_t>(o) * H + i];
        g2[i] = (s0 + s1) * dsilu(a[H + i]);
    }
    __syncthreads();
    for (int i = threadIdx.x; i < H; i += kRadThreads) {
        float s0 = 0.0f, s1 = 0.0f;
        int j = 0;
#pragma unroll 8
        for (; j + 1 < H; j += 2) {
            s0 += g2[j] * W2[j * H + i];
            s1 += g2[j + 1] * W2[(j + 1) * H + i];
        }
        if (j < H) s0 += g2[j] * W2[j * H + i];
        grows[b * 2 * H + H + i] = (s0 + s1) * dsilu(a[i]);
        grows[b * 2 * H + i] = g2[i];
    }
}

// Weight gradients (rows summed in a fixed order):
//   gW3[o][i] = sum_b gF[b][o] h2[b][i], gb3[o] = sum_b gF[b][o]
//   gW2[j][i] = sum_b gz2[b][j] h1[b][i], gb2[j] = sum_b gz2[b][j]
//   gW1[j][i] = sum_b gz1[b][j] basis[b][i], gb1[j] = sum_b gz1[b][j]
// A workgroup takes 64 weights; its four waves sum interleaved quarters of the
// rows (b = 4 r + wave), combined in wave order through LDS.
constexpr int kRadWeights = 64;

__global__ void __launch_bounds__(kRadThreads)
k_radial_bwd_weights(const float* __restrict__ basis, const float* __restrict__ gF,
                     const float* __restrict__ acts, const float* __restrict__ grows, int B, int I, int H,
                     int O, float* __restrict__ gW1, float* __restrict__ gb1, float* __restrict__ gW2,
                     float* __restrict__ gb2, float* __restrict__ gW3, float* __restrict__ gb3) {
    __shared__ float part[4][kRadWeights];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t q = static_cast<int64_t>(blockIdx.x) * kRadWeights + lane;
    const int64_t n3 = static_cast<int64_t>(O) * (H + 1), n2 = static_cast<int64_t>(H) * (H + 1);
    const int64_t n1 = static_cast<int64_t>(H) * (I + 1);
    // the weight's left operand (row stride, column) and right operand (row
    // stride, column; -1 for a bias: a plain sum of the left operand)
    const float* L = gF;
    const float* R = basis;
    int64_t ls = 0, rs = 0;
    int lc = 0, rc = -1;
    float* out = nullptr;
    if (q < n3) {
        const int o = static_cast<int>(q / (H + 1)), i = static_cast<int>(q % (H + 1));
        L = gF; ls = O; lc = o;
        R = acts + 3 * H; rs = 4 * H; rc = i < H ? i : -1;
        out = i < H ? gW3 + static_cast<int64_t>(o) * H + i : gb3 + o;
    } else if (q < n3 + n2) {
        const int64_t r = q - n3;
        const int j = static_cast<int>(r / (H + 1)), i = static_cast<int>(r % (H + 1));
        L = grows; ls = 2 * H; lc = j;
        R = acts + 2 * H; rs = 4 * H; rc = i < H ? i : -1;
        out = i < H ? gW2 + static_cast<int64_t>(j) * H + i : gb2 + j;
    } else if (q < n3 + n2 + n1) {
        const int64_t r = q - n3 - n2;
        const int j = static_cast<int>(r / (I + 1)), i = static_cast<int>(r % (I + 1));
        L = grows + H; ls = 2 * H; lc = j;
        R = basis; rs = I; rc = i < I ? i : -1;
        out = i < I ? gW1 + static_cast<int64_t>(j) * I + i : gb1 + j;
    }
    float a = 0.0f;
    if (out) {
        // unrolled: eight rows' loads in flight ahead of the (ordered) sum
        if (rc >= 0) {
#pragma unroll 8
            for (int b = wave; b < B; b += 4) a += L[b * ls + lc] * R[b * rs + rc];
        } else {
#pragma unroll 8
            for (int b = wave; b < B; b += 4) a += L[b * ls + lc];
        }
    }
    part[wave][lane] = a;
    __syncthreads();
    if (wave == 0 && out) *out = (part[0][lane] + part[1][lane]) + (part[2][lane] + part[3][lane]);
}

int radial_check(int B, int I, int H, int O) {
    if (B < 1 || I < 1 || H < 1 || O < 1) return fail(FEQ_ERR_INVALID, "radial network: empty shape");
    if (I > FEQ_RADIAL_MAX_WIDTH || H > FEQ_RADIAL_MAX_WIDTH || O > FEQ_RADIAL_MAX_OUT)
        return fail(FEQ_ERR_UNSUPPORTED, "radial network of width %d / %d and %d outputs exceeds the kernels",
                    I, H, O);
    return FEQ_OK;
}

}  // namespace
}  // namespace feq

using namespace feq;

extern "C" int feq_radial_supported(int32_t rows, int32_t in_dim, int32_t hidden, int32_t out_dim) {
    return rows >= 1 && in_dim >= 1 && hidden >= 1 && out_dim >= 1 && in_dim <= FEQ_RADIAL_MAX_WIDTH &&
           hidden <= FEQ_RADIAL_MAX_WIDTH && out_dim <= FEQ_RADIAL_MAX_OUT;
}

extern "C" size_t feq_radial_workspace(int32_t rows, int32_t hidden) {
    return rows < 1 || hidden < 1 ? 0 : sizeof(float) * 2 * static_cast<size_t>(rows) * hidden;
}

extern "C" int feq_radial_fwd(const float* basis, int32_t rows, int32_t in_dim, int32_t hidden,
                              int32_t out_dim, const float* W1, const float* b1, const float* W2,
                              const float* b2, const float* W3, const float* b3, float* F, float* acts,
                              feq_stream_t stream) {
    if (int rc = radial_check(rows, in_dim, hidden, out_dim)) return rc;
    if (!basis || !W1 || !b1 || !W2 || !b2 || !W3 || !b3 || !F || !acts) return fail(FEQ_ERR_INVALID, "NULL pointer");
    const size_t lds = sizeof(float) * (static_cast<size_t>(in_dim) + 4 * static_cast<size_t>(hidden));
    FEQ_LAUNCH("k_radial_fwd", k_radial_fwd, dim3(static_cast<unsigned>(rows)), dim3(kRadThreads), lds,
               stream_of(stream), basis, W1, b1, W2, b2, W3, b3, in_dim, hidden, out_dim, F, acts);
    return FEQ_OK;
}

extern "C" int feq_radial_bwd(const float* basis, int32_t rows, int32_t in_dim, int32_t hidden,
                              int32_t out_dim, const float* W2, const float* W3, const float* acts,
                              const float* grad_F, float* gW1, float* gb1, float* gW2, float* gb2,
                              float* gW3, float* gb3, void* ws, size_t ws_bytes, feq_stream_t stream) {
    if (int rc = radial_check(rows, in_dim, hidden, out_dim)) return rc;
    if (!basis || !W2 || !W3 || !acts || !grad_F || !gW1 || !gb1 || !gW2 || !gb2 || !gW3 || !gb3)
        return fail(FEQ_ERR_INVALID, "NULL pointer");
    if (!ws || ws_bytes < sizeof(float) * 2 * static_cast<size_t>(rows) * hidden)
        return fail(FEQ_ERR_WORKSPACE, "radial network workspace too small");
    float* grows = static_cast<float*>(ws);
    hipStream_t s = stream_of(stream);
    const size_t lds = sizeof(float) * (static_cast<size_t>(out_dim) + hidden);
    FEQ_LAUNCH("k_radial_bwd", k_radial_bwd_rows, dim3(static_cast<unsigned>(rows)), dim3(kRadThreads), lds, s,
               W2, W3, grad_F, acts, hidden, out_dim, grows);
    const int64_t nw = static_cast<int64_t>(out_dim) * (hidden + 1) + static_cast<int64_t>(hidden) * (hidden + 1) +
                       static_cast<int64_t>(hidden) * (in_dim + 1);
    FEQ_LAUNCH("k_radial_bwd", k_radial_bwd_weights, dim3(static_cast<unsigned>(ceil_div(nw, kRadWeights))),
               dim3(kRadThreads), 0, s, basis, grad_F, acts, grows, rows, in_dim, hidden, out_dim, gW1, gb1, gW2,
               gb2, gW3, gb3);
    return FEQ_OK;
}

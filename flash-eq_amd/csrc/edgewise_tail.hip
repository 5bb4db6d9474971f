// Tail of the fused backward passes, shared by the split-fp16 and fp32-MFMA
// families: the binned radial-function gradient from the per-edge gradient
// dF_e (lo/hi split with the interpolation weights, as the reference's table
// gradient, block_diagonal.cu:990-1036), the distance gradient, and the
// deterministic sums of per-workgroup partials.
#include "feq_internal.h"

#include <algorithm>

namespace feq {
namespace {

constexpr int kThreads = 256;

// l_in + l_out of every weight slot w < wdim of a layout, into fl (LDS).
__device__ void weight_lsum(const feq_layout& L, int* fl) {
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
    __syncthreads();
}

// Binned radial-function gradient of one edge chunk: dF[lo] += (1 - t) dF_e and
// dF[lo + 1] += t dF_e.  Thread t serves the columns c = t % kw (+ kThreads
// multiples when kw > kThreads) of edge stream t / kw; every stream keeps its
// own LDS histogram, so each cell has one writer and a fixed summation order.
// One partial histogram per workgroup.
__global__ void __launch_bounds__(kThreads)
k_ewm_hist(feq_binning B, int kw, int streams, int64_t E, int64_t chunk,
           const float* __restrict__ dist, const float* __restrict__ dFe,
           float* __restrict__ hist_part) {
    extern __shared__ float sh[];
    const int hsz = (B.num_bins + 1) * kw;
    float* sT = sh + static_cast<int64_t>(streams) * hsz;
    int* sLo = reinterpret_cast<int*>(sT + chunk);
    for (int q = threadIdx.x; q < streams * hsz; q += kThreads) sh[q] = 0.0f;
    const int64_t e_begin = blockIdx.x * chunk;
    const int n = static_cast<int>(E - e_begin < chunk ? E - e_begin : chunk);
    for (int q = threadIdx.x; q < n; q += kThreads) {
        const EdgeBin eb = edge_bin(dist[e_begin + q], B);
        sLo[q] = eb.lo;
        sT[q] = eb.t;
    }
    __syncthreads();
    const int per = kw <= kThreads ? kw : kThreads;   // threads per stream
    const int st = threadIdx.x / per;
    if (st < streams) {
        float* h = sh + static_cast<int64_t>(st) * hsz;
        for (int c = threadIdx.x % per; c < kw; c += per)
            for (int q = st; q < n; q += streams) {
                const float v = dFe[(e_begin + q) * kw + c];
                const int lo = sLo[q];
                const float t = sT[q];
                h[lo * kw + c] += (1.0f - t) * v;
                h[(lo + 1) * kw + c] += t * v;
            }
    }
    __syncthreads();
    float* out = hist_part + static_cast<int64_t>(blockIdx.x) * hsz;
    for (int q = threadIdx.x; q < hsz; q += kThreads) {
        float acc = sh[q];
        for (int v = 1; v < streams; ++v) acc += sh[static_cast<int64_t>(v) * hsz + q];
        out[q] = acc;
    }
}

// Distance gradient from dF_e, one thread per edge (sums in slot order):
// dr = dt/dr sum (F[hi] - F[lo]) dF_e + [l > 0 pairs] sigma/(r(r+sigma)) sum (l_i+l_o) F_e dF_e.
__global__ void __launch_bounds__(kThreads)
k_ewm_dr(feq_layout L, feq_binning B, int K, int64_t E, const float* __restrict__ dist,
         const float* __restrict__ F, const float* __restrict__ dFe, float* __restrict__ gdist) {
    extern __shared__ int fl[];   // l_in + l_out per weight slot (wdim entries)
    weight_lsum(L, fl);
    const int64_t e = blockIdx.x * static_cast<int64_t>(kThreads) + threadIdx.x;
    if (e >= E) return;
    const int kw = K * L.wdim;
    const float r = dist[e];
    const EdgeBin eb = edge_bin(r, B);
    const float* flo = F + static_cast<int64_t>(eb.lo) * kw;
    const float* g = dFe + e * kw;
    float st = 0.0f, ss = 0.0f;
    for (int q = 0; q < kw; ++q) {
        const float gv = g[q], lo = flo[q], hi = flo[kw + q];
        st += (hi - lo) * gv;
        ss += static_cast<float>(fl[q % L.wdim]) * lerp_bins(lo, hi, eb.t) * gv;
    }
    const float sigma = B.sh_scale;
    float v = st * eb.dtdr;
    if (L.has_lpos) v += ss * (sigma / (r * (r + sigma)));
    gdist[e] = v;
}

// out[s * n + q] = sum of part[g * n + q] over the groups g of slice s
// (blockIdx.y), in increasing g.
__global__ void k_sum_partials(const float* __restrict__ part, int groups, int per_slice,
                               int64_t n, float* __restrict__ out) {
    const int64_t q = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
    if (q >= n) return;
    const int g0 = blockIdx.y * per_slice;
    const int g1 = g0 + per_slice < groups ? g0 + per_slice : groups;
    float acc = 0.0f;
    for (int g = g0; g < g1; ++g) acc += part[static_cast<int64_t>(g) * n + q];
    out[blockIdx.y * n + q] = acc;
}

constexpr int kSliceGroups = 32;   // partials summed per thread in one pass

size_t reduce_tmp_floats(int groups, int64_t n) {
    return groups > kSliceGroups ? static_cast<size_t>((groups + kSliceGroups - 1) / kSliceGroups) * n
                                 : 0;
}

// Deterministic sum of `groups` partial arrays of n floats: slices of at most
// kSliceGroups partials into tmp, then the slices into out.
int reduce_partials(const float* part, int groups, int64_t n, float* out, float* tmp,
                    hipStream_t s) {
    const unsigned nb = static_cast<unsigned>(ceil_div(n, 256));
    if (groups <= kSliceGroups) {
        FEQ_LAUNCH("k_sum_partials", k_sum_partials, dim3(nb, 1), dim3(256), 0, s, part, groups,
                   groups, n, out);
        return FEQ_OK;
    }
    const int slices = (groups + kSliceGroups - 1) / kSliceGroups;
    FEQ_LAUNCH("k_sum_partials", k_sum_partials, dim3(nb, slices), dim3(256), 0, s, part, groups,
               kSliceGroups, n, tmp);
    FEQ_LAUNCH("k_sum_partials", k_sum_partials, dim3(nb, 1), dim3(256), 0, s, tmp, slices, slices,
               n, out);
    return FEQ_OK;
}

constexpr int64_t kBinChunk = 256;   // edges per histogram workgroup
constexpr size_t kHistLds = 64 * 1024;

// Histogram streams per workgroup (0: the histogram does not fit LDS).
int hist_streams(const feq_binning& B, int kw) {
    const size_t hbytes = 4 * static_cast<size_t>(B.num_bins + 1) * kw;
    const size_t avail = kHistLds - 8 * kBinChunk;
    int st = kw <= kThreads ? kThreads / kw : 1;
    while (st > 0 && st * hbytes > avail) --st;
    return st;
}

size_t hist_lds(const feq_binning& B, int kw, int streams) {
    return 4 * static_cast<size_t>(streams) * (B.num_bins + 1) * kw + 8 * kBinChunk;
}

}  // namespace

bool ew_tail_supported(const feq_binning& B, int kw) { return hist_streams(B, kw) >= 1; }

size_t ew_tail_floats(const feq_binning& B, int kw, int64_t E, int groups, int64_t ncc) {
    const int nchunks = static_cast<int>(ceil_div(E, kBinChunk));
    const int64_t hsz = (B.num_bins + 1) * static_cast<int64_t>(kw);
    const size_t tmp = std::max(reduce_tmp_floats(groups, ncc), reduce_tmp_floats(nchunks, hsz));
    return align_up(static_cast<size_t>(nchunks) * hsz, 64) + align_up(tmp, 64) + 64;
}

int ew_tail(const feq_layout& L, const feq_binning& B, int K, int64_t E, const float* dist,
            const float* F, const float* dFe, const float* dCp, int groups, int64_t ncc, float* gC,
            float* gF, float* gdist, float* tail, hipStream_t s) {
    const int kw = K * L.wdim;
    const int streams = hist_streams(B, kw);
    if (streams < 1) return fail(FEQ_ERR_UNSUPPORTED, "radial-function histogram does not fit LDS");
    const size_t hlds = hist_lds(B, kw, streams);
    const int nchunks = static_cast<int>(ceil_div(E, kBinChunk));
    const int64_t hsz = (B.num_bins + 1) * static_cast<int64_t>(kw);
    float* hp = tail;
    float* tmp = tail + align_up(static_cast<size_t>(nchunks) * hsz, 64);
    if (hlds > 64 * 1024)
        FEQ_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&k_ewm_hist),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(hlds)));
    FEQ_LAUNCH("k_ewm_hist", k_ewm_hist, dim3(nchunks), dim3(kThreads), hlds, s, B, kw, streams,
               E, kBinChunk, dist, dFe, hp);
    if (gdist)
        FEQ_LAUNCH("k_ewm_dr", k_ewm_dr, dim3(ceil_div(E, kThreads)), dim3(kThreads),
                   sizeof(int) * L.wdim, s, L, B, K, E, dist, F, dFe, gdist);
    if (int rc = reduce_partials(dCp, groups, ncc, gC, tmp, s)) return rc;
    return reduce_partials(hp, nchunks, hsz, gF, tmp, s);
}

}  // namespace feq

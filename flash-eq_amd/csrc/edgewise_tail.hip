// Tail of the fused backward passes, shared by the edgewise families: the
// binned radial-function gradient from the per-edge gradient dF_e (lo/hi split
// with the interpolation weights, as the reference's table gradient,
// block_diagonal.cu:990-1036), the distance gradient, and the deterministic
// sums of per-workgroup partials.
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

// Binned radial-function gradient: dF[lo] += (1 - t) dF_e and dF[lo + 1] += t dF_e.
// Two forms.  Narrow rows (a few private histograms fit LDS): every wave owns a private LDS histogram and a contiguous run of edges, and
// adds into it in edge order (plain read-add-write; LDS float atomics are
// several times slower), so every cell's summation order is fixed and the
// result is deterministic.  Lane c serves the columns c, c + 64, ... of an edge.  Edges
// are taken in batches of kHistBatch whose loads are issued together, one batch
// ahead.  One
// partial histogram per workgroup (its waves' histograms summed in wave order).
constexpr int kHistBatch = 16;

// PAIR (even rows, 8-byte aligned): lane c owns the adjacent columns c0 + 2c and
// c0 + 2c + 1 of each 128-column block, one 8-byte load and one 8-byte LDS read
// and write per cell pair.  Otherwise lane c owns the columns c0 + c and c0 + 64 + c.
// Both forms add every cell's edges in edge order with the same operations.
template <bool PAIR>
__global__ void __launch_bounds__(kThreads)
k_ewm_hist(feq_binning B, int kw_row, int cw0, int kw, int64_t E, int64_t per_wave,
           const float* __restrict__ dist, const float* __restrict__ dFe,
           float* __restrict__ hist_part) {
    extern __shared__ __align__(16) float sh[];   // 8-byte cell pairs in the PAIR form
    const int waves = blockDim.x / 64;
    const int hsz = (B.num_bins + 1) * kw;
    for (int q = threadIdx.x; q < waves * hsz; q += blockDim.x) sh[q] = 0.0f;
    __syncthreads();
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    float* h = sh + static_cast<int64_t>(wave) * hsz;
    const int64_t e_begin = (static_cast<int64_t>(blockIdx.x) * waves + wave) * per_wave;
    const int64_t e_end = e_begin + per_wave < E ? e_begin + per_wave : E;
    for (int c0 = 0; c0 < kw; c0 += 128) {
        // columns of the lane's two slots (in-bounds loads: clamped, not added)
        const int ca = PAIR ? c0 + 2 * lane : c0 + lane, cb = PAIR ? ca + 1 : c0 + 64 + lane;
        const bool ina = ca < kw, inb = cb < kw;
        const int la = ina ? ca : (PAIR ? kw - 2 : kw - 1), lb = inb ? cb : kw - 1;
        // Batch of kHistBatch edges from e: lane j < kHistBatch bins edge e + j.
        // The loads are unconditional (rows past the run repeat its last edge and
        // are not added; a batch wholly past it reads the last edge), and the
        // bins are computed only where the batch is added, so nothing waits on a
        // batch's loads before the batch ahead of it is added in: the compiler's
        // in-order load counter then keeps the next batch in flight.
        struct Batch {
            float va[kHistBatch], vb[kHistBatch];
            float r;
        };
        auto load = [&](int64_t e, Batch& b) {
            const int64_t ec = e < e_end ? e : e_end - 1;
            const int nb = static_cast<int>(e_end - ec < kHistBatch ? e_end - ec : kHistBatch);
            const int jl = (lane % kHistBatch) < nb ? lane % kHistBatch : nb - 1;
            b.r = dist[ec + jl];
#pragma unroll
            for (int j = 0; j < kHistBatch; ++j) {
                const float* row = dFe + (ec + (j < nb ? j : nb - 1)) * kw_row + cw0;
                if constexpr (PAIR) {
                    const float2 v = *reinterpret_cast<const float2*>(row + la);
                    b.va[j] = v.x;
                    b.vb[j] = v.y;
                } else {
                    b.va[j] = row[la];
                    b.vb[j] = row[lb];
                }
            }
        };
        auto add = [&](int64_t e, const Batch& b) {
            const int nb = static_cast<int>(e_end - e < kHistBatch ? e_end - e : kHistBatch);
            const EdgeBin eb = edge_bin(b.r, B);
            if constexpr (PAIR) {
                // Edges in groups of four.  When a group's lower bins are pairwise
                // at least two apart its cells are distinct, and all its reads are
                // issued before any write (one LDS round trip instead of four);
                // otherwise its edges go one at a time.  Every cell receives its
                // edges in edge order either way.
#pragma unroll
                for (int g = 0; g < kHistBatch; g += 4) {
                    int lo[4];
                    float t[4];
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        lo[q] = __builtin_amdgcn_readlane(eb.lo, g + q);
                        t[q] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(eb.t), g + q));
                    }
                    bool apart = g + 3 < nb;
#pragma unroll
                    for (int q = 0; q < 4; ++q)
#pragma unroll
                        for (int r = q + 1; r < 4; ++r)
                            apart = apart && (lo[q] - lo[r] >= 2 || lo[r] - lo[q] >= 2);
                    if (!ina) continue;
                    if (apart) {
                        float2 c[4][2];
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            c[q][0] = *reinterpret_cast<const float2*>(h + lo[q] * kw + ca);
                            c[q][1] = *reinterpret_cast<const float2*>(h + lo[q] * kw + kw + ca);
                        }
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            const float u = 1.0f - t[q], va = b.va[g + q], vb = b.vb[g + q];
                            *reinterpret_cast<float2*>(h + lo[q] * kw + ca) =
                                make_float2(c[q][0].x + u * va, c[q][0].y + u * vb);
                            *reinterpret_cast<float2*>(h + lo[q] * kw + kw + ca) =
                                make_float2(c[q][1].x + t[q] * va, c[q][1].y + t[q] * vb);
                        }
                    } else {
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            if (g + q >= nb) break;
                            float2* p0 = reinterpret_cast<float2*>(h + lo[q] * kw + ca);
                            float2* p1 = reinterpret_cast<float2*>(h + lo[q] * kw + kw + ca);
                            const float2 a = *p0, c = *p1;
                            const float u = 1.0f - t[q], va = b.va[g + q], vb = b.vb[g + q];
                            *p0 = make_float2(a.x + u * va, a.y + u * vb);
                            *p1 = make_float2(c.x + t[q] * va, c.y + t[q] * vb);
                        }
                    }
                }
                return;
            }
#pragma unroll
            for (int j = 0; j < kHistBatch; ++j) {
                if (j < nb) {
                    const int lo = __builtin_amdgcn_readlane(eb.lo, j);
                    const float t = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(eb.t), j));
                    float* hl = h + lo * kw;
                    // read-add-write: the wave's LDS operations execute in issue
                    // order, so the next edge's reads see these writes (a lane's
                    // four cells are distinct: read all, then write)
                    const float a0 = ina ? hl[ca] : 0.0f, a1 = ina ? hl[kw + ca] : 0.0f;
                    const float b0 = inb ? hl[cb] : 0.0f, b1 = inb ? hl[kw + cb] : 0.0f;
                    if (ina) {
                        hl[ca] = a0 + (1.0f - t) * b.va[j];
                        hl[kw + ca] = a1 + t * b.va[j];
                    }
                    if (inb) {
                        hl[cb] = b0 + (1.0f - t) * b.vb[j];
                        hl[kw + cb] = b1 + t * b.vb[j];
                    }
                }
            }
        };
        Batch b0, b1;
        int64_t e = e_begin;
        if (e < e_end) {
            load(e, b0);
            for (;;) {
                load(e + kHistBatch, b1);
                add(e, b0);
                e += kHistBatch;
                if (e >= e_end) break;
                load(e + kHistBatch, b0);
                add(e, b1);
                e += kHistBatch;
                if (e >= e_end) break;
            }
        }
    }
    __syncthreads();
    float* out = hist_part + static_cast<int64_t>(blockIdx.x) * (B.num_bins + 1) * kw_row + cw0;
    for (int q = threadIdx.x; q < hsz; q += blockDim.x) {
        float acc = sh[q];
        for (int v = 1; v < waves; ++v) acc += sh[static_cast<int64_t>(v) * hsz + q];
        out[(q / kw) * kw_row + q % kw] = acc;
    }
}

// Wide rows (no room for several histograms in LDS): the edges are grouped by lower bin (a stable CSR by bin from the library's
// radix sort) and the sorted positions cut into tiles of kBinTile.  Per bin n
// the kernels form S0[n] = sum (1 - t) dF_e and S1[n] = sum t dF_e over the
// bin's edges in sorted order; dF[b] = S0[b] + S1[b - 1].  A workgroup (tile,
// column block) walks its positions in order and closes every run of equal
// bins: a bin inside the tile is written whole, a bin that crosses a tile
// boundary leaves a partial row per tile (slot 0 for the tile's first run,
// slot 1 for its last), summed in tile order by the output kernel.  No
// atomics and no LDS histogram: every cell's summation order is fixed, so the
// result is deterministic, and the work spreads over tiles x column blocks
// whatever the row width.
constexpr int kBinTile = 256;     // sorted positions per tile
constexpr int kBinBatch = 8;      // loads in flight per thread

__global__ void k_ewm_keys(feq_binning B, int64_t E, const float* __restrict__ dist,
                           int64_t* __restrict__ lo) {
    const int64_t e = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
    if (e < E) lo[e] = bin_index(dist[e], B);
}

__device__ __forceinline__ bool bin_crosses_tiles(int b, int e) { return b / kBinTile != (e - 1) / kBinTile; }

// grid (tiles, column blocks of blockDim.x); S holds S0 rows [0, nb) then S1 rows.
__global__ void __launch_bounds__(kThreads)
k_ewm_binsum(feq_binning B, int kw, int64_t E, const float* __restrict__ dist,
             const float* __restrict__ dFe, const int32_t* __restrict__ perm,
             const int32_t* __restrict__ offsets, float* __restrict__ S, float* __restrict__ part) {
    __shared__ int spe[kBinTile], slo[kBinTile];
    __shared__ float st[kBinTile];
    const int nb = B.num_bins;
    const int64_t tile = blockIdx.x;
    const int64_t p0 = tile * kBinTile;
    const int np = static_cast<int>(E - p0 < kBinTile ? E - p0 : kBinTile);
    for (int j = threadIdx.x; j < np; j += blockDim.x) {
        const int e = perm[p0 + j];
        const EdgeBin eb = edge_bin(dist[e], B);
        spe[j] = e;
        slo[j] = eb.lo;
        st[j] = eb.t;
    }
    __syncthreads();
    const int c = blockIdx.y * blockDim.x + threadIdx.x;
    if (c >= kw) return;
    float a0 = 0.0f, a1 = 0.0f;
    int js = 0;   // first position of the current run
    for (int j0 = 0; j0 < np; j0 += kBinBatch) {
        float v[kBinBatch];
#pragma unroll
        for (int q = 0; q < kBinBatch; ++q) {
            const int j = j0 + q < np ? j0 + q : np - 1;
            v[q] = dFe[static_cast<int64_t>(spe[j]) * kw + c];
        }
#pragma unroll
        for (int q = 0; q < kBinBatch; ++q) {
            const int j = j0 + q;
            if (j >= np) break;
            const float t = st[j];
            a0 += (1.0f - t) * v[q];
            a1 += t * v[q];
            const int n = slo[j];
            if (j + 1 < np && slo[j + 1] == n) continue;
            if (bin_crosses_tiles(offsets[n], offsets[n + 1])) {
                const int64_t row = (2 * tile + (js == 0 ? 0 : 1)) * 2;
                part[row * kw + c] = a0;
                part[(row + 1) * kw + c] = a1;
            } else {
                S[static_cast<int64_t>(n) * kw + c] = a0;
                S[static_cast<int64_t>(nb + n) * kw + c] = a1;
            }
            a0 = a1 = 0.0f;
            js = j + 1;
        }
    }
}

// S0 (comp 0) or S1 (comp 1) of bin n at column c: zero for an empty bin, the
// tile partials in tile order for a bin that crosses tiles, else the row
// k_ewm_binsum wrote.
__device__ __forceinline__ float bin_sum(const float* __restrict__ S, const float* __restrict__ part,
                                         const int32_t* __restrict__ offsets, int nb, int kw, int n,
                                         int comp, int c) {
    const int b = offsets[n], e = offsets[n + 1];
    if (b >= e) return 0.0f;
    if (!bin_crosses_tiles(b, e)) return S[static_cast<int64_t>(comp * nb + n) * kw + c];
    const int t0 = b / kBinTile, t1 = (e - 1) / kBinTile;
    float acc = 0.0f;
    for (int t = t0; t <= t1; ++t) {
        const int slot = (t == t0 && b % kBinTile != 0) ? 1 : 0;
        acc += part[((2 * static_cast<int64_t>(t) + slot) * 2 + comp) * kw + c];
    }
    return acc;
}

// dF[b] = S0[b] + S1[b - 1], b = 0 .. nb; grid (nb + 1, column blocks).
__global__ void __launch_bounds__(kThreads)
k_ewm_binout(feq_binning B, int kw, const float* __restrict__ S, const float* __restrict__ part,
             const int32_t* __restrict__ offsets, float* __restrict__ gF) {
    const int nb = B.num_bins, b = blockIdx.x;
    const int c = blockIdx.y * blockDim.x + threadIdx.x;
    if (c >= kw) return;
    float v = 0.0f;
    if (b < nb) v = bin_sum(S, part, offsets, nb, kw, b, 0, c);
    if (b > 0) v += bin_sum(S, part, offsets, nb, kw, b - 1, 1, c);
    gF[static_cast<int64_t>(b) * kw + c] = v;
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
#pragma unroll 8
    for (int g = g0; g < g1; ++g) acc += part[static_cast<int64_t>(g) * n + q];
    out[blockIdx.y * n + q] = acc;
}

// k_sum_partials over several jobs in one launch: job j owns the workgroups
// [start[j], start[j + 1]), nb[j] per slice; each sums the same partials in
// the same order as k_sum_partials.
struct SliceJobs {
    const float* part[2 * kMaxPartialJobs];
    float* out[2 * kMaxPartialJobs];
    int64_t n[2 * kMaxPartialJobs];
    int groups[2 * kMaxPartialJobs], per_slice[2 * kMaxPartialJobs];
    int64_t nb[2 * kMaxPartialJobs];
    int64_t start[2 * kMaxPartialJobs + 1];
    int count;
};

__global__ void __launch_bounds__(256)
k_sum_slices_multi(SliceJobs J) {
    const int64_t b = blockIdx.x;
    int j = 0;
    while (j + 1 < J.count && b >= J.start[j + 1]) ++j;
    const int64_t local = b - J.start[j], nb = J.nb[j], n = J.n[j];
    const int slice = static_cast<int>(local / nb);
    const int64_t q = (local - slice * nb) * 256 + threadIdx.x;
    if (q >= n) return;
    const int g0 = slice * J.per_slice[j];
    const int g1 = g0 + J.per_slice[j] < J.groups[j] ? g0 + J.per_slice[j] : J.groups[j];
    const float* part = J.part[j];
    float acc = 0.0f;
#pragma unroll 8
    for (int g = g0; g < g1; ++g) acc += part[static_cast<int64_t>(g) * n + q];
    J.out[j][slice * n + q] = acc;
}

// Few sums of many partials (n <= kSmallN): a workgroup per output, its
// threads summing interleaved partials, combined by a fixed tree in LDS.
__global__ void __launch_bounds__(256)
k_sum_partials_small(const float* __restrict__ part, int groups, int64_t n, float* __restrict__ out) {
    __shared__ float s[256];
    const int64_t q = blockIdx.x;
    float acc = 0.0f;
    for (int g = threadIdx.x; g < groups; g += 256) acc += part[static_cast<int64_t>(g) * n + q];
    s[threadIdx.x] = acc;
    __syncthreads();
    for (int h = 128; h > 0; h >>= 1) {
        if (threadIdx.x < h) s[threadIdx.x] += s[threadIdx.x + h];
        __syncthreads();
    }
    if (threadIdx.x == 0) out[q] = s[0];
}

constexpr int64_t kSmallN = 256;

// k_sum_partials_small over several jobs: workgroup b sums output b - start[j]
// of the job j whose range [start[j], start[j + 1]) holds b.
struct PartialJobs {
    const float* part[kMaxPartialJobs];
    float* out[kMaxPartialJobs];
    int64_t n[kMaxPartialJobs];
    int groups[kMaxPartialJobs];
    int64_t start[kMaxPartialJobs + 1];
    int count;
};

__global__ void __launch_bounds__(256)
k_sum_partials_multi(PartialJobs J) {
    __shared__ float s[256];
    const int64_t b = blockIdx.x;
    int j = 0;
    while (j + 1 < J.count && b >= J.start[j + 1]) ++j;
    const int64_t q = b - J.start[j], n = J.n[j];
    const float* part = J.part[j];
    const int groups = J.groups[j];
    float acc = 0.0f;
    for (int g = threadIdx.x; g < groups; g += 256) acc += part[static_cast<int64_t>(g) * n + q];
    s[threadIdx.x] = acc;
    __syncthreads();
    for (int h = 128; h > 0; h >>= 1) {
        if (threadIdx.x < h) s[threadIdx.x] += s[threadIdx.x + h];
        __syncthreads();
    }
    if (threadIdx.x == 0) J.out[j][q] = s[0];
}

constexpr int kSliceGroups = 32;   // partials summed per thread in one pass

size_t reduce_tmp_floats(int groups, int64_t n) {
    return groups > kSliceGroups ? static_cast<size_t>((groups + kSliceGroups - 1) / kSliceGroups) * n
                                 : 0;
}

}  // namespace

// Deterministic sum of `groups` partial arrays of n floats: slices of at most
// kSliceGroups partials into tmp, then the slices into out (up to kSmallN
// outputs: one launch, a workgroup per output).
int reduce_partials(const float* part, int groups, int64_t n, float* out, float* tmp,
                    hipStream_t s) {
    const unsigned nb = static_cast<unsigned>(ceil_div(n, 256));
    if (n <= kSmallN && groups > kSliceGroups) {
        FEQ_LAUNCH("k_sum_partials", k_sum_partials_small, dim3(static_cast<unsigned>(n)), dim3(256), 0, s,
                   part, groups, n, out);
        return FEQ_OK;
    }
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

int reduce_partials_multi(const PartialJob* jobs, int njobs, hipStream_t s) {
    if (njobs < 1) return FEQ_OK;
    bool small = njobs <= kMaxPartialJobs;
    for (int j = 0; j < njobs && small; ++j) small = jobs[j].n <= kSmallN && jobs[j].groups > kSliceGroups;
    if (!small && njobs > kMaxPartialJobs) {
        for (int j = 0; j < njobs; ++j)
            if (int rc = reduce_partials(jobs[j].part, jobs[j].groups, jobs[j].n, jobs[j].out, jobs[j].tmp, s))
                return rc;
        return FEQ_OK;
    }
    if (!small) {
        // the first slices of every job in one launch, the sums of the slices
        // in a second (the same sums, in the same order, as reduce_partials;
        // no partials: zeros); few-output jobs keep their own one-launch form
        SliceJobs L1{}, L2{};
        auto add = [](SliceJobs& J, const float* part, int groups, int per_slice, int64_t n, float* out) {
            const int slices = groups > 0 ? (groups + per_slice - 1) / per_slice : 1;
            const int k = J.count++;
            J.part[k] = part;
            J.out[k] = out;
            J.n[k] = n;
            J.groups[k] = groups;
            J.per_slice[k] = per_slice;
            J.nb[k] = ceil_div(n, 256);
            J.start[k + 1] = J.start[k] + J.nb[k] * slices;
        };
        for (int j = 0; j < njobs; ++j) {
            const PartialJob& p = jobs[j];
            if (p.n <= 0) continue;
            if (p.n <= kSmallN && p.groups > kSliceGroups) {
                if (int rc = reduce_partials(p.part, p.groups, p.n, p.out, p.tmp, s)) return rc;
            } else if (p.groups <= kSliceGroups) {
                add(L1, p.part, p.groups > 0 ? p.groups : 0, p.groups > 0 ? p.groups : 1, p.n, p.out);
            } else {
                const int slices = (p.groups + kSliceGroups - 1) / kSliceGroups;
                add(L1, p.part, p.groups, kSliceGroups, p.n, p.tmp);
                add(L2, p.tmp, slices, slices, p.n, p.out);
            }
        }
        for (const SliceJobs* J : {&L1, &L2})
            if (J->count > 0)
                FEQ_LAUNCH("k_sum_partials", k_sum_slices_multi, dim3(static_cast<unsigned>(J->start[J->count])),
                           dim3(256), 0, s, *J);
        return FEQ_OK;
    }
    PartialJobs J{};
    J.count = njobs;
    J.start[0] = 0;
    for (int j = 0; j < njobs; ++j) {
        J.part[j] = jobs[j].part;
        J.out[j] = jobs[j].out;
        J.n[j] = jobs[j].n;
        J.groups[j] = jobs[j].groups;
        J.start[j + 1] = J.start[j] + jobs[j].n;
    }
    if (J.start[njobs] == 0) return FEQ_OK;
    FEQ_LAUNCH("k_sum_partials", k_sum_partials_multi, dim3(static_cast<unsigned>(J.start[njobs])), dim3(256), 0,
               s, J);
    return FEQ_OK;
}

namespace {

constexpr int kHistCUs = 256;              // histogram workgroups per CU-round (fixed: the order is set by E alone)
constexpr size_t kHistLds = 160 * 1024;

// Launch shape of the histogram kernel: waves (private histograms) per
// workgroup and workgroups.  Rows small enough for six histograms in a CU's
// LDS take workgroups of two waves, three or four per CU (more waves resident,
// each walking fewer edges: the walk is bound by LDS and load latency, not by
// bandwidth); otherwise up to four waves in one workgroup per CU.  The shape
// depends on the layout alone, so the summation order is fixed.
struct HistShape {
    int waves, groups;
};
HistShape hist_shape(const feq_binning& B, int kw) {
    const size_t hbytes = 4 * static_cast<size_t>(B.num_bins + 1) * kw;
    const size_t per_cu = kHistLds / hbytes;
    if (per_cu >= 6) return {2, kHistCUs * static_cast<int>(per_cu >= 8 ? 4 : 3)};
    return {static_cast<int>(per_cu < 4 ? per_cu : 4), kHistCUs};
}

// Workgroups for E edges: the shape's, or fewer for few edges (at least 64
// edges per wave), so that a small graph does not zero, write and sum hundreds
// of empty histograms.  Set by E and the layout alone: a fixed order.
int hist_groups(const feq_binning& B, int kw, int64_t E) {
    const HistShape hs = hist_shape(B, kw);
    const int64_t need = ceil_div(E > 0 ? E : 1, static_cast<int64_t>(hs.waves) * 64);
    return static_cast<int>(need < hs.groups ? need : hs.groups);
}

// The LDS histograms serve rows for which at least two fit a workgroup's LDS;
// wider rows take the sorted-bin form.
bool use_hist(const feq_binning& B, int kw) { return hist_shape(B, kw).waves >= 2; }

// Workspace of the binned gradient, carved from `tail` in this order.
struct BinWs {
    int64_t* keys;
    int32_t* perm;
    int32_t* offsets;
    void* csr;
    float* S;
    float* part;
    float* tmp;    // the channel patterns' partial sums
    float* htmp;   // the histogram partials' sums (reduced in the same launches)
    size_t bytes;
};

BinWs bin_ws(const feq_binning& B, int kw, int64_t E, int groups, int64_t ncc, void* base) {
    Carver cv(base);
    BinWs w{};
    const int64_t hsz = (B.num_bins + 1) * static_cast<int64_t>(kw);
    const size_t tmp = reduce_tmp_floats(groups, ncc) + 1;
    size_t htmp = 0;
    if (use_hist(B, kw)) {
        // per-workgroup histogram partials
        const int groups = hist_groups(B, kw, E);
        w.part = cv.take<float>(static_cast<size_t>(groups) * hsz);
        htmp = reduce_tmp_floats(groups, hsz);
    } else {
        const int64_t ntiles = ceil_div(E, kBinTile);
        w.keys = cv.take<int64_t>(E);
        w.perm = cv.take<int32_t>(E);
        w.offsets = cv.take<int32_t>(B.num_bins + 1);
        w.csr = cv.take<char>(feq_csr_workspace(E, B.num_bins));
        w.S = cv.take<float>(2 * static_cast<size_t>(B.num_bins) * kw);
        w.part = cv.take<float>(4 * static_cast<size_t>(ntiles) * kw);
    }
    w.tmp = cv.take<float>(tmp);
    w.htmp = htmp ? cv.take<float>(htmp) : nullptr;
    w.bytes = cv.used + 256;
    return w;
}

}  // namespace

bool ew_tail_supported(const feq_binning& B, int kw) { return B.num_bins >= 1 && kw >= 1; }

size_t ew_tail_floats(const feq_binning& B, int kw, int64_t E, int groups, int64_t ncc) {
    return (bin_ws(B, kw, E, groups, ncc, nullptr).bytes + 3) / 4;
}

int ew_tail(const feq_layout& L, const feq_binning& B, int K, int64_t E, const float* dist,
            const float* F, const float* dFe, const float* dCp, int groups, int64_t ncc, float* gC,
            float* gF, float* gdist, float* tail, hipStream_t s) {
    const int kw = K * L.wdim;
    const int nb = B.num_bins;
    if (!ew_tail_supported(B, kw)) return fail(FEQ_ERR_UNSUPPORTED, "empty radial-function rows");
    if (E == 0) {
        if (groups > 0)
            if (int rc = reduce_partials(dCp, groups, ncc, gC, tail, s)) return rc;
        return fill_zero(gF, static_cast<int64_t>(nb + 1) * kw, s);
    }
    const BinWs w = bin_ws(B, kw, E, groups, ncc, tail);
    PartialJob jobs[2];
    int njobs = 0;
    if (use_hist(B, kw)) {
        const HistShape hs = hist_shape(B, kw);
        const int waves = hs.waves, groups = hist_groups(B, kw, E);
        const size_t hlds = 4 * static_cast<size_t>(waves) * (nb + 1) * kw;
        const int64_t per_wave = ceil_div(E, static_cast<int64_t>(groups) * waves);
        if (kw % 2 == 0 && reinterpret_cast<uintptr_t>(dFe) % 8 == 0) {
            FEQ_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&k_ewm_hist<true>),
                                        hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kHistLds)));
            FEQ_LAUNCH("k_ewm_hist", k_ewm_hist<true>, dim3(groups), dim3(64 * waves), hlds, s, B, kw, 0,
                       kw, E, per_wave, dist, dFe, w.part);
        } else {
            FEQ_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&k_ewm_hist<false>),
                                        hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kHistLds)));
            FEQ_LAUNCH("k_ewm_hist", k_ewm_hist<false>, dim3(groups), dim3(64 * waves), hlds, s, B, kw, 0,
                       kw, E, per_wave, dist, dFe, w.part);
        }
        jobs[njobs++] = PartialJob{w.part, groups, (nb + 1) * static_cast<int64_t>(kw), gF, w.htmp};
    } else {
        FEQ_LAUNCH("k_ewm_keys", k_ewm_keys, dim3(ceil_div(E, kThreads)), dim3(kThreads), 0, s, B, E,
                   dist, w.keys);
        if (int rc = feq_csr_by_dst(w.keys, E, nb, w.perm, w.offsets, w.csr, feq_csr_workspace(E, nb),
                                    reinterpret_cast<feq_stream_t>(s)))
            return rc;
        const int bt = kw < kThreads ? static_cast<int>(ceil_div(kw, 64)) * 64 : kThreads;
        const unsigned cbs = static_cast<unsigned>(ceil_div(kw, bt));
        FEQ_LAUNCH("k_ewm_binsum", k_ewm_binsum, dim3(static_cast<unsigned>(ceil_div(E, kBinTile)), cbs),
                   dim3(bt), 0, s, B, kw, E, dist, dFe, w.perm, w.offsets, w.S, w.part);
        FEQ_LAUNCH("k_ewm_binout", k_ewm_binout, dim3(static_cast<unsigned>(nb + 1), cbs), dim3(bt), 0, s,
                   B, kw, w.S, w.part, w.offsets, gF);
    }
    if (gdist)
        FEQ_LAUNCH("k_ewm_dr", k_ewm_dr, dim3(ceil_div(E, kThreads)), dim3(kThreads),
                   sizeof(int) * L.wdim, s, L, B, K, E, dist, F, dFe, gdist);
    // the binned gradient's and the channel patterns' partial sums together
    if (groups > 0) jobs[njobs++] = PartialJob{dCp, groups, ncc, gC, w.tmp};
    return reduce_partials_multi(jobs, njobs, s);
}

}  // namespace feq

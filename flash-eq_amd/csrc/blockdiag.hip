// Generic block-diagonal radial mix (the reference's pybind forward/backward),
// in float32 and float64.
//
// Features and outputs are in the m-first basis; the radial table has the
// reference layout (num_bins+1, Cout, Cin, Wdim).  Semantics follow
// block_diagonal.cu:558-1161 (see flasheq.h for the entry points):
//   y[e,co,slot] = sum_{ci,i} lerp_t(T)[co,ci,w(o,i)] s^(l_i+l_o) x[e,ci,slot_i]
// with the 2x2 [[a, b], [-b, a]] structure on (+m, -m) pairs for m > 0.
//
// Forward and feature gradient: one workgroup per edge, the edge's row staged
// in LDS, every thread producing whole outputs.  Table gradient: the edges are
// grouped by lower bin (a CSR built by the library's radix sort), and one
// workgroup per (table row b, slice of the (co, ci, w) weights) sums the
// contributions of the edges in bins b (weight 1 - t) and b - 1 (weight t) in a
// fixed order: no atomics, every row written, the same bits on every run.
// Distance gradient: one workgroup per edge, a fixed-order workgroup sum.
#include "feq_internal.h"

namespace feq {
namespace {

constexpr int kThreads = 256;

struct SlotRef {
    int blk;  // m-block index, -1 when the slot has no partner block
    int o;    // index inside the block
    int c;    // 0 = +m (re) component, 1 = -m (im)
};

__device__ __forceinline__ SlotRef find_out_slot(const feq_layout& L, int slot) {
    for (int k = 0; k < L.nblocks; ++k) {
        const int m = L.blk[k][0], no = L.blk[k][2], off = L.blk[k][4];
        const int w = m == 0 ? 1 : 2;
        if (slot >= off && slot < off + w * no) {
            const int rel = slot - off;
            return {k, rel / w, rel % w};
        }
    }
    return {-1, 0, 0};
}

__device__ __forceinline__ SlotRef find_in_slot(const feq_layout& L, int slot) {
    for (int k = 0; k < L.nblocks; ++k) {
        const int m = L.blk[k][0], ni = L.blk[k][1], off = L.blk[k][3];
        const int w = m == 0 ? 1 : 2;
        if (slot >= off && slot < off + w * ni) {
            const int rel = slot - off;
            return {k, rel / w, rel % w};
        }
    }
    return {-1, 0, 0};
}

template <class T>
__device__ __forceinline__ T lerp_t(T lo, T hi, T t) {
    return lo + t * (hi - lo);
}

// Weight w's place in the layout: input slot (the +m slot of a pair), output
// slot, degree sum and the component (0: a, 1: b of the 2x2 block; m = 0: -1).
struct WeightRef {
    int is, os, lsum, comp;
};

__device__ __forceinline__ WeightRef weight_ref(const feq_layout& L, int w) {
    int k = L.nblocks - 1;
    while (k > 0 && w < L.blk[k][5]) --k;
    const int m = L.blk[k][0], ni = L.blk[k][1];
    const int in_off = L.blk[k][3], out_off = L.blk[k][4], w_off = L.blk[k][5];
    const int rel = w - w_off;
    WeightRef r;
    if (m == 0) {
        r.is = in_off + rel % ni;
        r.os = out_off + rel / ni;
        r.comp = -1;
    } else {
        const int pair = rel >> 1;
        r.is = in_off + 2 * (pair % ni);
        r.os = out_off + 2 * (pair / ni);
        r.comp = rel & 1;
    }
    r.lsum = L.lslot_in[r.is] + L.lslot_out[r.os];
    return r;
}

// d y / d T for one weight, before the solid-harmonic factor (block_diagonal.cu:514-517)
template <class T>
__device__ __forceinline__ T weight_grad(const WeightRef& r, const T* xr, const T* gr) {
    if (r.comp < 0) return xr[r.is] * gr[r.os];
    const T fr = xr[r.is], fi = xr[r.is + 1], g_r = gr[r.os], g_i = gr[r.os + 1];
    return r.comp == 0 ? fr * g_r + fi * g_i : fi * g_r - fr * g_i;
}

template <class T>
__global__ void __launch_bounds__(kThreads)
k_bd_fwd(feq_layout L, feq_binning B, const T* __restrict__ x, const T* __restrict__ table,
         const T* __restrict__ dist, T* __restrict__ y) {
    extern __shared__ char smem[];
    T* sx = reinterpret_cast<T*>(smem);  // (cin, din) of this edge
    const int64_t e = blockIdx.x;
    const int cin = L.cin, din = L.din, cout = L.cout, dout = L.dout, wd = L.wdim;
    for (int q = threadIdx.x; q < cin * din; q += kThreads) sx[q] = x[e * cin * din + q];
    __syncthreads();
    const T r = dist[e];
    const EdgeBinT<T> eb = edge_bin_t<T>(r, B);
    const T t = eb.t;
    const T sw = r / (r + static_cast<T>(B.sh_scale));
    const int64_t tstride = static_cast<int64_t>(cout) * cin * wd;
    const T* tlo = table + eb.lo * tstride;
    const T* thi = tlo + tstride;
    for (int q = threadIdx.x; q < cout * dout; q += kThreads) {
        const int co = q / dout, slot = q % dout;
        const SlotRef s = find_out_slot(L, slot);
        T acc = T(0);
        if (s.blk >= 0) {
            const int m = L.blk[s.blk][0], ni = L.blk[s.blk][1];
            const int in_off = L.blk[s.blk][3], w_off = L.blk[s.blk][5];
            const int lo_l = L.lslot_out[slot];
            for (int i = 0; i < ni; ++i) {
                const int islot = in_off + (m == 0 ? i : 2 * i);
                const T sc = ipow_t<T>(sw, lo_l + L.lslot_in[islot]);
                const int64_t wb = static_cast<int64_t>(co) * cin * wd;
                if (m == 0) {
                    const int w = w_off + s.o * ni + i;
                    for (int ci = 0; ci < cin; ++ci) {
                        const int64_t a = wb + static_cast<int64_t>(ci) * wd + w;
                        acc += lerp_t<T>(tlo[a], thi[a], t) * sc * sx[ci * din + islot];
                    }
                } else {
                    const int w = w_off + 2 * (s.o * ni + i);
                    for (int ci = 0; ci < cin; ++ci) {
                        const int64_t a = wb + static_cast<int64_t>(ci) * wd + w;
                        const T wa = lerp_t<T>(tlo[a], thi[a], t) * sc;
                        const T wb2 = lerp_t<T>(tlo[a + 1], thi[a + 1], t) * sc;
                        const T fr = sx[ci * din + islot], fi = sx[ci * din + islot + 1];
                        acc += s.c == 0 ? (wa * fr + wb2 * fi) : (wa * fi - wb2 * fr);
                    }
                }
            }
        }
        y[e * cout * dout + q] = acc;
    }
}

template <class T>
__global__ void __launch_bounds__(kThreads)
k_bd_bwd_x(feq_layout L, feq_binning B, const T* __restrict__ gy, const T* __restrict__ table,
           const T* __restrict__ dist, T* __restrict__ gx) {
    extern __shared__ char smem[];
    T* sg = reinterpret_cast<T*>(smem);  // (cout, dout) gradient row of this edge
    const int64_t e = blockIdx.x;
    const int cin = L.cin, din = L.din, cout = L.cout, dout = L.dout, wd = L.wdim;
    for (int q = threadIdx.x; q < cout * dout; q += kThreads) sg[q] = gy[e * cout * dout + q];
    __syncthreads();
    const T r = dist[e];
    const EdgeBinT<T> eb = edge_bin_t<T>(r, B);
    const T t = eb.t;
    const T sw = r / (r + static_cast<T>(B.sh_scale));
    const int64_t tstride = static_cast<int64_t>(cout) * cin * wd;
    const T* tlo = table + eb.lo * tstride;
    const T* thi = tlo + tstride;
    for (int q = threadIdx.x; q < cin * din; q += kThreads) {
        const int ci = q / din, slot = q % din;
        const SlotRef s = find_in_slot(L, slot);
        T acc = T(0);
        if (s.blk >= 0) {
            const int m = L.blk[s.blk][0], ni = L.blk[s.blk][1], no = L.blk[s.blk][2];
            const int out_off = L.blk[s.blk][4], w_off = L.blk[s.blk][5];
            const int li = L.lslot_in[slot];
            for (int o = 0; o < no; ++o) {
                const int oslot = out_off + (m == 0 ? o : 2 * o);
                const T sc = ipow_t<T>(sw, li + L.lslot_out[oslot]);
                if (m == 0) {
                    const int w = w_off + o * ni + s.o;
                    for (int co = 0; co < cout; ++co) {
                        const int64_t a = (static_cast<int64_t>(co) * cin + ci) * wd + w;
                        acc += lerp_t<T>(tlo[a], thi[a], t) * sc * sg[co * dout + oslot];
                    }
                } else {
                    const int w = w_off + 2 * (o * ni + s.o);
                    for (int co = 0; co < cout; ++co) {
                        const int64_t a = (static_cast<int64_t>(co) * cin + ci) * wd + w;
                        const T wa = lerp_t<T>(tlo[a], thi[a], t) * sc;
                        const T wb2 = lerp_t<T>(tlo[a + 1], thi[a + 1], t) * sc;
                        const T gr = sg[co * dout + oslot], gi = sg[co * dout + oslot + 1];
                        acc += s.c == 0 ? (wa * gr - wb2 * gi) : (wb2 * gr + wa * gi);
                    }
                }
            }
        }
        gx[e * cin * din + q] = acc;
    }
}

// ---- table gradient by bin ---------------------------------------------------------
// Per edge: lower bin (as the sort key) and the solid-harmonic base s.
template <class T>
__global__ void k_bd_bins(feq_binning B, int64_t E, const T* __restrict__ dist,
                          int64_t* __restrict__ lo) {
    const int64_t e = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
    if (e < E) lo[e] = bin_index(static_cast<float>(dist[e]), B);
}

constexpr int kTbNJ = 16;          // weights per thread in the table-gradient kernel
constexpr int kTbEdges = 8;        // edges staged per step

// Workgroup (b, slice): table row b, weights (co, ci, w) of the slice, q = the
// slice-local index (co - co0) ci_n wd + (ci - ci0) wd + w; thread t owns
// q = t + 256 j.  grid.y enumerates (co block, ci block).
template <class T>
__global__ void __launch_bounds__(kThreads)
k_bd_bwd_table(feq_layout L, feq_binning B, int64_t E, const T* __restrict__ gy,
               const T* __restrict__ x, const T* __restrict__ dist, const int32_t* __restrict__ perm,
               const int32_t* __restrict__ offsets, int ob, int ib, T* __restrict__ gtable) {
    extern __shared__ char smem[];
    const int cin = L.cin, din = L.din, cout = L.cout, dout = L.dout, wd = L.wdim;
    const int nb = B.num_bins;
    const int b = blockIdx.x;
    const int ncib = (cin + ib - 1) / ib;
    const int co0 = (blockIdx.y / ncib) * ob, ci0 = (blockIdx.y % ncib) * ib;
    const int con = min(ob, cout - co0), cin_n = min(ib, cin - ci0);
    const int nq = con * cin_n * wd;
    T* sx = reinterpret_cast<T*>(smem);                   // [kTbEdges][ib][din]
    T* sg = sx + kTbEdges * ib * din;                      // [kTbEdges][ob][dout]
    T* sw = sg + kTbEdges * ob * dout;                     // [kTbEdges][2 lmax + 1]: weight * s^l
    const int npw = 2 * (FEQ_MAX_BLOCKS - 1) + 1;

    // this thread's weights: fixed for the launch
    WeightRef ref[kTbNJ];
    int xo[kTbNJ], go[kTbNJ];
    T acc[kTbNJ];
#pragma unroll
    for (int j = 0; j < kTbNJ; ++j) {
        const int q = threadIdx.x + kThreads * j;
        acc[j] = T(0);
        if (q < nq) {
            const int w = q % wd, ci = (q / wd) % cin_n, co = q / (wd * cin_n);
            ref[j] = weight_ref(L, w);
            xo[j] = ci * din;
            go[j] = co * dout;
        } else {
            ref[j] = WeightRef{0, 0, 0, -1};
            xo[j] = go[j] = 0;
        }
    }
    // edges of bin b (weight 1 - t) then of bin b - 1 (weight t)
    const int seg_lo0 = b < nb ? offsets[b] : 0, seg_lo1 = b < nb ? offsets[b + 1] : 0;
    const int seg_hi0 = b > 0 ? offsets[b - 1] : 0, seg_hi1 = b > 0 ? offsets[b] : 0;
    const int n_lo = seg_lo1 - seg_lo0, n_all = n_lo + (seg_hi1 - seg_hi0);
    for (int base = 0; base < n_all; base += kTbEdges) {
        const int ne = min(kTbEdges, n_all - base);
        __syncthreads();
        for (int q = threadIdx.x; q < ne * ib * din; q += kThreads) {
            const int k = q / (ib * din), rest = q % (ib * din), ci = rest / din, d = rest % din;
            const int pos = base + k;
            const int64_t e = perm[pos < n_lo ? seg_lo0 + pos : seg_hi0 + pos - n_lo];
            sx[q] = ci < cin_n ? x[(e * cin + ci0 + ci) * din + d] : T(0);
        }
        for (int q = threadIdx.x; q < ne * ob * dout; q += kThreads) {
            const int k = q / (ob * dout), rest = q % (ob * dout), co = rest / dout, d = rest % dout;
            const int pos = base + k;
            const int64_t e = perm[pos < n_lo ? seg_lo0 + pos : seg_hi0 + pos - n_lo];
            sg[q] = co < con ? gy[(e * cout + co0 + co) * dout + d] : T(0);
        }
        if (threadIdx.x < ne) {
            const int pos = base + threadIdx.x;
            const int64_t e = perm[pos < n_lo ? seg_lo0 + pos : seg_hi0 + pos - n_lo];
            const T r = dist[e];
            const EdgeBinT<T> eb = edge_bin_t<T>(r, B);
            const T wgt = pos < n_lo ? T(1) - eb.t : eb.t;
            const T s = r / (r + static_cast<T>(B.sh_scale));
            T p = wgt;
            for (int l = 0; l < npw; ++l) {
                sw[threadIdx.x * npw + l] = p;
                p *= s;
            }
        }
        __syncthreads();
        for (int k = 0; k < ne; ++k) {
            const T* xr = sx + k * ib * din;
            const T* gr = sg + k * ob * dout;
            const T* pw = sw + k * npw;
#pragma unroll
            for (int j = 0; j < kTbNJ; ++j)
                acc[j] += pw[ref[j].lsum] * weight_grad<T>(ref[j], xr + xo[j], gr + go[j]);
        }
    }
    const int64_t tstride = static_cast<int64_t>(cout) * cin * wd;
#pragma unroll
    for (int j = 0; j < kTbNJ; ++j) {
        const int q = threadIdx.x + kThreads * j;
        if (q < nq) {
            const int w = q % wd, ci = (q / wd) % cin_n, co = q / (wd * cin_n);
            gtable[b * tstride + (static_cast<int64_t>(co0 + co) * cin + ci0 + ci) * wd + w] = acc[j];
        }
    }
}

template <class T>
__device__ __forceinline__ T block_sum(T v, T* red) {
    for (int off = 32; off > 0; off >>= 1) v += __shfl_down(v, off, 64);
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[wid] = v;
    __syncthreads();
    T s = T(0);
    if (threadIdx.x == 0)
        for (int w = 0; w < kThreads / 64; ++w) s += red[w];
    return s;
}

// Distance gradient (block_diagonal.cu:990-1036, 1113-1160):
//   dr = (sum_w (T_hi - T_lo) s^L u) dt/dr + sum_w W s^L u L sigma / (r (r + sigma)),
// u the unscaled weight gradient; NaN at r = 0 when an l > 0 pair exists.
template <class T>
__global__ void __launch_bounds__(kThreads)
k_bd_bwd_r(feq_layout L, feq_binning B, const T* __restrict__ gy, const T* __restrict__ x,
           const T* __restrict__ table, const T* __restrict__ dist, T* __restrict__ gdist) {
    extern __shared__ char smem[];
    const int64_t e = blockIdx.x;
    const int cin = L.cin, din = L.din, cout = L.cout, dout = L.dout, wd = L.wdim;
    T* sx = reinterpret_cast<T*>(smem);
    T* sg = sx + cin * din;
    __shared__ T red[kThreads / 64];
    for (int q = threadIdx.x; q < cin * din; q += kThreads) sx[q] = x[e * cin * din + q];
    for (int q = threadIdx.x; q < cout * dout; q += kThreads) sg[q] = gy[e * cout * dout + q];
    __syncthreads();
    const T r = dist[e];
    const EdgeBinT<T> eb = edge_bin_t<T>(r, B);
    const T t = eb.t;
    const T sigma = static_cast<T>(B.sh_scale);
    const T sw = r / (r + sigma);
    const T deriv = sigma / (r * (r + sigma));
    const int64_t tstride = static_cast<int64_t>(cout) * cin * wd;
    const T* tlo = table + eb.lo * tstride;
    const T* thi = tlo + tstride;
    T acc_t = T(0), acc_s = T(0);
    for (int64_t q = threadIdx.x; q < tstride; q += kThreads) {
        const int w = static_cast<int>(q % wd);
        const int ci = static_cast<int>((q / wd) % cin);
        const int co = static_cast<int>(q / (static_cast<int64_t>(wd) * cin));
        const WeightRef ref = weight_ref(L, w);
        const T u = weight_grad<T>(ref, sx + ci * din, sg + co * dout);
        const T sc = ipow_t<T>(sw, ref.lsum);
        const T wl = tlo[q], wh = thi[q];
        acc_t += (wh - wl) * sc * u;
        if (ref.lsum > 0) acc_s += lerp_t<T>(wl, wh, t) * u * sc * static_cast<T>(ref.lsum) * deriv;
    }
    const T st = block_sum<T>(acc_t, red);
    const T ss = block_sum<T>(acc_s, red);
    if (threadIdx.x == 0) gdist[e] = st * eb.dtdr + ss;
}

template <class T>
__global__ void k_fill_zero_t(T* __restrict__ p, int64_t n) {
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x)
        p[i] = T(0);
}

// Slice of the (co, ci, w) weights per table-gradient workgroup: at most
// kTbNJ * 256 weights, whole ci rows when they fit, and the staged rows of
// kTbEdges edges within 48 KB of LDS.
constexpr size_t kTbLds = 48 * 1024;

void table_slices(const feq_layout& L, size_t elem, int& ob, int& ib) {
    const int cap = kTbNJ * kThreads;
    if (L.cin * L.wdim <= cap) {
        ib = L.cin;
        ob = cap / (L.cin * L.wdim);
        ob = ob > L.cout ? L.cout : ob;
    } else {
        ob = 1;
        ib = cap / L.wdim;
        ib = ib < 1 ? 1 : ib;
    }
    const int64_t rows = static_cast<int64_t>(kTbLds / (elem * kTbEdges));   // (ib din + ob dout) cap
    while (ob > 1 && ib * L.din + ob * L.dout > rows) --ob;
    while (ib > 1 && ib * L.din + ob * L.dout > rows) --ib;
}

template <class T>
size_t table_lds(const feq_layout& L, int ob, int ib) {
    return sizeof(T) * (static_cast<size_t>(kTbEdges) * (ib * L.din + ob * L.dout) +
                        kTbEdges * (2 * (FEQ_MAX_BLOCKS - 1) + 1));
}

size_t bin_ws_bytes(const feq_binning& b, int64_t E) {
    return align_up(sizeof(int64_t) * E, 256) + align_up(sizeof(int32_t) * E, 256) +
           align_up(sizeof(int32_t) * (b.num_bins + 1), 256) + feq_csr_workspace(E, b.num_bins) + 256;
}

template <class T>
int blockdiag_fwd(const feq_layout* L, const feq_binning* b, int64_t E, const T* x, const T* table,
                  const T* dist, T* y, feq_stream_t stream) {
    if (int rc = check_layout(L)) return rc;
    if (int rc = check_binning(b)) return rc;
    if (E < 0) return fail(FEQ_ERR_INVALID, "negative edge count");
    if (E == 0) return FEQ_OK;
    if (!x || !table || !dist || !y) return fail(FEQ_ERR_INVALID, "NULL pointer");
    if (E > 0x7fffffffLL) return fail(FEQ_ERR_UNSUPPORTED, "more than 2^31-1 edges");
    const size_t lds = sizeof(T) * L->cin * L->din;
    if (lds > 64 * 1024) return fail(FEQ_ERR_UNSUPPORTED, "Cin*Din too large for this kernel");
    auto k = k_bd_fwd<T>;
    FEQ_LAUNCH("k_bd_fwd", k, dim3(E), dim3(kThreads), lds, stream_of(stream), *L, *b, x, table,
               dist, y);
    return FEQ_OK;
}

template <class T>
int blockdiag_bwd(const feq_layout* L, const feq_binning* b, int64_t E, const T* gy, const T* x,
                  const T* table, const T* dist, T* gx, T* gtable, T* gdist, void* ws,
                  size_t ws_bytes, feq_stream_t stream) {
    if (int rc = check_layout(L)) return rc;
    if (int rc = check_binning(b)) return rc;
    if (E < 0) return fail(FEQ_ERR_INVALID, "negative edge count");
    if (!gtable) return fail(FEQ_ERR_INVALID, "grad_table is NULL");
    hipStream_t s = stream_of(stream);
    const int64_t tsize = static_cast<int64_t>(b->num_bins + 1) * L->cout * L->cin * L->wdim;
    if (E == 0) {
        auto z = k_fill_zero_t<T>;
        const int64_t blocks = ceil_div(tsize, 256) < 4096 ? ceil_div(tsize, 256) : 4096;
        FEQ_LAUNCH("k_fill_zero", z, dim3(blocks), dim3(256), 0, s, gtable, tsize);
        return FEQ_OK;
    }
    if (!gy || !x || !table || !dist || !gx) return fail(FEQ_ERR_INVALID, "NULL pointer");
    if (E > 0x7fffffffLL) return fail(FEQ_ERR_UNSUPPORTED, "more than 2^31-1 edges");
    if (!ws || ws_bytes < bin_ws_bytes(*b, E))
        return fail(FEQ_ERR_WORKSPACE, "block-diagonal workspace too small");
    const size_t lds_x = sizeof(T) * L->cout * L->dout;
    const size_t lds_r = sizeof(T) * (L->cin * L->din + L->cout * L->dout);
    if (lds_r > 64 * 1024) return fail(FEQ_ERR_UNSUPPORTED, "channel*dim too large for this kernel");
    int ob, ib;
    table_slices(*L, sizeof(T), ob, ib);
    const size_t lds_t = table_lds<T>(*L, ob, ib);
    if (lds_t > 64 * 1024) return fail(FEQ_ERR_UNSUPPORTED, "representation too large for this kernel");
    // the edges grouped by lower bin
    Carver cv(ws);
    int64_t* lo = cv.take<int64_t>(E);
    int32_t* perm = cv.take<int32_t>(E);
    int32_t* offsets = cv.take<int32_t>(b->num_bins + 1);
    void* csr_ws = cv.take<char>(feq_csr_workspace(E, b->num_bins));
    auto kb = k_bd_bins<T>;
    FEQ_LAUNCH("k_bd_bins", kb, dim3(ceil_div(E, 256)), dim3(256), 0, s, *b, E, dist, lo);
    if (int rc = feq_csr_by_dst(lo, E, b->num_bins, perm, offsets, csr_ws,
                                feq_csr_workspace(E, b->num_bins), stream))
        return rc;
    auto kx = k_bd_bwd_x<T>;
    FEQ_LAUNCH("k_bd_bwd_x", kx, dim3(E), dim3(kThreads), lds_x, s, *L, *b, gy, table, dist, gx);
    const int nslices = static_cast<int>(ceil_div(L->cout, ob) * ceil_div(L->cin, ib));
    auto kt = k_bd_bwd_table<T>;
    FEQ_LAUNCH("k_bd_bwd_table", kt, dim3(b->num_bins + 1, nslices), dim3(kThreads), lds_t, s, *L,
               *b, E, gy, x, dist, perm, offsets, ob, ib, gtable);
    if (gdist) {
        auto kr = k_bd_bwd_r<T>;
        FEQ_LAUNCH("k_bd_bwd_r", kr, dim3(E), dim3(kThreads), lds_r, s, *L, *b, gy, x, table, dist,
                   gdist);
    }
    return FEQ_OK;
}

__global__ void k_fill_zero(float* __restrict__ p, int64_t n) {
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x)
        p[i] = 0.0f;
}

}  // namespace

int fill_zero(float* p, int64_t n, hipStream_t s) {
    if (n <= 0) return FEQ_OK;
    const int64_t blocks = ceil_div(n, 256) < 4096 ? ceil_div(n, 256) : 4096;
    FEQ_LAUNCH("k_fill_zero", k_fill_zero, dim3(blocks), dim3(256), 0, s, p, n);
    return FEQ_OK;
}

}  // namespace feq

using namespace feq;

extern "C" size_t feq_blockdiag_workspace(const feq_layout* L, const feq_binning* b, int64_t E) {
    if (!L || !b || E <= 0) return 0;
    return bin_ws_bytes(*b, E);
}

extern "C" int feq_blockdiag_fwd(const feq_layout* L, const feq_binning* b, int64_t E,
                                 const float* x, const float* table, const float* dist, float* y,
                                 void*, size_t, feq_stream_t stream) {
    return blockdiag_fwd<float>(L, b, E, x, table, dist, y, stream);
}

extern "C" int feq_blockdiag_bwd(const feq_layout* L, const feq_binning* b, int64_t E,
                                 const float* gy, const float* x, const float* table,
                                 const float* dist, float* gx, float* gtable, float* gdist,
                                 void* ws, size_t ws_bytes, feq_stream_t stream) {
    return blockdiag_bwd<float>(L, b, E, gy, x, table, dist, gx, gtable, gdist, ws, ws_bytes, stream);
}

extern "C" int feq_blockdiag_fwd_f64(const feq_layout* L, const feq_binning* b, int64_t E,
                                     const double* x, const double* table, const double* dist,
                                     double* y, feq_stream_t stream) {
    return blockdiag_fwd<double>(L, b, E, x, table, dist, y, stream);
}

extern "C" int feq_blockdiag_bwd_f64(const feq_layout* L, const feq_binning* b, int64_t E,
                                     const double* gy, const double* x, const double* table,
                                     const double* dist, double* gx, double* gtable, double* gdist,
                                     void* ws, size_t ws_bytes, feq_stream_t stream) {
    return blockdiag_bwd<double>(L, b, E, gy, x, table, dist, gx, gtable, gdist, ws, ws_bytes,
                                 stream);
}

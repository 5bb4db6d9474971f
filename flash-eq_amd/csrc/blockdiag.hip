// Generic block-diagonal radial mix (the reference's pybind forward/backward).
//
// Features and outputs are in the m-first basis; the radial table has the
// reference layout (num_bins+1, Cout, Cin, Wdim).  Semantics follow
// block_diagonal.cu:558-1161 (see flasheq.h for the entry points):
//   y[e,co,slot] = sum_{ci,i} lerp_t(T)[co,ci,w(o,i)] s^(l_i+l_o) x[e,ci,slot_i]
// with the 2x2 [[a, b], [-b, a]] structure on (+m, -m) pairs for m > 0.
//
// One workgroup per edge; the edge's input (or output gradient) row is staged
// in LDS and every thread produces whole outputs, so there are no atomics
// except the table-gradient scatter.
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

__global__ void __launch_bounds__(kThreads)
k_bd_fwd(feq_layout L, feq_binning B, const float* __restrict__ x,
         const float* __restrict__ table, const float* __restrict__ dist,
         float* __restrict__ y) {
    extern __shared__ float sx[];  // (cin, din) of this edge
    const int64_t e = blockIdx.x;
    const int cin = L.cin, din = L.din, cout = L.cout, dout = L.dout, wd = L.wdim;
    for (int q = threadIdx.x; q < cin * din; q += kThreads) sx[q] = x[e * cin * din + q];
    __syncthreads();
    const float r = dist[e];
    const EdgeBin eb = edge_bin(r, B);
    const float t = eb.t;
    const float sw = r / (r + B.sh_scale);
    const int64_t tstride = static_cast<int64_t>(cout) * cin * wd;
    const float* tlo = table + eb.lo * tstride;
    const float* thi = tlo + tstride;
    for (int q = threadIdx.x; q < cout * dout; q += kThreads) {
        const int co = q / dout, slot = q % dout;
        const SlotRef s = find_out_slot(L, slot);
        float acc = 0.0f;
        if (s.blk >= 0) {
            const int m = L.blk[s.blk][0], ni = L.blk[s.blk][1];
            const int in_off = L.blk[s.blk][3], w_off = L.blk[s.blk][5];
            const int lo_l = L.lslot_out[slot];
            for (int i = 0; i < ni; ++i) {
                const int islot = in_off + (m == 0 ? i : 2 * i);
                const float sc = ipowf(sw, lo_l + L.lslot_in[islot]);
                const int64_t wb = static_cast<int64_t>(co) * cin * wd;
                if (m == 0) {
                    const int w = w_off + s.o * ni + i;
                    for (int ci = 0; ci < cin; ++ci) {
                        const int64_t a = wb + static_cast<int64_t>(ci) * wd + w;
                        acc += lerp_bins(tlo[a], thi[a], t) * sc * sx[ci * din + islot];
                    }
                } else {
                    const int w = w_off + 2 * (s.o * ni + i);
                    for (int ci = 0; ci < cin; ++ci) {
                        const int64_t a = wb + static_cast<int64_t>(ci) * wd + w;
                        const float wa = lerp_bins(tlo[a], thi[a], t) * sc;
                        const float wb2 = lerp_bins(tlo[a + 1], thi[a + 1], t) * sc;
                        const float fr = sx[ci * din + islot], fi = sx[ci * din + islot + 1];
                        acc += s.c == 0 ? (wa * fr + wb2 * fi) : (wa * fi - wb2 * fr);
                    }
                }
            }
        }
        y[e * cout * dout + q] = acc;
    }
}

__global__ void __launch_bounds__(kThreads)
k_bd_bwd_x(feq_layout L, feq_binning B, const float* __restrict__ gy,
           const float* __restrict__ table, const float* __restrict__ dist,
           float* __restrict__ gx) {
    extern __shared__ float sg[];  // (cout, dout) gradient row of this edge
    const int64_t e = blockIdx.x;
    const int cin = L.cin, din = L.din, cout = L.cout, dout = L.dout, wd = L.wdim;
    for (int q = threadIdx.x; q < cout * dout; q += kThreads) sg[q] = gy[e * cout * dout + q];
    __syncthreads();
    const float r = dist[e];
    const EdgeBin eb = edge_bin(r, B);
    const float t = eb.t;
    const float sw = r / (r + B.sh_scale);
    const int64_t tstride = static_cast<int64_t>(cout) * cin * wd;
    const float* tlo = table + eb.lo * tstride;
    const float* thi = tlo + tstride;
    for (int q = threadIdx.x; q < cin * din; q += kThreads) {
        const int ci = q / din, slot = q % din;
        const SlotRef s = find_in_slot(L, slot);
        float acc = 0.0f;
        if (s.blk >= 0) {
            const int m = L.blk[s.blk][0], ni = L.blk[s.blk][1], no = L.blk[s.blk][2];
            const int out_off = L.blk[s.blk][4], w_off = L.blk[s.blk][5];
            const int li = L.lslot_in[slot];
            for (int o = 0; o < no; ++o) {
                const int oslot = out_off + (m == 0 ? o : 2 * o);
                const float sc = ipowf(sw, li + L.lslot_out[oslot]);
                if (m == 0) {
                    const int w = w_off + o * ni + s.o;
                    for (int co = 0; co < cout; ++co) {
                        const int64_t a = (static_cast<int64_t>(co) * cin + ci) * wd + w;
                        acc += lerp_bins(tlo[a], thi[a], t) * sc * sg[co * dout + oslot];
                    }
                } else {
                    const int w = w_off + 2 * (o * ni + s.o);
                    for (int co = 0; co < cout; ++co) {
                        const int64_t a = (static_cast<int64_t>(co) * cin + ci) * wd + w;
                        const float wa = lerp_bins(tlo[a], thi[a], t) * sc;
                        const float wb2 = lerp_bins(tlo[a + 1], thi[a + 1], t) * sc;
                        const float gr = sg[co * dout + oslot], gi = sg[co * dout + oslot + 1];
                        acc += s.c == 0 ? (wa * gr - wb2 * gi) : (wb2 * gr + wa * gi);
                    }
                }
            }
        }
        gx[e * cin * din + q] = acc;
    }
}

__device__ __forceinline__ float block_sum(float v, float* red) {
    for (int off = 32; off > 0; off >>= 1) v += __shfl_down(v, off, 64);
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[wid] = v;
    __syncthreads();
    float s = 0.0f;
    if (threadIdx.x == 0)
        for (int w = 0; w < kThreads / 64; ++w) s += red[w];
    return s;
}

// Table gradient (atomic scatter into rows lo and lo+1) and distance gradient.
__global__ void __launch_bounds__(kThreads)
k_bd_bwd_t(feq_layout L, feq_binning B, const float* __restrict__ gy,
           const float* __restrict__ x, const float* __restrict__ table,
           const float* __restrict__ dist, float* __restrict__ gtable,
           float* __restrict__ gdist) {
    extern __shared__ float sm[];
    const int64_t e = blockIdx.x;
    const int cin = L.cin, din = L.din, cout = L.cout, dout = L.dout, wd = L.wdim;
    float* sx = sm;
    float* sg = sm + cin * din;
    __shared__ float red[kThreads / 64];
    for (int q = threadIdx.x; q < cin * din; q += kThreads) sx[q] = x[e * cin * din + q];
    for (int q = threadIdx.x; q < cout * dout; q += kThreads) sg[q] = gy[e * cout * dout + q];
    __syncthreads();
    const float r = dist[e];
    const EdgeBin eb = edge_bin(r, B);
    const float t = eb.t, omt = 1.0f - eb.t;
    const float sigma = B.sh_scale;
    const float sw = r / (r + sigma);
    const float deriv = sigma / (r * (r + sigma));
    const int64_t tstride = static_cast<int64_t>(cout) * cin * wd;
    const float* tlo = table + eb.lo * tstride;
    const float* thi = tlo + tstride;
    float* glo = gtable + eb.lo * tstride;
    float* ghi = glo + tstride;
    float acc_t = 0.0f, acc_s = 0.0f;
    const int64_t nw = tstride;
    for (int64_t q = threadIdx.x; q < nw; q += kThreads) {
        const int w = static_cast<int>(q % wd);
        const int ci = static_cast<int>((q / wd) % cin);
        const int co = static_cast<int>(q / (static_cast<int64_t>(wd) * cin));
        // locate the m-block of weight w
        int k = L.nblocks - 1;
        while (k > 0 && w < L.blk[k][5]) --k;
        const int m = L.blk[k][0], ni = L.blk[k][1];
        const int in_off = L.blk[k][3], out_off = L.blk[k][4], w_off = L.blk[k][5];
        const int rel = w - w_off;
        float gw, unscaled;
        int Lsum;
        if (m == 0) {
            const int o = rel / ni, i = rel % ni;
            const int is = in_off + i, os = out_off + o;
            Lsum = L.lslot_in[is] + L.lslot_out[os];
            unscaled = sx[ci * din + is] * sg[co * dout + os];
        } else {
            const int pair = rel >> 1, isb = rel & 1;
            const int o = pair / ni, i = pair % ni;
            const int is = in_off + 2 * i, os = out_off + 2 * o;
            Lsum = L.lslot_in[is] + L.lslot_out[os];
            const float fr = sx[ci * din + is], fi = sx[ci * din + is + 1];
            const float gr = sg[co * dout + os], gi = sg[co * dout + os + 1];
            unscaled = isb == 0 ? (fr * gr + fi * gi) : (fi * gr - fr * gi);
        }
        const float sc = ipowf(sw, Lsum);
        gw = sc * unscaled;
        atomicAdd(&glo[q], omt * gw);
        atomicAdd(&ghi[q], t * gw);
        if (gdist) {
            const float wl = tlo[q], wh = thi[q];
            acc_t += (wh - wl) * gw;
            if (Lsum > 0) acc_s += lerp_bins(wl, wh, t) * unscaled * sc * static_cast<float>(Lsum) * deriv;
        }
    }
    if (gdist) {
        const float st = block_sum(acc_t, red);
        const float ss = block_sum(acc_s, red);
        if (threadIdx.x == 0) gdist[e] = st * eb.dtdr + ss;
    }
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

extern "C" size_t feq_blockdiag_workspace(const feq_layout*, const feq_binning*, int64_t) {
    return 0;
}

extern "C" int feq_blockdiag_fwd(const feq_layout* L, const feq_binning* b, int64_t E,
                                 const float* x, const float* table, const float* dist, float* y,
                                 void*, size_t, feq_stream_t stream) {
    if (int rc = check_layout(L)) return rc;
    if (int rc = check_binning(b)) return rc;
    if (E < 0) return fail(FEQ_ERR_INVALID, "negative edge count");
    if (E == 0) return FEQ_OK;
    if (!x || !table || !dist || !y) return fail(FEQ_ERR_INVALID, "NULL pointer");
    if (E > 0x7fffffffLL) return fail(FEQ_ERR_UNSUPPORTED, "more than 2^31-1 edges");
    const size_t lds = sizeof(float) * L->cin * L->din;
    if (lds > 64 * 1024) return fail(FEQ_ERR_UNSUPPORTED, "Cin*Din too large for this kernel");
    FEQ_LAUNCH("k_bd_fwd", k_bd_fwd, dim3(E), dim3(kThreads), lds, stream_of(stream), *L, *b, x,
                       table, dist, y);
    return FEQ_OK;
}

extern "C" int feq_blockdiag_bwd(const feq_layout* L, const feq_binning* b, int64_t E,
                                 const float* gy, const float* x, const float* table,
                                 const float* dist, float* gx, float* gtable, float* gdist,
                                 void*, size_t, feq_stream_t stream) {
    if (int rc = check_layout(L)) return rc;
    if (int rc = check_binning(b)) return rc;
    if (E < 0) return fail(FEQ_ERR_INVALID, "negative edge count");
    if (!gtable) return fail(FEQ_ERR_INVALID, "grad_table is NULL");
    hipStream_t s = stream_of(stream);
    const int64_t tsize = static_cast<int64_t>(b->num_bins + 1) * L->cout * L->cin * L->wdim;
    if (int rc = fill_zero(gtable, tsize, s)) return rc;
    if (E == 0) return FEQ_OK;
    if (!gy || !x || !table || !dist || !gx) return fail(FEQ_ERR_INVALID, "NULL pointer");
    if (E > 0x7fffffffLL) return fail(FEQ_ERR_UNSUPPORTED, "more than 2^31-1 edges");
    const size_t lds_x = sizeof(float) * L->cout * L->dout;
    const size_t lds_t = sizeof(float) * (L->cin * L->din + L->cout * L->dout);
    if (lds_t > 64 * 1024) return fail(FEQ_ERR_UNSUPPORTED, "channel*dim too large for this kernel");
    FEQ_LAUNCH("k_bd_bwd_x", k_bd_bwd_x, dim3(E), dim3(kThreads), lds_x, s, *L, *b, gy, table, dist, gx);
    FEQ_LAUNCH("k_bd_bwd_t", k_bd_bwd_t, dim3(E), dim3(kThreads), lds_t, s, *L, *b, gy, x, table, dist,
                       gtable, gdist);
    return FEQ_OK;
}

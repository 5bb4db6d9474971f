// Library-level C ABI: errors, version, layout construction, edge binning.
#include "feq_internal.h"

#include <cstdlib>
#include <cstring>

namespace feq {

static thread_local std::string g_last_error;

void set_error(const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
}

int fail(int code, const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

int check_layout(const feq_layout* L) {
    if (!L) return fail(FEQ_ERR_INVALID, "layout is NULL");
    if (L->cin <= 0 || L->cout <= 0 || L->din <= 0 || L->dout <= 0 || L->wdim <= 0)
        return fail(FEQ_ERR_INVALID, "layout has non-positive sizes");
    if (L->din > FEQ_MAX_SLOTS || L->dout > FEQ_MAX_SLOTS)
        return fail(FEQ_ERR_UNSUPPORTED, "representation dimension exceeds %d", FEQ_MAX_SLOTS);
    if (L->nblocks <= 0 || L->nblocks > FEQ_MAX_BLOCKS)
        return fail(FEQ_ERR_INVALID, "layout has %d m-blocks", L->nblocks);
    return FEQ_OK;
}

int ew_path() {
    const char* g = getenv("FEQ_FORCE_GENERIC");
    if (g && g[0] == '1') return kPathGeneric;
    const char* v = getenv("FEQ_EW_PATH");
    if (!v) return kPathSplit;
    if (strcmp(v, "generic") == 0) return kPathGeneric;
    return kPathSplit;
}

bool force_generic() { return ew_path() == kPathGeneric; }

int check_binning(const feq_binning* b) {
    if (!b) return fail(FEQ_ERR_INVALID, "binning is NULL");
    if (b->num_bins < 1) return fail(FEQ_ERR_INVALID, "num_bins must be >= 1");
    return FEQ_OK;
}

}  // namespace feq

using namespace feq;

extern "C" const char* feq_last_error(void) { return g_last_error.c_str(); }

extern "C" int feq_abi_version(void) { return 1; }

extern "C" int feq_layout_init(feq_layout* out, const int32_t* lvals_in, int32_t n_in,
                               const int32_t* lvals_out, int32_t n_out, int32_t cin,
                               int32_t cout) {
    if (!out || !lvals_in || !lvals_out) return fail(FEQ_ERR_INVALID, "NULL argument");
    if (n_in < 1 || n_out < 1) return fail(FEQ_ERR_INVALID, "lvals must be non-empty");
    if (n_in > FEQ_MAX_IRREPS || n_out > FEQ_MAX_IRREPS)
        return fail(FEQ_ERR_UNSUPPORTED, "more than %d irreps in a representation", FEQ_MAX_IRREPS);
    if (cin < 1 || cout < 1) return fail(FEQ_ERR_INVALID, "multiplicities must be positive");
    std::memset(out, 0, sizeof(*out));
    int mmax = 0, din = 0, dout = 0, wdim = 0;
    for (int i = 0; i < n_in; ++i) {
        if (lvals_in[i] < 0) return fail(FEQ_ERR_INVALID, "negative degree");
        mmax = lvals_in[i] > mmax ? lvals_in[i] : mmax;
        din += 2 * lvals_in[i] + 1;
    }
    for (int i = 0; i < n_out; ++i) {
        if (lvals_out[i] < 0) return fail(FEQ_ERR_INVALID, "negative degree");
        mmax = lvals_out[i] > mmax ? lvals_out[i] : mmax;
        dout += 2 * lvals_out[i] + 1;
    }
    if (mmax >= FEQ_MAX_BLOCKS)
        return fail(FEQ_ERR_UNSUPPORTED,
                    "Maximum l-value (%d) exceeds supported limit (%d).", mmax, FEQ_MAX_BLOCKS - 1);
    if (din > FEQ_MAX_SLOTS || dout > FEQ_MAX_SLOTS)
        return fail(FEQ_ERR_UNSUPPORTED, "representation dimension exceeds %d", FEQ_MAX_SLOTS);
    for (int i = 0; i < n_in; ++i)
        for (int j = 0; j < n_out; ++j) {
            int a = lvals_in[i], b = lvals_out[j];
            wdim += 2 * (a < b ? a : b) + 1;
        }
    // m-first slots: every irrep's m=0 component, then for m = 1.. the
    // (+m, -m) pair of every irrep with l >= m, in lvals order.
    int in_off = 0, out_off = 0, w_off = 0, nb = 0;
    for (int m = 0; m <= mmax; ++m) {
        int ni = 0, no = 0;
        for (int i = 0; i < n_in; ++i) ni += lvals_in[i] >= m;
        for (int i = 0; i < n_out; ++i) no += lvals_out[i] >= m;
        if (ni == 0 || no == 0) continue;
        int* b = out->blk[nb++];
        b[0] = m; b[1] = ni; b[2] = no; b[3] = in_off; b[4] = out_off; b[5] = w_off;
        int k = m == 0 ? 1 : 2;
        in_off += k * ni;
        out_off += k * no;
        w_off += k * ni * no;
    }
    if (w_off != wdim) return fail(FEQ_ERR_INVALID, "internal: weight count mismatch");
    // per-slot degrees over the full m-first order (slots of m-blocks that are
    // empty on the other side are still present in the feature vector)
    int s = 0;
    for (int m = 0; m <= mmax; ++m)
        for (int i = 0; i < n_in; ++i)
            if (lvals_in[i] >= m)
                for (int c = 0; c < (m == 0 ? 1 : 2); ++c) out->lslot_in[s++] = (int8_t)lvals_in[i];
    s = 0;
    for (int m = 0; m <= mmax; ++m)
        for (int i = 0; i < n_out; ++i)
            if (lvals_out[i] >= m)
                for (int c = 0; c < (m == 0 ? 1 : 2); ++c) out->lslot_out[s++] = (int8_t)lvals_out[i];
    int lmax_in = 0, lmax_out = 0;
    for (int i = 0; i < n_in; ++i) lmax_in = lvals_in[i] > lmax_in ? lvals_in[i] : lmax_in;
    for (int i = 0; i < n_out; ++i) lmax_out = lvals_out[i] > lmax_out ? lvals_out[i] : lmax_out;
    out->cin = cin;
    out->cout = cout;
    out->din = din;
    out->dout = dout;
    out->wdim = wdim;
    out->nblocks = nb;
    out->has_lpos = (lmax_in + lmax_out) > 0;
    return FEQ_OK;
}

__global__ void k_bin_edges(feq_binning b, int64_t n, const float* __restrict__ r,
                            int32_t* __restrict__ lo, float* __restrict__ t) {
    int64_t e = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
    if (e >= n) return;
    EdgeBin s = edge_bin(r[e], b);
    lo[e] = s.lo;
    t[e] = s.t;
}

extern "C" int feq_bin_edges(const feq_binning* b, int64_t n, const float* dist, int32_t* lo,
                             float* t, feq_stream_t stream) {
    if (int rc = check_binning(b)) return rc;
    if (n < 0) return fail(FEQ_ERR_INVALID, "negative edge count");
    if (n == 0) return FEQ_OK;
    if (!dist || !lo || !t) return fail(FEQ_ERR_INVALID, "NULL pointer");
    const int threads = 256;
    FEQ_LAUNCH("k_bin_edges", k_bin_edges, dim3(ceil_div(n, threads)), dim3(threads), 0,
                       stream_of(stream), *b, n, dist, lo, t);
    return FEQ_OK;
}

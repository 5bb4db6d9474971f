// Internal helpers shared by the HIP translation units of libflasheq.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>

#include "flasheq.h"

namespace feq {

// ---- error reporting ---------------------------------------------------------
void set_error(const char* fmt, ...);
int fail(int code, const char* fmt, ...);

#define FEQ_HIP(call)                                                              \
    do {                                                                           \
        hipError_t e_ = (call);                                                    \
        if (e_ != hipSuccess)                                                      \
            return ::feq::fail(FEQ_ERR_HIP, "%s failed: %s", #call,                \
                               hipGetErrorString(e_));                             \
    } while (0)

#define FEQ_LAUNCH_CHECK(name)                                                     \
    do {                                                                           \
        hipError_t e_ = hipGetLastError();                                         \
        if (e_ != hipSuccess)                                                      \
            return ::feq::fail(FEQ_ERR_HIP, "launch of %s failed: %s", name,       \
                               hipGetErrorString(e_));                             \
    } while (0)

inline hipStream_t stream_of(feq_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

// Brackets one launch with timing events while feq_profile_enable(1) is in
// effect (profile.hip); otherwise does nothing.
class ProfScope {
   public:
    ProfScope(const char* name, hipStream_t s);
    ~ProfScope();
    ProfScope(const ProfScope&) = delete;
    ProfScope& operator=(const ProfScope&) = delete;

   private:
    const char* name_;
    hipStream_t s_;
    hipEvent_t a_;
};

// hipLaunchKernelGGL plus the profiling bracket and the launch-error check;
// returns from the enclosing function on a launch error.  `kern` must be a
// single token (bind template instantiations to a variable first).
#define FEQ_LAUNCH(name, kern, grid, block, lds, stream, ...)                      \
    do {                                                                           \
        {                                                                          \
            ::feq::ProfScope ps_(name, stream);                                    \
            hipLaunchKernelGGL(kern, grid, block, lds, stream, __VA_ARGS__);       \
        }                                                                          \
        FEQ_LAUNCH_CHECK(name);                                                    \
    } while (0)

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Zero-fill by kernel (never hipMemsetAsync: callers may capture the stream).
int fill_zero(float* p, int64_t n, hipStream_t s);

// Tail shared by the fused backward kernels (edgewise_tail.hip): binned
// radial-function gradient from dF_e (E, K wdim), distance gradient (gdist may
// be NULL), and the sums of `groups` channel-pattern partials of ncc floats.
// Deterministic sum of `groups` partial arrays of n floats into out (tmp holds
// ceil(groups / 32) * n floats when groups > 32).
int reduce_partials(const float* part, int groups, int64_t n, float* out, float* tmp,
                    hipStream_t s);

// Several reduce_partials in one launch when each is a few sums of many
// partials (n <= 256, groups > 32; otherwise one call each), with the same
// summation order, so the results are bitwise those of separate calls.
struct PartialJob {
    const float* part;
    int groups;
    int64_t n;
    float* out;
    float* tmp;
};
constexpr int kMaxPartialJobs = 4;
int reduce_partials_multi(const PartialJob* jobs, int njobs, hipStream_t s);

// `tail` holds ew_tail_floats(...) floats of workspace.  groups = 0: no dC partials.
bool ew_tail_supported(const feq_binning& B, int kw);
size_t ew_tail_floats(const feq_binning& B, int kw, int64_t E, int groups, int64_t ncc);
int ew_tail(const feq_layout& L, const feq_binning& B, int K, int64_t E, const float* dist,
            const float* F, const float* dFe, const float* dCp, int groups, int64_t ncc, float* gC,
            float* gF, float* gdist, float* tail, hipStream_t s);

// The input gradient of the message-passing form summed per source node inside
// the input-gradient kernel.  Tiles walk the edges in source order (perm,
// offsets: the CSR by source over the nsrc nodes); a tile sums its rows per
// node in tile order.  A node whose edges lie in one tile gets its row written
// by that tile; a node whose edges cross a tile boundary leaves one partial row
// per tile in part[(tile, slot)] (slot 0: the tile's first node, slot 1: its
// last), summed in tile order by a fix-up kernel, which also zeroes the rows of
// nodes without edges.  The same bits on every run, no atomics.
struct NodeScatter {
    const int32_t* perm;
    const int32_t* offsets;
    float* out;    // (nsrc, Cin, Din)
    float* part;   // (ntiles, 2, Cin, Din), carved from the backward's workspace
    // by CSR position p (edge perm[p]), formed per call in the workspace so that
    // the kernel's tile loads index them directly: the source row (-1 outside
    // [0, nsrc)), the distance and, for the pooled form, the destination
    const int32_t* src_pos;
    const float* dist_pos;
    const int32_t* dnode_pos;
};

// The V projection of attention fused with the attention's head weighting and
// sum pooling (attention.py:307-314 with pooling.py:21-30).  The forward walks
// the edges in destination order (perm, offsets: the CSR by destination over
// ndst nodes) and sums attn[e, head(c)] y_e[c, :] per destination node, a
// node crossing a tile boundary leaving partial rows as in NodeScatter; y_e is
// never written unless the caller keeps it (in destination order) for the
// backward.  The backward reads gy_e[c, :] = attn[e, head(c)] gout[dst[e], c, :]
// where the unfused form reads the per-edge gradient, so that is never formed
// either.  head(c) = min(c / hc, heads - 1); edges whose destination lies
// outside [0, ndst) add nothing and get a zero gradient.
constexpr int kPoolMaxHeads = 16;
struct DstPool {
    const int32_t* perm;
    const int32_t* offsets;
    const int64_t* dst;
    const float* attn;   // (E, heads)
    int64_t ndst;
    int heads;
    int hc;              // channels per head
    float* out;          // forward: (ndst, Cout, Dout)
    float* part;         // forward: (ntiles, 2, Cout, Dout), carved from the workspace
    const int64_t* src_pos;   // forward: src[perm[p]] by CSR position, formed per call
    const int32_t* node_pos;  // forward: destination by CSR position (-1 outside [0, ndst))
    const float* dist_pos;    // forward: distance by CSR position
};

// Gradients for the bases on the split kernels, with y = m Q^T and f = x P (m:
// the block-diagonal output before the rotation): the forward writes m to
// ym_out (E, Cout, Dout) in edge order when it is not NULL; the backward reads
// it back from ym and writes gQ (E, Dout, Dout) = gy^T m and gP (E, Din, Din) =
// x^T dL/df per edge when they are not NULL.
struct BasisGrads {
    float* ym_out;
    const float* ym;
    float* gP;
    float* gQ;
};

// Split-fp16 fast paths (edgewise_split.hip); -1 when the shape has none.
size_t ew_split_workspace(const feq_layout& L, int rank);
// nodes: with the per-node sums (NodeScatter partial rows).
size_t ew_split_bwd_workspace(const feq_layout& L, const feq_binning& B, int rank, int64_t E,
                              bool nodes);
// src (may be NULL): message-passing form, edge e reads row src[e] of the node
// table x (nsrc rows; indices outside [0, nsrc) read zeros).  ns (may be NULL,
// needs src): the input gradient summed per source node into ns->out instead
// of per edge into gx.  lp (message-passing form only, else ignored): one fp16
// product per operand pair instead of the three of the hi/lo split.
int ew_split_bwd(const feq_layout& L, const feq_binning& B, int rank, int64_t E, const float* gy,
                 const float* x, const int64_t* src, int64_t nsrc, const float* P, const float* Q,
                 const float* dist, const float* C, const float* F, float* gx, float* gC, float* gF,
                 float* gdist, const NodeScatter* ns, void* ws, size_t ws_bytes, bool lp, hipStream_t s,
                 const DstPool* dp = nullptr, const BasisGrads* bg = nullptr);
// dp (may be NULL, needs src): the pooled form; y then receives the per-edge
// rows in destination order, or is NULL.
int ew_split_fwd(const feq_layout& L, const feq_binning& B, int rank, int64_t E, const float* x,
                 const int64_t* src, int64_t nsrc, const float* P, const float* Q, const float* dist,
                 const float* C, const float* F, float* y, void* ws, size_t ws_bytes, bool lp,
                 hipStream_t s, const DstPool* dp = nullptr, const BasisGrads* bg = nullptr);
bool ew_split_supported(const feq_layout& L, const feq_binning& B, int rank, bool backward);
// Layouts whose split kernels form the bases' gradients (BasisGrads): the
// split shapes with a backward, not the scalar-output family.
bool ew_split_pq_supported(const feq_layout& L, const feq_binning& B, int rank);
// Layouts with the pooled form (the split shapes with Cin = 64, not the
// scalar-output family) and its forward workspace.
bool ew_pool_supported(const feq_layout& L, const feq_binning& B, int rank);
size_t ew_pool_fwd_workspace(const feq_layout& L, int rank, int64_t E);
// Rows of the nodes that the per-node sums of a tile walk did not write (nodes
// crossing 16-edge tile boundaries: their partial rows summed in tile order;
// nodes without edges: zeros).  row4 = Cin Din / 4.
int node_fix(const NodeScatter& ns, int64_t nsrc, int64_t row4, hipStream_t s);

// Scalar-output family (edgewise_scalar.hip): lvals_out = [0], Cin = 64, rank 4,
// reached through the split family's entry points above.
bool ew0_supported(const feq_layout& L, int rank);
size_t ew0_bwd_workspace(const feq_layout& L, const feq_binning& B, int rank, int64_t E, bool nodes);
int ew0_fwd(const feq_layout& L, const feq_binning& B, int rank, int64_t E, const float* x,
            const int64_t* src, int64_t nsrc, const float* P, const float* Q, const float* dist,
            const float* C, const float* F, float* y, float* ym, hipStream_t s);
int ew0_bwd(const feq_layout& L, const feq_binning& B, int rank, int64_t E, const float* gy,
            const float* x, const int64_t* src, int64_t nsrc, const float* P, const float* Q,
            const float* dist, const float* C, const float* F, float* gx, float* gC, float* gF,
            float* gdist, const NodeScatter* ns, void* ws, size_t ws_bytes, hipStream_t s,
            const float* ym = nullptr, float* gP = nullptr, float* gQ = nullptr);

// Kernel family of the fused edgewise layer.  The default tries the split-fp16
// kernels, then the shape-generic ones; FEQ_EW_PATH=generic (or
// FEQ_FORCE_GENERIC=1) uses only the generic ones, so tests can check the
// implementations against each other.
enum { kPathSplit = 0, kPathGeneric = 2 };
int ew_path();
bool force_generic();

// Checks shared by every layout-consuming entry point.
int check_layout(const feq_layout* L);
int check_binning(const feq_binning* b);

// Carves consecutive 256-byte aligned regions out of a caller workspace.
struct Carver {
    char* base;
    size_t used = 0;
    explicit Carver(void* p) : base(static_cast<char*>(p)) {}
    template <class T>
    T* take(size_t n) {
        used = align_up(used, 256);
        T* p = reinterpret_cast<T*>(base ? base + used : nullptr);
        used += n * sizeof(T);
        return p;
    }
};

// ---- per-edge distance state ---------------------------------------------------
// Lower bin index lo (hi = lo + 1), interpolation weight t, dt/dr.
// The index is found in float32 exactly as the reference kernel does
// (block_diagonal.cu:82-115): normalized = (r - p1) * p2 (linear) or
// (log(max(r, exp(p1))) - p1) * p2 * nb (log), clamped to [0, nb],
// lo = min(floor(normalized), nb - 1).  Linear t is not clamped (it
// extrapolates outside [min, max]); log t is clamped to <= 1 and r below the
// bin's lower edge maps to t = 0.  dt/dr follows binning_derivative (:121-138).
struct EdgeBin {
    int lo;
    float t;
    float dtdr;
};

// float32 log and exp rounded from float64 (correctly rounded but for values
// within 2^-29 of a rounding boundary): the bin index of a log-binned distance
// then depends on nothing but the float32 inputs, and the CPU oracle's
// float64-then-round restatement reproduces it bit for bit.
__device__ __forceinline__ float cr_logf(float x) { return static_cast<float>(log(static_cast<double>(x))); }
__device__ __forceinline__ float cr_expf(float x) { return static_cast<float>(exp(static_cast<double>(x))); }

// Lower bin index of distance r: the float32 index path of compute_binning.
__device__ __forceinline__ int bin_index(float r, const feq_binning& b) {
    const int nb = b.num_bins;
    float nrm;
    if (b.log_bins) {
        nrm = (cr_logf(fmaxf(r, cr_expf(b.p1))) - b.p1) * b.p2 * static_cast<float>(nb);
    } else {
        nrm = (r - b.p1) * b.p2;
    }
    nrm = fminf(fmaxf(nrm, 0.0f), static_cast<float>(nb));
    const int lo = static_cast<int>(floorf(nrm));
    return lo < nb - 1 ? lo : nb - 1;
}

__device__ __forceinline__ EdgeBin edge_bin(float r, const feq_binning& b) {
    EdgeBin s;
    const int lo = bin_index(r, b);
    s.lo = lo;
    if (b.log_bins) {
        const float ilbw = b.p2 * static_cast<float>(b.num_bins);
        const float log_lo = b.p1 + static_cast<float>(lo) / ilbw;
        const float e_lo = static_cast<float>(exp(static_cast<double>(log_lo)));
        const float e_hi = static_cast<float>(exp(static_cast<double>(log_lo + 1.0f / ilbw)));
        const float c = r > e_lo ? r : e_lo;
        float t = (c - e_lo) / (e_hi - e_lo);
        s.t = t < 1.0f ? t : 1.0f;
        s.dtdr = 1.0f / (e_hi - e_lo);
    } else {
        const float width = 1.0f / b.p2;
        const float e_lo = b.p1 + static_cast<float>(lo) * width;
        s.t = (r - e_lo) / width;
        s.dtdr = b.p2;
    }
    return s;
}

// Interpolated table value (1-t) lo + t hi, evaluated as lo + t (hi - lo):
// identical in exact arithmetic and well conditioned when linear bins
// extrapolate (|t| >> 1 beyond max_dist).
__device__ __forceinline__ float lerp_bins(float lo, float hi, float t) {
    return fmaf(t, hi - lo, lo);
}

// s^l for small non-negative integer l by repeated squaring (as ipow, :202-213).
template <class T>
__device__ __forceinline__ T ipow_t(T base, int e) {
    T r = T(1);
    while (e > 0) {
        if (e & 1) r *= base;
        base *= base;
        e >>= 1;
    }
    return r;
}
__device__ __forceinline__ float ipowf(float base, int e) { return ipow_t<float>(base, e); }

// Bin state with t and dt/dr in the feature precision T (the reference's
// InterpState<scalar_t>): the index in float32, t as compute_binning forms it
// in T (block_diagonal.cu:82-115), dt/dr as binning_derivative (:121-138).
template <class T>
struct EdgeBinT {
    int lo;
    T t;
    T dtdr;
};

template <class T>
__device__ __forceinline__ EdgeBinT<T> edge_bin_t(T r, const feq_binning& b) {
    EdgeBinT<T> s;
    const int lo = bin_index(static_cast<float>(r), b);
    s.lo = lo;
    if (b.log_bins) {
        const T ilbw = static_cast<T>(b.p2 * static_cast<float>(b.num_bins));
        const T log_lo = static_cast<T>(b.p1) + static_cast<T>(lo) / ilbw;
        const T e_lo = static_cast<T>(exp(static_cast<double>(log_lo)));
        const T e_hi = static_cast<T>(exp(static_cast<double>(log_lo + T(1) / ilbw)));
        const T c = r > e_lo ? r : e_lo;
        const T t = (c - e_lo) / (e_hi - e_lo);
        s.t = t < T(1) ? t : T(1);
        s.dtdr = T(1) / (e_hi - e_lo);
    } else {
        const T width = T(1) / static_cast<T>(b.p2);
        const T e_lo = static_cast<T>(b.p1) + static_cast<T>(lo) * width;
        s.t = (r - e_lo) / width;
        s.dtdr = static_cast<T>(b.p2);
    }
    return s;
}

}  // namespace feq

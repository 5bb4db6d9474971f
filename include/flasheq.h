/*
 * flasheq.h -- C ABI of the MI355X (gfx950) equivariant edge hot path.
 *
 * Plain pointers and sizes only.  Every device pointer is caller-owned memory
 * (the Python host side allocates it through PyTorch's caching allocator);
 * the library never allocates device memory.  Every entry point launches on
 * the caller's stream, returns FEQ_OK (0) or an FEQ_ERR_* code, and leaves a
 * human-readable message for feq_last_error() (thread-local).
 *
 * Reference interfaces replaced (paths are in the reference repository):
 *   feq_layout_init          block-layout bookkeeping of precompute_block_info
 *                            (flash_eq/cuda/csrc/block_diagonal.cu:1191-1266) and
 *                            _compute_block_sizes (flash_eq/cuda/block_diagonal.py:181-203)
 *   feq_bin_edges            compute_binning (block_diagonal.cu:82-115), exposed so
 *                            bin ids can be checked bit-exactly
 *   feq_blockdiag_fwd        pybind "forward"  -> block_diagonal_forward_cuda
 *                            (block_diagonal.cu:1268-1282, 1758-1761)
 *   feq_blockdiag_bwd        pybind "backward" -> block_diagonal_backward_cuda
 *                            (block_diagonal.cu:1543-1558, 1758-1761)
 *   feq_blockdiag_*_f64      their float64 dispatch (block_diagonal.cu:1332, 1605)
 *   feq_edgewise_fwd/_bwd    EquivariantEdgewiseLinear.forward = bmm(X,P) ->
 *                            block_diagonal_cuda(rw()) -> bmm(.,Q^T)
 *                            (flash_eq/layers/linear.py:100-160, radial.py:259-275),
 *                            fused, with the radial table kept in its separable
 *                            form T[b,o,i,w] = sum_k C[k,o,i] F[b,k,w]
 *   feq_wigner_basis         WignerDBasis.forward / WignerD.rot_to_ez
 *                            (flash_eq/representations/wigner.py:198-240, 341-370)
 *   feq_wigner_basis_bwd     its autograd backward (matrix_exp's, wigner.py:183)
 *   feq_csr_by_dst           grouping of edges by destination that the scatter
 *                            ops of pooling.py:21-30 / attention.py:124-141 imply
 *   feq_segment_sum          GraphPooling 'sum' forward (flash_eq/layers/pooling.py:21-30)
 *   feq_gather_rows          its backward (index_select of the node gradient)
 *   feq_attn_softmax_fwd/bwd EquivariantEdgeAttention logits + _neighbor_softmax
 *                            (flash_eq/layers/attention.py:92-141), with the Q/K
 *                            gathers of EquivariantAttention.forward
 *                            (attention.py:298-304) inside the kernels
 *   feq_attn_pool_fwd/bwd    _apply_attention + GraphPooling 'sum'
 *                            (flash_eq/layers/attention.py:143-167, pooling.py:21-30)
 *   feq_sepnorm_fwd/bwd      SeparableEquivariantLayerNorm.forward and its autograd
 *                            (flash_eq/layers/norm.py:177-246, 76-112)
 *   feq_eqnorm_fwd/bwd       EquivariantLayerNorm.forward (norm.py:148-174, RepNorm :51-73)
 *   feq_gate_*               EquivariantGating.forward (flash_eq/layers/gating.py:54-76)
 *                            around its nn.Linear, which stays a library GEMM
 *   feq_eqlinear_fwd/bwd_x/bwd_w
 *                            EquivariantLinear.forward and its autograd gradients
 *                            (flash_eq/layers/linear.py:242-268)
 *   feq_scale_add(_bwd)     the block's residual connections with LayerScale
 *                            (flash_eq/layers/transformer.py:23-38, 245, 252)
 *   feq_transpose, feq_column_sums, feq_dot_f64
 *                            PyTorch work inside the reference's modules: layout
 *                            changes around EquivariantLinear (linear.py:242-268),
 *                            bias gradients, scalar-parameter gradients
 */
#ifndef FLASHEQ_H
#define FLASHEQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Opaque stream handle; pass a hipStream_t (torch.cuda.current_stream().cuda_stream). */
typedef void* feq_stream_t;

enum {
    FEQ_OK = 0,
    FEQ_ERR_INVALID = 1,      /* bad argument, shape or size */
    FEQ_ERR_UNSUPPORTED = 2,  /* valid but outside this build's limits */
    FEQ_ERR_HIP = 3,          /* a HIP runtime call failed */
    FEQ_ERR_WORKSPACE = 4     /* workspace missing or too small */
};

#define FEQ_MAX_BLOCKS 17     /* m = 0..16: l <= 16 like the reference (block_diagonal.cu:172) */
#define FEQ_MAX_SLOTS 128     /* components per representation (dim) */
#define FEQ_MAX_IRREPS 32     /* irreps per representation */

/* m-first block layout of one (in_repr, out_repr) pair. */
typedef struct feq_layout {
    int32_t cin, cout;                    /* multiplicities */
    int32_t din, dout;                    /* representation dimensions */
    int32_t wdim;                         /* radial weights per channel pair */
    int32_t nblocks;                      /* non-empty m-blocks */
    int32_t blk[FEQ_MAX_BLOCKS][6];       /* m, n_in, n_out, in_off, out_off, w_off */
    int8_t lslot_in[FEQ_MAX_SLOTS];       /* l of every m-first input component */
    int8_t lslot_out[FEQ_MAX_SLOTS];      /* l of every m-first output component */
    int32_t has_lpos;                     /* any pair with l_in + l_out > 0 */
} feq_layout;

/* Distance binning: p1/p2 are SeparableRadialNet.binning_params() as float32. */
typedef struct feq_binning {
    float p1;          /* min_val (linear) or log(min_val) (log) */
    float p2;          /* num_bins/(max-min) (linear) or 1/log(max/min) (log) */
    int32_t num_bins;  /* table has num_bins + 1 rows */
    int32_t log_bins;  /* 0 linear, 1 logarithmic */
    float sh_scale;    /* solid-harmonic length scale sigma */
} feq_binning;

const char* feq_last_error(void);
int feq_abi_version(void);

/* ---- per-kernel timing (no reference counterpart: the reference times its
 * kernels from Python with CUDA events, scripts/profile_kernels.py:7-76) ------
 * While enabled, every kernel launch is bracketed by two events recorded on its
 * own stream.  feq_profile_summary waits for them and writes one line per
 * kernel, "name<TAB>launches<TAB>total_ms\n", then forgets the records.
 * Process-global, for one host thread. */
int feq_profile_enable(int on);
int feq_profile_summary(char* buf, size_t len);

/* Fill *out from the irrep degrees (host arrays, lvals order, duplicates allowed). */
int feq_layout_init(feq_layout* out, const int32_t* lvals_in, int32_t n_in,
                    const int32_t* lvals_out, int32_t n_out, int32_t cin, int32_t cout);

/* Per-edge lower bin index and interpolation weight t (float32 path). */
int feq_bin_edges(const feq_binning* b, int64_t num_edges, const float* dist,
                  int32_t* lo, float* t, feq_stream_t stream);

/* ---- generic block-diagonal op: table (num_bins+1, Cout, Cin, Wdim) ----------
 * The forward needs no workspace (pass NULL, 0).  The backward needs
 * feq_blockdiag_workspace bytes: it groups the edges by lower bin and sums the
 * table gradient per bin in a fixed order (no atomics: the same bits on every
 * run).  grad_dist may be NULL (not needed).  grad_x, grad_table and
 * grad_dist are overwritten. */
size_t feq_blockdiag_workspace(const feq_layout* L, const feq_binning* b, int64_t num_edges);
int feq_blockdiag_fwd(const feq_layout* L, const feq_binning* b, int64_t num_edges,
                      const float* x, const float* table, const float* dist, float* y,
                      void* workspace, size_t ws_bytes, feq_stream_t stream);
int feq_blockdiag_bwd(const feq_layout* L, const feq_binning* b, int64_t num_edges,
                      const float* grad_y, const float* x, const float* table, const float* dist,
                      float* grad_x, float* grad_table, float* grad_dist,
                      void* workspace, size_t ws_bytes, feq_stream_t stream);
/* The same op in float64: the reference dispatches the kernels on float64 as well
 * (block_diagonal.cu:1332, 1605, AT_DISPATCH_FLOATING_TYPES_AND_HALF); bin
 * indices in float32, t and dt/dr in float64, as its InterpState<double>. */
int feq_blockdiag_fwd_f64(const feq_layout* L, const feq_binning* b, int64_t num_edges,
                          const double* x, const double* table, const double* dist, double* y,
                          feq_stream_t stream);
int feq_blockdiag_bwd_f64(const feq_layout* L, const feq_binning* b, int64_t num_edges,
                          const double* grad_y, const double* x, const double* table,
                          const double* dist, double* grad_x, double* grad_table,
                          double* grad_dist, void* workspace, size_t ws_bytes,
                          feq_stream_t stream);

/* ---- fused EquivariantEdgewiseLinear (separable radial weights) ---------------
 * x (E, Cin, Din) standard basis; P (E, Din, Din); Q (E, Dout, Dout);
 * C (K, Cout, Cin) channel patterns; F (num_bins+1, K, Wdim) radial functions;
 * y (E, Cout, Dout) standard basis.  y = (Lambda(r) (x P)) Q^T.
 * Workspaces: feq_edgewise_fwd_workspace bytes for the forward (it keeps the
 * fp16-split channel patterns there; independent of num_edges) and
 * feq_edgewise_workspace bytes for the backward. */
size_t feq_edgewise_fwd_workspace(const feq_layout* L, const feq_binning* b, int32_t rank,
                                  int64_t num_edges);
size_t feq_edgewise_workspace(const feq_layout* L, const feq_binning* b, int32_t rank,
                              int64_t num_edges);
int feq_edgewise_fwd(const feq_layout* L, const feq_binning* b, int32_t rank, int64_t num_edges,
                     const float* x, const float* P, const float* Q, const float* dist,
                     const float* C, const float* F, float* y,
                     void* workspace, size_t ws_bytes, feq_stream_t stream);
/* Outputs may be NULL when not needed: grad_x, grad_dist, grad_P, grad_Q.
 * grad_C (K,Cout,Cin) and grad_F (num_bins+1,K,Wdim) are overwritten. */
int feq_edgewise_bwd(const feq_layout* L, const feq_binning* b, int32_t rank, int64_t num_edges,
                     const float* grad_y, const float* x, const float* P, const float* Q,
                     const float* dist, const float* C, const float* F,
                     float* grad_x, float* grad_C, float* grad_F, float* grad_dist,
                     float* grad_P, float* grad_Q,
                     void* workspace, size_t ws_bytes, feq_stream_t stream);
/* 1 when feq_edgewise_fwd and feq_edgewise_bwd have kernels for this layout
 * and rank (the shape-generic pair keeps an edge's rows and the workgroup's
 * channel-pattern gradient in at most 160 KB of LDS: Cin Din, Din^2, Dout^2,
 * Cout Dout and K Cout Cin floats), else 0; they then return
 * FEQ_ERR_UNSUPPORTED.  The reference accepts any layout with lmax <= 16
 * (block_diagonal.cu:1298); a caller routes the others through the
 * composition x P -> feq_blockdiag_* on the formed radial table -> Q^T
 * (flash_eq/layers/linear.py:131-160). */
int feq_edgewise_fused_supported(const feq_layout* L, const feq_binning* b, int32_t rank);

/* ---- gradients for the bases on the fused kernels ------------------------------
 * The reference gets grad_P and grad_Q from torch.bmm autograd around its
 * block-diagonal op (flash_eq/layers/linear.py:135, :160): with f = x P and
 * y = m Q^T (m the block-diagonal output before the rotation),
 *   grad_P[e] = x_e^T (dL/df)_e   (Din x Din),   grad_Q[e] = grad_y_e^T m_e   (Dout x Dout).
 * feq_edgewise_fwd_ym is the forward (src NULL: x holds edge rows, as
 * feq_edgewise_fwd; else x is a node table read at src, as
 * feq_edgewise_fwd_src_ex, flags alike) that also writes m to ym (E, Cout,
 * Dout).  feq_edgewise_bwd_pq is the backward that also writes grad_P
 * (E, Din, Din) and grad_Q (E, Dout, Dout) (each may be NULL; ym is required
 * with grad_Q), both formed inside the input-gradient kernel's tiles: grad_Q
 * from the grad_y and m rows its producers load, grad_P from the tile's dL/df
 * and x rows (scalar-output layouts, lvals_out = [0]: in the wave-per-edge
 * backward, grad_P zero outside the m = 0 columns that y reads).  src NULL: grad_x (E, Cin, Din) per edge, workspace
 * feq_edgewise_workspace bytes; src set: grad_x (num_src, Cin, Din) summed per
 * source node over the CSR by source perm_src / offsets_src, as
 * feq_edgewise_bwd_src_nodes_ex, workspace
 * feq_edgewise_bwd_src_nodes_workspace bytes.  Layouts:
 * feq_edgewise_pq_supported (1); the others return FEQ_ERR_UNSUPPORTED, and
 * the shape-generic feq_edgewise_bwd forms grad_P and grad_Q itself. */
int feq_edgewise_pq_supported(const feq_layout* L, const feq_binning* b, int32_t rank);
int feq_edgewise_fwd_ym(const feq_layout* L, const feq_binning* b, int32_t rank, int64_t num_edges,
                        const float* x, int64_t num_src, const int64_t* src, const float* P,
                        const float* Q, const float* dist, const float* C, const float* F, float* y,
                        float* ym, int32_t flags, void* workspace, size_t ws_bytes,
                        feq_stream_t stream);
int feq_edgewise_bwd_pq(const feq_layout* L, const feq_binning* b, int32_t rank, int64_t num_edges,
                        const float* grad_y, const float* x, int64_t num_src, const int64_t* src,
                        const int32_t* perm_src, const int32_t* offsets_src, const float* P,
                        const float* Q, const float* dist, const float* C, const float* F,
                        const float* ym, float* grad_x, float* grad_C, float* grad_F,
                        float* grad_dist, float* grad_P, float* grad_Q, int32_t flags,
                        void* workspace, size_t ws_bytes, feq_stream_t stream);

/* ---- message-passing form of the fused layer ---------------------------------
 * The same layer with its input gathered inside the kernels: x is a node table
 * (num_src, Cin, Din) and edge e reads row src[e] (int64; an index outside
 * [0, num_src) reads a zero row), i.e. feq_edgewise_fwd(x[src], ...) without
 * materialising x[src] (reference: the x[src] gather before
 * EquivariantEdgewiseLinear in layers/attention.py:307-310).  The backward
 * writes the per-edge input gradient grad_x_edges (E, Cin, Din); the caller
 * sums it over the edges of each source node (feq_segment_sum over a CSR by
 * source).  Workspaces as for feq_edgewise_fwd/_bwd.  Only the layouts that
 * feq_edgewise_src_supported accepts (1) have these kernels; the others return
 * FEQ_ERR_UNSUPPORTED, and the caller gathers and calls feq_edgewise_fwd/_bwd. */
int feq_edgewise_src_supported(const feq_layout* L, const feq_binning* b, int32_t rank);
int feq_edgewise_fwd_src(const feq_layout* L, const feq_binning* b, int32_t rank, int64_t num_edges,
                         const float* x, int64_t num_src, const int64_t* src, const float* P,
                         const float* Q, const float* dist, const float* C, const float* F, float* y,
                         void* workspace, size_t ws_bytes, feq_stream_t stream);
/* Allocation-free form of feq_edgewise_fwd_src.  No counterpart in the
 * reference: it is for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Its scratch
 * (the split channel patterns) lives in a static device array of
 * FEQ_NOALLOC_SCRATCH_BYTES per device instead of a caller workspace; layouts
 * needing more are rejected with FEQ_ERR_UNSUPPORTED.  Calls that overlap on
 * one device race on that array.  Calls nothing that allocates. */
#define FEQ_NOALLOC_SCRATCH_BYTES (256 * 1024)
#define FEQ_MAX_DEVICES 64
int feq_edgewise_fwd_src_noalloc(const feq_layout* L, const feq_binning* b, int32_t rank,
                                 int64_t num_edges, const float* x, int64_t num_src,
                                 const int64_t* src, const float* P, const float* Q,
                                 const float* dist, const float* C, const float* F, float* y,
                                 feq_stream_t stream);
int feq_edgewise_bwd_src(const feq_layout* L, const feq_binning* b, int32_t rank, int64_t num_edges,
                         const float* grad_y, const float* x, int64_t num_src, const int64_t* src,
                         const float* P, const float* Q, const float* dist, const float* C,
                         const float* F, float* grad_x_edges, float* grad_C, float* grad_F,
                         float* grad_dist, void* workspace, size_t ws_bytes, feq_stream_t stream);
/* The same backward with the input gradient summed per source node inside the
 * kernel: grad_x_nodes (num_src, Cin, Din) = the scatter-sum over src of the
 * per-edge gradient (reference: the backward of the x[src] gather, index_select,
 * summed with atomics; attention.py:307-310).  perm_src / offsets_src (int32,
 * E and num_src + 1 entries) are the CSR by source (feq_csr_by_dst with src as
 * the key); the kernel walks the edges in that order and sums each node's rows
 * in CSR order (nodes whose edges cross a 16-edge tile boundary through two
 * partial rows per tile, summed in tile order).  Every node row is written,
 * zeros for nodes without edges; deterministic.  Workspace:
 * feq_edgewise_bwd_src_nodes_workspace bytes. */
size_t feq_edgewise_bwd_src_nodes_workspace(const feq_layout* L, const feq_binning* b, int32_t rank,
                                            int64_t num_edges);
int feq_edgewise_bwd_src_nodes(const feq_layout* L, const feq_binning* b, int32_t rank,
                               int64_t num_edges, const float* grad_y, const float* x,
                               int64_t num_src, const int64_t* src, const int32_t* perm_src,
                               const int32_t* offsets_src, const float* P, const float* Q,
                               const float* dist, const float* C, const float* F,
                               float* grad_x_nodes, float* grad_C, float* grad_F, float* grad_dist,
                               void* workspace, size_t ws_bytes, feq_stream_t stream);

/* Forms of feq_edgewise_fwd_src / feq_edgewise_bwd_src_nodes with a flags
 * word (flags = 0: identical to them).  The reference dispatches its kernel on
 * the tensor dtype (block_diagonal.cu:1332, AT_DISPATCH_FLOATING_TYPES_AND_HALF)
 * and computes at that precision; here the data stay float32 and the caller
 * states the accuracy it needs.  FEQ_EW_HALF_ACCURACY: the channel mixes use
 * one fp16 matrix-core product per operand pair instead of the three of the
 * hi/lo split: each operand is rounded to fp16 after its power-of-two scaling,
 * so a product carries a relative error up to about 2^-10 and a sum an error
 * up to about 2^-10 of the sum of its absolute terms, far inside the bfloat16
 * bar of 2e-2, for a third of the matrix-core work and half the split work.  For modules that
 * compute in bfloat16 or float16. */
#define FEQ_EW_HALF_ACCURACY 1
int feq_edgewise_fwd_src_ex(const feq_layout* L, const feq_binning* b, int32_t rank,
                            int64_t num_edges, const float* x, int64_t num_src, const int64_t* src,
                            const float* P, const float* Q, const float* dist, const float* C,
                            const float* F, float* y, int32_t flags, void* workspace,
                            size_t ws_bytes, feq_stream_t stream);
int feq_edgewise_bwd_src_nodes_ex(const feq_layout* L, const feq_binning* b, int32_t rank,
                                  int64_t num_edges, const float* grad_y, const float* x,
                                  int64_t num_src, const int64_t* src, const int32_t* perm_src,
                                  const int32_t* offsets_src, const float* P, const float* Q,
                                  const float* dist, const float* C, const float* F,
                                  float* grad_x_nodes, float* grad_C, float* grad_F,
                                  float* grad_dist, int32_t flags, void* workspace, size_t ws_bytes,
                                  feq_stream_t stream);

/* The V projection of EquivariantAttention fused with the attention's head
 * weighting and sum pooling.  The reference makes three passes over (E, Cout,
 * Dout) tensors: the layer over x[src] (attention.py:307-310), attn * V
 * (attention.py:311-313) and the scatter-sum to dst (pooling.py:21-30).  Here
 * out (num_dst, Cout, Dout)[n, c, :] = sum over the edges e into n of
 * attn[e, h(c)] y_e[c, :], y_e the layer's output for edge e (as
 * feq_edgewise_fwd_src_ex, flags alike), attn (E, heads) float32,
 * h(c) = min(c / chan_per_head, heads - 1); heads <= 16, chan_per_head a
 * multiple of 4.  The kernel walks the edges in the order of the CSR by
 * destination (perm_dst, offsets_dst over num_dst nodes: feq_csr_by_dst with
 * dst as the key) and sums each node's rows in that order (nodes crossing a
 * 16-edge tile boundary through partial rows summed in tile order), so the
 * result is deterministic; every node row is written; edges whose dst lies
 * outside [0, num_dst) add nothing.  The rows y_e are not formed unless y_pos
 * is given: y_pos (E, Cout, Dout) then receives them in CSR position order
 * (row p holds edge perm_dst[p]), the form feq_attn_pool_grad_attn reads.
 * Layouts: feq_edgewise_pool_supported.  Workspace:
 * feq_edgewise_fwd_src_pool_workspace bytes. */
int feq_edgewise_pool_supported(const feq_layout* L, const feq_binning* b, int32_t rank);
size_t feq_edgewise_fwd_src_pool_workspace(const feq_layout* L, const feq_binning* b, int32_t rank,
                                           int64_t num_edges);
int feq_edgewise_fwd_src_pool(const feq_layout* L, const feq_binning* b, int32_t rank,
                              int64_t num_edges, const float* x, int64_t num_src, const int64_t* src,
                              const float* P, const float* Q, const float* dist, const float* C,
                              const float* F, const float* attn, int32_t heads,
                              int32_t chan_per_head, const int64_t* dst, const int32_t* perm_dst,
                              const int32_t* offsets_dst, int64_t num_dst, float* out, float* y_pos,
                              int32_t flags, void* workspace, size_t ws_bytes, feq_stream_t stream);
/* Its backward: feq_edgewise_bwd_src_nodes_ex with the per-edge gradient
 * grad_y[e, c, :] = attn[e, h(c)] grad_out[dst[e], c, :] read inside the
 * kernels (never formed); grad_out (num_dst, Cout, Dout).  Edges whose dst lies
 * outside [0, num_dst) get zero gradients.  The attention weights' gradient is
 * feq_attn_pool_grad_attn's.  Workspace: feq_edgewise_bwd_src_nodes_workspace
 * bytes. */
int feq_edgewise_bwd_src_pool(const feq_layout* L, const feq_binning* b, int32_t rank,
                              int64_t num_edges, const float* grad_out, const float* attn,
                              int32_t heads, int32_t chan_per_head, const int64_t* dst,
                              int64_t num_dst, const float* x, int64_t num_src, const int64_t* src,
                              const int32_t* perm_src, const int32_t* offsets_src, const float* P,
                              const float* Q, const float* dist, const float* C, const float* F,
                              float* grad_x_nodes, float* grad_C, float* grad_F, float* grad_dist,
                              int32_t flags, void* workspace, size_t ws_bytes, feq_stream_t stream);

/* The pooled form with the gradients for the bases (as feq_edgewise_fwd_ym /
 * feq_edgewise_bwd_pq for the message-passing form): the forward also writes
 * m (E, Cout, Dout), the rows before the Q rotation, in edge order; the
 * backward writes grad_P (E, Din, Din) and grad_Q (E, Dout, Dout) (each may be
 * NULL; ym is required with grad_Q) with grad_y[e] = attn[e, h(c)]
 * grad_out[dst[e]] (zero for edges without a destination).  Layouts:
 * feq_edgewise_pq_supported. */
int feq_edgewise_fwd_src_pool_ym(const feq_layout* L, const feq_binning* b, int32_t rank,
                                 int64_t num_edges, const float* x, int64_t num_src, const int64_t* src,
                                 const float* P, const float* Q, const float* dist, const float* C,
                                 const float* F, const float* attn, int32_t heads,
                                 int32_t chan_per_head, const int64_t* dst, const int32_t* perm_dst,
                                 const int32_t* offsets_dst, int64_t num_dst, float* out, float* y_pos,
                                 float* ym, int32_t flags, void* workspace, size_t ws_bytes,
                                 feq_stream_t stream);
int feq_edgewise_bwd_src_pool_pq(const feq_layout* L, const feq_binning* b, int32_t rank,
                                 int64_t num_edges, const float* grad_out, const float* attn,
                                 int32_t heads, int32_t chan_per_head, const int64_t* dst,
                                 int64_t num_dst, const float* x, int64_t num_src, const int64_t* src,
                                 const int32_t* perm_src, const int32_t* offsets_src, const float* P,
                                 const float* Q, const float* dist, const float* C, const float* F,
                                 const float* ym, float* grad_x_nodes, float* grad_C, float* grad_F,
                                 float* grad_dist, float* grad_P, float* grad_Q, int32_t flags,
                                 void* workspace, size_t ws_bytes, feq_stream_t stream);

/* ---- Wigner-D basis ------------------------------------------------------------
 * plan: host-built per-representation constants (see feq_wigner_plan_size);
 * out (E, dim, dim): column j = column perm[j] of D(g), g e_z = dir/|dir|. */
size_t feq_wigner_plan_doubles(const int32_t* lvals, int32_t n);
int feq_wigner_basis(const int32_t* lvals, int32_t n, const double* plan_dev,
                     const int32_t* perm_dev, int64_t num_edges, const float* dirs,
                     float* out, feq_stream_t stream);
/* Backward of feq_wigner_basis: grad_dirs (E, 3) = d<grad_out, M>/d dirs, the
 * exact derivative of the reference's matrix_exp path (autograd through
 * rot_to_ez and matrix_exp, flash_eq/representations/wigner.py:144-240, 358-367)
 * in closed form: dD/dangle = X D and dD/dphi = [G2, D] for the axis generator
 * X, chained through the axis normalisation, arccos and d = v/(|v|+eps).
 * grad_out (E, dim, dim) float32; grad_dirs is written (not accumulated). */
int feq_wigner_basis_bwd(const int32_t* lvals, int32_t n, const double* plan_dev,
                         const int32_t* perm_dev, int64_t num_edges, const float* dirs,
                         const float* grad_out, float* grad_dirs, feq_stream_t stream);
/* float64 forms of the two above, for a WignerDBasis of float64 directions
 * (a module moved with .double(): its rot_to_ez and matrix_exp run in float64,
 * wigner.py:132-142, 198-240): the edge frame in float64 with the clamp of d_z
 * to [-1 + eps, 1 - eps] as written (in float32 its bounds round to +-1). */
int feq_wigner_basis_f64(const int32_t* lvals, int32_t n, const double* plan_dev,
                         const int32_t* perm_dev, int64_t num_edges, const double* dirs,
                         double* out, feq_stream_t stream);
int feq_wigner_basis_bwd_f64(const int32_t* lvals, int32_t n, const double* plan_dev,
                             const int32_t* perm_dev, int64_t num_edges, const double* dirs,
                             const double* grad_out, double* grad_dirs, feq_stream_t stream);

/* ---- graph ops -----------------------------------------------------------------
 * CSR by destination: perm (E) lists edge ids grouped by dst in increasing
 * order, stable within a node; offsets (N+1). */
size_t feq_csr_workspace(int64_t num_edges, int64_t num_nodes);
int feq_csr_by_dst(const int64_t* dst, int64_t num_edges, int64_t num_nodes,
                   int32_t* perm, int32_t* offsets, void* workspace, size_t ws_bytes,
                   feq_stream_t stream);
/* out[n, :] = sum over the node's edges (perm order) of x[e, :]; row = C*D floats. */
int feq_segment_sum(const float* x, int64_t row, const int32_t* perm, const int32_t* offsets,
                    int64_t num_nodes, float* out, feq_stream_t stream);
/* out[e, :] = src[idx[e], :] for 0 <= idx[e] < num_src, else 0. */
int feq_gather_rows(const float* src, int64_t num_src, int64_t row, const int64_t* idx,
                    int64_t num_rows, float* out, feq_stream_t stream);
/* out[0] = sum of y[i]^2 (the sum-of-squares loss of the reference's benchmark,
 * benchmarks/compare_all.py: (out**2).sum()), deterministic (a fixed grid of
 * partials summed in a fixed order) and free of memsets, so it can be recorded
 * in a HIP graph.  Workspace: feq_sum_squares_workspace() bytes. */
size_t feq_sum_squares_workspace(void);
int feq_sum_squares(const float* y, int64_t n, float* out, void* workspace, size_t ws_bytes,
                    feq_stream_t stream);
/* The same for bfloat16 y (16-bit storage): squares and sums in float32, out float32. */
int feq_sum_squares_bf16(const void* y, int64_t n, float* out, void* workspace, size_t ws_bytes,
                         feq_stream_t stream);

/* The radial network of SeparableRadialNet at the bin edges (radial.py:200-275:
 * trunk = Linear(in_dim, hidden), SiLU, Linear(hidden, hidden), SiLU; head =
 * Linear(hidden, out_dim)): F (rows, out_dim) = head(trunk(basis)) for the
 * (rows, in_dim) sinusoidal basis, float32, weights row-major as nn.Linear
 * holds them (W1 (hidden, in_dim), W2 (hidden, hidden), W3 (out_dim, hidden)).
 * The reference runs these few hundred thousand flops as a dozen library
 * launches per step; here the forward is one launch (a workgroup per row) and
 * the backward two.  acts (rows, 4 hidden floats) receives the trunk's
 * activations for feq_radial_bwd, which writes (does not accumulate) the six
 * parameter gradients from grad_F, deterministically; its workspace is
 * feq_radial_workspace(rows, hidden) bytes.  Shapes: feq_radial_supported. */
#define FEQ_RADIAL_MAX_WIDTH 1024
#define FEQ_RADIAL_MAX_OUT 4096
int feq_radial_supported(int32_t rows, int32_t in_dim, int32_t hidden, int32_t out_dim);
size_t feq_radial_workspace(int32_t rows, int32_t hidden);
int feq_radial_fwd(const float* basis, int32_t rows, int32_t in_dim, int32_t hidden, int32_t out_dim,
                   const float* W1, const float* b1, const float* W2, const float* b2, const float* W3,
                   const float* b3, float* F, float* acts, feq_stream_t stream);
int feq_radial_bwd(const float* basis, int32_t rows, int32_t in_dim, int32_t hidden, int32_t out_dim,
                   const float* W2, const float* W3, const float* acts, const float* grad_F,
                   float* grad_W1, float* grad_b1, float* grad_W2, float* grad_b2, float* grad_W3,
                   float* grad_b3, void* workspace, size_t ws_bytes, feq_stream_t stream);

/* High-degree form for bfloat16 features (canonical lvals 0..6 in and out,
 * Cin = Cout in {64, 128}, rank 4): x (E, Cin, Din), P, Q, y and the gradients
 * of x and y are bf16 (uint16 storage), dist, C, F and their gradients float32.
 * Same interface and results as feq_edgewise_fwd/_bwd (EquivariantEdgewiseLinear,
 * flash_eq/layers/linear.py:100-160) to bf16 accuracy: the GEMMs against the
 * channel patterns run on bf16 matrix cores with float32 accumulation.  The
 * backward forms no P/Q gradients.  The workspace holds rotated features and
 * staging (about 8 * E * Din * Cin bytes for the backward) and per-workgroup
 * partials of the channel-pattern gradient. */
int feq_edgewise_hl_supported(const feq_layout* layout, const feq_binning* binning, int32_t rank);
size_t feq_edgewise_hl_workspace(const feq_layout* layout, const feq_binning* binning, int32_t rank,
                                 int64_t num_edges, int32_t backward);
int feq_edgewise_hl_fwd(const feq_layout* layout, const feq_binning* binning, int32_t rank,
                        int64_t num_edges, const void* x, const void* P, const void* Q,
                        const float* dist, const float* C, const float* F, void* y, void* fs_out,
                        void* workspace, size_t workspace_bytes, feq_stream_t stream);
/* fs_out (nullable, bf16 (E, Din, Cin)): receives the rotated, s^l-scaled input
 * s^l (x P) in slot-major order; passing it to feq_edgewise_hl_bwd as fs_in
 * (nullable) spares the backward that rotation. */
int feq_edgewise_hl_bwd(const feq_layout* layout, const feq_binning* binning, int32_t rank,
                        int64_t num_edges, const void* grad_y, const void* x, const void* P,
                        const void* Q, const float* dist, const float* C, const float* F,
                        void* grad_x, float* grad_C, float* grad_F, float* grad_dist,
                        const void* fs_in, void* workspace, size_t workspace_bytes,
                        feq_stream_t stream);

/* Attention over head-major rows: a row of Q, K or V holds heads*head_dim floats,
 * head h at offset h*head_dim; row r of a table T starts at T + r*ld (floats).
 * Edges are visited in the CSR by destination (perm, offsets, num_nodes);
 * edges whose destination lies outside [0, num_nodes) get zero weights and
 * gradients.  Two forms:
 *   edge form (q_idx = k_idx = NULL): edge e reads row e of Q and of K;
 *   node form (q_idx = dst, k_idx = src): edge e reads row dst[e] of the node
 *     table Q (num_nodes rows) and row k_idx[e] of the node table K (num_k rows;
 *     an index outside [0, num_k) reads a zero row) -- the gathers of
 *     attention.py:298-304 done inside the kernels.
 * logits[e,h] = scale <Q_h, K_h> - dist[e]/decay (decay <= 0: no decay term);
 * scale is a device pointer to one float (exp(log_scale), attention.py:95-96),
 * read by the kernels, so no host synchronisation is needed to pass it;
 * attn = per-destination softmax with max shift and +1e-8 in the denominator
 * (attention.py:92-141).  qk_out (E, heads; nullable) receives scale <Q_h, K_h>.
 * Limit: head_dim <= 16 * V * 64 / NG, NG = next power of two >= heads (at most
 * 64), V = 4 when every row start is 16-byte aligned, else 1. */
int feq_attn_softmax_fwd(const float* Q, int64_t ldq, const float* K, int64_t ldk,
                         const int64_t* q_idx, const int64_t* k_idx, int64_t num_k,
                         const float* dist, int64_t num_edges, int32_t heads, int32_t head_dim,
                         const float* scale, float decay, const int32_t* perm,
                         const int32_t* offsets, int64_t num_nodes, float* attn, float* qk_out,
                         feq_stream_t stream);
/* Given grad_attn (E, heads): grad_logits (E, heads) = attn (grad_attn - S), S the
 * per-destination sum of attn*grad_attn (the caller forms the log-scale gradient
 * sum(grad_logits*qk) and the distance gradient -sum_h grad_logits/decay from it).
 * Edge form: grad_Q[e], grad_K[e] (E rows).  Node form: grad_Q (num_nodes rows)
 * and grad_K (num_k rows) summed per node, every row written; grad_K walks the
 * CSR of the edges by k_idx (perm_k, offsets_k), so num_k is that CSR's node
 * count (offsets_k has num_k + 1 entries).  With num_edges == 0, perm and
 * perm_k may be NULL and every gradient row is written as zero. */
int feq_attn_softmax_bwd(const float* Q, int64_t ldq, const float* K, int64_t ldk,
                         const int64_t* q_idx, const int64_t* k_idx, int64_t num_k,
                         const float* attn, const float* grad_attn, int64_t num_edges,
                         int32_t heads, int32_t head_dim, const float* scale, const int32_t* perm,
                         const int32_t* offsets, int64_t num_nodes, const int32_t* perm_k,
                         const int32_t* offsets_k, float* grad_Q, int64_t ldgq, float* grad_K,
                         int64_t ldgk, float* grad_logits, feq_stream_t stream);
/* The node form of feq_attn_softmax_fwd / _bwd on component-major node tables:
 * element (node n, channel c, component d) of Q, K, grad_Q and grad_K at
 * [d * comp_stride + n * ld + c] (the layout the fused QK projection writes:
 * Q = channels [0, mult), K = the same table from channel mult on), head h
 * the channels [h * head_channels, (h + 1) * head_channels) of every component
 * (head_dim = head_channels * dim).  The weights, logits and gradients are the
 * node-major form's up to the order of each head's dot-product sum.  No
 * counterpart in the reference (its Q and K are edge tensors). */
int feq_attn_softmax_fwd_cm(const float* Q, const float* K, int64_t ld, int64_t comp_stride,
                            int32_t dim, const int64_t* q_idx, const int64_t* k_idx, int64_t num_k,
                            const float* dist, int64_t num_edges, int32_t heads,
                            int32_t head_channels, const float* scale, float decay,
                            const int32_t* perm, const int32_t* offsets, int64_t num_nodes,
                            float* attn, float* qk_out, feq_stream_t stream);
int feq_attn_softmax_bwd_cm(const float* Q, const float* K, int64_t ld, int64_t comp_stride,
                            int32_t dim, const int64_t* q_idx, const int64_t* k_idx, int64_t num_k,
                            const float* attn, const float* grad_attn, int64_t num_edges,
                            int32_t heads, int32_t head_channels, const float* scale,
                            const int32_t* perm, const int32_t* offsets, int64_t num_nodes,
                            const int32_t* perm_k, const int32_t* offsets_k, float* grad_Q,
                            float* grad_K, float* grad_logits, feq_stream_t stream);
/* out[n,c,:] = sum_{e in seg(n)} attn[e, c / (mult/H)] * V[e,c,:]; V (E, mult, dim). */
int feq_attn_pool_fwd(const float* V, const float* attn, int64_t num_edges, int32_t mult,
                      int32_t dim, int32_t heads, const int32_t* perm, const int32_t* offsets,
                      int64_t num_nodes, float* out, feq_stream_t stream);
/* grad_V[e] = attn[e,h(c)] * gout[dst[e]]; grad_attn[e,h] = sum_{c in h, d} V*gout[dst],
 * walking the CSR by destination (gout[n] read once per node). */
int feq_attn_pool_bwd(const float* V, const float* attn, const float* grad_out,
                      const int32_t* perm, const int32_t* offsets, int64_t num_edges,
                      int64_t num_nodes, int32_t mult, int32_t dim, int32_t heads,
                      float* grad_V, float* grad_attn, feq_stream_t stream);
/* grad_attn[e, h] = sum_{c in h, d} V_pos[p, c, d] grad_out[n, c, d] for the edge
 * e = perm[p] at position p of node n's CSR segment (perm, offsets: the CSR by
 * destination); V_pos holds the per-edge rows in position order, as
 * feq_edgewise_fwd_src_pool keeps them (the attention-weight half of
 * feq_attn_pool_bwd; grad_V is not formed).  Edges outside the nodes get 0. */
int feq_attn_pool_grad_attn(const float* V_pos, const float* grad_out, const int32_t* perm,
                            const int32_t* offsets, int64_t num_edges, int64_t num_nodes,
                            int32_t mult, int32_t dim, int32_t heads, float* grad_attn,
                            feq_stream_t stream);

/* ---- node-side neighbours of the path (transformer block norms, gating) ----
 * Node tables x, y, gy, gx are (N, mult, dim) float32, contiguous; the layout is
 * the irreps' degrees lvals[nreps] (component offsets follow from 2l+1) and the
 * channel count mult <= FEQ_NODE_MAX_MULT.  Parameter gradients are written
 * (not accumulated) and are deterministic. */
#define FEQ_NODE_MAX_MULT 256
#define FEQ_NODE_MAX_SCALARS 8   /* l = 0 irreps per layout (separable norm) */

/* SeparableEquivariantLayerNorm (norm.py:177-246): l = 0 components get a
 * LayerNorm over channels, (v - mu) / (sd + eps) * w_s + b_s with w_s, b_s
 * (mult, nscalar) (_ChannelLayerNorm, norm.py:76-93); the l > 0 components
 * v * w_h[c] / sqrt(mean(v^2) + eps) over all channels and l > 0 components of a
 * node (_EquivariantRMSNorm, norm.py:96-112).  w_s/b_s may be NULL without
 * scalars, w_h without l > 0 irreps. */
int feq_sepnorm_fwd(const int32_t* lvals, int32_t nreps, int32_t mult, int64_t num_nodes,
                    const float* x, const float* w_s, const float* b_s, const float* w_h,
                    float eps, float* y, feq_stream_t stream);
size_t feq_sepnorm_workspace(const int32_t* lvals, int32_t nreps, int32_t mult,
                             int64_t num_nodes);
/* The same with y (forward) or grad_y (backward) component-major (dim, N, mult),
 * the layout of the channel-mixing maps that follow the norm in the block's
 * MLP; x and grad_x stay node-major; mult * dim at most 1152. */
int feq_sepnorm_fwd_cm(const int32_t* lvals, int32_t nreps, int32_t mult, int64_t num_nodes,
                       const float* x, const float* w_s, const float* b_s, const float* w_h,
                       float eps, float* y, feq_stream_t stream);
int feq_sepnorm_bwd(const int32_t* lvals, int32_t nreps, int32_t mult, int64_t num_nodes,
                    const float* grad_y, const float* x, const float* w_s, const float* w_h,
                    float eps, float* grad_x, float* grad_w_s, float* grad_b_s,
                    float* grad_w_h, void* workspace, size_t workspace_bytes,
                    feq_stream_t stream);
int feq_sepnorm_bwd_cm(const int32_t* lvals, int32_t nreps, int32_t mult, int64_t num_nodes,
                       const float* grad_y, const float* x, const float* w_s, const float* w_h,
                       float eps, float* grad_x, float* grad_w_s, float* grad_b_s,
                       float* grad_w_h, void* workspace, size_t workspace_bytes,
                       feq_stream_t stream);
/* feq_sepnorm_bwd (cm = 0) or _bwd_cm (cm != 0) with grad_x = the norm's input
 * gradient + grad_x_add (node-major, like grad_x): the gradient of an input
 * that also feeds a second branch (the block's residual connection), summed as
 * grad_x is written instead of in a separate pass.  No counterpart in the
 * reference, whose autograd adds the branches' gradients; mult * dim at most
 * 1152. */
int feq_sepnorm_bwd_add(const int32_t* lvals, int32_t nreps, int32_t mult, int64_t num_nodes,
                        const float* grad_y, const float* x, const float* w_s, const float* w_h,
                        float eps, const float* grad_x_add, float* grad_x, float* grad_w_s,
                        float* grad_b_s, float* grad_w_h, void* workspace, size_t workspace_bytes,
                        int32_t cm, feq_stream_t stream);

/* EquivariantLayerNorm (norm.py:148-174): per irrep k, n = sqrt(sum x^2 + eps)
 * (RepNorm, norm.py:51-73); y = x * LayerNorm_c(n)[w_ln, b_ln, ln_eps] / (n + eps),
 * or x / (n + eps) when w_ln = b_ln = NULL (one channel: no LayerNorm). */
int feq_eqnorm_fwd(const int32_t* lvals, int32_t nreps, int32_t mult, int64_t num_nodes,
                   const float* x, const float* w_ln, const float* b_ln, float eps,
                   float ln_eps, float* y, feq_stream_t stream);
size_t feq_eqnorm_workspace(const int32_t* lvals, int32_t nreps, int32_t mult,
                            int64_t num_nodes);
/* The same with y (forward) or grad_y (backward) component-major (dim, N, mult),
 * as feq_sepnorm_fwd_cm / _bwd_cm (the attention's QK projection follows this
 * norm); mult * dim at most 1152. */
int feq_eqnorm_fwd_cm(const int32_t* lvals, int32_t nreps, int32_t mult, int64_t num_nodes,
                      const float* x, const float* w_ln, const float* b_ln, float eps,
                      float ln_eps, float* y, feq_stream_t stream);
int feq_eqnorm_bwd_cm(const int32_t* lvals, int32_t nreps, int32_t mult, int64_t num_nodes,
                      const float* grad_y, const float* x, const float* w_ln, const float* b_ln,
                      float eps, float ln_eps, float* grad_x, float* grad_w_ln, float* grad_b_ln,
                      void* workspace, size_t workspace_bytes, feq_stream_t stream);
/* feq_eqnorm_bwd / _bwd_cm with grad_x = the norm's input gradient +
 * grad_x_add (node-major), as feq_sepnorm_bwd_add (the attention's input feeds
 * both this norm and the V projection).  No counterpart in the reference. */
int feq_eqnorm_bwd_add(const int32_t* lvals, int32_t nreps, int32_t mult, int64_t num_nodes,
                       const float* grad_y, const float* x, const float* w_ln, const float* b_ln,
                       float eps, float ln_eps, const float* grad_x_add, float* grad_x,
                       float* grad_w_ln, float* grad_b_ln, void* workspace, size_t workspace_bytes,
                       int32_t cm, feq_stream_t stream);
int feq_eqnorm_bwd(const int32_t* lvals, int32_t nreps, int32_t mult, int64_t num_nodes,
                   const float* grad_y, const float* x, const float* w_ln, const float* b_ln,
                   float eps, float ln_eps, float* grad_x, float* grad_w_ln, float* grad_b_ln,
                   void* workspace, size_t workspace_bytes, feq_stream_t stream);

/* EquivariantGating (gating.py:54-76) as norms -> [caller's Linear] -> apply:
 * norms (N, mult, nreps) = sqrt(sum_irrep x^2 + eps); y = x * sigmoid(lin)
 * broadcast over each irrep's components, lin (N, mult, nreps) the Linear's output.
 * Backward: grad_lin = sigmoid'(lin) * sum_irrep gy x (feed it to the Linear's
 * backward for grad_norms), then grad_x = gy sigmoid(lin) + x grad_norms / norms.
 * component_major != 0: x, y, grad_y, grad_x are (dim, N, mult) instead (the
 * layout EquivariantLinear's per-irrep GEMMs produce and consume); norms, lin
 * and their gradients are (N, mult, nreps) either way. */
int feq_gate_norms(const int32_t* lvals, int32_t nreps, int32_t mult, int64_t num_nodes,
                   int32_t component_major, const float* x, float eps, float* norms,
                   feq_stream_t stream);
int feq_gate_apply(const int32_t* lvals, int32_t nreps, int32_t mult, int64_t num_nodes,
                   int32_t component_major, const float* x, const float* lin, float* y,
                   feq_stream_t stream);
int feq_gate_bwd_lin(const int32_t* lvals, int32_t nreps, int32_t mult, int64_t num_nodes,
                     int32_t component_major, const float* grad_y, const float* x,
                     const float* lin, float* grad_lin, feq_stream_t stream);
int feq_gate_bwd_x(const int32_t* lvals, int32_t nreps, int32_t mult, int64_t num_nodes,
                   int32_t component_major, const float* grad_y, const float* x,
                   const float* lin, const float* norms, const float* grad_norms, float* grad_x,
                   feq_stream_t stream);

/* ---- dense helpers of the node-side layers ------------------------------------
 * The reference leaves this work to PyTorch inside its modules: its
 * EquivariantLinear forms all degrees in one broadcast product and a gather
 * (linear.py:242-268), which this build runs as one GEMM per degree on
 * component-major (dim, rows, c) tables, moved to and from node-major
 * (rows, c, dim) by feq_transpose; the bias gradients of its Linear and
 * EquivariantLinear biases (linear.py:262-266) are autograd's sums over rows;
 * and the gradients of scalar parameters, EquivariantAttention's log_scale
 * (attention.py:64-70) and LayerScale's gamma (transformer.py:35-39), are dot
 * products.  Here each is one deterministic pass, free of memsets (safe in HIP
 * graphs). */

/* EquivariantLinear (linear.py:242-268) on component-major tables: for each
 * component d of the representation (irrep k(d) of lvals[0..nreps)),
 *   y[d] = x[d] W_k^T (+ bias[:, bias_cols[k]] when irrep k is scalar and
 *   bias_cols[k] >= 0),
 * x (dim, rows, cin), y (dim, rows, cout), weight (nreps cout, cin) as the
 * module's parameter, bias (cout, nbias) or NULL.  feq_eqlinear_bwd_x is the
 * input gradient grad_x[d] = grad_y[d] W_k.  One launch for every component
 * (plus one that splits the weight): the products on the fp16 matrix cores
 * with split operands (hi + lo of power-of-two-scaled values, three products),
 * float32 accumulation: a float32 GEMM's accuracy.  Channel counts:
 * feq_eqlinear_supported(cin, cout) (32, 64 or 128 each); x and workspace 16-byte aligned; workspace
 * feq_eqlinear_workspace(nreps, cin, cout) bytes. */
int feq_eqlinear_supported(int32_t cin, int32_t cout);
size_t feq_eqlinear_workspace(int32_t nreps, int32_t cin, int32_t cout);
int feq_eqlinear_fwd(const int32_t* lvals, int32_t nreps, int64_t rows, int32_t cin, int32_t cout,
                     const float* x, const float* weight, const float* bias, int32_t nbias,
                     const int32_t* bias_cols, float* y, void* workspace, size_t ws_bytes,
                     feq_stream_t stream);
int feq_eqlinear_bwd_x(const int32_t* lvals, int32_t nreps, int64_t rows, int32_t cin, int32_t cout,
                       const float* grad_y, const float* weight, float* grad_x, void* workspace,
                       size_t ws_bytes, feq_stream_t stream);
/* The parameter gradients: grad_w[k] = sum over the rows of irrep k's components
 * of grad_y^T x ((nreps cout, cin), as weight), and, with grad_b (cout, nbias),
 * grad_b[:, bias_cols[k]] = sum of grad_y over those rows for each scalar irrep
 * k with bias_cols[k] >= 0.  Per-workgroup partials over 64-row chunks (split
 * fp16 products, per-column scales), summed in a fixed order: the same bits on
 * every run.  grad_y and x as above (component-major, 16-byte aligned);
 * workspace feq_eqlinear_bwd_w_workspace bytes (it depends on rows). */
size_t feq_eqlinear_bwd_w_workspace(const int32_t* lvals, int32_t nreps, int64_t rows, int32_t cin,
                                    int32_t cout);
int feq_eqlinear_bwd_w(const int32_t* lvals, int32_t nreps, int64_t rows, int32_t cin, int32_t cout,
                       const float* grad_y, const float* x, int32_t nbias, const int32_t* bias_cols,
                       float* grad_w, float* grad_b, void* workspace, size_t ws_bytes,
                       feq_stream_t stream);

/* out[b][j][i] = in[b][i][j] for in (batch, rows, cols) of elem_bytes-wide
 * elements (2, 4 or 8); out must not overlap in. */
int feq_transpose(const void* in, int64_t batch, int64_t rows, int64_t cols,
                  int32_t elem_bytes, void* out, feq_stream_t stream);
/* out[j] = sum over i of in[i][j] for in (rows, cols) float32 (elem_bytes 4,
 * float32 sums) or float64 (8).  rows = 0 writes zeros.  Partial sums per row
 * chunk are combined in a fixed order: the result does not depend on timing. */
size_t feq_column_sums_workspace(int64_t rows, int64_t cols, int32_t elem_bytes);
int feq_column_sums(const void* in, int64_t rows, int64_t cols, int32_t elem_bytes, void* out,
                    void* workspace, size_t ws_bytes, feq_stream_t stream);
/* The residual connection with LayerScale, x + gamma * y (transformer.py:245 and
 * :252 of the reference, LayerScale :23-38), in one pass: out = x + scale[0] y
 * (n floats, scale a device scalar).  Its backward for grad_out g in one pass:
 * grad_y = scale[0] g (may be NULL) and grad_scale[0] = sum of g * y, products
 * and sum in float64 in a fixed order (may be NULL; workspace
 * feq_dot_f64_workspace() bytes when set).  The gradient for x is g itself. */
int feq_scale_add(const float* x, const float* y, const float* scale, int64_t n, float* out,
                  feq_stream_t stream);
int feq_scale_add_bwd(const float* grad_out, const float* y, const float* scale, int64_t n,
                      float* grad_y, float* grad_scale, void* workspace, size_t ws_bytes,
                      feq_stream_t stream);
/* out = tables[0] + ... + tables[num_tables - 1] (1..16 float32 tables of n
 * floats, summed in that order): the gradients of a tensor read by several
 * consumers (the transformer's bases, used by every layer) in one pass instead
 * of autograd's pairwise sums.  No counterpart in the reference. */
int feq_sum_tables(const float* const* tables, int32_t num_tables, int64_t n, float* out,
                   feq_stream_t stream);
/* The same residual with y component-major (dim, N, mult), x and out node-major
 * (N, mult, dim): the block's MLP output joins the residual stream without a
 * separate transpose.  The backward writes grad_y component-major (may be NULL)
 * and grad_scale (may be NULL); workspace feq_scale_add_cm_workspace() bytes.
 * mult * dim at most 1152. */
int feq_scale_add_cm(const float* x, const float* y, const float* scale, int64_t num_nodes, int32_t mult,
                     int32_t dim, float* out, feq_stream_t stream);
size_t feq_scale_add_cm_workspace(void);
int feq_scale_add_cm_bwd(const float* grad_out, const float* y, const float* scale, int64_t num_nodes,
                         int32_t mult, int32_t dim, float* grad_y, float* grad_scale, void* workspace,
                         size_t ws_bytes, feq_stream_t stream);
/* out[0] = (float) sum of (double) a[i] * b[i], the products and their sum in
 * float64 in a fixed order (many products that largely cancel). */
size_t feq_dot_f64_workspace(void);
int feq_dot_f64(const float* a, const float* b, int64_t n, float* out, void* workspace,
                size_t ws_bytes, feq_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* FLASHEQ_H */

// Edge attention of EquivariantAttention: logits, per-destination softmax,
// head weighting with sum pooling, and their backward passes.
//
// Rows are head-major: a row of Q, K or V holds H * Dh floats, head h at offset
// h * Dh (attention.py:157-167 splits channel c into head c / (mult / H), so a
// head of an (mult, dim) row is the contiguous run of (mult / H) * dim floats).
// Row r of a table T starts at T + r * ld.
//
// Every kernel gives one wave to one CSR segment (the edges into one node, or
// out of one node for the K gradient), four waves per workgroup; segment N is
// the tail of edges whose node index lies outside the graph.  Inside a wave,
// head h0 + g is served by the G = 64 / NG lanes of group g (NG = heads per
// pass, a power of two); lane j of a group holds the V-float chunks
// j, j + G, j + 2 G, ... of the head's Dh values (at most NT of them), so a
// row is read with coalesced 16-byte loads and a head's dot product is a sum
// over the G lanes of its group (xor shuffles).  Edges are processed four at a
// time so that four rows per lane are in flight.  Segments are summed in CSR
// order: results are deterministic, without atomics.
//
// Node form: Q is a node table read at the segment's destination (loaded once
// per segment, held in registers) and K a node table read at k_idx[e] (the
// gather of attention.py:298-304 done inside the kernel); edge form: Q and K
// are (E, H * Dh) tables read at row e.
#include "feq_internal.h"

#include <type_traits>

namespace feq {
namespace {

constexpr int kWaves = 4;  // segments per workgroup
constexpr int kUE = 4;     // edges in flight per wave

template <int V>
__device__ inline void ldv(const float* __restrict__ p, float (&v)[V]) {
    if constexpr (V == 4) {
        const float4 t = *reinterpret_cast<const float4*>(p);
        v[0] = t.x;
        v[1] = t.y;
        v[2] = t.z;
        v[3] = t.w;
    } else {
        v[0] = *p;
    }
}

template <int V>
__device__ inline void stv(float* __restrict__ p, const float (&v)[V]) {
    if constexpr (V == 4)
        *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
    else
        *p = v[0];
}

// Chunks j, j + G, ... (< NC) of one head of a row; zeros where absent or !ok.
template <int V, int NT>
__device__ inline void ld_head(const float* __restrict__ head, int j, int G, int NC, bool ok,
                               float (&v)[NT][V]) {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const int c = j + G * t;
        if (ok && c < NC) {
            ldv<V>(head + c * V, v[t]);
        } else {
#pragma unroll
            for (int u = 0; u < V; ++u) v[t][u] = 0.0f;
        }
    }
}

template <int V, int NT>
__device__ inline void st_head(float* __restrict__ head, int j, int G, int NC, bool ok,
                               const float (&v)[NT][V]) {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const int c = j + G * t;
        if (ok && c < NC) stv<V>(head + c * V, v[t]);
    }
}

template <int V, int NT>
__device__ inline void st_head_scaled(float* __restrict__ head, int j, int G, int NC, bool ok,
                                      float a, const float (&v)[NT][V]) {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const int c = j + G * t;
        if (ok && c < NC) {
            float w[V];
#pragma unroll
            for (int u = 0; u < V; ++u) w[u] = a * v[t][u];
            stv<V>(head + c * V, w);
        }
    }
}

// Layout of the Q / K node tables' heads: head h of row n starts at
// n * ld + h * hs, and its chunk c (V floats) at (c / cpd) * cs + (c % cpd) * V
// from there.  Node-major rows (n, channel, component): hs = Dh, cpd = Dh / V,
// cs = 0 (the head's Dh floats are contiguous).  Component-major tables
// (component, n, channel): hs = hc (channels per head), cpd = hc / V, cs = the
// component stride (the head's hc channels of each component are contiguous).
struct HeadLayout {
    int64_t hs;
    int cpd;
    int64_t cs;
};

// The offsets of the lane's chunks j, j + G, ... within a head.
template <int V, int NT>
__device__ inline void head_offsets(const HeadLayout& hl, int j, int G, int64_t (&off)[NT]) {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const int c = j + G * t;
        const int g = c / hl.cpd;
        off[t] = g * hl.cs + static_cast<int64_t>(c - g * hl.cpd) * V;
    }
}

template <int V, int NT>
__device__ inline void ld_head_o(const float* __restrict__ head, const int64_t (&off)[NT], int j, int G, int NC,
                                 bool ok, float (&v)[NT][V]) {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const int c = j + G * t;
        if (ok && c < NC) {
            ldv<V>(head + off[t], v[t]);
        } else {
#pragma unroll
            for (int u = 0; u < V; ++u) v[t][u] = 0.0f;
        }
    }
}

template <int V, int NT>
__device__ inline void st_head_o(float* __restrict__ head, const int64_t (&off)[NT], int j, int G, int NC, bool ok,
                                 const float (&v)[NT][V]) {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const int c = j + G * t;
        if (ok && c < NC) stv<V>(head + off[t], v[t]);
    }
}

template <int V, int NT>
__device__ inline float dot_head(const float (&a)[NT][V], const float (&b)[NT][V]) {
    float s = 0.0f;
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int u = 0; u < V; ++u) s += a[t][u] * b[t][u];
    return s;
}

// Sum over the G lanes of an aligned lane group (G a power of two).
__device__ inline float group_sum(float v, int G) {
    for (int o = G >> 1; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// The wave's segment: node n (n == N: the tail of out-of-range edges), its
// first CSR position b and edge count.  False for waves past the tail.
__device__ inline bool wave_segment(const int32_t* __restrict__ offsets, int64_t N, int64_t E,
                                    int64_t& n, int& b, int& cnt) {
    n = static_cast<int64_t>(blockIdx.x) * kWaves +
        __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
    if (n > N) return false;
    b = offsets[n];
    cnt = (n < N ? offsets[n + 1] : static_cast<int>(E)) - b;
    return true;
}

// The segment's edge indices and gathered row indices, one lane per position of
// a 64-position chunk: loaded once per chunk, so the row loads of the chunk's
// edges go out without waiting on index loads edge by edge.  chunk_at reads
// position i's values (i wave-uniform) from the lane that loaded them.
// Row r of the gathered table: ridx[e] (node form, -1 outside [0, nr)) or e.
struct SegChunk {
    int e, r;
    template <bool GATHER>
    __device__ __forceinline__ void load(const int32_t* __restrict__ perm, int b, int cnt, int i0,
                                         const int64_t* __restrict__ ridx, int64_t nr) {
        const int p = i0 + static_cast<int>(threadIdx.x & 63);
        e = p < cnt ? perm[b + p] : 0;
        if constexpr (GATHER) {
            const int64_t rr = p < cnt ? ridx[e] : -1;
            r = rr >= 0 && rr < nr ? static_cast<int>(rr) : -1;
        } else {
            r = p < cnt ? e : -1;
        }
    }
    __device__ __forceinline__ int edge(int i) const { return __builtin_amdgcn_readlane(e, i & 63); }
    __device__ __forceinline__ int row(int i) const { return __builtin_amdgcn_readlane(r, i & 63); }
};

// ---- logits + softmax --------------------------------------------------------
// logit[e,h] = scale <Q[row q(e), h], K[row k(e), h]> - dist[e] / decay (decay > 0),
// attn = exp(logit - max) / (sum exp(logit - max) + 1e-8) over the segment
// (attention.py:92-141).  The maximum and the sum are carried together while
// the logits are formed (s <- s exp(m - l) + 1 on a new maximum); the logits
// are stored, then normalised in a second pass by the lane that stored them.
template <int V, int NT, bool NODE>
__global__ void __launch_bounds__(64 * kWaves)
k_att_fwd(const float* __restrict__ Q, int64_t ldq, const float* __restrict__ K, int64_t ldk,
          const int64_t* __restrict__ kidx, int64_t nk, const float* __restrict__ dist, int64_t E,
          int H, int Dh, int lgG, const float* __restrict__ scale_p, float decay,
          const int32_t* __restrict__ perm, const int32_t* __restrict__ offsets, int64_t N,
          float* __restrict__ attn, float* __restrict__ qk, HeadLayout hl) {
    const float scale = *scale_p;
    int64_t n;
    int b, cnt;
    if (!wave_segment(offsets, N, E, n, b, cnt)) return;
    const int lane = threadIdx.x & 63;
    if (n == N) {  // destination outside the graph: weight 0
        for (int t = lane; t < cnt * H; t += 64) {
            const int64_t e = perm[b + t / H];
            attn[e * H + t % H] = 0.0f;
            if (qk) qk[e * H + t % H] = 0.0f;
        }
        return;
    }
    const int G = 1 << lgG, NG = 64 >> lgG, g = lane >> lgG, j = lane & (G - 1);
    const int NC = Dh / V;
    // edges in flight: kUE, fewer when a lane's share of a head row is long
    // (16 chunks of 4 floats: the rows of kUE edges, and in the edge form the
    // Q rows too, would not fit the registers)
    constexpr int UE = NT * V >= 64 ? (NODE ? 2 : 1) : NT * V >= 32 ? 2 : kUE;
    static_assert(64 % UE == 0, "chunks of 64 positions hold whole groups of UE edges");
    int64_t off[NT];
    head_offsets<V, NT>(hl, j, G, off);
    for (int h0 = 0; h0 < H; h0 += NG) {
        const int h = h0 + g;
        const bool hv = h < H;
        float q[NT][V];
        if constexpr (NODE) ld_head_o<V, NT>(Q + n * ldq + h * hl.hs, off, j, G, NC, hv && cnt > 0, q);
        float m = -INFINITY, s = 0.0f;
        SegChunk sc{};
        for (int i0 = 0; i0 < cnt; i0 += UE) {
            if ((i0 & 63) == 0) sc.load<NODE>(perm, b, cnt, i0, kidx, nk);
            int64_t eu[UE];
            float k[UE][NT][V];
#pragma unroll
            for (int u = 0; u < UE; ++u) {
                const bool live = i0 + u < cnt;
                const int iu = live ? i0 + u : i0;
                eu[u] = sc.edge(iu);
                const int64_t kr = sc.row(iu);
                const bool ok = hv && live && kr >= 0;
                ld_head_o<V, NT>(K + (ok ? kr : 0) * ldk + h * hl.hs, off, j, G, NC, ok, k[u]);
            }
            float dot[UE];
            if constexpr (NODE) {
#pragma unroll
                for (int u = 0; u < UE; ++u) dot[u] = dot_head<V, NT>(q, k[u]);
            } else {
#pragma unroll
                for (int u = 0; u < UE; ++u) {
                    float qe[NT][V];
                    ld_head_o<V, NT>(Q + eu[u] * ldq + h * hl.hs, off, j, G, NC, hv && i0 + u < cnt, qe);
                    dot[u] = dot_head<V, NT>(qe, k[u]);
                }
            }
#pragma unroll
            for (int u = 0; u < UE; ++u) dot[u] = group_sum(dot[u], G);
#pragma unroll
            for (int u = 0; u < UE; ++u) {
                if (i0 + u >= cnt) break;
                const int64_t e = eu[u];
                const float qkv = dot[u] * scale;
                float lg = qkv;
                if (decay > 0.0f) lg -= dist[e] / decay;
                if (hv && ((i0 + u) & (G - 1)) == j) {
                    attn[e * H + h] = lg;
                    if (qk) qk[e * H + h] = qkv;
                }
                if (lg > m) {
                    s = s * expf(m - lg) + 1.0f;
                    m = lg;
                } else {
                    s += expf(lg - m);
                }
            }
        }
        if (hv)
            for (int i = j; i < cnt; i += G) {
                const int64_t e = perm[b + i];
                attn[e * H + h] = expf(attn[e * H + h] - m) / (s + 1e-8f);
            }
    }
}

// ---- softmax backward, by destination -------------------------------------------
// glogit[e,h] = attn (gattn - S_h), S_h = sum over the segment of attn gattn.
// Node form: gQ[n] = sum_e glogit scale K[row k(e)] (every node row written);
// edge form: gQ[e] = glogit scale K[e], gK[e] = glogit scale Q[e].
template <int V, int NT, bool NODE>
__global__ void __launch_bounds__(64 * kWaves)
k_att_bwd_dst(const float* __restrict__ Q, int64_t ldq, const float* __restrict__ K, int64_t ldk,
              const int64_t* __restrict__ kidx, int64_t nk, const float* __restrict__ attn,
              const float* __restrict__ gattn, int64_t E, int H, int Dh, int lgG,
              const float* __restrict__ scale_p, const int32_t* __restrict__ perm,
              const int32_t* __restrict__ offsets, int64_t N, float* __restrict__ gQ, int64_t ldgq,
              float* __restrict__ gK, int64_t ldgk, float* __restrict__ glogit, HeadLayout hl) {
    const float scale = *scale_p;
    int64_t n;
    int b, cnt;
    if (!wave_segment(offsets, N, E, n, b, cnt)) return;
    const int lane = threadIdx.x & 63;
    if (n == N) {  // destination outside the graph: zero gradients
        for (int t = lane; t < cnt * H; t += 64) glogit[static_cast<int64_t>(perm[b + t / H]) * H + t % H] = 0.0f;
        if (!NODE)
            for (int i = 0; i < cnt; ++i) {
                const int64_t e = perm[b + i];
                for (int c = lane; c < H * Dh; c += 64) {
                    gQ[e * ldgq + c] = 0.0f;
                    gK[e * ldgk + c] = 0.0f;
                }
            }
        return;
    }
    const int G = 1 << lgG, NG = 64 >> lgG, g = lane >> lgG, j = lane & (G - 1);
    const int NC = Dh / V;
    int64_t off[NT];
    head_offsets<V, NT>(hl, j, G, off);
    for (int h0 = 0; h0 < H; h0 += NG) {
        const int h = h0 + g;
        const bool hv = h < H;
        float sp = 0.0f;
        if (hv)
            for (int i = j; i < cnt; i += G) {
                const int64_t e = perm[b + i];
                sp += attn[e * H + h] * gattn[e * H + h];
            }
        const float S = group_sum(sp, G);
        float acc[NT][V];
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int u = 0; u < V; ++u) acc[t][u] = 0.0f;
        SegChunk sc{};
        for (int i0 = 0; i0 < cnt; i0 += kUE) {
            if ((i0 & 63) == 0) sc.load<NODE>(perm, b, cnt, i0, kidx, nk);
            int64_t eu[kUE];
            float gl[kUE];
            float k[kUE][NT][V];
#pragma unroll
            for (int u = 0; u < kUE; ++u) {
                const bool live = i0 + u < cnt;
                const int iu = live ? i0 + u : i0;
                eu[u] = sc.edge(iu);
                const int64_t e = eu[u];
                const int64_t kr = sc.row(iu);
                const bool ok = hv && live && kr >= 0;
                ld_head_o<V, NT>(K + (ok ? kr : 0) * ldk + h * hl.hs, off, j, G, NC, ok, k[u]);
                gl[u] = (hv && live) ? attn[e * H + h] * (gattn[e * H + h] - S) : 0.0f;
                if (hv && live && ((i0 + u) & (G - 1)) == j) glogit[e * H + h] = gl[u];
            }
#pragma unroll
            for (int u = 0; u < kUE; ++u) {
                const float w = gl[u] * scale;
                if constexpr (NODE) {
#pragma unroll
                    for (int t = 0; t < NT; ++t)
#pragma unroll
                        for (int v = 0; v < V; ++v) acc[t][v] += w * k[u][t][v];
                } else {
                    const bool live = hv && i0 + u < cnt;
                    const int64_t e = eu[u];
                    st_head_scaled<V, NT>(gQ + e * ldgq + h * Dh, j, G, NC, live, w, k[u]);
                    float qe[NT][V];
                    ld_head<V, NT>(Q + e * ldq + h * Dh, j, G, NC, live, qe);
                    st_head_scaled<V, NT>(gK + e * ldgk + h * Dh, j, G, NC, live, w, qe);
                }
            }
        }
        if constexpr (NODE) st_head_o<V, NT>(gQ + n * ldgq + h * hl.hs, off, j, G, NC, hv, acc);
    }
}

// ---- K gradient of the node form, by source ----------------------------------------
// gK[m] = sum over the edges out of m (CSR by source) of glogit[e,h] scale Q[q(e)];
// every row of gK is written.
template <int V, int NT>
__global__ void __launch_bounds__(64 * kWaves)
k_att_bwd_src(const float* __restrict__ Q, int64_t ldq, const int64_t* __restrict__ qidx,
              int64_t nq, const float* __restrict__ glogit, int64_t E, int H, int Dh, int lgG,
              const float* __restrict__ scale_p, const int32_t* __restrict__ perm,
              const int32_t* __restrict__ offsets, int64_t NK, float* __restrict__ gK, int64_t ldgk,
              HeadLayout hl) {
    const float scale = *scale_p;
    int64_t n;
    int b, cnt;
    if (!wave_segment(offsets, NK, E, n, b, cnt) || n == NK) return;
    const int lane = threadIdx.x & 63;
    const int G = 1 << lgG, NG = 64 >> lgG, g = lane >> lgG, j = lane & (G - 1);
    const int NC = Dh / V;
    int64_t off[NT];
    head_offsets<V, NT>(hl, j, G, off);
    for (int h0 = 0; h0 < H; h0 += NG) {
        const int h = h0 + g;
        const bool hv = h < H;
        float acc[NT][V];
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int u = 0; u < V; ++u) acc[t][u] = 0.0f;
        SegChunk sc{};
        for (int i0 = 0; i0 < cnt; i0 += kUE) {
            if ((i0 & 63) == 0) sc.load<true>(perm, b, cnt, i0, qidx, nq);
            float gl[kUE];
            float q[kUE][NT][V];
#pragma unroll
            for (int u = 0; u < kUE; ++u) {
                const bool live = i0 + u < cnt;
                const int iu = live ? i0 + u : i0;
                const int64_t e = sc.edge(iu);
                const int64_t qr = sc.row(iu);
                const bool ok = hv && live && qr >= 0;
                ld_head_o<V, NT>(Q + (ok ? qr : 0) * ldq + h * hl.hs, off, j, G, NC, ok, q[u]);
                gl[u] = ok ? glogit[e * H + h] * scale : 0.0f;
            }
#pragma unroll
            for (int u = 0; u < kUE; ++u)
#pragma unroll
                for (int t = 0; t < NT; ++t)
#pragma unroll
                    for (int v = 0; v < V; ++v) acc[t][v] += gl[u] * q[u][t][v];
        }
        st_head_o<V, NT>(gK + n * ldgk + h * hl.hs, off, j, G, NC, hv, acc);
    }
}

// ---- head weighting + sum pooling ---------------------------------------------------
// out[n, h] = sum over the segment of attn[e,h] V[e, h]  (V rows of H * Dh floats).
template <int V, int NT>
__global__ void __launch_bounds__(64 * kWaves)
k_pool_fwd(const float* __restrict__ Vt, const float* __restrict__ attn, int64_t E, int H, int Dh,
           int lgG, const int32_t* __restrict__ perm, const int32_t* __restrict__ offsets,
           int64_t N, float* __restrict__ out) {
    int64_t n;
    int b, cnt;
    if (!wave_segment(offsets, N, E, n, b, cnt) || n == N) return;
    const int lane = threadIdx.x & 63;
    const int G = 1 << lgG, NG = 64 >> lgG, g = lane >> lgG, j = lane & (G - 1);
    const int NC = Dh / V;
    const int64_t row = static_cast<int64_t>(H) * Dh;
    for (int h0 = 0; h0 < H; h0 += NG) {
        const int h = h0 + g;
        const bool hv = h < H;
        float acc[NT][V];
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int u = 0; u < V; ++u) acc[t][u] = 0.0f;
        for (int i0 = 0; i0 < cnt; i0 += kUE) {
            float a[kUE];
            float v[kUE][NT][V];
#pragma unroll
            for (int u = 0; u < kUE; ++u) {
                const bool live = hv && i0 + u < cnt;
                const int64_t e = perm[b + (i0 + u < cnt ? i0 + u : i0)];
                a[u] = live ? attn[e * H + h] : 0.0f;
                ld_head<V, NT>(Vt + e * row + h * Dh, j, G, NC, live, v[u]);
            }
#pragma unroll
            for (int u = 0; u < kUE; ++u)
#pragma unroll
                for (int t = 0; t < NT; ++t)
#pragma unroll
                    for (int w = 0; w < V; ++w) acc[t][w] += a[u] * v[u][t][w];
        }
        st_head<V, NT>(out + n * row + h * Dh, j, G, NC, hv, acc);
    }
}

// gV[e, h] = attn[e,h] gout[n, h]; gattn[e,h] = <V[e, h], gout[n, h]> for the
// edges into n (gout[n] loaded once per segment); out-of-range edges get zeros.
// VPOS: V holds the rows in CSR position order (row b + i, as the pooled
// edgewise forward keeps them) and only gattn is formed (gV is not written).
template <int V, int NT, bool VPOS>
__global__ void __launch_bounds__(64 * kWaves)
k_pool_bwd(const float* __restrict__ Vt, const float* __restrict__ attn,
           const float* __restrict__ gout, int64_t E, int H, int Dh, int lgG,
           const int32_t* __restrict__ perm, const int32_t* __restrict__ offsets, int64_t N,
           float* __restrict__ gV, float* __restrict__ gattn) {
    int64_t n;
    int b, cnt;
    if (!wave_segment(offsets, N, E, n, b, cnt)) return;
    const int lane = threadIdx.x & 63;
    const int64_t row = static_cast<int64_t>(H) * Dh;
    if (n == N) {
        for (int t = lane; t < cnt * H; t += 64) gattn[static_cast<int64_t>(perm[b + t / H]) * H + t % H] = 0.0f;
        if (VPOS) return;
        for (int i = 0; i < cnt; ++i) {
            const int64_t e = perm[b + i];
            for (int64_t c = lane; c < row; c += 64) gV[e * row + c] = 0.0f;
        }
        return;
    }
    const int G = 1 << lgG, NG = 64 >> lgG, g = lane >> lgG, j = lane & (G - 1);
    const int NC = Dh / V;
    for (int h0 = 0; h0 < H; h0 += NG) {
        const int h = h0 + g;
        const bool hv = h < H;
        float go[NT][V];
        ld_head<V, NT>(gout + n * row + h * Dh, j, G, NC, hv && cnt > 0, go);
        for (int i0 = 0; i0 < cnt; i0 += kUE) {
            int64_t eu[kUE];
            float a[kUE];
            float v[kUE][NT][V];
#pragma unroll
            for (int u = 0; u < kUE; ++u) {
                const bool live = hv && i0 + u < cnt;
                const int pos = b + (i0 + u < cnt ? i0 + u : i0);
                eu[u] = perm[pos];
                a[u] = live && !VPOS ? attn[eu[u] * H + h] : 0.0f;   // VPOS: attn unused (NULL)
                ld_head<V, NT>(Vt + (VPOS ? static_cast<int64_t>(pos) : eu[u]) * row + h * Dh, j, G, NC,
                               live, v[u]);
            }
            float dot[kUE];
#pragma unroll
            for (int u = 0; u < kUE; ++u) dot[u] = group_sum(dot_head<V, NT>(v[u], go), G);
#pragma unroll
            for (int u = 0; u < kUE; ++u) {
                const bool live = hv && i0 + u < cnt;
                if (live && ((i0 + u) & (G - 1)) == j) gattn[eu[u] * H + h] = dot[u];
                if (!VPOS) st_head_scaled<V, NT>(gV + eu[u] * row + h * Dh, j, G, NC, live, a[u], go);
            }
        }
    }
}

// ---- launch configuration ------------------------------------------------------------
struct HeadCfg {
    int V;    // floats per chunk (4: 16-byte accesses)
    int NT;   // chunks per lane, template bound
    int lgG;  // log2 lanes per head group
};

bool al16(const void* p) { return p == nullptr || (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Chunking of a head of Dh floats: 16-byte chunks when every row start is
// 16-byte aligned (Dh, all row strides a multiple of 4 floats and aligned
// bases), else single floats; heads per pass NG = next power of two >= H (at
// most 64), G = 64 / NG lanes per head.
int head_cfg(int H, int Dh, std::initializer_list<int64_t> lds,
             std::initializer_list<const void*> ptrs, HeadCfg& c) {
    if (H < 1) return fail(FEQ_ERR_INVALID, "num_heads must be positive");
    if (Dh < 1) return fail(FEQ_ERR_INVALID, "head dim must be positive");
    bool vec = Dh % 4 == 0;
    for (int64_t ld : lds) vec = vec && ld % 4 == 0;
    for (const void* p : ptrs) vec = vec && al16(p);
    c.V = vec ? 4 : 1;
    int ng = 1;
    while (ng < H && ng < 64) ng <<= 1;
    const int G = 64 / ng;
    c.lgG = 0;
    while ((1 << c.lgG) < G) ++c.lgG;
    const int nt = (Dh / c.V + G - 1) / G;
    if (nt > 16)
        return fail(FEQ_ERR_UNSUPPORTED,
                    "head dim %d too large for %d heads (at most %d floats per head)", Dh, H,
                    16 * G * c.V);
    c.NT = nt <= 1 ? 1 : nt <= 2 ? 2 : nt <= 4 ? 4 : nt <= 8 ? 8 : 16;
    return FEQ_OK;
}

template <int N>
using IC = std::integral_constant<int, N>;

// Calls fn(IC<V>, IC<NT>) for the configuration's template arguments.
template <typename Fn>
int with_cfg(const HeadCfg& c, Fn&& fn) {
    auto pick = [&](auto VV) -> int {
        switch (c.NT) {
            case 1: return fn(VV, IC<1>{});
            case 2: return fn(VV, IC<2>{});
            case 4: return fn(VV, IC<4>{});
            case 8: return fn(VV, IC<8>{});
            default: return fn(VV, IC<16>{});
        }
    };
    return c.V == 4 ? pick(IC<4>{}) : pick(IC<1>{});
}

dim3 seg_grid(int64_t segments) { return dim3(static_cast<unsigned>(ceil_div(segments, kWaves))); }

int check_graph(int64_t E, int64_t N) {
    if (E < 0 || N < 1) return fail(FEQ_ERR_INVALID, "invalid graph sizes");
    if (E > 0x7fffffffLL) return fail(FEQ_ERR_UNSUPPORTED, "more than 2^31-1 edges");
    return FEQ_OK;
}

}  // namespace
}  // namespace feq

using namespace feq;

namespace {

// The node-major (cs = 0: rows of heads * head_dim floats, ld / ldg their
// strides) and component-major (cs > 0: element (n, channel c, component d)
// at d cs + n ld + c, hc channels per head, head_dim = hc * dim) forms share
// these.
int softmax_fwd(const float* Q, int64_t ldq, const float* K, int64_t ldk, const int64_t* q_idx,
                const int64_t* k_idx, int64_t num_k, const float* dist, int64_t num_edges, int32_t heads,
                int32_t head_dim, int32_t hc, int64_t cs, const float* scale, float decay, const int32_t* perm,
                const int32_t* offsets, int64_t num_nodes, float* attn, float* qk_out, hipStream_t s) {
    if (!scale) return fail(FEQ_ERR_INVALID, "NULL scale (a device float)");
    if (int rc = check_graph(num_edges, num_nodes)) return rc;
    const bool node = q_idx != nullptr;
    if (node != (k_idx != nullptr)) return fail(FEQ_ERR_INVALID, "q_idx and k_idx must both be given or both be NULL");
    if (num_edges == 0) return FEQ_OK;
    if (!Q || !K || !perm || !offsets || !attn) return fail(FEQ_ERR_INVALID, "NULL pointer");
    if (decay > 0.0f && !dist) return fail(FEQ_ERR_INVALID, "distance decay needs distances");
    const int64_t row = static_cast<int64_t>(heads) * (cs ? hc : head_dim);
    if (ldq < row || ldk < row) return fail(FEQ_ERR_INVALID, "row stride shorter than the heads' values");
    const int64_t nk = node ? num_k : num_edges;
    HeadCfg c;
    if (int rc = cs ? head_cfg(heads, head_dim, {ldq, ldk, hc, cs}, {Q, K}, c)
                    : head_cfg(heads, head_dim, {ldq, ldk}, {Q, K}, c))
        return rc;
    const HeadLayout hl = cs ? HeadLayout{hc, hc / c.V, cs} : HeadLayout{head_dim, head_dim / c.V, 0};
    return with_cfg(c, [&](auto VV, auto TT) -> int {
        constexpr int V = decltype(VV)::value, NT = decltype(TT)::value;
        if (node) {
            auto kern = k_att_fwd<V, NT, true>;
            FEQ_LAUNCH("k_att_fwd", kern, seg_grid(num_nodes + 1), dim3(64 * kWaves), 0, s, Q, ldq,
                       K, ldk, k_idx, nk, dist, num_edges, heads, head_dim, c.lgG, scale, decay,
                       perm, offsets, num_nodes, attn, qk_out, hl);
        } else {
            auto kern = k_att_fwd<V, NT, false>;
            FEQ_LAUNCH("k_att_fwd", kern, seg_grid(num_nodes + 1), dim3(64 * kWaves), 0, s, Q, ldq,
                       K, ldk, k_idx, nk, dist, num_edges, heads, head_dim, c.lgG, scale, decay,
                       perm, offsets, num_nodes, attn, qk_out, hl);
        }
        return FEQ_OK;
    });
}

int softmax_bwd(const float* Q, int64_t ldq, const float* K, int64_t ldk, const int64_t* q_idx,
                const int64_t* k_idx, int64_t num_k, const float* attn, const float* grad_attn,
                int64_t num_edges, int32_t heads, int32_t head_dim, int32_t hc, int64_t cs, const float* scale,
                const int32_t* perm, const int32_t* offsets, int64_t num_nodes, const int32_t* perm_k,
                const int32_t* offsets_k, float* grad_Q, int64_t ldgq, float* grad_K, int64_t ldgk,
                float* grad_logits, hipStream_t s) {
    if (!scale) return fail(FEQ_ERR_INVALID, "NULL scale (a device float)");
    if (int rc = check_graph(num_edges, num_nodes)) return rc;
    const bool node = q_idx != nullptr;
    if (node != (k_idx != nullptr)) return fail(FEQ_ERR_INVALID, "q_idx and k_idx must both be given or both be NULL");
    // node form: grad_Q gets one row per destination segment (num_nodes rows),
    // grad_K one row per segment of the CSR by k_idx (num_k rows, offsets_k has
    // num_k + 1 entries); rows without edges are written as zeros
    if (node && (num_k < 1 || !offsets_k || (num_edges > 0 && !perm_k)))
        return fail(FEQ_ERR_INVALID, "the node form needs the CSR of the edges by k_idx");
    const int64_t row = static_cast<int64_t>(heads) * (cs ? hc : head_dim);
    if (ldq < row || ldk < row || ldgq < row || ldgk < row)
        return fail(FEQ_ERR_INVALID, "row stride shorter than the heads' values");
    if (!grad_Q || !grad_K || !offsets) return fail(FEQ_ERR_INVALID, "NULL pointer");
    if (num_edges > 0 && (!Q || !K || !attn || !grad_attn || !perm || !grad_logits))
        return fail(FEQ_ERR_INVALID, "NULL pointer");
    HeadCfg c;
    if (int rc = cs ? head_cfg(heads, head_dim, {ldq, ldk, ldgq, ldgk, hc, cs}, {Q, K, grad_Q, grad_K}, c)
                    : head_cfg(heads, head_dim, {ldq, ldk, ldgq, ldgk}, {Q, K, grad_Q, grad_K}, c))
        return rc;
    const HeadLayout hl = cs ? HeadLayout{hc, hc / c.V, cs} : HeadLayout{head_dim, head_dim / c.V, 0};
    if (!node && num_edges == 0) return FEQ_OK;
    const int64_t nk = node ? num_k : num_edges;
    return with_cfg(c, [&](auto VV, auto TT) -> int {
        constexpr int V = decltype(VV)::value, NT = decltype(TT)::value;
        if (node) {
            auto kd = k_att_bwd_dst<V, NT, true>;
            FEQ_LAUNCH("k_att_bwd_dst", kd, seg_grid(num_nodes + 1), dim3(64 * kWaves), 0, s, Q,
                       ldq, K, ldk, k_idx, nk, attn, grad_attn, num_edges, heads, head_dim, c.lgG,
                       scale, perm, offsets, num_nodes, grad_Q, ldgq, grad_K, ldgk, grad_logits, hl);
            auto ks = k_att_bwd_src<V, NT>;
            FEQ_LAUNCH("k_att_bwd_src", ks, seg_grid(num_k + 1), dim3(64 * kWaves), 0, s, Q, ldq,
                       q_idx, num_nodes, grad_logits, num_edges, heads, head_dim, c.lgG, scale,
                       perm_k, offsets_k, num_k, grad_K, ldgk, hl);
        } else {
            auto kd = k_att_bwd_dst<V, NT, false>;
            FEQ_LAUNCH("k_att_bwd_dst", kd, seg_grid(num_nodes + 1), dim3(64 * kWaves), 0, s, Q,
                       ldq, K, ldk, k_idx, nk, attn, grad_attn, num_edges, heads, head_dim, c.lgG,
                       scale, perm, offsets, num_nodes, grad_Q, ldgq, grad_K, ldgk, grad_logits, hl);
        }
        return FEQ_OK;
    });
}

}  // namespace

extern "C" int feq_attn_softmax_fwd(const float* Q, int64_t ldq, const float* K, int64_t ldk,
                                    const int64_t* q_idx, const int64_t* k_idx, int64_t num_k,
                                    const float* dist, int64_t num_edges, int32_t heads,
                                    int32_t head_dim, const float* scale, float decay,
                                    const int32_t* perm, const int32_t* offsets, int64_t num_nodes,
                                    float* attn, float* qk_out, feq_stream_t stream) {
    return softmax_fwd(Q, ldq, K, ldk, q_idx, k_idx, num_k, dist, num_edges, heads, head_dim, 0, 0, scale, decay,
                       perm, offsets, num_nodes, attn, qk_out, stream_of(stream));
}

extern "C" int feq_attn_softmax_fwd_cm(const float* Q, const float* K, int64_t ld, int64_t comp_stride,
                                       int32_t dim, const int64_t* q_idx, const int64_t* k_idx, int64_t num_k,
                                       const float* dist, int64_t num_edges, int32_t heads,
                                       int32_t head_channels, const float* scale, float decay,
                                       const int32_t* perm, const int32_t* offsets, int64_t num_nodes,
                                       float* attn, float* qk_out, feq_stream_t stream) {
    if (dim < 1 || head_channels < 1 || comp_stride < 1) return fail(FEQ_ERR_INVALID, "invalid sizes");
    if (!q_idx || !k_idx) return fail(FEQ_ERR_INVALID, "the component-major tables are node tables");
    return softmax_fwd(Q, ld, K, ld, q_idx, k_idx, num_k, dist, num_edges, heads, head_channels * dim,
                       head_channels, comp_stride, scale, decay, perm, offsets, num_nodes, attn, qk_out,
                       stream_of(stream));
}

extern "C" int feq_attn_softmax_bwd(const float* Q, int64_t ldq, const float* K, int64_t ldk,
                                    const int64_t* q_idx, const int64_t* k_idx, int64_t num_k,
                                    const float* attn, const float* grad_attn, int64_t num_edges,
                                    int32_t heads, int32_t head_dim, const float* scale,
                                    const int32_t* perm, const int32_t* offsets, int64_t num_nodes,
                                    const int32_t* perm_k, const int32_t* offsets_k,
                                    float* grad_Q, int64_t ldgq, float* grad_K, int64_t ldgk,
                                    float* grad_logits, feq_stream_t stream) {
    return softmax_bwd(Q, ldq, K, ldk, q_idx, k_idx, num_k, attn, grad_attn, num_edges, heads, head_dim, 0, 0,
                       scale, perm, offsets, num_nodes, perm_k, offsets_k, grad_Q, ldgq, grad_K, ldgk, grad_logits,
                       stream_of(stream));
}

extern "C" int feq_attn_softmax_bwd_cm(const float* Q, const float* K, int64_t ld, int64_t comp_stride,
                                       int32_t dim, const int64_t* q_idx, const int64_t* k_idx, int64_t num_k,
                                       const float* attn, const float* grad_attn, int64_t num_edges,
                                       int32_t heads, int32_t head_channels, const float* scale,
                                       const int32_t* perm, const int32_t* offsets, int64_t num_nodes,
                                       const int32_t* perm_k, const int32_t* offsets_k, float* grad_Q,
                                       float* grad_K, float* grad_logits, feq_stream_t stream) {
    if (dim < 1 || head_channels < 1 || comp_stride < 1) return fail(FEQ_ERR_INVALID, "invalid sizes");
    if (!q_idx || !k_idx) return fail(FEQ_ERR_INVALID, "the component-major tables are node tables");
    return softmax_bwd(Q, ld, K, ld, q_idx, k_idx, num_k, attn, grad_attn, num_edges, heads, head_channels * dim,
                       head_channels, comp_stride, scale, perm, offsets, num_nodes, perm_k, offsets_k, grad_Q, ld,
                       grad_K, ld, grad_logits, stream_of(stream));
}

extern "C" int feq_attn_pool_fwd(const float* V, const float* attn, int64_t num_edges,
                                 int32_t mult, int32_t dim, int32_t heads, const int32_t* perm,
                                 const int32_t* offsets, int64_t num_nodes, float* out,
                                 feq_stream_t stream) {
    if (heads < 1 || mult % heads) return fail(FEQ_ERR_INVALID, "num_heads must divide mult");
    if (dim < 1) return fail(FEQ_ERR_INVALID, "invalid sizes");
    if (int rc = check_graph(num_edges, num_nodes)) return rc;
    if (!offsets || !out || (num_edges > 0 && (!V || !attn || !perm)))
        return fail(FEQ_ERR_INVALID, "NULL pointer");
    const int Dh = mult / heads * dim;
    HeadCfg c;
    if (int rc = head_cfg(heads, Dh, {}, {V, out}, c)) return rc;
    hipStream_t s = stream_of(stream);
    return with_cfg(c, [&](auto VV, auto TT) -> int {
        constexpr int Vw = decltype(VV)::value, NT = decltype(TT)::value;
        auto kern = k_pool_fwd<Vw, NT>;
        FEQ_LAUNCH("k_pool_fwd", kern, seg_grid(num_nodes), dim3(64 * kWaves), 0, s, V, attn,
                   num_edges, heads, Dh, c.lgG, perm, offsets, num_nodes, out);
        return FEQ_OK;
    });
}

extern "C" int feq_attn_pool_bwd(const float* V, const float* attn, const float* grad_out,
                                 const int32_t* perm, const int32_t* offsets, int64_t num_edges,
                                 int64_t num_nodes, int32_t mult, int32_t dim, int32_t heads,
                                 float* grad_V, float* grad_attn, feq_stream_t stream) {
    if (heads < 1 || mult % heads) return fail(FEQ_ERR_INVALID, "num_heads must divide mult");
    if (dim < 1) return fail(FEQ_ERR_INVALID, "invalid sizes");
    if (int rc = check_graph(num_edges, num_nodes)) return rc;
    if (num_edges == 0) return FEQ_OK;
    if (!V || !attn || !grad_out || !perm || !offsets || !grad_V || !grad_attn)
        return fail(FEQ_ERR_INVALID, "NULL pointer");
    const int Dh = mult / heads * dim;
    HeadCfg c;
    if (int rc = head_cfg(heads, Dh, {}, {V, grad_out, grad_V}, c)) return rc;
    hipStream_t s = stream_of(stream);
    return with_cfg(c, [&](auto VV, auto TT) -> int {
        constexpr int Vw = decltype(VV)::value, NT = decltype(TT)::value;
        auto kern = k_pool_bwd<Vw, NT, false>;
        FEQ_LAUNCH("k_pool_bwd", kern, seg_grid(num_nodes + 1), dim3(64 * kWaves), 0, s, V, attn,
                   grad_out, num_edges, heads, Dh, c.lgG, perm, offsets, num_nodes, grad_V,
                   grad_attn);
        return FEQ_OK;
    });
}

extern "C" int feq_attn_pool_grad_attn(const float* V_pos, const float* grad_out,
                                       const int32_t* perm, const int32_t* offsets, int64_t num_edges,
                                       int64_t num_nodes, int32_t mult, int32_t dim, int32_t heads,
                                       float* grad_attn, feq_stream_t stream) {
    if (heads < 1 || mult % heads) return fail(FEQ_ERR_INVALID, "num_heads must divide mult");
    if (dim < 1) return fail(FEQ_ERR_INVALID, "invalid sizes");
    if (int rc = check_graph(num_edges, num_nodes)) return rc;
    if (num_edges == 0) return FEQ_OK;
    if (!V_pos || !grad_out || !perm || !offsets || !grad_attn) return fail(FEQ_ERR_INVALID, "NULL pointer");
    const int Dh = mult / heads * dim;
    HeadCfg c;
    if (int rc = head_cfg(heads, Dh, {}, {V_pos, grad_out}, c)) return rc;
    hipStream_t s = stream_of(stream);
    return with_cfg(c, [&](auto VV, auto TT) -> int {
        constexpr int Vw = decltype(VV)::value, NT = decltype(TT)::value;
        auto kern = k_pool_bwd<Vw, NT, true>;
        FEQ_LAUNCH("k_pool_grad_attn", kern, seg_grid(num_nodes + 1), dim3(64 * kWaves), 0, s, V_pos,
                   static_cast<const float*>(nullptr), grad_out, num_edges, heads, Dh, c.lgG, perm,
                   offsets, num_nodes, static_cast<float*>(nullptr), grad_attn);
        return FEQ_OK;
    });
}

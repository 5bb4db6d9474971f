/*
 * Per-edge C restatement of the reference block-diagonal kernels (oracle).
 *
 * TEST INFRASTRUCTURE ONLY -- built by oracle/Makefile into oracle/_build and
 * loaded by oracle/cref.py; never linked into the product library.
 *
 * Follows flash_eq/cuda/csrc/block_diagonal.cu:
 *   compute_binning          :82-115   (float32 index path, t in scalar_t)
 *   binning_derivative       :121-138
 *   ipow / setup_edge        :202-213, :307-319  (s = r/(r+sigma), scale = s^(l_in+l_out))
 *   forward_m0 / forward_mpos            :558-733
 *   backward_features_m0 / _mpos         :747-917
 *   backward_table_m0 / _mpos            :931-1161 (dT lo/hi split, dr terms)
 *   precompute_block_info                :1191-1266 (m-block offsets)
 * Written from the semantics, one edge at a time, in the order the kernels
 * accumulate; OpenMP parallelises over edges (and over output channels for dT,
 * so every sum is accumulated in a fixed order).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define MAXB 64

typedef struct {
    int nb;                       /* number of m-blocks */
    int m[MAXB], n_in[MAXB], n_out[MAXB], in_off[MAXB], out_off[MAXB], w_off[MAXB];
    int l_in[MAXB][MAXB], l_out[MAXB][MAXB];
} blocks_t;

static int build_blocks(const int* lin, int nlin, const int* lout, int nlout, blocks_t* b) {
    int mmax = 0, in_off = 0, out_off = 0, w_off = 0;
    for (int i = 0; i < nlin; ++i) if (lin[i] > mmax) mmax = lin[i];
    for (int i = 0; i < nlout; ++i) if (lout[i] > mmax) mmax = lout[i];
    b->nb = 0;
    for (int m = 0; m <= mmax; ++m) {
        int ni = 0, no = 0;
        int k = b->nb;
        if (k >= MAXB) return -1;
        for (int i = 0; i < nlin; ++i) if (lin[i] >= m) { if (ni >= MAXB) return -1; b->l_in[k][ni++] = lin[i]; }
        for (int i = 0; i < nlout; ++i) if (lout[i] >= m) { if (no >= MAXB) return -1; b->l_out[k][no++] = lout[i]; }
        if (ni == 0 || no == 0) continue;
        b->m[k] = m; b->n_in[k] = ni; b->n_out[k] = no;
        b->in_off[k] = in_off; b->out_off[k] = out_off; b->w_off[k] = w_off;
        b->nb++;
        int mul = m == 0 ? 1 : 2;
        in_off += mul * ni; out_off += mul * no; w_off += mul * ni * no;
    }
    return 0;
}

/* float32 log/exp rounded from double (correctly rounded), as the kernels form them */
static float cr_logf(float x) { return (float)log((double)x); }
static float cr_expf(float x) { return (float)exp((double)x); }

#define DEFINE_ORACLE(T, SUF)                                                               \
static T ipow_##SUF(T base, int e) {                                                       \
    T r = (T)1;                                                                             \
    while (e > 0) { if (e & 1) r *= base; base *= base; e >>= 1; }                         \
    return r;                                                                               \
}                                                                                           \
static void binning_##SUF(T dist, float p1, float p2, int nbins, int logb,                 \
                          int* lo, int* hi, T* t, T* dtdr) {                               \
    float nrm;                                                                              \
    if (logb) nrm = (cr_logf(fmaxf((float)dist, cr_expf(p1))) - p1) * p2 * (float)nbins;  \
    else      nrm = ((float)dist - p1) * p2;                                               \
    nrm = fminf(fmaxf(nrm, 0.0f), (float)nbins);                                           \
    int l = (int)floorf(nrm); if (l > nbins - 1) l = nbins - 1;                            \
    *lo = l; *hi = (l + 1 < nbins) ? l + 1 : nbins;                                         \
    if (logb) {                                                                             \
        T ilbw = (T)(p2 * (float)nbins);                                                    \
        T lel = (T)p1 + (T)l / ilbw;                                                        \
        T el = (T)exp((double)lel);                                                         \
        T eh = (T)exp((double)(lel + (T)1 / ilbw));                                         \
        T c = dist > el ? dist : el;                                                        \
        T tt = (c - el) / (eh - el);                                                        \
        *t = tt < (T)1 ? tt : (T)1;                                                         \
        *dtdr = (T)1 / (eh - el);                                                           \
    } else {                                                                                \
        T bw = (T)1 / (T)p2;                                                                \
        T el = (T)p1 + (T)l * bw;                                                           \
        *t = (dist - el) / bw;                                                              \
        *dtdr = (T)p2;                                                                      \
    }                                                                                       \
}                                                                                           \
int feqo_fwd_##SUF(int64_t E, int cin, int cout, int din, int dout, int wdim,              \
                   const int* lin, int nlin, const int* lout, int nlout,                   \
                   float p1, float p2, int nbins, int logb, float sigma,                   \
                   const T* x, const T* tab, const T* r, T* y) {                           \
    blocks_t B; if (build_blocks(lin, nlin, lout, nlout, &B)) return -1;                   \
    const int64_t ts = (int64_t)cout * cin * wdim;                                         \
    _Pragma("omp parallel for schedule(static)")                                            \
    for (int64_t e = 0; e < E; ++e) {                                                       \
        int lo, hi; T t, dd; binning_##SUF(r[e], p1, p2, nbins, logb, &lo, &hi, &t, &dd);   \
        T omt = (T)1 - t;                                                                   \
        T sw = r[e] / (r[e] + (T)sigma);                                                    \
        const T* xe = x + e * cin * din;                                                    \
        T* ye = y + e * cout * dout;                                                        \
        for (int q = 0; q < cout * dout; ++q) ye[q] = 0;                                   \
        for (int k = 0; k < B.nb; ++k) {                                                    \
            int ni = B.n_in[k], no = B.n_out[k];                                            \
            for (int co = 0; co < cout; ++co) for (int o = 0; o < no; ++o) {                \
                T are = 0, aim = 0;                                                         \
                for (int ci = 0; ci < cin; ++ci) for (int i = 0; i < ni; ++i) {             \
                    T sc = ipow_##SUF(sw, B.l_in[k][i] + B.l_out[k][o]);                    \
                    int64_t wb = (int64_t)co * cin * wdim + (int64_t)ci * wdim + B.w_off[k]; \
                    if (B.m[k] == 0) {                                                      \
                        int64_t w = wb + o * ni + i;                                        \
                        T wt = omt * tab[lo * ts + w] + t * tab[hi * ts + w];               \
                        are += wt * sc * xe[ci * din + B.in_off[k] + i];                    \
                    } else {                                                                \
                        int64_t w = wb + 2 * (o * ni + i);                                  \
                        T a = (omt * tab[lo * ts + w] + t * tab[hi * ts + w]) * sc;         \
                        T b = (omt * tab[lo * ts + w + 1] + t * tab[hi * ts + w + 1]) * sc; \
                        T fr = xe[ci * din + B.in_off[k] + 2 * i];                          \
                        T fi = xe[ci * din + B.in_off[k] + 2 * i + 1];                      \
                        are += a * fr + b * fi;                                             \
                        aim += a * fi - b * fr;                                             \
                    }                                                                       \
                }                                                                           \
                if (B.m[k] == 0) ye[co * dout + B.out_off[k] + o] = are;                    \
                else { ye[co * dout + B.out_off[k] + 2 * o] = are;                          \
                       ye[co * dout + B.out_off[k] + 2 * o + 1] = aim; }                    \
            }                                                                               \
        }                                                                                   \
    }                                                                                       \
    return 0;                                                                               \
}                                                                                           \
int feqo_bwd_##SUF(int64_t E, int cin, int cout, int din, int dout, int wdim,              \
                   const int* lin, int nlin, const int* lout, int nlout,                   \
                   float p1, float p2, int nbins, int logb, float sigma,                   \
                   const T* gy, const T* x, const T* tab, const T* r,                      \
                   T* gx, T* gt, T* gr) {                                                   \
    blocks_t B; if (build_blocks(lin, nlin, lout, nlout, &B)) return -1;                   \
    const int64_t ts = (int64_t)cout * cin * wdim;                                         \
    /* grad_features and grad_distances: per edge */                                      \
    _Pragma("omp parallel for schedule(static)")                                            \
    for (int64_t e = 0; e < E; ++e) {                                                       \
        int lo, hi; T t, dd; binning_##SUF(r[e], p1, p2, nbins, logb, &lo, &hi, &t, &dd);   \
        T omt = (T)1 - t;                                                                   \
        T sw = r[e] / (r[e] + (T)sigma);                                                    \
        T deriv = (T)sigma / (r[e] * (r[e] + (T)sigma));                                    \
        const T* xe = x + e * cin * din; const T* ge = gy + e * cout * dout;                \
        T* gxe = gx + e * cin * din;                                                        \
        for (int q = 0; q < cin * din; ++q) gxe[q] = 0;                                    \
        T acc_t = 0, acc_s = 0;                                                             \
        for (int k = 0; k < B.nb; ++k) {                                                    \
            int ni = B.n_in[k], no = B.n_out[k];                                            \
            for (int ci = 0; ci < cin; ++ci) for (int i = 0; i < ni; ++i) {                 \
                T gre = 0, gim = 0;                                                         \
                for (int co = 0; co < cout; ++co) for (int o = 0; o < no; ++o) {            \
                    int L = B.l_in[k][i] + B.l_out[k][o];                                   \
                    T sc = ipow_##SUF(sw, L);                                               \
                    int64_t wb = (int64_t)co * cin * wdim + (int64_t)ci * wdim + B.w_off[k]; \
                    if (B.m[k] == 0) {                                                      \
                        int64_t w = wb + o * ni + i;                                        \
                        T wlo = tab[lo * ts + w], whi = tab[hi * ts + w];                   \
                        T f = xe[ci * din + B.in_off[k] + i];                               \
                        T g = ge[co * dout + B.out_off[k] + o];                             \
                        T wt = (omt * wlo + t * whi) * sc;                                  \
                        gre += wt * g;                                                      \
                        T gw = sc * f * g;                                                  \
                        acc_t += (whi - wlo) * gw;                                          \
                        if (L > 0) acc_s += (omt * wlo + t * whi) * f * g * sc * (T)L * deriv; \
                    } else {                                                                \
                        int64_t w = wb + 2 * (o * ni + i);                                  \
                        T alo = tab[lo * ts + w], ahi = tab[hi * ts + w];                   \
                        T blo = tab[lo * ts + w + 1], bhi = tab[hi * ts + w + 1];           \
                        T a = (omt * alo + t * ahi) * sc, b = (omt * blo + t * bhi) * sc;   \
                        T gr_ = ge[co * dout + B.out_off[k] + 2 * o];                       \
                        T gi_ = ge[co * dout + B.out_off[k] + 2 * o + 1];                   \
                        gre += a * gr_ - b * gi_;                                           \
                        gim += b * gr_ + a * gi_;                                           \
                        T fr = xe[ci * din + B.in_off[k] + 2 * i];                          \
                        T fi = xe[ci * din + B.in_off[k] + 2 * i + 1];                      \
                        T ga = fr * gr_ + fi * gi_, gb = fi * gr_ - fr * gi_;               \
                        acc_t += (ahi - alo) * sc * ga + (bhi - blo) * sc * gb;             \
                        acc_s += (omt * alo + t * ahi) * ga * sc * (T)L * deriv;            \
                        acc_s += (omt * blo + t * bhi) * gb * sc * (T)L * deriv;            \
                    }                                                                       \
                }                                                                           \
                if (B.m[k] == 0) gxe[ci * din + B.in_off[k] + i] = gre;                     \
                else { gxe[ci * din + B.in_off[k] + 2 * i] = gre;                           \
                       gxe[ci * din + B.in_off[k] + 2 * i + 1] = gim; }                     \
            }                                                                               \
        }                                                                                   \
        if (gr) gr[e] = acc_t * dd + acc_s;                                                 \
    }                                                                                       \
    /* grad_table: parallel over output channel, edges in order */                         \
    memset(gt, 0, sizeof(T) * (size_t)(nbins + 1) * ts);                                   \
    _Pragma("omp parallel for schedule(static)")                                            \
    for (int co = 0; co < cout; ++co) {                                                     \
        for (int64_t e = 0; e < E; ++e) {                                                   \
            int lo, hi; T t, dd; binning_##SUF(r[e], p1, p2, nbins, logb, &lo, &hi, &t, &dd); \
            T omt = (T)1 - t;                                                               \
            T sw = r[e] / (r[e] + (T)sigma);                                                \
            const T* xe = x + e * cin * din; const T* ge = gy + e * cout * dout;            \
            for (int k = 0; k < B.nb; ++k) {                                                \
                int ni = B.n_in[k], no = B.n_out[k];                                        \
                for (int ci = 0; ci < cin; ++ci) for (int o = 0; o < no; ++o)               \
                for (int i = 0; i < ni; ++i) {                                              \
                    T sc = ipow_##SUF(sw, B.l_in[k][i] + B.l_out[k][o]);                    \
                    int64_t wb = (int64_t)co * cin * wdim + (int64_t)ci * wdim + B.w_off[k]; \
                    if (B.m[k] == 0) {                                                      \
                        int64_t w = wb + o * ni + i;                                        \
                        T gw = sc * xe[ci * din + B.in_off[k] + i] * ge[co * dout + B.out_off[k] + o]; \
                        gt[lo * ts + w] += omt * gw; gt[hi * ts + w] += t * gw;             \
                    } else {                                                                \
                        int64_t w = wb + 2 * (o * ni + i);                                  \
                        T fr = xe[ci * din + B.in_off[k] + 2 * i];                          \
                        T fi = xe[ci * din + B.in_off[k] + 2 * i + 1];                      \
                        T gr_ = ge[co * dout + B.out_off[k] + 2 * o];                       \
                        T gi_ = ge[co * dout + B.out_off[k] + 2 * o + 1];                   \
                        T ga = sc * (fr * gr_ + fi * gi_), gb = sc * (fi * gr_ - fr * gi_); \
                        gt[lo * ts + w] += omt * ga; gt[hi * ts + w] += t * ga;             \
                        gt[lo * ts + w + 1] += omt * gb; gt[hi * ts + w + 1] += t * gb;     \
                    }                                                                       \
                }                                                                           \
            }                                                                               \
        }                                                                                   \
    }                                                                                       \
    return 0;                                                                               \
}                                                                                           \
void feqo_binning_##SUF(int64_t E, const T* r, float p1, float p2, int nbins, int logb,    \
                        int32_t* lo, T* t) {                                                \
    for (int64_t e = 0; e < E; ++e) { int l, h; T tt, dd;                                   \
        binning_##SUF(r[e], p1, p2, nbins, logb, &l, &h, &tt, &dd); lo[e] = l; t[e] = tt; } \
}

DEFINE_ORACLE(double, f64)
DEFINE_ORACLE(float, f32)

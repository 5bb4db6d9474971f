// Compile-time m-first layout of a canonical representation pair
// (lvals = 0..LIN in, 0..LOUT out): slot offsets, radial-weight offsets and the
// list of (out slot, in slot, weight, sign) terms of the per-edge mixing
// matrix, as fixed by the m-block layout of block_diagonal.cu:1220-1258 (2x2
// [[a, b], [-b, a]] blocks on the (+m, -m) pairs for m > 0).
#pragma once

#include <hip/hip_runtime.h>

#include <array>
#include <utility>

namespace feq {
// Internal linkage on purpose: the compiler folds loads from the constexpr
// term tables only when each translation unit owns its copy.
namespace {

struct Term {
    int o, i, w, neg;
};

template <int LIN, int LOUT>
struct Canon {
    static constexpr int DIN = (LIN + 1) * (LIN + 1);
    static constexpr int DOUT = (LOUT + 1) * (LOUT + 1);
    static constexpr int MMIN = LIN < LOUT ? LIN : LOUT;
    static constexpr int nin(int m) { return LIN - m + 1; }
    static constexpr int nout(int m) { return LOUT - m + 1; }
    static constexpr int in_off(int m) {
        int o = 0;
        for (int q = 0; q < m; ++q) o += (q ? 2 : 1) * nin(q);
        return o;
    }
    static constexpr int out_off(int m) {
        int o = 0;
        for (int q = 0; q < m; ++q) o += (q ? 2 : 1) * nout(q);
        return o;
    }
    static constexpr int w_off(int m) {
        int o = 0;
        for (int q = 0; q < m; ++q) o += (q ? 2 : 1) * nin(q) * nout(q);
        return o;
    }
    static constexpr int WD = w_off(MMIN + 1);
    static constexpr int count() {
        int n = 0;
        for (int m = 0; m <= MMIN; ++m) n += (m ? 4 : 1) * nin(m) * nout(m);
        return n;
    }
    static constexpr int NT = count();
    static constexpr std::array<Term, NT> make_terms() {
        std::array<Term, NT> t{};
        int n = 0;
        for (int m = 0; m <= MMIN; ++m) {
            const int ni = nin(m), no = nout(m), io = in_off(m), oo = out_off(m), wo = w_off(m);
            for (int o = 0; o < no; ++o)
                for (int i = 0; i < ni; ++i) {
                    if (m == 0) {
                        t[n++] = Term{oo + o, io + i, wo + o * ni + i, 0};
                    } else {
                        const int wa = wo + 2 * (o * ni + i);
                        const int ro = oo + 2 * o, im_o = ro + 1, ri = io + 2 * i, im_i = ri + 1;
                        t[n++] = Term{ro, ri, wa, 0};          // re += a f_re
                        t[n++] = Term{ro, im_i, wa + 1, 0};    // re += b f_im
                        t[n++] = Term{im_o, im_i, wa, 0};      // im += a f_im
                        t[n++] = Term{im_o, ri, wa + 1, 1};    // im -= b f_re
                    }
                }
        }
        return t;
    }
    static constexpr std::array<Term, NT> terms = make_terms();
    // l_in + l_out of radial weight w: in m-block m, pair (o, i) joins degrees
    // m + i (in) and m + o (out).
    static constexpr std::array<int, WD> make_wl() {
        std::array<int, WD> v{};
        for (int m = 0; m <= MMIN; ++m)
            for (int o = 0; o < nout(m); ++o)
                for (int i = 0; i < nin(m); ++i) {
                    if (m == 0) {
                        v[w_off(m) + o * nin(m) + i] = o + i;
                    } else {
                        v[w_off(m) + 2 * (o * nin(m) + i)] = 2 * m + o + i;
                        v[w_off(m) + 2 * (o * nin(m) + i) + 1] = 2 * m + o + i;
                    }
                }
        return v;
    }
    static constexpr std::array<int, WD> wl = make_wl();
    // wl packed 4 bits per weight, for lookups with a run-time index
    static constexpr int NWW = (WD + 15) / 16;
    static constexpr std::array<unsigned long long, NWW> make_wl_words() {
        std::array<unsigned long long, NWW> w{};
        for (int j = 0; j < WD; ++j) w[j / 16] |= static_cast<unsigned long long>(wl[j]) << (4 * (j % 16));
        return w;
    }
    static constexpr std::array<unsigned long long, NWW> wl_words = make_wl_words();
    static __device__ __forceinline__ int wl_of(int w) {
        unsigned long long word = wl_words[0];
#pragma unroll
        for (int n = 1; n < NWW; ++n) word = (w >> 4) == n ? wl_words[n] : word;
        return static_cast<int>((word >> (4 * (w & 15))) & 15u);
    }
};

// l of every m-first component of a canonical representation with lmax L
template <int L>
struct SlotL {
    static constexpr std::array<int, (L + 1) * (L + 1)> make() {
        std::array<int, (L + 1) * (L + 1)> v{};
        int s = 0;
        for (int l = 0; l <= L; ++l) v[s++] = l;
        for (int m = 1; m <= L; ++m)
            for (int l = m; l <= L; ++l) {
                v[s++] = l;
                v[s++] = l;
            }
        return v;
    }
    static constexpr std::array<int, (L + 1) * (L + 1)> l = make();
};

// Degree-block structure of a Wigner-D basis matrix of a canonical
// representation (lvals = 0..L): row d is in the standard (l, m) order,
// column j in the m-first order, and the entry can be non-zero only when
// deg(d) == SlotL<L>::l[j] (the matrix is block diagonal over irreps).
template <int L>
struct DegreeBlocks {
    static constexpr int D = (L + 1) * (L + 1);
    static constexpr int NW = (D * D + 31) / 32;
    static constexpr int deg(int d) {
        int l = 0;
        while ((l + 1) * (l + 1) <= d) ++l;
        return l;
    }
    // m-first slots of degree l: slots[l * l .. (l + 1) * (l + 1))
    static constexpr std::array<int, D> make_slots() {
        std::array<int, D> v{};
        std::array<int, L + 1> fill{};
        for (int j = 0; j < D; ++j) {
            const int l = SlotL<L>::l[j];
            v[l * l + fill[l]++] = j;
        }
        return v;
    }
    static constexpr std::array<int, D> slots = make_slots();
    // bit (d D + j) set where the entry lies outside the blocks
    static constexpr std::array<unsigned, NW> make_offmask() {
        std::array<unsigned, NW> m{};
        for (int d = 0; d < D; ++d)
            for (int j = 0; j < D; ++j)
                if (deg(d) != SlotL<L>::l[j]) m[(d * D + j) / 32] |= 1u << ((d * D + j) % 32);
        return m;
    }
    static constexpr std::array<unsigned, NW> offmask = make_offmask();
};

// Compile-time loop: f(std::integral_constant<int, 0>{}), ..., up to N - 1.
template <class Fn, int... Is>
__device__ __forceinline__ void static_for_impl(Fn&& f, std::integer_sequence<int, Is...>) {
    (f(std::integral_constant<int, Is>{}), ...);
}
template <int N, class Fn>
__device__ __forceinline__ void static_for(Fn&& f) {
    static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// The terms of Canon<LIN, LOUT> grouped by input slot (BY_OUT = false) or by
// output slot (BY_OUT = true): group s holds terms [start[s], start[s + 1]).
template <int LIN, int LOUT, bool BY_OUT>
struct TermGroups {
    using T = Canon<LIN, LOUT>;
    static constexpr int NS = BY_OUT ? T::DOUT : T::DIN;
    static constexpr std::array<int, NS + 1> make_start() {
        std::array<int, NS + 1> st{};
        for (int t = 0; t < T::NT; ++t) st[(BY_OUT ? T::terms[t].o : T::terms[t].i) + 1]++;
        for (int s = 0; s < NS; ++s) st[s + 1] += st[s];
        return st;
    }
    static constexpr std::array<int, NS + 1> start = make_start();
    static constexpr std::array<Term, T::NT> make_sorted() {
        std::array<Term, T::NT> out{};
        std::array<int, NS> fill{};
        for (int t = 0; t < T::NT; ++t) {
            const int s = BY_OUT ? T::terms[t].o : T::terms[t].i;
            out[start[s] + fill[s]++] = T::terms[t];
        }
        return out;
    }
    static constexpr std::array<Term, T::NT> sorted = make_sorted();
    static constexpr int count(int s) { return start[s + 1] - start[s]; }
    // last group (in increasing group order) that uses radial weight w
    static constexpr std::array<int, T::WD> make_last() {
        std::array<int, T::WD> l{};
        for (int w = 0; w < T::WD; ++w) l[w] = -1;
        for (int t = 0; t < T::NT; ++t) {
            const int s = BY_OUT ? T::terms[t].o : T::terms[t].i;
            if (s > l[T::terms[t].w]) l[T::terms[t].w] = s;
        }
        return l;
    }
    static constexpr std::array<int, T::WD> last = make_last();
};

}  // namespace
}  // namespace feq

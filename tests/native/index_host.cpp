// Host build of the device index code (na_common.h): the same window rule,
// neighbour enumeration and inverse (key -> queries) enumeration the kernels
// run, exported for the CPU tests through ctypes.
#include <cstdint>
#include <set>
#include <tuple>

#include "na_common.h"

namespace {

na::Prob make(const natten_problem_t* p) {
    na::Prob P{};
    P.B = 1; P.Hq = 1; P.Hkv = 1; P.rep = 1; P.Dqk = 1; P.Dv = 1;
    P.kv = 1; P.nout = 1; P.nkey = 1;
    for (int a = 0; a < 3; ++a) {
        P.ax[a] = {p->length[a], p->out_length[a], p->kernel[a], p->dilation[a], p->stride[a], p->causal[a]};
        P.kv *= p->kernel[a];
        P.nout *= p->out_length[a];
        P.nkey *= p->length[a];
    }
    return P;
}

}  // namespace

extern "C" {

int host_window_start(int i, int L, int K, int d) { return na::window_start(i, L, K, d); }

// flat[o, e] and valid[o, e] exactly as the device map kernel defines them,
// but built from for_each_neighbor (the enumeration the attention kernels use).
void host_neighbor_map(const natten_problem_t* p, int64_t* flat, uint8_t* valid) {
    const na::Prob P = make(p);
    long long o = 0;
    for (int o0 = 0; o0 < P.ax[0].out; ++o0)
        for (int o1 = 0; o1 < P.ax[1].out; ++o1)
            for (int o2 = 0; o2 < P.ax[2].out; ++o2, ++o) {
                const int i0 = o0 * P.ax[0].st, i1 = o1 * P.ax[1].st, i2 = o2 * P.ax[2].st;
                na::for_each_neighbor(P, i0, i1, i2, [&](int j0, int j1, int j2, int e, bool ok) {
                    auto clamp = [](int j, int L) { return j < 0 ? 0 : (j > L - 1 ? L - 1 : j); };
                    const int c0 = clamp(j0, P.ax[0].len), c1 = clamp(j1, P.ax[1].len), c2 = clamp(j2, P.ax[2].len);
                    flat[o * P.kv + e] = (static_cast<int64_t>(c0) * P.ax[1].len + c1) * P.ax[2].len + c2;
                    valid[o * P.kv + e] = ok ? 1 : 0;
                });
            }
}

// Number of (query, neighbour, key) triples on which the forward enumeration
// (query -> neighbours, valid only) and the inverse enumeration (key ->
// queries) disagree.  0 means the gradient kernels visit exactly the pairs
// the forward kernels use.
long long host_inverse_mismatch(const natten_problem_t* p) {
    const na::Prob P = make(p);
    std::set<std::tuple<int, int, int, int, int, int, int>> fwd, inv;
    for (int o0 = 0; o0 < P.ax[0].out; ++o0)
        for (int o1 = 0; o1 < P.ax[1].out; ++o1)
            for (int o2 = 0; o2 < P.ax[2].out; ++o2) {
                const int i0 = o0 * P.ax[0].st, i1 = o1 * P.ax[1].st, i2 = o2 * P.ax[2].st;
                na::for_each_neighbor(P, i0, i1, i2, [&](int j0, int j1, int j2, int e, bool ok) {
                    if (ok) fwd.insert({o0, o1, o2, e, j0, j1, j2});
                });
            }
    for (int m0 = 0; m0 < P.ax[0].len; ++m0)
        for (int m1 = 0; m1 < P.ax[1].len; ++m1)
            for (int m2 = 0; m2 < P.ax[2].len; ++m2)
                na::for_each_query(P, m0, m1, m2, [&](int o0, int o1, int o2, int, int, int, int e) {
                    inv.insert({o0, o1, o2, e, m0, m1, m2});
                });
    long long bad = 0;
    for (auto& t : fwd) bad += inv.count(t) ? 0 : 1;
    for (auto& t : inv) bad += fwd.count(t) ? 0 : 1;
    return bad;
}

// Class-coordinate closed forms (class_ws, class_span) against the window
// rule on positions and brute-force membership, for every residue class of
// axis 2.  Returns the number of disagreements.
long long host_class_mismatch(const natten_problem_t* p) {
    const na::Prob P = make(p);
    const na::Axis& A = P.ax[2];
    long long bad = 0;
    for (int r = 0; r < A.dil; ++r) {
        const na::ClassAxis c = na::class_axis(A, r);
        if (c.n != (A.len - r + A.dil - 1) / A.dil) ++bad;
        for (int j = 0; j < c.n; ++j) {
            const int want = (na::axis_first(A, r + j * A.dil) - r) / A.dil;
            if (na::class_ws(c, j) != want) ++bad;
        }
        for (int u = 0; u < c.n; ++u) {
            int lo, hi;
            na::class_span(c, u, lo, hi);
            for (int j = 0; j < c.n; ++j) {
                const int ws = na::class_ws(c, j);
                const bool member = u >= ws && u <= ws + A.k - 1 && u >= 0;
                const bool in = j >= lo && j <= hi;
                if (member != in) ++bad;
            }
        }
    }
    return bad;
}

}  // extern "C"

extern "C" {

// Number of n in [0, n_max) (stepping by `step`, plus the last 4096 below
// n_max) for which the multiply-high division disagrees with n / d.
long long host_fastdiv_errors(uint32_t d, int n_max, int step) {
    const na::FastDiv f = na::make_fastdiv(d);
    long long bad = 0;
    for (long long n = 0; n < n_max; n += step)
        if (na::fdiv(static_cast<int>(n), f) != static_cast<int>(n / d)) ++bad;
    for (long long n = n_max > 4096 ? n_max - 4096 : 0; n < n_max; ++n)
        if (na::fdiv(static_cast<int>(n), f) != static_cast<int>(n / d)) ++bad;
    return bad;
}

}  // extern "C"

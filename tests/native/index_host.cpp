// Host build of the device index code (na_common.h): the same window rule,
// neighbour enumeration and inverse (key -> queries) enumeration the kernels
// run, exported for the CPU tests through ctypes.
#include <algorithm>
#include <cstdint>
#include <set>
#include <tuple>
#include <vector>

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

// Query-item closed forms (query_ws, query_span) on axis 2 against the
// window rule at position stride * t and brute-force membership; the axis
// has dilation 1 when strided.  Returns the number of disagreements.
long long host_query_item_mismatch(const natten_problem_t* p) {
    const na::Prob P = make(p);
    const na::Axis& A = P.ax[2];
    long long bad = 0;
    for (int r = 0; r < A.dil; ++r) {
        const na::ClassAxis c = na::class_axis(A, r);
        const int nq = na::query_items(A, c.n);
        if (nq != (A.st == 1 ? c.n : A.out)) ++bad;
        for (int t = 0; t < nq; ++t) {
            const int want = (na::axis_first(A, r + t * A.st * A.dil) - r) / A.dil;
            if (A.st > 1 && na::query_ws(c, t) != want) ++bad;
        }
        for (int u = 0; u < c.n; ++u) {
            int lo, hi;
            na::query_span(c, u, lo, hi);
            for (int t = 0; t < nq; ++t) {
                const int f = na::axis_first(A, r + t * A.st * A.dil);
                const int m = r + u * A.dil;
                const bool member = m >= f && m <= f + (A.k - 1) * A.dil && (m - f) % A.dil == 0;
                const bool in = t >= lo && t <= hi;
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

extern "C" {

// Tile geometry (axis_geometry, shared by the host-built tables and the
// kernels) against brute force on one axis: for every residue class, tile
// of T items and wave item range [wl, wh], the union box must equal the
// min/max of the coordinates the tile's items need (their window members,
// or the query items attending a key) and the wave box must contain what
// the wave's items need, equal to it when every key is attended.  With
// stride s > 1 (dilation 1) query item t is the query at position s*t.
// Returns the number of mismatches.
long long host_tile_geometry_mismatch(int L, int K, int d, int causal, int T, int key, int s) {
    const int out = (L + s - 1) / s;
    na::Axis A{L, out, K, d, s, causal};
    long long bad = 0;
    const na::FastDiv fd = na::make_fastdiv(static_cast<uint32_t>(d));
    for (int r = 0; r < d && r < L; ++r) {
        const int n = (L - r + d - 1) / d;
        const int nq = s == 1 ? n : out;
        const int items = key ? n : nq;
        // coordinates needed by item j: [need_lo[j], need_hi[j]]
        std::vector<int> need_lo(items, 1 << 30), need_hi(items, -(1 << 30));
        for (int qj = 0; qj < nq; ++qj) {
            const int i = r + qj * s * d;
            const int f = na::axis_first(A, i);
            for (int x = 0; x < K; ++x) {
                const int m = f + x * d;
                if (m < 0 || m >= L) continue;
                const int mj = (m - r) / d;
                const int item = key ? mj : qj, other = key ? qj : mj;
                need_lo[item] = std::min(need_lo[item], other);
                need_hi[item] = std::max(need_hi[item], other);
            }
        }
        bool all_attended = true;
        for (int j = 0; j < items; ++j) all_attended = all_attended && need_lo[j] <= need_hi[j];
        for (int t = 0; t * T < items; ++t) {
            for (int wl = 0; wl < T; ++wl)
                for (int wh = wl; wh < T; ++wh) {
                    const na::AxisGeo g =
                        na::axis_geometry(L, K, d, causal, L % d, s, out, T, t, r, wl, wh, key != 0, fd);
                    const int J = t * T, E = std::min(T, items - J);
                    if (g.J != J || g.E != E || g.n != n || !g.tile_ok) { ++bad; continue; }
                    int ulo = 1 << 30, uhi = -(1 << 30);
                    for (int j = J; j < J + E; ++j) {
                        ulo = std::min(ulo, need_lo[j]);
                        uhi = std::max(uhi, need_hi[j]);
                    }
                    if (ulo <= uhi && (g.lo != ulo || g.U != uhi - ulo + 1)) { ++bad; continue; }
                    const int whc = std::min(wh, E - 1);
                    int blo = 1 << 30, bhi = -(1 << 30);
                    for (int j = J + wl; j <= J + whc; ++j) {
                        blo = std::min(blo, need_lo[j]);
                        bhi = std::max(bhi, need_hi[j]);
                    }
                    const bool has = blo <= bhi;
                    if (!has) continue;
                    const int rlo = blo - g.lo, rhi = bhi - g.lo;
                    if (!g.wave_ok || g.glo > rlo || g.ghi < rhi) { ++bad; continue; }
                    if (all_attended && (g.glo != rlo || g.ghi != rhi)) ++bad;
                }
        }
    }
    return bad;
}

}  // extern "C"

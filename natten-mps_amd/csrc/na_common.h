// Shared device-side definitions for the neighbourhood-attention kernels:
// problem descriptors, the window rule, element conversion and vector I/O.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "natten_hip.h"

namespace na {

// ---------------------------------------------------------------------------
// Problem description passed by value to every kernel.
// ---------------------------------------------------------------------------

struct Axis {
    int len;     // key/value extent
    int out;     // number of query positions
    int k;       // kernel size
    int dil;     // dilation
    int st;      // stride
    int causal;  // 0 / 1
};

struct Prob {
    int B, Hq, Hkv, rep;   // rep = Hq / Hkv
    int Dqk, Dv;
    int has_scale;
    float scale;
    Axis ax[3];
    int kv;                // K0*K1*K2
    int nout;              // out0*out1*out2
    int nkey;              // len0*len1*len2
};

struct Lay {
    long long b, s0, s1, s2, h;
    __host__ __device__ long long at(int bb, int p0, int p1, int p2, int hh) const {
        return bb * b + p0 * s0 + p1 * s1 + p2 * s2 + hh * h;
    }
};

// ---------------------------------------------------------------------------
// Window rule.  Non-causal start of the window of query position i on an axis
// of length L, kernel K, dilation d (utils/window.py:91-111 of the
// reference): centred, shifted inwards at the borders, and for d > 1 kept on
// the residue class of i.  Causal windows start at i-(K-1)d and are clipped
// by validity (j >= 0) rather than shifted.
// ---------------------------------------------------------------------------

__host__ __device__ inline int window_start(int i, int L, int K, int d) {
    const int half = K / 2;
    if (d <= 1) {
        int s = i - half;
        if (s < 0) s = 0;
        if (i + half >= L) s += L - i - half - 1;
        return s;
    }
    if (i - half * d < 0) return i % d;
    if (i + half * d >= L) {
        const int r = i % d;
        const int full = (L / d) * d;
        const int tail = L - full;
        return (r < tail) ? (L - tail + r - 2 * half * d) : (full + r - K * d);
    }
    return i - half * d;
}

__host__ __device__ inline int axis_first(const Axis& a, int i) {
    return a.causal ? i - (a.k - 1) * a.dil : window_start(i, a.len, a.k, a.dil);
}

// Range [t_lo, t_hi] of offsets t such that query position i = m + t*dil has
// key position m inside its window (and is inside the axis).  Window starts
// are non-decreasing along a residue class, so the set is contiguous in t.
// Returns false when empty.  The caller still filters by stride and out.
// A non-causal window lies within K*dil of its query (an even kernel at the
// right border does not contain the query itself), hence t in [-K, K].
__host__ __device__ inline bool axis_query_range(const Axis& a, int m, int& t_lo, int& t_hi) {
    int lo = a.causal ? 0 : -a.k;
    int hi = a.causal ? a.k - 1 : a.k;
    // clip to 0 <= m + t*dil < len
    while (lo <= hi && m + lo * a.dil < 0) ++lo;
    while (hi >= lo && m + hi * a.dil >= a.len) --hi;
    if (a.causal) { t_lo = lo; t_hi = hi; return lo <= hi; }
    while (lo <= hi) {
        const int i = m + lo * a.dil;
        const int f = window_start(i, a.len, a.k, a.dil);
        if (m <= f + (a.k - 1) * a.dil) break;  // m >= f holds on this side
        ++lo;
    }
    while (hi >= lo) {
        const int i = m + hi * a.dil;
        const int f = window_start(i, a.len, a.k, a.dil);
        if (m >= f) break;
        --hi;
    }
    t_lo = lo; t_hi = hi;
    return lo <= hi;
}

// Division by an invariant d >= 1 of 0 <= n < 2^31 with one multiply-high:
// with l = ceil(log2 d) and m = floor(2^32 (2^l - d) / d) + 1,
//   n / d = (mulhi(n, m) + n) >> l
// (the round-up method of Granlund and Montgomery, "Division by invariant
// integers using multiplication", 1994; n + mulhi stays below 2^32 for
// n < 2^31).  The kernels decode workgroup indices with it, in scalar
// registers, instead of the emulated integer division.
struct FastDiv {
    uint32_t mul, shift, d;
};

inline FastDiv make_fastdiv(uint32_t d) {
    uint32_t l = 0;
    while ((1ull << l) < d) ++l;
    const uint64_t m = ((1ull << 32) * ((1ull << l) - d)) / d + 1;
    return FastDiv{static_cast<uint32_t>(m), l, d};
}

__host__ __device__ inline int fdiv(int n, const FastDiv& f) {
    const uint32_t u = static_cast<uint32_t>(n);
    const uint32_t hi = static_cast<uint32_t>((static_cast<uint64_t>(u) * f.mul) >> 32);
    return static_cast<int>((hi + u) >> f.shift);
}

// Residue-class view of one axis.  With dilation d the positions r, r+d, ...
// form class r with n = ceil((L - r)/d) members; a window never leaves its
// class and, in class coordinates j = (i - r)/d, is the undilated run
// [ws(j), ws(j) + K - 1].  The window rule above becomes, with h = K/2:
//   causal:      ws(j) = j - (K - 1)
//   non-causal:  ws(j) = 0 for j < h;  B for j + h >= n;  j - h otherwise,
// with B = n - 1 - 2h when d == 1 or r < L % d, and B = n - K otherwise (the
// two agree for odd K).  No divisions: kernels evaluate it per lane.
//
// Queries: with stride s (the tile kernels take s > 1 only with d == 1, so
// the axis is one class) the query items t = 0 .. ceil(n/s)-1 sit at class
// coordinates qs*t, qs = s; with s == 1 items and class coordinates agree.
struct ClassAxis {
    int n, K, h, B, causal;
    int qs;  // query step
};

__host__ __device__ inline ClassAxis class_axis(const Axis& a, int r) {
    ClassAxis c;
    c.n = (a.len - r + a.dil - 1) / a.dil;
    c.K = a.k;
    c.h = a.k / 2;
    c.causal = a.causal;
    c.B = (a.dil == 1 || r < a.len % a.dil) ? c.n - 1 - 2 * c.h : c.n - a.k;
    c.qs = a.st;
    return c;
}

__host__ __device__ inline int class_ws(const ClassAxis& c, int j) {
    if (c.causal) return j - (c.K - 1);
    if (j < c.h) return 0;
    if (j + c.h >= c.n) return c.B;
    return j - c.h;
}

// Class range [jlo, jhi] of the queries whose windows hold key u (empty when
// jlo > jhi).  ws is non-decreasing, so {j : ws(j) <= u} is a prefix and
// {j : ws(j) + K - 1 >= u} a suffix of the class.
__host__ __device__ inline void class_span(const ClassAxis& c, int u, int& jlo, int& jhi) {
    if (c.causal) {
        jlo = u;
        jhi = u + c.K - 1 < c.n - 1 ? u + c.K - 1 : c.n - 1;
        return;
    }
    jhi = u >= c.B ? c.n - 1 : u + c.h;
    const int v = u - c.K + 1;  // smallest j with ws(j) >= v
    if (v <= 0)
        jlo = 0;
    else if (v + c.h < c.n - c.h)
        jlo = v + c.h;
    else
        jlo = c.B >= v ? c.n - c.h : c.n;
}

// Window start of query item t.
__host__ __device__ inline int query_ws(const ClassAxis& c, int t) { return class_ws(c, c.qs * t); }

// Query items [tlo, thi] whose windows hold key u (empty when tlo > thi): the
// class span's members at multiples of qs.  The span lies in [0, n], so
// thi <= (n-1)/qs, the last item.
__host__ __device__ inline void query_span(const ClassAxis& c, int u, int& tlo, int& thi) {
    class_span(c, u, tlo, thi);
    if (c.qs != 1) {
        tlo = (tlo + c.qs - 1) / c.qs;
        thi = thi / c.qs;
    }
}

// Query items on an axis: ceil(n/qs), which is the axis's output extent.
__host__ __device__ inline int query_items(const Axis& a, int n) { return a.st == 1 ? n : a.out; }

// Admissible box of a query item (its window) or key (its attending query
// items) in class coordinates.
__host__ __device__ inline void item_box(const ClassAxis& c, int j, bool key_side, int& lo, int& hi) {
    if (!key_side) {
        lo = query_ws(c, j);
        hi = lo + c.K - 1;
    } else {
        query_span(c, j, lo, hi);
    }
}

__host__ __device__ inline int imin(int a, int b) { return a < b ? a : b; }
__host__ __device__ inline int imax(int a, int b) { return a > b ? a : b; }

// One axis of a tile: class (n, B) of residue r, tile origin J = tT, clipped
// extent E, the union [lo, lo+U) of its queries' windows (key: of the
// queries attending its keys), and the admissible box [glo, ghi] of the
// wave's items [wl, wh] (union-relative, clipped to the union).  Window ends
// are non-decreasing along the axis, so the box follows from its corners.
struct AxisGeo {
    int J, E, lo, U, n, B, glo, ghi, tile_ok, wave_ok;
};

__host__ __device__ inline AxisGeo axis_geometry(int len, int K, int dil, int causal, int lenmod, int st, int out,
                                                 int T, int t, int r, int wl, int wh, bool key, const FastDiv& fd) {
    AxisGeo o;
    ClassAxis c;
    c.n = dil == 1 ? len : fdiv(len - r + dil - 1, fd);
    c.K = K;
    c.h = K >> 1;
    c.causal = causal;
    c.B = (dil == 1 || r < lenmod) ? c.n - 1 - 2 * c.h : c.n - K;
    c.qs = st;
    o.n = c.n;
    o.B = c.B;
    o.J = t * T;
    const int jend = imin(o.J + T, key || st == 1 ? c.n : out) - 1;
    o.E = jend - o.J + 1;
    int lo, hi;
    if (!key) {
        lo = imax(query_ws(c, o.J), 0);
        hi = imin(query_ws(c, jend) + K - 1, c.n - 1);
    } else {
        // both span ends are non-decreasing in the key; keys attended by
        // nobody (past the last window at an even-kernel border, or at the
        // end of a strided axis) leave hi unchanged
        int x2;
        query_span(c, o.J, lo, x2);
        query_span(c, jend, x2, hi);
    }
    o.lo = lo;
    o.U = hi >= lo ? hi - lo + 1 : 0;
    const int whc = imin(wh, o.E - 1);
    int bl, bh, el, eh;
    item_box(c, o.J + wl, key, bl, bh);
    item_box(c, o.J + imax(whc, wl), key, el, eh);
    o.glo = imax(bl - lo, 0);
    o.ghi = imin(eh - lo, o.U - 1);
    o.tile_ok = o.E > 0 ? 1 : 0;
    o.wave_ok = (wl <= whc && o.glo <= o.ghi) ? 1 : 0;
    return o;
}

// f(j0, j1, j2, e, valid) for each neighbour e (row-major over the kernel) of
// the query at (i0, i1, i2).  Invalid (causal) neighbours have j < 0 on some
// axis and must not be dereferenced.
template <class F>
__host__ __device__ inline void for_each_neighbor(const Prob& p, int i0, int i1, int i2, F&& f) {
    const Axis &A0 = p.ax[0], &A1 = p.ax[1], &A2 = p.ax[2];
    const int f0 = axis_first(A0, i0), f1 = axis_first(A1, i1), f2 = axis_first(A2, i2);
    int e = 0;
    for (int x = 0; x < A0.k; ++x) {
        const int j0 = f0 + x * A0.dil;
        for (int y = 0; y < A1.k; ++y) {
            const int j1 = f1 + y * A1.dil;
            for (int z = 0; z < A2.k; ++z, ++e) {
                const int j2 = f2 + z * A2.dil;
                f(j0, j1, j2, e, (j0 >= 0) & (j1 >= 0) & (j2 >= 0));
            }
        }
    }
}

// f(o0, o1, o2, i0, i1, i2, e) for every query (output index o, position i)
// whose window holds the key at (m0, m1, m2) as neighbour e (valid pairs only).
template <class F>
__host__ __device__ inline void for_each_query(const Prob& p, int m0, int m1, int m2, F&& f) {
    const Axis &A0 = p.ax[0], &A1 = p.ax[1], &A2 = p.ax[2];
    int l0, h0, l1, h1, l2, h2;
    if (!axis_query_range(A0, m0, l0, h0)) return;
    if (!axis_query_range(A1, m1, l1, h1)) return;
    if (!axis_query_range(A2, m2, l2, h2)) return;
    for (int t0 = l0; t0 <= h0; ++t0) {
        const int i0 = m0 + t0 * A0.dil;
        if (i0 % A0.st) continue;
        const int o0 = i0 / A0.st;
        if (o0 >= A0.out) continue;
        const int x = (m0 - axis_first(A0, i0)) / A0.dil;
        for (int t1 = l1; t1 <= h1; ++t1) {
            const int i1 = m1 + t1 * A1.dil;
            if (i1 % A1.st) continue;
            const int o1 = i1 / A1.st;
            if (o1 >= A1.out) continue;
            const int y = (m1 - axis_first(A1, i1)) / A1.dil;
            for (int t2 = l2; t2 <= h2; ++t2) {
                const int i2 = m2 + t2 * A2.dil;
                if (i2 % A2.st) continue;
                const int o2 = i2 / A2.st;
                if (o2 >= A2.out) continue;
                const int z = (m2 - axis_first(A2, i2)) / A2.dil;
                f(o0, o1, o2, i0, i1, i2, (x * A1.k + y) * A2.k + z);
            }
        }
    }
}

// Split iteration for latency-bound vector kernels: `split` lane groups share
// one query (key); group `sp` takes every split-th index of the outermost
// axis whose kernel extent exceeds 1, so each group walks about 1/split of
// the neighbours (attending queries) and the loads of the groups are in
// flight together.  The callers combine the groups' partial results.
__host__ __device__ inline int split_axis(const Prob& p) {
    return p.ax[0].k > 1 ? 0 : p.ax[1].k > 1 ? 1 : 2;
}

template <class F>
__device__ __forceinline__ void for_each_neighbor_split(const Prob& p, int i0, int i1, int i2, int sp, int split,
                                                        F&& f) {
    const Axis &A0 = p.ax[0], &A1 = p.ax[1], &A2 = p.ax[2];
    const int f0 = axis_first(A0, i0), f1 = axis_first(A1, i1), f2 = axis_first(A2, i2);
    const int sa = split_axis(p);
    const int x0 = sa == 0 ? sp : 0, xs = sa == 0 ? split : 1;
    const int y0 = sa == 1 ? sp : 0, ys = sa == 1 ? split : 1;
    const int z0 = sa == 2 ? sp : 0, zs = sa == 2 ? split : 1;
    for (int x = x0; x < A0.k; x += xs) {
        const int j0 = f0 + x * A0.dil;
        for (int y = y0; y < A1.k; y += ys) {
            const int j1 = f1 + y * A1.dil;
            for (int z = z0; z < A2.k; z += zs) {
                const int j2 = f2 + z * A2.dil;
                f(j0, j1, j2, (x * A1.k + y) * A2.k + z, (j0 >= 0) & (j1 >= 0) & (j2 >= 0));
            }
        }
    }
}

template <class F>
__device__ __forceinline__ void for_each_query_split(const Prob& p, int m0, int m1, int m2, int sp, int split,
                                                     F&& f) {
    const Axis &A0 = p.ax[0], &A1 = p.ax[1], &A2 = p.ax[2];
    int l0, h0, l1, h1, l2, h2;
    if (!axis_query_range(A0, m0, l0, h0)) return;
    if (!axis_query_range(A1, m1, l1, h1)) return;
    if (!axis_query_range(A2, m2, l2, h2)) return;
    const int sa = split_axis(p);
    const int s0 = sa == 0 ? split : 1, s1 = sa == 1 ? split : 1, s2 = sa == 2 ? split : 1;
    for (int t0 = l0 + (sa == 0 ? sp : 0); t0 <= h0; t0 += s0) {
        const int i0 = m0 + t0 * A0.dil;
        if (i0 % A0.st) continue;
        const int o0 = i0 / A0.st;
        if (o0 >= A0.out) continue;
        const int x = (m0 - axis_first(A0, i0)) / A0.dil;
        for (int t1 = l1 + (sa == 1 ? sp : 0); t1 <= h1; t1 += s1) {
            const int i1 = m1 + t1 * A1.dil;
            if (i1 % A1.st) continue;
            const int o1 = i1 / A1.st;
            if (o1 >= A1.out) continue;
            const int y = (m1 - axis_first(A1, i1)) / A1.dil;
            for (int t2 = l2 + (sa == 2 ? sp : 0); t2 <= h2; t2 += s2) {
                const int i2 = m2 + t2 * A2.dil;
                if (i2 % A2.st) continue;
                const int o2 = i2 / A2.st;
                if (o2 >= A2.out) continue;
                const int z = (m2 - axis_first(A2, i2)) / A2.dil;
                f(o0, o1, o2, i0, i1, i2, (x * A1.k + y) * A2.k + z);
            }
        }
    }
}

// NATTEN 0.17's relative-position-bias start (get_pb_start) of query i on an
// axis of length len, kernel K, dilation d (extras/allin1/reference_impl.py:30-41):
// the bias index of the query's neighbour e along the axis is start + e.
__host__ __device__ inline int pb_start(int i, int len, int K, int d) {
    const int nh = K / 2;
    if (d <= 1) return nh + (i < nh ? nh - i : 0) + (i + nh >= len ? len - i - 1 - nh : 0);
    if (i - nh * d < 0) return K - 1 - i / d;
    if (i + nh * d >= len) return (len - i - 1) / d;
    return nh;
}

// ---------------------------------------------------------------------------
// Element types.  bf16 is carried as raw bits; fp32 -> bf16 rounds to nearest
// even with NaN kept quiet, the same rounding torch uses.
// ---------------------------------------------------------------------------

struct bf16 { uint16_t x; };
using f16 = _Float16;

__device__ __forceinline__ float to_f(float v) { return v; }
__device__ __forceinline__ float to_f(f16 v) { return static_cast<float>(v); }
__device__ __forceinline__ float to_f(bf16 v) { return __uint_as_float(static_cast<uint32_t>(v.x) << 16); }

template <typename T> __device__ __forceinline__ T from_f(float f);
template <> __device__ __forceinline__ float from_f<float>(float f) { return f; }
template <> __device__ __forceinline__ f16 from_f<f16>(float f) { return static_cast<f16>(f); }
template <> __device__ __forceinline__ bf16 from_f<bf16>(float f) {
    uint32_t u = __float_as_uint(f);
    bf16 r;
    if ((u & 0x7fffffffu) > 0x7f800000u) { r.x = static_cast<uint16_t>((u >> 16) | 0x40u); return r; }
    u += 0x7fffu + ((u >> 16) & 1u);
    r.x = static_cast<uint16_t>(u >> 16);
    return r;
}

// N consecutive elements starting at p[d0], converted to float.  `vec` means
// p + d0 is aligned to N*sizeof(T) bytes and D % N == 0 (so d0 < D implies the
// whole run is in range).  Otherwise a guarded scalar path.
template <typename T, int N>
__device__ __forceinline__ void load_run(const T* __restrict__ p, int d0, int D, bool vec, float (&out)[N]) {
    if (vec) {
        if (d0 < D) {
            constexpr int NW = (N * (int)sizeof(T)) / 16;
            static_assert(NW >= 1, "run must cover at least 16 bytes");
            uint4 raw[NW];
            const uint4* src = reinterpret_cast<const uint4*>(p + d0);
#pragma unroll
            for (int w = 0; w < NW; ++w) raw[w] = src[w];
            const T* e = reinterpret_cast<const T*>(raw);
#pragma unroll
            for (int j = 0; j < N; ++j) out[j] = to_f(e[j]);
        } else {
#pragma unroll
            for (int j = 0; j < N; ++j) out[j] = 0.f;
        }
    } else {
#pragma unroll
        for (int j = 0; j < N; ++j) out[j] = (d0 + j < D) ? to_f(p[d0 + j]) : 0.f;
    }
}

template <typename T, int N>
__device__ __forceinline__ void store_run(T* __restrict__ p, int d0, int D, bool vec, const float (&in)[N]) {
    if (vec) {
        if (d0 < D) {
            constexpr int NW = (N * (int)sizeof(T)) / 16;
            T e[N];
#pragma unroll
            for (int j = 0; j < N; ++j) e[j] = from_f<T>(in[j]);
            const uint4* src = reinterpret_cast<const uint4*>(e);
            uint4* dst = reinterpret_cast<uint4*>(p + d0);
#pragma unroll
            for (int w = 0; w < NW; ++w) dst[w] = src[w];
        }
    } else {
#pragma unroll
        for (int j = 0; j < N; ++j)
            if (d0 + j < D) p[d0 + j] = from_f<T>(in[j]);
    }
}

// Sum over the LPQ consecutive lanes that share one query.
template <int LPQ>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int m = LPQ / 2; m >= 1; m >>= 1) v += __shfl_xor(v, m, LPQ);
    return v;
}

// Sum / max over the `split` lane groups (LPQ lanes each, consecutive) of
// one query or key, in a fixed butterfly order.
template <int LPQ>
__device__ __forceinline__ float split_sum(float v, int split) {
    for (int m = split >> 1; m >= 1; m >>= 1) v += __shfl_xor(v, m * LPQ);
    return v;
}

template <int LPQ>
__device__ __forceinline__ float split_max(float v, int split) {
    for (int m = split >> 1; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m * LPQ));
    return v;
}

// Workgroup barrier after ordinary LDS stores (ds_write) that other waves
// read next.  The compiler emits no LDS counter wait before a workgroup
// barrier (it takes LDS operations as ordered across waves); on MI355X a
// store issued just before the barrier was not always seen by another
// wave's read after it, so the wait is explicit here.
__device__ __forceinline__ void lds_publish_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __syncthreads();
}

// Blocks are dealt round-robin to the 8 XCDs; remap so that each XCD works on
// one contiguous range of logical blocks (neighbouring tiles share K/V lines in
// that XCD's L2).  Identity on the tail that does not fill all 8.
__device__ __forceinline__ int xcd_block(int bid, int nb) {
    const int per = nb >> 3;
    const int full = per << 3;
    if (bid >= full) return bid;
    return (bid & 7) * per + (bid >> 3);
}

}  // namespace na

// Exact per-item evaluation of the fused and split products, for the MFMA
// tile kernels.  A tile kernel computes every (query, slot) pair of its
// staged union and removes the pairs outside a query's window by arithmetic
// (a -inf bias or exponent offset, or a zero weight).  With finite inputs
// that is exact.  A NaN or Inf inside the union but outside an item's window
// can still reach the item, through 0 * Inf or -inf + Inf inside a product,
// and then always as NaN or Inf, never as a wrong finite value: it reaches
// either every dim of the item (through a probability or a score gradient)
// or only the dims that hold the non-finite element.  So every tile kernel
// checks each lane's part of its results and, where it is not finite,
// recomputes that lane's dims here from global memory over the item's true
// window (or the true set of queries attending it), in the reference's
// order of operations: logits scaled after the contraction, softmax as
// exp(s - max) over the sum.  With finite inputs none of this runs.
//
// The code is kept lean in registers, since a kernel's register budget is
// the maximum over all its code: windows in residue-class form (no
// divisions per neighbour), plain loops without unrolling.
//
// Each of the four lanes of an item (the MFMA column layout) evaluates full
// logits and keeps its own 4 * D/16 output dims: d = 16 db + 4 grp + i.
#pragma once

#include "na_common.h"

namespace na {

typedef float f32x4_t __attribute__((ext_vector_type(4)));

// a . b over D elements (16-byte aligned rows, D % 8 == 0), fp32 accumulation
// in element order.
template <typename T, int D>
__device__ __forceinline__ float exact_dot(const T* __restrict__ a, const T* __restrict__ b) {
    float s = 0.f;
    if constexpr (sizeof(T) == 4) {
#pragma unroll 1
        for (int c = 0; c < D; c += 4) {
            const float4 x = *reinterpret_cast<const float4*>(a + c);
            const float4 y = *reinterpret_cast<const float4*>(b + c);
            s = fmaf(x.x, y.x, s);
            s = fmaf(x.y, y.y, s);
            s = fmaf(x.z, y.z, s);
            s = fmaf(x.w, y.w, s);
        }
    } else {
#pragma unroll 1
        for (int c = 0; c < D; c += 8) {
            const uint4 x = *reinterpret_cast<const uint4*>(a + c);
            const uint4 y = *reinterpret_cast<const uint4*>(b + c);
            const T* xe = reinterpret_cast<const T*>(&x);
            const T* ye = reinterpret_cast<const T*>(&y);
#pragma unroll
            for (int e = 0; e < 8; ++e) s = fmaf(to_f(xe[e]), to_f(ye[e]), s);
        }
    }
    return s;
}

// acc += w * x over the lane's own dims of row x.
template <typename T, int D>
__device__ __forceinline__ void exact_axpy(float w, const T* __restrict__ x, int grp, f32x4_t (&acc)[D / 16]) {
#pragma unroll
    for (int db = 0; db < D / 16; ++db) {
        if constexpr (sizeof(T) == 4) {
            const float4 r = *reinterpret_cast<const float4*>(x + db * 16 + grp * 4);
            acc[db][0] = fmaf(w, r.x, acc[db][0]);
            acc[db][1] = fmaf(w, r.y, acc[db][1]);
            acc[db][2] = fmaf(w, r.z, acc[db][2]);
            acc[db][3] = fmaf(w, r.w, acc[db][3]);
        } else {
            const uint2 r = *reinterpret_cast<const uint2*>(x + db * 16 + grp * 4);
            const T* e = reinterpret_cast<const T*>(&r);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[db][i] = fmaf(w, to_f(e[i]), acc[db][i]);
        }
    }
}

template <int N>
__device__ __forceinline__ void exact_zero(f32x4_t (&acc)[N]) {
#pragma unroll
    for (int db = 0; db < N; ++db) acc[db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
}

// Element offset of position (i0, i1, i2) under spatial strides s.
struct Strides3 {
    int s0, s1, s2;
    __device__ __forceinline__ int at(int i0, int i1, int i2) const { return i0 * s0 + i1 * s1 + i2 * s2; }
};

// One axis of an item in residue-class form: residue r, class coordinate j,
// and the class's window rule.  A query item's j is its item index (the
// output index on a strided axis, which is one class).
struct ExactAxis {
    int r, j, dil;
    ClassAxis c;
};

__device__ __forceinline__ ExactAxis exact_axis(const Axis& A, int pos) {
    ExactAxis e;
    e.dil = A.dil;
    e.r = pos % A.dil;
    e.j = pos / A.dil;
    e.c = class_axis(A, e.r);
    return e;
}

// f(j0, j1, j2, e) over the valid neighbours of the query whose axes are x
// (e: kernel index, row-major over the axes).
template <class F>
__device__ __forceinline__ void exact_window(const ExactAxis (&x)[3], F&& f) {
    const int w0 = query_ws(x[0].c, x[0].j), w1 = query_ws(x[1].c, x[1].j), w2 = query_ws(x[2].c, x[2].j);
    const int K0 = x[0].c.K, K1 = x[1].c.K, K2 = x[2].c.K;
#pragma unroll 1
    for (int a = 0; a < K0; ++a) {
        if (w0 + a < 0) continue;
        const int j0 = x[0].r + (w0 + a) * x[0].dil;
#pragma unroll 1
        for (int b = 0; b < K1; ++b) {
            if (w1 + b < 0) continue;
            const int j1 = x[1].r + (w1 + b) * x[1].dil;
#pragma unroll 1
            for (int c = 0; c < K2; ++c) {
                if (w2 + c < 0) continue;
                f(j0, j1, x[2].r + (w2 + c) * x[2].dil, (a * K1 + b) * K2 + c);
            }
        }
    }
}

// f(i0, i1, i2, e) over the query items whose window holds the key whose
// axes are x, as their neighbour e; i is the item's output index (its
// position at stride 1).
template <class F>
__device__ __forceinline__ void exact_attending(const ExactAxis (&x)[3], F&& f) {
    int l0, h0, l1, h1, l2, h2;
    query_span(x[0].c, x[0].j, l0, h0);
    query_span(x[1].c, x[1].j, l1, h1);
    query_span(x[2].c, x[2].j, l2, h2);
    const int K1 = x[1].c.K, K2 = x[2].c.K;
#pragma unroll 1
    for (int a = l0; a <= h0; ++a) {
        const int i0 = x[0].r + a * x[0].dil, e0 = x[0].j - query_ws(x[0].c, a);
#pragma unroll 1
        for (int b = l1; b <= h1; ++b) {
            const int i1 = x[1].r + b * x[1].dil, e1 = x[1].j - query_ws(x[1].c, b);
#pragma unroll 1
            for (int c = l2; c <= h2; ++c)
                f(i0, i1, x[2].r + c * x[2].dil, (e0 * K1 + e1) * K2 + x[2].j - query_ws(x[2].c, c));
        }
    }
}

// Forward of one query: acc = softmax(scale q.k) v over its window (the
// normalised output), lse natural log.  kb, vb: (batch, kv head) bases.
template <typename T, int D>
__device__ __forceinline__ void exact_forward(float scale, const ExactAxis (&x)[3], const T* __restrict__ q_row,
                                              const T* __restrict__ kb, Strides3 ks, const T* __restrict__ vb,
                                              Strides3 vs, int grp, f32x4_t (&acc)[D / 16], float& lse) {
    float m = -INFINITY;
    exact_window(x, [&](int j0, int j1, int j2, int) {
        m = __builtin_elementwise_maximum(m, exact_dot<T, D>(q_row, kb + ks.at(j0, j1, j2)) * scale);
    });
    float l = 0.f;
    exact_zero(acc);
    exact_window(x, [&](int j0, int j1, int j2, int) {
        const float e = expf(exact_dot<T, D>(q_row, kb + ks.at(j0, j1, j2)) * scale - m);
        l += e;
        exact_axpy<T, D>(e, vb + vs.at(j0, j1, j2), grp, acc);
    });
    const float inv = 1.f / l;
#pragma unroll
    for (int db = 0; db < D / 16; ++db) acc[db] *= inv;
    lse = m + logf(l);
}

// Global keys of one (batch, kv head) for the exact paths: rows k + j * ks,
// v + j * vs, j < n (every query attends them besides its window).
template <typename T>
struct ExactGlobal {
    const T *k, *v;
    int ks, vs, n;
};

// exact_forward over the window and the global keys together.
template <typename T, int D>
__device__ __forceinline__ void exact_forward_global(float scale, const ExactAxis (&x)[3], const T* __restrict__ q_row,
                                                     const T* __restrict__ kb, Strides3 ks,
                                                     const T* __restrict__ vb, Strides3 vs,
                                                     const ExactGlobal<T>& g, int grp, f32x4_t (&acc)[D / 16],
                                                     float& lse) {
    float m = -INFINITY;
    exact_window(x, [&](int j0, int j1, int j2, int) {
        m = __builtin_elementwise_maximum(m, exact_dot<T, D>(q_row, kb + ks.at(j0, j1, j2)) * scale);
    });
#pragma unroll 1
    for (int j = 0; j < g.n; ++j)
        m = __builtin_elementwise_maximum(m, exact_dot<T, D>(q_row, g.k + j * g.ks) * scale);
    float l = 0.f;
    exact_zero(acc);
    exact_window(x, [&](int j0, int j1, int j2, int) {
        const float e = expf(exact_dot<T, D>(q_row, kb + ks.at(j0, j1, j2)) * scale - m);
        l += e;
        exact_axpy<T, D>(e, vb + vs.at(j0, j1, j2), grp, acc);
    });
#pragma unroll 1
    for (int j = 0; j < g.n; ++j) {
        const float e = expf(exact_dot<T, D>(q_row, g.k + j * g.ks) * scale - m);
        l += e;
        exact_axpy<T, D>(e, g.v + j * g.vs, grp, acc);
    }
    const float inv = 1.f / l;
#pragma unroll
    for (int db = 0; db < D / 16; ++db) acc[db] *= inv;
    lse = m + logf(l);
}

// Query side of the backward: acc = sum P (dP - delta) k over the window
// (times scale by the caller), P = exp(scale q.k - lse), dP = dO . v.
template <typename T, int D>
__device__ __forceinline__ void exact_backward_q(float scale, const ExactAxis (&x)[3], const T* __restrict__ q_row,
                                                 const T* __restrict__ do_row, float lse, float delta,
                                                 const T* __restrict__ kb, Strides3 ks, const T* __restrict__ vb,
                                                 Strides3 vs, int grp, f32x4_t (&acc)[D / 16]) {
    exact_zero(acc);
    exact_window(x, [&](int j0, int j1, int j2, int) {
        const T* kr = kb + ks.at(j0, j1, j2);
        const float pr = expf(exact_dot<T, D>(q_row, kr) * scale - lse);
        const float dp = exact_dot<T, D>(do_row, vb + vs.at(j0, j1, j2));
        exact_axpy<T, D>(pr * (dp - delta), kr, grp, acc);
    });
}

// exact_backward_q over the window and the global keys together.
template <typename T, int D>
__device__ __forceinline__ void exact_backward_q_global(float scale, const ExactAxis (&x)[3],
                                                        const T* __restrict__ q_row, const T* __restrict__ do_row,
                                                        float lse, float delta, const T* __restrict__ kb, Strides3 ks,
                                                        const T* __restrict__ vb, Strides3 vs,
                                                        const ExactGlobal<T>& g, int grp, f32x4_t (&acc)[D / 16]) {
    exact_backward_q<T, D>(scale, x, q_row, do_row, lse, delta, kb, ks, vb, vs, grp, acc);
#pragma unroll 1
    for (int j = 0; j < g.n; ++j) {
        const T* kr = g.k + j * g.ks;
        const float pr = expf(exact_dot<T, D>(q_row, kr) * scale - lse);
        const float dp = exact_dot<T, D>(do_row, g.v + j * g.vs);
        exact_axpy<T, D>(pr * (dp - delta), kr, grp, acc);
    }
}

// Key side of the backward for one key of one q head (the caller sums the
// q heads of its GQA group): over every query attending the key,
//   gv += P dO   (GV)   or   gk += P (dP - delta) q   (!GV; times scale by
// the caller).  One gradient per call keeps the accumulators to D/4 floats.
template <typename T, int D, bool GV>
__device__ __forceinline__ void exact_backward_kv(float scale, const ExactAxis (&x)[3], const T* __restrict__ k_row,
                                                  const T* __restrict__ v_row, const T* __restrict__ qb, Strides3 qs,
                                                  const T* __restrict__ dob, Strides3 dos,
                                                  const float* __restrict__ lseb, Strides3 ls,
                                                  const float* __restrict__ deb, Strides3 des, int grp,
                                                  f32x4_t (&g)[D / 16]) {
    exact_attending(x, [&](int i0, int i1, int i2, int) {
        const T* qr = qb + qs.at(i0, i1, i2);
        const T* dr = dob + dos.at(i0, i1, i2);
        const float pr = expf(exact_dot<T, D>(qr, k_row) * scale - lseb[ls.at(i0, i1, i2)]);
        if constexpr (GV) {
            exact_axpy<T, D>(pr, dr, grp, g);
        } else {
            const float dp = exact_dot<T, D>(dr, v_row);
            exact_axpy<T, D>(pr * (dp - deb[des.at(i0, i1, i2)]), qr, grp, g);
        }
    });
}

// Split products.  Query side: acc = sum over valid neighbours e of
// w_row[e] x[nbr(e)]; key side: acc = sum over the queries attending the key
// of w[q][e(q, key)] x[q] (times mul by the caller).
template <typename T, int D>
__device__ __forceinline__ void exact_wsum(const ExactAxis (&x)[3], const T* __restrict__ w_row,
                                           const T* __restrict__ xb, Strides3 xs, int grp, f32x4_t (&acc)[D / 16]) {
    exact_zero(acc);
    exact_window(x, [&](int j0, int j1, int j2, int e) {
        exact_axpy<T, D>(to_f(w_row[e]), xb + xs.at(j0, j1, j2), grp, acc);
    });
}

template <typename T, int D>
__device__ __forceinline__ void exact_wsum_key(const ExactAxis (&x)[3], const T* __restrict__ wb, Strides3 ws,
                                               const T* __restrict__ xb, Strides3 xs, int grp,
                                               f32x4_t (&acc)[D / 16]) {
    exact_zero(acc);
    exact_attending(x, [&](int i0, int i1, int i2, int e) {
        exact_axpy<T, D>(to_f(wb[ws.at(i0, i1, i2) + e]), xb + xs.at(i0, i1, i2), grp, acc);
    });
}

}  // namespace na

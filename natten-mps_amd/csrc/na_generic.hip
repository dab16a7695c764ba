// Generic neighbourhood-attention kernels: every rank (as three padded axes),
// dtype (fp32 / fp16 / bf16), kernel size, dilation, stride, causal mask and
// GQA ratio.  Vector-ALU (FMA) kernels with fp32 accumulation.
//
// Work mapping: a "group" of LPQ consecutive lanes owns one query (or one key,
// for the key-centric gradient kernels); each lane owns DPL consecutive head
// dims, so a group covers up to DPL*LPQ dims and dot products finish with a
// log2(LPQ)-step butterfly.  Queries are enumerated (b, o0, o1, o2, h) with the
// head fastest, so one wave reads whole [H, D] token rows.  K/V neighbours are
// read straight from global memory; the overlap between neighbouring windows
// is served by L1/L2 (blocks are remapped so each XCD walks a contiguous
// range).
#include <cstdlib>

#include "na_launch.h"

namespace na {

namespace {

struct QPos {
    int b, h, o0, o1, o2, i0, i1, i2;
};

__device__ __forceinline__ QPos decode_query(const Prob& p, long long qi) {
    QPos r;
    r.h = static_cast<int>(qi % p.Hq);
    long long t = qi / p.Hq;
    r.o2 = static_cast<int>(t % p.ax[2].out); t /= p.ax[2].out;
    r.o1 = static_cast<int>(t % p.ax[1].out); t /= p.ax[1].out;
    r.o0 = static_cast<int>(t % p.ax[0].out);
    r.b = static_cast<int>(t / p.ax[0].out);
    r.i0 = r.o0 * p.ax[0].st;
    r.i1 = r.o1 * p.ax[1].st;
    r.i2 = r.o2 * p.ax[2].st;
    return r;
}

struct KPos {
    int b, h, m0, m1, m2;
};

__device__ __forceinline__ KPos decode_key(const Prob& p, long long ki, int heads) {
    KPos r;
    r.h = static_cast<int>(ki % heads);
    long long t = ki / heads;
    r.m2 = static_cast<int>(t % p.ax[2].len); t /= p.ax[2].len;
    r.m1 = static_cast<int>(t % p.ax[1].len); t /= p.ax[1].len;
    r.m0 = static_cast<int>(t % p.ax[0].len);
    r.b = static_cast<int>(t / p.ax[0].len);
    return r;
}

__device__ __forceinline__ long long group_index(int lpq) {
    const int blk = xcd_block(blockIdx.x, gridDim.x);
    return (static_cast<long long>(blk) * blockDim.x + threadIdx.x) / lpq;
}

// Variable-length problems: lens[b * 3 + a] is sample b's extent on padded
// axis a (stride 1).  It replaces the problem's (maximum) extent in the window
// rule; positions past it are padding.  A sample whose extents fall outside
// [kernel * dilation, maximum], or hit the even-kernel-equal-to-length case,
// is all padding.  False: (i0, i1, i2) is padding for its sample.
__device__ __forceinline__ bool sample_extent(Prob& p, const int* __restrict__ lens, int b, int i0, int i1,
                                              int i2) {
    int L[3];
    bool ok = true;
#pragma unroll
    for (int a = 0; a < 3; ++a) {
        const Axis& A = p.ax[a];
        L[a] = lens[b * 3 + a];
        ok = ok && L[a] >= A.k * A.dil && L[a] <= A.len &&
             !(!A.causal && A.dil == 1 && (A.k % 2) == 0 && A.k == L[a]);
    }
    if (!ok || i0 >= L[0] || i1 >= L[1] || i2 >= L[2]) return false;
#pragma unroll
    for (int a = 0; a < 3; ++a) p.ax[a].len = p.ax[a].out = L[a];
    return true;
}

template <typename T, int DPL>
__device__ __forceinline__ void store_zero(T* g, int d0, int D, int vec) {
    float z[DPL];
#pragma unroll
    for (int j = 0; j < DPL; ++j) z[j] = 0.f;
    store_run<T, DPL>(g, d0, D, vec, z);
}

// ---------------------------------------------------------------------------
// Pipelined walks.  A group's walk over its neighbours (or attending
// queries) waits on each step's loads; with `walk_*_pipelined` the loads of
// the next U steps are already in flight.  `fetch` issues a step's loads and
// returns the raw registers (no use of the loaded values, so no wait), `use`
// consumes them, in the same order as the plain walk.  Only for 16-byte
// aligned runs (`vec`): lanes past the head dim read the row start and drop
// it when unpacking; masked (causal) neighbours load from a clamped position
// and are skipped by `use`.  fetch(j0, j1, j2, e) gets the neighbour's
// position and index, use(step, e, valid) its registers.
// ---------------------------------------------------------------------------
template <typename T, int N>
struct Raw {
    static constexpr int NW = (N * static_cast<int>(sizeof(T))) / 16;
    uint4 w[NW];
};

template <typename T, int N>
__device__ __forceinline__ Raw<T, N> fetch_run(const T* __restrict__ p, int d0, int D) {
    Raw<T, N> r;
    const uint4* src = reinterpret_cast<const uint4*>(p + (d0 < D ? d0 : 0));
#pragma unroll
    for (int w = 0; w < Raw<T, N>::NW; ++w) r.w[w] = src[w];
    return r;
}

template <typename T, int N>
__device__ __forceinline__ void unpack_run(const Raw<T, N>& r, int d0, int D, float (&out)[N]) {
    const T* e = reinterpret_cast<const T*>(r.w);
#pragma unroll
    for (int j = 0; j < N; ++j) out[j] = d0 < D ? to_f(e[j]) : 0.f;
}

// Steps in flight: about 8 runs of 16 bytes per lane.
template <typename T, int DPL, int RUNS>
constexpr int pipe_depth() {
    constexpr int w = Raw<T, DPL>::NW * RUNS;
    return w >= 4 ? 2 : 8 / w;
}

template <int U, class Fetch, class Use>
__device__ __forceinline__ void walk_neighbors_pipelined(const Prob& p, int i0, int i1, int i2, int sp, int split,
                                                         Fetch&& fetch, Use&& use) {
    const Axis &A0 = p.ax[0], &A1 = p.ax[1], &A2 = p.ax[2];
    const int f0 = axis_first(A0, i0), f1 = axis_first(A1, i1), f2 = axis_first(A2, i2);
    const int sa = split_axis(p);
    const int x0 = sa == 0 ? sp : 0, xs = sa == 0 ? split : 1;
    const int y0 = sa == 1 ? sp : 0, ys = sa == 1 ? split : 1;
    const int z0 = sa == 2 ? sp : 0, zs = sa == 2 ? split : 1;
    const int nx = x0 < A0.k ? (A0.k - x0 + xs - 1) / xs : 0;
    const int ny = y0 < A1.k ? (A1.k - y0 + ys - 1) / ys : 0;
    const int nz = z0 < A2.k ? (A2.k - z0 + zs - 1) / zs : 0;
    const int total = nx * ny * nz;
    using P = decltype(fetch(0, 0, 0, 0));
    int x = x0, y = y0, z = z0;
    // blocks of U steps: every fetch of a block is issued before the first
    // use, unconditionally (past the end the cursor stays on the last step),
    // so the compiler waits for each step's loads with the rest in flight
    for (int i = 0; i < total; i += U) {
        P buf[U];
        int eb[U];
        bool okb[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int j0 = f0 + x * A0.dil, j1 = f1 + y * A1.dil, j2 = f2 + z * A2.dil;
            okb[u] = (j0 >= 0) & (j1 >= 0) & (j2 >= 0);
            eb[u] = (x * A1.k + y) * A2.k + z;
            buf[u] = fetch(j0 < 0 ? 0 : j0, j1 < 0 ? 0 : j1, j2 < 0 ? 0 : j2, eb[u]);
            if (i + u + 1 < total) {
                if ((z += zs) >= A2.k) {
                    z = z0;
                    if ((y += ys) >= A1.k) {
                        y = y0;
                        x += xs;
                    }
                }
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
            if (i + u < total) use(buf[u], eb[u], okb[u]);
    }
}

// ---------------------------------------------------------------------------
// Fused forward with online softmax.
// ---------------------------------------------------------------------------
template <typename T, int DPL, int LPQ>
__global__ __launch_bounds__(256) void k_forward(Prob p, int vec, int split, const int* __restrict__ lens,
                                                 const T* __restrict__ q, Lay lq,
                                                 const T* __restrict__ k, Lay lk,
                                                 const T* __restrict__ v, Lay lv,
                                                 T* __restrict__ out, Lay lo,
                                                 float* __restrict__ lse, Lay ll) {
    const long long qi = group_index(LPQ * split);
    if (qi >= static_cast<long long>(p.B) * p.nout * p.Hq) return;
    const int d0 = (threadIdx.x % LPQ) * DPL;
    const int sp = (threadIdx.x / LPQ) % split;
    const QPos Q = decode_query(p, qi);
    const int hk = Q.h / p.rep;
    if (lens && !sample_extent(p, lens, Q.b, Q.i0, Q.i1, Q.i2)) {
        if (sp == 0) store_zero<T, DPL>(out + lo.at(Q.b, Q.o0, Q.o1, Q.o2, Q.h), d0, p.Dv, vec);
        if (sp == 0 && d0 == 0) lse[ll.at(Q.b, Q.o0, Q.o1, Q.o2, Q.h)] = 0.f;
        return;
    }

    float qv[DPL];
    load_run<T, DPL>(q + lq.at(Q.b, Q.i0, Q.i1, Q.i2, Q.h), d0, p.Dqk, vec, qv);
    float m = -INFINITY, l = 0.f, acc[DPL];
#pragma unroll
    for (int j = 0; j < DPL; ++j) acc[j] = 0.f;

    const auto step = [&](const float (&kv)[DPL], const float (&vv)[DPL]) {
        float s = 0.f;
#pragma unroll
        for (int j = 0; j < DPL; ++j) s = fmaf(qv[j], kv[j], s);
        s = group_sum<LPQ>(s) * p.scale;
        if (s > m) {
            const float c = expf(m - s);
            l *= c;
#pragma unroll
            for (int j = 0; j < DPL; ++j) acc[j] *= c;
            m = s;
        }
        const float e = expf(s - m);
        l += e;
#pragma unroll
        for (int j = 0; j < DPL; ++j) acc[j] = fmaf(e, vv[j], acc[j]);
    };
    if (vec) {
        struct Step {
            Raw<T, DPL> k, v;
        };
        walk_neighbors_pipelined<pipe_depth<T, DPL, 2>()>(
            p, Q.i0, Q.i1, Q.i2, sp, split,
            [&](int j0, int j1, int j2, int) {
                return Step{fetch_run<T, DPL>(k + lk.at(Q.b, j0, j1, j2, hk), d0, p.Dqk),
                            fetch_run<T, DPL>(v + lv.at(Q.b, j0, j1, j2, hk), d0, p.Dv)};
            },
            [&](const Step& st, int, bool ok) {
                if (!ok) return;
                float kv[DPL], vv[DPL];
                unpack_run<T, DPL>(st.k, d0, p.Dqk, kv);
                unpack_run<T, DPL>(st.v, d0, p.Dv, vv);
                step(kv, vv);
            });
    } else {
        for_each_neighbor_split(p, Q.i0, Q.i1, Q.i2, sp, split, [&](int j0, int j1, int j2, int, bool ok) {
            if (!ok) return;
            float kv[DPL], vv[DPL];
            load_run<T, DPL>(k + lk.at(Q.b, j0, j1, j2, hk), d0, p.Dqk, vec, kv);
            load_run<T, DPL>(v + lv.at(Q.b, j0, j1, j2, hk), d0, p.Dv, vec, vv);
            step(kv, vv);
        });
    }

    if (split > 1) {
        // merge the groups' softmax states (a group may have seen no neighbour)
        const float mall = split_max<LPQ>(m, split);
        const float c = m == -INFINITY ? 0.f : expf(m - mall);
        l = split_sum<LPQ>(l * c, split);
#pragma unroll
        for (int j = 0; j < DPL; ++j) acc[j] = split_sum<LPQ>(acc[j] * c, split);
        m = mall;
    }
#pragma unroll
    for (int j = 0; j < DPL; ++j) acc[j] = acc[j] / l;
    if (sp == 0) store_run<T, DPL>(out + lo.at(Q.b, Q.o0, Q.o1, Q.o2, Q.h), d0, p.Dv, vec, acc);
    if (sp == 0 && d0 == 0) lse[ll.at(Q.b, Q.o0, Q.o1, Q.o2, Q.h)] = m + logf(l);
}

// ---------------------------------------------------------------------------
// Split QK: logits per neighbour (unscaled unless has_scale), -inf if invalid.
// ---------------------------------------------------------------------------
template <typename T, int DPL, int LPQ>
__global__ __launch_bounds__(256) void k_qk(Prob p, int vec,
                                            const T* __restrict__ q, Lay lq,
                                            const T* __restrict__ k, Lay lk,
                                            T* __restrict__ attn, Lay la) {
    const long long qi = group_index(LPQ);
    if (qi >= static_cast<long long>(p.B) * p.nout * p.Hq) return;
    const int d0 = (threadIdx.x % LPQ) * DPL;
    const QPos Q = decode_query(p, qi);
    float qv[DPL];
    load_run<T, DPL>(q + lq.at(Q.b, Q.i0, Q.i1, Q.i2, Q.h), d0, p.Dqk, vec, qv);
    T* row = attn + la.at(Q.b, Q.o0, Q.o1, Q.o2, Q.h);
    if (vec) {
        walk_neighbors_pipelined<pipe_depth<T, DPL, 1>()>(
            p, Q.i0, Q.i1, Q.i2, 0, 1,
            [&](int j0, int j1, int j2, int) { return fetch_run<T, DPL>(k + lk.at(Q.b, j0, j1, j2, Q.h), d0, p.Dqk); },
            [&](const Raw<T, DPL>& r, int e, bool ok) {
                float kv[DPL];
                unpack_run<T, DPL>(r, d0, p.Dqk, kv);
                float acc = 0.f;
#pragma unroll
                for (int j = 0; j < DPL; ++j) acc = fmaf(qv[j], kv[j], acc);
                float s = ok ? group_sum<LPQ>(acc) : -INFINITY;
                if (p.has_scale) s *= p.scale;
                if (d0 == 0) row[e] = from_f<T>(s);
            });
        return;
    }
    for_each_neighbor(p, Q.i0, Q.i1, Q.i2, [&](int j0, int j1, int j2, int e, bool ok) {
        float s = -INFINITY;
        if (ok) {
            float kv[DPL];
            load_run<T, DPL>(k + lk.at(Q.b, j0, j1, j2, Q.h), d0, p.Dqk, vec, kv);
            float acc = 0.f;
#pragma unroll
            for (int j = 0; j < DPL; ++j) acc = fmaf(qv[j], kv[j], acc);
            s = group_sum<LPQ>(acc);
        }
        if (p.has_scale) s *= p.scale;
        if (d0 == 0) row[e] = from_f<T>(s);
    });
}

// Accumulator of the split ops' gathers (AV output, dq, dk, dv): a sum over
// a whole window (or over every query attending a key), hundreds of products
// in 3-D.  For fp32 operands it runs in double -- a product of two fp32
// values is exact there, so the result is the correctly rounded sum, and no
// summation-order noise of fp32 (which passes 1e-5 relative at 3-D window
// sizes) reaches the output; 16-bit operands keep fp32 accumulators.
template <typename T>
struct GatherAcc {
    using type = float;
};
template <>
struct GatherAcc<float> {
    using type = double;
};

template <typename A>
__device__ __forceinline__ A gather_fma(float a, float b, A acc) {
    return static_cast<A>(a) * static_cast<A>(b) + acc;
}

// acc (times mul) rounded to float for store_run.
template <typename A, int DPL>
__device__ __forceinline__ void gather_out(const A (&acc)[DPL], float mul, float (&out)[DPL]) {
#pragma unroll
    for (int j = 0; j < DPL; ++j) out[j] = static_cast<float>(acc[j] * static_cast<A>(mul));
}

// ---------------------------------------------------------------------------
// Split AV: out = sum_valid attn * v.
// ---------------------------------------------------------------------------
template <typename T, int DPL, int LPQ>
__global__ __launch_bounds__(256) void k_av(Prob p, int vec,
                                            const T* __restrict__ attn, Lay la,
                                            const T* __restrict__ v, Lay lv,
                                            T* __restrict__ out, Lay lo) {
    const long long qi = group_index(LPQ);
    if (qi >= static_cast<long long>(p.B) * p.nout * p.Hq) return;
    const int d0 = (threadIdx.x % LPQ) * DPL;
    const QPos Q = decode_query(p, qi);
    const T* row = attn + la.at(Q.b, Q.o0, Q.o1, Q.o2, Q.h);
    using A = typename GatherAcc<T>::type;
    A acc[DPL];
#pragma unroll
    for (int j = 0; j < DPL; ++j) acc[j] = 0;
    if (vec) {
        struct Step {
            Raw<T, DPL> v;
            T a;
        };
        walk_neighbors_pipelined<pipe_depth<T, DPL, 1>()>(
            p, Q.i0, Q.i1, Q.i2, 0, 1,
            [&](int j0, int j1, int j2, int e) {
                return Step{fetch_run<T, DPL>(v + lv.at(Q.b, j0, j1, j2, Q.h), d0, p.Dv), row[e]};
            },
            [&](Step& st, int, bool ok) {
                if (!ok) return;
                const float a = to_f(st.a);
                float vv[DPL];
                unpack_run<T, DPL>(st.v, d0, p.Dv, vv);
#pragma unroll
                for (int j = 0; j < DPL; ++j) acc[j] = gather_fma(a, vv[j], acc[j]);
            });
    } else {
        for_each_neighbor(p, Q.i0, Q.i1, Q.i2, [&](int j0, int j1, int j2, int e, bool ok) {
            if (!ok) return;
            const float a = to_f(row[e]);
            float vv[DPL];
            load_run<T, DPL>(v + lv.at(Q.b, j0, j1, j2, Q.h), d0, p.Dv, vec, vv);
#pragma unroll
            for (int j = 0; j < DPL; ++j) acc[j] = gather_fma(a, vv[j], acc[j]);
        });
    }
    float res[DPL];
    gather_out(acc, 1.f, res);
    store_run<T, DPL>(out + lo.at(Q.b, Q.o0, Q.o1, Q.o2, Q.h), d0, p.Dv, vec, res);
}

// ---------------------------------------------------------------------------
// Fused backward, query side: delta = dO.O - dlse, and
// dq = scale * sum_k P (dO.v_k - delta) k_k with P = exp(scale q.k - lse).
// ---------------------------------------------------------------------------
template <typename T, int DPL, int LPQ>
__global__ __launch_bounds__(256) void k_bwd_dq(Prob p, int vec, int split, const int* __restrict__ lens,
                                                const T* __restrict__ q, Lay lq,
                                                const T* __restrict__ k, Lay lk,
                                                const T* __restrict__ v, Lay lv,
                                                const T* __restrict__ o, Lay lo,
                                                const T* __restrict__ dout, Lay ldo,
                                                const float* __restrict__ lse, Lay ll,
                                                const float* __restrict__ dlse, Lay ldl,
                                                T* __restrict__ dq, Lay ldq,
                                                float* __restrict__ delta, Lay lde) {
    const long long qi = group_index(LPQ * split);
    if (qi >= static_cast<long long>(p.B) * p.nout * p.Hq) return;
    const int d0 = (threadIdx.x % LPQ) * DPL;
    const int sp = (threadIdx.x / LPQ) % split;
    const QPos Q = decode_query(p, qi);
    const int hk = Q.h / p.rep;
    if (lens && !sample_extent(p, lens, Q.b, Q.i0, Q.i1, Q.i2)) {
        if (sp == 0) store_zero<T, DPL>(dq + ldq.at(Q.b, Q.i0, Q.i1, Q.i2, Q.h), d0, p.Dqk, vec);
        if (sp == 0 && d0 == 0) delta[lde.at(Q.b, Q.o0, Q.o1, Q.o2, Q.h)] = 0.f;
        return;
    }

    float qv[DPL], dov[DPL];
    load_run<T, DPL>(q + lq.at(Q.b, Q.i0, Q.i1, Q.i2, Q.h), d0, p.Dqk, vec, qv);
    load_run<T, DPL>(dout + ldo.at(Q.b, Q.o0, Q.o1, Q.o2, Q.h), d0, p.Dv, vec, dov);
    const float L = lse[ll.at(Q.b, Q.o0, Q.o1, Q.o2, Q.h)];
    float di = 0.f;
    if constexpr (sizeof(T) == 4) {
        // delta = dO . O: exact enough when O was stored in fp32.
        float ov[DPL];
        load_run<T, DPL>(o + lo.at(Q.b, Q.o0, Q.o1, Q.o2, Q.h), d0, p.Dv, vec, ov);
#pragma unroll
        for (int j = 0; j < DPL; ++j) di = fmaf(dov[j], ov[j], di);
        di = group_sum<LPQ>(di);
    } else {
        // 16-bit O carries ~2^-9 relative rounding; use the equivalent
        // delta = sum_k P_k (dO . v_k) from an extra pass instead.
        for_each_neighbor_split(p, Q.i0, Q.i1, Q.i2, sp, split, [&](int j0, int j1, int j2, int, bool ok) {
            if (!ok) return;
            float kv[DPL], vv[DPL];
            load_run<T, DPL>(k + lk.at(Q.b, j0, j1, j2, hk), d0, p.Dqk, vec, kv);
            load_run<T, DPL>(v + lv.at(Q.b, j0, j1, j2, hk), d0, p.Dv, vec, vv);
            float s = 0.f, dp = 0.f;
#pragma unroll
            for (int j = 0; j < DPL; ++j) { s = fmaf(qv[j], kv[j], s); dp = fmaf(dov[j], vv[j], dp); }
            s = group_sum<LPQ>(s) * p.scale;
            dp = group_sum<LPQ>(dp);
            di = fmaf(expf(s - L), dp, di);
        });
        di = split_sum<LPQ>(di, split);
    }
    if (dlse) di -= dlse[ldl.at(Q.b, Q.o0, Q.o1, Q.o2, Q.h)];
    if (sp == 0 && d0 == 0) delta[lde.at(Q.b, Q.o0, Q.o1, Q.o2, Q.h)] = di;

    float acc[DPL];
#pragma unroll
    for (int j = 0; j < DPL; ++j) acc[j] = 0.f;
    const auto step = [&](const float (&kv)[DPL], const float (&vv)[DPL]) {
        float s = 0.f, dp = 0.f;
#pragma unroll
        for (int j = 0; j < DPL; ++j) { s = fmaf(qv[j], kv[j], s); dp = fmaf(dov[j], vv[j], dp); }
        s = group_sum<LPQ>(s) * p.scale;
        dp = group_sum<LPQ>(dp);
        const float ds = expf(s - L) * (dp - di);
#pragma unroll
        for (int j = 0; j < DPL; ++j) acc[j] = fmaf(ds, kv[j], acc[j]);
    };
    if (vec) {
        struct Step {
            Raw<T, DPL> k, v;
        };
        walk_neighbors_pipelined<pipe_depth<T, DPL, 2>()>(
            p, Q.i0, Q.i1, Q.i2, sp, split,
            [&](int j0, int j1, int j2, int) {
                return Step{fetch_run<T, DPL>(k + lk.at(Q.b, j0, j1, j2, hk), d0, p.Dqk),
                            fetch_run<T, DPL>(v + lv.at(Q.b, j0, j1, j2, hk), d0, p.Dv)};
            },
            [&](const Step& st, int, bool ok) {
                if (!ok) return;
                float kv[DPL], vv[DPL];
                unpack_run<T, DPL>(st.k, d0, p.Dqk, kv);
                unpack_run<T, DPL>(st.v, d0, p.Dv, vv);
                step(kv, vv);
            });
    } else {
        for_each_neighbor_split(p, Q.i0, Q.i1, Q.i2, sp, split, [&](int j0, int j1, int j2, int, bool ok) {
            if (!ok) return;
            float kv[DPL], vv[DPL];
            load_run<T, DPL>(k + lk.at(Q.b, j0, j1, j2, hk), d0, p.Dqk, vec, kv);
            load_run<T, DPL>(v + lv.at(Q.b, j0, j1, j2, hk), d0, p.Dv, vec, vv);
            step(kv, vv);
        });
    }
#pragma unroll
    for (int j = 0; j < DPL; ++j) acc[j] = split_sum<LPQ>(acc[j], split) * p.scale;
    if (sp == 0) store_run<T, DPL>(dq + ldq.at(Q.b, Q.i0, Q.i1, Q.i2, Q.h), d0, p.Dqk, vec, acc);
}

// ---------------------------------------------------------------------------
// Fused backward, key side: for each key/value position and kv head, gather
// over the queries (of every q head in the GQA group) whose windows hold it:
// dv = sum P dO,  dk = scale * sum P (dO.v - delta) q.  Deterministic (no
// atomics); recomputes P from q, k and lse.
// ---------------------------------------------------------------------------
template <typename T, int DPL, int LPQ>
__global__ __launch_bounds__(256) void k_bwd_dkdv(Prob p, int vec, int split, const int* __restrict__ lens,
                                                  const T* __restrict__ q, Lay lq,
                                                  const T* __restrict__ k, Lay lk,
                                                  const T* __restrict__ v, Lay lv,
                                                  const T* __restrict__ dout, Lay ldo,
                                                  const float* __restrict__ lse, Lay ll,
                                                  const float* __restrict__ delta, Lay lde,
                                                  T* __restrict__ dk, Lay ldk,
                                                  T* __restrict__ dv, Lay ldv) {
    const long long ki = group_index(LPQ * split);
    if (ki >= static_cast<long long>(p.B) * p.nkey * p.Hkv) return;
    const int d0 = (threadIdx.x % LPQ) * DPL;
    const int sp = (threadIdx.x / LPQ) % split;
    const KPos K = decode_key(p, ki, p.Hkv);
    if (lens && !sample_extent(p, lens, K.b, K.m0, K.m1, K.m2)) {
        if (sp == 0) store_zero<T, DPL>(dk + ldk.at(K.b, K.m0, K.m1, K.m2, K.h), d0, p.Dqk, vec);
        if (sp == 0) store_zero<T, DPL>(dv + ldv.at(K.b, K.m0, K.m1, K.m2, K.h), d0, p.Dv, vec);
        return;
    }

    float kv[DPL], vv[DPL], gk[DPL], gv[DPL];
    load_run<T, DPL>(k + lk.at(K.b, K.m0, K.m1, K.m2, K.h), d0, p.Dqk, vec, kv);
    load_run<T, DPL>(v + lv.at(K.b, K.m0, K.m1, K.m2, K.h), d0, p.Dv, vec, vv);
#pragma unroll
    for (int j = 0; j < DPL; ++j) { gk[j] = 0.f; gv[j] = 0.f; }

    for_each_query_split(p, K.m0, K.m1, K.m2, sp, split, [&](int o0, int o1, int o2, int i0, int i1, int i2, int) {
        for (int r = 0; r < p.rep; ++r) {
            const int h = K.h * p.rep + r;
            float qv[DPL], dov[DPL];
            load_run<T, DPL>(q + lq.at(K.b, i0, i1, i2, h), d0, p.Dqk, vec, qv);
            load_run<T, DPL>(dout + ldo.at(K.b, o0, o1, o2, h), d0, p.Dv, vec, dov);
            const float L = lse[ll.at(K.b, o0, o1, o2, h)];
            const float di = delta[lde.at(K.b, o0, o1, o2, h)];
            float s = 0.f, dp = 0.f;
#pragma unroll
            for (int j = 0; j < DPL; ++j) { s = fmaf(qv[j], kv[j], s); dp = fmaf(dov[j], vv[j], dp); }
            s = group_sum<LPQ>(s) * p.scale;
            dp = group_sum<LPQ>(dp);
            const float pr = expf(s - L);
            const float ds = pr * (dp - di);
#pragma unroll
            for (int j = 0; j < DPL; ++j) {
                gv[j] = fmaf(pr, dov[j], gv[j]);
                gk[j] = fmaf(ds, qv[j], gk[j]);
            }
        }
    });
#pragma unroll
    for (int j = 0; j < DPL; ++j) {
        gk[j] = split_sum<LPQ>(gk[j], split) * p.scale;
        gv[j] = split_sum<LPQ>(gv[j], split);
    }
    if (sp == 0) store_run<T, DPL>(dk + ldk.at(K.b, K.m0, K.m1, K.m2, K.h), d0, p.Dqk, vec, gk);
    if (sp == 0) store_run<T, DPL>(dv + ldv.at(K.b, K.m0, K.m1, K.m2, K.h), d0, p.Dv, vec, gv);
}

// ---------------------------------------------------------------------------
// Split QK backward.  dq (query side) and dk (key side); grad of an invalid
// entry is zero, and both carry the logit scale when has_scale.
// ---------------------------------------------------------------------------
template <typename T, int DPL, int LPQ>
__global__ __launch_bounds__(256) void k_qk_bwd_q(Prob p, int vec,
                                                  const T* __restrict__ da, Lay lda,
                                                  const T* __restrict__ k, Lay lk,
                                                  T* __restrict__ dq, Lay ldq) {
    const long long qi = group_index(LPQ);
    if (qi >= static_cast<long long>(p.B) * p.nout * p.Hq) return;
    const int d0 = (threadIdx.x % LPQ) * DPL;
    const QPos Q = decode_query(p, qi);
    const T* row = da + lda.at(Q.b, Q.o0, Q.o1, Q.o2, Q.h);
    using A = typename GatherAcc<T>::type;
    A acc[DPL];
#pragma unroll
    for (int j = 0; j < DPL; ++j) acc[j] = 0;
    if (vec) {
        struct Step {
            Raw<T, DPL> k;
            T g;
        };
        walk_neighbors_pipelined<pipe_depth<T, DPL, 1>()>(
            p, Q.i0, Q.i1, Q.i2, 0, 1,
            [&](int j0, int j1, int j2, int e) {
                return Step{fetch_run<T, DPL>(k + lk.at(Q.b, j0, j1, j2, Q.h), d0, p.Dqk), row[e]};
            },
            [&](Step& st, int, bool ok) {
                if (!ok) return;
                const float g = to_f(st.g);
                float kv[DPL];
                unpack_run<T, DPL>(st.k, d0, p.Dqk, kv);
#pragma unroll
                for (int j = 0; j < DPL; ++j) acc[j] = gather_fma(g, kv[j], acc[j]);
            });
    } else {
        for_each_neighbor(p, Q.i0, Q.i1, Q.i2, [&](int j0, int j1, int j2, int e, bool ok) {
            if (!ok) return;
            const float g = to_f(row[e]);
            float kv[DPL];
            load_run<T, DPL>(k + lk.at(Q.b, j0, j1, j2, Q.h), d0, p.Dqk, vec, kv);
#pragma unroll
            for (int j = 0; j < DPL; ++j) acc[j] = gather_fma(g, kv[j], acc[j]);
        });
    }
    float res[DPL];
    gather_out(acc, p.has_scale ? p.scale : 1.f, res);
    store_run<T, DPL>(dq + ldq.at(Q.b, Q.i0, Q.i1, Q.i2, Q.h), d0, p.Dqk, vec, res);
}

template <typename T, int DPL, int LPQ>
__global__ __launch_bounds__(256) void k_qk_bwd_k(Prob p, int vec,
                                                  const T* __restrict__ da, Lay lda,
                                                  const T* __restrict__ q, Lay lq,
                                                  T* __restrict__ dk, Lay ldk) {
    const long long ki = group_index(LPQ);
    if (ki >= static_cast<long long>(p.B) * p.nkey * p.Hkv) return;
    const int d0 = (threadIdx.x % LPQ) * DPL;
    const KPos K = decode_key(p, ki, p.Hkv);
    using A = typename GatherAcc<T>::type;
    A acc[DPL];
#pragma unroll
    for (int j = 0; j < DPL; ++j) acc[j] = 0;
    for_each_query(p, K.m0, K.m1, K.m2, [&](int o0, int o1, int o2, int i0, int i1, int i2, int e) {
        const float g = to_f(da[lda.at(K.b, o0, o1, o2, K.h) + e]);
        float qv[DPL];
        load_run<T, DPL>(q + lq.at(K.b, i0, i1, i2, K.h), d0, p.Dqk, vec, qv);
#pragma unroll
        for (int j = 0; j < DPL; ++j) acc[j] = gather_fma(g, qv[j], acc[j]);
    });
    float res[DPL];
    gather_out(acc, p.has_scale ? p.scale : 1.f, res);
    store_run<T, DPL>(dk + ldk.at(K.b, K.m0, K.m1, K.m2, K.h), d0, p.Dqk, vec, res);
}

// ---------------------------------------------------------------------------
// Split AV backward: dattn (query side) and dv (key side).
// ---------------------------------------------------------------------------
template <typename T, int DPL, int LPQ>
__global__ __launch_bounds__(256) void k_av_bwd_a(Prob p, int vec,
                                                  const T* __restrict__ dout, Lay ldo,
                                                  const T* __restrict__ v, Lay lv,
                                                  T* __restrict__ da, Lay lda) {
    const long long qi = group_index(LPQ);
    if (qi >= static_cast<long long>(p.B) * p.nout * p.Hq) return;
    const int d0 = (threadIdx.x % LPQ) * DPL;
    const QPos Q = decode_query(p, qi);
    float dov[DPL];
    load_run<T, DPL>(dout + ldo.at(Q.b, Q.o0, Q.o1, Q.o2, Q.h), d0, p.Dv, vec, dov);
    T* row = da + lda.at(Q.b, Q.o0, Q.o1, Q.o2, Q.h);
    if (vec) {
        walk_neighbors_pipelined<pipe_depth<T, DPL, 1>()>(
            p, Q.i0, Q.i1, Q.i2, 0, 1,
            [&](int j0, int j1, int j2, int) { return fetch_run<T, DPL>(v + lv.at(Q.b, j0, j1, j2, Q.h), d0, p.Dv); },
            [&](const Raw<T, DPL>& r, int e, bool ok) {
                float vv[DPL];
                unpack_run<T, DPL>(r, d0, p.Dv, vv);
                float acc = 0.f;
#pragma unroll
                for (int j = 0; j < DPL; ++j) acc = fmaf(dov[j], vv[j], acc);
                const float g = ok ? group_sum<LPQ>(acc) : 0.f;
                if (d0 == 0) row[e] = from_f<T>(g);
            });
        return;
    }
    for_each_neighbor(p, Q.i0, Q.i1, Q.i2, [&](int j0, int j1, int j2, int e, bool ok) {
        float g = 0.f;
        if (ok) {
            float vv[DPL];
            load_run<T, DPL>(v + lv.at(Q.b, j0, j1, j2, Q.h), d0, p.Dv, vec, vv);
            float acc = 0.f;
#pragma unroll
            for (int j = 0; j < DPL; ++j) acc = fmaf(dov[j], vv[j], acc);
            g = group_sum<LPQ>(acc);
        }
        if (d0 == 0) row[e] = from_f<T>(g);
    });
}

template <typename T, int DPL, int LPQ>
__global__ __launch_bounds__(256) void k_av_bwd_v(Prob p, int vec,
                                                  const T* __restrict__ dout, Lay ldo,
                                                  const T* __restrict__ attn, Lay la,
                                                  T* __restrict__ dv, Lay ldv) {
    const long long ki = group_index(LPQ);
    if (ki >= static_cast<long long>(p.B) * p.nkey * p.Hkv) return;
    const int d0 = (threadIdx.x % LPQ) * DPL;
    const KPos K = decode_key(p, ki, p.Hkv);
    using A = typename GatherAcc<T>::type;
    A acc[DPL];
#pragma unroll
    for (int j = 0; j < DPL; ++j) acc[j] = 0;
    for_each_query(p, K.m0, K.m1, K.m2, [&](int o0, int o1, int o2, int, int, int, int e) {
        const float a = to_f(attn[la.at(K.b, o0, o1, o2, K.h) + e]);
        float dov[DPL];
        load_run<T, DPL>(dout + ldo.at(K.b, o0, o1, o2, K.h), d0, p.Dv, vec, dov);
#pragma unroll
        for (int j = 0; j < DPL; ++j) acc[j] = gather_fma(a, dov[j], acc[j]);
    });
    float res[DPL];
    gather_out(acc, 1.f, res);
    store_run<T, DPL>(dv + ldv.at(K.b, K.m0, K.m1, K.m2, K.h), d0, p.Dv, vec, res);
}

// ---------------------------------------------------------------------------
// Neighbourhood map export (one thread per (query position, neighbour)).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_map(Prob p, int64_t* __restrict__ flat, uint8_t* __restrict__ valid) {
    const long long t = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= static_cast<long long>(p.nout) * p.kv) return;
    const int e = static_cast<int>(t % p.kv);
    long long oq = t / p.kv;
    const int o2 = static_cast<int>(oq % p.ax[2].out); oq /= p.ax[2].out;
    const int o1 = static_cast<int>(oq % p.ax[1].out); oq /= p.ax[1].out;
    const int o0 = static_cast<int>(oq);
    const int z = e % p.ax[2].k, y = (e / p.ax[2].k) % p.ax[1].k, x = e / (p.ax[2].k * p.ax[1].k);
    const int os[3] = {o0, o1, o2}, ks[3] = {x, y, z};
    long long f = 0;
    bool ok = true;
    for (int a = 0; a < 3; ++a) {
        const Axis& A = p.ax[a];
        const int i = os[a] * A.st;
        int j = axis_first(A, i) + ks[a] * A.dil;
        if (A.causal) {
            ok = ok && (j >= 0) && (j <= i);
            j = j < 0 ? 0 : (j > A.len - 1 ? A.len - 1 : j);
        }
        f = f * A.len + j;
    }
    flat[t] = f;
    valid[t] = ok ? 1 : 0;
}

}  // namespace

// ---------------------------------------------------------------------------
// Launchers.
// ---------------------------------------------------------------------------

namespace {

// Lanes-per-query / dims-per-lane configurations, chosen from the head dim.
template <template <typename, int, int> class Launch, typename T, typename... Args>
hipError_t by_dim(int D, Args&&... args) {
    if (D <= 8) return Launch<T, 8, 1>::run(args...);
    if (D <= 16) return Launch<T, 8, 2>::run(args...);
    if (D <= 32) return Launch<T, 8, 4>::run(args...);
    if (D <= 64) return Launch<T, 8, 8>::run(args...);
    if (D <= 128) return Launch<T, 8, 16>::run(args...);
    return Launch<T, 16, 16>::run(args...);
}

template <template <typename, int, int> class Launch, typename... Args>
hipError_t by_type(int dtype, int D, Args&&... args) {
    switch (dtype) {
        case NATTEN_F32: return by_dim<Launch, float>(D, args...);
        case NATTEN_F16: return by_dim<Launch, f16>(D, args...);
        default: return by_dim<Launch, bf16>(D, args...);
    }
}

inline unsigned grid_for(long long groups, int lpq) {
    const long long threads = groups * lpq;
    return static_cast<unsigned>((threads + 255) / 256);
}

// Lane groups per query (key) for the fused vector kernels.  Each group walks
// its neighbours (attending queries) one after another, every step waiting
// on its loads, so a small problem (few groups) is bound by that chain.
// Splitting the walk over up to 8 groups, until the launch holds about 8
// waves per SIMD of a 256-CU device, shortens the chain; groups stay within
// one wave (lpq * split <= 64) and never outnumber the split axis's kernel
// positions.  NATTEN_HIP_SPLIT=n fixes it (tuning).
inline int choose_split(const Prob& p, long long groups, int lpq) {
    static const int forced = [] {
        const char* e = std::getenv("NATTEN_HIP_SPLIT");
        return e ? std::atoi(e) : 0;
    }();
    const int kmax = p.ax[split_axis(p)].k;
    constexpr long long kTargetWaves = 256LL * 4 * 8;
    int split = 1;
    if (forced > 0) {
        while (split * 2 <= forced && split * 2 * lpq <= 64) split *= 2;
        return split;
    }
    const long long waves = (groups * lpq + 63) / 64;
    while (split < 8 && split * 2 * lpq <= 64 && split * 2 <= kmax && waves * split < kTargetWaves) split *= 2;
    return split;
}

template <typename T, int DPL, int LPQ>
struct LForward {
    static hipError_t run(const Prob& p, int vec, const int* lens, const void* q, Lay lq, const void* k, Lay lk,
                          const void* v, Lay lv, void* o, Lay lo, float* lse, Lay ll, hipStream_t s) {
        const long long n = static_cast<long long>(p.B) * p.nout * p.Hq;
        const int split = choose_split(p, n, LPQ);
        NA_LAUNCH(lens ? "na_varlen_forward" : "na_forward", (k_forward<T, DPL, LPQ>),
                  dim3(grid_for(n, LPQ * split)), dim3(256), 0, s, p, vec, split, lens, (const T*)q, lq, (const T*)k, lk, (const T*)v, lv, (T*)o, lo, lse,
                  ll);
        return hipGetLastError();
    }
};

template <typename T, int DPL, int LPQ>
struct LQK {
    static hipError_t run(const Prob& p, int vec, const void* q, Lay lq, const void* k, Lay lk, void* a, Lay la,
                          hipStream_t s) {
        const long long n = static_cast<long long>(p.B) * p.nout * p.Hq;
        NA_LAUNCH("na_qk", (k_qk<T, DPL, LPQ>), dim3(grid_for(n, LPQ)), dim3(256), 0, s, p, vec, (const T*)q, lq,
                           (const T*)k, lk, (T*)a, la);
        return hipGetLastError();
    }
};

template <typename T, int DPL, int LPQ>
struct LAV {
    static hipError_t run(const Prob& p, int vec, const void* a, Lay la, const void* v, Lay lv, void* o, Lay lo,
                          hipStream_t s) {
        const long long n = static_cast<long long>(p.B) * p.nout * p.Hq;
        NA_LAUNCH("na_av", (k_av<T, DPL, LPQ>), dim3(grid_for(n, LPQ)), dim3(256), 0, s, p, vec, (const T*)a, la,
                           (const T*)v, lv, (T*)o, lo);
        return hipGetLastError();
    }
};

template <typename T, int DPL, int LPQ>
struct LBackward {
    static hipError_t run(const Prob& p, int vec, const int* lens, const void* q, Lay lq, const void* k, Lay lk,
                          const void* v, Lay lv, const void* o, Lay lo, const void* dout, Lay ldo, const float* lse,
                          Lay ll, const float* dlse, Lay ldl, void* dq, Lay ldq, void* dk, Lay ldk, void* dv,
                          Lay ldv, float* delta, Lay lde, hipStream_t s) {
        const long long nq = static_cast<long long>(p.B) * p.nout * p.Hq;
        const int sq = choose_split(p, nq, LPQ);
        NA_LAUNCH(lens ? "na_varlen_bwd_dq" : "na_bwd_dq", (k_bwd_dq<T, DPL, LPQ>), dim3(grid_for(nq, LPQ * sq)),
                  dim3(256), 0, s, p, vec, sq, lens, (const T*)q, lq, (const T*)k, lk, (const T*)v, lv, (const T*)o, lo,
                  (const T*)dout, ldo, lse, ll, dlse, ldl, (T*)dq, ldq, delta, lde);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        const long long nk = static_cast<long long>(p.B) * p.nkey * p.Hkv;
        const int sk = choose_split(p, nk, LPQ);
        NA_LAUNCH(lens ? "na_varlen_bwd_dkdv" : "na_bwd_dkdv", (k_bwd_dkdv<T, DPL, LPQ>),
                  dim3(grid_for(nk, LPQ * sk)), dim3(256), 0, s, p, vec, sk, lens, (const T*)q, lq, (const T*)k, lk,
                  (const T*)v, lv, (const T*)dout, ldo, lse, ll, (const float*)delta, lde, (T*)dk, ldk, (T*)dv,
                  ldv);
        return hipGetLastError();
    }
};

template <typename T, int DPL, int LPQ>
struct LQKBwd {
    static hipError_t run(const Prob& p, int vec, const void* da, Lay lda, const void* q, Lay lq, const void* k,
                          Lay lk, void* dq, Lay ldq, void* dk, Lay ldk, int sides, hipStream_t s) {
        if (sides & kQuerySide) {
            const long long nq = static_cast<long long>(p.B) * p.nout * p.Hq;
            NA_LAUNCH("na_qk_bwd_q", (k_qk_bwd_q<T, DPL, LPQ>), dim3(grid_for(nq, LPQ)), dim3(256), 0, s, p, vec,
                      (const T*)da, lda, (const T*)k, lk, (T*)dq, ldq);
            const hipError_t e = hipGetLastError();
            if (e != hipSuccess) return e;
        }
        if (!(sides & kKeySide)) return hipSuccess;
        const long long nk = static_cast<long long>(p.B) * p.nkey * p.Hkv;
        NA_LAUNCH("na_qk_bwd_k", (k_qk_bwd_k<T, DPL, LPQ>), dim3(grid_for(nk, LPQ)), dim3(256), 0, s, p, vec,
                           (const T*)da, lda, (const T*)q, lq, (T*)dk, ldk);
        return hipGetLastError();
    }
};

template <typename T, int DPL, int LPQ>
struct LAVBwd {
    static hipError_t run(const Prob& p, int vec, const void* dout, Lay ldo, const void* a, Lay la, const void* v,
                          Lay lv, void* da, Lay lda, void* dv, Lay ldv, int sides, hipStream_t s) {
        if (sides & kQuerySide) {
            const long long nq = static_cast<long long>(p.B) * p.nout * p.Hq;
            NA_LAUNCH("na_av_bwd_a", (k_av_bwd_a<T, DPL, LPQ>), dim3(grid_for(nq, LPQ)), dim3(256), 0, s, p, vec,
                      (const T*)dout, ldo, (const T*)v, lv, (T*)da, lda);
            const hipError_t e = hipGetLastError();
            if (e != hipSuccess) return e;
        }
        if (!(sides & kKeySide)) return hipSuccess;
        const long long nk = static_cast<long long>(p.B) * p.nkey * p.Hkv;
        NA_LAUNCH("na_av_bwd_v", (k_av_bwd_v<T, DPL, LPQ>), dim3(grid_for(nk, LPQ)), dim3(256), 0, s, p, vec,
                           (const T*)dout, ldo, (const T*)a, la, (T*)dv, ldv);
        return hipGetLastError();
    }
};

}  // namespace

hipError_t generic_forward(const Prob& p, int vec, const void* q, Lay lq, const void* k, Lay lk, const void* v,
                           Lay lv, void* o, Lay lo, float* lse, Lay ll, int dtype, hipStream_t s, const int* lens) {
    return by_type<LForward>(dtype, p.Dqk > p.Dv ? p.Dqk : p.Dv, p, vec, lens, q, lq, k, lk, v, lv, o, lo, lse, ll,
                             s);
}

hipError_t generic_qk(const Prob& p, int vec, const void* q, Lay lq, const void* k, Lay lk, void* a, Lay la,
                      int dtype, hipStream_t s) {
    return by_type<LQK>(dtype, p.Dqk, p, vec, q, lq, k, lk, a, la, s);
}

hipError_t generic_av(const Prob& p, int vec, const void* a, Lay la, const void* v, Lay lv, void* o, Lay lo,
                      int dtype, hipStream_t s) {
    return by_type<LAV>(dtype, p.Dv, p, vec, a, la, v, lv, o, lo, s);
}

hipError_t generic_backward(const Prob& p, int vec, const void* q, Lay lq, const void* k, Lay lk, const void* v,
                            Lay lv, const void* o, Lay lo, const void* dout, Lay ldo, const float* lse, Lay ll,
                            const float* dlse, Lay ldl, void* dq, Lay ldq, void* dk, Lay ldk, void* dv, Lay ldv,
                            float* delta, Lay lde, int dtype, hipStream_t s, const int* lens) {
    return by_type<LBackward>(dtype, p.Dqk > p.Dv ? p.Dqk : p.Dv, p, vec, lens, q, lq, k, lk, v, lv, o, lo, dout,
                              ldo, lse, ll, dlse, ldl, dq, ldq, dk, ldk, dv, ldv, delta, lde, s);
}

hipError_t generic_qk_backward(const Prob& p, int vec, const void* da, Lay lda, const void* q, Lay lq,
                               const void* k, Lay lk, void* dq, Lay ldq, void* dk, Lay ldk, int dtype,
                               hipStream_t s, int sides) {
    return by_type<LQKBwd>(dtype, p.Dqk, p, vec, da, lda, q, lq, k, lk, dq, ldq, dk, ldk, sides, s);
}

hipError_t generic_av_backward(const Prob& p, int vec, const void* dout, Lay ldo, const void* a, Lay la,
                               const void* v, Lay lv, void* da, Lay lda, void* dv, Lay ldv, int dtype,
                               hipStream_t s, int sides) {
    return by_type<LAVBwd>(dtype, p.Dv, p, vec, dout, ldo, a, la, v, lv, da, lda, dv, ldv, sides, s);
}

hipError_t neighborhood_map(const Prob& p, int64_t* flat, uint8_t* valid, hipStream_t s) {
    const long long n = static_cast<long long>(p.nout) * p.kv;
    if (n == 0) return hipSuccess;
    NA_LAUNCH("na_map", k_map, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s, p, flat, valid);
    return hipGetLastError();
}

}  // namespace na

// DiNAT-style split ops with relative position bias (the reference's
// extras/allin1: extras/allin1/functional.py:47-570, reference_impl.py:9-41).
//
//   logits[b, p, h, e] = q[b, p, h] . k[b, pos(p, e), h] + rpb[h, bias(p, e)]
//                        (-inf where the neighbour is invalid)
//   out[b, p, h]       = sum over valid e of attn[b, p, h, e] v[b, pos(p, e), h]
//
// for 1-D and 2-D (square kernel, one dilation), with NATTEN 0.17's shifted
// windows: a phase-aligned start per axis (the query's residue class mod the
// dilation), window end min(len, start + K * dil), and the bias start of
// get_pb_start; a neighbour is valid when 0 <= pos < end, and its bias index
// is clamped to [0, 2K-2].  Those rules differ from the main operators' for
// an even kernel with dilation (starts can be negative there), so these ops
// carry their own.
//
// Axes are padded to two: a 1-D problem is (1, L) with kernel (1, K), and its
// bias has extent (1, 2K-1).  Vector-ALU kernels, fp32 accumulation, one
// thread per output element; dk, dv and the bias gradient are deterministic
// gathers (no atomics).
//
// For odd kernels the shifted window is the main operators' window (start,
// end and neighbour order), so the C entry points send the products of
// these ops to the split tile kernels where those apply (k_dot_mfma adds the
// bias as it stores the logits), and this file reduces the bias gradient
// (rpb_qk_backward).  An
// odd kernel's bias start lies in [0, K-1], so the bias index of neighbour e
// is start + e without clamping and each (query, bias index) pair has at
// most one neighbour: the two-pass reduction below gathers per bias index
// over LDS chunks of queries instead of scanning the tensor once per index.
#include "na_launch.h"

namespace na {

namespace {

struct RAxis {
    int len, K, nh, dil;
};

// extras/allin1/reference_impl.py:9-22
__device__ __forceinline__ int rpb_start(int i, const RAxis& a) {
    const int d = a.dil, di = i % d, ip = i / d;
    int lp = (a.len + d - 1) / d;
    const int npad = lp * d - a.len;
    lp -= (di >= d - npad) ? 1 : 0;
    const int s = max(ip - a.nh, 0) + ((ip + a.nh >= lp) ? (lp - ip - a.nh - 1) : 0);
    return s * d + di;
}

// reference_impl.py:25-27 (half-open end)
__device__ __forceinline__ int rpb_end(int start, const RAxis& a) { return min(a.len, start + a.K * a.dil); }

// reference_impl.py:30-41 (pb_start, na_common.h)
__device__ __forceinline__ int rpb_bias_start(int i, const RAxis& a) { return pb_start(i, a.len, a.K, a.dil); }

struct RProb {
    int B, H, Dqk, Dv;
    RAxis ax[2];
    int kv;     // K0 * K1
    int rs[2];  // bias extent per axis, 2K-1
};

__device__ __forceinline__ int clampi(int x, int lo, int hi) { return x < lo ? lo : (x > hi ? hi : x); }

// Neighbour e of query (p0, p1): key position per axis, validity, bias index.
struct RNb {
    int k0, k1, bias;
    bool ok;
};

__device__ __forceinline__ RNb rpb_neighbor(const RProb& p, int p0, int p1, int e) {
    const int e0 = e / p.ax[1].K, e1 = e - e0 * p.ax[1].K;
    const int s0 = rpb_start(p0, p.ax[0]), s1 = rpb_start(p1, p.ax[1]);
    RNb n;
    n.k0 = s0 + e0 * p.ax[0].dil;
    n.k1 = s1 + e1 * p.ax[1].dil;
    n.ok = n.k0 >= 0 && n.k0 < rpb_end(s0, p.ax[0]) && n.k1 >= 0 && n.k1 < rpb_end(s1, p.ax[1]);
    const int b0 = clampi(rpb_bias_start(p0, p.ax[0]) + e0, 0, p.rs[0] - 1);
    const int b1 = clampi(rpb_bias_start(p1, p.ax[1]) + e1, 0, p.rs[1] - 1);
    n.bias = b0 * p.rs[1] + b1;
    return n;
}

__device__ __forceinline__ long long at2(const Lay& l, int b, int i0, int i1, int h) {
    return b * l.b + i0 * l.s1 + i1 * l.s2 + h * l.h;
}

// (b, p0, p1, h, x) with x fastest, from a flat thread index over extent n_x.
struct RIdx {
    int b, p0, p1, h, x;
};

__device__ __forceinline__ bool rpb_index(const RProb& p, int nx, RIdx& r) {
    long long t = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    const long long total = static_cast<long long>(p.B) * p.ax[0].len * p.ax[1].len * p.H * nx;
    if (t >= total) return false;
    r.x = static_cast<int>(t % nx);
    t /= nx;
    r.h = static_cast<int>(t % p.H);
    t /= p.H;
    r.p1 = static_cast<int>(t % p.ax[1].len);
    t /= p.ax[1].len;
    r.p0 = static_cast<int>(t % p.ax[0].len);
    r.b = static_cast<int>(t / p.ax[0].len);
    return true;
}

template <typename T>
__global__ __launch_bounds__(256) void k_rpb_qk(RProb p, const T* __restrict__ q, Lay lq, const T* __restrict__ k,
                                                Lay lk, const T* __restrict__ rpb, T* __restrict__ attn, Lay la) {
    RIdx r;
    if (!rpb_index(p, p.kv, r)) return;
    const RNb n = rpb_neighbor(p, r.p0, r.p1, r.x);
    float s = -INFINITY;
    if (n.ok) {
        const T* qp = q + at2(lq, r.b, r.p0, r.p1, r.h);
        const T* kp = k + at2(lk, r.b, n.k0, n.k1, r.h);
        float acc = 0.f;
        for (int d = 0; d < p.Dqk; ++d) acc = fmaf(to_f(qp[d]), to_f(kp[d]), acc);
        if (rpb) acc += to_f(rpb[r.h * p.rs[0] * p.rs[1] + n.bias]);
        s = acc;
    }
    attn[at2(la, r.b, r.p0, r.p1, r.h) + r.x] = from_f<T>(s);
}

template <typename T>
__global__ __launch_bounds__(256) void k_rpb_av(RProb p, const T* __restrict__ attn, Lay la, const T* __restrict__ v,
                                                Lay lv, T* __restrict__ out, Lay lo) {
    RIdx r;
    if (!rpb_index(p, p.Dv, r)) return;
    const T* ap = attn + at2(la, r.b, r.p0, r.p1, r.h);
    float acc = 0.f;
    for (int e = 0; e < p.kv; ++e) {
        const RNb n = rpb_neighbor(p, r.p0, r.p1, e);
        if (n.ok) acc = fmaf(to_f(ap[e]), to_f(v[at2(lv, r.b, n.k0, n.k1, r.h) + r.x]), acc);
    }
    out[at2(lo, r.b, r.p0, r.p1, r.h) + r.x] = from_f<T>(acc);
}

// dq[d] = sum over valid e of dattn[e] k(e)[d]  (invalid neighbours read the
// zero padding in the reference, so they add nothing)
template <typename T>
__global__ __launch_bounds__(256) void k_rpb_dq(RProb p, const T* __restrict__ da, Lay lda, const T* __restrict__ k,
                                                Lay lk, T* __restrict__ dq, Lay ldq) {
    RIdx r;
    if (!rpb_index(p, p.Dqk, r)) return;
    const T* ap = da + at2(lda, r.b, r.p0, r.p1, r.h);
    float acc = 0.f;
    for (int e = 0; e < p.kv; ++e) {
        const RNb n = rpb_neighbor(p, r.p0, r.p1, e);
        if (n.ok) acc = fmaf(to_f(ap[e]), to_f(k[at2(lk, r.b, n.k0, n.k1, r.h) + r.x]), acc);
    }
    dq[at2(ldq, r.b, r.p0, r.p1, r.h) + r.x] = from_f<T>(acc);
}

// dattn[e] = valid ? dout . v(e) : 0
template <typename T>
__global__ __launch_bounds__(256) void k_rpb_dattn(RProb p, const T* __restrict__ dout, Lay ldo,
                                                   const T* __restrict__ v, Lay lv, T* __restrict__ da, Lay lda) {
    RIdx r;
    if (!rpb_index(p, p.kv, r)) return;
    const RNb n = rpb_neighbor(p, r.p0, r.p1, r.x);
    float acc = 0.f;
    if (n.ok) {
        const T* gp = dout + at2(ldo, r.b, r.p0, r.p1, r.h);
        const T* vp = v + at2(lv, r.b, n.k0, n.k1, r.h);
        for (int d = 0; d < p.Dv; ++d) acc = fmaf(to_f(gp[d]), to_f(vp[d]), acc);
    }
    da[at2(lda, r.b, r.p0, r.p1, r.h) + r.x] = from_f<T>(acc);
}

// Key side: out[m][d] = sum over the (query, neighbour) pairs whose valid
// neighbour is key m of w(query, e) * x(query)[d].  A query attends keys of
// its own residue class at most K class steps away (K, not K-1: the shifted
// start of an even kernel with dilation can sit one step further), so the
// candidates per axis are the 2K+1 class members around m.
template <typename T>
__global__ __launch_bounds__(256) void k_rpb_keyside(RProb p, const T* __restrict__ w, Lay lw,
                                                     const T* __restrict__ x, Lay lx, int D, T* __restrict__ out,
                                                     Lay lout) {
    RIdx r;
    if (!rpb_index(p, D, r)) return;
    const int m0 = r.p0, m1 = r.p1;
    const RAxis &A0 = p.ax[0], &A1 = p.ax[1];
    float acc = 0.f;
    for (int t0 = -A0.K; t0 <= A0.K; ++t0) {
        const int i0 = m0 + t0 * A0.dil;
        if (i0 < 0 || i0 >= A0.len) continue;
        const int s0 = rpb_start(i0, A0);
        const int u0 = m0 - s0;
        if (u0 < 0 || u0 % A0.dil || u0 / A0.dil >= A0.K || m0 >= rpb_end(s0, A0)) continue;
        const int e0 = u0 / A0.dil;
        for (int t1 = -A1.K; t1 <= A1.K; ++t1) {
            const int i1 = m1 + t1 * A1.dil;
            if (i1 < 0 || i1 >= A1.len) continue;
            const int s1 = rpb_start(i1, A1);
            const int u1 = m1 - s1;
            if (u1 < 0 || u1 % A1.dil || u1 / A1.dil >= A1.K || m1 >= rpb_end(s1, A1)) continue;
            const int e = e0 * A1.K + u1 / A1.dil;
            acc = fmaf(to_f(w[at2(lw, r.b, i0, i1, r.h) + e]), to_f(x[at2(lx, r.b, i0, i1, r.h) + r.x]), acc);
        }
    }
    out[at2(lout, r.b, m0, m1, r.h) + r.x] = from_f<T>(acc);
}

// Bias gradient: one workgroup per (head, bias index), summing dattn over
// every (batch, query, neighbour) whose clamped bias index is it -- valid or
// not, as the bias enters every logit.
template <typename T>
__global__ __launch_bounds__(256) void k_rpb_dbias(RProb p, const T* __restrict__ da, Lay lda, T* __restrict__ drpb) {
    __shared__ float part[256];
    const int nb = p.rs[0] * p.rs[1];
    const int h = blockIdx.x / nb, rb = blockIdx.x % nb;
    const int r0 = rb / p.rs[1], r1 = rb % p.rs[1];
    const long long npos = static_cast<long long>(p.B) * p.ax[0].len * p.ax[1].len;
    float acc = 0.f;
    for (long long t = threadIdx.x; t < npos; t += blockDim.x) {
        const int i1 = static_cast<int>(t % p.ax[1].len);
        long long u = t / p.ax[1].len;
        const int i0 = static_cast<int>(u % p.ax[0].len);
        const int b = static_cast<int>(u / p.ax[0].len);
        const int pb0 = rpb_bias_start(i0, p.ax[0]), pb1 = rpb_bias_start(i1, p.ax[1]);
        const T* ap = da + at2(lda, b, i0, i1, h);
        for (int e0 = 0; e0 < p.ax[0].K; ++e0) {
            if (clampi(pb0 + e0, 0, p.rs[0] - 1) != r0) continue;
            for (int e1 = 0; e1 < p.ax[1].K; ++e1)
                if (clampi(pb1 + e1, 0, p.rs[1] - 1) == r1) acc += to_f(ap[e0 * p.ax[1].K + e1]);
        }
    }
    part[threadIdx.x] = acc;
    lds_publish_barrier();
    for (int s = blockDim.x / 2; s > 0; s >>= 1) {
        if (threadIdx.x < s) part[threadIdx.x] += part[threadIdx.x + s];
        lds_publish_barrier();
    }
    if (threadIdx.x == 0) drpb[h * nb + rb] = from_f<T>(part[0]);
}

// Bias gradient, odd kernels, pass 1: workgroup (h, g) takes kDbChunk
// consecutive queries (flattened (batch, p0, p1) order) of head h, with one
// thread per neighbour e (kv <= 256, ceil(kv / 64) waves).  Queries with the
// same bias starts (pb0, pb1) -- every interior query, and runs along the
// borders -- send entry e to the same bias index (pb0 + e0, pb1 + e1), so a
// thread keeps a running sum over such a run and adds it to its wave's LDS
// table when the starts change: within a run the wave's entries hit
// distinct indices, and a wave's LDS operations keep their order, so no
// barrier is needed until the wave tables are summed (in wave order) into
// part[(h * nb + index) * G + g].  Every sum has a fixed order.
constexpr int kDbChunk = 64;
constexpr int kDbLoads = 16;  // queries whose loads are issued together

template <typename T>
__global__ __launch_bounds__(256) void k_rpb_dbias_part(RProb p, const T* __restrict__ da, Lay lda,
                                                        float* __restrict__ part, int G, int npos) {
    extern __shared__ float dbs[];
    const int nb = p.rs[0] * p.rs[1], K1 = p.ax[1].K, nw = blockDim.x >> 6;
    long long* rowoff = reinterpret_cast<long long*>(dbs);           // kDbChunk
    int* st = reinterpret_cast<int*>(rowoff + kDbChunk);              // 2 * kDbChunk
    float* bins = reinterpret_cast<float*>(st + 2 * kDbChunk);        // nw * nb
    const int h = blockIdx.x / G, g = blockIdx.x - (blockIdx.x / G) * G;
    const int t0 = g * kDbChunk, n = min(npos - t0, kDbChunk);
    if (threadIdx.x < kDbChunk) {
        // the chunk's queries, decoded once: row offset and bias starts
        const int t = t0 + threadIdx.x;
        if (threadIdx.x < n) {
            const int i1 = t % p.ax[1].len, u = t / p.ax[1].len;
            const int i0 = u % p.ax[0].len;
            rowoff[threadIdx.x] = at2(lda, u / p.ax[0].len, i0, i1, h);
            st[2 * threadIdx.x] = rpb_bias_start(i0, p.ax[0]);
            st[2 * threadIdx.x + 1] = rpb_bias_start(i1, p.ax[1]);
        }
    }
    for (int i = threadIdx.x; i < nw * nb; i += blockDim.x) bins[i] = 0.f;
    lds_publish_barrier();
    const int e = threadIdx.x;
    const bool mine = e < p.kv;
    const int e0 = e / K1, e1 = e - (e / K1) * K1;
    float* wbins = bins + (threadIdx.x >> 6) * nb;
    float acc = 0.f;
    int c0 = -1, c1 = -1;  // the current run's bias starts (none yet)
    const int ec = mine ? e : 0;  // loads at a valid address; unused past kv
    for (int jb = 0; jb < n; jb += kDbLoads) {
        // unconditional loads (queries past the chunk re-read its last row) so
        // that all of them are in flight before the first is used
        T xr[kDbLoads];
#pragma unroll
        for (int i = 0; i < kDbLoads; ++i) xr[i] = da[rowoff[min(jb + i, n - 1)] + ec];
        float x[kDbLoads];
#pragma unroll
        for (int i = 0; i < kDbLoads; ++i) x[i] = to_f(xr[i]);
#pragma unroll
        for (int i = 0; i < kDbLoads; ++i) {
            if (jb + i >= n) break;
            const int s0 = st[2 * (jb + i)], s1 = st[2 * (jb + i) + 1];
            if (s0 != c0 || s1 != c1) {  // s0, s1 are the same in every lane
                // a lane's flush may update an entry that another lane of
                // this wave flushed earlier: order the wave's LDS accesses
                // explicitly instead of relying on the compiler keeping them
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                if (c0 >= 0 && mine) wbins[(c0 + e0) * p.rs[1] + c1 + e1] += acc;
                c0 = s0;
                c1 = s1;
                acc = 0.f;
            }
            acc += x[i];
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (c0 >= 0 && mine) wbins[(c0 + e0) * p.rs[1] + c1 + e1] += acc;
    lds_publish_barrier();
    for (int i = threadIdx.x; i < nb; i += blockDim.x) {
        float sum = 0.f;
        for (int w = 0; w < nw; ++w) sum += bins[w * nb + i];
        part[(static_cast<long long>(h) * nb + i) * G + g] = sum;
    }
}

// Pass 2: one wave per (h, index): lane l sums the partials g = l, l + 64,
// ... in order (consecutive in memory across the lanes), then a fixed
// butterfly over the lanes.
template <typename T>
__global__ __launch_bounds__(256) void k_rpb_dbias_sum(RProb p, const float* __restrict__ part, int G,
                                                       T* __restrict__ drpb) {
    const int nb = p.rs[0] * p.rs[1];
    const int t = static_cast<int>(blockIdx.x * 4 + (threadIdx.x >> 6)), lane = threadIdx.x & 63;
    if (t >= p.H * nb) return;
    const float* row = part + static_cast<long long>(t) * G;
    float s = 0.f;
    for (int g = lane; g < G; g += 64) s += row[g];
    for (int m = 32; m >= 1; m >>= 1) s += __shfl_xor(s, m);
    if (lane == 0) drpb[t] = from_f<T>(s);
}

long long rpb_rows(const RProb& p) { return static_cast<long long>(p.B) * p.ax[0].len * p.ax[1].len * p.H; }

// The two-pass bias gradient applies to odd kernels of at most 256
// neighbours (one thread each).
bool dbias_two_pass(const RProb& p) {
    return (p.ax[0].K % 2) == 1 && (p.ax[1].K % 2) == 1 && p.kv <= 256 && rpb_rows(p) < (1LL << 31);
}

// Workgroups per head of pass 1: one per chunk of kDbChunk queries.
int dbias_groups(const RProb& p) {
    const long long npos = static_cast<long long>(p.B) * p.ax[0].len * p.ax[1].len;
    return static_cast<int>((npos + kDbChunk - 1) / kDbChunk);
}

unsigned rgrid(const RProb& p, int nx) {
    const long long n = static_cast<long long>(p.B) * p.ax[0].len * p.ax[1].len * p.H * nx;
    return static_cast<unsigned>((n + 255) / 256);
}

template <typename T>
hipError_t rpb_qk_t(const RProb& p, const void* q, Lay lq, const void* k, Lay lk, const void* rpb, void* attn, Lay la,
                    hipStream_t s) {
    NA_LAUNCH("na_rpb_qk", k_rpb_qk<T>, dim3(rgrid(p, p.kv)), dim3(256), 0, s, p, (const T*)q, lq, (const T*)k, lk,
              (const T*)rpb, (T*)attn, la);
    return hipGetLastError();
}

template <typename T>
hipError_t rpb_av_t(const RProb& p, const void* attn, Lay la, const void* v, Lay lv, void* out, Lay lo,
                    hipStream_t s) {
    NA_LAUNCH("na_rpb_av", k_rpb_av<T>, dim3(rgrid(p, p.Dv)), dim3(256), 0, s, p, (const T*)attn, la, (const T*)v, lv,
              (T*)out, lo);
    return hipGetLastError();
}

// Floats of the two-pass bias gradient's partial sums (0: the one-pass
// kernel serves the problem).
size_t dbias_work_floats(const RProb& p) {
    if (!dbias_two_pass(p)) return 0;
    return static_cast<size_t>(p.H) * dbias_groups(p) * p.rs[0] * p.rs[1];
}

// The bias gradient: two passes through the caller's workspace when it holds
// dbias_work_floats floats, else the one-pass kernel (no workspace).
template <typename T>
hipError_t rpb_dbias_t(const RProb& p, const void* da, Lay lda, void* drpb, float* work, size_t work_floats,
                       hipStream_t s) {
    const int nb = p.rs[0] * p.rs[1];
    const size_t need = dbias_work_floats(p);
    if (need > 0 && work && work_floats >= need) {
        const int G = dbias_groups(p);
        const int nw = (p.kv + 63) / 64;  // one thread per neighbour
        const size_t shm =
            kDbChunk * (sizeof(long long) + 2 * sizeof(int)) + static_cast<size_t>(nw) * nb * sizeof(float);
        const int npos = static_cast<int>(rpb_rows(p) / p.H);
        NA_LAUNCH("na_rpb_dbias_part", k_rpb_dbias_part<T>, dim3(static_cast<unsigned>(p.H * G)), dim3(64 * nw), shm,
                  s, p, (const T*)da, lda, work, G, npos);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        NA_LAUNCH("na_rpb_dbias_sum", k_rpb_dbias_sum<T>, dim3(static_cast<unsigned>((p.H * nb + 3) / 4)), dim3(256),
                  0, s, p, (const float*)work, G, (T*)drpb);
        return hipGetLastError();
    }
    NA_LAUNCH("na_rpb_dbias", k_rpb_dbias<T>, dim3(static_cast<unsigned>(p.H * nb)), dim3(256), 0, s, p,
              (const T*)da, lda, (T*)drpb);
    return hipGetLastError();
}

template <typename T>
hipError_t rpb_qk_bwd_t(const RProb& p, const void* da, Lay lda, const void* q, Lay lq, const void* k, Lay lk,
                        void* dq, Lay ldq, void* dk, Lay ldk, void* drpb, float* work, size_t work_floats,
                        hipStream_t s, int sides) {
    hipError_t e = hipSuccess;
    if (sides & kQuerySide) {
        NA_LAUNCH("na_rpb_dq", k_rpb_dq<T>, dim3(rgrid(p, p.Dqk)), dim3(256), 0, s, p, (const T*)da, lda, (const T*)k,
                  lk, (T*)dq, ldq);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    if (sides & kKeySide) {
        NA_LAUNCH("na_rpb_dk", k_rpb_keyside<T>, dim3(rgrid(p, p.Dqk)), dim3(256), 0, s, p, (const T*)da, lda,
                  (const T*)q, lq, p.Dqk, (T*)dk, ldk);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    return drpb ? rpb_dbias_t<T>(p, da, lda, drpb, work, work_floats, s) : hipSuccess;
}


template <typename T>
hipError_t rpb_av_bwd_t(const RProb& p, const void* dout, Lay ldo, const void* attn, Lay la, const void* v, Lay lv,
                        void* da, Lay lda, void* dv, Lay ldv, hipStream_t s, int sides) {
    if (sides & kQuerySide) {
        NA_LAUNCH("na_rpb_dattn", k_rpb_dattn<T>, dim3(rgrid(p, p.kv)), dim3(256), 0, s, p, (const T*)dout, ldo,
                  (const T*)v, lv, (T*)da, lda);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    if (!(sides & kKeySide)) return hipSuccess;
    NA_LAUNCH("na_rpb_dv", k_rpb_keyside<T>, dim3(rgrid(p, p.Dv)), dim3(256), 0, s, p, (const T*)attn, la,
              (const T*)dout, ldo, p.Dv, (T*)dv, ldv);
    return hipGetLastError();
}

RProb to_rprob(const Prob& P) {
    RProb r{};
    r.B = P.B;
    r.H = P.Hq;
    r.Dqk = P.Dqk;
    r.Dv = P.Dv;
    for (int a = 0; a < 2; ++a) {
        const Axis& A = P.ax[a + 1];
        r.ax[a] = RAxis{A.len, A.k, A.k / 2, A.dil};
        r.rs[a] = 2 * A.k - 1;
    }
    r.kv = r.ax[0].K * r.ax[1].K;
    return r;
}

}  // namespace

hipError_t rpb_qk(const Prob& P, const void* q, Lay lq, const void* k, Lay lk, const void* rpb, void* attn, Lay la,
                  int dtype, hipStream_t s) {
    const RProb p = to_rprob(P);
    if (dtype == NATTEN_F32) return rpb_qk_t<float>(p, q, lq, k, lk, rpb, attn, la, s);
    if (dtype == NATTEN_F16) return rpb_qk_t<f16>(p, q, lq, k, lk, rpb, attn, la, s);
    return rpb_qk_t<bf16>(p, q, lq, k, lk, rpb, attn, la, s);
}

hipError_t rpb_av(const Prob& P, const void* attn, Lay la, const void* v, Lay lv, void* out, Lay lo, int dtype,
                  hipStream_t s) {
    const RProb p = to_rprob(P);
    if (dtype == NATTEN_F32) return rpb_av_t<float>(p, attn, la, v, lv, out, lo, s);
    if (dtype == NATTEN_F16) return rpb_av_t<f16>(p, attn, la, v, lv, out, lo, s);
    return rpb_av_t<bf16>(p, attn, la, v, lv, out, lo, s);
}

hipError_t rpb_qk_backward(const Prob& P, const void* da, Lay lda, const void* q, Lay lq, const void* k, Lay lk,
                           void* dq, Lay ldq, void* dk, Lay ldk, void* drpb, int dtype, hipStream_t s, int sides,
                           float* work, size_t work_floats) {
    const RProb p = to_rprob(P);
    if (dtype == NATTEN_F32)
        return rpb_qk_bwd_t<float>(p, da, lda, q, lq, k, lk, dq, ldq, dk, ldk, drpb, work, work_floats, s, sides);
    if (dtype == NATTEN_F16)
        return rpb_qk_bwd_t<f16>(p, da, lda, q, lq, k, lk, dq, ldq, dk, ldk, drpb, work, work_floats, s, sides);
    return rpb_qk_bwd_t<bf16>(p, da, lda, q, lq, k, lk, dq, ldq, dk, ldk, drpb, work, work_floats, s, sides);
}

size_t rpb_dbias_workspace(const Prob& P) { return dbias_work_floats(to_rprob(P)); }

hipError_t rpb_av_backward(const Prob& P, const void* dout, Lay ldo, const void* attn, Lay la, const void* v, Lay lv,
                           void* da, Lay lda, void* dv, Lay ldv, int dtype, hipStream_t s, int sides) {
    const RProb p = to_rprob(P);
    if (dtype == NATTEN_F32) return rpb_av_bwd_t<float>(p, dout, ldo, attn, la, v, lv, da, lda, dv, ldv, s, sides);
    if (dtype == NATTEN_F16) return rpb_av_bwd_t<f16>(p, dout, ldo, attn, la, v, lv, da, lda, dv, ldv, s, sides);
    return rpb_av_bwd_t<bf16>(p, dout, ldo, attn, la, v, lv, da, lda, dv, ldv, s, sides);
}

}  // namespace na

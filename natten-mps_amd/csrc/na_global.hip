// Key side of the backward for global keys: extra tokens that every query
// attends besides its neighbourhood (the reference's additional_keys /
// additional_values, functional.py:74-110 with the merge of merge.py:21-156,
// here folded into the fused kernels).  The forward and the dQ kernel take
// them as extra 32-key chunks of their online softmax (na_mfma.hip, GLOBAL
// instances); this file computes their gradients:
//   dv_g = sum over all queries q (every q head of the GQA group) of P dO,
//   dk_g = scale * sum P (dP - delta) q,
// with P = exp(scale q.k_g - lse) and dP = dO.v_g, from the forward's lse and
// the backward's delta.
//
// A workgroup (one wave) holds 16 global keys as MFMA fragments and walks a
// slice of the query rows (q head within the group x query position), 32
// rows at a time staged in LDS as the key-side tile kernel stages a union;
// the products are those of k_bwd_kv_mfma.  Slices write fp32 partial sums;
// a second pass adds them in slice order (deterministic) and rounds once.
#include "na_tile.h"

namespace na {

namespace {

template <typename T>
struct GlobalKvArgs {
    Prob p;
    const T *q, *dout;
    const float *lse, *delta;
    LayK lq, ldo, ll, lde;
    GlobalKeys<T> g;
    float* part;  // [splits][B][Hkv][blocks * 16][2][D]: dk then dv
    int rows, rows_per_split, blocks;
    FastDiv nout, out2, out1;
};

// Query row r of a kv head's group -> q head within the group (r / nout) and
// position (i0, i1, i2), row-major over the axes.
template <typename T>
__device__ __forceinline__ int row_head_pos(const GlobalKvArgs<T>& a, int r, int (&i)[3]) {
    const int h_in = fdiv(r, a.nout);
    int pos = r - h_in * static_cast<int>(a.nout.d);
    int t = fdiv(pos, a.out2);
    i[2] = pos - t * static_cast<int>(a.out2.d);
    pos = t;
    t = fdiv(pos, a.out1);
    i[1] = pos - t * static_cast<int>(a.out1.d);
    i[0] = t;
    return h_in;
}

template <typename T, int D>
__global__ __launch_bounds__(64) void k_global_kv(GlobalKvArgs<T> a) {
    constexpr int LD = lds_dim<D>(), P = LD / 8, R = 64 / P;
    constexpr int E = static_cast<int>(sizeof(T));
    __shared__ __attribute__((aligned(16))) T Qs[32 * LD];
    __shared__ __attribute__((aligned(16))) T Gs[32 * LD];
    __shared__ __attribute__((aligned(16))) float NL[32];
    __shared__ __attribute__((aligned(16))) float ND[32];
    const Prob& p = a.p;
    const int lane = threadIdx.x, col = lane & 15, grp = lane >> 4;
    int x = blockIdx.x;
    const int kblk = x % a.blocks;
    x /= a.blocks;
    const int hk = x % p.Hkv;
    x /= p.Hkv;
    const int b = x % p.B;
    const int split = x / p.B;
    const int j = kblk * 16 + col;
    const bool key_ok = j < a.g.n;

    // the 16 keys and values as MFMA fragments (zero past n)
    uint4 kf[D / 32], vf[D / 32];
    load_frags<T, D>(a.g.k + b * a.g.kb + hk * a.g.kh, static_cast<long long>(j) * a.g.ks, key_ok, grp, kf);
    load_frags<T, D>(a.g.v + b * a.g.vb + hk * a.g.vh, static_cast<long long>(j) * a.g.vs, key_ok, grp, vf);
    f32x4_t gk[D / 16], gv[D / 16];
#pragma unroll
    for (int db = 0; db < D / 16; ++db) gk[db] = gv[db] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    const T* qb = a.q + b * a.lq.b;
    const T* gb = a.dout + b * a.ldo.b;
    const float* lb = a.lse + b * a.ll.b;
    const float* db_ = a.delta + b * a.lde.b;
    const __amdgpu_buffer_rsrc_t rq =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(qb), static_cast<short>(0), kPlaneBytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rg =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(gb), static_cast<short>(0), kPlaneBytes, 0x00020000);
    const float sc2 = p.scale * kLog2e;
    const f32x4_t zero[2] = {f32x4_t{0.f, 0.f, 0.f, 0.f}, f32x4_t{0.f, 0.f, 0.f, 0.f}};
    const int r_end = min(a.rows, (split + 1) * a.rows_per_split);
    for (int r0 = split * a.rows_per_split; r0 < r_end; r0 += 32) {
        // 32 rows of q and dO, swizzled as a staged union (slot = row - r0)
#pragma unroll
        for (int i = 0; i < 32 / R; ++i) {
            const int slot = i * R + lane / P, r = r0 + slot;
            int pos[3];
            const int h = hk * p.rep + row_head_pos(a, min(r, a.rows - 1), pos);
            const int piece16 = ((lane % P) ^ swz<LD>(slot)) << 4;
            const bool ok = r < r_end && (piece16 >> 4) < D / 8;
            const int oq = h * static_cast<int>(a.lq.h) + vol_off(a.lq, pos);
            const int og = h * static_cast<int>(a.ldo.h) + vol_off(a.ldo, pos);
            const uint32_t vq = ok ? static_cast<uint32_t>(oq * E + piece16) : kOutOfRange;
            const uint32_t vg = ok ? static_cast<uint32_t>(og * E + piece16) : kOutOfRange;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rq, (lds_void_t*)(Qs + i * R * LD), 16, vq, 0, 0, 0);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rg, (lds_void_t*)(Gs + i * R * LD), 16, vg, 0, 0, 0);
        }
        // per row: -lse * log2 e and -delta (-inf / 0 past the slice)
        if (lane < 32) {
            const int r = r0 + lane;
            float nl = -INFINITY, nd = 0.f;
            if (r < r_end) {
                int pos[3];
                const int h = hk * p.rep + row_head_pos(a, r, pos);
                nl = -lb[h * a.ll.h + vol_off(a.ll, pos)] * kLog2e;
                nd = -db_[h * a.lde.h + vol_off(a.lde, pos)];
            }
            NL[lane] = nl;
            ND[lane] = nd;
        }
        wait_loads();
        lds_publish_barrier();  // staged rows and the per-row scalars
        const int s0 = 8 * grp;
        const f32x4_t ndc[2] = {*reinterpret_cast<const f32x4_t*>(ND + s0),
                                *reinterpret_cast<const f32x4_t*>(ND + s0 + 4)};
        const f32x4_t nl[2] = {*reinterpret_cast<const f32x4_t*>(NL + s0),
                               *reinterpret_cast<const f32x4_t*>(NL + s0 + 4)};
        f32x4_t s[2], dp[2];
        score_chunk<T, D>(Qs, 0, col, grp, kf, zero, s);
        score_chunk<T, D>(Gs, 0, col, grp, vf, ndc, dp);
#pragma unroll
        for (int bb = 0; bb < 2; ++bb)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                s[bb][i] = __builtin_amdgcn_exp2f(fmaf(s[bb][i], sc2, nl[bb][i]));
                dp[bb][i] *= s[bb][i];
            }
        accumulate_chunk<T, D>(Gs, 0, lane, pack8<T>(s), gv);
        accumulate_chunk<T, D>(Qs, 0, lane, pack8<T>(dp), gk);
        __syncthreads();  // the rows are no longer read
    }
    // the lane's dims 16 db + 4 grp .. +3 of key j
    float* out = a.part + ((((static_cast<long long>(split) * p.B + b) * p.Hkv + hk) * a.blocks + kblk) * 16 + col) *
                              (2 * D);
#pragma unroll
    for (int db = 0; db < D / 16; ++db) {
        *reinterpret_cast<f32x4_t*>(out + 16 * db + 4 * grp) = gk[db];
        *reinterpret_cast<f32x4_t*>(out + D + 16 * db + 4 * grp) = gv[db];
    }
}

// dk_g = scale * sum over slices, dv_g = sum over slices, in slice order.
template <typename T>
__global__ __launch_bounds__(256) void k_global_reduce(const float* __restrict__ part, int splits, int B, int Hkv,
                                                       int blocks, int n, int D, float scale, T* __restrict__ dk,
                                                       LayK ldk, T* __restrict__ dv, LayK ldv) {
    const long long total = static_cast<long long>(B) * Hkv * n * D;
    const long long idx = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= total) return;
    const int d = static_cast<int>(idx % D);
    long long t = idx / D;
    const int j = static_cast<int>(t % n);
    t /= n;
    const int hk = static_cast<int>(t % Hkv);
    const int b = static_cast<int>(t / Hkv);
    const long long per_split = static_cast<long long>(B) * Hkv * blocks * 16 * 2 * D;
    const float* src = part + ((static_cast<long long>(b) * Hkv + hk) * blocks * 16 + j) * 2 * D + d;
    float sk = 0.f, sv = 0.f;
    for (int s = 0; s < splits; ++s) {
        sk += src[s * per_split];
        sv += src[s * per_split + D];
    }
    dk[b * ldk.b + hk * ldk.h + static_cast<long long>(j) * ldk.s2 + d] = from_f<T>(sk * scale);
    dv[b * ldv.b + hk * ldv.h + static_cast<long long>(j) * ldv.s2 + d] = from_f<T>(sv);
}

// Slices of the query rows: about 2048 workgroups in all, each slice a
// multiple of 32 rows and at least 64 (unless the rows are fewer).
struct GlobalSplit {
    int rows, rows_per_split, splits, blocks;
};

GlobalSplit global_split(const Prob& p, int n) {
    GlobalSplit s;
    s.rows = p.rep * p.nout;
    s.blocks = (n + 15) / 16;
    const long long groups = static_cast<long long>(p.B) * p.Hkv * s.blocks;
    const long long want = std::max<long long>(1, (2048 + groups - 1) / groups);
    const long long cap = std::max<long long>(1, (s.rows + 63) / 64);
    const long long splits = std::min(want, cap);
    s.rows_per_split = static_cast<int>(((s.rows + splits - 1) / splits + 31) / 32 * 32);
    s.splits = (s.rows + s.rows_per_split - 1) / s.rows_per_split;
    return s;
}

// Byte offsets of a q-side operand within one batch (every head and position)
// stay in 31 bits, strides non-negative.
bool batch_offsets_fit(const Prob& p, const Lay& l, int esz) {
    if (l.b < 0 || l.h < 0 || l.s0 < 0 || l.s1 < 0 || l.s2 < 0) return false;
    long long last = (static_cast<long long>(p.Hq) - 1) * l.h;
    for (int a = 0; a < 3; ++a) {
        const long long st = a == 0 ? l.s0 : a == 1 ? l.s1 : l.s2;
        last += (static_cast<long long>(p.ax[a].out) - 1) * st;
    }
    return (last + 256) * esz < kPlaneBytes;
}

template <typename T, int D>
hipError_t run_global_kv(const Prob& p, const void* q, Lay lq, const void* dout, Lay ldo, const float* lse, Lay ll,
                         const float* delta, Lay lde, const GlobalSet& g, void* dk, Lay ldk, void* dv, Lay ldv,
                         float* work, hipStream_t s) {
    const GlobalSplit sp = global_split(p, g.n);
    GlobalKvArgs<T> a{};
    a.p = p;
    a.q = static_cast<const T*>(q);
    a.dout = static_cast<const T*>(dout);
    a.lse = lse;
    a.delta = delta;
    a.lq = to_k(lq);
    a.ldo = to_k(ldo);
    a.ll = to_k(ll);
    a.lde = to_k(lde);
    a.g = GlobalKeys<T>{static_cast<const T*>(g.k), static_cast<const T*>(g.v), g.lk.b, g.lk.h, g.lv.b, g.lv.h,
                        static_cast<int>(g.lk.s2), static_cast<int>(g.lv.s2), g.n};
    a.part = work;
    a.rows = sp.rows;
    a.rows_per_split = sp.rows_per_split;
    a.blocks = sp.blocks;
    a.nout = make_fastdiv(static_cast<uint32_t>(p.nout));
    a.out2 = make_fastdiv(static_cast<uint32_t>(p.ax[2].out));
    a.out1 = make_fastdiv(static_cast<uint32_t>(p.ax[1].out));
    const long long grid = static_cast<long long>(sp.splits) * p.B * p.Hkv * sp.blocks;
    NA_LAUNCH("na_global_kv_mfma", (k_global_kv<T, D>), dim3(static_cast<unsigned>(grid)), dim3(64), 0, s, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const long long total = static_cast<long long>(p.B) * p.Hkv * g.n * D;
    NA_LAUNCH("na_global_reduce", k_global_reduce<T>, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0,
              s, (const float*)work, sp.splits, p.B, p.Hkv, sp.blocks, g.n, D, p.scale, static_cast<T*>(dk), to_k(ldk),
              static_cast<T*>(dv), to_k(ldv));
    return hipGetLastError();
}

}  // namespace

bool mfma_global_key_ok(const Prob& p, int dtype, const GlobalSet& g) {
    if (dtype == NATTEN_F32 || g.n < 1 || !(p.Dqk == 32 || p.Dqk == 64 || p.Dqk == 96 || p.Dqk == 128) ||
        p.Dqk != p.Dv)
        return false;
    for (const Lay* l : {&g.lk, &g.lv})
        if (l->b < 0 || l->h < 0 || l->s2 < 0 ||
            (static_cast<long long>(g.n) * l->s2 + 256) * 2 >= kPlaneBytes)
            return false;
    const GlobalSplit sp = global_split(p, g.n);
    const long long grid = static_cast<long long>(sp.splits) * p.B * p.Hkv * sp.blocks;
    return grid < (1LL << 31) && static_cast<long long>(p.rep) * p.nout < (1LL << 31);
}

bool mfma_global_batch_fit(const Prob& p, const Lay& lq, const Lay& ldo) {
    return batch_offsets_fit(p, lq, 2) && batch_offsets_fit(p, ldo, 2);
}

size_t global_workspace_floats(const Prob& p, int n) {
    const GlobalSplit sp = global_split(p, n);
    return static_cast<size_t>(sp.splits) * p.B * p.Hkv * sp.blocks * 16 * 2 * std::max(p.Dqk, p.Dv);
}

hipError_t mfma_global_key_backward(const Prob& p, const void* q, Lay lq, const void* dout, Lay ldo, const float* lse,
                                    Lay ll, const float* delta, Lay lde, const GlobalSet& g, void* dk, Lay ldk,
                                    void* dv, Lay ldv, float* work, int dtype, hipStream_t s) {
    if (!batch_offsets_fit(p, lq, 2) || !batch_offsets_fit(p, ldo, 2)) return hipErrorInvalidValue;
#define NA_GKV(TT, DD) return run_global_kv<TT, DD>(p, q, lq, dout, ldo, lse, ll, delta, lde, g, dk, ldk, dv, ldv, work, s)
    if (dtype == NATTEN_BF16) {
        if (p.Dqk == 32) NA_GKV(bf16, 32);
        if (p.Dqk == 64) NA_GKV(bf16, 64);
        if (p.Dqk == 96) NA_GKV(bf16, 96);
        NA_GKV(bf16, 128);
    }
    if (p.Dqk == 32) NA_GKV(f16, 32);
    if (p.Dqk == 64) NA_GKV(f16, 64);
    if (p.Dqk == 96) NA_GKV(f16, 96);
    NA_GKV(f16, 128);
#undef NA_GKV
}

}  // namespace na

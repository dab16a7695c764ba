// MFMA tile kernels (gfx950, bf16 / fp16, stride 1, head dim 32/64/128):
// forward, backward-dQ (query-centric) and backward-dK/dV (key-centric).
//
// Tiling.  With dilation d an axis splits into d residue classes; a query and
// every key of its window share the class, and inside a class the window is
// an undilated run of K positions (class coordinates j = (i - r) / d).  A
// workgroup owns a box of up to 64 queries (or keys) of one class triple
// (r0, r1, r2) and one (batch, head).  The union of their windows (or, for
// keys, of the queries attending them) is a box in class coordinates, staged
// one axis-0 plane ("slice") at a time in LDS, slot = (u1-lo1)*U2 + (u2-lo2),
// zero padded to a multiple of 32, both row-major (Xs[slot][D]) and, where a
// product contracts over slots, transposed (Xt[D][slot]).
//
// Each wave owns 16 queries (keys) and walks the staged slots 32 at a time
// with v_mfma_f32_16x16x32: the score block is computed with the slots as
// MFMA rows, split over two 16-row blocks whose rows interleave so that every
// lane ends up holding 8 consecutive slots of one query (key) -- exactly the
// B-operand layout of the following product that contracts over those slots.
// Softmax runs in the log2 domain in fp32; probabilities and score gradients
// enter the second product rounded to the input dtype, accumulators are fp32.
//
// MFMA lane layout (16x16x32): A row = lane%16, B column = lane%16, both with
// k = 8*(lane/16) .. +7; C column = lane%16, rows 4*(lane/16) .. +3.
#include "na_launch.h"

namespace na {

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr int kPad = 8;  // elements of padding per LDS row (spreads rows over banks)

template <typename T>
struct Mma;

template <>
struct Mma<bf16> {
    __device__ static __forceinline__ f32x4_t run(uint4 a, uint4 b, f32x4_t c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                       __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
    }
    __device__ static __forceinline__ uint32_t pack(float lo, float hi) {
        return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t{lo, hi}), bf16x2_t));
    }
};

template <>
struct Mma<f16> {
    __device__ static __forceinline__ f32x4_t run(uint4 a, uint4 b, f32x4_t c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                      __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
    }
    __device__ static __forceinline__ uint32_t pack(float lo, float hi) {
        return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t{lo, hi}), f16x2_t));
    }
};

template <typename T>
__device__ __forceinline__ uint4 pack8(const float (&v)[8]) {
    return make_uint4(Mma<T>::pack(v[0], v[1]), Mma<T>::pack(v[2], v[3]), Mma<T>::pack(v[4], v[5]),
                      Mma<T>::pack(v[6], v[7]));
}

__device__ __forceinline__ int imin16(int v) {
#pragma unroll
    for (int m = 1; m < 16; m <<= 1) v = min(v, __shfl_xor(v, m));
    return v;
}

__device__ __forceinline__ int imax16(int v) {
#pragma unroll
    for (int m = 1; m < 16; m <<= 1) v = max(v, __shfl_xor(v, m));
    return v;
}

__device__ __forceinline__ float sum_groups(float v) {
    v += __shfl_xor(v, 16);
    return v + __shfl_xor(v, 32);
}

__device__ __forceinline__ float max_groups(float v) {
    v = fmaxf(v, __shfl_xor(v, 16));
    return fmaxf(v, __shfl_xor(v, 32));
}

}  // namespace

// Host-chosen tile: extents (class coordinates) of a workgroup's box, tiles
// per class per axis, waves per workgroup, and the staged slice layout: slot
// = a1 * rowlen + a2 for union row a1 and column a2, with rowlen = 2^rowshift
// >= 8 covering the widest union row (so a lane's 8 consecutive slots never
// straddle two rows), `slots` = staged slots per slice (multiple of 32).
struct TileShape {
    int T[3];
    int ntile[3];
    int waves;
    int slots;
    int rowlen;
    int rowshift;
};

namespace {

struct Block {
    int b, h, r[3], J[3], E[3], lo[3], U[3];
    ClassAxis c[3];
};

// Workgroup -> (batch, head, residues, tile origin J, clipped extent E) and
// the union box [lo, lo+U) of the windows of its queries (key_tile = false)
// or of the queries attending its keys (key_tile = true).  False: empty tile.
__device__ __forceinline__ bool decode_block(const Prob& p, const TileShape& ts, int heads, bool key_tile,
                                             Block& k) {
    int bid = xcd_block(blockIdx.x, gridDim.x);
    k.h = bid % heads;
    bid /= heads;
    int t[3];
    for (int a = 2; a >= 0; --a) {
        t[a] = bid % ts.ntile[a];
        bid /= ts.ntile[a];
        k.r[a] = bid % p.ax[a].dil;
        bid /= p.ax[a].dil;
    }
    k.b = bid;
    for (int a = 0; a < 3; ++a) {
        const ClassAxis c = class_axis(p.ax[a], k.r[a]);
        k.c[a] = c;
        k.J[a] = t[a] * ts.T[a];
        const int jend = min(k.J[a] + ts.T[a], c.n) - 1;
        k.E[a] = jend - k.J[a] + 1;
        if (k.E[a] <= 0) return false;
        int lo, hi;
        if (!key_tile) {
            lo = max(class_ws(c, k.J[a]), 0);
            hi = min(class_ws(c, jend) + c.K - 1, c.n - 1);
        } else {
            // both span ends are non-decreasing in the key; keys attended by
            // nobody (only past the last window at an even-kernel border) sit
            // at the end and leave hi unchanged
            int x;
            class_span(c, k.J[a], lo, x);
            class_span(c, jend, x, hi);
        }
        k.lo[a] = lo;
        k.U[a] = hi >= lo ? hi - lo + 1 : 0;
    }
    return true;
}

// Stage the slice of the union at axis-0 position p0 (all slots < `slots`):
// rows[slot][D] row-major and/or trans[D][slot] transposed, zeros past the
// union.  Offsets inside one (batch, head, axis-0 plane) fit in 32 bits
// (checked on the host).
template <typename T, int D>
__device__ __forceinline__ void stage(const Prob& p, const Block& k, const TileShape& ts, const T* __restrict__ g,
                                      Lay lay, int h, int p0, T* rows, T* trans) {
    constexpr int V8 = D / 8;
    const int slots = ts.slots;
    const int part = threadIdx.x % V8;
    const T* base = g + static_cast<long long>(k.b) * lay.b + static_cast<long long>(h) * lay.h +
                    static_cast<long long>(p0) * lay.s0 + part * 8;
    const int s1 = static_cast<int>(lay.s1), s2 = static_cast<int>(lay.s2);
    const int d1 = p.ax[1].dil, d2 = p.ax[2].dil;
    const int c1 = k.r[1] + k.lo[1] * d1, c2 = k.r[2] + k.lo[2] * d2;
#pragma unroll 2
    for (int sp = threadIdx.x / V8; 2 * sp < slots; sp += blockDim.x / V8) {
        // the pair 2sp, 2sp+1 shares a union row (rowlen is even)
        const int a1 = (2 * sp) >> ts.rowshift, a2 = (2 * sp) & (ts.rowlen - 1);
        const bool row_ok = a1 < k.U[1];
        const T* src = base + (c1 + a1 * d1) * s1 + (c2 + a2 * d2) * s2;
        uint4 x[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            x[e] = make_uint4(0, 0, 0, 0);
            if (row_ok && a2 + e < k.U[2]) x[e] = *reinterpret_cast<const uint4*>(src + e * d2 * s2);
        }
        if (rows) {
#pragma unroll
            for (int e = 0; e < 2; ++e) *reinterpret_cast<uint4*>(rows + (2 * sp + e) * (D + kPad) + part * 8) = x[e];
        }
        if (trans) {
            const uint16_t* a = reinterpret_cast<const uint16_t*>(&x[0]);
            const uint16_t* b = reinterpret_cast<const uint16_t*>(&x[1]);
#pragma unroll
            for (int j = 0; j < 8; ++j)
                *reinterpret_cast<uint32_t*>(trans + (part * 8 + j) * (slots + kPad) + 2 * sp) =
                    static_cast<uint32_t>(a[j]) | (static_cast<uint32_t>(b[j]) << 16);
        }
    }
}

// Stage per-slot fp32 values (lse in the log2 domain, delta) of the slice.
__device__ __forceinline__ void stage_scalars(const Prob& p, const Block& k, const TileShape& ts, int h, int p0,
                                              const float* __restrict__ lse, Lay ll, const float* __restrict__ delta,
                                              Lay lde, float* L2s, float* Ds) {
    for (int s = threadIdx.x; s < ts.slots; s += blockDim.x) {
        float l2 = 0.f, dd = 0.f;
        const int a1 = s >> ts.rowshift, a2 = s & (ts.rowlen - 1);
        if (a1 < k.U[1] && a2 < k.U[2]) {
            const int p1 = k.r[1] + (k.lo[1] + a1) * p.ax[1].dil, p2 = k.r[2] + (k.lo[2] + a2) * p.ax[2].dil;
            l2 = lse[ll.at(k.b, p0, p1, p2, h)] * kLog2e;
            dd = delta[lde.at(k.b, p0, p1, p2, h)];
        }
        L2s[s] = l2;
        Ds[s] = dd;
    }
}

// One lane's query (or key) of the wave: class coordinates and position.
struct Item {
    bool valid;
    int j[3], pos[3];
};

__device__ __forceinline__ Item wave_item(const Prob& p, const Block& k, int wave, int col) {
    Item it;
    const int n = k.E[0] * k.E[1] * k.E[2];
    const int f = wave * 16 + col;
    it.valid = f < n;
    const int ff = it.valid ? f : 0;
    const int e2 = ff % k.E[2], e1 = (ff / k.E[2]) % k.E[1], e0 = ff / (k.E[2] * k.E[1]);
    const int e[3] = {e0, e1, e2};
    for (int a = 0; a < 3; ++a) {
        it.j[a] = k.J[a] + e[a];
        it.pos[a] = k.r[a] + it.j[a] * p.ax[a].dil;
    }
    return it;
}

// The lane's admissible box in union-relative coordinates [rel_lo, rel_hi]
// per axis (windows for a query, attending queries for a key), and the
// wave-wide slot range covering all of them (for skipping slices/chunks).
struct Span {
    int lo[3], hi[3];   // lane, relative to the union origin
    int wlo[3], whi[3]; // wave
};

__device__ __forceinline__ Span lane_span(const Prob& p, const Block& k, const Item& it, bool key_side) {
    Span sp;
    for (int a = 0; a < 3; ++a) {
        int lo, hi;
        if (!key_side) {
            lo = class_ws(k.c[a], it.j[a]);
            hi = lo + k.c[a].K - 1;
        } else {
            class_span(k.c[a], it.j[a], lo, hi);
        }
        sp.lo[a] = lo - k.lo[a];
        sp.hi[a] = hi - k.lo[a];
        const bool live = it.valid && lo <= hi;
        sp.wlo[a] = imin16(live ? max(sp.lo[a], 0) : 1 << 30);
        sp.whi[a] = imax16(live ? min(sp.hi[a], k.U[a] - 1) : -(1 << 30));
    }
    return sp;
}

// Bit e set when slot s0 + e (s0 a multiple of 8, so all in one union row) is
// admissible for this lane: its row in [lo1, hi1] and column in [lo2, hi2].
// Padding columns lie past hi2 and padding rows past hi1.
__device__ __forceinline__ unsigned chunk_mask(const Span& sp, bool in0, int s0, const TileShape& ts) {
    const int a1 = s0 >> ts.rowshift, a2 = s0 & (ts.rowlen - 1);
    if (!in0 || a1 < sp.lo[1] || a1 > sp.hi[1]) return 0u;
    const int lo = sp.lo[2] - a2, hi = sp.hi[2] - a2;  // admissible bit range
    if (hi < 0 || lo > 7) return 0u;
    return (0xFFu << (lo > 0 ? lo : 0)) & (0xFFu >> (hi < 7 ? 7 - hi : 0));
}

// First and last chunk covering the wave's admissible box.
__device__ __forceinline__ void chunk_range(const Span& sp, const TileShape& ts, int& c0, int& c1) {
    c0 = (sp.wlo[1] * ts.rowlen + sp.wlo[2]) >> 5;
    c1 = (sp.whi[1] * ts.rowlen + sp.whi[2]) >> 5;
}

// Score block: rows = 32 slots of chunk c (A operand from row-major LDS),
// columns = the wave's 16 items (B operand fragments).  Returns the lane's 8
// slots 32c + 8grp + [0..7] in order.
template <typename T, int D>
__device__ __forceinline__ void score_chunk(const T* rows, int c, int col, int grp, const uint4 (&frag)[D / 32],
                                            float (&out)[8]) {
#pragma unroll
    for (int b = 0; b < 2; ++b) {
        const int row = 32 * c + 8 * (col >> 2) + 4 * b + (col & 3);
        f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < D / 32; ++ks) {
            const uint4 a = *reinterpret_cast<const uint4*>(rows + row * (D + kPad) + ks * 32 + grp * 8);
            acc = Mma<T>::run(a, frag[ks], acc);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) out[4 * b + i] = acc[i];
    }
}

// acc[db] (16 head dims x 16 items) += trans[d][32 slots of chunk c] * packed.
template <typename T, int D>
__device__ __forceinline__ void accumulate_chunk(const T* trans, int slots, int c, int col, int grp, uint4 packed,
                                                 f32x4_t (&acc)[D / 16]) {
#pragma unroll
    for (int db = 0; db < D / 16; ++db) {
        const uint4 a = *reinterpret_cast<const uint4*>(trans + (db * 16 + col) * (slots + kPad) + 32 * c + 8 * grp);
        acc[db] = Mma<T>::run(a, packed, acc[db]);
    }
}

template <typename T, int D>
__device__ __forceinline__ void load_frags(const T* __restrict__ g, long long off, bool valid, int grp,
                                           uint4 (&f)[D / 32]) {
#pragma unroll
    for (int ks = 0; ks < D / 32; ++ks)
        f[ks] = valid ? *reinterpret_cast<const uint4*>(g + off + ks * 32 + grp * 8) : make_uint4(0, 0, 0, 0);
}

// Store the lane's 4 consecutive head dims per 16-dim block (scaled).
template <typename T, int D>
__device__ __forceinline__ void store_rows(T* __restrict__ g, long long off, int grp, const f32x4_t (&acc)[D / 16],
                                           float mul) {
#pragma unroll
    for (int db = 0; db < D / 16; ++db) {
        const uint2 w = make_uint2(Mma<T>::pack(acc[db][0] * mul, acc[db][1] * mul),
                                   Mma<T>::pack(acc[db][2] * mul, acc[db][3] * mul));
        *reinterpret_cast<uint2*>(g + off + db * 16 + grp * 4) = w;
    }
}

// ---------------------------------------------------------------------------
// Forward: out = softmax(scale q.k) v over each window, lse (natural log).
// ---------------------------------------------------------------------------
template <typename T, int D>
__global__ __launch_bounds__(256) void k_fwd_mfma(Prob p, TileShape ts, const T* __restrict__ q, Lay lq,
                                                  const T* __restrict__ kg, Lay lk, const T* __restrict__ vg,
                                                  Lay lv, T* __restrict__ out, Lay lo, float* __restrict__ lse,
                                                  Lay ll) {
    extern __shared__ __align__(16) unsigned char smem[];
    Block blk;
    if (!decode_block(p, ts, p.Hq, false, blk)) return;
    const int slots = ts.slots;
    T* Ks = reinterpret_cast<T*>(smem);
    T* Vt = Ks + slots * (D + kPad);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, col = lane & 15, grp = lane >> 4;
    const int hk = blk.h / p.rep;

    const Item it = wave_item(p, blk, wave, col);
    const Span sp = lane_span(p, blk, it, false);
    uint4 qf[D / 32];
    load_frags<T, D>(q, lq.at(blk.b, it.pos[0], it.pos[1], it.pos[2], blk.h), it.valid, grp, qf);

    f32x4_t acc[D / 16];
#pragma unroll
    for (int db = 0; db < D / 16; ++db) acc[db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    float m = -INFINITY, lsum = 0.f;  // running max and sum, log2 domain (scores times scale*log2 e)
    const float sc2 = p.scale * kLog2e;
    int c0, c1;
    chunk_range(sp, ts, c0, c1);

    for (int u0 = 0; u0 < blk.U[0]; ++u0) {
        const int p0 = blk.r[0] + (blk.lo[0] + u0) * p.ax[0].dil;
        __syncthreads();
        stage<T, D>(p, blk, ts, kg, lk, hk, p0, Ks, nullptr);
        stage<T, D>(p, blk, ts, vg, lv, hk, p0, nullptr, Vt);
        __syncthreads();
        if (u0 < sp.wlo[0] || u0 > sp.whi[0]) continue;
        const bool in0 = it.valid && u0 >= sp.lo[0] && u0 <= sp.hi[0];
        for (int c = c0; c <= c1; ++c) {
            float sv[8];
            score_chunk<T, D>(Ks, c, col, grp, qf, sv);
            const unsigned msk = chunk_mask(sp, in0, 32 * c + 8 * grp, ts);
            float cmax = -INFINITY;
#pragma unroll
            for (int e = 0; e < 8; ++e) cmax = fmaxf(cmax, (msk >> e) & 1u ? sv[e] : -INFINITY);
            const float mnew = fmaxf(m, max_groups(cmax) * sc2);
            const float mref = mnew == -INFINITY ? 0.f : mnew;
            const float corr = __builtin_amdgcn_exp2f(m - mref);
            m = mnew;
            lsum *= corr;
#pragma unroll
            for (int db = 0; db < D / 16; ++db) acc[db] *= corr;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                sv[e] = (msk >> e) & 1u ? __builtin_amdgcn_exp2f(fmaf(sv[e], sc2, -mref)) : 0.f;
                lsum += sv[e];
            }
            accumulate_chunk<T, D>(Vt, slots, c, col, grp, pack8<T>(sv), acc);
        }
    }

    lsum = sum_groups(lsum);
    if (!it.valid) return;
    store_rows<T, D>(out, lo.at(blk.b, it.pos[0], it.pos[1], it.pos[2], blk.h), grp, acc, 1.f / lsum);
    if (grp == 0) lse[ll.at(blk.b, it.pos[0], it.pos[1], it.pos[2], blk.h)] = (m + __log2f(lsum)) * kLn2;
}

// ---------------------------------------------------------------------------
// Backward, query side: delta = dO . O - dlse (written for the key side) and
// dq = scale * sum_k P (dP - delta) k, with P = exp(scale q.k - lse) and
// dP = dO . v.
// ---------------------------------------------------------------------------
template <typename T, int D>
__global__ __launch_bounds__(256) void k_bwd_q_mfma(Prob p, TileShape ts, const T* __restrict__ q, Lay lq,
                                                    const T* __restrict__ kg, Lay lk, const T* __restrict__ vg,
                                                    Lay lv, const T* __restrict__ o, Lay lo,
                                                    const T* __restrict__ dout, Lay ldo,
                                                    const float* __restrict__ lse, Lay ll,
                                                    const float* __restrict__ dlse, Lay ldl, T* __restrict__ dq,
                                                    Lay ldq, float* __restrict__ delta, Lay lde) {
    extern __shared__ __align__(16) unsigned char smem[];
    Block blk;
    if (!decode_block(p, ts, p.Hq, false, blk)) return;
    const int slots = ts.slots;
    T* Ks = reinterpret_cast<T*>(smem);
    T* Vs = Ks + slots * (D + kPad);
    T* Kt = Vs + slots * (D + kPad);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, col = lane & 15, grp = lane >> 4;
    const int hk = blk.h / p.rep;

    const Item it = wave_item(p, blk, wave, col);
    const Span sp = lane_span(p, blk, it, false);
    uint4 qf[D / 32], gf[D / 32], of[D / 32];
    const long long qoff = lq.at(blk.b, it.pos[0], it.pos[1], it.pos[2], blk.h);
    load_frags<T, D>(q, qoff, it.valid, grp, qf);
    load_frags<T, D>(dout, ldo.at(blk.b, it.pos[0], it.pos[1], it.pos[2], blk.h), it.valid, grp, gf);
    load_frags<T, D>(o, lo.at(blk.b, it.pos[0], it.pos[1], it.pos[2], blk.h), it.valid, grp, of);
    const float L2 = it.valid ? lse[ll.at(blk.b, it.pos[0], it.pos[1], it.pos[2], blk.h)] * kLog2e : 0.f;
    // delta from this lane's 8 head dims per 32, summed over the 4 lane groups
    float di = 0.f;
#pragma unroll
    for (int ks = 0; ks < D / 32; ++ks) {
        const T* g8 = reinterpret_cast<const T*>(&gf[ks]);
        const T* o8 = reinterpret_cast<const T*>(&of[ks]);
#pragma unroll
        for (int e = 0; e < 8; ++e) di = fmaf(to_f(g8[e]), to_f(o8[e]), di);
    }
    di = sum_groups(di);
    if (dlse && it.valid) di -= dlse[ldl.at(blk.b, it.pos[0], it.pos[1], it.pos[2], blk.h)];
    if (it.valid && grp == 0) delta[lde.at(blk.b, it.pos[0], it.pos[1], it.pos[2], blk.h)] = di;
    const float sc2 = p.scale * kLog2e;
    int c0, c1;
    chunk_range(sp, ts, c0, c1);

    f32x4_t acc[D / 16];
#pragma unroll
    for (int db = 0; db < D / 16; ++db) acc[db] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    for (int u0 = 0; u0 < blk.U[0]; ++u0) {
        const int p0 = blk.r[0] + (blk.lo[0] + u0) * p.ax[0].dil;
        __syncthreads();
        stage<T, D>(p, blk, ts, kg, lk, hk, p0, Ks, Kt);
        stage<T, D>(p, blk, ts, vg, lv, hk, p0, Vs, nullptr);
        __syncthreads();
        if (u0 < sp.wlo[0] || u0 > sp.whi[0]) continue;
        const bool in0 = it.valid && u0 >= sp.lo[0] && u0 <= sp.hi[0];
        for (int c = c0; c <= c1; ++c) {
            float sv[8], dp[8];
            score_chunk<T, D>(Ks, c, col, grp, qf, sv);
            score_chunk<T, D>(Vs, c, col, grp, gf, dp);
            const unsigned msk = chunk_mask(sp, in0, 32 * c + 8 * grp, ts);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float pe = (msk >> e) & 1u ? __builtin_amdgcn_exp2f(fmaf(sv[e], sc2, -L2)) : 0.f;
                sv[e] = pe * (dp[e] - di);
            }
            accumulate_chunk<T, D>(Kt, slots, c, col, grp, pack8<T>(sv), acc);
        }
    }
    if (!it.valid) return;
    store_rows<T, D>(dq, ldq.at(blk.b, it.pos[0], it.pos[1], it.pos[2], blk.h), grp, acc, p.scale);
}

// ---------------------------------------------------------------------------
// Backward, key side: for each key/value position, over every query (of each
// q head in the GQA group) whose window holds it:
//   dv = sum P dO,   dk = scale * sum P (dP - delta) q.
// ---------------------------------------------------------------------------
template <typename T, int D>
__global__ __launch_bounds__(256) void k_bwd_kv_mfma(Prob p, TileShape ts, const T* __restrict__ q, Lay lq,
                                                     const T* __restrict__ kg, Lay lk, const T* __restrict__ vg,
                                                     Lay lv, const T* __restrict__ dout, Lay ldo,
                                                     const float* __restrict__ lse, Lay ll,
                                                     const float* __restrict__ delta, Lay lde,
                                                     T* __restrict__ dk, Lay ldk, T* __restrict__ dv, Lay ldv) {
    extern __shared__ __align__(16) unsigned char smem[];
    Block blk;
    if (!decode_block(p, ts, p.Hkv, true, blk)) return;
    const int slots = ts.slots;
    T* Qs = reinterpret_cast<T*>(smem);
    T* Gs = Qs + slots * (D + kPad);
    T* Qt = Gs + slots * (D + kPad);
    T* Gt = Qt + D * (slots + kPad);
    float* L2s = reinterpret_cast<float*>(Gt + D * (slots + kPad));
    float* Ds = L2s + slots;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, col = lane & 15, grp = lane >> 4;

    const Item it = wave_item(p, blk, wave, col);
    const Span sp = lane_span(p, blk, it, true);
    uint4 kf[D / 32], vf[D / 32];
    load_frags<T, D>(kg, lk.at(blk.b, it.pos[0], it.pos[1], it.pos[2], blk.h), it.valid, grp, kf);
    load_frags<T, D>(vg, lv.at(blk.b, it.pos[0], it.pos[1], it.pos[2], blk.h), it.valid, grp, vf);
    const float sc2 = p.scale * kLog2e;
    int c0, c1;
    chunk_range(sp, ts, c0, c1);

    f32x4_t gk[D / 16], gv[D / 16];
#pragma unroll
    for (int db = 0; db < D / 16; ++db) {
        gk[db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        gv[db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }

    for (int r = 0; r < p.rep; ++r) {
        const int h = blk.h * p.rep + r;
        for (int u0 = 0; u0 < blk.U[0]; ++u0) {
            const int p0 = blk.r[0] + (blk.lo[0] + u0) * p.ax[0].dil;
            __syncthreads();
            stage<T, D>(p, blk, ts, q, lq, h, p0, Qs, Qt);
            stage<T, D>(p, blk, ts, dout, ldo, h, p0, Gs, Gt);
            stage_scalars(p, blk, ts, h, p0, lse, ll, delta, lde, L2s, Ds);
            __syncthreads();
            if (u0 < sp.wlo[0] || u0 > sp.whi[0]) continue;
            const bool in0 = it.valid && u0 >= sp.lo[0] && u0 <= sp.hi[0];
            for (int c = c0; c <= c1; ++c) {
                float sv[8], dp[8];
                score_chunk<T, D>(Qs, c, col, grp, kf, sv);
                score_chunk<T, D>(Gs, c, col, grp, vf, dp);
                const int s0 = 32 * c + 8 * grp;
                const unsigned msk = chunk_mask(sp, in0, s0, ts);
                const float4 la = *reinterpret_cast<const float4*>(L2s + s0);
                const float4 lb = *reinterpret_cast<const float4*>(L2s + s0 + 4);
                const float4 da = *reinterpret_cast<const float4*>(Ds + s0);
                const float4 db4 = *reinterpret_cast<const float4*>(Ds + s0 + 4);
                const float l2[8] = {la.x, la.y, la.z, la.w, lb.x, lb.y, lb.z, lb.w};
                const float dd[8] = {da.x, da.y, da.z, da.w, db4.x, db4.y, db4.z, db4.w};
                float pe[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    pe[e] = (msk >> e) & 1u ? __builtin_amdgcn_exp2f(fmaf(sv[e], sc2, -l2[e])) : 0.f;
                    sv[e] = pe[e] * (dp[e] - dd[e]);
                }
                accumulate_chunk<T, D>(Gt, slots, c, col, grp, pack8<T>(pe), gv);
                accumulate_chunk<T, D>(Qt, slots, c, col, grp, pack8<T>(sv), gk);
            }
        }
    }
    if (!it.valid) return;
    store_rows<T, D>(dk, ldk.at(blk.b, it.pos[0], it.pos[1], it.pos[2], blk.h), grp, gk, p.scale);
    store_rows<T, D>(dv, ldv.at(blk.b, it.pos[0], it.pos[1], it.pos[2], blk.h), grp, gv, 1.f);
}

}  // namespace

// ---------------------------------------------------------------------------
// Host side: eligibility, tile choice, launches.
// ---------------------------------------------------------------------------

namespace {

enum Kind { kForward = 0, kBackwardQ = 1, kBackwardKV = 2 };

constexpr size_t kLdsBudget = 64 * 1024;

int n_class_h(const Axis& A, int r) { return (A.len - r + A.dil - 1) / A.dil; }

// Largest union extent on one axis over every class and tile (the same
// spans decode_block computes on the device).
int union_extent(const Axis& A, int T, bool key_tile) {
    int best = 1;
    for (int r = 0; r < A.dil; ++r) {
        const ClassAxis c = class_axis(A, r);
        for (int J = 0; J < c.n; J += T) {
            const int jend = (J + T < c.n ? J + T : c.n) - 1;
            int lo, hi, x;
            if (!key_tile) {
                lo = class_ws(c, J);
                lo = lo > 0 ? lo : 0;
                hi = class_ws(c, jend) + c.K - 1;
                hi = hi < c.n - 1 ? hi : c.n - 1;
            } else {
                class_span(c, J, lo, x);
                class_span(c, jend, x, hi);
            }
            if (hi - lo + 1 > best) best = hi - lo + 1;
        }
    }
    return best;
}

size_t lds_bytes(Kind kind, int slots, int D) {
    const size_t rows = static_cast<size_t>(slots) * (D + kPad) * 2;
    const size_t trans = static_cast<size_t>(D) * (slots + kPad) * 2;
    switch (kind) {
        case kForward: return rows + trans;
        case kBackwardQ: return 2 * rows + trans;
        default: return 2 * rows + 2 * trans + 2 * static_cast<size_t>(slots) * 4;
    }
}

// Workgroup box in class coordinates: up to 64 items (4 waves), innermost
// axis first; halved until the staged union fits the LDS budget.
bool choose_tile(const Prob& p, Kind kind, int D, TileShape& ts) {
    int n[3];
    for (int a = 0; a < 3; ++a) n[a] = n_class_h(p.ax[a], 0);  // class 0 is the longest
    for (int items = 64; items >= 16; items /= 2) {
        if (n[0] == 1 && n[1] == 1) {
            ts.T[2] = n[2] < items ? n[2] : items;
            ts.T[1] = ts.T[0] = 1;
        } else {
            ts.T[2] = n[2] < 8 ? n[2] : 8;
            const int r1 = items / ts.T[2] > 0 ? items / ts.T[2] : 1;
            ts.T[1] = n[1] < r1 ? n[1] : r1;
            const int r0 = items / (ts.T[2] * ts.T[1]) > 0 ? items / (ts.T[2] * ts.T[1]) : 1;
            ts.T[0] = n[0] < r0 ? n[0] : r0;
        }
        for (int a = 0; a < 3; ++a) ts.ntile[a] = (n[a] + ts.T[a] - 1) / ts.T[a];
        const int cnt = ts.T[0] * ts.T[1] * ts.T[2];
        ts.waves = (cnt + 15) / 16;
        const int u1 = union_extent(p.ax[1], ts.T[1], kind == kBackwardKV);
        const int u2 = union_extent(p.ax[2], ts.T[2], kind == kBackwardKV);
        ts.rowshift = 3;
        while ((1 << ts.rowshift) < u2) ++ts.rowshift;
        ts.rowlen = 1 << ts.rowshift;
        ts.slots = ((u1 * ts.rowlen + 31) / 32) * 32;
        if (lds_bytes(kind, ts.slots, D) <= kLdsBudget) return true;
    }
    return false;
}

template <typename K>
void allow_lds(K kernel, size_t bytes) {
    if (bytes > 64 * 1024)
        hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                            static_cast<int>(bytes));
}

long long grid_blocks(const Prob& p, const TileShape& ts, int heads) {
    long long nb = static_cast<long long>(p.B) * heads;
    for (int a = 0; a < 3; ++a) nb *= static_cast<long long>(p.ax[a].dil) * ts.ntile[a];
    return nb;
}

// 32-bit offsets inside one (batch, head, axis-0 plane) for every operand.
bool offsets_fit(const Prob& p, std::initializer_list<Lay> lays) {
    for (const Lay& l : lays) {
        const long long m = (static_cast<long long>(p.ax[1].len) - 1) * (l.s1 < 0 ? -l.s1 : l.s1) +
                            (static_cast<long long>(p.ax[2].len) - 1) * (l.s2 < 0 ? -l.s2 : l.s2) + 256;
        if (m >= (1LL << 31)) return false;
    }
    return true;
}

template <typename T, int D>
hipError_t launch_fwd(const Prob& p, const void* q, Lay lq, const void* k, Lay lk, const void* v, Lay lv, void* o,
                      Lay lo, float* lse, Lay ll, hipStream_t s) {
    TileShape ts{};
    choose_tile(p, kForward, D, ts);
    const size_t shm = lds_bytes(kForward, ts.slots, D);
    allow_lds(k_fwd_mfma<T, D>, shm);
    NA_LAUNCH("na_fwd_mfma", (k_fwd_mfma<T, D>), dim3(static_cast<unsigned>(grid_blocks(p, ts, p.Hq))),
              dim3(64 * ts.waves), shm, s, p, ts, (const T*)q, lq, (const T*)k, lk, (const T*)v, lv, (T*)o, lo, lse,
              ll);
    return hipGetLastError();
}

template <typename T, int D>
hipError_t launch_bwd(const Prob& p, const void* q, Lay lq, const void* k, Lay lk, const void* v, Lay lv,
                      const void* o, Lay lo, const void* dout, Lay ldo, const float* lse, Lay ll,
                      const float* dlse, Lay ldl, void* dq, Lay ldq, void* dk, Lay ldk, void* dv, Lay ldv,
                      float* delta, Lay lde, hipStream_t s) {
    TileShape tq{}, tk{};
    choose_tile(p, kBackwardQ, D, tq);
    choose_tile(p, kBackwardKV, D, tk);
    const size_t shq = lds_bytes(kBackwardQ, tq.slots, D), shk = lds_bytes(kBackwardKV, tk.slots, D);
    allow_lds(k_bwd_q_mfma<T, D>, shq);
    allow_lds(k_bwd_kv_mfma<T, D>, shk);
    NA_LAUNCH("na_bwd_q_mfma", (k_bwd_q_mfma<T, D>), dim3(static_cast<unsigned>(grid_blocks(p, tq, p.Hq))),
              dim3(64 * tq.waves), shq, s, p, tq, (const T*)q, lq, (const T*)k, lk, (const T*)v, lv,
              (const T*)o, lo, (const T*)dout, ldo, lse, ll, dlse, ldl, (T*)dq, ldq, delta, lde);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    NA_LAUNCH("na_bwd_kv_mfma", (k_bwd_kv_mfma<T, D>), dim3(static_cast<unsigned>(grid_blocks(p, tk, p.Hkv))),
              dim3(64 * tk.waves), shk, s, p, tk, (const T*)q, lq, (const T*)k, lk, (const T*)v, lv,
              (const T*)dout, ldo, lse, ll, (const float*)delta, lde, (T*)dk, ldk, (T*)dv, ldv);
    return hipGetLastError();
}

}  // namespace

bool mfma_eligible(const Prob& p, int dtype, int D, bool aligned, bool backward) {
    if (dtype == NATTEN_F32 || !aligned || !(p.scale > 0.f)) return false;
    if (p.Dqk != p.Dv || !(D == 32 || D == 64 || D == 128)) return false;
    for (int a = 0; a < 3; ++a)
        if (p.ax[a].st != 1) return false;
    TileShape ts{};
    if (!choose_tile(p, kForward, D, ts)) return false;
    if (backward && (!choose_tile(p, kBackwardQ, D, ts) || !choose_tile(p, kBackwardKV, D, ts))) return false;
    // grid and per-plane offsets stay in 32 bits
    if (grid_blocks(p, ts, p.Hq) >= (1LL << 31)) return false;
    return true;
}

bool mfma_offsets_fit(const Prob& p, std::initializer_list<Lay> lays) { return offsets_fit(p, lays); }

hipError_t mfma_forward(const Prob& p, const void* q, Lay lq, const void* k, Lay lk, const void* v, Lay lv, void* o,
                        Lay lo, float* lse, Lay ll, int dtype, hipStream_t s) {
#define NA_FWD(T, DD) return launch_fwd<T, DD>(p, q, lq, k, lk, v, lv, o, lo, lse, ll, s)
    if (dtype == NATTEN_BF16) {
        if (p.Dqk == 32) NA_FWD(bf16, 32);
        if (p.Dqk == 64) NA_FWD(bf16, 64);
        NA_FWD(bf16, 128);
    }
    if (p.Dqk == 32) NA_FWD(f16, 32);
    if (p.Dqk == 64) NA_FWD(f16, 64);
    NA_FWD(f16, 128);
#undef NA_FWD
}

hipError_t mfma_backward(const Prob& p, const void* q, Lay lq, const void* k, Lay lk, const void* v, Lay lv,
                         const void* o, Lay lo, const void* dout, Lay ldo, const float* lse, Lay ll,
                         const float* dlse, Lay ldl, void* dq, Lay ldq, void* dk, Lay ldk, void* dv, Lay ldv,
                         float* delta, Lay lde, int dtype, hipStream_t s) {
#define NA_BWD(T, DD)                                                                                            \
    return launch_bwd<T, DD>(p, q, lq, k, lk, v, lv, o, lo, dout, ldo, lse, ll, dlse, ldl, dq, ldq, dk, ldk, dv, \
                             ldv, delta, lde, s)
    if (dtype == NATTEN_BF16) {
        if (p.Dqk == 32) NA_BWD(bf16, 32);
        if (p.Dqk == 64) NA_BWD(bf16, 64);
        NA_BWD(bf16, 128);
    }
    if (p.Dqk == 32) NA_BWD(f16, 32);
    if (p.Dqk == 64) NA_BWD(f16, 64);
    NA_BWD(f16, 128);
#undef NA_BWD
}

}  // namespace na

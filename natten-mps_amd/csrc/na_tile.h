// Device helpers of the MFMA tile kernels (na_mfma.hip): MFMA wrappers and lane layouts, LDS staging
// by buffer loads, the score and accumulation products over 32-slot chunks,
// operand layouts, tile geometry, and the kernels' argument structs.  The
// tiling these serve is described at the top of na_mfma.hip.
#pragma once

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <initializer_list>
#include <mutex>
#include <type_traits>
#include <vector>

#include "na_exact.h"
#include "na_launch.h"

namespace na {

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4_t lds_i16x4_t;
typedef __attribute__((address_space(3))) void lds_void_t;

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
// Items (queries or keys) per workgroup: 16 per wave.  The fused kernels
// take up to kMaxFusedItems (8 waves), the split kernels up to kMaxItems.
constexpr int kMaxItems = 64;
constexpr int kMaxFusedItems = 128;
constexpr int kMaxWaves = kMaxFusedItems / 16;
// bytes of LDS before the staged operands (see lds_base)
constexpr int kLdsPad = 16;
// buffer range of a staged plane; out-of-union slots read at kOutOfRange
constexpr int kPlaneBytes = 0x7FFFFFF0;
constexpr uint32_t kOutOfRange = 0x80000000u;

template <typename T>
struct Mma;

template <>
struct Mma<bf16> {
    static constexpr uint32_t kOnes = 0x3F803F80u;  // two bf16 1.0
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
    static constexpr uint32_t kOnes = 0x3C003C00u;  // two fp16 1.0
    __device__ static __forceinline__ f32x4_t run(uint4 a, uint4 b, f32x4_t c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                      __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
    }
    __device__ static __forceinline__ uint32_t pack(float lo, float hi) {
        return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t{lo, hi}), f16x2_t));
    }
};

template <typename T>
__device__ __forceinline__ uint4 pack8(const f32x4_t (&v)[2]) {
    return make_uint4(Mma<T>::pack(v[0][0], v[0][1]), Mma<T>::pack(v[0][2], v[0][3]),
                      Mma<T>::pack(v[1][0], v[1][1]), Mma<T>::pack(v[1][2], v[1][3]));
}

// Reductions over the four 16-lane rows of the wave (lanes i, i+16, i+32,
// i+48): v_permlane16_swap / v_permlane32_swap exchange rows between two
// registers, here both the same value.
// NaN-propagating maximum (v_maximum3_f32 on gfx950, no operand quieting).
__device__ __forceinline__ float fmaxp(float a, float b) { return __builtin_elementwise_maximum(a, b); }

__device__ __forceinline__ float max_rows(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxp(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxp(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

__device__ __forceinline__ float sum_rows(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// delta = dO . O of a query from the dQ kernel's own products: the sum over
// its window of P dP (dP = dO . v), equal to dO . O in exact arithmetic (O is
// the P-weighted sum of v), so the dQ kernels need not read O.  The lane's
// part over one chunk, its 2 x 4 slots in order (the order k_lean_bwd_q
// sums them in); a masked slot has P = 0.
__device__ __forceinline__ float delta_part(const f32x4_t (&s)[2], const f32x4_t (&dp)[2], float sc2, float off,
                                            float part) {
#pragma unroll
    for (int bb = 0; bb < 2; ++bb)
#pragma unroll
        for (int i = 0; i < 4; ++i) part = fmaf(__builtin_amdgcn_exp2f(fmaf(s[bb][i], sc2, off)), dp[bb][i], part);
    return part;
}

// Sum of a lane's accumulators (plus `extra`): not finite exactly when one
// of them is not finite (a sum of finite accumulators of this size cannot
// overflow).
template <int N>
__device__ __forceinline__ float lane_sum(const f32x4_t (&a)[N], float extra) {
    float s = extra;
#pragma unroll
    for (int db = 0; db < N; ++db) s += (a[db][0] + a[db][1]) + (a[db][2] + a[db][3]);
    return s;
}

// True when a lane's part of an item's result is not finite: the lane then
// recomputes its dims exactly (na_exact.h).  A contamination from outside the
// window reaches either every dim of an item (through a probability or score
// gradient) or only the dims that hold a non-finite operand element, so the
// lanes of one item need not agree: each lane's finite dims are exact.
// Tested on the exponent bits, independent of floating-point flags.
__device__ __forceinline__ bool item_nonfinite(float lane_total) {
    return (__float_as_uint(lane_total) & 0x7F800000u) == 0x7F800000u;
}

// x, hidden from value numbering: the recompute after a walk derives the
// lane's position afresh instead of keeping the walk's copy live through it.
__device__ __forceinline__ int opaque(int x) {
    asm volatile("" : "+v"(x));
    return x;
}

__device__ __forceinline__ float max8(const f32x4_t (&s)[2]) {
    const float a = fmaxp(fmaxp(s[0][0], s[0][1]), s[0][2]);
    const float b = fmaxp(fmaxp(s[0][3], s[1][0]), s[1][1]);
    const float c = fmaxp(fmaxp(s[1][2], s[1][3]), a);
    return fmaxp(b, c);
}

// acc + the 8 products of two runs of 8 16-bit elements, in pairs
// (v_dot2_f32_bf16 / v_dot2_f32_f16, fp32 accumulation).  Every tile kernel
// forms delta = dO . O with it in one order (per 8-dim piece, pieces of a
// lane in k-step order, then the four lanes of an item pairwise), so that
// the kernels that compute delta agree bit for bit.
template <typename T>
__device__ __forceinline__ float dot8(uint4 x, uint4 y, float acc) {
    const uint32_t xs[4] = {x.x, x.y, x.z, x.w}, ys[4] = {y.x, y.y, y.z, y.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if constexpr (std::is_same<T, bf16>::value)
            acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, xs[i]), __builtin_bit_cast(bf16x2_t, ys[i]),
                                                  acc, false);
        else
            acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, xs[i]), __builtin_bit_cast(f16x2_t, ys[i]), acc,
                                         false);
    }
    return acc;
}

// XOR swizzle of the 16-byte pieces of LDS row `row` (D / 8 pieces per row):
// the 16 rows one score-operand read touches (rows 8x + y + 4b, x, y < 4)
// land on distinct banks for every head dim.
template <int D>
__host__ __device__ constexpr int swz(int row) {
    if constexpr (D == 32) return (row >> 3) & 3;
    else if constexpr (D == 64) return (((row >> 3) & 3) << 1) | ((row >> 1) & 1);
    else return (((row >> 3) & 3) << 2) | (row & 3);
}

// Staging moves R = 64 / (D/8) rows per wave instruction; the swizzle of row
// iR + l (l < R) splits into disjoint bits of i and of l, so the lane part of
// the LDS/global offsets is fixed for a whole tile.
// Elements per LDS row for head dim D: 96 is stored as 128 (the last four
// 16-byte pieces stay unread), so that rows keep a power-of-two number of
// pieces and every lane layout and swizzle of head dim 128 applies.
template <int D>
__host__ __device__ constexpr int lds_dim() {
    return D == 96 ? 128 : D;
}

template <int D>
constexpr bool swz_splits() {
    constexpr int R = 64 / (D / 8);
    for (int i = 0; i < 256; ++i)
        for (int l = 0; l < R; ++l)
            if (swz<D>(i * R + l) != (swz<D>(i * R) ^ swz<D>(l))) return false;
    return true;
}
static_assert(swz_splits<32>() && swz_splits<64>() && swz_splits<128>(), "swizzle must split");

__device__ __forceinline__ void wait_loads() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

}  // namespace

// Host-chosen tile: power-of-two extents T = 2^tshift (class coordinates) of a
// workgroup's box, tiles per class per axis, waves per workgroup, the staged
// slice layout (slot = a1 * 2^rowshift + a2, `slots` per slice, a multiple of
// 32), len % dil per axis, the run of heads a workgroup works through for
// its box, and divisors for decoding the workgroup index.
struct TileShape {
    int T[3], tshift[3], ntile[3];
    int waves, slots, rowshift;
    int lenmod[3];
    int nheads, h_per;  // heads, and how many of them one workgroup runs
    FastDiv rep, hchunks, spatial, tiles[3], dil[3];
    FastDiv hg, hgroups;  // head chunks per group (fastest), groups (slowest within a batch)
};

// Workgroup x (after the XCD remap) -> batch b, head chunk hc and spatial
// tile s: head chunks vary fastest in groups of hg, then the spatial tile,
// then the group, then the batch.  With hg = hchunks (one group) this is
// heads fastest, then tiles, then batches.
__device__ __forceinline__ void decode_block(const TileShape& ts, int x, int& b, int& hc, int& s) {
    const int q1 = fdiv(x, ts.hg);
    const int hl = x - q1 * static_cast<int>(ts.hg.d);
    const int q2 = fdiv(q1, ts.spatial);
    s = q1 - q2 * static_cast<int>(ts.spatial.d);
    b = fdiv(q2, ts.hgroups);
    hc = (q2 - b * static_cast<int>(ts.hgroups.d)) * static_cast<int>(ts.hg.d) + hl;
}

// Operand layout as the kernels take it: 64-bit batch and head strides, and
// 32-bit strides inside one (batch, head) (the host checks the offsets fit).
struct LayK {
    long long b, h;
    int s0, s1, s2, pad;
};

namespace {

struct Block {
    int b, h0, h1;  // batch and run of heads [h0, h1)
    int r[3], J[3], E[3], lo[3], U[3];
    ClassAxis c[3];
};

// The wave's part of the tile: items f = 16w .. 16w+15 in row-major tile
// order; with power-of-two extents they cover a box, items [il, ih] per axis
// (before clipping to the tile's extent).
__host__ __device__ inline void wave_items(const TileShape& ts, int wave, int (&il)[3], int (&ih)[3]) {
    const int f0 = wave * 16, s2 = ts.tshift[2], s1 = ts.tshift[1];
    if (ts.T[2] >= 16) {
        il[2] = f0 & (ts.T[2] - 1);
        ih[2] = il[2] + 15;
        il[1] = ih[1] = (f0 >> s2) & (ts.T[1] - 1);
        il[0] = ih[0] = f0 >> (s2 + s1);
    } else if (ts.T[2] * ts.T[1] >= 16) {
        il[2] = 0;
        ih[2] = ts.T[2] - 1;
        il[1] = (f0 >> s2) & (ts.T[1] - 1);
        ih[1] = il[1] + (16 >> s2) - 1;
        il[0] = ih[0] = f0 >> (s2 + s1);
    } else {
        il[2] = 0;
        ih[2] = ts.T[2] - 1;
        il[1] = 0;
        ih[1] = ts.T[1] - 1;
        il[0] = f0 >> (s2 + s1);
        ih[0] = il[0] + (16 >> (s2 + s1)) - 1;
    }
}

// The wave's admissible box (union-relative) and the chunks c0..c1 covering it.
struct WaveGeo {
    bool any;
    int lo[3], hi[3];
    int c0, c1;
};

// Host-built per-tile geometry records (kRecDwords ints per spatial tile):
//   [0..2] r   [3..5] J   [6..8] E   [9..11] lo   [12..14] U   [15..17] n
//   [18..20] B   [21] nonempty   then per wave w < kMaxWaves at 24 + 8w:
//   any, lo0, hi0, lo1, hi1, lo2, hi2, c0 | c1 << 16
constexpr int kRecDwords = 128;
static_assert(24 + 8 * kMaxWaves <= kRecDwords, "geometry record too small");

__host__ __device__ inline void spatial_coords(const TileShape& ts, int s, int (&t)[3], int (&r)[3]) {
    for (int a = 2; a >= 0; --a) {
        int q = fdiv(s, ts.tiles[a]);
        t[a] = s - q * static_cast<int>(ts.tiles[a].d);
        s = q;
        q = fdiv(s, ts.dil[a]);
        r[a] = s - q * static_cast<int>(ts.dil[a].d);
        s = q;
    }
}

// Workgroup -> (batch, run of heads, residues, tile origin J, clipped extent
// E) and the union box [lo, lo+U) of the windows of its queries (KEY false)
// or of the queries attending its keys (KEY true), plus the wave's box.  The
// geometry is the same for every (batch, head).  Heads vary fastest, then
// tiles, then batch, so that neighbouring tiles (which share halo rows) run
// close together in time on the same XCD.  With a host-built table (geo) the
// tile's record is read with scalar loads; without one the per-axis work
// runs with one axis per lane (lanes 0, 1, 2) and is read back into scalar
// registers.  False: empty tile.
//
// Variable-length problems (VARLEN, lens = int32 [batch][3] sample extents,
// no table): p and ts describe the padded extents; the sample's own extent
// takes the padded one's place in the geometry (with len % dil to match), so
// tiles past it are empty, and a sample whose extents are out of range
// (below kernel * dilation, above the padded extent, or an even kernel equal
// to a non-causal, undilated extent) has no tiles at all.
template <bool KEY, bool VARLEN = false>
__device__ __forceinline__ bool tile_geometry(const Prob& p, const TileShape& ts, const int* __restrict__ geo,
                                              int wave, Block& k, WaveGeo& g, const int* __restrict__ lens = nullptr) {
    int hc, s;
    decode_block(ts, xcd_block(blockIdx.x, gridDim.x), k.b, hc, s);
    k.h0 = hc * ts.h_per;
    k.h1 = min(k.h0 + ts.h_per, ts.nheads);
    int vlen[3], vmod[3];
    if constexpr (VARLEN) {
        bool ok = true;
#pragma unroll
        for (int a = 0; a < 3; ++a) {
            const Axis& A = p.ax[a];
            const int L = __builtin_amdgcn_readfirstlane(lens[k.b * 3 + a]);
            ok = ok && L >= A.k * A.dil && L <= A.len && !(!A.causal && A.dil == 1 && (A.k % 2) == 0 && A.k == L);
            vlen[a] = L;
            vmod[a] = L - fdiv(L, ts.dil[a]) * A.dil;
        }
        if (!ok) return false;
    }

    if (!VARLEN && geo) {
        const int* rec = geo + s * kRecDwords;
#pragma unroll
        for (int a = 0; a < 3; ++a) {
            k.r[a] = rec[a];
            k.J[a] = rec[3 + a];
            k.E[a] = rec[6 + a];
            k.lo[a] = rec[9 + a];
            k.U[a] = rec[12 + a];
            k.c[a].n = rec[15 + a];
            k.c[a].B = rec[18 + a];
            k.c[a].K = p.ax[a].k;
            k.c[a].h = p.ax[a].k >> 1;
            k.c[a].causal = p.ax[a].causal;
            k.c[a].qs = p.ax[a].st;
        }
        const int* wr = rec + 24 + 8 * wave;
        g.any = wr[0] != 0;
#pragma unroll
        for (int a = 0; a < 3; ++a) {
            g.lo[a] = wr[1 + 2 * a];
            g.hi[a] = wr[2 + 2 * a];
        }
        g.c0 = wr[7] & 0xFFFF;
        g.c1 = wr[7] >> 16;
        return rec[21] != 0;
    }

    int t[3];
    spatial_coords(ts, s, t, k.r);
    int il[3], ih[3];
    wave_items(ts, wave, il, ih);

    // one axis per lane
    const int lane = threadIdx.x & 63;
    const bool l0 = lane == 0, l1 = lane == 1;
#define NA_PICK(field) (l0 ? (field(0)) : l1 ? (field(1)) : (field(2)))
#define F_LEN(a) (VARLEN ? vlen[a] : p.ax[a].len)
#define F_K(a) p.ax[a].k
#define F_DIL(a) p.ax[a].dil
#define F_CAUSAL(a) p.ax[a].causal
#define F_ST(a) p.ax[a].st
#define F_OUT(a) (VARLEN ? vlen[a] : p.ax[a].out)
#define F_LENMOD(a) (VARLEN ? vmod[a] : ts.lenmod[a])
#define F_T(a) ts.T[a]
#define F_DMUL(a) ts.dil[a].mul
#define F_DSH(a) ts.dil[a].shift
#define F_TT(a) t[a]
#define F_RR(a) k.r[a]
#define F_IL(a) il[a]
#define F_IH(a) ih[a]
    const int dil = NA_PICK(F_DIL);
    const FastDiv fd{static_cast<uint32_t>(NA_PICK(F_DMUL)), static_cast<uint32_t>(NA_PICK(F_DSH)),
                     static_cast<uint32_t>(dil)};
    const AxisGeo ag = axis_geometry(NA_PICK(F_LEN), NA_PICK(F_K), dil, NA_PICK(F_CAUSAL), NA_PICK(F_LENMOD),
                                     NA_PICK(F_ST), NA_PICK(F_OUT), NA_PICK(F_T), NA_PICK(F_TT), NA_PICK(F_RR),
                                     NA_PICK(F_IL), NA_PICK(F_IH), KEY, fd);
#undef F_LEN
#undef F_K
#undef F_DIL
#undef F_CAUSAL
#undef F_ST
#undef F_OUT
#undef F_LENMOD
#undef F_T
#undef F_DMUL
#undef F_DSH
#undef F_TT
#undef F_RR
#undef F_IL
#undef F_IH
#undef NA_PICK

    bool nonempty = true;
    g.any = true;
#pragma unroll
    for (int a = 0; a < 3; ++a) {
        k.J[a] = __builtin_amdgcn_readlane(ag.J, a);
        k.E[a] = __builtin_amdgcn_readlane(ag.E, a);
        k.lo[a] = __builtin_amdgcn_readlane(ag.lo, a);
        k.U[a] = __builtin_amdgcn_readlane(ag.U, a);
        k.c[a].n = __builtin_amdgcn_readlane(ag.n, a);
        k.c[a].B = __builtin_amdgcn_readlane(ag.B, a);
        k.c[a].K = p.ax[a].k;
        k.c[a].h = p.ax[a].k >> 1;
        k.c[a].causal = p.ax[a].causal;
        k.c[a].qs = p.ax[a].st;
        g.lo[a] = __builtin_amdgcn_readlane(ag.glo, a);
        g.hi[a] = __builtin_amdgcn_readlane(ag.ghi, a);
        nonempty = nonempty && __builtin_amdgcn_readlane(ag.tile_ok, a) != 0;
        g.any = g.any && __builtin_amdgcn_readlane(ag.wave_ok, a) != 0;
    }
    g.c0 = (g.lo[1] * (1 << ts.rowshift) + g.lo[2]) >> 5;
    g.c1 = (g.hi[1] * (1 << ts.rowshift) + g.hi[2]) >> 5;
    return nonempty;
}

// A key tile whose union is empty on some axis: no query attends its keys
// (they lie past the last window at an even-kernel border, or past the
// last query's window on a strided axis), so every gradient it owns is
// zero.  Query tiles always have a union (every window holds a key).
__device__ __forceinline__ bool empty_union(const Block& k) {
    return k.U[0] == 0 || k.U[1] == 0 || k.U[2] == 0;
}

// One lane's query (or key): validity, position and admissible box
// (union-relative; empty on axis 0 for lanes past the tile).
struct Lane {
    bool valid;
    int pos[3], lo[3], hi[3];
};

__device__ __forceinline__ Lane lane_item(const Prob& p, const TileShape& ts, const Block& k, int wave, int col,
                                          bool key_side) {
    Lane ln;
    const int f = wave * 16 + col, s2 = ts.tshift[2], s1 = ts.tshift[1];
    int e[3];
    e[2] = f & (ts.T[2] - 1);
    e[1] = (f >> s2) & (ts.T[1] - 1);
    e[0] = f >> (s2 + s1);
    ln.valid = e[0] < k.E[0] && e[1] < k.E[1] && e[2] < k.E[2];
    for (int a = 0; a < 3; ++a) {
        const int j = k.J[a] + (ln.valid ? e[a] : 0);
        ln.pos[a] = k.r[a] + j * p.ax[a].dil;
        int lo, hi;
        item_box(k.c[a], j, key_side, lo, hi);
        ln.lo[a] = lo - k.lo[a];
        ln.hi[a] = hi - k.lo[a];
    }
    if (!ln.valid) {
        ln.lo[0] = 1 << 30;
        ln.hi[0] = -1;
    }
    return ln;
}

// Column part of the mask for chunk c as the score MFMA's accumulator input:
// 0 where the lane's slot 32c + 8grp + 4b + i lies in its column range, -inf
// elsewhere.
__device__ __forceinline__ void column_bias(const Lane& ln, int rowshift, int c, int grp, f32x4_t (&bias)[2]) {
    const int col0 = (32 * c + 8 * grp) & ((1 << rowshift) - 1);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const int cc = col0 + e;
        bias[e >> 2][e & 3] = (cc >= ln.lo[2] && cc <= ln.hi[2]) ? 0.f : -INFINITY;
    }
}

__device__ __forceinline__ bool row_ok(const Lane& ln, int rowshift, bool in0, int c, int grp) {
    const int row = (32 * c + 8 * grp) >> rowshift;
    return in0 && row >= ln.lo[1] && row <= ln.hi[1];
}

// Per-(batch, head) base pointer and the 32-bit offset of a position inside
// it (the host checks that every such offset fits in 31 bits).
template <typename T>
__device__ __forceinline__ T* bh_ptr(T* g, const LayK& lay, int b, int h) {
    return g + static_cast<long long>(b) * lay.b + static_cast<long long>(h) * lay.h;
}

__device__ __forceinline__ int vol_off(const LayK& lay, const int (&pos)[3]) {
    return pos[0] * lay.s0 + pos[1] * lay.s1 + pos[2] * lay.s2;
}

__device__ __forceinline__ Strides3 strides3(const LayK& lay) { return Strides3{lay.s0, lay.s1, lay.s2}; }

template <typename T>
__device__ __forceinline__ const T* plane_of(const T* g, const LayK& lay, int b, int h, int p0) {
    return bh_ptr(g, lay, b, h) + p0 * lay.s0;
}

// Staging of union slices into X[slot][D], two operands at a time (same
// slot layout, own strides; one when PAIR is false): each wave instruction moves R = 64 / (D/8)
// rows, lane l the 16-byte piece l % (D/8) of row l / (D/8), holding logical
// piece (l % (D/8)) ^ swz(row).  With slot = iR + l/(D/8), union row and
// column split into an instruction part (scalar) and a lane part fixed per
// tile.  In-plane offsets fit in 31 bits and strides are non-negative
// (checked on the host).
struct StageMap {
    int lrow, lcol;    // lane's row / column inside an instruction's rows
    int lane_a, lane_b;  // lane part of the byte offset, operands a and b
    int kb16;          // lane part of the swizzled piece, times 16
};

template <typename T, int D>
__device__ __forceinline__ StageMap stage_map(const Prob& p, const TileShape& ts, const LayK& la, const LayK& lb,
                                              int lane) {
    constexpr int P = lds_dim<D>() / 8;
    StageMap m;
    const int l = lane / P;
    m.lrow = l >> ts.rowshift;
    m.lcol = l & ((1 << ts.rowshift) - 1);
    const int d1 = p.ax[1].dil, d2 = p.ax[2].dil;
    m.lane_a = (m.lrow * d1 * la.s1 + m.lcol * d2 * la.s2) * static_cast<int>(sizeof(T));
    m.lane_b = (m.lrow * d1 * lb.s1 + m.lcol * d2 * lb.s2) * static_cast<int>(sizeof(T));
    m.kb16 = ((lane % P) ^ swz<lds_dim<D>()>(l)) << 4;
    return m;
}

template <typename T, int D, bool PAIR = true>
__device__ __forceinline__ void stage_pair(const Prob& p, const Block& k, const TileShape& ts, const StageMap& m,
                                           const T* plane_a, const LayK& la, T* Xa, const T* plane_b, const LayK& lb,
                                           T* Xb, int wave) {
    constexpr int LD = lds_dim<D>(), R = 64 / (LD / 8);
    const __amdgpu_buffer_rsrc_t ra =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(plane_a), static_cast<short>(0), kPlaneBytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rb =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(plane_b), static_cast<short>(0), kPlaneBytes, 0x00020000);
    const int d1 = p.ax[1].dil, d2 = p.ax[2].dil;
    const int c1 = k.r[1] + k.lo[1] * d1, c2 = k.r[2] + k.lo[2] * d2;
    const int mask2 = (1 << ts.rowshift) - 1;
    const int n_inst = ts.slots / R;
    constexpr int E = static_cast<int>(sizeof(T));
    for (int i = wave; i < n_inst; i += ts.waves) {
        // instruction part in scalar registers; the lane part was fixed per tile
        const int irow = (i * R) >> ts.rowshift, icol = (i * R) & mask2;
        const int r1 = c1 + irow * d1, r2 = c2 + icol * d2;
        const int sa = __builtin_amdgcn_readfirstlane((r1 * la.s1 + r2 * la.s2) * E);
        const int sb = __builtin_amdgcn_readfirstlane((r1 * lb.s1 + r2 * lb.s2) * E);
        const int kbh = __builtin_amdgcn_readfirstlane(swz<LD>(i * R) << 4);
        const int lim_r = __builtin_amdgcn_readfirstlane(k.U[1] - irow);
        const int lim_c = __builtin_amdgcn_readfirstlane(k.U[2] - icol);
        const int kb = m.kb16 ^ kbh;
        // out-of-union slots: set bit 31, past the buffer range (offsets < 2^31)
        // (head dim 96: the pieces past the row's 12 are padding, not loaded)
        const uint32_t bad = ((m.lrow < lim_r && m.lcol < lim_c && (LD == D || (kb >> 4) < D / 8)) ? 0u
                                                                                                  : kOutOfRange);
        const uint32_t oa = static_cast<uint32_t>(sa + m.lane_a + kb) | bad;
        const uint32_t ob = static_cast<uint32_t>(sb + m.lane_b + kb) | bad;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_void_t*)(Xa + i * R * LD), 16, oa, 0, 0, 0);
        if constexpr (PAIR)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_void_t*)(Xb + i * R * LD), 16, ob, 0, 0, 0);
    }
}

// Score block of chunk c: rows = its 32 slots (A operand, row-major X),
// columns = the wave's 16 items (B fragments); out[b] starts from bias[b].
// The lane receives slots 32c + 8grp + 4b + i (i < 4) in out[b][i].
template <typename T, int D>
__device__ __forceinline__ void score_chunk(const T* X, int c, int col, int grp, const uint4 (&frag)[D / 32],
                                            const f32x4_t (&bias)[2], f32x4_t (&out)[2]) {
#pragma unroll
    for (int b = 0; b < 2; ++b) {
        const int row = 32 * c + 8 * (col >> 2) + 4 * b + (col & 3);
        f32x4_t acc = bias[b];
#pragma unroll
        for (int ks = 0; ks < D / 32; ++ks) {
            const int kb = (ks * 4 + grp) ^ swz<lds_dim<D>()>(row);
            const uint4 a = *reinterpret_cast<const uint4*>(X + row * lds_dim<D>() + kb * 8);
            acc = Mma<T>::run(a, frag[ks], acc);
        }
        out[b] = acc;
    }
}

// acc[db] (16 head dims x 16 items) += X^T[db*16 .. +15][32 slots of chunk c]
// * packed.  The A operand (row = head dim, k = 8 consecutive slots) comes
// from row-major X through two transposing reads: in 16-lane row g, lane j
// points at X[32c + 8g + j/4 (+4)][db*16 + 4(j%4) ..] and lane i receives
// X[32c + 8g + m (+4)][db*16 + i], m < 4.
template <typename T, int D>
__device__ __forceinline__ void accumulate_chunk(const T* X, int c, int lane, uint4 packed, f32x4_t (&acc)[D / 16]) {
    const int g = lane >> 4, j = lane & 15;
    const int r0 = 32 * c + 8 * g + (j >> 2), r1 = r0 + 4;
    const int sub = (j & 1) * 4;
#pragma unroll
    for (int db = 0; db < D / 16; ++db) {
        const int kb = 2 * db + ((j & 3) >> 1);
        constexpr int LD = lds_dim<D>();
        const T* a0 = X + r0 * LD + ((kb ^ swz<LD>(r0)) * 8) + sub;
        const T* a1 = X + r1 * LD + ((kb ^ swz<LD>(r1)) * 8) + sub;
        const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)a0);
        const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)a1);
        const uint2 l2 = __builtin_bit_cast(uint2, lo), h2 = __builtin_bit_cast(uint2, hi);
        acc[db] = Mma<T>::run(make_uint4(l2.x, l2.y, h2.x, h2.y), packed, acc[db]);
    }
}

template <typename T, int D>
__device__ __forceinline__ void load_frags(const T* __restrict__ g, long long off, bool valid, int grp,
                                           uint4 (&f)[D / 32]) {
#pragma unroll
    for (int ks = 0; ks < D / 32; ++ks)
        f[ks] = valid ? *reinterpret_cast<const uint4*>(g + off + ks * 32 + grp * 8) : make_uint4(0, 0, 0, 0);
}

// Global keys, 32 at a time: rows j0 .. j0+31 of the keys and values of one
// (batch, kv head) into the 32 slots of Xk / Xv, laid out and swizzled as a
// staged union (slot = row - j0); rows past n load as zeros.  Each wave
// instruction moves 512 / D rows; the workgroup's waves share them.
template <typename T, int D>
__device__ __forceinline__ void stage_global(const T* kb, int ks, const T* vb, int vs, int j0, int n, T* Xk, T* Xv,
                                             int wave, int waves, int lane) {
    constexpr int LD = lds_dim<D>(), P = LD / 8, R = 64 / P;
    constexpr int E = static_cast<int>(sizeof(T));
    const __amdgpu_buffer_rsrc_t rk =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(kb), static_cast<short>(0), kPlaneBytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rv =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(vb), static_cast<short>(0), kPlaneBytes, 0x00020000);
    const int l = lane / P;
    for (int i = wave; i < 32 / R; i += waves) {
        const int slot = i * R + l, j = j0 + slot;
        const int piece16 = ((lane % P) ^ swz<LD>(slot)) << 4;
        const bool ok = j < n && (piece16 >> 4) < D / 8;
        const uint32_t ok_k = ok ? static_cast<uint32_t>(j * ks * E + piece16) : kOutOfRange;
        const uint32_t ok_v = ok ? static_cast<uint32_t>(j * vs * E + piece16) : kOutOfRange;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (lds_void_t*)(Xk + i * R * LD), 16, ok_k, 0, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (lds_void_t*)(Xv + i * R * LD), 16, ok_v, 0, 0, 0);
    }
}

// Score-MFMA accumulator input for a block of 32 global keys starting at j0:
// 0 for the lane's slots (8 grp + e) that hold a key, -inf past n.
__device__ __forceinline__ void global_bias(int j0, int n, int grp, f32x4_t (&bias)[2]) {
    const int lim = n - j0 - 8 * grp;
#pragma unroll
    for (int e = 0; e < 8; ++e) bias[e >> 2][e & 3] = e < lim ? 0.f : -INFINITY;
}

// Store the lane's 4 consecutive head dims per 16-dim block (scaled).
template <typename T, int D>
__device__ __forceinline__ void store_rows(T* __restrict__ g, long long off, int grp, const f32x4_t (&acc)[D / 16],
                                           float mul) {
#pragma unroll
    for (int db = 0; db < D / 16; ++db) {
        if constexpr (sizeof(T) == 4) {
            *reinterpret_cast<float4*>(g + off + db * 16 + grp * 4) =
                make_float4(acc[db][0] * mul, acc[db][1] * mul, acc[db][2] * mul, acc[db][3] * mul);
        } else {
            const uint2 w = make_uint2(Mma<T>::pack(acc[db][0] * mul, acc[db][1] * mul),
                                       Mma<T>::pack(acc[db][2] * mul, acc[db][3] * mul));
            *reinterpret_cast<uint2*>(g + off + db * 16 + grp * 4) = w;
        }
    }
}

// The staged operands start at LDS address kLdsPad, reached through a
// constant address instead of the dynamic `extern __shared__` symbol: the
// compiler then folds the base into each ds_read's offset field (through the
// symbol it re-adds the base with one VALU per LDS address and chunk).  Not
// address 0: a constant 0 becomes a null pointer, and the generic null
// pointer is not LDS.  Every launch allocates kLdsPad more bytes.
__device__ __forceinline__ unsigned char* lds_base() {
    return (unsigned char*)((__attribute__((address_space(3))) unsigned char*)(kLdsPad));
}

__device__ __forceinline__ int kv_head(const TileShape& ts, int h) { return ts.rep.d == 1 ? h : fdiv(h, ts.rep); }

// Operand layout groups a kernel instance assumes (chosen by the host).
// kLayOne: every 16-bit operand has q's layout and every fp32 row operand
// lse's.  kLayTwo: the query-side 16-bit operands (q, out, dO, dq) share q's
// layout, the key-side ones (k, v, dk, dv) k's, the fp32 rows lse's (GQA).
// kLayFour: q its own; k and v one; out, dO and dq one; dk and dv one (q,
// k and v as views of one packed tensor, the gradients and out contiguous,
// as the nn modules call).  kLayGeneral: each operand its own.  Fewer
// distinct layouts keep fewer registers live, which at head dim 32 removes
// the SGPR spills and at head dim 64 the VGPR spills of the dQ kernel.
constexpr int kLayGeneral = 0, kLayOne = 1, kLayTwo = 2, kLayFour = 3;
// v read at k's layout; out (and what shares it) at its own layout.
template <int LAY>
constexpr bool kVAtK = LAY == kLayTwo || LAY == kLayFour;
template <int LAY>
constexpr bool kOwnOut = LAY == kLayGeneral || LAY == kLayFour;

// Waves per SIMD an instance is built for (4: at most 128 VGPRs, 5: at most
// 96; 1: no constraint).  Saying so lets the register allocator trade VGPRs
// for SGPRs instead of spilling SGPRs.  The choices are the measured best on
// MI355X: at head dim 32 the forward without the per-chunk column pattern
// fits 5 waves; the backward kernels at 96 VGPRs serialise their
// transposing LDS reads (the dK/dV kernel also spills), and at 4 waves they
// run 2 % (dQ) and 7 % (dK/dV) faster; at head dim 64 the forward and the
// wide dK/dV kernel fit 4, and the dQ kernel, whose tiles mostly leave room
// for 2 to 4 workgroups per CU, runs 3-10 % faster with the registers of 2.
// WIDE instances handle unions whose rows exceed 32 slots, where the column
// mask changes from chunk to chunk; keeping them apart leaves the common
// instance its smaller register need.
enum KernelId { kKernFwd, kKernBwdQ, kKernBwdKV };

constexpr int waves_per_simd(KernelId k, int D, bool wide) {
    if (D == 32) return wide || k != kKernFwd ? 4 : 5;
    if (D == 64) return k == kKernBwdQ ? 2 : k == kKernFwd || wide ? 4 : 1;
    return 1;
}

#define NA_OCCUPANCY(K, D, WIDE) __attribute__((amdgpu_waves_per_eu(waves_per_simd(K, D, WIDE))))

// Chunks per online-softmax group in the forward (one max reduction and one
// rescale per group); two keep head dim 32 within 96 VGPRs.
template <int D>
constexpr int fwd_group() {
    return D == 32 ? 2 : 4;
}

// Walk of a workgroup over its (batch, head) pairs and axis-0 slices.  The
// loads of the next slice are issued as soon as the current one is no longer
// read, and the very first right after decoding the tile, so that the
// per-lane setup runs while they are in flight.
struct Walk {
    int h, u0, b;
};

__device__ __forceinline__ void walk_start(const Block& k, Walk& w) {
    w.h = k.h0;
    w.u0 = 0;
    w.b = k.b;
}

// Advance to the next slice; false past the last one.  `new_pair` reports a
// change of head.
__device__ __forceinline__ bool walk_next(const Block& k, Walk& w, bool& new_pair) {
    new_pair = false;
    if (++w.u0 < k.U[0]) return true;
    w.u0 = 0;
    if (++w.h >= k.h1) return false;
    new_pair = true;
    return true;
}

// True when the next (q head) h1 of the walk reads the staged K/V of h0
// unchanged: one slice per head and the same kv head (GQA group).
__device__ __forceinline__ bool same_rows(const TileShape& ts, const Block& k, int h0, int h1) {
    return k.U[0] == 1 && kv_head(ts, h0) == kv_head(ts, h1);
}

__device__ __forceinline__ int slice_pos(const Prob& p, const Block& k, int u0) {
    return k.r[0] + (k.lo[0] + u0) * p.ax[0].dil;
}

// Kernel arguments, one struct per kernel: the kernel receives it by value
// (its only explicit argument, so it sits at offset 0 of the kernel-argument
// segment), and the exact recomputation after a walk reads it again from
// there through the segment pointer -- so the walk holds none of the
// pointers and layouts only the recomputation needs.
// Global keys: extra tokens every query attends besides its neighbourhood
// (the reference's additional_keys / additional_values), rows [B, n, Hkv,
// D] with element strides; query head h reads kv head h / rep.  n == 0:
// none.  Offsets inside one (batch, kv head) fit in 31 bits (host check).
template <typename T>
struct GlobalKeys {
    const T *k, *v;
    long long kb, kh, vb, vh;  // batch / head strides
    int ks, vs;                // token strides
    int n;
};

template <typename T>
struct FwdArgs {
    Prob p;
    TileShape ts;
    const int* geo;
    const T *q, *k, *v;
    T* out;
    float* lse;
    LayK lq, lk, lv, lo, ll;
    GlobalKeys<T> gk;
    const int* lens;  // variable-length instances: int32 [batch][3] sample extents
};

template <typename T>
struct BwdQArgs {
    Prob p;
    TileShape ts;
    const int* geo;
    const T *q, *k, *v, *o, *dout;
    const float *lse, *dlse;
    T* dq;
    float* delta;
    LayK lq, lk, lv, lo, ldo, ll, ldl, ldq, lde;
    GlobalKeys<T> gk;
    const int* lens;
};

template <typename T>
struct BwdKvArgs {
    Prob p;
    TileShape ts;
    const int* geo;
    const T *q, *k, *v, *dout;
    const float *lse, *delta;
    T *dk, *dv;
    LayK lq, lk, lv, ldo, ll, lde, ldk, ldv;
    const int* lens;
};

// Split products: weights w (rows of KV entries), staged operand x, out.
template <typename T>
struct WsumArgs {
    Prob p;
    TileShape ts;
    const int* geo;
    const T *w, *x;
    T* out;
    LayK lw, lx, lo;
    float mul;
};

// Variable-length problems, for the exact recomputation: the problem and
// tile shape with sample b's own extents (lens[b * 3 + a]) in place of the
// padded ones (and len % dil to match), b from the XCD-remapped workgroup
// index x.  False when the sample's extents are out of range (the rule of
// tile_geometry).  The walks themselves keep the padded problem and take the
// sample's extents in tile_geometry only.
__device__ __forceinline__ bool varlen_view(const Prob& p0, const TileShape& ts0, const int* __restrict__ lens, int x,
                                            Prob& p, TileShape& ts) {
    int b, hc, s;
    decode_block(ts0, x, b, hc, s);
    p = p0;
    ts = ts0;
    bool ok = true;
#pragma unroll
    for (int a = 0; a < 3; ++a) {
        const Axis& A = p0.ax[a];
        const int L = __builtin_amdgcn_readfirstlane(lens[b * 3 + a]);
        ok = ok && L >= A.k * A.dil && L <= A.len && !(!A.causal && A.dil == 1 && (A.k % 2) == 0 && A.k == L);
        p.ax[a].len = p.ax[a].out = L;
        ts.lenmod[a] = L - fdiv(L, ts0.dil[a]) * A.dil;
    }
    return ok;
}

// The lane's item from the (XCD-remapped) workgroup index x alone (the
// decode of tile_geometry without the unions): batch, the workgroup's run of
// heads [h0, h1) and the position (a query item's output index on a strided
// axis); false for lanes past the tile.
template <bool KEY>
__device__ __forceinline__ bool lane_position(const Prob& p, const TileShape& ts, int x, int wave, int col, int& b,
                                              int& h0, int& h1, int (&pos)[3]) {
    int hc, s;
    decode_block(ts, x, b, hc, s);
    h0 = hc * ts.h_per;
    h1 = min(h0 + ts.h_per, ts.nheads);
    int t[3], r[3];
    spatial_coords(ts, s, t, r);
    const int f = wave * 16 + col, s2 = ts.tshift[2], s1 = ts.tshift[1];
    const int e[3] = {f >> (s2 + s1), (f >> s2) & (ts.T[1] - 1), f & (ts.T[2] - 1)};
    bool ok = true;
#pragma unroll
    for (int a = 0; a < 3; ++a) {
        const int n = !KEY && p.ax[a].st != 1 ? p.ax[a].out : fdiv(p.ax[a].len - r[a] + p.ax[a].dil - 1, ts.dil[a]);
        const int j = t[a] * ts.T[a] + e[a];
        ok = ok && j < n;
        pos[a] = r[a] + j * p.ax[a].dil;
    }
    return ok;
}

// The kernel's argument segment as a generic pointer, hidden from value
// numbering, so that what the recomputation reads through it are fresh
// scalar loads rather than values the walk would have to keep live.  Valid
// in kernel code only (the recomputation is inlined into its kernel).
__device__ __forceinline__ const void* kernargs() {
    auto ka = __builtin_amdgcn_kernarg_segment_ptr();
    asm volatile("" : "+s"(ka));
    return (const void*)ka;  // address-space conversion to a generic pointer
}


// ---------------------------------------------------------------------------
// Host helpers shared by the launchers.
// ---------------------------------------------------------------------------

// Static-LDS audit: lds_base() places the staged operands at the constant
// LDS address kLdsPad, which is sound only while no kernel instance declares
// static __shared__ memory (that would sit at address 0 and overlap them).
// Every instance is asked once per process; one with static LDS turns the
// whole tile path off (the vector kernels take every call) with a message.
struct LdsAudit {
    int checked = 0, bad = 0;
};

template <typename K>
void audit_one(K kernel, const char* what, LdsAudit& a) {
    hipFuncAttributes attr{};
    if (hipFuncGetAttributes(&attr, reinterpret_cast<const void*>(kernel)) != hipSuccess) {
        (void)hipGetLastError();
        ++a.bad;
        std::fprintf(stderr, "natten_hip: cannot read the attributes of %s; MFMA tile kernels disabled\n", what);
        return;
    }
    ++a.checked;
    if (attr.sharedSizeBytes != 0) {
        ++a.bad;
        std::fprintf(stderr,
                     "natten_hip: %s has %zu bytes of static LDS, which would overlap the operands staged at LDS "
                     "address %d; MFMA tile kernels disabled\n",
                     what, static_cast<size_t>(attr.sharedSizeBytes), kLdsPad);
    }
}

int n_class_h(const Axis& A, int r) { return (A.len - r + A.dil - 1) / A.dil; }

int pow2_at_least(int x) {
    int p = 1;
    while (p < x) p <<= 1;
    return p;
}

int log2_of(int x) {
    int l = 0;
    while ((1 << l) < x) ++l;
    return l;
}

// Largest union extent on one axis over every class and tile (the same
// spans axis_geometry computes for each tile).
int union_extent(const Axis& A, int T, bool key_tile) {
    int best = 1;
    for (int r = 0; r < A.dil; ++r) {
        const ClassAxis c = class_axis(A, r);
        const int items = key_tile ? c.n : query_items(A, c.n);
        for (int J = 0; J < items; J += T) {
            const int jend = (J + T < items ? J + T : items) - 1;
            int lo, hi, x;
            if (!key_tile) {
                lo = query_ws(c, J);
                lo = lo > 0 ? lo : 0;
                hi = query_ws(c, jend) + c.K - 1;
                hi = hi < c.n - 1 ? hi : c.n - 1;
            } else {
                query_span(c, J, lo, x);
                query_span(c, jend, x, hi);
            }
            if (hi - lo + 1 > best) best = hi - lo + 1;
        }
    }
    return best;
}

// Largest union extent on one axis over every extent from K * dil up to
// A.len (the samples of a variable-length problem; the same spans
// axis_geometry computes for each tile).  A tile's union depends on the
// extent only through the windows it meets at the axis ends, so per extent
// the tiles within 2K + 2T of either end are evaluated, plus one interior
// tile; the result is cached per (axis, tile extent, side).
int union_extent_upto(const Axis& A, int T, bool key_tile) {
    struct Entry {
        int len, k, dil, causal, T, key, u;
    };
    static std::mutex mu;
    static std::vector<Entry> cache;
    {
        std::lock_guard<std::mutex> g(mu);
        for (const Entry& e : cache)
            if (e.len == A.len && e.k == A.k && e.dil == A.dil && e.causal == A.causal && e.T == T &&
                e.key == (key_tile ? 1 : 0))
                return e.u;
    }
    int best = 1;
    const int reach = 2 * A.k + 2 * T;
    for (int L = A.k * A.dil; L <= A.len; ++L) {
        Axis B = A;
        B.len = B.out = L;
        for (int r = 0; r < B.dil && r < L; ++r) {
            const ClassAxis c = class_axis(B, r);
            const auto span = [&](int J) {
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
            };
            const int ntiles = (c.n + T - 1) / T;
            for (int t = 0; t < ntiles; ++t) {
                const int J = t * T;
                if (J < reach || J + T > c.n - reach || t == ntiles / 2) span(J);
            }
        }
    }
    std::lock_guard<std::mutex> g(mu);
    cache.push_back(Entry{A.len, A.k, A.dil, A.causal, T, key_tile ? 1 : 0, best});
    return best;
}

// Workgroups of `kernel` (block threads, shm bytes of LDS) resident on the
// current device at once; cached per (kernel, block, shm, device).
template <typename K>
long long resident_blocks(K kernel, int block, size_t shm) {
    struct Entry {
        const void* f;
        int block;
        size_t shm;
        int dev;
        long long n;
    };
    static std::mutex mu;
    static std::vector<Entry> cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) dev = 0;
    const void* f = reinterpret_cast<const void*>(kernel);
    std::lock_guard<std::mutex> g(mu);
    for (const Entry& e : cache)
        if (e.f == f && e.block == block && e.shm == shm && e.dev == dev) return e.n;
    int per_cu = 0, cus = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, block, shm) != hipSuccess || per_cu < 1)
        per_cu = 1;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1) cus = 1;
    cache.push_back(Entry{f, block, shm, dev, static_cast<long long>(per_cu) * cus});
    return cache.back().n;
}

// Every operand: non-negative strides and every offset inside one (batch,
// head) (plus a row of 128 head dims) in 31 bits; staged operands' in-plane
// byte offsets (axes 1 and 2) inside the buffer range of a plane.
bool offsets_fit(const Prob& p, std::initializer_list<Lay> lays) {
    for (const Lay& l : lays) {
        if (l.b < 0 || l.s0 < 0 || l.s1 < 0 || l.s2 < 0 || l.h < 0) return false;
        const long long plane = (static_cast<long long>(p.ax[1].len) - 1) * l.s1 +
                                (static_cast<long long>(p.ax[2].len) - 1) * l.s2 + 128;
        const long long vol = (static_cast<long long>(p.ax[0].len) - 1) * l.s0 + plane;
        if (plane * 2 >= kPlaneBytes || vol >= (1LL << 31)) return false;
    }
    return true;
}

LayK to_k(const Lay& l) { return LayK{l.b, l.h, static_cast<int>(l.s0), static_cast<int>(l.s1), static_cast<int>(l.s2), 0}; }

template <typename K>
hipError_t allow_lds(K kernel, size_t bytes) {
    if (bytes <= 64 * 1024) return hipSuccess;
    return hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                               static_cast<int>(bytes));
}

bool same_lay(const Lay& a, const Lay& b) {
    return a.b == b.b && a.h == b.h && a.s0 == b.s0 && a.s1 == b.s1 && a.s2 == b.s2;
}

bool all_same(std::initializer_list<Lay> g) {
    for (const Lay& l : g)
        if (!same_lay(l, *g.begin())) return false;
    return true;
}

// Layout group for a launch from its query-side and key-side 16-bit operands
// and its fp32 row operands (first of each list is the one the kernel reads).
int layout_group(std::initializer_list<Lay> qside, std::initializer_list<Lay> kvside,
                 std::initializer_list<Lay> rows) {
    if (!all_same(rows)) return kLayGeneral;
    if (all_same(qside) && all_same(kvside)) return same_lay(*qside.begin(), *kvside.begin()) ? kLayOne : kLayTwo;
    // kLayFour: qside = q, then out, dO, dq sharing one layout; kvside = k, v,
    // then dk, dv, each pair sharing one
    if (kvside.size() % 2 != 0) return kLayGeneral;
    for (const Lay* l = kvside.begin(); l != kvside.end(); l += 2)
        if (!same_lay(l[0], l[1])) return kLayGeneral;
    for (const Lay* l = qside.begin() + 1; l != qside.end(); ++l)
        if (!same_lay(*l, qside.begin()[1])) return kLayGeneral;
    return kLayFour;
}

}  // namespace

}  // namespace na

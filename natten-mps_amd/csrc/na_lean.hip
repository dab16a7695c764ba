// Lean tile kernels (gfx950, bf16 / fp16 / fp32, head dim 32 or 64, stride
// 1): forward, backward dQ and backward dK/dV for 2-D problems, for 1-D
// problems (ONE_D: a tile is 64 consecutive items of a residue class, 16 per
// wave, its window union staged 16 slots to a row and masked per 32-slot
// chunk), and for fp32 3-D problems (D3: the 2-D tile at one depth walks
// its window's depth planes).  Every operand is read or written at its own
// strides (k and v, and dk and dv, share one), and the key side walks the
// q heads of its kv head's group (GQA).
//
// They serve the common case of the MFMA tile path with a fixed tile and
// fixed lane layouts, so that a wave spends its instructions on the products
// and the softmax instead of on general tile geometry:
//
// * A workgroup owns an 8 x 8 box of queries (keys) of one class pair (r1,
//   r2) and one (batch, head); wave w owns box rows 2w and 2w+1, lane column
//   n = lane % 16 the item (2w + n/8, n%8).  In class coordinates a window is
//   an undilated K1 x K2 run; window starts are non-decreasing along an axis
//   and grow by at most one per item, so the union of the box's windows (of
//   the queries attending the box's keys) spans at most 7 + K rows and a
//   wave's own two rows at most K1 + 1 of them.
// * LDS holds the union row-major with 16 slots per union row (K2 <= 9 keeps
//   a row's windows inside 16 columns), two union rows per 32-slot chunk;
//   rows and columns past the union are staged from outside the buffer's
//   range and read as zeros.  16-byte pieces are XOR-swizzled by slot as in
//   the general tile kernels (swz, na_tile.h).
// * Everything a tile needs beyond the problem is one host-built record of
//   16 dwords (positions of the box and the union, extents, and every item's
//   window start per axis relative to the union), read with one scalar load.
// * The forward computes all of a wave's score blocks first (K1 + 1 union
//   rows at most), takes one maximum per query and exponentiates once: no
//   online rescaling.
//
// MFMA layouts are those of na_mfma.hip (16x16x32): in a chunk the lane
// (n, g = lane / 16) holds the 8 consecutive slots 8g .. 8g+7 of item n
// (union row 2c + g/2, columns 8(g%2) ..), the B operand of the product that
// contracts over slots; that product reads its A operand transposed out of
// LDS with ds_read_b64_tr_b16.
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <vector>

#include "na_tile.h"

namespace na {

namespace {

constexpr int kLeanRec = 16;                 // dwords per tile record
constexpr uint32_t kLeanOOR = 0x40000000u;   // offset past every staged plane's range (planes < 2^30 bytes)
constexpr int kLeanWaves = 4;

// Staged rows of a query tile reading NCH chunks per wave: a wave's first
// row is at most 6 (2-D: union rows of its window) or 3 (1-D: 16 items per
// wave, windows start at most one slot apart per item).
template <bool ONE_D>
__host__ __device__ constexpr int lean_rows(int nch) {
    return 2 * nch + (ONE_D ? 4 : 6);
}

// Element types: bf16 / fp16 (v_mfma_f32_16x16x32, the products' operands
// 8 elements per lane) and fp32 (v_mfma_f32_16x16x4_f32, one element per
// lane and k-step).  A staged row of D elements is as wide as kRowD 16-bit
// elements: staging and the XOR swizzle act on its 16-byte pieces as for a
// 16-bit row of that width.  A lane's fragment of a row (the B operand of
// the products over head dims) is kNF 16-byte pieces: 16-bit, dims 32 j +
// 8 g .. + 7 of piece j for lane group g; fp32, dims (D / 4) g + 4 j .. + 3,
// so that k-step ks of the fp32 product takes dim (D / 4) g + ks.
template <typename T>
constexpr bool kF32 = sizeof(T) == 4;
template <typename T, int D>
constexpr int kRowD = D * static_cast<int>(sizeof(T)) / 2;
template <typename T, int D>
constexpr int kNF = D * static_cast<int>(sizeof(T)) / 64;
// Offset variants of the transposed reads (fp32: per low slot bits that the
// swizzle takes, see lean_tr_off).
template <typename T, int D>
constexpr int kTV = !kF32<T> ? 2 : (D == 32 ? 2 : 4);
constexpr int kLeanEsz2 = 2;

// Byte offset of fragment piece j of lane group g inside a row.
template <typename T, int D>
__device__ __forceinline__ int lean_frag_off(int j, int g) {
    return kF32<T> ? g * D + j * 16 : j * 64 + g * 16;
}

typedef unsigned int v2u32_t __attribute__((ext_vector_type(2)));
typedef unsigned int v4u32_t __attribute__((ext_vector_type(4)));

// Layout of one operand group: batch and head strides, and the element
// strides of the spatial axes (axis 0 of a 2-D problem has extent 1).
struct LeanLay {
    long long b, h;
    int s1, s2, s0;
};

// Workgroup decode of the tile kernels.  2-D: heads fastest, then the tile,
// then the batch.  3-D: the heads of a group of hg fastest, then the
// in-plane tile, then the depth position, then the head group, then the
// batch -- the tiles of neighbouring depths, which stage the same planes,
// run close together on one XCD while the planes of only hg heads are live.
struct LeanTask {
    int b, h, t, z;
};

struct LeanDecode {
    FastDiv heads, tiles;       // 2-D
    FastDiv hg, zlen, hgroups;  // 3-D: heads per group, depth extent, groups
};

template <bool D3>
__device__ __forceinline__ LeanTask lean_task(const LeanDecode& d, int x) {
    LeanTask k;
    if constexpr (!D3) {
        const int bt = fdiv(x, d.heads);
        k.h = x - bt * static_cast<int>(d.heads.d);
        k.b = fdiv(bt, d.tiles);
        k.t = bt - k.b * static_cast<int>(d.tiles.d);
        k.z = 0;
    } else {
        const int x1 = fdiv(x, d.hg);
        const int hl = x - x1 * static_cast<int>(d.hg.d);
        const int x2 = fdiv(x1, d.tiles);
        k.t = x1 - x2 * static_cast<int>(d.tiles.d);
        const int x3 = fdiv(x2, d.zlen);
        k.z = x2 - x3 * static_cast<int>(d.zlen.d);
        k.b = fdiv(x3, d.hgroups);
        k.h = (x3 - k.b * static_cast<int>(d.hgroups.d)) * static_cast<int>(d.hg.d) + hl;
    }
    return k;
}

// Depth planes of a 3-D tile: planes z0 + j d for j in [j0, n).  Query
// tiles: the key planes of the window of depth z (a causal window's planes
// below 0 skipped); key tiles: the query planes whose windows hold z.
struct LeanDepth {
    int z0, d, j0, n;
};

__device__ __forceinline__ LeanDepth lean_depth_q(const Axis& A, int z) {
    LeanDepth w{axis_first(A, z), A.dil, 0, A.k};
    while (w.z0 + w.j0 * w.d < 0) ++w.j0;
    return w;
}

__device__ __forceinline__ LeanDepth lean_depth_k(const Axis& A, int z) {
    int lo, hi;
    if (!axis_query_range(A, z, lo, hi)) return LeanDepth{z, A.dil, 0, 0};
    return LeanDepth{z, A.dil, lo, hi + 1};
}

template <typename T>
struct LeanFwdArgs {
    const int* rec;
    const T *q, *k, *v;
    T* out;
    float* lse;
    LeanLay lq, lk, ll, lo;       // q; k and v; lse; out
    LeanDecode dec;               // workgroup decode
    FastDiv rep;                  // kv head = h / rep
    int d1, d2, K1, K2;
    uint32_t qbytes, kbytes, obytes;  // byte range of one (batch, head) plane of q / k / out
    float sc2;                    // scale * log2(e)
    Prob p;                       // for the exact recomputation
};

// Signed byte i (0..7) of the pair (lo, hi).
__device__ __forceinline__ int sbyte(int lo, int hi, int i) {
    const int w = i < 4 ? lo : hi;
    return (w << (24 - 8 * (i & 3))) >> 24;
}

// Logical 16-byte piece that lands at physical piece `pp` of slot `slot`.
template <int D>
__device__ __forceinline__ int lean_piece(int pp, int slot) {
    return pp ^ swz<D>(slot);
}

// Staging of union rows [0, nst) of two operands sharing one layout into
// Xa / Xb (16 slots per row): rows at or past U1 and columns at or past U2
// load from outside the range (zeros).  Rows are dealt to the waves in turn.
template <typename T, int D, int NW = kLeanWaves>
__device__ __forceinline__ void lean_stage(__amdgpu_buffer_rsrc_t ra, __amdgpu_buffer_rsrc_t rb, T* Xa, T* Xb,
                                           int base, int step1, int step2, int U1, int U2, int nst, int wave,
                                           int lane) {
    constexpr int R = kRowD<T, D>;
    constexpr int P = R / 8, SPI = 64 / P, HALVES = 16 / SPI;
    static_assert(NW % 2 == 0, "a wave's rows must keep one parity");
    // lane part of the offset per half row; a wave's rows i = wave + 4j all
    // have the parity of `wave`, which fixes the swizzle's row bit
    uint32_t off[HALVES];
    const int pp = lane % P;
#pragma unroll
    for (int hf = 0; hf < HALVES; ++hf) {
        const int c = hf * SPI + lane / P;
        const int slot = (wave & 1) * 16 + c;
        off[hf] = c < U2 ? static_cast<uint32_t>(c * step2 + lean_piece<R>(pp, slot) * 16) : kLeanOOR;
    }
#pragma unroll 1
    for (int i = wave; i < nst; i += NW) {
        const uint32_t ro = i < U1 ? static_cast<uint32_t>(base + i * step1) : kLeanOOR;
#pragma unroll
        for (int hf = 0; hf < HALVES; ++hf) {
            const uint32_t o = off[hf] + ro;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_void_t*)(Xa + (i * 16 + hf * SPI) * D), 16, o, 0, 0,
                                                     0);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_void_t*)(Xb + (i * 16 + hf * SPI) * D), 16, o, 0, 0,
                                                     0);
        }
    }
}

// Staging of one operand's union rows [0, nst) (as lean_stage, one operand).
template <typename T, int D>
__device__ __forceinline__ void lean_stage1(__amdgpu_buffer_rsrc_t ra, T* Xa, int base, int step1, int step2, int U1,
                                            int U2, int nst, int wave, int lane) {
    constexpr int R = kRowD<T, D>;
    constexpr int P = R / 8, SPI = 64 / P, HALVES = 16 / SPI;
    uint32_t off[HALVES];
    const int pp = lane % P;
#pragma unroll
    for (int hf = 0; hf < HALVES; ++hf) {
        const int c = hf * SPI + lane / P;
        const int slot = (wave & 1) * 16 + c;
        off[hf] = c < U2 ? static_cast<uint32_t>(c * step2 + lean_piece<R>(pp, slot) * 16) : kLeanOOR;
    }
#pragma unroll 1
    for (int i = wave; i < nst; i += kLeanWaves) {
        const uint32_t ro = i < U1 ? static_cast<uint32_t>(base + i * step1) : kLeanOOR;
#pragma unroll
        for (int hf = 0; hf < HALVES; ++hf) {
            const uint32_t o = off[hf] + ro;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_void_t*)(Xa + (i * 16 + hf * SPI) * D), 16, o, 0, 0,
                                                     0);
        }
    }
}

template <typename T>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t lean_rsrc(const T* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(p), static_cast<short>(0), static_cast<int>(bytes),
                                             0x00020000);
}

// LDS byte offsets (from the operand's base) of the lane's score A operand
// for blocks b = 0, 1 of chunk 0 of a wave whose rows start at union row
// `first`, k-step ks: slot 8(n/4) + 4b + n%4, logical piece 4ks + g.
template <typename T, int D>
__device__ __forceinline__ int lean_score_off(int first, int col, int grp, int b, int ks) {
    constexpr int R = kRowD<T, D>;
    const int slot = first * 16 + 8 * (col >> 2) + 4 * b + (col & 3);
    const int piece = kF32<T> ? (D / 16) * grp + ks : ks * 4 + grp;
    return slot * R * 2 + (piece ^ swz<R>(slot)) * 16;
}

// LDS byte offset of the lane's transposing read (rows r0 or r1 = r0 + 4 of
// chunk 0, 16-dim block db): see accumulate_chunk in na_tile.h.
// fp32: the A operand of k-step kk (0..7) for lane (m, g) is element
// d = 16 db + m of slot 8 g + kk of the chunk; variant v carries the slot
// bits below 8 that the swizzle reads ((kk >> 1) & 1 at D = 32, kk & 3 at
// D = 64), and the read adds kk rows.
template <typename T, int D>
__device__ __forceinline__ int lean_tr_off(int first, int lane, int hi, int db) {
    const int g = lane >> 4, j = lane & 15;
    if constexpr (kF32<T>) {
        constexpr int R = kRowD<T, D>;
        const int s0 = first * 16 + 8 * g;
        const int rep = s0 + (D == 32 ? 2 * hi : hi);
        return s0 * R * 2 + (((4 * db + (j >> 2)) ^ swz<R>(rep)) * 16) + (j & 3) * 4;
    }
    const int r = first * 16 + 8 * g + (j >> 2) + 4 * hi;
    const int kb = 2 * db + ((j & 3) >> 1);
    return r * D * 2 + (kb ^ swz<D>(r)) * 16 + (j & 1) * 8;
}

template <typename T, int D>
__device__ __forceinline__ f32x4_t lean_score(const unsigned char* X, const int (&aoff)[2][kNF<T, D>], int c, int b,
                                              const uint4 (&frag)[kNF<T, D>], f32x4_t acc) {
    if constexpr (kF32<T>) {
        constexpr int R = kRowD<T, D>;
#pragma unroll
        for (int j = 0; j < kNF<T, D>; ++j) {
            const uint4 a = *reinterpret_cast<const uint4*>(X + aoff[b][j] + c * 32 * R * 2);
            const uint32_t av[4] = {a.x, a.y, a.z, a.w};
            const uint32_t bv[4] = {frag[j].x, frag[j].y, frag[j].z, frag[j].w};
#pragma unroll
            for (int e = 0; e < 4; ++e)
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(av[e]), __uint_as_float(bv[e]), acc, 0, 0,
                                                            0);
        }
        return acc;
    } else {
#pragma unroll
        for (int ks = 0; ks < D / 32; ++ks) {
            const uint4 a = *reinterpret_cast<const uint4*>(X + aoff[b][ks] + c * 32 * D * 2);
            acc = Mma<T>::run(a, frag[ks], acc);
        }
        return acc;
    }
}

// acc[db] += X^T[db block][chunk c slots] * packed (B operand: 8 slots of the lane's item).
template <typename T, int D>
__device__ __forceinline__ void lean_accumulate(const unsigned char* X, const int (&toff)[2][D / 16], int c,
                                                uint4 packed, f32x4_t (&acc)[D / 16]) {
#pragma unroll
    for (int db = 0; db < D / 16; ++db) {
        const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(X + toff[0][db] + c * 32 * D * 2));
        const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(X + toff[1][db] + c * 32 * D * 2));
        const uint2 l2 = __builtin_bit_cast(uint2, lo), h2 = __builtin_bit_cast(uint2, hi);
        acc[db] = Mma<T>::run(make_uint4(l2.x, l2.y, h2.x, h2.y), packed, acc[db]);
    }
}

// acc[db] += X^T[db block][chunk c slots] * p, p the lane's 8 slot values
// (16-bit: rounded to T and packed as the B operand; fp32: k-step kk takes
// slot 8 g + kk, value p[kk / 4][kk % 4]).
template <typename T, int D>
__device__ __forceinline__ void lean_acc(const unsigned char* X, const int (&toff)[kTV<T, D>][D / 16], int c,
                                         const f32x4_t (&p)[2], f32x4_t (&acc)[D / 16]) {
    if constexpr (kF32<T>) {
        constexpr int R = kRowD<T, D>;
#pragma unroll
        for (int db = 0; db < D / 16; ++db)
#pragma unroll
            for (int kk = 0; kk < 8; ++kk) {
                const int v = D == 32 ? ((kk >> 1) & 1) : (kk & 3);
                const float a = *reinterpret_cast<const float*>(X + toff[v][db] + (c * 32 + kk) * R * 2);
                acc[db] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, p[kk >> 2][kk & 3], acc[db], 0, 0, 0);
            }
    } else {
        lean_accumulate<T, D>(X, toff, c, pack8<T>(p), acc);
    }
}

// acc + the products of two fragment pieces (16-bit: dot8, 8 elements in
// pairs; fp32: 4 elements in order).
template <typename T>
__device__ __forceinline__ float lean_dot(uint4 x, uint4 y, float acc) {
    if constexpr (kF32<T>) {
        acc = fmaf(__uint_as_float(x.x), __uint_as_float(y.x), acc);
        acc = fmaf(__uint_as_float(x.y), __uint_as_float(y.y), acc);
        acc = fmaf(__uint_as_float(x.z), __uint_as_float(y.z), acc);
        return fmaf(__uint_as_float(x.w), __uint_as_float(y.w), acc);
    } else {
        return dot8<T>(x, y, acc);
    }
}

// Store of the lane's 4 consecutive dims of 16-dim block db (times mul) into
// the row at byte offset `row`.
template <typename T>
__device__ __forceinline__ void lean_store4(__amdgpu_buffer_rsrc_t rs, int row, int db, int grp, f32x4_t v, float mul) {
    if constexpr (kF32<T>) {
        const uint4 w = make_uint4(__float_as_uint(v[0] * mul), __float_as_uint(v[1] * mul), __float_as_uint(v[2] * mul),
                                   __float_as_uint(v[3] * mul));
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4u32_t, w), rs, row + db * 64 + grp * 16, 0, 0);
    } else {
        const uint2 w = make_uint2(Mma<T>::pack(v[0] * mul, v[1] * mul), Mma<T>::pack(v[2] * mul, v[3] * mul));
        __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(v2u32_t, w), rs, row + db * 32 + grp * 8, 0, 0);
    }
}

// Column mask of the lane as the score MFMA's accumulator input: slot
// columns 8(g%2) + 4b + i inside [clo, clo + K2) -> 0, else -inf.
__device__ __forceinline__ void lean_colbias(int clo, int K2, int grp, f32x4_t (&bias)[2]) {
    const int c0 = 8 * (grp & 1) - clo;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const unsigned cc = static_cast<unsigned>(c0 + e);
        bias[e >> 2][e & 3] = cc < static_cast<unsigned>(K2) ? 0.f : -INFINITY;
    }
}

// 1-D tiles (64 consecutive class items per tile, 16 per wave, the union's
// slots 16 to a staged row): the class rule of the tile's residue class from
// its record (class size r[6], border start r[7]) and the axis.
__device__ __forceinline__ ClassAxis lean_class1d(const int* r, const Axis& A) {
    ClassAxis c;
    c.n = r[6];
    c.K = A.k;
    c.h = A.k / 2;
    c.B = r[7];
    c.causal = A.causal;
    c.qs = 1;
    return c;
}

// Mask of chunk c for a lane whose valid slots (counted from the wave's
// first staged row) are [lo, lo + w), as the score MFMA's accumulator input:
// the lane's slots 32c + 8g + 4b + i -> 0 inside, -inf outside.
__device__ __forceinline__ void lean_chunkbias(int c, int lo, int w, int grp, f32x4_t (&bias)[2]) {
    const int t0 = 32 * c + 8 * grp - lo;
#pragma unroll
    for (int e = 0; e < 8; ++e)
        bias[e >> 2][e & 3] = static_cast<unsigned>(t0 + e) < static_cast<unsigned>(w) ? 0.f : -INFINITY;
}

template <typename T, int D>
__device__ __forceinline__ void lean_redo_fwd(const void* kargs, int z, int pos1, int pos2, int b, int h, int hk,
                                              int grp) {
    const LeanFwdArgs<T>& A = *static_cast<const LeanFwdArgs<T>*>(kargs);
    ExactAxis x[3];
    x[0] = exact_axis(A.p.ax[0], z);
    x[1] = exact_axis(A.p.ax[1], pos1);
    x[2] = exact_axis(A.p.ax[2], pos2);
    const T* qp = A.q + b * A.lq.b + h * A.lq.h;
    const T* kp = A.k + b * A.lk.b + hk * A.lk.h;
    const T* vp = A.v + b * A.lk.b + hk * A.lk.h;
    const Strides3 ks{A.lk.s0, A.lk.s1, A.lk.s2};
    const int qo = z * A.lq.s0 + pos1 * A.lq.s1 + pos2 * A.lq.s2;
    f32x4_t acc[D / 16];
    float lse_v;
    exact_forward<T, D>(A.p.scale, x, qp + qo, kp, ks, vp, ks, grp, acc, lse_v);
    store_rows<T, D>(A.out + b * A.lo.b + h * A.lo.h, z * A.lo.s0 + pos1 * A.lo.s1 + pos2 * A.lo.s2, grp, acc, 1.f);
    if (grp == 0) A.lse[b * A.ll.b + h * A.ll.h + z * A.ll.s0 + pos1 * A.ll.s1 + pos2 * A.ll.s2] = lse_v;
}

// ---------------------------------------------------------------------------
// Forward.  NCH chunks (2 NCH >= K1 + 1 union rows) per wave.  3-D (D3):
// the tile walks its window's key planes, staging each plane's union in
// turn, with one online-softmax rescale per plane; 2-D: one plane, one
// maximum, no rescale.
// ---------------------------------------------------------------------------
// HP q heads per workgroup (HP = 2: two q heads of one kv head's group,
// waves 0-3 and 4-7, share the staged K/V rows).
template <typename T, int D, int NCH, bool D3 = false, bool ONE_D = false, int HP = 1>
__global__ __launch_bounds__(64 * kLeanWaves * HP) void k_lean_fwd(LeanFwdArgs<T> a) {
    constexpr int NR = lean_rows<ONE_D>(NCH), NF = kNF<T, D>, TV = kTV<T, D>, ES = sizeof(T);
    static_assert(!(D3 && HP > 1), "one head per workgroup for depth walks");
    unsigned char* smem = lds_base();
    T* Ks = reinterpret_cast<T*>(smem);
    T* Vs = Ks + NR * 16 * D;
    const int lane = threadIdx.x & 63, col = lane & 15, grp = lane >> 4;
    const int wave_wg = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wave = wave_wg & (kLeanWaves - 1);  // the wave's place in its head's tile
    const LeanTask tk = lean_task<D3>(a.dec, xcd_block(blockIdx.x, gridDim.x));
    const int b = tk.b, h = tk.h * HP + (wave_wg / kLeanWaves), t = tk.t, z = tk.z;
    const int hk = a.rep.d == 1 ? h : fdiv(h, a.rep);
    const int* r = a.rec + t * kLeanRec;
    const int pr0 = r[0], pc0 = r[1], ur0 = r[2], uc0 = r[3], ext = r[4], nst = r[5];
    const int U1 = ext & 0xFF, U2 = (ext >> 8) & 0xFF, E1 = (ext >> 16) & 0xFF, E2 = (ext >> 24) & 0xFF;
    LeanDepth dw{0, 0, 0, 1};
    if constexpr (D3) dw = lean_depth_q(a.p.ax[0], z);

    // stage the union's K and V rows (of the first key plane; 1-D: union
    // slots 16 to a row)
    const long long kvo = b * a.lk.b + hk * a.lk.h;
    const int ks2 = a.lk.s2 * a.d2 * ES;
    const int kst = ONE_D ? ur0 * a.lk.s2 * ES : (ur0 * a.lk.s1 + uc0 * a.lk.s2) * ES;
    const int ks1 = ONE_D ? 16 * ks2 : a.lk.s1 * a.d1 * ES;
    const auto stage = [&](int j) {
        const long long o = kvo + static_cast<long long>(dw.z0 + j * dw.d) * a.lk.s0;
        lean_stage<T, D, kLeanWaves * HP>(lean_rsrc(a.k + o, a.kbytes), lean_rsrc(a.v + o, a.kbytes), Ks, Vs, kst,
                                          ks1, ks2, U1, U2, nst, wave_wg, lane);
    };
    stage(dw.j0);

    // the lane's query and its window, relative to the wave's first staged
    // union row (2-D: window rows [rlo, rlo + K1) and columns [clo, clo +
    // K2); 1-D: window slots [rlo, rlo + K))
    bool valid;
    int pos1, pos2, first, rlo, clo = 0;
    if constexpr (ONE_D) {
        const ClassAxis c = lean_class1d(r, a.p.ax[2]);
        const int item = 16 * wave + col, E = (ext >> 16) & 0xFF;
        valid = item < E;
        pos1 = 0;
        pos2 = pr0 + item * a.d2;
        const int ow = class_ws(c, pc0 + 16 * wave) - uc0;
        first = __builtin_amdgcn_readfirstlane(ow > 0 ? ow >> 4 : 0);
        rlo = valid ? class_ws(c, pc0 + item) - uc0 - 16 * first : 1 << 20;
    } else {
        const int qr = 2 * wave + (col >> 3), qc = col & 7;
        valid = qr < E1 && qc < E2;
        pos1 = pr0 + qr * a.d1;
        pos2 = pc0 + qc * a.d2;
        const int w0 = sbyte(r[6], r[7], 2 * wave), w1 = sbyte(r[6], r[7], 2 * wave + 1);
        first = __builtin_amdgcn_readfirstlane(w0 > 0 ? w0 : 0);
        rlo = valid ? ((col >> 3) ? w1 : w0) - first : 1 << 20;
        clo = sbyte(r[8], r[9], qc);
    }
    const int qoff = pos1 * a.lq.s1 + pos2 * a.lq.s2;
    const long long qbo = b * a.lq.b + h * a.lq.h + static_cast<long long>(z) * a.lq.s0;
    uint4 qf[NF];
    {
        const __amdgpu_buffer_rsrc_t rq = lean_rsrc(a.q + qbo, a.qbytes);
#pragma unroll
        for (int ks = 0; ks < NF; ++ks) {
            const uint32_t o = valid ? static_cast<uint32_t>(qoff * ES + lean_frag_off<T, D>(ks, grp)) : kLeanOOR;
            qf[ks] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rq, o, 0, 0));
        }
    }
    f32x4_t cb[2];
    if constexpr (!ONE_D) lean_colbias(clo, a.K2, grp, cb);
    int aoff[2][NF], toff[TV][D / 16];
#pragma unroll
    for (int bb = 0; bb < 2; ++bb)
#pragma unroll
        for (int ks = 0; ks < NF; ++ks) aoff[bb][ks] = lean_score_off<T, D>(first, col, grp, bb, ks);
#pragma unroll
    for (int hi = 0; hi < TV; ++hi)
#pragma unroll
        for (int db = 0; db < D / 16; ++db) toff[hi][db] = lean_tr_off<T, D>(first, lane, hi, db);

    const unsigned char* Kb = reinterpret_cast<const unsigned char*>(Ks);
    const unsigned char* Vb = reinterpret_cast<const unsigned char*>(Vs);
    f32x4_t acc[D / 16], lacc = f32x4_t{0.f, 0.f, 0.f, 0.f};
    float lpart = 0.f, m = -INFINITY;
#pragma unroll
    for (int db = 0; db < D / 16; ++db) acc[db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll 1
    for (int j = dw.j0; j < dw.n; ++j) {
        wait_loads();
        __syncthreads();
        f32x4_t s[NCH][2];
        bool rv[NCH];
        float mx = -INFINITY;
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            if constexpr (ONE_D) {
                lean_chunkbias(c, rlo, a.K2, grp, cb);
                rv[c] = true;
            } else {
                const int row = 2 * c + (grp >> 1) - rlo;
                rv[c] = static_cast<unsigned>(row) < static_cast<unsigned>(a.K1);
            }
            s[c][0] = lean_score<T, D>(Kb, aoff, c, 0, qf, cb[0]);
            s[c][1] = lean_score<T, D>(Kb, aoff, c, 1, qf, cb[1]);
            mx = fmaxp(mx, rv[c] ? max8(s[c]) : -INFINITY);
        }
        float mref;
        if constexpr (D3) {
            // online softmax over the planes: one rescale per plane
            const float mnew = fmaxp(m, max_rows(mx) * a.sc2);
            mref = mnew == -INFINITY ? 0.f : mnew;
            const float corr = __builtin_amdgcn_exp2f(m - mref);
            m = mnew;
            lacc *= corr;
            lpart *= corr;
#pragma unroll
            for (int db = 0; db < D / 16; ++db) acc[db] *= corr;
        } else {
            m = max_rows(mx) * a.sc2;
            mref = m == -INFINITY ? 0.f : m;
        }
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            const float off = rv[c] ? -mref : -INFINITY;
#pragma unroll
            for (int bb = 0; bb < 2; ++bb)
#pragma unroll
                for (int i = 0; i < 4; ++i) s[c][bb][i] = __builtin_amdgcn_exp2f(fmaf(s[c][bb][i], a.sc2, off));
            if constexpr (kF32<T>) {
                // row sums of the probabilities themselves, in slot order
#pragma unroll
                for (int bb = 0; bb < 2; ++bb)
#pragma unroll
                    for (int i = 0; i < 4; ++i) lpart += s[c][bb][i];
                lean_acc<T, D>(Vb, toff, c, s[c], acc);
            } else {
                // row sums from one more MFMA against ones: the same rounded P as the product
                const uint4 pk = pack8<T>(s[c]);
                lean_accumulate<T, D>(Vb, toff, c, pk, acc);
                const uint4 ones = make_uint4(Mma<T>::kOnes, Mma<T>::kOnes, Mma<T>::kOnes, Mma<T>::kOnes);
                lacc = Mma<T>::run(ones, pk, lacc);
            }
        }
        if constexpr (D3) {
            if (j + 1 < dw.n) {
                __syncthreads();  // the plane is no longer read
                stage(j + 1);
            }
        }
    }
    const float lsum = kF32<T> ? sum_rows(lpart) : lacc[0];
    const bool redo = valid && item_nonfinite(lane_sum(acc, lsum));
    if (valid) {
        const float inv = 1.f / lsum;
        const __amdgpu_buffer_rsrc_t ro =
            lean_rsrc(a.out + (b * a.lo.b + h * a.lo.h + static_cast<long long>(z) * a.lo.s0), a.obytes);
        const int ooff = pos1 * a.lo.s1 + pos2 * a.lo.s2;
#pragma unroll
        for (int db = 0; db < D / 16; ++db) lean_store4<T>(ro, ooff * ES, db, grp, acc[db], inv);
        if (grp == 0)
            a.lse[b * a.ll.b + h * a.ll.h + static_cast<long long>(z) * a.ll.s0 + pos1 * a.ll.s1 + pos2 * a.ll.s2] =
                (m + __log2f(lsum)) * kLn2;
    }
    if (redo) lean_redo_fwd<T, D>(kernargs(), opaque(z), opaque(pos1), opaque(pos2), b, h, hk, grp);
}


template <typename T>
struct LeanBwdArgs {
    const int *rec, *rec_k;       // query-tile and key-tile records
    const T *q, *k, *v, *o, *dout;
    const float *lse, *dlse;
    T *dq, *dk, *dv;
    float* delta;
    LeanLay lq, lk, ll;           // q; k and v; lse, dlse and delta
    LeanLay lo, ldo, ldq, ldk;    // out; dout; dq; dk and dv
    LeanDecode dec;               // task decode
    FastDiv rep;
    int nr;                       // LDS rows of a key tile
    int d1, d2, K1, K2;
    uint32_t qbytes, kbytes, obytes, dobytes, dqbytes, dkbytes;  // plane byte ranges
    float sc2, scale;
    Prob p;
};

template <typename T, int D>
__device__ __forceinline__ void lean_redo_bwd_q(const void* kargs, int z, int pos1, int pos2, int b, int h, int hk,
                                                int grp) {
    const LeanBwdArgs<T>& A = *static_cast<const LeanBwdArgs<T>*>(kargs);
    ExactAxis x[3];
    x[0] = exact_axis(A.p.ax[0], z);
    x[1] = exact_axis(A.p.ax[1], pos1);
    x[2] = exact_axis(A.p.ax[2], pos2);
    const long long qb = b * A.lq.b + h * A.lq.h, kb = b * A.lk.b + hk * A.lk.h;
    const long long lb = b * A.ll.b + h * A.ll.h + z * A.ll.s0 + pos1 * A.ll.s1 + pos2 * A.ll.s2;
    const Strides3 ks{A.lk.s0, A.lk.s1, A.lk.s2};
    const int qo = z * A.lq.s0 + pos1 * A.lq.s1 + pos2 * A.lq.s2;
    const T* do_row = A.dout + (b * A.ldo.b + h * A.ldo.h + z * A.ldo.s0 + pos1 * A.ldo.s1 + pos2 * A.ldo.s2);
    float di = exact_dot<T, D>(do_row,
                               A.o + (b * A.lo.b + h * A.lo.h + z * A.lo.s0 + pos1 * A.lo.s1 + pos2 * A.lo.s2));
    if (A.dlse) di -= A.dlse[lb];
    f32x4_t acc[D / 16];
    exact_backward_q<T, D>(A.p.scale, x, A.q + qb + qo, do_row, A.lse[lb], di, A.k + kb, ks, A.v + kb, ks, grp, acc);
    store_rows<T, D>(A.dq + (b * A.ldq.b + h * A.ldq.h), z * A.ldq.s0 + pos1 * A.ldq.s1 + pos2 * A.ldq.s2, grp, acc,
                     A.p.scale);
}

template <typename T, int D>
__device__ __forceinline__ void lean_redo_bwd_kv(const void* kargs, int z, int pos1, int pos2, int b, int hk,
                                                 int grp) {
    const LeanBwdArgs<T>& A = *static_cast<const LeanBwdArgs<T>*>(kargs);
    ExactAxis x[3];
    x[0] = exact_axis(A.p.ax[0], z);
    x[1] = exact_axis(A.p.ax[1], pos1);
    x[2] = exact_axis(A.p.ax[2], pos2);
    const long long kb = b * A.lk.b + hk * A.lk.h, gb = b * A.ldk.b + hk * A.ldk.h;
    const int ko = z * A.lk.s0 + pos1 * A.lk.s1 + pos2 * A.lk.s2, go = z * A.ldk.s0 + pos1 * A.ldk.s1 + pos2 * A.ldk.s2;
    const Strides3 qs{A.lq.s0, A.lq.s1, A.lq.s2}, gs{A.ldo.s0, A.ldo.s1, A.ldo.s2}, ls{A.ll.s0, A.ll.s1, A.ll.s2};
    f32x4_t g[D / 16];
    const int rep = A.p.rep;
    exact_zero(g);
#pragma unroll 1
    for (int h = hk * rep; h < (hk + 1) * rep; ++h) {
        const long long qb = b * A.lq.b + h * A.lq.h, lb = b * A.ll.b + h * A.ll.h;
        const long long db = b * A.ldo.b + h * A.ldo.h;
        exact_backward_kv<T, D, true>(A.p.scale, x, A.k + kb + ko, A.v + kb + ko, A.q + qb, qs, A.dout + db, gs,
                                      A.lse + lb, ls, A.delta + lb, ls, grp, g);
    }
    store_rows<T, D>(A.dv + gb, go, grp, g, 1.f);
    exact_zero(g);
#pragma unroll 1
    for (int h = hk * rep; h < (hk + 1) * rep; ++h) {
        const long long qb = b * A.lq.b + h * A.lq.h, lb = b * A.ll.b + h * A.ll.h;
        const long long db = b * A.ldo.b + h * A.ldo.h;
        exact_backward_kv<T, D, false>(A.p.scale, x, A.k + kb + ko, A.v + kb + ko, A.q + qb, qs, A.dout + db, gs,
                                       A.lse + lb, ls, A.delta + lb, ls, grp, g);
    }
    store_rows<T, D>(A.dk + gb, go, grp, g, A.p.scale);
}

// ---------------------------------------------------------------------------
// Backward, query side: delta = dO . O - dlse (written for the key side),
// dq = scale * sum P (dP - delta) k with P = exp(scale q.k - lse).  delta
// comes from the kernel's own products, sum over the window of P dP (equal
// to dO . O), in a first pass that keeps every chunk's P and dP; O is read
// only where that sum is not finite.
// ---------------------------------------------------------------------------
// Query tile of task x (lean_task).  3-D (D3): delta = dO . O from the rows
// (the products of one plane do not hold the window's sum), the dP products
// start from -delta, and the tile walks its window's key planes.
template <typename T, int D, int NCH, bool D3 = false, bool ONE_D = false, int HP = 1>
__device__ __forceinline__ void lean_bwd_q_tile(const LeanBwdArgs<T>& a, int x) {
    constexpr int NR = lean_rows<ONE_D>(NCH), NF = kNF<T, D>, TV = kTV<T, D>, ES = sizeof(T);
    static_assert(!(D3 && HP > 1), "one head per workgroup for depth walks");
    unsigned char* smem = lds_base();
    T* Ks = reinterpret_cast<T*>(smem);
    T* Vs = Ks + NR * 16 * D;
    const int lane = threadIdx.x & 63, col = lane & 15, grp = lane >> 4;
    const int wave_wg = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wave = wave_wg & (kLeanWaves - 1);  // the wave's place in its head's tile
    const LeanTask tk = lean_task<D3>(a.dec, x);
    const int b = tk.b, h = tk.h * HP + (wave_wg / kLeanWaves), t = tk.t, z = tk.z;
    const int hk = a.rep.d == 1 ? h : fdiv(h, a.rep);
    const int* r = a.rec + t * kLeanRec;
    const int pr0 = r[0], pc0 = r[1], ur0 = r[2], uc0 = r[3], ext = r[4], nst = r[5];
    const int U1 = ext & 0xFF, U2 = (ext >> 8) & 0xFF, E1 = (ext >> 16) & 0xFF, E2 = (ext >> 24) & 0xFF;
    LeanDepth dw{0, 0, 0, 1};
    if constexpr (D3) dw = lean_depth_q(a.p.ax[0], z);
    const long long kvo = b * a.lk.b + hk * a.lk.h;
    const int ks2 = a.lk.s2 * a.d2 * ES;
    const int kst = ONE_D ? ur0 * a.lk.s2 * ES : (ur0 * a.lk.s1 + uc0 * a.lk.s2) * ES;
    const int ks1 = ONE_D ? 16 * ks2 : a.lk.s1 * a.d1 * ES;
    const auto stage = [&](int j) {
        const long long o = kvo + static_cast<long long>(dw.z0 + j * dw.d) * a.lk.s0;
        lean_stage<T, D, kLeanWaves * HP>(lean_rsrc(a.k + o, a.kbytes), lean_rsrc(a.v + o, a.kbytes), Ks, Vs, kst,
                                          ks1, ks2, U1, U2, nst, wave_wg, lane);
    };
    stage(dw.j0);
    // the lane's query and its window (as in k_lean_fwd)
    bool valid;
    int pos1, pos2, first, rlo, clo = 0;
    if constexpr (ONE_D) {
        const ClassAxis c = lean_class1d(r, a.p.ax[2]);
        const int item = 16 * wave + col, E = (ext >> 16) & 0xFF;
        valid = item < E;
        pos1 = 0;
        pos2 = pr0 + item * a.d2;
        const int ow = class_ws(c, pc0 + 16 * wave) - uc0;
        first = __builtin_amdgcn_readfirstlane(ow > 0 ? ow >> 4 : 0);
        rlo = valid ? class_ws(c, pc0 + item) - uc0 - 16 * first : 1 << 20;
    } else {
        const int qr = 2 * wave + (col >> 3), qc = col & 7;
        valid = qr < E1 && qc < E2;
        pos1 = pr0 + qr * a.d1;
        pos2 = pc0 + qc * a.d2;
        const int w0 = sbyte(r[6], r[7], 2 * wave), w1 = sbyte(r[6], r[7], 2 * wave + 1);
        first = __builtin_amdgcn_readfirstlane(w0 > 0 ? w0 : 0);
        rlo = valid ? ((col >> 3) ? w1 : w0) - first : 1 << 20;
        clo = sbyte(r[8], r[9], qc);
    }
    const long long zl = z;
    const int qoff = pos1 * a.lq.s1 + pos2 * a.lq.s2;
    const long long qbo = b * a.lq.b + h * a.lq.h + zl * a.lq.s0;
    const long long lo = b * a.ll.b + h * a.ll.h + zl * a.ll.s0 + pos1 * a.ll.s1 + pos2 * a.ll.s2;
    const int goff = pos1 * a.ldo.s1 + pos2 * a.ldo.s2;
    const long long gbo = b * a.ldo.b + h * a.ldo.h + zl * a.ldo.s0;
    const int ooff = pos1 * a.lo.s1 + pos2 * a.lo.s2;
    const long long obo = b * a.lo.b + h * a.lo.h + zl * a.lo.s0;
    uint4 qf[NF], gf[NF], of[NF];
    {
        const __amdgpu_buffer_rsrc_t rq = lean_rsrc(a.q + qbo, a.qbytes);
        const __amdgpu_buffer_rsrc_t rg = lean_rsrc(a.dout + gbo, a.dobytes);
#pragma unroll
        for (int ks = 0; ks < NF; ++ks) {
            const uint32_t o = valid ? static_cast<uint32_t>(qoff * ES + lean_frag_off<T, D>(ks, grp)) : kLeanOOR;
            const uint32_t og = valid ? static_cast<uint32_t>(goff * ES + lean_frag_off<T, D>(ks, grp)) : kLeanOOR;
            qf[ks] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rq, o, 0, 0));
            gf[ks] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rg, og, 0, 0));
        }
        if constexpr (D3) {
            const __amdgpu_buffer_rsrc_t ro = lean_rsrc(a.o + obo, a.obytes);
#pragma unroll
            for (int ks = 0; ks < NF; ++ks) {
                const uint32_t o = valid ? static_cast<uint32_t>(ooff * ES + lean_frag_off<T, D>(ks, grp)) : kLeanOOR;
                of[ks] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(ro, o, 0, 0));
            }
        }
    }
    const float L2 = valid ? a.lse[lo] * kLog2e : 0.f;
    const float dl = (valid && a.dlse) ? a.dlse[lo] : 0.f;
    f32x4_t cb[2];
    if constexpr (!ONE_D) lean_colbias(clo, a.K2, grp, cb);
    // chunk c's mask (1-D) and row offset of the exponent (2-D: -inf where
    // the row test fails)
    const auto chunk_mask = [&](int c, float& off) {
        if constexpr (ONE_D) {
            lean_chunkbias(c, rlo, a.K2, grp, cb);
            off = -L2;
        } else {
            const int row = 2 * c + (grp >> 1) - rlo;
            off = static_cast<unsigned>(row) < static_cast<unsigned>(a.K1) ? -L2 : -INFINITY;
        }
    };
    int aoff[2][NF], toff[TV][D / 16];
#pragma unroll
    for (int bb = 0; bb < 2; ++bb)
#pragma unroll
        for (int ks = 0; ks < NF; ++ks) aoff[bb][ks] = lean_score_off<T, D>(first, col, grp, bb, ks);
#pragma unroll
    for (int hi = 0; hi < TV; ++hi)
#pragma unroll
        for (int db = 0; db < D / 16; ++db) toff[hi][db] = lean_tr_off<T, D>(first, lane, hi, db);

    const unsigned char* Kb = reinterpret_cast<const unsigned char*>(Ks);
    const unsigned char* Vb = reinterpret_cast<const unsigned char*>(Vs);
    f32x4_t acc[D / 16];
#pragma unroll
    for (int db = 0; db < D / 16; ++db) acc[db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    if constexpr (D3) {
        // delta from this lane's head dims, summed over the 4 lane rows
        float di = 0.f;
#pragma unroll
        for (int ks = 0; ks < NF; ++ks) di = lean_dot<T>(gf[ks], of[ks], di);
        di = sum_rows(di) - dl;
        if (valid && grp == 0) a.delta[lo] = di;
        const f32x4_t nd[2] = {f32x4_t{-di, -di, -di, -di}, f32x4_t{-di, -di, -di, -di}};
#pragma unroll 1
        for (int j = dw.j0; j < dw.n; ++j) {
            wait_loads();
            __syncthreads();
#pragma unroll
            for (int c = 0; c < NCH; ++c) {
                float off;
                chunk_mask(c, off);
                f32x4_t ds[2];
#pragma unroll
                for (int bb = 0; bb < 2; ++bb) {
                    const f32x4_t sc = lean_score<T, D>(Kb, aoff, c, bb, qf, cb[bb]);
                    const f32x4_t dp = lean_score<T, D>(Vb, aoff, c, bb, gf, nd[bb]);
#pragma unroll
                    for (int i = 0; i < 4; ++i) ds[bb][i] = __builtin_amdgcn_exp2f(fmaf(sc[i], a.sc2, off)) * dp[i];
                }
                lean_acc<T, D>(Kb, toff, c, ds, acc);
            }
            if (j + 1 < dw.n) {
                __syncthreads();  // the plane is no longer read
                stage(j + 1);
            }
        }
    } else {
        wait_loads();
        __syncthreads();
        // P and dP (= dO . v) of every chunk first, and delta = sum over the
        // window of P dP (= dO . O) from them; where that is not finite (a
        // non-finite operand outside the window reaching the sum through a
        // masked slot), dO . O from the rows
        f32x4_t pr[NCH][2], dpr[NCH][2];
        float di;
        {
            const f32x4_t zero = f32x4_t{0.f, 0.f, 0.f, 0.f};
            float part = 0.f;
#pragma unroll
            for (int c = 0; c < NCH; ++c) {
                float off;
                chunk_mask(c, off);
#pragma unroll
                for (int bb = 0; bb < 2; ++bb) {
                    const f32x4_t sc = lean_score<T, D>(Kb, aoff, c, bb, qf, cb[bb]);
                    dpr[c][bb] = lean_score<T, D>(Vb, aoff, c, bb, gf, zero);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        pr[c][bb][i] = __builtin_amdgcn_exp2f(fmaf(sc[i], a.sc2, off));
                        part = fmaf(pr[c][bb][i], dpr[c][bb][i], part);
                    }
                }
            }
            di = sum_rows(part) - dl;
            if (valid && !(__builtin_fabsf(di) <= __FLT_MAX__))
                di = exact_dot<T, D>(a.dout + gbo + goff, a.o + obo + ooff) - dl;
        }
        if (valid && grp == 0) a.delta[lo] = di;
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            f32x4_t ds[2];
#pragma unroll
            for (int bb = 0; bb < 2; ++bb)
#pragma unroll
                for (int i = 0; i < 4; ++i) ds[bb][i] = pr[c][bb][i] * (dpr[c][bb][i] - di);
            lean_acc<T, D>(Kb, toff, c, ds, acc);
        }
    }
    const bool redo = valid && item_nonfinite(lane_sum(acc, 0.f));
    if (valid) {
        const __amdgpu_buffer_rsrc_t rd = lean_rsrc(a.dq + (b * a.ldq.b + h * a.ldq.h + zl * a.ldq.s0), a.dqbytes);
        const int dqoff = pos1 * a.ldq.s1 + pos2 * a.ldq.s2;
#pragma unroll
        for (int db = 0; db < D / 16; ++db) lean_store4<T>(rd, dqoff * ES, db, grp, acc[db], a.scale);
    }
    if (redo) lean_redo_bwd_q<T, D>(kernargs(), opaque(z), opaque(pos1), opaque(pos2), b, h, hk, grp);
}

// ---------------------------------------------------------------------------
// Backward, key side: over the queries attending each key (of every q head
// of its kv head's group), dv = sum P dO and dk = scale * sum P (dP - delta)
// q.  The union
// of the attending queries is staged (q and dO rows, and per slot
// -lse log2 e and -delta); a wave walks its own union rows, at most
// MAXCH chunks.
// ---------------------------------------------------------------------------
// Key tile of task x (lean_task; heads are kv heads): reads the delta rows
// the query tiles wrote.  The tile walks the q heads of its kv head's group
// (GQA: rep of them) and, 3-D (D3), the query planes whose windows hold its
// key plane, staging each (plane, q head)'s union in turn.
// A wave walks at most MAXC chunks (the host checks its rows fit).
template <typename T, int D, int MAXC, bool D3 = false, bool ONE_D = false>
__device__ __forceinline__ void lean_bwd_kv_tile(const LeanBwdArgs<T>& a, int x) {
    constexpr int NF = kNF<T, D>, TV = kTV<T, D>, ES = sizeof(T);
    const int nr = a.nr;
    unsigned char* smem = lds_base();
    T* Qs = reinterpret_cast<T*>(smem);
    T* Gs = Qs + nr * 16 * D;
    float* NL = reinterpret_cast<float*>(Gs + nr * 16 * D);  // nr * 16 slots, then 8 x -inf
    float* ND = NL + nr * 16 + 8;
    const int lane = threadIdx.x & 63, col = lane & 15, grp = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const LeanTask tk = lean_task<D3>(a.dec, x);
    const int b = tk.b, hk = tk.h, t = tk.t, z = tk.z;  // kv head
    const int rep = static_cast<int>(a.rep.d), h0 = hk * rep;
    const int* r = a.rec_k + t * kLeanRec;
    const int pr0 = r[0], pc0 = r[1], ur0 = r[2], uc0 = r[3], ext = r[4], nst = r[5];
    const int U1 = ext & 0xFF, U2 = (ext >> 8) & 0xFF, E1 = (ext >> 16) & 0xFF, E2 = (ext >> 24) & 0xFF;
    // the lane's key (1-D: item 16 w + n of the tile's 64)
    const int kr = 2 * wave + (col >> 3), kc = col & 7, item = 16 * wave + col;
    const bool valid = ONE_D ? item < E1 : (kr < E1 && kc < E2);
    const int pos1 = ONE_D ? 0 : pr0 + kr * a.d1, pos2 = ONE_D ? pr0 + item * a.d2 : pc0 + kc * a.d2;
    const long long zl = z;
    const int koff = pos1 * a.lk.s1 + pos2 * a.lk.s2;
    const long long kbo = b * a.lk.b + hk * a.lk.h + zl * a.lk.s0;
    const int dkoff = pos1 * a.ldk.s1 + pos2 * a.ldk.s2;
    const long long dkbo = b * a.ldk.b + hk * a.ldk.h + zl * a.ldk.s0;
    LeanDepth dw{0, 0, 0, 1};
    if constexpr (D3) dw = lean_depth_k(a.p.ax[0], z);
    if (r[14] || dw.n <= dw.j0) {  // no query attends these keys
        if (valid) {
            const __amdgpu_buffer_rsrc_t rk = lean_rsrc(a.dk + dkbo, a.dkbytes);
            const __amdgpu_buffer_rsrc_t rv = lean_rsrc(a.dv + dkbo, a.dkbytes);
            const f32x4_t zr = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int db = 0; db < D / 16; ++db) {
                lean_store4<T>(rk, dkoff * ES, db, grp, zr, 1.f);
                lean_store4<T>(rv, dkoff * ES, db, grp, zr, 1.f);
            }
        }
        return;
    }
    // per-slot -lse log2 e and -delta: slot threadIdx.x (and up, past 256 slots)
    const auto slot_pos = [&](int sidx, bool& in) {
        if constexpr (ONE_D) {
            in = sidx < r[8];  // the union's members
            return (ur0 + (in ? sidx : 0) * a.d2) * a.ll.s2;
        }
        const int u = sidx >> 4, cc = sidx & 15;
        in = u < U1 && cc < U2;
        return (ur0 + (in ? u : 0) * a.d1) * a.ll.s1 + (uc0 + (in ? cc : 0) * a.d2) * a.ll.s2;
    };
    bool sin;
    const int sp = slot_pos(threadIdx.x, sin);
    // query plane j of q head h: q and dO rows, and the lse / delta rows
    const auto plane = [&](int j) { return static_cast<long long>(dw.z0 + j * dw.d); };
    const auto lbase = [&](int j, int h) { return b * a.ll.b + h * a.ll.h + plane(j) * a.ll.s0; };
    const bool same_qg = a.lq.s1 == a.ldo.s1 && a.lq.s2 == a.ldo.s2;
    const auto stage = [&](int j, int h, float& sl, float& sd) {
        const long long lb = lbase(j, h);
        sl = a.lse[lb + sp];
        sd = a.delta[lb + sp];
        const __amdgpu_buffer_rsrc_t rq = lean_rsrc(a.q + (b * a.lq.b + h * a.lq.h + plane(j) * a.lq.s0), a.qbytes);
        const __amdgpu_buffer_rsrc_t rg =
            lean_rsrc(a.dout + (b * a.ldo.b + h * a.ldo.h + plane(j) * a.ldo.s0), a.dobytes);
        // union rows: 2-D one row per union row; 1-D 16 union slots per row
        const auto base = [&](const LeanLay& l) { return (ONE_D ? ur0 * l.s2 : ur0 * l.s1 + uc0 * l.s2) * ES; };
        const auto step1 = [&](const LeanLay& l) { return ONE_D ? 16 * l.s2 * a.d2 * ES : l.s1 * a.d1 * ES; };
        if (same_qg) {
            lean_stage<T, D>(rq, rg, Qs, Gs, base(a.lq), step1(a.lq), a.lq.s2 * a.d2 * ES, U1, U2, nst, wave, lane);
        } else {
            // q and dO rows at different strides (a packed qkv tensor's views)
            lean_stage1<T, D>(rq, Qs, base(a.lq), step1(a.lq), a.lq.s2 * a.d2 * ES, U1, U2, nst, wave, lane);
            lean_stage1<T, D>(rg, Gs, base(a.ldo), step1(a.ldo), a.ldo.s2 * a.d2 * ES, U1, U2, nst, wave, lane);
        }
    };
    float sl, sd;
    stage(dw.j0, h0, sl, sd);
    uint4 kf[NF], vf[NF];
    {
        const __amdgpu_buffer_rsrc_t rk = lean_rsrc(a.k + kbo, a.kbytes);
        const __amdgpu_buffer_rsrc_t rv = lean_rsrc(a.v + kbo, a.kbytes);
#pragma unroll
        for (int ks = 0; ks < NF; ++ks) {
            const uint32_t o = valid ? static_cast<uint32_t>(koff * ES + lean_frag_off<T, D>(ks, grp)) : kLeanOOR;
            kf[ks] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rk, o, 0, 0));
            vf[ks] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rv, o, 0, 0));
        }
    }
    // the wave's first staged row and chunk count; the lane's attending
    // queries (2-D: rows [rlo, rlo + rn) and columns [clo, chi]; 1-D: slots
    // [rlo, rlo + rn) from the first row); an unattended key has an empty range
    int first, nch, rlo, rn;
    f32x4_t cb[2];
    if constexpr (ONE_D) {
        first = __builtin_amdgcn_readfirstlane(sbyte(r[9], r[9], wave));
        nch = __builtin_amdgcn_readfirstlane(sbyte(r[10], r[10], wave));
        int alo, ahi;
        class_span(lean_class1d(r, a.p.ax[2]), pc0 + (valid ? item : 0), alo, ahi);
        rlo = alo - uc0 - 16 * first;
        rn = valid ? ahi - alo + 1 : 0;
    } else {
        first = __builtin_amdgcn_readfirstlane(sbyte(r[6], r[7], 2 * wave));
        const int last = __builtin_amdgcn_readfirstlane(sbyte(r[10], r[11], 2 * wave + 1));
        nch = (last - first + 2) >> 1;
        rlo = sbyte(r[6], r[7], kr) - first;
        rn = valid ? sbyte(r[10], r[11], kr) - first - rlo + 1 : 0;
        const int clo = sbyte(r[8], r[9], kc), chi = sbyte(r[12], r[13], kc);
        lean_colbias(clo, chi >= clo ? chi - clo + 1 : 0, grp, cb);
    }
    int aoff[2][NF], toff[TV][D / 16];
#pragma unroll
    for (int bb = 0; bb < 2; ++bb)
#pragma unroll
        for (int ks = 0; ks < NF; ++ks) aoff[bb][ks] = lean_score_off<T, D>(first, col, grp, bb, ks);
#pragma unroll
    for (int hi = 0; hi < TV; ++hi)
#pragma unroll
        for (int db = 0; db < D / 16; ++db) toff[hi][db] = lean_tr_off<T, D>(first, lane, hi, db);

    const unsigned char* Qb = reinterpret_cast<const unsigned char*>(Qs);
    const unsigned char* Gb = reinterpret_cast<const unsigned char*>(Gs);
    f32x4_t gk[D / 16], gv[D / 16];
#pragma unroll
    for (int db = 0; db < D / 16; ++db) gk[db] = gv[db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    const float* nlp = NL + first * 16 + 8 * grp;
    const float* ndp = ND + first * 16 + 8 * grp;
    const float* ninf = NL + nr * 16;
    // the (plane, q head) steps: heads fastest
    int j = dw.j0, h = h0;
#pragma unroll 1
    while (true) {
        wait_loads();
        if (static_cast<int>(threadIdx.x) < nr * 16) {
            NL[threadIdx.x] = sin ? -sl * kLog2e : 0.f;
            ND[threadIdx.x] = sin ? -sd : 0.f;
        }
        // the exponent offsets of lanes whose row test fails: P = 0
        if (threadIdx.x < 8) NL[nr * 16 + threadIdx.x] = -INFINITY;
        {
            const long long lb = lbase(j, h);
            for (int s = threadIdx.x + 64 * kLeanWaves; s < nr * 16; s += 64 * kLeanWaves) {
                bool in;
                const int o = slot_pos(s, in);
                NL[s] = in ? -a.lse[lb + o] * kLog2e : 0.f;
                ND[s] = in ? -a.delta[lb + o] : 0.f;
            }
        }
        lds_publish_barrier();
#pragma unroll
        for (int c = 0; c < MAXC; ++c) {
            if (c >= nch) break;  // wave-uniform
            const float* nlc;
            if constexpr (ONE_D) {
                lean_chunkbias(c, rlo, rn > 0 ? rn : 0, grp, cb);
                nlc = nlp + 32 * c;
            } else {
                const int row = 2 * c + (grp >> 1) - rlo;
                // a failed row test reads the -inf entries (one select per chunk)
                nlc = (row >= 0 && row < rn) ? nlp + 32 * c : ninf;
            }
            const f32x4_t nd[2] = {*reinterpret_cast<const f32x4_t*>(ndp + 32 * c),
                                   *reinterpret_cast<const f32x4_t*>(ndp + 32 * c + 4)};
            const f32x4_t nl[2] = {*reinterpret_cast<const f32x4_t*>(nlc), *reinterpret_cast<const f32x4_t*>(nlc + 4)};
            f32x4_t s[2], dp[2];
#pragma unroll
            for (int bb = 0; bb < 2; ++bb) {
                s[bb] = lean_score<T, D>(Qb, aoff, c, bb, kf, cb[bb]);
                dp[bb] = lean_score<T, D>(Gb, aoff, c, bb, vf, nd[bb]);
            }
#pragma unroll
            for (int bb = 0; bb < 2; ++bb)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    s[bb][i] = __builtin_amdgcn_exp2f(fmaf(s[bb][i], a.sc2, nl[bb][i]));
                    dp[bb][i] *= s[bb][i];
                }
            lean_acc<T, D>(Gb, toff, c, s, gv);
            lean_acc<T, D>(Qb, toff, c, dp, gk);
        }
        if (++h == h0 + rep) {
            h = h0;
            if (++j >= dw.n) break;
        }
        __syncthreads();  // the staged rows and their scalars are no longer read
        stage(j, h, sl, sd);
    }
    const bool redo = valid && item_nonfinite(lane_sum(gk, lane_sum(gv, 0.f)));
    if (valid) {
        const __amdgpu_buffer_rsrc_t rk = lean_rsrc(a.dk + dkbo, a.dkbytes);
        const __amdgpu_buffer_rsrc_t rv = lean_rsrc(a.dv + dkbo, a.dkbytes);
#pragma unroll
        for (int db = 0; db < D / 16; ++db) {
            lean_store4<T>(rk, dkoff * ES, db, grp, gk[db], a.scale);
            lean_store4<T>(rv, dkoff * ES, db, grp, gv[db], 1.f);
        }
    }
    if (redo) lean_redo_bwd_kv<T, D>(kernargs(), opaque(z), opaque(pos1), opaque(pos2), b, hk, grp);
}

// Waves per SIMD the key-side kernel is built for: 5 (at most 96 VGPRs) for
// the 16-bit 2-D kernel at head dim 32, whose LDS holds 5 workgroups per CU
// (the dQ kernel at 96 VGPRs spills and runs slower at 5 waves than at 4);
// no constraint otherwise.
constexpr int lean_kv_waves(int D, bool f32, bool d3, bool one_d) { return D == 32 && !f32 && !d3 && !one_d ? 5 : 1; }

template <typename T, int D, int NCH, bool D3 = false, bool ONE_D = false, int HP = 1>
__global__ __launch_bounds__(64 * kLeanWaves * HP) void k_lean_bwd_q(LeanBwdArgs<T> a) {
    lean_bwd_q_tile<T, D, NCH, D3, ONE_D, HP>(a, xcd_block(blockIdx.x, gridDim.x));
}

template <typename T, int D, int MAXC, bool D3 = false, bool ONE_D = false>
__global__ __launch_bounds__(64 * kLeanWaves) __attribute__((amdgpu_waves_per_eu(
    lean_kv_waves(D, kF32<T>, D3, ONE_D)))) void k_lean_bwd_kv(LeanBwdArgs<T> a) {
    lean_bwd_kv_tile<T, D, MAXC, D3, ONE_D>(a, xcd_block(blockIdx.x, gridDim.x));
}

// ---------------------------------------------------------------------------
// Split ops, key side: out[k] = mul * sum over the queries q attending key k
// of w[q][e(q, k)] x[q] (the dk of QK's backward with w = dattn, x = q; the
// dv of AV's backward with w = attn, x = dO).  Key tiles as in k_lean_bwd_kv:
// the union of the attending queries is staged, x rows by the 16-byte DMA
// (16 slots per union row) and, of each union query's row of w (KV
// entries), only the band of window rows that meet the key tile, by 16-byte
// DMA into one slot per union column (about a third of the row at K = 7;
// the band's layout is given where the kernel stages it).  In class coordinates
// e(q, k) = (J1(k) - ws1(q)) K2 + (J2(k) - ws2(q)); the host tables d1[u] =
// J1(first key) - ws1(union row u) and d2[u] (per union column) make it
// (d1[u1] + kr) K2 + (d2[u2] + kc) for the lane's key (kr, kc), and the pair
// is attended exactly when both terms lie in [0, K).  The weights of a chunk
// are then one LDS entry each, gathered into the B operand of the product
// that contracts over the chunk's 32 slots (as the key side's P in
// k_lean_bwd_kv).  The w rows share one 2-byte phase (lead) per (batch, head):
// the host checks that the row strides are even.
// ---------------------------------------------------------------------------
template <typename T>
struct LeanWsumKeyArgs {
    const int* rec;               // two records per key tile: the key record, then d1 / d2
    const T *w, *x;
    T* out;
    LeanLay lw, lx, lo;
    FastDiv heads, tiles;
    int nr;                       // LDS rows
    int d1, d2, K1, K2;
    uint32_t xbytes, wbytes;      // byte ranges of one (batch, head) plane of x and of w
    float mul;
    Prob p;
};

template <typename T, int D>
__device__ __forceinline__ void lean_redo_wsum_key(const void* kargs, int pos1, int pos2, int b, int h, int grp) {
    const LeanWsumKeyArgs<T>& A = *static_cast<const LeanWsumKeyArgs<T>*>(kargs);
    ExactAxis x[3];
    x[0] = exact_axis(A.p.ax[0], 0);
    x[1] = exact_axis(A.p.ax[1], pos1);
    x[2] = exact_axis(A.p.ax[2], pos2);
    f32x4_t acc[D / 16];
    exact_wsum_key<T, D>(x, A.w + b * A.lw.b + h * A.lw.h, Strides3{0, A.lw.s1, A.lw.s2},
                         A.x + b * A.lx.b + h * A.lx.h, Strides3{0, A.lx.s1, A.lx.s2}, grp, acc);
    store_rows<T, D>(A.out + b * A.lo.b + h * A.lo.h, pos1 * A.lo.s1 + pos2 * A.lo.s2, grp, acc, A.mul);
}

template <typename T, int D, int MAXC>
__global__ __launch_bounds__(64 * kLeanWaves) void k_lean_wsum_key(LeanWsumKeyArgs<T> a) {
    const int nr = a.nr;
    unsigned char* smem = lds_base();
    T* Xs = reinterpret_cast<T*>(smem);
    uint32_t* Ws32 = reinterpret_cast<uint32_t*>(Xs + nr * 16 * D);
    const int lane = threadIdx.x & 63, col = lane & 15, grp = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int x = xcd_block(blockIdx.x, gridDim.x);
    const int bt = fdiv(x, a.heads);
    const int h = x - bt * static_cast<int>(a.heads.d);
    const int b = fdiv(bt, a.tiles);
    const int t = bt - b * static_cast<int>(a.tiles.d);
    const int* r = a.rec + t * (2 * kLeanRec);
    const int* r2 = r + kLeanRec;
    const int pr0 = r[0], pc0 = r[1], ur0 = r[2], uc0 = r[3], ext = r[4], nst = r[5];
    const int U1 = ext & 0xFF, U2 = (ext >> 8) & 0xFF, E1 = (ext >> 16) & 0xFF, E2 = (ext >> 24) & 0xFF;
    const int kr = 2 * wave + (col >> 3), kc = col & 7;
    const bool valid = kr < E1 && kc < E2;
    const int pos1 = pr0 + kr * a.d1, pos2 = pc0 + kc * a.d2;
    const int ooff = pos1 * a.lo.s1 + pos2 * a.lo.s2;
    const long long obo = b * a.lo.b + h * a.lo.h;
    if (r[14]) {  // no query attends these keys
        if (valid) {
            const __amdgpu_buffer_rsrc_t ro = lean_rsrc(a.out + obo, kLeanOOR);
#pragma unroll
            for (int db = 0; db < D / 16; ++db)
                __builtin_amdgcn_raw_buffer_store_b64(v2u32_t{0u, 0u}, ro, ooff * 2 + db * 32 + grp * 8, 0, 0);
        }
        return;
    }
    // x rows of the union
    const long long xo = b * a.lx.b + h * a.lx.h;
    lean_stage1<T, D>(lean_rsrc(a.x + xo, a.xbytes), Xs, (ur0 * a.lx.s1 + uc0 * a.lx.s2) * 2, a.lx.s1 * a.d1 * 2,
                      a.lx.s2 * a.d2 * 2, U1, U2, nst, wave, lane);
    // w rows of the union, each over its band only: union row u's queries
    // meet the tile's key rows kr < E1 at window rows e1 = d1[u] + kr, so
    // the band is [lo, hi] = [d1[u], d1[u] + E1 - 1] clipped to [0, K1), n
    // rows, entries [lo K2, (hi + 1) K2).  It is staged from the word that
    // holds its first entry (entry sb = (lead + lo K2) rounded down to even,
    // counted from the plane's word-aligned base) in n16 = (n K2 + 8) / 8
    // chunks of 16 bytes, enough for either phase.  Row u's slots (union
    // columns cc < U2) start at chunk W_u + cc n16_u, W_u = U2 (n16_0 + ... +
    // n16_{u-1}); chunk t of a row goes to lane t % 64 of the row's DMA
    // instruction t / 64.  Lane u of each 16 holds row u's W, n16 and sb.
    const T* wplane = a.w + b * a.lw.b + h * a.lw.h;
    const int lead = static_cast<int>((reinterpret_cast<uintptr_t>(wplane) >> 1) & 1);
    int bw = 0, bn, bs;
    {
        const int u = lane & 15;
        const int d1u = u < 8 ? sbyte(r2[0], r2[1], u) : sbyte(r2[2], r2[3], u - 8);
        const int lo = max(d1u, 0), hi = min(d1u + E1 - 1, a.K1 - 1);
        bn = u < U1 && hi >= lo ? ((hi - lo + 1) * a.K2 + 8) >> 3 : 0;
        bs = (lead + lo * a.K2) & ~1;
        int run = 0;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            bw = u == v ? run : bw;
            run += __builtin_amdgcn_readlane(bn, v);
        }
        bw *= U2;
    }
    {
        const __amdgpu_buffer_rsrc_t rw = lean_rsrc(wplane - lead, a.wbytes);
        const int rs = a.lw.s1 * a.d1 * 2, cs = a.lw.s2 * a.d2 * 2;  // bytes between union rows / columns
        const int rbase = (ur0 * a.lw.s1 + uc0 * a.lw.s2) * 2;
        // union rows round-robin over the waves; lanes past a row's chunks
        // stay inactive (no LDS write), so rows never overlap
#pragma unroll 1
        for (int u = wave; u < U1; u += kLeanWaves) {
            const int n = __builtin_amdgcn_readlane(bn, u);
            if (n == 0) continue;
            const int w0 = __builtin_amdgcn_readlane(bw, u), sb = __builtin_amdgcn_readlane(bs, u);
            const int cnt = U2 * n, ro = rbase + u * rs + 2 * sb;
            const float rn = __builtin_amdgcn_rcpf(static_cast<float>(n));
#pragma unroll 1
            for (int t0 = 0; t0 < cnt; t0 += 64) {
                // slot cc and chunk k (t < 16 * 11: the float quotient is
                // exact to far below the 1 / (2 n) margin)
                const int t = t0 + lane;
                const int cc = static_cast<int>((static_cast<float>(t) + 0.5f) * rn);
                const int k = t - cc * n;
                if (t < cnt)
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (lds_void_t*)(Ws32 + 4 * (w0 + t0)), 16,
                                                             static_cast<uint32_t>(ro + cc * cs + 16 * k), 0, 0, 0);
            }
        }
    }
    // the wave's union rows [first, last] (of the key record)
    const int first = __builtin_amdgcn_readfirstlane(sbyte(r[6], r[7], 2 * wave));
    const int last = __builtin_amdgcn_readfirstlane(sbyte(r[10], r[11], 2 * wave + 1));
    const int nch = (last - first + 2) >> 1;
    // the lane's 8 slots of a chunk: union columns 8 (g % 2) + j (past the
    // union: the last column, whose entries the masks drop); window entry
    // offsets lead + e2 of the lane's key column and the column masks, two
    // entries per word.  Window entry ew of union row u sits at entry ew -
    // sb_u of its slot.
    const int c0 = 8 * (grp & 1), clast = U2 - 1;
    int cp[8];
    uint32_t cm[4];
    {
        const int t0 = (grp & 1) ? r2[6] : r2[4], t1 = (grp & 1) ? r2[7] : r2[5];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int e2 = sbyte(t0, t1, j) + kc;
            cp[j] = lead + e2;
            const uint32_t ok = static_cast<unsigned>(e2) < static_cast<unsigned>(a.K2) ? 0xFFFFu : 0u;
            if (j & 1)
                cm[j >> 1] |= ok << 16;
            else
                cm[j >> 1] = ok;
        }
    }
    int toff[2][D / 16];
#pragma unroll
    for (int hi = 0; hi < 2; ++hi)
#pragma unroll
        for (int db = 0; db < D / 16; ++db) toff[hi][db] = lean_tr_off<T, D>(first, lane, hi, db);

    const int d10 = r2[0], d11 = r2[1], d12 = r2[2], d13 = r2[3];  // d1 bytes of union rows 0-15

    wait_loads();
    __syncthreads();

    const unsigned char* Xb = reinterpret_cast<const unsigned char*>(Xs);
    const uint16_t* Ws = reinterpret_cast<const uint16_t*>(Ws32);
    f32x4_t acc[D / 16];
#pragma unroll
    for (int db = 0; db < D / 16; ++db) acc[db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < MAXC; ++c) {
        if (c >= nch) break;  // wave-uniform
        // union row of the lane's slots, its d1 entry (rows past the table: none attend)
        const int ua = first + 2 * c, ub = ua + 1;
        const int da = ua < 8 ? sbyte(d10, d11, ua) : (ua < 16 ? sbyte(d12, d13, ua - 8) : -100);
        const int dbb = ub < 8 ? sbyte(d10, d11, ub) : (ub < 16 ? sbyte(d12, d13, ub - 8) : -100);
        const bool second = grp >> 1;
        const int e1 = (second ? dbb : da) + kr;
        const bool rok = valid && static_cast<unsigned>(e1) < static_cast<unsigned>(a.K1);
        // the band of the lane's union row (a valid e1 lies in it)
        const int ra = min(ua, 15), rb = min(ub, 15);
        const int wa = __builtin_amdgcn_readlane(bw, ra), na = __builtin_amdgcn_readlane(bn, ra);
        const int sa = __builtin_amdgcn_readlane(bs, ra), wb2 = __builtin_amdgcn_readlane(bw, rb);
        const int nb = __builtin_amdgcn_readlane(bn, rb), sb2 = __builtin_amdgcn_readlane(bs, rb);
        const int pe = 8 * (second ? nb : na);  // entries per slot of the row
        const int base = rok ? 8 * (second ? wb2 : wa) - (second ? sb2 : sa) + e1 * a.K2 : 0;
        uint32_t wv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t lo16 = Ws[base + min(c0 + 2 * i, clast) * pe + cp[2 * i]];
            const uint32_t hi16 = Ws[base + min(c0 + 2 * i + 1, clast) * pe + cp[2 * i + 1]];
            wv[i] = rok ? ((lo16 | (hi16 << 16)) & cm[i]) : 0u;
        }
        lean_accumulate<T, D>(Xb, toff, c, make_uint4(wv[0], wv[1], wv[2], wv[3]), acc);
    }
    const bool redo = valid && item_nonfinite(lane_sum(acc, 0.f));
    if (valid) {
        const __amdgpu_buffer_rsrc_t ro = lean_rsrc(a.out + obo, kLeanOOR);
#pragma unroll
        for (int db = 0; db < D / 16; ++db) {
            const uint2 wo = make_uint2(Mma<T>::pack(acc[db][0] * a.mul, acc[db][1] * a.mul),
                                        Mma<T>::pack(acc[db][2] * a.mul, acc[db][3] * a.mul));
            __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(v2u32_t, wo), ro, ooff * 2 + db * 32 + grp * 8,
                                                  0, 0);
        }
    }
    if (redo) lean_redo_wsum_key<T, D>(kernargs(), opaque(pos1), opaque(pos2), b, h, grp);
}

}  // namespace

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
namespace {

// Tile records of one problem geometry (axes 1 and 2), query tiles (key
// false) or key tiles (key true), cached per device for the process.
struct LeanGeo {
    int dev, key;
    int len[2], k[2], dil[2], causal[2];
    int* ptr;
    int ntiles, nst_max, rows_max, u2_max;
    int wchunks_max;        // split key tiles: the most 16-byte chunks of staged w bands
    std::vector<int> host;  // source of the asynchronous upload, kept with the table
    TableUpload up;
};

struct LeanAxisTile {
    int pos0, upos0, E, U;
    int J, lo;   // class coordinates of the first item and of the union's first member
    int ws[8];   // per item: window start (key tiles: first attending query), union-relative
    int we[8];   // key tiles: last attending query, union-relative
};

// Tile t of class r on one axis: items J = 8t .. 8t+7 (class coordinates).
bool lean_axis_tile(const Axis& A, int r, int t, bool key, LeanAxisTile& o) {
    const ClassAxis c = class_axis(A, r);
    const int J = 8 * t;
    const int jend = std::min(J + 8, c.n) - 1;
    o.E = jend - J + 1;
    int lo, hi;
    if (!key) {
        lo = std::max(class_ws(c, J), 0);
        hi = std::min(class_ws(c, jend) + c.K - 1, c.n - 1);
    } else {
        int x;
        class_span(c, J, lo, x);
        class_span(c, jend, x, hi);
        if (hi < lo) return false;
    }
    o.U = hi - lo + 1;
    o.J = J;
    o.lo = lo;
    o.pos0 = r + J * A.dil;
    o.upos0 = r + lo * A.dil;
    for (int e = 0; e < 8; ++e) {
        const int j = std::min(J + e, jend);
        if (!key) {
            o.ws[e] = class_ws(c, j) - lo;
            o.we[e] = o.ws[e] + c.K - 1;
        } else {
            int a0, a1;
            class_span(c, j, a0, a1);
            o.ws[e] = a0 - lo;
            o.we[e] = a1 - lo;
        }
    }
    return true;
}

int pack_bytes(const int* v, int i0) {
    uint32_t w = 0;
    for (int e = 0; e < 4; ++e) w |= (static_cast<uint32_t>(v[i0 + e]) & 0xFFu) << (8 * e);
    return static_cast<int>(w);
}

// d[u] = J - ws(lo + u) over the union members u < U of a key tile's axis
// (the entry offset of the tile's first key in member u's window), -100
// past the union; packed as 16 signed bytes.
void split_table(const Axis& A, int r, const LeanAxisTile& a, int* out4) {
    const ClassAxis c = class_axis(A, r);
    int d[16];
    for (int u = 0; u < 16; ++u) d[u] = u < a.U ? a.J - class_ws(c, a.lo + u) : -100;
    for (int i = 0; i < 4; ++i) out4[i] = pack_bytes(d, 4 * i);
}

// 16-byte chunks per union column that a split key tile stages of its w
// rows: union row u only its band of window rows that meet the tile's key
// rows, n of them, in (n K2 + 8) / 8 chunks.
int split_chunks(const Axis& A, int r, const LeanAxisTile& a, int K2) {
    const ClassAxis c = class_axis(A, r);
    int sum = 0;
    for (int u = 0; u < a.U; ++u) {
        const int d = a.J - class_ws(c, a.lo + u);
        const int lo = std::max(d, 0), hi = std::min(d + a.E - 1, A.k - 1);
        if (hi >= lo) sum += ((hi - lo + 1) * K2 + 8) >> 3;
    }
    return sum;
}

// A 1-D problem (axes 0 and 1 of extent 1): tiles of 64 consecutive class
// items along axis 2.
bool lean_1d(const Prob& p) { return p.ax[0].len == 1 && p.ax[1].len == 1 && p.ax[1].k == 1; }

// Chunks of 32 slots a wave of a 1-D query tile reads: its 16 windows from
// the staged row holding the first of them (up to 15 slots in).
int lean_nch_1d(int K) { return std::max(1, (K + 30 + 31) / 32); }

// Records of the 1-D tiles (one per 64 class items of each residue class):
// query tiles (key false) pos0, J, the union's first position and class
// coordinate, ext (staged rows | 16 << 8 | items << 16), rows to stage, the
// class size and border start, the union's size; key tiles also each
// wave's first staged row (bytes of [9]) and chunk count (bytes of [10]),
// and [14] = 1 where no query attends the tile.  False when a wave's
// windows (attending spans) do not fit nch (key tiles: nch + 2) chunks.
bool lean_records_1d(const Prob& p, bool key, int nch, std::vector<int>& h, int& nst_max, int& rows_max) {
    const Axis& A = p.ax[2];
    for (int r = 0; r < A.dil; ++r) {
        const ClassAxis c = class_axis(A, r);
        for (int J = 0; J < c.n; J += 64) {
            const int E = std::min(64, c.n - J), jend = J + E - 1;
            int rec[kLeanRec] = {};
            rec[0] = r + J * A.dil;
            rec[1] = J;
            rec[6] = c.n;
            rec[7] = c.B;
            int U0, Uend;
            if (!key) {
                U0 = std::max(class_ws(c, J), 0);
                Uend = std::min(class_ws(c, jend) + c.K - 1, c.n - 1);
            } else {
                U0 = c.n;
                Uend = -1;
                for (int u = J; u <= jend; ++u) {
                    int lo, hi;
                    class_span(c, u, lo, hi);
                    if (lo <= hi) {
                        U0 = std::min(U0, lo);
                        Uend = std::max(Uend, hi);
                    }
                }
            }
            if (Uend < U0) {  // key tile that no query attends: extents only (zero gradients)
                rec[4] = E << 16;
                rec[14] = 1;
                h.insert(h.end(), rec, rec + kLeanRec);
                continue;
            }
            const int NU = Uend - U0 + 1, rows = (NU + 15) / 16;
            int nst = rows, fb[4] = {}, nb[4] = {};
            for (int w = 0; w < 4 && 16 * w < E; ++w) {
                const int u0 = J + 16 * w, u1 = std::min(u0 + 15, jend);
                int first, end = 0;  // end: one past the wave's last slot, from its first row
                if (!key) {
                    first = std::max(class_ws(c, u0) - U0, 0) >> 4;
                    for (int j = u0; j <= u1; ++j) end = std::max(end, class_ws(c, j) - U0 - 16 * first + c.K);
                } else {
                    int wlo = c.n, whi = -1;
                    for (int u = u0; u <= u1; ++u) {
                        int lo, hi;
                        class_span(c, u, lo, hi);
                        if (lo <= hi) {
                            wlo = std::min(wlo, lo);
                            whi = std::max(whi, hi);
                        }
                    }
                    if (whi < wlo) continue;  // no key of the wave is attended
                    first = (wlo - U0) >> 4;
                    end = whi - U0 - 16 * first + 1;
                }
                const int need = (end + 31) / 32;
                if (need > (key ? nch + 2 : nch)) return false;
                fb[w] = first;
                nb[w] = need;
                nst = std::max(nst, first + 2 * (key ? need : nch));
                rows_max = std::max(rows_max, 2 * need);
            }
            rec[2] = r + U0 * A.dil;
            rec[3] = U0;
            rec[4] = rows | (16 << 8) | (E << 16);
            rec[5] = nst;
            rec[8] = NU;
            rec[9] = pack_bytes(fb, 0);
            rec[10] = pack_bytes(nb, 0);
            nst_max = std::max(nst_max, nst);
            h.insert(h.end(), rec, rec + kLeanRec);
        }
    }
    return true;
}

// Builds (or finds) the records.  Query tiles: rows of a wave start at
// max(ws[2w], 0) and span at most K1 + 1 rows; nst = rows to stage.  Mode:
// 0 query tiles, 1 key tiles, 2 key tiles of the split key side (each key
// record followed by a second one holding the d1 / d2 tables).
const LeanGeo* lean_geometry(const Prob& p, int mode, int nch, hipStream_t s) {
    static std::mutex mu;
    static std::vector<LeanGeo*> cache;
    const bool key = mode != 0;
    const int per_tile = mode == 2 ? 2 * kLeanRec : kLeanRec;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return nullptr;
    LeanGeo k{};
    k.dev = dev;
    k.key = mode;
    for (int a = 0; a < 2; ++a) {
        k.len[a] = p.ax[a + 1].len;
        k.k[a] = p.ax[a + 1].k;
        k.dil[a] = p.ax[a + 1].dil;
        k.causal[a] = p.ax[a + 1].causal;
    }
    std::lock_guard<std::mutex> g(mu);
    for (LeanGeo* e : cache)
        if (std::memcmp(e, &k, offsetof(LeanGeo, ptr)) == 0) return table_ready(e->up, s) ? e : nullptr;
    if (!device_alloc_allowed()) return nullptr;
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &st) != hipSuccess || st != hipStreamCaptureStatusNone) return nullptr;
    const Axis &A1 = p.ax[1], &A2 = p.ax[2];
    std::vector<int> h;
    int nst_max = 0, rows_max = 0, u2_max = 1, wch_max = 0;
    if (lean_1d(p)) {
        if (mode == 2 || !lean_records_1d(p, key, nch, h, nst_max, rows_max)) return nullptr;
    } else {
    for (int r1 = 0; r1 < A1.dil; ++r1) {
        const int n1 = (A1.len - r1 + A1.dil - 1) / A1.dil;
        for (int r2 = 0; r2 < A2.dil; ++r2) {
            const int n2 = (A2.len - r2 + A2.dil - 1) / A2.dil;
            for (int t1 = 0; t1 < (n1 + 7) / 8; ++t1) {
                LeanAxisTile a1;
                const bool ok1 = lean_axis_tile(A1, r1, t1, key, a1);
                for (int t2 = 0; t2 < (n2 + 7) / 8; ++t2) {
                    LeanAxisTile a2;
                    const bool ok2 = lean_axis_tile(A2, r2, t2, key, a2);
                    int rec[kLeanRec] = {};
                    if (ok1 && ok2) {
                        if (a2.U > 16) return nullptr;  // eligibility should have excluded it
                        // rows a wave reads: query tiles NCH chunks from max(ws, 0);
                        // key tiles its own attending rows, in whole chunks
                        int nst = 0;
                        for (int w = 0; w < 4; ++w) {
                            const int f = key ? a1.ws[2 * w] : std::max(a1.ws[2 * w], 0);
                            const int rows = a1.we[2 * w + 1] - f + 1;
                            rows_max = std::max(rows_max, rows);
                            nst = std::max(nst, f + (key ? 2 * ((std::max(rows, 0) + 1) / 2) : 2 * nch));
                        }
                        nst = std::max(nst, a1.U);
                        nst_max = std::max(nst_max, nst);
                        u2_max = std::max(u2_max, a2.U);
                        rec[0] = a1.pos0;
                        rec[1] = a2.pos0;
                        rec[2] = a1.upos0;
                        rec[3] = a2.upos0;
                        rec[4] = a1.U | (a2.U << 8) | (a1.E << 16) | (a2.E << 24);
                        rec[5] = nst;
                        rec[6] = pack_bytes(a1.ws, 0);
                        rec[7] = pack_bytes(a1.ws, 4);
                        rec[8] = pack_bytes(a2.ws, 0);
                        rec[9] = pack_bytes(a2.ws, 4);
                        rec[10] = pack_bytes(a1.we, 0);
                        rec[11] = pack_bytes(a1.we, 4);
                        rec[12] = pack_bytes(a2.we, 0);
                        rec[13] = pack_bytes(a2.we, 4);
                    } else {
                        // a key tile that no query attends: extents only (zero gradients)
                        rec[0] = ok1 ? a1.pos0 : r1 + 8 * t1 * A1.dil;
                        rec[1] = ok2 ? a2.pos0 : r2 + 8 * t2 * A2.dil;
                        rec[4] = (std::min(8, n1 - 8 * t1) << 16) | (std::min(8, n2 - 8 * t2) << 24);
                        rec[14] = 1;
                    }
                    h.insert(h.end(), rec, rec + kLeanRec);
                    if (mode == 2) {
                        int tab[kLeanRec] = {};
                        if (ok1 && ok2) {
                            if (a1.U > 16) return nullptr;
                            split_table(A1, r1, a1, tab);
                            split_table(A2, r2, a2, tab + 4);
                            wch_max = std::max(wch_max, split_chunks(A1, r1, a1, A2.k) * a2.U);
                        }
                        h.insert(h.end(), tab, tab + kLeanRec);
                    }
                }
            }
        }
    }
    }
    if (!key && nst_max > (lean_1d(p) ? lean_rows<true>(nch) : lean_rows<false>(nch))) return nullptr;
    if (key && nst_max > 32) return nullptr;
    int* d = nullptr;
    const size_t bytes = h.size() * sizeof(int);
    if (hipMalloc(reinterpret_cast<void**>(&d), bytes) != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
    }
    LeanGeo* e = new LeanGeo(k);
    e->host = std::move(h);
    // stream-ordered upload; the host copy lives as long as the table
    if (table_upload(e->up, d, e->host.data(), bytes, s) != hipSuccess) {
        (void)hipGetLastError();
        (void)hipFree(d);
        delete e;
        return nullptr;
    }
    e->ptr = d;
    e->ntiles = static_cast<int>(e->host.size() / per_tile);
    e->nst_max = nst_max;
    e->rows_max = rows_max;
    e->u2_max = u2_max;
    e->wchunks_max = wch_max;
    cache.push_back(e);
    return e;
}

LeanLay lean_lay(const Lay& l) {
    return LeanLay{l.b, l.h, static_cast<int>(l.s1), static_cast<int>(l.s2), static_cast<int>(l.s0)};
}

// A 3-D problem: the tiles walk depth planes (axis 0 of a 2-D problem has
// extent 1).
bool lean_3d(const Prob& p) { return p.ax[0].len > 1; }

LeanDecode lean_decode(const Prob& p, int heads, int ntiles) {
    LeanDecode d;
    d.heads = make_fastdiv(heads);
    d.tiles = make_fastdiv(ntiles);
    const int hg = heads % 2 == 0 ? 2 : 1;
    d.hg = make_fastdiv(hg);
    d.zlen = make_fastdiv(p.ax[0].len);
    d.hgroups = make_fastdiv(heads / hg);
    return d;
}

// Byte range of one (batch, head) plane of an operand of head dim D
// (elements of esz bytes).
uint32_t plane_bytes(const Prob& p, const Lay& l, int D, int esz = 2) {
    const long long v = ((static_cast<long long>(p.ax[1].len) - 1) * l.s1 +
                         (static_cast<long long>(p.ax[2].len) - 1) * l.s2 + D) * esz;
    return static_cast<uint32_t>(v);
}

// Two q heads per workgroup for GQA (NATTEN_HIP_LEAN_PAIRS=0 turns it off).
bool lean_head_pairs() {
    static const bool on = [] {
        const char* e = std::getenv("NATTEN_HIP_LEAN_PAIRS");
        return !(e && std::strcmp(e, "0") == 0);
    }();
    return on;
}

bool lean_switch() {
    static const bool on = [] {
        const char* e = std::getenv("NATTEN_HIP_LEAN");
        return !(e && std::strcmp(e, "0") == 0);
    }();
    return on;
}

// The lean kernels address LDS from the constant offset of lds_base(), as
// the general tile kernels do: every instance is checked once per process
// for static LDS (which would overlap it); one with static LDS turns the
// lean path off with a message.
template <typename T, int D, int NCH>
void lean_audit_one(LdsAudit& a) {
    audit_one(k_lean_fwd<T, D, NCH>, "k_lean_fwd", a);
    audit_one(k_lean_bwd_q<T, D, NCH>, "k_lean_bwd_q", a);
    audit_one(k_lean_bwd_kv<T, D, NCH + 2>, "k_lean_bwd_kv", a);
    audit_one(k_lean_fwd<T, D, NCH, false, true>, "k_lean_fwd (1-D)", a);
    if constexpr (!kF32<T>) {
        audit_one(k_lean_fwd<T, D, NCH, false, false, 2>, "k_lean_fwd (head pairs)", a);
        audit_one(k_lean_fwd<T, D, NCH, false, true, 2>, "k_lean_fwd (1-D, head pairs)", a);
        audit_one(k_lean_bwd_q<T, D, NCH, false, false, 2>, "k_lean_bwd_q (head pairs)", a);
        audit_one(k_lean_bwd_q<T, D, NCH, false, true, 2>, "k_lean_bwd_q (1-D, head pairs)", a);
    }
    audit_one(k_lean_bwd_q<T, D, NCH, false, true>, "k_lean_bwd_q (1-D)", a);
    audit_one(k_lean_bwd_kv<T, D, NCH + 2, false, true>, "k_lean_bwd_kv (1-D)", a);
    if constexpr (!kF32<T>) {
        audit_one(k_lean_wsum_key<T, D, NCH + 2>, "k_lean_wsum_key", a);
    } else {
        audit_one(k_lean_fwd<T, D, NCH, true>, "k_lean_fwd (3-D)", a);
        audit_one(k_lean_bwd_q<T, D, NCH, true>, "k_lean_bwd_q (3-D)", a);
        audit_one(k_lean_bwd_kv<T, D, NCH + 2, true>, "k_lean_bwd_kv (3-D)", a);
    }
}

template <typename T, int D>
void lean_audit_dim(LdsAudit& a) {
    lean_audit_one<T, D, 1>(a);
    lean_audit_one<T, D, 2>(a);
    lean_audit_one<T, D, 3>(a);
    lean_audit_one<T, D, 4>(a);
    lean_audit_one<T, D, 5>(a);
}

const LdsAudit& lean_audit() {
    static const LdsAudit result = [] {
        LdsAudit a;
        lean_audit_dim<bf16, 32>(a);
        lean_audit_dim<bf16, 64>(a);
        lean_audit_dim<f16, 32>(a);
        lean_audit_dim<f16, 64>(a);
        lean_audit_dim<float, 32>(a);
        lean_audit_dim<float, 64>(a);
        return a;
    }();
    return result;
}

bool lean_static_lds_ok() { return lean_audit().bad == 0; }

// Chunks per wave for kernel K1 (query side): K1 + 1 rows.
int lean_nch(int K1) { return (K1 + 2) / 2; }

}  // namespace

// Lean path eligibility: a 2-D (or 2-D-padded) problem at stride 1, or an
// fp32 3-D one at stride 1 (the 16-bit ones run faster on the general tile
// kernels, whose 3-D tiles share each staged plane between two depths; in
// fp32 those have no instances), head dim 32 or 64 for q, k and v, K2 <= 9,
// K1 <= 9, in-plane extents below 2^15, planes below 2^30 bytes (and a
// (batch, head) volume's element offsets in 31 bits for 3-D).  Every
// operand has its own layout, except that the operands staged or stored
// together share one: kvside lists pairs (k, v) and (dk, dv), and the fp32
// rows (lse, delta, dlse) share one.
bool lean_eligible(const Prob& p, int dtype, bool aligned, std::initializer_list<Lay> qside,
                   std::initializer_list<Lay> kvside, std::initializer_list<Lay> rows) {
    if (!lean_switch() || !aligned || !(p.scale > 0.f) || !lean_static_lds_ok()) return false;
    if (p.Dqk != p.Dv || (p.Dqk != 32 && p.Dqk != 64)) return false;
    // 1-D problems run as 64-item tiles along axis 2 (K <= 129: at most 5
    // chunks per wave); a short first in-plane axis otherwise stays on the
    // general tiles
    const bool d1 = lean_1d(p), d3 = lean_3d(p);
    if (d1) {
        const Axis& A = p.ax[2];
        if (A.st != 1 || A.k > 129 || lean_nch_1d(A.k) > 5 || A.len >= (1 << 30)) return false;
    } else {
        if (p.ax[1].len < 8) return false;
        if (!d3 && p.ax[0].k != 1) return false;
        if (d3 && (dtype != NATTEN_F32 || p.ax[0].st != 1 || p.ax[0].len >= (1 << 15))) return false;
        for (int a = 1; a < 3; ++a) {
            const Axis& A = p.ax[a];
            if (A.st != 1 || A.k > 9 || A.len >= (1 << 15)) return false;
        }
    }
    if (kvside.size() % 2 != 0 || !all_same(rows)) return false;
    for (const Lay* l = kvside.begin(); l != kvside.end(); l += 2)
        if (!same_lay(l[0], l[1])) return false;
    const long long z1 = static_cast<long long>(p.ax[0].len) - 1;
    const int esz = dtype == NATTEN_F32 ? 4 : 2;
    for (const auto& side : {qside, kvside}) {
        for (const Lay& l : side) {
            if (l.s1 < 0 || l.s2 < 0 || l.b < 0 || l.h < 0 || l.s0 < 0) return false;
            const long long v = (static_cast<long long>(p.ax[1].len) - 1) * l.s1 +
                                (static_cast<long long>(p.ax[2].len) - 1) * l.s2 + p.Dqk;
            if (v * esz >= (1LL << 30)) return false;
            if (d3 && z1 * l.s0 + v >= (1LL << 31)) return false;
        }
    }
    // fp32 rows (lse, delta, dlse): element offsets in 31 bits
    const Lay& r = *rows.begin();
    if (r.s1 < 0 || r.s2 < 0 || r.b < 0 || r.h < 0 || r.s0 < 0) return false;
    if (z1 * r.s0 + (static_cast<long long>(p.ax[1].len) - 1) * r.s1 +
            (static_cast<long long>(p.ax[2].len) - 1) * r.s2 >=
        (1LL << 31))
        return false;
    return true;
}

int lean_lds_audit(int* checked) {
    const LdsAudit& a = lean_audit();
    if (checked) *checked = a.checked;
    return a.bad == 0 ? 1 : 0;
}

template <typename T, int D, int NCH, bool D3, bool ONE_D = false, int HP = 1>
hipError_t lean_fwd_run(const Prob& p, const LeanGeo* g, const void* q, Lay lq, const void* k, Lay lk,
                        const void* v, void* o, Lay lo, float* lse, Lay ll, hipStream_t s) {
    LeanFwdArgs<T> a{};
    a.rec = g->ptr;
    a.q = static_cast<const T*>(q);
    a.k = static_cast<const T*>(k);
    a.v = static_cast<const T*>(v);
    a.out = static_cast<T*>(o);
    a.lse = lse;
    a.lq = lean_lay(lq);
    a.lk = lean_lay(lk);
    a.ll = lean_lay(ll);
    a.lo = lean_lay(lo);
    a.dec = lean_decode(p, p.Hq / HP, g->ntiles);
    a.rep = make_fastdiv(p.rep);
    a.d1 = p.ax[1].dil;
    a.d2 = p.ax[2].dil;
    a.K1 = p.ax[1].k;
    a.K2 = p.ax[2].k;
    a.qbytes = plane_bytes(p, lq, D, sizeof(T));
    a.kbytes = plane_bytes(p, lk, D, sizeof(T));
    a.obytes = plane_bytes(p, lo, D, sizeof(T));
    a.sc2 = p.scale * kLog2e;
    a.p = p;
    const long long blocks = static_cast<long long>(p.B) * (p.Hq / HP) * g->ntiles * p.ax[0].len;
    if (blocks >= (1LL << 31)) return hipErrorNotSupported;
    const size_t shm = kLdsPad + static_cast<size_t>(2) * lean_rows<ONE_D>(NCH) * 16 * D * sizeof(T);
    if (shm > 160 * 1024) return hipErrorNotSupported;
    auto kern = k_lean_fwd<T, D, NCH, D3, ONE_D, HP>;
    const hipError_t e = allow_lds(kern, shm);
    if (e != hipSuccess) return e;
    NA_LAUNCH("na_fwd_lean", kern, dim3(static_cast<unsigned>(blocks)), dim3(64 * kLeanWaves * HP), shm, s, a);
    return hipGetLastError();
}

// Forward on the lean kernels; hipErrorNotSupported when this problem has no
// lean launch (the caller then takes the general tile kernels).
hipError_t lean_forward(const Prob& p, const void* q, Lay lq, const void* k, Lay lk, const void* v, Lay lv, void* o,
                        Lay lo, float* lse, Lay ll, int dtype, hipStream_t s) {
    (void)lv;
    const bool d1 = lean_1d(p), d3 = lean_3d(p);
    const int nch = d1 ? lean_nch_1d(p.ax[2].k) : lean_nch(p.ax[1].k);
    if (static_cast<long long>(p.B) * p.Hq * p.ax[0].len * 4096 >= (1LL << 31)) return hipErrorNotSupported;
    const LeanGeo* g = lean_geometry(p, 0, nch, s);
    if (!g) return hipErrorNotSupported;
    // 3-D instances exist for fp32 only (the eligibility keeps 16-bit 3-D away)
#define NA_LF_ARGS p, g, q, lq, k, lk, v, o, lo, lse, ll, s
    // GQA with an even group: two q heads per workgroup share the staged K/V
    const bool pairs = p.rep % 2 == 0 && lean_head_pairs();
#define NA_LF(T, DD, N)                                                                                 \
    return d1 ? (pairs ? lean_fwd_run<T, DD, N, false, true, 2>(NA_LF_ARGS)                             \
                       : lean_fwd_run<T, DD, N, false, true>(NA_LF_ARGS))                               \
              : (pairs ? lean_fwd_run<T, DD, N, false, false, 2>(NA_LF_ARGS) : lean_fwd_run<T, DD, N, false>(NA_LF_ARGS))
#define NA_LF3(T, DD, N)                                                                         \
    return d1 ? lean_fwd_run<T, DD, N, false, true>(NA_LF_ARGS)                                  \
              : (d3 ? lean_fwd_run<T, DD, N, true>(NA_LF_ARGS) : lean_fwd_run<T, DD, N, false>(NA_LF_ARGS))
#define NA_LF_N(T, DD, F)    \
    switch (nch) {           \
        case 1: F(T, DD, 1); \
        case 2: F(T, DD, 2); \
        case 3: F(T, DD, 3); \
        case 4: F(T, DD, 4); \
        default: F(T, DD, 5); \
    }
    if (d3 && dtype != NATTEN_F32) return hipErrorNotSupported;
    if (dtype == NATTEN_BF16) {
        if (p.Dqk == 32) NA_LF_N(bf16, 32, NA_LF);
        NA_LF_N(bf16, 64, NA_LF);
    }
    if (dtype == NATTEN_F32) {
        if (p.Dqk == 32) NA_LF_N(float, 32, NA_LF3);
        NA_LF_N(float, 64, NA_LF3);
    }
    if (p.Dqk == 32) NA_LF_N(f16, 32, NA_LF);
    NA_LF_N(f16, 64, NA_LF);
#undef NA_LF_N
#undef NA_LF3
#undef NA_LF
#undef NA_LF_ARGS
}

template <typename T, int D>
LeanBwdArgs<T> lean_bwd_args(const Prob& p, const void* q, Lay lq, const void* k, Lay lk, const void* v,
                             const void* o, Lay lo, const void* dout, Lay ldo, const float* lse, Lay ll,
                             const float* dlse, void* dq, Lay ldq, void* dk, Lay ldk, void* dv, float* delta) {
    LeanBwdArgs<T> a{};
    a.q = static_cast<const T*>(q);
    a.k = static_cast<const T*>(k);
    a.v = static_cast<const T*>(v);
    a.o = static_cast<const T*>(o);
    a.dout = static_cast<const T*>(dout);
    a.lse = lse;
    a.dlse = dlse;
    a.dq = static_cast<T*>(dq);
    a.dk = static_cast<T*>(dk);
    a.dv = static_cast<T*>(dv);
    a.delta = delta;
    a.lq = lean_lay(lq);
    a.lk = lean_lay(lk);
    a.ll = lean_lay(ll);
    a.lo = lean_lay(lo);
    a.ldo = lean_lay(ldo);
    a.ldq = lean_lay(ldq);
    a.ldk = lean_lay(ldk);
    a.rep = make_fastdiv(p.rep);
    a.d1 = p.ax[1].dil;
    a.d2 = p.ax[2].dil;
    a.K1 = p.ax[1].k;
    a.K2 = p.ax[2].k;
    a.qbytes = plane_bytes(p, lq, D, sizeof(T));
    a.kbytes = plane_bytes(p, lk, D, sizeof(T));
    a.obytes = plane_bytes(p, lo, D, sizeof(T));
    a.dobytes = plane_bytes(p, ldo, D, sizeof(T));
    a.dqbytes = plane_bytes(p, ldq, D, sizeof(T));
    a.dkbytes = plane_bytes(p, ldk, D, sizeof(T));
    a.sc2 = p.scale * kLog2e;
    a.scale = p.scale;
    a.p = p;
    return a;
}

template <typename T, int D, int NCH, bool D3, bool ONE_D = false, int HP = 1>
hipError_t lean_bwd_run(const Prob& p, const LeanGeo* gq, const LeanGeo* gk, const LeanBwdArgs<T>& base,
                        hipStream_t s) {
    LeanBwdArgs<T> a = base;
    a.rec = gq->ptr;
    a.rec_k = gk->ptr;
    a.dec = lean_decode(p, p.Hq / HP, gq->ntiles);
    a.nr = std::max(gk->nst_max, 1);
    const size_t shm_q = kLdsPad + static_cast<size_t>(2) * lean_rows<ONE_D>(NCH) * 16 * D * sizeof(T);
    const size_t shm_k =
        kLdsPad + static_cast<size_t>(a.nr) * 16 * (2 * D * sizeof(T) + 2 * sizeof(float)) + 8 * sizeof(float);
    const long long tasks = static_cast<long long>(p.B) * (p.Hq / HP) * gq->ntiles * p.ax[0].len;
    if (tasks >= (1LL << 31) || shm_q > 160 * 1024 || shm_k > 160 * 1024) return hipErrorNotSupported;
    auto kq = k_lean_bwd_q<T, D, NCH, D3, ONE_D, HP>;
    hipError_t e = allow_lds(kq, shm_q);
    if (e != hipSuccess) return e;
    NA_LAUNCH("na_bwd_q_lean", kq, dim3(static_cast<unsigned>(tasks)), dim3(64 * kLeanWaves * HP), shm_q, s, a);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    auto kern = k_lean_bwd_kv<T, D, NCH + 2, D3, ONE_D>;
    if ((e = allow_lds(kern, shm_k)) != hipSuccess) return e;
    // key tiles over the kv heads, each walking the q heads of its group
    LeanBwdArgs<T> ak = a;
    ak.dec = lean_decode(p, p.Hkv, gq->ntiles);
    const long long ktasks = static_cast<long long>(p.B) * p.Hkv * gq->ntiles * p.ax[0].len;
    NA_LAUNCH("na_bwd_kv_lean", kern, dim3(static_cast<unsigned>(ktasks)), dim3(64 * kLeanWaves), shm_k, s, ak);
    return hipGetLastError();
}

// Backward on the lean kernels; hipErrorNotSupported
// when this problem has no lean launch.
hipError_t lean_backward(const Prob& p, const void* q, Lay lq, const void* k, Lay lk, const void* v, Lay lv,
                         const void* o, Lay lo, const void* dout, Lay ldo, const float* lse, Lay ll,
                         const float* dlse, Lay ldl, void* dq, Lay ldq, void* dk, Lay ldk, void* dv, Lay ldv,
                         float* delta, Lay lde, int dtype, hipStream_t s) {
    (void)lv;
    (void)ldv;
    if (!same_lay(ll, lde) || (dlse && !same_lay(ll, ldl))) return hipErrorNotSupported;
    if (static_cast<long long>(p.B) * p.Hq * p.ax[0].len * 8192 >= (1LL << 31)) return hipErrorNotSupported;
    const bool d1 = lean_1d(p), d3 = lean_3d(p);
    if (d3 && dtype != NATTEN_F32) return hipErrorNotSupported;  // 3-D instances exist for fp32 only
    const int nch = d1 ? lean_nch_1d(p.ax[2].k) : lean_nch(p.ax[1].k);
    const LeanGeo* gq = lean_geometry(p, 0, nch, s);
    const LeanGeo* gk = gq ? lean_geometry(p, 1, nch, s) : nullptr;
    if (!gq || !gk || gq->ntiles != gk->ntiles || gk->rows_max > 2 * (nch + 2)) return hipErrorNotSupported;
#define NA_LB_A(T, DD) \
    lean_bwd_args<T, DD>(p, q, lq, k, lk, v, o, lo, dout, ldo, lse, ll, dlse, dq, ldq, dk, ldk, dv, delta)
    // GQA with an even group: two q heads per dQ workgroup share the staged K/V
    const bool pairs = p.rep % 2 == 0 && lean_head_pairs();
#define NA_LB(T, DD, N)                                                                          \
    return d1 ? (pairs ? lean_bwd_run<T, DD, N, false, true, 2>(p, gq, gk, NA_LB_A(T, DD), s)     \
                       : lean_bwd_run<T, DD, N, false, true>(p, gq, gk, NA_LB_A(T, DD), s))       \
              : (pairs ? lean_bwd_run<T, DD, N, false, false, 2>(p, gq, gk, NA_LB_A(T, DD), s)    \
                       : lean_bwd_run<T, DD, N, false>(p, gq, gk, NA_LB_A(T, DD), s))
#define NA_LB3(T, DD, N)                                                              \
    return d1 ? lean_bwd_run<T, DD, N, false, true>(p, gq, gk, NA_LB_A(T, DD), s)     \
              : (d3 ? lean_bwd_run<T, DD, N, true>(p, gq, gk, NA_LB_A(T, DD), s)      \
                    : lean_bwd_run<T, DD, N, false>(p, gq, gk, NA_LB_A(T, DD), s))
#define NA_LB_N(T, DD, F)    \
    switch (nch) {           \
        case 1: F(T, DD, 1); \
        case 2: F(T, DD, 2); \
        case 3: F(T, DD, 3); \
        case 4: F(T, DD, 4); \
        default: F(T, DD, 5); \
    }
    if (dtype == NATTEN_BF16) {
        if (p.Dqk == 32) NA_LB_N(bf16, 32, NA_LB);
        NA_LB_N(bf16, 64, NA_LB);
    }
    if (dtype == NATTEN_F32) {
        if (p.Dqk == 32) NA_LB_N(float, 32, NA_LB3);
        NA_LB_N(float, 64, NA_LB3);
    }
    if (p.Dqk == 32) NA_LB_N(f16, 32, NA_LB);
    NA_LB_N(f16, 64, NA_LB);
#undef NA_LB_N
#undef NA_LB3
#undef NA_LB
#undef NA_LB_A
}

// Split ops, key side, on the 8x8 key tiles: eligibility beyond the general
// lean checks -- one head count, w's row strides even (one 2-byte phase of
// the w rows per (batch, head)), w's plane below 2^30 bytes, at least 6
// window entries (one 16-byte chunk per w row).
bool lean_wsum_key_eligible(const Prob& p, int dtype, int D, bool aligned, const Lay& lw, const Lay& lx,
                            const Lay& lo) {
    if (!lean_switch() || dtype == NATTEN_F32 || !aligned || !lean_static_lds_ok()) return false;
    if (p.Hq != p.Hkv || (D != 32 && D != 64)) return false;
    if (p.ax[0].len != 1 || p.ax[0].k != 1 || p.ax[1].len < 8) return false;
    if (p.kv < 6) return false;  // a w row's window is staged in 16-byte chunks
    for (int a = 1; a < 3; ++a) {
        const Axis& A = p.ax[a];
        if (A.st != 1 || A.k > 9 || A.len >= (1 << 15)) return false;
    }
    for (const Lay& l : {lx, lo, lw}) {
        if (l.s1 < 0 || l.s2 < 0 || l.b < 0 || l.h < 0) return false;
        const long long v = ((static_cast<long long>(p.ax[1].len) - 1) * l.s1 +
                             (static_cast<long long>(p.ax[2].len) - 1) * l.s2 + std::max(D, p.kv + 2)) * 2;
        if (v >= (1LL << 30)) return false;
    }
    return (lw.s1 & 1) == 0 && (lw.s2 & 1) == 0;
}

namespace {

template <typename T, int D, int MAXC>
hipError_t lean_wsum_key_run(const char* name, const Prob& p, const LeanGeo* g, const void* w, Lay lw, const void* x,
                             Lay lx, void* o, Lay lo, float mul, hipStream_t s) {
    LeanWsumKeyArgs<T> a{};
    a.rec = g->ptr;
    a.w = static_cast<const T*>(w);
    a.x = static_cast<const T*>(x);
    a.out = static_cast<T*>(o);
    a.lw = lean_lay(lw);
    a.lx = lean_lay(lx);
    a.lo = lean_lay(lo);
    a.heads = make_fastdiv(p.Hq);
    a.tiles = make_fastdiv(g->ntiles);
    a.nr = std::max(g->nst_max, 1);
    a.d1 = p.ax[1].dil;
    a.d2 = p.ax[2].dil;
    a.K1 = p.ax[1].k;
    a.K2 = p.ax[2].k;
    a.xbytes = plane_bytes(p, lx, D);
    const long long wb = ((static_cast<long long>(p.ax[1].len) - 1) * lw.s1 +
                          (static_cast<long long>(p.ax[2].len) - 1) * lw.s2 + p.kv + 1) * 2;
    a.wbytes = static_cast<uint32_t>((wb + 3) & ~3LL);
    a.mul = mul;
    a.p = p;
    // x rows (16 slots per union row), the w bands (the most chunks of any
    // tile), and room for the gather's masked reads, which end less than 16
    // entries past the last slot
    const size_t shm = kLdsPad + static_cast<size_t>(a.nr) * 16 * D * sizeof(T) +
                       (static_cast<size_t>(g->wchunks_max) + 2) * 16;
    if (shm > 160 * 1024) return hipErrorNotSupported;
    auto kern = k_lean_wsum_key<T, D, MAXC>;
    hipError_t e = allow_lds(kern, shm);
    if (e != hipSuccess) return e;
    const long long tasks = static_cast<long long>(p.B) * p.Hq * g->ntiles;
    NA_LAUNCH(name, kern, dim3(static_cast<unsigned>(tasks)), dim3(64 * kLeanWaves), shm, s, a);
    return hipGetLastError();
}

// Launch names of the key-side split ops on these kernels.
const char* lean_key_name(const char* name) {
    if (std::strcmp(name, "na_qk_bwd_k_mfma") == 0) return "na_qk_bwd_k_lean";
    if (std::strcmp(name, "na_av_bwd_v_mfma") == 0) return "na_av_bwd_v_lean";
    if (std::strcmp(name, "na_rpb_dk_mfma") == 0) return "na_rpb_dk_lean";
    if (std::strcmp(name, "na_rpb_dv_mfma") == 0) return "na_rpb_dv_lean";
    return name;
}

}  // namespace

hipError_t lean_wsum_key(const char* name, const Prob& p, int D, const void* w, Lay lw, const void* x, Lay lx,
                         void* o, Lay lo, float mul, int dtype, hipStream_t s) {
    const int nch = lean_nch(p.ax[1].k);
    if (static_cast<long long>(p.B) * p.Hq * 8192 >= (1LL << 31)) return hipErrorNotSupported;
    const LeanGeo* g = lean_geometry(p, 2, nch, s);
    if (!g || g->rows_max > 2 * (nch + 2)) return hipErrorNotSupported;
    name = lean_key_name(name);
#define NA_LW(T, DD, N) return lean_wsum_key_run<T, DD, N + 2>(name, p, g, w, lw, x, lx, o, lo, mul, s)
#define NA_LW_N(T, DD)          \
    switch (nch) {              \
        case 1: NA_LW(T, DD, 1); \
        case 2: NA_LW(T, DD, 2); \
        case 3: NA_LW(T, DD, 3); \
        case 4: NA_LW(T, DD, 4); \
        default: NA_LW(T, DD, 5); \
    }
    if (dtype == NATTEN_BF16) {
        if (D == 32) NA_LW_N(bf16, 32);
        NA_LW_N(bf16, 64);
    }
    if (D == 32) NA_LW_N(f16, 32);
    NA_LW_N(f16, 64);
#undef NA_LW_N
#undef NA_LW
}

}  // namespace na

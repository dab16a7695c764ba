// MFMA tile kernels (gfx950, bf16 / fp16, stride 1, head dim 32/64/128):
// forward, backward-dQ (query-centric) and backward-dK/dV (key-centric).
//
// Tiling.  With dilation d an axis splits into d residue classes; a query and
// every key of its window share the class, and inside a class the window is
// an undilated run of K positions (class coordinates j = (i - r) / d).  A
// workgroup owns a box of up to 64 queries (or keys) of one class triple
// (r0, r1, r2) and one (batch, head), with power-of-two extents T[a].  The
// union of their windows (or, for keys, of the queries attending them) is a
// box in class coordinates, staged one axis-0 plane ("slice") at a time in
// LDS: slot = a1 * rowlen + a2 for union row a1 and column a2, rowlen =
// 2^rowshift >= 8, the slot count padded to a multiple of 32.
//
// LDS holds each staged operand once, row-major X[slot][D], the 16-byte
// pieces of a row permuted by an XOR swizzle of the slot (spreads the MFMA
// operand reads over the banks).  Rows arrive straight from global memory
// through buffer loads into LDS (no register round trip); slots outside the
// union load out of the buffer's range and land as zeros.  Products that
// contract over slots read their operand transposed with ds_read_b64_tr_b16.
//
// Each wave owns 16 queries (keys) and walks the staged slots 32 at a time
// ("chunks") with v_mfma_f32_16x16x32: the score block is computed with the
// slots as MFMA rows, split over two 16-row blocks whose rows interleave so
// that every lane ends up holding 8 consecutive slots of one query (key) --
// exactly the B-operand layout of the following product over those slots.
//
// Masking.  A lane's 8 slots lie in one union row (rowlen >= 8), so the
// window test splits into a row test (one per lane and chunk) and a column
// test, which is fixed per lane for the whole tile when rows are at most 32
// slots.  Columns enter the score MFMA as its accumulator input (0 or -inf);
// a failed row test moves the lane's exponent offset to -inf, so its
// probabilities come out exactly 0.
//
// Softmax runs in the log2 domain in fp32; probabilities and score gradients
// enter the second product rounded to the input dtype, accumulators are fp32.
// Row sums of the forward come from the same rounded probabilities through
// one more MFMA against a block of ones.
//
// MFMA lane layout (16x16x32): A row = lane%16, B column = lane%16, both with
// k = 8*(lane/16) .. +7; C column = lane%16, rows 4*(lane/16) .. +3.
#include <algorithm>
#include <cstddef>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <type_traits>
#include <vector>

#include "na_tile.h"

namespace na {

namespace {

// ---------------------------------------------------------------------------
// Forward: out = softmax(scale q.k) v over each window, lse (natural log).
// Online softmax over groups of fwd_group<D>() chunks (one max reduction and
// one rescale per group).
// ---------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ ExactGlobal<T> exact_global(const GlobalKeys<T>& g, int b, int hk) {
    return ExactGlobal<T>{g.k + b * g.kb + hk * g.kh, g.v + b * g.vb + hk * g.vh, g.ks, g.vs, g.n};
}

template <typename T, int D, int LAY, bool WIDE, bool GLOBAL, bool VARLEN>
__device__ __forceinline__ void redo_fwd(const void* kargs, int wg, int wave, int col, int grp) {
    const FwdArgs<T>& A = *static_cast<const FwdArgs<T>*>(kargs);
    Prob pv;
    TileShape tv;
    if constexpr (VARLEN) varlen_view(A.p, A.ts, A.lens, wg, pv, tv);
    const Prob& P = VARLEN ? pv : A.p;
    const TileShape& TS = VARLEN ? tv : A.ts;
    const LayK &aq = A.lq, &ak = LAY == kLayOne ? aq : A.lk, &av = LAY == kLayOne ? aq : kVAtK<LAY> ? A.lk : A.lv;
    const LayK &ao = kOwnOut<LAY> ? A.lo : aq, &al = A.ll;
    int b, h0, h1, pos[3];
    if (!lane_position<false>(P, TS, wg, wave, col, b, h0, h1, pos)) return;
    ExactAxis x[3];
    for (int a = 0; a < 3; ++a) x[a] = exact_axis(P.ax[a], pos[a]);
    f32x4_t acc[D / 16];
#pragma unroll 1
    for (int h = h0; h < h1; ++h) {
        const int hk = kv_head(TS, h);
        float lse_v;
        if constexpr (GLOBAL)
            exact_forward_global<T, D>(P.scale, x, bh_ptr(A.q, aq, b, h) + vol_off(aq, pos), bh_ptr(A.k, ak, b, hk),
                                       strides3(ak), bh_ptr(A.v, av, b, hk), strides3(av),
                                       exact_global(A.gk, b, hk), grp, acc, lse_v);
        else
            exact_forward<T, D>(P.scale, x, bh_ptr(A.q, aq, b, h) + vol_off(aq, pos), bh_ptr(A.k, ak, b, hk),
                                strides3(ak), bh_ptr(A.v, av, b, hk), strides3(av), grp, acc, lse_v);
        store_rows<T, D>(bh_ptr(A.out, ao, b, h), vol_off(ao, pos), grp, acc, 1.f);
        if (grp == 0) bh_ptr(A.lse, al, b, h)[vol_off(al, pos)] = lse_v;
    }
}

// FLAT: every workgroup runs one (batch, head) over one slice (axis 0 of
// extent 1, one head per workgroup): the walk has one step, and its
// bookkeeping compiles away.
template <typename T, int D, int LAY, bool WIDE, bool GLOBAL, bool VARLEN = false, bool FLAT = false>
__global__ __launch_bounds__(64 * kMaxWaves) NA_OCCUPANCY(kKernFwd, D, WIDE) void k_fwd_mfma(FwdArgs<T> args) {
    const Prob& p = args.p;
    const TileShape& ts = args.ts;
    const int* __restrict__ geo = args.geo;
    const T* __restrict__ q = args.q;
    const T* __restrict__ kg = args.k;
    const T* __restrict__ vg = args.v;
    T* __restrict__ out = args.out;
    float* __restrict__ lse = args.lse;
    const LayK &lq = args.lq, &lk_in = args.lk, &lv_in = args.lv, &lo_in = args.lo, &ll = args.ll;
    const LayK& lk = LAY == kLayOne ? lq : lk_in;
    const LayK& lv = LAY == kLayOne ? lq : kVAtK<LAY> ? lk_in : lv_in;
    const LayK& lo = kOwnOut<LAY> ? lo_in : lq;
    unsigned char* smem = lds_base();
    constexpr bool KEY_SIDE = false;
    T* Ks = reinterpret_cast<T*>(smem);
    T* Vs = Ks + ts.slots * lds_dim<D>();
    const int lane = threadIdx.x & 63, col = lane & 15, grp = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: scalar loops
    Block blk;
    WaveGeo wg;
    if (!tile_geometry<KEY_SIDE, VARLEN>(p, ts, geo, wave, blk, wg, args.lens)) return;
    const StageMap sm = stage_map<T, D>(p, ts, lk, lv, lane);
    Walk w;
    walk_start(blk, w);
    {
        const int p0 = slice_pos(p, blk, 0), hk = kv_head(ts, w.h);
        stage_pair<T, D>(p, blk, ts, sm, plane_of(kg, lk, w.b, hk, p0), lk, Ks, plane_of(vg, lv, w.b, hk, p0), lv,
                         Vs, wave);
    }
    const Lane ln = lane_item(p, ts, blk, wave, col, false);
    f32x4_t cb[2];
    if constexpr (!WIDE) column_bias(ln, ts.rowshift, 0, grp, cb);
    const uint4 ones = make_uint4(Mma<T>::kOnes, Mma<T>::kOnes, Mma<T>::kOnes, Mma<T>::kOnes);
    const float sc2 = p.scale * kLog2e;

    uint4 qf[D / 32];
    f32x4_t acc[D / 16], lacc;
    float m;
    bool more = true, fresh = true, redo = false;
    while (more) {
        const int b = w.b, h = w.h, u0 = w.u0;
        if (fresh) {
            load_frags<T, D>(bh_ptr(q, lq, b, h), vol_off(lq, ln.pos), ln.valid, grp, qf);
#pragma unroll
            for (int db = 0; db < D / 16; ++db) acc[db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
            lacc = f32x4_t{0.f, 0.f, 0.f, 0.f};
            m = -INFINITY;  // running max, log2 domain (scores times scale * log2 e)
        }
        wait_loads();
        __syncthreads();
        if (wg.any && u0 >= wg.lo[0] && u0 <= wg.hi[0]) {
            const bool in0 = u0 >= ln.lo[0] && u0 <= ln.hi[0];
            const auto chunks = [&](auto) {
                constexpr int FG = fwd_group<D>();
                for (int c = wg.c0; c <= wg.c1; c += FG) {
                    const int n = min(FG, wg.c1 - c + 1);
                    f32x4_t s[FG][2];
                    bool rv[FG];
                    float cm = -INFINITY;
#pragma unroll
                    for (int g = 0; g < FG; ++g) {
                        if (g < n) {
                            if constexpr (!WIDE) {
                                score_chunk<T, D>(Ks, c + g, col, grp, qf, cb, s[g]);
                            } else {
                                f32x4_t bias[2];
                                column_bias(ln, ts.rowshift, c + g, grp, bias);
                                score_chunk<T, D>(Ks, c + g, col, grp, qf, bias, s[g]);
                            }
                            rv[g] = row_ok(ln, ts.rowshift, in0, c + g, grp);
                            cm = fmaxp(cm, rv[g] ? max8(s[g]) : -INFINITY);
                        }
                    }
                    const float mnew = fmaxp(m, max_rows(cm) * sc2);
                    const float mref = mnew == -INFINITY ? 0.f : mnew;
                    const float corr = __builtin_amdgcn_exp2f(m - mref);
                    m = mnew;
                    lacc *= corr;
#pragma unroll
                    for (int db = 0; db < D / 16; ++db) acc[db] *= corr;
#pragma unroll
                    for (int g = 0; g < FG; ++g) {
                        if (g < n) {
                            const float off = rv[g] ? -mref : -INFINITY;
#pragma unroll
                            for (int bb = 0; bb < 2; ++bb)
#pragma unroll
                                for (int i = 0; i < 4; ++i)
                                    s[g][bb][i] = __builtin_amdgcn_exp2f(fmaf(s[g][bb][i], sc2, off));
                            const uint4 pk = pack8<T>(s[g]);
                            accumulate_chunk<T, D>(Vs, c + g, lane, pk, acc);
                            lacc = Mma<T>::run(ones, pk, lacc);
                        }
                    }
                }
            };
            chunks(std::integral_constant<bool, WIDE>{});
        }
        if constexpr (FLAT) {
            more = false;
        } else {
            more = walk_next(blk, w, fresh);
            __syncthreads();  // the slice is no longer read
        }
        if constexpr (GLOBAL) {
            // the finished head's global keys, 32 at a time, continue the
            // same online softmax (every key valid up to n)
            if (fresh || !more) {
                const GlobalKeys<T>& g = args.gk;
                const int hk = kv_head(ts, h);
                const T* gkb = g.k + b * g.kb + hk * g.kh;
                const T* gvb = g.v + b * g.vb + hk * g.vh;
                T* Xk = Vs + ts.slots * lds_dim<D>();
                T* Xv = Xk + 32 * lds_dim<D>();
                for (int j0 = 0; j0 < g.n; j0 += 32) {
                    stage_global<T, D>(gkb, g.ks, gvb, g.vs, j0, g.n, Xk, Xv, wave, ts.waves, lane);
                    wait_loads();
                    __syncthreads();
                    f32x4_t xb[2], s[2];
                    global_bias(j0, g.n, grp, xb);
                    score_chunk<T, D>(Xk, 0, col, grp, qf, xb, s);
                    const float mnew = fmaxp(m, max_rows(max8(s)) * sc2);
                    const float mref = mnew == -INFINITY ? 0.f : mnew;
                    const float corr = __builtin_amdgcn_exp2f(m - mref);
                    m = mnew;
                    lacc *= corr;
#pragma unroll
                    for (int db = 0; db < D / 16; ++db) acc[db] *= corr;
#pragma unroll
                    for (int bb = 0; bb < 2; ++bb)
#pragma unroll
                        for (int i = 0; i < 4; ++i) s[bb][i] = __builtin_amdgcn_exp2f(fmaf(s[bb][i], sc2, -mref));
                    const uint4 pk = pack8<T>(s);
                    accumulate_chunk<T, D>(Xv, 0, lane, pk, acc);
                    lacc = Mma<T>::run(ones, pk, lacc);
                    __syncthreads();  // the global rows are no longer read
                }
            }
        }
        if (more && !same_rows(ts, blk, h, w.h)) {
            const int p0 = slice_pos(p, blk, w.u0), hk = kv_head(ts, w.h);
            stage_pair<T, D>(p, blk, ts, sm, plane_of(kg, lk, w.b, hk, p0), lk, Ks, plane_of(vg, lv, w.b, hk, p0),
                             lv, Vs, wave);
        }
        if (fresh || !more) {
            redo = redo || (item_nonfinite(lane_sum(acc, lacc[0])) && ln.valid);
            if (ln.valid) {
                const float lsum = lacc[0];
                store_rows<T, D>(bh_ptr(out, lo, b, h), vol_off(lo, ln.pos), grp, acc, 1.f / lsum);
                if (grp == 0) bh_ptr(lse, ll, b, h)[vol_off(ll, ln.pos)] = (m + __log2f(lsum)) * kLn2;
            }
        }
    }
    // items whose tile result was not finite: exact recomputation (the
    // walk's state is dead here, so this costs the loop no registers)
    if (redo) redo_fwd<T, D, LAY, WIDE, GLOBAL, VARLEN>(kernargs(), xcd_block(blockIdx.x, gridDim.x), wave, col, grp);
}

// ---------------------------------------------------------------------------
// Backward, query side: delta = dO . O - dlse (written for the key side) and
// dq = scale * sum_k P (dP - delta) k, with P = exp(scale q.k - lse) and
// dP = dO . v.  The dP product starts from -delta.
// ---------------------------------------------------------------------------
template <typename T, int D, int LAY, bool WIDE, bool GLOBAL, bool VARLEN>
__device__ __forceinline__ void redo_bwd_q(const void* kargs, int wg, int wave, int col, int grp) {
    const BwdQArgs<T>& A = *static_cast<const BwdQArgs<T>*>(kargs);
    Prob pv;
    TileShape tv;
    if constexpr (VARLEN) varlen_view(A.p, A.ts, A.lens, wg, pv, tv);
    const Prob& P = VARLEN ? pv : A.p;
    const TileShape& TS = VARLEN ? tv : A.ts;
    const LayK &aq = A.lq, &ak = LAY == kLayOne ? aq : A.lk, &av = LAY == kLayOne ? aq : kVAtK<LAY> ? A.lk : A.lv;
    const LayK &ao = kOwnOut<LAY> ? A.lo : aq, &ado = LAY == kLayGeneral ? A.ldo : ao;
    const LayK &adq = LAY == kLayGeneral ? A.ldq : ao, &al = A.ll, &adl = LAY == kLayGeneral ? A.ldl : al;
    int b, h0, h1, pos[3];
    if (!lane_position<false>(P, TS, wg, wave, col, b, h0, h1, pos)) return;
    ExactAxis x[3];
    for (int a = 0; a < 3; ++a) x[a] = exact_axis(P.ax[a], pos[a]);
    f32x4_t acc[D / 16];
#pragma unroll 1
    for (int h = h0; h < h1; ++h) {
        const int hk = kv_head(TS, h);
        const T* do_row = bh_ptr(A.dout, ado, b, h) + vol_off(ado, pos);
        float di = exact_dot<T, D>(do_row, bh_ptr(A.o, ao, b, h) + vol_off(ao, pos));
        if (A.dlse) di -= bh_ptr(A.dlse, adl, b, h)[vol_off(adl, pos)];
        if constexpr (GLOBAL)
            exact_backward_q_global<T, D>(P.scale, x, bh_ptr(A.q, aq, b, h) + vol_off(aq, pos), do_row,
                                          bh_ptr(A.lse, al, b, h)[vol_off(al, pos)], di, bh_ptr(A.k, ak, b, hk),
                                          strides3(ak), bh_ptr(A.v, av, b, hk), strides3(av),
                                          exact_global(A.gk, b, hk), grp, acc);
        else
            exact_backward_q<T, D>(P.scale, x, bh_ptr(A.q, aq, b, h) + vol_off(aq, pos), do_row,
                                   bh_ptr(A.lse, al, b, h)[vol_off(al, pos)], di, bh_ptr(A.k, ak, b, hk),
                                   strides3(ak), bh_ptr(A.v, av, b, hk), strides3(av), grp, acc);
        store_rows<T, D>(bh_ptr(A.dq, adq, b, h), vol_off(adq, pos), grp, acc, P.scale);
    }
}

// FLAT as for k_fwd_mfma.  PDP: one slice per head (axis 0 of extent 1:
// 1-D and 2-D problems) and no global keys; delta from the kernel's own
// products (the sum over the window of P dP, which equals dO . O) in a first
// pass over the chunks, so O is not read, and dS = P (dP - delta) with dP
// from a zero accumulator (the 2-D tile kernel's arithmetic, bit for bit).
// Otherwise delta = dO . O from the rows and dP is accumulated from -delta.
template <typename T, int D, int LAY, bool WIDE, bool GLOBAL, bool VARLEN = false, bool FLAT = false, bool PDP = false>
__global__ __launch_bounds__(64 * kMaxWaves) NA_OCCUPANCY(kKernBwdQ, D, WIDE) void k_bwd_q_mfma(BwdQArgs<T> args) {
    static_assert(!PDP || (!GLOBAL && !VARLEN), "delta from P dP: one slice per head, no global keys");
    const Prob& p = args.p;
    const TileShape& ts = args.ts;
    const int* __restrict__ geo = args.geo;
    const T* __restrict__ q = args.q;
    const T* __restrict__ kg = args.k;
    const T* __restrict__ vg = args.v;
    const T* __restrict__ o = args.o;
    const T* __restrict__ dout = args.dout;
    const float* __restrict__ lse = args.lse;
    const float* __restrict__ dlse = args.dlse;
    T* __restrict__ dq = args.dq;
    float* __restrict__ delta = args.delta;
    const LayK &lq = args.lq, &lk_in = args.lk, &lv_in = args.lv, &lo_in = args.lo, &ldo_in = args.ldo;
    const LayK &ll = args.ll, &ldl_in = args.ldl, &ldq_in = args.ldq, &lde_in = args.lde;
    const LayK& lk = LAY == kLayOne ? lq : lk_in;
    const LayK& lv = LAY == kLayOne ? lq : kVAtK<LAY> ? lk_in : lv_in;
    const LayK& lo = kOwnOut<LAY> ? lo_in : lq;
    const LayK& ldo = LAY == kLayGeneral ? ldo_in : lo;
    const LayK& ldq = LAY == kLayGeneral ? ldq_in : lo;
    const LayK& ldl = LAY == kLayGeneral ? ldl_in : ll;
    const LayK& lde = LAY == kLayGeneral ? lde_in : ll;
    unsigned char* smem = lds_base();
    constexpr bool KEY_SIDE = false;
    T* Ks = reinterpret_cast<T*>(smem);
    T* Vs = Ks + ts.slots * lds_dim<D>();
    const int lane = threadIdx.x & 63, col = lane & 15, grp = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: scalar loops
    Block blk;
    WaveGeo wg;
    if (!tile_geometry<KEY_SIDE, VARLEN>(p, ts, geo, wave, blk, wg, args.lens)) return;
    const StageMap sm = stage_map<T, D>(p, ts, lk, lv, lane);
    Walk w;
    walk_start(blk, w);
    {
        const int p0 = slice_pos(p, blk, 0), hk = kv_head(ts, w.h);
        stage_pair<T, D>(p, blk, ts, sm, plane_of(kg, lk, w.b, hk, p0), lk, Ks, plane_of(vg, lv, w.b, hk, p0), lv,
                         Vs, wave);
    }
    const Lane ln = lane_item(p, ts, blk, wave, col, false);
    const float sc2 = p.scale * kLog2e;
    f32x4_t cb[2];
    if constexpr (!WIDE) column_bias(ln, ts.rowshift, 0, grp, cb);

    uint4 qf[D / 32], gf[D / 32];
    f32x4_t acc[D / 16], nd[2];
    float L2, dsub = 0.f;
    bool more = true, fresh = true, redo = false;
    while (more) {
        const int b = w.b, h = w.h, u0 = w.u0;
        if (fresh) {
            load_frags<T, D>(bh_ptr(q, lq, b, h), vol_off(lq, ln.pos), ln.valid, grp, qf);
            load_frags<T, D>(bh_ptr(dout, ldo, b, h), vol_off(ldo, ln.pos), ln.valid, grp, gf);
            L2 = ln.valid ? bh_ptr(lse, ll, b, h)[vol_off(ll, ln.pos)] * kLog2e : 0.f;
            if constexpr (!PDP) {
                uint4 of[D / 32];
                load_frags<T, D>(bh_ptr(o, lo, b, h), vol_off(lo, ln.pos), ln.valid, grp, of);
                // delta from this lane's 8 head dims per 32, summed over the 4 lane rows
                float di = 0.f;
#pragma unroll
                for (int ks = 0; ks < D / 32; ++ks) di = dot8<T>(gf[ks], of[ks], di);
                di = sum_rows(di);
                if (dlse && ln.valid) di -= bh_ptr(dlse, ldl, b, h)[vol_off(ldl, ln.pos)];
                if (ln.valid && grp == 0) bh_ptr(delta, lde, b, h)[vol_off(lde, ln.pos)] = di;
                nd[0] = nd[1] = f32x4_t{-di, -di, -di, -di};
            }
#pragma unroll
            for (int db = 0; db < D / 16; ++db) acc[db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        }
        wait_loads();
        __syncthreads();
        if (PDP && fresh) {
            float part = 0.f;
            if (wg.any && u0 >= wg.lo[0] && u0 <= wg.hi[0]) {
                const bool in0 = u0 >= ln.lo[0] && u0 <= ln.hi[0];
                const f32x4_t zero[2] = {f32x4_t{0.f, 0.f, 0.f, 0.f}, f32x4_t{0.f, 0.f, 0.f, 0.f}};
                for (int c = wg.c0; c <= wg.c1; ++c) {
                    f32x4_t s[2], dp[2];
                    if constexpr (!WIDE) {
                        score_chunk<T, D>(Ks, c, col, grp, qf, cb, s);
                    } else {
                        f32x4_t bias[2];
                        column_bias(ln, ts.rowshift, c, grp, bias);
                        score_chunk<T, D>(Ks, c, col, grp, qf, bias, s);
                    }
                    score_chunk<T, D>(Vs, c, col, grp, gf, zero, dp);
                    part = delta_part(s, dp, sc2, row_ok(ln, ts.rowshift, in0, c, grp) ? -L2 : -INFINITY, part);
                }
            }
            float di = sum_rows(part);
            if (dlse && ln.valid) di -= bh_ptr(dlse, ldl, b, h)[vol_off(ldl, ln.pos)];
            // a non-finite operand outside the window can reach the sum
            // through a masked slot: dO . O from the rows there
            if (ln.valid && !(__builtin_fabsf(di) <= __FLT_MAX__)) {
                di = exact_dot<T, D>(bh_ptr(dout, ldo, b, h) + vol_off(ldo, ln.pos),
                                     bh_ptr(o, lo, b, h) + vol_off(lo, ln.pos));
                if (dlse) di -= bh_ptr(dlse, ldl, b, h)[vol_off(ldl, ln.pos)];
            }
            if (ln.valid && grp == 0) bh_ptr(delta, lde, b, h)[vol_off(lde, ln.pos)] = di;
            nd[0] = nd[1] = f32x4_t{0.f, 0.f, 0.f, 0.f};
            dsub = di;
        }
        if (wg.any && u0 >= wg.lo[0] && u0 <= wg.hi[0]) {
            const bool in0 = u0 >= ln.lo[0] && u0 <= ln.hi[0];
            const auto chunks = [&](auto) {
                for (int c = wg.c0; c <= wg.c1; ++c) {
                    f32x4_t s[2], dp[2];
                    if constexpr (!WIDE) {
                        score_chunk<T, D>(Ks, c, col, grp, qf, cb, s);
                    } else {
                        f32x4_t bias[2];
                        column_bias(ln, ts.rowshift, c, grp, bias);
                        score_chunk<T, D>(Ks, c, col, grp, qf, bias, s);
                    }
                    score_chunk<T, D>(Vs, c, col, grp, gf, nd, dp);
                    const float off = row_ok(ln, ts.rowshift, in0, c, grp) ? -L2 : -INFINITY;
#pragma unroll
                    for (int bb = 0; bb < 2; ++bb)
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const float e = __builtin_amdgcn_exp2f(fmaf(s[bb][i], sc2, off));
                            if constexpr (PDP) s[bb][i] = e * (dp[bb][i] - dsub);
                            else s[bb][i] = e * dp[bb][i];
                        }
                    accumulate_chunk<T, D>(Ks, c, lane, pack8<T>(s), acc);
                }
            };
            chunks(std::integral_constant<bool, WIDE>{});
        }
        if constexpr (FLAT) {
            more = false;
        } else {
            more = walk_next(blk, w, fresh);
            __syncthreads();  // the slice is no longer read
        }
        if constexpr (GLOBAL) {
            // the finished head's global keys, 32 at a time
            if (fresh || !more) {
                const GlobalKeys<T>& g = args.gk;
                const int hk = kv_head(ts, h);
                const T* gkb = g.k + b * g.kb + hk * g.kh;
                const T* gvb = g.v + b * g.vb + hk * g.vh;
                T* Xk = Vs + ts.slots * lds_dim<D>();
                T* Xv = Xk + 32 * lds_dim<D>();
                for (int j0 = 0; j0 < g.n; j0 += 32) {
                    stage_global<T, D>(gkb, g.ks, gvb, g.vs, j0, g.n, Xk, Xv, wave, ts.waves, lane);
                    wait_loads();
                    __syncthreads();
                    f32x4_t xb[2], s[2], dp[2];
                    global_bias(j0, g.n, grp, xb);
                    score_chunk<T, D>(Xk, 0, col, grp, qf, xb, s);
                    score_chunk<T, D>(Xv, 0, col, grp, gf, nd, dp);
#pragma unroll
                    for (int bb = 0; bb < 2; ++bb)
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            s[bb][i] = __builtin_amdgcn_exp2f(fmaf(s[bb][i], sc2, -L2)) * dp[bb][i];
                    accumulate_chunk<T, D>(Xk, 0, lane, pack8<T>(s), acc);
                    __syncthreads();  // the global rows are no longer read
                }
            }
        }
        if (more && !same_rows(ts, blk, h, w.h)) {
            const int p0 = slice_pos(p, blk, w.u0), hk = kv_head(ts, w.h);
            stage_pair<T, D>(p, blk, ts, sm, plane_of(kg, lk, w.b, hk, p0), lk, Ks, plane_of(vg, lv, w.b, hk, p0),
                             lv, Vs, wave);
        }
        if (fresh || !more) {
            redo = redo || (item_nonfinite(lane_sum(acc, 0.f)) && ln.valid);
            if (ln.valid) store_rows<T, D>(bh_ptr(dq, ldq, b, h), vol_off(ldq, ln.pos), grp, acc, p.scale);
        }
    }
    if (redo) redo_bwd_q<T, D, LAY, WIDE, GLOBAL, VARLEN>(kernargs(), xcd_block(blockIdx.x, gridDim.x), wave, col, grp);
}

// ---------------------------------------------------------------------------
// Backward, key side: for each key/value position, over every query (of each
// q head in the GQA group) whose window holds it:
//   dv = sum P dO,   dk = scale * sum P (dP - delta) q.
// Per staged slot: -lse * log2 e and -delta (fp32); 8 further -inf entries
// serve lanes whose row test fails.  Runs over (batch, kv head) pairs; the
// walk's slices cover the GQA group's q heads one after the other.
// ---------------------------------------------------------------------------
// One slice's per-slot scalars in two steps, so that their loads travel with
// the slice's staging loads instead of after them: scalar_loads issues the
// loads of slot threadIdx.x (for slots outside the union an unconditional
// load of a valid position, the union's first, so that both loads are in
// flight together), scalar_store writes the values once the loads have
// landed and handles the slots past the workgroup's threads (unions of more
// slots than threads) with ordinary dependent loads.
struct SlotScalars {
    float nl, nd;
};

__device__ __forceinline__ void slot_position(const Prob& p, const Block& k, const TileShape& ts, int s, bool& in,
                                              int& p1, int& p2) {
    const int a1 = s >> ts.rowshift, a2 = s & ((1 << ts.rowshift) - 1);
    in = s < ts.slots && a1 < k.U[1] && a2 < k.U[2];
    p1 = k.r[1] + (k.lo[1] + (in ? a1 : 0)) * p.ax[1].dil;
    p2 = k.r[2] + (k.lo[2] + (in ? a2 : 0)) * p.ax[2].dil;
}

__device__ __forceinline__ SlotScalars scalar_loads(const Prob& p, const Block& k, const TileShape& ts, int b, int h,
                                                    int p0, const float* __restrict__ lse, const LayK& ll,
                                                    const float* __restrict__ delta, const LayK& lde) {
    bool in;
    int p1, p2;
    slot_position(p, k, ts, threadIdx.x, in, p1, p2);
    const float l = (bh_ptr(lse, ll, b, h) + p0 * ll.s0)[p1 * ll.s1 + p2 * ll.s2];
    const float d = (bh_ptr(delta, lde, b, h) + p0 * lde.s0)[p1 * lde.s1 + p2 * lde.s2];
    return SlotScalars{in ? -l * kLog2e : 0.f, in ? -d : 0.f};
}

__device__ __forceinline__ void scalar_store(const Prob& p, const Block& k, const TileShape& ts, int b, int h, int p0,
                                             const float* __restrict__ lse, const LayK& ll,
                                             const float* __restrict__ delta, const LayK& lde, SlotScalars sc,
                                             float* NL, float* ND) {
    if (static_cast<int>(threadIdx.x) < ts.slots) {
        NL[threadIdx.x] = sc.nl;
        ND[threadIdx.x] = sc.nd;
    }
    for (int s = threadIdx.x + blockDim.x; s < ts.slots; s += blockDim.x) {
        bool in;
        int p1, p2;
        slot_position(p, k, ts, s, in, p1, p2);
        float nl = 0.f, nd = 0.f;
        if (in) {
            nl = -(bh_ptr(lse, ll, b, h) + p0 * ll.s0)[p1 * ll.s1 + p2 * ll.s2] * kLog2e;
            nd = -(bh_ptr(delta, lde, b, h) + p0 * lde.s0)[p1 * lde.s1 + p2 * lde.s2];
        }
        NL[s] = nl;
        ND[s] = nd;
    }
}

template <typename T, int D, int LAY, bool WIDE, bool VARLEN>
__device__ __forceinline__ void redo_bwd_kv(const void* kargs, int wg, int wave, int col, int grp) {
    const BwdKvArgs<T>& A = *static_cast<const BwdKvArgs<T>*>(kargs);
    Prob pv;
    TileShape tv;
    if constexpr (VARLEN) varlen_view(A.p, A.ts, A.lens, wg, pv, tv);
    const Prob& P = VARLEN ? pv : A.p;
    const TileShape& TS = VARLEN ? tv : A.ts;
    const LayK &aq = A.lq, &ak = LAY == kLayOne ? aq : A.lk, &av = LAY == kLayOne ? aq : kVAtK<LAY> ? A.lk : A.lv;
    const LayK& adk = LAY == kLayOne ? aq : LAY == kLayTwo ? A.lk : A.ldk;
    const LayK& adv = LAY == kLayOne ? aq : LAY == kLayTwo ? A.lk : LAY == kLayFour ? A.ldk : A.ldv;
    const LayK &ado = kOwnOut<LAY> ? A.ldo : aq, &al = A.ll, &ade = LAY == kLayGeneral ? A.lde : al;
    int b, h0, h1, pos[3];
    if (!lane_position<true>(P, TS, wg, wave, col, b, h0, h1, pos)) return;
    ExactAxis x[3];
    for (int a = 0; a < 3; ++a) x[a] = exact_axis(P.ax[a], pos[a]);
    f32x4_t g[D / 16];
    const int rep = P.rep;
#pragma unroll 1
    for (int hk = h0; hk < h1; ++hk) {
        const T* k_row = bh_ptr(A.k, ak, b, hk) + vol_off(ak, pos);
        const T* v_row = bh_ptr(A.v, av, b, hk) + vol_off(av, pos);
        // dv, then dk, each summed over the q heads of the group
        exact_zero(g);
#pragma unroll 1
        for (int h = hk * rep; h < (hk + 1) * rep; ++h)
            exact_backward_kv<T, D, true>(P.scale, x, k_row, v_row, bh_ptr(A.q, aq, b, h), strides3(aq),
                                          bh_ptr(A.dout, ado, b, h), strides3(ado), bh_ptr(A.lse, al, b, h),
                                          strides3(al), bh_ptr(A.delta, ade, b, h), strides3(ade), grp, g);
        store_rows<T, D>(bh_ptr(A.dv, adv, b, hk), vol_off(adv, pos), grp, g, 1.f);
        exact_zero(g);
#pragma unroll 1
        for (int h = hk * rep; h < (hk + 1) * rep; ++h)
            exact_backward_kv<T, D, false>(P.scale, x, k_row, v_row, bh_ptr(A.q, aq, b, h), strides3(aq),
                                           bh_ptr(A.dout, ado, b, h), strides3(ado), bh_ptr(A.lse, al, b, h),
                                           strides3(al), bh_ptr(A.delta, ade, b, h), strides3(ade), grp, g);
        store_rows<T, D>(bh_ptr(A.dk, adk, b, hk), vol_off(adk, pos), grp, g, P.scale);
    }
}

// FLAT: one slice and one (batch, kv head) per workgroup with one q head
// per kv head (axis 0 of extent 1, no GQA): the walk has one step.
template <typename T, int D, int LAY, bool WIDE, bool VARLEN = false, bool FLAT = false>
__global__ __launch_bounds__(64 * kMaxWaves) NA_OCCUPANCY(kKernBwdKV, D, WIDE) void k_bwd_kv_mfma(BwdKvArgs<T> args) {
    const Prob& p = args.p;
    const TileShape& ts = args.ts;
    const int* __restrict__ geo = args.geo;
    const T* __restrict__ q = args.q;
    const T* __restrict__ kg = args.k;
    const T* __restrict__ vg = args.v;
    const T* __restrict__ dout = args.dout;
    const float* __restrict__ lse = args.lse;
    const float* __restrict__ delta = args.delta;
    T* __restrict__ dk = args.dk;
    T* __restrict__ dv = args.dv;
    const LayK &lq = args.lq, &lk_in = args.lk, &lv_in = args.lv, &ldo_in = args.ldo, &ll = args.ll;
    const LayK &lde_in = args.lde, &ldk_in = args.ldk, &ldv_in = args.ldv;
    const LayK& lk = LAY == kLayOne ? lq : lk_in;
    const LayK& lv = LAY == kLayOne ? lq : kVAtK<LAY> ? lk_in : lv_in;
    const LayK& ldk = LAY == kLayOne ? lq : LAY == kLayTwo ? lk_in : ldk_in;
    const LayK& ldv = LAY == kLayOne ? lq : LAY == kLayTwo ? lk_in : LAY == kLayFour ? ldk_in : ldv_in;
    const LayK& ldo = kOwnOut<LAY> ? ldo_in : lq;
    const LayK& lde = LAY == kLayGeneral ? lde_in : ll;
    unsigned char* smem = lds_base();
    constexpr bool KEY_SIDE = true;
    const int slots = ts.slots;
    T* Qs = reinterpret_cast<T*>(smem);
    T* Gs = Qs + slots * lds_dim<D>();
    float* NL = reinterpret_cast<float*>(Gs + slots * lds_dim<D>());  // slots + 8
    float* ND = NL + slots + 8;                            // slots
    const int lane = threadIdx.x & 63, col = lane & 15, grp = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: scalar loops
    Block blk;
    WaveGeo wg;
    if (!tile_geometry<KEY_SIDE, VARLEN>(p, ts, geo, wave, blk, wg, args.lens)) return;
    const Lane ln = lane_item(p, ts, blk, wave, col, true);
    if (empty_union(blk)) {
        f32x4_t z[D / 16];
        exact_zero(z);
        if (ln.valid)
            for (int hk = blk.h0; hk < blk.h1; ++hk) {
                store_rows<T, D>(bh_ptr(dk, ldk, blk.b, hk), vol_off(ldk, ln.pos), grp, z, 1.f);
                store_rows<T, D>(bh_ptr(dv, ldv, blk.b, hk), vol_off(ldv, ln.pos), grp, z, 1.f);
            }
        return;
    }
    const int rep = static_cast<int>(ts.rep.d);
    const StageMap sm = stage_map<T, D>(p, ts, lq, ldo, lane);
    // the walk runs over (batch, kv head, q head of the group, slice): its
    // slice counter spans rep * U0
    Walk w;
    walk_start(blk, w);
    const int nsl = rep * blk.U[0];
    // the staged slice's head and axis-0 position (its scalars are stored
    // after the wait that precedes the slice's chunks)
    int st_h = w.h * rep, st_p0 = slice_pos(p, blk, 0);
    SlotScalars sc = scalar_loads(p, blk, ts, w.b, st_h, st_p0, lse, ll, delta, lde);
    stage_pair<T, D>(p, blk, ts, sm, plane_of(q, lq, w.b, st_h, st_p0), lq, Qs, plane_of(dout, ldo, w.b, st_h, st_p0),
                     ldo, Gs, wave);
    if (threadIdx.x < 8) NL[slots + threadIdx.x] = -INFINITY;
    const float sc2 = p.scale * kLog2e;
    f32x4_t cb[2];
    if constexpr (!WIDE) column_bias(ln, ts.rowshift, 0, grp, cb);

    uint4 kf[D / 32], vf[D / 32];
    f32x4_t gk[D / 16], gv[D / 16];
    bool more = true, fresh = true, redo = false;
    int sl = 0;  // slice index within the pair: q head (sl / U0) and axis-0 slice (sl % U0)
    while (more) {
        const int b = w.b, hk = w.h, u0 = sl % blk.U[0];
        if (fresh) {
            load_frags<T, D>(bh_ptr(kg, lk, b, hk), vol_off(lk, ln.pos), ln.valid, grp, kf);
            load_frags<T, D>(bh_ptr(vg, lv, b, hk), vol_off(lv, ln.pos), ln.valid, grp, vf);
#pragma unroll
            for (int db = 0; db < D / 16; ++db) {
                gk[db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
                gv[db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
            }
        }
        wait_loads();
        scalar_store(p, blk, ts, b, st_h, st_p0, lse, ll, delta, lde, sc, NL, ND);
        lds_publish_barrier();  // staged rows and the slice's -lse / -delta
        if (wg.any && u0 >= wg.lo[0] && u0 <= wg.hi[0]) {
            const bool in0 = u0 >= ln.lo[0] && u0 <= ln.hi[0];
            const auto chunks = [&](auto) {
                for (int c = wg.c0; c <= wg.c1; ++c) {
                    const int s0 = 32 * c + 8 * grp;
                    const f32x4_t ndc[2] = {*reinterpret_cast<const f32x4_t*>(ND + s0),
                                            *reinterpret_cast<const f32x4_t*>(ND + s0 + 4)};
                    f32x4_t s[2], dp[2];
                    if constexpr (!WIDE) {
                        score_chunk<T, D>(Qs, c, col, grp, kf, cb, s);
                    } else {
                        f32x4_t bias[2];
                        column_bias(ln, ts.rowshift, c, grp, bias);
                        score_chunk<T, D>(Qs, c, col, grp, kf, bias, s);
                    }
                    score_chunk<T, D>(Gs, c, col, grp, vf, ndc, dp);
                    const float* nlp = row_ok(ln, ts.rowshift, in0, c, grp) ? NL + s0 : NL + slots;
                    const f32x4_t nl[2] = {*reinterpret_cast<const f32x4_t*>(nlp),
                                           *reinterpret_cast<const f32x4_t*>(nlp + 4)};
#pragma unroll
                    for (int bb = 0; bb < 2; ++bb)
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            s[bb][i] = __builtin_amdgcn_exp2f(fmaf(s[bb][i], sc2, nl[bb][i]));
                            dp[bb][i] *= s[bb][i];
                        }
                    accumulate_chunk<T, D>(Gs, c, lane, pack8<T>(s), gv);
                    accumulate_chunk<T, D>(Qs, c, lane, pack8<T>(dp), gk);
                }
            };
            chunks(std::integral_constant<bool, WIDE>{});
        }
        // next slice: within the pair (q heads x axis-0 slices), else the next pair
        if constexpr (FLAT) {
            more = false;
        } else {
            fresh = false;
            if (++sl >= nsl) {
                sl = 0;
                more = ++w.h < blk.h1;
                fresh = true;
            }
        }
        // a finished pair's results go out first, so that its accumulators
        // are dead while the next slice's loads are issued
        if (fresh) {
            redo = redo || (item_nonfinite(lane_sum(gk, lane_sum(gv, 0.f))) && ln.valid);
            if (ln.valid) {
                store_rows<T, D>(bh_ptr(dk, ldk, b, hk), vol_off(ldk, ln.pos), grp, gk, p.scale);
                store_rows<T, D>(bh_ptr(dv, ldv, b, hk), vol_off(ldv, ln.pos), grp, gv, 1.f);
            }
        }
        if constexpr (!FLAT) __syncthreads();  // the slice is no longer read
        if (more) {
            st_h = w.h * rep + sl / blk.U[0];
            st_p0 = slice_pos(p, blk, sl % blk.U[0]);
            sc = scalar_loads(p, blk, ts, w.b, st_h, st_p0, lse, ll, delta, lde);
            stage_pair<T, D>(p, blk, ts, sm, plane_of(q, lq, w.b, st_h, st_p0), lq, Qs,
                             plane_of(dout, ldo, w.b, st_h, st_p0), ldo, Gs, wave);
        }
    }
    if (redo) redo_bwd_kv<T, D, LAY, WIDE, VARLEN>(kernargs(), xcd_block(blockIdx.x, gridDim.x), wave, col, grp);
}

// ---------------------------------------------------------------------------
// Split products, query side (the split QK / AV ops and the query side of
// their backward), over the union the forward stages:
//   k_dot_mfma:  out[q][e] = mul * (a[q] . x[nbr(q, e)]) for each valid
//                neighbour e, `fill` for the others (QK: a = q, x = k,
//                fill -inf; AV backward dattn: a = dO, x = v, fill 0);
//   k_wsum_mfma: out[q] = mul * sum over valid e of w[q][e] x[nbr(q, e)]
//                (AV: w = attn, x = v; QK backward dq: w = dattn, x = k).
//
// Rows of KV entries (row-major over the kernel axes, contiguous in global
// memory) pass through an LDS block per wave: 16 rows, one per query.  A
// lane's 8 slots of a chunk are consecutive columns of one union row, i.e.
// consecutive entries of one kernel row where they meet the window; each
// entry outside the window is redirected to a zero (reads) or scratch
// (writes) entry by one select on its address, so the chunk loop has no
// branches.  Global memory sees whole rows: one 16-bit buffer access per
// query, lanes over consecutive entries, the row's offset in a scalar
// register.
// ---------------------------------------------------------------------------

// LDS block of one wave, in 16-bit entries: 16 rows of `pitch` entries
// (kernel rows of p2 = K2 entries), then 8 zero entries (reads outside the
// window) and 8 entries that writes outside the window go to.
struct RowBlock {
    int p2, pitch;
};

__host__ __device__ inline RowBlock row_block(const Prob& p) {
    RowBlock r;
    r.p2 = p.ax[2].k;
    r.pitch = (p.ax[0].k * p.ax[1].k * r.p2 + 1) & ~1;
    return r;
}

__host__ __device__ inline int row_block_entries(const Prob& p) { return 16 * row_block(p).pitch + 16; }

// Position in a row block of the entries e = lane + 64 t (t < 4) a lane
// moves between global memory and LDS, -1 past the row's end.
__device__ __forceinline__ void lane_entries(const Prob& p, const RowBlock& rb, int lane, int (&pos)[4]) {
    const int k2 = p.ax[2].k;
    // e / k2 for e < 256, k2 <= 256: (e + 1/2) / k2 lies at least 1/(2 k2) from
    // an integer, far beyond the float rounding of the product
    const float inv = 1.f / static_cast<float>(k2);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const int e = lane + 64 * t;
        const int row = static_cast<int>((static_cast<float>(e) + 0.5f) * inv);
        pos[t] = e < p.kv ? row * rb.p2 + (e - row * k2) : -1;
    }
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rows_rsrc(const void* base) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0), kPlaneBytes, 0x00020000);
}

// Bias-table offset of a query's first neighbour: pb1 * (2 K2 - 1) + pb2,
// with pb = pb_start of the query's position per axis (in [0, K - 1] for odd
// kernels, so start + e needs no clamping).
__device__ __forceinline__ int bias_origin(const Prob& p, const Lane& ln) {
    return pb_start(ln.pos[1], p.ax[1].len, p.ax[1].k, p.ax[1].dil) * (2 * p.ax[2].k - 1) +
           pb_start(ln.pos[2], p.ax[2].len, p.ax[2].k, p.ax[2].dil);
}

// v[qq] += bias of entry e (kernel row e / K2 on axis 1, column e % K2) of
// the wave's query qq: bias[h] at origin(qq) + e1 (2 K2 - 1) + e2, where
// `origin` (bias_origin of each lane's query) was formed with every lane
// active and is read from lane qq.  Table reads in groups of four queries:
// the entry's part of the offset per lane, the query's in a scalar register.
template <typename T>
__device__ __forceinline__ void add_bias(const Prob& p, const T* __restrict__ bias, int h, int origin, int e,
                                         uint16_t (&v)[16]) {
    const int K1 = p.ax[1].k, K2 = p.ax[2].k, r1 = 2 * K1 - 1, r2 = 2 * K2 - 1;
    const int e1 = e / K2, e2 = e - (e / K2) * K2;
    const int mine = origin;
    const __amdgpu_buffer_rsrc_t rt = rows_rsrc(bias + h * r1 * r2);
    const int vo = (e1 * r2 + e2) * 2;
#pragma unroll
    for (int g = 0; g < 16; g += 4) {
        uint16_t x[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
            x[i] = __builtin_amdgcn_raw_buffer_load_b16(rt, vo, __builtin_amdgcn_readlane(mine, g + i) * 2, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            T y, b;
            __builtin_memcpy(&y, &v[g + i], 2);
            __builtin_memcpy(&b, &x[i], 2);
            const T z = from_f<T>(to_f(y) + to_f(b));
            __builtin_memcpy(&v[g + i], &z, 2);
        }
    }
}

// SAME: the two [B, *sp, H, D] operands share one layout (one set of strides
// kept in scalar registers instead of two).
// FLAT (here and in k_wsum_mfma, k_wsum_key_mfma) as for k_fwd_mfma.
// BIAS: `bias`, a relative-position bias [H, 2 K1 - 1, 2 K2 - 1], is added
// to each stored entry at index (pb_start + e) per axis, for odd kernels
// with axis 0 of kernel 1 (the DiNAT QK+RPB op); its own instances, so the
// other products keep their registers.
template <typename T, int D, bool SAME, bool FLAT = false, bool BIAS = false>
__global__ __launch_bounds__(256) void k_dot_mfma(Prob p, TileShape ts, const int* __restrict__ geo,
                                                  const T* __restrict__ a, LayK la_in, const T* __restrict__ xg,
                                                  LayK lx, T* __restrict__ out, LayK lo, float mul, float fill,
                                                  const T* __restrict__ bias) {
    const LayK& la = SAME ? lx : la_in;
    unsigned char* smem = lds_base();
    T* Xs = reinterpret_cast<T*>(smem);
    const int lane = threadIdx.x & 63, col = lane & 15, grp = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: scalar loops
    const RowBlock rb = row_block(p);
    uint16_t* const Rw = reinterpret_cast<uint16_t*>(Xs + ts.slots * D) + wave * row_block_entries(p);
    uint16_t* const dummy = Rw + 16 * rb.pitch + 8;
    Block blk;
    WaveGeo wg;
    if (!tile_geometry<false>(p, ts, geo, wave, blk, wg)) return;
    const StageMap sm = stage_map<T, D>(p, ts, lx, lx, lane);
    Walk w;
    walk_start(blk, w);
    {
        const T* pl = plane_of(xg, lx, w.b, w.h, slice_pos(p, blk, 0));
        stage_pair<T, D, false>(p, blk, ts, sm, pl, lx, Xs, pl, lx, Xs, wave);
    }
    const Lane ln = lane_item(p, ts, blk, wave, col, false);
    const int orow = ln.valid ? vol_off(lo, ln.pos) : -1;
    const int borigin = BIAS ? bias_origin(p, ln) : 0;
    int epos[4];
    lane_entries(p, rb, lane, epos);
    const f32x4_t zero[2] = {f32x4_t{0.f, 0.f, 0.f, 0.f}, f32x4_t{0.f, 0.f, 0.f, 0.f}};
    const uint32_t fill2 = Mma<T>::pack(fill, fill);
    const uint4 fill8 = make_uint4(fill2, fill2, fill2, fill2);
    uint16_t* const myrow = Rw + col * rb.pitch;
    const int nfill = rb.pitch * 2;  // 16-byte pieces of the 16 rows
    uint4 af[D / 32];
    bool more = true, fresh = true;
    while (more) {
        const int b = w.b, h = w.h, u0 = w.u0;
        if (fresh) {
            load_frags<T, D>(bh_ptr(a, la, b, h), vol_off(la, ln.pos), ln.valid, grp, af);
            for (int i = lane; i < nfill; i += 64) reinterpret_cast<uint4*>(Rw)[i] = fill8;
        }
        wait_loads();
        __syncthreads();
        if (wg.any && u0 >= wg.lo[0] && u0 <= wg.hi[0]) {
            const bool in0 = u0 >= ln.lo[0] && u0 <= ln.hi[0];
            for (int c = wg.c0; c <= wg.c1; ++c) {
                f32x4_t sc[2];
                score_chunk<T, D>(Xs, c, col, grp, af, zero, sc);
                const int s0 = 32 * c + 8 * grp, r = s0 >> ts.rowshift, col0 = s0 & ((1 << ts.rowshift) - 1);
                const bool rok = in0 && r >= ln.lo[1] && r <= ln.hi[1];
                const int e0 = ((u0 - ln.lo[0]) * p.ax[1].k + r - ln.lo[1]) * rb.p2 + col0 - ln.lo[2];
                const int d = rok ? col0 - ln.lo[2] : 0x40000000;
                const unsigned k2 = static_cast<unsigned>(p.ax[2].k);
#pragma unroll
                for (int i = 0; i < 8; i += 2) {
                    const uint32_t v = Mma<T>::pack(sc[i >> 2][i & 3] * mul, sc[i >> 2][(i & 3) + 1] * mul);
                    uint16_t* a0 = static_cast<unsigned>(d + i) < k2 ? myrow + e0 + i : dummy;
                    uint16_t* a1 = static_cast<unsigned>(d + i + 1) < k2 ? myrow + e0 + i + 1 : dummy;
                    *a0 = static_cast<uint16_t>(v);
                    *a1 = static_cast<uint16_t>(v >> 16);
                }
            }
        }
        if constexpr (FLAT) {
            more = false;
        } else {
            more = walk_next(blk, w, fresh);
            __syncthreads();  // the slice is no longer read
        }
        if (more) {
            const T* pl = plane_of(xg, lx, w.b, w.h, slice_pos(p, blk, w.u0));
            stage_pair<T, D, false>(p, blk, ts, sm, pl, lx, Xs, pl, lx, Xs, wave);
        }
        if (fresh || !more) {
            // the 16 rows, 64 entries at a time: all LDS reads, then the stores
            const __amdgpu_buffer_rsrc_t ro = rows_rsrc(bh_ptr(out, lo, b, h));
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                if (64 * t >= p.kv) break;
                if (epos[t] >= 0) {
                    uint16_t v[16];
#pragma unroll
                    for (int qq = 0; qq < 16; ++qq) v[qq] = Rw[qq * rb.pitch + epos[t]];
                    if constexpr (BIAS) add_bias<T>(p, bias, h, borigin, lane + 64 * t, v);
#pragma unroll
                    for (int qq = 0; qq < 16; ++qq) {
                        const int off = __builtin_amdgcn_readlane(orow, qq);
                        if (off >= 0) __builtin_amdgcn_raw_buffer_store_b16(v[qq], ro, (lane + 64 * t) * 2, off * 2, 0);
                    }
                }
            }
        }
    }
}

template <typename T, int D, bool SAME>
__device__ __forceinline__ void redo_wsum(const void* kargs, int wg, int wave, int col, int grp) {
    const WsumArgs<T>& A = *static_cast<const WsumArgs<T>*>(kargs);
    const LayK &aw = A.lw, &ax = A.lx, &ao = SAME ? ax : A.lo;
    int b, h0, h1, pos[3];
    if (!lane_position<false>(A.p, A.ts, wg, wave, col, b, h0, h1, pos)) return;
    ExactAxis x[3];
    for (int a = 0; a < 3; ++a) x[a] = exact_axis(A.p.ax[a], pos[a]);
    f32x4_t acc[D / 16];
#pragma unroll 1
    for (int h = h0; h < h1; ++h) {
        exact_wsum<T, D>(x, bh_ptr(A.w, aw, b, h) + vol_off(aw, pos), bh_ptr(A.x, ax, b, h), strides3(ax), grp, acc);
        store_rows<T, D>(bh_ptr(A.out, ao, b, h), vol_off(ao, pos), grp, acc, A.mul);
    }
}

template <typename T, int D, bool SAME, bool FLAT = false>
__global__ __launch_bounds__(256) void k_wsum_mfma(WsumArgs<T> args) {
    const Prob& p = args.p;
    const TileShape& ts = args.ts;
    const int* __restrict__ geo = args.geo;
    const T* __restrict__ wt = args.w;
    const T* __restrict__ xg = args.x;
    T* __restrict__ out = args.out;
    const LayK &lw = args.lw, &lx = args.lx, &lo_in = args.lo;
    const float mul = args.mul;
    const LayK& lo = SAME ? lx : lo_in;
    unsigned char* smem = lds_base();
    T* Xs = reinterpret_cast<T*>(smem);
    const int lane = threadIdx.x & 63, col = lane & 15, grp = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: scalar loops
    const RowBlock rb = row_block(p);
    uint16_t* const Rw = reinterpret_cast<uint16_t*>(Xs + ts.slots * D) + wave * row_block_entries(p);
    const uint16_t* const zeros = Rw + 16 * rb.pitch;
    Block blk;
    WaveGeo wg;
    if (!tile_geometry<false>(p, ts, geo, wave, blk, wg)) return;
    const StageMap sm = stage_map<T, D>(p, ts, lx, lx, lane);
    Walk w;
    walk_start(blk, w);
    {
        const T* pl = plane_of(xg, lx, w.b, w.h, slice_pos(p, blk, 0));
        stage_pair<T, D, false>(p, blk, ts, sm, pl, lx, Xs, pl, lx, Xs, wave);
    }
    const Lane ln = lane_item(p, ts, blk, wave, col, false);
    const int wrow = ln.valid ? vol_off(lw, ln.pos) : -1;
    int epos[4];
    lane_entries(p, rb, lane, epos);
    const uint16_t* const myrow = Rw + col * rb.pitch;
    const int nclear = rb.pitch * 2 + 2;  // 16-byte pieces of the block
    f32x4_t acc[D / 16];
    bool more = true, fresh = true, redo = false;
    while (more) {
        const int b = w.b, h = w.h, u0 = w.u0;
        if (fresh) {
#pragma unroll
            for (int db = 0; db < D / 16; ++db) acc[db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
            for (int i = lane; i < nclear; i += 64) reinterpret_cast<uint4*>(Rw)[i] = make_uint4(0u, 0u, 0u, 0u);
            // the 16 rows, 64 entries at a time: all loads, then the LDS
            // writes (rows of queries past the tile read row 0 and are never
            // read back)
            const __amdgpu_buffer_rsrc_t rw = rows_rsrc(bh_ptr(wt, lw, b, h));
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                if (64 * t >= p.kv) break;
                if (epos[t] >= 0) {
                    uint16_t v[16];
#pragma unroll
                    for (int qq = 0; qq < 16; ++qq)
                        v[qq] = __builtin_amdgcn_raw_buffer_load_b16(
                            rw, (lane + 64 * t) * 2, max(__builtin_amdgcn_readlane(wrow, qq), 0) * 2, 0);
#pragma unroll
                    for (int qq = 0; qq < 16; ++qq) Rw[qq * rb.pitch + epos[t]] = v[qq];
                }
            }
        }
        wait_loads();
        __syncthreads();
        if (wg.any && u0 >= wg.lo[0] && u0 <= wg.hi[0]) {
            const bool in0 = u0 >= ln.lo[0] && u0 <= ln.hi[0];
            for (int c = wg.c0; c <= wg.c1; ++c) {
                const int s0 = 32 * c + 8 * grp, r = s0 >> ts.rowshift, col0 = s0 & ((1 << ts.rowshift) - 1);
                const bool rok = in0 && r >= ln.lo[1] && r <= ln.hi[1];
                const int e0 = ((u0 - ln.lo[0]) * p.ax[1].k + r - ln.lo[1]) * rb.p2 + col0 - ln.lo[2];
                const int d = rok ? col0 - ln.lo[2] : 0x40000000;
                const unsigned k2 = static_cast<unsigned>(p.ax[2].k);
                uint32_t wv[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint16_t* a0 = static_cast<unsigned>(d + 2 * i) < k2 ? myrow + e0 + 2 * i : zeros;
                    const uint16_t* a1 = static_cast<unsigned>(d + 2 * i + 1) < k2 ? myrow + e0 + 2 * i + 1 : zeros;
                    wv[i] = static_cast<uint32_t>(*a0) | (static_cast<uint32_t>(*a1) << 16);
                }
                accumulate_chunk<T, D>(Xs, c, lane, make_uint4(wv[0], wv[1], wv[2], wv[3]), acc);
            }
        }
        if constexpr (FLAT) {
            more = false;
        } else {
            more = walk_next(blk, w, fresh);
            __syncthreads();  // the slice is no longer read
        }
        if (more) {
            const T* pl = plane_of(xg, lx, w.b, w.h, slice_pos(p, blk, w.u0));
            stage_pair<T, D, false>(p, blk, ts, sm, pl, lx, Xs, pl, lx, Xs, wave);
        }
        if (fresh || !more) {
            redo = redo || (item_nonfinite(lane_sum(acc, 0.f)) && ln.valid);
            if (ln.valid) store_rows<T, D>(bh_ptr(out, lo, b, h), vol_off(lo, ln.pos), grp, acc, mul);
        }
    }
    if (redo) redo_wsum<T, D, SAME>(kernargs(), xcd_block(blockIdx.x, gridDim.x), wave, col, grp);
}

// ---------------------------------------------------------------------------
// Split products, key side: out[k] = mul * sum over the queries q whose
// window holds key k of w[q][e(q, k)] x[q]  (QK backward dk: w = dattn,
// x = q, mul = scale; AV backward dv: w = attn, x = dO).  Key tiles as in
// the key-side backward: per slice, the union of the queries attending the
// tile's keys is staged (x rows by DMA, and each query's row of w, slot
// after slot, KV entries each).  In class coordinates e(q, k) = keylin(k) -
// base(q), keylin = sum_a j_a M_a over the key, base = sum_a ws_a(q) M_a
// over the query's window start (M = K1 K2, K2, 1); a per-slot table
// OFF[s] = s KV - base(q_s) leaves one add per (key, slot).  Pairs outside
// the key's query box are masked: rows per chunk, columns per slot.
// ---------------------------------------------------------------------------

// Entries per slot of the key-side weight rows in LDS: a row plus one
// entry of parity, rounded to whole 32-bit words.
__host__ __device__ inline int key_row_pitch(const Prob& p) { return (p.kv + 2) & ~1; }

// Rows of w of one slice's union queries into Ws (pitch entries per slot)
// and the entry table OFF.  Rows are read as aligned 32-bit words, two rows
// per wave instruction (lanes 0-31 and 32-63), only the words that hold
// entries of the row; a row whose first entry sits in the upper half of
// its word lands one entry late in LDS, which OFF accounts for.
template <typename T>
__device__ __forceinline__ void stage_key_rows(const Prob& p, const Block& k, const TileShape& ts, int b, int h,
                                               int u0, const T* __restrict__ wt, const LayK& lw, int* OFF,
                                               uint16_t* Ws, int wave, int lane) {
    const int slots = ts.slots, kv = p.kv, mask2 = (1 << ts.rowshift) - 1, pitch = key_row_pitch(p);
    const int k1 = p.ax[1].k, k2 = p.ax[2].k, d1 = p.ax[1].dil, d2 = p.ax[2].dil;
    const T* wb = bh_ptr(wt, lw, b, h) + slice_pos(p, k, u0) * lw.s0;
    const int lead = static_cast<int>((reinterpret_cast<uintptr_t>(wb) >> 1) & 1);  // wb is 4-byte aligned + 2 lead
    const __amdgpu_buffer_rsrc_t rw = rows_rsrc(wb - lead);
    // in-plane offset of slot s's row, -1 for slots outside the union (not
    // loaded; their LDS rows are never read unmasked)
    const auto row_off = [&](int s) {
        const int a1 = s >> ts.rowshift, a2 = s & mask2;
        return (a1 < k.U[1] && a2 < k.U[2])
                   ? (k.r[1] + (k.lo[1] + a1) * d1) * lw.s1 + (k.r[2] + (k.lo[2] + a2) * d2) * lw.s2
                   : -1;
    };
    const int ws0 = class_ws(k.c[0], k.lo[0] + u0);
    for (int s = threadIdx.x; s < slots; s += blockDim.x) {
        const int a1 = s >> ts.rowshift, a2 = s & mask2;
        const int base = (ws0 * k1 + class_ws(k.c[1], k.lo[1] + a1)) * k2 + class_ws(k.c[2], k.lo[2] + a2);
        OFF[s] = s * pitch + ((max(row_off(s), 0) + lead) & 1) - base;
    }
    uint32_t* Ws32 = reinterpret_cast<uint32_t*>(Ws);
    const int half = lane >> 5, groups = ((kv + 2) / 2 + 31) / 32;  // 32-word groups of a row
    for (int sb = wave * 16; sb < slots; sb += 16 * ts.waves) {
        const int offs = row_off(sb + (lane & 15));  // lanes 0..15: slots sb .. sb + 15
        for (int g = 0; g < groups; ++g) {
            const int j = (lane & 31) + 32 * g;
            uint32_t v[8];
            bool in[8];
#pragma unroll
            for (int m = 0; m < 8; ++m) {
                const int o0 = __builtin_amdgcn_readlane(offs, 2 * m);
                const int o1 = __builtin_amdgcn_readlane(offs, 2 * m + 1);
                const int off = half ? o1 : o0;
                const int first = off + lead;  // entry index from the aligned base
                in[m] = off >= 0 && j < (((first & 1) + kv + 1) >> 1);  // words holding entries of the row
                v[m] = in[m] ? __builtin_amdgcn_raw_buffer_load_b32(rw, ((first >> 1) + j) * 4, 0, 0) : 0u;
            }
#pragma unroll
            for (int m = 0; m < 8; ++m)
                if (in[m]) Ws32[(sb + 2 * m + half) * (pitch >> 1) + j] = v[m];
        }
    }
}

template <typename T, int D, bool SAME>
__device__ __forceinline__ void redo_wsum_key(const void* kargs, int wg, int wave, int col, int grp) {
    const WsumArgs<T>& A = *static_cast<const WsumArgs<T>*>(kargs);
    const LayK &aw = A.lw, &ax = A.lx, &ao = SAME ? ax : A.lo;
    int b, h0, h1, pos[3];
    if (!lane_position<true>(A.p, A.ts, wg, wave, col, b, h0, h1, pos)) return;
    ExactAxis x[3];
    for (int a = 0; a < 3; ++a) x[a] = exact_axis(A.p.ax[a], pos[a]);
    f32x4_t acc[D / 16];
#pragma unroll 1
    for (int h = h0; h < h1; ++h) {
        exact_wsum_key<T, D>(x, bh_ptr(A.w, aw, b, h), strides3(aw), bh_ptr(A.x, ax, b, h), strides3(ax), grp, acc);
        store_rows<T, D>(bh_ptr(A.out, ao, b, h), vol_off(ao, pos), grp, acc, A.mul);
    }
}

template <typename T, int D, bool SAME, bool FLAT = false>
__global__ __launch_bounds__(256) void k_wsum_key_mfma(WsumArgs<T> args) {
    const Prob& p = args.p;
    const TileShape& ts = args.ts;
    const int* __restrict__ geo = args.geo;
    const T* __restrict__ wt = args.w;
    const T* __restrict__ xg = args.x;
    T* __restrict__ out = args.out;
    const LayK &lw = args.lw, &lx = args.lx, &lo_in = args.lo;
    const float mul = args.mul;
    const LayK& lo = SAME ? lx : lo_in;
    unsigned char* smem = lds_base();
    const int slots = ts.slots;
    T* Xs = reinterpret_cast<T*>(smem);
    int* OFF = reinterpret_cast<int*>(Xs + slots * D);
    uint16_t* Ws = reinterpret_cast<uint16_t*>(OFF + slots);
    const int lane = threadIdx.x & 63, col = lane & 15, grp = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: scalar loops
    Block blk;
    WaveGeo wg;
    if (!tile_geometry<true>(p, ts, geo, wave, blk, wg)) return;
    const Lane ln = lane_item(p, ts, blk, wave, col, true);
    if (empty_union(blk)) {
        f32x4_t z[D / 16];
        exact_zero(z);
        if (ln.valid)
            for (int h = blk.h0; h < blk.h1; ++h)
                store_rows<T, D>(bh_ptr(out, lo, blk.b, h), vol_off(lo, ln.pos), grp, z, 1.f);
        return;
    }
    const StageMap sm = stage_map<T, D>(p, ts, lx, lx, lane);
    Walk w;
    walk_start(blk, w);
    int keylin;
    {
        const int f = wave * 16 + col, s2 = ts.tshift[2], s1 = ts.tshift[1];
        const int e2 = f & (ts.T[2] - 1), e1 = (f >> s2) & (ts.T[1] - 1), e0 = f >> (s2 + s1);
        keylin = ((blk.J[0] + e0) * p.ax[1].k + blk.J[1] + e1) * p.ax[2].k + blk.J[2] + e2;
    }
    const int last = slots * key_row_pitch(p) - 1;
    // column masks (two entries per word) of the lane's 8 slots; fixed per
    // tile when union rows are at most 32 slots
    const auto col_masks = [&](int c, uint32_t (&cm)[4]) {
        const int col0 = (32 * c + 8 * grp) & ((1 << ts.rowshift) - 1);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int ca = col0 + 2 * i, cb = ca + 1;
            cm[i] = ((ca >= ln.lo[2] && ca <= ln.hi[2]) ? 0xFFFFu : 0u) |
                    ((cb >= ln.lo[2] && cb <= ln.hi[2]) ? 0xFFFF0000u : 0u);
        }
    };
    uint32_t cm0[4];
    col_masks(0, cm0);
    const bool wide = ts.rowshift > 5;
    f32x4_t acc[D / 16];
    bool more = true, fresh = true, redo = false;
    while (more) {
        const int b = w.b, h = w.h, u0 = w.u0;
        {
            // one staging site (the walk's first slice and every later one)
            const T* pl = plane_of(xg, lx, b, h, slice_pos(p, blk, u0));
            stage_pair<T, D, false>(p, blk, ts, sm, pl, lx, Xs, pl, lx, Xs, wave);
            stage_key_rows<T>(p, blk, ts, b, h, u0, wt, lw, OFF, Ws, wave, lane);
        }
        if (fresh) {
#pragma unroll
            for (int db = 0; db < D / 16; ++db) acc[db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        }
        wait_loads();
        lds_publish_barrier();  // staged rows, the rows of w and OFF
        if (wg.any && u0 >= wg.lo[0] && u0 <= wg.hi[0]) {
            const bool in0 = u0 >= ln.lo[0] && u0 <= ln.hi[0];
            for (int c = wg.c0; c <= wg.c1; ++c) {
                const int s0 = 32 * c + 8 * grp;
                uint32_t cm[4] = {cm0[0], cm0[1], cm0[2], cm0[3]};
                if (wide) col_masks(c, cm);
                const bool rok = row_ok(ln, ts.rowshift, in0, c, grp);
                const int4 oa = *reinterpret_cast<const int4*>(OFF + s0);
                const int4 ob = *reinterpret_cast<const int4*>(OFF + s0 + 4);
                const int o[8] = {oa.x, oa.y, oa.z, oa.w, ob.x, ob.y, ob.z, ob.w};
                uint32_t wv[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int ia = min(max(o[2 * i] + keylin, 0), last);
                    const int ib = min(max(o[2 * i + 1] + keylin, 0), last);
                    const uint32_t v = static_cast<uint32_t>(Ws[ia]) | (static_cast<uint32_t>(Ws[ib]) << 16);
                    wv[i] = rok ? (v & cm[i]) : 0u;
                }
                accumulate_chunk<T, D>(Xs, c, lane, make_uint4(wv[0], wv[1], wv[2], wv[3]), acc);
            }
        }
        if constexpr (FLAT) {
            more = false;
        } else {
            more = walk_next(blk, w, fresh);
            __syncthreads();  // the slice is no longer read
        }
        if (fresh || !more) {
            redo = redo || (item_nonfinite(lane_sum(acc, 0.f)) && ln.valid);
            if (ln.valid) store_rows<T, D>(bh_ptr(out, lo, b, h), vol_off(lo, ln.pos), grp, acc, mul);
        }
    }
    if (redo) redo_wsum_key<T, D, SAME>(kernargs(), xcd_block(blockIdx.x, gridDim.x), wave, col, grp);
}

}  // namespace

// ---------------------------------------------------------------------------
// Host side: eligibility, tile choice, launches.
// ---------------------------------------------------------------------------

namespace {

enum Kind { kForward = 0, kBackwardQ = 1, kBackwardKV = 2, kSplit = 3, kSplitKey = 4 };

// Entries per row (KV) up to which the split kernels take a call (a lane
// moves at most 4 entries of a row), and the LDS their row blocks may take
// per workgroup.
constexpr int kSplitMaxKV = 256;
constexpr size_t kSplitRowsBudget = 48 * 1024;
// LDS of the key-side split kernel per workgroup (x rows, OFF and the rows
// of w of one slice's queries).
constexpr size_t kSplitKeyLds = 128 * 1024;

constexpr size_t kLdsBudget = 64 * 1024;
// A problem whose staged union does not fit kLdsBudget even at 16 items
// (head dim 96/128 with wide unions: strided axes, long kernels near the
// borders) takes a tile of up to kLdsBudgetLarge: fewer workgroups per CU,
// still the matrix cores.
constexpr size_t kLdsBudgetLarge = 128 * 1024;

// Staged operands (split kernels: one; their row blocks come on top).
size_t lds_bytes(Kind kind, int slots, int D) {
    const size_t rows = static_cast<size_t>(slots) * (D == 96 ? 128 : D) * 2;
    if (kind == kSplit || kind == kSplitKey) return kLdsPad + rows;
    return kLdsPad + (kind == kBackwardKV ? 2 * rows + (2 * static_cast<size_t>(slots) + 8) * 4 : 2 * rows);
}

// Head chunks per group of the workgroup order (decode_block).  A 3-D
// window (K0 > 1) takes groups of 2: with every head of a tile in a row the
// K/V planes that neighbouring depth tiles share (all heads of a region)
// outgrow an XCD's L2 before the next depth tile reads them, and the
// kernels fetched 1.3-1.8x their compulsory bytes at config 5; in pairs
// they fetch 1.03-1.04x, and the lse / delta rows are still written two
// heads at a time.  Otherwise all chunks form one group (heads fastest).
// NATTEN_HIP_HEAD_GROUP=g (a divisor of the chunk count) overrides (tuning).
void set_h_per(const Prob& p, TileShape& ts, int per) {
    static const int forced = [] {
        const char* e = std::getenv("NATTEN_HIP_HEAD_GROUP");
        return e ? std::atoi(e) : 0;
    }();
    ts.h_per = per;
    const int chunks = (ts.nheads + per - 1) / per;
    ts.hchunks = make_fastdiv(static_cast<uint32_t>(chunks));
    int g = chunks;
    if (forced > 0 && chunks % forced == 0)
        g = forced;
    else if (forced <= 0 && p.ax[0].k > 1 && chunks >= 4 && chunks % 2 == 0)
        g = 2;
    ts.hg = make_fastdiv(static_cast<uint32_t>(g));
    ts.hgroups = make_fastdiv(static_cast<uint32_t>(chunks / g));
}

// Largest box of the fused kernels' tiles: 64 items (4 waves) unless
// NATTEN_HIP_TILE_ITEMS asks for 16, 32 or 128 (tuning).
int fused_items() {
    static const int n = [] {
        const char* e = std::getenv("NATTEN_HIP_TILE_ITEMS");
        const int v = e ? std::atoi(e) : 0;
        return (v == 16 || v == 32 || v == 64 || v == kMaxFusedItems) ? v : kMaxItems;
    }();
    return n;
}

// NATTEN_HIP_TILE_SHAPE=t0,t1,t2 (powers of two, product 16..128) fixes the
// first box tried for the fused kernels (tuning); null when unset.
const int* forced_shape() {
    static int shape[3] = {0, 0, 0};
    static const bool set = [] {
        const char* e = std::getenv("NATTEN_HIP_TILE_SHAPE");
        int t[3];
        if (!e || std::sscanf(e, "%d,%d,%d", &t[0], &t[1], &t[2]) != 3) return false;
        const long long prod = static_cast<long long>(t[0]) * t[1] * t[2];
        for (int a = 0; a < 3; ++a)
            if (t[a] < 1 || (t[a] & (t[a] - 1)) != 0) return false;
        if (prod < 16 || prod > kMaxFusedItems) return false;
        for (int a = 0; a < 3; ++a) shape[a] = t[a];
        return true;
    }();
    return set ? shape : nullptr;
}

// 3-D forward and dQ tiles first try two depth planes of 8 x 8 items (8
// waves): a depth window of K0 then stages K0 + 1 slices for two planes
// instead of K0 for one. On config 5 (16 x 32 x 32, K 3 x 7 x 7, head dim
// 64) that made both kernels about 11 % faster; the dK/dV kernel, limited by
// its registers to one such workgroup per CU, keeps 64 items.
bool deep_query_tile(const Prob& p, Kind kind, const int (&n)[3]) {
    return (kind == kForward || kind == kBackwardQ) && fused_items() == kMaxItems && n[0] >= 2 &&
           p.ax[0].k > 1 && n[1] >= 8 && n[2] >= 8;
}

// LDS a forward / dQ workgroup adds for global keys: 32 key and 32 value rows.
size_t global_lds(int D) { return static_cast<size_t>(2 * 32) * (D == 96 ? 128 : D) * 2; }

// Workgroup box in class coordinates (query items on a strided axis): up to
// 64 items (4 waves), power-of-two extents, innermost axis first (8 wide
// unless the problem is 1-D); halved until the staged union fits the LDS
// budget, kLdsBudget first, then kLdsBudgetLarge.
bool choose_tile(const Prob& p, Kind kind, int D, TileShape& ts, size_t extra_lds = 0, bool varlen = false) {
    const bool key_tile = kind == kBackwardKV || kind == kSplitKey;
    const bool fused = kind == kForward || kind == kBackwardQ || kind == kBackwardKV;
    int n[3];  // items per axis: keys, or query items (output extent when strided); class 0 is the longest
    for (int a = 0; a < 3; ++a) n[a] = key_tile ? n_class_h(p.ax[a], 0) : query_items(p.ax[a], n_class_h(p.ax[a], 0));
    // box T (power-of-two extents): its waves, staged union and LDS fit
    const auto fits = [&](const int (&T)[3], size_t budget) {
        for (int a = 0; a < 3; ++a) {
            ts.T[a] = T[a];
            ts.tshift[a] = log2_of(T[a]);
            ts.ntile[a] = (n[a] + T[a] - 1) / T[a];
        }
        ts.waves = std::max(1, (T[0] * T[1] * T[2] + 15) / 16);
        // variable-length samples: sized for every extent up to the padded one
        const int u1 = varlen ? union_extent_upto(p.ax[1], T[1], key_tile) : union_extent(p.ax[1], T[1], key_tile);
        const int u2 = varlen ? union_extent_upto(p.ax[2], T[2], key_tile) : union_extent(p.ax[2], T[2], key_tile);
        ts.rowshift = std::max(3, log2_of(u2));
        ts.slots = ((u1 * (1 << ts.rowshift) + 31) / 32) * 32;
        return lds_bytes(kind, ts.slots, D) + extra_lds <= budget;
    };
    const auto finish = [&]() {
        ts.nheads = key_tile ? p.Hkv : p.Hq;
        set_h_per(p, ts, 1);
        ts.rep = make_fastdiv(static_cast<uint32_t>(p.rep));
        long long spatial = 1;
        for (int a = 0; a < 3; ++a) {
            ts.tiles[a] = make_fastdiv(static_cast<uint32_t>(ts.ntile[a]));
            ts.dil[a] = make_fastdiv(static_cast<uint32_t>(p.ax[a].dil));
            ts.lenmod[a] = p.ax[a].len % p.ax[a].dil;
            spatial *= static_cast<long long>(ts.ntile[a]) * p.ax[a].dil;
        }
        if (spatial >= (1LL << 31)) return false;
        ts.spatial = make_fastdiv(static_cast<uint32_t>(spatial));
        return true;
    };
    if (const int* forced = fused ? forced_shape() : nullptr) {
        int T[3];
        for (int a = 0; a < 3; ++a) T[a] = std::min(pow2_at_least(n[a]), forced[a]);
        if (fits(T, kLdsBudget)) return finish();
    } else if (fused && deep_query_tile(p, kind, n)) {
        const int T[3] = {2, 8, 8};
        if (fits(T, kLdsBudget)) return finish();
    }
    for (int pass = 0; pass < 2; ++pass) {
        const size_t budget = pass == 0 ? kLdsBudget : kLdsBudgetLarge;
        for (int items = fused ? fused_items() : kMaxItems; items >= 16; items /= 2) {
            const auto shape = [&](int w2, int (&T)[3]) {
                if (n[0] == 1 && n[1] == 1) {
                    T[2] = std::min(pow2_at_least(n[2]), items);
                    T[1] = T[0] = 1;
                } else {
                    T[2] = std::min(pow2_at_least(n[2]), w2);
                    T[1] = std::min(pow2_at_least(n[1]), std::max(items / T[2], 1));
                    T[0] = std::min(pow2_at_least(n[0]), std::max(items / (T[2] * T[1]), 1));
                }
            };
            if (!varlen) {
                int T[3];
                shape(8, T);
                if (fits(T, budget)) return finish();
                continue;
            }
            // variable length: the union that every sample extent allows can
            // cross a power of two at the default width (a row pitch twice as
            // wide), so the widths 8, 4 and 16 compete on LDS
            int best[3] = {0, 0, 0};
            size_t best_lds = 0;
            for (const int w2 : {8, 4, 16}) {
                int T[3];
                shape(w2, T);
                if (!fits(T, budget)) continue;
                const size_t lds = lds_bytes(kind, ts.slots, D);
                if (best[0] == 0 || lds < best_lds) {
                    for (int a = 0; a < 3; ++a) best[a] = T[a];
                    best_lds = lds;
                }
            }
            if (best[0] != 0 && fits(best, budget)) return finish();
        }
    }
    return false;
}

long long spatial_tiles(const Prob& p, const TileShape& ts) {
    long long nb = 1;
    for (int a = 0; a < 3; ++a) nb *= static_cast<long long>(p.ax[a].dil) * ts.ntile[a];
    return nb;
}

long long grid_blocks(const Prob& p, const TileShape& ts) {
    return spatial_tiles(p, ts) * p.B * static_cast<long long>(ts.hchunks.d);
}

// Heads per workgroup: one unless the grid would still fill the device about
// twice over with more; NATTEN_HIP_HEADS_PER=n fixes it (tuning).
void fit_h_per(const Prob& p, TileShape& ts, long long resident) {
    static const int forced = [] {
        const char* e = std::getenv("NATTEN_HIP_HEADS_PER");
        return e ? std::atoi(e) : 0;
    }();
    const long long cells = spatial_tiles(p, ts) * p.B;
    long long per = forced > 0 ? forced : (cells * ts.nheads) / (4 * resident);
    per = std::max(1LL, std::min<long long>(per, ts.nheads));
    set_h_per(p, ts, static_cast<int>(per));
}

// Per-tile geometry records, built on the host once per (device, tile kind,
// problem geometry) and kept for the life of the process; launches read
// their tile's record instead of recomputing it.  Not built while the stream
// is being captured or inside a NoDeviceAlloc scope (the kernels then compute
// the geometry themselves), nor past kGeoMaxBytes in total.  NATTEN_HIP_GEOMETRY=device disables the
// tables (A/B and tests).
constexpr size_t kGeoMaxBytes = size_t(64) << 20;

struct GeoEntry {
    int dev, key;
    int len[3], k[3], dil[3], st[3], causal[3], T[3], waves, rowshift;
    int* ptr;
    std::vector<int>* host;  // source of the asynchronous upload, kept with the table
    TableUpload* up;
};

thread_local bool t_no_device_alloc = false;

}  // namespace

hipError_t table_upload(TableUpload& u, void* d, const void* h, size_t bytes, hipStream_t s) {
    hipError_t e = hipEventCreateWithFlags(&u.ev, hipEventDisableTiming);
    if (e != hipSuccess) return e;
    e = hipMemcpyAsync(d, h, bytes, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = hipEventRecord(u.ev, s);
    if (e != hipSuccess) {
        (void)hipEventDestroy(u.ev);
        u.ev = nullptr;
        return e;
    }
    u.stream = s;
    return hipSuccess;
}

bool table_ready(TableUpload& u, hipStream_t s) {
    if (u.done) return true;
    // Under capture the upload's event is neither queried nor waited on (a
    // graph may be replayed on any stream, after any amount of other work):
    // until an ordinary call has seen the upload complete, a captured launch
    // declines the table and its kernels compute the geometry themselves.
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &st) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    if (st != hipStreamCaptureStatusNone) return false;
    const hipError_t q = hipEventQuery(u.ev);
    if (q == hipSuccess) {
        u.done = true;
        return true;
    }
    if (q != hipErrorNotReady) {
        (void)hipGetLastError();
        return false;
    }
    if (s == u.stream) return true;  // stream order covers the copy
    return hipStreamWaitEvent(s, u.ev, 0) == hipSuccess;
}

namespace {

const int* geometry_table(const Prob& p, const TileShape& ts, bool key_tile, hipStream_t stream) {
    const char* env = std::getenv("NATTEN_HIP_GEOMETRY");
    if (env && std::strcmp(env, "device") == 0) return nullptr;
    static std::mutex mu;
    static std::vector<GeoEntry> cache;
    static size_t total = 0;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return nullptr;
    GeoEntry key{};
    key.dev = dev;
    key.key = key_tile ? 1 : 0;
    for (int a = 0; a < 3; ++a) {
        key.len[a] = p.ax[a].len;
        key.k[a] = p.ax[a].k;
        key.dil[a] = p.ax[a].dil;
        key.st[a] = p.ax[a].st;
        key.causal[a] = p.ax[a].causal;
        key.T[a] = ts.T[a];
    }
    key.waves = ts.waves;
    key.rowshift = ts.rowshift;
    std::lock_guard<std::mutex> g(mu);
    for (const GeoEntry& e : cache)
        if (std::memcmp(&e, &key, offsetof(GeoEntry, ptr)) == 0) return table_ready(*e.up, stream) ? e.ptr : nullptr;
    if (!device_alloc_allowed()) return nullptr;
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &st) != hipSuccess || st != hipStreamCaptureStatusNone) return nullptr;
    const long long S = ts.spatial.d;
    const size_t bytes = static_cast<size_t>(S) * kRecDwords * sizeof(int);
    if (total + bytes > kGeoMaxBytes) return nullptr;
    auto* hv = new std::vector<int>(static_cast<size_t>(S) * kRecDwords, 0);
    std::vector<int>& h = *hv;
    for (int s = 0; s < S; ++s) {
        int* rec = h.data() + static_cast<size_t>(s) * kRecDwords;
        int t[3], r[3];
        spatial_coords(ts, s, t, r);
        int nonempty = 1;
        for (int w = 0; w < kMaxWaves; ++w) {
            int il[3], ih[3];
            wave_items(ts, w, il, ih);
            int* wr = rec + 24 + 8 * w;
            int any = w < ts.waves ? 1 : 0, glo[3], ghi[3];
            for (int a = 0; a < 3; ++a) {
                const AxisGeo ag = axis_geometry(p.ax[a].len, p.ax[a].k, p.ax[a].dil, p.ax[a].causal, ts.lenmod[a],
                                                 p.ax[a].st, p.ax[a].out, ts.T[a], t[a], r[a], il[a], ih[a],
                                                 key_tile, ts.dil[a]);
                if (w == 0) {
                    rec[a] = r[a];
                    rec[3 + a] = ag.J;
                    rec[6 + a] = ag.E;
                    rec[9 + a] = ag.lo;
                    rec[12 + a] = ag.U;
                    rec[15 + a] = ag.n;
                    rec[18 + a] = ag.B;
                    nonempty &= ag.tile_ok;
                }
                any &= ag.wave_ok;
                glo[a] = ag.glo;
                ghi[a] = ag.ghi;
            }
            wr[0] = any;
            for (int a = 0; a < 3; ++a) {
                wr[1 + 2 * a] = glo[a];
                wr[2 + 2 * a] = ghi[a];
            }
            const int c0 = (glo[1] * (1 << ts.rowshift) + glo[2]) >> 5;
            const int c1 = (ghi[1] * (1 << ts.rowshift) + ghi[2]) >> 5;
            wr[7] = (c0 & 0xFFFF) | (c1 << 16);
        }
        rec[21] = nonempty;
    }
    int* d = nullptr;
    if (hipMalloc(reinterpret_cast<void**>(&d), bytes) != hipSuccess) {
        (void)hipGetLastError();
        delete hv;
        return nullptr;
    }
    auto* up = new TableUpload;
    if (table_upload(*up, d, h.data(), bytes, stream) != hipSuccess) {
        (void)hipGetLastError();
        (void)hipFree(d);
        delete up;
        delete hv;
        return nullptr;
    }
    key.ptr = d;
    key.host = hv;
    key.up = up;
    cache.push_back(key);
    total += bytes;
    return d;
}

template <typename T>
GlobalKeys<T> to_global(const GlobalSet* g) {
    GlobalKeys<T> r{};
    if (g) {
        r.k = static_cast<const T*>(g->k);
        r.v = static_cast<const T*>(g->v);
        r.kb = g->lk.b;
        r.kh = g->lk.h;
        r.vb = g->lv.b;
        r.vh = g->lv.h;
        r.ks = static_cast<int>(g->lk.s2);
        r.vs = static_cast<int>(g->lv.s2);
        r.n = g->n;
    }
    return r;
}

// A launch whose workgroups each walk a single step (FLAT instances): axis 0
// of extent 1 (one slice per tile), one head per workgroup, and for key
// tiles one q head per kv head.  Built for the shared layout groups with
// rows of at most 32 slots.
template <int LAY, bool WIDE, bool GLOBAL, bool VARLEN>
constexpr bool kHasFlat = !WIDE && !GLOBAL && !VARLEN && LAY != kLayGeneral;

bool flat_walk(const Prob& p, const TileShape& ts, bool key_tile) {
    return p.ax[0].len == 1 && p.ax[0].k == 1 && ts.h_per == 1 && (!key_tile || p.rep == 1);
}

template <typename T, int D, int LAY, bool WIDE, bool GLOBAL, bool VARLEN = false>
hipError_t run_fwd(const Prob& p, TileShape ts, const void* q, Lay lq, const void* k, Lay lk, const void* v, Lay lv,
                   void* o, Lay lo, float* lse, Lay ll, const GlobalSet* g, hipStream_t s, const int* lens = nullptr) {
    auto kern = k_fwd_mfma<T, D, LAY, WIDE, GLOBAL, VARLEN>;
    const size_t shm = lds_bytes(kForward, ts.slots, D) + (GLOBAL ? global_lds(D) : 0);
    hipError_t e = allow_lds(kern, shm);
    if (e != hipSuccess) return e;
    fit_h_per(p, ts, resident_blocks(kern, 64 * ts.waves, shm));
    if constexpr (kHasFlat<LAY, WIDE, GLOBAL, VARLEN>) {
        if (flat_walk(p, ts, false)) {
            kern = k_fwd_mfma<T, D, LAY, WIDE, GLOBAL, VARLEN, true>;
            if ((e = allow_lds(kern, shm)) != hipSuccess) return e;
        }
    }
    const int* geo = VARLEN ? nullptr : geometry_table(p, ts, false, s);
    const FwdArgs<T> a{p,   ts,       geo,      (const T*)q, (const T*)k, (const T*)v, (T*)o,
                       lse, to_k(lq), to_k(lk), to_k(lv),    to_k(lo),    to_k(ll),    to_global<T>(g), lens};
    NA_LAUNCH(VARLEN ? "na_varlen_fwd_mfma" : GLOBAL ? "na_fwd_global_mfma" : "na_fwd_mfma", kern, dim3(static_cast<unsigned>(grid_blocks(p, ts))),
              dim3(64 * ts.waves), shm, s, a);
    return hipGetLastError();
}

template <typename T, int D, int LAY, bool GLOBAL>
hipError_t launch_fwd(const Prob& p, const void* q, Lay lq, const void* k, Lay lk, const void* v, Lay lv, void* o,
                      Lay lo, float* lse, Lay ll, const GlobalSet* g, hipStream_t s) {
    TileShape ts{};
    if (!choose_tile(p, kForward, D, ts, GLOBAL ? global_lds(D) : 0)) return hipErrorInvalidValue;
    if (ts.rowshift > 5) return run_fwd<T, D, LAY, true, GLOBAL>(p, ts, q, lq, k, lk, v, lv, o, lo, lse, ll, g, s);
    return run_fwd<T, D, LAY, false, GLOBAL>(p, ts, q, lq, k, lk, v, lv, o, lo, lse, ll, g, s);
}

template <typename T, int D>
hipError_t launch_fwd(const Prob& p, const void* q, Lay lq, const void* k, Lay lk, const void* v, Lay lv, void* o,
                      Lay lo, float* lse, Lay ll, const GlobalSet* g, hipStream_t s) {
    // global-key instances exist for the general layout group only
    if (g) return launch_fwd<T, D, kLayGeneral, true>(p, q, lq, k, lk, v, lv, o, lo, lse, ll, g, s);
    switch (layout_group({lq, lo}, {lk, lv}, {ll})) {
        case kLayOne:
            return launch_fwd<T, D, kLayOne, false>(p, q, lq, k, lk, v, lv, o, lo, lse, ll, nullptr, s);
        case kLayTwo:
            return launch_fwd<T, D, kLayTwo, false>(p, q, lq, k, lk, v, lv, o, lo, lse, ll, nullptr, s);
        case kLayFour:
            return launch_fwd<T, D, kLayFour, false>(p, q, lq, k, lk, v, lv, o, lo, lse, ll, nullptr, s);
        default:
            return launch_fwd<T, D, kLayGeneral, false>(p, q, lq, k, lk, v, lv, o, lo, lse, ll, nullptr, s);
    }
}

template <typename T, int D, int LAY, bool WIDE, bool GLOBAL, bool VARLEN = false>
hipError_t run_bwd_q(const Prob& p, TileShape ts, const void* q, Lay lq, const void* k, Lay lk, const void* v,
                     Lay lv, const void* o, Lay lo, const void* dout, Lay ldo, const float* lse, Lay ll,
                     const float* dlse, Lay ldl, void* dq, Lay ldq, float* delta, Lay lde, const GlobalSet* g,
                     hipStream_t s, const int* lens = nullptr) {
    // delta from P dP where the walk has one slice per head
    constexpr bool kPdpOk = !GLOBAL && !VARLEN;
    const bool pdp = kPdpOk && p.ax[0].len == 1;
    auto kern = pdp ? k_bwd_q_mfma<T, D, LAY, WIDE, GLOBAL, VARLEN, false, kPdpOk>
                    : k_bwd_q_mfma<T, D, LAY, WIDE, GLOBAL, VARLEN>;
    const size_t shm = lds_bytes(kBackwardQ, ts.slots, D) + (GLOBAL ? global_lds(D) : 0);
    hipError_t e = allow_lds(kern, shm);
    if (e != hipSuccess) return e;
    fit_h_per(p, ts, resident_blocks(kern, 64 * ts.waves, shm));
    if constexpr (kHasFlat<LAY, WIDE, GLOBAL, VARLEN>) {
        if (flat_walk(p, ts, false)) {
            kern = pdp ? k_bwd_q_mfma<T, D, LAY, WIDE, GLOBAL, VARLEN, true, kPdpOk>
                       : k_bwd_q_mfma<T, D, LAY, WIDE, GLOBAL, VARLEN, true>;
            if ((e = allow_lds(kern, shm)) != hipSuccess) return e;
        }
    }
    const int* geo = VARLEN ? nullptr : geometry_table(p, ts, false, s);
    const BwdQArgs<T> a{p,        ts,       geo,      (const T*)q, (const T*)k, (const T*)v, (const T*)o,
                        (const T*)dout, lse, dlse,  (T*)dq,      delta,       to_k(lq),    to_k(lk),
                        to_k(lv), to_k(lo), to_k(ldo), to_k(ll),  to_k(ldl),   to_k(ldq),   to_k(lde),
                        to_global<T>(g), lens};
    NA_LAUNCH(VARLEN ? "na_varlen_bwd_q_mfma" : GLOBAL ? "na_bwd_q_global_mfma" : "na_bwd_q_mfma", kern,
              dim3(static_cast<unsigned>(grid_blocks(p, ts))), dim3(64 * ts.waves), shm, s, a);
    return hipGetLastError();
}

template <typename T, int D, int LAY, bool WIDE, bool VARLEN = false>
hipError_t run_bwd_kv(const Prob& p, TileShape ts, const void* q, Lay lq, const void* k, Lay lk, const void* v,
                      Lay lv, const void* dout, Lay ldo, const float* lse, Lay ll, const float* delta, Lay lde,
                      void* dk, Lay ldk, void* dv, Lay ldv, hipStream_t s, const int* lens = nullptr) {
    auto kern = k_bwd_kv_mfma<T, D, LAY, WIDE, VARLEN>;
    const size_t shm = lds_bytes(kBackwardKV, ts.slots, D);
    hipError_t e = allow_lds(kern, shm);
    if (e != hipSuccess) return e;
    fit_h_per(p, ts, resident_blocks(kern, 64 * ts.waves, shm));
    if constexpr (kHasFlat<LAY, WIDE, false, VARLEN>) {
        if (flat_walk(p, ts, true)) {
            kern = k_bwd_kv_mfma<T, D, LAY, WIDE, VARLEN, true>;
            if ((e = allow_lds(kern, shm)) != hipSuccess) return e;
        }
    }
    const int* geo = VARLEN ? nullptr : geometry_table(p, ts, true, s);
    const BwdKvArgs<T> a{p,        ts,       geo,       (const T*)q, (const T*)k, (const T*)v, (const T*)dout,
                         lse,      delta,    (T*)dk,    (T*)dv,      to_k(lq),    to_k(lk),    to_k(lv),
                         to_k(ldo), to_k(ll), to_k(lde), to_k(ldk),  to_k(ldv), lens};
    NA_LAUNCH(VARLEN ? "na_varlen_bwd_kv_mfma" : "na_bwd_kv_mfma", kern, dim3(static_cast<unsigned>(grid_blocks(p, ts))), dim3(64 * ts.waves), shm, s, a);
    return hipGetLastError();
}

template <typename T, int D, int LAY, bool GLOBAL>
hipError_t launch_bwd(const Prob& p, const void* q, Lay lq, const void* k, Lay lk, const void* v, Lay lv,
                      const void* o, Lay lo, const void* dout, Lay ldo, const float* lse, Lay ll,
                      const float* dlse, Lay ldl, void* dq, Lay ldq, void* dk, Lay ldk, void* dv, Lay ldv,
                      float* delta, Lay lde, const GlobalSet* g, hipStream_t s) {
    TileShape tq{}, tk{};
    if (!choose_tile(p, kBackwardQ, D, tq, GLOBAL ? global_lds(D) : 0) || !choose_tile(p, kBackwardKV, D, tk))
        return hipErrorInvalidValue;
    hipError_t e = tq.rowshift > 5
                       ? run_bwd_q<T, D, LAY, true, GLOBAL>(p, tq, q, lq, k, lk, v, lv, o, lo, dout, ldo, lse, ll,
                                                            dlse, ldl, dq, ldq, delta, lde, g, s)
                       : run_bwd_q<T, D, LAY, false, GLOBAL>(p, tq, q, lq, k, lk, v, lv, o, lo, dout, ldo, lse, ll,
                                                             dlse, ldl, dq, ldq, delta, lde, g, s);
    if (e != hipSuccess) return e;
    if (tk.rowshift > 5)
        return run_bwd_kv<T, D, LAY, true>(p, tk, q, lq, k, lk, v, lv, dout, ldo, lse, ll, delta, lde, dk, ldk, dv,
                                           ldv, s);
    return run_bwd_kv<T, D, LAY, false>(p, tk, q, lq, k, lk, v, lv, dout, ldo, lse, ll, delta, lde, dk, ldk, dv, ldv,
                                        s);
}

template <typename T, int D>
hipError_t launch_bwd(const Prob& p, const void* q, Lay lq, const void* k, Lay lk, const void* v, Lay lv,
                      const void* o, Lay lo, const void* dout, Lay ldo, const float* lse, Lay ll,
                      const float* dlse, Lay ldl, void* dq, Lay ldq, void* dk, Lay ldk, void* dv, Lay ldv,
                      float* delta, Lay lde, const GlobalSet* gs, hipStream_t s) {
    // global-key instances exist for the general layout group only
    if (gs)
        return launch_bwd<T, D, kLayGeneral, true>(p, q, lq, k, lk, v, lv, o, lo, dout, ldo, lse, ll, dlse, ldl, dq,
                                                   ldq, dk, ldk, dv, ldv, delta, lde, gs, s);
    // without dlse its layout is never read
    const int g = layout_group({lq, lo, ldo, ldq}, {lk, lv, ldk, ldv}, {ll, lde, dlse ? ldl : ll});
#define NA_BWD_LAY(L)                                                                                                 \
    return launch_bwd<T, D, L, false>(p, q, lq, k, lk, v, lv, o, lo, dout, ldo, lse, ll, dlse, ldl, dq, ldq, dk, ldk, \
                                      dv, ldv, delta, lde, nullptr, s)
    switch (g) {
        case kLayOne:
            NA_BWD_LAY(kLayOne);
        case kLayTwo:
            NA_BWD_LAY(kLayTwo);
        case kLayFour:
            NA_BWD_LAY(kLayFour);
        default:
            NA_BWD_LAY(kLayGeneral);
    }
#undef NA_BWD_LAY
}

// ---------------------------------------------------------------------------
// Variable-length problems on the fused tile kernels (their VARLEN instances,
// general layout group): tile shape and LDS sized for the padded extents and
// every smaller one, geometry computed in the kernels per sample, and the
// padding positions zeroed by k_varlen_pad_zero afterwards.
// ---------------------------------------------------------------------------

// Zeroing target: rows of `width` elements of `esz` bytes (16-byte aligned
// when width > 1) at every head below `heads`, or one fp32 scalar per head.
struct PadTarget {
    void* base;
    LayK lay;
    int heads, width, esz;
};

struct PadArgs {
    Prob p;
    const int* lens;
    int n;
    PadTarget t[4];
};

// One thread per (batch, padded position, head): where the position is
// padding for its sample (past its extent on some axis, or the whole sample
// when its extents are out of range) every target's row of that head
// becomes zero.
__global__ __launch_bounds__(256) void k_varlen_pad_zero(PadArgs a) {
    const Prob& p = a.p;
    const int n0 = p.ax[0].len, n1 = p.ax[1].len, n2 = p.ax[2].len;
    const int hmax = p.Hq > p.Hkv ? p.Hq : p.Hkv;
    const long long vol = static_cast<long long>(n0) * n1 * n2;
    long long id = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (id >= vol * p.B * hmax) return;
    const int h = static_cast<int>(id % hmax);
    id /= hmax;
    const int b = static_cast<int>(id / vol);
    long long r = id - b * vol;
    const int i2 = static_cast<int>(r % n2);
    r /= n2;
    const int i1 = static_cast<int>(r % n1), i0 = static_cast<int>(r / n1);
    const int pos[3] = {i0, i1, i2};
    bool keep = true;
    for (int ax = 0; ax < 3; ++ax) {
        const Axis& A = p.ax[ax];
        const int L = a.lens[b * 3 + ax];
        keep = keep && L >= A.k * A.dil && L <= A.len && !(!A.causal && A.dil == 1 && (A.k % 2) == 0 && A.k == L) &&
               pos[ax] < L;
    }
    if (keep) return;
    for (int t = 0; t < a.n; ++t) {
        const PadTarget& g = a.t[t];
        if (h >= g.heads) continue;
        const long long row = b * g.lay.b + static_cast<long long>(i0) * g.lay.s0 +
                              static_cast<long long>(i1) * g.lay.s1 + static_cast<long long>(i2) * g.lay.s2 +
                              h * g.lay.h;
        char* at = static_cast<char*>(g.base) + row * g.esz;
        if (g.width == 1) {
            *reinterpret_cast<float*>(at) = 0.f;
        } else {
            for (int c = 0; c < g.width * g.esz; c += 16) *reinterpret_cast<uint4*>(at + c) = make_uint4(0, 0, 0, 0);
        }
    }
}

hipError_t varlen_pad_zero(const Prob& p, const int* lens, std::initializer_list<PadTarget> targets, hipStream_t s) {
    PadArgs a{};
    a.p = p;
    a.lens = lens;
    for (const PadTarget& t : targets) a.t[a.n++] = t;
    const long long n =
        static_cast<long long>(p.B) * p.ax[0].len * p.ax[1].len * p.ax[2].len * (p.Hq > p.Hkv ? p.Hq : p.Hkv);
    NA_LAUNCH("na_varlen_pad_zero", k_varlen_pad_zero, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s,
              a);
    return hipGetLastError();
}

template <typename T, int D>
hipError_t launch_varlen_fwd(const Prob& p, const int* lens, const void* q, Lay lq, const void* k, Lay lk,
                             const void* v, Lay lv, void* o, Lay lo, float* lse, Lay ll, hipStream_t s) {
    TileShape ts{};
    if (!choose_tile(p, kForward, D, ts, 0, true)) return hipErrorInvalidValue;
    const hipError_t e =
        ts.rowshift > 5
            ? run_fwd<T, D, kLayGeneral, true, false, true>(p, ts, q, lq, k, lk, v, lv, o, lo, lse, ll, nullptr, s, lens)
            : run_fwd<T, D, kLayGeneral, false, false, true>(p, ts, q, lq, k, lk, v, lv, o, lo, lse, ll, nullptr, s,
                                                             lens);
    if (e != hipSuccess) return e;
    return varlen_pad_zero(p, lens, {PadTarget{o, to_k(lo), p.Hq, p.Dv, 2}, PadTarget{lse, to_k(ll), p.Hq, 1, 4}}, s);
}

template <typename T, int D>
hipError_t launch_varlen_bwd(const Prob& p, const int* lens, const void* q, Lay lq, const void* k, Lay lk,
                             const void* v, Lay lv, const void* o, Lay lo, const void* dout, Lay ldo, const float* lse,
                             Lay ll, void* dq, Lay ldq, void* dk, Lay ldk, void* dv, Lay ldv, float* delta, Lay lde,
                             hipStream_t s) {
    TileShape tq{}, tk{};
    if (!choose_tile(p, kBackwardQ, D, tq, 0, true) || !choose_tile(p, kBackwardKV, D, tk, 0, true))
        return hipErrorInvalidValue;
    hipError_t e = tq.rowshift > 5
                       ? run_bwd_q<T, D, kLayGeneral, true, false, true>(p, tq, q, lq, k, lk, v, lv, o, lo, dout, ldo,
                                                                         lse, ll, nullptr, Lay{}, dq, ldq, delta, lde,
                                                                         nullptr, s, lens)
                       : run_bwd_q<T, D, kLayGeneral, false, false, true>(p, tq, q, lq, k, lk, v, lv, o, lo, dout, ldo,
                                                                          lse, ll, nullptr, Lay{}, dq, ldq, delta, lde,
                                                                          nullptr, s, lens);
    if (e != hipSuccess) return e;
    e = tk.rowshift > 5 ? run_bwd_kv<T, D, kLayGeneral, true, true>(p, tk, q, lq, k, lk, v, lv, dout, ldo, lse, ll,
                                                                     delta, lde, dk, ldk, dv, ldv, s, lens)
                        : run_bwd_kv<T, D, kLayGeneral, false, true>(p, tk, q, lq, k, lk, v, lv, dout, ldo, lse, ll,
                                                                      delta, lde, dk, ldk, dv, ldv, s, lens);
    if (e != hipSuccess) return e;
    return varlen_pad_zero(p, lens,
                           {PadTarget{dq, to_k(ldq), p.Hq, p.Dqk, 2}, PadTarget{dk, to_k(ldk), p.Hkv, p.Dqk, 2},
                            PadTarget{dv, to_k(ldv), p.Hkv, p.Dv, 2}, PadTarget{delta, to_k(lde), p.Hq, 1, 4}},
                           s);
}

// Split kernels: one staged operand plus a row block per wave.  Heads of q
// and k/v are equal for the split ops (rep 1).
size_t split_lds_bytes(const Prob& p, const TileShape& ts, int D) {
    return lds_bytes(kSplit, ts.slots, D) + static_cast<size_t>(ts.waves) * row_block_entries(p) * 2;
}

template <typename T, int D, bool SAME>
hipError_t run_dot_as(const char* name, const Prob& p, const void* a, Lay la, const void* x, Lay lx, void* o, Lay lo,
                   float mul, float fill, const void* bias, hipStream_t s) {
    TileShape ts{};
    if (!choose_tile(p, kSplit, D, ts)) return hipErrorInvalidValue;
    auto kern = bias ? k_dot_mfma<T, D, SAME, false, true> : k_dot_mfma<T, D, SAME>;
    const size_t shm = split_lds_bytes(p, ts, D);
    hipError_t e = allow_lds(kern, shm);
    if (e != hipSuccess) return e;
    fit_h_per(p, ts, resident_blocks(kern, 64 * ts.waves, shm));
    if (flat_walk(p, ts, false)) {
        kern = bias ? k_dot_mfma<T, D, SAME, true, true> : k_dot_mfma<T, D, SAME, true>;
        if ((e = allow_lds(kern, shm)) != hipSuccess) return e;
    }
    const int* geo = geometry_table(p, ts, false, s);
    NA_LAUNCH(name, kern, dim3(static_cast<unsigned>(grid_blocks(p, ts))), dim3(64 * ts.waves), shm, s, p, ts, geo,
              (const T*)a, to_k(la), (const T*)x, to_k(lx), (T*)o, to_k(lo), mul, fill, (const T*)bias);
    return hipGetLastError();
}

template <typename T, int D>
hipError_t run_dot(const char* name, const Prob& p, const void* a, Lay la, const void* x, Lay lx, void* o, Lay lo,
                   float mul, float fill, const void* bias, hipStream_t s) {
    if (same_lay(la, lx)) return run_dot_as<T, D, true>(name, p, a, la, x, lx, o, lo, mul, fill, bias, s);
    return run_dot_as<T, D, false>(name, p, a, la, x, lx, o, lo, mul, fill, bias, s);
}

template <typename T, int D, bool SAME>
hipError_t run_wsum_as(const char* name, const Prob& p, const void* w, Lay lw, const void* x, Lay lx, void* o, Lay lo,
                    float mul, hipStream_t s) {
    TileShape ts{};
    if (!choose_tile(p, kSplit, D, ts)) return hipErrorInvalidValue;
    auto kern = k_wsum_mfma<T, D, SAME>;
    const size_t shm = split_lds_bytes(p, ts, D);
    hipError_t e = allow_lds(kern, shm);
    if (e != hipSuccess) return e;
    fit_h_per(p, ts, resident_blocks(kern, 64 * ts.waves, shm));
    if (flat_walk(p, ts, false)) {
        kern = k_wsum_mfma<T, D, SAME, true>;
        if ((e = allow_lds(kern, shm)) != hipSuccess) return e;
    }
    const int* geo = geometry_table(p, ts, false, s);
    const WsumArgs<T> a{p, ts, geo, (const T*)w, (const T*)x, (T*)o, to_k(lw), to_k(lx), to_k(lo), mul};
    NA_LAUNCH(name, kern, dim3(static_cast<unsigned>(grid_blocks(p, ts))), dim3(64 * ts.waves), shm, s, a);
    return hipGetLastError();
}

template <typename T, int D>
hipError_t run_wsum(const char* name, const Prob& p, const void* w, Lay lw, const void* x, Lay lx, void* o, Lay lo,
                    float mul, hipStream_t s) {
    if (same_lay(lx, lo)) return run_wsum_as<T, D, true>(name, p, w, lw, x, lx, o, lo, mul, s);
    return run_wsum_as<T, D, false>(name, p, w, lw, x, lx, o, lo, mul, s);
}

// Key-side split kernel: the staged operand, OFF (one int per slot) and the
// slots' rows of KV 16-bit entries.
size_t split_key_lds_bytes(const Prob& p, const TileShape& ts, int D) {
    return lds_bytes(kSplitKey, ts.slots, D) + static_cast<size_t>(ts.slots) * (4 + 2 * key_row_pitch(p));
}

template <typename T, int D, bool SAME>
hipError_t run_wsum_key_as(const char* name, const Prob& p, const void* w, Lay lw, const void* x, Lay lx, void* o,
                        Lay lo, float mul, hipStream_t s) {
    TileShape ts{};
    if (!choose_tile(p, kSplitKey, D, ts)) return hipErrorInvalidValue;
    auto kern = k_wsum_key_mfma<T, D, SAME>;
    const size_t shm = split_key_lds_bytes(p, ts, D);
    hipError_t e = allow_lds(kern, shm);
    if (e != hipSuccess) return e;
    fit_h_per(p, ts, resident_blocks(kern, 64 * ts.waves, shm));
    if (flat_walk(p, ts, true)) {
        kern = k_wsum_key_mfma<T, D, SAME, true>;
        if ((e = allow_lds(kern, shm)) != hipSuccess) return e;
    }
    const int* geo = geometry_table(p, ts, true, s);
    const WsumArgs<T> a{p, ts, geo, (const T*)w, (const T*)x, (T*)o, to_k(lw), to_k(lx), to_k(lo), mul};
    NA_LAUNCH(name, kern, dim3(static_cast<unsigned>(grid_blocks(p, ts))), dim3(64 * ts.waves), shm, s, a);
    return hipGetLastError();
}

template <typename T, int D>
hipError_t run_wsum_key(const char* name, const Prob& p, const void* w, Lay lw, const void* x, Lay lx, void* o,
                        Lay lo, float mul, hipStream_t s) {
    if (same_lay(lx, lo)) return run_wsum_key_as<T, D, true>(name, p, w, lw, x, lx, o, lo, mul, s);
    return run_wsum_key_as<T, D, false>(name, p, w, lw, x, lx, o, lo, mul, s);
}

// Rows of KV entries: non-negative strides, and every entry of one (batch,
// head) at a byte offset inside the buffer range of a row resource
// (kPlaneBytes): the row kernels form byte offsets as 2 * (element offset)
// in 32-bit arithmetic, and an access past the range would read zeros or
// drop the store without any error.
bool rows_fit(const Prob& p, const Lay& l) {
    if (l.b < 0 || l.s0 < 0 || l.s1 < 0 || l.s2 < 0 || l.h < 0) return false;
    const long long vol = (static_cast<long long>(p.ax[0].len) - 1) * l.s0 +
                          (static_cast<long long>(p.ax[1].len) - 1) * l.s1 +
                          (static_cast<long long>(p.ax[2].len) - 1) * l.s2 + p.kv;
    return (vol + 8) * 2 < kPlaneBytes;
}

// The tile kernels walk every query position of an axis up to its length: a
// split op whose attention tensor covers fewer query positions than the
// value tensor has (allowed at stride 1) goes to the vector kernels, which
// decode over the attention extent.
bool full_query_extent(const Prob& p) {
    for (int a = 0; a < 3; ++a)
        if (p.ax[a].st != 1 || p.ax[a].out != p.ax[a].len) return false;
    return true;
}

template <typename T, int D, int LAY>
void audit_fused(LdsAudit& a) {
    audit_one(k_fwd_mfma<T, D, LAY, false, false>, "k_fwd_mfma", a);
    audit_one(k_fwd_mfma<T, D, LAY, true, false>, "k_fwd_mfma (wide)", a);
    audit_one(k_bwd_q_mfma<T, D, LAY, false, false>, "k_bwd_q_mfma", a);
    audit_one(k_bwd_q_mfma<T, D, LAY, true, false>, "k_bwd_q_mfma (wide)", a);
    audit_one(k_bwd_q_mfma<T, D, LAY, false, false, false, false, true>, "k_bwd_q_mfma (P dP)", a);
    audit_one(k_bwd_q_mfma<T, D, LAY, true, false, false, false, true>, "k_bwd_q_mfma (wide, P dP)", a);
    audit_one(k_bwd_kv_mfma<T, D, LAY, false>, "k_bwd_kv_mfma", a);
    audit_one(k_bwd_kv_mfma<T, D, LAY, true>, "k_bwd_kv_mfma (wide)", a);
    if constexpr (kHasFlat<LAY, false, false, false>) {
        audit_one(k_fwd_mfma<T, D, LAY, false, false, false, true>, "k_fwd_mfma (flat)", a);
        audit_one(k_bwd_q_mfma<T, D, LAY, false, false, false, true>, "k_bwd_q_mfma (flat)", a);
        audit_one(k_bwd_q_mfma<T, D, LAY, false, false, false, true, true>, "k_bwd_q_mfma (flat, P dP)", a);
        audit_one(k_bwd_kv_mfma<T, D, LAY, false, false, true>, "k_bwd_kv_mfma (flat)", a);
    }
}

template <typename T, int D>
void audit_varlen(LdsAudit& a) {
    audit_one(k_fwd_mfma<T, D, kLayGeneral, false, false, true>, "k_fwd_mfma (varlen)", a);
    audit_one(k_fwd_mfma<T, D, kLayGeneral, true, false, true>, "k_fwd_mfma (wide, varlen)", a);
    audit_one(k_bwd_q_mfma<T, D, kLayGeneral, false, false, true>, "k_bwd_q_mfma (varlen)", a);
    audit_one(k_bwd_q_mfma<T, D, kLayGeneral, true, false, true>, "k_bwd_q_mfma (wide, varlen)", a);
    audit_one(k_bwd_kv_mfma<T, D, kLayGeneral, false, true>, "k_bwd_kv_mfma (varlen)", a);
    audit_one(k_bwd_kv_mfma<T, D, kLayGeneral, true, true>, "k_bwd_kv_mfma (wide, varlen)", a);
}

template <typename T, int D>
void audit_dim(LdsAudit& a) {
    audit_varlen<T, D>(a);
    audit_one(k_fwd_mfma<T, D, kLayGeneral, false, true>, "k_fwd_mfma (global keys)", a);
    audit_one(k_fwd_mfma<T, D, kLayGeneral, true, true>, "k_fwd_mfma (wide, global keys)", a);
    audit_one(k_bwd_q_mfma<T, D, kLayGeneral, false, true>, "k_bwd_q_mfma (global keys)", a);
    audit_one(k_bwd_q_mfma<T, D, kLayGeneral, true, true>, "k_bwd_q_mfma (wide, global keys)", a);
    audit_fused<T, D, kLayGeneral>(a);
    audit_fused<T, D, kLayOne>(a);
    audit_fused<T, D, kLayTwo>(a);
    audit_fused<T, D, kLayFour>(a);
    audit_one(k_dot_mfma<T, D, true>, "k_dot_mfma", a);
    audit_one(k_dot_mfma<T, D, false>, "k_dot_mfma", a);
    audit_one(k_wsum_mfma<T, D, true>, "k_wsum_mfma", a);
    audit_one(k_wsum_mfma<T, D, false>, "k_wsum_mfma", a);
    audit_one(k_wsum_key_mfma<T, D, true>, "k_wsum_key_mfma", a);
    audit_one(k_wsum_key_mfma<T, D, false>, "k_wsum_key_mfma", a);
    audit_one(k_dot_mfma<T, D, true, true>, "k_dot_mfma (flat)", a);
    audit_one(k_dot_mfma<T, D, false, true>, "k_dot_mfma (flat)", a);
    audit_one(k_dot_mfma<T, D, true, false, true>, "k_dot_mfma (bias)", a);
    audit_one(k_dot_mfma<T, D, false, false, true>, "k_dot_mfma (bias)", a);
    audit_one(k_dot_mfma<T, D, true, true, true>, "k_dot_mfma (flat, bias)", a);
    audit_one(k_dot_mfma<T, D, false, true, true>, "k_dot_mfma (flat, bias)", a);
    audit_one(k_wsum_mfma<T, D, true, true>, "k_wsum_mfma (flat)", a);
    audit_one(k_wsum_mfma<T, D, false, true>, "k_wsum_mfma (flat)", a);
    audit_one(k_wsum_key_mfma<T, D, true, true>, "k_wsum_key_mfma (flat)", a);
    audit_one(k_wsum_key_mfma<T, D, false, true>, "k_wsum_key_mfma (flat)", a);
}

// Head dim 96 has fused instances only (the split ops keep the vector
// kernels there).
template <typename T>
void audit_dim96(LdsAudit& a) {
    audit_one(k_fwd_mfma<T, 96, kLayGeneral, false, true>, "k_fwd_mfma (global keys)", a);
    audit_one(k_fwd_mfma<T, 96, kLayGeneral, true, true>, "k_fwd_mfma (wide, global keys)", a);
    audit_one(k_bwd_q_mfma<T, 96, kLayGeneral, false, true>, "k_bwd_q_mfma (global keys)", a);
    audit_one(k_bwd_q_mfma<T, 96, kLayGeneral, true, true>, "k_bwd_q_mfma (wide, global keys)", a);
    audit_fused<T, 96, kLayGeneral>(a);
    audit_fused<T, 96, kLayOne>(a);
    audit_fused<T, 96, kLayTwo>(a);
    audit_fused<T, 96, kLayFour>(a);
    audit_varlen<T, 96>(a);
}

const LdsAudit& lds_audit() {
    static const LdsAudit result = [] {
        LdsAudit a;
        audit_dim96<bf16>(a);
        audit_dim96<f16>(a);
        audit_dim<bf16, 32>(a);
        audit_dim<bf16, 64>(a);
        audit_dim<bf16, 128>(a);
        audit_dim<f16, 32>(a);
        audit_dim<f16, 64>(a);
        audit_dim<f16, 128>(a);
        return a;
    }();
    return result;
}

}  // namespace

NoDeviceAlloc::NoDeviceAlloc() : prev_(t_no_device_alloc) { t_no_device_alloc = true; }
NoDeviceAlloc::~NoDeviceAlloc() { t_no_device_alloc = prev_; }
bool device_alloc_allowed() { return !t_no_device_alloc; }

bool mfma_static_lds_ok() { return lds_audit().bad == 0; }

int mfma_lds_audit(int* checked) {
    const LdsAudit& a = lds_audit();
    if (checked) *checked = a.checked;
    return a.bad == 0 ? 1 : 0;
}

bool mfma_split_eligible(const Prob& p, int dtype, int D, bool aligned, const Lay& rows,
                         std::initializer_list<Lay> staged) {
    if (dtype == NATTEN_F32 || !aligned || p.rep != 1 || !mfma_static_lds_ok()) return false;
    if (!(D == 32 || D == 64 || D == 128) || p.kv > kSplitMaxKV) return false;
    if (static_cast<size_t>(4) * row_block_entries(p) * 2 > kSplitRowsBudget) return false;
    if (!full_query_extent(p)) return false;
    TileShape ts{};
    if (!choose_tile(p, kSplit, D, ts) || grid_blocks(p, ts) >= (1LL << 31)) return false;
    return rows_fit(p, rows) && offsets_fit(p, staged);
}

bool mfma_split_key_eligible(const Prob& p, int dtype, int D, bool aligned, const Lay& rows,
                             std::initializer_list<Lay> staged) {
    if (dtype == NATTEN_F32 || !aligned || p.rep != 1 || !mfma_static_lds_ok()) return false;
    if (!(D == 32 || D == 64 || D == 128) || p.kv > kSplitMaxKV) return false;
    if (!full_query_extent(p)) return false;
    TileShape ts{};
    if (!choose_tile(p, kSplitKey, D, ts) || grid_blocks(p, ts) >= (1LL << 31)) return false;
    if (split_key_lds_bytes(p, ts, D) > kSplitKeyLds)
        return false;
    return rows_fit(p, rows) && offsets_fit(p, staged);
}

hipError_t mfma_split_wsum_key(const char* name, const Prob& p, int D, const void* w, Lay lw, const void* x, Lay lx,
                               void* o, Lay lo, float mul, int dtype, hipStream_t s) {
    // the 8x8 key tiles first (2-D, head dim 32 / 64, K <= 9); their
    // operands' alignment is the one mfma_split_key_eligible checked
    if (lean_wsum_key_eligible(p, dtype, D, true, lw, lx, lo)) {
        const hipError_t e = lean_wsum_key(name, p, D, w, lw, x, lx, o, lo, mul, dtype, s);
        if (e != hipErrorNotSupported) return e;
    }
#define NA_WSUMK(T, DD) return run_wsum_key<T, DD>(name, p, w, lw, x, lx, o, lo, mul, s)
    if (dtype == NATTEN_BF16) {
        if (D == 32) NA_WSUMK(bf16, 32);
        if (D == 64) NA_WSUMK(bf16, 64);
        NA_WSUMK(bf16, 128);
    }
    if (D == 32) NA_WSUMK(f16, 32);
    if (D == 64) NA_WSUMK(f16, 64);
    NA_WSUMK(f16, 128);
#undef NA_WSUMK
}

hipError_t mfma_split_dot(const char* name, const Prob& p, int D, const void* a, Lay la, const void* x, Lay lx,
                          void* o, Lay lo, float mul, float fill, int dtype, hipStream_t s, const void* bias) {
#define NA_DOT(T, DD) return run_dot<T, DD>(name, p, a, la, x, lx, o, lo, mul, fill, bias, s)
    if (dtype == NATTEN_BF16) {
        if (D == 32) NA_DOT(bf16, 32);
        if (D == 64) NA_DOT(bf16, 64);
        NA_DOT(bf16, 128);
    }
    if (D == 32) NA_DOT(f16, 32);
    if (D == 64) NA_DOT(f16, 64);
    NA_DOT(f16, 128);
#undef NA_DOT
}

hipError_t mfma_split_wsum(const char* name, const Prob& p, int D, const void* w, Lay lw, const void* x, Lay lx,
                           void* o, Lay lo, float mul, int dtype, hipStream_t s) {
#define NA_WSUM(T, DD) return run_wsum<T, DD>(name, p, w, lw, x, lx, o, lo, mul, s)
    if (dtype == NATTEN_BF16) {
        if (D == 32) NA_WSUM(bf16, 32);
        if (D == 64) NA_WSUM(bf16, 64);
        NA_WSUM(bf16, 128);
    }
    if (D == 32) NA_WSUM(f16, 32);
    if (D == 64) NA_WSUM(f16, 64);
    NA_WSUM(f16, 128);
#undef NA_WSUM
}

// The tile kernels index q and dq, like out, lse and dO, by query item: on
// an axis with stride s item t is position s*t, so their spatial strides
// scale by s.
static Lay item_lay(const Prob& p, Lay l) {
    l.s0 *= p.ax[0].st;
    l.s1 *= p.ax[1].st;
    l.s2 *= p.ax[2].st;
    return l;
}

bool mfma_eligible(const Prob& p, int dtype, int D, bool aligned, bool backward, bool global) {
    if (dtype == NATTEN_F32 || !aligned || !(p.scale > 0.f) || !mfma_static_lds_ok()) return false;
    if (p.Dqk != p.Dv || !(D == 32 || D == 64 || D == 96 || D == 128)) return false;
    // a strided axis must be one residue class (its query items then sit at
    // class coordinates stride * t); global keys come at stride 1 only
    for (int a = 0; a < 3; ++a)
        if (p.ax[a].st != 1 && (p.ax[a].dil != 1 || global)) return false;
    // tile indices (the launch grid) stay in 31 bits
    const size_t extra = global ? global_lds(D) : 0;
    TileShape ts{};
    if (!choose_tile(p, kForward, D, ts, extra) || grid_blocks(p, ts) >= (1LL << 31)) return false;
    if (backward) {
        if (!choose_tile(p, kBackwardQ, D, ts, extra) || grid_blocks(p, ts) >= (1LL << 31)) return false;
        if (!choose_tile(p, kBackwardKV, D, ts) || grid_blocks(p, ts) >= (1LL << 31)) return false;
    }
    return true;
}

bool mfma_offsets_fit(const Prob& p, std::initializer_list<Lay> lays) { return offsets_fit(p, lays); }

bool mfma_varlen_eligible(const Prob& p, int dtype, int D, bool aligned, bool backward) {
    if (dtype == NATTEN_F32 || !aligned || !(p.scale > 0.f) || !mfma_static_lds_ok()) return false;
    if (p.Dqk != p.Dv || !(D == 32 || D == 64 || D == 96 || D == 128)) return false;
    for (int a = 0; a < 3; ++a)
        if (p.ax[a].st != 1) return false;
    TileShape ts{};
    if (!choose_tile(p, kForward, D, ts, 0, true) || grid_blocks(p, ts) >= (1LL << 31)) return false;
    if (backward) {
        if (!choose_tile(p, kBackwardQ, D, ts, 0, true) || grid_blocks(p, ts) >= (1LL << 31)) return false;
        if (!choose_tile(p, kBackwardKV, D, ts, 0, true) || grid_blocks(p, ts) >= (1LL << 31)) return false;
    }
    // the padding kernel's grid: one thread per (batch, position, head)
    return static_cast<long long>(p.B) * p.ax[0].len * p.ax[1].len * p.ax[2].len * (p.Hq > p.Hkv ? p.Hq : p.Hkv) <
           (1LL << 31) * 255LL;
}

hipError_t mfma_varlen_forward(const Prob& p, const int* lens, const void* q, Lay lq, const void* k, Lay lk,
                               const void* v, Lay lv, void* o, Lay lo, float* lse, Lay ll, int dtype, hipStream_t s) {
#define NA_VFWD(T, DD) return launch_varlen_fwd<T, DD>(p, lens, q, lq, k, lk, v, lv, o, lo, lse, ll, s)
    if (dtype == NATTEN_BF16) {
        if (p.Dqk == 32) NA_VFWD(bf16, 32);
        if (p.Dqk == 64) NA_VFWD(bf16, 64);
        if (p.Dqk == 96) NA_VFWD(bf16, 96);
        NA_VFWD(bf16, 128);
    }
    if (p.Dqk == 32) NA_VFWD(f16, 32);
    if (p.Dqk == 64) NA_VFWD(f16, 64);
    if (p.Dqk == 96) NA_VFWD(f16, 96);
    NA_VFWD(f16, 128);
#undef NA_VFWD
}

hipError_t mfma_varlen_backward(const Prob& p, const int* lens, const void* q, Lay lq, const void* k, Lay lk,
                                const void* v, Lay lv, const void* o, Lay lo, const void* dout, Lay ldo,
                                const float* lse, Lay ll, void* dq, Lay ldq, void* dk, Lay ldk, void* dv, Lay ldv,
                                float* delta, Lay lde, int dtype, hipStream_t s) {
#define NA_VBWD(T, DD)                                                                                                 \
    return launch_varlen_bwd<T, DD>(p, lens, q, lq, k, lk, v, lv, o, lo, dout, ldo, lse, ll, dq, ldq, dk, ldk, dv, ldv, \
                                    delta, lde, s)
    if (dtype == NATTEN_BF16) {
        if (p.Dqk == 32) NA_VBWD(bf16, 32);
        if (p.Dqk == 64) NA_VBWD(bf16, 64);
        if (p.Dqk == 96) NA_VBWD(bf16, 96);
        NA_VBWD(bf16, 128);
    }
    if (p.Dqk == 32) NA_VBWD(f16, 32);
    if (p.Dqk == 64) NA_VBWD(f16, 64);
    if (p.Dqk == 96) NA_VBWD(f16, 96);
    NA_VBWD(f16, 128);
#undef NA_VBWD
}

hipError_t mfma_forward(const Prob& p, const void* q, Lay lq, const void* k, Lay lk, const void* v, Lay lv, void* o,
                        Lay lo, float* lse, Lay ll, int dtype, hipStream_t s, const GlobalSet* g) {
    lq = item_lay(p, lq);
#define NA_FWD(T, DD) return launch_fwd<T, DD>(p, q, lq, k, lk, v, lv, o, lo, lse, ll, g, s)
    if (dtype == NATTEN_BF16) {
        if (p.Dqk == 32) NA_FWD(bf16, 32);
        if (p.Dqk == 64) NA_FWD(bf16, 64);
        if (p.Dqk == 96) NA_FWD(bf16, 96);
        NA_FWD(bf16, 128);
    }
    if (p.Dqk == 32) NA_FWD(f16, 32);
    if (p.Dqk == 64) NA_FWD(f16, 64);
    if (p.Dqk == 96) NA_FWD(f16, 96);
    NA_FWD(f16, 128);
#undef NA_FWD
}

hipError_t mfma_backward(const Prob& p, const void* q, Lay lq, const void* k, Lay lk, const void* v, Lay lv,
                         const void* o, Lay lo, const void* dout, Lay ldo, const float* lse, Lay ll,
                         const float* dlse, Lay ldl, void* dq, Lay ldq, void* dk, Lay ldk, void* dv, Lay ldv,
                         float* delta, Lay lde, int dtype, hipStream_t s, const GlobalSet* g) {
    lq = item_lay(p, lq);
    ldq = item_lay(p, ldq);
#define NA_BWD(T, DD)                                                                                            \
    return launch_bwd<T, DD>(p, q, lq, k, lk, v, lv, o, lo, dout, ldo, lse, ll, dlse, ldl, dq, ldq, dk, ldk, dv, \
                             ldv, delta, lde, g, s)
    if (dtype == NATTEN_BF16) {
        if (p.Dqk == 32) NA_BWD(bf16, 32);
        if (p.Dqk == 64) NA_BWD(bf16, 64);
        if (p.Dqk == 96) NA_BWD(bf16, 96);
        NA_BWD(bf16, 128);
    }
    if (p.Dqk == 32) NA_BWD(f16, 32);
    if (p.Dqk == 64) NA_BWD(f16, 64);
    if (p.Dqk == 96) NA_BWD(f16, 96);
    NA_BWD(f16, 128);
#undef NA_BWD
}

}  // namespace na

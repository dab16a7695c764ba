/*
 * natten_hip.h -- C ABI of the MI355X (gfx950) neighbourhood-attention library
 * (libnatten_hip.so).
 *
 * Plain pointers, sizes and element strides; no torch types.  The caller owns
 * every buffer (inputs, outputs, workspaces) and the stream.  The only device
 * memory the library allocates itself is the tile geometry of each problem
 * shape (a few hundred bytes per tile of the general tile kernels, 64 bytes
 * per 8x8 tile of the 2-D ones), built on the first call with that shape
 * outside stream capture, uploaded by an asynchronous copy on that call's
 * stream (no host synchronisation) and kept until the process ends; a later
 * call on another stream waits for that copy on its own stream.  During
 * capture, in natten_hip_backward_noalloc, or when the general tables would
 * pass 64 MiB, the general kernels compute the same geometry themselves and
 * the 2-D ones leave the problem to them.  Workspaces (global keys, the
 * relative-position-bias gradient) are the caller's, sized by the
 * natten_hip_*_workspace queries.  Every entry point returns 0 on success and a
 * non-zero natten_status_t otherwise, with a message available from
 * natten_hip_last_error().  Launches are asynchronous on `stream` (a
 * hipStream_t; NULL = the default stream).
 *
 * Tensor conventions (spatial-first, as the reference's public API):
 *   q      [B, *sp,     Hq,  Dqk]      k  [B, *sp, Hkv, Dqk]    v [B, *sp, Hkv, Dv]
 *   out    [B, *sp_out, Hq,  Dv]       lse / delta [B, *sp_out, Hq]  (fp32)
 *   attn   [B, *sp_out, H,   KV]       KV = prod(kernel), row-major over the axes
 * `*sp` always has three axes here, outermost first: a rank-r problem pads the
 * leading 3-r axes with length 1, kernel 1, dilation 1, stride 1, non-causal.
 * Each tensor is described by a natten_layout_t of element strides; the
 * innermost dimension (D, or KV for attn, or nothing for lse) must be
 * contiguous.
 *
 * Reference interfaces these entry points replace (paths under
 * /root/reference/src/natten_mps):
 *   natten_hip_forward         _core/metal.py:452-558  na{1,2,3}d_fused_forward
 *                              (and the forward_with_lse hooks :592-621,
 *                              :845-874, :1051-1080)
 *   natten_hip_qk_forward      _core/metal.py:181-224, 273-338, 882-949  na{r}d_qk_forward
 *   natten_hip_av_forward      _core/metal.py:227-265, 341-401, 952-1012 na{r}d_av_forward
 *   natten_hip_backward        _core/metal.py:1088-1330 na{r}d_fused_backward
 *   natten_hip_qk_backward     _core/metal.py:1352-1470 (q/k backward kernels)
 *   natten_hip_av_backward     _core/metal.py:1473-1611 (a/v backward kernels)
 *   natten_hip_neighborhood_map _core/pure.py:91-129, 335-387 (index maps; the
 *                              Metal backend has no equivalent export)
 *   natten_hip_varlen_forward  _core/metal.py:624-811 na{1,2,3}d_varlen_forward
 *                              (and _core/pure.py:573-673)
 *   natten_hip_varlen_backward functional.py:721-754, 804-835, 860-893 (the
 *                              per-sample autograd loops of _NA{1,2,3}DVarlenFunction)
 *   natten_hip_rpb_qk_forward  extras/allin1/functional.py:47-100, 153-250 and
 *                              extras/allin1/metal.py (natten{1,2}dqkrpb)
 *   natten_hip_rpb_av_forward  extras/allin1/functional.py:103-150, 253-325 (natten{1,2}dav)
 *   natten_hip_rpb_qk_backward extras/allin1/functional.py:333-365, 413-448 (QK+RPB backward;
 *   natten_hip_rpb_qk_backward_ws  the same op with the caller's workspace for
 *   natten_hip_rpb_dbias_workspace the bias gradient's partial sums)
 *   natten_hip_rpb_av_backward extras/allin1/functional.py:368-400, 451-485 (AV backward)
 */
#ifndef NATTEN_HIP_H
#define NATTEN_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NATTEN_HIP_ABI_VERSION 1

typedef enum {
    NATTEN_OK = 0,
    NATTEN_ERR_INVALID = 1,     /* bad shape / parameter / alignment */
    NATTEN_ERR_UNSUPPORTED = 2, /* valid input outside what the kernels cover */
    NATTEN_ERR_LAUNCH = 3       /* HIP launch error */
} natten_status_t;

typedef enum { NATTEN_F32 = 0, NATTEN_F16 = 1, NATTEN_BF16 = 2 } natten_dtype_t;

typedef struct {
    int32_t batch;
    int32_t heads_q;       /* query heads (= heads of attn/out)                  */
    int32_t heads_kv;      /* key/value heads; heads_q % heads_kv == 0 (GQA)     */
    int32_t dim_qk;        /* head dim of q and k                                */
    int32_t dim_v;         /* head dim of v and out                              */
    int32_t dtype;         /* natten_dtype_t of q, k, v, out, attn and gradients */
    int32_t has_scale;     /* split QK / its backward: 0 = logits left unscaled  */
    float scale;           /* softmax scale (fused ops), logit scale (split QK)  */
    int32_t length[3];     /* key/value spatial extent per axis                  */
    int32_t out_length[3]; /* query positions per axis (ceil(len/stride), or the
                              attn extent for the split ops at stride 1)         */
    int32_t kernel[3];
    int32_t dilation[3];
    int32_t stride[3];
    int32_t causal[3];
} natten_problem_t;

typedef struct {
    int64_t batch;
    int64_t axis[3];
    int64_t head;
} natten_layout_t;

/* Library / ABI introspection. */
int natten_hip_abi_version(void);
const char *natten_hip_last_error(void);

/* Audit of the MFMA tile kernels (no counterpart in the reference): they
 * address their staged operands at a constant LDS offset, which is sound
 * only while no kernel instance declares static LDS.  Every instance is
 * checked once per process (needs a device); returns 1 when the tile path
 * is enabled, 0 when an instance has static LDS (the vector kernels then
 * take every call and a message names it on stderr).  *checked (may be
 * NULL) receives the number of instances whose attributes were read. */
int natten_hip_mfma_lds_check(int32_t *checked);

/* Fused forward: out = softmax(scale * q k^T over each neighbourhood) v, and
 * lse = log-sum-exp of the scaled logits (natural log).  Native GQA: query
 * head h reads key/value head h / (Hq/Hkv). */
int natten_hip_forward(const natten_problem_t *p,
                       const void *q, const natten_layout_t *lq,
                       const void *k, const natten_layout_t *lk,
                       const void *v, const natten_layout_t *lv,
                       void *out, const natten_layout_t *lo,
                       float *lse, const natten_layout_t *llse,
                       void *stream);

/* Fused backward.  Inputs: q, k, v, the forward's out and lse, dout, and an
 * optional upstream gradient of lse (dlse, NULL if none).  Outputs: dq (zeroed
 * by the caller at off-stride positions when any stride > 1), dk, dv, at the
 * shapes of q, k, v (dk/dv summed over each GQA group).  delta is an fp32
 * workspace shaped like lse. */
int natten_hip_backward(const natten_problem_t *p,
                        const void *q, const natten_layout_t *lq,
                        const void *k, const natten_layout_t *lk,
                        const void *v, const natten_layout_t *lv,
                        const void *out, const natten_layout_t *lo,
                        const void *dout, const natten_layout_t *ldo,
                        const float *lse, const natten_layout_t *llse,
                        const float *dlse, const natten_layout_t *ldlse,
                        void *dq, const natten_layout_t *ldq,
                        void *dk, const natten_layout_t *ldk,
                        void *dv, const natten_layout_t *ldv,
                        float *delta, const natten_layout_t *ldelta,
                        void *stream);

/* Global keys (additional_keys / additional_values of the reference's
 * na{1,2,3}d, functional.py:74-110 and :285-299 with merge.py:21-156 -- there
 * a split NA pass, dense attention over the extra tokens and a merge of the
 * two by their log-sum-exps).  Here the extra tokens are keys that every query
 * attends besides its neighbourhood, inside the fused kernels: out is the
 * softmax over the neighbourhood and the global keys together, lse its
 * log-sum-exp.  gk / gv are [B, n_global, heads_kv, dim] (layout: batch,
 * head, and the token stride in axis[2]; axis[0], axis[1] unused).  These
 * entry points serve the MFMA tile path only (bf16/fp16, dim_qk == dim_v in
 * {32, 64, 96, 128}, stride 1, aligned operands) and return
 * NATTEN_ERR_UNSUPPORTED otherwise; natten_hip_global_supported answers that
 * from the problem alone (1 / 0; backward != 0 also checks the backward).
 * The backward also writes dgk / dgv (summed over every query of each GQA
 * group) and needs an fp32 workspace of natten_hip_global_workspace(p, n)
 * floats (-1: invalid problem). */
int natten_hip_global_supported(const natten_problem_t *p, int32_t n_global, int32_t backward);
int64_t natten_hip_global_workspace(const natten_problem_t *p, int32_t n_global);
int natten_hip_forward_global(const natten_problem_t *p,
                              const void *q, const natten_layout_t *lq,
                              const void *k, const natten_layout_t *lk,
                              const void *v, const natten_layout_t *lv,
                              const void *gk, const natten_layout_t *lgk,
                              const void *gv, const natten_layout_t *lgv,
                              int32_t n_global,
                              void *out, const natten_layout_t *lo,
                              float *lse, const natten_layout_t *llse,
                              void *stream);
int natten_hip_backward_global(const natten_problem_t *p,
                               const void *q, const natten_layout_t *lq,
                               const void *k, const natten_layout_t *lk,
                               const void *v, const natten_layout_t *lv,
                               const void *gk, const natten_layout_t *lgk,
                               const void *gv, const natten_layout_t *lgv,
                               int32_t n_global,
                               const void *out, const natten_layout_t *lo,
                               const void *dout, const natten_layout_t *ldo,
                               const float *lse, const natten_layout_t *llse,
                               const float *dlse, const natten_layout_t *ldlse,
                               void *dq, const natten_layout_t *ldq,
                               void *dk, const natten_layout_t *ldk,
                               void *dv, const natten_layout_t *ldv,
                               void *dgk, const natten_layout_t *ldgk,
                               void *dgv, const natten_layout_t *ldgv,
                               float *delta, const natten_layout_t *ldelta,
                               float *work, int64_t work_floats,
                               void *stream);

/* Allocation-free fused backward (no counterpart in the reference): the same
 * computation and results as natten_hip_backward, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  It takes no delta workspace: the delta
 * rows live in a static device array of the library, at most 4 Mi floats
 * (batch x query positions x heads_q <= 4,194,304; larger problems return
 * NATTEN_ERR_UNSUPPORTED), one copy per GPU, held until the process ends.
 * It calls no hipMalloc/hipFree: the tile kernels then compute their geometry
 * themselves unless a table for the shape already exists.  Calls that overlap
 * on one GPU share that array and race; serialise them (one stream, or
 * events). */
int natten_hip_backward_noalloc(const natten_problem_t *p,
                                const void *q, const natten_layout_t *lq,
                                const void *k, const natten_layout_t *lk,
                                const void *v, const natten_layout_t *lv,
                                const void *out, const natten_layout_t *lo,
                                const void *dout, const natten_layout_t *ldo,
                                const float *lse, const natten_layout_t *llse,
                                const float *dlse, const natten_layout_t *ldlse,
                                void *dq, const natten_layout_t *ldq,
                                void *dk, const natten_layout_t *ldk,
                                void *dv, const natten_layout_t *ldv,
                                void *stream);

/* Split QK: attn[.., kv] = q . k_neighbour (times scale if has_scale); entries
 * of causally invalid neighbours are -inf (times scale).  heads_q == heads_kv. */
int natten_hip_qk_forward(const natten_problem_t *p,
                          const void *q, const natten_layout_t *lq,
                          const void *k, const natten_layout_t *lk,
                          void *attn, const natten_layout_t *la,
                          void *stream);

/* Split AV: out = sum over valid neighbours of attn * v_neighbour. */
int natten_hip_av_forward(const natten_problem_t *p,
                          const void *attn, const natten_layout_t *la,
                          const void *v, const natten_layout_t *lv,
                          void *out, const natten_layout_t *lo,
                          void *stream);

/* Split QK backward: dq = sum dattn * k, dk = sum dattn * q over valid pairs,
 * each times scale when has_scale.  dq must be zeroed by the caller at
 * off-stride positions when any stride > 1. */
int natten_hip_qk_backward(const natten_problem_t *p,
                           const void *dattn, const natten_layout_t *lda,
                           const void *q, const natten_layout_t *lq,
                           const void *k, const natten_layout_t *lk,
                           void *dq, const natten_layout_t *ldq,
                           void *dk, const natten_layout_t *ldk,
                           void *stream);

/* Split AV backward: dattn = dout . v_neighbour (0 for invalid neighbours),
 * dv = sum attn * dout over valid pairs. */
int natten_hip_av_backward(const natten_problem_t *p,
                           const void *dout, const natten_layout_t *ldo,
                           const void *attn, const natten_layout_t *la,
                           const void *v, const natten_layout_t *lv,
                           void *dattn, const natten_layout_t *lda,
                           void *dv, const natten_layout_t *ldv,
                           void *stream);

/* The flattened neighbour index map of the fused op, computed on the device:
 * flat[o, kv] (int64, row-major over the padded three axes, causal indices
 * clamped to the axis) and valid[o, kv] (uint8), o over all query positions.
 * Same values as the reference's _build_2d/_build_3d_neighborhood. */
int natten_hip_neighborhood_map(const natten_problem_t *p,
                                int64_t *flat, uint8_t *valid,
                                void *stream);

/* Variable-length fused forward / backward.  The problem describes the
 * padded (maximum) extents, stride 1; lens (device memory, int32 [batch][3],
 * padded axes first as in `length`) holds each sample's own extent per axis,
 * with kernel * dilation <= lens[b][a] <= length[a].  Sample b attends within
 * its own extent exactly as an unpadded problem of that size would; outputs
 * and gradients at padding positions are zero (lse and delta there are 0).
 * A sample whose extents are out of range (or an even kernel equal to its
 * extent, non-causal, dilation 1) comes out all zero.  Other arguments as for
 * natten_hip_forward / natten_hip_backward. */
int natten_hip_varlen_forward(const natten_problem_t *p, const int32_t *lens,
                              const void *q, const natten_layout_t *lq,
                              const void *k, const natten_layout_t *lk,
                              const void *v, const natten_layout_t *lv,
                              void *out, const natten_layout_t *lo,
                              float *lse, const natten_layout_t *llse,
                              void *stream);

int natten_hip_varlen_backward(const natten_problem_t *p, const int32_t *lens,
                               const void *q, const natten_layout_t *lq,
                               const void *k, const natten_layout_t *lk,
                               const void *v, const natten_layout_t *lv,
                               const void *out, const natten_layout_t *lo,
                               const void *dout, const natten_layout_t *ldo,
                               const float *lse, const natten_layout_t *llse,
                               void *dq, const natten_layout_t *ldq,
                               void *dk, const natten_layout_t *ldk,
                               void *dv, const natten_layout_t *ldv,
                               float *delta, const natten_layout_t *ldelta,
                               void *stream);

/* Relative-position-bias split ops of DiNAT-style models (1-D or 2-D: the
 * padded axis 0 has length and kernel 1; stride 1, non-causal, heads_q ==
 * heads_kv).  They follow NATTEN 0.17's shifted windows: per axis, the start
 * is phase-aligned to the query's residue class mod the dilation and may be
 * negative near the borders for an even kernel, the window ends at
 * min(len, start + kernel * dilation), and a neighbour is valid when it lies
 * in [0, end).  Its bias index per axis is get_pb_start(query) + its offset,
 * clamped to [0, 2K-2].
 *   rpb_qk:  attn = q . k_neighbour + rpb[h, bias]   (-inf when invalid; the
 *            logits are not scaled: scale q beforehand); rpb may be NULL
 *   rpb_av:  out = sum over valid neighbours of attn * v_neighbour
 *   rpb_qk_backward: dq, dk over valid pairs; drpb (may be NULL) sums dattn
 *            over every entry at each bias index
 *   rpb_av_backward: dattn (0 for invalid neighbours), dv
 * rpb and drpb are contiguous [H, 2K1-1, 2K2-1] (1-D: [H, 2K-1]) in the
 * problem's dtype; attn is [B, *sp, H, K1*K2].  Odd kernels in bf16/fp16 at
 * head dims 32/64/128 run on the split MFMA tile kernels: there rpb_qk
 * rounds q . k to the dtype before adding the bias (one more rounding).
 * drpb is reduced in one pass by natten_hip_rpb_qk_backward; where
 * natten_hip_rpb_dbias_workspace(p) is positive, natten_hip_rpb_qk_backward_ws
 * given an fp32 workspace of that many floats reduces it in two passes
 * (partial sums per slice of the queries, then one fixed-order sum: the same
 * value, several times faster on large images).  A workspace that is NULL or
 * smaller takes the one-pass kernel.  0 from the query: the one pass serves
 * the problem; -1: invalid problem. */
int natten_hip_rpb_qk_forward(const natten_problem_t *p,
                              const void *q, const natten_layout_t *lq,
                              const void *k, const natten_layout_t *lk,
                              const void *rpb,
                              void *attn, const natten_layout_t *la,
                              void *stream);

int natten_hip_rpb_av_forward(const natten_problem_t *p,
                              const void *attn, const natten_layout_t *la,
                              const void *v, const natten_layout_t *lv,
                              void *out, const natten_layout_t *lo,
                              void *stream);

int natten_hip_rpb_qk_backward(const natten_problem_t *p,
                               const void *dattn, const natten_layout_t *lda,
                               const void *q, const natten_layout_t *lq,
                               const void *k, const natten_layout_t *lk,
                               void *dq, const natten_layout_t *ldq,
                               void *dk, const natten_layout_t *ldk,
                               void *drpb,
                               void *stream);

int64_t natten_hip_rpb_dbias_workspace(const natten_problem_t *p);
int natten_hip_rpb_qk_backward_ws(const natten_problem_t *p,
                                  const void *dattn, const natten_layout_t *lda,
                                  const void *q, const natten_layout_t *lq,
                                  const void *k, const natten_layout_t *lk,
                                  void *dq, const natten_layout_t *ldq,
                                  void *dk, const natten_layout_t *ldk,
                                  void *drpb,
                                  float *work, int64_t work_floats,
                                  void *stream);

int natten_hip_rpb_av_backward(const natten_problem_t *p,
                               const void *dout, const natten_layout_t *ldo,
                               const void *attn, const natten_layout_t *la,
                               const void *v, const natten_layout_t *lv,
                               void *dattn, const natten_layout_t *lda,
                               void *dv, const natten_layout_t *ldv,
                               void *stream);

/* Per-kernel timing (no counterpart in the reference; for benchmarks and
 * profiling).  While enabled, every kernel launch of the library is bracketed
 * by two HIP events on its stream.  natten_hip_profile_read waits for the
 * recorded events, folds them into per-kernel totals, copies up to
 * max_entries of them to `out` (may be NULL) and returns the number of
 * kernels seen; reset != 0 clears the totals afterwards. */
typedef struct {
    char name[64];
    int64_t launches;
    double total_ms;
    double min_ms;
    double max_ms;
} natten_kernel_stat_t;

int natten_hip_profile_enable(int on);
int natten_hip_profile_read(natten_kernel_stat_t *out, int max_entries, int reset);

#ifdef __cplusplus
}
#endif

#endif /* NATTEN_HIP_H */

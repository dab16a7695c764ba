// Host-side launch entry points shared between the kernel files and the C ABI.
#pragma once

#include "na_common.h"

namespace na {

// Optional event timing around each launch (na_profile.hip).
void prof_begin(const char* name, hipStream_t s);
void prof_end(hipStream_t s);

// `lens` (device, int32 [B][3]): per-sample extents of a variable-length
// problem, or null.
hipError_t generic_forward(const Prob& p, int vec, const void* q, Lay lq, const void* k, Lay lk, const void* v,
                           Lay lv, void* o, Lay lo, float* lse, Lay ll, int dtype, hipStream_t s,
                           const int* lens = nullptr);
hipError_t generic_qk(const Prob& p, int vec, const void* q, Lay lq, const void* k, Lay lk, void* a, Lay la,
                      int dtype, hipStream_t s);
hipError_t generic_av(const Prob& p, int vec, const void* a, Lay la, const void* v, Lay lv, void* o, Lay lo,
                      int dtype, hipStream_t s);
hipError_t generic_backward(const Prob& p, int vec, const void* q, Lay lq, const void* k, Lay lk, const void* v,
                            Lay lv, const void* o, Lay lo, const void* dout, Lay ldo, const float* lse, Lay ll,
                            const float* dlse, Lay ldl, void* dq, Lay ldq, void* dk, Lay ldk, void* dv, Lay ldv,
                            float* delta, Lay lde, int dtype, hipStream_t s, const int* lens = nullptr);
// Split backward: `sides` selects the query side (dq / dattn) and the key
// side (dk / dv).
constexpr int kQuerySide = 1, kKeySide = 2;
hipError_t generic_qk_backward(const Prob& p, int vec, const void* da, Lay lda, const void* q, Lay lq,
                               const void* k, Lay lk, void* dq, Lay ldq, void* dk, Lay ldk, int dtype,
                               hipStream_t s, int sides = kQuerySide | kKeySide);
hipError_t generic_av_backward(const Prob& p, int vec, const void* dout, Lay ldo, const void* a, Lay la,
                               const void* v, Lay lv, void* da, Lay lda, void* dv, Lay ldv, int dtype,
                               hipStream_t s, int sides = kQuerySide | kKeySide);
hipError_t neighborhood_map(const Prob& p, int64_t* flat, uint8_t* valid, hipStream_t s);

// Relative-position-bias split ops (na_rpb.hip): padded axes 1 and 2 carry
// the problem; rpb / drpb are contiguous [H, 2K1-1, 2K2-1] (rpb may be null).
hipError_t rpb_qk(const Prob& p, const void* q, Lay lq, const void* k, Lay lk, const void* rpb, void* attn, Lay la,
                  int dtype, hipStream_t s);
hipError_t rpb_av(const Prob& p, const void* attn, Lay la, const void* v, Lay lv, void* out, Lay lo, int dtype,
                  hipStream_t s);
// `sides` as for the generic backward (drpb is reduced whenever non-null,
// in two passes through `work` when it holds rpb_dbias_workspace floats,
// else in one pass).
hipError_t rpb_qk_backward(const Prob& p, const void* da, Lay lda, const void* q, Lay lq, const void* k, Lay lk,
                           void* dq, Lay ldq, void* dk, Lay ldk, void* drpb, int dtype, hipStream_t s,
                           int sides = kQuerySide | kKeySide, float* work = nullptr, size_t work_floats = 0);
size_t rpb_dbias_workspace(const Prob& p);
hipError_t rpb_av_backward(const Prob& p, const void* dout, Lay ldo, const void* attn, Lay la, const void* v, Lay lv,
                           void* da, Lay lda, void* dv, Lay ldv, int dtype, hipStream_t s,
                           int sides = kQuerySide | kKeySide);


}  // namespace na

// Launch with optional event timing (see na_profile.hip).
#define NA_LAUNCH(name, kernel, grid, block, shmem, stream, ...)                     \
    do {                                                                             \
        ::na::prof_begin(name, stream);                                              \
        hipLaunchKernelGGL(kernel, grid, block, shmem, stream, __VA_ARGS__);         \
        ::na::prof_end(stream);                                                      \
    } while (0)

namespace na {

// While a NoDeviceAlloc object lives on a thread, launches from that thread
// allocate no device memory: the tile kernels read a geometry table only if
// one was already built for the shape and otherwise compute the geometry
// themselves (the same values).
class NoDeviceAlloc {
public:
    NoDeviceAlloc();
    ~NoDeviceAlloc();
    NoDeviceAlloc(const NoDeviceAlloc&) = delete;
    NoDeviceAlloc& operator=(const NoDeviceAlloc&) = delete;

private:
    bool prev_;
};
bool device_alloc_allowed();

// A device table (tile geometry) filled by an asynchronous copy on the stream
// that first needed it.  table_upload enqueues the copy of `bytes` from `h`
// (which the caller keeps alive as long as the table) and records an event;
// table_ready says whether a launch on `s` may read the table now, after
// making `s` wait for the copy when it was enqueued on another stream and is
// not known to be complete (false under stream capture in that case: the
// caller then does without the table).  Callers hold their cache's lock.
struct TableUpload {
    hipStream_t stream = nullptr;
    hipEvent_t ev = nullptr;
    bool done = false;
};
hipError_t table_upload(TableUpload& u, void* d, const void* h, size_t bytes, hipStream_t s);
bool table_ready(TableUpload& u, hipStream_t s);

// Global keys of a fused call (the reference's additional_keys): rows of
// keys and values [B, n, Hkv, D] with their batch / head strides and the
// token stride in s2.
struct GlobalSet {
    const void *k, *v;
    Lay lk, lv;
    int n;
};

// MFMA tile path (na_mfma.hip): bf16/fp16, stride 1, equal head dims 32/64/96/128
// (96 stored as 128-wide LDS rows).
// mfma_static_lds_ok: no tile kernel instance declares static LDS (checked
// once per process); mfma_lds_audit returns 1 when so, 0 otherwise, and the
// number of instances whose attributes were read.
bool mfma_static_lds_ok();
int mfma_lds_audit(int* checked);
// `global`: with global keys (their LDS on top of the tiles').
bool mfma_eligible(const Prob& p, int dtype, int D, bool aligned, bool backward, bool global = false);
bool mfma_offsets_fit(const Prob& p, std::initializer_list<Lay> lays);

// Variable-length fused forward / backward on the MFMA tile kernels: the
// problem describes the padded extents (stride 1), lens (device, int32
// [batch][3]) each sample's own; padding positions of every output are
// zeroed.  Eligibility as for the tile path, with LDS sized for every
// sample extent up to the padded one.
bool mfma_varlen_eligible(const Prob& p, int dtype, int D, bool aligned, bool backward);
hipError_t mfma_varlen_forward(const Prob& p, const int* lens, const void* q, Lay lq, const void* k, Lay lk,
                               const void* v, Lay lv, void* o, Lay lo, float* lse, Lay ll, int dtype, hipStream_t s);
hipError_t mfma_varlen_backward(const Prob& p, const int* lens, const void* q, Lay lq, const void* k, Lay lk,
                                const void* v, Lay lv, const void* o, Lay lo, const void* dout, Lay ldo,
                                const float* lse, Lay ll, void* dq, Lay ldq, void* dk, Lay ldk, void* dv, Lay ldv,
                                float* delta, Lay lde, int dtype, hipStream_t s);
hipError_t mfma_forward(const Prob& p, const void* q, Lay lq, const void* k, Lay lk, const void* v, Lay lv, void* o,
                        Lay lo, float* lse, Lay ll, int dtype, hipStream_t s, const GlobalSet* g = nullptr);
hipError_t mfma_backward(const Prob& p, const void* q, Lay lq, const void* k, Lay lk, const void* v, Lay lv,
                         const void* o, Lay lo, const void* dout, Lay ldo, const float* lse, Lay ll,
                         const float* dlse, Lay ldl, void* dq, Lay ldq, void* dk, Lay ldk, void* dv, Lay ldv,
                         float* delta, Lay lde, int dtype, hipStream_t s, const GlobalSet* g = nullptr);

// Lean 2-D tile kernels (na_lean.hip): 2-D problems at stride 1, bf16/fp16,
// head dim 32 or 64, kernel sizes up to 9, q-side and k-side operands each
// in one layout.  The launchers return hipErrorNotSupported when they have
// no launch for the problem (no tile table can be built: stream capture or a
// no-allocation scope), and the caller then takes the general tile kernels.
bool lean_eligible(const Prob& p, int dtype, bool aligned, std::initializer_list<Lay> qside,
                   std::initializer_list<Lay> kvside, std::initializer_list<Lay> rows);
// Static-LDS audit of the lean instances (as mfma_lds_audit).
int lean_lds_audit(int* checked);
// Split ops' key side (out[k] = mul * sum over attending q of w[q][e] x[q])
// on the 8x8 key tiles; hipErrorNotSupported when there is no launch (the
// caller then takes the general split kernel).
bool lean_wsum_key_eligible(const Prob& p, int dtype, int D, bool aligned, const Lay& lw, const Lay& lx,
                            const Lay& lo);
hipError_t lean_wsum_key(const char* name, const Prob& p, int D, const void* w, Lay lw, const void* x, Lay lx,
                         void* o, Lay lo, float mul, int dtype, hipStream_t s);
hipError_t lean_forward(const Prob& p, const void* q, Lay lq, const void* k, Lay lk, const void* v, Lay lv, void* o,
                        Lay lo, float* lse, Lay ll, int dtype, hipStream_t s);
hipError_t lean_backward(const Prob& p, const void* q, Lay lq, const void* k, Lay lk, const void* v, Lay lv,
                         const void* o, Lay lo, const void* dout, Lay ldo, const float* lse, Lay ll,
                         const float* dlse, Lay ldl, void* dq, Lay ldq, void* dk, Lay ldk, void* dv, Lay ldv,
                         float* delta, Lay lde, int dtype, hipStream_t s);

// Key side of the global keys' backward (na_global.hip): dk and dv of the
// global keys (summed over every query of each q head of the group), from the
// forward's lse and the backward's delta.  Partial sums over slices of the
// queries go to `work` (global_workspace_floats of them), then one pass adds
// them in a fixed order.  mfma_global_key_ok: the problem fits the kernel.
bool mfma_global_key_ok(const Prob& p, int dtype, const GlobalSet& g);
// The key side's q / dO operands: every offset within one batch in 31 bits.
bool mfma_global_batch_fit(const Prob& p, const Lay& lq, const Lay& ldo);
size_t global_workspace_floats(const Prob& p, int n);
hipError_t mfma_global_key_backward(const Prob& p, const void* q, Lay lq, const void* dout, Lay ldo, const float* lse,
                                    Lay ll, const float* delta, Lay lde, const GlobalSet& g, void* dk, Lay ldk,
                                    void* dv, Lay ldv, float* work, int dtype, hipStream_t s);

// Split ops on the MFMA tile path, query side: `rows` is the operand of KV
// entries per query (attn or dattn), `staged` the operands staged per tile.
bool mfma_split_eligible(const Prob& p, int dtype, int D, bool aligned, const Lay& rows,
                         std::initializer_list<Lay> staged);
// out[q][e] = mul * (a[q] . x[nbr(q, e)]), `fill` at invalid neighbours;
// `bias` (relative-position bias [H, 2 K1 - 1, 2 K2 - 1], odd kernels, axis
// 0 of kernel 1) adds bias[h, pb_start + e] per axis to every entry.
hipError_t mfma_split_dot(const char* name, const Prob& p, int D, const void* a, Lay la, const void* x, Lay lx,
                          void* o, Lay lo, float mul, float fill, int dtype, hipStream_t s,
                          const void* bias = nullptr);
// Key side: out[k] = mul * sum over the queries q attending k of w[q][e(q, k)] x[q].
bool mfma_split_key_eligible(const Prob& p, int dtype, int D, bool aligned, const Lay& rows,
                             std::initializer_list<Lay> staged);
hipError_t mfma_split_wsum_key(const char* name, const Prob& p, int D, const void* w, Lay lw, const void* x, Lay lx,
                               void* o, Lay lo, float mul, int dtype, hipStream_t s);
// out[q] = mul * sum over valid e of w[q][e] x[nbr(q, e)].
hipError_t mfma_split_wsum(const char* name, const Prob& p, int D, const void* w, Lay lw, const void* x, Lay lx,
                           void* o, Lay lo, float mul, int dtype, hipStream_t s);

}  // namespace na

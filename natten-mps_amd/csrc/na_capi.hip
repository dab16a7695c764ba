// C ABI of libnatten_hip.so (declared in include/natten_hip.h): argument
// validation, problem set-up and kernel selection.  The caller passes every
// buffer; the only device memory the library allocates is the tile-geometry
// tables of na_mfma.hip, and natten_hip_backward_noalloc allocates none.
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>

#include "na_launch.h"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

int launch_status(hipError_t e, const char* what) {
    if (e == hipSuccess) return NATTEN_OK;
    return fail(NATTEN_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(e));
}

na::Lay to_lay(const natten_layout_t* l) {
    na::Lay r{};
    if (l) {
        r.b = l->batch;
        r.s0 = l->axis[0];
        r.s1 = l->axis[1];
        r.s2 = l->axis[2];
        r.h = l->head;
    }
    return r;
}

int elem_size(int dtype) { return dtype == NATTEN_F32 ? 4 : 2; }

// Validates the problem and fills the kernel-side descriptor.  `fused` ops use
// out = ceil(len/stride); split ops may use a shorter query extent at stride 1.
// `shifted_windows` (the relative-position-bias ops, whose window rule
// covers an even kernel equal to the axis) skips that one rejection.
int make_prob(const natten_problem_t* p, bool fused, na::Prob& P, bool shifted_windows = false) {
    if (!p) return fail(NATTEN_ERR_INVALID, "problem is NULL");
    if (p->dtype < NATTEN_F32 || p->dtype > NATTEN_BF16) return fail(NATTEN_ERR_INVALID, "bad dtype %d", p->dtype);
    if (p->batch < 1 || p->heads_q < 1 || p->heads_kv < 1)
        return fail(NATTEN_ERR_INVALID, "batch and heads must be >= 1");
    if (p->heads_q % p->heads_kv != 0)
        return fail(NATTEN_ERR_INVALID, "heads_q (%d) must be divisible by heads_kv (%d)", p->heads_q, p->heads_kv);
    if (p->dim_qk < 1 || p->dim_v < 1) return fail(NATTEN_ERR_INVALID, "head dims must be >= 1");
    if (p->dim_qk > 256 || p->dim_v > 256)
        return fail(NATTEN_ERR_UNSUPPORTED, "head dims above 256 are not supported (got %d, %d)", p->dim_qk,
                    p->dim_v);
    P.B = p->batch;
    P.Hq = p->heads_q;
    P.Hkv = p->heads_kv;
    P.rep = p->heads_q / p->heads_kv;
    P.Dqk = p->dim_qk;
    P.Dv = p->dim_v;
    P.has_scale = p->has_scale ? 1 : 0;
    P.scale = p->scale;
    P.kv = 1;
    P.nout = 1;
    P.nkey = 1;
    for (int a = 0; a < 3; ++a) {
        na::Axis& A = P.ax[a];
        A.len = p->length[a];
        A.out = p->out_length[a];
        A.k = p->kernel[a];
        A.dil = p->dilation[a];
        A.st = p->stride[a];
        A.causal = p->causal[a] ? 1 : 0;
        if (A.len < 1 || A.k < 1 || A.dil < 1 || A.st < 1)
            return fail(NATTEN_ERR_INVALID, "axis %d: length, kernel, dilation and stride must be >= 1", a);
        if (static_cast<long long>(A.k) * A.dil > A.len)
            return fail(NATTEN_ERR_INVALID, "axis %d: dilation*kernel (%d*%d) exceeds length %d", a, A.dil, A.k,
                        A.len);
        const int full = (A.len + A.st - 1) / A.st;
        if (fused ? (A.out != full) : (A.out < 1 || A.out > full || (A.st != 1 && A.out != full)))
            return fail(NATTEN_ERR_INVALID, "axis %d: query extent %d does not match length %d / stride %d", a,
                        A.out, A.len, A.st);
        // The reference rule places the window at -1 only in this case (even
        // kernel equal to the axis, no dilation, non-causal); no defined result.
        if (!shifted_windows && !A.causal && A.dil == 1 && (A.k % 2) == 0 && A.k == A.len)
            return fail(NATTEN_ERR_UNSUPPORTED,
                        "axis %d: an even kernel (%d) equal to the axis length is not supported", a, A.k);
        P.kv *= A.k;
        P.nout *= A.out;
        P.nkey *= A.len;
    }
    return NATTEN_OK;
}

// Dims per lane used by the generic kernels for head dim D.
int dpl_for(int D) { return D <= 128 ? 8 : 16; }

struct Run {
    const void* ptr;
    const natten_layout_t* lay;
    int D;
};

// True when every operand can be read in aligned runs of `dpl` elements:
// 16-byte aligned base, its head dim and every stride a multiple of dpl.
bool runs_aligned(int dpl, std::initializer_list<Run> ts) {
    for (auto& t : ts) {
        if (!t.ptr) continue;
        if (t.D % dpl) return false;
        if (reinterpret_cast<uintptr_t>(t.ptr) % 16) return false;
        const natten_layout_t* l = t.lay;
        if (!l) return false;
        if (l->batch % dpl || l->axis[0] % dpl || l->axis[1] % dpl || l->axis[2] % dpl || l->head % dpl) return false;
    }
    return true;
}

// NATTEN_HIP_KERNELS=generic selects the vector-ALU kernels everywhere (for
// A/B comparisons); by default the MFMA tile kernels serve every eligible call.
bool use_mfma() {
    static const bool on = [] {
        const char* e = std::getenv("NATTEN_HIP_KERNELS");
        return !(e && std::strcmp(e, "generic") == 0);
    }();
    return on;
}

bool any_null(std::initializer_list<const void*> ps) {
    for (auto p : ps)
        if (!p) return true;
    return false;
}

}  // namespace

extern "C" {

int natten_hip_abi_version(void) { return NATTEN_HIP_ABI_VERSION; }

const char* natten_hip_last_error(void) { return g_err; }

int natten_hip_mfma_lds_check(int32_t* checked) {
    int n = 0, n_lean = 0;
    const int ok = na::mfma_lds_audit(&n);
    const int ok_lean = na::lean_lds_audit(&n_lean);
    if (checked) *checked = n + n_lean;
    return ok && ok_lean ? 1 : 0;
}

int natten_hip_forward(const natten_problem_t* p, const void* q, const natten_layout_t* lq, const void* k,
                       const natten_layout_t* lk, const void* v, const natten_layout_t* lv, void* out,
                       const natten_layout_t* lo, float* lse, const natten_layout_t* llse, void* stream) {
    na::Prob P;
    int rc = make_prob(p, true, P);
    if (rc) return rc;
    if (any_null({q, k, v, out, lse, lq, lk, lv, lo, llse})) return fail(NATTEN_ERR_INVALID, "NULL operand");
    const int D = P.Dqk > P.Dv ? P.Dqk : P.Dv;
    const int vec =
        runs_aligned(dpl_for(D), {{q, lq, P.Dqk}, {k, lk, P.Dqk}, {v, lv, P.Dv}, {out, lo, P.Dv}}) ? 1 : 0;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    // the lean 2-D tiles first (their checks are cheap), then the general tiles
    if (use_mfma() && na::lean_eligible(P, p->dtype, vec != 0, {to_lay(lq), to_lay(lo)}, {to_lay(lk), to_lay(lv)},
                                        {to_lay(llse)})) {
        const hipError_t e = na::lean_forward(P, q, to_lay(lq), k, to_lay(lk), v, to_lay(lv), out, to_lay(lo), lse,
                                              to_lay(llse), p->dtype, s);
        if (e != hipErrorNotSupported) return launch_status(e, "forward");
    }
    if (use_mfma() && na::mfma_eligible(P, p->dtype, D, vec != 0, false) &&
        na::mfma_offsets_fit(P, {to_lay(lq), to_lay(lk), to_lay(lv), to_lay(lo), to_lay(llse)})) {
        return launch_status(na::mfma_forward(P, q, to_lay(lq), k, to_lay(lk), v, to_lay(lv), out, to_lay(lo), lse,
                                              to_lay(llse), p->dtype, s),
                             "forward");
    }
    return launch_status(na::generic_forward(P, vec, q, to_lay(lq), k, to_lay(lk), v, to_lay(lv), out, to_lay(lo),
                                             lse, to_lay(llse), p->dtype, s),
                         "forward");
}

namespace {

// Shared body of the two backward entry points (the problem already checked).
int backward_impl(const natten_problem_t* p, const na::Prob& P, const void* q, const natten_layout_t* lq,
                  const void* k, const natten_layout_t* lk, const void* v, const natten_layout_t* lv,
                  const void* out, const natten_layout_t* lo, const void* dout, const natten_layout_t* ldo,
                  const float* lse, const natten_layout_t* llse, const float* dlse, const natten_layout_t* ldlse,
                  void* dq, const natten_layout_t* ldq, void* dk, const natten_layout_t* ldk, void* dv,
                  const natten_layout_t* ldv, float* delta, const natten_layout_t* ldelta, void* stream) {
    if (any_null({q, k, v, out, dout, lse, dq, dk, dv, delta, lq, lk, lv, lo, ldo, llse, ldq, ldk, ldv, ldelta}))
        return fail(NATTEN_ERR_INVALID, "NULL operand");
    if (dlse && !ldlse) return fail(NATTEN_ERR_INVALID, "dlse given without a layout");
    const int D = P.Dqk > P.Dv ? P.Dqk : P.Dv;
    const int vec = runs_aligned(dpl_for(D), {{q, lq, P.Dqk}, {k, lk, P.Dqk}, {v, lv, P.Dv}, {out, lo, P.Dv},
                                              {dout, ldo, P.Dv}, {dq, ldq, P.Dqk}, {dk, ldk, P.Dqk}, {dv, ldv, P.Dv}})
                        ? 1
                        : 0;
    // the lean 2-D tiles first (their checks are cheap), then the general tiles
    if (use_mfma() &&
        na::lean_eligible(P, p->dtype, vec != 0, {to_lay(lq), to_lay(lo), to_lay(ldo), to_lay(ldq)},
                          {to_lay(lk), to_lay(lv), to_lay(ldk), to_lay(ldv)},
                          dlse ? std::initializer_list<na::Lay>{to_lay(llse), to_lay(ldelta), to_lay(ldlse)}
                               : std::initializer_list<na::Lay>{to_lay(llse), to_lay(ldelta)})) {
        const hipError_t e = na::lean_backward(
            P, q, to_lay(lq), k, to_lay(lk), v, to_lay(lv), out, to_lay(lo), dout, to_lay(ldo), lse, to_lay(llse),
            dlse, to_lay(ldlse), dq, to_lay(ldq), dk, to_lay(ldk), dv, to_lay(ldv), delta, to_lay(ldelta), p->dtype,
            static_cast<hipStream_t>(stream));
        if (e != hipErrorNotSupported) return launch_status(e, "backward");
    }
    if (use_mfma() && na::mfma_eligible(P, p->dtype, D, vec != 0, true) &&
        na::mfma_offsets_fit(P, {to_lay(lq), to_lay(lk), to_lay(lv), to_lay(lo), to_lay(ldo), to_lay(llse),
                                 to_lay(ldq), to_lay(ldk), to_lay(ldv), to_lay(ldelta)}) &&
        (!dlse || na::mfma_offsets_fit(P, {to_lay(ldlse)}))) {
        return launch_status(na::mfma_backward(P, q, to_lay(lq), k, to_lay(lk), v, to_lay(lv), out, to_lay(lo), dout,
                                               to_lay(ldo), lse,
                                               to_lay(llse), dlse, to_lay(ldlse), dq, to_lay(ldq), dk, to_lay(ldk), dv,
                                               to_lay(ldv), delta, to_lay(ldelta), p->dtype,
                                               static_cast<hipStream_t>(stream)),
                             "backward");
    }
    return launch_status(
        na::generic_backward(P, vec, q, to_lay(lq), k, to_lay(lk), v, to_lay(lv), out, to_lay(lo), dout, to_lay(ldo),
                             lse, to_lay(llse), dlse, to_lay(ldlse), dq, to_lay(ldq), dk, to_lay(ldk), dv,
                             to_lay(ldv), delta, to_lay(ldelta), p->dtype, static_cast<hipStream_t>(stream)),
        "backward");
}

// Device scratch of natten_hip_backward_noalloc: its fp32 delta rows
// (batch x query positions x query heads), at most kScratchFloats of them.
// Each GPU the library runs on holds its own copy until the process ends.
// The kernels write every delta entry before any is read, so nothing needs
// clearing between calls; two calls that overlap on one GPU race on it.
constexpr size_t kScratchFloats = size_t(4) << 20;  // 16 MiB
static __device__ __align__(256) float scratch[kScratchFloats];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch[kMaxDevices];

// Device address of `scratch` on the current device, looked up once per
// device.  In host code the name `scratch` is a host-side stand-in; only the
// looked-up address may reach a kernel.
int scratch_ptr(float** out) {
    int dev = -1;
    const hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail(NATTEN_ERR_LAUNCH, "backward_noalloc: hipGetDevice: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices) return fail(NATTEN_ERR_UNSUPPORTED, "backward_noalloc: device %d", dev);
    std::lock_guard<std::mutex> g(g_scratch_mu);
    if (!g_scratch[dev]) {
        void* ptr = nullptr;
        const hipError_t es = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (es != hipSuccess || !ptr)
            return fail(NATTEN_ERR_LAUNCH, "backward_noalloc: hipGetSymbolAddress(scratch): %s",
                        hipGetErrorString(es));
        g_scratch[dev] = static_cast<float*>(ptr);
    }
    *out = g_scratch[dev];
    return NATTEN_OK;
}

}  // namespace

int natten_hip_backward(const natten_problem_t* p, const void* q, const natten_layout_t* lq, const void* k,
                        const natten_layout_t* lk, const void* v, const natten_layout_t* lv, const void* out,
                        const natten_layout_t* lo, const void* dout, const natten_layout_t* ldo, const float* lse,
                        const natten_layout_t* llse, const float* dlse, const natten_layout_t* ldlse, void* dq,
                        const natten_layout_t* ldq, void* dk, const natten_layout_t* ldk, void* dv,
                        const natten_layout_t* ldv, float* delta, const natten_layout_t* ldelta, void* stream) {
    na::Prob P;
    int rc = make_prob(p, true, P);
    if (rc) return rc;
    return backward_impl(p, P, q, lq, k, lk, v, lv, out, lo, dout, ldo, lse, llse, dlse, ldlse, dq, ldq, dk, ldk, dv,
                         ldv, delta, ldelta, stream);
}

int natten_hip_backward_noalloc(const natten_problem_t* p, const void* q, const natten_layout_t* lq, const void* k,
                                const natten_layout_t* lk, const void* v, const natten_layout_t* lv, const void* out,
                                const natten_layout_t* lo, const void* dout, const natten_layout_t* ldo,
                                const float* lse, const natten_layout_t* llse, const float* dlse,
                                const natten_layout_t* ldlse, void* dq, const natten_layout_t* ldq, void* dk,
                                const natten_layout_t* ldk, void* dv, const natten_layout_t* ldv, void* stream) {
    na::Prob P;
    int rc = make_prob(p, true, P);
    if (rc) return rc;
    const long long rows = static_cast<long long>(P.B) * P.nout * P.Hq;
    if (rows > static_cast<long long>(kScratchFloats))
        return fail(NATTEN_ERR_UNSUPPORTED,
                    "backward_noalloc: %lld delta rows (batch x query positions x heads) exceed the scratch "
                    "maximum of %zu; use natten_hip_backward with a caller workspace",
                    rows, kScratchFloats);
    float* delta = nullptr;
    rc = scratch_ptr(&delta);
    if (rc) return rc;
    // delta rows contiguous: [B, out0, out1, out2, Hq]
    natten_layout_t ld{};
    ld.head = 1;
    ld.axis[2] = P.Hq;
    ld.axis[1] = ld.axis[2] * P.ax[2].out;
    ld.axis[0] = ld.axis[1] * P.ax[1].out;
    ld.batch = ld.axis[0] * P.ax[0].out;
    const na::NoDeviceAlloc no_alloc;
    return backward_impl(p, P, q, lq, k, lk, v, lv, out, lo, dout, ldo, lse, llse, dlse, ldlse, dq, ldq, dk, ldk, dv,
                         ldv, delta, &ld, stream);
}

namespace {

// Global keys from the ABI: layouts [B, n, Hkv, D] with the token stride in
// axis[2]; checks shared by the two global-key entry points.
int make_global(const na::Prob& P, const void* gk, const natten_layout_t* lgk, const void* gv,
                const natten_layout_t* lgv, int32_t n, na::GlobalSet& g) {
    if (n < 1) return fail(NATTEN_ERR_INVALID, "global keys: n_global must be >= 1 (got %d)", n);
    if (any_null({gk, gv, lgk, lgv})) return fail(NATTEN_ERR_INVALID, "NULL global key operand");
    g.k = gk;
    g.v = gv;
    g.lk = to_lay(lgk);
    g.lv = to_lay(lgv);
    g.n = n;
    if (!runs_aligned(8, {{gk, lgk, P.Dqk}, {gv, lgv, P.Dv}}))
        return fail(NATTEN_ERR_UNSUPPORTED, "global keys: operands must be 16-byte aligned with strides in 8s");
    return NATTEN_OK;
}

// The global-key path: the MFMA tile kernels with global-key chunks.
bool global_eligible(const na::Prob& P, int dtype, int vec, const na::GlobalSet& g, bool backward) {
    const int D = P.Dqk > P.Dv ? P.Dqk : P.Dv;
    return use_mfma() && na::mfma_eligible(P, dtype, D, vec != 0, backward, true) &&
           na::mfma_global_key_ok(P, dtype, g);
}

}  // namespace

int natten_hip_global_supported(const natten_problem_t* p, int32_t n_global, int32_t backward) {
    na::Prob P;
    if (make_prob(p, true, P)) return 0;
    na::GlobalSet g{};
    g.n = n_global;
    g.lk.s2 = g.lv.s2 = static_cast<long long>(p->heads_kv) * p->dim_qk;
    g.lk.h = g.lv.h = p->dim_qk;
    return n_global >= 1 && P.scale > 0.f && global_eligible(P, p->dtype, 1, g, backward != 0) ? 1 : 0;
}

int64_t natten_hip_global_workspace(const natten_problem_t* p, int32_t n_global) {
    na::Prob P;
    if (make_prob(p, true, P) || n_global < 1) return -1;
    return static_cast<int64_t>(na::global_workspace_floats(P, n_global));
}

int natten_hip_forward_global(const natten_problem_t* p, const void* q, const natten_layout_t* lq, const void* k,
                              const natten_layout_t* lk, const void* v, const natten_layout_t* lv, const void* gk,
                              const natten_layout_t* lgk, const void* gv, const natten_layout_t* lgv,
                              int32_t n_global, void* out, const natten_layout_t* lo, float* lse,
                              const natten_layout_t* llse, void* stream) {
    na::Prob P;
    int rc = make_prob(p, true, P);
    if (rc) return rc;
    if (any_null({q, k, v, out, lse, lq, lk, lv, lo, llse})) return fail(NATTEN_ERR_INVALID, "NULL operand");
    na::GlobalSet g{};
    rc = make_global(P, gk, lgk, gv, lgv, n_global, g);
    if (rc) return rc;
    const int D = P.Dqk > P.Dv ? P.Dqk : P.Dv;
    const int vec =
        runs_aligned(dpl_for(D), {{q, lq, P.Dqk}, {k, lk, P.Dqk}, {v, lv, P.Dv}, {out, lo, P.Dv}}) ? 1 : 0;
    if (!global_eligible(P, p->dtype, vec, g, false) ||
        !na::mfma_offsets_fit(P, {to_lay(lq), to_lay(lk), to_lay(lv), to_lay(lo), to_lay(llse)}))
        return fail(NATTEN_ERR_UNSUPPORTED,
                    "global keys run on the MFMA tile kernels only (bf16/fp16, head dim 32/64/96/128, stride 1, "
                    "aligned operands)");
    return launch_status(na::mfma_forward(P, q, to_lay(lq), k, to_lay(lk), v, to_lay(lv), out, to_lay(lo), lse,
                                          to_lay(llse), p->dtype, static_cast<hipStream_t>(stream), &g),
                         "forward_global");
}

int natten_hip_backward_global(const natten_problem_t* p, const void* q, const natten_layout_t* lq, const void* k,
                               const natten_layout_t* lk, const void* v, const natten_layout_t* lv, const void* gk,
                               const natten_layout_t* lgk, const void* gv, const natten_layout_t* lgv,
                               int32_t n_global, const void* out, const natten_layout_t* lo, const void* dout,
                               const natten_layout_t* ldo, const float* lse, const natten_layout_t* llse,
                               const float* dlse, const natten_layout_t* ldlse, void* dq, const natten_layout_t* ldq,
                               void* dk, const natten_layout_t* ldk, void* dv, const natten_layout_t* ldv, void* dgk,
                               const natten_layout_t* ldgk, void* dgv, const natten_layout_t* ldgv, float* delta,
                               const natten_layout_t* ldelta, float* work, int64_t work_floats, void* stream) {
    na::Prob P;
    int rc = make_prob(p, true, P);
    if (rc) return rc;
    if (any_null({q, k, v, out, dout, lse, dq, dk, dv, delta, lq, lk, lv, lo, ldo, llse, ldq, ldk, ldv, ldelta, dgk,
                  dgv, ldgk, ldgv, work}))
        return fail(NATTEN_ERR_INVALID, "NULL operand");
    if (dlse && !ldlse) return fail(NATTEN_ERR_INVALID, "dlse given without a layout");
    na::GlobalSet g{};
    rc = make_global(P, gk, lgk, gv, lgv, n_global, g);
    if (rc) return rc;
    if (!runs_aligned(8, {{dgk, ldgk, P.Dqk}, {dgv, ldgv, P.Dv}}))
        return fail(NATTEN_ERR_UNSUPPORTED, "global keys: gradients must be 16-byte aligned with strides in 8s");
    const size_t need = na::global_workspace_floats(P, n_global);
    if (work_floats < 0 || static_cast<size_t>(work_floats) < need)
        return fail(NATTEN_ERR_INVALID, "backward_global: workspace of %lld floats, %zu needed",
                    static_cast<long long>(work_floats), need);
    const int D = P.Dqk > P.Dv ? P.Dqk : P.Dv;
    const int vec = runs_aligned(dpl_for(D), {{q, lq, P.Dqk}, {k, lk, P.Dqk}, {v, lv, P.Dv}, {out, lo, P.Dv},
                                              {dout, ldo, P.Dv}, {dq, ldq, P.Dqk}, {dk, ldk, P.Dqk}, {dv, ldv, P.Dv}})
                        ? 1
                        : 0;
    // every check of both launches before the first: an unsupported problem
    // is rejected with no output written
    if (!global_eligible(P, p->dtype, vec, g, true) ||
        !na::mfma_offsets_fit(P, {to_lay(lq), to_lay(lk), to_lay(lv), to_lay(lo), to_lay(ldo), to_lay(llse),
                                  to_lay(ldq), to_lay(ldk), to_lay(ldv), to_lay(ldelta)}) ||
        (dlse && !na::mfma_offsets_fit(P, {to_lay(ldlse)})) || !na::mfma_global_batch_fit(P, to_lay(lq), to_lay(ldo)))
        return fail(NATTEN_ERR_UNSUPPORTED,
                    "global keys run on the MFMA tile kernels only (bf16/fp16, head dim 32/64/96/128, stride 1, "
                    "aligned operands)");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    rc = launch_status(na::mfma_backward(P, q, to_lay(lq), k, to_lay(lk), v, to_lay(lv), out, to_lay(lo), dout,
                                         to_lay(ldo), lse, to_lay(llse), dlse, to_lay(ldlse), dq, to_lay(ldq), dk,
                                         to_lay(ldk), dv, to_lay(ldv), delta, to_lay(ldelta), p->dtype, s, &g),
                       "backward_global");
    if (rc) return rc;
    return launch_status(na::mfma_global_key_backward(P, q, to_lay(lq), dout, to_lay(ldo), lse, to_lay(llse), delta,
                                                      to_lay(ldelta), g, dgk, to_lay(ldgk), dgv, to_lay(ldgv), work,
                                                      p->dtype, s),
                         "backward_global (global keys)");
}

int natten_hip_qk_forward(const natten_problem_t* p, const void* q, const natten_layout_t* lq, const void* k,
                          const natten_layout_t* lk, void* attn, const natten_layout_t* la, void* stream) {
    na::Prob P;
    int rc = make_prob(p, false, P);
    if (rc) return rc;
    if (P.rep != 1) return fail(NATTEN_ERR_INVALID, "split QK needs heads_q == heads_kv");
    if (any_null({q, k, attn, lq, lk, la})) return fail(NATTEN_ERR_INVALID, "NULL operand");
    const int vec = runs_aligned(dpl_for(P.Dqk), {{q, lq, P.Dqk}, {k, lk, P.Dqk}}) ? 1 : 0;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (use_mfma() && na::mfma_split_eligible(P, p->dtype, P.Dqk, vec != 0, to_lay(la), {to_lay(lq), to_lay(lk)}))
        return launch_status(na::mfma_split_dot("na_qk_mfma", P, P.Dqk, q, to_lay(lq), k, to_lay(lk), attn,
                                                to_lay(la), P.has_scale ? P.scale : 1.f, -INFINITY, p->dtype, s),
                             "qk_forward");
    return launch_status(na::generic_qk(P, vec, q, to_lay(lq), k, to_lay(lk), attn, to_lay(la), p->dtype, s),
                         "qk_forward");
}

int natten_hip_av_forward(const natten_problem_t* p, const void* attn, const natten_layout_t* la, const void* v,
                          const natten_layout_t* lv, void* out, const natten_layout_t* lo, void* stream) {
    na::Prob P;
    int rc = make_prob(p, false, P);
    if (rc) return rc;
    if (P.rep != 1) return fail(NATTEN_ERR_INVALID, "split AV needs heads_q == heads_kv");
    if (any_null({attn, v, out, la, lv, lo})) return fail(NATTEN_ERR_INVALID, "NULL operand");
    const int vec = runs_aligned(dpl_for(P.Dv), {{v, lv, P.Dv}, {out, lo, P.Dv}}) ? 1 : 0;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (use_mfma() && na::mfma_split_eligible(P, p->dtype, P.Dv, vec != 0, to_lay(la), {to_lay(lv), to_lay(lo)}))
        return launch_status(na::mfma_split_wsum("na_av_mfma", P, P.Dv, attn, to_lay(la), v, to_lay(lv), out,
                                                 to_lay(lo), 1.f, p->dtype, s),
                             "av_forward");
    return launch_status(na::generic_av(P, vec, attn, to_lay(la), v, to_lay(lv), out, to_lay(lo), p->dtype, s),
                         "av_forward");
}

int natten_hip_qk_backward(const natten_problem_t* p, const void* dattn, const natten_layout_t* lda, const void* q,
                           const natten_layout_t* lq, const void* k, const natten_layout_t* lk, void* dq,
                           const natten_layout_t* ldq, void* dk, const natten_layout_t* ldk, void* stream) {
    na::Prob P;
    int rc = make_prob(p, false, P);
    if (rc) return rc;
    if (P.rep != 1) return fail(NATTEN_ERR_INVALID, "split QK needs heads_q == heads_kv");
    if (any_null({dattn, q, k, dq, dk, lda, lq, lk, ldq, ldk})) return fail(NATTEN_ERR_INVALID, "NULL operand");
    const int vec =
        runs_aligned(dpl_for(P.Dqk), {{q, lq, P.Dqk}, {k, lk, P.Dqk}, {dq, ldq, P.Dqk}, {dk, ldk, P.Dqk}}) ? 1 : 0;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    int sides = na::kQuerySide | na::kKeySide;
    if (use_mfma() &&
        na::mfma_split_eligible(P, p->dtype, P.Dqk, vec != 0, to_lay(lda), {to_lay(lk), to_lay(ldq)})) {
        const int rc2 = launch_status(na::mfma_split_wsum("na_qk_bwd_q_mfma", P, P.Dqk, dattn, to_lay(lda), k,
                                                          to_lay(lk), dq, to_lay(ldq), P.has_scale ? P.scale : 1.f,
                                                          p->dtype, s),
                                      "qk_backward");
        if (rc2) return rc2;
        sides = na::kKeySide;
    }
    if (use_mfma() &&
        na::mfma_split_key_eligible(P, p->dtype, P.Dqk, vec != 0, to_lay(lda), {to_lay(lq), to_lay(ldk)})) {
        const int rc2 = launch_status(na::mfma_split_wsum_key("na_qk_bwd_k_mfma", P, P.Dqk, dattn, to_lay(lda), q,
                                                              to_lay(lq), dk, to_lay(ldk),
                                                              P.has_scale ? P.scale : 1.f, p->dtype, s),
                                      "qk_backward");
        if (rc2) return rc2;
        sides &= ~na::kKeySide;
    }
    if (!sides) return NATTEN_OK;
    return launch_status(na::generic_qk_backward(P, vec, dattn, to_lay(lda), q, to_lay(lq), k, to_lay(lk), dq,
                                                 to_lay(ldq), dk, to_lay(ldk), p->dtype, s, sides),
                         "qk_backward");
}

int natten_hip_av_backward(const natten_problem_t* p, const void* dout, const natten_layout_t* ldo,
                           const void* attn, const natten_layout_t* la, const void* v, const natten_layout_t* lv,
                           void* dattn, const natten_layout_t* lda, void* dv, const natten_layout_t* ldv,
                           void* stream) {
    na::Prob P;
    int rc = make_prob(p, false, P);
    if (rc) return rc;
    if (P.rep != 1) return fail(NATTEN_ERR_INVALID, "split AV needs heads_q == heads_kv");
    if (any_null({dout, attn, v, dattn, dv, ldo, la, lv, lda, ldv})) return fail(NATTEN_ERR_INVALID, "NULL operand");
    const int vec = runs_aligned(dpl_for(P.Dv), {{dout, ldo, P.Dv}, {v, lv, P.Dv}, {dv, ldv, P.Dv}}) ? 1 : 0;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    int sides = na::kQuerySide | na::kKeySide;
    if (use_mfma() &&
        na::mfma_split_eligible(P, p->dtype, P.Dv, vec != 0, to_lay(lda), {to_lay(ldo), to_lay(lv)})) {
        const int rc2 = launch_status(na::mfma_split_dot("na_av_bwd_a_mfma", P, P.Dv, dout, to_lay(ldo), v,
                                                         to_lay(lv), dattn, to_lay(lda), 1.f, 0.f, p->dtype, s),
                                      "av_backward");
        if (rc2) return rc2;
        sides = na::kKeySide;
    }
    if (use_mfma() &&
        na::mfma_split_key_eligible(P, p->dtype, P.Dv, vec != 0, to_lay(la), {to_lay(ldo), to_lay(ldv)})) {
        const int rc2 = launch_status(na::mfma_split_wsum_key("na_av_bwd_v_mfma", P, P.Dv, attn, to_lay(la), dout,
                                                              to_lay(ldo), dv, to_lay(ldv), 1.f, p->dtype, s),
                                      "av_backward");
        if (rc2) return rc2;
        sides &= ~na::kKeySide;
    }
    if (!sides) return NATTEN_OK;
    return launch_status(na::generic_av_backward(P, vec, dout, to_lay(ldo), attn, to_lay(la), v, to_lay(lv), dattn,
                                                 to_lay(lda), dv, to_lay(ldv), p->dtype, s, sides),
                         "av_backward");
}

int natten_hip_varlen_forward(const natten_problem_t* p, const int32_t* lens, const void* q,
                              const natten_layout_t* lq, const void* k, const natten_layout_t* lk, const void* v,
                              const natten_layout_t* lv, void* out, const natten_layout_t* lo, float* lse,
                              const natten_layout_t* llse, void* stream) {
    na::Prob P;
    int rc = make_prob(p, true, P);
    if (rc) return rc;
    if (any_null({lens, q, k, v, out, lse, lq, lk, lv, lo, llse})) return fail(NATTEN_ERR_INVALID, "NULL operand");
    for (int a = 0; a < 3; ++a)
        if (P.ax[a].st != 1) return fail(NATTEN_ERR_INVALID, "variable-length attention needs stride 1");
    const int D = P.Dqk > P.Dv ? P.Dqk : P.Dv;
    const int vec =
        runs_aligned(dpl_for(D), {{q, lq, P.Dqk}, {k, lk, P.Dqk}, {v, lv, P.Dv}, {out, lo, P.Dv}}) ? 1 : 0;
    if (use_mfma() && na::mfma_varlen_eligible(P, p->dtype, D, vec != 0, false) &&
        na::mfma_offsets_fit(P, {to_lay(lq), to_lay(lk), to_lay(lv), to_lay(lo), to_lay(llse)}))
        return launch_status(na::mfma_varlen_forward(P, lens, q, to_lay(lq), k, to_lay(lk), v, to_lay(lv), out,
                                                     to_lay(lo), lse, to_lay(llse), p->dtype,
                                                     static_cast<hipStream_t>(stream)),
                             "varlen_forward");
    return launch_status(na::generic_forward(P, vec, q, to_lay(lq), k, to_lay(lk), v, to_lay(lv), out, to_lay(lo),
                                             lse, to_lay(llse), p->dtype, static_cast<hipStream_t>(stream), lens),
                         "varlen_forward");
}

int natten_hip_varlen_backward(const natten_problem_t* p, const int32_t* lens, const void* q,
                               const natten_layout_t* lq, const void* k, const natten_layout_t* lk, const void* v,
                               const natten_layout_t* lv, const void* out, const natten_layout_t* lo,
                               const void* dout, const natten_layout_t* ldo, const float* lse,
                               const natten_layout_t* llse, void* dq, const natten_layout_t* ldq, void* dk,
                               const natten_layout_t* ldk, void* dv, const natten_layout_t* ldv, float* delta,
                               const natten_layout_t* ldelta, void* stream) {
    na::Prob P;
    int rc = make_prob(p, true, P);
    if (rc) return rc;
    if (any_null({lens, q, k, v, out, dout, lse, dq, dk, dv, delta, lq, lk, lv, lo, ldo, llse, ldq, ldk, ldv,
                  ldelta}))
        return fail(NATTEN_ERR_INVALID, "NULL operand");
    for (int a = 0; a < 3; ++a)
        if (P.ax[a].st != 1) return fail(NATTEN_ERR_INVALID, "variable-length attention needs stride 1");
    const int D = P.Dqk > P.Dv ? P.Dqk : P.Dv;
    const int vec = runs_aligned(dpl_for(D), {{q, lq, P.Dqk}, {k, lk, P.Dqk}, {v, lv, P.Dv}, {out, lo, P.Dv},
                                              {dout, ldo, P.Dv}, {dq, ldq, P.Dqk}, {dk, ldk, P.Dqk}, {dv, ldv, P.Dv}})
                        ? 1
                        : 0;
    if (use_mfma() && na::mfma_varlen_eligible(P, p->dtype, D, vec != 0, true) &&
        na::mfma_offsets_fit(P, {to_lay(lq), to_lay(lk), to_lay(lv), to_lay(lo), to_lay(ldo), to_lay(llse),
                                 to_lay(ldq), to_lay(ldk), to_lay(ldv), to_lay(ldelta)}))
        return launch_status(na::mfma_varlen_backward(P, lens, q, to_lay(lq), k, to_lay(lk), v, to_lay(lv), out,
                                                      to_lay(lo), dout, to_lay(ldo), lse, to_lay(llse), dq,
                                                      to_lay(ldq), dk, to_lay(ldk), dv, to_lay(ldv), delta,
                                                      to_lay(ldelta), p->dtype, static_cast<hipStream_t>(stream)),
                             "varlen_backward");
    return launch_status(
        na::generic_backward(P, vec, q, to_lay(lq), k, to_lay(lk), v, to_lay(lv), out, to_lay(lo), dout, to_lay(ldo),
                             lse, to_lay(llse), nullptr, na::Lay{}, dq, to_lay(ldq), dk, to_lay(ldk), dv, to_lay(ldv),
                             delta, to_lay(ldelta), p->dtype, static_cast<hipStream_t>(stream), lens),
        "varlen_backward");
}

// Relative-position-bias ops: rank <= 2 (padded axis 0 of length and kernel
// 1), stride 1, non-causal, equal head counts.
static int make_rpb_prob(const natten_problem_t* p, na::Prob& P) {
    int rc = make_prob(p, true, P, true);
    if (rc) return rc;
    if (P.rep != 1) return fail(NATTEN_ERR_INVALID, "relative-position-bias ops need heads_q == heads_kv");
    if (P.ax[0].len != 1 || P.ax[0].k != 1)
        return fail(NATTEN_ERR_INVALID, "relative-position-bias ops are 1-D or 2-D (axis 0 must be trivial)");
    for (int a = 0; a < 3; ++a)
        if (P.ax[a].st != 1 || P.ax[a].causal)
            return fail(NATTEN_ERR_INVALID, "relative-position-bias ops need stride 1 and no causal mask");
    return NATTEN_OK;
}

// Odd kernels on every axis: the shifted window of these ops is the main
// operators' window (same start, end and neighbour order), so their products
// run on the split tile kernels where those apply (the logits kernel adds
// the bias as it stores them; na_rpb.hip reduces the bias gradient).
static bool rpb_on_tiles(const na::Prob& P) {
    if (!use_mfma()) return false;
    for (int a = 0; a < 3; ++a)
        if (P.ax[a].k % 2 == 0) return false;
    return true;
}

int natten_hip_rpb_qk_forward(const natten_problem_t* p, const void* q, const natten_layout_t* lq, const void* k,
                              const natten_layout_t* lk, const void* rpb, void* attn, const natten_layout_t* la,
                              void* stream) {
    na::Prob P;
    int rc = make_rpb_prob(p, P);
    if (rc) return rc;
    if (any_null({q, k, attn, lq, lk, la})) return fail(NATTEN_ERR_INVALID, "NULL operand");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const bool vec = runs_aligned(dpl_for(P.Dqk), {{q, lq, P.Dqk}, {k, lk, P.Dqk}});
    if (rpb_on_tiles(P) && na::mfma_split_eligible(P, p->dtype, P.Dqk, vec, to_lay(la), {to_lay(lq), to_lay(lk)})) {
        return launch_status(na::mfma_split_dot("na_rpb_qk_mfma", P, P.Dqk, q, to_lay(lq), k, to_lay(lk), attn,
                                                to_lay(la), 1.f, -INFINITY, p->dtype, s, rpb),
                             "rpb_qk_forward");
    }
    return launch_status(na::rpb_qk(P, q, to_lay(lq), k, to_lay(lk), rpb, attn, to_lay(la), p->dtype, s),
                         "rpb_qk_forward");
}

int natten_hip_rpb_av_forward(const natten_problem_t* p, const void* attn, const natten_layout_t* la, const void* v,
                              const natten_layout_t* lv, void* out, const natten_layout_t* lo, void* stream) {
    na::Prob P;
    int rc = make_rpb_prob(p, P);
    if (rc) return rc;
    if (any_null({attn, v, out, la, lv, lo})) return fail(NATTEN_ERR_INVALID, "NULL operand");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const bool vec = runs_aligned(dpl_for(P.Dv), {{v, lv, P.Dv}, {out, lo, P.Dv}});
    if (rpb_on_tiles(P) && na::mfma_split_eligible(P, p->dtype, P.Dv, vec, to_lay(la), {to_lay(lv), to_lay(lo)}))
        return launch_status(na::mfma_split_wsum("na_rpb_av_mfma", P, P.Dv, attn, to_lay(la), v, to_lay(lv), out,
                                                 to_lay(lo), 1.f, p->dtype, s),
                             "rpb_av_forward");
    return launch_status(na::rpb_av(P, attn, to_lay(la), v, to_lay(lv), out, to_lay(lo), p->dtype, s),
                         "rpb_av_forward");
}

namespace {

int rpb_qk_backward_impl(const natten_problem_t* p, const void* dattn, const natten_layout_t* lda, const void* q,
                         const natten_layout_t* lq, const void* k, const natten_layout_t* lk, void* dq,
                         const natten_layout_t* ldq, void* dk, const natten_layout_t* ldk, void* drpb, float* work,
                         int64_t work_floats, void* stream) {
    na::Prob P;
    int rc = make_rpb_prob(p, P);
    if (rc) return rc;
    if (any_null({dattn, q, k, dq, dk, lda, lq, lk, ldq, ldk})) return fail(NATTEN_ERR_INVALID, "NULL operand");
    if (work_floats < 0) return fail(NATTEN_ERR_INVALID, "rpb_qk_backward: negative workspace size");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    int sides = na::kQuerySide | na::kKeySide;
    if (rpb_on_tiles(P)) {
        const bool vec =
            runs_aligned(dpl_for(P.Dqk), {{q, lq, P.Dqk}, {k, lk, P.Dqk}, {dq, ldq, P.Dqk}, {dk, ldk, P.Dqk}});
        if (na::mfma_split_eligible(P, p->dtype, P.Dqk, vec, to_lay(lda), {to_lay(lk), to_lay(ldq)})) {
            rc = launch_status(na::mfma_split_wsum("na_rpb_dq_mfma", P, P.Dqk, dattn, to_lay(lda), k, to_lay(lk), dq,
                                                   to_lay(ldq), 1.f, p->dtype, s),
                               "rpb_qk_backward");
            if (rc) return rc;
            sides &= ~na::kQuerySide;
        }
        if (na::mfma_split_key_eligible(P, p->dtype, P.Dqk, vec, to_lay(lda), {to_lay(lq), to_lay(ldk)})) {
            rc = launch_status(na::mfma_split_wsum_key("na_rpb_dk_mfma", P, P.Dqk, dattn, to_lay(lda), q, to_lay(lq),
                                                       dk, to_lay(ldk), 1.f, p->dtype, s),
                               "rpb_qk_backward");
            if (rc) return rc;
            sides &= ~na::kKeySide;
        }
    }
    return launch_status(na::rpb_qk_backward(P, dattn, to_lay(lda), q, to_lay(lq), k, to_lay(lk), dq, to_lay(ldq), dk,
                                             to_lay(ldk), drpb, p->dtype, s, sides, work,
                                             static_cast<size_t>(work_floats)),
                         "rpb_qk_backward");
}

}  // namespace

int natten_hip_rpb_qk_backward(const natten_problem_t* p, const void* dattn, const natten_layout_t* lda,
                               const void* q, const natten_layout_t* lq, const void* k, const natten_layout_t* lk,
                               void* dq, const natten_layout_t* ldq, void* dk, const natten_layout_t* ldk, void* drpb,
                               void* stream) {
    return rpb_qk_backward_impl(p, dattn, lda, q, lq, k, lk, dq, ldq, dk, ldk, drpb, nullptr, 0, stream);
}

int64_t natten_hip_rpb_dbias_workspace(const natten_problem_t* p) {
    na::Prob P;
    if (make_rpb_prob(p, P)) return -1;
    return static_cast<int64_t>(na::rpb_dbias_workspace(P));
}

int natten_hip_rpb_qk_backward_ws(const natten_problem_t* p, const void* dattn, const natten_layout_t* lda,
                                  const void* q, const natten_layout_t* lq, const void* k, const natten_layout_t* lk,
                                  void* dq, const natten_layout_t* ldq, void* dk, const natten_layout_t* ldk,
                                  void* drpb, float* work, int64_t work_floats, void* stream) {
    return rpb_qk_backward_impl(p, dattn, lda, q, lq, k, lk, dq, ldq, dk, ldk, drpb, work, work_floats, stream);
}

int natten_hip_rpb_av_backward(const natten_problem_t* p, const void* dout, const natten_layout_t* ldo,
                               const void* attn, const natten_layout_t* la, const void* v, const natten_layout_t* lv,
                               void* dattn, const natten_layout_t* lda, void* dv, const natten_layout_t* ldv,
                               void* stream) {
    na::Prob P;
    int rc = make_rpb_prob(p, P);
    if (rc) return rc;
    if (any_null({dout, attn, v, dattn, dv, ldo, la, lv, lda, ldv})) return fail(NATTEN_ERR_INVALID, "NULL operand");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    int sides = na::kQuerySide | na::kKeySide;
    if (rpb_on_tiles(P)) {
        const bool vec = runs_aligned(dpl_for(P.Dv), {{dout, ldo, P.Dv}, {v, lv, P.Dv}, {dv, ldv, P.Dv}});
        if (na::mfma_split_eligible(P, p->dtype, P.Dv, vec, to_lay(lda), {to_lay(ldo), to_lay(lv)})) {
            rc = launch_status(na::mfma_split_dot("na_rpb_dattn_mfma", P, P.Dv, dout, to_lay(ldo), v, to_lay(lv),
                                                  dattn, to_lay(lda), 1.f, 0.f, p->dtype, s),
                               "rpb_av_backward");
            if (rc) return rc;
            sides &= ~na::kQuerySide;
        }
        if (na::mfma_split_key_eligible(P, p->dtype, P.Dv, vec, to_lay(la), {to_lay(ldo), to_lay(ldv)})) {
            rc = launch_status(na::mfma_split_wsum_key("na_rpb_dv_mfma", P, P.Dv, attn, to_lay(la), dout, to_lay(ldo),
                                                       dv, to_lay(ldv), 1.f, p->dtype, s),
                               "rpb_av_backward");
            if (rc) return rc;
            sides &= ~na::kKeySide;
        }
    }
    if (!sides) return NATTEN_OK;
    return launch_status(na::rpb_av_backward(P, dout, to_lay(ldo), attn, to_lay(la), v, to_lay(lv), dattn,
                                             to_lay(lda), dv, to_lay(ldv), p->dtype, s, sides),
                         "rpb_av_backward");
}

int natten_hip_neighborhood_map(const natten_problem_t* p, int64_t* flat, uint8_t* valid, void* stream) {
    na::Prob P;
    int rc = make_prob(p, true, P);
    if (rc) return rc;
    if (any_null({flat, valid})) return fail(NATTEN_ERR_INVALID, "NULL operand");
    return launch_status(na::neighborhood_map(P, flat, valid, static_cast<hipStream_t>(stream)), "neighborhood_map");
}

}  // extern "C"

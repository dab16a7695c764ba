// Host binding of the fused forward / backward and of the split QK / AV ops
// (and their backward) for the 'hip' backend: the per-call work of
// natten_mps_amd/_core/hip.py (output allocation, the C call, the status
// check) in C++ on top of the C ABI, so an eager call pays a few
// microseconds of host time instead of the ctypes marshalling of ten to
// twenty arguments and one torch allocation per output from Python.
//
// A FusedCall holds what is fixed per call signature (shapes, strides,
// dtype, parameters): the problem descriptor and the element-stride layouts
// that hip.py computed once, and the output shapes.  forward / backward
// allocate the outputs from torch's device caching allocator on the inputs'
// device and call natten_hip_forward / natten_hip_backward on the stream
// given (the raw hipStream_t of torch's current stream).  Errors map as in
// the ctypes path: invalid input -> ValueError, unsupported ->
// NotImplementedError, launch failure -> RuntimeError.
//
// SplitCall does the same for the four split ops (qk, av, qk_bwd, av_bwd)
// and the four relative-position-bias ops (rpb_qk, rpb_av, rpb_qk_bwd,
// rpb_av_bwd).
//
// fwd / bwd (and qk / av / qk_bwd / av_bwd) are the per-call entry of
// hip.py: they take the backend hook's own arguments, build the signature
// key from the tensors' metadata and the parameter sequences, and run the
// call object registered for that key on torch's current stream of the
// inputs' device; None when no call is
// registered (hip.py then checks the arguments, builds the signature and
// registers it) or when an argument needs hip.py's handling (a non-unit
// innermost stride, lse / dlse that are not contiguous fp32, parameters that
// are not sequences of ints).
//
// Reference: the backend hooks this serves are those the autograd factory
// calls (autograd/_factory.py:37-38,66-67 of /root/reference/src/natten_mps)
// the split ops' forward and backward hooks (_core/ops.py:98-152), and the
// relative-position-bias ops of extras/allin1 (extras/allin1/functional.py).
#include <torch/extension.h>

#include <ATen/hip/EmptyTensor.h>
#include <c10/core/DeviceGuard.h>
#include <c10/core/impl/DeviceGuardImplInterface.h>
#include <c10/hip/HIPCachingAllocator.h>
#include <c10/hip/HIPStream.h>

#include <cstring>
#include <optional>
#include <string>
#include <vector>

#include "natten_hip.h"

namespace {

[[noreturn]] void raise_status(int rc, const char* what) {
    const std::string msg = std::string("natten hip ") + what + ": " + natten_hip_last_error();
    if (rc == NATTEN_ERR_INVALID) throw pybind11::value_error(msg);
    if (rc == NATTEN_ERR_UNSUPPORTED) {
        PyErr_SetString(PyExc_NotImplementedError, msg.c_str());
        throw pybind11::error_already_set();
    }
    throw std::runtime_error(msg);
}

// Layout slots: forward q k v out lse; backward q k v out dO lse dlse dq dk dv delta.
constexpr int kFwdLays = 5, kBwdLays = 11;

// A device tensor from torch's caching allocator (no dispatcher round trip).
at::Tensor alloc(at::IntArrayRef shape, at::ScalarType dt, const at::Device& d) {
    return at::detail::empty_cuda(shape, dt, d, std::nullopt);
}

int64_t numel(at::IntArrayRef shape) {
    int64_t n = 1;
    for (int64_t x : shape) n *= x;
    return n;
}

// Several results of one call carved from one caching-allocator block (one
// allocator call instead of one per result): each part starts on a 256-byte
// boundary, and the block is given back when the last part is freed.
struct Block {
    std::vector<int64_t> off;
    int64_t bytes = 0;
    c10::Storage st;

    int add(int64_t nbytes) {
        bytes = (bytes + 255) & ~int64_t(255);
        off.push_back(bytes);
        bytes += nbytes;
        return static_cast<int>(off.size()) - 1;
    }
    void allocate(const at::Device& d) { st = alloc({std::max<int64_t>(bytes, 1)}, at::kByte, d).storage(); }
    at::Tensor part(int i, at::IntArrayRef shape, at::ScalarType dt) const {
        at::Tensor t = at::detail::make_tensor<c10::TensorImpl>(
            c10::Storage(st), c10::DispatchKeySet(c10::DispatchKey::CUDA), c10::scalarTypeToTypeMeta(dt));
        t.unsafeGetTensorImpl()->set_sizes_contiguous(shape);
        t.unsafeGetTensorImpl()->set_storage_offset(off[i] / static_cast<int64_t>(c10::elementSize(dt)));
        return t;
    }
};

// Workspace from the caching allocator on the current device for one call:
// given back when the call returns (or throws).  The block belongs to the
// stream it was taken for, so the allocator hands it out again only to work
// ordered after this call's kernels on that stream.
struct Workspace {
    void* ptr = nullptr;
    Workspace(size_t bytes, hipStream_t s)
        : ptr(bytes ? c10::hip::HIPCachingAllocator::raw_alloc_with_stream(bytes, s) : nullptr) {}
    ~Workspace() {
        if (ptr) c10::hip::HIPCachingAllocator::raw_delete(ptr);
    }
    Workspace(const Workspace&) = delete;
    Workspace& operator=(const Workspace&) = delete;
};

struct FusedCall {
    natten_problem_t prob;
    std::vector<natten_layout_t> lay;
    std::vector<int64_t> out_shape, lse_shape;
    bool strided;

    FusedCall(const pybind11::bytes& prob_bytes, const pybind11::bytes& lay_bytes, std::vector<int64_t> out_shape_,
              std::vector<int64_t> lse_shape_, bool strided_)
        : out_shape(std::move(out_shape_)), lse_shape(std::move(lse_shape_)), strided(strided_) {
        const std::string p = prob_bytes, l = lay_bytes;
        if (p.size() != sizeof(natten_problem_t)) throw pybind11::value_error("FusedCall: problem size mismatch");
        if (l.size() % sizeof(natten_layout_t) != 0) throw pybind11::value_error("FusedCall: layout size mismatch");
        std::memcpy(&prob, p.data(), sizeof(prob));
        lay.resize(l.size() / sizeof(natten_layout_t));
        std::memcpy(lay.data(), l.data(), l.size());
    }

    std::tuple<at::Tensor, at::Tensor> forward(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                                               int64_t stream) const {
        if (lay.size() != kFwdLays) throw pybind11::value_error("FusedCall.forward: not a forward signature");
        c10::OptionalDeviceGuard guard;
        if (current_index() != q.get_device()) guard.reset_device(q.device());
        // out and lse share one block (the autograd Function keeps both)
        Block blk;
        blk.add(numel(out_shape) * static_cast<int64_t>(c10::elementSize(q.scalar_type())));
        blk.add(numel(lse_shape) * static_cast<int64_t>(sizeof(float)));
        blk.allocate(q.device());
        at::Tensor out = blk.part(0, out_shape, q.scalar_type());
        at::Tensor lse = blk.part(1, lse_shape, at::kFloat);
        const int rc = natten_hip_forward(&prob, q.data_ptr(), &lay[0], k.data_ptr(), &lay[1], v.data_ptr(), &lay[2],
                                          out.data_ptr(), &lay[3], lse.data_ptr<float>(), &lay[4],
                                          reinterpret_cast<void*>(stream));
        if (rc != NATTEN_OK) raise_status(rc, "forward");
        return {out, lse};
    }

    std::tuple<at::Tensor, at::Tensor, at::Tensor> backward(const at::Tensor& q, const at::Tensor& k,
                                                            const at::Tensor& v, const at::Tensor& out,
                                                            const at::Tensor& d_out, const at::Tensor& lse,
                                                            const std::optional<at::Tensor>& d_lse,
                                                            int64_t stream) const {
        if (lay.size() != kBwdLays) throw pybind11::value_error("FusedCall.backward: not a backward signature");
        c10::OptionalDeviceGuard guard;
        if (current_index() != q.get_device()) guard.reset_device(q.device());
        // dq, dk, dv and the delta rows from one block; delta's part lives as
        // long as the gradients (lse-sized, one float per query and head)
        Block blk;
        const auto bytes = [](const at::Tensor& t) {
            return t.numel() * static_cast<int64_t>(c10::elementSize(t.scalar_type()));
        };
        blk.add(bytes(q));
        blk.add(bytes(k));
        blk.add(bytes(v));
        blk.add(numel(lse_shape) * static_cast<int64_t>(sizeof(float)));
        blk.allocate(q.device());
        at::Tensor dq = blk.part(0, q.sizes(), q.scalar_type());
        // dq is zeroed where stride > 1 leaves positions that are not queries
        if (strided) dq.zero_();
        at::Tensor dk = blk.part(1, k.sizes(), k.scalar_type());
        at::Tensor dv = blk.part(2, v.sizes(), v.scalar_type());
        float* const delta = static_cast<float*>(blk.st.mutable_data()) + blk.off[3] / sizeof(float);
        const float* dl = d_lse.has_value() ? d_lse->data_ptr<float>() : nullptr;
        const int rc = natten_hip_backward(
            &prob, q.data_ptr(), &lay[0], k.data_ptr(), &lay[1], v.data_ptr(), &lay[2], out.data_ptr(), &lay[3],
            d_out.data_ptr(), &lay[4], lse.data_ptr<float>(), &lay[5], dl, dl ? &lay[6] : nullptr, dq.data_ptr(),
            &lay[7], dk.data_ptr(), &lay[8], dv.data_ptr(), &lay[9], delta, &lay[10],
            reinterpret_cast<void*>(stream));
        if (rc != NATTEN_OK) raise_status(rc, "backward");
        return {dq, dk, dv};
    }

    static int current_index() {
        return c10::impl::getDeviceGuardImpl(c10::DeviceType::CUDA)->getDevice().index();
    }
};

// The split ops (QK, AV and their backward), as FusedCall: the problem and
// layouts of one call signature, fixed.  Layout slots: QK q k attn; AV attn v
// out; QK backward dattn q k dq dk; AV backward dout attn v dattn dv.
// The relative-position-bias ops (natten_hip_rpb_*) use the same slots: QK
// q k attn (plus the bias table, no layout); AV attn v out; QK backward dattn
// q k dq dk (plus the bias gradient and its workspace); AV backward dout attn
// v dattn dv.
enum SplitOp { kQk = 0, kAv = 1, kQkBwd = 2, kAvBwd = 3, kRpbQk = 4, kRpbAv = 5, kRpbQkBwd = 6, kRpbAvBwd = 7 };
constexpr int kSplitOps = 8;
constexpr size_t kSplitLays[kSplitOps] = {3, 3, 5, 5, 3, 3, 5, 5};

struct SplitCall {
    int op;
    natten_problem_t prob;
    std::vector<natten_layout_t> lay;
    std::vector<int64_t> out_shape;  // QK: attn; AV: out; RPB QK backward: the bias gradient
    bool zero_dq;                    // QK backward: dq zeroed where strides leave non-query positions
    int64_t work_floats = 0;         // RPB QK backward: the bias gradient's workspace

    SplitCall(int op_, const pybind11::bytes& prob_bytes, const pybind11::bytes& lay_bytes,
              std::vector<int64_t> out_shape_, bool zero_dq_, int64_t work_floats_)
        : op(op_), out_shape(std::move(out_shape_)), zero_dq(zero_dq_), work_floats(work_floats_) {
        const std::string p = prob_bytes, l = lay_bytes;
        if (op < 0 || op >= kSplitOps) throw pybind11::value_error("SplitCall: unknown op");
        if (work_floats < 0) throw pybind11::value_error("SplitCall: negative workspace");
        if (p.size() != sizeof(natten_problem_t)) throw pybind11::value_error("SplitCall: problem size mismatch");
        if (l.size() != kSplitLays[op] * sizeof(natten_layout_t))
            throw pybind11::value_error("SplitCall: layout size mismatch");
        std::memcpy(&prob, p.data(), sizeof(prob));
        lay.resize(kSplitLays[op]);
        std::memcpy(lay.data(), l.data(), l.size());
    }

    void want(int o) const {
        if (op != o) throw pybind11::value_error("SplitCall: called as another op");
    }

    at::Tensor qk(const at::Tensor& q, const at::Tensor& k, int64_t stream) const {
        want(kQk);
        c10::OptionalDeviceGuard guard;
        if (FusedCall::current_index() != q.get_device()) guard.reset_device(q.device());
        at::Tensor attn = alloc(out_shape, q.scalar_type(), q.device());
        const int rc = natten_hip_qk_forward(&prob, q.data_ptr(), &lay[0], k.data_ptr(), &lay[1], attn.data_ptr(),
                                             &lay[2], reinterpret_cast<void*>(stream));
        if (rc != NATTEN_OK) raise_status(rc, "qk_forward");
        return attn;
    }

    at::Tensor av(const at::Tensor& attn, const at::Tensor& v, int64_t stream) const {
        want(kAv);
        c10::OptionalDeviceGuard guard;
        if (FusedCall::current_index() != v.get_device()) guard.reset_device(v.device());
        at::Tensor out = alloc(out_shape, v.scalar_type(), v.device());
        const int rc = natten_hip_av_forward(&prob, attn.data_ptr(), &lay[0], v.data_ptr(), &lay[1], out.data_ptr(),
                                             &lay[2], reinterpret_cast<void*>(stream));
        if (rc != NATTEN_OK) raise_status(rc, "av_forward");
        return out;
    }

    std::tuple<at::Tensor, at::Tensor> qk_backward(const at::Tensor& da, const at::Tensor& q, const at::Tensor& k,
                                                   int64_t stream) const {
        want(kQkBwd);
        c10::OptionalDeviceGuard guard;
        if (FusedCall::current_index() != q.get_device()) guard.reset_device(q.device());
        at::Tensor dq = alloc(q.sizes(), q.scalar_type(), q.device());
        if (zero_dq) dq.zero_();
        at::Tensor dk = alloc(k.sizes(), k.scalar_type(), k.device());
        const int rc = natten_hip_qk_backward(&prob, da.data_ptr(), &lay[0], q.data_ptr(), &lay[1], k.data_ptr(),
                                              &lay[2], dq.data_ptr(), &lay[3], dk.data_ptr(), &lay[4],
                                              reinterpret_cast<void*>(stream));
        if (rc != NATTEN_OK) raise_status(rc, "qk_backward");
        return {dq, dk};
    }

    std::tuple<at::Tensor, at::Tensor> av_backward(const at::Tensor& dout, const at::Tensor& attn,
                                                   const at::Tensor& v, int64_t stream) const {
        want(kAvBwd);
        c10::OptionalDeviceGuard guard;
        if (FusedCall::current_index() != v.get_device()) guard.reset_device(v.device());
        at::Tensor da = alloc(attn.sizes(), attn.scalar_type(), attn.device());
        at::Tensor dv = alloc(v.sizes(), v.scalar_type(), v.device());
        const int rc = natten_hip_av_backward(&prob, dout.data_ptr(), &lay[0], attn.data_ptr(), &lay[1],
                                              v.data_ptr(), &lay[2], da.data_ptr(), &lay[3], dv.data_ptr(), &lay[4],
                                              reinterpret_cast<void*>(stream));
        if (rc != NATTEN_OK) raise_status(rc, "av_backward");
        return {da, dv};
    }

    at::Tensor rpb_qk(const at::Tensor& q, const at::Tensor& k, const std::optional<at::Tensor>& rpb,
                      int64_t stream) const {
        want(kRpbQk);
        c10::OptionalDeviceGuard guard;
        if (FusedCall::current_index() != q.get_device()) guard.reset_device(q.device());
        at::Tensor attn = alloc(out_shape, q.scalar_type(), q.device());
        const int rc = natten_hip_rpb_qk_forward(&prob, q.data_ptr(), &lay[0], k.data_ptr(), &lay[1],
                                                 rpb.has_value() ? rpb->data_ptr() : nullptr, attn.data_ptr(),
                                                 &lay[2], reinterpret_cast<void*>(stream));
        if (rc != NATTEN_OK) raise_status(rc, "rpb_qk_forward");
        return attn;
    }

    at::Tensor rpb_av(const at::Tensor& attn, const at::Tensor& v, int64_t stream) const {
        want(kRpbAv);
        c10::OptionalDeviceGuard guard;
        if (FusedCall::current_index() != v.get_device()) guard.reset_device(v.device());
        at::Tensor out = alloc(v.sizes(), v.scalar_type(), v.device());
        const int rc = natten_hip_rpb_av_forward(&prob, attn.data_ptr(), &lay[0], v.data_ptr(), &lay[1],
                                                 out.data_ptr(), &lay[2], reinterpret_cast<void*>(stream));
        if (rc != NATTEN_OK) raise_status(rc, "rpb_av_forward");
        return out;
    }

    // (dq, dk, drpb); drpb None without a bias (an empty out_shape)
    pybind11::tuple rpb_qk_backward(const at::Tensor& da, const at::Tensor& q, const at::Tensor& k,
                                    int64_t stream) const {
        want(kRpbQkBwd);
        c10::OptionalDeviceGuard guard;
        if (FusedCall::current_index() != q.get_device()) guard.reset_device(q.device());
        at::Tensor dq = alloc(q.sizes(), q.scalar_type(), q.device());
        at::Tensor dk = alloc(k.sizes(), k.scalar_type(), k.device());
        std::optional<at::Tensor> drpb;
        if (!out_shape.empty()) drpb = alloc(out_shape, q.scalar_type(), q.device());
        const Workspace work(static_cast<size_t>(drpb ? work_floats : 0) * sizeof(float),
                             reinterpret_cast<hipStream_t>(stream));
        const int rc = natten_hip_rpb_qk_backward_ws(
            &prob, da.data_ptr(), &lay[0], q.data_ptr(), &lay[1], k.data_ptr(), &lay[2], dq.data_ptr(), &lay[3],
            dk.data_ptr(), &lay[4], drpb ? drpb->data_ptr() : nullptr, static_cast<float*>(work.ptr),
            work.ptr ? work_floats : 0, reinterpret_cast<void*>(stream));
        if (rc != NATTEN_OK) raise_status(rc, "rpb_qk_backward");
        return pybind11::make_tuple(dq, dk, drpb ? pybind11::cast(*drpb) : pybind11::none());
    }

    std::tuple<at::Tensor, at::Tensor> rpb_av_backward(const at::Tensor& dout, const at::Tensor& attn,
                                                       const at::Tensor& v, int64_t stream) const {
        want(kRpbAvBwd);
        c10::OptionalDeviceGuard guard;
        if (FusedCall::current_index() != v.get_device()) guard.reset_device(v.device());
        at::Tensor da = alloc(attn.sizes(), attn.scalar_type(), attn.device());
        at::Tensor dv = alloc(v.sizes(), v.scalar_type(), v.device());
        const int rc = natten_hip_rpb_av_backward(&prob, dout.data_ptr(), &lay[0], attn.data_ptr(), &lay[1],
                                                  v.data_ptr(), &lay[2], da.data_ptr(), &lay[3], dv.data_ptr(),
                                                  &lay[4], reinterpret_cast<void*>(stream));
        if (rc != NATTEN_OK) raise_status(rc, "rpb_av_backward");
        return {da, dv};
    }
};

// ---------------------------------------------------------------------------
// signature cache of the per-call entry
// ---------------------------------------------------------------------------

// The key: rank, each tensor's dtype, device, sizes and strides, the
// parameter sequences and the scale argument, as 64-bit words.
struct Key {
    static constexpr int kMax = 160;
    int64_t w[kMax];
    int n = 0;
    bool ok = true;

    void put(int64_t x) {
        if (n < kMax) w[n++] = x;
        else ok = false;
    }
    // inner: the innermost stride must be 1; fp32c: fp32 and contiguous
    void tensor(const at::Tensor& t, bool inner, bool fp32c = false) {
        if (!t.defined() || !t.is_cuda()) {
            ok = false;
            return;
        }
        const int64_t d = t.dim();
        put(static_cast<int64_t>(t.scalar_type()));
        put(t.get_device());
        put(d);
        const auto sz = t.sizes(), st = t.strides();
        for (int64_t i = 0; i < d; ++i) {
            put(sz[i]);
            put(st[i]);
        }
        if (inner && (d == 0 || st[d - 1] != 1)) ok = false;
        if (fp32c && (t.scalar_type() != at::kFloat || !t.is_contiguous())) ok = false;
    }
    void ints(pybind11::handle h) {
        PyObject* o = h.ptr();
        if (!PyTuple_Check(o) && !PyList_Check(o)) {
            ok = false;
            return;
        }
        const Py_ssize_t len = PySequence_Fast_GET_SIZE(o);
        put(len);
        for (Py_ssize_t i = 0; i < len; ++i) {
            PyObject* it = PySequence_Fast_GET_ITEM(o, i);
            if (!PyLong_Check(it)) {
                ok = false;
                return;
            }
            const long long x = PyLong_AsLongLong(it);
            if (x == -1 && PyErr_Occurred()) {
                PyErr_Clear();
                ok = false;
                return;
            }
            put(x);
        }
    }
    void scale(pybind11::handle h) {
        PyObject* o = h.ptr();
        if (o == Py_None) {
            put(0);
            put(0);
        } else if (PyFloat_CheckExact(o)) {
            const double x = PyFloat_AS_DOUBLE(o);
            int64_t bits;
            std::memcpy(&bits, &x, sizeof(bits));
            put(1);
            put(bits);
        } else {
            ok = false;
        }
    }
    bool operator==(const Key& o) const { return n == o.n && std::memcmp(w, o.w, n * sizeof(int64_t)) == 0; }
};

template <typename C>
struct Entry {
    Key key;
    C* call;
    pybind11::object owner;
};

constexpr size_t kCacheMax = 64;
std::vector<Entry<FusedCall>> g_fwd, g_bwd;
std::vector<Entry<SplitCall>> g_split[kSplitOps];

template <typename C>
const C* find(const std::vector<Entry<C>>& cache, const Key& k) {
    if (!k.ok) return nullptr;
    for (const Entry<C>& e : cache)
        if (e.key == k) return e.call;
    return nullptr;
}

template <typename C>
bool remember(std::vector<Entry<C>>& cache, const Key& k, pybind11::object call) {
    if (!k.ok) return false;
    if (cache.size() >= kCacheMax) cache.clear();
    cache.push_back(Entry<C>{k, call.cast<C*>(), std::move(call)});
    return true;
}

void clear_all() {
    g_fwd.clear();
    g_bwd.clear();
    for (auto& c : g_split) c.clear();
}

Key fwd_key(int64_t rank, const at::Tensor& q, const at::Tensor& k, const at::Tensor& v, pybind11::handle ks,
            pybind11::handle st, pybind11::handle dil, pybind11::handle causal, pybind11::handle scale) {
    Key key;
    key.put(rank);
    key.tensor(q, true);
    key.tensor(k, true);
    key.tensor(v, true);
    key.ints(ks);
    key.ints(st);
    key.ints(dil);
    key.ints(causal);
    key.scale(scale);
    return key;
}

Key bwd_key(int64_t rank, const at::Tensor& dout, const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
            const at::Tensor& out, const at::Tensor& lse, pybind11::handle ks, pybind11::handle dil,
            pybind11::handle st, pybind11::handle causal, pybind11::handle scale,
            const std::optional<at::Tensor>& dlse) {
    Key key;
    key.put(rank);
    key.tensor(q, true);
    key.tensor(k, true);
    key.tensor(v, true);
    key.tensor(out, true);
    key.tensor(dout, true);
    key.tensor(lse, false, true);
    if (dlse.has_value()) key.tensor(*dlse, false, true);
    else key.put(-1);
    key.ints(ks);
    key.ints(dil);
    key.ints(st);
    key.ints(causal);
    key.scale(scale);
    return key;
}

int64_t current_stream(const at::Tensor& t) {
    return reinterpret_cast<int64_t>(c10::hip::getCurrentHIPStream(t.get_device()).stream());
}

pybind11::object fwd(int64_t rank, const at::Tensor& q, const at::Tensor& k, const at::Tensor& v, pybind11::handle ks,
                     pybind11::handle st, pybind11::handle dil, pybind11::handle causal, pybind11::handle scale) {
    const FusedCall* c = find(g_fwd, fwd_key(rank, q, k, v, ks, st, dil, causal, scale));
    if (!c) return pybind11::none();
    return pybind11::cast(c->forward(q, k, v, current_stream(q)));
}

bool fwd_register(int64_t rank, const at::Tensor& q, const at::Tensor& k, const at::Tensor& v, pybind11::handle ks,
                  pybind11::handle st, pybind11::handle dil, pybind11::handle causal, pybind11::handle scale,
                  pybind11::object call) {
    return remember(g_fwd, fwd_key(rank, q, k, v, ks, st, dil, causal, scale), std::move(call));
}

pybind11::object bwd(int64_t rank, const at::Tensor& dout, const at::Tensor& q, const at::Tensor& k,
                     const at::Tensor& v, const at::Tensor& out, const at::Tensor& lse, pybind11::handle ks,
                     pybind11::handle dil, pybind11::handle st, pybind11::handle causal, pybind11::handle scale,
                     const std::optional<at::Tensor>& dlse) {
    const FusedCall* c = find(g_bwd, bwd_key(rank, dout, q, k, v, out, lse, ks, dil, st, causal, scale, dlse));
    if (!c) return pybind11::none();
    return pybind11::cast(c->backward(q, k, v, out, dout, lse, dlse, current_stream(q)));
}

bool bwd_register(int64_t rank, const at::Tensor& dout, const at::Tensor& q, const at::Tensor& k,
                  const at::Tensor& v, const at::Tensor& out, const at::Tensor& lse, pybind11::handle ks,
                  pybind11::handle dil, pybind11::handle st, pybind11::handle causal, pybind11::handle scale,
                  const std::optional<at::Tensor>& dlse, pybind11::object call) {
    return remember(g_bwd, bwd_key(rank, dout, q, k, v, out, lse, ks, dil, st, causal, scale, dlse),
                    std::move(call));
}

// Split ops: the key of op `op` over its input tensors (every one with a
// unit innermost stride), the parameter sequences and the scale argument
// (None for AV and its backward).
Key split_key(int op, int64_t rank, std::initializer_list<const at::Tensor*> ts, pybind11::handle ks,
              pybind11::handle dil, pybind11::handle st, pybind11::handle causal, pybind11::handle scale) {
    Key key;
    key.put(op);
    key.put(rank);
    for (const at::Tensor* t : ts) key.tensor(*t, true);
    key.ints(ks);
    key.ints(dil);
    key.ints(st);
    key.ints(causal);
    key.scale(scale);
    return key;
}

pybind11::object qk(int64_t rank, const at::Tensor& q, const at::Tensor& k, pybind11::handle ks, pybind11::handle dil,
                    pybind11::handle st, pybind11::handle causal, pybind11::handle scale) {
    const SplitCall* c = find(g_split[kQk], split_key(kQk, rank, {&q, &k}, ks, dil, st, causal, scale));
    if (!c) return pybind11::none();
    return pybind11::cast(c->qk(q, k, current_stream(q)));
}

pybind11::object av(int64_t rank, const at::Tensor& attn, const at::Tensor& v, pybind11::handle ks,
                    pybind11::handle dil, pybind11::handle st, pybind11::handle causal) {
    const SplitCall* c =
        find(g_split[kAv], split_key(kAv, rank, {&attn, &v}, ks, dil, st, causal, pybind11::none()));
    if (!c) return pybind11::none();
    return pybind11::cast(c->av(attn, v, current_stream(v)));
}

pybind11::object qk_bwd(int64_t rank, const at::Tensor& da, const at::Tensor& q, const at::Tensor& k,
                        pybind11::handle ks, pybind11::handle dil, pybind11::handle st, pybind11::handle causal,
                        pybind11::handle scale) {
    const SplitCall* c =
        find(g_split[kQkBwd], split_key(kQkBwd, rank, {&da, &q, &k}, ks, dil, st, causal, scale));
    if (!c) return pybind11::none();
    return pybind11::cast(c->qk_backward(da, q, k, current_stream(q)));
}

pybind11::object av_bwd(int64_t rank, const at::Tensor& dout, const at::Tensor& attn, const at::Tensor& v,
                        pybind11::handle ks, pybind11::handle dil, pybind11::handle st, pybind11::handle causal) {
    const SplitCall* c = find(g_split[kAvBwd],
                              split_key(kAvBwd, rank, {&dout, &attn, &v}, ks, dil, st, causal, pybind11::none()));
    if (!c) return pybind11::none();
    return pybind11::cast(c->av_backward(dout, attn, v, current_stream(v)));
}

// Relative-position-bias ops: the key of op `op` over its input tensors, a
// flag (the bias table's presence or, for QK backward, whether a bias
// gradient is asked for) and the kernel and dilation sequences.
Key rpb_key(int op, int64_t rank, std::initializer_list<const at::Tensor*> ts, const at::Tensor* table, int flag,
            pybind11::handle ks, pybind11::handle dil) {
    Key key;
    key.put(op);
    key.put(rank);
    for (const at::Tensor* t : ts) key.tensor(*t, true);
    if (table) key.tensor(*table, true);
    key.put(flag);
    key.ints(ks);
    key.ints(dil);
    return key;
}

pybind11::object rpb_qk(int64_t rank, const at::Tensor& q, const at::Tensor& k, const std::optional<at::Tensor>& rpb,
                        pybind11::handle ks, pybind11::handle dil) {
    const SplitCall* c = find(g_split[kRpbQk], rpb_key(kRpbQk, rank, {&q, &k}, rpb ? &*rpb : nullptr,
                                                       rpb.has_value(), ks, dil));
    if (!c) return pybind11::none();
    return pybind11::cast(c->rpb_qk(q, k, rpb, current_stream(q)));
}

pybind11::object rpb_av(int64_t rank, const at::Tensor& attn, const at::Tensor& v, pybind11::handle ks,
                        pybind11::handle dil) {
    const SplitCall* c = find(g_split[kRpbAv], rpb_key(kRpbAv, rank, {&attn, &v}, nullptr, 0, ks, dil));
    if (!c) return pybind11::none();
    return pybind11::cast(c->rpb_av(attn, v, current_stream(v)));
}

pybind11::object rpb_qk_bwd(int64_t rank, const at::Tensor& da, const at::Tensor& q, const at::Tensor& k,
                            bool with_rpb, pybind11::handle ks, pybind11::handle dil) {
    const SplitCall* c =
        find(g_split[kRpbQkBwd], rpb_key(kRpbQkBwd, rank, {&da, &q, &k}, nullptr, with_rpb, ks, dil));
    if (!c) return pybind11::none();
    return c->rpb_qk_backward(da, q, k, current_stream(q));
}

pybind11::object rpb_av_bwd(int64_t rank, const at::Tensor& dout, const at::Tensor& attn, const at::Tensor& v,
                            pybind11::handle ks, pybind11::handle dil) {
    const SplitCall* c = find(g_split[kRpbAvBwd], rpb_key(kRpbAvBwd, rank, {&dout, &attn, &v}, nullptr, 0, ks, dil));
    if (!c) return pybind11::none();
    return pybind11::cast(c->rpb_av_backward(dout, attn, v, current_stream(v)));
}

// ts: the op's input tensors in argument order (RPB QK: q, k and the bias
// table when there is one); flag as in rpb_key.
bool rpb_register(int64_t rank, const std::vector<at::Tensor>& ts, int flag, pybind11::handle ks,
                  pybind11::handle dil, pybind11::object call) {
    const int op = call.cast<SplitCall&>().op;
    if (op < kRpbQk) throw pybind11::value_error("rpb_register: not a relative-position-bias op");
    Key key;
    if (op == kRpbQk) {
        if (ts.size() != 2 + (flag ? 1 : 0)) throw pybind11::value_error("rpb_register: wrong number of tensors");
        key = rpb_key(op, rank, {&ts[0], &ts[1]}, flag ? &ts[2] : nullptr, flag, ks, dil);
    } else if (op == kRpbAv) {
        if (ts.size() != 2) throw pybind11::value_error("rpb_register: wrong number of tensors");
        key = rpb_key(op, rank, {&ts[0], &ts[1]}, nullptr, flag, ks, dil);
    } else {
        if (ts.size() != 3) throw pybind11::value_error("rpb_register: wrong number of tensors");
        key = rpb_key(op, rank, {&ts[0], &ts[1], &ts[2]}, nullptr, flag, ks, dil);
    }
    return remember(g_split[op], key, std::move(call));
}

bool split_register(int64_t rank, const std::vector<at::Tensor>& ts, pybind11::handle ks, pybind11::handle dil,
                    pybind11::handle st, pybind11::handle causal, pybind11::handle scale, pybind11::object call) {
    const int op = call.cast<SplitCall&>().op;
    if (op > kAvBwd) throw pybind11::value_error("split_register: a relative-position-bias op (rpb_register)");
    const size_t n = op == kQk || op == kAv ? 2 : 3;
    if (ts.size() != n) throw pybind11::value_error("split_register: wrong number of tensors");
    const Key key = n == 2 ? split_key(op, rank, {&ts[0], &ts[1]}, ks, dil, st, causal, scale)
                           : split_key(op, rank, {&ts[0], &ts[1], &ts[2]}, ks, dil, st, causal, scale);
    return remember(g_split[op], key, std::move(call));
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
    m.doc() = "Host binding of the fused and split entry points for the 'hip' backend";
    m.attr("abi_version") = natten_hip_abi_version();
    pybind11::class_<FusedCall>(m, "FusedCall")
        .def(pybind11::init<const pybind11::bytes&, const pybind11::bytes&, std::vector<int64_t>,
                            std::vector<int64_t>, bool>())
        .def("forward", &FusedCall::forward)
        .def("backward", &FusedCall::backward);
    m.def("fwd", &fwd, "cached fused forward: (out, lse), or None when the signature is not registered");
    m.def("fwd_register", &fwd_register, "register the FusedCall of a forward signature");
    m.def("bwd", &bwd, "cached fused backward: (dq, dk, dv), or None when the signature is not registered");
    m.def("bwd_register", &bwd_register, "register the FusedCall of a backward signature");
    pybind11::class_<SplitCall>(m, "SplitCall")
        .def(pybind11::init<int, const pybind11::bytes&, const pybind11::bytes&, std::vector<int64_t>, bool,
                            int64_t>(),
             pybind11::arg("op"), pybind11::arg("prob"), pybind11::arg("layouts"), pybind11::arg("out_shape"),
             pybind11::arg("zero_dq"), pybind11::arg("work_floats") = 0)
        .def_readonly("op", &SplitCall::op)
        .def("qk", &SplitCall::qk)
        .def("av", &SplitCall::av)
        .def("qk_backward", &SplitCall::qk_backward)
        .def("av_backward", &SplitCall::av_backward)
        .def("rpb_qk", &SplitCall::rpb_qk)
        .def("rpb_av", &SplitCall::rpb_av)
        .def("rpb_qk_backward", &SplitCall::rpb_qk_backward)
        .def("rpb_av_backward", &SplitCall::rpb_av_backward);
    m.def("rpb_qk", &rpb_qk, "cached relative-position-bias QK: attn, or None");
    m.def("rpb_av", &rpb_av, "cached relative-position-bias AV: out, or None");
    m.def("rpb_qk_bwd", &rpb_qk_bwd, "cached relative-position-bias QK backward: (dq, dk, drpb), or None");
    m.def("rpb_av_bwd", &rpb_av_bwd, "cached relative-position-bias AV backward: (dattn, dv), or None");
    m.def("rpb_register", &rpb_register, "register the SplitCall of a relative-position-bias op signature");
    m.def("qk", &qk, "cached split QK: attn, or None when the signature is not registered");
    m.def("av", &av, "cached split AV: out, or None when the signature is not registered");
    m.def("qk_bwd", &qk_bwd, "cached split QK backward: (dq, dk), or None");
    m.def("av_bwd", &av_bwd, "cached split AV backward: (dattn, dv), or None");
    m.def("split_register", &split_register,
          "register the SplitCall of a split-op signature (its input tensors in the op's argument order)");
    m.def("clear", &clear_all, "drop every registered signature");
    // the cached objects hold Python references: release them before the
    // interpreter's own teardown
    auto atexit = pybind11::module_::import("atexit");
    atexit.attr("register")(pybind11::cpp_function(&clear_all));
}

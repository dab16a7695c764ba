// Host binding of the fused forward / backward for the 'hip' backend: the
// per-call work of natten_mps_amd/_core/hip.py (output allocation, the C
// call, the status check) in C++ on top of the C ABI, so an eager step pays
// a few microseconds of host time instead of the ctypes marshalling of ten to
// twenty arguments and one torch allocation per output from Python.
//
// A FusedCall holds what is fixed per call signature (shapes, strides,
// dtype, parameters): the problem descriptor and the element-stride layouts
// that hip.py computed once, and the output shapes.  forward / backward
// allocate the outputs with ATen on the inputs' device and call
// natten_hip_forward / natten_hip_backward on the stream given (the raw
// hipStream_t of torch's current stream, passed by the caller).  Errors map
// as in the ctypes path: invalid input -> ValueError, unsupported ->
// NotImplementedError, launch failure -> RuntimeError.
//
// Reference: the backend hooks this serves are those the autograd factory
// calls (autograd/_factory.py:37-38,66-67 of /root/reference/src/natten_mps).
#include <torch/extension.h>

#include <c10/core/DeviceGuard.h>
#include <c10/core/impl/DeviceGuardImplInterface.h>

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
        at::Tensor out = at::empty(out_shape, q.options());
        at::Tensor lse = at::empty(lse_shape, q.options().dtype(at::kFloat));
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
        // dq is zeroed where stride > 1 leaves positions that are not queries
        at::Tensor dq = strided ? at::zeros(q.sizes(), q.options()) : at::empty(q.sizes(), q.options());
        at::Tensor dk = at::empty(k.sizes(), k.options());
        at::Tensor dv = at::empty(v.sizes(), v.options());
        at::Tensor delta = at::empty(lse_shape, q.options().dtype(at::kFloat));
        const float* dl = d_lse.has_value() ? d_lse->data_ptr<float>() : nullptr;
        const int rc = natten_hip_backward(
            &prob, q.data_ptr(), &lay[0], k.data_ptr(), &lay[1], v.data_ptr(), &lay[2], out.data_ptr(), &lay[3],
            d_out.data_ptr(), &lay[4], lse.data_ptr<float>(), &lay[5], dl, dl ? &lay[6] : nullptr, dq.data_ptr(),
            &lay[7], dk.data_ptr(), &lay[8], dv.data_ptr(), &lay[9], delta.data_ptr<float>(), &lay[10],
            reinterpret_cast<void*>(stream));
        if (rc != NATTEN_OK) raise_status(rc, "backward");
        return {dq, dk, dv};
    }

    static int current_index() {
        return c10::impl::getDeviceGuardImpl(c10::DeviceType::CUDA)->getDevice().index();
    }
};

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
    m.doc() = "Host binding of natten_hip_forward / natten_hip_backward for the 'hip' backend";
    m.attr("abi_version") = natten_hip_abi_version();
    pybind11::class_<FusedCall>(m, "FusedCall")
        .def(pybind11::init<const pybind11::bytes&, const pybind11::bytes&, std::vector<int64_t>,
                            std::vector<int64_t>, bool>())
        .def("forward", &FusedCall::forward)
        .def("backward", &FusedCall::backward);
}

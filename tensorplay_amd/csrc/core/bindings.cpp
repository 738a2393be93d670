// Python bindings (pybind11; nanobind, which the reference uses, is not in this
// image).  The method overloads mirror TensorPlay's reduction surface
// (/root/reference/src/bindings/python/Tensor.cpp:1099-1224): each reduction
// takes dim as an int or a list, keepdim, and (sum/mean) a keyword dtype;
// var/std take correction.  topk is added.  C++ exceptions map to the Python
// exception of the same name (as src/bindings/python/init.cpp:13-38).
#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include <sstream>

#include "Allocator.h"
#include "Dispatcher.h"
#include "Exception.h"
#include "Tensor.h"
#include "tpr_rocm.h"

namespace py = pybind11;
using namespace tensorplay;

namespace {

DType dtype_from_numpy(const py::dtype& dt) {
    const char k = dt.kind();
    const size_t sz = dt.itemsize();
    if (k == 'f' && sz == 4) return DType::Float32;
    if (k == 'f' && sz == 8) return DType::Float64;
    if (k == 'i' && sz == 8) return DType::Int64;
    if (k == 'i' && sz == 4) return DType::Int32;
    if (k == 'i' && sz == 2) return DType::Int16;
    if (k == 'i' && sz == 1) return DType::Int8;
    if (k == 'u' && sz == 1) return DType::UInt8;
    if (k == 'u' && sz == 2) return DType::UInt16;
    if (k == 'u' && sz == 4) return DType::UInt32;
    if (k == 'u' && sz == 8) return DType::UInt64;
    if (k == 'b') return DType::Bool;
    TP_THROW(TypeError, "unsupported numpy dtype");
}

py::dtype numpy_dtype(DType t) {
    switch (t) {
        case DType::Float32: return py::dtype::of<float>();
        case DType::Float64: return py::dtype::of<double>();
        case DType::Int64: return py::dtype::of<int64_t>();
        case DType::Int32: return py::dtype::of<int32_t>();
        case DType::Int16: return py::dtype::of<int16_t>();
        case DType::Int8: return py::dtype::of<int8_t>();
        case DType::UInt8: return py::dtype::of<uint8_t>();
        case DType::UInt16: return py::dtype::of<uint16_t>();
        case DType::UInt32: return py::dtype::of<uint32_t>();
        case DType::UInt64: return py::dtype::of<uint64_t>();
        case DType::Bool: return py::dtype::of<bool>();
        default: TP_THROW(TypeError, "no numpy dtype for this tensor dtype");
    }
}

Device to_device(const py::object& o) {
    if (py::isinstance<Device>(o)) return o.cast<Device>();
    return Device(o.cast<std::string>());
}

Tensor from_numpy(py::array arr, std::optional<DType> dtype, const py::object& device) {
    py::array c = py::array::ensure(arr, py::array::c_style | py::array::forcecast);
    DType dt = dtype_from_numpy(c.dtype());
    if (dtype && *dtype != dt) {
        c = py::array(numpy_dtype(*dtype), py::array::ShapeContainer(c.shape(), c.shape() + c.ndim()));
        py::array src = py::array::ensure(arr, py::array::c_style | py::array::forcecast);
        py::module_::import("numpy").attr("copyto")(c, src, py::arg("casting") = "unsafe");
        dt = *dtype;
    }
    std::vector<int64_t> shape(c.shape(), c.shape() + c.ndim());
    return Tensor::fromHost(c.data(), shape, dt, to_device(device));
}

py::array to_numpy(const Tensor& t) {
    std::vector<py::ssize_t> shape(t.shape().begin(), t.shape().end());
    py::array out(numpy_dtype(t.dtype()), shape);
    t.copyToHost(out.mutable_data());
    return out;
}

std::string repr(const Tensor& t) {
    std::ostringstream os;
    os << "tensor(shape=[";
    for (size_t i = 0; i < t.shape().size(); ++i) os << (i ? ", " : "") << t.shape()[i];
    os << "], dtype=" << toString(t.dtype()) << ", device=" << t.device().str() << ")";
    return os.str();
}

DType opt_dtype(const std::optional<DType>& d) { return d.value_or(DType::Undefined); }

}  // namespace

PYBIND11_MODULE(_C, m) {
    m.doc() = "tensorplay_amd native core: P10-shaped tensor + dispatcher with a ROCm backend";

    py::register_exception_translator([](std::exception_ptr p) {
        try {
            if (p) std::rethrow_exception(p);
        } catch (const IndexError& e) {
            PyErr_SetString(PyExc_IndexError, e.what());
        } catch (const TypeError& e) {
            PyErr_SetString(PyExc_TypeError, e.what());
        } catch (const ValueError& e) {
            PyErr_SetString(PyExc_ValueError, e.what());
        } catch (const NotImplementedError& e) {
            PyErr_SetString(PyExc_NotImplementedError, e.what());
        } catch (const RuntimeError& e) {
            PyErr_SetString(PyExc_RuntimeError, e.what());
        }
    });

    py::enum_<DType>(m, "DType")
        .value("uint8", DType::UInt8).value("int8", DType::Int8).value("int16", DType::Int16)
        .value("int32", DType::Int32).value("int64", DType::Int64).value("uint16", DType::UInt16)
        .value("uint32", DType::UInt32).value("uint64", DType::UInt64).value("float32", DType::Float32)
        .value("float64", DType::Float64).value("bool", DType::Bool).value("undefined", DType::Undefined);

    py::class_<Device>(m, "Device")
        .def(py::init<const std::string&>())
        .def_property_readonly("type", [](const Device& d) { return d.is_cpu() ? "cpu" : "rocm"; })
        .def_property_readonly("index", [](const Device& d) { return d.index; })
        .def("__repr__", [](const Device& d) { return "device('" + d.str() + "')"; })
        .def("__str__", &Device::str)
        .def("__eq__", [](const Device& a, const Device& b) { return a == b; });

    py::class_<Tensor> t(m, "TensorBase");
    t.def_property_readonly("shape", [](const Tensor& x) { return std::vector<int64_t>(x.shape()); })
        .def_property_readonly("dtype", &Tensor::dtype)
        .def_property_readonly("device", &Tensor::device)
        .def_property_readonly("ndim", &Tensor::dim)
        .def("dim", &Tensor::dim)
        .def("numel", &Tensor::numel)
        .def("size", [](const Tensor& x, std::optional<int64_t> d) -> py::object {
            if (d) return py::int_(x.size(*d));
            return py::cast(std::vector<int64_t>(x.shape()));
        }, py::arg("dim") = py::none())
        .def("stride", [](const Tensor& x) { return std::vector<int64_t>(x.strides()); })
        .def("storage_offset", &Tensor::storage_offset)
        .def("is_contiguous", &Tensor::is_contiguous)
        .def("contiguous", &Tensor::contiguous)
        .def("clone", &Tensor::clone)
        .def("data_ptr", [](const Tensor& x) { return reinterpret_cast<uintptr_t>(x.data_ptr()); })
        .def("record_stream", [](const Tensor& x, uintptr_t s) { x.record_stream(reinterpret_cast<void*>(s)); },
             py::arg("stream"))
        .def("transpose", &Tensor::transpose)
        .def("permute", [](const Tensor& x, const std::vector<int64_t>& d) { return x.permute(d); })
        .def("reshape", [](const Tensor& x, const std::vector<int64_t>& s) { return x.reshape(s); })
        .def("to", [](const Tensor& x, const py::object& arg) {
            if (py::isinstance<DType>(arg)) return x.to(arg.cast<DType>());
            return x.to(to_device(arg));
        })
        .def("copy_", [](Tensor& x, const Tensor& src) { return x.copy_(src); }, py::arg("src"))
        .def("cpu", &Tensor::cpu)
        .def("rocm", [](const Tensor& x, int index) { return x.to(Device(DeviceType::ROCm, index)); },
             py::arg("index") = 0)
        .def("numpy", &to_numpy)
        .def("item", [](const Tensor& x) -> py::object {
            if (isIntegralType(x.dtype(), false)) return py::int_(x.item_int());
            if (x.dtype() == DType::Bool) return py::bool_(x.item() != 0.0);
            return py::float_(x.item());
        })
        .def("__repr__", &repr)
        .def("__getitem__", [](const Tensor& x, int64_t i) {
            if (x.dim() == 0) TP_THROW(IndexError, "invalid index of a 0-dim tensor");
            const int64_t n = x.shape()[0];
            if (i < 0) i += n;
            if (i < 0 || i >= n) TP_THROW(IndexError, "index out of range");
            std::vector<int64_t> sz(x.shape().begin() + 1, x.shape().end());
            std::vector<int64_t> st(x.strides().begin() + 1, x.strides().end());
            return x.as_strided(sz, st, x.storage_offset() + i * x.strides()[0]);
        });

    // ---- reductions (Tensor.cpp:1101-1224 overload set) ----
    using V = std::vector<int64_t>;
    t.def("sum", [](const Tensor& s, std::optional<DType> dt) { return s.sum(opt_dtype(dt)); },
          py::kw_only(), py::arg("dtype") = py::none())
        .def("sum", [](const Tensor& s, const V& d, bool k, std::optional<DType> dt) { return s.sum(d, k, opt_dtype(dt)); },
             py::arg("dim"), py::arg("keepdim") = false, py::kw_only(), py::arg("dtype") = py::none())
        .def("sum", [](const Tensor& s, int64_t d, bool k, std::optional<DType> dt) { return s.sum(V{d}, k, opt_dtype(dt)); },
             py::arg("dim"), py::arg("keepdim") = false, py::kw_only(), py::arg("dtype") = py::none())
        .def("mean", [](const Tensor& s, std::optional<DType> dt) { return s.mean(opt_dtype(dt)); },
             py::kw_only(), py::arg("dtype") = py::none())
        .def("mean", [](const Tensor& s, const V& d, bool k, std::optional<DType> dt) { return s.mean(d, k, opt_dtype(dt)); },
             py::arg("dim"), py::arg("keepdim") = false, py::kw_only(), py::arg("dtype") = py::none())
        .def("mean", [](const Tensor& s, int64_t d, bool k, std::optional<DType> dt) { return s.mean(V{d}, k, opt_dtype(dt)); },
             py::arg("dim"), py::arg("keepdim") = false, py::kw_only(), py::arg("dtype") = py::none())
        .def("max", [](const Tensor& s) { return s.max(); })
        .def("max", [](const Tensor& s, const V& d, bool k) { return s.max(d, k); }, py::arg("dim"),
             py::arg("keepdim") = false)
        .def("max", [](const Tensor& s, int64_t d, bool k) { return s.max(V{d}, k); }, py::arg("dim"),
             py::arg("keepdim") = false)
        .def("min", [](const Tensor& s) { return s.min(); })
        .def("min", [](const Tensor& s, const V& d, bool k) { return s.min(d, k); }, py::arg("dim"),
             py::arg("keepdim") = false)
        .def("min", [](const Tensor& s, int64_t d, bool k) { return s.min(V{d}, k); }, py::arg("dim"),
             py::arg("keepdim") = false)
        .def("argmax", [](const Tensor& s, std::optional<int64_t> d, bool k) { return s.argmax(d, k); },
             py::arg("dim") = py::none(), py::arg("keepdim") = false)
        .def("argmin", [](const Tensor& s, std::optional<int64_t> d, bool k) { return s.argmin(d, k); },
             py::arg("dim") = py::none(), py::arg("keepdim") = false)
        .def("var", [](const Tensor& s, int64_t c) { return s.var(c); }, py::arg("correction") = 1)
        .def("var", [](const Tensor& s, const V& d, int64_t c, bool k) { return s.var(d, c, k); }, py::arg("dim"),
             py::arg("correction") = 1, py::arg("keepdim") = false)
        .def("var", [](const Tensor& s, int64_t d, int64_t c, bool k) { return s.var(V{d}, c, k); }, py::arg("dim"),
             py::arg("correction") = 1, py::arg("keepdim") = false)
        .def("std", [](const Tensor& s, int64_t c) { return s.std(c); }, py::arg("correction") = 1)
        .def("std", [](const Tensor& s, const V& d, int64_t c, bool k) { return s.std(d, c, k); }, py::arg("dim"),
             py::arg("correction") = 1, py::arg("keepdim") = false)
        .def("std", [](const Tensor& s, int64_t d, int64_t c, bool k) { return s.std(V{d}, c, k); }, py::arg("dim"),
             py::arg("correction") = 1, py::arg("keepdim") = false)
        .def("prod", [](const Tensor& s, std::optional<DType> dt) { return s.prod(opt_dtype(dt)); },
             py::kw_only(), py::arg("dtype") = py::none())
        .def("prod", [](const Tensor& s, const V& d, bool k, std::optional<DType> dt) { return s.prod(d, k, opt_dtype(dt)); },
             py::arg("dim"), py::arg("keepdim") = false, py::kw_only(), py::arg("dtype") = py::none())
        .def("prod", [](const Tensor& s, int64_t d, bool k, std::optional<DType> dt) { return s.prod(V{d}, k, opt_dtype(dt)); },
             py::arg("dim"), py::arg("keepdim") = false, py::kw_only(), py::arg("dtype") = py::none())
        .def("all", [](const Tensor& s) { return s.all(); })
        .def("all", [](const Tensor& s, const V& d, bool k) { return s.all(d, k); }, py::arg("dim"),
             py::arg("keepdim") = false)
        .def("all", [](const Tensor& s, int64_t d, bool k) { return s.all(V{d}, k); }, py::arg("dim"),
             py::arg("keepdim") = false)
        .def("any", [](const Tensor& s) { return s.any(); })
        .def("any", [](const Tensor& s, const V& d, bool k) { return s.any(d, k); }, py::arg("dim"),
             py::arg("keepdim") = false)
        .def("any", [](const Tensor& s, int64_t d, bool k) { return s.any(V{d}, k); }, py::arg("dim"),
             py::arg("keepdim") = false)
        .def("median", [](const Tensor& s) { return s.median(); })
        .def("norm", [](const Tensor& s, double p) { return s.norm(p); }, py::arg("p") = 2.0)
        .def("norm", [](const Tensor& s, const V& d, double p, bool k) { return s.norm(d, p, k); }, py::arg("dim"),
             py::arg("p") = 2.0, py::arg("keepdim") = false)
        .def("norm", [](const Tensor& s, int64_t d, double p, bool k) { return s.norm(V{d}, p, k); }, py::arg("dim"),
             py::arg("p") = 2.0, py::arg("keepdim") = false)
        .def("topk", [](const Tensor& s, int64_t k, int64_t d, bool largest, bool sorted) {
            return s.topk(k, d, largest, sorted);
        }, py::arg("k"), py::arg("dim") = -1, py::arg("largest") = true, py::arg("sorted") = true)
        .def("softmax", [](const Tensor& s, int64_t d, std::optional<DType> dt) { return s.softmax(d, opt_dtype(dt)); },
             py::arg("dim"), py::arg("dtype") = py::none())
        .def("log_softmax", [](const Tensor& s, int64_t d, std::optional<DType> dt) {
            return s.log_softmax(d, opt_dtype(dt));
        }, py::arg("dim"), py::arg("dtype") = py::none());

    // ---- function-only schemas (tensorplay/functional.py:313-317, 496-500) ----
    m.def("softmax", [](const Tensor& s, int64_t d, std::optional<DType> dt) { return s.softmax(d, opt_dtype(dt)); },
          py::arg("self"), py::arg("dim"), py::arg("dtype") = py::none());
    m.def("log_softmax", [](const Tensor& s, int64_t d, std::optional<DType> dt) {
        return s.log_softmax(d, opt_dtype(dt));
    }, py::arg("self"), py::arg("dim"), py::arg("dtype") = py::none());
    m.def("nll_loss", [](const Tensor& s, const Tensor& t, std::optional<Tensor> w, int64_t r, int64_t ig) {
        return nll_loss(s, t, w, r, ig);
    }, py::arg("self"), py::arg("target"), py::arg("weight") = py::none(), py::arg("reduction") = 1,
       py::arg("ignore_index") = -100);
    m.def("nll_loss_backward", [](const Tensor& g, const Tensor& s, const Tensor& t, std::optional<Tensor> w,
                                  int64_t r, int64_t ig, std::optional<Tensor> tw) {
        return nll_loss_backward(g, s, t, w, r, ig, tw.value_or(Tensor()));
    }, py::arg("grad_output"), py::arg("self"), py::arg("target"), py::arg("weight") = py::none(),
       py::arg("reduction") = 1, py::arg("ignore_index") = -100, py::arg("total_weight") = py::none());
    m.def("topk_topp_sample", [](const Tensor& s, const Tensor& u, int64_t k, double t, double p) {
        return topk_topp_sample(s, u, k, t, p);
    }, py::arg("self"), py::arg("uniforms"), py::arg("k") = 50, py::arg("temperature") = 1.0, py::arg("top_p") = 1.0);
    m.def("sum_backward", [](const Tensor& g, const Tensor& s, const V& d, bool k) { return sum_backward(g, s, d, k); },
          py::arg("grad"), py::arg("self"), py::arg("dim") = V{}, py::arg("keepdim") = false);
    m.def("mean_backward", [](const Tensor& g, const Tensor& s, const V& d, bool k) { return mean_backward(g, s, d, k); },
          py::arg("grad"), py::arg("self"), py::arg("dim") = V{}, py::arg("keepdim") = false);
    m.def("var_backward", [](const Tensor& g, const Tensor& s, const V& d, int64_t c, bool k) {
        return var_backward(g, s, d, c, k);
    }, py::arg("grad"), py::arg("self"), py::arg("dim") = V{}, py::arg("correction") = 1, py::arg("keepdim") = false);
    m.def("std_backward", [](const Tensor& g, const Tensor& s, const Tensor& r, const V& d, int64_t c, bool k) {
        return std_backward(g, s, r, d, c, k);
    }, py::arg("grad"), py::arg("self"), py::arg("result"), py::arg("dim") = V{}, py::arg("correction") = 1,
       py::arg("keepdim") = false);
    m.def("_softmax_backward_data", [](const Tensor& g, const Tensor& y, int64_t d) {
        return _softmax_backward_data(g, y, d, DType::Float32);
    }, py::arg("grad_output"), py::arg("output"), py::arg("dim"));
    m.def("_log_softmax_backward_data", [](const Tensor& g, const Tensor& y, int64_t d) {
        return _log_softmax_backward_data(g, y, d, DType::Float32);
    }, py::arg("grad_output"), py::arg("output"), py::arg("dim"));

    // ---- factories ----
    m.def("tensor", &from_numpy, py::arg("data"), py::arg("dtype") = py::none(), py::arg("device") = "cpu");
    m.def("empty", [](const V& shape, DType dt, const py::object& dev) { return Tensor::empty(shape, dt, to_device(dev)); },
          py::arg("shape"), py::arg("dtype") = DType::Float32, py::arg("device") = "cpu");
    m.def("_from_device_ptr", [](uintptr_t ptr, const V& shape, const V& strides, DType dt, int index, py::object owner) {
        auto keep = std::shared_ptr<void>(new py::object(std::move(owner)), [](void* p) {
            py::gil_scoped_acquire g;
            delete static_cast<py::object*>(p);
        });
        return Tensor::fromExternal(reinterpret_cast<void*>(ptr), shape, strides, dt, Device(DeviceType::ROCm, index), keep);
    }, py::arg("ptr"), py::arg("shape"), py::arg("strides"), py::arg("dtype"), py::arg("device_index"), py::arg("owner"),
       "Wraps device memory owned by `owner` (e.g. a torch tensor) without copying.");
    m.def("_reduction_shape", &reductionShape);
    m.def("_registered_ops", [](const std::string& key) {
        if (key == "ROCm") return Dispatcher::singleton().registeredOps(DispatchKey::ROCm);
        if (key == "CPU") return Dispatcher::singleton().registeredOps(DispatchKey::CPU);
        TP_THROW(ValueError, "unknown dispatch key " + key);
    });

    auto r = m.def_submodule("_rocm", "ROCm device runtime");
    r.def("is_available", [] { return rocmDeviceCount() > 0; });
    r.def("device_count", &rocmDeviceCount);
    r.def("synchronize", &synchronize, py::arg("device") = 0);
    r.def("set_stream", [](uintptr_t s, int dev) { setCurrentStream(dev, reinterpret_cast<void*>(s)); },
          py::arg("stream"), py::arg("device") = 0);
    r.def("current_stream", [](int dev) { return reinterpret_cast<uintptr_t>(currentStream(dev)); },
          py::arg("device") = 0);
    r.def("empty_cache", &emptyCache);
    r.def("release_stream_blocks", [](uintptr_t s, int dev) { releaseStreamBlocks(dev, reinterpret_cast<void*>(s)); },
          py::arg("stream"), py::arg("device") = 0);
    r.def("memory_stats", [](int dev) {
        AllocatorStats s = allocatorStats(dev);
        py::dict d;
        d["allocated_bytes"] = s.allocated_bytes;
        d["cached_bytes"] = s.cached_bytes;
        d["pending_bytes"] = s.pending_bytes;
        d["device_allocs"] = s.device_allocs;
        d["requests"] = s.requests;
        d["leaked_bytes"] = s.leaked_bytes;
        return d;
    }, py::arg("device") = 0);
    r.def("abi_version", [] { return tpr_abi_version(); });
}

// Python bindings of the host core: the `oxitorch_amd._native` module.
// Restates the PyO3 surface of crates/oxi-bindings/src/lib.rs (PyTensor and
// the free functions) over the device-backed Var graph, and the exception
// mapping of crates/oxi-bindings/src/error.rs:22-32.
#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include <algorithm>
#include <cmath>
#include <sstream>

#include "host.h"

namespace py = pybind11;
using namespace oxt;

namespace {

struct PyTensor {
  Var v;
  explicit PyTensor(Var var) : v(std::move(var)) {}
  const Tensor& value() const { return v.value(); }
};

PyTensor leaf(Tensor t, bool rg = false) { return PyTensor(Var::leaf(std::move(t), rg)); }

// "cpu", or a HIP device: "hip" / "cuda" (the bound device, OXI_HIP_DEVICE
// before the first device use) or "hip:N" / "cuda:N", which binds device N
// (crates/oxi-core/src/lib.rs:139-146: a device is a family and an index).
// The library runs on one device per process.
Dev parse_device(const py::object& d) {
  if (d.is_none()) return default_device();
  const std::string s = py::str(d);
  if (s == "cpu" || s == "cpu:0") return Dev::Cpu;
  const size_t colon = s.find(':');
  const std::string fam = s.substr(0, colon);
  if (fam != "hip" && fam != "cuda")
    err_invalid("unknown device \"" + s + "\" (expected \"cpu\", \"hip\" or \"hip:N\")");
  if (colon == std::string::npos) return Dev::Hip;
  const std::string idx = s.substr(colon + 1);
  if (idx.empty() || idx.size() > 6 || idx.find_first_not_of("0123456789") != std::string::npos)
    err_invalid("invalid device index in \"" + s + "\"");
  bind_device(std::stoi(idx));
  return Dev::Hip;
}

// buffer_to_f32 (bindings lib.rs:31-42)
Tensor from_buffer(const py::object& obj, Dev d) {
  py::buffer_info info;
  try {
    info = py::reinterpret_borrow<py::buffer>(obj).request();
  } catch (const std::exception&) {
    throw py::type_error("expected a numpy array or f32 buffer object");
  }
  if (info.format != py::format_descriptor<float>::format() || info.itemsize != 4)
    throw py::type_error("expected a numpy array or f32 buffer object");
  Shape shape(info.shape.begin(), info.shape.end());
  // C-contiguity check
  ssize_t expect = 4;
  for (int i = (int)info.ndim - 1; i >= 0; --i) {
    if (info.shape[i] != 1 && info.strides[i] != expect)
      throw py::value_error("only contiguous numpy arrays are accepted at the boundary; call .copy() first");
    expect *= info.shape[i];
  }
  return t_from_host(static_cast<const float*>(info.ptr), shape, d);
}

bool is_f32_buffer(const py::object& obj) {
  if (!py::isinstance<py::buffer>(obj)) return false;
  try {
    py::buffer_info info = py::reinterpret_borrow<py::buffer>(obj).request();
    return info.format == py::format_descriptor<float>::format();
  } catch (...) {
    return false;
  }
}

std::string fmt_float(float v) {
  std::ostringstream o;
  o << v;
  return o.str();
}

// Display of Tensor (crates/oxi-tensor/src/lib.rs:1168-1209)
std::string display(const Tensor& t) {
  std::vector<float> data = t_to_host(t);
  std::ostringstream o;
  if (t.ndim() == 0) {
    o << fmt_float(data.empty() ? 0.f : data[0]);
    return o.str();
  }
  o << "Tensor(shape=" << fmt_shape(t.shape) << ", dtype=float32, device=" << dev_name(t.dev()) << ")\n";
  if (t.ndim() == 1) {
    for (size_t i = 0; i < data.size() && i < 6; ++i) o << "  [" << i << "] " << fmt_float(data[i]) << "\n";
    if (data.size() > 6) o << "  ... (" << data.size() - 6 << " more)\n";
  } else {
    const int64_t rows = std::min<int64_t>(t.shape[0], 6);
    const int64_t cols = t.shape.back();
    for (int64_t r = 0; r < rows; ++r) {
      o << "  [";
      for (int64_t c = 0; c < cols && r * cols + c < (int64_t)data.size(); ++c)
        o << (c ? ", " : "") << fmt_float(data[(size_t)(r * cols + c)]);
      o << "]\n";
    }
    if (t.shape[0] > 6) o << "  ... (" << t.shape[0] - 6 << " more rows)\n";
  }
  return o.str();
}

// Binary-dunder operand: a tensor or a Python number promoted to a constant
// leaf of self's shape (bindings lib.rs:51-104).
Var operand(const PyTensor& self, const py::object& other) {
  if (py::isinstance<PyTensor>(other)) return other.cast<PyTensor&>().v;
  if (py::isinstance<py::float_>(other) || py::isinstance<py::int_>(other)) {
    const float c = (float)other.cast<double>();
    return Var::leaf(t_scalar_full(self.value().shape, c, self.value().dev()), false);
  }
  throw py::type_error("operands must be oxitorch.Tensor or a Python number");
}

PyTensor reduce_all(const PyTensor& self, Reduce kind) {  // bindings lib.rs:126-143
  if (self.v.requires_grad() && (kind == Reduce::Sum || kind == Reduce::Mean)) {
    const int nd = self.value().ndim();
    if (nd == 0) return self;
    Var v = self.v;
    for (int d = 0; d < nd; ++d) v = aops::reduce(v, kind, d, true);
    return PyTensor(aops::reshape(v, {}));
  }
  return leaf(t_reduce_all(kind, self.value()));
}

PyTensor dim_reduce(const PyTensor& self, Reduce kind, const py::object& dim, bool keepdim) {
  if (dim.is_none()) return reduce_all(self, kind);
  return PyTensor(aops::reduce(self.v, kind, dim.cast<int64_t>(), keepdim));
}

PyTensor narrow_impl(const PyTensor& self, int64_t dim, int64_t lo, int64_t hi, int64_t by) {
  if (by == 1 && self.v.requires_grad()) return PyTensor(aops::narrow(self.v, dim, lo, hi, by));
  return leaf(t_narrow(self.value(), dim, lo, hi, by));
}

PyTensor select_impl(const PyTensor& self, int64_t dim, int64_t index) {
  const Tensor& t = self.value();
  if (self.v.requires_grad()) {
    const int d = normalize_dim(dim, t.ndim());
    const int64_t idx = index < 0 ? t.shape[d] + index : index;
    const Tensor probe = t_select(t, d, idx);  // validates the index
    Var w = aops::narrow(self.v, d, idx, idx + 1, 1);
    return PyTensor(aops::reshape(w, probe.shape));
  }
  return leaf(t_select(t, dim, index));
}

// Integer ids as PyO3 extracts a Vec<i64>: any sequence of integers (items
// with __index__; floats and str are refused with TypeError, values outside
// int64 with OverflowError). A 1-d numpy integer array is read through its
// buffer instead of item by item: that is the embedding's hot input.
std::vector<int64_t> int_ids(const py::handle& obj) {
  if (py::isinstance<py::array>(obj)) {
    const py::array a = py::reinterpret_borrow<py::array>(obj);
    const char kind = a.dtype().kind();
    if (a.ndim() == 1 && (kind == 'i' || kind == 'u')) {
      const auto c = py::array_t<int64_t, py::array::c_style | py::array::forcecast>::ensure(a);
      if (!c) throw py::error_already_set();
      if (kind == 'u' && a.dtype().itemsize() == 8) {
        // uint64 values above INT64_MAX do not fit, as for a Python int
        const auto u = py::array_t<uint64_t, py::array::c_style | py::array::forcecast>::ensure(a);
        for (py::ssize_t i = 0; i < u.size(); ++i)
          if (u.data()[i] > (uint64_t)INT64_MAX) {
            PyErr_SetString(PyExc_OverflowError, "Python int too large to convert to C long long");
            throw py::error_already_set();
          }
      }
      return std::vector<int64_t>(c.data(), c.data() + c.size());
    }
  }
  if (PyUnicode_Check(obj.ptr())) throw py::type_error("Can't extract `str` to `Vec`");
  PyObject* seq = PySequence_Fast(obj.ptr(), "expected a sequence of integers");
  if (!seq) throw py::error_already_set();
  const Py_ssize_t n = PySequence_Fast_GET_SIZE(seq);
  PyObject** items = PySequence_Fast_ITEMS(seq);
  std::vector<int64_t> out((size_t)n);
  for (Py_ssize_t i = 0; i < n; ++i) {
    PyObject* it = items[i];
    long long v;
    if (PyLong_CheckExact(it)) {
      v = PyLong_AsLongLong(it);
    } else {
      PyObject* ix = PyNumber_Index(it);
      if (!ix) {
        Py_DECREF(seq);
        throw py::error_already_set();
      }
      v = PyLong_AsLongLong(ix);
      Py_DECREF(ix);
    }
    if (v == -1 && PyErr_Occurred()) {
      Py_DECREF(seq);
      throw py::error_already_set();
    }
    out[(size_t)i] = (int64_t)v;
  }
  Py_DECREF(seq);
  return out;
}

PyTensor index_select_impl(const PyTensor& self, int64_t dim, const std::vector<int64_t>& idx) {
  if (self.v.requires_grad()) return PyTensor(aops::index_select(self.v, dim, idx));
  return leaf(t_index_select(self.value(), dim, idx));
}

PyTensor apply_detached(const PyTensor& self, const std::string& name) {
  return leaf(t_unary_op(name, self.value()));
}

// PyTensor.apply (bindings lib.rs:682-710): differentiable for the listed ops,
// detached for the rest.
PyTensor apply(const PyTensor& self, const std::string& name) {
  if (self.v.requires_grad()) {
    if (name == "relu") return PyTensor(aops::relu(self.v));
    if (name == "sigmoid") return PyTensor(aops::sigmoid(self.v));
    if (name == "tanh") return PyTensor(aops::tanh(self.v));
    if (name == "exp") return PyTensor(aops::exp(self.v));
    if (name == "log") return PyTensor(aops::log(self.v));
    if (name == "sqrt") return PyTensor(aops::sqrt(self.v));
    if (name == "neg") return PyTensor(aops::neg(self.v));
    if (name == "abs") return PyTensor(aops::abs(self.v));
  }
  return apply_detached(self, name);
}

py::array_t<float> to_numpy(const PyTensor& self) {
  std::vector<float> v = t_to_host(self.value());
  std::vector<ssize_t> shape(self.value().shape.begin(), self.value().shape.end());
  py::array_t<float> a(shape);
  if (!v.empty()) std::memcpy(a.mutable_data(), v.data(), v.size() * sizeof(float));
  return a;
}

PyTensor& tensor_item(const py::handle& item) {
  if (!py::isinstance<PyTensor>(item)) throw py::type_error("optimizer parameters must be oxitorch.Tensor objects");
  return item.cast<PyTensor&>();
}

// step_all (bindings lib.rs:815-826): the optimizer advances each Var in
// list order and rebinds the caller's Tensor objects, which keep their
// identity; those before a failing parameter stay advanced. A Tensor listed
// twice is refused before any step, as the reference's exclusive borrow of
// each list element refuses it.
template <class F>
void step_all(const py::list& params, F&& step) {
  std::vector<Var*> vars;
  vars.reserve(params.size());
  for (const py::handle& item : params) {
    Var* v = &tensor_item(item).v;
    if (std::find(vars.begin(), vars.end(), v) != vars.end())
      throw std::runtime_error("Already borrowed: the same Tensor appears twice in the parameter list");
    vars.push_back(v);
  }
  step(vars);
}

void zero_grads(const py::list& params) {  // RustSgd::zero_grad (bindings lib.rs:864-872)
  for (const py::handle& item : params) tensor_item(item).v.zero_grad();
}

}  // namespace

PYBIND11_MODULE(_native, m) {
  m.doc() = "oxitorch_amd native host core: device tensors, autograd graph, fused hot-path ops";
  m.attr("__version__") = "0.1.0";

  py::register_exception_translator([](std::exception_ptr p) {
    try {
      if (p) std::rethrow_exception(p);
    } catch (const Error& e) {
      switch (e.kind()) {
        case ErrKind::InvalidArgument:
        case ErrKind::ShapeMismatch:
          PyErr_SetString(PyExc_ValueError, e.what());
          break;
        case ErrKind::NotImplemented:
          PyErr_SetString(PyExc_NotImplementedError, e.what());
          break;
        default:
          PyErr_SetString(PyExc_RuntimeError, e.what());
      }
    }
  });

  py::class_<PyTensor>(m, "Tensor")
      .def(py::init([](const py::object& buffer, bool requires_grad, const py::object& device) {
             const Dev d = parse_device(device);
             if (is_f32_buffer(buffer)) return leaf(from_buffer(buffer, d), requires_grad);
             std::vector<float> data;
             try {
               data = buffer.cast<std::vector<float>>();
             } catch (const py::cast_error&) {
               throw py::type_error("expected a numpy array, f32 buffer, or sequence of numbers");
             }
             return leaf(t_from_host(data.data(), {(int64_t)data.size()}, d), requires_grad);
           }),
           py::arg("buffer"), py::arg("requires_grad") = false, py::arg("device") = py::none())
      .def("__repr__", [](const PyTensor& s) { return display(s.value()); })
      .def("__str__", [](const PyTensor& s) { return display(s.value()); })
      .def("__len__",
           [](const PyTensor& s) -> int64_t {
             if (s.value().ndim() == 0) throw py::type_error("len() of a 0-d tensor");
             return s.value().shape[0];
           })
      .def("__getitem__",
           [](const PyTensor& s, const py::object& key) -> PyTensor {
             if (py::isinstance<py::int_>(key)) return select_impl(s, 0, key.cast<int64_t>());
             if (py::isinstance<py::slice>(key)) {
               py::slice sl = key.cast<py::slice>();
               const py::object st = sl.attr("start"), sp = sl.attr("stop"), by = sl.attr("step");
               const int64_t lo = st.is_none() ? 0 : st.cast<int64_t>();
               const int64_t hi = sp.is_none() ? INT64_MAX : sp.cast<int64_t>();
               const int64_t step = by.is_none() ? 1 : by.cast<int64_t>();
               return narrow_impl(s, 0, lo, hi, step);
             }
             try {
               return index_select_impl(s, 0, key.cast<std::vector<int64_t>>());
             } catch (const py::cast_error&) {
               throw py::type_error("tensor indices must be integers, slices, or integer lists");
             }
           })
      .def("__add__", [](const PyTensor& s, const py::object& o) { return PyTensor(aops::add(s.v, operand(s, o))); })
      .def("__radd__", [](const PyTensor& s, const py::object& o) { return PyTensor(aops::add(s.v, operand(s, o))); })
      .def("__sub__", [](const PyTensor& s, const py::object& o) { return PyTensor(aops::sub(s.v, operand(s, o))); })
      .def("__rsub__",
           [](const PyTensor& s, const py::object& o) {
             if (py::isinstance<PyTensor>(o)) return PyTensor(aops::sub(o.cast<PyTensor&>().v, s.v));
             return PyTensor(aops::add(aops::neg(s.v), operand(s, o)));  // c - t = (-t) + c
           })
      .def("__mul__", [](const PyTensor& s, const py::object& o) { return PyTensor(aops::mul(s.v, operand(s, o))); })
      .def("__rmul__", [](const PyTensor& s, const py::object& o) { return PyTensor(aops::mul(s.v, operand(s, o))); })
      .def("__truediv__",
           [](const PyTensor& s, const py::object& o) { return PyTensor(aops::div(s.v, operand(s, o))); })
      .def("__rtruediv__",
           [](const PyTensor& s, const py::object& o) {
             if (py::isinstance<PyTensor>(o)) return PyTensor(aops::div(o.cast<PyTensor&>().v, s.v));
             // c / t = c * t^(-1)
             Var inv = aops::pow(s.v, Var::leaf(t_scalar_full(s.value().shape, -1.0f, s.value().dev()), false));
             return PyTensor(aops::mul(inv, operand(s, o)));
           })
      .def("__pow__",
           [](const PyTensor& s, const py::object& o, const py::object&) {
             if (py::isinstance<PyTensor>(o)) return PyTensor(aops::pow(s.v, o.cast<PyTensor&>().v));
             if (s.v.requires_grad()) return PyTensor(aops::pow(s.v, operand(s, o)));
             return leaf(t_binary(OXI_BINARY_POW, s.value(), operand(s, o).value()));
           },
           py::arg("other"), py::arg("modulo") = py::none())
      .def("__neg__", [](const PyTensor& s) { return PyTensor(aops::neg(s.v)); })
      .def("__abs__",
           [](const PyTensor& s) {
             if (s.v.requires_grad()) return PyTensor(aops::abs(s.v));
             return leaf(t_unary_op("abs", s.value()));
           })
      .def("__eq__", [](const PyTensor& s, const PyTensor& o) { return leaf(t_cmp_op("eq", s.value(), o.value())); })
      .def("__ne__", [](const PyTensor& s, const PyTensor& o) { return leaf(t_cmp_op("ne", s.value(), o.value())); })
      .def("__lt__", [](const PyTensor& s, const PyTensor& o) { return leaf(t_cmp_op("lt", s.value(), o.value())); })
      .def("__le__", [](const PyTensor& s, const PyTensor& o) { return leaf(t_cmp_op("le", s.value(), o.value())); })
      .def("__gt__", [](const PyTensor& s, const PyTensor& o) { return leaf(t_cmp_op("gt", s.value(), o.value())); })
      .def("__ge__", [](const PyTensor& s, const PyTensor& o) { return leaf(t_cmp_op("ge", s.value(), o.value())); })
      .def("__matmul__",
           [](const PyTensor&, const PyTensor&) -> PyTensor {
             err_notimpl("matmul (SGEMM) is outside this build's device hot path");
           })
      .def("__float__",
           [](const PyTensor& s) -> double {
             std::vector<float> v = t_to_host(s.value());
             if (v.size() != 1) {
               throw py::type_error("only one-element tensors can be converted to float, got " +
                                    std::to_string(v.size()) + " elements");
             }
             return (double)v[0];
           })
      // ---- autograd
      .def_property_readonly("requires_grad", [](const PyTensor& s) { return s.v.requires_grad(); })
      .def_property(
          "grad",
          [](const PyTensor& s) -> py::object {
            auto g = s.v.grad();
            if (!g) return py::none();
            return py::cast(leaf(*g));
          },
          // `t.grad = None` clears the gradient (the reference's setter takes a
          // Tensor only, crates/oxi-bindings/src/lib.rs:354-358)
          [](const PyTensor& s, const py::object& g) {
            if (g.is_none()) s.v.clear_grad();
            else s.v.set_grad(g.cast<PyTensor&>().value());
          })
      .def("detach", [](const PyTensor& s) { return leaf(s.value()); })
      .def(
          "backward",
          [](const PyTensor& s, const py::object& grad, bool retain_graph) {
            std::optional<Tensor> seed;
            if (!grad.is_none()) seed = grad.cast<PyTensor&>().value();
            backward(s.v, seed, retain_graph);
          },
          py::arg("grad") = py::none(), py::kw_only(), py::arg("retain_graph") = false)
      .def("zero_grad", [](const PyTensor& s) { s.v.zero_grad(); })
      .def("numpy", &to_numpy)
      // ---- metadata
      .def_property_readonly("shape",
                             [](const PyTensor& s) { return std::vector<int64_t>(s.value().shape); })
      .def_property_readonly("dtype", [](const PyTensor&) { return std::string("float32"); })
      .def_property_readonly("device", [](const PyTensor& s) { return dev_name(s.value().dev()); })
      .def_property_readonly("ndim", [](const PyTensor& s) { return s.value().ndim(); })
      .def_property_readonly("strides", [](const PyTensor& s) { return std::vector<int64_t>(s.value().strides); })
      .def("numel", [](const PyTensor& s) { return s.value().numel(); })
      .def("is_contiguous", [](const PyTensor& s) { return s.value().is_contiguous(); })
      // ---- device movement
      .def(
          "to",
          [](const PyTensor& s, const py::object& device) {
            const Dev d = parse_device(device);
            if (d == s.value().dev()) return s;
            return leaf(t_to(s.value(), d), s.v.requires_grad() && !s.v.op_name());
          },
          py::arg("device"))
      .def("cpu", [](const PyTensor& s) { return leaf(t_to(s.value(), Dev::Cpu)); })
      .def("hip", [](const PyTensor& s) { return leaf(t_to(s.value(), Dev::Hip)); })
      // ---- elementwise & reductions
      .def("add", [](const PyTensor& s, const PyTensor& o) { return PyTensor(aops::add(s.v, o.v)); })
      .def("sub", [](const PyTensor& s, const PyTensor& o) { return PyTensor(aops::sub(s.v, o.v)); })
      .def("mul", [](const PyTensor& s, const PyTensor& o) { return PyTensor(aops::mul(s.v, o.v)); })
      .def("div", [](const PyTensor& s, const PyTensor& o) { return PyTensor(aops::div(s.v, o.v)); })
      .def("pow", [](const PyTensor& s, const PyTensor& o) { return PyTensor(aops::pow(s.v, o.v)); })
      .def("matmul",
           [](const PyTensor&, const PyTensor&) -> PyTensor {
             err_notimpl("matmul (SGEMM) is outside this build's device hot path");
           })
      .def("bmm",
           [](const PyTensor&, const PyTensor&) -> PyTensor {
             err_notimpl("bmm is outside this build's device hot path");
           })
      .def(
          "sum", [](const PyTensor& s, const py::object& dim, bool keepdim) { return dim_reduce(s, Reduce::Sum, dim, keepdim); },
          py::arg("dim") = py::none(), py::arg("keepdim") = false)
      .def(
          "mean", [](const PyTensor& s, const py::object& dim, bool keepdim) { return dim_reduce(s, Reduce::Mean, dim, keepdim); },
          py::arg("dim") = py::none(), py::arg("keepdim") = false)
      .def(
          "max", [](const PyTensor& s, const py::object& dim, bool keepdim) { return dim_reduce(s, Reduce::Max, dim, keepdim); },
          py::arg("dim") = py::none(), py::arg("keepdim") = false)
      .def(
          "min", [](const PyTensor& s, const py::object& dim, bool keepdim) { return dim_reduce(s, Reduce::Min, dim, keepdim); },
          py::arg("dim") = py::none(), py::arg("keepdim") = false)
      .def(
          "argmax",
          [](const PyTensor& s, int64_t dim, bool keepdim) { return leaf(t_reduce(Reduce::ArgMax, s.value(), dim, keepdim)); },
          py::arg("dim"), py::arg("keepdim") = false)
      .def(
          "argmin",
          [](const PyTensor& s, int64_t dim, bool keepdim) { return leaf(t_reduce(Reduce::ArgMin, s.value(), dim, keepdim)); },
          py::arg("dim"), py::arg("keepdim") = false)
      .def(
          "norm", [](const PyTensor& s, int64_t dim, bool keepdim) { return PyTensor(aops::reduce(s.v, Reduce::Norm, dim, keepdim)); },
          py::arg("dim"), py::arg("keepdim") = false)
      // ---- views & indexing
      .def("reshape",
           [](const PyTensor& s, const std::vector<int64_t>& shape) {
             if (s.v.requires_grad()) return PyTensor(aops::reshape(s.v, shape));
             return leaf(t_reshape(s.value(), shape));
           })
      .def("view",
           [](const PyTensor& s, const std::vector<int64_t>& shape) {
             if (s.v.requires_grad()) return PyTensor(aops::reshape(s.v, shape));
             return leaf(t_reshape(s.value(), shape));
           })
      .def("transpose",
           [](const PyTensor& s) {
             if (s.v.requires_grad()) return PyTensor(aops::transpose(s.v));
             return leaf(t_transpose(s.value()));
           })
      .def("permute",
           [](const PyTensor& s, const std::vector<int64_t>& dims) {
             if (s.v.requires_grad()) return PyTensor(aops::permute(s.v, dims));
             return leaf(t_permute(s.value(), dims));
           })
      .def("narrow", &narrow_impl)
      .def("select", &select_impl)
      .def("index_select",
           [](const PyTensor& s, int64_t dim, const py::object& idx) { return index_select_impl(s, dim, int_ids(idx)); })
      .def("gather", [](const PyTensor& s, const py::object& idx) { return index_select_impl(s, 0, int_ids(idx)); })
      // bindings lib.rs:650-673: differentiable when either operand needs a gradient
      .def("scatter",
           [](const PyTensor& s, const py::object& ids, const PyTensor& values) {
             const std::vector<int64_t> idx = int_ids(ids);
             if (s.v.requires_grad() || values.v.requires_grad())
               return PyTensor(aops::scatter_dim0(s.v, idx, values.v));
             return leaf(t_scatter_dim0(s.value(), idx, values.value()));
           })
      .def("masked_select",
           [](const PyTensor& s, const PyTensor& mask) {
             if (s.v.requires_grad() || mask.v.requires_grad()) return PyTensor(aops::masked_select(s.v, mask.v));
             return leaf(t_masked_select(s.value(), mask.value()));
           })
      .def("contiguous", [](const PyTensor& s) { return leaf(t_contiguous(s.value())); })
      .def("apply", &apply)
      .def("broadcast_to",
           [](const PyTensor& s, const std::vector<int64_t>& shape) {
             if (s.v.requires_grad()) return PyTensor(aops::broadcast_to(s.v, shape));
             return leaf(t_broadcast_to(s.value(), shape));
           })
      .def("tolist", [](const PyTensor& s) { return t_to_host(s.value()); })
      .def("item", [](const PyTensor& s) -> float {
        if (s.value().numel() != 1)
          throw py::value_error("only one-element tensors can be converted to scalars (got " +
                                std::to_string(s.value().numel()) + ")");
        return t_to_host(s.value())[0];
      });

  // ---- free functions (bindings lib.rs:744-799)
  m.def(
      "zeros", [](const std::vector<int64_t>& shape, const py::object& device) { return leaf(t_zeros(validate_shape(shape), parse_device(device))); },
      py::arg("shape"), py::arg("device") = py::none());
  m.def(
      "full",
      [](const std::vector<int64_t>& shape, float value, bool requires_grad, const py::object& device) {
        return leaf(t_full(validate_shape(shape), value, parse_device(device)), requires_grad);
      },
      py::arg("shape"), py::arg("value"), py::arg("requires_grad") = false, py::arg("device") = py::none());
  m.def(
      "eye",
      [](int64_t n, const py::object& device) {
        std::vector<float> v((size_t)(n * n), 0.f);
        for (int64_t i = 0; i < n; ++i) v[(size_t)(i * n + i)] = 1.f;
        return leaf(t_from_host(v.data(), {n, n}, parse_device(device)));
      },
      py::arg("n"), py::arg("device") = py::none());
  m.def(
      "from_numpy",
      [](const py::object& array, bool requires_grad, const py::object& device) {
        if (!py::isinstance<py::buffer>(array)) throw py::type_error("expected a numpy array or f32 buffer object");
        return leaf(from_buffer(array, parse_device(device)), requires_grad);
      },
      py::arg("array"), py::arg("requires_grad") = false, py::arg("device") = py::none());
  m.def("current_device", []() { return hip_device_index(); },
        "Index of the HIP device the library is bound to (or will bind at its first device use).");
  m.def("device_count", []() {
    int n = 0;
    hip_check(oxi_hip_device_count(&n));
    return n;
  });
  m.def("is_grad_enabled", &is_grad_enabled);
  m.def("set_grad_enabled", &set_grad_enabled);
  m.def("fuse_norm_act", &fuse_norm_act,
        "Whether backward runs a norm VJP and the VJP of an activation on its output as one pass.");
  m.def("set_fuse_norm_act", &set_fuse_norm_act, "Turn the fused norm + activation VJP on or off; returns the old value.");
  m.def("fused_norm_act_passes", &fused_norm_act_passes, "Fused norm + activation VJP passes run in this process.");
  m.def("ce_one_pass", &ce_one_pass,
        "Whether cross_entropy's forward also writes the gradient for backward()'s implicit seed.");
  m.def("set_ce_one_pass", &set_ce_one_pass,
        "Turn cross_entropy's one-pass forward + seed-1 gradient on or off; returns the old value.");
  m.def("version", []() { return std::string("0.1.0"); });
  m.def("synchronize", []() { hip_check(oxi_hip_sync()); });
  m.def("memory_stats", []() {
    size_t a = 0, b = 0;
    hip_check(oxi_hip_memory_stats(&a, &b));
    return py::make_tuple(a, b);
  });
  m.def("set_default_device", [](const py::object& d) { set_default_device(parse_device(d)); });
  m.def("get_default_device", []() { return dev_name(default_device()); });

  // ---- fused hot-path ops, called by oxitorch_amd.nn.functional
  m.def(
      "rms_norm",
      [](const PyTensor& x, const PyTensor& w, float eps, const py::object& mode) {
        aops::NormVjp md = mode.is_none() ? aops::norm_vjp_mode()
                                          : (mode.cast<std::string>() == "exact" ? aops::NormVjp::Exact : aops::NormVjp::Ref);
        return PyTensor(aops::rms_norm(x.v, w.v, eps, md));
      },
      py::arg("x"), py::arg("weight"), py::arg("eps") = 1e-6f, py::arg("vjp") = py::none());
  m.def(
      "layer_norm",
      [](const PyTensor& x, const py::object& w, const py::object& b, float eps, const py::object& mode) {
        aops::NormVjp md = mode.is_none() ? aops::norm_vjp_mode()
                                          : (mode.cast<std::string>() == "exact" ? aops::NormVjp::Exact : aops::NormVjp::Ref);
        std::optional<Var> wv, bv;
        if (!w.is_none()) wv = w.cast<PyTensor&>().v;
        if (!b.is_none()) bv = b.cast<PyTensor&>().v;
        return PyTensor(aops::layer_norm(x.v, wv, bv, eps, md));
      },
      py::arg("x"), py::arg("weight"), py::arg("bias"), py::arg("eps") = 1e-5f, py::arg("vjp") = py::none());
  m.def(
      "gelu",
      [](const PyTensor& x, const std::string& approximate) {
        int a;
        if (approximate == "tanh") a = OXI_GELU_TANH;
        else if (approximate == "none" || approximate == "erf") a = OXI_GELU_ERF;
        else err_invalid("gelu approximate must be \"tanh\" or \"none\", got \"" + approximate + "\"");
        return PyTensor(aops::gelu(x.v, a));
      },
      py::arg("x"), py::arg("approximate") = "tanh");
  m.def("silu", [](const PyTensor& x) { return PyTensor(aops::silu(x.v)); });
  m.def(
      "softmax", [](const PyTensor& x, int64_t dim) { return PyTensor(aops::softmax(x.v, dim, false)); },
      py::arg("x"), py::arg("dim") = -1);
  m.def(
      "log_softmax", [](const PyTensor& x, int64_t dim) { return PyTensor(aops::softmax(x.v, dim, true)); },
      py::arg("x"), py::arg("dim") = -1);
  m.def("cross_entropy", [](const PyTensor& logits, const py::object& targets) {
    return PyTensor(aops::cross_entropy(logits.v, int_ids(targets)));
  });
  m.def("embedding", [](const py::object& indices, const PyTensor& w) {
    return PyTensor(aops::embedding(int_ids(indices), w.v));
  });

  // Elementwise clamp on the device (binary max then min against scalar
  // constants), for gradient-value clipping; detached.
  m.def("clamp", [](const PyTensor& x, float lo, float hi) {
    const Tensor& t = x.value();
    Tensor a = t_binary_op("max", t, t_scalar_full(t.shape, lo, t.dev()));
    return leaf(t_binary_op("min", a, t_scalar_full(t.shape, hi, t.dev())));
  });

  // ---- tensor-column loader (bindings data.rs:115-365): columns live in HBM,
  // batches are device gathers in the epoch's (optionally shuffled) order
  py::class_<LoaderIter>(m, "LoaderIter")
      .def("__iter__", [](py::object self) { return self; })
      .def("__next__", [](LoaderIter& it) {
        std::vector<Tensor> cols;
        if (!it.next(&cols)) throw py::stop_iteration();
        py::list out;
        for (Tensor& t : cols) out.append(py::cast(leaf(std::move(t))));
        return out;
      });
  py::class_<Loader>(m, "DataLoader")
      .def(py::init([](const py::list& columns, int64_t batch_size, bool shuffle, bool drop_last,
                       std::optional<uint64_t> seed, int64_t num_workers, const py::object& transforms,
                       uint64_t transform_seed) {
             if (!transforms.is_none())
               err_notimpl("native batch transforms (crop/flip/normalize) are outside this build's device path");
             (void)transform_seed;
             std::vector<Tensor> cols;
             for (const py::handle& c : columns) {
               if (!py::isinstance<PyTensor>(c)) throw py::type_error("DataLoader columns must be oxitorch.Tensor");
               cols.push_back(c.cast<PyTensor&>().value());
             }
             if (batch_size < 0 || num_workers < 0) throw py::value_error("batch_size and num_workers must be >= 0");
             return Loader(cols, batch_size, shuffle, drop_last, seed, num_workers);
           }),
           py::arg("columns"), py::arg("batch_size") = 1, py::arg("shuffle") = false, py::arg("drop_last") = false,
           py::arg("seed") = py::none(), py::arg("num_workers") = 0, py::arg("transforms") = py::none(),
           py::arg("transform_seed") = 0)
      .def_property_readonly("n", &Loader::n)
      .def_property_readonly("batch_size", &Loader::batch_size)
      .def("__iter__", &Loader::iter);
  // NumPy RandomState(seed).permutation(n), as the loader shuffles
  m.def("_mt19937_permutation", [](uint32_t seed, int64_t n) { return Mt19937(seed).permutation(n); });
  // epoch_plan (batch.rs:269-292) as (start, length) pairs
  m.def("_epoch_plan", &epoch_plan);

  // ---- optimizers (bindings lib.rs:807-936): state lives in the host core,
  // each step rebinds the given Tensor objects to their updated leaves.
  py::class_<Sgd>(m, "RustSgd")
      .def(py::init([](double lr, double momentum, bool nesterov) {
             if (nesterov && momentum <= 0.0) throw py::value_error("nesterov momentum requires momentum > 0");
             return Sgd((float)lr, (float)momentum, nesterov);
           }),
           py::arg("lr") = 0.01, py::arg("momentum") = 0.0, py::arg("nesterov") = false)
      .def_property(
          "lr", [](const Sgd& o) { return (double)o.lr(); }, [](Sgd& o, double lr) { o.set_lr((float)lr); })
      .def_static("zero_grad", &zero_grads)
      .def("step", [](Sgd& o, const py::list& params) { step_all(params, [&](std::vector<Var*>& v) { o.step(v); }); });
  py::class_<AdamW>(m, "RustAdamW")
      .def(py::init([](double lr, std::pair<double, double> betas, double eps, double weight_decay, bool decoupled) {
             return AdamW((float)lr, (float)betas.first, (float)betas.second, (float)eps, (float)weight_decay,
                          decoupled);
           }),
           py::arg("lr") = 1e-3, py::arg("betas") = std::make_pair(0.9, 0.999), py::arg("eps") = 1e-8,
           py::arg("weight_decay") = 1e-2, py::arg("decoupled") = true)
      .def_property(
          "lr", [](const AdamW& o) { return (double)o.lr(); }, [](AdamW& o, double lr) { o.set_lr((float)lr); })
      .def_static("zero_grad", &zero_grads)
      .def("step",
           [](AdamW& o, const py::list& params) { step_all(params, [&](std::vector<Var*>& v) { o.step(v); }); });
}

// Tensor storage, layout algebra, views and device dispatch.
// Restates crates/oxi-tensor/src/{layout.rs, lib.rs} with a Host|Device
// storage variant; compute goes through the liboxihip C-ABI.
#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <numeric>
#include <sstream>

#include "host.h"

namespace oxt {

// ---- errors -------------------------------------------------------------------

void err_invalid(const std::string& m) { throw Error(ErrKind::InvalidArgument, "invalid argument: " + m); }
void err_shape(const std::string& l, const std::string& r) {
  throw Error(ErrKind::ShapeMismatch, "shape mismatch: " + l + " vs " + r);
}
void err_notimpl(const std::string& m) { throw Error(ErrKind::NotImplemented, "not implemented: " + m); }
void err_oob(const std::string& m) { throw Error(ErrKind::OutOfBounds, "out of bounds: " + m); }
void err_other(const std::string& m) { throw Error(ErrKind::Other, m); }
void err_invalid_plain(const std::string& m) { throw Error(ErrKind::InvalidArgument, m); }

void hip_check(int rc) {
  if (rc == OXI_OK) return;
  const char* m = oxi_hip_last_error();
  const std::string msg = m ? m : "";
  switch (rc) {
    case OXI_INVALID_ARGUMENT: throw Error(ErrKind::InvalidArgument, "invalid argument: " + msg);
    case OXI_SHAPE_MISMATCH: throw Error(ErrKind::ShapeMismatch, msg);
    case OXI_NOT_IMPLEMENTED: throw Error(ErrKind::NotImplemented, "not implemented: " + msg);
    case OXI_OUT_OF_BOUNDS: throw Error(ErrKind::OutOfBounds, "out of bounds: " + msg);
    default: throw Error(ErrKind::Other, msg);
  }
}

// ---- layout (layout.rs) ------------------------------------------------------

std::string fmt_shape(const Shape& s) {
  std::ostringstream o;
  o << "[";
  for (size_t i = 0; i < s.size(); ++i) o << (i ? ", " : "") << s[i];
  o << "]";
  return o.str();
}

Shape row_major_strides(const Shape& s) {
  Shape st(s.size(), 0);
  int64_t acc = 1;
  for (int i = (int)s.size() - 1; i >= 0; --i) {
    st[i] = acc;
    acc *= s[i];
  }
  return st;
}

int64_t element_count(const Shape& s) {
  int64_t n = 1;
  for (auto d : s) n *= d;
  return n;
}

Shape validate_shape(const std::vector<int64_t>& dims) {
  for (auto d : dims)
    if (d < 0) err_invalid("dimensions must be non-negative, got " + fmt_shape(dims));
  __int128 n = 1;
  for (auto d : dims) {
    n *= d;
    if (n > ((__int128)1 << 62)) err_invalid("number of elements for shape " + fmt_shape(dims) + " overflows usize");
  }
  return dims;
}

Shape broadcast_shapes(const Shape& a, const Shape& b) {
  const size_t rank = std::max(a.size(), b.size());
  Shape out(rank);
  for (size_t i = 0; i < rank; ++i) {
    const int64_t ia = (int64_t)i - (int64_t)(rank - a.size());
    const int64_t ib = (int64_t)i - (int64_t)(rank - b.size());
    const int64_t da = ia >= 0 ? a[ia] : 1;
    const int64_t db = ib >= 0 ? b[ib] : 1;
    if (da != db && da != 1 && db != 1) err_shape(fmt_shape(a), fmt_shape(b));
    out[i] = std::max(da, db);
  }
  return out;
}

Shape broadcast_strides(const Shape& shape, const Shape& strides, const Shape& out) {
  broadcast_shapes(shape, out);
  if (shape.size() > out.size()) err_shape(fmt_shape(shape), fmt_shape(out));
  Shape r(out.size(), 0);
  const size_t off = out.size() - shape.size();
  for (size_t i = off; i < out.size(); ++i) {
    const size_t j = i - off;
    if (shape[j] != 1) {
      if (shape[j] != out[i]) err_shape(fmt_shape(shape), fmt_shape(out));
      r[i] = strides[j];
    }
  }
  return r;
}

int normalize_dim(int64_t dim, int ndim) {
  const int64_t d = dim < 0 ? ndim + dim : dim;
  if (d < 0 || d >= ndim)
    err_invalid("dim " + std::to_string(dim) + " out of range for " + std::to_string(ndim) + "-D tensor");
  return (int)d;
}

// ---- storage ----------------------------------------------------------------

namespace {
Dev g_default = Dev::Hip;
}
Dev default_device() { return g_default; }
void set_default_device(Dev d) { g_default = d; }
int hip_device_index() {
  int d = 0;
  hip_check(oxi_hip_default_device(&d));
  return d;
}

std::string dev_name(Dev d) {
  if (d == Dev::Cpu) return "cpu";
  int i = 0;
  return oxi_hip_default_device(&i) == OXI_OK ? "hip:" + std::to_string(i) : std::string("hip");
}

void bind_device(int index) {
  int n = 0;
  hip_check(oxi_hip_device_count(&n));
  if (n > 0 && index >= n)
    err_invalid("device index " + std::to_string(index) + " out of range for " + std::to_string(n) +
                " HIP device(s)");
  int cur = -1;
  hip_check(oxi_hip_current_device(&cur));
  if (cur >= 0 && cur != index)
    err_invalid("this process runs on hip:" + std::to_string(cur) + " (one device per process); hip:" +
                std::to_string(index) + " needs a process of its own, e.g. with OXI_HIP_DEVICE=" +
                std::to_string(index));
  if (cur < 0) hip_check(oxi_hip_init(index));
}

Storage::Storage(Dev d, size_t bytes) : dev(d), nbytes(bytes) {
  if (bytes == 0) return;
  if (d == Dev::Cpu) {
    ptr = std::aligned_alloc(64, (bytes + 63) / 64 * 64);
    if (!ptr) err_other("host allocation of " + std::to_string(bytes) + " bytes failed");
  } else {
    hip_check(oxi_hip_alloc(bytes, &ptr));
  }
}

std::shared_ptr<Storage> Storage::adopt_device(void* ptr, size_t bytes) {
  auto s = std::make_shared<Storage>(Dev::Hip, 0);
  s->ptr = ptr;
  s->nbytes = ptr ? bytes : 0;
  return s;
}

Storage::~Storage() {
  if (!ptr) return;
  if (dev == Dev::Cpu) std::free(ptr);
  else (void)oxi_hip_free(ptr);
}

Tensor Tensor::empty(const Shape& shape, Dev d) {
  validate_shape(shape);
  Tensor t;
  t.st = std::make_shared<Storage>(d, sizeof(float) * (size_t)element_count(shape));
  t.shape = shape;
  t.strides = row_major_strides(shape);
  return t;
}

Tensor Tensor::with_strides(std::shared_ptr<Storage> st, int64_t offset, Shape shape, Shape strides) {
  Tensor t;
  t.st = std::move(st);
  t.offset = offset;
  t.shape = std::move(shape);
  t.strides = std::move(strides);
  return t;
}

void require_hip(const Tensor& t, const char* what) {
  if (t.dev() != Dev::Hip)
    err_notimpl(std::string(what) +
                " on a host (cpu) tensor: compute runs on the HIP device in this build; call .to(\"hip\") first");
}

// ---- constructors / transfers -----------------------------------------------

Tensor t_full(const Shape& shape, float v, Dev d) {
  Tensor t = Tensor::empty(shape, d);
  const int64_t n = t.numel();
  if (d == Dev::Cpu) {
    std::fill(t.data(), t.data() + n, v);
  } else {
    hip_check(oxi_fill(t.data(), n, v));
  }
  return t;
}

Tensor t_zeros(const Shape& shape, Dev d) { return t_full(shape, 0.0f, d); }
Tensor t_ones_like(const Tensor& t) { return t_full(t.shape, 1.0f, t.dev()); }

Tensor t_scalar_full(const Shape& shape, float v, Dev d) {
  validate_shape(shape);
  Tensor one = t_full({1}, v, d);
  return Tensor::with_strides(one.st, 0, shape, Shape(shape.size(), 0));
}

Tensor t_from_host(const float* data, const Shape& shape, Dev d) {
  Tensor t = Tensor::empty(shape, d);
  const size_t bytes = sizeof(float) * (size_t)t.numel();
  if (!bytes) return t;
  if (d == Dev::Cpu) std::memcpy(t.data(), data, bytes);
  else hip_check(oxi_hip_upload(t.data(), data, bytes));  // staged, no stream wait
  return t;
}

std::vector<float> t_to_host(const Tensor& t) {
  const int64_t n = t.numel();
  std::vector<float> out((size_t)n);
  if (n == 0) return out;
  if (t.dev() == Dev::Hip) {
    Tensor c = t_contiguous(t);
    // staged through the pinned ring: double-buffered chunks beat a plain
    // waiting copy from pageable memory
    hip_check(oxi_hip_download(out.data(), c.data(), sizeof(float) * (size_t)n));
    return out;
  }
  // host: walk the strides row-major (iterate::map_n general path)
  Shape idx(t.shape.size(), 0);
  const float* base = t.data();
  for (int64_t e = 0; e < n; ++e) {
    int64_t off = 0;
    for (size_t d = 0; d < idx.size(); ++d) off += idx[d] * t.strides[d];
    out[(size_t)e] = base[off];
    for (int d = (int)idx.size() - 1; d >= 0; --d) {
      if (++idx[d] < t.shape[d]) break;
      idx[d] = 0;
    }
  }
  return out;
}

Tensor t_to(const Tensor& t, Dev d) {
  if (t.dev() == d) return t;
  if (d == Dev::Cpu) {
    std::vector<float> v = t_to_host(t);
    return t_from_host(v.data(), t.shape, Dev::Cpu);
  }
  std::vector<float> v = t_to_host(t);
  return t_from_host(v.data(), t.shape, Dev::Hip);
}

// ---- views ----------------------------------------------------------------------

Tensor t_contiguous(const Tensor& t) {
  if (t.is_contiguous()) return t;
  if (t.dev() == Dev::Cpu) {
    std::vector<float> v = t_to_host(t);
    return t_from_host(v.data(), t.shape, Dev::Cpu);
  }
  return t_unary(OXI_UNARY_IDENTITY, t);
}

Tensor t_reshape(const Tensor& t, const std::vector<int64_t>& new_shape) {
  int infer = 0;
  for (auto d : new_shape) infer += d == -1;
  if (infer > 1) err_invalid("can only infer one dimension with -1");
  const int64_t numel = t.numel();
  Shape dims;
  int inferred_at = -1;
  int64_t known = 1;
  for (size_t i = 0; i < new_shape.size(); ++i) {
    const int64_t d = new_shape[i];
    if (d == -1) {
      inferred_at = (int)i;
      dims.push_back(1);
    } else if (d < 0) {
      err_invalid("invalid dimension " + std::to_string(d) + " in reshape");
    } else {
      dims.push_back(d);
      known *= d;
    }
  }
  if (inferred_at >= 0) {
    if (known == 0 || numel % known != 0)
      err_invalid("cannot reshape " + std::to_string(numel) + " elements into shape " + fmt_shape(new_shape));
    dims[inferred_at] = numel / known;
  }
  if (element_count(dims) != numel)
    err_invalid("cannot reshape " + std::to_string(numel) + " elements into shape " + fmt_shape(new_shape));
  const Tensor src = t.is_contiguous() ? t : t_contiguous(t);
  return Tensor::with_strides(src.st, src.offset, dims, row_major_strides(dims));
}

Tensor t_permute(const Tensor& t, const std::vector<int64_t>& order) {
  if ((int)order.size() != t.ndim())
    err_invalid("permute expects " + std::to_string(t.ndim()) + " dims, got " + std::to_string(order.size()));
  std::vector<bool> seen(t.ndim(), false);
  Shape sh, st;
  for (auto d : order) {
    const int dim = normalize_dim(d, t.ndim());
    if (seen[dim]) err_invalid("repeated dim " + std::to_string(d) + " in permute");
    seen[dim] = true;
    sh.push_back(t.shape[dim]);
    st.push_back(t.strides[dim]);
  }
  return Tensor::with_strides(t.st, t.offset, sh, st);
}

Tensor t_transpose(const Tensor& t) {
  if (t.ndim() != 2) err_invalid("transpose() expects a 2-D tensor; use permute for other ranks");
  return t_permute(t, {1, 0});
}

Tensor t_broadcast_to(const Tensor& t, const Shape& out_shape) {
  return Tensor::with_strides(t.st, t.offset, out_shape, broadcast_strides(t.shape, t.strides, out_shape));
}

Tensor t_narrow(const Tensor& t, int64_t dim, int64_t lo, int64_t hi, int64_t by) {
  const int d = normalize_dim(dim, t.ndim());
  const int64_t len = t.shape[d];
  if (by <= 0) err_notimpl("negative slice steps are not supported yet");
  auto resolve = [len](int64_t v) -> int64_t {
    if (v < 0) return std::max<int64_t>(0, len + v);
    return std::min(v, len);
  };
  const int64_t l = resolve(lo);
  const int64_t h = std::max(resolve(hi), l);
  const int64_t n = h <= l ? 0 : (h - l + by - 1) / by;
  Shape sh = t.shape, st = t.strides;
  sh[d] = n;
  st[d] *= by;
  return Tensor::with_strides(t.st, t.offset + l * t.strides[d], sh, st);
}

Tensor t_select(const Tensor& t, int64_t dim, int64_t index) {
  const int d = normalize_dim(dim, t.ndim());
  const int64_t len = t.shape[d];
  const int64_t i = index < 0 ? len + index : index;
  if (i < 0 || i >= len)
    err_oob("index " + std::to_string(i) + " out of range for dim " + std::to_string(d) + " of size " +
            std::to_string(len));
  Shape sh = t.shape, st = t.strides;
  sh.erase(sh.begin() + d);
  st.erase(st.begin() + d);
  return Tensor::with_strides(t.st, t.offset + i * t.strides[d], sh, st);
}

// ---- registry lookups (crates/oxi-tensor/src/ops.rs:55-220) ----------------------

namespace {
const char* const UNARY_NAMES[] = {"neg", "abs", "sqrt", "rsqrt", "exp", "log", "log2", "log10", "sin", "cos",
                                   "tanh", "relu", "sigmoid", "floor", "ceil", "round", "sign", "square",
                                   "reciprocal"};
const char* const BINARY_NAMES[] = {"add", "sub", "mul", "div", "pow", "min", "max"};
const char* const CMP_NAMES[] = {"eq", "ne", "lt", "le", "gt", "ge"};

std::string quoted(const std::string& s) { return "\"" + s + "\""; }
}  // namespace

int unary_id(const std::string& name) {
  for (int i = 0; i < (int)(sizeof UNARY_NAMES / sizeof *UNARY_NAMES); ++i)
    if (name == UNARY_NAMES[i]) return i;
  err_invalid("unknown unary op " + quoted(name));
}

int binary_id(const std::string& name) {
  for (int i = 0; i < (int)(sizeof BINARY_NAMES / sizeof *BINARY_NAMES); ++i)
    if (name == BINARY_NAMES[i]) return i;
  err_invalid("unknown binary op " + quoted(name));
}

int cmp_id(const std::string& name) {
  for (int i = 0; i < (int)(sizeof CMP_NAMES / sizeof *CMP_NAMES); ++i)
    if (name == CMP_NAMES[i]) return OXI_CMP_EQ + i;
  err_invalid("unknown comparison op " + quoted(name));
}

// ---- elementwise dispatch ----------------------------------------------------------

namespace {
// Dense layout test: strides form a permutation of a row-major layout.
bool dense_layout(const Shape& shape, const Shape& strides) {
  std::vector<int> order(shape.size());
  std::iota(order.begin(), order.end(), 0);
  std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return strides[a] > strides[b]; });
  int64_t expect = 1;
  for (int i = (int)order.size() - 1; i >= 0; --i) {
    const int d = order[i];
    if (shape[d] == 1) continue;
    if (strides[d] != expect) return false;
    expect *= shape[d];
  }
  return true;
}
}  // namespace

Shape result_strides(const Shape& shape, const std::vector<const Tensor*>& ins) {
  if (ins.empty()) return row_major_strides(shape);
  const Shape& s0 = ins[0]->strides;
  if (ins[0]->shape != shape || !dense_layout(shape, s0)) return row_major_strides(shape);
  for (const Tensor* t : ins)
    if (t->shape != shape || t->strides != s0) return row_major_strides(shape);
  return s0;
}

namespace {
Tensor alloc_like(const Shape& shape, const Shape& strides, Dev d) {
  // a dense layout covers exactly numel elements starting at offset 0
  Tensor t = Tensor::empty(shape, d);
  t.strides = strides;
  return t;
}
}  // namespace

Tensor t_unary(int op, const Tensor& a, bool preserve) {
  require_hip(a, "unary op");
  const Shape st = preserve ? result_strides(a.shape, {&a}) : row_major_strides(a.shape);
  Tensor y = alloc_like(a.shape, st, Dev::Hip);
  hip_check(oxi_unary(op, a.data(), a.strides.data(), y.data(), y.strides.data(), a.shape.data(), a.ndim()));
  return y;
}

Tensor t_binary(int op, const Tensor& a, const Tensor& b, bool preserve) {
  const Shape out = broadcast_shapes(a.shape, b.shape);
  require_hip(a, "binary op");
  require_hip(b, "binary op");
  const Shape sa = broadcast_strides(a.shape, a.strides, out);
  const Shape sb = broadcast_strides(b.shape, b.strides, out);
  Shape st = row_major_strides(out);
  if (preserve) st = result_strides(out, {&a, &b});
  Tensor y = alloc_like(out, st, Dev::Hip);
  hip_check(oxi_binary(op, a.data(), sa.data(), b.data(), sb.data(), y.data(), y.strides.data(), out.data(),
                       (int)out.size()));
  return y;
}

Tensor t_unary_op(const std::string& name, const Tensor& a) { return t_unary(unary_id(name), a); }
Tensor t_binary_op(const std::string& name, const Tensor& a, const Tensor& b) {
  return t_binary(binary_id(name), a, b);
}
Tensor t_cmp_op(const std::string& name, const Tensor& a, const Tensor& b) { return t_binary(cmp_id(name), a, b); }
Tensor t_add(const Tensor& a, const Tensor& b) { return t_binary(OXI_BINARY_ADD, a, b); }
Tensor t_mul_scalar(const Tensor& a, float c) {
  return t_binary(OXI_BINARY_MUL, a, t_scalar_full(a.shape, c, a.dev()), true);
}

void t_copy_into(const Tensor& dst, const Tensor& src) {
  require_hip(dst, "copy");
  require_hip(src, "copy");
  if (dst.shape != src.shape) err_shape(fmt_shape(src.shape), fmt_shape(dst.shape));
  hip_check(oxi_unary(OXI_UNARY_IDENTITY, src.data(), src.strides.data(), dst.data(), dst.strides.data(),
                      src.shape.data(), src.ndim()));
}

// ---- reductions (lib.rs:519-604) -------------------------------------------------

Tensor t_reduce(Reduce kind, const Tensor& t, int64_t dim, bool keepdim) {
  if (t.ndim() == 0) err_invalid("dim " + std::to_string(dim) + " out of range for 0-D tensor");
  const int d = normalize_dim(dim, t.ndim());
  const int64_t len = t.shape[d];
  if (len == 0 && (kind == Reduce::ArgMax || kind == Reduce::ArgMin))
    err_invalid("cannot compute argmax/argmin over a zero-length dim");
  if (len == 0 && (kind == Reduce::Max || kind == Reduce::Min))
    err_invalid("cannot compute max/min over a zero-length dim");
  require_hip(t, "reduce");
  Shape out_shape = t.shape;
  if (keepdim) out_shape[d] = 1;
  else out_shape.erase(out_shape.begin() + d);
  Tensor y = Tensor::empty(out_shape, Dev::Hip);
  hip_check(oxi_reduce((int)kind, t.data(), t.strides.data(), t.shape.data(), t.ndim(), d, y.data()));
  return y;
}

Tensor t_reduce_all(Reduce kind, const Tensor& t) {
  // reduce_strip over the flat row-major values (bindings lib.rs:139-142)
  Tensor flat = t_reshape(t, {t.numel()});
  if (t.numel() == 0) {
    if (kind == Reduce::Sum || kind == Reduce::Mean || kind == Reduce::Norm) return t_zeros({}, t.dev());
    err_invalid("cannot compute min/max/argmax/argmin over an empty reduction");
  }
  return t_reshape(t_reduce(kind, flat, 0, false), {});
}

// ---- index_select (lib.rs:665-703) ---------------------------------------------------

std::vector<int64_t> resolve_indices(const std::vector<int64_t>& idx, int64_t len, int dim) {
  std::vector<int64_t> out(idx.size());
  for (size_t k = 0; k < idx.size(); ++k) {
    const int64_t i = idx[k];
    const int64_t r = i < 0 ? len + i : i;
    if (r < 0 || r >= len)
      err_oob("index " + std::to_string(i) + " out of range for dim " + std::to_string(dim) + " of size " +
              std::to_string(len));
    out[k] = r;
  }
  return out;
}

std::shared_ptr<Storage> device_i64(const std::vector<int64_t>& v) {
  auto s = std::make_shared<Storage>(Dev::Hip, sizeof(int64_t) * v.size());
  if (!v.empty()) hip_check(oxi_hip_upload(s->ptr, v.data(), sizeof(int64_t) * v.size()));
  return s;
}

Tensor t_index_select_dev(const Tensor& t, int d, const std::shared_ptr<Storage>& ids, int64_t n) {
  require_hip(t, "index_select");
  const Tensor src = t_contiguous(t);
  int64_t outer = 1, inner = 1;
  for (int i = 0; i < d; ++i) outer *= t.shape[i];
  for (int i = d + 1; i < t.ndim(); ++i) inner *= t.shape[i];
  Shape out_shape = t.shape;
  out_shape[d] = n;
  Tensor y = Tensor::empty(out_shape, Dev::Hip);
  if (y.numel() == 0) return y;
  hip_check(oxi_index_select(src.data(), outer, t.shape[d], inner, static_cast<const int64_t*>(ids->ptr), n,
                             y.data()));
  return y;
}

Tensor t_index_select(const Tensor& t, int64_t dim, const std::vector<int64_t>& indices) {
  if (t.ndim() == 0) err_invalid("dim " + std::to_string(dim) + " out of range for 0-D tensor");
  const int d = normalize_dim(dim, t.ndim());
  const std::vector<int64_t> idx = resolve_indices(indices, t.shape[d], d);
  require_hip(t, "index_select");
  return t_index_select_dev(t, d, device_i64(idx), (int64_t)idx.size());
}

Tensor t_scatter_dim0(const Tensor& base, const std::vector<int64_t>& indices, const Tensor& values) {
  if (base.ndim() == 0) err_invalid("scatter_dim0 requires at least a 1-D tensor");
  Shape expect = base.shape;
  expect[0] = (int64_t)indices.size();
  if (values.shape != expect) err_shape(fmt_shape(values.shape), fmt_shape(expect));
  const int64_t rows = base.shape[0];
  const std::vector<int64_t> idx = resolve_indices(indices, rows, 0);
  require_hip(base, "scatter");
  require_hip(values, "scatter");
  const Tensor b = t_contiguous(base);
  const Tensor v = t_contiguous(values);
  int64_t inner = 1;
  for (int d = 1; d < base.ndim(); ++d) inner *= base.shape[d];
  Tensor y = Tensor::empty(base.shape, Dev::Hip);
  if (y.numel() == 0) return y;
  auto ids = device_i64(idx);
  hip_check(oxi_scatter_rows(b.data(), rows, inner, static_cast<const int64_t*>(ids->ptr), (int64_t)idx.size(),
                             v.data(), y.data()));
  return y;
}

Tensor t_masked_select(const Tensor& x, const Tensor& mask, std::shared_ptr<Storage>* record) {
  const Shape grid = broadcast_shapes(x.shape, mask.shape);
  const Shape xs = broadcast_strides(x.shape, x.strides, grid);
  const Shape ms = broadcast_strides(mask.shape, mask.strides, grid);
  require_hip(x, "masked_select");
  require_hip(mask, "masked_select");
  void* rec = nullptr;
  if (record) {
    int64_t nb = 0;
    hip_check(oxi_masked_select_record_bytes(grid.data(), (int)grid.size(), &nb));
    *record = std::make_shared<Storage>(Dev::Hip, (size_t)nb);
    rec = (*record)->ptr;
  }
  float* picks = nullptr;
  int64_t count = 0;
  hip_check(oxi_masked_select(x.data(), xs.data(), mask.data(), ms.data(), grid.data(), (int)grid.size(), &picks,
                              &count, rec));
  Tensor y;
  y.st = Storage::adopt_device(picks, sizeof(float) * (size_t)count);
  y.shape = {count};
  y.strides = {1};
  return y;
}

}  // namespace oxt

// Host core of oxitorch_amd: the C++ restatement of the reference's Rust
// tensor engine (crates/oxi-tensor), autograd graph (crates/oxi-autograd) and
// error convention (crates/oxi-core), with a device storage variant whose
// compute is dispatched through the liboxihip C-ABI (include/oxihip.h).
//
// Storage is Host or Device (HIP) behind a refcounted handle; views share it.
// Every compute op runs on the device; host tensors only stage data
// (from/to numpy, .cpu()). There is no CPU compute fallback.
#pragma once

#include <cstdint>
#include <deque>
#include <functional>
#include <future>
#include <memory>
#include <mutex>
#include <optional>
#include <string>
#include <vector>

#include "oxihip.h"

namespace oxt {

// ---- errors (crates/oxi-core/src/lib.rs:186-211) ---------------------------

enum class ErrKind : int { InvalidArgument = 1, ShapeMismatch = 2, NotImplemented = 3, OutOfBounds = 4, Other = 5 };

class Error : public std::exception {
 public:
  Error(ErrKind k, std::string msg) : kind_(k), msg_(std::move(msg)) {}
  const char* what() const noexcept override { return msg_.c_str(); }
  ErrKind kind() const { return kind_; }

 private:
  ErrKind kind_;
  std::string msg_;
};

// Display formats of OxitorchError.
[[noreturn]] void err_invalid(const std::string& m);                      // "invalid argument: m"
[[noreturn]] void err_shape(const std::string& l, const std::string& r);  // "shape mismatch: l vs r"
[[noreturn]] void err_notimpl(const std::string& m);                      // "not implemented: m"
[[noreturn]] void err_oob(const std::string& m);                          // "out of bounds: m"
[[noreturn]] void err_other(const std::string& m);                        // "m"
[[noreturn]] void err_invalid_plain(const std::string& m);                // ValueError "m" (no prefix)
// Raises the Error matching an oxi_status, with liboxihip's message.
void hip_check(int rc);

// ---- shapes (crates/oxi-tensor/src/layout.rs) -----------------------------

using Shape = std::vector<int64_t>;
std::string fmt_shape(const Shape& s);  // Rust Debug of a Vec: "[2, 3]"
Shape row_major_strides(const Shape& s);
int64_t element_count(const Shape& s);
Shape validate_shape(const std::vector<int64_t>& dims);
Shape broadcast_shapes(const Shape& a, const Shape& b);
Shape broadcast_strides(const Shape& shape, const Shape& strides, const Shape& out);
int normalize_dim(int64_t dim, int ndim);

// ---- storage + tensor (crates/oxi-tensor/src/lib.rs:24-58) ------------------

enum class Dev { Cpu, Hip };
Dev default_device();
void set_default_device(Dev d);
std::string dev_name(Dev d);
// Binds the library to HIP device `index` at the first device use ("hip:N"):
// ValueError past the visible devices or when another device is bound.
void bind_device(int index);
// The bound HIP device, or the one the first device use will bind.
int hip_device_index();

struct Storage {
  Dev dev;
  void* ptr = nullptr;
  size_t nbytes = 0;
  Storage(Dev d, size_t bytes);
  ~Storage();
  Storage(const Storage&) = delete;
  Storage& operator=(const Storage&) = delete;
  // Takes ownership of a device block from oxi_hip_alloc (freed with oxi_hip_free).
  static std::shared_ptr<Storage> adopt_device(void* ptr, size_t bytes);
};

class Tensor {
 public:
  std::shared_ptr<Storage> st;
  int64_t offset = 0;  // in elements
  Shape shape;
  Shape strides;

  int64_t numel() const { return element_count(shape); }
  int ndim() const { return (int)shape.size(); }
  bool is_contiguous() const { return strides == row_major_strides(shape); }
  Dev dev() const { return st ? st->dev : default_device(); }
  float* data() const { return st ? static_cast<float*>(st->ptr) + offset : nullptr; }

  static Tensor empty(const Shape& shape, Dev d);
  static Tensor with_strides(std::shared_ptr<Storage> st, int64_t offset, Shape shape, Shape strides);
};

// Raises NotImplemented for a host tensor reaching device compute.
void require_hip(const Tensor& t, const char* what);

// ---- constructors and transfers -----------------------------------------------

Tensor t_full(const Shape& shape, float v, Dev d);         // dense fill (Tensor::full)
Tensor t_zeros(const Shape& shape, Dev d);
Tensor t_ones_like(const Tensor& t);
// A constant of `shape` backed by one element with zero strides: the value of
// the reference's full-tensor scalar promotion (bindings lib.rs:86-89) without
// an E-sized fill.
Tensor t_scalar_full(const Shape& shape, float v, Dev d);
Tensor t_from_host(const float* data, const Shape& shape, Dev d);
std::vector<float> t_to_host(const Tensor& t);  // row-major values
Tensor t_to(const Tensor& t, Dev d);

// ---- views (lib.rs:620-825) --------------------------------------------------

Tensor t_reshape(const Tensor& t, const std::vector<int64_t>& new_shape);
Tensor t_permute(const Tensor& t, const std::vector<int64_t>& order);
Tensor t_transpose(const Tensor& t);
Tensor t_broadcast_to(const Tensor& t, const Shape& out_shape);
Tensor t_narrow(const Tensor& t, int64_t dim, int64_t lo, int64_t hi, int64_t by);
Tensor t_select(const Tensor& t, int64_t dim, int64_t index);
Tensor t_contiguous(const Tensor& t);

// ---- device dispatch (lib.rs:263-357, 478-576, 665-703) ------------------------

int unary_id(const std::string& name);   // InvalidArgument for unknown names
int binary_id(const std::string& name);
int cmp_id(const std::string& name);
Tensor t_unary(int op, const Tensor& a, bool preserve_layout = false);
Tensor t_binary(int op, const Tensor& a, const Tensor& b, bool preserve_layout = false);
Tensor t_unary_op(const std::string& name, const Tensor& a);
Tensor t_binary_op(const std::string& name, const Tensor& a, const Tensor& b);
Tensor t_cmp_op(const std::string& name, const Tensor& a, const Tensor& b);
Tensor t_add(const Tensor& a, const Tensor& b);
Tensor t_mul_scalar(const Tensor& a, float c);

enum class Reduce : int { Sum = 0, Mean, Max, Min, ArgMax, ArgMin, Norm };
Tensor t_reduce(Reduce kind, const Tensor& t, int64_t dim, bool keepdim);
// Full reduction to a 0-d tensor (reduce_strip over all elements).
Tensor t_reduce_all(Reduce kind, const Tensor& t);
// Validates all indices first (negative wrap); OutOfBounds with the reference text.
std::vector<int64_t> resolve_indices(const std::vector<int64_t>& idx, int64_t len, int dim);
Tensor t_index_select(const Tensor& t, int64_t dim, const std::vector<int64_t>& indices);
// index_select along normalized dim `d` with ids already on the device (resolved, n of them).
Tensor t_index_select_dev(const Tensor& t, int d, const std::shared_ptr<Storage>& ids, int64_t n);
// Copies `src` into the (possibly strided) view `dst` of the same shape.
void t_copy_into(const Tensor& dst, const Tensor& src);
// Tensor::scatter_dim0 (lib.rs:895-932): rows indices[p] of `base` replaced by
// values[p], last write wins; the reference's argument checks and messages.
Tensor t_scatter_dim0(const Tensor& base, const std::vector<int64_t>& indices, const Tensor& values);
// Tensor::masked_select (lib.rs:939-961): 1-D picks over the broadcast grid.
// With `record`, also keeps the selection's record for the VJP.
Tensor t_masked_select(const Tensor& x, const Tensor& mask, std::shared_ptr<Storage>* record = nullptr);

// Strides for an elementwise result: the operands' common dense layout when
// they all share one (keeps a permuted gradient permuted), else row-major.
Shape result_strides(const Shape& shape, const std::vector<const Tensor*>& ins);
// A device int64 buffer holding `v` (kept alive by the returned storage).
std::shared_ptr<Storage> device_i64(const std::vector<int64_t>& v);

// ---- autograd graph (crates/oxi-autograd/src/graph.rs) ------------------------

bool is_grad_enabled();
bool set_grad_enabled(bool on);  // returns the previous mode

class Var;
// A VJP gets the upstream gradient and which inputs need a gradient; it
// returns one optional gradient per input (unset = not needed / none).
using Vjp = std::function<std::vector<std::optional<Tensor>>(const Tensor& g, const std::vector<bool>& needs)>;

// What a norm node keeps so that its VJP can absorb the VJP of an activation
// applied to its output (oxi_*_norm_act_bwd).
struct NormSaved {
  bool ln = false;
  Tensor x, w, b, mean, rstd;  // contiguous; w, b unused unless has_w / has_b
  bool has_w = false, has_b = false;
  int64_t rows = 0, H = 0;
  int mode = 0;         // OXI_NORM_VJP_*
  int wi = -1, bi = -1;  // input slots of w and b, -1 when absent
};

// The gradient of an intermediate that a fused backward pass did not write:
// formed on first read by the VJP(s) that would have formed it in the
// node-by-node order, so it holds the same values.
struct DeferredGrad {
  std::function<Tensor()> make;
  std::optional<Tensor> value;
  std::mutex mu;
  Tensor get() {
    std::lock_guard<std::mutex> lk(mu);
    if (!value) {
      value = make();
      make = nullptr;  // drops what the recipe held
    }
    return *value;
  }
};

struct Node {
  Tensor value;
  const char* op = nullptr;
  std::vector<Var> inputs;
  std::mutex mu;
  std::optional<Vjp> vjp;
  std::optional<Tensor> grad;
  std::shared_ptr<DeferredGrad> dgrad;  // when set (and grad is not), the gradient to form on read
  bool requires_grad = false;
  std::shared_ptr<const NormSaved> norm;  // set on layer_norm / rms_norm nodes
  int act = -1;                            // OXI_ACT_* on gelu / silu nodes
  std::vector<int64_t> perm;               // on permute / transpose nodes: the forward order
};

class Var {
 public:
  std::shared_ptr<Node> node;

  static Var leaf(Tensor value, bool requires_grad);
  static Var op(Tensor value, const char* name, std::vector<Var> inputs, Vjp vjp);
  const Tensor& value() const { return node->value; }
  bool requires_grad() const { return node->requires_grad; }
  const char* op_name() const { return node->op; }
  std::optional<Tensor> grad() const;
  void set_grad(const Tensor& g) const;
  void clear_grad() const;  // no gradient (as before the first backward)
  void zero_grad() const;
  void accumulate_grad(const Tensor& g) const;
};

Tensor unbroadcast(const Tensor& g, const Shape& shape);
void backward(const Var& root, std::optional<Tensor> seed, bool retain_graph);
// Whether `g` is (a view of) the seed backward() made itself, ones
// everywhere, in the backward pass now running on this thread.
bool is_implicit_seed(const Tensor& g);
// Whether backward runs norm + activation VJPs as one pass (OXI_FUSE_NORM_ACT,
// default on; the setter overrides the environment and returns the old value).
bool fuse_norm_act();
bool set_fuse_norm_act(bool on);
// Whether cross_entropy's forward also writes the gradient for backward()'s
// implicit seed when the logits require grad (OXI_CE_ONE_PASS, default on).
bool ce_one_pass();
bool set_ce_one_pass(bool on);
uint64_t fused_norm_act_passes();  // fused passes run so far in this process

// ---- differentiable ops (crates/oxi-autograd/src/ops.rs) ------------------------

namespace aops {
Var add(const Var& a, const Var& b);
Var sub(const Var& a, const Var& b);
Var mul(const Var& a, const Var& b);
Var div(const Var& a, const Var& b);
Var pow(const Var& a, const Var& b);
Var neg(const Var& x);
Var abs(const Var& x);
Var exp(const Var& x);
Var log(const Var& x);
Var sqrt(const Var& x);
Var tanh(const Var& x);
Var sigmoid(const Var& x);
Var relu(const Var& x);
Var reduce(const Var& x, Reduce kind, int64_t dim, bool keepdim);
Var reshape(const Var& x, const std::vector<int64_t>& shape);
Var permute(const Var& x, const std::vector<int64_t>& order);
Var transpose(const Var& x);
Var broadcast_to(const Var& x, const Shape& shape);
Var narrow(const Var& x, int64_t dim, int64_t lo, int64_t hi, int64_t by);
Var index_select(const Var& x, int64_t dim, const std::vector<int64_t>& indices);
Var scatter_dim0(const Var& base, const std::vector<int64_t>& indices, const Var& values);
Var masked_select(const Var& x, const Var& mask);

// Fused hot-path nodes: one graph node and one kernel per direction.
enum class NormVjp { Ref = OXI_NORM_VJP_REF, Exact = OXI_NORM_VJP_EXACT };
NormVjp norm_vjp_mode();  // OXI_NORM_VJP=ref|exact (default ref)
// The fused VJP of act(norm(x)) for upstream g (the activation output's
// gradient): fills dy (the norm output's gradient) and one gradient per norm
// input as `need` asks. False, with nothing computed, when the rows do not
// vectorize; the caller then runs the two VJPs.
// The norm's VJP as one pass with what backward folds into it: an activation
// on the norm output (act >= 0: g is the activation's upstream gradient and
// *dy receives the norm output's gradient; OXI_ACT_NONE: g is the norm
// output's gradient) and, with lsum, the sum of dx over a leading dim of
// `lead` rows (*lsum receives it, shape (rows / lead, H)). Returns false,
// having run nothing, when the kernels do not take this shape.
bool norm_vjp_fused(const NormSaved& s, int act, const Tensor& g, const std::vector<bool>& need, Tensor* dy,
                    std::vector<std::optional<Tensor>>& grads, int64_t lead = 0, Tensor* lsum = nullptr);
Var rms_norm(const Var& x, const Var& w, float eps, NormVjp mode);
Var layer_norm(const Var& x, const std::optional<Var>& w, const std::optional<Var>& b, float eps, NormVjp mode);
Var gelu(const Var& x, int approximate);
Var silu(const Var& x);
Var softmax(const Var& x, int64_t dim, bool log);
Var cross_entropy(const Var& logits, const std::vector<int64_t>& targets);
Var embedding(const std::vector<int64_t>& indices, const Var& weight);
}  // namespace aops

// ---- optimizers (crates/oxi-autograd/src/optim.rs) ------------------------------
// All state (velocities, moments, per-parameter step counters) lives here as
// device tensors, indexed by parameter position and allocated lazily on the
// first step that parameter has a gradient. Each step rebinds the parameter to
// a fresh requires_grad leaf holding the updated values (optim.rs:24-28).

class Sgd {
 public:
  Sgd(float lr, float momentum, bool nesterov) : lr_(lr), momentum_(momentum), nesterov_(nesterov) {}
  float lr() const { return lr_; }
  void set_lr(float lr) { lr_ = lr; }
  void step_param(size_t index, Var& param);
  void step(std::vector<Var*>& params);

 private:
  float lr_, momentum_;
  bool nesterov_;
  std::vector<std::optional<Tensor>> velocities_;
};

class AdamW {
 public:
  AdamW(float lr, float beta1, float beta2, float eps, float weight_decay, bool decoupled)
      : lr_(lr), beta1_(beta1), beta2_(beta2), eps_(eps), wd_(weight_decay), decoupled_(decoupled) {}
  float lr() const { return lr_; }
  void set_lr(float lr) { lr_ = lr; }
  void step_param(size_t index, Var& param);
  void step(std::vector<Var*>& params);

 private:
  float lr_, beta1_, beta2_, eps_, wd_;
  bool decoupled_;
  std::vector<std::optional<Tensor>> moments_, sq_moments_;
  std::vector<uint64_t> steps_;
};

// ---- tensor-column loader (crates/oxi-data, crates/oxi-bindings/src/data.rs) ------

// MT19937 with NumPy RandomState(seed) streams (crates/oxi-data/src/rng.rs).
class Mt19937 {
 public:
  explicit Mt19937(uint32_t seed);
  uint32_t next_u32();
  uint64_t below(uint64_t bound);                // uniform in [0, bound), NumPy's masked rejection
  std::vector<int64_t> permutation(int64_t n);   // RandomState.permutation(n)

 private:
  void twist();
  uint32_t mt_[624];
  int mti_;
};

// (start, length) of each batch of an epoch over n rows (batch.rs:269-292).
std::vector<std::pair<int64_t, int64_t>> epoch_plan(int64_t n, int64_t batch_size, bool drop_last);

struct LoaderIter {
  std::vector<Tensor> columns;
  std::shared_ptr<Storage> order;  // this epoch's row order, int64 on the device
  std::vector<std::pair<int64_t, int64_t>> batches;
  size_t pos = 0;
  bool next(std::vector<Tensor>* out);  // false once the epoch is done
};

class Loader {
 public:
  Loader(const std::vector<Tensor>& columns, int64_t batch_size, bool shuffle, bool drop_last,
         std::optional<uint64_t> seed, int64_t num_workers);
  int64_t n() const { return n_; }
  int64_t batch_size() const { return batch_size_; }
  LoaderIter iter();

 private:
  std::vector<int64_t> next_order();
  void prefetch_orders();
  std::vector<Tensor> columns_;  // contiguous, device-resident
  // the next shuffled epochs' orders, computed on host threads while the
  // current epoch runs (the permutation is the loader's only host work)
  std::deque<std::future<std::vector<int64_t>>> pending_;
  int64_t n_ = 0, batch_size_ = 1;
  bool shuffle_ = false, drop_last_ = false;
  std::optional<uint64_t> seed_;
  uint64_t epoch_ = 0;
  int64_t workers_ = 0;
};

}  // namespace oxt

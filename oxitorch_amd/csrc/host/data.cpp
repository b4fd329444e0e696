// The tensor-column loader of the host core (crates/oxi-data/src/{batch,rng}.rs,
// crates/oxi-bindings/src/data.rs): the dataset's columns live in HBM for the
// loader's lifetime, each epoch's row order is uploaded once, and a batch is
// one device gather of all columns at an offset into that order. No batch
// crosses PCIe; the only host work, the shuffled orders of the coming epochs,
// runs on host threads (num_workers of them, at least one) while the current
// epoch is consumed.
#include <algorithm>
#include <stdexcept>
#include <string>

#include "host.h"

namespace oxt {

// ---- MT19937 with NumPy RandomState streams (crates/oxi-data/src/rng.rs:8-121)

Mt19937::Mt19937(uint32_t seed) {
  mt_[0] = seed;
  for (uint32_t i = 1; i < 624; ++i) mt_[i] = 1812433253u * (mt_[i - 1] ^ (mt_[i - 1] >> 30)) + i;
  mti_ = 624;
}

namespace {
// One word of the twist: the top bit of `cur`, the low 31 of `nxt`, mixed
// into the word 397 places on (branch-free form of the twist matrix).
inline uint32_t twist_word(uint32_t cur, uint32_t nxt, uint32_t far) {
  const uint32_t y = (cur & 0x80000000u) | (nxt & 0x7fffffffu);
  return far ^ (y >> 1) ^ (0x9908b0dfu & (0u - (y & 1u)));
}
}  // namespace

// In place, in index order: words past 623-397 read already-twisted words,
// as the generator defines.
void Mt19937::twist() {
  int i = 0;
  for (; i < 624 - 397; ++i) mt_[i] = twist_word(mt_[i], mt_[i + 1], mt_[i + 397]);
  for (; i < 623; ++i) mt_[i] = twist_word(mt_[i], mt_[i + 1], mt_[i + 397 - 624]);
  mt_[623] = twist_word(mt_[623], mt_[0], mt_[396]);
  mti_ = 0;
}

uint32_t Mt19937::next_u32() {
  if (mti_ >= 624) twist();
  uint32_t y = mt_[mti_++];
  y ^= y >> 11;
  y ^= (y << 7) & 0x9d2c5680u;
  y ^= (y << 15) & 0xefc60000u;
  y ^= y >> 18;
  return y;
}

// NumPy's masked rejection for a uniform integer in [0, bound).
uint64_t Mt19937::below(uint64_t bound) {
  const uint32_t top = (uint32_t)(bound - 1);
  uint32_t mask = top;
  mask |= mask >> 1;
  mask |= mask >> 2;
  mask |= mask >> 4;
  mask |= mask >> 8;
  mask |= mask >> 16;
  for (;;) {
    const uint32_t v = next_u32() & mask;
    if (v <= top) return v;
  }
}

// RandomState.permutation(n): Fisher-Yates from the back.
std::vector<int64_t> Mt19937::permutation(int64_t n) {
  std::vector<int64_t> idx((size_t)n);
  for (int64_t i = 0; i < n; ++i) idx[(size_t)i] = i;
  for (int64_t i = n - 1; i >= 1; --i) std::swap(idx[(size_t)i], idx[(size_t)below((uint64_t)i + 1)]);
  return idx;
}

// ---- epoch plans (batch.rs:269-292) --------------------------------------------

std::vector<std::pair<int64_t, int64_t>> epoch_plan(int64_t n, int64_t batch_size, bool drop_last) {
  if (batch_size < 1) err_invalid("batch_size must be >= 1");
  std::vector<std::pair<int64_t, int64_t>> batches;
  for (int64_t start = 0; start < n; start += batch_size) {
    const int64_t len = std::min(batch_size, n - start);
    const bool last = start + len >= n;
    // a short last batch is dropped, unless it is the only batch
    if (last && drop_last && len < batch_size && !batches.empty()) break;
    batches.emplace_back(start, len);
  }
  return batches;
}

// ---- the loader (bindings data.rs:115-270) ----------------------------------------

Loader::Loader(const std::vector<Tensor>& columns, int64_t batch_size, bool shuffle, bool drop_last,
               std::optional<uint64_t> seed, int64_t num_workers)
    : batch_size_(batch_size), shuffle_(shuffle), drop_last_(drop_last), seed_(seed), workers_(num_workers) {
  if (columns.empty()) err_invalid_plain("DataLoader needs at least one tensor column");
  for (const Tensor& c : columns)
    if (c.ndim() == 0) err_invalid_plain("DataLoader columns need a row dimension (got a 0-d tensor)");
  n_ = columns[0].shape[0];
  if (n_ == 0) err_invalid_plain("DataLoader dataset is empty");
  if (batch_size < 1) err_invalid_plain("batch_size must be >= 1");
  for (size_t i = 0; i < columns.size(); ++i)
    if (columns[i].shape[0] != n_)
      err_invalid_plain("column " + std::to_string(i) + " has " + std::to_string(columns[i].shape[0]) +
                        " rows, expected " + std::to_string(n_));
  // the dataset goes to HBM once and stays there
  for (const Tensor& c : columns) columns_.push_back(t_contiguous(c.dev() == Dev::Hip ? c : t_to(c, Dev::Hip)));
}

// Keeps the orders of the next epochs in flight on host threads: each
// epoch's seed is fixed in advance, so they are independent. `num_workers`
// (the reference's host thread count) sets how many, at least one.
void Loader::prefetch_orders() {
  const size_t depth = (size_t)std::max<int64_t>(1, workers_);
  while (pending_.size() < depth) {
    // EpochSeeds::next (data.rs:40-48): base + epoch, truncated to 32 bits
    const uint32_t seed = (uint32_t)(*seed_ + epoch_++);
    const int64_t n = n_;
    pending_.push_back(std::async(std::launch::async, [seed, n]() { return Mt19937(seed).permutation(n); }));
  }
}

std::vector<int64_t> Loader::next_order() {
  if (shuffle_ && seed_) {
    prefetch_orders();
    std::vector<int64_t> order = pending_.front().get();
    pending_.pop_front();
    prefetch_orders();
    return order;
  }
  std::vector<int64_t> order((size_t)n_);
  for (int64_t i = 0; i < n_; ++i) order[(size_t)i] = i;
  return order;
}

LoaderIter Loader::iter() {
  LoaderIter it;
  it.columns = columns_;
  it.order = device_i64(next_order());
  it.batches = epoch_plan(n_, batch_size_, drop_last_);
  return it;
}

bool LoaderIter::next(std::vector<Tensor>* out) {
  if (pos >= batches.size()) return false;
  const auto [start, len] = batches[pos++];
  const int64_t* ids = static_cast<const int64_t*>(order->ptr) + start;
  out->clear();
  // every column of the batch in one launch (gather_columns, batch.rs:406-423)
  std::vector<oxi_batch_column> cols;
  cols.reserve(columns.size());
  for (const Tensor& c : columns) {
    Shape shape = c.shape;
    shape[0] = len;
    int64_t inner = 1;
    for (size_t d = 1; d < shape.size(); ++d) inner *= shape[d];
    Tensor b = Tensor::empty(shape, Dev::Hip);
    if (b.numel() > 0) cols.push_back({c.data(), b.data(), inner});
    out->push_back(std::move(b));
  }
  if (!cols.empty()) hip_check(oxi_batch_gather(cols.data(), (int)cols.size(), columns[0].shape[0], ids, len));
  return true;
}

}  // namespace oxt

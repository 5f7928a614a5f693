// hip::Runtime: host-side validation and dispatch of every runtime op onto
// the gfx950 kernel library (include/templit_hip.h).
//
// Each op follows the validation of its metal::Runtime counterpart in
// src/my_metal/runtime.cpp (cited per op) so that callers see the same
// exceptions for the same misuse, then enqueues the kernel(s) on the
// context stream. Where the Metal runtime composes several kernels
// (RMS: hadamard+sum+divide+add+sqrt, runtime.cpp:1031-1052; RMSNorm: RMS +
// divide, 1060-1072) this runtime calls one fused kernel with the same
// arithmetic. Metal-specific choices that are not semantics (threadgroup
// geometry, pipeline selection by alignment) have no counterpart here: the
// kernel library picks MFMA tile shapes and launch geometry for gfx950.
#include "my_hip/runtime.h"

#include "RTensor/infer_shape.h"
#include "templit_hip.h"

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <list>
#include <memory>
#include <numeric>
#include <optional>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include "templit/runnable.h"

namespace hip {

static_assert(templit::Runnable<Runtime::Tensor, Runtime>,
              "hip::Runtime must provide the passes::Runnable operation surface");

namespace {

using Tensor = Runtime::Tensor;
using IndexTensor = Runtime::IndexTensor;
using shape_type = rtensor::shape_type;

constexpr float kRmsEpsilon = 1e-6f; // added inside the sqrt, runtime.cpp:1044-1052

enum Op : uint32_t {
  kAdd = 1, kAddScalar, kSub, kHadamard, kDivide, kDivideScalar, kPow, kSigmoid, kSqrt, kExp,
  kGelu, kGeluDerivative, kCopy, kMult, kTranspose, kSplit, kMerge, kSum, kSumToShape,
  kMaxToShape, kArgmax, kSoftmax, kCrossEntropy, kCrossEntropyDerivative, kRms, kRmsNorm,
  kEmbedding, kScatterAdd, kScatterIndex, kSquaredNorm, kClip, kAdamW, kRmsNormGain,
  kSoftmaxDerivative, kGeluBackward, kRmsNormDerivative, kAttention, kAttentionBackward,
};

void check(int code, const char *what) { detail::check(code, what); }

// ---- views materialised on demand -------------------------------------------
// The reference executor transposes an operand into a fresh destination and
// hands it straight to one matrix product (MULT_LHS/RHS_DERIVATIVE,
// include/passes/execute.h:187-232), and copies a gradient's first
// contribution into its slot (context.h:73-89). Such a destination is kept
// as a view of its source -- the source tensor (held alive), the
// destination's shape and the source's element strides per destination dim
// -- and filled by one transpose or copy kernel only when its bytes are
// needed: when an op other than mult and the broadcast binary ops (which
// read strided operands) reads it, when the destination or the source is
// written, or on host access (the Storage hook). Either way the consuming
// kernels see the same values.
//
// A batched product whose batch entries chain into its inner dimension
// (MULT_RHS_DERIVATIVE's per-sequence weight gradient X_b^T . G_b, which
// the executor then sums over the batch with sum_to_shape) is kept pending
// the same way: sum_to_shape over exactly its batch dims runs one product
// with the batch folded into K, and anything else that needs the bytes runs
// the batched product.
struct ProductPlan {
  Tensor b;                                  // the second operand's data (held)
  uint32_t M, K, N, a_rs, a_cs, b_rs, b_cs;  // source = the first operand's data
  std::vector<uint32_t> batch, sa, sb, sc;   // merged batch dims
};
struct PendingView {
  Tensor source;
  shape_type shape, strides;
  std::shared_ptr<const ProductPlan> product; // set: a pending product, not a view
};

// Keyed by the destination's storage block. Never destroyed: views still
// pending at exit hold device memory the context may already have released.
std::unordered_map<const void *, PendingView> &pending_views() {
  static auto *views = new std::unordered_map<const void *, PendingView>();
  return *views;
}
using ViewIt = std::unordered_map<const void *, PendingView>::iterator;

// The blocks pending views read (their sources and deferred products' B
// operands), each with the destinations of those views: a write to a block
// fills the views that read it without a scan of every view. Views enter
// and leave through put_view and take_view only.
std::unordered_map<const void *, std::vector<const void *>> &view_readers() {
  static auto *readers = new std::unordered_map<const void *, std::vector<const void *>>();
  return *readers;
}
void index_view(const void *dst, const PendingView &v, bool add) {
  auto &readers = view_readers();
  const auto one = [&](const void *block) {
    if (add) {
      readers[block].push_back(dst);
      return;
    }
    const auto r = readers.find(block);
    if (r == readers.end()) return;
    auto &list = r->second;
    if (const auto i = std::find(list.begin(), list.end(), dst); i != list.end()) list.erase(i);
    if (list.empty()) readers.erase(r);
  };
  one(v.source.get_storage()->data());
  if (v.product) one(v.product->b.get_storage()->data());
}
void put_view(const void *dst, PendingView &&v) {
  auto &views = pending_views();
  index_view(dst, v, true);
  const auto it = views.find(dst);
  if (it == views.end()) {
    views.emplace(dst, std::move(v));
    return;
  }
  index_view(dst, it->second, false);
  PendingView dead = std::exchange(it->second, std::move(v)); // released after the update
}
PendingView take_view(ViewIt it) {
  index_view(it->first, it->second, false);
  PendingView v = std::move(it->second);
  pending_views().erase(it);
  return v;
}

// ---- value identities and the result cache ----------------------------------
// Every block carries the identity of the value it holds: a fresh number
// whenever a kernel or the host writes it, the source's number when it
// becomes a copy (a pending copy holds the same bytes), and a number derived
// from the transpose and its input's number for a transposed view.
// Filling a pending view changes nothing (the logical contents stay).
//
// The reference executor evaluates a gradient expression once per path to
// a leaf (the local gradients of include/passes/execute.h are recomputed
// for every use of a node), so its backward computes the same products
// from the same values several times. An op whose code, parameters, input
// values and shapes and output shape match a cached result whose block
// still holds that value makes its destination a pending copy of that block
// instead of running (`reuse`); results are cached (`remember`) up to a byte
// budget, least recently used first out. Equal identities mean equal bytes,
// so results are exactly those of running every op.
using ValueId = uint64_t;
ValueId g_next_value = 1;
ValueId fresh_value() { return g_next_value++; }

std::unordered_map<const void *, ValueId> &block_values() {
  static auto *values = new std::unordered_map<const void *, ValueId>();
  return *values;
}
ValueId value_of(const void *block) {
  auto [it, inserted] = block_values().try_emplace(block, 0);
  if (inserted) it->second = fresh_value();
  return it->second;
}
void set_value(const void *block, ValueId v) { block_values()[block] = v; }
void written(const void *block) { set_value(block, fresh_value()); }

struct MemoKey {
  std::vector<uint64_t> words;
  bool operator==(const MemoKey &o) const { return words == o.words; }
};
struct MemoKeyHash {
  size_t operator()(const MemoKey &k) const {
    uint64_t h = 0xcbf29ce484222325ull;
    for (uint64_t w : k.words) {
      h ^= w;
      h *= 0x100000001b3ull;
    }
    return size_t(h);
  }
};
struct MemoEntry {
  ValueId value;
  Tensor result; // holds the block
  size_t bytes;
  std::list<MemoKey>::iterator age;
};
struct ResultCache {
  std::unordered_map<MemoKey, MemoEntry, MemoKeyHash> entries;
  std::list<MemoKey> ages;                        // most recent first
  // the entries of each result block (pointers to their keys in `entries`)
  std::unordered_map<const void *, std::vector<const MemoKey *>> blocks;
  std::unordered_map<MemoKey, ValueId, MemoKeyHash> derived; // transposed views
  size_t bytes = 0;
};
ResultCache &cache() {
  static auto *c = new ResultCache();
  return *c;
}
// Byte budget of the cache; TEMPLIT_HIP_RESULT_CACHE_MB overrides (0 turns
// reuse off).
size_t cache_budget() {
  static const size_t budget = [] {
    const char *env = std::getenv("TEMPLIT_HIP_RESULT_CACHE_MB");
    return env ? size_t(std::strtoull(env, nullptr, 10)) << 20 : size_t(1) << 30;
  }();
  return budget;
}

struct KeyBuilder {
  MemoKey key;
  explicit KeyBuilder(uint32_t op) { key.words.push_back(op); }
  template <typename T> KeyBuilder &tensor(const RTensor<HIP, T> &t) {
    key.words.push_back(t.get_storage() ? value_of(t.get_storage()->data()) : 0);
    dims(t.shape());
    return *this;
  }
  KeyBuilder &dims(std::span<const uint32_t> d) {
    key.words.push_back(d.size());
    key.words.insert(key.words.end(), d.begin(), d.end());
    return *this;
  }
  KeyBuilder &scalar(float v) {
    uint32_t bits;
    std::memcpy(&bits, &v, 4);
    key.words.push_back(bits);
    return *this;
  }
};

void forget(std::unordered_map<MemoKey, MemoEntry, MemoKeyHash>::iterator it) {
  ResultCache &c = cache();
  c.bytes -= it->second.bytes;
  c.ages.erase(it->second.age);
  const void *block = it->second.result.get_storage()->data();
  if (const auto b = c.blocks.find(block); b != c.blocks.end()) {
    auto &keys = b->second;
    keys.erase(std::remove(keys.begin(), keys.end(), &it->first), keys.end());
    if (keys.empty()) c.blocks.erase(b);
  }
  MemoEntry dead = std::move(it->second); // released after the erase
  c.entries.erase(it);
}

// The derived identity of a transposed view of value `v`.
ValueId derived_value(MemoKey &&key) {
  auto &derived = cache().derived;
  if (derived.size() > (size_t(1) << 16)) derived.clear(); // new numbers from here on
  auto [it, inserted] = derived.try_emplace(std::move(key), 0);
  if (inserted) it->second = fresh_value();
  return it->second;
}

bool contiguous(std::span<const uint32_t> shape, std::span<const uint32_t> strides) {
  uint64_t expect = 1;
  for (size_t i = shape.size(); i-- > 0;) {
    if (shape[i] != 1 && strides[i] != expect) return false;
    expect *= shape[i];
  }
  return true;
}

void materialise(const void *base) {
  auto &views = pending_views();
  const auto it = views.find(base);
  if (it == views.end()) return;
  PendingView v = take_view(it); // (its source may be released on return)
  float *dst = static_cast<float *>(const_cast<void *>(base));
  const float *src = v.source.get_storage()->data();
  size_t n = 1;
  for (const uint32_t d : v.shape) n *= d;
  if (n == 0) return;
  if (const ProductPlan *p = v.product.get()) {
    const size_t r = v.shape.size();
    check(tlh_matmul(src, p->b.get_storage()->data(), dst, p->M, p->K, p->N, p->a_rs, p->a_cs,
                     p->b_rs, p->b_cs, v.shape[r - 1], 1, uint32_t(p->batch.size()),
                     p->batch.data(), p->sa.data(), p->sb.data(), p->sc.data(), stream()),
          "materialise product");
    return;
  }
  if (contiguous(v.shape, v.strides))
    check(tlh_copy(src, dst, n, stream()), "materialise copy");
  else
    check(tlh_transpose(src, dst, uint32_t(v.shape.size()), v.shape.data(), v.strides.data(),
                        stream()),
          "materialise transpose");
}

// ---- squared norms collected per scalar -------------------------------------
// Compiled::step(max_norm) accumulates every gradient's squared norm into one
// scalar, a call per tensor (include/passes/compile.h:241-245), and reads it
// only in the clips that follow. The calls are collected per scalar and run
// as one multi-tensor launch plus one add into the scalar when the scalar is
// read or written, when one of the collected gradients is about to be
// written, or at submit().
struct PendingNorm {
  Tensor s;
  std::vector<Tensor> grads;
};
std::unordered_map<const void *, PendingNorm> &pending_norms() {
  static auto *norms = new std::unordered_map<const void *, PendingNorm>();
  return *norms;
}
void flush_norm(const void *s_block);           // the collection into this scalar, if any
void flush_norms_reading(const void *block);    // every collection holding this gradient

// ---- AdamW updates collected ---------------------------------------------------
// exec::step updates every parameter with its own adamW call (the
// optimiser's update, include/optimiser/AdamW.h); in-place updates that share
// the hyper-parameter scalars are collected and run as one multi-tensor
// launch at submit(), or before anything reads or writes a parameter or
// moment they update, or writes a gradient or scalar they read.
struct AdamEntry {
  Tensor p, g, m1, m2;
  uint32_t step;
};
struct PendingAdam {
  std::vector<AdamEntry> entries;
  Tensor beta1, beta2, decay, lr;
  float eps = 0.0f;
  std::unordered_map<const void *, int> writes, reads; // blocks -> uses
};
PendingAdam &pending_adam() {
  static auto *adam = new PendingAdam();
  return *adam;
}
bool adam_pending() { return !pending_adam().entries.empty(); }
void flush_adam();

// ---- in-place clips batched ---------------------------------------------------------
// Compiled::step(max_norm) clips each gradient in place with a call of its
// own (compile.h:246-249). Consecutive in-place clips by one norm and bound
// are batched and run as one multi-tensor launch before the runtime does
// anything else (the next op, a host access, submit), so every other
// operation finds them done. A gradient slot that is still a pending copy
// of its one contribution is clipped from the copy's source into the slot,
// so the copy is never made.
struct ClipEntry {
  Tensor g;   // written whole
  Tensor src; // read: g itself, or the source of the copy g was
};
struct ClipBatch {
  std::vector<ClipEntry> entries;
  Tensor s;
  float max_norm = 0.0f;
};
ClipBatch &clip_batch() {
  static auto *batch = new ClipBatch();
  return *batch;
}
void flush_clips();
void flush_linear(); // the product waiting for its bias (see below)
void drop_linear();
bool add_bias_to_product(const Tensor &a, const Tensor &b, Tensor &o);
bool gelu_of_product(const Tensor &a, Tensor &o);
void settle(const void *base); // runs collected work that reads or writes this block

// Before a kernel or the host reads block `base`.
void reading(const void *base) {
  if (adam_pending() && pending_adam().writes.count(base)) flush_adam();
  if (!pending_norms().empty()) flush_norm(base);
  if (!pending_views().empty()) materialise(base);
}

// Before a kernel or the host writes block `base`: its own pending view
// first (partial and in-place writes keep the rest), then every view whose
// source is this block, which needs its current contents.
void writing(const void *base) {
  if (adam_pending() && (pending_adam().writes.count(base) || pending_adam().reads.count(base)))
    flush_adam();
  if (!pending_norms().empty()) {
    flush_norm(base);
    flush_norms_reading(base);
  }
  auto &views = pending_views();
  if (views.empty()) return;
  materialise(base);
  const auto r = view_readers().find(base);
  if (r == view_readers().end()) return;
  const std::vector<const void *> readers = r->second; // (materialise edits the index)
  for (const void *dst : readers) materialise(dst);
}

void storage_hook(const void *base, int kind) {
  if (kind == detail::kAccessShutdown) { // the context goes: drop every view
    auto dead = std::move(pending_views());
    pending_views().clear();
    view_readers().clear();
    auto dead_norms = std::move(pending_norms());
    pending_norms().clear();
    PendingAdam dead_adam = std::move(pending_adam());
    pending_adam() = PendingAdam{};
    ClipBatch dead_clips = std::move(clip_batch());
    clip_batch() = ClipBatch{};
    drop_linear();
    auto dead_results = std::move(cache().entries);
    cache().entries.clear();
    cache().ages.clear();
    cache().blocks.clear();
    cache().bytes = 0;
    return;
  }
  if (kind == detail::kAccessRelease) {
    block_values().erase(base); // the pool may hand the block out again
    if (const auto it = pending_norms().find(base); it != pending_norms().end()) {
      PendingNorm dead = std::move(it->second); // nobody can read this scalar any more
      pending_norms().erase(it);
    }
    auto &views = pending_views();
    const auto it = views.find(base);
    if (it == views.end()) return;
    PendingView dead = take_view(it); // destroyed after the erase
    return;
  }
  flush_linear(); // a host access sees them done
  flush_clips();
  if (kind == detail::kAccessRead) {
    reading(base);
  } else {
    writing(base);
    written(base);
  }
}

// The device pointer a kernel reads t's elements from. A block that is a
// pending copy (a contiguous view of its source: the same bytes in the same
// order) is read at its source, which the view holds; any other pending
// view or product is filled first.
template <typename T> const T *in(const RTensor<HIP, T> &t) {
  if (!t.get_storage()) throw std::logic_error("operation on an uninitialised tensor");
  const T *p = t.get_storage()->data();
  if constexpr (std::is_same_v<T, float>) {
    auto &views = pending_views();
    if (!views.empty()) {
      const auto it = views.find(p);
      if (it != views.end() && !it->second.product &&
          contiguous(it->second.shape, it->second.strides))
        return it->second.source.get_storage()->data();
      reading(p);
    }
  }
  return p;
}
template <typename T> T *out(RTensor<HIP, T> &t) {
  if (!t.get_storage()) throw std::logic_error("operation on an uninitialised tensor");
  T *p = t.get_storage()->data();
  if constexpr (std::is_same_v<T, float>) writing(p);
  written(p);
  return p;
}

void flush_norm(const void *s_block) {
  auto node = pending_norms().extract(s_block);
  if (node.empty()) return;
  PendingNorm pn = std::move(node.mapped());
  const size_t n = pn.grads.size();
  // device tables: n gradient pointers, then n element counts (u64 each)
  std::vector<uint64_t> table(2 * n);
  for (size_t i = 0; i < n; ++i) {
    table[i] = reinterpret_cast<uintptr_t>(in(pn.grads[i]));
    table[n + i] = pn.grads[i].numel();
  }
  Tensor tables({uint32_t(4 * n)});
  tables.get_storage()->write(
      std::span<const float>(reinterpret_cast<const float *>(table.data()), 4 * n), 0);
  Tensor partials({uint32_t(TLH_NORM_PARTIALS + 1)}); // the last element takes the sum
  float *part = out(partials);
  const float *tab = in(tables);
  check(tlh_gradient_squared_norm_multi(reinterpret_cast<const float *const *>(tab),
                                        reinterpret_cast<const uint64_t *>(tab + 2 * n),
                                        uint32_t(n), part, part + TLH_NORM_PARTIALS, stream()),
        "accumulate_gradient_squared_norm");
  float *acc = pn.s.get_storage()->data(); // (not pending: filled when the collection began)
  const uint32_t one = 1;
  check(tlh_add(acc, part + TLH_NORM_PARTIALS, acc, 1, &one, &one, &one, stream()),
        "accumulate_gradient_squared_norm");
}

void flush_adam() {
  PendingAdam pa = std::move(pending_adam());
  pending_adam() = PendingAdam{};
  const size_t n = pa.entries.size();
  if (n == 0) return;
  // device tables: p, g, m1, m2 pointers and sizes (u64 each), steps (u32)
  std::vector<uint64_t> table(5 * n + (n + 1) / 2, 0);
  uint32_t *steps = reinterpret_cast<uint32_t *>(table.data() + 5 * n);
  for (size_t i = 0; i < n; ++i) {
    AdamEntry &e = pa.entries[i];
    table[i] = reinterpret_cast<uintptr_t>(e.p.get_storage()->data());
    table[n + i] = reinterpret_cast<uintptr_t>(in(e.g));
    table[2 * n + i] = reinterpret_cast<uintptr_t>(e.m1.get_storage()->data());
    table[3 * n + i] = reinterpret_cast<uintptr_t>(e.m2.get_storage()->data());
    table[4 * n + i] = e.p.numel();
    steps[i] = e.step;
  }
  const size_t floats = 2 * table.size();
  Tensor tables({uint32_t(floats)});
  tables.get_storage()->write(
      std::span<const float>(reinterpret_cast<const float *>(table.data()), floats), 0);
  const float *t = in(tables);
  const auto ptrs = [&](size_t k) { return reinterpret_cast<float *const *>(t + 2 * k * n); };
  check(tlh_adamw_multi(ptrs(0), reinterpret_cast<const float *const *>(ptrs(1)), ptrs(2), ptrs(3),
                        reinterpret_cast<const uint64_t *>(t + 8 * n),
                        reinterpret_cast<const uint32_t *>(t + 10 * n), uint32_t(n),
                        in(pa.beta1), in(pa.beta2), in(pa.decay), in(pa.lr), pa.eps, nullptr,
                        0.0f, stream()),
        "adamW");
}

void flush_clips() {
  if (clip_batch().entries.empty()) return;
  ClipBatch b = std::move(clip_batch());
  clip_batch() = ClipBatch{};
  const size_t n = b.entries.size();
  // device tables: source pointers, destination pointers, element counts
  // (u64 each)
  std::vector<uint64_t> table(3 * n);
  for (size_t i = 0; i < n; ++i) {
    ClipEntry &e = b.entries[i];
    float *dst = out(e.g); // readers of the old values first
    table[i] = reinterpret_cast<uintptr_t>(
        e.src.get_storage() == e.g.get_storage() ? dst : e.src.get_storage()->data());
    table[n + i] = reinterpret_cast<uintptr_t>(dst);
    table[2 * n + i] = e.g.numel();
  }
  Tensor tables({uint32_t(6 * n)});
  tables.get_storage()->write(
      std::span<const float>(reinterpret_cast<const float *>(table.data()), 6 * n), 0);
  const float *t = in(tables);
  check(tlh_clip_multi(reinterpret_cast<const float *const *>(t),
                       reinterpret_cast<float *const *>(t + 2 * n),
                       reinterpret_cast<const uint64_t *>(t + 4 * n), uint32_t(n), in(b.s),
                       b.max_norm, stream()),
        "clip_gradient");
}

void flush_norms_reading(const void *block) {
  std::vector<const void *> hits;
  for (const auto &[sb, pn] : pending_norms())
    for (const Tensor &g : pn.grads)
      if (g.get_storage()->data() == block) {
        hits.push_back(sb);
        break;
      }
  for (const void *sb : hits) flush_norm(sb);
}

// Before an op overwrites every element of `o` without reading it: views
// and products still pending on o's block keep that block -- it moves to a
// storage of their own -- and o's storage takes a fresh block from the
// pool, so nothing is copied. (The executor rewrites its node buffers each
// step while views of last step's values are still pending.)
std::optional<Tensor> move_aside(Tensor &o) {
  settle(o.get_storage()->data());
  auto &views = pending_views();
  ResultCache &c = cache();
  auto *os = o.get_storage();
  const void *base = os->data();
  const auto r = view_readers().find(base);
  const std::vector<const void *> readers =
      r == view_readers().end() ? std::vector<const void *>{} : r->second;
  const bool cached = c.blocks.count(base) > 0;
  if (!cached && readers.empty()) return std::nullopt;
  if (os->size() == 0 || os->size() > UINT32_MAX) {
    writing(base);
    return std::nullopt;
  }
  // the readers (and cached results) are pointed at the new storage first,
  // then the blocks swap; the old block keeps its value identity
  Tensor holder({uint32_t(os->size())});
  for (const void *dst : readers) { // (their blocks keep the address `base`)
    PendingView &v = views.at(dst);
    if (v.source.get_storage()->data() == base) v.source = holder;
    if (v.product && v.product->b.get_storage()->data() == base) {
      auto plan = std::make_shared<ProductPlan>(*v.product);
      plan->b = holder;
      v.product = std::move(plan);
    }
  }
  if (cached) {
    std::vector<MemoKey> stale;
    for (const MemoKey *key : c.blocks.at(base)) {
      MemoEntry &e = c.entries.find(*key)->second;
      if (e.result.numel() == os->size()) e.result = holder.view(e.result.shape());
      else stale.push_back(*key);
    }
    for (const MemoKey &key : stale) forget(c.entries.find(key));
  }
  os->exchange_block(*holder.get_storage());
  written(os->data());
  return holder;
}

// Runs the collected work that reads block `base` or writes it (squared
// norms of or into it, AdamW updates of or from it), before its contents
// change.
void settle(const void *base) {
  if (adam_pending() && (pending_adam().writes.count(base) || pending_adam().reads.count(base)))
    flush_adam();
  if (pending_norms().empty()) return;
  flush_norm(base);
  flush_norms_reading(base);
}

// Drops the pending view of block `base`, if any, without filling it.
void drop_view(const void *base) {
  settle(base);
  auto &views = pending_views();
  const auto it = views.find(base);
  if (it == views.end()) return;
  PendingView dead = take_view(it); // destroyed after the erase
}

// The pending view of `t` when it covers t exactly (its own shape).
const PendingView *view_of(const Tensor &t) {
  auto &views = pending_views();
  if (views.empty() || !t.get_storage()) return nullptr;
  const auto it = views.find(t.get_storage()->data());
  return it != views.end() && it->second.shape == t.shape() && !it->second.product
             ? &it->second
             : nullptr;
}

// `o` becomes a view of `a`, o's dim d being a's dim perm[d] (a transpose,
// or with the identity a copy of the same shape). o's previous contents are
// dead (a pending view of o is dropped) and views reading o are filled
// first. A pending `a` is composed: o then views a's source.
void defer_view(const Tensor &a, Tensor &o, const std::vector<size_t> &perm) {
  if (!o.get_storage() || !a.get_storage())
    throw std::logic_error("operation on an uninitialised tensor");
  if (a.get_storage() == o.get_storage())
    throw std::invalid_argument("view of a tensor into its own storage");
  drop_view(o.get_storage()->data());
  move_aside(o);
  const void *dst = o.get_storage()->data();
  shape_type strides(perm.size());
  Tensor source = a;
  const auto copy = pending_views().find(a.get_storage()->data());
  if (const PendingView *v = view_of(a)) {
    source = v->source;
    for (size_t d = 0; d < perm.size(); ++d) strides[d] = v->strides[perm[d]];
  } else if (copy != pending_views().end() && !copy->second.product &&
             contiguous(copy->second.shape, copy->second.strides) &&
             contiguous(a.shape(), a.strides())) {
    // a reshape of a pending copy (split_last_dim aliases its input): the
    // same bytes in the same order at the copy's source
    source = copy->second.source;
    for (size_t d = 0; d < perm.size(); ++d) strides[d] = a.strides()[perm[d]];
  } else {
    reading(a.get_storage()->data()); // a view's source is never pending
    for (size_t d = 0; d < perm.size(); ++d) strides[d] = a.strides()[perm[d]];
  }
  if (source.get_storage() == o.get_storage())
    throw std::invalid_argument("view of a tensor into its own storage");
  put_view(dst, PendingView{std::move(source), o.shape(), std::move(strides)});
  // a copy holds a's value; a transposed view a value derived from it
  bool identity = o.shape() == a.shape();
  for (size_t d = 0; d < perm.size(); ++d) identity = identity && perm[d] == d;
  if (identity) {
    set_value(dst, value_of(a.get_storage()->data()));
  } else {
    std::vector<uint32_t> order(perm.begin(), perm.end());
    set_value(dst, derived_value(std::move(KeyBuilder(kTranspose).tensor(a).dims(order).key)));
  }
}

// `o` (same element count, another shape) becomes a view of the elements
// of `a` in order.
void defer_reshape(const Tensor &a, Tensor &o) {
  if (o.shape() == a.shape()) {
    std::vector<size_t> identity(o.shape().size());
    std::iota(identity.begin(), identity.end(), size_t(0));
    defer_view(a, o, identity);
    return;
  }
  if (a.get_storage() == o.get_storage())
    throw std::invalid_argument("view of a tensor into its own storage");
  drop_view(o.get_storage()->data());
  move_aside(o);
  // the same bytes: a's source when a is itself a pending copy, else a
  // (filled first if it is another pending view)
  Tensor source = a;
  const auto it = pending_views().find(a.get_storage()->data());
  if (it != pending_views().end() && !it->second.product &&
      contiguous(it->second.shape, it->second.strides))
    source = it->second.source;
  else
    reading(a.get_storage()->data());
  put_view(o.get_storage()->data(), PendingView{std::move(source), o.shape(), o.strides()});
  set_value(o.get_storage()->data(), value_of(a.get_storage()->data()));
}

// True when block `base` holds a still valid cached result of an op other
// than `op`. An in-place op of another kind that rewrote it would end a
// chain of reusable results: the softmax derivative p * (g - rowsum(g * p))
// is evaluated once per path through the scores, and each evaluation writes
// the product over the difference it reads.
bool holds_other_result(const void *base, uint32_t op) {
  ResultCache &c = cache();
  const auto b = c.blocks.find(base);
  if (b == c.blocks.end()) return false;
  const ValueId v = value_of(base);
  for (const MemoKey *key : b->second)
    if (c.entries.find(*key)->second.value == v && key->words[0] != op) return true;
  return false;
}

// The destination of an op that writes every element of `o`: unless one of
// `inputs` shares o's storage and so reads it, a pending view of o is
// dropped unfilled (its bytes are dead) and views reading o keep its old
// block (move_aside); otherwise views reading o are filled first.
float *dest(Tensor &o, std::initializer_list<const Tensor *> inputs) {
  if (!o.get_storage()) throw std::logic_error("operation on an uninitialised tensor");
  bool read = false;
  for (const Tensor *t : inputs) read = read || t->get_storage() == o.get_storage();
  if (!read) {
    drop_view(o.get_storage()->data());
    move_aside(o);
  }
  return out(o);
}

// A cached result for `key`: o already holds it, or o becomes a pending copy
// of the cached block (its old contents treated as by an op that
// overwrites it whole). False when there is none and the op must run.
bool reuse(const MemoKey &key, Tensor &o) {
  ResultCache &c = cache();
  if (cache_budget() == 0 || !o.get_storage() || c.entries.empty()) return false;
  const auto it = c.entries.find(key);
  if (it == c.entries.end()) return false;
  MemoEntry &e = it->second;
  if (value_of(e.result.get_storage()->data()) != e.value || e.result.shape() != o.shape()) {
    forget(it); // the block was written since
    return false;
  }
  c.ages.splice(c.ages.begin(), c.ages, e.age);
  if (value_of(o.get_storage()->data()) == e.value) return true;
  const Tensor source = e.result; // (defer_view may reorder the cache)
  std::vector<size_t> identity(o.shape().size());
  std::iota(identity.begin(), identity.end(), size_t(0));
  defer_view(source, o, identity);
  return true;
}

// Caches o (just written by the op `key` describes) as that op's result.
void remember(MemoKey &&key, const Tensor &o) {
  ResultCache &c = cache();
  const size_t budget = cache_budget();
  if (budget == 0 || !o.get_storage() || o.numel() == 0) return;
  const size_t bytes = o.numel() * sizeof(float);
  if (bytes > budget / 4) return;
  if (const auto it = c.entries.find(key); it != c.entries.end()) forget(it);
  const void *block = o.get_storage()->data();
  c.ages.push_front(key);
  const auto it =
      c.entries.emplace(std::move(key), MemoEntry{value_of(block), o, bytes, c.ages.begin()}).first;
  c.blocks[block].push_back(&it->first);
  c.bytes += bytes;
  while (c.bytes > budget) forget(c.entries.find(c.ages.back()));
}

// An op that writes every element of o and whose result `key` determines:
// a cached result is reused, else `launch(destination pointer)` runs (with
// dest's treatment of o) and its result is cached.
template <typename F>
void cached(KeyBuilder &key, Tensor &o, std::initializer_list<const Tensor *> inputs, F &&launch) {
  if (reuse(key.key, o)) return;
  launch(dest(o, inputs));
  remember(std::move(key.key), o);
}

// An operand read through its strides: a pending view reads its source
// (when `unit_inner`, only if one of the last two strides is 1, as the
// GEMM needs); anything else is materialised.
struct Operand {
  const float *ptr;
  shape_type strides;
  const Tensor *holder; // the tensor whose storage holds the data
};
Operand operand(const Tensor &t, bool unit_inner) {
  if (const PendingView *v = view_of(t)) {
    const shape_type &st = v->strides;
    const size_t r = st.size();
    if (!unit_inner || (r >= 2 && (st[r - 1] == 1 || st[r - 2] == 1)))
      return {v->source.get_storage()->data(), st, &v->source};
  }
  return {in(t), t.strides(), &t};
}

// Element strides of `shape`/`strides` right-aligned to `out_shape`, 0 on
// broadcast dims (runtime.cpp:18-39).
std::vector<uint32_t> broadcast_strides(std::span<const uint32_t> shape,
                                        std::span<const uint32_t> strides,
                                        std::span<const uint32_t> out_shape) {
  if (shape.size() > out_shape.size()) throw std::runtime_error("invalid broadcast");
  std::vector<uint32_t> result(out_shape.size(), 0);
  const size_t offset = out_shape.size() - shape.size();
  for (size_t i = 0; i < shape.size(); ++i) {
    if (shape[i] == out_shape[offset + i]) result[offset + i] = strides[i];
    else if (shape[i] != 1) throw std::runtime_error("invalid broadcast");
  }
  return result;
}

using BinaryFn = int (*)(const float *, const float *, float *, uint32_t, const uint32_t *,
                         const uint32_t *, const uint32_t *, void *);
using UnaryFn = int (*)(const float *, float *, size_t, void *);
using ScalarFn = int (*)(const float *, float, float *, size_t, void *);

void require_same_count(const Tensor &a, const Tensor &o, const char *op) {
  if (a.numel() != o.numel())
    throw std::invalid_argument(std::string(op) + " destination has incorrect shape");
}

// rows x cols view of a tensor whose last dim is the row.
struct Rows {
  size_t rows;
  uint32_t cols;
};
Rows as_rows(const Tensor &t, const char *op) {
  if (t.shape().empty() || t.shape().back() == 0)
    throw std::invalid_argument(std::string(op) + " requires a non-empty final dimension");
  return {t.numel() / t.shape().back(), t.shape().back()};
}

// Drops unit batch dims and merges neighbours that are contiguous in all
// three operands, so the kernel's 4 batch dims cover any practical rank.
struct Batch {
  std::vector<uint32_t> shape, sa, sb, sc;
};
Batch simplify_batch(std::span<const uint32_t> shape, const std::vector<uint32_t> &sa,
                     const std::vector<uint32_t> &sb, std::span<const uint32_t> sc) {
  Batch out;
  for (size_t i = 0; i < shape.size(); ++i) {
    if (shape[i] == 1) continue;
    if (!out.shape.empty()) {
      const size_t j = out.shape.size() - 1;
      const auto merges = [&](uint32_t outer, uint32_t inner) {
        return uint64_t(outer) == uint64_t(inner) * shape[i];
      };
      if (merges(out.sa[j], sa[i]) && merges(out.sb[j], sb[i]) && merges(out.sc[j], sc[i])) {
        out.shape[j] *= shape[i];
        out.sa[j] = sa[i];
        out.sb[j] = sb[i];
        out.sc[j] = sc[i];
        continue;
      }
    }
    out.shape.push_back(shape[i]);
    out.sa.push_back(sa[i]);
    out.sb.push_back(sb[i]);
    out.sc.push_back(sc[i]);
  }
  return out;
}

} // namespace

struct Runtime::State {
  bool recording = false;
  bool submitted = false;
  bool graph_mode = false;
  bool capturing = false;
  bool profiling = false;
  uint64_t signature = 0;
  std::unordered_map<uint64_t, void *> graphs; // op/shape sequence -> executable graph
  void *launched = nullptr;
  GraphStats stats;
};

Runtime::Runtime() : state_(std::make_unique<State>()) {
  if (!initialised()) throw std::logic_error("HIP must be initialised before Runtime");
  detail::set_access_hook(&storage_hook);
}

Runtime::~Runtime() { cleanup(); }

void Runtime::require_recording(const char *op, bool run_clips) const {
  if (!state_->recording)
    throw std::logic_error(std::string("HIP runtime execution has not started (") + op + ")");
  flush_linear();
  if (run_clips) flush_clips();
}

// FNV-1a over the op and its output shape: the key of a recorded sequence.
void Runtime::note(uint32_t op, std::span<const uint32_t> shape) {
  if (!state_->capturing) return;
  uint64_t h = state_->signature;
  const auto mix = [&h](uint64_t v) {
    h ^= v;
    h *= 0x100000001b3ull;
  };
  mix(op);
  mix(shape.size());
  for (uint32_t d : shape) mix(d);
  state_->signature = h;
}

// ---- lifecycle (runtime.cpp:170-317) ----------------------------------------

void Runtime::start() {
  State &s = *state_;
  if (s.recording || s.submitted) throw std::logic_error("HIP runtime execution already started");
  if (s.graph_mode) {
    // Host transfers made while recording happen at record time; nothing
    // queued earlier may still be running when they do.
    check(tlh_stream_synchronize(stream()), "hipStreamSynchronize");
    check(tlh_graph_begin_capture_relaxed(stream()), "hipStreamBeginCapture");
    hip::detail::defer_releases(true);
    s.capturing = true;
    s.signature = 0xcbf29ce484222325ull;
  }
  s.recording = true;
}

void Runtime::submit() {
  State &s = *state_;
  if (!s.recording) throw std::logic_error("HIP runtime execution has not started");
  flush_linear();
  flush_clips();
  while (!pending_norms().empty()) flush_norm(pending_norms().begin()->first);
  flush_adam();
  s.recording = false;
  s.submitted = true;
  if (!s.capturing) return;
  s.capturing = false;
  void *graph = nullptr;
  int st = tlh_graph_end_capture_graph(stream(), &graph);
  if (st != 0) {
    s.submitted = false;
    hip::detail::defer_releases(false);
    check(st, "hipStreamEndCapture");
  }
  s.stats.captures += 1;
  void *&exec = s.graphs[s.signature];
  int updated = 0;
  if (exec) {
    st = tlh_graph_exec_update(exec, graph, &updated);
    if (st == 0 && updated) s.stats.updates += 1;
  }
  if (st == 0 && !updated) {
    if (exec) tlh_graph_destroy(exec);
    exec = nullptr;
    st = tlh_graph_instantiate(graph, &exec);
    if (st == 0) s.stats.instantiations += 1;
  }
  tlh_graph_free(graph);
  if (st == 0) st = tlh_graph_launch(exec, stream());
  // Blocks released during the capture may be reused from here on: later
  // work is queued after the graph, and the next capture's start() waits
  // for the graph before any record-time host transfer.
  hip::detail::defer_releases(false);
  if (st != 0) {
    s.submitted = false;
    check(st, "hipGraphLaunch");
  }
}

void Runtime::wait() {
  State &s = *state_;
  if (!s.submitted || s.recording)
    throw std::logic_error("HIP runtime execution has not been submitted");
  s.submitted = false;
  check(tlh_stream_synchronize(stream()), "HIP runtime execution");
}

namespace {
void forget_recorded_work() noexcept {
  ResultCache &c = cache();
  auto dead_results = std::move(c.entries);
  c.entries.clear();
  c.ages.clear();
  c.blocks.clear();
  c.derived.clear();
  c.bytes = 0;
  block_values().clear(); // every block takes a fresh identity on next use
  auto dead_norms = std::move(pending_norms());
  pending_norms().clear();
  PendingAdam dead_adam = std::move(pending_adam());
  pending_adam() = PendingAdam{};
  ClipBatch dead_clips = std::move(clip_batch());
  clip_batch() = ClipBatch{};
  drop_linear();
}
} // namespace

void Runtime::abort() noexcept {
  State &s = *state_;
  if (s.capturing) {
    void *graph = nullptr;
    if (tlh_graph_end_capture_graph(stream(), &graph) == 0) tlh_graph_free(graph);
    hip::detail::defer_releases(false); // the dropped graph never runs
    s.capturing = false;
    // Nothing recorded in the dropped graph ran: cached results and value
    // identities may name blocks it was to write, and the collected norm and
    // AdamW calls belong to it.
    forget_recorded_work();
  }
  s.recording = false;
  s.submitted = false;
}


void Runtime::cleanup() noexcept {
  if (!state_) return;
  State &s = *state_;
  const bool had_work = s.recording || s.submitted;
  abort();
  if (had_work && initialised()) tlh_stream_synchronize(stream());
  for (auto &[key, exec] : s.graphs) tlh_graph_destroy(exec);
  s.graphs.clear();
  if (s.profiling) {
    tlh_range_pop();
    s.profiling = false;
  }
}

void Runtime::start_profile(std::string_view output_path) {
  if (state_->profiling) throw std::logic_error("a profile span is already open");
  const std::string name(output_path);
  check(tlh_range_push(name.c_str()), "roctxRangePush");
  state_->profiling = true;
}

void Runtime::end_profile() {
  if (!state_->profiling) return;
  tlh_range_pop();
  state_->profiling = false;
}

void Runtime::set_graph_mode(bool enabled) {
  if (state_->recording || state_->submitted)
    throw std::logic_error("graph mode can only change between executions");
  state_->graph_mode = enabled;
}
bool Runtime::graph_mode() const { return state_->graph_mode; }
Runtime::GraphStats Runtime::graph_stats() const { return state_->stats; }

// ---- elementwise (runtime.cpp:65-136, 321-373, 1073-1081, 1170-1186) -------

namespace {
void binary(Runtime &, const Tensor &a, const Tensor &b, Tensor &o, BinaryFn fn, const char *what,
            uint32_t op) {
  broadcast_strides(a.shape(), a.strides(), o.shape()); // shape checks first
  broadcast_strides(b.shape(), b.strides(), o.shape());
  if (o.numel() == 0) return;
  KeyBuilder key(op);
  key.tensor(a).tensor(b).dims(o.shape());
  if (reuse(key.key, o)) return;
  // An in-place op on a destination that is still a view (a gradient slot
  // holding a copy of its first contribution, then add(slot, g, slot),
  // context.h:73-89): the op writes every element of o, so the inputs that
  // are o read the view's source and the copy is never made. (No view ever
  // reads a block that is itself a pending view.)
  auto &views = pending_views();
  const void *ob_ = o.get_storage() ? static_cast<const void *>(o.get_storage()->data()) : nullptr;
  if (ob_) settle(ob_); // (before the lookup: it may fill views)
  const auto self = ob_ ? views.find(ob_) : views.end();
  const bool same_a = a.get_storage() == o.get_storage(), same_b = b.get_storage() == o.get_storage();
  if (self != views.end() && !self->second.product && (same_a || same_b) &&
      (!same_a || a.shape() == o.shape()) && (!same_b || b.shape() == o.shape())) {
    PendingView v = take_view(self); // holds the source until the launch
    const Operand src{v.source.get_storage()->data(), v.strides, &v.source};
    const Operand oa = same_a ? src : operand(a, false), ob = same_b ? src : operand(b, false);
    const auto sa = broadcast_strides(a.shape(), oa.strides, o.shape());
    const auto sb = broadcast_strides(b.shape(), ob.strides, o.shape());
    check(fn(oa.ptr, ob.ptr, o.get_storage()->data(), uint32_t(o.shape().size()),
             o.shape().data(), sa.data(), sb.data(), stream()),
          what);
    written(o.get_storage()->data());
    remember(std::move(key.key), o);
    return;
  }
  // An in-place op over a cached result of another op: the result keeps the
  // old block, which the op reads, and o takes a fresh one (move_aside), so
  // the next evaluation of the same expression still finds it.
  if ((same_a || same_b) && ob_ && self == views.end() && holds_other_result(ob_, op) &&
      (!same_a || (a.shape() == o.shape() && a.strides() == o.strides())) &&
      (!same_b || (b.shape() == o.shape() && b.strides() == o.strides()))) {
    if (const std::optional<Tensor> old = move_aside(o)) {
      const Operand src{old->get_storage()->data(), o.strides(), &*old};
      const Operand oa = same_a ? src : operand(a, false), ob = same_b ? src : operand(b, false);
      const auto sa = broadcast_strides(a.shape(), oa.strides, o.shape());
      const auto sb = broadcast_strides(b.shape(), ob.strides, o.shape());
      check(fn(oa.ptr, ob.ptr, out(o), uint32_t(o.shape().size()), o.shape().data(), sa.data(),
               sb.data(), stream()),
            what);
      remember(std::move(key.key), o);
      return;
    }
  }
  // the destination first: views of it are filled before it is written
  float *dst = dest(o, {&a, &b});
  const Operand oa = operand(a, false), ob = operand(b, false);
  const auto sa = broadcast_strides(a.shape(), oa.strides, o.shape());
  const auto sb = broadcast_strides(b.shape(), ob.strides, o.shape());
  check(fn(oa.ptr, ob.ptr, dst, uint32_t(o.shape().size()), o.shape().data(), sa.data(),
           sb.data(), stream()),
        what);
  remember(std::move(key.key), o);
}

// For an op on one input that rewrites o in place (a is o) while o's block
// holds a cached result of another op (the executor's
// divide(mean, D, mean) after the sum that produced mean): the result moves
// aside, and the returned block holding it is what the op reads.
std::optional<Tensor> in_place_aside(const Tensor &a, Tensor &o, uint32_t op) {
  if (a.get_storage() != o.get_storage() || !o.get_storage()) return std::nullopt;
  const void *base = o.get_storage()->data();
  if (pending_views().count(base) || !holds_other_result(base, op)) return std::nullopt;
  return move_aside(o);
}

void unary(const Tensor &a, Tensor &o, UnaryFn fn, const char *what, uint32_t op) {
  require_same_count(a, o, what);
  if (o.numel() == 0) return;
  KeyBuilder key(op);
  key.tensor(a).dims(o.shape());
  if (reuse(key.key, o)) return;
  if (const std::optional<Tensor> old = in_place_aside(a, o, op)) {
    check(fn(old->get_storage()->data(), out(o), o.numel(), stream()), what);
    remember(std::move(key.key), o);
    return;
  }
  cached(key, o, {&a}, [&](float *dst) { check(fn(in(a), dst, o.numel(), stream()), what); });
}

void scalar_op(const Tensor &a, float v, Tensor &o, ScalarFn fn, const char *what, uint32_t op) {
  if (a.shape() != o.shape())
    throw std::invalid_argument("scalar operation input and output shapes must match");
  if (o.numel() == 0) return;
  KeyBuilder key(op);
  key.tensor(a).scalar(v);
  if (reuse(key.key, o)) return;
  if (const std::optional<Tensor> old = in_place_aside(a, o, op)) {
    check(fn(old->get_storage()->data(), v, out(o), o.numel(), stream()), what);
    remember(std::move(key.key), o);
    return;
  }
  cached(key, o, {&a}, [&](float *dst) { check(fn(in(a), v, dst, o.numel(), stream()), what); });
}
} // namespace

void Runtime::add(const Tensor &a, const Tensor &b, Tensor &o) {
  if (state_->recording && add_bias_to_product(a, b, o)) {
    note(kAdd, o.shape());
    return;
  }
  require_recording("add");
  note(kAdd, o.shape());
  binary(*this, a, b, o, tlh_add, "add", kAdd);
}
void Runtime::sub(const Tensor &a, const Tensor &b, Tensor &o) {
  require_recording("sub");
  note(kSub, o.shape());
  binary(*this, a, b, o, tlh_sub, "sub", kSub);
}
void Runtime::hadamard(const Tensor &a, const Tensor &b, Tensor &o) {
  require_recording("hadamard");
  note(kHadamard, o.shape());
  binary(*this, a, b, o, tlh_hadamard, "hadamard", kHadamard);
}
void Runtime::divide(const Tensor &a, const Tensor &b, Tensor &o) {
  require_recording("divide");
  note(kDivide, o.shape());
  binary(*this, a, b, o, tlh_divide, "divide", kDivide);
}
void Runtime::add(const Tensor &a, kernel_type v, Tensor &o) {
  require_recording("add");
  note(kAddScalar, o.shape());
  scalar_op(a, v, o, tlh_add_scalar, "add_scalar", kAddScalar);
}
void Runtime::divide(const Tensor &a, kernel_type v, Tensor &o) {
  require_recording("divide");
  note(kDivideScalar, o.shape());
  scalar_op(a, v, o, tlh_divide_scalar, "divide_scalar", kDivideScalar);
}
void Runtime::pow(const Tensor &a, kernel_type v, Tensor &o) {
  require_recording("pow");
  note(kPow, o.shape());
  scalar_op(a, v, o, tlh_pow_scalar, "pow_scalar", kPow);
}
void Runtime::sigmoid(const Tensor &a, Tensor &o) {
  require_recording("sigmoid");
  note(kSigmoid, o.shape());
  unary(a, o, tlh_sigmoid, "sigmoid", kSigmoid);
}
void Runtime::sqrt(const Tensor &a, Tensor &o) {
  require_recording("sqrt");
  note(kSqrt, o.shape());
  unary(a, o, tlh_sqrt, "sqrt", kSqrt);
}
void Runtime::exp(const Tensor &a, Tensor &o) {
  require_recording("exp");
  note(kExp, o.shape());
  unary(a, o, tlh_exp, "exp", kExp);
}
void Runtime::GELU(const Tensor &a, Tensor &o) {
  if (state_->recording && gelu_of_product(a, o)) {
    note(kGelu, o.shape());
    return;
  }
  require_recording("GELU");
  note(kGelu, o.shape());
  unary(a, o, tlh_gelu, "GELU", kGelu);
}
void Runtime::GELU_derivative(const Tensor &a, Tensor &o) {
  require_recording("GELU_derivative");
  note(kGeluDerivative, o.shape());
  unary(a, o, tlh_gelu_derivative, "GELU_derivative", kGeluDerivative);
}

void Runtime::copy(const Tensor &a, Tensor &o) {
  require_recording("copy");
  if (a.shape() != o.shape()) throw std::invalid_argument("copy destination has incorrect shape");
  note(kCopy, o.shape());
  if (o.numel() == 0 || a.get_storage() == o.get_storage()) return;
  // kept as a view of `a` until something needs o's bytes (see defer_view)
  defer_reshape(a, o);
}

// sub then in-place hadamard (runtime.cpp:843-848).
void Runtime::sqe(const Tensor &prediction, const Tensor &target, Tensor &o) {
  sub(prediction, target, o);
  hadamard(o, o, o);
}

// ---- products and layout ----------------------------------------------------

// Batched broadcasting matmul (runtime.cpp:375-505) on the fp32 MFMA GEMM.
namespace {
// One (batched) product; K-chunk partials (tail split / split-K) come from
// the pool and return to it on exit: their next user is queued after this
// work, and while a graph is being captured the pool holds released blocks
// back until the graph launches.
void run_product(const float *a, const float *b, float *c, uint32_t M, uint32_t K, uint32_t N,
                 uint32_t a_rs, uint32_t a_cs, uint32_t b_rs, uint32_t b_cs, uint32_t c_rs,
                 uint32_t c_cs, const Batch &batch, size_t ws_elems) {
  const uint32_t nb = uint32_t(batch.shape.size());
  if (ws_elems == 0 || ws_elems > UINT32_MAX) {
    check(tlh_matmul(a, b, c, M, K, N, a_rs, a_cs, b_rs, b_cs, c_rs, c_cs, nb, batch.shape.data(),
                     batch.sa.data(), batch.sb.data(), batch.sc.data(), stream()),
          "mult");
    return;
  }
  Tensor partials({uint32_t(ws_elems)});
  check(tlh_matmul_ws(a, b, c, M, K, N, a_rs, a_cs, b_rs, b_cs, c_rs, c_cs, nb,
                      batch.shape.data(), batch.sa.data(), batch.sb.data(), batch.sc.data(),
                      out(partials), ws_elems, stream()),
        "mult");
}

// ---- a product waiting for its bias -----------------------------------------------
// The executor's LINEAR is mult(x, W, y) then add(y, bias, y)
// (execute.h:242-253), and the FFN's first LINEAR is followed by GELU(y, g)
// (execute.h:477-482). The product mult would launch waits for the next call
// instead: an in-place add of a bias row to it becomes the product's epilogue
// (tlh_matmul_bias_ws: the same bits as the add after the product), and the
// product with its bias waits again for a GELU of it into another tensor,
// which the epilogue writes too (the pre-activation stays in y). Anything
// else (any op, a host access, submit) launches what is pending first.
struct PendingLinear {
  bool armed = false;
  Tensor a_hold, b_hold, o; // the operands' blocks and the destination, kept
  const float *a = nullptr, *b = nullptr;
  float *c = nullptr;
  uint32_t M = 0, K = 0, N = 0, a_rs = 0, a_cs = 0, b_rs = 0, b_cs = 0, c_rs = 0, c_cs = 0;
  Batch batch;
  size_t ws_elems = 0;
  Tensor bias_hold; // set: the bias row joins the epilogue
  const float *bias = nullptr;
};
PendingLinear &pending_linear() {
  static auto *linear = new PendingLinear();
  return *linear;
}
void drop_linear() {
  PendingLinear dead = std::move(pending_linear());
  pending_linear() = PendingLinear{};
}
// Launches the pending product: plain, with its bias, or (gelu_out) with its
// bias into c and GELU of that into gelu_out.
void launch_linear(float *gelu_out) {
  if (!pending_linear().armed) return;
  PendingLinear p = std::move(pending_linear());
  pending_linear() = PendingLinear{};
  const float *bias = p.bias;
  if (!bias) {
    run_product(p.a, p.b, p.c, p.M, p.K, p.N, p.a_rs, p.a_cs, p.b_rs, p.b_cs, p.c_rs, p.c_cs,
                p.batch, p.ws_elems);
    return;
  }
  Tensor partials;
  float *ws = nullptr;
  if (p.ws_elems > 0 && p.ws_elems <= UINT32_MAX) {
    partials = Tensor({uint32_t(p.ws_elems)});
    ws = out(partials);
  }
  const Batch &bt = p.batch;
  float *c = gelu_out ? gelu_out : p.c;
  float *pre = gelu_out ? p.c : nullptr;
  check(tlh_matmul_bias_ws(p.a, p.b, c, bias, pre, p.M, p.K, p.N, p.a_rs, p.a_cs, p.b_rs,
                           p.b_cs, p.c_rs, p.c_cs, uint32_t(bt.shape.size()), bt.shape.data(),
                           bt.sa.data(), bt.sb.data(), bt.sc.data(), ws, ws ? p.ws_elems : 0,
                           stream()),
        gelu_out ? "mult + bias + GELU" : "mult + bias");
}
void flush_linear() { launch_linear(nullptr); }

// add(y, bias, y) on the product waiting for its bias: the bias joins its
// epilogue (and the product waits on, for a GELU of it).
bool add_bias_to_product(const Tensor &a, const Tensor &b, Tensor &o) {
  PendingLinear &pl = pending_linear();
  if (!pl.armed || pl.bias || !o.get_storage() || !b.get_storage() ||
      a.get_storage() != o.get_storage() || o.get_storage() != pl.o.get_storage() ||
      b.get_storage() == o.get_storage() || a.shape() != o.shape() ||
      a.strides() != o.strides() || o.shape() != pl.o.shape() || o.strides() != pl.o.strides() ||
      pl.c_cs != 1 || o.shape().back() != pl.N)
    return false;
  // b: one row of N contiguous values, broadcast over every other dim
  if (b.shape().empty() || b.shape().back() != pl.N || b.numel() != pl.N ||
      b.strides().back() != 1)
    return false;
  KeyBuilder key(kAdd);
  key.tensor(a).tensor(b).dims(o.shape());
  const float *bias = in(b);
  PendingLinear &p = pending_linear(); // (in() runs nothing that launches it)
  p.bias = bias;
  p.bias_hold = b;
  written(o.get_storage()->data());
  remember(std::move(key.key), o);
  return true;
}

// GELU(y, g) of the product with its bias, g another tensor of y's shape:
// one launch writes y (the pre-activation) and g.
bool gelu_of_product(const Tensor &a, Tensor &o) {
  const PendingLinear &pl = pending_linear();
  if (!pl.armed || !pl.bias || !a.get_storage() || !o.get_storage() ||
      a.get_storage() != pl.o.get_storage() || o.get_storage() == a.get_storage() ||
      a.shape() != pl.o.shape() || a.strides() != pl.o.strides() || o.shape() != a.shape() ||
      !contiguous(a.shape(), a.strides()) || !contiguous(o.shape(), o.strides()) ||
      pl.c_cs != 1 || pl.c_rs != pl.N || pl.a_cs != 1 || pl.a_rs != pl.K)
    return false;
  // batch entries only as rows of one tall product: a shared right operand,
  // packed rows of the left and of the output (tlh_matmul_bias_ws refuses
  // other batches with a GELU)
  uint64_t rows = pl.M;
  for (size_t i = pl.batch.shape.size(); i-- > 0;) {
    if (pl.batch.sb[i] != 0 || pl.batch.sa[i] != rows * pl.K || pl.batch.sc[i] != rows * pl.N)
      return false;
    rows *= pl.batch.shape[i];
  }
  if (rows > 0x7fffffffu) return false;
  // (g must not be a block the product reads: one launch reads and writes)
  const auto *g_store = o.get_storage();
  if (g_store == pl.a_hold.get_storage() || g_store == pl.b_hold.get_storage() ||
      g_store == pl.bias_hold.get_storage())
    return false;
  KeyBuilder key(kGelu);
  key.tensor(a).dims(o.shape());
  float *g = dest(o, {&a}); // (o is overwritten whole)
  if (!pending_linear().armed) return false; // (not reached: dest launches nothing pending)
  launch_linear(g);
  remember(std::move(key.key), o);
  return true;
}
} // namespace

void Runtime::mult(const Tensor &a, const Tensor &b, Tensor &o) {
  require_recording("mult");
  const shape_type expected = rtensor::infer_mult(a.shape(), b.shape());
  if (o.shape() != expected) throw std::invalid_argument("matmul destination has incorrect shape");
  note(kMult, o.shape());
  const size_t ra = a.shape().size(), rb = b.shape().size(), ro = o.shape().size();
  const uint32_t M = a.shape()[ra - 2], K = a.shape()[ra - 1], N = b.shape()[rb - 1];
  const std::span<const uint32_t> out_batch(o.shape().data(), ro - 2);
  const auto sa = broadcast_strides(std::span(a.shape()).first(ra - 2),
                                    std::span(a.strides()).first(ra - 2), out_batch);
  const auto sb = broadcast_strides(std::span(b.shape()).first(rb - 2),
                                    std::span(b.strides()).first(rb - 2), out_batch);
  const Batch batch =
      simplify_batch(out_batch, sa, sb, std::span(o.strides()).first(ro - 2));
  if (batch.shape.size() > 4)
    throw std::invalid_argument("matmul supports at most 4 non-mergeable batch dimensions");
  if (o.numel() == 0) return;
  if (K == 0) { // empty inner dimension: the product is all zeros
    check(tlh_fill_f32(out(o), 0.0f, o.numel(), stream()), "mult");
    return;
  }
  KeyBuilder key(kMult);
  key.tensor(a).tensor(b).dims(o.shape());
  if (reuse(key.key, o)) return;
  // the destination first (views of it are filled before it is written),
  // then the operands: a pending transpose is read through its strides
  float *dst = dest(o, {&a, &b});
  Operand oa = operand(a, true), ob = operand(b, true);
  Batch vb = simplify_batch(
      out_batch,
      broadcast_strides(std::span(a.shape()).first(ra - 2), std::span(oa.strides).first(ra - 2),
                        out_batch),
      broadcast_strides(std::span(b.shape()).first(rb - 2), std::span(ob.strides).first(rb - 2),
                        out_batch),
      std::span(o.strides()).first(ro - 2));
  if (vb.shape.size() > 4) { // the views' batch dims do not merge: fill them
    oa = {in(a), a.strides(), &a};
    ob = {in(b), b.strides(), &b};
    vb = batch;
  }
  const uint32_t a_rs = oa.strides[ra - 2], a_cs = oa.strides[ra - 1];
  const uint32_t b_rs = ob.strides[rb - 2], b_cs = ob.strides[rb - 1];
  const uint32_t c_rs = o.strides()[ro - 2], c_cs = o.strides()[ro - 1];
  const uint32_t nb = uint32_t(vb.shape.size());
  size_t ws_elems = 0;
  check(tlh_matmul_workspace_size(M, K, N, a_rs, a_cs, b_rs, b_cs, c_rs, c_cs, nb,
                                  vb.shape.data(), vb.sa.data(), vb.sb.data(), vb.sc.data(),
                                  &ws_elems),
        "mult");
  // A batched product whose batch entries continue its inner dimension in
  // both operands (entry i+1 starts where entry i's K run would go on) is
  // kept pending: a following sum over the batch becomes one product over
  // K * entries (see sum_to_shape). Only products that need no scratch and
  // write a contiguous destination that no operand shares are deferred.
  const auto chains = [&](const std::vector<uint32_t> &st, uint64_t k_stride) {
    for (size_t i = nb; i-- > 0;) {
      if (st[i] != k_stride) return false;
      k_stride *= vb.shape[i];
    }
    return true;
  };
  const auto *os = o.get_storage();
  if (nb > 0 && ws_elems == 0 && contiguous(o.shape(), o.strides()) &&
      chains(vb.sa, uint64_t(K) * a_cs) && chains(vb.sb, uint64_t(K) * b_rs) &&
      oa.holder->get_storage() != os && ob.holder->get_storage() != os &&
      oa.ptr == oa.holder->get_storage()->data() && ob.ptr == ob.holder->get_storage()->data()) {
    auto plan = std::make_shared<ProductPlan>(
        ProductPlan{*ob.holder, M, K, N, a_rs, a_cs, b_rs, b_cs, vb.shape, vb.sa, vb.sb, vb.sc});
    put_view(dst, PendingView{*oa.holder, o.shape(), o.strides(), std::move(plan)});
    remember(std::move(key.key), o);
    return;
  }
  // launched by the next call (see pending_linear)
  pending_linear() = PendingLinear{true,  *oa.holder, *ob.holder, o,    oa.ptr, ob.ptr,
                                   dst,   M,          K,          N,    a_rs,   a_cs,
                                   b_rs,  b_cs,       c_rs,       c_cs, vb,     ws_elems};
  remember(std::move(key.key), o);
}

// Swap of two dims (runtime.cpp:529-569): a view of `a` filled on demand.
void Runtime::transpose(const Tensor &a, Tensor &o, int32_t dim_a, int32_t dim_b) {
  require_recording("transpose");
  if (a.shape().size() < 2) throw std::invalid_argument("transpose requires rank >= 2");
  const size_t x = rtensor::normalise_dimension(a.shape().size(), dim_a);
  const size_t y = rtensor::normalise_dimension(a.shape().size(), dim_b);
  if (x == y) throw std::invalid_argument("transpose dimensions must be different");
  if (o.shape() != rtensor::infer_transpose(a.shape(), dim_a, dim_b))
    throw std::invalid_argument("transpose destination has incorrect shape");
  if (a.shape().size() > 8) throw std::invalid_argument("transpose supports rank <= 8");
  note(kTranspose, o.shape());
  if (o.numel() == 0) return;
  shape_type strides = a.strides();
  std::swap(strides[x], strides[y]);
  if (a.get_storage() != o.get_storage()) {
    // kept as a strided view of `a` until something needs o's bytes
    std::vector<size_t> perm(a.shape().size());
    std::iota(perm.begin(), perm.end(), size_t(0));
    std::swap(perm[x], perm[y]);
    defer_view(a, o, perm);
    return;
  }
  float *dst = out(o); // destinations before sources throughout (see `in`)
  check(tlh_transpose(in(a), dst, uint32_t(o.shape().size()), o.shape().data(), strides.data(),
                      stream()),
        "transpose");
}

// The Metal runtime copies a contiguous view into the destination
// (runtime.cpp:571-593); the bytes do not move, so this is one device copy.
void Runtime::split_last_dim(const Tensor &a, Tensor &o, uint32_t outer, uint32_t inner) {
  require_recording("split_last_dim");
  if (o.shape() != rtensor::infer_split_last_dim(a.shape(), outer, inner))
    throw std::invalid_argument("split_last_dim destination has incorrect shape");
  note(kSplit, o.shape());
  // A reshape of contiguous data: the destination becomes a view of `a`, as
  // the reference CPU runtime does (CPU/runtime.h:53-63), instead of a copy.
  const std::vector<uint32_t> shape = o.shape();
  o = a.view(shape);
}

void Runtime::merge_last_dims(const Tensor &a, Tensor &o, uint32_t outer, uint32_t inner) {
  require_recording("merge_last_dims");
  if (o.shape() != rtensor::infer_merge_last_dims(a.shape(), outer, inner))
    throw std::invalid_argument("merge_last_dims destination has incorrect shape");
  note(kMerge, o.shape());
  const std::vector<uint32_t> shape = o.shape(); // a view of `a` (CPU/runtime.h:65-75)
  o = a.view(shape);
}

// ---- reductions ----------------------------------------------------------------

void Runtime::sum(const Tensor &a, Tensor &o) { // runtime.cpp:506-518
  require_recording("sum");
  if (o.numel() != 1) throw std::invalid_argument("sum destination must hold one element");
  note(kSum, a.shape());
  KeyBuilder key(kSum);
  key.tensor(a).dims(o.shape());
  cached(key, o, {&a},
         [&](float *dst) { check(tlh_sum(in(a), a.numel(), dst, stream()), "sum"); });
}

void Runtime::sum(const Tensor &a, size_t axis, Tensor &o) { // runtime.cpp:520-527
  require_recording("sum");
  if (axis >= a.shape().size()) throw std::out_of_range("sum axis out of range");
  sum_to_shape(a, o.shape(), o);
}

// runtime.cpp:661-739: reduce every dim where the (right-aligned) target is
// 1 and the input is not; leading dims beyond the target's rank are reduced
// away; no reduced dim means a copy.
void Runtime::sum_to_shape(const Tensor &a, std::span<const uint32_t> shape, Tensor &o) {
  require_recording("sum_to_shape");
  const auto &as = a.shape();
  if (shape.size() > as.size())
    throw std::invalid_argument("cannot reduce to a shape with a higher rank");
  if (o.shape().size() != shape.size() || !std::equal(shape.begin(), shape.end(), o.shape().begin()))
    throw std::invalid_argument("sum_to_shape destination has incorrect shape");
  shape_type aligned(as.size(), 1);
  std::copy(shape.begin(), shape.end(), aligned.begin() + (as.size() - shape.size()));
  bool reduces = false;
  for (size_t i = 0; i < as.size(); ++i) {
    if (as[i] == aligned[i]) continue;
    if (aligned[i] != 1) throw std::invalid_argument("invalid reduce_to_shape");
    reduces = true;
  }
  if (as.size() > 8) throw std::invalid_argument("sum_to_shape supports rank <= 8");
  note(kSumToShape, o.shape());
  if (a.numel() == 0) {
    if (o.numel()) check(tlh_fill_f32(out(o), 0.0f, o.numel(), stream()), "sum_to_shape");
    return;
  }
  if (!reduces) {
    // the same elements in the same order: a view of `a`
    if (a.get_storage() != o.get_storage() && o.numel() > 0) defer_reshape(a, o);
    return;
  }
  KeyBuilder key(kSumToShape);
  key.tensor(a).dims(o.shape());
  if (reuse(key.key, o)) return;
  reduce_to(a, aligned, o);
  remember(std::move(key.key), o);
}

// The reducing part of sum_to_shape (`aligned`: the target right-aligned to
// a's rank).
void Runtime::reduce_to(const Tensor &a, const std::vector<uint32_t> &aligned, Tensor &o) {
  const auto &as = a.shape();
  // The sum over every batch dim of a pending batched product whose entries
  // chain into K: one product over K * entries, written straight into o.
  // `a` stays pending (its sources are unchanged).
  if (const auto it = pending_views().find(a.get_storage()->data());
      it != pending_views().end() && it->second.product && it->second.shape == as &&
      a.get_storage() != o.get_storage() && it->second.source.get_storage() != o.get_storage() &&
      it->second.product->b.get_storage() != o.get_storage()) {
    const size_t r = as.size();
    bool batch_only = aligned[r - 2] == as[r - 2] && aligned[r - 1] == as[r - 1];
    for (size_t i = 0; i + 2 < r; ++i) batch_only = batch_only && aligned[i] == 1;
    if (batch_only) {
      const PendingView v = it->second; // holds the sources until the launch
      const ProductPlan &p = *v.product;
      uint64_t k = p.K;
      for (const uint32_t d : p.batch) k *= d;
      if (k <= UINT32_MAX) {
        float *dst = dest(o, {&a});
        const Batch none;
        size_t ws_elems = 0;
        check(tlh_matmul_workspace_size(p.M, uint32_t(k), p.N, p.a_rs, p.a_cs, p.b_rs, p.b_cs,
                                        p.N, 1, 0, nullptr, nullptr, nullptr, nullptr, &ws_elems),
              "sum_to_shape");
        run_product(v.source.get_storage()->data(), p.b.get_storage()->data(), dst, p.M,
                    uint32_t(k), p.N, p.a_rs, p.a_cs, p.b_rs, p.b_cs, p.N, 1, none, ws_elems);
        return;
      }
    }
  }
  size_t ws_elems = 0;
  check(tlh_sum_to_shape_workspace(uint32_t(as.size()), as.data(), aligned.data(), &ws_elems),
        "sum_to_shape");
  float *dst = dest(o, {&a});
  if (ws_elems == 0) {
    check(tlh_sum_to_shape(in(a), dst, uint32_t(as.size()), as.data(), aligned.data(), stream()),
          "sum_to_shape");
    return;
  }
  // Row-chunk partials of a tall column sum, returned to the pool on exit
  // (stream-ordered reuse; held back while a graph is being captured).
  Tensor partials({uint32_t(ws_elems)});
  check(tlh_sum_to_shape_ws(in(a), dst, uint32_t(as.size()), as.data(), aligned.data(),
                            out(partials), ws_elems, stream()),
        "sum_to_shape");
}

// reduce_to_shape with the max kernel (runtime.cpp:595-659, 741-745): same
// rank, at most one shrinking dim; nothing to shrink aliases the input.
void Runtime::max_to_shape(const Tensor &a, std::span<const uint32_t> shape, Tensor &o) {
  require_recording("max_to_shape");
  const auto &as = a.shape();
  if (shape.size() != as.size()) throw std::invalid_argument("cannot reduce to shape if ranks differ");
  size_t shrinking = 0;
  for (size_t i = 0; i < as.size(); ++i) {
    if (as[i] == shape[i]) continue;
    if (shape[i] != 1) throw std::invalid_argument("invalid reduce_to_shape");
    if (++shrinking > 1)
      throw std::invalid_argument("reduce_to_shape currently supports only one shrinking dimension");
  }
  if (shrinking == 0) {
    o = a;
    return;
  }
  if (o.shape().size() != shape.size() || !std::equal(shape.begin(), shape.end(), o.shape().begin()))
    throw std::invalid_argument("max_to_shape destination has incorrect shape");
  if (as.size() > 8) throw std::invalid_argument("max_to_shape supports rank <= 8");
  note(kMaxToShape, o.shape());
  if (o.numel() == 0) return;
  float *dst = out(o);
  check(tlh_max_to_shape(in(a), dst, uint32_t(as.size()), as.data(), shape.data(), stream()),
        "max_to_shape");
}

// Index of the first maximum (runtime.cpp:850-918).
void Runtime::argmax(const Tensor &a, IndexTensor &o) {
  require_recording("argmax");
  if (a.numel() == 0) throw std::invalid_argument("argmax requires a non-empty tensor");
  if (o.numel() != 1) throw std::invalid_argument("argmax destination must hold one index");
  note(kArgmax, a.shape());
  uint32_t *dst = out(o);
  check(tlh_argmax(in(a), a.numel(), dst, stream()), "argmax");
}

// ---- row ops -----------------------------------------------------------------------

void Runtime::softmax(const Tensor &x, Tensor &o) { // runtime.cpp:747-766
  require_recording("softmax");
  const Rows r = as_rows(x, "softmax");
  if (o.shape() != x.shape()) throw std::invalid_argument("softmax destination has incorrect shape");
  note(kSoftmax, o.shape());
  if (r.rows == 0) return;
  KeyBuilder key(kSoftmax);
  key.tensor(x);
  cached(key, o, {&x},
         [&](float *dst) { check(tlh_softmax(in(x), dst, r.rows, r.cols, stream()), "softmax"); });
}

void Runtime::cross_entropy(const Tensor &logits, const IndexTensor &targets, Tensor &o) {
  require_recording("cross_entropy"); // runtime.cpp:768-804
  const shape_type expected = rtensor::infer_cross_entropy(logits.shape(), targets.shape());
  if (o.shape() != expected)
    throw std::invalid_argument("cross_entropy destination must match target shape with a "
                                "trailing singleton dimension");
  note(kCrossEntropy, logits.shape());
  const Rows r = as_rows(logits, "cross_entropy");
  if (r.rows == 0) return;
  KeyBuilder key(kCrossEntropy);
  key.tensor(logits).tensor(targets).dims(o.shape());
  cached(key, o, {&logits}, [&](float *dst) {
    check(tlh_cross_entropy_rows(in(logits), in(targets), dst, r.rows, r.cols, stream()),
          "cross_entropy");
  });
}

void Runtime::cross_entropy_derivative(const Tensor &logits, const IndexTensor &targets,
                                       Tensor &o) { // runtime.cpp:806-841
  require_recording("cross_entropy_derivative");
  (void)rtensor::infer_cross_entropy(logits.shape(), targets.shape());
  if (o.shape() != logits.shape())
    throw std::invalid_argument("cross_entropy_derivative destination must match logits shape");
  note(kCrossEntropyDerivative, o.shape());
  const Rows r = as_rows(logits, "cross_entropy_derivative");
  if (r.rows == 0) return;
  KeyBuilder key(kCrossEntropyDerivative);
  key.tensor(logits).tensor(targets);
  cached(key, o, {&logits}, [&](float *dst) {
    check(tlh_cross_entropy_rows_backward(in(logits), in(targets), dst, r.rows, r.cols, nullptr,
                                          stream()),
          "cross_entropy_derivative");
  });
}

void Runtime::RMS(const Tensor &a, Tensor &o) { // runtime.cpp:1031-1058
  require_recording("RMS");
  RMS_impl(a, o);
}

void Runtime::RMS_impl(const Tensor &a, Tensor &o) {
  if (a.shape().empty()) throw std::invalid_argument("RMS requires rank >= 1");
  if (o.shape() != rtensor::infer_rms(a.shape()))
    throw std::invalid_argument("RMS destination has incorrect shape");
  note(kRms, a.shape());
  if (a.numel() == 0) return;
  KeyBuilder key(kRms);
  key.tensor(a);
  cached(key, o, {&a}, [&](float *dst) {
    check(tlh_rms(in(a), dst, a.numel() / a.shape().back(), a.shape().back(), kRmsEpsilon,
                  stream()),
          "RMS");
  });
}

void Runtime::RMSNorm(const Tensor &a, Tensor &o) { // runtime.cpp:1060-1072
  require_recording("RMSNorm");
  if (o.shape() != a.shape()) throw std::invalid_argument("RMSNorm destination has incorrect shape");
  if (a.shape().empty()) throw std::invalid_argument("RMSNorm requires rank >= 1");
  note(kRmsNorm, a.shape());
  if (a.numel() == 0) return;
  KeyBuilder key(kRmsNorm);
  key.tensor(a);
  cached(key, o, {&a}, [&](float *dst) {
    check(tlh_rms_norm(in(a), nullptr, dst, nullptr, a.numel() / a.shape().back(),
                       a.shape().back(), kRmsEpsilon, stream()),
          "RMSNorm");
  });
}

// ---- embedding (runtime.cpp:920-1030) ------------------------------------------------

void Runtime::embedding_lookup(const Tensor &w, const IndexTensor &ids, Tensor &o) {
  require_recording("embedding_lookup");
  if (w.shape().size() != 2) throw std::invalid_argument("embedding weights must have rank 2");
  shape_type expected = ids.shape();
  expected.push_back(w.shape().back());
  if (o.shape() != expected) throw std::invalid_argument("embedding output shape does not match IDs");
  note(kEmbedding, o.shape());
  if (o.numel() == 0) return;
  KeyBuilder key(kEmbedding);
  key.tensor(w).tensor(ids);
  cached(key, o, {&w}, [&](float *dst) {
    check(tlh_embedding_lookup(in(w), w.shape()[0], w.shape()[1], in(ids), ids.numel(), dst,
                               stream()),
          "embedding_lookup");
  });
}

void Runtime::gather_rows(const Tensor &values, const IndexTensor &ids, Tensor &o) {
  embedding_lookup(values, ids, o);
}

namespace {
void validate_scatter(const Tensor &values, const IndexTensor &ids, const Tensor &dst) {
  if (dst.shape().size() != 2) throw std::invalid_argument("scatter destination must have rank 2");
  shape_type expected = ids.shape();
  expected.push_back(dst.shape().back());
  if (values.shape() != expected)
    throw std::invalid_argument("scatter input shape does not match IDs and embedding size");
}
void scatter(const Tensor &values, const IndexTensor &ids, Tensor &dst) {
  if (values.numel() == 0) return;
  float *d = out(dst);
  check(tlh_scatter_add_rows(in(values), in(ids), ids.numel(), dst.shape()[1], d, dst.shape()[0],
                             stream()),
        "scatter_add_rows");
}
} // namespace

void Runtime::scatter_add_rows(const Tensor &base, const IndexTensor &ids, const Tensor &values,
                               Tensor &o) {
  require_recording("scatter_add_rows");
  if (base.shape() != o.shape())
    throw std::invalid_argument("scatter base and destination shapes must match");
  validate_scatter(values, ids, o);
  note(kScatterAdd, o.shape());
  if (o.numel() && base.get_storage() != o.get_storage()) {
    float *dst = dest(o, {&base});
    check(tlh_copy(in(base), dst, o.numel(), stream()), "scatter_add_rows");
  }
  scatter(values, ids, o);
}

void Runtime::scatter_index(const Tensor &values, const IndexTensor &ids, Tensor &o) {
  require_recording("scatter_index");
  validate_scatter(values, ids, o);
  note(kScatterIndex, o.shape());
  if (o.numel()) check(tlh_fill_f32(out(o), 0.0f, o.numel(), stream()), "scatter_index");
  scatter(values, ids, o);
}

// ---- optimiser (runtime.cpp:1083-1168) -----------------------------------------------------

void Runtime::accumulate_gradient_squared_norm(const Tensor &g, Tensor &s) {
  require_recording("accumulate_gradient_squared_norm");
  if (s.numel() != 1) throw std::invalid_argument("gradient norm destination must be a scalar");
  note(kSquaredNorm, g.shape());
  if (g.numel() == 0) return;
  // collected (see pending_norms): the first call fills whatever reads or is
  // pending on s, later ones only give s a new value identity
  auto &norms = pending_norms();
  const void *sb = s.get_storage()->data();
  auto it = norms.find(sb);
  if (it == norms.end()) {
    out(s);
    it = norms.emplace(sb, PendingNorm{s, {}}).first;
  } else {
    written(sb);
  }
  it->second.grads.push_back(g);
  if (it->second.grads.size() >= 2048) flush_norm(sb); // the multi-tensor kernel's limit
}

void Runtime::clip_gradient(const Tensor &g, const Tensor &s, kernel_type max_norm, Tensor &o) {
  require_recording("clip_gradient", false);
  if (s.numel() != 1) throw std::invalid_argument("gradient norm input must be a scalar");
  if (g.shape() != o.shape())
    throw std::invalid_argument("gradient clipping input and destination shapes must match");
  if (!(max_norm > 0.0f) || !std::isfinite(max_norm))
    throw std::invalid_argument("maximum gradient norm must be finite and positive");
  note(kClip, g.shape());
  if (g.numel() == 0) return;
  // the norm first: its collection may read g's pending view
  if (s.get_storage()) settle(s.get_storage()->data());
  if (o.get_storage()) settle(o.get_storage()->data());
  // in place: the clip joins the batch (see clip_batch). A slot that is a
  // pending copy is read at the copy's source; any other pending view of g
  // is filled first. The batch runs first when this clip reads or writes a
  // block that one of its clips writes or reads, or takes another norm or
  // bound.
  if (g.get_storage() == o.get_storage() && g.strides() == o.strides() && s.get_storage()) {
    const void *gb = g.get_storage()->data();
    const auto source = [&]() -> Tensor {
      if (const PendingView *v = view_of(g); v && v->strides == g.strides()) return v->source;
      if (pending_views().count(gb)) reading(gb);
      return g;
    };
    Tensor src = source();
    ClipBatch &cb = clip_batch();
    bool fits = cb.entries.empty() ||
                (cb.s.get_storage() == s.get_storage() && cb.max_norm == max_norm &&
                 cb.entries.size() < 2048); // the multi-tensor kernel's limit
    const void *sb = src.get_storage()->data();
    for (size_t i = 0; fits && i < cb.entries.size(); ++i) {
      const void *eg = cb.entries[i].g.get_storage()->data();
      const void *es = cb.entries[i].src.get_storage()->data();
      fits = eg != gb && eg != sb && es != gb;
    }
    if (!fits) {
      flush_clips(); // (it may have filled g's copy: look again)
      src = source();
    }
    if (src.get_storage() != g.get_storage()) drop_view(gb); // every element is written
    ClipBatch &b = clip_batch();
    if (b.entries.empty()) {
      b.s = s;
      b.max_norm = max_norm;
    }
    b.entries.push_back(ClipEntry{g, std::move(src)});
    return;
  }
  flush_clips();
  // in place on a slot that still holds a copy: read the copy's source and
  // write every element of the slot, so the copy is never made
  if (const PendingView *v = view_of(g);
      v && v->strides == g.strides() && g.get_storage() == o.get_storage()) {
    PendingView copy = *v; // holds the source until the launch
    drop_view(o.get_storage()->data());
    check(tlh_clip_gradient(copy.source.get_storage()->data(), in(s), max_norm,
                            o.get_storage()->data(), g.numel(), stream()),
          "clip_gradient");
    written(o.get_storage()->data());
    return;
  }
  float *dst = dest(o, {&g, &s});
  check(tlh_clip_gradient(in(g), in(s), max_norm, dst, g.numel(), stream()), "clip_gradient");
}

void Runtime::adamW(const Tensor &p, const Tensor &g, Tensor &o, Tensor &m1, Tensor &m2,
                    const Tensor &beta1, const Tensor &beta2, const Tensor &decay,
                    const Tensor &lr, kernel_type epsilon, uint32_t step) {
  require_recording("adamW");
  if (g.shape() != p.shape() || o.shape() != p.shape() || m1.shape() != p.shape() ||
      m2.shape() != p.shape())
    throw std::invalid_argument("AdamW tensor shapes must match");
  if (beta1.numel() != 1 || beta2.numel() != 1 || decay.numel() != 1 || lr.numel() != 1)
    throw std::invalid_argument("AdamW parameters must be scalars");
  if (step == 0) throw std::invalid_argument("AdamW step must be greater than zero");
  note(kAdamW, p.shape());
  if (p.numel() == 0) return;
  const auto *bs1 = beta1.get_storage(), *bs2 = beta2.get_storage();
  const auto *ds = decay.get_storage(), *ls = lr.get_storage();
  if (o.get_storage() == p.get_storage() && bs1 && bs2 && ds && ls) {
    // in place: collected (see pending_adam)
    PendingAdam &pa = pending_adam();
    if (adam_pending() && (pa.beta1.get_storage() != bs1 || pa.beta2.get_storage() != bs2 ||
                           pa.decay.get_storage() != ds || pa.lr.get_storage() != ls ||
                           pa.eps != epsilon))
      flush_adam();
    out(o); // fills what is pending on the blocks the update writes
    out(m1);
    out(m2);
    PendingAdam &group = pending_adam(); // (the writes above may have run a group)
    if (!adam_pending()) {
      group.beta1 = beta1;
      group.beta2 = beta2;
      group.decay = decay;
      group.lr = lr;
      group.eps = epsilon;
    }
    group.entries.push_back(AdamEntry{p, g, m1, m2, step});
    for (const void *b : {static_cast<const void *>(p.get_storage()->data()),
                          static_cast<const void *>(m1.get_storage()->data()),
                          static_cast<const void *>(m2.get_storage()->data())})
      ++group.writes[b];
    for (const void *b : {static_cast<const void *>(g.get_storage()->data()),
                          static_cast<const void *>(bs1->data()),
                          static_cast<const void *>(bs2->data()),
                          static_cast<const void *>(ds->data()),
                          static_cast<const void *>(ls->data())})
      ++group.reads[b];
    if (group.entries.size() >= 2048) flush_adam(); // the multi-tensor kernel's limit
    return;
  }
  float *po = out(o), *pm1 = out(m1), *pm2 = out(m2);
  check(tlh_adamw(in(p), in(g), po, pm1, pm2, in(beta1), in(beta2), in(decay), in(lr),
                  epsilon, step, p.numel(), stream()),
        "adamW");
}

// ---- fused extensions ---------------------------------------------------------------------------

void Runtime::RMSNorm(const Tensor &a, const Tensor &gain, kernel_type epsilon, Tensor &o) {
  require_recording("RMSNorm");
  if (o.shape() != a.shape()) throw std::invalid_argument("RMSNorm destination has incorrect shape");
  const Rows r = as_rows(a, "RMSNorm");
  const bool has_gain = gain.get_storage() != nullptr;
  if (has_gain && gain.numel() != r.cols)
    throw std::invalid_argument("RMSNorm gain must have one value per column");
  note(kRmsNormGain, a.shape());
  if (r.rows == 0) return;
  KeyBuilder key(kRmsNormGain);
  key.tensor(a).tensor(gain).scalar(epsilon);
  cached(key, o, {&a, &gain}, [&](float *dst) {
    check(tlh_rms_norm(in(a), has_gain ? in(gain) : nullptr, dst, nullptr, r.rows, r.cols,
                       epsilon, stream()),
          "RMSNorm");
  });
}

void Runtime::softmax_derivative(const Tensor &grad, const Tensor &y, Tensor &o) {
  require_recording("softmax_derivative");
  if (grad.shape() != y.shape() || o.shape() != y.shape())
    throw std::invalid_argument("softmax_derivative shapes must match");
  const Rows r = as_rows(y, "softmax_derivative");
  note(kSoftmaxDerivative, y.shape());
  if (r.rows == 0) return;
  KeyBuilder key(kSoftmaxDerivative);
  key.tensor(grad).tensor(y);
  cached(key, o, {&grad, &y}, [&](float *dst) {
    check(tlh_softmax_backward(in(grad), in(y), dst, r.rows, r.cols, stream()),
          "softmax_derivative");
  });
}

void Runtime::GELU_backward(const Tensor &grad, const Tensor &x, Tensor &o) {
  require_recording("GELU_backward");
  if (grad.shape() != x.shape() || o.shape() != x.shape())
    throw std::invalid_argument("GELU_backward shapes must match");
  note(kGeluBackward, x.shape());
  if (x.numel() == 0) return;
  KeyBuilder key(kGeluBackward);
  key.tensor(grad).tensor(x);
  cached(key, o, {&grad, &x}, [&](float *dst) {
    check(tlh_gelu_backward(in(grad), in(x), dst, x.numel(), stream()), "GELU_backward");
  });
}

void Runtime::RMSNorm_derivative(const Tensor &grad, const Tensor &x, Tensor &o) {
  require_recording("RMSNorm_derivative");
  if (grad.shape() != x.shape() || o.shape() != x.shape())
    throw std::invalid_argument("RMSNorm_derivative shapes must match");
  const Rows r = as_rows(x, "RMSNorm_derivative");
  note(kRmsNormDerivative, x.shape());
  if (r.rows == 0) return;
  KeyBuilder key(kRmsNormDerivative);
  key.tensor(grad).tensor(x);
  cached(key, o, {&grad, &x}, [&](float *dst) {
    check(tlh_rms_norm_backward(in(grad), in(x), nullptr, dst, nullptr, r.rows, r.cols,
                                kRmsEpsilon, 0.0f, stream()),
          "RMSNorm_derivative");
  });
}

namespace {
struct AttentionDims {
  uint32_t b, h, t, d;
};
AttentionDims attention_dims(const Tensor &q, const Tensor &k, const Tensor &v) {
  if (q.shape().size() != 4 || k.shape() != q.shape() || v.shape() != q.shape())
    throw std::invalid_argument("attention operands must all be [B, H, T, 64]");
  const AttentionDims d{q.shape()[0], q.shape()[1], q.shape()[2], q.shape()[3]};
  if (d.d != 64) throw std::invalid_argument("attention head dimension must be 64");
  return d;
}
void require_lse(const Tensor &lse, const AttentionDims &d) {
  if (lse.numel() != size_t(d.b) * d.h * d.t)
    throw std::invalid_argument("attention log-sum-exp must hold B*H*T values");
}
} // namespace

void Runtime::causal_attention(const Tensor &q, const Tensor &k, const Tensor &v, kernel_type scale,
                               Tensor &o, Tensor &lse) {
  require_recording("causal_attention");
  const AttentionDims d = attention_dims(q, k, v);
  if (o.shape() != q.shape()) throw std::invalid_argument("attention output has incorrect shape");
  require_lse(lse, d);
  note(kAttention, q.shape());
  if (q.numel() == 0) return;
  float *po = out(o), *plse = out(lse);
  check(tlh_attention_forward(in(q), in(k), in(v), po, plse, d.b, d.h, d.t, d.d, scale, 1, 0,
                              stream()),
        "causal_attention");
}

void Runtime::causal_attention_backward(const Tensor &q, const Tensor &k, const Tensor &v,
                                        const Tensor &o, const Tensor &grad_out, const Tensor &lse,
                                        kernel_type scale, Tensor &grad_q, Tensor &grad_k,
                                        Tensor &grad_v) {
  require_recording("causal_attention_backward");
  const AttentionDims d = attention_dims(q, k, v);
  if (o.shape() != q.shape() || grad_out.shape() != q.shape() || grad_q.shape() != q.shape() ||
      grad_k.shape() != q.shape() || grad_v.shape() != q.shape())
    throw std::invalid_argument("attention gradients must match the operands' shape");
  require_lse(lse, d);
  note(kAttentionBackward, q.shape());
  if (q.numel() == 0) return;
  // Per-row dot(dO, O) workspace, returned to the pool on exit
  // (stream-ordered reuse; held back while a graph is being captured).
  Tensor delta({d.b, d.h, d.t});
  float *pd = out(delta), *pq = out(grad_q), *pk = out(grad_k), *pv = out(grad_v);
  check(tlh_attention_backward(in(q), in(k), in(v), in(o), in(grad_out), in(lse), pd, pq, pk, pv,
                               d.b, d.h, d.t, d.d, scale, 1, 0, 0, stream()),
        "causal_attention_backward");
}

} // namespace hip

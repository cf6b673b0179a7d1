// The cyclic-attention operators registered from C++: white_matter::cyclic_attn_fwd,
// cyclic_attn_bwd, cyclic_attn_doc_fwd and cyclic_attn_doc_bwd, with the names,
// argument names and output layouts of the reference's registration
// (src/white_matter/ops/cyclic_attention/_tilelang/registration.py:164-302).
//
// The model calls these operators once per (layer, residue) and pass, more
// than a thousand times per training step (registration.py:247-251), on
// problems of a few hundred microseconds of GPU work. Registering them from
// Python (torch.library.custom_op) costs about 80 us of dispatch per forward
// and 220 us per forward + backward on the host before any work of ours, so
// they are defined here: the CUDA kernels fill wmx_attn_args and call the C
// ABI of libwmx_attn.so directly, and the autograd kernel is a C++
// torch::autograd::Function whose backward calls cyclic_attn(_doc)_bwd through
// the dispatcher (so dispatch modes, the FLOP counter and selective
// checkpointing still see every operator by name).
//
// Document metadata is packed once per (metadata tensors, shapes, stride,
// residue) into varlen segments by the Python packer, reached through the
// registered operator white_matter::_cyclic_schedule on a cache miss; the
// entries hold the metadata tensors (so their identity stays a valid key) and
// their version counters (so in-place changes are seen).
#include <ATen/ATen.h>
#include <ATen/core/dispatch/Dispatcher.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/autograd.h>
#include <torch/library.h>

#include <array>
#include <cmath>
#include <cstring>
#include <list>
#include <map>
#include <memory>
#include <mutex>
#include <utility>
#include <vector>

#include "wmx_attn.h"

namespace {

using at::Tensor;
using torch::autograd::AutogradContext;
using torch::autograd::variable_list;

// ------------------------------------------------------------ operands ----
bool vector_ready(const Tensor& x) {
  if (x.stride(-1) != 1 && x.size(-1) != 1) return false;
  if (reinterpret_cast<uintptr_t>(x.data_ptr()) % 16) return false;
  for (int64_t d = 0; d + 1 < x.dim(); ++d)
    if (x.size(d) > 1 && x.stride(d) % 8) return false;
  return true;
}

// bf16 with unit head_dim stride and 16-byte aligned rows; strided views
// (cache channels, capacity padding, BQHD storage) are kept without a copy
Tensor operand(Tensor x) {
  if (x.scalar_type() != at::kBFloat16) x = x.to(at::kBFloat16);
  if (vector_ready(x)) return x;
  x = x.contiguous();
  return vector_ready(x) ? x : x.clone();
}

// [batch, head, token] element strides of a 4-D tensor; size-1 dims give 0
void strides3(const Tensor& x, int64_t (&out)[3]) {
  for (int d = 0; d < 3; ++d) out[d] = x.size(d) > 1 ? x.stride(d) : 0;
}

void check_rc(int rc, const char* what) {
  TORCH_CHECK(rc == WMX_OK, what, " failed (", rc, "): ", wmx_last_error());
}

void check_residue(int64_t stride, int64_t residue) {
  // residue -1 is the strict-past shift of residue 0
  TORCH_CHECK_VALUE(-1 <= residue && residue < stride, "cyclic residue must be in [-1, ", stride, "), got ", residue);
}

void check_shapes(const Tensor& Q, const Tensor& K, const Tensor& V) {
  TORCH_CHECK_VALUE(Q.dim() == 4 && K.dim() == 4 && K.sizes() == V.sizes() && Q.size(0) == K.size(0) &&
                        Q.size(3) == K.size(3),
                    "Q/K/V require matching batch/head_dim and K/V shapes");
  TORCH_CHECK_VALUE(Q.size(1) % K.size(1) == 0, "Q/K/V require divisible query/KV heads");
}

void check_documents(const std::array<Tensor, 4>& m, const Tensor& Q, const Tensor& K) {
  const int64_t lens[4] = {Q.size(2), K.size(2), Q.size(2), K.size(2)};
  for (int i = 0; i < 4; ++i)
    TORCH_CHECK_VALUE(m[i].dim() == 2 && m[i].size(0) == Q.size(0) && m[i].size(1) == lens[i] &&
                          m[i].device() == Q.device(),
                      "document metadata shape/device does not match Q/K/V");
}

// ------------------------------------------------------- schedule cache ----
enum { kDocMode = 0, kEmpty = 1, kPacked = 2 };

// The metadata tensors a cache entry was built from, held weakly: an entry
// never keeps its metadata alive, and is dropped once any of them is freed
// (a weak reference keeps the TensorImpl's address reserved, so a live tensor
// never aliases a dead entry's). Version counters make in-place changes miss.
using WeakImpl = c10::weak_intrusive_ptr<c10::TensorImpl, c10::UndefinedTensorImpl>;

uint32_t version_of(const Tensor& t) { return t.unsafeGetTensorImpl()->version_counter().current_version(); }

struct MetaKey {
  std::vector<WeakImpl> refs;
  std::vector<uint32_t> versions;

  explicit MetaKey(const std::array<Tensor, 4>& m) {
    for (const Tensor& t : m) {
      refs.emplace_back(t.getIntrusivePtr());
      versions.push_back(version_of(t));
    }
  }
  bool expired() const {
    for (const WeakImpl& r : refs)
      if (r.expired()) return true;
    return false;
  }
  bool matches(const std::array<Tensor, 4>& m) const {
    for (size_t i = 0; i < refs.size(); ++i)
      if (refs[i]._unsafe_get_target() != m[i].unsafeGetTensorImpl() || versions[i] != version_of(m[i])) return false;
    return true;
  }
};

// A tensor in the given dtype and contiguous, or an undefined tensor when the
// input already is one (the caller then uses the input itself, so the cache
// holds no strong reference to it).
Tensor converted(const Tensor& t, at::ScalarType dtype) {
  if (t.scalar_type() == dtype && t.is_contiguous()) return Tensor();
  return t.to(dtype).contiguous();
}

const Tensor& either(const Tensor& own, const Tensor& given) { return own.defined() ? own : given; }

// Most-recently-used list of shared entries, bounded in count; every lookup
// drops the entries whose metadata was freed.
template <typename Entry>
struct WeakCache {
  std::mutex mutex;
  std::list<std::shared_ptr<Entry>> entries;
  static constexpr size_t kMaxEntries = 256;

  template <typename Same>
  std::shared_ptr<Entry> find(const std::array<Tensor, 4>& m, Same&& same) {
    std::lock_guard<std::mutex> lock(mutex);
    for (auto it = entries.begin(); it != entries.end();) {
      if ((*it)->key.expired()) {
        it = entries.erase(it);
        continue;
      }
      if (same(**it) && (*it)->key.matches(m)) {
        auto hit = *it;
        if (it != entries.begin()) entries.splice(entries.begin(), entries, it);
        return hit;
      }
      ++it;
    }
    return nullptr;
  }
  void insert(std::shared_ptr<Entry> e) {
    std::lock_guard<std::mutex> lock(mutex);
    entries.push_front(std::move(e));
    while (entries.size() > kMaxEntries) entries.pop_back();
  }
  int64_t size() {
    std::lock_guard<std::mutex> lock(mutex);
    for (auto it = entries.begin(); it != entries.end();) it = (*it)->key.expired() ? entries.erase(it) : std::next(it);
    return (int64_t)entries.size();
  }
  void clear() {
    std::lock_guard<std::mutex> lock(mutex);
    entries.clear();
  }
};

struct Schedule {
  MetaKey key;  // the metadata tensors the entry was built from
  int64_t q_len, k_len, stride, offset;
  int status = kDocMode;
  // packed segments (status kPacked), see wmx_attn_args
  Tensor qi, ki, cu_q, cu_k, q_units, k_units, ds_offsets;
  // the fused backward's segments and the other backward kernels' lists
  // without them (wmx_attn_args f_units, q_units, k_units)
  Tensor f_units, bq_units, bk_units;
  int64_t num_segments = 0, max_q = 0, max_k = 0, layout = 0, keys_unique = 1, ds_elements = 0, key_tile = 0;
  // int32 contiguous copies of the document arrays that were not (status kDocMode)
  std::array<Tensor, 4> docs;

  explicit Schedule(const std::array<Tensor, 4>& m) : key(m) {}
};

WeakCache<Schedule> g_cyclic_cache;

// The packed schedule of these metadata tensors at this stride and residue
// offset, built on a miss by the Python packer
// (white_matter::_cyclic_schedule: [facts, query_indices, key_indices,
// cu_queries, cu_keys, q_units, k_units, ds_offsets, f_units, bq_units,
// bk_units], facts = int64 CPU {status, num_segments, max_queries, max_keys,
// segment_layout, keys_unique, ds_elements, key_tile}).
std::shared_ptr<Schedule> schedule_for(const std::array<Tensor, 4>& m, int64_t q_len, int64_t k_len, int64_t stride,
                                       int64_t offset) {
  auto same = [&](const Schedule& s) {
    return s.q_len == q_len && s.k_len == k_len && s.stride == stride && s.offset == offset;
  };
  if (auto hit = g_cyclic_cache.find(m, same)) return hit;
  static auto packer = c10::Dispatcher::singleton()
                           .findSchemaOrThrow("white_matter::_cyclic_schedule", "")
                           .typed<std::vector<Tensor>(const Tensor&, const Tensor&, const Tensor&, const Tensor&,
                                                      int64_t, int64_t, int64_t, int64_t)>();
  auto s = std::make_shared<Schedule>(m);
  s->q_len = q_len;
  s->k_len = k_len;
  s->stride = stride;
  s->offset = offset;
  std::vector<Tensor> built;
  {
    at::AutoDispatchBelowADInplaceOrView below;
    built = packer.call(m[0], m[1], m[2], m[3], q_len, k_len, stride, offset);
  }
  TORCH_CHECK(!built.empty() && built[0].numel() == 8, "_cyclic_schedule returned an unexpected result");
  const Tensor facts = built[0].to(at::kLong).contiguous();
  const int64_t* f = facts.data_ptr<int64_t>();
  s->status = (int)f[0];
  if (s->status == kPacked) {
    TORCH_CHECK(built.size() == 11, "_cyclic_schedule returned an unexpected result");
    s->num_segments = f[1];
    s->max_q = f[2];
    s->max_k = f[3];
    s->layout = f[4];
    s->keys_unique = f[5];
    s->ds_elements = f[6];
    s->key_tile = f[7];
    s->qi = built[1].contiguous();
    s->ki = built[2].contiguous();
    s->cu_q = built[3].to(at::kInt).contiguous();
    s->cu_k = built[4].to(at::kInt).contiguous();
    s->q_units = built[5].to(at::kInt).contiguous();
    s->k_units = built[6].to(at::kInt).contiguous();
    s->ds_offsets = built[7].to(at::kLong).contiguous();
    s->f_units = built[8].to(at::kInt).contiguous();
    s->bq_units = built[9].to(at::kInt).contiguous();
    s->bk_units = built[10].to(at::kInt).contiguous();
  } else if (s->status == kDocMode) {
    for (int i = 0; i < 4; ++i) s->docs[i] = converted(m[i], at::kInt);
  }
  g_cyclic_cache.insert(s);
  return s;
}

// --------------------------------------------------------- launch glue ----
// The fused short-segment backward loads consecutive query and key slots as
// strided tiles: both layout bits, and token strides of at least head_dim and
// below 2^23 elements (as wmx_attn_bwd checks).
bool fused_fits(const wmx_attn_args& a) {
  auto fits = [&](const int64_t* st) { return st[2] >= a.head_dim && st[2] < (int64_t(1) << 23); };
  return (a.segment_layout & 3) == 3 && fits(a.q_stride) && fits(a.k_stride) && fits(a.v_stride) && fits(a.do_stride);
}

void fill_common(wmx_attn_args& a, const Tensor& q, const Tensor& k, const Tensor& v, const Tensor& o, const Tensor& lse,
                 double scale) {
  a.q = q.data_ptr();
  a.k = k.data_ptr();
  a.v = v.data_ptr();
  a.o = o.data_ptr();
  a.lse = lse.data_ptr<float>();
  strides3(q, a.q_stride);
  strides3(k, a.k_stride);
  strides3(v, a.v_stride);
  strides3(o, a.o_stride);
  a.batch = (int32_t)q.size(0);
  a.q_heads = (int32_t)q.size(1);
  a.kv_heads = (int32_t)k.size(1);
  a.q_len = (int32_t)q.size(2);
  a.kv_len = (int32_t)k.size(2);
  a.head_dim = (int32_t)q.size(3);
  a.softmax_scale = (float)scale;
}

// Visibility: packed segments (query_offset unused), document arrays, or the
// plain strided bound.
void fill_visibility(wmx_attn_args& a, const Schedule* s, const std::array<Tensor, 4>* meta, int64_t stride,
                     int64_t residue, const Tensor& q, const Tensor& k, bool backward) {
  a.query_stride = (int32_t)stride;
  a.query_offset = (int32_t)residue;
  if (!s) return;
  if (s->status == kPacked) {
    a.query_indices = s->qi.data_ptr<int64_t>();
    a.key_indices = s->ki.data_ptr<int64_t>();
    a.cu_queries = s->cu_q.data_ptr<int32_t>();
    a.cu_keys = s->cu_k.data_ptr<int32_t>();
    a.num_segments = (int32_t)s->num_segments;
    a.max_queries = (int32_t)s->max_q;
    a.max_keys = (int32_t)s->max_k;
    a.query_extent = (int32_t)q.size(2);
    a.key_extent = (int32_t)k.size(2);
    a.keys_unique = (int32_t)s->keys_unique;
    a.segment_layout = (int32_t)s->layout;
    a.q_units = s->q_units.data_ptr<int32_t>();
    a.num_q_units = (int32_t)s->q_units.size(0);
    a.k_units = s->k_units.data_ptr<int32_t>();
    a.num_k_units = (int32_t)s->k_units.size(0);
    TORCH_CHECK(s->q_units.size(1) == s->k_units.size(1), "q_units and k_units must have entries of one width");
    a.unit_fields = (int32_t)s->q_units.size(1);
    a.key_tile = (int32_t)s->key_tile;
    if (backward) {
      a.ds_offsets = s->ds_offsets.data_ptr<int64_t>();
      a.ds_elements = s->ds_elements;
      if (s->f_units.defined() && s->f_units.size(0) > 0 && q.size(1) == k.size(1) &&
          s->f_units.size(1) == WMX_UNIT_FIELDS && a.unit_fields == WMX_UNIT_FIELDS) {
        // short segments through the fused kernel; the tiled kernels take the
        // rest (an empty list still passes a valid pointer, with count 0)
        a.f_units = s->f_units.data_ptr<int32_t>();
        a.num_f_units = (int32_t)s->f_units.size(0);
        a.q_units = s->bq_units.numel() ? s->bq_units.data_ptr<int32_t>() : a.f_units;
        a.num_q_units = (int32_t)s->bq_units.size(0);
        a.k_units = s->bk_units.numel() ? s->bk_units.data_ptr<int32_t>() : a.f_units;
        a.num_k_units = (int32_t)s->bk_units.size(0);
      }
    }
  } else if (s->status == kDocMode) {
    a.q_seg = either(s->docs[0], (*meta)[0]).data_ptr<int32_t>();
    a.k_seg = either(s->docs[1], (*meta)[1]).data_ptr<int32_t>();
    a.q_start = either(s->docs[2], (*meta)[2]).data_ptr<int32_t>();
    a.k_qend = either(s->docs[3], (*meta)[3]).data_ptr<int32_t>();
  }
}

hipStream_t stream_of(const Tensor& t) { return c10::hip::getCurrentHIPStream(t.device().index()).stream(); }

std::tuple<Tensor, Tensor> forward_impl(const Tensor& Q, const Tensor& K, const Tensor& V,
                                        const std::array<Tensor, 4>* meta, int64_t stride, int64_t residue) {
  check_residue(stride, residue);
  check_shapes(Q, K, V);
  c10::OptionalDeviceGuard guard(Q.device());
  const Tensor q = operand(Q), k = operand(K), v = operand(V);
  const int64_t batch = Q.size(0), heads = Q.size(1), length = Q.size(2), dim = Q.size(3);
  std::shared_ptr<Schedule> s;
  if (meta) {
    check_documents(*meta, Q, K);
    s = schedule_for(*meta, length, K.size(2), stride, residue);
  }
  // (B, Tq, H, D) storage exposed as a (B, H, Tq, D) view
  Tensor out = at::empty({batch, length, heads, dim}, q.options()).transpose(1, 2);
  Tensor lse = at::empty({batch, heads, length}, q.options().dtype(at::kFloat));
  if (s && s->status == kEmpty) {
    out.zero_();
    lse.fill_(INFINITY);
  } else {
    wmx_attn_args a;
    std::memset(&a, 0, sizeof(a));
    fill_common(a, q, k, v, out, lse, std::pow((double)dim, -0.5));
    fill_visibility(a, s.get(), meta, stride, residue, q, k, false);
    check_rc(wmx_attn_fwd(&a, stream_of(q)), "wmx_attn_fwd");
  }
  if (Q.scalar_type() != at::kBFloat16) out = out.to(Q.scalar_type());
  return {out, lse};
}

std::tuple<Tensor, Tensor, Tensor> backward_impl(const Tensor& Q, const Tensor& K, const Tensor& V,
                                                 const std::array<Tensor, 4>* meta, const Tensor& Out, const Tensor& Lse,
                                                 const Tensor& dOut, int64_t stride, int64_t residue) {
  check_residue(stride, residue);
  check_shapes(Q, K, V);
  TORCH_CHECK_VALUE(Out.sizes() == Q.sizes() && dOut.sizes() == Q.sizes() && Lse.dim() == 3 &&
                        Lse.size(0) == Q.size(0) && Lse.size(1) == Q.size(1) && Lse.size(2) == Q.size(2),
                    "Out/dOut/Lse do not match Q");
  c10::OptionalDeviceGuard guard(Q.device());
  const Tensor q = operand(Q), k = operand(K), v = operand(V), o = operand(Out), g = operand(dOut);
  const Tensor lse = Lse.to(at::kFloat).contiguous();
  std::shared_ptr<Schedule> s;
  if (meta) {
    check_documents(*meta, Q, K);
    s = schedule_for(*meta, Q.size(2), K.size(2), stride, residue);
  }
  Tensor dq = at::empty(q.sizes(), q.options());
  Tensor dk = at::empty(k.sizes(), k.options());
  Tensor dv = at::empty(v.sizes(), v.options());
  if (s && s->status == kEmpty) {
    dq.zero_();
    dk.zero_();
    dv.zero_();
  } else {
    Tensor delta = at::empty(lse.sizes(), lse.options());
    wmx_attn_args a;
    std::memset(&a, 0, sizeof(a));
    fill_common(a, q, k, v, o, lse, std::pow((double)Q.size(3), -0.5));
    fill_visibility(a, s.get(), meta, stride, residue, q, k, true);
    a.dout = g.data_ptr();
    a.delta = delta.data_ptr<float>();
    strides3(g, a.do_stride);
    a.dq = dq.data_ptr();
    a.dk = dk.data_ptr();
    a.dv = dv.data_ptr();
    strides3(dq, a.dq_stride);
    strides3(dk, a.dk_stride);
    strides3(dv, a.dv_stride);
    if (a.f_units && !fused_fits(a)) {
      // the tiled kernels for every segment
      a.f_units = nullptr;
      a.num_f_units = 0;
      a.q_units = s->q_units.data_ptr<int32_t>();
      a.num_q_units = (int32_t)s->q_units.size(0);
      a.k_units = s->k_units.data_ptr<int32_t>();
      a.num_k_units = (int32_t)s->k_units.size(0);
    }
    const int64_t need = wmx_attn_bwd_workspace_size(&a);
    Tensor workspace;
    if (need > 0) {
      workspace = at::empty({need}, q.options().dtype(at::kByte));
      a.workspace = workspace.data_ptr();
      a.workspace_bytes = need;
    }
    check_rc(wmx_attn_bwd(&a, stream_of(q)), "wmx_attn_bwd");
  }
  // contiguous, in Q's dtype (the reference's fake: registration.py:199-212)
  if (Q.scalar_type() != at::kBFloat16) {
    dq = dq.to(Q.scalar_type());
    dk = dk.to(Q.scalar_type());
    dv = dv.to(Q.scalar_type());
  }
  return {dq, dk, dv};
}

// ------------------------------------------------------- CUDA kernels ----
std::tuple<Tensor, Tensor> cyclic_attn_fwd(const Tensor& Q, const Tensor& K, const Tensor& V, int64_t K_stride,
                                           int64_t residue, int64_t block_M) {
  (void)block_M;  // schema compatibility: tiles are fixed per head_dim
  return forward_impl(Q, K, V, nullptr, K_stride, residue);
}

std::tuple<Tensor, Tensor, Tensor> cyclic_attn_bwd(const Tensor& Q, const Tensor& K, const Tensor& V, const Tensor& Out,
                                                   const Tensor& Lse, const Tensor& dOut, int64_t K_stride,
                                                   int64_t residue, int64_t block_M) {
  (void)block_M;
  return backward_impl(Q, K, V, nullptr, Out, Lse, dOut, K_stride, residue);
}

std::tuple<Tensor, Tensor> cyclic_attn_doc_fwd(const Tensor& Q, const Tensor& K, const Tensor& V, const Tensor& QSeg,
                                               const Tensor& KSeg, const Tensor& QStart, const Tensor& KQEnd,
                                               int64_t K_stride, int64_t residue, int64_t block_M) {
  (void)block_M;
  const std::array<Tensor, 4> meta = {QSeg, KSeg, QStart, KQEnd};
  return forward_impl(Q, K, V, &meta, K_stride, residue);
}

std::tuple<Tensor, Tensor, Tensor> cyclic_attn_doc_bwd(const Tensor& Q, const Tensor& K, const Tensor& V,
                                                       const Tensor& QSeg, const Tensor& KSeg, const Tensor& QStart,
                                                       const Tensor& KQEnd, const Tensor& Out, const Tensor& Lse,
                                                       const Tensor& dOut, int64_t K_stride, int64_t residue,
                                                       int64_t block_M) {
  (void)block_M;
  const std::array<Tensor, 4> meta = {QSeg, KSeg, QStart, KQEnd};
  return backward_impl(Q, K, V, &meta, Out, Lse, dOut, K_stride, residue);
}

// ------------------------------------------------------------ autograd ----
// Forward below the autograd key, saving Q/K/V (and the document tensors),
// O and LSE; the backward calls the registered backward operator.
struct CyclicFn : public torch::autograd::Function<CyclicFn> {
  static variable_list forward(AutogradContext* ctx, const Tensor& Q, const Tensor& K, const Tensor& V, int64_t K_stride,
                               int64_t residue, int64_t block_M) {
    static auto op = c10::Dispatcher::singleton()
                         .findSchemaOrThrow("white_matter::cyclic_attn_fwd", "")
                         .typed<decltype(cyclic_attn_fwd)>();
    Tensor out, lse;
    {
      at::AutoDispatchBelowADInplaceOrView below;
      std::tie(out, lse) = op.call(Q, K, V, K_stride, residue, block_M);
    }
    ctx->save_for_backward({Q, K, V, out, lse});
    ctx->saved_data["s"] = K_stride;
    ctx->saved_data["r"] = residue;
    ctx->saved_data["m"] = block_M;
    ctx->mark_non_differentiable({lse});
    ctx->set_materialize_grads(false);
    return {out, lse};
  }
  static variable_list backward(AutogradContext* ctx, variable_list grads) {
    static auto op = c10::Dispatcher::singleton()
                         .findSchemaOrThrow("white_matter::cyclic_attn_bwd", "")
                         .typed<decltype(cyclic_attn_bwd)>();
    const auto t = ctx->get_saved_variables();
    const Tensor dout = grads[0].defined() ? grads[0] : at::zeros_like(t[3]);
    auto [dq, dk, dv] = op.call(t[0], t[1], t[2], t[3], t[4], dout, ctx->saved_data["s"].toInt(),
                                ctx->saved_data["r"].toInt(), ctx->saved_data["m"].toInt());
    return {dq, dk, dv, Tensor(), Tensor(), Tensor()};
  }
};

struct CyclicDocFn : public torch::autograd::Function<CyclicDocFn> {
  static variable_list forward(AutogradContext* ctx, const Tensor& Q, const Tensor& K, const Tensor& V,
                               const Tensor& QSeg, const Tensor& KSeg, const Tensor& QStart, const Tensor& KQEnd,
                               int64_t K_stride, int64_t residue, int64_t block_M) {
    static auto op = c10::Dispatcher::singleton()
                         .findSchemaOrThrow("white_matter::cyclic_attn_doc_fwd", "")
                         .typed<decltype(cyclic_attn_doc_fwd)>();
    Tensor out, lse;
    {
      at::AutoDispatchBelowADInplaceOrView below;
      std::tie(out, lse) = op.call(Q, K, V, QSeg, KSeg, QStart, KQEnd, K_stride, residue, block_M);
    }
    ctx->save_for_backward({Q, K, V, QSeg, KSeg, QStart, KQEnd, out, lse});
    ctx->saved_data["s"] = K_stride;
    ctx->saved_data["r"] = residue;
    ctx->saved_data["m"] = block_M;
    ctx->mark_non_differentiable({lse});
    ctx->set_materialize_grads(false);
    return {out, lse};
  }
  static variable_list backward(AutogradContext* ctx, variable_list grads) {
    static auto op = c10::Dispatcher::singleton()
                         .findSchemaOrThrow("white_matter::cyclic_attn_doc_bwd", "")
                         .typed<decltype(cyclic_attn_doc_bwd)>();
    const auto t = ctx->get_saved_variables();
    const Tensor dout = grads[0].defined() ? grads[0] : at::zeros_like(t[7]);
    auto [dq, dk, dv] = op.call(t[0], t[1], t[2], t[3], t[4], t[5], t[6], t[7], t[8], dout,
                                ctx->saved_data["s"].toInt(), ctx->saved_data["r"].toInt(),
                                ctx->saved_data["m"].toInt());
    return {dq, dk, dv, Tensor(), Tensor(), Tensor(), Tensor(), Tensor(), Tensor(), Tensor()};
  }
};

std::tuple<Tensor, Tensor> cyclic_attn_fwd_autograd(const Tensor& Q, const Tensor& K, const Tensor& V,
                                                    int64_t K_stride, int64_t residue, int64_t block_M) {
  auto r = CyclicFn::apply(Q, K, V, K_stride, residue, block_M);
  return {r[0], r[1]};
}

std::tuple<Tensor, Tensor> cyclic_attn_doc_fwd_autograd(const Tensor& Q, const Tensor& K, const Tensor& V,
                                                        const Tensor& QSeg, const Tensor& KSeg, const Tensor& QStart,
                                                        const Tensor& KQEnd, int64_t K_stride, int64_t residue,
                                                        int64_t block_M) {
  auto r = CyclicDocFn::apply(Q, K, V, QSeg, KSeg, QStart, KQEnd, K_stride, residue, block_M);
  return {r[0], r[1]};
}

// ==================================================== strict operators ====
// white_matter::strict_packed_fwd/bwd (packed documents: Jacobi passes and
// packed prefill), strict_dense_fwd/bwd (per-row bounds: cached prefill,
// single-query training) and strict_decode (one query token over the KV
// pool), the kernels behind strict_causal_attention
// (reference ops/strict_causal_attention.py:338-474). The public function and
// its validation stay in Python; these operators are what it calls.

// What the kernels need beyond a packed schedule's own tensors, derived by
// the Python planner once per schedule and call shape: the covering schedule
// (the user's segments, then runs of rows no segment holds), its flags, the
// rows no segment writes and the work lists.
struct PackedPlan {
  MetaKey key;
  std::array<int64_t, 7> shape;  // max_queries, max_keys, batch, length, key_slots, heads, kv_heads
  bool covered = false;          // false: the schedule runs as given
  Tensor qi, ki, cu_q, cu_k;     // the covering schedule (or converted copies), else undefined
  Tensor out_gaps, dq_gaps, dkv_gaps, q_units, k_units, ds_offsets;
  int64_t num_segments = 0, max_q = 0, max_k = 0, layout = 0, keys_unique = 1, ds_elements = 0, key_tile = 0;

  explicit PackedPlan(const std::array<Tensor, 4>& m) : key(m) {}
};

WeakCache<PackedPlan> g_plan_cache;

// facts = int64 CPU {num_segments, max_queries, max_keys, segment_layout,
// keys_unique, ds_elements, covered, key_tile}; then query_indices, key_indices,
// cu_queries, cu_keys (of the covering schedule; the given tensors when not
// covered), out_gaps, dq_gaps, dkv_gaps, q_units, k_units, ds_offsets
std::shared_ptr<PackedPlan> packed_plan(const std::array<Tensor, 4>& m, int64_t max_queries, int64_t max_keys,
                                        const Tensor& Q, const Tensor& K) {
  const std::array<int64_t, 7> shape = {max_queries, max_keys, Q.size(0), Q.size(2), K.size(2), Q.size(1), K.size(1)};
  auto same = [&](const PackedPlan& p) { return p.shape == shape; };
  if (auto hit = g_plan_cache.find(m, same)) return hit;
  static auto planner = c10::Dispatcher::singleton()
                            .findSchemaOrThrow("white_matter::_packed_plan", "")
                            .typed<std::vector<Tensor>(const Tensor&, const Tensor&, const Tensor&, const Tensor&,
                                                       int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t)>();
  std::vector<Tensor> built;
  {
    at::AutoDispatchBelowADInplaceOrView below;
    built = planner.call(m[0], m[1], m[2], m[3], shape[0], shape[1], shape[2], shape[3], shape[4], shape[5], shape[6]);
  }
  TORCH_CHECK(built.size() == 11 && built[0].numel() == 8, "_packed_plan returned an unexpected result");
  auto p = std::make_shared<PackedPlan>(m);
  p->shape = shape;
  const Tensor facts = built[0].to(at::kLong).contiguous();
  const int64_t* f = facts.data_ptr<int64_t>();
  p->num_segments = f[0];
  p->max_q = f[1];
  p->max_k = f[2];
  p->layout = f[3];
  p->keys_unique = f[4];
  p->ds_elements = f[5];
  p->covered = f[6] != 0;
  p->key_tile = f[7];
  if (p->covered) {
    p->qi = built[1].to(at::kLong).contiguous();
    p->ki = built[2].to(at::kLong).contiguous();
    p->cu_q = built[3].to(at::kInt).contiguous();
    p->cu_k = built[4].to(at::kInt).contiguous();
  } else {  // the given tensors run as they are unless they need converting
    p->qi = converted(m[0], at::kLong);
    p->ki = converted(m[1], at::kLong);
    p->cu_q = converted(m[2], at::kInt);
    p->cu_k = converted(m[3], at::kInt);
  }
  p->out_gaps = built[5];
  p->dq_gaps = built[6];
  p->dkv_gaps = built[7];
  p->q_units = built[8].to(at::kInt).contiguous();
  p->k_units = built[9].to(at::kInt).contiguous();
  p->ds_offsets = built[10].to(at::kLong).contiguous();
  g_plan_cache.insert(p);
  return p;
}

void fill_plan(wmx_attn_args& a, const PackedPlan& p, const std::array<Tensor, 4>& m, const Tensor& q, const Tensor& k,
               bool backward) {
  a.query_stride = 1;
  a.query_offset = 0;
  a.query_indices = either(p.qi, m[0]).data_ptr<int64_t>();
  a.key_indices = either(p.ki, m[1]).data_ptr<int64_t>();
  a.cu_queries = either(p.cu_q, m[2]).data_ptr<int32_t>();
  a.cu_keys = either(p.cu_k, m[3]).data_ptr<int32_t>();
  a.num_segments = (int32_t)p.num_segments;
  a.max_queries = (int32_t)p.max_q;
  a.max_keys = (int32_t)p.max_k;
  a.query_extent = (int32_t)q.size(2);
  a.key_extent = (int32_t)k.size(2);
  a.keys_unique = (int32_t)p.keys_unique;
  a.segment_layout = (int32_t)p.layout;
  a.q_units = p.q_units.data_ptr<int32_t>();
  a.num_q_units = (int32_t)p.q_units.size(0);
  a.k_units = p.k_units.data_ptr<int32_t>();
  a.num_k_units = (int32_t)p.k_units.size(0);
  TORCH_CHECK(p.q_units.size(1) == p.k_units.size(1), "q_units and k_units must have entries of one width");
  a.unit_fields = (int32_t)p.q_units.size(1);
  a.key_tile = (int32_t)p.key_tile;
  if (backward) {
    a.ds_offsets = p.ds_offsets.data_ptr<int64_t>();
    a.ds_elements = p.ds_elements;
  }
}

void check_strict_shapes(const Tensor& Q, const Tensor& K, const Tensor& V) {
  TORCH_CHECK_VALUE(Q.dim() == 4 && K.dim() == 4 && K.sizes() == V.sizes() && Q.size(0) == K.size(0) &&
                        Q.size(3) == K.size(3) && Q.size(1) % K.size(1) == 0,
                    "Q/K/V require matching batch/head_dim and divisible heads");
}

// Zero the rows of a gradient or output that no kernel writes.
void zero_rows(const Tensor& flat, const Tensor& rows) {
  if (rows.defined() && rows.numel()) flat.index_fill_(0, rows, 0);
}

// Backward launch shared by the packed and dense operators: delta, dK/dV
// (and the dS buffer), dQ; a is filled but for the gradient fields.
void launch_backward(wmx_attn_args& a, const Tensor& q, const Tensor& g, const Tensor& dq, const Tensor& dk,
                     const Tensor& dv, const Tensor& lse) {
  Tensor delta = at::empty(lse.sizes(), lse.options());
  a.dout = g.data_ptr();
  a.delta = delta.data_ptr<float>();
  strides3(g, a.do_stride);
  a.dq = dq.data_ptr();
  a.dk = dk.data_ptr();
  a.dv = dv.data_ptr();
  strides3(dq, a.dq_stride);
  strides3(dk, a.dk_stride);
  strides3(dv, a.dv_stride);
  const int64_t need = wmx_attn_bwd_workspace_size(&a);
  Tensor workspace;
  if (need > 0) {
    workspace = at::empty({need}, q.options().dtype(at::kByte));
    a.workspace = workspace.data_ptr();
    a.workspace_bytes = need;
  }
  check_rc(wmx_attn_bwd(&a, stream_of(q)), "wmx_attn_bwd");
}

std::tuple<Tensor, Tensor> strict_packed_fwd(const Tensor& query, const Tensor& key, const Tensor& value,
                                             const Tensor& query_indices, const Tensor& key_indices,
                                             const Tensor& cu_queries, const Tensor& cu_keys, int64_t max_queries,
                                             int64_t max_keys, double scale) {
  check_strict_shapes(query, key, value);
  c10::OptionalDeviceGuard guard(query.device());
  const std::array<Tensor, 4> m = {query_indices, key_indices, cu_queries, cu_keys};
  const auto plan = packed_plan(m, max_queries, max_keys, query, key);
  const Tensor q = operand(query), k = operand(key), v = operand(value);
  const int64_t batch = q.size(0), heads = q.size(1), length = q.size(2), dim = q.size(3);
  Tensor out = at::empty({batch, length, heads, dim}, q.options());
  zero_rows(out.view({batch * length, heads * dim}), plan->out_gaps);
  Tensor lse = at::empty({batch, heads, length}, q.options().dtype(at::kFloat));
  wmx_attn_args a;
  std::memset(&a, 0, sizeof(a));
  fill_common(a, q, k, v, out.transpose(1, 2), lse, scale);
  fill_plan(a, *plan, m, q, k, false);
  check_rc(wmx_attn_fwd(&a, stream_of(q)), "wmx_attn_fwd");
  return {out, lse};
}

std::tuple<Tensor, Tensor, Tensor> strict_packed_bwd(const Tensor& query, const Tensor& key, const Tensor& value,
                                                     const Tensor& out, const Tensor& lse, const Tensor& dout,
                                                     const Tensor& query_indices, const Tensor& key_indices,
                                                     const Tensor& cu_queries, const Tensor& cu_keys,
                                                     int64_t max_queries, int64_t max_keys, double scale) {
  check_strict_shapes(query, key, value);
  c10::OptionalDeviceGuard guard(query.device());
  const std::array<Tensor, 4> m = {query_indices, key_indices, cu_queries, cu_keys};
  const auto plan = packed_plan(m, max_queries, max_keys, query, key);
  const Tensor q = operand(query), k = operand(key), v = operand(value);
  const Tensor o = operand(out.transpose(1, 2)), g = operand(dout.transpose(1, 2));
  const Tensor l = lse.to(at::kFloat).contiguous();
  const int64_t dim = q.size(3);
  Tensor dq = at::empty(q.sizes(), q.options());
  Tensor dk = at::empty(k.sizes(), k.options());
  Tensor dv = at::empty(v.sizes(), v.options());
  zero_rows(dq.view({-1, dim}), plan->dq_gaps);
  zero_rows(dk.view({-1, dim}), plan->dkv_gaps);
  zero_rows(dv.view({-1, dim}), plan->dkv_gaps);
  wmx_attn_args a;
  std::memset(&a, 0, sizeof(a));
  fill_common(a, q, k, v, o, l, scale);
  fill_plan(a, *plan, m, q, k, true);
  launch_backward(a, q, g, dq, dk, dv, l);
  return {dq, dk, dv};
}

// Dense problems: key slot j is visible to query i of row b iff
// j <= min(offset_b + i, limit_b), or j == 0 with keep_slot0, and
// key_mask[b, j] when given (offset_b = row_offset[b] or query_offset).
void fill_dense(wmx_attn_args& a, int64_t query_offset, const c10::optional<Tensor>& row_offset,
                const c10::optional<Tensor>& row_limit, const Tensor& mask, bool keep_slot0) {
  a.query_stride = 1;
  a.query_offset = (int32_t)query_offset;
  if (row_offset) a.row_offset = row_offset->data_ptr<int32_t>();
  if (row_limit) a.row_limit = row_limit->data_ptr<int32_t>();
  a.keep_slot0 = keep_slot0 ? 1 : 0;
  if (mask.defined()) {
    a.key_mask = mask.data_ptr<uint8_t>();
    a.key_mask_stride = mask.stride(0);
  }
}

c10::optional<Tensor> row_bounds(const c10::optional<Tensor>& t) {
  if (!t) return c10::nullopt;
  TORCH_CHECK_VALUE(t->scalar_type() == at::kInt, "row bounds must be int32");
  return t->contiguous();
}

Tensor mask_bytes(const c10::optional<Tensor>& key_mask) {
  if (!key_mask) return Tensor();
  return key_mask->contiguous().view(at::kByte);
}

constexpr int64_t kQueryTile = 128;

std::tuple<Tensor, Tensor> strict_dense_fwd(const Tensor& query, const Tensor& key, const Tensor& value,
                                            int64_t query_offset, const c10::optional<Tensor>& row_offset,
                                            const c10::optional<Tensor>& row_limit,
                                            const c10::optional<Tensor>& key_mask, bool keep_slot0, double scale) {
  check_strict_shapes(query, key, value);
  c10::OptionalDeviceGuard guard(query.device());
  const Tensor q = operand(query), k = operand(key), v = operand(value);
  const int64_t batch = q.size(0), heads = q.size(1), length = q.size(2), dim = q.size(3);
  const auto offsets = row_bounds(row_offset), limits = row_bounds(row_limit);
  const Tensor mask = mask_bytes(key_mask);
  Tensor out = at::empty({batch, length, heads, dim}, q.options());
  Tensor lse = at::empty({batch, heads, length}, q.options().dtype(at::kFloat));
  wmx_attn_args a;
  std::memset(&a, 0, sizeof(a));
  fill_common(a, q, k, v, out.transpose(1, 2), lse, scale);
  fill_dense(a, query_offset, offsets, limits, mask, keep_slot0);
  // a chunk of queries after a long cached prefix: 256-row workgroups read
  // each key/value tile once for twice the rows (the prefix dominates)
  const int64_t tile = length > kQueryTile && k.size(2) >= 4 * length ? 256 : kQueryTile;
  a.query_tile = tile == 256 ? 256 : 0;
  Tensor units;
  if (offsets || limits) {
    // ragged rows (cached prefixes): the heaviest tiles first, listed by one kernel
    units = at::empty({batch * ((length + tile - 1) / tile), 2}, q.options().dtype(at::kInt));
    check_rc(wmx_dense_units(&a, units.data_ptr<int32_t>(), stream_of(q)), "wmx_dense_units");
    a.q_units = units.data_ptr<int32_t>();
    a.num_q_units = (int32_t)units.size(0);
  }
  check_rc(wmx_attn_fwd(&a, stream_of(q)), "wmx_attn_fwd");
  return {out, lse};
}

std::tuple<Tensor, Tensor, Tensor> strict_dense_bwd(const Tensor& query, const Tensor& key, const Tensor& value,
                                                    const Tensor& out, const Tensor& lse, const Tensor& dout,
                                                    int64_t query_offset, const c10::optional<Tensor>& row_offset,
                                                    const c10::optional<Tensor>& row_limit,
                                                    const c10::optional<Tensor>& key_mask, bool keep_slot0,
                                                    double scale) {
  check_strict_shapes(query, key, value);
  c10::OptionalDeviceGuard guard(query.device());
  const Tensor q = operand(query), k = operand(key), v = operand(value);
  const Tensor o = operand(out.transpose(1, 2)), g = operand(dout.transpose(1, 2));
  const Tensor l = lse.to(at::kFloat).contiguous();
  const auto offsets = row_bounds(row_offset), limits = row_bounds(row_limit);
  const Tensor mask = mask_bytes(key_mask);
  Tensor dq = at::empty(q.sizes(), q.options());
  Tensor dk = at::empty(k.sizes(), k.options());
  Tensor dv = at::empty(v.sizes(), v.options());
  wmx_attn_args a;
  std::memset(&a, 0, sizeof(a));
  fill_common(a, q, k, v, o, l, scale);
  fill_dense(a, query_offset, offsets, limits, mask, keep_slot0);
  launch_backward(a, q, g, dq, dk, dv, l);
  return {dq, dk, dv};
}

// The split-merge counters of wmx_decode per (device, stream): zero when
// created, left zero by every launch (the last split of a (row, KV head)
// resets its counter), so calls in order on one stream share them. Buffers are
// kept for the life of the process, also when a larger one replaces them: a
// captured graph may hold their addresses.
struct DecodeCounters {
  std::mutex mutex;
  std::map<std::pair<int, hipStream_t>, std::vector<Tensor>> by_stream;

  int32_t* get(const Tensor& like, hipStream_t stream, int64_t count) {
    std::lock_guard<std::mutex> lock(mutex);
    auto& kept = by_stream[{(int)like.get_device(), stream}];
    if (kept.empty() || kept.back().numel() < count)
      kept.push_back(at::zeros({std::max<int64_t>(count, 4096)}, like.options().dtype(at::kInt)));
    return kept.back().data_ptr<int32_t>();
  }
};
DecodeCounters g_decode_counters;

// One query token per row into out (B, 1, H, D) bf16, any strides with a unit
// head_dim stride.
void decode_into(const Tensor& out, const Tensor& query, const Tensor& key, const Tensor& value,
                 const c10::optional<Tensor>& query_start, int64_t query_start_value,
                 const c10::optional<Tensor>& kv_lengths, const c10::optional<Tensor>& key_mask, bool use_dummy,
                 double scale, int64_t num_splits) {
  check_strict_shapes(query, key, value);
  TORCH_CHECK_VALUE(query.size(2) == 1, "strict_decode takes one query token per row");
  c10::OptionalDeviceGuard guard(query.device());
  const Tensor q = operand(query), k = operand(key), v = operand(value);
  const int64_t batch = q.size(0), heads = q.size(1), dim = q.size(3);
  TORCH_CHECK_VALUE(out.scalar_type() == at::kBFloat16 && out.device() == q.device() && out.dim() == 4 &&
                        out.size(0) == batch && out.size(1) == 1 && out.size(2) == heads && out.size(3) == dim &&
                        out.stride(3) == 1,
                    "strict_decode_out: out must be a bf16 (B, 1, H, D) tensor on the query's device with a unit "
                    "head_dim stride");
  const Tensor o = out.select(1, 0);
  wmx_decode_args a;
  std::memset(&a, 0, sizeof(a));
  a.q = q.data_ptr();
  a.k = k.data_ptr();
  a.v = v.data_ptr();
  a.o = o.data_ptr();
  a.q_stride[0] = q.stride(0);
  a.q_stride[1] = q.stride(1);
  strides3(k, a.k_stride);
  strides3(v, a.v_stride);
  a.o_stride[0] = o.stride(0);
  a.o_stride[1] = o.stride(1);
  Tensor starts, lengths;
  // one value for every row (a pool's shared length) is read in place by
  // all rows rather than copied out per row
  const bool shared = batch > 1 && query_start && query_start->numel() == 1 &&
                      (!kv_lengths || kv_lengths->numel() == 1);
  if (query_start) {
    TORCH_CHECK_VALUE(query_start->numel() == 1 || query_start->numel() == batch,
                      "query_start must hold one value or one per batch row");
    starts = query_start->to(q.device(), at::kLong);
    starts = (shared ? starts.reshape({1}) : starts.expand({batch})).contiguous();
    a.query_start = starts.data_ptr<int64_t>();
  } else {
    a.query_start_scalar = query_start_value;
  }
  if (kv_lengths) {
    TORCH_CHECK_VALUE(kv_lengths->numel() == batch || (shared && kv_lengths->numel() == 1),
                      "kv_lengths must hold one value per batch row");
    lengths = kv_lengths->to(q.device(), at::kLong).reshape({-1}).contiguous();
    a.kv_lengths = lengths.data_ptr<int64_t>();
  }
  a.lengths_broadcast = shared ? 1 : 0;
  const Tensor mask = mask_bytes(key_mask);
  if (mask.defined()) {
    a.key_mask = mask.data_ptr<uint8_t>();
    a.key_mask_stride = mask.stride(0);
  }
  a.batch = (int32_t)batch;
  a.q_heads = (int32_t)heads;
  a.kv_heads = (int32_t)k.size(1);
  a.capacity = (int32_t)k.size(2);
  a.head_dim = (int32_t)dim;
  a.use_dummy = use_dummy ? 1 : 0;
  a.num_splits = (int32_t)num_splits;
  a.softmax_scale = (float)scale;
  a.counters = g_decode_counters.get(q, stream_of(q), batch * k.size(1));
  const int64_t need = wmx_decode_workspace_size(&a);
  Tensor workspace = at::empty({std::max<int64_t>(need, 16)}, q.options().dtype(at::kByte));
  a.workspace = workspace.data_ptr();
  a.workspace_bytes = need;
  check_rc(wmx_decode(&a, stream_of(q)), "wmx_decode");
}

Tensor strict_decode(const Tensor& query, const Tensor& key, const Tensor& value,
                     const c10::optional<Tensor>& query_start, int64_t query_start_value,
                     const c10::optional<Tensor>& kv_lengths, const c10::optional<Tensor>& key_mask, bool use_dummy,
                     double scale, int64_t num_splits) {
  check_strict_shapes(query, key, value);
  Tensor out = at::empty({query.size(0), 1, query.size(1), query.size(3)}, query.options().dtype(at::kBFloat16));
  decode_into(out, query, key, value, query_start, query_start_value, kv_lengths, key_mask, use_dummy, scale,
              num_splits);
  return out;
}

// The same into a caller's buffer (a decode loop's output rows, so the loop
// needs no stacking copy).
void strict_decode_out(const Tensor& out, const Tensor& query, const Tensor& key, const Tensor& value,
                       const c10::optional<Tensor>& query_start, int64_t query_start_value,
                       const c10::optional<Tensor>& kv_lengths, const c10::optional<Tensor>& key_mask, bool use_dummy,
                       double scale, int64_t num_splits) {
  decode_into(out, query, key, value, query_start, query_start_value, kv_lengths, key_mask, use_dummy, scale,
              num_splits);
}

// ------------------------------------------------- strict autograd ----
// Forward below the autograd key, saving what the backward operator reads;
// gradients are returned in the inputs' dtypes.
Tensor in_dtype(const Tensor& t, const Tensor& like) {
  return t.scalar_type() == like.scalar_type() ? t : t.to(like.scalar_type());
}

struct StrictPackedFn : public torch::autograd::Function<StrictPackedFn> {
  static variable_list forward(AutogradContext* ctx, const Tensor& query, const Tensor& key, const Tensor& value,
                               const Tensor& qi, const Tensor& ki, const Tensor& cq, const Tensor& ck,
                               int64_t max_queries, int64_t max_keys, double scale) {
    static auto op = c10::Dispatcher::singleton()
                         .findSchemaOrThrow("white_matter::strict_packed_fwd", "")
                         .typed<decltype(strict_packed_fwd)>();
    Tensor out, lse;
    {
      at::AutoDispatchBelowADInplaceOrView below;
      std::tie(out, lse) = op.call(query, key, value, qi, ki, cq, ck, max_queries, max_keys, scale);
    }
    ctx->save_for_backward({query, key, value, out, lse, qi, ki, cq, ck});
    ctx->saved_data["mq"] = max_queries;
    ctx->saved_data["mk"] = max_keys;
    ctx->saved_data["scale"] = scale;
    ctx->mark_non_differentiable({lse});
    ctx->set_materialize_grads(false);
    return {out, lse};
  }
  static variable_list backward(AutogradContext* ctx, variable_list grads) {
    static auto op = c10::Dispatcher::singleton()
                         .findSchemaOrThrow("white_matter::strict_packed_bwd", "")
                         .typed<decltype(strict_packed_bwd)>();
    const auto t = ctx->get_saved_variables();
    const Tensor dout = grads[0].defined() ? grads[0] : at::zeros_like(t[3]);
    auto [dq, dk, dv] = op.call(t[0], t[1], t[2], t[3], t[4], dout, t[5], t[6], t[7], t[8],
                                ctx->saved_data["mq"].toInt(), ctx->saved_data["mk"].toInt(),
                                ctx->saved_data["scale"].toDouble());
    return {in_dtype(dq, t[0]), in_dtype(dk, t[1]), in_dtype(dv, t[2]), Tensor(), Tensor(), Tensor(), Tensor(),
            Tensor(),           Tensor(),           Tensor()};
  }
};

struct StrictDenseFn : public torch::autograd::Function<StrictDenseFn> {
  static variable_list forward(AutogradContext* ctx, const Tensor& query, const Tensor& key, const Tensor& value,
                               int64_t query_offset, const c10::optional<Tensor>& row_offset,
                               const c10::optional<Tensor>& row_limit, const c10::optional<Tensor>& key_mask,
                               bool keep_slot0, double scale) {
    static auto op = c10::Dispatcher::singleton()
                         .findSchemaOrThrow("white_matter::strict_dense_fwd", "")
                         .typed<decltype(strict_dense_fwd)>();
    Tensor out, lse;
    {
      at::AutoDispatchBelowADInplaceOrView below;
      std::tie(out, lse) = op.call(query, key, value, query_offset, row_offset, row_limit, key_mask, keep_slot0, scale);
    }
    // undefined tensors stand for the absent optional bounds and mask
    ctx->save_for_backward({query, key, value, out, lse, row_offset.value_or(Tensor()), row_limit.value_or(Tensor()),
                            key_mask.value_or(Tensor())});
    ctx->saved_data["offset"] = query_offset;
    ctx->saved_data["slot0"] = keep_slot0;
    ctx->saved_data["scale"] = scale;
    ctx->mark_non_differentiable({lse});
    ctx->set_materialize_grads(false);
    return {out, lse};
  }
  static variable_list backward(AutogradContext* ctx, variable_list grads) {
    static auto op = c10::Dispatcher::singleton()
                         .findSchemaOrThrow("white_matter::strict_dense_bwd", "")
                         .typed<decltype(strict_dense_bwd)>();
    const auto t = ctx->get_saved_variables();
    const Tensor dout = grads[0].defined() ? grads[0] : at::zeros_like(t[3]);
    auto opt = [](const Tensor& x) { return x.defined() ? c10::optional<Tensor>(x) : c10::nullopt; };
    auto [dq, dk, dv] = op.call(t[0], t[1], t[2], t[3], t[4], dout, ctx->saved_data["offset"].toInt(), opt(t[5]),
                                opt(t[6]), opt(t[7]), ctx->saved_data["slot0"].toBool(),
                                ctx->saved_data["scale"].toDouble());
    return {in_dtype(dq, t[0]), in_dtype(dk, t[1]), in_dtype(dv, t[2]), Tensor(), Tensor(), Tensor(), Tensor(),
            Tensor(),           Tensor()};
  }
};

std::tuple<Tensor, Tensor> strict_packed_fwd_autograd(const Tensor& query, const Tensor& key, const Tensor& value,
                                                      const Tensor& qi, const Tensor& ki, const Tensor& cq,
                                                      const Tensor& ck, int64_t max_queries, int64_t max_keys,
                                                      double scale) {
  auto r = StrictPackedFn::apply(query, key, value, qi, ki, cq, ck, max_queries, max_keys, scale);
  return {r[0], r[1]};
}

std::tuple<Tensor, Tensor> strict_dense_fwd_autograd(const Tensor& query, const Tensor& key, const Tensor& value,
                                                     int64_t query_offset, const c10::optional<Tensor>& row_offset,
                                                     const c10::optional<Tensor>& row_limit,
                                                     const c10::optional<Tensor>& key_mask, bool keep_slot0,
                                                     double scale) {
  auto r = StrictDenseFn::apply(query, key, value, query_offset, row_offset, row_limit, key_mask, keep_slot0, scale);
  return {r[0], r[1]};
}

int64_t packed_plan_cache_size() { return g_plan_cache.size(); }

void packed_plan_cache_clear() { g_plan_cache.clear(); }

// Entries currently cached (for tests).
int64_t cyclic_schedule_cache_size() { return g_cyclic_cache.size(); }

void cyclic_schedule_cache_clear() { g_cyclic_cache.clear(); }

}  // namespace

TORCH_LIBRARY_FRAGMENT(white_matter, m) {
  m.def("cyclic_attn_fwd(Tensor Q, Tensor K, Tensor V, int K_stride, int residue, int block_M) -> (Tensor, Tensor)");
  m.def(
      "cyclic_attn_bwd(Tensor Q, Tensor K, Tensor V, Tensor Out, Tensor Lse, Tensor dOut, int K_stride, int residue, "
      "int block_M) -> (Tensor, Tensor, Tensor)");
  m.def(
      "cyclic_attn_doc_fwd(Tensor Q, Tensor K, Tensor V, Tensor QSeg, Tensor KSeg, Tensor QStart, Tensor KQEnd, "
      "int K_stride, int residue, int block_M) -> (Tensor, Tensor)");
  m.def(
      "cyclic_attn_doc_bwd(Tensor Q, Tensor K, Tensor V, Tensor QSeg, Tensor KSeg, Tensor QStart, Tensor KQEnd, "
      "Tensor Out, Tensor Lse, Tensor dOut, int K_stride, int residue, int block_M) -> (Tensor, Tensor, Tensor)");
  m.def("_cyclic_schedule_cache_size() -> int", &cyclic_schedule_cache_size);
  m.def("_cyclic_schedule_cache_clear() -> ()", &cyclic_schedule_cache_clear);
  m.def(
      "strict_packed_fwd(Tensor query, Tensor key, Tensor value, Tensor query_indices, Tensor key_indices, "
      "Tensor cu_queries, Tensor cu_keys, int max_queries, int max_keys, float scale) -> (Tensor, Tensor)");
  m.def(
      "strict_packed_bwd(Tensor query, Tensor key, Tensor value, Tensor out, Tensor lse, Tensor dout, "
      "Tensor query_indices, Tensor key_indices, Tensor cu_queries, Tensor cu_keys, int max_queries, int max_keys, "
      "float scale) -> (Tensor, Tensor, Tensor)");
  m.def(
      "strict_dense_fwd(Tensor query, Tensor key, Tensor value, int query_offset, Tensor? row_offset, "
      "Tensor? row_limit, Tensor? key_mask, bool keep_slot0, float scale) -> (Tensor, Tensor)");
  m.def(
      "strict_dense_bwd(Tensor query, Tensor key, Tensor value, Tensor out, Tensor lse, Tensor dout, "
      "int query_offset, Tensor? row_offset, Tensor? row_limit, Tensor? key_mask, bool keep_slot0, float scale) "
      "-> (Tensor, Tensor, Tensor)");
  m.def(
      "strict_decode(Tensor query, Tensor key, Tensor value, Tensor? query_start, int query_start_value, "
      "Tensor? kv_lengths, Tensor? key_mask, bool use_dummy, float scale, int num_splits) -> Tensor");
  m.def(
      "strict_decode_out(Tensor(a!) out, Tensor query, Tensor key, Tensor value, Tensor? query_start, "
      "int query_start_value, Tensor? kv_lengths, Tensor? key_mask, bool use_dummy, float scale, int num_splits) "
      "-> ()");
  m.def("_packed_plan_cache_size() -> int", &packed_plan_cache_size);
  m.def("_packed_plan_cache_clear() -> ()", &packed_plan_cache_clear);
}

TORCH_LIBRARY_IMPL(white_matter, CUDA, m) {
  m.impl("cyclic_attn_fwd", &cyclic_attn_fwd);
  m.impl("cyclic_attn_bwd", &cyclic_attn_bwd);
  m.impl("cyclic_attn_doc_fwd", &cyclic_attn_doc_fwd);
  m.impl("cyclic_attn_doc_bwd", &cyclic_attn_doc_bwd);
  m.impl("strict_packed_fwd", &strict_packed_fwd);
  m.impl("strict_packed_bwd", &strict_packed_bwd);
  m.impl("strict_dense_fwd", &strict_dense_fwd);
  m.impl("strict_dense_bwd", &strict_dense_bwd);
  m.impl("strict_decode", &strict_decode);
  m.impl("strict_decode_out", &strict_decode_out);
}

TORCH_LIBRARY_IMPL(white_matter, Autograd, m) {
  m.impl("cyclic_attn_fwd", &cyclic_attn_fwd_autograd);
  m.impl("cyclic_attn_doc_fwd", &cyclic_attn_doc_fwd_autograd);
  m.impl("strict_packed_fwd", &strict_packed_fwd_autograd);
  m.impl("strict_dense_fwd", &strict_dense_fwd_autograd);
}

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
#include <memory>
#include <mutex>

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

struct Schedule {
  std::array<Tensor, 4> meta;         // the metadata tensors the entry was built from
  std::array<uint32_t, 4> versions;
  int64_t q_len, k_len, stride, offset;
  int status = kDocMode;
  // packed segments (status kPacked), see wmx_attn_args
  Tensor qi, ki, cu_q, cu_k, q_units, k_units, ds_offsets;
  int64_t num_segments = 0, max_q = 0, max_k = 0, layout = 0, keys_unique = 1, ds_elements = 0;
  // int32 contiguous document arrays (status kDocMode)
  std::array<Tensor, 4> docs;
};

std::mutex g_cache_mutex;
std::list<std::shared_ptr<Schedule>> g_cache;  // most recently used first
constexpr size_t kCacheEntries = 256;

uint32_t version_of(const Tensor& t) { return t.unsafeGetTensorImpl()->version_counter().current_version(); }

std::shared_ptr<Schedule> find_schedule(const std::array<Tensor, 4>& m, int64_t q_len, int64_t k_len, int64_t stride,
                                        int64_t offset) {
  std::lock_guard<std::mutex> lock(g_cache_mutex);
  for (auto it = g_cache.begin(); it != g_cache.end(); ++it) {
    const Schedule& s = **it;
    if (s.q_len != q_len || s.k_len != k_len || s.stride != stride || s.offset != offset) continue;
    bool same = true;
    for (int i = 0; i < 4 && same; ++i)
      same = s.meta[i].unsafeGetTensorImpl() == m[i].unsafeGetTensorImpl() && s.versions[i] == version_of(m[i]);
    if (!same) continue;
    auto hit = *it;
    if (it != g_cache.begin()) g_cache.splice(g_cache.begin(), g_cache, it);
    return hit;
  }
  return nullptr;
}

// The packed schedule of these metadata tensors at this stride and residue
// offset, built on a miss by the Python packer
// (white_matter::_cyclic_schedule: [facts, query_indices, key_indices,
// cu_queries, cu_keys, q_units, k_units, ds_offsets], facts = int64 CPU
// {status, num_segments, max_queries, max_keys, segment_layout, keys_unique,
// ds_elements}).
std::shared_ptr<Schedule> schedule_for(const std::array<Tensor, 4>& m, int64_t q_len, int64_t k_len, int64_t stride,
                                       int64_t offset) {
  if (auto hit = find_schedule(m, q_len, k_len, stride, offset)) return hit;
  static auto packer = c10::Dispatcher::singleton()
                           .findSchemaOrThrow("white_matter::_cyclic_schedule", "")
                           .typed<std::vector<Tensor>(const Tensor&, const Tensor&, const Tensor&, const Tensor&,
                                                      int64_t, int64_t, int64_t, int64_t)>();
  auto s = std::make_shared<Schedule>();
  s->meta = m;
  for (int i = 0; i < 4; ++i) s->versions[i] = version_of(m[i]);
  s->q_len = q_len;
  s->k_len = k_len;
  s->stride = stride;
  s->offset = offset;
  std::vector<Tensor> built;
  {
    at::AutoDispatchBelowADInplaceOrView below;
    built = packer.call(m[0], m[1], m[2], m[3], q_len, k_len, stride, offset);
  }
  TORCH_CHECK(!built.empty() && built[0].numel() == 7, "_cyclic_schedule returned an unexpected result");
  const Tensor facts = built[0].to(at::kLong).contiguous();
  const int64_t* f = facts.data_ptr<int64_t>();
  s->status = (int)f[0];
  if (s->status == kPacked) {
    TORCH_CHECK(built.size() == 8, "_cyclic_schedule returned an unexpected result");
    s->num_segments = f[1];
    s->max_q = f[2];
    s->max_k = f[3];
    s->layout = f[4];
    s->keys_unique = f[5];
    s->ds_elements = f[6];
    s->qi = built[1].contiguous();
    s->ki = built[2].contiguous();
    s->cu_q = built[3].to(at::kInt).contiguous();
    s->cu_k = built[4].to(at::kInt).contiguous();
    s->q_units = built[5].to(at::kInt).contiguous();
    s->k_units = built[6].to(at::kInt).contiguous();
    s->ds_offsets = built[7].to(at::kLong).contiguous();
  } else if (s->status == kDocMode) {
    for (int i = 0; i < 4; ++i) s->docs[i] = m[i].to(at::kInt).contiguous();
  }
  std::lock_guard<std::mutex> lock(g_cache_mutex);
  g_cache.push_front(s);
  while (g_cache.size() > kCacheEntries) g_cache.pop_back();
  return s;
}

// --------------------------------------------------------- launch glue ----
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
void fill_visibility(wmx_attn_args& a, const Schedule* s, int64_t stride, int64_t residue, const Tensor& q,
                     const Tensor& k, bool backward) {
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
    if (backward) {
      a.ds_offsets = s->ds_offsets.data_ptr<int64_t>();
      a.ds_elements = s->ds_elements;
    }
  } else if (s->status == kDocMode) {
    a.q_seg = s->docs[0].data_ptr<int32_t>();
    a.k_seg = s->docs[1].data_ptr<int32_t>();
    a.q_start = s->docs[2].data_ptr<int32_t>();
    a.k_qend = s->docs[3].data_ptr<int32_t>();
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
    fill_visibility(a, s.get(), stride, residue, q, k, false);
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
    fill_visibility(a, s.get(), stride, residue, q, k, true);
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

// Entries currently cached (for tests).
int64_t cyclic_schedule_cache_size() {
  std::lock_guard<std::mutex> lock(g_cache_mutex);
  return (int64_t)g_cache.size();
}

void cyclic_schedule_cache_clear() {
  std::lock_guard<std::mutex> lock(g_cache_mutex);
  g_cache.clear();
}

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
}

TORCH_LIBRARY_IMPL(white_matter, CUDA, m) {
  m.impl("cyclic_attn_fwd", &cyclic_attn_fwd);
  m.impl("cyclic_attn_bwd", &cyclic_attn_bwd);
  m.impl("cyclic_attn_doc_fwd", &cyclic_attn_doc_fwd);
  m.impl("cyclic_attn_doc_bwd", &cyclic_attn_doc_bwd);
}

TORCH_LIBRARY_IMPL(white_matter, Autograd, m) {
  m.impl("cyclic_attn_fwd", &cyclic_attn_fwd_autograd);
  m.impl("cyclic_attn_doc_fwd", &cyclic_attn_doc_fwd_autograd);
}

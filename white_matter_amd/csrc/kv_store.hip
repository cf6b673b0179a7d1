// KV-pool store for gfx950: K-norm, weight, RoPE, casts and the pool slot
// scatter in one pass over the group's keys and values (the eager reference
// sequence modules/kv_pool.py:163-172,216 and blocks/_execution/cyclic.py:
// 448-458 makes about eight passes over the keys). HBM-bound: each thread
// moves 8 consecutive elements of a row with 16-byte accesses.
#include "wmx_kernels.h"

namespace wmx {

// Value source: none (keys only), fp32 or bf16.
enum ValueKind { kNoValue = 0, kValueF32 = 1, kValueBF16 = 2 };

// One (b, c, t, head group) per D/8 consecutive lanes (token-fastest, so
// neighbouring lanes read and write neighbouring rows); each thread then
// walks its group's heads, U at a time with all their loads issued before any
// is used (no branch between them: the last group repeats its final head
// instead of testing), so cos, sin, the norm weight and the slot are read
// once per token and group instead of once per row. One group of all heads
// where there are many tokens; one head per group for a decode step's few
// rows, whose latency chain is then one round trip. KEY_BF16 selects the
// reference's rounding after every step.
template <int D, bool KEY_BF16, int VALUE>
__global__ __launch_bounds__(256) void kv_store_kernel(const wmx_kv_store_args a, int64_t tokens_total,
                                                       int head_groups) {
  // Every product and sum is rounded on its own, as the eager sequence does:
  // a fused multiply-add would skip the rounding of y * cos.
#pragma clang fp contract(off)
  constexpr int LD = D / 8;                    // lanes holding data
  constexpr int L = LD <= 8 ? 8 : 16;          // lanes per row (a power of two; D = 96 leaves 4 idle)
  constexpr int U = 4;                         // heads in flight per thread
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t unit = gid / L;
  const int l = (int)(gid % L);  // this lane's elements: 8 l .. 8 l + 7
  const int64_t r = unit / head_groups;
  const int hg = (int)(unit - r * head_groups);
  // A row's L lanes are aligned and share r and hg, so they leave together
  // and the shuffles below never read a lane that has left.
  if (r >= tokens_total) return;
  const int t = (int)(r % a.tokens);
  const int64_t bc = r / a.tokens;
  const int c = (int)(bc % a.channels);
  const int b = (int)(bc / a.channels);
  const int per_group = (a.heads + head_groups - 1) / head_groups;
  const int h_begin = hg * per_group, h_end = min(h_begin + per_group, a.heads);
  if (h_begin >= h_end) return;
  // out-of-range slots are not written; the check waits for the slot only at
  // the stores, so the loads below do not
  const int64_t slot = a.slots[t];
  const bool slot_ok = slot >= 0 && slot < a.pool_slots;
  const int d0 = 8 * l;
  // idle lanes (D = 96) take part in the shuffles with zeros and store nothing
  const bool data = l < LD;
  const int dl = data ? d0 : 0;
  auto rnd = [](float x) { return KEY_BF16 ? round_bf16(x) : x; };

  float w[8], cs[8], sn[8];
  load8(a.k_norm_weight, (int64_t)c * D + dl, a.weight_dtype == WMX_DTYPE_BF16, w);
  const int64_t ro = a.rope_by_slot ? (slot_ok ? slot : 0) * a.rope_stride[1] + dl
                                    : (int64_t)b * a.rope_stride[0] + (int64_t)t * a.rope_stride[1] + dl;
  load8(a.cos, ro, a.rope_dtype == WMX_DTYPE_BF16, cs);
  load8(a.sin, ro, a.rope_dtype == WMX_DTYPE_BF16, sn);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    w[e] = rnd(w[e]);
    cs[e] = rnd(cs[e]);
    sn[e] = rnd(sn[e]);
  }
  // rotate_half: element d pairs with d +- D/2, held by the lane LD/2 away
  const bool low = d0 < D / 2;
  const int partner = (int)(gid & 63) + (low ? LD / 2 : -(LD / 2));  // lane in the wave
  const int64_t key_row = (int64_t)b * a.key_stride[0] + (int64_t)c * a.key_stride[1] + (int64_t)t * a.key_stride[3] + dl;
  const int64_t kpool_row =
      (int64_t)b * a.key_pool_stride[0] + (int64_t)c * a.key_pool_stride[1] + slot * a.key_pool_stride[3] + dl;
  const int64_t value_row =
      (int64_t)b * a.value_stride[0] + (int64_t)c * a.value_stride[1] + (int64_t)t * a.value_stride[3] + dl;
  const int64_t vpool_row =
      (int64_t)b * a.value_pool_stride[0] + (int64_t)c * a.value_pool_stride[1] + slot * a.value_pool_stride[3] + dl;

  for (int h0 = h_begin; h0 < h_end; h0 += U) {
    float x[U][8], v[U][8];
    int hu[U];
#pragma unroll
    for (int u = 0; u < U; ++u) hu[u] = min(h0 + u, h_end - 1);
#pragma unroll
    for (int u = 0; u < U; ++u) load8<true>(a.key, key_row + hu[u] * a.key_stride[2], KEY_BF16, x[u]);
    if constexpr (VALUE != kNoValue) {
#pragma unroll
      for (int u = 0; u < U; ++u) load8<true>(a.value, value_row + hu[u] * a.value_stride[2], VALUE == kValueBF16, v[u]);
    }
    __builtin_amdgcn_sched_barrier(0);  // keep every load of the group ahead of the first use
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float ss = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = fmaf(x[u][e], x[u][e], ss);
      if (!data) ss = 0.f;
#pragma unroll
      for (int o = L / 2; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
      const float inv = 1.f / sqrtf(ss / (float)D + a.eps);
      float y[8], out[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) y[e] = rnd(rnd(x[u][e] * inv) * w[e]);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float other = __shfl(y[e], data ? partner : 0);
        const float rot = low ? -other : other;
        out[e] = rnd(rnd(y[e] * cs[e]) + rnd(rot * sn[e]));
      }
      if (data && slot_ok && h0 + u < h_end) {
        store8_bf16(a.key_pool, kpool_row + hu[u] * a.key_pool_stride[2], out);
        if constexpr (VALUE != kNoValue) store8_bf16(a.value_pool, vpool_row + hu[u] * a.value_pool_stride[2], v[u]);
      }
    }
  }
}

template <int D, bool KEY_BF16>
void launch_kv_store_d(const wmx_kv_store_args& a, int64_t rows, int groups, dim3 grid, hipStream_t stream) {
  if (!a.value)
    hipLaunchKernelGGL((kv_store_kernel<D, KEY_BF16, kNoValue>), grid, dim3(256), 0, stream, a, rows, groups);
  else if (a.value_dtype == WMX_DTYPE_BF16)
    hipLaunchKernelGGL((kv_store_kernel<D, KEY_BF16, kValueBF16>), grid, dim3(256), 0, stream, a, rows, groups);
  else
    hipLaunchKernelGGL((kv_store_kernel<D, KEY_BF16, kValueF32>), grid, dim3(256), 0, stream, a, rows, groups);
}

int launch_kv_store(const wmx_kv_store_args& a, hipStream_t stream) {
  const int64_t rows = (int64_t)a.batch * a.channels * a.tokens;
  if (rows == 0 || a.heads == 0) return WMX_OK;
  const int64_t lanes = a.head_dim <= 64 ? 8 : 16;  // lanes per row, as in the kernel
  // threads walk all heads of a token where that still gives every CU four
  // workgroups (1024 x 256 threads); fewer rows (a decode step) split the heads
  int64_t groups = 1;
  while (groups < a.heads && rows * groups * lanes < 1024 * 256) groups *= 2;
  if (groups > a.heads) groups = a.heads;
  const int64_t threads = rows * groups * lanes;
  if ((threads + 255) / 256 > UINT32_MAX) return WMX_E_UNSUPPORTED;
  const dim3 grid((unsigned)((threads + 255) / 256));
  const bool kb = a.key_dtype == WMX_DTYPE_BF16;
  if (a.head_dim == 64) {
    if (kb) launch_kv_store_d<64, true>(a, rows, (int)groups, grid, stream);
    else launch_kv_store_d<64, false>(a, rows, (int)groups, grid, stream);
  } else if (a.head_dim == 96) {
    if (kb) launch_kv_store_d<96, true>(a, rows, (int)groups, grid, stream);
    else launch_kv_store_d<96, false>(a, rows, (int)groups, grid, stream);
  } else if (a.head_dim == 128) {
    if (kb) launch_kv_store_d<128, true>(a, rows, (int)groups, grid, stream);
    else launch_kv_store_d<128, false>(a, rows, (int)groups, grid, stream);
  } else {
    return WMX_E_UNSUPPORTED;
  }
  return WMX_OK;
}

// ------------------------------------------------------------ backward ----
// Rows per workgroup of the backward: (256 / L) tokens of one (b, c), each
// thread walking the heads of its token like the forward.
template <int D>
constexpr int bwd_lanes() { return D / 8 <= 8 ? 8 : 16; }

int64_t kv_store_bwd_chunks(const wmx_kv_store_bwd_args& a) {
  const int rows = 256 / (a.head_dim <= 64 ? 8 : 16);
  return ((int64_t)a.tokens + rows - 1) / rows;
}

int64_t kv_store_bwd_workspace_size(const wmx_kv_store_bwd_args& a) {
  return (int64_t)a.batch * a.channels * kv_store_bwd_chunks(a) * a.head_dim * (int64_t)sizeof(float);
}

// Workgroup (b, c, token chunk). Per row: y = x * inv, du = g cos +
// rot^T(g sin), dx = inv (du w - y mean(du w y)); the workgroup's part of
// grad_weight[c] (sum of du y over its rows and heads) goes to the workspace.
template <int D, bool KEY_BF16>
__global__ __launch_bounds__(256) void kv_store_bwd_kernel(const wmx_kv_store_bwd_args a, int chunks) {
  constexpr int LD = D / 8;
  constexpr int L = bwd_lanes<D>();
  constexpr int RB = 256 / L;
  __shared__ float red[4][D];
  const int bc = blockIdx.x / chunks, chunk = blockIdx.x - bc * chunks;
  const int b = bc / a.channels, c = bc - b * a.channels;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int l = tid % L;
  const int t = chunk * RB + tid / L;
  const bool row_ok = t < a.tokens;
  const int d0 = 8 * l;
  const bool data = l < LD;
  const bool live = row_ok && data;
  const int dl = data ? d0 : 0;
  const int tl = row_ok ? t : 0;
  const bool low = d0 < D / 2;
  const int partner = data ? lane + (low ? LD / 2 : -(LD / 2)) : lane;

  float wt[8], cs[8], sn[8];
  load8(a.k_norm_weight, (int64_t)c * D + dl, a.weight_dtype == WMX_DTYPE_BF16, wt);
  const int64_t ro = (int64_t)b * a.rope_stride[0] + (int64_t)tl * a.rope_stride[1] + dl;
  load8(a.cos, ro, a.rope_dtype == WMX_DTYPE_BF16, cs);
  load8(a.sin, ro, a.rope_dtype == WMX_DTYPE_BF16, sn);
  const int64_t key_row = (int64_t)b * a.key_stride[0] + (int64_t)c * a.key_stride[1] + (int64_t)tl * a.key_stride[3] + dl;
  const int64_t g_row =
      (int64_t)b * a.grad_out_stride[0] + (int64_t)c * a.grad_out_stride[1] + (int64_t)tl * a.grad_out_stride[3] + dl;
  const int64_t dk_row =
      (int64_t)b * a.grad_key_stride[0] + (int64_t)c * a.grad_key_stride[1] + (int64_t)tl * a.grad_key_stride[3] + dl;
  float dw[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) dw[e] = 0.f;

  for (int h = 0; h < a.heads; ++h) {
    float x[8], g[8];
    load8(a.key, key_row + (int64_t)h * a.key_stride[2], KEY_BF16, x);
    load8(a.grad_out, g_row + (int64_t)h * a.grad_out_stride[2], true, g);
    if (!live) {
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = g[e] = 0.f;
    }
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) ss = fmaf(x[e], x[e], ss);
#pragma unroll
    for (int o = L / 2; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
    const float inv = 1.f / sqrtf(ss / (float)D + a.eps);
    float y[8], du[8], dot = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      y[e] = x[e] * inv;
      const float other = __shfl(g[e] * sn[e], partner);
      du[e] = g[e] * cs[e] + (low ? other : -other);
      dw[e] = fmaf(du[e], y[e], dw[e]);
      du[e] *= wt[e];
      dot = fmaf(du[e], y[e], dot);
    }
#pragma unroll
    for (int o = L / 2; o > 0; o >>= 1) dot += __shfl_xor(dot, o);
    const float mean = dot / (float)D;
    float dx[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) dx[e] = inv * (du[e] - y[e] * mean);
    if (live) {
      const int64_t off = dk_row + (int64_t)h * a.grad_key_stride[2];
      if constexpr (KEY_BF16) {
        store8_bf16(a.grad_key, off, dx);
      } else {
        float* dst = (float*)a.grad_key + off;
        *reinterpret_cast<f32x4*>(dst) = f32x4{dx[0], dx[1], dx[2], dx[3]};
        *reinterpret_cast<f32x4*>(dst + 4) = f32x4{dx[4], dx[5], dx[6], dx[7]};
      }
    }
  }
  // the workgroup's grad_weight part: rows of a wave, then the four waves in order
#pragma unroll
  for (int e = 0; e < 8; ++e) {
#pragma unroll
    for (int o = L; o < 64; o <<= 1) dw[e] += __shfl_xor(dw[e], o);
  }
  if (lane < L && data) {
#pragma unroll
    for (int e = 0; e < 8; ++e) red[w][d0 + e] = dw[e];
  }
  __syncthreads();
  if (tid < D) {
    float* part = (float*)a.workspace + (int64_t)blockIdx.x * D;
    part[tid] = ((red[0][tid] + red[1][tid]) + red[2][tid]) + red[3][tid];
  }
}

// grad_weight[c, d] = the parts of every (b, chunk) of channel c, added in
// order (eight interleaved partial sums, combined in a fixed order).
__global__ __launch_bounds__(128) void kv_store_bwd_reduce_kernel(const wmx_kv_store_bwd_args a, int chunks) {
  const int c = blockIdx.x, d = threadIdx.x;
  if (d >= a.head_dim) return;
  const int D = a.head_dim;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  const int64_t per_b = (int64_t)chunks;
  const int n = a.batch * chunks;
  int i = 0;
  for (; i + 8 <= n; i += 8) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int k = i + u, bb = k / chunks, ch = k - bb * chunks;
      acc[u] += ((const float*)a.workspace)[(((int64_t)bb * a.channels + c) * per_b + ch) * D + d];
    }
  }
  for (; i < n; ++i) {
    const int bb = i / chunks, ch = i - bb * chunks;
    acc[i & 7] += ((const float*)a.workspace)[(((int64_t)bb * a.channels + c) * per_b + ch) * D + d];
  }
  a.grad_weight[(int64_t)c * D + d] = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
}

template <int D>
static void launch_kv_store_bwd_d(const wmx_kv_store_bwd_args& a, unsigned blocks, int chunks, hipStream_t stream) {
  if (a.key_dtype == WMX_DTYPE_BF16)
    hipLaunchKernelGGL((kv_store_bwd_kernel<D, true>), dim3(blocks), dim3(256), 0, stream, a, chunks);
  else
    hipLaunchKernelGGL((kv_store_bwd_kernel<D, false>), dim3(blocks), dim3(256), 0, stream, a, chunks);
}

int launch_kv_store_bwd(const wmx_kv_store_bwd_args& a, hipStream_t stream) {
  const int64_t chunks = kv_store_bwd_chunks(a);
  const int64_t blocks = (int64_t)a.batch * a.channels * chunks;
  if (a.channels == 0) return WMX_OK;
  if (blocks > UINT32_MAX || chunks > INT32_MAX) return WMX_E_UNSUPPORTED;
  if (blocks > 0) {
    switch (a.head_dim) {
      case 64: launch_kv_store_bwd_d<64>(a, (unsigned)blocks, (int)chunks, stream); break;
      case 96: launch_kv_store_bwd_d<96>(a, (unsigned)blocks, (int)chunks, stream); break;
      case 128: launch_kv_store_bwd_d<128>(a, (unsigned)blocks, (int)chunks, stream); break;
      default: return WMX_E_UNSUPPORTED;
    }
  }
  hipLaunchKernelGGL(kv_store_bwd_reduce_kernel, dim3((unsigned)a.channels), dim3(128), 0, stream, a, (int)chunks);
  return WMX_OK;
}

}  // namespace wmx

// Single-query decode over a KV pool for gfx950: bandwidth-bound split-K.
//
// Replaces the reference's cached decode (flash_attn_with_kvcache /
// aten._flash_attention_forward with seqused_k,
// src/white_matter/ops/flash_attention.py:15-103) and its key_mask packing
// (src/white_matter/ops/strict_causal_attention.py:238-263): the mask is
// applied while streaming, so the cache is never gathered or copied.
//
// Work unit: one workgroup = (batch row b, KV head, key split). It streams
// its key range once and serves all G = Hq/Hkv query heads of the KV head,
// so each K/V byte is read from HBM once. A key row of D bf16 is read by
// LPR lanes with 16-byte loads (D=128: 16 lanes, 4 rows per wave load),
// UNROLL row groups are in flight per wave. Scores are dot products on the
// VALU (arithmetic intensity ~2G flop/byte, far below the MFMA ridge).
// K/V rows are read with nontemporal loads (streamed once). Each split writes
// an unnormalised (o, max, sum) partial, merged in log-sum-exp form into the
// bf16 output either by the last split of its (row, KV head) to finish (with
// the caller's counters: a vector-memory atomic counts the finished splits,
// the last one merges every split's partial in split order and resets the
// counter) or by a second kernel (without). Both merges add the same terms in
// the same order, so the outputs are bit-identical. A single split writes its
// output itself.
#include <climits>

#include "wmx_kernels.h"

namespace wmx {

constexpr int kDecodeChunkMin = 256;
// With counters, launches of at most kDecodeMergeBlocks workgroups (four per
// CU) and at most kDecodeMergeSplits splits merge in the last split to
// finish: there a second kernel's launch and tail are most of the merge's
// cost (the C5 decode loop: 0.313 -> 0.289 ms per token). Larger launches keep
// the combine kernel: the atomic round trip at the end of each of their many
// workgroups costs more (C4 decode, 4096 workgroups: 0.177 -> 0.19 ms).
constexpr int kDecodeMergeSplits = 64;
constexpr int64_t kDecodeMergeBlocks = 4 * 256;

bool decode_merges_in_split(const wmx_decode_args& a, int nsplit) {
  return a.counters && nsplit > 1 && nsplit <= kDecodeMergeSplits &&
         (int64_t)nsplit * a.batch * a.kv_heads <= kDecodeMergeBlocks;
}

struct DecodeLen {
  int64_t len;        // keys j < len may be visible
  bool masked;        // key_mask applies
};

__device__ __forceinline__ DecodeLen decode_len(const wmx_decode_args& a, int b) {
  const int rb = a.lengths_broadcast ? 0 : b;
  const int64_t start = a.query_start ? a.query_start[rb] : a.query_start_scalar;
  int64_t bound = start;
  if (a.kv_lengths) bound = min(bound, a.kv_lengths[rb]);
  DecodeLen r;
  if (a.key_mask) {
    r.len = bound + a.use_dummy;
    r.masked = true;
  } else {
    const int64_t cap = (int64_t)a.capacity - a.use_dummy;
    bound = bound < 0 ? 0 : (bound > cap ? cap : bound);
    r.len = bound + a.use_dummy;
    r.masked = false;
  }
  if (r.len > a.capacity) r.len = a.capacity;
  return r;
}

// Partials that another workgroup may merge in the same launch are written
// and read with agent-coherent accesses (relaxed agent-scope atomics: the
// sc1 forms of global_store / global_load), which reach the point where all
// XCDs' accesses meet without writing back or invalidating whole L2 caches.
__device__ __forceinline__ void store_partial(float* p, float v, bool shared) {
  if (shared) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else {
    *p = v;  // read by the combine kernel after this launch
  }
}
__device__ __forceinline__ float load_shared(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Cross-lane exchanges without the LDS crossbar (ds_bpermute) that
// __shfl_xor compiles to: DPP within rows of 16 lanes, v_permlane16_swap /
// v_permlane32_swap across them. A decode workgroup is often the only wave on
// its SIMD, so the crossbar's latency is not hidden there.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}
// x of lane l ^ OFF, exactly, for OFF in {1, 2, 8, 16, 32}
template <int OFF>
__device__ __forceinline__ float lane_xor(float x) {
  if constexpr (OFF == 1) {
    return dpp_mov<0xB1>(x);  // quad_perm [1, 0, 3, 2]
  } else if constexpr (OFF == 2) {
    return dpp_mov<0x4E>(x);  // quad_perm [2, 3, 0, 1]
  } else if constexpr (OFF == 8) {
    return dpp_mov<0x128>(x);  // row_ror:8 (rows of 16 lanes)
  } else if constexpr (OFF == 16) {
    // swaps rows 1 and 3 of the first operand with rows 0 and 2 of the second
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float((threadIdx.x & 16) ? r[0] : r[1]);
  } else {
    static_assert(OFF == 32, "lane_xor: 1, 2, 8, 16 or 32");
    // swaps the upper half of the first operand with the lower half of the second
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float((threadIdx.x & 32) ? r[0] : r[1]);
  }
}

// Sum over the LPR (8 or 16) consecutive lanes of a key row, the same value
// in all of them: quads first (exact xor), then half rows and rows by
// mirroring, which equals the xor partner once each quad (half row) holds one
// value.
template <int LPR>
__device__ __forceinline__ float row_sum(float acc) {
  acc += lane_xor<1>(acc);
  acc += lane_xor<2>(acc);
  acc += dpp_mov<0x141>(acc);  // row_half_mirror: the other quad of the half row
  if constexpr (LPR == 16) acc += dpp_mov<0x140>(acc);  // row_mirror: the other half row
  return acc;
}

// One step of the merge of a wave's row slots: the (m, l, o) of lane l and
// lane l ^ OFF (same dims, another slot) combined in log-sum-exp form.
template <int OFF, int G>
__device__ __forceinline__ void merge_slots(float (&m)[G], float (&l)[G], float (&o)[G][8]) {
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float mo = lane_xor<OFF>(m[g]);
    const float lo = lane_xor<OFF>(l[g]);
    const float mx = fmaxf(fmaxf(m[g], mo), kMaxFloor);
    const float sa = __builtin_amdgcn_exp2f(m[g] - mx), sb = __builtin_amdgcn_exp2f(mo - mx);
    l[g] = l[g] * sa + lo * sb;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[g][e] = o[g][e] * sa + lane_xor<OFF>(o[g][e]) * sb;
    m[g] = fmaxf(m[g], mo);
  }
}

// Merge the nsplit partials of query head h of row b in split order (the
// log-sum-exp form of decode_combine_kernel) into output element d.
__device__ __forceinline__ float merge_splits(const float* ws_o, const float* ws_ml, int64_t prow0, int nsplit, int D,
                                              int d) {
  float mx = kMaxFloor;
  for (int s = 0; s < nsplit; ++s) mx = fmaxf(mx, ws_ml[(prow0 + s) * 2]);
  float lsum = 0.f, acc = 0.f;
  for (int s = 0; s < nsplit; ++s) {
    const float w = __builtin_amdgcn_exp2f(ws_ml[(prow0 + s) * 2] - mx);
    lsum += ws_ml[(prow0 + s) * 2 + 1] * w;
    acc += ws_o[(prow0 + s) * D + d] * w;
  }
  return lsum > 0.f ? acc / lsum : 0.f;
}

// G query heads of one KV head per workgroup, from head head_offset of the
// KV head's group on (groups of more than 8 heads run in several launches);
// NW waves per workgroup, each taking every NW-th group of key rows
template <int D, int G, int NW>
__global__ __launch_bounds__(64 * NW) void decode_split_kernel(const wmx_decode_args a, int chunk, int head_offset,
                                                            int32_t* counters) {
  constexpr int LPR = D <= 64 ? 8 : 16;   // lanes per key row
  constexpr int RPW = 64 / LPR;           // rows per wave load
  // key rows in flight per lane: eight for one head; four for a head group,
  // whose accumulators take the registers (fewer rows, more resident waves)
  constexpr int kDecodeUnroll = G == 1 ? 8 : 4;
  constexpr int ROWS_ITER = NW * RPW * kDecodeUnroll;
  __shared__ float lds_m[NW][G], lds_l[NW][G];
  __shared__ __attribute__((aligned(16))) float lds_o[NW][G][D];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int dch = lane % LPR, rslot = lane / LPR;
  const bool dlive = 8 * dch < D;
  // split-major order: consecutive workgroups (dealt round-robin over the 8
  // XCDs) take different (row, KV head) pairs of one split, so every XCD gets
  // an even share of each split whatever the rows' lengths, and the first
  // splits (which every nonempty row has) start first
  const int pairs = a.batch * a.kv_heads;
  const int split = blockIdx.x / pairs, pair = blockIdx.x - split * pairs;
  const int b = pair / a.kv_heads, hk = pair - b * a.kv_heads;
  const int nsplit = gridDim.x / pairs;
  const int group = a.q_heads / a.kv_heads;
  const int h0 = hk * group + head_offset;  // first query head of this workgroup

  const DecodeLen dl = decode_len(a, b);
  const int64_t j_begin = (int64_t)split * chunk;
  int64_t j_end = j_begin + chunk;
  if (j_end > dl.len) j_end = dl.len;

  const float qscale = a.softmax_scale * kLog2e;
  float q[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    u32x4 w = {0u, 0u, 0u, 0u};
    if (dlive) w = load16((const bf16*)a.q + (int64_t)b * a.q_stride[0] + (int64_t)(h0 + g) * a.q_stride[1] + 8 * dch);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      q[g][2 * e] = bf16_lo(w[e]) * qscale;
      q[g][2 * e + 1] = bf16_hi(w[e]) * qscale;
    }
  }
  float m[G], l[G], o[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = kNegInf;
    l[g] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[g][e] = 0.f;
  }

  const bf16* kbase = (const bf16*)a.k + (int64_t)b * a.k_stride[0] + (int64_t)hk * a.k_stride[1] + 8 * dch;
  const bf16* vbase = (const bf16*)a.v + (int64_t)b * a.v_stride[0] + (int64_t)hk * a.v_stride[1] + 8 * dch;
  const uint8_t* kmask = a.key_mask ? a.key_mask + (int64_t)b * a.key_mask_stride : nullptr;

  for (int64_t it = j_begin; it < j_end; it += ROWS_ITER) {
    u32x4 kw[kDecodeUnroll], vw[kDecodeUnroll];
    bool vis[kDecodeUnroll];
#pragma unroll
    for (int u = 0; u < kDecodeUnroll; ++u) {
      const int64_t j = it + (int64_t)(u * NW + wave) * RPW + rslot;
      bool ok = j < j_end;
      if (ok && dl.masked) ok = kmask[j] != 0;
      vis[u] = ok;
      u32x4 zk = {0u, 0u, 0u, 0u}, zv = {0u, 0u, 0u, 0u};
      if (ok && dlive) {
        // each K/V byte is read once: nontemporal loads stream past the caches
        // (measured 4.74 -> 5.17 TB/s on the C4 decode)
        zk = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(kbase + j * a.k_stride[2]));
        zv = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(vbase + j * a.v_stride[2]));
      }
      kw[u] = zk;
      vw[u] = zv;
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float s[kDecodeUnroll];
      float smax = kNegInf;
#pragma unroll
      for (int u = 0; u < kDecodeUnroll; ++u) {
        float acc = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          acc = fmaf(q[g][2 * e], bf16_lo(kw[u][e]), acc);
          acc = fmaf(q[g][2 * e + 1], bf16_hi(kw[u][e]), acc);
        }
        acc = row_sum<LPR>(acc);
        s[u] = vis[u] ? acc : kNegInf;
        smax = fmaxf(smax, s[u]);
      }
      const float m_new = fmaxf(m[g], smax);
      const float m_use = fmaxf(m_new, kMaxFloor);
      const float alpha = __builtin_amdgcn_exp2f(m[g] - m_use);
      l[g] *= alpha;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[g][e] *= alpha;
#pragma unroll
      for (int u = 0; u < kDecodeUnroll; ++u) {
        const float p = __builtin_amdgcn_exp2f(s[u] - m_use);
        l[g] += p;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          o[g][2 * e] = fmaf(p, bf16_lo(vw[u][e]), o[g][2 * e]);
          o[g][2 * e + 1] = fmaf(p, bf16_hi(vw[u][e]), o[g][2 * e + 1]);
        }
      }
      m[g] = m_new;
    }
  }

  // merge the RPW row slots of the wave (lanes with equal dch)
  if constexpr (LPR == 8) merge_slots<8, G>(m, l, o);
  merge_slots<16, G>(m, l, o);
  merge_slots<32, G>(m, l, o);
  if (rslot == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      if (dch == 0) {
        lds_m[wave][g] = m[g];
        lds_l[wave][g] = l[g];
      }
      if (dlive) {
#pragma unroll
        for (int e = 0; e < 8; ++e) lds_o[wave][g][8 * dch + e] = o[g][e];
      }
    }
  }
  __syncthreads();
  if (nsplit == 1) {
    // the split is the whole row: merge the 4 waves and write the bf16 output
    // (the same sums the combine kernel would form from one partial)
    for (int idx = tid; idx < G * D; idx += 64 * NW) {
      const int g = idx / D, d = idx % D;
      float mx = kMaxFloor;
#pragma unroll
      for (int w = 0; w < NW; ++w) mx = fmaxf(mx, lds_m[w][g]);
      float acc = 0.f, lsum = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const float s = __builtin_amdgcn_exp2f(lds_m[w][g] - mx);
        acc += lds_o[w][g][d] * s;
        lsum += lds_l[w][g] * s;
      }
      const float r = lsum > 0.f ? acc / lsum : 0.f;
      ((bf16*)a.o)[(int64_t)b * a.o_stride[0] + (int64_t)(h0 + g) * a.o_stride[1] + d] = (__bf16)r;
    }
    return;
  }
  // merge the 4 waves and write the split's partial row
  float* ws_o = (float*)a.workspace;
  float* ws_ml = ws_o + (int64_t)a.batch * a.q_heads * nsplit * D;
  for (int idx = tid; idx < G * D; idx += 64 * NW) {
    const int g = idx / D, d = idx % D;
    float mx = kMaxFloor;
#pragma unroll
    for (int w = 0; w < NW; ++w) mx = fmaxf(mx, lds_m[w][g]);
    float acc = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) acc += lds_o[w][g][d] * __builtin_amdgcn_exp2f(lds_m[w][g] - mx);
    const int64_t prow = ((int64_t)b * a.q_heads + h0 + g) * nsplit + split;
    store_partial(ws_o + prow * D + d, acc, counters != nullptr);
    if (d == 0) {
      float lsum = 0.f, mraw = kNegInf;
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        lsum += lds_l[w][g] * __builtin_amdgcn_exp2f(lds_m[w][g] - mx);
        mraw = fmaxf(mraw, lds_m[w][g]);
      }
      store_partial(ws_ml + prow * 2 + 0, mraw == kNegInf ? kNegInf : mx, counters != nullptr);
      store_partial(ws_ml + prow * 2 + 1, lsum, counters != nullptr);
    }
  }
  if (!counters) return;  // decode_combine_kernel merges the splits
  // The last split of (b, hk) to finish merges them all. Every thread waits
  // until its coherent partial stores have completed, the workgroup meets,
  // and one lane counts this split with a vector-memory atomic; the split
  // that sees nsplit - 1 earlier counts reads every split's partial with
  // coherent loads, merges, and resets the counter for the next launch.
  __shared__ int last_lds;
  __shared__ float ml_lds[G][kDecodeMergeSplits][2];
  __builtin_amdgcn_s_waitcnt(0);  // vmcnt(0) expcnt(0) lgkmcnt(0): the partial stores have landed
  __syncthreads();
  if (tid == 0) last_lds = atomicAdd(counters + pair, 1) == nsplit - 1;
  __syncthreads();
  if (!last_lds) return;
  // every split's (max, sum) of the G heads into LDS and, in the same round
  // trip, each thread's first output element's rows of the first 8 splits;
  // then each output element from 8 splits' rows at a time: the same terms
  // in the same order as merge_splits
  const int64_t head0 = ((int64_t)b * a.q_heads + h0) * nsplit;  // partial row of (h0, split 0)
  auto orow_of = [&](int idx) { return ws_o + (head0 + (int64_t)(idx / D) * nsplit) * D + idx % D; };
  float first[8];
  if (tid < G * D) {
    const float* orow = orow_of(tid);
#pragma unroll
    for (int u = 0; u < 8; ++u) first[u] = u < nsplit ? load_shared(orow + (int64_t)u * D) : 0.f;
  }
  for (int i = tid; i < G * nsplit * 2; i += 64 * NW) {
    const int g = i / (nsplit * 2), r = i - g * nsplit * 2;
    (&ml_lds[g][0][0])[r] = load_shared(ws_ml + (head0 + (int64_t)g * nsplit) * 2 + r);
  }
  __syncthreads();
  for (int idx = tid; idx < G * D; idx += 64 * NW) {
    const int g = idx / D, d = idx % D;
    const float* orow = orow_of(idx);
    float mx = kMaxFloor;
    for (int s = 0; s < nsplit; ++s) mx = fmaxf(mx, ml_lds[g][s][0]);
    float lsum = 0.f, acc = 0.f;
    for (int s0 = 0; s0 < nsplit; s0 += 8) {
      float ov[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        if (idx == tid && s0 == 0) {
          ov[u] = first[u];
        } else {
          ov[u] = s0 + u < nsplit ? load_shared(orow + (int64_t)(s0 + u) * D) : 0.f;
        }
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        if (s0 + u < nsplit) {
          const float w = __builtin_amdgcn_exp2f(ml_lds[g][s0 + u][0] - mx);
          lsum += ml_lds[g][s0 + u][1] * w;
          acc += ov[u] * w;
        }
      }
    }
    const float r = lsum > 0.f ? acc / lsum : 0.f;
    ((bf16*)a.o)[(int64_t)b * a.o_stride[0] + (int64_t)(h0 + g) * a.o_stride[1] + d] = (__bf16)r;
  }
  if (tid == 0) __hip_atomic_store(counters + pair, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One workgroup of D threads per (b, query head): merge the splits.
__global__ void decode_combine_kernel(const wmx_decode_args a, int nsplit) {
  const int D = a.head_dim;
  const int h = blockIdx.x, b = blockIdx.y, d = threadIdx.x;
  if (d >= D) return;
  const float* ws_o = (const float*)a.workspace;
  const float* ws_ml = ws_o + (int64_t)a.batch * a.q_heads * nsplit * D;
  const float r = merge_splits(ws_o, ws_ml, ((int64_t)b * a.q_heads + h) * nsplit, nsplit, D, d);
  ((bf16*)a.o)[(int64_t)b * a.o_stride[0] + (int64_t)h * a.o_stride[1] + d] = (__bf16)r;
}

int decode_num_splits(const wmx_decode_args& a) {
  if (a.num_splits > 0) return a.num_splits;
  // at least 4 workgroups per CU (256 CUs) and chunks of at most 1024 keys,
  // with chunks of at least kDecodeChunkMin keys (C4, B=32 over 8192 slots:
  // 8 splits, 6.5 TB/s at 16 KV heads against 6.2 at 4 splits and 5.4 at 64)
  const int64_t units = (int64_t)a.batch * a.kv_heads;
  int64_t splits = (4 * 256 + units - 1) / units;
  const int64_t by_chunk = (a.capacity + 1023) / 1024;
  if (splits < by_chunk) splits = by_chunk;
  const int64_t max_splits = (a.capacity + kDecodeChunkMin - 1) / kDecodeChunkMin;
  if (splits > max_splits) splits = max_splits;
  if (splits < 1) splits = 1;
  return (int)splits;
}

int64_t decode_workspace_size(const wmx_decode_args& a) {
  const int64_t s = decode_num_splits(a);
  return (int64_t)a.batch * a.q_heads * s * (a.head_dim + 2) * (int64_t)sizeof(float);
}

template <int D, int G>
static void launch_decode_t(const wmx_decode_args& a, int nsplit, int chunk, int head_offset, hipStream_t stream) {
  const int64_t blocks = (int64_t)nsplit * a.batch * a.kv_heads;  // <= INT32_MAX (checked by the caller)
  int32_t* counters = decode_merges_in_split(a, nsplit) ? a.counters : nullptr;
  // Long launches (beyond the in-split merge's 1024 workgroups, so several
  // rounds per CU) of one head per KV head run eight waves per workgroup:
  // twice the rows in flight per CU (C4 at Hkv 16: 0.181 -> 0.178 ms; head
  // pairs measured slower, 0.105 -> 0.108 ms at Hkv 8). Short launches keep
  // four, whose workgroups all fit in one round (eight-wave workgroups of
  // ~130 registers fit one per CU).
  if (G == 1 && blocks > kDecodeMergeBlocks)
    hipLaunchKernelGGL((decode_split_kernel<D, G, 8>), dim3((unsigned)blocks), dim3(512), 0, stream, a, chunk,
                       head_offset, counters);
  else
    hipLaunchKernelGGL((decode_split_kernel<D, G, 4>), dim3((unsigned)blocks), dim3(256), 0, stream, a, chunk,
                       head_offset, counters);
}

// Any group size: up to 8 query heads share one read of each K/V row; larger
// groups take one launch per 8 heads (and the remainder).
template <int D>
static int launch_decode_d(const wmx_decode_args& a, int nsplit, int chunk, hipStream_t stream) {
  const int group = a.q_heads / a.kv_heads;
  for (int off = 0; off < group; off += 8) {
    switch (group - off < 8 ? group - off : 8) {
      case 1: launch_decode_t<D, 1>(a, nsplit, chunk, off, stream); break;
      case 2: launch_decode_t<D, 2>(a, nsplit, chunk, off, stream); break;
      case 3: launch_decode_t<D, 3>(a, nsplit, chunk, off, stream); break;
      case 4: launch_decode_t<D, 4>(a, nsplit, chunk, off, stream); break;
      case 5: launch_decode_t<D, 5>(a, nsplit, chunk, off, stream); break;
      case 6: launch_decode_t<D, 6>(a, nsplit, chunk, off, stream); break;
      case 7: launch_decode_t<D, 7>(a, nsplit, chunk, off, stream); break;
      default: launch_decode_t<D, 8>(a, nsplit, chunk, off, stream); break;
    }
  }
  return WMX_OK;
}

int launch_decode(const wmx_decode_args& a, hipStream_t stream) {
  if (a.batch == 0 || a.q_heads == 0) return WMX_OK;
  const int nsplit = decode_num_splits(a);
  if ((int64_t)nsplit * a.batch * a.kv_heads > INT32_MAX) return WMX_E_UNSUPPORTED;
  int chunk = (a.capacity + nsplit - 1) / nsplit;
  chunk = (chunk + 63) / 64 * 64;
  if (chunk < 64) chunk = 64;
  int rc;
  switch (a.head_dim) {
    case 64: rc = launch_decode_d<64>(a, nsplit, chunk, stream); break;
    case 96: rc = launch_decode_d<96>(a, nsplit, chunk, stream); break;
    case 128: rc = launch_decode_d<128>(a, nsplit, chunk, stream); break;
    default: return WMX_E_UNSUPPORTED;
  }
  if (rc != WMX_OK) return rc;
  if (nsplit == 1 || decode_merges_in_split(a, nsplit)) return WMX_OK;  // the split kernel wrote the output
  const int threads = (a.head_dim + 63) / 64 * 64;
  hipLaunchKernelGGL(decode_combine_kernel, dim3(a.q_heads, a.batch), dim3(threads), 0, stream, a, nsplit);
  return WMX_OK;
}

}  // namespace wmx

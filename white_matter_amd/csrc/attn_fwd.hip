// Flash-style attention forward for gfx950 (CDNA4), bf16 in, fp32 accumulate.
//
// One workgroup = 4 wave64s = 128 query rows of one (batch or segment,
// query head); each wave owns 32 query rows. Key/value tiles of 64 rows are
// staged through registers into LDS (K row-major, V transposed and
// swizzled) and shared by the 4 waves; the next tile's global loads are in
// flight while the current tile is computed.
//
// Each wave computes S^T = K Q^T so that a lane owns one query column: the
// softmax row statistics are per-lane scalars plus one exchange with
// lane ^ 32, and the output accumulator O^T = V^T P^T is rescaled by a
// per-lane factor (skipped for the whole wave when no row maximum moved).
// P never leaves registers (see the k-order note in wmx_device.h). Masks
// (strided causal bound, per-row offset/limit, key mask, documents, varlen
// segments) are evaluated only on tiles that can contain a masked pair;
// tiles nobody in the workgroup can see are never loaded, and rows beyond
// the workgroup's reach are zero-filled so NaN in unused cache capacity
// cannot leak.
//
// Semantics follow the reference's portable path
// (src/white_matter/ops/cyclic_attention/reference.py:10-42,
//  src/white_matter/ops/strict_causal_attention.py:279-322) with the
// accelerated path's numerics contract (exp2 online softmax with the
// rescale-by-exactly-one guard, natural-log LSE, zero rows for empty
// visibility; _tilelang/forward.py:99-131).
#include "attn_tiles.h"

namespace wmx {

constexpr int kFwdBM = 128;  // query rows per workgroup
constexpr int kFwdBN = 64;   // keys per tile

template <int D, int MODE>
__global__ __launch_bounds__(256, 2) void attn_fwd_kernel(const wmx_attn_args a) {
  constexpr int BM = kFwdBM, BN = kFwdBN;
  constexpr int KLD = D + 8;     // K tile row stride (elements): per-row 16-byte operand reads
  constexpr int VLD = tr_ld(D);  // V tile row stride (elements): transpose reads
  constexpr int KS = D / 16;  // MFMA k-steps over head_dim
  constexpr int DB = D / 32;  // 32-row blocks of O^T

  __shared__ __attribute__((aligned(16))) bf16 k_lds[BN * KLD];
  __shared__ __attribute__((aligned(16))) bf16 v_lds[BN * VLD];
  __shared__ int kseg_lds[BN];
  __shared__ int kqend_lds[BN];
  __shared__ int red_lds[4];

  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int half = lane >> 5, col = lane & 31;

  // ---- resolve the problem this workgroup works on ----
  const int qtiles = ((MODE == kVarlen ? a.max_queries : a.q_len) + BM - 1) / BM;
  const unsigned outer = MODE == kVarlen ? (unsigned)a.num_segments : (unsigned)a.batch;
  unsigned unit;
  if (!logical_unit((unsigned)qtiles * outer * a.q_heads, unit)) return;
  const int q0 = (qtiles - 1 - (int)(unit % qtiles)) * BM;
  const unsigned rest = unit / qtiles;
  const int h = MODE == kVarlen ? (int)(rest / outer) : (int)(rest % a.q_heads);
  const int grp = MODE == kVarlen ? (int)(rest % outer) : (int)(rest / a.q_heads);
  const int hk = h / (a.q_heads / a.kv_heads);
  Problem<MODE> pb;
  pb.init(a, grp);
  const int b = pb.b, nq = pb.nq, nk = pb.nk;
  if (q0 >= nq) return;
  auto lim_of = [&](int i) { return pb.bound.lim(i); };
  const bool slot0 = a.keep_slot0 && nk > 0;
  const int lim_max_wg = lim_of(min(q0 + BM, nq) - 1);

  // ---- this lane's query row ----
  const int i = q0 + wave * 32 + col;
  const bool valid_q = i < nq;
  const int lim_i = lim_of(i);
  const int wave_first = q0 + wave * 32;
  const bool wave_live = wave_first < nq;
  const int lim_min_wave = lim_of(wave_first);
  const int lim_max_wave = lim_of(min(wave_first + 31, nq - 1));

  int qb, qt;
  pb.query_loc(valid_q ? i : q0, qb, qt);
  bf16x8 qf[KS];
  {
    const bf16* qrow = (const bf16*)a.q + (int64_t)qb * a.q_stride[0] + (int64_t)h * a.q_stride[1] +
                       (int64_t)qt * a.q_stride[2] + 8 * half;
    const u32x4 z = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const u32x4 w = load16(qrow + 16 * s);
      qf[s] = as_bf16x8(valid_q ? w : z);
    }
  }

  int qseg_i = 0, qstart_i = 0, kt_begin_main = 0;
  if constexpr (MODE == kDoc) {
    if (valid_q) {
      qseg_i = a.q_seg[(int64_t)b * a.q_len + i];
      qstart_i = a.q_start[(int64_t)b * a.q_len + i];
    }
    // smallest document start over the workgroup's rows bounds the first key tile
    int v = INT_MAX;
    if (tid < BM && q0 + tid < nq) v = a.q_start[(int64_t)b * a.q_len + q0 + tid];
    for (int o = 32; o > 0; o >>= 1) v = min(v, __shfl_xor(v, o));
    if (lane == 0) red_lds[wave] = v;
    __syncthreads();
    v = min(min(red_lds[0], red_lds[1]), min(red_lds[2], red_lds[3]));
    kt_begin_main = v < 0 ? 0 : v / BN;
  }
  // document of this wave's rows when they all share one (ids are sorted)
  int qseg_w = 0, qstart_w = 0;
  bool q_uniform = false;
  if constexpr (MODE == kDoc) {
    qseg_w = __builtin_amdgcn_readfirstlane(qseg_i);
    q_uniform = __all(!valid_q || qseg_i == qseg_w);
    int v = valid_q ? qstart_i : INT_MIN;
    for (int o = 32; o > 0; o >>= 1) v = max(v, __shfl_xor(v, o));
    qstart_w = __builtin_amdgcn_readfirstlane(v);  // largest document start of the wave's rows
  }

  // ---- key tile range: tile 0 stays when it holds the shared dummy ----
  int kt_end = (lim_max_wg + 1 + BN - 1) / BN;
  if (slot0 && kt_end < 1) kt_end = 1;
  const int first_main = kt_begin_main > 1 ? kt_begin_main : 1;
  const bool gap = (MODE == kDoc) && first_main > 1;
  const int ntiles = gap ? 1 + max(0, kt_end - first_main) : kt_end;
  auto tile_of = [&](int it) { return gap ? (it == 0 ? 0 : first_main + it - 1) : it; };

  // key row j of this problem as a global pointer into K (or V)
  auto key_ptr = [&](const void* base, const int64_t* st, int j, bool& ok) -> const bf16* {
    ok = j < nk && (j <= lim_max_wg || (slot0 && j == 0));
    if (MODE == kDense && a.key_mask) ok = ok && a.key_mask[(int64_t)b * a.key_mask_stride + min(j, nk - 1)] != 0;
    int kb, kt;
    pb.key_loc(ok ? j : 0, kb, kt);
    return row_at(base, st, kb, hk, kt);
  };
  // Affine key rows (dense rows, or a varlen segment whose keys 1.. are
  // consecutive slots of one row): slot(j) = first + j for j >= 1 and key 0
  // at slot0, read from a per-workgroup slice base.
  const bool affine = MODE != kVarlen || (a.segment_layout & kKeysConsecutive);
  int kb0 = b, kslot0 = 0, kfirst = 0;
  if (nk > 0) {
    pb.key_loc(0, kb0, kslot0);
    if (nk > 1) {
      int kb1, kslot1;
      pb.key_loc(1, kb1, kslot1);
      kfirst = kslot1 - 1;
    } else {
      kfirst = kslot0;
    }
  }
  const bf16* kslice = row_at(a.k, a.k_stride, kb0, hk, 0);
  const bf16* vslice = row_at(a.v, a.v_stride, kb0, hk, 0);
  const int64_t kst = a.k_stride[2], vst = a.v_stride[2];
  // a tile whose rows are all in range and inside the workgroup's reach
  auto tile_full = [&](int n0) {
    return affine && !(MODE == kDense && a.key_mask) && n0 + BN <= nk && n0 + BN - 1 <= lim_max_wg && n0 > 0;
  };

  PairTile<BN, D> ktile, vtile;
  auto load_tile = [&](int n0) {
    if (tile_full(n0)) {
      ktile.load(tid, [&](int r, bool& ok) { ok = true; return kslice + (int64_t)(kfirst + n0 + r) * kst; });
      vtile.load(tid, [&](int r, bool& ok) { ok = true; return vslice + (int64_t)(kfirst + n0 + r) * vst; });
    } else {
      ktile.load(tid, [&](int r, bool& ok) { return key_ptr(a.k, a.k_stride, n0 + r, ok); });
      vtile.load(tid, [&](int r, bool& ok) { return key_ptr(a.v, a.v_stride, n0 + r, ok); });
    }
  };

  f32x16 oacc[DB];
#pragma unroll
  for (int d = 0; d < DB; ++d) oacc[d] = f32x16{};
  float m_run = kNegInf, l_run = 0.f;
  const float sl2 = a.softmax_scale * kLog2e;  // > 0 (checked on the host)

  // One key tile of this wave's online softmax and PV product.
  auto tile_step = [&](int n0, bool masked) {
    f32x16 sacc[BN / 32];
#pragma unroll
    for (int nb = 0; nb < BN / 32; ++nb) {
      sacc[nb] = f32x16{};
#pragma unroll
      for (int s = 0; s < KS; ++s)
        sacc[nb] = mfma32(lds_row_operand(k_lds, KLD, nb * 32 + col, s, half), qf[s], sacc[nb]);
    }

    if (masked) {
      // keeps this block a real (wave-uniform) branch instead of selects
      __asm__ volatile("");
#pragma unroll
      for (int nb = 0; nb < BN / 32; ++nb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int jl = nb * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
          const int j = n0 + jl;
          bool keep = (j <= lim_i) || (slot0 && j == 0);
          if constexpr (MODE == kDense) {
            if (a.key_mask) keep = keep && kseg_lds[jl] != 0;
          }
          if constexpr (MODE == kDoc) {
            const int ksg = kseg_lds[jl];
            keep = keep && j < nk && ((ksg == qseg_i && j >= qstart_i) || ksg == -1) && (i < kqend_lds[jl]);
          }
          sacc[nb][r] = keep ? sacc[nb][r] : kNegInf;
        }
      }
    }
    float rmax = kNegInf;
#pragma unroll
    for (int nb = 0; nb < BN / 32; ++nb)
#pragma unroll
      for (int r = 0; r < 16; ++r) rmax = fmaxf(rmax, sacc[nb][r]);
    rmax = max_halves(rmax);
    const float m_new = fmaxf(m_run, rmax * sl2);
    const float m_use = fmaxf(m_new, kMaxFloor);
    float rsum = 0.f;
#pragma unroll
    for (int nb = 0; nb < BN / 32; ++nb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = __builtin_amdgcn_exp2f(fmaf(sacc[nb][r], sl2, -m_use));
        sacc[nb][r] = p;
        rsum += p;
      }
    }
    rsum = sum_halves(rsum);
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
    l_run = l_run * alpha + rsum;
    m_run = m_new;
    if (__any(alpha != 1.f)) {
#pragma unroll
      for (int d = 0; d < DB; ++d) oacc[d] *= alpha;
    }

#pragma unroll
    for (int s = 0; s < BN / 16; ++s) {
      const bf16x8 pb = acc_kperm_operand(sacc[s >> 1], s);
#pragma unroll
      for (int d = 0; d < DB; ++d) oacc[d] = mfma32(lds_tr_operand(v_lds, VLD, d * 32, s, lane), pb, oacc[d]);
    }
  };

  if (ntiles > 0) load_tile(tile_of(0) * BN);
  for (int it = 0; it < ntiles; ++it) {
    const int n0 = tile_of(it) * BN;
    __syncthreads();
    ktile.store_rows(tid, k_lds, KLD);
    vtile.store_rows(tid, v_lds, VLD);
    if constexpr (MODE == kDoc) {
      if (tid < BN) {
        const int j = n0 + tid;
        kseg_lds[tid] = j < nk ? a.k_seg[(int64_t)b * a.kv_len + j] : INT_MIN;
        kqend_lds[tid] = j < nk ? a.k_qend[(int64_t)b * a.kv_len + j] : 0;
      }
    } else if constexpr (MODE == kDense) {
      if (a.key_mask && tid < BN) {
        const int j = n0 + tid;
        kseg_lds[tid] = j < nk ? (int)a.key_mask[(int64_t)b * a.key_mask_stride + j] : 0;
      }
    }
    __syncthreads();
    if (it + 1 < ntiles) load_tile(tile_of(it + 1) * BN);

    const bool wave_sees = wave_live && (n0 <= lim_max_wave || (slot0 && n0 == 0));
    if (!wave_sees) continue;

    // Per-element masks are needed on the causal diagonal, at document
    // boundaries and under a key mask; the wave decides uniformly.
    bool masked = !((n0 + BN - 1 <= lim_min_wave) && (n0 + BN <= nk));
    if constexpr (MODE == kDense) masked = masked || a.key_mask != nullptr;
    if constexpr (MODE == kDoc) {
      // a tile is document-interior for this wave when all 32 query ids and
      // all 64 key ids equal one id: the document rule then keeps every pair
      // (with n0 >= every row's document start and every key's query end past
      // the wave's last row, all three parts of the document rule hold)
      const int i_last = min(wave_first + 31, nq - 1);
      masked = masked || !(q_uniform && n0 >= qstart_w && __all(kseg_lds[lane] == qseg_w && kqend_lds[lane] > i_last));
    }
    tile_step(n0, masked);
  }

  if (!valid_q) return;
  const float inv = l_run > 0.f ? 1.f / l_run : 0.f;
  bf16* orow = (bf16*)a.o + (int64_t)qb * a.o_stride[0] + (int64_t)h * a.o_stride[1] + (int64_t)qt * a.o_stride[2];
  store_acc_row<DB>(orow, oacc, inv, half);
  if (half == 0) {
    const float lse = l_run > 0.f ? (m_run + __log2f(l_run)) * kLn2 : kPosInf;
    a.lse[((int64_t)qb * a.q_heads + h) * a.q_len + qt] = lse;
  }
}

template <int D, int MODE>
static int launch_fwd_t(const wmx_attn_args& a, hipStream_t stream) {
  const int64_t qtiles = ((MODE == kVarlen ? a.max_queries : a.q_len) + kFwdBM - 1) / kFwdBM;
  const int64_t outer = MODE == kVarlen ? a.num_segments : a.batch;
  const int64_t units = qtiles * outer * a.q_heads;
  if (units <= 0) return WMX_OK;
  const int64_t blocks = logical_grid(units);
  if (blocks > INT_MAX) return WMX_E_UNSUPPORTED;
  hipLaunchKernelGGL((attn_fwd_kernel<D, MODE>), dim3((unsigned)blocks), dim3(256), 0, stream, a);
  return WMX_OK;
}

template <int MODE>
static int launch_fwd_mode(const wmx_attn_args& a, hipStream_t stream) {
  switch (a.head_dim) {
    case 64: return launch_fwd_t<64, MODE>(a, stream);
    case 96: return launch_fwd_t<96, MODE>(a, stream);
    case 128: return launch_fwd_t<128, MODE>(a, stream);
    default: return WMX_E_UNSUPPORTED;
  }
}

int launch_fwd(const wmx_attn_args& a, hipStream_t stream) {
  if (a.query_indices) return launch_fwd_mode<kVarlen>(a, stream);
  if (a.q_seg) return launch_fwd_mode<kDoc>(a, stream);
  return launch_fwd_mode<kDense>(a, stream);
}

}  // namespace wmx

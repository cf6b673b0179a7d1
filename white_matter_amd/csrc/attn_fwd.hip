// Flash-style attention forward for gfx950 (CDNA4), bf16 in, fp32 accumulate.
//
// One workgroup = 4 wave64s = 128 query rows of one (batch, query head);
// each wave owns 32 query rows. Key/value tiles of 64 rows are staged in
// LDS (K row-major, V transposed) and shared by the 4 waves.
//
// Each wave computes S^T = K Q^T so that a lane owns one query column: the
// softmax row statistics are then per-lane scalars plus one exchange with
// lane ^ 32, and the output accumulator O^T = V^T P^T is rescaled by a
// per-lane factor. P never leaves registers (see the k-order note in
// wmx_device.h). Masking (strided causal bound, per-row offset/limit,
// key mask, documents, varlen segments) is evaluated only on tiles that
// can contain a masked pair; tiles nobody in the workgroup can see are
// never loaded (tile skipping), and rows beyond the workgroup's reach are
// zero-filled on load so that NaN in unused cache capacity cannot leak.
//
// Semantics follow the reference's portable path
// (src/white_matter/ops/cyclic_attention/reference.py:10-42,
//  src/white_matter/ops/strict_causal_attention.py:279-322) and its
// numerics contract (exp2 online softmax with the rescale-by-exactly-one
// guard, natural-log LSE, zero rows for empty visibility).
#include <climits>

#include "wmx_kernels.h"

namespace wmx {

template <int D>
struct FwdTile {
  static constexpr int BM = 128;
  static constexpr int BN = 64;
  static constexpr int KLD = D + 8;   // K tile row stride (elements)
  static constexpr int VLD = BN + 8;  // V^T tile row stride (elements)
};

template <int D, int MODE>
__global__ __launch_bounds__(256) void attn_fwd_kernel(const wmx_attn_args a) {
  using Tl = FwdTile<D>;
  constexpr int BM = Tl::BM, BN = Tl::BN, KLD = Tl::KLD, VLD = Tl::VLD;
  constexpr int KS = D / 16;          // MFMA k-steps over head_dim
  constexpr int DB = D / 32;          // 32-row blocks of O^T
  constexpr int CPR = D / 8;          // 16-byte chunks per row
  constexpr int KCH = BN * CPR / 256; // K chunks per thread
  constexpr int VCH = (BN / 2 * CPR + 255) / 256;  // V row-pair chunks per thread

  __shared__ __attribute__((aligned(16))) bf16 k_lds[BN * KLD];
  __shared__ __attribute__((aligned(16))) bf16 vt_lds[D * VLD];
  __shared__ int kseg_lds[BN];
  __shared__ int kqend_lds[BN];
  __shared__ int red_lds[4];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int half = lane >> 5, col = lane & 31;
  const int h = blockIdx.y;
  const int hk = h / (a.q_heads / a.kv_heads);

  // ---- resolve the problem this workgroup works on ----
  int b = 0, nq, nk, q0, qs = 0, ks = 0;
  int64_t offset, limit, qstride;
  if constexpr (MODE == kVarlen) {
    const int qtiles = (a.max_queries + BM - 1) / BM;
    const int seg = blockIdx.x / qtiles;
    const int tile = qtiles - 1 - (int)(blockIdx.x % qtiles);
    qs = a.cu_queries[seg];
    nq = a.cu_queries[seg + 1] - qs;
    ks = a.cu_keys[seg];
    nk = a.cu_keys[seg + 1] - ks;
    q0 = tile * BM;
    if (q0 >= nq) return;
    offset = nk - nq;
    limit = INT_MAX;
    qstride = 1;
  } else {
    b = blockIdx.z;
    nq = a.q_len;
    nk = a.kv_len;
    q0 = (gridDim.x - 1 - blockIdx.x) * BM;
    offset = a.row_offset ? a.row_offset[b] : a.query_offset;
    limit = a.row_limit ? a.row_limit[b] : INT_MAX;
    qstride = a.query_stride;
  }
  auto lim_of = [&](int i) -> int {
    int64_t l = offset + qstride * (int64_t)i;
    l = l < limit ? l : limit;
    l = l < (int64_t)nk - 1 ? l : (int64_t)nk - 1;
    return (int)(l < -1 ? -1 : l);
  };
  const int q_last = min(q0 + BM, nq) - 1;
  const int lim_max_wg = lim_of(q_last);
  const bool slot0 = a.keep_slot0 && nk > 0;

  // ---- this lane's query row ----
  const int i = q0 + wave * 32 + col;
  const bool valid_q = i < nq;
  const int lim_i = lim_of(i);
  const int wave_first = q0 + wave * 32;
  const bool wave_live = wave_first < nq;
  const int lim_min_wave = lim_of(wave_first);
  const int lim_max_wave = lim_of(min(wave_first + 31, nq - 1));

  int qb = b, qt = i;
  if constexpr (MODE == kVarlen) {
    if (valid_q) split_flat(a.query_indices[qs + i], a.query_extent, qb, qt);
  }
  const RowSource qsrc{(const bf16*)a.q, a.q_stride[0], a.q_stride[1], a.q_stride[2]};
  bf16x8 qf[KS];
  {
    const bf16* qrow = row_ptr(qsrc, qb, h, qt);
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      u32x4 w = {0u, 0u, 0u, 0u};
      if (valid_q) w = load16(qrow + 16 * s + 8 * half);
      qf[s] = as_bf16x8(w);
    }
  }

  int qseg_i = 0, qstart_i = 0;
  int kt_begin_main = 0;
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

  // ---- key tile range ----
  int kt_end = (lim_max_wg + 1 + BN - 1) / BN;
  if (slot0 && kt_end < 1) kt_end = 1;
  const int first_main = kt_begin_main > 1 ? kt_begin_main : 1;
  const bool gap = (MODE == kDoc) && first_main > 1;
  const int ntiles = gap ? 1 + max(0, kt_end - first_main) : kt_end;
  auto tile_of = [&](int it) { return gap ? (it == 0 ? 0 : first_main + it - 1) : it; };

  const RowSource ksrc{(const bf16*)a.k, a.k_stride[0], a.k_stride[1], a.k_stride[2]};
  const RowSource vsrc{(const bf16*)a.v, a.v_stride[0], a.v_stride[1], a.v_stride[2]};
  auto key_row_valid = [&](int j) -> bool {
    if (j >= nk) return false;
    if (!(j <= lim_max_wg || (slot0 && j == 0))) return false;
    if (MODE == kDense && a.key_mask) return a.key_mask[(int64_t)b * a.key_mask_stride + j] != 0;
    return true;
  };
  auto key_loc = [&](int j, int& kb, int& kt) {
    if constexpr (MODE == kVarlen) {
      split_flat(a.key_indices[ks + j], a.key_extent, kb, kt);
    } else {
      kb = b;
      kt = j;
    }
  };

  u32x4 kreg[KCH];
  u32x4 vreg[VCH][2];
  auto load_tile = [&](int n0) {
#pragma unroll
    for (int r = 0; r < KCH; ++r) {
      const int c = tid + 256 * r;
      const int row = c / CPR, cc = c % CPR;
      const int j = n0 + row;
      u32x4 w = {0u, 0u, 0u, 0u};
      if (key_row_valid(j)) {
        int kb, kt;
        key_loc(j, kb, kt);
        w = load16(row_ptr(ksrc, kb, hk, kt) + 8 * cc);
      }
      kreg[r] = w;
    }
#pragma unroll
    for (int r = 0; r < VCH; ++r) {
      const int c = tid + 256 * r;
      const int p = c / CPR, cc = c % CPR;
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int j = n0 + 2 * p + u;
        u32x4 w = {0u, 0u, 0u, 0u};
        if (c < BN / 2 * CPR && key_row_valid(j)) {
          int kb, kt;
          key_loc(j, kb, kt);
          w = load16(row_ptr(vsrc, kb, hk, kt) + 8 * cc);
        }
        vreg[r][u] = w;
      }
    }
  };
  auto store_tile = [&](int n0) {
#pragma unroll
    for (int r = 0; r < KCH; ++r) {
      const int c = tid + 256 * r;
      const int row = c / CPR, cc = c % CPR;
      *reinterpret_cast<u32x4*>(&k_lds[row * KLD + 8 * cc]) = kreg[r];
    }
#pragma unroll
    for (int r = 0; r < VCH; ++r) {
      const int c = tid + 256 * r;
      if (c < BN / 2 * CPR) {
        const int p = c / CPR, cc = c % CPR;
        const u32x4 x = vreg[r][0], y = vreg[r][1];
        uint32_t* dst = reinterpret_cast<uint32_t*>(&vt_lds[(8 * cc) * VLD + 2 * p]);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          dst[(2 * e) * (VLD / 2)] = (x[e] & 0xffffu) | (y[e] << 16);
          dst[(2 * e + 1) * (VLD / 2)] = (x[e] >> 16) | (y[e] & 0xffff0000u);
        }
      }
    }
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
  };

  f32x16 oacc[DB];
#pragma unroll
  for (int d = 0; d < DB; ++d) oacc[d] = f32x16{};
  float m_run = kNegInf, l_run = 0.f;
  const float sl2 = a.softmax_scale * kLog2e;

  if (ntiles > 0) load_tile(tile_of(0) * BN);
  for (int it = 0; it < ntiles; ++it) {
    const int n0 = tile_of(it) * BN;
    __syncthreads();
    store_tile(n0);
    __syncthreads();
    if (it + 1 < ntiles) load_tile(tile_of(it + 1) * BN);

    const bool wave_sees = wave_live && (n0 <= lim_max_wave || (slot0 && n0 == 0));
    if (!wave_sees) continue;

    f32x16 sacc[BN / 32];
#pragma unroll
    for (int nb = 0; nb < BN / 32; ++nb) {
      sacc[nb] = f32x16{};
      const bf16* krow = &k_lds[(nb * 32 + col) * KLD + 8 * half];
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        sacc[nb] = mfma32(as_bf16x8(*reinterpret_cast<const u32x4*>(krow + 16 * s)), qf[s], sacc[nb]);
      }
    }

    const bool full = (MODE != kDoc) && !(MODE == kDense && a.key_mask) && (n0 + BN - 1 <= lim_min_wave) &&
                      (n0 + BN <= nk);
    float rmax = kNegInf;
#pragma unroll
    for (int nb = 0; nb < BN / 32; ++nb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float x = sacc[nb][r] * sl2;
        if (!full) {
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
          x = keep ? x : kNegInf;
        }
        sacc[nb][r] = x;
        rmax = fmaxf(rmax, x);
      }
    }
    rmax = fmaxf(rmax, xor32(rmax));
    const float m_new = fmaxf(m_run, rmax);
    const float m_use = fmaxf(m_new, kMaxFloor);
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
    float rsum = 0.f;
#pragma unroll
    for (int nb = 0; nb < BN / 32; ++nb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = __builtin_amdgcn_exp2f(sacc[nb][r] - m_use);
        sacc[nb][r] = p;
        rsum += p;
      }
    }
    rsum += xor32(rsum);
    l_run = l_run * alpha + rsum;
    m_run = m_new;
#pragma unroll
    for (int d = 0; d < DB; ++d) oacc[d] *= alpha;

#pragma unroll
    for (int s = 0; s < BN / 16; ++s) {
      const f32x16& src = sacc[s >> 1];
      const int base = 8 * (s & 1);
      u32x4 pw;
      pw[0] = pack_bf16x2(src[base + 0], src[base + 1]);
      pw[1] = pack_bf16x2(src[base + 2], src[base + 3]);
      pw[2] = pack_bf16x2(src[base + 4], src[base + 5]);
      pw[3] = pack_bf16x2(src[base + 6], src[base + 7]);
      const bf16x8 pb = as_bf16x8(pw);
#pragma unroll
      for (int d = 0; d < DB; ++d) {
        const bf16* vrow = &vt_lds[(d * 32 + col) * VLD + 16 * s + 4 * half];
        const u32x2 lo = *reinterpret_cast<const u32x2*>(vrow);
        const u32x2 hi = *reinterpret_cast<const u32x2*>(vrow + 8);
        const u32x4 va = {lo[0], lo[1], hi[0], hi[1]};
        oacc[d] = mfma32(as_bf16x8(va), pb, oacc[d]);
      }
    }
  }

  if (!valid_q) return;
  const float inv = l_run > 0.f ? 1.f / l_run : 0.f;
  int ob = b, ot = i;
  if constexpr (MODE == kVarlen) { ob = qb; ot = qt; }
  bf16* orow = (bf16*)a.o + (int64_t)ob * a.o_stride[0] + (int64_t)h * a.o_stride[1] + (int64_t)ot * a.o_stride[2];
#pragma unroll
  for (int d = 0; d < DB; ++d) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      u32x2 w;
      w[0] = pack_bf16x2(oacc[d][4 * g + 0] * inv, oacc[d][4 * g + 1] * inv);
      w[1] = pack_bf16x2(oacc[d][4 * g + 2] * inv, oacc[d][4 * g + 3] * inv);
      store8(orow + d * 32 + 8 * g + 4 * half, w);
    }
  }
  if (half == 0) {
    const float lse = l_run > 0.f ? (m_run + __log2f(l_run)) * kLn2 : kPosInf;
    a.lse[((int64_t)ob * a.q_heads + h) * a.q_len + ot] = lse;
  }
}

template <int D, int MODE>
static int launch_fwd_t(const wmx_attn_args& a, hipStream_t stream) {
  constexpr int BM = FwdTile<D>::BM;
  dim3 grid;
  if (MODE == kVarlen) {
    if (a.num_segments <= 0 || a.max_queries <= 0) return WMX_OK;
    const int64_t qtiles = (a.max_queries + BM - 1) / BM;
    grid = dim3((unsigned)(qtiles * a.num_segments), a.q_heads, 1);
  } else {
    grid = dim3((a.q_len + BM - 1) / BM, a.q_heads, a.batch);
  }
  hipLaunchKernelGGL((attn_fwd_kernel<D, MODE>), grid, dim3(256), 0, stream, a);
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

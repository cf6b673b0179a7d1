// Flash-style attention forward for gfx950 (CDNA4), bf16 in, fp32 accumulate.
//
// One workgroup = NW wave64s (4, or 8 for query_tile 256) = 32 NW query rows
// of one (batch row or varlen segment, query head); each wave owns 32 rows. Key/value tiles of 64
// rows go from global memory straight into double-buffered LDS (direct-to-LDS
// loads, no staging registers): the next tile streams in while the current
// one is computed. Rows outside the problem or past the workgroup's reach
// arrive as zeros, so NaN in unused cache capacity cannot leak.
//
// Each wave computes S^T = K Q^T so that a lane owns one query column: the
// softmax row statistics are per-lane scalars plus one exchange with
// lane ^ 32, and the output accumulator O^T = V^T P^T is rescaled by a
// per-lane factor (skipped for the whole wave when no row maximum moved).
// P never leaves registers (see the k-order note in wmx_device.h); V^T is
// read from the row-major V tile with transpose reads. Masks (strided causal
// bound, per-row offset/limit, key mask, documents, varlen segments) are
// evaluated only on tiles that can contain a masked pair; tiles nobody in the
// workgroup can see are never loaded.
//
// Semantics follow the reference's portable path
// (src/white_matter/ops/cyclic_attention/reference.py:10-42,
//  src/white_matter/ops/strict_causal_attention.py:279-322) with the
// accelerated path's numerics contract (exp2 online softmax with the
// rescale-by-exactly-one guard, natural-log LSE, zero rows for empty
// visibility; _tilelang/forward.py:99-131).
#include <type_traits>

#include "attn_tiles.h"

namespace wmx {

constexpr int kFwdBN = 64;  // keys per tile

// NW waves of 32 query rows each: 4 (128 rows, two workgroups per CU) by
// default; 8 (256 rows, one per CU) when few query tiles share long key
// ranges, so each key/value tile streamed from HBM serves twice the rows.
template <int D, int MODE, int NW>
__global__ __launch_bounds__(64 * NW, NW == 4 ? 2 : 1) void attn_fwd_kernel(const wmx_attn_args args) {
  const wmx_attn_args& a = args;
  constexpr int BM = 32 * NW, BN = kFwdBN;
  static_assert(BN == kTileRows, "one LDS tile per key tile");
  constexpr int KS = D / 16;  // MFMA k-steps over head_dim
  constexpr int DB = D / 32;  // 32-row blocks of O^T

  // Two buffers indexed by compile-time constants only (the tile loop is
  // unrolled by two): the compiler then sees that loads streaming into one
  // buffer never alias reads of the other and does not wait for the prefetch
  // before computing, and buffer offsets fold into instruction immediates.
  __shared__ __attribute__((aligned(1024))) bf16 k_lds0[kTileElems];
  __shared__ __attribute__((aligned(1024))) bf16 k_lds1[kTileElems];
  __shared__ __attribute__((aligned(1024))) bf16 v_lds0[kTileElems];
  __shared__ __attribute__((aligned(1024))) bf16 v_lds1[kTileElems];
  __shared__ int meta_lds[2][2][BN];  // per buffer: key ids (or key mask), key query ends
  __shared__ int red_lds[NW];

  // ---- the work units: (batch row or segment, query tile, head) ----
  const int qtiles = ((MODE == kVarlen ? a.max_queries : a.q_len) + BM - 1) / BM;
  const unsigned outer = MODE == kVarlen ? (unsigned)a.num_segments : (unsigned)a.batch;
  const int32_t* list = a.q_units;  // (batch row or segment, tile) pairs, heaviest first
  const uint32_t count = list ? (uint32_t)a.num_q_units : (uint32_t)qtiles * outer;

  // this workgroup's unit: BM query rows of one (batch row or segment, query head)
  TileUnit tu;
  tu.decode(a.q_heads, count, list != nullptr, qtiles, list, (int)outer, true,  // heaviest (last) query tiles first
            MODE == kVarlen ? a.unit_fields : 2);
  if (!tu.ok) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int half = lane >> 5, col = lane & 31;
  const int q0 = tu.tile * BM;
  const int h = tu.head, grp = tu.grp;
  const int hk = h / (a.q_heads / a.kv_heads);
  Problem<MODE> pb;
  pb.init(a, grp, tu);
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
    v = red_lds[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) v = min(v, red_lds[w]);
    kt_begin_main = __builtin_amdgcn_readfirstlane(v < 0 ? 0 : v / BN);  // uniform: keeps the tile loop scalar
  }
  // document of this wave's rows when they all share one (ids are sorted),
  // and the smallest document start of its rows: the wave sees no key below
  // it outside tile 0 (which holds the only keys of every document, as in
  // the reference's tile skipping)
  int qseg_w = 0, qstart_w = 0, qstart_min_w = 0;
  bool q_uniform = false;
  if constexpr (MODE == kDoc) {
    qseg_w = __builtin_amdgcn_readfirstlane(qseg_i);
    q_uniform = __all(!valid_q || qseg_i == qseg_w);
    int v = valid_q ? qstart_i : INT_MIN, u = valid_q ? qstart_i : INT_MAX;
    for (int o = 32; o > 0; o >>= 1) {
      v = max(v, __shfl_xor(v, o));
      u = min(u, __shfl_xor(u, o));
    }
    qstart_w = __builtin_amdgcn_readfirstlane(v);  // largest document start of the wave's rows
    qstart_min_w = __builtin_amdgcn_readfirstlane(u);
  }

  // ---- key tile range: tile 0 stays when it holds the shared dummy ----
  int kt_end = (lim_max_wg + 1 + BN - 1) / BN;
  if (slot0 && kt_end < 1) kt_end = 1;
  const int first_main = kt_begin_main > 1 ? kt_begin_main : 1;
  const bool gap = (MODE == kDoc) && first_main > 1;
  const int ntiles = gap ? 1 + max(0, kt_end - first_main) : kt_end;
  auto tile_of = [&](int it) { return gap ? (it == 0 ? 0 : first_main + it - 1) : it; };

  // ---- key/value tiles: keys [0, reach) are visible to some row of the workgroup ----
  TileDMA<D, NW> dma;
  dma.init(wave, lane);
  KeyTiles<MODE, D, NW> keys;
  keys.init(a, pb, hk, slot0 ? max(lim_max_wg + 1, 1) : lim_max_wg + 1, dma);
  // masking metadata of a key tile, loaded into a register while the tile
  // streams in and stored to LDS once the previous buffer is free
  auto load_meta = [&](int n0) -> int {
    const int j = n0 + (tid & 63);
    if constexpr (MODE == kDoc) {
      if (tid < 64) return j < nk ? a.k_seg[(int64_t)b * a.kv_len + j] : INT_MIN;
      if (tid < 128) return j < nk ? a.k_qend[(int64_t)b * a.kv_len + j] : 0;
    } else if constexpr (MODE == kDense) {
      if (a.key_mask && tid < 64) return j < nk ? (int)a.key_mask[(int64_t)b * a.key_mask_stride + j] : 0;
    }
    return 0;
  };
  auto store_meta = [&](int buf, int v) {
    if (MODE == kDoc || (MODE == kDense && a.key_mask)) {
      if (tid < 128) meta_lds[buf][tid >> 6][tid & 63] = v;
    }
  };

  f32x16 oacc[DB];
#pragma unroll
  for (int d = 0; d < DB; ++d) oacc[d] = f32x16{};
  float m_run = kNegInf, l_run = 0.f;
  const float sl2 = a.softmax_scale * kLog2e;  // > 0 (checked on the host)

  // One key tile of this wave's online softmax and PV product.
  RowReads<KS> krd;
  krd.init(col, half);
  TrReads<DB> vrd;
  vrd.init(lane);
  auto tile_step = [&](int n0, int buf, const bf16* kt, const bf16* vt, bool masked) __attribute__((always_inline)) {
    krd.refresh();
    vrd.refresh();
    f32x16 sacc[BN / 32];
#pragma unroll
    for (int nb = 0; nb < BN / 32; ++nb) sacc[nb] = f32x16{};
    // k-step major, each operand read PF k-steps ahead of its product (the
    // scheduling barriers keep the compiler from sinking the reads next to
    // their uses, where every product would wait out the LDS latency)
    constexpr int PF = KS < 4 ? KS : 4;
    bf16x8 kop[KS][BN / 32];
#pragma unroll
    for (int s = 0; s < PF; ++s) {
#pragma unroll
      for (int nb = 0; nb < BN / 32; ++nb) kop[s][nb] = krd.get(kt, s, nb);
    }
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      __builtin_amdgcn_sched_barrier(0);
      if (s + PF < KS) {
#pragma unroll
        for (int nb = 0; nb < BN / 32; ++nb) kop[s + PF][nb] = krd.get(kt, s + PF, nb);
      }
#pragma unroll
      for (int nb = 0; nb < BN / 32; ++nb) sacc[nb] = mfma32(kop[s][nb], qf[s], sacc[nb]);
    }
    __builtin_amdgcn_sched_barrier(0);

    if (masked) {
      // keeps this block a real (wave-uniform) branch instead of selects
      __asm__ volatile("");
      // element r of block nb holds key j = n0 + 4 half + c with the constant
      // c = 32 nb + 8 (r / 4) + r % 4: the rules become compares of c against
      // per-lane bounds formed once per tile
      const int base = n0 + 4 * half;
      const int lim_c = lim_i - base;                         // j <= lim_i
      const bool dummy_here = slot0 && n0 == 0 && half == 0;  // j == 0 is c == 0 there
      const int nk_c = nk - base, qstart_c = qstart_i - base; // j < nk, j >= qstart_i
#pragma unroll
      for (int nb = 0; nb < BN / 32; ++nb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int c = nb * 32 + 8 * (r >> 2) + (r & 3);
          const int jl = c + 4 * half;  // key within the tile (LDS metadata index)
          // bitwise forms: every term is evaluated, no per-lane branches
          bool keep = c <= lim_c;
          if (c == 0) keep = keep | dummy_here;
          if constexpr (MODE == kDense) {
            if (a.key_mask) keep = keep & (meta_lds[buf][0][jl] != 0);
          }
          if constexpr (MODE == kDoc) {
            const int ksg = meta_lds[buf][0][jl], kqe = meta_lds[buf][1][jl];
            keep = keep & (c < nk_c) & (((ksg == qseg_i) & (c >= qstart_c)) | (ksg == -1)) & (i < kqe);
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

    // V^T operands one k-step ahead of their products
    bf16x8 vop[BN / 16][DB];
#pragma unroll
    for (int d = 0; d < DB; ++d) vop[0][d] = vrd.get(vt, d, 0);
#pragma unroll
    for (int s = 0; s < BN / 16; ++s) {
      __builtin_amdgcn_sched_barrier(0);
      if (s + 1 < BN / 16) {
#pragma unroll
        for (int d = 0; d < DB; ++d) vop[s + 1][d] = vrd.get(vt, d, s + 1);
      }
      const bf16x8 pb = acc_kperm_operand(sacc[s >> 1], s);
#pragma unroll
      for (int d = 0; d < DB; ++d) oacc[d] = mfma32(vop[s][d], pb, oacc[d]);
    }
    __builtin_amdgcn_sched_barrier(0);
  };

  // One iteration of the tile loop on buffer B (tile `it` resident there),
  // prefetching tile it + 1 into the other buffer.
  auto iteration = [&](auto bufc, int it) __attribute__((always_inline)) {
    constexpr int B = decltype(bufc)::value;
    bf16* const kcur = B ? k_lds1 : k_lds0;
    bf16* const vcur = B ? v_lds1 : v_lds0;
    bf16* const knext = B ? k_lds0 : k_lds1;
    bf16* const vnext = B ? v_lds0 : v_lds1;
    const int n0 = tile_of(it) * BN;
    // tile `it` (and its metadata) has landed; every wave is done with the other buffer
    dma_barrier();
    const bool more = it + 1 < ntiles;
    int next_meta = 0;
    if (more) {
      const int n1 = tile_of(it + 1) * BN;
      keys.issue(a, pb, dma, n1, knext, vnext);
      next_meta = load_meta(n1);
    }
    bool wave_sees = wave_live && (n0 <= lim_max_wave || (slot0 && n0 == 0));
    if constexpr (MODE == kDoc) wave_sees = wave_sees && (n0 == 0 || n0 + BN > qstart_min_w);
    if (wave_sees) {
      // Per-element masks are needed on the causal diagonal, at document
      // boundaries and under a key mask; the wave decides uniformly.
      bool masked = !((n0 + BN - 1 <= lim_min_wave) && (n0 + BN <= nk));
      if constexpr (MODE == kDense) masked = masked || a.key_mask != nullptr;
      if constexpr (MODE == kDoc) {
        // a tile is document-interior for this wave when all 32 query ids and
        // all 64 key ids equal one id: the document rule then keeps every pair
        // (with n0 >= every row's document start and every key's query end
        // past the wave's last row, all three parts of the document rule hold)
        const int i_last = min(wave_first + 31, nq - 1);
        masked = masked || !(q_uniform && n0 >= qstart_w &&
                             __all(meta_lds[B][0][lane] == qseg_w && meta_lds[B][1][lane] > i_last));
      }
      tile_step(n0, B, kcur, vcur, masked);
    }
    if (more) store_meta(B ^ 1, next_meta);
  };

  if (ntiles > 0) {
    const int n0 = tile_of(0) * BN;
    keys.issue(a, pb, dma, n0, k_lds0, v_lds0);
    store_meta(0, load_meta(n0));
  }
  lgkm_settle();  // no scalar load of the prologue stays pending into the tile loop
  for (int it = 0; it < ntiles; it += 2) {
    iteration(std::integral_constant<int, 0>{}, it);
    if (it + 1 < ntiles) iteration(std::integral_constant<int, 1>{}, it + 1);
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

template <int D, int MODE, int NW>
static int launch_fwd_t(const wmx_attn_args& a, hipStream_t stream) {
  constexpr int BM = 32 * NW;
  const int64_t qtiles = ((MODE == kVarlen ? a.max_queries : a.q_len) + BM - 1) / BM;
  const int64_t outer = MODE == kVarlen ? a.num_segments : a.batch;
  const int64_t per_head = a.q_units ? a.num_q_units : qtiles * outer;
  const int64_t units = per_head * a.q_heads;
  if (units <= 0) return WMX_OK;
  if (units > UINT32_MAX) return WMX_E_UNSUPPORTED;
  hipLaunchKernelGGL((attn_fwd_kernel<D, MODE, NW>), dim3((unsigned)units), dim3(64 * NW), 0, stream, a);
  return WMX_OK;
}

template <int MODE, int NW>
static int launch_fwd_rows(const wmx_attn_args& a, hipStream_t stream) {
  switch (a.head_dim) {
    case 64: return launch_fwd_t<64, MODE, NW>(a, stream);
    case 96: return launch_fwd_t<96, MODE, NW>(a, stream);
    case 128: return launch_fwd_t<128, MODE, NW>(a, stream);
    default: return WMX_E_UNSUPPORTED;
  }
}

template <int MODE>
static int launch_fwd_mode(const wmx_attn_args& a, hipStream_t stream) {
  return a.query_tile == 256 ? launch_fwd_rows<MODE, 8>(a, stream) : launch_fwd_rows<MODE, 4>(a, stream);
}

int launch_fwd(const wmx_attn_args& a, hipStream_t stream) {
  if (a.query_indices) return launch_fwd_mode<kVarlen>(a, stream);
  if (a.q_seg) return launch_fwd_mode<kDoc>(a, stream);
  return launch_fwd_mode<kDense>(a, stream);
}

}  // namespace wmx

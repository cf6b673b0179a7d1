// Attention backward for gfx950 (CDNA4): delta, dQ and dK/dV kernels.
//
// Math (softmax scale c, exp2 form, LSE in natural log from the forward):
//   P  = exp2(S * c * log2e - LSE * log2e)   on visible pairs, else 0
//   dP = dO V^T,  dS = P * (dP - delta),  delta = rowsum(dO * O)
//   dQ = c * dS K,  dK = c * dS^T Q,  dV = P^T dO
// following the reference's backward contract
// (src/white_matter/ops/cyclic_attention/_tilelang/backward_query.py:86-109,
//  backward_key_value.py:102-132, backward_preprocess.py:34-49).
//
// Deterministic kernels, no atomics on the dense paths:
//   dKV : key-parallel (128 keys and 8 waves, or 64 keys and 4 waves), loops
//         over the query heads of the KV head and over the query tiles of 32
//         that can see the key tile;
//         a lane owns one key column of S = Q K^T; dV^T = dO^T P and
//         dK^T = Q^T dS accumulate in registers. With a dS buffer in the
//         workspace it also stores dS^T (bf16, the value its dK product
//         uses) for every query tile it visits.
//   dQ  : query-parallel (4 waves x 32 query rows), loops over visible key
//         tiles of 64; dQ^T = K^T dS^T accumulates in registers. The stored-
//         dS form streams K and dS^T tiles and runs after dKV; the recompute
//         form (no dS buffer) evaluates S^T = K Q^T and dP^T = V dO^T itself,
//         a lane owning one query column so its LSE and delta are scalars.
// Varlen schedules whose key rows repeat across segments: where only the
// dummy slot of each batch row is shared, each segment stores its part of the
// dummy's dK/dV and a second kernel adds the parts in segment order (the same
// result on every run); where other rows repeat (capped histories), dK/dV
// accumulate in fp32 workspace rows with atomics, converted once at the end.
#include <type_traits>

#include "attn_tiles.h"

namespace wmx {

// ---------------------------------------------------------------- delta ----
// 16 lanes per row, 8 elements per lane; a thread takes kDeltaRows rows (16
// apart) with all their loads issued before any is used, so each thread has
// kDeltaRows x 32 bytes in flight; 16 kDeltaRows rows per 256-thread block.
constexpr int kDeltaRows = 4;
template <int D>
__global__ __launch_bounds__(256) void bwd_delta_kernel(const wmx_attn_args a, int64_t rows) {
  const int tid = threadIdx.x;
  const int l16 = tid & 15;
  const int r0 = (int)blockIdx.x * 16 * kDeltaRows + (tid >> 4);  // rows < 2^31 (checked on the host)
  const bool lane_live = 8 * l16 < D;
  u32x4 ow[kDeltaRows], gw[kDeltaRows];
#pragma unroll
  for (int k = 0; k < kDeltaRows; ++k) {
    const int r = r0 + 16 * k;
    ow[k] = gw[k] = u32x4{0u, 0u, 0u, 0u};
    if (r < rows && lane_live) {
      const int i = (int)((unsigned)r % (unsigned)a.q_len);
      const int bh = (int)((unsigned)r / (unsigned)a.q_len);
      const int h = (int)((unsigned)bh % (unsigned)a.q_heads);
      const int b = (int)((unsigned)bh / (unsigned)a.q_heads);
      ow[k] = load16((const bf16*)a.o + (int64_t)b * a.o_stride[0] + (int64_t)h * a.o_stride[1] +
                     (int64_t)i * a.o_stride[2] + 8 * l16);
      gw[k] = load16((const bf16*)a.dout + (int64_t)b * a.do_stride[0] + (int64_t)h * a.do_stride[1] +
                     (int64_t)i * a.do_stride[2] + 8 * l16);
    }
  }
#pragma unroll
  for (int k = 0; k < kDeltaRows; ++k) {
    float acc = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      acc = fmaf(bf16_lo(ow[k][e]), bf16_lo(gw[k][e]), acc);
      acc = fmaf(bf16_hi(ow[k][e]), bf16_hi(gw[k][e]), acc);
    }
#pragma unroll
    for (int o = 8; o > 0; o >>= 1) acc += __shfl_xor(acc, o);
    const int r = r0 + 16 * k;
    if (r < rows && l16 == 0) a.delta[r] = acc;
  }
}

// ------------------------------------------------------------------- dQ ----
// One workgroup = 128 query rows (4 waves x 32) of one (batch row or segment,
// query head), Q and dO rows in registers. Key/value tiles of 64 rows stream
// through double-buffered LDS exactly as in the forward; the K tile is read
// row-wise for S^T = K Q^T and with transpose reads for dQ^T = K^T dS^T.
template <int D, int MODE>
__global__ __launch_bounds__(256, 2) void attn_bwd_dq_kernel(const wmx_attn_args args) {
  const wmx_attn_args& a = args;
  constexpr int BM = 128, BN = 64;
  static_assert(BN == kTileRows, "one LDS tile per key tile");
  constexpr int KS = D / 16, DB = D / 32;
  // two buffers as distinct arrays with static roles (see the forward)
  __shared__ __attribute__((aligned(1024))) bf16 k_lds0[kTileElems];
  __shared__ __attribute__((aligned(1024))) bf16 k_lds1[kTileElems];
  __shared__ __attribute__((aligned(1024))) bf16 v_lds0[kTileElems];
  __shared__ __attribute__((aligned(1024))) bf16 v_lds1[kTileElems];
  __shared__ int meta_lds[2][2][BN];  // per buffer: key ids (or key mask), key query ends
  __shared__ int red_lds[4];

  const int qtiles = ((MODE == kVarlen ? a.max_queries : a.q_len) + BM - 1) / BM;
  const unsigned outer = MODE == kVarlen ? (unsigned)a.num_segments : (unsigned)a.batch;
  const int32_t* list = a.q_units;  // (batch row or segment, tile) pairs, heaviest first
  const uint32_t count = list ? (uint32_t)a.num_q_units : (uint32_t)qtiles * outer;

  // this workgroup's unit: 128 query rows of one (batch row or segment, query head)
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
  const bool slot0 = a.keep_slot0 && nk > 0;
  const int lim_max_wg = pb.bound.lim(min(q0 + BM, nq) - 1);
  const int i = q0 + wave * 32 + col;
  const bool valid_q = i < nq;
  const int lim_i = pb.bound.lim(i);
  const int wave_first = q0 + wave * 32;
  const bool wave_live = wave_first < nq;
  const int lim_min_wave = pb.bound.lim(wave_first);
  const int lim_max_wave = pb.bound.lim(min(wave_first + 31, nq - 1));

  int qb, qt;
  pb.query_loc(valid_q ? i : q0, qb, qt);
  bf16x8 qf[KS], gf[KS];
  float lse2, delta;
  {
    const bf16* qrow = row_at(a.q, a.q_stride, qb, h, qt) + 8 * half;
    const bf16* grow = row_at(a.dout, a.do_stride, qb, h, qt) + 8 * half;
    const u32x4 z = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const u32x4 wq = load16(qrow + 16 * s), wg = load16(grow + 16 * s);
      qf[s] = as_bf16x8(valid_q ? wq : z);
      gf[s] = as_bf16x8(valid_q ? wg : z);
    }
    const int64_t r = ((int64_t)qb * a.q_heads + h) * a.q_len + qt;
    lse2 = valid_q ? a.lse[r] * kLog2e : kPosInf;
    delta = valid_q ? a.delta[r] : 0.f;
  }

  int qseg_i = 0, qstart_i = 0, kt_begin_main = 0, qstart_min_w = 0;
  if constexpr (MODE == kDoc) {
    if (valid_q) {
      qseg_i = a.q_seg[(int64_t)b * a.q_len + i];
      qstart_i = a.q_start[(int64_t)b * a.q_len + i];
    }
    int v = INT_MAX;
    if (tid < BM && q0 + tid < nq) v = a.q_start[(int64_t)b * a.q_len + q0 + tid];
    for (int o = 32; o > 0; o >>= 1) v = min(v, __shfl_xor(v, o));
    if (lane == 0) red_lds[wave] = v;
    __syncthreads();
    v = min(min(red_lds[0], red_lds[1]), min(red_lds[2], red_lds[3]));
    kt_begin_main = __builtin_amdgcn_readfirstlane(v < 0 ? 0 : v / BN);  // uniform: keeps the tile loop scalar
    // smallest document start of this wave's rows: no key below it outside tile 0
    int u = valid_q ? qstart_i : INT_MAX;
    for (int o = 32; o > 0; o >>= 1) u = min(u, __shfl_xor(u, o));
    qstart_min_w = __builtin_amdgcn_readfirstlane(u);
  }
  int kt_end = (lim_max_wg + 1 + BN - 1) / BN;
  if (slot0 && kt_end < 1) kt_end = 1;
  const int first_main = kt_begin_main > 1 ? kt_begin_main : 1;
  const bool gap = (MODE == kDoc) && first_main > 1;
  const int ntiles = gap ? 1 + max(0, kt_end - first_main) : kt_end;
  auto tile_of = [&](int it) { return gap ? (it == 0 ? 0 : first_main + it - 1) : it; };

  TileDMA<D> dma;
  dma.init(wave, lane);
  KeyTiles<MODE, D> keys;
  keys.init(a, pb, hk, slot0 ? max(lim_max_wg + 1, 1) : lim_max_wg + 1, dma);
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

  f32x16 dqacc[DB];
#pragma unroll
  for (int d = 0; d < DB; ++d) dqacc[d] = f32x16{};
  const float sl2 = a.softmax_scale * kLog2e;
  RowReads<KS> rrd;
  rrd.init(col, half);
  TrReads<DB> trd;
  trd.init(lane);

  auto tile_step = [&](int n0, int buf, const bf16* kt, const bf16* vt, bool masked) __attribute__((always_inline)) {
    rrd.refresh();
    trd.refresh();
    f32x16 sacc[BN / 32], pacc[BN / 32];
#pragma unroll
    for (int nb = 0; nb < BN / 32; ++nb) {
      sacc[nb] = f32x16{};
      pacc[nb] = f32x16{};
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        sacc[nb] = mfma32(rrd.get(kt, s, nb), qf[s], sacc[nb]);
        pacc[nb] = mfma32(rrd.get(vt, s, nb), gf[s], pacc[nb]);
      }
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
          bool keep = (j <= lim_i) | (slot0 & (j == 0));
          if constexpr (MODE == kDense) {
            if (a.key_mask) keep = keep & (meta_lds[buf][0][jl] != 0);
          }
          if constexpr (MODE == kDoc) {
            const int ksg = meta_lds[buf][0][jl], kqe = meta_lds[buf][1][jl];
            keep = keep & (j < nk) & (((ksg == qseg_i) & (j >= qstart_i)) | (ksg == -1)) & (i < kqe);
          }
          sacc[nb][r] = keep ? sacc[nb][r] : kNegInf;
        }
      }
    }
#pragma unroll
    for (int nb = 0; nb < BN / 32; ++nb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        // a masked score is -inf and gives p = 0 exactly (lse is finite or +inf)
        const float p = __builtin_amdgcn_exp2f(fmaf(sacc[nb][r], sl2, -lse2));
        sacc[nb][r] = p * (pacc[nb][r] - delta);
      }
    }
#pragma unroll
    for (int s = 0; s < BN / 16; ++s) {
      const bf16x8 ds = acc_kperm_operand(sacc[s >> 1], s);
#pragma unroll
      for (int d = 0; d < DB; ++d) dqacc[d] = mfma32(trd.get(kt, d, s), ds, dqacc[d]);
    }
  };

  auto iteration = [&](auto bufc, int it) __attribute__((always_inline)) {
    constexpr int B = decltype(bufc)::value;
    const bf16* kcur = B ? k_lds1 : k_lds0;
    const bf16* vcur = B ? v_lds1 : v_lds0;
    const int n0 = tile_of(it) * BN;
    dma_barrier();
    const bool more = it + 1 < ntiles;
    int next_meta = 0;
    if (more) {
      const int n1 = tile_of(it + 1) * BN;
      keys.issue(a, pb, dma, n1, B ? k_lds0 : k_lds1, B ? v_lds0 : v_lds1);
      next_meta = load_meta(n1);
    }
    bool wave_sees = wave_live && (n0 <= lim_max_wave || (slot0 && n0 == 0));
    if constexpr (MODE == kDoc) wave_sees = wave_sees && (n0 == 0 || n0 + BN > qstart_min_w);
    if (wave_sees) {
      bool masked = !((n0 + BN - 1 <= lim_min_wave) && (n0 + BN <= nk));
      if constexpr (MODE == kDense) masked = masked || a.key_mask != nullptr;
      if constexpr (MODE == kDoc) masked = true;
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
  bf16* dqrow = (bf16*)row_at(a.dq, a.dq_stride, qb, h, qt);
  store_acc_row<DB>(dqrow, dqacc, a.softmax_scale, half);
}

// ------------------------------------------------------- dQ from dS ----
// One workgroup = 128 query rows (4 waves x 32) of one (batch row or segment,
// query head): dQ^T = K^T dS^T over the visible key tiles of 64, with the K
// tile and the dS^T tile (64 keys x the workgroup's 128 queries, written by
// the dK/dV kernel) streaming through double-buffered LDS; both operands are
// transpose reads. The dK/dV kernel stores every (key, query) pair of each
// query tile it visits, zeros for invisible pairs, and visits every tile a
// wave here reads under the causal/offset bound, so only document masks
// (whose rows past a key's document end the dK/dV kernel skips) are applied
// here.
template <int D, int MODE>
__global__ __launch_bounds__(256, 2) void attn_bwd_dq_ds_kernel(const wmx_attn_args args) {
  const wmx_attn_args& a = args;
  constexpr int BM = 128, BN = 64;
  static_assert(BN == kTileRows && BM == kRowElems, "one LDS tile per key tile, one row per query tile");
  constexpr int DB = D / 32;
  __shared__ __attribute__((aligned(1024))) bf16 k_lds0[kTileElems];
  __shared__ __attribute__((aligned(1024))) bf16 k_lds1[kTileElems];
  __shared__ __attribute__((aligned(1024))) bf16 s_lds0[kTileElems];
  __shared__ __attribute__((aligned(1024))) bf16 s_lds1[kTileElems];
  __shared__ int meta_lds[2][2][BN];  // per buffer: key document ids, key query ends
  __shared__ int red_lds[4];

  const int qtiles = ((MODE == kVarlen ? a.max_queries : a.q_len) + BM - 1) / BM;
  const unsigned outer = MODE == kVarlen ? (unsigned)a.num_segments : (unsigned)a.batch;
  const int32_t* list = a.q_units;  // (batch row or segment, tile) pairs, heaviest first
  const uint32_t count = list ? (uint32_t)a.num_q_units : (uint32_t)qtiles * outer;
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
  const bool slot0 = a.keep_slot0 && nk > 0;
  const int lim_max_wg = pb.bound.lim(min(q0 + BM, nq) - 1);
  const int i = q0 + wave * 32 + col;
  const bool valid_q = i < nq;
  const int lim_i = pb.bound.lim(i);
  const int wave_first = q0 + wave * 32;
  const bool wave_live = wave_first < nq;
  const int lim_max_wave = pb.bound.lim(min(wave_first + 31, nq - 1));

  int qseg_i = 0, qstart_i = 0, kt_begin_main = 0, qstart_min_w = 0;
  if constexpr (MODE == kDoc) {
    if (valid_q) {
      qseg_i = a.q_seg[(int64_t)b * a.q_len + i];
      qstart_i = a.q_start[(int64_t)b * a.q_len + i];
    }
    int v = INT_MAX;
    if (tid < BM && q0 + tid < nq) v = a.q_start[(int64_t)b * a.q_len + q0 + tid];
    for (int o = 32; o > 0; o >>= 1) v = min(v, __shfl_xor(v, o));
    if (lane == 0) red_lds[wave] = v;
    __syncthreads();
    v = min(min(red_lds[0], red_lds[1]), min(red_lds[2], red_lds[3]));
    kt_begin_main = __builtin_amdgcn_readfirstlane(v < 0 ? 0 : v / BN);  // uniform: keeps the tile loop scalar
    // smallest document start of this wave's rows: no key below it outside tile 0
    int u = valid_q ? qstart_i : INT_MAX;
    for (int o = 32; o > 0; o >>= 1) u = min(u, __shfl_xor(u, o));
    qstart_min_w = __builtin_amdgcn_readfirstlane(u);
  }
  int kt_end = (lim_max_wg + 1 + BN - 1) / BN;
  if (slot0 && kt_end < 1) kt_end = 1;
  const int first_main = kt_begin_main > 1 ? kt_begin_main : 1;
  const bool gap = (MODE == kDoc) && first_main > 1;
  const int ntiles = gap ? 1 + max(0, kt_end - first_main) : kt_end;
  auto tile_of = [&](int it) { return gap ? (it == 0 ? 0 : first_main + it - 1) : it; };

  const int reach = slot0 ? max(lim_max_wg + 1, 1) : lim_max_wg + 1;
  TileDMA<D> dma;
  dma.init(wave, lane);
  KeyTiles<MODE, D> keys;
  keys.init(a, pb, hk, reach, dma);
  // dS^T tile: rows = keys n0 .. n0 + 63 (zeros past the reach), columns =
  // this workgroup's queries
  TileDMA<kRowElems> sdma;
  sdma.init(wave, lane);
  const int64_t ld = ds_ld(nq);
  const bf16* ds = (const bf16*)((const char*)a.workspace + bwd_ds_offset(a)) + q0;
  if constexpr (MODE == kVarlen) {
    ds += h * a.ds_elements + ds_offset_of(a, grp, tu);
  } else {
    ds += ((int64_t)b * a.q_heads + h) * a.kv_len * ld;
  }
  auto issue_ds = [&](int n0, bf16* tile) __attribute__((always_inline)) {
    const int nvalid = min(max(reach - n0, 0), kTileRows);
    sdma.issue_strided_rows_once(make_rsrc(ds + (int64_t)n0 * ld, nvalid * (int)ld * 2), tile, (int)ld * 2);
  };
  auto load_meta = [&](int n0) -> int {
    const int j = n0 + (tid & 63);
    if constexpr (MODE == kDoc) {
      if (tid < 64) return j < nk ? a.k_seg[(int64_t)b * a.kv_len + j] : INT_MIN;
      if (tid < 128) return j < nk ? a.k_qend[(int64_t)b * a.kv_len + j] : 0;
    }
    return 0;
  };
  auto store_meta = [&](int buf, int v) {
    if constexpr (MODE == kDoc) {
      if (tid < 128) meta_lds[buf][tid >> 6][tid & 63] = v;
    }
  };

  f32x16 dqacc[DB];
#pragma unroll
  for (int d = 0; d < DB; ++d) dqacc[d] = f32x16{};
  TrReads<DB> trd;  // K^T: rows d, contraction over keys
  trd.init(lane);
  TrReads<1> srd;  // dS^T: this wave's 32 query columns, contraction over keys
  srd.init(lane, 32 * wave);

  auto tile_step = [&](int n0, int buf, const bf16* kt, const bf16* st) __attribute__((always_inline)) {
    trd.refresh();
    srd.refresh();
    // operands one k-step ahead of their products
    bf16x8 sop[BN / 16], kop[BN / 16][DB];
    sop[0] = srd.get(st, 0, 0);
#pragma unroll
    for (int d = 0; d < DB; ++d) kop[0][d] = trd.get(kt, d, 0);
#pragma unroll
    for (int s = 0; s < BN / 16; ++s) {
      __builtin_amdgcn_sched_barrier(0);
      if (s + 1 < BN / 16) {
        sop[s + 1] = srd.get(st, 0, s + 1);
#pragma unroll
        for (int d = 0; d < DB; ++d) kop[s + 1][d] = trd.get(kt, d, s + 1);
      }
      bf16x8 op = sop[s];
      if constexpr (MODE == kDoc) {
        // element e is key n0 + 16 s + 8 (e / 4) + 4 half + e % 4
        u32x4 w = __builtin_bit_cast(u32x4, op);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int jl = 16 * s + 8 * (e >> 2) + 4 * half + (e & 3);
          const int j = n0 + jl;
          const int ksg = meta_lds[buf][0][jl], kqe = meta_lds[buf][1][jl];
          const bool keep = ((j <= lim_i) | (slot0 & (j == 0))) & (j < nk) &
                            (((ksg == qseg_i) & (j >= qstart_i)) | (ksg == -1)) & (i < kqe);
          const uint32_t m = (e & 1) ? 0xffff0000u : 0x0000ffffu;
          w[e >> 1] &= keep ? 0xffffffffu : ~m;
        }
        op = as_bf16x8(w);
      }
#pragma unroll
      for (int d = 0; d < DB; ++d) dqacc[d] = mfma32(kop[s][d], op, dqacc[d]);
    }
    __builtin_amdgcn_sched_barrier(0);
  };

  auto iteration = [&](auto bufc, int it) __attribute__((always_inline)) {
    constexpr int B = decltype(bufc)::value;
    const bf16* kcur = B ? k_lds1 : k_lds0;
    const bf16* scur = B ? s_lds1 : s_lds0;
    const int n0 = tile_of(it) * BN;
    dma_barrier();
    const bool more = it + 1 < ntiles;
    int next_meta = 0;
    if (more) {
      const int n1 = tile_of(it + 1) * BN;
      issue_key_tile(keys, a, pb, dma, n1, B ? k_lds0 : k_lds1);
      issue_ds(n1, B ? s_lds0 : s_lds1);
      next_meta = load_meta(n1);
    }
    bool wave_sees = wave_live && (n0 <= lim_max_wave || (slot0 && n0 == 0));
    if constexpr (MODE == kDoc) wave_sees = wave_sees && (n0 == 0 || n0 + BN > qstart_min_w);
    if (wave_sees) tile_step(n0, B, kcur, scur);
    if (more) store_meta(B ^ 1, next_meta);
  };

  if (ntiles > 0) {
    const int n0 = tile_of(0) * BN;
    issue_key_tile(keys, a, pb, dma, n0, k_lds0);
    issue_ds(n0, s_lds0);
    store_meta(0, load_meta(n0));
  }
  lgkm_settle();  // no scalar load of the prologue stays pending into the tile loop
  for (int it = 0; it < ntiles; it += 2) {
    iteration(std::integral_constant<int, 0>{}, it);
    if (it + 1 < ntiles) iteration(std::integral_constant<int, 1>{}, it + 1);
  }

  if (!valid_q) return;
  int qb, qt;
  pb.query_loc(i, qb, qt);
  bf16* dqrow = (bf16*)row_at(a.dq, a.dq_stride, qb, h, qt);
  store_acc_row<DB>(dqrow, dqacc, a.softmax_scale, half);
}

// ------------------------------------------------------------------ dKV ----
// One workgroup = 32 NP keys of one (batch row or segment, kv head) and 2 NP
// waves: wave pair p (waves p and p + NP) owns keys 32p .. 32p + 31. NP = 4:
// 128 keys, eight waves, one workgroup per CU (a pair shares SIMD p); NP = 2:
// 64 keys, four waves, two workgroups per CU, so that one workgroup's setup
// (its unit's bounds, K/V rows and first query tiles) overlaps the other's
// tile loop. The pair splits the work so each wave holds half of the state:
//   wave p     ("S side")  holds K rows, computes S = Q K^T, the mask and
//              P = exp2(S c log2e - lse), hands P to its partner through LDS
//              and accumulates dV^T = dO^T P;
//   wave p + 4 ("dP side") holds V rows, computes dP = dO V^T, takes P and
//              forms dS = P (dP - delta), and accumulates dK^T = Q^T dS.
// Query and output-gradient tiles of 32 rows for every query head of the
// group stream through four LDS buffers with NP = 4 (direct-to-LDS loads
// issued by the S side two tiles ahead), three with NP = 2 (one tile ahead);
// each tile is read row-wise for S and dP and by transpose reads for dV and
// dK. The dP side works one tile behind the S side: in step j the S side
// takes tile j and the dP side tile j - 1, whose P the S side left in that
// tile's hand-over buffer in step j - 1. The two waves of a pair then never
// wait for each other inside a step (one workgroup barrier per step), and
// one's matrix products overlap the other's vector work.
template <int D, int MODE, bool ATOMIC, bool DS, int NP>
__global__ __launch_bounds__(128 * NP, NP == 2 ? 2 : 1) void attn_bwd_dkv_kernel(const wmx_attn_args args) {
  const wmx_attn_args& a = args;
  static_assert(NP == 2 || NP == 4, "two or four wave pairs");
  constexpr int BNK = 32 * NP, BMQ = 32, NW = 2 * NP;
  // Q/dO tile buffers, and P hand-over buffers (one per tile buffer): NBUF - 2
  // tiles are loaded ahead of the S side's (the dP side holds the one
  // behind). Four for eight waves (two tiles ahead); three for four waves,
  // whose LDS then fits twice per CU (one tile ahead: the other workgroup
  // covers the wait).
  constexpr int NBUF = NP == 4 ? 4 : 3, DIST = NBUF - 2;
  constexpr int KS = D / 16, DB = D / 32;
  constexpr int kTile32 = BMQ * kRowElems;  // 8 KB: the first 32 rows of the tile layout
  // buffers indexed by compile-time constants only (the loop is unrolled by
  // NBUF): prefetches into one buffer are then known not to alias reads of
  // the others, so reads never wait for the prefetch
  __shared__ __attribute__((aligned(1024))) bf16 q_lds[NBUF][kTile32];
  __shared__ __attribute__((aligned(1024))) bf16 g_lds[NBUF][kTile32];
  // P of tile t from the S side to the dP side: [t % NBUF][pair][register quad][lane]
  __shared__ __attribute__((aligned(16))) f32x4 p_lds[NBUF][NP][4][64];
  // lse, delta, document id and start of the tile's rows (entries past BMQ:
  // the 4-byte direct-to-LDS loads of lanes 32 .. 63, never read)
  __shared__ __attribute__((aligned(16))) float stat_lds[NBUF][2][64];
  __shared__ __attribute__((aligned(16))) int qdoc_lds[NBUF][2][64];
  __shared__ int red_lds[NW];
  // per key of the workgroup: first query row that sees it, document id,
  // document query end (kept in LDS rather than in registers)
  __shared__ int key_lds[3][BNK];

  const int group = a.q_heads / a.kv_heads;

  const int ktiles = ((MODE == kVarlen ? a.max_keys : a.kv_len) + BNK - 1) / BNK;
  const unsigned outer = MODE == kVarlen ? (unsigned)a.num_segments : (unsigned)a.batch;
  const int32_t* list = MODE == kVarlen ? a.k_units : nullptr;
  const uint32_t count = list ? (uint32_t)a.num_k_units : (uint32_t)ktiles * outer;

  // this workgroup's unit: 128 keys of one (batch row or segment, kv head)
  TileUnit tu;
  tu.decode(a.kv_heads, count, list != nullptr, ktiles, list, (int)outer, false,  // low key tiles see the most queries
            MODE == kVarlen ? a.unit_fields : 2);
  if (!tu.ok) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int half = lane >> 5, col = lane & 31;
  const int pair = wave & (NP - 1);
  const bool dp_side = wave >= NP;  // wave-uniform role
  const int n0 = tu.tile * BNK;
  const int hk = tu.head, grp = tu.grp;
  Problem<MODE> pb;
  pb.init(a, grp, tu);
  const int b = pb.b, nq = pb.nq, nk = pb.nk;
  if (n0 >= nk) return;
  const bool slot0 = a.keep_slot0 && nk > 0;

  // this lane's key (shared by the two waves of the pair)
  const int n = n0 + pair * 32 + col;
  const bool valid_k = n < nk;
  bool k_live = valid_k;
  if (MODE == kDense && a.key_mask) k_live = k_live && a.key_mask[(int64_t)b * a.key_mask_stride + min(n, nk - 1)] != 0;
  int kb, kslot;
  pb.key_loc(valid_k ? n : n0, kb, kslot);
  int kseg_n = 0, kqend_n = 0;
  if constexpr (MODE == kDoc) {
    if (valid_k) {
      kseg_n = a.k_seg[(int64_t)b * a.kv_len + n];
      kqend_n = a.k_qend[(int64_t)b * a.kv_len + n];
    }
  }
  // query rows that can see any key of the workgroup / of this pair
  const int m_begin = (slot0 && n0 == 0) ? 0 : pb.bound.first_row(n0, nq);
  int m_end = nq;
  if constexpr (MODE == kDoc) {
    int v = valid_k ? kqend_n : 0;
    for (int o = 32; o > 0; o >>= 1) v = max(v, __shfl_xor(v, o));
    if (lane == 0) red_lds[wave] = v;
    __syncthreads();
    v = red_lds[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) v = max(v, red_lds[w]);
    m_end = __builtin_amdgcn_readfirstlane(min(m_end, v));  // uniform: keeps the tile loop scalar
  }
  const int pair_key0 = n0 + pair * 32;
  const bool pair_live = pair_key0 < nk;

  // dS^T rows of this lane's key: block of (problem, query head hq) at
  // ds_key + hq * ds_head, query i at element i
  bf16* ds_key = nullptr;
  int64_t ds_head = 0;
  if constexpr (DS) {
    const int64_t ld = ds_ld(nq);
    bf16* ds = (bf16*)((char*)a.workspace + bwd_ds_offset(a));
    if constexpr (MODE == kVarlen) {
      ds_head = a.ds_elements;
      ds += ds_offset_of(a, grp, tu);
    } else {
      ds_head = (int64_t)a.kv_len * ld;
      ds += (int64_t)b * a.q_heads * ds_head;
    }
    ds_key = ds + (int64_t)(valid_k ? n : n0) * ld + 8 * half;
  }
  const int pair_m_begin = (slot0 && pair_key0 == 0) ? 0 : pb.bound.first_row(pair_key0, nq);

  // K rows on the S side, V rows on the dP side
  bf16x8 kvf[KS];
  {
    const bf16* row = dp_side ? row_at(a.v, a.v_stride, kb, hk, kslot) : row_at(a.k, a.k_stride, kb, hk, kslot);
    const u32x4 z = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const u32x4 w = load16(row + 8 * half + 16 * s);
      kvf[s] = as_bf16x8(k_live ? w : z);
    }
  }
  // dV^T on the S side, dK^T on the dP side
  f32x16 acc[DB];
#pragma unroll
  for (int d = 0; d < DB; ++d) acc[d] = f32x16{};
  const float sl2 = a.softmax_scale * kLog2e;

  // ---- query tiles: (head, first row) pairs over the group's heads ----
  const int m_first = (m_begin / BMQ) * BMQ;
  const int nqt = m_end > m_first ? (m_end - m_first + BMQ - 1) / BMQ : 0;
  const int total = nqt * group;
  // the S-side waves load every tile
  TileDMA<D, NP, BMQ> dma;
  dma.init(pair, lane);
  QueryTiles<MODE, D, NP, BMQ> qrows;
  qrows.init(a, pb);
  RowReads<KS> rrd;
  rrd.init(col, half);
  TrReads<DB> trd;
  trd.init(lane);

  // tile t is (query head hk * group + t / nqt, first row m_first + BMQ (t % nqt))
  struct Cursor {
    int hq, m0;
  };
  auto advance = [&](Cursor& c) {
    c.m0 += BMQ;
    if (c.m0 >= m_end) {
      c.m0 = m_first;
      ++c.hq;
    }
  };
  auto active = [&](int m0) { return pair_live && m0 + BMQ > pair_m_begin; };  // uniform over the pair

  // per-row statistics (and document metadata) of query tile (hq, m0), loaded
  // by wave 0 straight into LDS buffer B with the tile (one 4-byte direct-to-
  // LDS load per array: no registers, no waits until the step barrier). Rows
  // past nq read as zeros; their scores are masked.
  auto issue_meta = [&](auto bufc, int hq, int m0) __attribute__((always_inline)) {
    constexpr int B = decltype(bufc)::value;
    if (wave == 0) {
      // rows of a dense problem, or of a segment with consecutive query slots,
      // are consecutive entries of LSE, delta and the document arrays
      const bool consecutive = MODE != kVarlen || (a.segment_layout & kQueriesConsecutive);
      if (consecutive) {
        // one buffer resource per array, this lane's row at byte 4 * lane
        // (rows past nq fall outside the resource and read as zeros)
        const int nvalid = min(max(nq - m0, 0), BMQ) * 4;  // lanes past the tile read zeros
        const int64_t r0 = ((int64_t)qrows.qrow * a.q_heads + hq) * a.q_len + qrows.qfirst + m0;
        const rsrc_t rl = make_rsrc(a.lse + r0, nvalid), rd = make_rsrc(a.delta + r0, nvalid);
        rsrc_t rs, rq;
        if constexpr (MODE == kDoc) {
          const int64_t d0 = (int64_t)b * a.q_len + m0;
          rs = make_rsrc(a.q_seg + d0, nvalid);
          rq = make_rsrc(a.q_start + d0, nvalid);
        }
        const unsigned off = 4u * lane;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rl, (lds_void*)&stat_lds[B][0][0], 4, off, 0, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rd, (lds_void*)&stat_lds[B][1][0], 4, off, 0, 0, 0);
        if constexpr (MODE == kDoc) {
          __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)&qdoc_lds[B][0][0], 4, off, 0, 0, 0);
          __builtin_amdgcn_raw_ptr_buffer_load_lds(rq, (lds_void*)&qdoc_lds[B][1][0], 4, off, 0, 0, 0);
        }
      } else if constexpr (MODE == kVarlen) {
        const int m = m0 + lane;
        const bool ok = m < nq;
        int rb, rt;
        pb.query_loc(ok ? m : 0, rb, rt);
        const int64_t idx = ((int64_t)rb * a.q_heads + hq) * a.q_len + rt;
        const void* zero = (const void*)kZeroChunk;
        __builtin_amdgcn_global_load_lds(ok ? (const void*)(a.lse + idx) : zero, (lds_void*)&stat_lds[B][0][0], 4, 0, 0);
        __builtin_amdgcn_global_load_lds(ok ? (const void*)(a.delta + idx) : zero, (lds_void*)&stat_lds[B][1][0], 4, 0, 0);
        lgkm_settle();
      }
    }
  };
  // tile (hq, m0) and its statistics into buffer B (S side only)
  auto issue_tile = [&](auto bufc, const Cursor& c) __attribute__((always_inline)) {
    constexpr int B = decltype(bufc)::value;
    bf16* const qt = q_lds[B];
    bf16* const gt = g_lds[B];
    issue_meta(bufc, c.hq, c.m0);
    qrows.issue(a, pb, dma, c.hq, c.m0, qt, gt);
  };

  // first query row that sees this lane's key (INT_MAX for a dead key): the
  // causal/offset rule is then one comparison per score. Read back from LDS
  // in each step (published by the first step barrier).
  if (!dp_side && half == 0) {
    key_lds[0][pair * 32 + col] = !k_live ? INT_MAX : (slot0 && n == 0) ? 0 : pb.bound.first_row(n, nq);
    key_lds[1][pair * 32 + col] = kseg_n;
    key_lds[2][pair * 32 + col] = kqend_n;
  }

  // S side, one tile (in Q/dO buffer B, its P to hand-over buffer B % 2)
  auto s_step = [&](auto bufc, int m0) __attribute__((always_inline)) {
    constexpr int B = decltype(bufc)::value;
    const bf16* const qt = q_lds[B];
    const bf16* const gt = g_lds[B];
    rrd.refresh();
    trd.refresh();
    f32x16 sacc = f32x16{};
    // S = Q K^T, k-step major, each Q operand read PF k-steps ahead of its
    // product (the scheduling barriers keep the compiler from sinking the
    // reads next to their uses, where every product would wait out the LDS
    // latency)
    constexpr int PF = KS < 4 ? KS : 4;
    bf16x8 op[KS];
#pragma unroll
    for (int s = 0; s < PF; ++s) op[s] = rrd.get(qt, s, 0);
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      __builtin_amdgcn_sched_barrier(0);
      if (s + PF < KS) op[s + PF] = rrd.get(qt, s + PF, 0);
      sacc = mfma32(op[s], kvf[s], sacc);
    }
    __builtin_amdgcn_sched_barrier(0);
    // the rows' lse and the first dO^T operands, read while the products drain
    f32x4 l4s[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) l4s[g] = *reinterpret_cast<const f32x4*>(&stat_lds[B][0][8 * g + 4 * half]);
    bf16x8 top[BMQ / 16][DB];
#pragma unroll
    for (int d = 0; d < DB; ++d) top[0][d] = trd.get(gt, d, 0);
    // every pair of the tile is visible to this pair's keys: no per-element mask
    const bool full = (MODE == kVarlen || (MODE == kDense && !a.key_mask)) && m0 >= pair_m_begin &&
                      m0 + BMQ <= nq && pb.bound.lim(m0) >= pair_key0 + 31;
    if (!full) {
      // keeps this block a real (wave-uniform) branch instead of selects
      __asm__ volatile("");
      const int kl = pair * 32 + col;
      const int lo = key_lds[0][kl] - m0, hi = nq - m0;  // rows ml in [lo, hi) see the key
      int kseg = 0, kqend = 0;
      if constexpr (MODE == kDoc) {
        kseg = key_lds[1][kl];
        kqend = key_lds[2][kl];
      }
      // element r is row ml = 4 half + c with the constant c = 8 (r / 4) + r % 4:
      // the row rules become compares of c against per-lane bounds
      const int lo_c = lo - 4 * half, hi_c = hi - 4 * half, kqend_c = kqend - m0 - 4 * half;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int c = 8 * (r >> 2) + (r & 3);
        const int ml = c + 4 * half;
        bool keep = (c >= lo_c) & (c < hi_c);
        if constexpr (MODE == kDoc) {
          const int qsg = qdoc_lds[B][0][ml], qst = qdoc_lds[B][1][ml];
          keep = keep & (((qsg == kseg) & (n >= qst)) | (kseg == -1)) & (c < kqend_c);
        }
        sacc[r] = keep ? sacc[r] : kNegInf;
      }
    }
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const f32x4 l4 = l4s[g];
      f32x4 p4;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        // a masked score is -inf and gives p = 0 exactly (lse is finite or +inf)
        p4[e] = __builtin_amdgcn_exp2f(fmaf(sacc[4 * g + e], sl2, -l4[e] * kLog2e));
        sacc[4 * g + e] = p4[e];
      }
      p_lds[B][pair][g][lane] = p4;
    }
    // dV^T += dO^T P, the transposed operands one k-step ahead of their products
#pragma unroll
    for (int s = 0; s < BMQ / 16; ++s) {
      __builtin_amdgcn_sched_barrier(0);
      if (s + 1 < BMQ / 16) {
#pragma unroll
        for (int d = 0; d < DB; ++d) top[s + 1][d] = trd.get(gt, d, s + 1);
      }
      const bf16x8 pop = acc_kperm_operand(sacc, s);
#pragma unroll
      for (int d = 0; d < DB; ++d) acc[d] = mfma32(top[s][d], pop, acc[d]);
    }
    __builtin_amdgcn_sched_barrier(0);
  };

  // dP side, one tile (in Q/dO buffer B, its P in hand-over buffer B % 2)
  auto dp_step = [&](auto bufc, int hq, int m0) __attribute__((always_inline)) {
    constexpr int B = decltype(bufc)::value;
    const bf16* const qt = q_lds[B];
    const bf16* const gt = g_lds[B];
    rrd.refresh();
    trd.refresh();
    f32x16 dacc = f32x16{};
    // dP = dO V^T
    constexpr int PF = KS < 4 ? KS : 4;
    bf16x8 op[KS];
#pragma unroll
    for (int s = 0; s < PF; ++s) op[s] = rrd.get(gt, s, 0);
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      __builtin_amdgcn_sched_barrier(0);
      if (s + PF < KS) op[s + PF] = rrd.get(gt, s + PF, 0);
      dacc = mfma32(op[s], kvf[s], dacc);
    }
    __builtin_amdgcn_sched_barrier(0);
    // dS = P (dP - delta) per k-step (its two register quads), P and delta
    // and the Q^T operands read one k-step ahead; dK^T += Q^T dS
    bf16x8 top[BMQ / 16][DB];
    f32x4 d4s[BMQ / 16][2], p4s[BMQ / 16][2];
    auto read_pd = [&](int s) __attribute__((always_inline)) {
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int g = 2 * s + q;
        d4s[s][q] = *reinterpret_cast<const f32x4*>(&stat_lds[B][1][8 * g + 4 * half]);
        p4s[s][q] = p_lds[B][pair][g][lane];
      }
    };
    read_pd(0);
#pragma unroll
    for (int d = 0; d < DB; ++d) top[0][d] = trd.get(qt, d, 0);
    bf16* ds_row = nullptr;
    if constexpr (DS) ds_row = ds_key + hq * ds_head + m0;
#pragma unroll
    for (int s = 0; s < BMQ / 16; ++s) {
      __builtin_amdgcn_sched_barrier(0);
      if (s + 1 < BMQ / 16) {
        read_pd(s + 1);
#pragma unroll
        for (int d = 0; d < DB; ++d) top[s + 1][d] = trd.get(qt, d, s + 1);
      }
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int g = 2 * s + q;
#pragma unroll
        for (int e = 0; e < 4; ++e) dacc[4 * g + e] = p4s[s][q][e] * (dacc[4 * g + e] - d4s[s][q][e]);
      }
      const bf16x8 sop = acc_kperm_operand(dacc, s);
      if constexpr (DS) {
        // operand element e is query m0 + 16 s + 8 (e / 4) + 4 half + e % 4;
        // swapping dwords with the partner lane (lane ^ 32) gives each lane
        // the 8 queries 16 s + 8 half .. + 7 of its key: one 16-byte store
        const u32x4 w = __builtin_bit_cast(u32x4, sop);
        const auto lo = __builtin_amdgcn_permlane32_swap(w[0], w[2], false, false);
        const auto hi = __builtin_amdgcn_permlane32_swap(w[1], w[3], false, false);
        if (valid_k) *reinterpret_cast<u32x4*>(ds_row + 16 * s) = u32x4{lo[0], hi[0], lo[1], hi[1]};
      }
#pragma unroll
      for (int d = 0; d < DB; ++d) acc[d] = mfma32(top[s][d], sop, acc[d]);
    }
    __builtin_amdgcn_sched_barrier(0);
  };

  // Step j: the S side takes tile j (buffer j % NBUF) and issues tile
  // j + DIST; the dP side takes tile j - 1. Steps run j = 0 .. total, one
  // workgroup barrier each: after it, tile j and P of tile j - 1 are in LDS,
  // and the buffer of tile j + DIST (last read for tile j + DIST - NBUF =
  // j - 2) is free.
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I3 = std::integral_constant<int, NBUF - 1>;  // the last buffer (3 or 2)
  if (!dp_side) {
    Cursor cur{hk * group, m_first}, pf = cur;
    if (total > 0) issue_tile(I0{}, pf);
    advance(pf);
    if constexpr (DIST > 1) {
      if (total > 1) issue_tile(I1{}, pf);
      advance(pf);
    }
    lgkm_settle();  // no scalar load of the prologue stays pending into the tile loop
    auto step = [&](auto bufc, int j) __attribute__((always_inline)) {
      constexpr int B = decltype(bufc)::value;
      // tile j has landed (with two tiles ahead, tile j + 1's loads, issued
      // after it, may still fly)
      if (DIST > 1 && j + 1 < total) {
        lds_sync<2 * TileDMA<D, NP, BMQ>::kInstr>();
      } else {
        lds_sync<0>();
      }
      if (j + DIST < total) {
        issue_tile(std::integral_constant<int, (B + DIST) % NBUF>{}, pf);
        advance(pf);
      }
      if (j < total) {
        if (active(cur.m0)) s_step(bufc, cur.m0);
        advance(cur);
      }
    };
    for (int j = 0; j <= total; j += NBUF) {
      step(I0{}, j);
      if (j + 1 <= total) step(I1{}, j + 1);
      if (j + 2 <= total) step(I2{}, j + 2);
      if constexpr (NBUF == 4) {
        if (j + 3 <= total) step(I3{}, j + 3);
      }
    }
  } else {
    Cursor cur{hk * group, m_first};
    lgkm_settle();
    // step j works on tile j - 1 in buffer (j - 1) % NBUF
    auto step = [&](auto bufc, int j) __attribute__((always_inline)) {
      constexpr int B = decltype(bufc)::value;
      lds_barrier();  // its own LDS reads done; the dS stores keep flying
      if (j >= 1) {
        if (active(cur.m0)) {
          dp_step(bufc, cur.hq, cur.m0);
        } else if constexpr (DS) {
          // the dQ kernel reads every key row of a visited tile: zeros for a
          // pair that sees none of its rows
          if (valid_k) {
            bf16* row = ds_key + cur.hq * ds_head + cur.m0;
#pragma unroll
            for (int s = 0; s < BMQ / 16; ++s) *reinterpret_cast<u32x4*>(row + 16 * s) = u32x4{0u, 0u, 0u, 0u};
          }
        }
        advance(cur);
      }
    };
    for (int j = 0; j <= total; j += NBUF) {
      step(I3{}, j);
      if (j + 1 <= total) step(I0{}, j + 1);
      if (j + 2 <= total) step(I1{}, j + 2);
      if constexpr (NBUF == 4) {
        if (j + 3 <= total) step(I2{}, j + 3);
      }
    }
  }

  if (!valid_k) return;
  const float scale = dp_side ? a.softmax_scale : 1.f;
  if constexpr (ATOMIC) {
    // fp32 accumulators laid out [key row][kv head][D]; dK first, then dV
    const int64_t row = (int64_t)kb * a.key_extent + kslot;
    float* dst = (float*)a.workspace + (row * a.kv_heads + hk) * D +
                 (dp_side ? 0 : (int64_t)a.batch * a.key_extent * a.kv_heads * D);
#pragma unroll
    for (int d = 0; d < DB; ++d) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int dd = d * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
        atomicAdd(dst + dd, acc[d][r] * scale);
      }
    }
  } else {
    if (MODE == kVarlen && a.keys_unique == 2 && kslot == 0) {
      // the dummy slot shared by the segments of a batch row: this segment's
      // part, [dK, dV][segment][kv head][D], and its mark (the dummy's batch
      // row + 1); dummy_reduce_kernel adds the parts in segment order
      float* dst = (float*)((char*)a.workspace + bwd_dummy_mark_bytes(a)) +
                   (((dp_side ? 0 : (int64_t)a.num_segments) + grp) * a.kv_heads + hk) * D;
#pragma unroll
      for (int d = 0; d < DB; ++d) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int dd = d * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
          dst[dd] = acc[d][r] * scale;
        }
      }
      if (!dp_side) ((int32_t*)a.workspace)[grp] = kb + 1;
      return;
    }
    bf16* dst = dp_side ? (bf16*)row_at(a.dk, a.dk_stride, kb, hk, kslot) : (bf16*)row_at(a.dv, a.dv_stride, kb, hk, kslot);
    store_acc_row<DB>(dst, acc, scale, half);
  }
}

// ----------------------------------------------- varlen accumulator glue ----
__global__ void zero_f32_kernel(float* p, int64_t n) {
  const int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (i + 3 < n) {
    *reinterpret_cast<f32x4*>(p + i) = f32x4{0.f, 0.f, 0.f, 0.f};
  } else {
    for (int64_t k = i; k < n; ++k) p[k] = 0.f;
  }
}

// The dummy slot's dK/dV where only it repeats: for every batch row, the sum
// of the parts of the segments marked with that row, added in segment order,
// stored as bf16 at slot 0 (zero for a row that no segment marks). Block
// (b, c) covers elements c * 256 .. of the [dK, dV][kv head][D] rows of b;
// the segments are taken 256 at a time, the marked ones listed in LDS in
// order (wave ballots and a prefix over the four waves).
__global__ __launch_bounds__(256) void dummy_reduce_kernel(const wmx_attn_args a, int cols) {
  __shared__ int list[256];
  __shared__ int wave_count[4];
  const int per_side = a.kv_heads * a.head_dim;
  const int b = blockIdx.x / cols;
  const int e = (blockIdx.x - b * cols) * 256 + threadIdx.x;
  const bool live = e < 2 * per_side;
  const int side = live ? e / per_side : 0;
  const int rem = live ? e - side * per_side : 0;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int32_t* marks = (const int32_t*)a.workspace;
  const float* parts = (const float*)((const char*)a.workspace + bwd_dummy_mark_bytes(a)) +
                       (int64_t)side * a.num_segments * per_side + rem;
  float sum = 0.f;
  for (int c0 = 0; c0 < a.num_segments; c0 += 256) {
    const int s = c0 + threadIdx.x;
    const bool mine = s < a.num_segments && marks[s] == b + 1;
    const uint64_t ballot = __ballot(mine);
    if (lane == 0) wave_count[w] = __popcll(ballot);
    __syncthreads();
    int base = 0;
    for (int i = 0; i < w; ++i) base += wave_count[i];
    const int total = wave_count[0] + wave_count[1] + wave_count[2] + wave_count[3];
    if (mine) list[base + __popcll(ballot & ((1ull << lane) - 1))] = s;
    __syncthreads();
    if (live) {
      for (int i = 0; i < total; ++i) sum += parts[(int64_t)list[i] * per_side];
    }
    __syncthreads();  // list and wave_count are rewritten by the next chunk
  }
  if (!live) return;
  const int h = rem / a.head_dim, d = rem - h * a.head_dim;
  void* out = side == 0 ? a.dk : a.dv;
  const int64_t* st = side == 0 ? a.dk_stride : a.dv_stride;
  ((bf16*)out)[(int64_t)b * st[0] + (int64_t)h * st[1] + d] = (__bf16)sum;
}

// Convert the fp32 [B*R][Hkv][D] accumulators (R = bwd_acc_rows, every key
// slot) to bf16 dK/dV with their strides.
__global__ void acc_to_bf16_kernel(const wmx_attn_args a) {
  const int D = a.head_dim;
  const int64_t rows = bwd_acc_rows(a);
  const int64_t total = (int64_t)a.batch * rows * a.kv_heads * D;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const int d = (int)(idx % D);
  const int64_t rh = idx / D;
  const int h = (int)(rh % a.kv_heads);
  const int64_t row = rh / a.kv_heads;
  const int b = (int)(row / rows);
  const int slot = (int)(row % rows);
  const float* acck = (const float*)a.workspace;
  const float* accv = acck + total;
  ((bf16*)a.dk)[(int64_t)b * a.dk_stride[0] + (int64_t)h * a.dk_stride[1] + (int64_t)slot * a.dk_stride[2] + d] =
      (__bf16)acck[idx];
  ((bf16*)a.dv)[(int64_t)b * a.dv_stride[0] + (int64_t)h * a.dv_stride[1] + (int64_t)slot * a.dv_stride[2] + d] =
      (__bf16)accv[idx];
}

// ------------------------------------------------------------- launchers ----
int launch_bwd_preprocess(const wmx_attn_args& a, hipStream_t stream) {
  const int64_t rows = (int64_t)a.batch * a.q_heads * a.q_len;
  if (rows == 0) return WMX_OK;
  if (rows + 16 * kDeltaRows > INT32_MAX) return WMX_E_UNSUPPORTED;
  const int64_t blocks = (rows + 16 * kDeltaRows - 1) / (16 * kDeltaRows);
  const dim3 grid((unsigned)blocks);
  switch (a.head_dim) {
    case 64: hipLaunchKernelGGL(bwd_delta_kernel<64>, grid, dim3(256), 0, stream, a, rows); break;
    case 96: hipLaunchKernelGGL(bwd_delta_kernel<96>, grid, dim3(256), 0, stream, a, rows); break;
    case 128: hipLaunchKernelGGL(bwd_delta_kernel<128>, grid, dim3(256), 0, stream, a, rows); break;
    default: return WMX_E_UNSUPPORTED;
  }
  return WMX_OK;
}

// Largest dS buffer the backward uses (beyond it dQ recomputes S and dP).
constexpr int64_t kMaxDsBytes = (int64_t)4 << 30;

int64_t bwd_ds_bytes(const wmx_attn_args& a) {
  int64_t elems = 0;
  if (a.query_indices) {
    if (!a.ds_offsets || a.ds_elements <= 0) return 0;
    if (__builtin_mul_overflow(a.ds_elements, (int64_t)a.q_heads, &elems)) return 0;
  } else {
    const int64_t per = (int64_t)a.kv_len * ds_ld(a.q_len);
    if (__builtin_mul_overflow(per, (int64_t)a.batch * a.q_heads, &elems)) return 0;
  }
  // 64 rows of a query row block must stay within 32-bit buffer offsets
  const int64_t ld = ds_ld(a.query_indices ? a.max_queries : a.q_len);
  if (elems <= 0 || elems > kMaxDsBytes / 2 || ld * 2 * kTileRows >= ((int64_t)1 << 31)) return 0;
  return elems * 2;
}

int64_t bwd_min_workspace_size(const wmx_attn_args& a) { return bwd_acc_bytes(a); }

int64_t bwd_workspace_size(const wmx_attn_args& a) {
  const int64_t ds = bwd_ds_bytes(a);
  return ds > 0 ? bwd_ds_offset(a) + ds : bwd_acc_bytes(a);
}

bool bwd_uses_ds(const wmx_attn_args& a) {
  const int64_t ds = bwd_ds_bytes(a);
  return ds > 0 && a.workspace && a.workspace_bytes >= bwd_ds_offset(a) + ds;
}

// keys_unique 2: the segments' dummy marks start at zero; after every kernel
// that writes dummy parts, the parts are summed in segment order.
static int launch_dummy_marks_clear(const wmx_attn_args& a, hipStream_t stream) {
  const int64_t marks = bwd_dummy_mark_bytes(a) / (int64_t)sizeof(int32_t);
  hipLaunchKernelGGL(zero_f32_kernel, dim3((unsigned)((marks / 4 + 256) / 256)), dim3(256), 0, stream,
                     (float*)a.workspace, marks);
  return WMX_OK;
}
static int launch_dummy_reduce(const wmx_attn_args& a, hipStream_t stream) {
  const int cols = (2 * a.kv_heads * a.head_dim + 255) / 256;
  if ((int64_t)a.batch * cols > UINT32_MAX) return WMX_E_UNSUPPORTED;
  hipLaunchKernelGGL(dummy_reduce_kernel, dim3((unsigned)(a.batch * cols)), dim3(256), 0, stream, a, cols);
  return WMX_OK;
}

template <int D, int MODE>
static int launch_dq_t(const wmx_attn_args& a, hipStream_t stream) {
  const int64_t qtiles = ((MODE == kVarlen ? a.max_queries : a.q_len) + 127) / 128;
  const int64_t per_head =
      a.q_units ? a.num_q_units : qtiles * (MODE == kVarlen ? a.num_segments : a.batch);
  const int64_t units = per_head * a.q_heads;
  if (units <= 0) return WMX_OK;
  if (units > UINT32_MAX) return WMX_E_UNSUPPORTED;
  if (bwd_uses_ds(a)) {
    hipLaunchKernelGGL((attn_bwd_dq_ds_kernel<D, MODE>), dim3((unsigned)units), dim3(256), 0, stream, a);
  } else {
    hipLaunchKernelGGL((attn_bwd_dq_kernel<D, MODE>), dim3((unsigned)units), dim3(256), 0, stream, a);
  }
  return WMX_OK;
}

template <int D, int MODE, bool ATOMIC, bool DS>
static void launch_dkv_kernel(const wmx_attn_args& a, dim3 grid, hipStream_t stream) {
  if (a.key_tile == 64) {
    hipLaunchKernelGGL((attn_bwd_dkv_kernel<D, MODE, ATOMIC, DS, 2>), grid, dim3(256), 0, stream, a);
  } else {
    hipLaunchKernelGGL((attn_bwd_dkv_kernel<D, MODE, ATOMIC, DS, 4>), grid, dim3(512), 0, stream, a);
  }
}

// dummy_steps: with keys_unique 2, clear the segments' marks first and sum the
// dummy's parts after (false when the caller brackets several kernels with
// those steps itself).
template <int D, int MODE>
static int launch_dkv_t(const wmx_attn_args& a, hipStream_t stream, bool dummy_steps = true) {
  const int bnk = a.key_tile == 64 ? 64 : 128;
  const int64_t ktiles = ((MODE == kVarlen ? a.max_keys : a.kv_len) + bnk - 1) / bnk;
  const int64_t per_head =
      (MODE == kVarlen && a.k_units) ? a.num_k_units : ktiles * (MODE == kVarlen ? a.num_segments : a.batch);
  const int64_t units = per_head * a.kv_heads;
  if (units <= 0) return WMX_OK;
  if (units > UINT32_MAX) return WMX_E_UNSUPPORTED;
  const dim3 grid((unsigned)units);
  const bool ds = bwd_uses_ds(a);
  if (MODE == kVarlen && a.keys_unique == 2) {
    // slot 0 through per-segment parts and an ordered sum, every other row stored directly
    if (dummy_steps) {
      const int rc = launch_dummy_marks_clear(a, stream);
      if (rc != WMX_OK) return rc;
    }
    if (ds) launch_dkv_kernel<D, MODE, false, true>(a, grid, stream);
    else launch_dkv_kernel<D, MODE, false, false>(a, grid, stream);
    if (dummy_steps) return launch_dummy_reduce(a, stream);
  } else if (MODE == kVarlen && a.keys_unique != 1) {
    // any key row may repeat: every row through fp32 atomics
    const int64_t n = bwd_acc_bytes(a) / (int64_t)sizeof(float);
    hipLaunchKernelGGL(zero_f32_kernel, dim3((unsigned)((n / 4 + 256) / 256)), dim3(256), 0, stream,
                       (float*)a.workspace, n);
    if (ds) {
      launch_dkv_kernel<D, MODE, true, true>(a, grid, stream);
    } else {
      launch_dkv_kernel<D, MODE, true, false>(a, grid, stream);
    }
    const int64_t total = n / 2;
    hipLaunchKernelGGL(acc_to_bf16_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, a);
  } else if (ds) {
    launch_dkv_kernel<D, MODE, false, true>(a, grid, stream);
  } else {
    launch_dkv_kernel<D, MODE, false, false>(a, grid, stream);
  }
  return WMX_OK;
}

template <int MODE>
static int launch_part(const wmx_attn_args& a, hipStream_t stream, bool dq) {
  switch (a.head_dim) {
    case 64: return dq ? launch_dq_t<64, MODE>(a, stream) : launch_dkv_t<64, MODE>(a, stream);
    case 96: return dq ? launch_dq_t<96, MODE>(a, stream) : launch_dkv_t<96, MODE>(a, stream);
    case 128: return dq ? launch_dq_t<128, MODE>(a, stream) : launch_dkv_t<128, MODE>(a, stream);
    default: return WMX_E_UNSUPPORTED;
  }
}

static int launch_bwd_part(const wmx_attn_args& a, hipStream_t stream, bool dq) {
  if (a.query_indices) return launch_part<kVarlen>(a, stream, dq);
  if (a.q_seg) return launch_part<kDoc>(a, stream, dq);
  return launch_part<kDense>(a, stream, dq);
}

int launch_bwd_dq(const wmx_attn_args& a, hipStream_t stream) { return launch_bwd_part(a, stream, true); }
int launch_bwd_dkv(const wmx_attn_args& a, hipStream_t stream) { return launch_bwd_part(a, stream, false); }

// Listed short segments through the fused kernel, the rest through dK/dV and
// dQ (the caller's k_units and q_units exclude the listed segments).
static int launch_bwd_fused(const wmx_attn_args& a, hipStream_t stream) {
  const bool parts = a.keys_unique == 2;
  int rc = parts ? launch_dummy_marks_clear(a, stream) : WMX_OK;
  if (rc == WMX_OK) rc = launch_bwd_seg(a, stream);
  if (rc == WMX_OK) {
    switch (a.head_dim) {
      case 64: rc = launch_dkv_t<64, kVarlen>(a, stream, false); break;
      case 96: rc = launch_dkv_t<96, kVarlen>(a, stream, false); break;
      case 128: rc = launch_dkv_t<128, kVarlen>(a, stream, false); break;
      default: rc = WMX_E_UNSUPPORTED;
    }
  }
  if (rc == WMX_OK) rc = launch_bwd_dq(a, stream);
  if (rc == WMX_OK && parts) rc = launch_dummy_reduce(a, stream);
  return rc;
}

int launch_bwd(const wmx_attn_args& a, hipStream_t stream) {
  int rc = launch_bwd_preprocess(a, stream);
  if (rc == WMX_OK && a.f_units && a.num_f_units > 0) return launch_bwd_fused(a, stream);
  if (bwd_uses_ds(a)) {
    // dQ reads the dS that the dK/dV kernel stores
    if (rc == WMX_OK) rc = launch_bwd_dkv(a, stream);
    if (rc == WMX_OK) rc = launch_bwd_dq(a, stream);
  } else {
    if (rc == WMX_OK) rc = launch_bwd_dq(a, stream);
    if (rc == WMX_OK) rc = launch_bwd_dkv(a, stream);
  }
  return rc;
}

}  // namespace wmx

// Explicit instantiations of the launched kernels: every launcher above then
// finds its host stub even where the compiler would not emit one for an
// instantiation first seen next to a branch it folds away.
namespace wmx {
#define WMX_DKV_KERNELS(D, M, A, S)                                                 \
  template __global__ void attn_bwd_dkv_kernel<D, M, A, S, 2>(const wmx_attn_args); \
  template __global__ void attn_bwd_dkv_kernel<D, M, A, S, 4>(const wmx_attn_args);
#define WMX_BWD_KERNELS_MODE(D, M)                                                 \
  template __global__ void attn_bwd_dq_kernel<D, M>(const wmx_attn_args);          \
  template __global__ void attn_bwd_dq_ds_kernel<D, M>(const wmx_attn_args);       \
  WMX_DKV_KERNELS(D, M, false, false)                                              \
  WMX_DKV_KERNELS(D, M, false, true)
#define WMX_BWD_KERNELS(D)                                                          \
  WMX_BWD_KERNELS_MODE(D, kDense)                                                   \
  WMX_BWD_KERNELS_MODE(D, kDoc)                                                     \
  WMX_BWD_KERNELS_MODE(D, kVarlen)                                                  \
  WMX_DKV_KERNELS(D, kVarlen, true, false)                                        \
  WMX_DKV_KERNELS(D, kVarlen, true, true)
WMX_BWD_KERNELS(64)
WMX_BWD_KERNELS(96)
WMX_BWD_KERNELS(128)
#undef WMX_BWD_KERNELS
#undef WMX_BWD_KERNELS_MODE
#undef WMX_DKV_KERNELS
}  // namespace wmx

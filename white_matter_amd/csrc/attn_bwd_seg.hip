// Fused backward of short varlen segments for gfx950 (CDNA4).
//
// One workgroup (8 waves) per (segment, head) of a segment with at most 128
// queries holds all of the segment's Q and dO rows in LDS and walks its keys
// in 64-row tiles. Per tile it forms S, dP, P and dS for every (query, key)
// pair, stores the tile's dK and dV rows (complete: no other workgroup sees
// these keys) and accumulates dQ in registers over the tiles; dQ is stored
// once at the end. No dS buffer, no second kernel for dQ, and each K/V row is
// read once. Key-tiled dK/dV and query-tiled dQ workgroups of such segments
// run about one query tile each, so their setup (bounds, K/V rows, first tile)
// is most of their time; here the setup is paid once per segment.
//
// Math as the other backward kernels (attn_bwd.hip): P = exp2(S c log2e -
// LSE log2e), dS = P (dP - delta), dV = P^T dO, dK = c dS^T Q, dQ = c dS K,
// with P and dS rounded to bf16 where they enter a product (the reference's
// backward contract: src/white_matter/ops/cyclic_attention/_tilelang/
// backward_key_value.py:102-132, backward_query.py:86-109).
//
// Step of key tile t (keys 64 t .. 64 t + 63), waves w = 0..7:
//   phase 1: wave w takes query block pqb (32 rows) and key half pkh (32
//            keys): S^T = K Q^T and dP^T = V dO^T (a lane owns one query
//            column, so its LSE and delta are scalars), P and dS to LDS as
//            [query][key] bf16;
//   phase 2: dV^T = dO^T P and dK^T = Q^T dS per (key half, 32 columns of D)
//            block, contracted over the query blocks that see the tile;
//            dQ^T += K^T dS^T per (query block, 32 columns of D).
// Two barriers per step. K tiles are double-buffered (the next one issued at
// the step's start); V has one buffer, refilled after the phase-1 barrier
// (phase 2 reads no V; a second V buffer measured no faster). A step's dK/dV
// rows are stored at the start of the next step, so that they complete while
// that step runs: the step barrier waits for every vector-memory operation of
// its wave, and stores issued at the end of a step would be waited for at
// once.
#include "attn_tiles.h"

namespace wmx {

constexpr int kSegRows = 128;  // queries a workgroup holds
constexpr int kSegKeys = 64;   // keys per step

// P and dS of one step: [query][key] bf16, query rows kPdLd = 68 elements
// (136 bytes, 34 dwords) apart. Row reads (32 queries x 8 bytes per 32 lanes)
// then hit 32 distinct even dwords (34 q mod 64): conflict-free; transposed
// reads (4 consecutive rows x 16 dwords per 32 lanes) are at most two-way.
// Every address is a per-lane base plus constants (no swizzle to recompute).
constexpr int kPdLd = kSegKeys + 4;

// Byte offset of this lane's transposed reads of key columns c0 .. c0 + 31
// (accumulator k-order of k-step s: rows 16 s + 8 (e / 4) + 4 half + e % 4
// for element e, as tile_tr_operand): k-step s adds 16 rows, the second
// 8-byte read 8 rows, both immediates.
__device__ __forceinline__ int pd_tr_base(int c0, int lane) {
  const int li = lane & 15, g = lane >> 4;
  const int c = c0 + 16 * (g & 1) + 4 * (li & 3);
  const int r = 4 * (g >> 1) + (li >> 2);
  return 2 * (r * kPdLd + c);
}
__device__ __forceinline__ bf16x8 pd_tr_get(const bf16* t, int base, int s) {
  const char* p = (const char*)t + base + 32 * kPdLd * s;
  const u32x2 lo = lds_read_tr4((const bf16*)p);
  const u32x2 hi = lds_read_tr4((const bf16*)(p + 16 * kPdLd));
  const u32x4 v = {lo[0], lo[1], hi[0], hi[1]};
  return as_bf16x8(v);
}

// Keys of query row q in the same k-order (16 s + 8 (e / 4) + 4 half + e % 4):
// base 2 (q kPdLd + 4 half); k-step s adds 32 s bytes, the second read 16.
__device__ __forceinline__ bf16x8 pd_row_get(const bf16* t, int base, int s) {
  const char* p = (const char*)t + base + 32 * s;
  const u32x2 lo = *reinterpret_cast<const u32x2*>(p);
  const u32x2 hi = *reinterpret_cast<const u32x2*>(p + 16);
  const u32x4 v = {lo[0], lo[1], hi[0], hi[1]};
  return as_bf16x8(v);
}

// Accumulator rows (32 columns of D, this lane's key or query) scaled and
// stored as bf16: after a dword swap with the partner lane (lane ^ 32, same
// column) each lane writes 8 consecutive elements, twice. Both lanes of a
// pair must execute it; `live` guards the stores only.
__device__ __forceinline__ void store_block_row(bf16* row, const f32x16& acc, float scale, int half, bool live) {
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int r = 8 * t;
    const u32x4 w = {pack_bf16x2(acc[r + 0] * scale, acc[r + 1] * scale), pack_bf16x2(acc[r + 2] * scale, acc[r + 3] * scale),
                     pack_bf16x2(acc[r + 4] * scale, acc[r + 5] * scale), pack_bf16x2(acc[r + 6] * scale, acc[r + 7] * scale)};
    const auto lo = __builtin_amdgcn_permlane32_swap(w[0], w[2], false, false);
    const auto hi = __builtin_amdgcn_permlane32_swap(w[1], w[3], false, false);
    if (live) *reinterpret_cast<u32x4*>(row + 16 * t + 8 * half) = u32x4{lo[0], hi[0], lo[1], hi[1]};
  }
}

template <int D, bool DUMMY>
__global__ __launch_bounds__(512, 1) void attn_bwd_seg_kernel(const wmx_attn_args args) {
  const wmx_attn_args& a = args;
  constexpr int NW = 8;
  constexpr int KS = D / 16, DB = D / 32;
  constexpr int QS = kSegRows / 16;  // query k-steps of phase 2
  // 32-column blocks of D per wave in dQ
  constexpr int PB = (DB + 1) / 2;
  // phase 2: a wave owns one 32-column block of dV or dK and NKH key halves
  // (both halves for D >= 96: 2 DB blocks of each kind for 8 waves)
  constexpr int NKH = DB >= 3 ? 2 : 1;
  using DMA = TileDMA<D, NW>;
  // Q and dO of the segment: 128 rows each (two 64-row tiles, one stack)
  __shared__ __attribute__((aligned(1024))) bf16 q_lds[2 * kTileElems];
  __shared__ __attribute__((aligned(1024))) bf16 g_lds[2 * kTileElems];
  // K tiles (double-buffered: distinct arrays, so a prefetch into one is
  // known not to alias reads of the other) and the V tile
  __shared__ __attribute__((aligned(1024))) bf16 k_lds0[kTileElems];
  __shared__ __attribute__((aligned(1024))) bf16 k_lds1[kTileElems];
  __shared__ __attribute__((aligned(1024))) bf16 v_lds[kTileElems];
  __shared__ __attribute__((aligned(16))) bf16 p_lds[kSegRows * kPdLd];
  __shared__ __attribute__((aligned(16))) bf16 s_lds[kSegRows * kPdLd];

  // the segment from its work-list entry (fields required by the host): its
  // queries are slots qslot0 .. of row qrow, key 0 is slot kslot0 and key
  // j >= 1 slot kslot1 + j - 1 of row krow (consecutive layouts, checked by
  // the host)
  TileUnit tu;
  tu.decode(a.q_heads, (uint32_t)a.num_f_units, true, 1, a.f_units, a.num_segments, false, WMX_UNIT_FIELDS);
  if (!tu.ok) return;
  const int nq = tu.nq, nk = tu.nk, h = tu.head;
  if (nq <= 0 || nq > kSegRows || nk <= 0) return;  // the host lists only such segments
  const Bounds bound{(int64_t)nk - 1 - (int64_t)a.query_stride * (nq - 1), INT_MAX, a.query_stride, nk};
  auto key_slot = [&](int j) { return j == 0 ? tu.kslot0 : tu.kslot1 + j - 1; };

  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int half = lane >> 5, col = lane & 31;
  const int nqb = (nq + 31) >> 5;  // query blocks holding rows
  const int nt = (nk + kSegKeys - 1) / kSegKeys;
  // phase 1: query block pqb, key half pkh; waves 0-3 (one per SIMD) take
  // query blocks 0 and 1, so a segment of at most 64 queries keeps every
  // SIMD busy
  const int pqb = ((wave >> 2) << 1) | ((wave >> 1) & 1), pkh = wave & 1;
  const int qi = 32 * pqb + col;  // this lane's query in phase 1
  // phase 2: unit u = (kind, column block db) with key halves kb2 .. kb2 + NKH
  const int p2_u = NKH == 2 ? wave : wave >> 1;
  const bool p2_live = p2_u < 2 * DB;
  const bool p2_k = p2_u >= DB;  // dK (else dV)
  const int db = p2_live ? p2_u % DB : 0, kb2 = NKH == 2 ? 0 : wave & 1;
  // dQ^T: query block dqb, columns dq0 .. dq0 + PB
  const int dqb = wave >> 1, dq0 = (wave & 1) * PB;
  // byte offsets into P and dS: phase 1's writes (query qi, keys 32 pkh + 4 half
  // + 8 g), phase 2's transposed reads (key halves kb2 ..), dQ's row reads
  int pd_w = 2 * (qi * kPdLd + 32 * pkh + 4 * half), pd_q = 2 * ((32 * dqb + col) * kPdLd + 4 * half);
  int pd_b[NKH];
#pragma unroll
  for (int i = 0; i < NKH; ++i) pd_b[i] = pd_tr_base(32 * (kb2 + i), lane);

  // this lane's query statistics (phase 1)
  const float sl2 = a.softmax_scale * kLog2e;
  float nl2 = 0.f, dlt = 0.f;
  int lim = -1;  // last key this lane's query sees (-1: none)
  if (qi < nq) {
    const int64_t idx = ((int64_t)tu.qrow * a.q_heads + h) * a.q_len + tu.qslot0 + qi;
    nl2 = -a.lse[idx] * kLog2e;
    dlt = a.delta[idx];
    lim = bound.lim(qi);
  }

  DMA dma;
  dma.init(wave, lane);
  {
    // Q and dO rows, strided from the segment's first query slot; rows past
    // nq fall outside the buffer resources and read as zeros
    const int64_t qb = (int64_t)tu.qrow * a.q_stride[0] + (int64_t)h * a.q_stride[1];
    const int64_t gb = (int64_t)tu.qrow * a.do_stride[0] + (int64_t)h * a.do_stride[1];
    const int qrb = (int)a.q_stride[2] * 2, grb = (int)a.do_stride[2] * 2;
    unsigned qoff[DMA::kInstr], goff[DMA::kInstr];
    dma.strided_offsets(qrb, qoff);
    dma.strided_offsets(grb, goff);
    for (int m0 = 0; m0 < nq; m0 += kTileRows) {
      const int nvalid = min(nq - m0, kTileRows);
      const int64_t slot = tu.qslot0 + m0;
      dma.issue_strided(make_rsrc((const bf16*)a.q + qb + slot * a.q_stride[2], nvalid * qrb), q_lds + m0 * kRowElems, qoff);
      dma.issue_strided(make_rsrc((const bf16*)a.dout + gb + slot * a.do_stride[2], nvalid * grb), g_lds + m0 * kRowElems,
                        goff);
    }
  }
  // K/V rows: tile 0 gathered (key 0 may sit apart from the others), later
  // tiles strided from slot kslot1 + n0 - 1
  const bf16* kslice = (const bf16*)a.k + (int64_t)tu.krow * a.k_stride[0] + (int64_t)h * a.k_stride[1];
  const bf16* vslice = (const bf16*)a.v + (int64_t)tu.krow * a.v_stride[0] + (int64_t)h * a.v_stride[1];
  const int krb = (int)a.k_stride[2] * 2, vrb = (int)a.v_stride[2] * 2;
  unsigned koff[DMA::kInstr], voff[DMA::kInstr];
  dma.strided_offsets(krb, koff);
  dma.strided_offsets(vrb, voff);
  auto issue_k = [&](bf16* tile, int n0) __attribute__((always_inline)) {
    const int64_t slot = (int64_t)tu.kslot1 + n0 - 1;
    dma.issue_strided(make_rsrc(kslice + slot * a.k_stride[2], min(nk - n0, kTileRows) * krb), tile, koff);
  };
  auto issue_v = [&](int n0) __attribute__((always_inline)) {
    const int64_t slot = (int64_t)tu.kslot1 + n0 - 1;
    dma.issue_strided(make_rsrc(vslice + slot * a.v_stride[2], min(nk - n0, kTileRows) * vrb), v_lds, voff);
  };
  dma.issue_gathered2(k_lds0, v_lds, [&](int tr, bool& ok, const bf16*& kp, const bf16*& vp) {
    ok = tr < nk;
    const int64_t slot = ok ? key_slot(tr) : tu.kslot0;
    kp = kslice + slot * a.k_stride[2];
    vp = vslice + slot * a.v_stride[2];
  });

  // row-read offsets with the wave's 32-row block folded in: K and V rows of
  // key half pkh, Q and dO rows of query block pqb
  RowReads<KS> rkv, rqg;
  rkv.init(col, half);
  rqg.init(col, half);
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    rkv.off[s] += 8192 * pkh;
    rqg.off[s] += 8192 * pqb;
  }
  TrReads<PB> trq;  // transposed reads of the wave's dQ columns of D (K^T)
  trq.init(lane, 32 * dq0);

  // operands that every step reuses, read from LDS once the tiles have
  // landed: the wave's Q rows (phase 1, B operands of S^T over D) and its
  // Q^T or dO^T columns over the 128 queries (phase 2, A operands); the dO
  // rows of dP^T stay in LDS (registers: at D = 128 holding them as well
  // spills)
  bf16x8 qreg[KS], areg[QS];
  auto fill_registers = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int s = 0; s < KS; ++s) qreg[s] = rqg.get(q_lds, s, 0);
    TrReads<1> tra;
    tra.init(lane, 32 * db);
    const bf16* const a_src = p2_k ? q_lds : g_lds;
#pragma unroll
    for (int s = 0; s < QS; ++s) areg[s] = tra.get(a_src, 0, s);
  };

  f32x16 qacc[PB], kvacc[NKH];
#pragma unroll
  for (int i = 0; i < PB; ++i) qacc[i] = f32x16{};

  // stores of step t's dK or dV blocks (held in kvacc)
  auto store_kv = [&](int t) __attribute__((always_inline)) {
    if (!p2_live) return;
    const float scale = p2_k ? a.softmax_scale : 1.f;
#pragma unroll
    for (int i = 0; i < NKH; ++i) {
      const int j = t * kSegKeys + 32 * (kb2 + i) + col;
      const bool live = j < nk;
      const int64_t slot = key_slot(live ? j : 0);
      bf16* row = p2_k ? (bf16*)row_at(a.dk, a.dk_stride, tu.krow, h, (int)slot)
                       : (bf16*)row_at(a.dv, a.dv_stride, tu.krow, h, (int)slot);
      bool direct = live;
      if constexpr (DUMMY) {
        // the row's dummy (slot 0, shared by its segments): this segment's
        // part, [dK, dV][segment][kv head][D] fp32, and its mark (row + 1);
        // the parts are summed in segment order by dummy_reduce_kernel
        if (t == 0 && kb2 + i == 0 && tu.kslot0 == 0) {
          if (live && j == 0) {
            float* dst = (float*)((char*)a.workspace + bwd_dummy_mark_bytes(a)) +
                         (((p2_k ? 0 : (int64_t)a.num_segments) + tu.grp) * a.kv_heads + h) * D + 32 * db;
#pragma unroll
            for (int r = 0; r < 16; ++r) dst[8 * (r >> 2) + 4 * half + (r & 3)] = kvacc[i][r] * scale;
            if (!p2_k && db == 0) ((int32_t*)a.workspace)[tu.grp] = tu.krow + 1;
          }
          direct = live && j != 0;
        }
      }
      store_block_row(row + 32 * db, kvacc[i], scale, half, direct);
    }
  };

  // phase 1 of step t on tiles kt, vt: S^T and dP^T chains interleaved
  auto phase1 = [&](const bf16* kt, const bf16* vt, int t) __attribute__((always_inline)) {
    rkv.refresh();
    rqg.refresh();
    opaque(pd_w);
    constexpr int PF = KS < 2 ? KS : 2;
    f32x16 sacc = f32x16{}, dacc = f32x16{};
    bf16x8 ka[KS], va[KS], ga[KS];
#pragma unroll
    for (int s = 0; s < PF; ++s) {
      ka[s] = rkv.get(kt, s, 0);
      va[s] = rkv.get(vt, s, 0);
      ga[s] = rqg.get(g_lds, s, 0);
    }
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      __builtin_amdgcn_sched_barrier(0);
      if (s + PF < KS) {
        ka[s + PF] = rkv.get(kt, s + PF, 0);
        va[s + PF] = rkv.get(vt, s + PF, 0);
        ga[s + PF] = rqg.get(g_lds, s + PF, 0);
      }
      sacc = mfma32(ka[s], qreg[s], sacc);
      dacc = mfma32(va[s], ga[s], dacc);
    }
    __builtin_amdgcn_sched_barrier(0);
    // register r holds key kbase + 8 (r / 4) + 4 half + r % 4 of this lane's query
    const int kbase = t * kSegKeys + 32 * pkh;
    const bool full = 32 * pqb + 31 < nq && bound.lim(32 * pqb) >= kbase + 31;
    if (!full) {
      __asm__ volatile("");
      const int lim_c = lim - kbase - 4 * half;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int c = 8 * (r >> 2) + (r & 3);
        sacc[r] = c <= lim_c ? sacc[r] : kNegInf;
      }
    }
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      float p[4], ds[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        // a masked score is -inf and gives p = 0 exactly
        p[e] = __builtin_amdgcn_exp2f(fmaf(sacc[4 * g + e], sl2, nl2));
        ds[e] = p[e] * (dacc[4 * g + e] - dlt);
      }
      *reinterpret_cast<u32x2*>((char*)p_lds + pd_w + 16 * g) = u32x2{pack_bf16x2(p[0], p[1]), pack_bf16x2(p[2], p[3])};
      *reinterpret_cast<u32x2*>((char*)s_lds + pd_w + 16 * g) = u32x2{pack_bf16x2(ds[0], ds[1]), pack_bf16x2(ds[2], ds[3])};
    }
  };

  // phase 2 of step t: dV^T or dK^T blocks over query k-steps s0 .. s1 - 1
  // (the B operand, P or dS of the wave's key half, shared by its blocks),
  // then dQ^T += K^T dS^T over the tile's 64 keys
  auto phase2 = [&](const bf16* kt, int s0, int s1, bool dq_live) __attribute__((always_inline)) {
    trq.refresh();
    opaque(pd_q);
#pragma unroll
    for (int i = 0; i < NKH; ++i) opaque(pd_b[i]);
#pragma unroll
    for (int i = 0; i < NKH; ++i) kvacc[i] = f32x16{};
    // unrolled over the 4 query blocks (the A operands are registers indexed
    // by the k-step), the blocks outside [s0 / 2, s1 / 2) skipped; a block's
    // B operands are all read before its products, and nothing is carried
    // from one block to the next (no register copies at the skipped blocks'
    // joins). The B array is named, not selected at run time: reads through
    // a selected pointer wait for the V tile's direct-to-LDS loads (the
    // compiler cannot tell the arrays apart)
    auto kv_blocks = [&](const bf16* src) __attribute__((always_inline)) {
#pragma unroll
      for (int qb = 0; qb < QS / 2; ++qb) {
        if (2 * qb >= s0 && 2 * qb < s1) {
          __builtin_amdgcn_sched_barrier(0);
          bf16x8 cb[2][NKH];
#pragma unroll
          for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int i = 0; i < NKH; ++i) cb[j][i] = pd_tr_get(src, pd_b[i], 2 * qb + j);
          __builtin_amdgcn_sched_barrier(0);  // all reads issued before the first product
#pragma unroll
          for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int i = 0; i < NKH; ++i) kvacc[i] = mfma32(areg[2 * qb + j], cb[j][i], kvacc[i]);
        }
      }
    };
    if (p2_live) {
      if (p2_k) kv_blocks(s_lds);
      else kv_blocks(p_lds);
    }
    __builtin_amdgcn_sched_barrier(0);
    if (dq_live) {
      // two groups of two key k-steps: a group's operands read before its
      // products
#pragma unroll
      for (int hs = 0; hs < kSegKeys / 32; ++hs) {
        __builtin_amdgcn_sched_barrier(0);
        bf16x8 cb[2], ca[2][PB];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          cb[j] = pd_row_get(s_lds, pd_q, 2 * hs + j);
#pragma unroll
          for (int i = 0; i < PB; ++i)
            if (dq0 + i < DB) ca[j][i] = trq.get(kt, i, 2 * hs + j);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int i = 0; i < PB; ++i)
            if (dq0 + i < DB) qacc[i] = mfma32(ca[j][i], cb[j], qacc[i]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  auto step = [&](auto bufc, int t) __attribute__((always_inline)) {
    constexpr int B = decltype(bufc)::value;
    bf16* const kt = B == 0 ? k_lds0 : k_lds1;
    bf16* const kn = B == 0 ? k_lds1 : k_lds0;
    // K(t) and V(t) have landed (the newest loads), and every wave is past
    // step t - 1 (its reads of P, dS, K(t - 1))
    dma_barrier();
    if (t == 0) fill_registers();
    if (t > 0) store_kv(t - 1);
    if (t + 1 < nt) issue_k(kn, (t + 1) * kSegKeys);
    // query blocks that see any key of the tile: from the block of the first
    // row that sees its first key (rows see more keys as they go)
    const int qbmin = bound.first_row(t * kSegKeys, nq) >> 5;
    if (pqb < nqb && pqb >= qbmin) phase1(kt, v_lds, t);
    lds_barrier();  // P and dS written; every wave is past its reads of V(t)
    if (t + 1 < nt) issue_v((t + 1) * kSegKeys);
    phase2(kt, 2 * qbmin, 2 * nqb, dqb < nqb && dqb >= qbmin);
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  for (int t = 0; t < nt; t += 2) {
    step(I0{}, t);
    if (t + 1 < nt) step(I1{}, t + 1);
  }
  store_kv(nt - 1);

  // dQ rows of query block dqb
  if (dqb < nqb) {
    const int q = 32 * dqb + col;
    bf16* row = (bf16*)row_at(a.dq, a.dq_stride, tu.qrow, h, tu.qslot0 + (q < nq ? q : 0));
#pragma unroll
    for (int i = 0; i < PB; ++i)
      if (dq0 + i < DB) store_block_row(row + 32 * (dq0 + i), qacc[i], a.softmax_scale, half, q < nq);
  }
}

template <int D>
static void launch_seg_d(const wmx_attn_args& a, dim3 grid, hipStream_t stream) {
  if (a.keys_unique == 2) {
    hipLaunchKernelGGL((attn_bwd_seg_kernel<D, true>), grid, dim3(512), 0, stream, a);
  } else {
    hipLaunchKernelGGL((attn_bwd_seg_kernel<D, false>), grid, dim3(512), 0, stream, a);
  }
}

int launch_bwd_seg(const wmx_attn_args& a, hipStream_t stream) {
  const int64_t units = (int64_t)a.num_f_units * a.q_heads;
  if (units <= 0) return WMX_OK;
  if (units > UINT32_MAX) return WMX_E_UNSUPPORTED;
  const dim3 grid((unsigned)units);
  switch (a.head_dim) {
    case 64: launch_seg_d<64>(a, grid, stream); break;
    case 96: launch_seg_d<96>(a, grid, stream); break;
    case 128: launch_seg_d<128>(a, grid, stream); break;
    default: return WMX_E_UNSUPPORTED;
  }
  return WMX_OK;
}

#define WMX_SEG_KERNELS(D)                                                   \
  template __global__ void attn_bwd_seg_kernel<D, false>(const wmx_attn_args); \
  template __global__ void attn_bwd_seg_kernel<D, true>(const wmx_attn_args);
WMX_SEG_KERNELS(64)
WMX_SEG_KERNELS(96)
WMX_SEG_KERNELS(128)
#undef WMX_SEG_KERNELS

}  // namespace wmx

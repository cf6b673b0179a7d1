// Per-workgroup problem resolution shared by the attention kernels.
//
// A workgroup owns either 128 query rows (forward, dQ) or 128 key rows (dK/dV)
// of one (batch row or varlen segment, head). These structs decode its
// logical index (heaviest units first over all heads), locate its rows, and
// evaluate the visibility bound
//   lim(i) = clamp(min(offset + stride * i, limit), -1, nk - 1)
// of wmx_attn_args.
#pragma once

#include <climits>

#include "lds_tiles.h"
#include "wmx_kernels.h"

namespace wmx {

// One work unit of a query- or key-tiled kernel: a batch row or varlen
// segment, a 128-row tile of it, and a head. Per head, units u = 0 .. count-1
// are heaviest first: u names a listed (segment, tile) pair when a work list
// is given (sorted by the host), else tile u / groups of batch row u % groups,
// tiles counted from the last one when `descending` (the heaviest query tiles
// of a causal problem are the last, the heaviest key tiles the first).
//
// Blocks start in index order as CU slots free up and are dealt round-robin
// over the 8 XCDs (block b runs on XCD b % 8). When the heads split evenly
// over the XCDs, XCD x takes heads [x H/8, (x+1) H/8), so every unit of a head
// shares one L2, in unit-major order (unit u of each of its heads, then unit
// u + 1: heaviest first over its heads) or head-major order (all units of
// one head, then the next head: fewer heads resident at a time). Otherwise
// units are unit-major over all heads. A launch has exactly count * heads
// blocks.
struct TileUnit {
  int grp, tile, head;
  bool ok;
  // the segment's bounds from a work-list entry that carries them (read
  // together, kept in scalar registers); has_fields is false when the list
  // holds (segment or row, tile) pairs only
  bool has_fields;
  int qs, nq, ks, nk, qrow, qslot0, qslot1, krow, kslot0, kslot1;
  int64_t ds_off;
  // fields: ints per list entry (2, or WMX_UNIT_FIELDS)
  __device__ __forceinline__ void decode(int heads, uint32_t count, bool unit_major, int tiles,
                                         const int32_t* list, int num_groups, bool descending, int fields = 2) {
    decode_at(blockIdx.x, heads, count, unit_major, tiles, list, num_groups, descending, fields);
  }
  // The same for logical block index b (a persistent grid's units).
  __device__ __forceinline__ void decode_at(uint32_t b, int heads, uint32_t count, bool unit_major, int tiles,
                                            const int32_t* list, int num_groups, bool descending, int fields = 2) {
    has_fields = false;
    const uint32_t nh = (uint32_t)heads;
    uint32_t u;
    if ((nh & 7u) == 0) {
      const uint32_t hpx = nh >> 3, x = b & 7u, s = b >> 3;
      if (unit_major) {
        u = s / hpx;
        head = (int)(x * hpx + (s - u * hpx));
      } else {
        const uint32_t hl = s / count;
        u = s - hl * count;
        head = (int)(x * hpx + hl);
      }
    } else {
      u = b / nh;
      head = (int)(b - u * nh);
    }
    ok = u < count && head < heads;
    if (!ok) return;
    if (list) {
      const int32_t* e = list + (size_t)(fields >= WMX_UNIT_FIELDS ? WMX_UNIT_FIELDS : 2) * u;
      if (fields >= WMX_UNIT_FIELDS) {
        has_fields = true;
        auto rd = [&](int f) { return __builtin_amdgcn_readfirstlane(e[f]); };
        qs = rd(WMX_UNIT_QUERY_START);
        nq = rd(WMX_UNIT_QUERIES);
        ks = rd(WMX_UNIT_KEY_START);
        nk = rd(WMX_UNIT_KEYS);
        qrow = rd(WMX_UNIT_QUERY_ROW);
        qslot0 = rd(WMX_UNIT_QUERY_SLOT0);
        qslot1 = rd(WMX_UNIT_QUERY_SLOT1);
        krow = rd(WMX_UNIT_KEY_ROW);
        kslot0 = rd(WMX_UNIT_KEY_SLOT0);
        kslot1 = rd(WMX_UNIT_KEY_SLOT1);
        ds_off = (int64_t)(uint32_t)rd(WMX_UNIT_DS_LO) | ((int64_t)rd(WMX_UNIT_DS_HI) << 32);
      }
      grp = __builtin_amdgcn_readfirstlane(e[WMX_UNIT_SEGMENT]);
      tile = __builtin_amdgcn_readfirstlane(e[WMX_UNIT_TILE]);
    } else {
      const int t = (int)(u / (uint32_t)num_groups);
      grp = (int)(u - (uint32_t)t * num_groups);
      tile = descending ? tiles - 1 - t : t;
    }
    ok = (unsigned)grp < (unsigned)num_groups && tile >= 0;
  }
};

struct Bounds {
  int64_t offset, limit, stride;
  int nk;
  __device__ __forceinline__ int lim(int i) const {
    int64_t l = offset + stride * (int64_t)i;
    l = l < limit ? l : limit;
    l = l < (int64_t)nk - 1 ? l : (int64_t)nk - 1;
    return (int)(l < -1 ? -1 : l);
  }
  // Smallest query row whose bound reaches key j (nq when none does).
  __device__ __forceinline__ int first_row(int j, int nq) const {
    if (j > nk - 1 || limit < j) return nq;
    const int64_t need = (int64_t)j - offset;
    if (need <= 0) return 0;
    if (stride == 1) return need < nq ? (int)need : nq;
    const int64_t num = need + stride - 1;
    // a 32-bit division where the operands fit (the 64-bit one is a long
    // instruction sequence in every workgroup's setup)
    const int64_t m = num <= INT32_MAX ? (int64_t)((uint32_t)num / (uint32_t)stride) : num / stride;
    return m < nq ? (int)m : nq;
  }
};

// The rows of one problem (a batch row of a dense call, or a varlen segment).
template <int MODE>
struct Problem {
  int b;        // batch row (dense / documents)
  int nq, nk;   // query and key rows
  Bounds bound;
  SegmentRows qrows, krows;  // varlen only

  // grp = batch row or segment index; the bounds come from the unit's
  // work-list entry when it carries them, else from cu_queries, cu_keys and
  // the index arrays (three dependent loads).
  __device__ __forceinline__ void init(const wmx_attn_args& a, int grp, const TileUnit& tu) {
    b = grp;
    if constexpr (MODE == kVarlen) {
      if (tu.has_fields) {
        nq = tu.nq;
        nk = tu.nk;
        if (nq > 0)
          qrows.set(a.query_indices + tu.qs, a.query_extent, a.segment_layout & kQueriesConsecutive,
                    a.segment_layout & kQueriesOneRow, false, tu.qrow, tu.qslot0, tu.qslot1);
        if (nk > 0)
          krows.set(a.key_indices + tu.ks, a.key_extent, a.segment_layout & kKeysConsecutive,
                    a.segment_layout & kKeysOneRow, true, tu.krow, tu.kslot0, tu.kslot1);
      } else {
        // one address for the whole wave: uniform values, kept in scalar registers
        const int qs = __builtin_amdgcn_readfirstlane(a.cu_queries[grp]);
        const int ks = __builtin_amdgcn_readfirstlane(a.cu_keys[grp]);
        nq = __builtin_amdgcn_readfirstlane(a.cu_queries[grp + 1]) - qs;
        nk = __builtin_amdgcn_readfirstlane(a.cu_keys[grp + 1]) - ks;
        if (nq > 0)
          qrows.init(a.query_indices + qs, nq, a.query_extent, a.segment_layout & kQueriesConsecutive,
                     a.segment_layout & kQueriesOneRow, false);
        if (nk > 0)
          krows.init(a.key_indices + ks, nk, a.key_extent, a.segment_layout & kKeysConsecutive,
                     a.segment_layout & kKeysOneRow, true);
      }
      // query i sees keys 0 .. nk - 1 - stride * (nq - 1 - i): the last query
      // sees every key of the segment (bottom-right causal at stride 1)
      bound = Bounds{(int64_t)nk - 1 - (int64_t)a.query_stride * (nq - 1), INT_MAX, a.query_stride, nk};
    } else {
      nq = a.q_len;
      nk = a.kv_len;
      bound = Bounds{a.row_offset ? __builtin_amdgcn_readfirstlane(a.row_offset[b]) : a.query_offset,
                     a.row_limit ? __builtin_amdgcn_readfirstlane(a.row_limit[b]) : INT_MAX, a.query_stride, nk};
    }
  }
  // (row, slot) of query row i and key row j (both must be in range)
  __device__ __forceinline__ void query_loc(int i, int& qb, int& qt) const {
    if constexpr (MODE == kVarlen) {
      qrows.locate(i, qb, qt);
    } else {
      qb = b;
      qt = i;
    }
  }
  __device__ __forceinline__ void key_loc(int j, int& kb, int& kt) const {
    if constexpr (MODE == kVarlen) {
      krows.locate(j, kb, kt);
    } else {
      kb = b;
      kt = j;
    }
  }
};

// Segment grp's dS block offset: from its work-list entry when it has one.
__device__ __forceinline__ int64_t ds_offset_of(const wmx_attn_args& a, int grp, const TileUnit& tu) {
  return tu.has_fields ? tu.ds_off : a.ds_offsets[grp];
}

__device__ __forceinline__ const bf16* row_at(const void* base, const int64_t* st, int b, int h, int t) {
  return (const bf16*)base + (int64_t)b * st[0] + (int64_t)h * st[1] + (int64_t)t * st[2];
}

// The key (and value) rows of one problem and kv head as 64-row LDS tiles.
// Keys [0, reach) are loaded, later rows read as zeros. Where the keys sit at
// a fixed stride in one row (dense rows; a varlen segment with consecutive
// slots from key 1 on) a tile is a strided load from a per-tile base;
// otherwise, and under a key mask (masked-out slots may hold anything), each
// row is located and gathered.
template <int MODE, int D, int NW = 4>
struct KeyTiles {
  const bf16 *kslice, *vslice;  // slot 0 of the keys' row, kv head hk
  int64_t kst, vst;             // slot strides (elements)
  int kfirst;                   // strided: key j at slot kfirst + j
  int reach;
  bool strided;
  unsigned koff[TileDMA<D, NW>::kInstr], voff[TileDMA<D, NW>::kInstr];
  int b, hk, nk;

  __device__ __forceinline__ void init(const wmx_attn_args& a, const Problem<MODE>& pb, int hk_, int reach_,
                                       const TileDMA<D, NW>& dma) {
    b = pb.b;
    hk = hk_;
    nk = pb.nk;
    reach = reach_;
    int kb0 = b, kslot0 = 0;
    kfirst = 0;
    if constexpr (MODE == kVarlen) {
      if (nk > 0) {
        pb.key_loc(0, kb0, kslot0);
        if (nk > 1) {
          int kb1, kslot1;
          pb.key_loc(1, kb1, kslot1);
          kfirst = kslot1 - 1;
        }
      }
    }
    kslice = row_at(a.k, a.k_stride, kb0, hk, 0);
    vslice = row_at(a.v, a.v_stride, kb0, hk, 0);
    kst = a.k_stride[2];
    vst = a.v_stride[2];
    const bool layout_ok = MODE != kVarlen || (a.segment_layout & kKeysConsecutive);
    const bool mask_free = !(MODE == kDense && a.key_mask);
    // rows must not overlap (zero rows past the buffer end) and 64 rows must
    // fit 32-bit offsets
    const bool stride_ok = kst >= D && vst >= D && kst < (1 << 23) && vst < (1 << 23);
    strided = layout_ok && mask_free && stride_ok;
    dma.strided_offsets(strided ? (int)kst * 2 : 0, koff);
    dma.strided_offsets(strided ? (int)vst * 2 : 0, voff);
  }

  template <class Args>
  __device__ __forceinline__ void issue(const Args& a, const Problem<MODE>& pb, const TileDMA<D, NW>& dma, int n0,
                                        bf16* ktile, bf16* vtile) const {
    if (strided && (MODE != kVarlen || n0 > 0)) {
      const int nvalid = min(max(reach - n0, 0), kTileRows);
      const int64_t slot = (int64_t)kfirst + n0;
      const rsrc_t rk = make_rsrc(kslice + slot * kst, nvalid * (int)kst * 2);
      const rsrc_t rv = make_rsrc(vslice + slot * vst, nvalid * (int)vst * 2);
      dma.issue_strided(rk, ktile, koff);
      dma.issue_strided(rv, vtile, voff);
    } else {
      dma.issue_gathered2(ktile, vtile, [&](int tr, bool& ok, const bf16*& kp, const bf16*& vp) {
        const int j = n0 + tr;
        ok = j < reach;
        if constexpr (MODE == kDense) {
          if (a.key_mask) ok = ok && a.key_mask[(int64_t)b * a.key_mask_stride + min(j, nk - 1)] != 0;
        }
        int kb, kt;
        pb.key_loc(ok ? j : 0, kb, kt);
        kp = row_at(a.k, a.k_stride, kb, hk, kt);
        vp = row_at(a.v, a.v_stride, kb, hk, kt);
      });
    }
  }
};

// The key rows alone (K tiles of the dQ kernel that reads a stored dS).
template <int MODE, int D, int NW>
__device__ __forceinline__ void issue_key_tile(const KeyTiles<MODE, D, NW>& kt, const wmx_attn_args& a,
                                               const Problem<MODE>& pb, const TileDMA<D, NW>& dma, int n0,
                                               bf16* ktile) {
  if (kt.strided && (MODE != kVarlen || n0 > 0)) {
    const int nvalid = min(max(kt.reach - n0, 0), kTileRows);
    const int64_t slot = (int64_t)kt.kfirst + n0;
    dma.issue_strided(make_rsrc(kt.kslice + slot * kt.kst, nvalid * (int)kt.kst * 2), ktile, kt.koff);
  } else {
    dma.issue_gathered1(ktile, [&](int tr, bool& ok, const bf16*& kp) {
      const int j = n0 + tr;
      ok = j < kt.reach;
      if constexpr (MODE == kDense) {
        if (a.key_mask) ok = ok && a.key_mask[(int64_t)kt.b * a.key_mask_stride + min(j, kt.nk - 1)] != 0;
      }
      int kb, ks;
      pb.key_loc(ok ? j : 0, kb, ks);
      kp = row_at(a.k, a.k_stride, kb, kt.hk, ks);
    });
  }
}

// The query and output-gradient rows of one problem as LDS tiles of ROWS rows
// (Q and dO share the row addressing), for any query head. Rows past nq read
// as zeros. Dense rows and varlen segments with consecutive query slots are
// strided loads; other varlen layouts gather each row.
template <int MODE, int D, int NW = 4, int ROWS = kTileRows>
struct QueryTiles {
  const bf16 *qslice, *gslice;  // slot 0 of the queries' row, head 0
  int64_t qst, gst, qhs, ghs;   // slot and head strides (elements)
  int qfirst;                   // strided: query m at slot qfirst + m of row qrow
  int qrow;
  int nq;
  bool strided;

  __device__ __forceinline__ void init(const wmx_attn_args& a, const Problem<MODE>& pb) {
    nq = pb.nq;
    int qb0 = pb.b;
    qfirst = 0;
    qrow = pb.b;
    if constexpr (MODE == kVarlen) {
      if (nq > 0) pb.query_loc(0, qb0, qfirst);
    }
    qrow = qb0;
    qslice = row_at(a.q, a.q_stride, qb0, 0, 0);
    gslice = row_at(a.dout, a.do_stride, qb0, 0, 0);
    qst = a.q_stride[2];
    gst = a.do_stride[2];
    qhs = a.q_stride[1];
    ghs = a.do_stride[1];
    const bool layout_ok = MODE != kVarlen || (a.segment_layout & kQueriesConsecutive);
    const bool stride_ok = qst >= D && gst >= D && qst < (1 << 23) && gst < (1 << 23);
    strided = layout_ok && stride_ok;
  }

  __device__ __forceinline__ void issue(const wmx_attn_args& a, const Problem<MODE>& pb,
                                        const TileDMA<D, NW, ROWS>& dma, int hq, int m0, bf16* qtile,
                                        bf16* gtile) const {
    if (strided) {
      const int nvalid = min(max(nq - m0, 0), ROWS);
      const int64_t slot = (int64_t)qfirst + m0;
      const rsrc_t rq = make_rsrc(qslice + hq * qhs + slot * qst, nvalid * (int)qst * 2);
      const rsrc_t rg = make_rsrc(gslice + hq * ghs + slot * gst, nvalid * (int)gst * 2);
      dma.issue_strided_rows(rq, qtile, (int)qst * 2);
      dma.issue_strided_rows(rg, gtile, (int)gst * 2);
    } else {
      dma.issue_gathered2(qtile, gtile, [&](int tr, bool& ok, const bf16*& qp, const bf16*& gp) {
        const int m = m0 + tr;
        ok = m < nq;
        int rb, rt;
        pb.query_loc(ok ? m : 0, rb, rt);
        qp = row_at(a.q, a.q_stride, rb, hq, rt);
        gp = row_at(a.dout, a.do_stride, rb, hq, rt);
      });
    }
  }
};

}  // namespace wmx

// Device helpers shared by the gfx950 attention kernels.
//
// Operand layouts of v_mfma_f32_32x32x16_bf16 (one wave64):
//   A (32 x 16): lane l holds row l % 32, k = 8 * (l / 32) + [0, 8)
//   B (16 x 32): lane l holds column l % 32, k = 8 * (l / 32) + [0, 8)
//   C (32 x 32): lane l, register r holds column l % 32,
//                row 8 * (r / 4) + 4 * (l / 32) + r % 4
// A product whose contraction index is read from an accumulator (for
// example P in O^T = V^T P^T) uses the accumulator's row order as its k
// order: lane half h supplies k = {16s + 4h + [0,4), 16s + 8 + 4h + [0,4)}
// for k-step s, which is registers 8(s%2) .. 8(s%2)+7 of 32-row block s/2.
// The other operand of that product reads the same k order from LDS.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "wmx_attn.h"

namespace wmx {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kNegInf = -__builtin_inff();
constexpr float kPosInf = __builtin_inff();
// An unchanged running maximum must rescale by exactly one, and a row that
// has seen only masked scores must produce zero weights (not NaN).
constexpr float kMaxFloor = -1e30f;

__device__ __forceinline__ f32x16 mfma32(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Two fp32 values to a packed bf16 pair (round to nearest even, hardware cvt).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  bf16x2 r;
  r[0] = (__bf16)lo;
  r[1] = (__bf16)hi;
  return __builtin_bit_cast(uint32_t, r);
}

__device__ __forceinline__ bf16x8 as_bf16x8(const u32x4& v) { return __builtin_bit_cast(bf16x8, v); }

__device__ __forceinline__ u32x4 load16(const bf16* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ void store8(bf16* p, const u32x2& v) { *reinterpret_cast<u32x2*>(p) = v; }

// -- row helpers of the HBM-bound kernels (KV-pool producer and store) --
// Round to bf16 (nearest even) and back: the reference's per-op rounding
// when the keys are bf16.
__device__ __forceinline__ float round_bf16(float x) { return (float)(__bf16)x; }

// Eight consecutive elements as fp32 from an fp32 or bf16 array. STREAM marks
// data read exactly once (the keys and values): a non-temporal load, which
// keeps it from displacing the cos/sin rows that every channel re-reads.
template <bool STREAM = false>
__device__ __forceinline__ void load8(const void* base, int64_t off, bool bf16_src, float (&v)[8]) {
  auto ld = [](const auto* p) { return STREAM ? __builtin_nontemporal_load(p) : *p; };
  if (bf16_src) {
    const u32x4 w = ld(reinterpret_cast<const u32x4*>((const bf16*)base + off));
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[2 * e] = bf16_lo(w[e]);
      v[2 * e + 1] = bf16_hi(w[e]);
    }
  } else {
    const f32x4 a = ld(reinterpret_cast<const f32x4*>((const float*)base + off));
    const f32x4 b = ld(reinterpret_cast<const f32x4*>((const float*)base + off + 4));
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[e] = a[e];
      v[4 + e] = b[e];
    }
  }
}

// Pool rows are written once and not read back by this kernel: non-temporal.
__device__ __forceinline__ void store8_bf16(void* base, int64_t off, const float (&v)[8]) {
  const u32x4 w = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]),
                   pack_bf16x2(v[6], v[7])};
  __builtin_nontemporal_store(w, reinterpret_cast<u32x4*>((bf16*)base + off));
}


// Reductions across the two halves of a wave (lane l with lane l ^ 32),
// with v_permlane32_swap: the two results hold x[l] and x[l ^ 32] in some order.
__device__ __forceinline__ float max_halves(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_halves(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Wave index as a scalar, so that values derived from it stay wave-uniform.
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// Row-addressing of one operand: dense (b fixed, row t) or varlen (flat index).
struct RowSource {
  const bf16* base;
  int64_t sb, sh, st;
};

__device__ __forceinline__ const bf16* row_ptr(const RowSource& s, int b, int h, int t) {
  return s.base + (int64_t)b * s.sb + (int64_t)h * s.sh + (int64_t)t * s.st;
}

// Flat varlen index -> (row, slot) for a row width `extent`.
__device__ __forceinline__ void split_flat(int64_t flat, int extent, int& b, int& t) {
  b = (int)(flat / extent);
  t = (int)(flat - (int64_t)b * extent);
}

// segment_layout bits of wmx_attn_args
constexpr int kQueriesConsecutive = 1;  // query i of a segment sits at slot t0 + i of one row
constexpr int kKeysConsecutive = 2;     // key j >= 1 sits at slot t1 + j - 1 of one row
constexpr int kQueriesOneRow = 4;       // every query of a segment is in the row of its first
constexpr int kKeysOneRow = 8;          // every key of a segment is in the row of its first

// Where the rows of one varlen segment live: one division per workgroup,
// then per-row slots by addition (consecutive layout) or by subtracting the
// row base from the gathered flat index (one row); the general case divides.
struct SegmentRows {
  const int64_t* idx;  // the segment's first flat index
  int extent;
  int layout;          // consecutive / one-row bits for this side
  bool from_one;       // consecutive from element 1 (keys: element 0 may be the dummy)
  int row;
  int64_t row_base;    // row * extent
  int slot0, slot1;    // slots of elements 0 and 1

  __device__ void init(const int64_t* first, int count, int extent_, bool consecutive, bool one_row, bool from_one_) {
    idx = first;
    extent = extent_;
    layout = (consecutive ? 1 : 0) | (one_row ? 2 : 0);
    from_one = from_one_;
    int t0 = 0;
    // one address for the whole wave: the values are uniform (scalar registers)
    split_flat(first[0], extent, row, t0);
    row = __builtin_amdgcn_readfirstlane(row);
    t0 = __builtin_amdgcn_readfirstlane(t0);
    row_base = (int64_t)row * extent;
    slot0 = t0;
    slot1 = __builtin_amdgcn_readfirstlane(count > 1 ? (int)(first[1] - row_base) : t0 + 1);
  }
  // The same from the entry's precomputed row and slots of elements 0 and 1.
  __device__ __forceinline__ void set(const int64_t* first, int extent_, bool consecutive, bool one_row, bool from_one_,
                                      int row_, int slot0_, int slot1_) {
    idx = first;
    extent = extent_;
    layout = (consecutive ? 1 : 0) | (one_row ? 2 : 0);
    from_one = from_one_;
    row = row_;
    row_base = (int64_t)row * extent;
    slot0 = slot0_;
    slot1 = slot1_;
  }
  __device__ __forceinline__ void locate(int j, int& b, int& t) const {
    if (layout & 1) {
      b = row;
      t = from_one ? (j == 0 ? slot0 : slot1 + j - 1) : slot0 + j;
    } else if (layout & 2) {
      b = row;
      t = (int)(idx[j] - row_base);
    } else {
      split_flat(idx[j], extent, b, t);
    }
  }
};

// Transposed LDS tiles t[d][n] are XOR-swizzled in groups of four elements:
// element (d, n) lives at d * ld + (n ^ tswz(d)). Groups of four stay
// contiguous (8-byte operand reads), and the 16 lanes that store one column
// chunk of a row pair hit 16 distinct banks instead of 2.
__device__ __forceinline__ int tswz(int d) { return ((d >> 3) & 7) << 2; }

// A [ROWS x D] bf16 tile staged through registers, read as row pairs so the
// same registers can be written to LDS row-major, transposed, or both.
// rp(r, ok) returns a dereferenceable global pointer for tile row r and sets
// ok = false for a row that must read as zeros (outside the problem or beyond
// every reader's reach); such rows are loaded from a valid row and zeroed, so
// the loads are branch-free.
template <int ROWS, int D, int NT = 256>
struct PairTile {
  static constexpr int CPR = D / 8;
  static constexpr int N = ROWS / 2 * CPR;
  static constexpr int PER = (N + NT - 1) / NT;
  u32x4 x[PER], y[PER];

  template <class RowPtr>
  __device__ __forceinline__ void load(int tid, RowPtr rp) {
#pragma unroll
    for (int r = 0; r < PER; ++r) {
      const int c = tid + NT * r;
      const int cl = c < N ? c : N - 1;
      const int p = cl / CPR, cc = cl % CPR;
      bool oka, okb;
      const bf16* ra = rp(2 * p, oka);
      const bf16* rb = rp(2 * p + 1, okb);
      const u32x4 wx = load16(ra + 8 * cc), wy = load16(rb + 8 * cc);
      const u32x4 z = {0u, 0u, 0u, 0u};
      x[r] = oka ? wx : z;
      y[r] = okb ? wy : z;
    }
  }
  // lds[row * ld + d]
  __device__ __forceinline__ void store_rows(int tid, bf16* lds, int ld) const {
#pragma unroll
    for (int r = 0; r < PER; ++r) {
      const int c = tid + NT * r;
      if (c < N) {
        const int p = c / CPR, cc = c % CPR;
        *reinterpret_cast<u32x4*>(lds + (2 * p) * ld + 8 * cc) = x[r];
        *reinterpret_cast<u32x4*>(lds + (2 * p + 1) * ld + 8 * cc) = y[r];
      }
    }
  }
  // lds[d * ld + (row ^ tswz(d))]; ld even, ROWS a multiple of 32
  __device__ __forceinline__ void store_cols(int tid, bf16* lds, int ld) const {
#pragma unroll
    for (int r = 0; r < PER; ++r) {
      const int c = tid + NT * r;
      if (c < N) {
        const int p = c / CPR, cc = c % CPR;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int d0 = 8 * cc + 2 * e;
          uint32_t* lo = reinterpret_cast<uint32_t*>(lds + d0 * ld + ((2 * p) ^ tswz(d0)));
          uint32_t* hi = reinterpret_cast<uint32_t*>(lds + (d0 + 1) * ld + ((2 * p) ^ tswz(d0 + 1)));
          *lo = (x[r][e] & 0xffffu) | (y[r][e] << 16);
          *hi = (x[r][e] >> 16) | (y[r][e] & 0xffff0000u);
        }
      }
    }
  }
};

// MFMA operand whose k order follows an accumulator's row order, read from a
// transposed, swizzled LDS tile: k = {16s + 4h + [0,4), 16s + 8 + 4h + [0,4)}.
__device__ __forceinline__ bf16x8 lds_kperm_operand(const bf16* t, int ld, int row, int s, int half) {
  const bf16* base = t + row * ld;
  const int sw = tswz(row);
  const u32x2 lo = *reinterpret_cast<const u32x2*>(base + ((16 * s + 4 * half) ^ sw));
  const u32x2 hi = *reinterpret_cast<const u32x2*>(base + ((16 * s + 8 + 4 * half) ^ sw));
  const u32x4 v = {lo[0], lo[1], hi[0], hi[1]};
  return as_bf16x8(v);
}

// Registers 8(s%2)..8(s%2)+7 of accumulator block acc as a bf16 MFMA operand.
__device__ __forceinline__ bf16x8 acc_kperm_operand(const f32x16& acc, int s) {
  const int base = 8 * (s & 1);
  u32x4 w;
  w[0] = pack_bf16x2(acc[base + 0], acc[base + 1]);
  w[1] = pack_bf16x2(acc[base + 2], acc[base + 3]);
  w[2] = pack_bf16x2(acc[base + 4], acc[base + 5]);
  w[3] = pack_bf16x2(acc[base + 6], acc[base + 7]);
  return as_bf16x8(w);
}

// Row of a row-major LDS tile as the MFMA operand for k-step s (k = d).
__device__ __forceinline__ bf16x8 lds_row_operand(const bf16* t, int ld, int row, int s, int half) {
  return as_bf16x8(*reinterpret_cast<const u32x4*>(t + row * ld + 16 * s + 8 * half));
}

// Store an accumulator holding X^T (rows d, column = this lane's row) as
// bf16 row x[d] scaled by `scale`. Lane (row, half) holds, per block d and
// group g, the columns d 32 + 8 g + 4 half + [0, 4); swapping dwords with its
// partner (lane ^ 32, the same row) gives it the 8 columns
// d 32 + 16 t + 8 half + [0, 8) of group pair t: one 16-byte store each. Both
// lanes of a pair must be active (they hold the same row).
template <int DB>
__device__ __forceinline__ void store_acc_row(bf16* row, const f32x16 (&acc)[DB], float scale, int half) {
#pragma unroll
  for (int d = 0; d < DB; ++d) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int r = 8 * t;
      const u32x4 w = {pack_bf16x2(acc[d][r + 0] * scale, acc[d][r + 1] * scale),
                       pack_bf16x2(acc[d][r + 2] * scale, acc[d][r + 3] * scale),
                       pack_bf16x2(acc[d][r + 4] * scale, acc[d][r + 5] * scale),
                       pack_bf16x2(acc[d][r + 6] * scale, acc[d][r + 7] * scale)};
      const auto lo = __builtin_amdgcn_permlane32_swap(w[0], w[2], false, false);
      const auto hi = __builtin_amdgcn_permlane32_swap(w[1], w[3], false, false);
      *reinterpret_cast<u32x4*>(row + d * 32 + 16 * t + 8 * half) = u32x4{lo[0], hi[0], lo[1], hi[1]};
    }
  }
}

}  // namespace wmx

namespace wmx {

// ds_read_b64_tr_b16 (gfx950): within each group of 16 lanes, lane li
// receives element li % 4 of the 8-byte chunks addressed by lanes li / 4 + 4k,
// k = 0..3 (checked on the device). If lane s of a group addresses
// t[(n0 + s / 4) * ld + d0 + 4 * (s % 4)], lane li receives
// t[(n0 + k) * ld + d0 + li] for k = 0..3: four consecutive rows of one column
// of a row-major tile, which is half of an MFMA operand whose contraction runs
// over the tile's rows.
__device__ __forceinline__ u32x2 lds_read_tr4(const bf16* p) {
  typedef short i16x4 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
  const i16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p));
  return __builtin_bit_cast(u32x2, v);
}

// MFMA operand (row index = lane % 32 of a 32-row block starting at column
// c0 of a row-major LDS tile t[n][c], contraction over the tile rows n in the
// accumulator k-order of k-step s): lane half h receives rows
// {16s + 4h + [0,4)} and {16s + 8 + 4h + [0,4)} of column c0 + lane % 32.
__device__ __forceinline__ bf16x8 lds_tr_operand(const bf16* t, int ld, int c0, int s, int lane) {
  const int li = lane & 15, g = lane >> 4;  // 16-lane group
  const int h = g >> 1;
  const int col = c0 + 16 * (g & 1) + 4 * (li & 3);
  const int row = 16 * s + 4 * h + (li >> 2);
  const u32x2 lo = lds_read_tr4(t + row * ld + col);
  const u32x2 hi = lds_read_tr4(t + (row + 8) * ld + col);
  const u32x4 v = {lo[0], lo[1], hi[0], hi[1]};
  return as_bf16x8(v);
}

// Row stride (elements) of a row-major tile read with lds_tr_operand: the 32
// lanes of one LDS pass read 4 rows x 16 dwords, so rows sit 16 (mod 64)
// dwords apart.
constexpr int tr_ld(int d) { return ((d / 2) % 64 == 16 || (d / 2) % 64 == 48) ? d : tr_ld(d + 8); }

}  // namespace wmx

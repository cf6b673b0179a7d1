// 64-row bf16 tiles in LDS, filled by direct-to-LDS loads (16 bytes per lane
// from global memory straight into LDS, no staging registers, no ds_write).
//
// Layout: a tile row holds 16 chunks of 16 bytes (up to 128 bf16; chunks past
// head_dim/8 are padding that no reader touches). Chunk c of row r is stored
// at chunk c ^ swz(r), swz(r) = 4 (r % 4) + (r / 4) % 4. With 64 banks of
// 4 bytes this keeps both read patterns of the kernels free of bank conflicts:
//   row operands - 16 lanes read 16 B of 16 different rows, same chunk;
//   tr operands  - 32 lanes read 8 B of 4 consecutive rows x 4 chunks
//                  (ds_read_b64_tr_b16, see wmx_device.h).
// One wave instruction fills 1 KB = 4 rows: lane l writes LDS bytes
// base + 16 l, i.e. physical chunk l % 16 of row l / 16, so the lane loads
// the logical chunk (l % 16) ^ swz(row).
//
// Two ways to fill a tile:
//   strided - rows at a fixed byte stride from a per-tile base, through a
//             buffer resource whose size ends at the last row to load: the
//             rows past it (outside the problem or past every reader's
//             reach) read as zeros, so NaN in unused cache capacity never
//             reaches the products;
//   gathered - one global address per row, zeros (from a zero chunk) for a
//             row that must not be read.
#pragma once

#include "wmx_device.h"

namespace wmx {

constexpr int kTileRows = 64;
constexpr int kRowElems = 128;
constexpr int kTileElems = kTileRows * kRowElems;  // 16 KB
constexpr unsigned kOutOfRange = 0x80000000u;      // past every tile buffer's size

__device__ __forceinline__ int tile_swz(int r) { return 4 * (r & 3) + ((r >> 2) & 3); }
__device__ __forceinline__ int tile_elem(int r, int c) { return r * kRowElems + 8 * (c ^ tile_swz(r)); }

// Row operand of k-step s (k = head_dim): row r, elements 16 s + 8 half .. + 8.
__device__ __forceinline__ bf16x8 tile_row_operand(const bf16* t, int r, int s, int half) {
  return as_bf16x8(*reinterpret_cast<const u32x4*>(t + tile_elem(r, 2 * s + half)));
}

// Transposed operand (contraction over tile rows, accumulator k-order of
// k-step s) for the 32 columns c0 .. c0 + 31, as lds_tr_operand.
__device__ __forceinline__ bf16x8 tile_tr_operand(const bf16* t, int c0, int s, int lane) {
  const int li = lane & 15, g = lane >> 4;
  const int col = c0 + 16 * (g & 1) + 4 * (li & 3);
  const int row = 16 * s + 4 * (g >> 1) + (li >> 2);
  const int within = col & 7;
  const u32x2 lo = lds_read_tr4(t + tile_elem(row, col >> 3) + within);
  const u32x2 hi = lds_read_tr4(t + tile_elem(row + 8, col >> 3) + within);
  const u32x4 v = {lo[0], lo[1], hi[0], hi[1]};
  return as_bf16x8(v);
}

// Keeps a value in a register as if it changed here: derived addresses are
// then formed at their use (register + immediate) instead of being hoisted
// out of the loop as one register per (buffer, k-step).
template <class T>
__device__ __forceinline__ void opaque(T& x) {
  __asm__ volatile("" : "+v"(x));
}
// The same for a wave-uniform value kept in a scalar register.
template <class T>
__device__ __forceinline__ void opaque_s(T& x) {
  __asm__ volatile("" : "+s"(x));
}

// This lane's byte offsets for the row operands of a 32-row block: row r
// (= lane % 32), k-steps s < KS. Row blocks 32 rows apart share the swizzle,
// so block nb adds the immediate 8192 nb.
template <int KS>
struct RowReads {
  int off[KS];
  __device__ __forceinline__ void init(int r, int half) {
#pragma unroll
    for (int s = 0; s < KS; ++s) off[s] = 2 * tile_elem(r, 2 * s + half);
  }
  __device__ __forceinline__ void refresh() {
#pragma unroll
    for (int s = 0; s < KS; ++s) opaque(off[s]);
  }
  __device__ __forceinline__ bf16x8 get(const bf16* t, int s, int nb) const {
    return as_bf16x8(*reinterpret_cast<const u32x4*>((const char*)t + off[s] + 8192 * nb));
  }
};

// This lane's byte offsets for transposed operands (see tile_tr_operand) of
// the 32-column blocks d < DB from column c0 on; k-step s adds 16 rows, the
// immediate 4096 s. Element e of the operand of k-step s comes from tile row
// 16 s + 8 (e / 4) + 4 (lane / 32) + e % 4.
template <int DB>
struct TrReads {
  int lo[DB], hi[DB];
  __device__ __forceinline__ void init(int lane, int c0 = 0) {
    const int li = lane & 15, g = lane >> 4;
    const int row = 4 * (g >> 1) + (li >> 2);
#pragma unroll
    for (int d = 0; d < DB; ++d) {
      const int c = c0 + 32 * d + 16 * (g & 1) + 4 * (li & 3);
      lo[d] = 2 * (tile_elem(row, c >> 3) + (c & 7));
      hi[d] = 2 * (tile_elem(row + 8, c >> 3) + (c & 7));
    }
  }
  __device__ __forceinline__ void refresh() {
#pragma unroll
    for (int d = 0; d < DB; ++d) {
      opaque(lo[d]);
      opaque(hi[d]);
    }
  }
  __device__ __forceinline__ bf16x8 get(const bf16* t, int d, int s) const {
    const char* base = (const char*)t + 4096 * s;
    const u32x2 l = lds_read_tr4((const bf16*)(base + lo[d]));
    const u32x2 h = lds_read_tr4((const bf16*)(base + hi[d]));
    const u32x4 v = {l[0], l[1], h[0], h[1]};
    return as_bf16x8(v);
  }
};

typedef __amdgpu_buffer_rsrc_t rsrc_t;
typedef __attribute__((address_space(3))) void lds_void;

// A raw byte buffer over [base, base + bytes); reads past it return zeros.
// Both arguments must be wave-uniform; they are moved to scalar registers
// explicitly so that the compiler never wraps a load in a per-lane loop.
__device__ __forceinline__ rsrc_t make_rsrc(const void* base, int bytes) {
  const uint64_t p = (uint64_t)base;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)p);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(p >> 32));
  void* up = (void*)(((uint64_t)hi << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(up, (short)0, __builtin_amdgcn_readfirstlane(bytes), 0x00020000);
}

// Source of the zero rows of gathered tiles.
static __device__ __attribute__((aligned(16))) const uint32_t kZeroChunk[4] = {0u, 0u, 0u, 0u};

// After global_load_lds: the compiler counts these direct-to-LDS loads (FLAT
// encoding) as LDS operations whose completion order it cannot track, and
// from then on waits for every outstanding LDS read (lgkmcnt(0)) wherever any
// one is needed, on every path that joins this one, so reads issued ahead of
// their products no longer overlap them. An explicit lgkmcnt(0) here settles
// that state once, on the path that issued the loads (buffer_load ... lds, the
// strided form, does not need it).
__device__ __forceinline__ void lgkm_settle() {
  __asm__ volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt left at their maximum
  __asm__ volatile("" ::: "memory");
}

// This thread's 16-byte slots of a ROWS-row tile (64, or the first 32 rows of
// the same layout) filled by NW waves: each wave fills ROWS / NW rows with
// ROWS / (4 NW) instructions of 4 rows.
template <int D, int NW = 4, int ROWS = kTileRows>
struct TileDMA {
  static constexpr int kInstr = ROWS / (4 * NW);  // instructions per wave per tile
  static_assert((NW == 2 || NW == 4 || NW == 8) && (ROWS == 32 || ROWS == 64) && kInstr >= 1,
                "2, 4 or 8 waves fill a tile");
  // Instruction r of wave w fills tile row 4 g + sub, g = kInstr w + r and
  // sub = lane / 16, whose swizzle is 4 sub + g % 4: the lane loads logical
  // chunk lc0 ^ (g % 4) with lc0 = (lane % 16) ^ 4 sub. Only these values are
  // kept; rows and offsets are formed per use.
  int wave, sub, lc0;

  __device__ __forceinline__ void init(int wave_, int lane) {
    wave = wave_;
    sub = lane >> 4;
    lc0 = (lane & 15) ^ (sub << 2);
  }
  __device__ __forceinline__ int group(int r) const { return wave * kInstr + r; }
  __device__ __forceinline__ int row(int r) const { return group(r) * 4 + sub; }
  // byte offset of this lane's chunk of instruction r in its row, or -1 for padding
  __device__ __forceinline__ int chunk16(int r) const {
    const int c = lc0 ^ (group(r) & 3);
    return (D == 128 || c < D / 8) ? 16 * c : -1;
  }
  __device__ __forceinline__ lds_void* dst(bf16* tile, int r) const { return (lds_void*)(tile + group(r) * 512); }
  // Per-lane byte offset of instruction r of a strided tile with row stride
  // row_bytes (0 <= row_bytes * ROWS < 2^31).
  __device__ __forceinline__ unsigned strided_offset(int r, int row_bytes) const {
    const int c = chunk16(r);
    return c < 0 ? kOutOfRange : (unsigned)(row(r) * row_bytes + c);
  }
  __device__ __forceinline__ void strided_offsets(int row_bytes, unsigned (&off)[kInstr]) const {
#pragma unroll
    for (int r = 0; r < kInstr; ++r) off[r] = strided_offset(r, row_bytes);
  }
  __device__ __forceinline__ void issue_strided(const rsrc_t& rs, bf16* tile, const unsigned (&off)[kInstr]) const {
#pragma unroll
    for (int r = 0; r < kInstr; ++r) __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, dst(tile, r), 16, off[r], 0, 0, 0);
  }
  // Offsets formed at issue time (no registers held between tiles: the
  // opaque row stride keeps the compiler from hoisting them out of the loop).
  __device__ __forceinline__ void issue_strided_rows(const rsrc_t& rs, bf16* tile, int row_bytes) const {
    opaque_s(row_bytes);
#pragma unroll
    for (int r = 0; r < kInstr; ++r)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, dst(tile, r), 16, strided_offset(r, row_bytes), 0, 0, 0);
  }
  // The same for data read once: the cache-policy immediate 2 is the
  // nontemporal hint on gfx950.
  __device__ __forceinline__ void issue_strided_rows_once(const rsrc_t& rs, bf16* tile, int row_bytes) const {
    opaque_s(row_bytes);
#pragma unroll
    for (int r = 0; r < kInstr; ++r)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, dst(tile, r), 16, strided_offset(r, row_bytes), 0, 0, 2);
  }
  // One tile: row(tr, ok, p) returns the address of tile row tr and sets
  // ok = false for a row that must read as zeros.
  template <class Row>
  __device__ __forceinline__ void issue_gathered1(bf16* t0, Row row_at_) const {
#pragma unroll
    for (int r = 0; r < kInstr; ++r) {
      bool ok;
      const bf16* p0;
      row_at_(row(r), ok, p0);
      const int c = chunk16(r);
      const void* s0 = (ok && c >= 0) ? (const void*)((const char*)p0 + c) : (const void*)kZeroChunk;
      __builtin_amdgcn_global_load_lds(s0, dst(t0, r), 16, 0, 0);
    }
    lgkm_settle();
  }
  // Two tiles whose rows are located together: rows(tr, ok, p0, p1) returns
  // the addresses of tile row tr and sets ok = false for a row that must read
  // as zeros.
  template <class Rows>
  __device__ __forceinline__ void issue_gathered2(bf16* t0, bf16* t1, Rows rows) const {
#pragma unroll
    for (int r = 0; r < kInstr; ++r) {
      bool ok;
      const bf16 *p0, *p1;
      rows(row(r), ok, p0, p1);
      const int c = chunk16(r);
      const bool use = ok && c >= 0;
      const void* s0 = use ? (const void*)((const char*)p0 + c) : (const void*)kZeroChunk;
      const void* s1 = use ? (const void*)((const char*)p1 + c) : (const void*)kZeroChunk;
      __builtin_amdgcn_global_load_lds(s0, dst(t0, r), 16, 0, 0);
      __builtin_amdgcn_global_load_lds(s1, dst(t1, r), 16, 0, 0);
    }
    lgkm_settle();
  }
};

// Workgroup barriers for data exchanged through LDS. Every wave waits for
// its own LDS operations and for its vector memory operations except the
// VM most recent ones (direct-to-LDS loads count as vector memory
// operations, and they complete in issue order), then the waves meet. The
// empty asm statements keep the compiler from moving memory accesses across
// the barrier; no global memory ordering is implied (the kernels exchange
// data through LDS only). s_waitcnt immediate: vmcnt [3:0] (high bits
// [15:14] zero), expcnt [6:4] = 7 (no wait), lgkmcnt [11:8] = 0.
template <int VM = 0>
__device__ __forceinline__ void lds_sync() {
  static_assert(VM >= 0 && VM <= 15, "vmcnt immediate");
  __asm__ volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0x0070 | VM);
  __builtin_amdgcn_s_barrier();
  __asm__ volatile("" ::: "memory");
}

// The tile loop's barrier: this wave's loads (the tile about to be read)
// have landed, and every wave is past its reads of the other buffer.
__device__ __forceinline__ void dma_barrier() { lds_sync<0>(); }

// Barrier for an LDS hand-over inside a tile step: global loads in flight
// (the next tile) keep flying (vmcnt left at its maximum, 63).
__device__ __forceinline__ void lds_barrier() {
  __asm__ volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);
  __builtin_amdgcn_s_barrier();
  __asm__ volatile("" ::: "memory");
}

}  // namespace wmx

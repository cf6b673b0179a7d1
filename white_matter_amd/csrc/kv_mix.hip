// KV-pool producer for gfx950: the token-local steps ahead of the per-channel
// projection (reference modules/kv_pool.py:97-160 `_project`,
// modules/routing.py:77-124 `Router`, `_RoutedMixer`).
//
//   premix: every source row of a token is RMS-normalised and scaled by the
//           K-side and the V-side pre-mix weights, rounded to bf16: the
//           router's input and the mixture's operand (one wave per row, both
//           sides from one read of the row);
//   mix:    per token, side and channel the routed sum over the sources,
//           rounded to bf16, RMS-normalised with the mix eps, scaled by the
//           channel gain and rounded to bf16, written in the projection's
//           input layout (channel, token, hidden) (one workgroup per token,
//           side and group of 8 channels; the token's premixed rows are read
//           once for all the group's channels);
//   router: between the two, the router logits of both sides, a split-K
//           MFMA GEMM over the premixed rows read in place: the whole row,
//           or the router's strided view of it (every source_stride-th
//           source block from source_start, routing.py:66-72) without a
//           gathered copy, then a reduce kernel that adds the chunks' fp32
//           partials in order with the bias and rounds once to bf16.
//
// premix and mix are HBM-bound: per token the sources are read once, the
// premixed rows written once and read twice (the router and the mixture),
// the channels written once. The eager sequence materialises the normalised sources, both
// premixed stacks, the mixtures, their normalisation and the gained copies.
#include "wmx_kernels.h"

namespace wmx {

namespace {

// Four consecutive elements as fp32 from an fp32 or bf16 array.
__device__ __forceinline__ void load4(const void* base, int64_t off, bool bf16_src, float (&v)[4]) {
  if (bf16_src) {
    const u32x2 w = *reinterpret_cast<const u32x2*>((const bf16*)base + off);
    v[0] = bf16_lo(w[0]);
    v[1] = bf16_hi(w[0]);
    v[2] = bf16_lo(w[1]);
    v[3] = bf16_hi(w[1]);
  } else {
    const f32x4 x = *reinterpret_cast<const f32x4*>((const float*)base + off);
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = x[e];
  }
}

// Eight fp32 values to eight bf16 at base + off (a plain store: the rows are
// read again soon).
__device__ __forceinline__ void store8_bf16_cached(void* base, int64_t off, const float (&v)[8]) {
  const u32x4 w = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]),
                   pack_bf16x2(v[6], v[7])};
  *reinterpret_cast<u32x4*>((bf16*)base + off) = w;
}

constexpr int kMixChannels = 8;  // channels per mix workgroup
constexpr int kMixBatch = 2;     // source rows whose loads are in flight together (few registers: more resident waves)

}  // namespace

// One wave per (token, source) row; lane l holds elements 512 c + 8 l + [0, 8)
// for c < CH (hidden <= 512 CH). Arithmetic in fp32 whatever the source
// dtype (the pool's fp32 residual policy): y = x * (1 / sqrt(mean(x^2) + eps)),
// p_side = bf16(y * w_side[s]).
template <int CH, bool SRC_BF16, bool W_BF16>
__global__ __launch_bounds__(256) void kv_premix_kernel(const wmx_kv_mix_args a, int64_t rows) {
#pragma clang fp contract(off)
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;  // wave-uniform
  const int lane = threadIdx.x & 63;
  const int s = (int)(r % a.num_sources);
  const int64_t n = r / a.num_sources;
  const int t = (int)(n % a.tokens), b = (int)(n / a.tokens);
  const int64_t src = (int64_t)b * a.source_stride[0] + (int64_t)t * a.source_stride[1] + (int64_t)s * a.source_stride[2];
  float x[CH][8];
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int d0 = 512 * c + 8 * lane;
    if (d0 < a.hidden) {
      load8(a.sources, src + d0, SRC_BF16, x[c]);
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = fmaf(x[c][e], x[c][e], ss);
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
  const float inv = 1.f / sqrtf(ss / (float)a.hidden + a.eps);
  const int64_t out = (n * a.num_sources + s) * a.hidden;
#pragma unroll
  for (int side = 0; side < 2; ++side) {
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int d0 = 512 * c + 8 * lane;
      if (d0 < a.hidden) {
        float w[8], y[8];
        load8(a.pre_mix[side], (int64_t)s * a.hidden + d0, W_BF16, w);
#pragma unroll
        for (int e = 0; e < 8; ++e) y[e] = (x[c][e] * inv) * w[e];
        store8_bf16_cached(a.premixed[side], out + d0, y);
      }
    }
  }
}

// Workgroup (token n, side, channel group) of NT threads; thread i holds
// elements 8 NT c + 8 i + [0, 8) for c < CH (hidden <= 8 NT CH), read and
// written as 16-byte vectors. For each channel j of the group:
// m = bf16(sum over s ascending of alpha[n, j, s] * p[n, s, :]) (fp32 products
// and sums), then out = bf16((m * (1 / sqrt(mean(m^2) + mix_eps))) * gain[j]).
template <int CH, bool W_BF16, int NT>
__global__ __launch_bounds__(NT) void kv_mix_kernel(const wmx_kv_mix_args a) {
#pragma clang fp contract(off)
  constexpr int NWV = NT / 64, CW = 8 * NT;
  __shared__ float alpha_lds[kMixChannels * WMX_KV_MIX_MAX_SOURCES];
  __shared__ float red[NWV][kMixChannels];
  const int64_t n = blockIdx.x;
  const int side = blockIdx.y;
  const int c0 = blockIdx.z * kMixChannels;
  const int nc = min(kMixChannels, a.channels - c0);
  const int S = a.num_sources, H = a.hidden;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  // this group's logits: channels c0 .. c0 + nc - 1 are contiguous rows of S
  const bf16* alpha = (const bf16*)a.alpha[side] + n * a.alpha_stride + (int64_t)c0 * S;
  for (int i = tid; i < nc * S; i += NT) alpha_lds[i] = (float)alpha[i];
  __syncthreads();

  float acc[kMixChannels][CH][8];
#pragma unroll
  for (int j = 0; j < kMixChannels; ++j)
#pragma unroll
    for (int c = 0; c < CH; ++c)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[j][c][e] = 0.f;
  const bf16* p = (const bf16*)a.premixed[side] + n * S * H;
  for (int s0 = 0; s0 < S; s0 += kMixBatch) {
    float pv[kMixBatch][CH][8];
#pragma unroll
    for (int u = 0; u < kMixBatch; ++u) {
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        const int d0 = CW * c + 8 * tid;
        if (s0 + u < S && d0 < H) {
          load8(p, (int64_t)(s0 + u) * H + d0, true, pv[u][c]);
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) pv[u][c][e] = 0.f;
        }
      }
    }
#pragma unroll
    for (int u = 0; u < kMixBatch; ++u) {
      if (s0 + u < S) {
#pragma unroll
        for (int j = 0; j < kMixChannels; ++j) {
          if (j < nc) {
            const float al = alpha_lds[j * S + s0 + u];
#pragma unroll
            for (int c = 0; c < CH; ++c)
#pragma unroll
              for (int e = 0; e < 8; ++e) acc[j][c][e] = fmaf(al, pv[u][c][e], acc[j][c][e]);
          }
        }
      }
    }
  }

  float ss[kMixChannels];
#pragma unroll
  for (int j = 0; j < kMixChannels; ++j) {
    ss[j] = 0.f;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const bool in = CW * c + 8 * tid < H;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float m = in ? round_bf16(acc[j][c][e]) : 0.f;
        acc[j][c][e] = m;
        ss[j] = fmaf(m, m, ss[j]);
      }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) ss[j] += __shfl_xor(ss[j], o);
    if (lane == 0) red[w][j] = ss[j];
  }
  __syncthreads();
  const int64_t tokens_total = (int64_t)a.batch * a.tokens;
#pragma unroll
  for (int j = 0; j < kMixChannels; ++j) {
    if (j >= nc) break;
    float total = 0.f;
#pragma unroll
    for (int v = 0; v < NWV; ++v) total += red[v][j];
    const float inv = 1.f / sqrtf(total / (float)H + a.mix_eps);
    const int64_t row = ((int64_t)(c0 + j) * tokens_total + n) * H;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int d0 = CW * c + 8 * tid;
      if (d0 < H) {
        float g[8], o[8];
        load8(a.gain[side], (int64_t)(c0 + j) * H + d0, W_BF16, g);
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = (acc[j][c][e] * inv) * g[e];
        store8_bf16(a.mixed[side], row + d0, o);
      }
    }
  }
}

// Router GEMM, one workgroup per (128-row tile, 1024-input chunk, side): four
// waves of 32 rows each, every logit of the tile in NB blocks of 32 columns.
// The weight rows of the chunk stream through LDS in stages of 64 inputs
// (double-buffered, 16-byte chunks swizzled by row so a wave's 32 rows read
// distinct banks); each lane reads its row's 8 inputs per product straight
// from HBM, one stage ahead. Partial sums, fp32, go to
// part[side][chunk][row][logit].
constexpr int kRouterRows = 128;
constexpr int kRouterStage = 64;

template <int NB>
__global__ __launch_bounds__(256, 2) void kv_router_kernel(const wmx_kv_router_args a, int chunks) {
  __shared__ __attribute__((aligned(16))) u32x4 w_lds[2][NB * 32][kRouterStage / 8];
  const int side = blockIdx.z, chunk = blockIdx.y;
  const int m0 = blockIdx.x * kRouterRows;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, col = lane & 31, half = lane >> 5;
  const int k0 = chunk * kRouterChunk, k1 = min(k0 + kRouterChunk, a.inputs);
  const int stages = (k1 - k0) / kRouterStage;
  const int row = m0 + wave * 32 + col;
  const bool row_ok = row < a.rows;
  // a row's inputs: its first `inputs` elements, or the blocks of the
  // selected sources (a stage never straddles two: widths are multiples of
  // kRouterStage)
  const int64_t row_stride = a.source_width ? a.row_stride : a.inputs;
  const bf16* arow = (const bf16*)a.premixed[side] + (int64_t)(row_ok ? row : 0) * row_stride + 8 * half;
  auto input_at = [&](int k) __attribute__((always_inline)) -> int64_t {
    if (!a.source_width) return k;
    const int block = k / a.source_width;
    return (int64_t)(a.source_start + block * a.source_stride) * a.source_width + (k - block * a.source_width);
  };
  const bf16* wgt = (const bf16*)a.weight[side];
  const u32x4 z = {0u, 0u, 0u, 0u};
  // this thread's weight chunks of a stage: chunk c = i * 256 + tid of the
  // stage's NB * 32 rows x 8 chunks
  auto load_w = [&](int k, u32x4 (&r)[NB]) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int c = i * 256 + tid, n = c >> 3;
      r[i] = n < a.logits ? load16(wgt + (int64_t)n * a.inputs + k + 8 * (c & 7)) : z;
    }
  };
  auto store_w = [&](int buf, const u32x4 (&r)[NB]) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int c = i * 256 + tid, n = c >> 3;
      w_lds[buf][n][(c & 7) ^ (n & 7)] = r[i];
    }
  };
  auto load_a = [&](int k, bf16x8 (&r)[kRouterStage / 16]) __attribute__((always_inline)) {
    const bf16* p = arow + input_at(k);
#pragma unroll
    for (int s = 0; s < kRouterStage / 16; ++s) r[s] = as_bf16x8(row_ok ? load16(p + 16 * s) : z);
  };

  f32x16 acc[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) acc[nb] = f32x16{};
  u32x4 wr[NB];
  bf16x8 aop[kRouterStage / 16], anext[kRouterStage / 16];
  load_w(k0, wr);
  load_a(k0, aop);
  store_w(0, wr);
  __syncthreads();
  for (int t = 0; t < stages; ++t) {
    const int buf = t & 1;
    const bool more = t + 1 < stages;
    if (more) {
      load_w(k0 + (t + 1) * kRouterStage, wr);
      load_a(k0 + (t + 1) * kRouterStage, anext);
    }
#pragma unroll
    for (int s = 0; s < kRouterStage / 16; ++s) {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const int n = nb * 32 + col;
        const bf16x8 wop = as_bf16x8(w_lds[buf][n][(2 * s + half) ^ (n & 7)]);
        acc[nb] = mfma32(aop[s], wop, acc[nb]);
      }
    }
    if (more) {
      store_w(buf ^ 1, wr);
#pragma unroll
      for (int s = 0; s < kRouterStage / 16; ++s) aop[s] = anext[s];
    }
    __syncthreads();
  }
  // element r of block nb: row m0 + 32 wave + 8 (r / 4) + 4 half + r % 4,
  // logit 32 nb + col
  float* part = (float*)a.workspace + ((int64_t)side * chunks + chunk) * a.rows * (int64_t)a.logits;
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int n = nb * 32 + col;
    if (n >= a.logits) continue;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int m = m0 + wave * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
      if (m < a.rows) part[(int64_t)m * a.logits + n] = acc[nb][r];
    }
  }
}

// alpha[side][m, n] = bf16(sum over chunks ascending of part + bias[n])
__global__ __launch_bounds__(256) void kv_router_reduce_kernel(const wmx_kv_router_args a, int chunks) {
  const int64_t per = (int64_t)a.rows * a.logits;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int side = blockIdx.y;
  if (i >= per) return;
  const float* part = (const float*)a.workspace + (int64_t)side * chunks * per + i;
  float sum = 0.f;
  // loads issued eight at a time, added in chunk order
#pragma unroll 8
  for (int c = 0; c < chunks; ++c) sum += part[(int64_t)c * per];
  const int n = (int)(i % a.logits);
  if (a.bias[side]) sum += (float)((const bf16*)a.bias[side])[n];
  ((bf16*)a.alpha[side])[i] = (bf16)sum;
}

int launch_kv_router(const wmx_kv_router_args& a, hipStream_t stream) {
  if (a.rows == 0) return WMX_OK;
  const int64_t chunks = kv_router_chunks(a);
  const int64_t tiles = (a.rows + kRouterRows - 1) / kRouterRows;
  const int64_t per = (int64_t)a.rows * a.logits;
  if (tiles > UINT32_MAX || chunks > 65535 || (per + 255) / 256 > UINT32_MAX) return WMX_E_UNSUPPORTED;
  const dim3 grid((unsigned)tiles, (unsigned)chunks, 2);
  const int nb = (a.logits + 31) / 32;
  switch (nb) {
    case 1: hipLaunchKernelGGL((kv_router_kernel<1>), grid, dim3(256), 0, stream, a, (int)chunks); break;
    case 2: hipLaunchKernelGGL((kv_router_kernel<2>), grid, dim3(256), 0, stream, a, (int)chunks); break;
    case 3: hipLaunchKernelGGL((kv_router_kernel<3>), grid, dim3(256), 0, stream, a, (int)chunks); break;
    case 4: hipLaunchKernelGGL((kv_router_kernel<4>), grid, dim3(256), 0, stream, a, (int)chunks); break;
    case 5: hipLaunchKernelGGL((kv_router_kernel<5>), grid, dim3(256), 0, stream, a, (int)chunks); break;
    case 6: hipLaunchKernelGGL((kv_router_kernel<6>), grid, dim3(256), 0, stream, a, (int)chunks); break;
    case 7: hipLaunchKernelGGL((kv_router_kernel<7>), grid, dim3(256), 0, stream, a, (int)chunks); break;
    case 8: hipLaunchKernelGGL((kv_router_kernel<8>), grid, dim3(256), 0, stream, a, (int)chunks); break;
    default: return WMX_E_UNSUPPORTED;
  }
  hipLaunchKernelGGL(kv_router_reduce_kernel, dim3((unsigned)((per + 255) / 256), 2), dim3(256), 0, stream, a,
                     (int)chunks);
  return WMX_OK;
}

template <int CH>
static void launch_premix_ch(const wmx_kv_mix_args& a, int64_t rows, hipStream_t stream) {
  const dim3 grid((unsigned)((rows + 3) / 4));
  const bool sb = a.source_dtype == WMX_DTYPE_BF16, wb = a.weight_dtype == WMX_DTYPE_BF16;
  if (sb && wb) hipLaunchKernelGGL((kv_premix_kernel<CH, true, true>), grid, dim3(256), 0, stream, a, rows);
  else if (sb) hipLaunchKernelGGL((kv_premix_kernel<CH, true, false>), grid, dim3(256), 0, stream, a, rows);
  else if (wb) hipLaunchKernelGGL((kv_premix_kernel<CH, false, true>), grid, dim3(256), 0, stream, a, rows);
  else hipLaunchKernelGGL((kv_premix_kernel<CH, false, false>), grid, dim3(256), 0, stream, a, rows);
}

int launch_kv_premix(const wmx_kv_mix_args& a, hipStream_t stream) {
  const int64_t rows = (int64_t)a.batch * a.tokens * a.num_sources;
  if (rows == 0) return WMX_OK;
  if ((rows + 3) / 4 > UINT32_MAX) return WMX_E_UNSUPPORTED;
  if (a.hidden <= 512) launch_premix_ch<1>(a, rows, stream);
  else if (a.hidden <= 1024) launch_premix_ch<2>(a, rows, stream);
  else if (a.hidden <= 2048) launch_premix_ch<4>(a, rows, stream);
  else launch_premix_ch<8>(a, rows, stream);
  return WMX_OK;
}

template <int CH, int NT>
static void launch_mix_ch(const wmx_kv_mix_args& a, dim3 grid, hipStream_t stream) {
  if (a.weight_dtype == WMX_DTYPE_BF16) hipLaunchKernelGGL((kv_mix_kernel<CH, true, NT>), grid, dim3(NT), 0, stream, a);
  else hipLaunchKernelGGL((kv_mix_kernel<CH, false, NT>), grid, dim3(NT), 0, stream, a);
}

int launch_kv_mix(const wmx_kv_mix_args& a, hipStream_t stream) {
  const int64_t tokens = (int64_t)a.batch * a.tokens;
  if (tokens == 0) return WMX_OK;
  if (tokens > UINT32_MAX) return WMX_E_UNSUPPORTED;
  const dim3 grid((unsigned)tokens, 2, (unsigned)((a.channels + kMixChannels - 1) / kMixChannels));
  if (a.hidden <= 1024) launch_mix_ch<1, 128>(a, grid, stream);
  else if (a.hidden <= 2048) launch_mix_ch<1, 256>(a, grid, stream);
  else launch_mix_ch<2, 256>(a, grid, stream);
  return WMX_OK;
}

}  // namespace wmx

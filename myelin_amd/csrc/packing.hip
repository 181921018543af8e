// Spike bitpacking for gfx950: 32 spikes per int32 word along the last
// dimension, bit i of word w = element 32*w + i (LSB first), padding bits 0.
//
// pack:   one lane per element; a wave ballot turns 64 consecutive elements
//         into two words.  Each wave handles 64 words (32 ballots) per pass
//         and lane j stores word j, so the word store is one coalesced
//         256-byte write and every element load is a coalesced wave load.
// unpack: one lane per 4 elements (same word), vector store of 4 outputs.
// counts: popcount with the padding bits of the last word masked.

#include "common.h"

namespace {

using myelin::kWave;

// ---- element predicates: "nonzero" exactly as ATen's (x != 0) ----------
struct F32 {
  using T = float;
  __device__ static bool nz(float v) { return v != 0.0f; }
};
struct F64 {
  using T = double;
  __device__ static bool nz(double v) { return v != 0.0; }
};
struct H16 {  // fp16 and bf16: zero iff all bits but the sign are zero
  using T = uint16_t;
  __device__ static bool nz(uint16_t v) { return (v & 0x7fffu) != 0; }
};
struct U8 {
  using T = uint8_t;
  __device__ static bool nz(uint8_t v) { return v != 0; }
};
struct I32 {
  using T = int32_t;
  __device__ static bool nz(int32_t v) { return v != 0; }
};
struct I64 {
  using T = int64_t;
  __device__ static bool nz(int64_t v) { return v != 0; }
};

// words: [rows, W]; total = rows * W.  ALIGNED: n % 32 == 0 so the element
// of (word g, bit i) is simply 32*g + i.
template <class E, bool ALIGNED>
__global__ __launch_bounds__(256) void pack_kernel(const typename E::T *__restrict__ src, int32_t *__restrict__ words,
                                                   int64_t total, int64_t W, int64_t n) {
  const int lane = static_cast<int>(threadIdx.x & (kWave - 1));
  const int64_t wave = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) >> 6;
  const int64_t g0 = wave * 64;  // first word of this wave
  if (g0 >= total) return;       // wave-uniform
  const int half = lane >> 5, bit = lane & 31;

  typename E::T v[32];
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    const int64_t g = g0 + 2 * i + half;
    v[i] = typename E::T(0);
    if (g < total) {
      if constexpr (ALIGNED) {
        v[i] = __builtin_nontemporal_load(src + g * 32 + bit);
      } else {
        const int64_t r = g / W;
        const int64_t col = (g - r * W) * 32 + bit;
        if (col < n) v[i] = src[r * n + col];
      }
    }
  }
  uint32_t mine = 0;
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    const uint64_t b = __ballot(E::nz(v[i]));
    const uint32_t lo = static_cast<uint32_t>(b), hi = static_cast<uint32_t>(b >> 32);
    mine = (lane == 2 * i) ? lo : mine;
    mine = (lane == 2 * i + 1) ? hi : mine;
  }
  if (g0 + lane < total) words[g0 + lane] = static_cast<int32_t>(mine);
}

// ALIGNED (n % 32 == 0): lane handles 4 consecutive elements of one word.
template <typename S>
__global__ __launch_bounds__(256) void unpack_aligned(const int32_t *__restrict__ words, S *__restrict__ dst,
                                                      int64_t quads, S one) {
  const int64_t q = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (q >= quads) return;
  const int64_t e = q * 4;
  const uint32_t w = static_cast<uint32_t>(words[e >> 5]);
  const uint32_t nib = (w >> (e & 31)) & 0xfu;
  S out[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) out[i] = ((nib >> i) & 1u) ? one : S(0);
  if constexpr (sizeof(S) == 4) {
    typedef uint32_t u4 __attribute__((ext_vector_type(4)));
    u4 t = {out[0], out[1], out[2], out[3]};
    __builtin_nontemporal_store(t, reinterpret_cast<u4 *>(dst + e));
  } else if constexpr (sizeof(S) == 2) {
    typedef uint16_t h4 __attribute__((ext_vector_type(4)));
    h4 t = {out[0], out[1], out[2], out[3]};
    __builtin_nontemporal_store(t, reinterpret_cast<h4 *>(dst + e));
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) dst[e + i] = out[i];
  }
}

template <typename S>
__global__ __launch_bounds__(256) void unpack_generic(const int32_t *__restrict__ words, S *__restrict__ dst,
                                                      int64_t total, int64_t n, int64_t W, S one) {
  const int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (e >= total) return;
  const int64_t r = e / n;
  const int64_t col = e - r * n;
  const uint32_t w = static_cast<uint32_t>(words[r * W + (col >> 5)]);
  dst[e] = ((w >> (col & 31)) & 1u) ? one : S(0);
}

// ---- counts --------------------------------------------------------------
inline int64_t cdiv64(int64_t a, int64_t b) { return (a + b - 1) / b; }

struct LeadInfo {
  int ndim;
  int64_t shape[8];
  int64_t out_stride[8];  // 0 for reduced dims
};

__device__ __forceinline__ int64_t out_index(int64_t row, const LeadInfo &li) {
  int64_t idx = 0;
  for (int d = li.ndim - 1; d >= 0; --d) {
    const int64_t s = li.shape[d];
    const int64_t q = row / s;
    idx += (row - q * s) * li.out_stride[d];
    row = q;
  }
  return idx;
}

__device__ __forceinline__ int64_t wave_sum(int64_t v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

// One wave per row.  DIRECT: out[row] = count (every leading dim kept);
// otherwise atomically accumulate into the kept-dims index (out zeroed).
template <bool DIRECT>
__global__ __launch_bounds__(256) void row_counts_wave(const int32_t *__restrict__ words, int64_t rows, int64_t W,
                                                       uint32_t last_mask, LeadInfo li, int64_t *__restrict__ out) {
  const int lane = static_cast<int>(threadIdx.x & (kWave - 1));
  const int64_t row = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) >> 6;
  if (row >= rows) return;
  const int32_t *rw = words + row * W;
  int64_t c = 0;
  for (int64_t j = lane; j < W; j += kWave) {
    uint32_t w = static_cast<uint32_t>(rw[j]);
    if (j == W - 1) w &= last_mask;
    c += __popc(w);
  }
  c = wave_sum(c);
  if (lane == 0) {
    if constexpr (DIRECT) {
      out[row] = c;
    } else {
      atomicAdd(reinterpret_cast<unsigned long long *>(out + out_index(row, li)), static_cast<unsigned long long>(c));
    }
  }
}

// One lane per row, for short rows (W < 16).
template <bool DIRECT>
__global__ __launch_bounds__(256) void row_counts_lane(const int32_t *__restrict__ words, int64_t rows, int64_t W,
                                                       uint32_t last_mask, LeadInfo li, int64_t *__restrict__ out) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (row >= rows) return;
  const int32_t *rw = words + row * W;
  int64_t c = 0;
  for (int64_t j = 0; j < W; ++j) {
    uint32_t w = static_cast<uint32_t>(rw[j]);
    if (j == W - 1) w &= last_mask;
    c += __popc(w);
  }
  if constexpr (DIRECT) {
    out[row] = c;
  } else {
    atomicAdd(reinterpret_cast<unsigned long long *>(out + out_index(row, li)), static_cast<unsigned long long>(c));
  }
}

// Counts whose kept leading dims form one contiguous block: output o sums
// the rows (a*P + o)*Q + i, a < A, i < Q (k = a*Q + i runs over AQ = A*Q).
// Blocks (o, s) of 16 waves split output o's AQ rows into S slices; wave q
// of a block takes k = q, q + 16, ... of its slice, four rows per pass, and
// wave 0 adds the 16 wave sums.  S == 1 stores the count; S > 1 adds the S
// slice counts atomically (out zeroed; a handful of atomics per output, and
// integer sums are order-independent).
constexpr int kBlkWaves = 16;

__global__ __launch_bounds__(1024) void row_counts_block(const int32_t *__restrict__ words, int64_t W,
                                                         uint32_t last_mask, int64_t P, int64_t Q, int64_t AQ,
                                                         int64_t slice, int atomic, int64_t *__restrict__ out) {
  __shared__ int64_t part[kBlkWaves];
  const int lane = static_cast<int>(threadIdx.x & 63), q = static_cast<int>(threadIdx.x >> 6);
  const int64_t o = blockIdx.x;
  const int64_t k_begin = static_cast<int64_t>(blockIdx.y) * slice;
  const int64_t k_end = (k_begin + slice < AQ) ? k_begin + slice : AQ;
  int64_t c = 0;
  for (int64_t k = k_begin + q; k < k_end; k += 4 * kBlkWaves) {
    const int32_t *rw[4];
    bool ok[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t kk = k + u * kBlkWaves;
      ok[u] = kk < k_end;
      const int64_t a = kk / Q, i = kk - a * Q;
      rw[u] = ok[u] ? words + ((a * P + o) * Q + i) * W : words;
    }
    for (int64_t j = lane; j < W; j += kWave) {
      const uint32_t m = (j == W - 1) ? last_mask : 0xffffffffu;
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (ok[u]) c += __popc(static_cast<uint32_t>(rw[u][j]) & m);
    }
  }
  c = wave_sum(c);
  if (lane == 0) part[q] = c;
  __syncthreads();
  if (threadIdx.x == 0) {
    int64_t t = 0;
#pragma unroll
    for (int i = 0; i < kBlkWaves; ++i) t += part[i];
    if (atomic)
      atomicAdd(reinterpret_cast<unsigned long long *>(out + o), static_cast<unsigned long long>(t));
    else
      out[o] = t;
  }
}

__global__ __launch_bounds__(256) void fill_i64(int64_t *__restrict__ p, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0;
}

// Per-neuron counts over R leading rows: words [R, K, W] -> out [K, n].
// Block = 8 waves x 64 word-columns; wave q walks rows r = q, q+8, ...
// inside the block's row range, 16 rows' loads issued before any is used.
// Bit counts are accumulated SWAR-style: acc[j] holds, in its 4 bytes, the
// counts of bits j, j+8, j+16, j+24.  A block spans at most 8 * 255 rows,
// so no byte passes 255 before the wave's counts are unpacked.  The 8
// waves are then reduced through LDS; a block covering all R rows stores,
// otherwise it atomically adds (out zeroed).
constexpr int kKeepWaves = 8;
constexpr int kKeepRows = kKeepWaves * 255;  // rows per block
constexpr int kKeepAhead = 16;               // row loads in flight per lane

__global__ __launch_bounds__(512) void keep_last_counts(const int32_t *__restrict__ words, int64_t R, int64_t KW,
                                                        int64_t W, int64_t n, int64_t *__restrict__ out,
                                                        int atomic) {
  __shared__ int32_t red[kKeepWaves - 1][32][64];
  const int lane = static_cast<int>(threadIdx.x & 63);
  const int q = static_cast<int>(threadIdx.x >> 6);
  const int64_t col = static_cast<int64_t>(blockIdx.x) * 64 + lane;  // (k, w) flattened
  const bool active = col < KW;
  const int64_t r_begin = static_cast<int64_t>(blockIdx.y) * kKeepRows;
  const int64_t r_end = (r_begin + kKeepRows < R) ? r_begin + kKeepRows : R;

  int32_t cnt[32];
  uint32_t acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = 0;
  if (active) {
    const int32_t *p = words + col;
    int64_t r = r_begin + q;
    for (; r + (kKeepAhead - 1) * kKeepWaves < r_end; r += kKeepAhead * kKeepWaves) {
      uint32_t w[kKeepAhead];
#pragma unroll
      for (int u = 0; u < kKeepAhead; ++u) w[u] = static_cast<uint32_t>(p[(r + u * kKeepWaves) * KW]);
#pragma unroll
      for (int u = 0; u < kKeepAhead; ++u)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] += (w[u] >> j) & 0x01010101u;
    }
    for (; r < r_end; r += kKeepWaves) {
      const uint32_t w = static_cast<uint32_t>(p[r * KW]);
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] += (w >> j) & 0x01010101u;
    }
  }
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int y = 0; y < 4; ++y) cnt[8 * y + j] = static_cast<int32_t>((acc[j] >> (8 * y)) & 0xffu);
  if (q > 0) {
#pragma unroll
    for (int b = 0; b < 32; ++b) red[q - 1][b][lane] = cnt[b];
  }
  __syncthreads();
  if (q == 0 && active) {
    for (int o = 0; o < kKeepWaves - 1; ++o)
#pragma unroll
      for (int b = 0; b < 32; ++b) cnt[b] += red[o][b][lane];
    const int64_t k = col / W;
    const int64_t w = col - k * W;
#pragma unroll
    for (int b = 0; b < 32; ++b) {
      const int64_t j = w * 32 + b;
      if (j < n) {
        int64_t *dst = out + k * n + j;
        if (atomic)
          atomicAdd(reinterpret_cast<unsigned long long *>(dst), static_cast<unsigned long long>(cnt[b]));
        else
          *dst = cnt[b];
      }
    }
  }
}

template <typename OUT>
__global__ __launch_bounds__(256) void rate_kernel(const int64_t *__restrict__ c, OUT *__restrict__ out, int64_t numel,
                                                   OUT denom) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < numel) out[i] = static_cast<OUT>(c[i]) / denom;
}

int64_t blocks(int64_t threads, int per = 256) { return (threads + per - 1) / per; }

template <class E>
int pack_typed(const void *src, int32_t *words, int64_t rows, int64_t n, hipStream_t s) {
  const int64_t W = (n + 31) / 32;
  const int64_t total = rows * W;
  const int64_t waves = (total + 63) / 64;
  const dim3 grid(blocks(waves * 64));
  const auto *p = static_cast<const typename E::T *>(src);
  if (n % 32 == 0)
    pack_kernel<E, true><<<grid, dim3(256), 0, s>>>(p, words, total, W, n);
  else
    pack_kernel<E, false><<<grid, dim3(256), 0, s>>>(p, words, total, W, n);
  return myelin::launched("pack");
}

template <typename S>
int unpack_typed(const int32_t *words, void *dst, int64_t rows, int64_t n, S one, hipStream_t s) {
  const int64_t W = (n + 31) / 32;
  S *d = static_cast<S *>(dst);
  if (n % 32 == 0 && myelin::aligned(dst, 4 * sizeof(S))) {
    const int64_t quads = rows * n / 4;
    unpack_aligned<S><<<dim3(blocks(quads)), dim3(256), 0, s>>>(words, d, quads, one);
  } else {
    const int64_t total = rows * n;
    unpack_generic<S><<<dim3(blocks(total)), dim3(256), 0, s>>>(words, d, total, n, W, one);
  }
  return myelin::launched("unpack");
}

}  // namespace

extern "C" int myelin_pack(const void *src, int dtype, int32_t *words, int64_t rows, int64_t n,
                           myelin_stream_t stream) {
  if (rows < 0 || n < 1) return myelin::invalid("pack: rows must be >= 0 and n >= 1");
  if (rows == 0) return MYELIN_OK;
  if (src == nullptr || words == nullptr) return myelin::invalid("pack: null pointer");
  hipStream_t s = myelin::as_hip(stream);
  switch (dtype) {
    case MYELIN_DT_F32: return pack_typed<F32>(src, words, rows, n, s);
    case MYELIN_DT_F64: return pack_typed<F64>(src, words, rows, n, s);
    case MYELIN_DT_F16:
    case MYELIN_DT_BF16: return pack_typed<H16>(src, words, rows, n, s);
    case MYELIN_DT_U8: return pack_typed<U8>(src, words, rows, n, s);
    case MYELIN_DT_I32: return pack_typed<I32>(src, words, rows, n, s);
    case MYELIN_DT_I64: return pack_typed<I64>(src, words, rows, n, s);
    default: return myelin::invalid("pack: unsupported dtype code %d", dtype);
  }
}

extern "C" int myelin_unpack(const int32_t *words, void *dst, int dtype, int64_t rows, int64_t n,
                             myelin_stream_t stream) {
  if (rows < 0 || n < 1) return myelin::invalid("unpack: rows must be >= 0 and n >= 1");
  if (rows == 0) return MYELIN_OK;
  if (words == nullptr || dst == nullptr) return myelin::invalid("unpack: null pointer");
  hipStream_t s = myelin::as_hip(stream);
  switch (dtype) {
    case MYELIN_DT_F32: return unpack_typed<uint32_t>(words, dst, rows, n, 0x3f800000u, s);
    case MYELIN_DT_F64: return unpack_typed<uint64_t>(words, dst, rows, n, 0x3ff0000000000000ull, s);
    case MYELIN_DT_F16: return unpack_typed<uint16_t>(words, dst, rows, n, uint16_t(0x3c00), s);
    case MYELIN_DT_BF16: return unpack_typed<uint16_t>(words, dst, rows, n, uint16_t(0x3f80), s);
    case MYELIN_DT_U8: return unpack_typed<uint8_t>(words, dst, rows, n, uint8_t(1), s);
    case MYELIN_DT_I32: return unpack_typed<uint32_t>(words, dst, rows, n, 1u, s);
    case MYELIN_DT_I64: return unpack_typed<uint64_t>(words, dst, rows, n, 1ull, s);
    default: return myelin::invalid("unpack: unsupported dtype code %d", dtype);
  }
}

extern "C" int myelin_packed_counts(const int32_t *words, int ndim_lead, const int64_t *lead_shape,
                                    uint32_t reduce_mask, int64_t n, int64_t *out, myelin_stream_t stream) {
  if (ndim_lead < 0 || ndim_lead > 8) return myelin::invalid("packed_counts: 0..8 leading dims supported");
  if (n < 1) return myelin::invalid("packed_counts: n must be >= 1");
  if (out == nullptr || (ndim_lead > 0 && lead_shape == nullptr)) return myelin::invalid("packed_counts: null pointer");
  LeadInfo li{};
  li.ndim = ndim_lead;
  int64_t rows = 1, kept = 1;
  for (int d = ndim_lead - 1; d >= 0; --d) {
    if (lead_shape[d] < 0) return myelin::invalid("packed_counts: negative dim");
    li.shape[d] = lead_shape[d];
    rows *= lead_shape[d];
    if (reduce_mask & (1u << d)) {
      li.out_stride[d] = 0;
    } else {
      li.out_stride[d] = kept;
      kept *= lead_shape[d];
    }
  }
  hipStream_t s = myelin::as_hip(stream);
  const uint32_t lead_mask = ndim_lead > 0 ? ((1u << ndim_lead) - 1u) : 0u;
  const bool direct = (reduce_mask & lead_mask) == 0;
  // kept leading dims [d0, d1] contiguous (or none kept): out = (row / Q) % P
  int d0 = -1, d1 = -1;
  for (int d = 0; d < ndim_lead; ++d)
    if (!(reduce_mask & (1u << d))) {
      if (d0 < 0) d0 = d;
      d1 = d;
    }
  bool block_ok = !direct;
  int64_t P = 1, Q = 1;
  if (block_ok) {
    for (int d = (d0 < 0 ? ndim_lead : d0); d <= d1; ++d) {
      if (reduce_mask & (1u << d)) block_ok = false;
      P *= lead_shape[d];
    }
    for (int d = (d1 < 0 ? ndim_lead : d1 + 1); d < ndim_lead; ++d) Q *= lead_shape[d];
  }
  // heavy reductions onto few outputs take the block kernel; others scatter
  const int64_t AQ = kept > 0 ? rows / kept : 0;
  block_ok = block_ok && kept <= 65535 && AQ >= 16;
  int64_t S = 1;
  if (block_ok) {
    S = cdiv64(256, kept);
    const int64_t by_rows = cdiv64(AQ, 64);
    if (S > by_rows) S = by_rows;
    if (S > 65535) S = 65535;
    if (S < 1) S = 1;
  }
  if (!direct && (!block_ok || S > 1)) {
    fill_i64<<<dim3(blocks(kept)), dim3(256), 0, s>>>(out, kept);
    if (int rc = myelin::launched("packed_counts zero")) return rc;
  }
  if (rows == 0) return MYELIN_OK;
  if (words == nullptr) return myelin::invalid("packed_counts: null words");
  const int64_t W = (n + 31) / 32;
  const int rem = static_cast<int>(n % 32);
  const uint32_t last_mask = rem ? ((1u << rem) - 1u) : 0xffffffffu;
  if (block_ok) {
    const int64_t slice = cdiv64(AQ, S);
    row_counts_block<<<dim3(static_cast<unsigned>(kept), static_cast<unsigned>(S)), dim3(1024), 0, s>>>(
        words, W, last_mask, P, Q, AQ, slice, S > 1 ? 1 : 0, out);
  } else if (W >= 16) {
    const dim3 grid(blocks(rows * 64));
    if (direct)
      row_counts_wave<true><<<grid, dim3(256), 0, s>>>(words, rows, W, last_mask, li, out);
    else
      row_counts_wave<false><<<grid, dim3(256), 0, s>>>(words, rows, W, last_mask, li, out);
  } else {
    const dim3 grid(blocks(rows));
    if (direct)
      row_counts_lane<true><<<grid, dim3(256), 0, s>>>(words, rows, W, last_mask, li, out);
    else
      row_counts_lane<false><<<grid, dim3(256), 0, s>>>(words, rows, W, last_mask, li, out);
  }
  return myelin::launched("packed_counts");
}

extern "C" int myelin_packed_counts_keep_last(const int32_t *words, int64_t R, int64_t K, int64_t n, int64_t *out,
                                              myelin_stream_t stream) {
  if (R < 0 || K < 0 || n < 1) return myelin::invalid("packed_counts_keep_last: bad sizes");
  if (out == nullptr) return myelin::invalid("packed_counts_keep_last: null out");
  hipStream_t s = myelin::as_hip(stream);
  const int64_t W = (n + 31) / 32;
  const int64_t KW = K * W;
  const int64_t out_n = K * n;
  if (out_n == 0) return MYELIN_OK;
  const int64_t row_blocks = (R + kKeepRows - 1) / kKeepRows;
  const int atomic = row_blocks > 1 ? 1 : 0;
  if (atomic || R == 0) {
    fill_i64<<<dim3(blocks(out_n)), dim3(256), 0, s>>>(out, out_n);
    if (int rc = myelin::launched("keep_last zero")) return rc;
  }
  if (R == 0) return MYELIN_OK;
  if (words == nullptr) return myelin::invalid("packed_counts_keep_last: null words");
  if (row_blocks > 65535) return myelin::invalid("packed_counts_keep_last: too many rows");
  const dim3 grid((KW + 63) / 64, row_blocks);
  keep_last_counts<<<grid, dim3(64 * kKeepWaves), 0, s>>>(words, R, KW, W, n, out, atomic);
  return myelin::launched("keep_last_counts");
}

extern "C" int myelin_counts_to_rate(const int64_t *counts, void *out, int dtype, int64_t numel, int64_t denominator,
                                     myelin_stream_t stream) {
  if (numel < 0) return myelin::invalid("counts_to_rate: negative numel");
  if (numel == 0) return MYELIN_OK;
  if (counts == nullptr || out == nullptr) return myelin::invalid("counts_to_rate: null pointer");
  hipStream_t s = myelin::as_hip(stream);
  const dim3 grid(blocks(numel));
  if (dtype == MYELIN_DT_F32) {
    rate_kernel<float><<<grid, dim3(256), 0, s>>>(counts, static_cast<float *>(out), numel,
                                                   static_cast<float>(denominator));
  } else if (dtype == MYELIN_DT_F64) {
    rate_kernel<double><<<grid, dim3(256), 0, s>>>(counts, static_cast<double *>(out), numel,
                                                    static_cast<double>(denominator));
  } else {
    return myelin::invalid("counts_to_rate: dtype must be F32 or F64");
  }
  return myelin::launched("counts_to_rate");
}

// Streamed synapse x_t @ W fused ahead of the LIF update, and the GEMMs and
// reverse recurrences of its backward, for gfx950.  In file order:
//
//  * gemm_kernel: 64 x 64 output tiles, 4 waves each owning a 32 x 32
//    quarter (v_mfma_f32_32x32x16_bf16 with fp32 accumulate, or
//    v_mfma_f32_32x32x2f32), operands staged through LDS; A may also be
//    packed spike bits.
//  * gemm_narrow / gemm_smallk: the readout shapes -- at most 32 output
//    columns (A streamed once straight into MFMA fragments) or K at most 32
//    (vector-ALU FMAs, 16-byte row stores).
//  * gemm_big: 128 x 128 tiles (each wave 2 x 2 MFMA blocks), register-
//    prefetched stages, XCD-grouped tile order; fp32 or bf16 operands.
//  * linear_lif_fwd / linear_lif_fwd_big: the current tile of a batch-row
//    block computed per time chunk, parked in LDS and consumed by the LIF
//    recurrence in registers, so currents never reach HBM.
//  * linear_pre_bwd (reverse recurrence -> G = dL/dI), col_sum (bias
//    gradient), lif_currents_fwd (the recurrence over precomputed currents),
//    bf16 operand copies, then the C ABI.
//
// MFMA operand fragments, per lane l of a wave (32 x 32 tiles):
//   A (32 x K-step): row l % 32, k = (l / 32) * KV + [0, KV)   (KV = 8 bf16 | 1 f32)
//   B (K-step x 32): col l % 32, same k
//   D (32 x 32):     col l % 32, row 8*(r/4) + 4*(l/32) + r%4 for acc register r
// Tiles stage through LDS k-contiguous ([row][k] for A, [col][k] for B), so a
// bf16 fragment is one 16-byte LDS read.

#include <type_traits>

#include "common.h"

namespace {

using myelin::kWave;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kTile = 64;  // output tile edge

template <int PREC>
struct Prec;
template <>
struct Prec<0> {  // fp32 MFMA
  using T = float;
  static constexpr int KS = 32;  // k per LDS stage
  static constexpr int KV = 1;   // k per lane per MFMA
  static constexpr int KM = 2;   // k per MFMA
  static constexpr int PAD = 4;  // rows of 36 floats: 16-byte fragment reads hit 64 distinct banks
};
template <>
struct Prec<1> {  // bf16 MFMA, fp32 accumulate
  using T = __bf16;
  static constexpr int KS = 64;
  static constexpr int KV = 8;
  static constexpr int KM = 16;
  static constexpr int PAD = 8;
};

template <int PREC>
struct Stage {
  using T = typename Prec<PREC>::T;
  static constexpr int LD = Prec<PREC>::KS + Prec<PREC>::PAD;  // padded row length (elements)
  alignas(16) T a[kTile][LD];
  alignas(16) T b[kTile][LD];
};

template <int PREC>
__device__ __forceinline__ typename Prec<PREC>::T cvt(float v) {
  if constexpr (PREC == 1)
    return static_cast<__bf16>(v);  // round to nearest even
  else
    return v;
}

typedef float f4 __attribute__((ext_vector_type(4)));

// One wave's MFMA over one LDS stage: acc += A[wm rows] x B[wn cols].
// fp32 fragments are read 16 bytes at a time: for each group of 8 k, lane l
// reads k0 + 4*(l/32) + [0, 4) and the i-th v_mfma_f32_32x32x2f32 takes
// element i (lanes < 32: k0 + i, lanes >= 32: k0 + 4 + i), so one LDS read
// feeds four MFMAs without bank conflicts.  Every fp32 tile path uses this
// k order, so all of them produce the same sums.
template <int PREC>
__device__ __forceinline__ void mfma_stage(const Stage<PREC> &st, int wm, int wn, int lane, f32x16 &acc) {
  constexpr int KS = Prec<PREC>::KS, KM = Prec<PREC>::KM, KV = Prec<PREC>::KV;
  const int r = 32 * wm + (lane & 31), c = 32 * wn + (lane & 31);
  if constexpr (PREC == 1) {
    const int kq = (lane >> 5) * KV;
#pragma unroll
    for (int kk = 0; kk < KS; kk += KM) {
      const bf16x8 av = *reinterpret_cast<const bf16x8 *>(&st.a[r][kk + kq]);
      const bf16x8 bv = *reinterpret_cast<const bf16x8 *>(&st.b[c][kk + kq]);
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, bv, acc, 0, 0, 0);
    }
  } else {
    const int kq = (lane >> 5) * 4;
#pragma unroll
    for (int kk = 0; kk < KS; kk += 8) {
      const f4 av = *reinterpret_cast<const f4 *>(&st.a[r][kk + kq]);
      const f4 bv = *reinterpret_cast<const f4 *>(&st.b[c][kk + kq]);
#pragma unroll
      for (int i = 0; i < 4; ++i) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i], bv[i], acc, 0, 0, 0);
    }
  }
}

// row index (within the wave's 32 x 32 quarter) of accumulator register r
__device__ __forceinline__ int acc_row(int r, int lane) { return 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3); }

// Stages one operand tile (64 rows x KS k) from global memory through
// registers into LDS.  Each thread owns NV float4 pieces.
//  KCONTIG: rows are k-contiguous in memory (base[e] = start of the row, or
//           null for a padding row); piece e covers k = koff[e] .. +3 of LDS
//           row roff[e].
//  otherwise: the 64 rows are contiguous along memory for a fixed k (stride
//           ld between k); piece e covers rows roff[e] .. +3 at k = koff[e];
//           nvalid[e] of those rows exist.
// VEC: 16-byte aligned pieces may be loaded as one float4.
template <int PREC, bool KCONTIG, bool VEC>
struct TileLoader {
  static constexpr int KS = Prec<PREC>::KS;
  static constexpr int NV = KS * kTile / 1024;
  const float *base[NV];
  int koff[NV], roff[NV], nvalid[NV];
  int64_t ld;
  float v[NV][4];

  // KCONTIG piece mapping for thread tid; the caller fills base[e] from row r = roff[e]
  __device__ __forceinline__ void map_kcontig(int tid) {
#pragma unroll
    for (int e = 0; e < NV; ++e) {
      const int idx = e * 256 + tid;
      roff[e] = idx / (KS / 4);
      koff[e] = 4 * (idx % (KS / 4));
      nvalid[e] = 4;
    }
  }
  // row-contiguous mapping: rows [row0, row0 + 64) of a [K x rows] array
  __device__ __forceinline__ void map_rowcontig(int tid, const float *ptr, int64_t row0, int64_t rows, int64_t ld_) {
    ld = ld_;
#pragma unroll
    for (int e = 0; e < NV; ++e) {
      const int idx = e * 256 + tid;
      koff[e] = idx / 16;
      roff[e] = 4 * (idx % 16);
      const int64_t left = rows - (row0 + roff[e]);
      nvalid[e] = left <= 0 ? 0 : (left >= 4 ? 4 : static_cast<int>(left));
      base[e] = ptr + row0 + roff[e];
    }
  }

  __device__ __forceinline__ void load(int64_t k0, int64_t kend) {
#pragma unroll
    for (int e = 0; e < NV; ++e) {
      v[e][0] = v[e][1] = v[e][2] = v[e][3] = 0.0f;
      if constexpr (KCONTIG) {
        const int64_t k = k0 + koff[e];
        if (base[e] != nullptr && k < kend) {
          const float *q = base[e] + k;
          if (VEC && k + 3 < kend) {
            const f4 t = *reinterpret_cast<const f4 *>(q);
            v[e][0] = t.x;
            v[e][1] = t.y;
            v[e][2] = t.z;
            v[e][3] = t.w;
          } else {
#pragma unroll
            for (int i = 0; i < 4; ++i)
              if (k + i < kend) v[e][i] = q[i];
          }
        }
      } else {
        const int64_t k = k0 + koff[e];
        if (k < kend && nvalid[e] > 0) {
          const float *q = base[e] + k * ld;
          if (VEC && nvalid[e] == 4) {
            const f4 t = *reinterpret_cast<const f4 *>(q);
            v[e][0] = t.x;
            v[e][1] = t.y;
            v[e][2] = t.z;
            v[e][3] = t.w;
          } else {
#pragma unroll
            for (int i = 0; i < 4; ++i)
              if (i < nvalid[e]) v[e][i] = q[i];
          }
        }
      }
    }
  }

  __device__ __forceinline__ void store(typename Prec<PREC>::T (*dst)[Stage<PREC>::LD]) const {
#pragma unroll
    for (int e = 0; e < NV; ++e) {
      if constexpr (KCONTIG && PREC == 0) {
        // fp32 rows are 16-byte aligned (36 floats) and koff a multiple of 4
        *reinterpret_cast<f4 *>(&dst[roff[e]][koff[e]]) = f4{v[e][0], v[e][1], v[e][2], v[e][3]};
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if constexpr (KCONTIG)
            dst[roff[e]][koff[e] + i] = cvt<PREC>(v[e][i]);
          else
            dst[roff[e] + i][koff[e]] = cvt<PREC>(v[e][i]);
        }
      }
    }
  }
};

// An operand held as packed spike bits (bit i of word w = column 32w + i,
// the format of myelin_pack), expanded to exact 0/1 on load; same interface
// as TileLoader.  KCONTIG: element (row, k) is bit k of the row's words.
// Otherwise (rows along mn): element (mn, k) is bit mn of row k's words
// (word k*ld + mn/32).  A piece's 4 elements never straddle a word.
template <int PREC, bool KCONTIG>
struct BitLoader {
  static constexpr int KS = Prec<PREC>::KS;
  static constexpr int NV = KS * kTile / 1024;
  const int32_t *base[NV];
  int koff[NV], roff[NV], nvalid[NV], sh[NV];
  int64_t ld;
  float v[NV][4];

  __device__ __forceinline__ void map_kcontig(int tid) {
#pragma unroll
    for (int e = 0; e < NV; ++e) {
      const int idx = e * 256 + tid;
      roff[e] = idx / (KS / 4);
      koff[e] = 4 * (idx % (KS / 4));
      nvalid[e] = 4;
      sh[e] = 0;
    }
  }
  __device__ __forceinline__ void map_rowcontig(int tid, const int32_t *ptr, int64_t row0, int64_t rows,
                                                int64_t ld_) {
    ld = ld_;
#pragma unroll
    for (int e = 0; e < NV; ++e) {
      const int idx = e * 256 + tid;
      koff[e] = idx / 16;
      roff[e] = 4 * (idx % 16);
      const int64_t left = rows - (row0 + roff[e]);
      nvalid[e] = left <= 0 ? 0 : (left >= 4 ? 4 : static_cast<int>(left));
      base[e] = ptr + (row0 + roff[e]) / 32;
      sh[e] = static_cast<int>((row0 + roff[e]) % 32);
    }
  }

  __device__ __forceinline__ void load(int64_t k0, int64_t kend) {
#pragma unroll
    for (int e = 0; e < NV; ++e) {
      uint32_t bits = 0;
      int n = 0;
      if constexpr (KCONTIG) {
        const int64_t k = k0 + koff[e];
        if (base[e] != nullptr && k < kend) {
          bits = static_cast<uint32_t>(base[e][k >> 5]) >> (k & 31);
          n = kend - k >= 4 ? 4 : static_cast<int>(kend - k);
        }
      } else {
        const int64_t k = k0 + koff[e];
        if (k < kend && nvalid[e] > 0) {
          bits = static_cast<uint32_t>(base[e][k * ld]) >> sh[e];
          n = nvalid[e];
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) v[e][i] = (i < n && ((bits >> i) & 1u)) ? 1.0f : 0.0f;
    }
  }

  __device__ __forceinline__ void store(typename Prec<PREC>::T (*dst)[Stage<PREC>::LD]) const {
#pragma unroll
    for (int e = 0; e < NV; ++e) {
      if constexpr (KCONTIG && PREC == 0) {
        // fp32 rows are 16-byte aligned (36 floats) and koff a multiple of 4
        *reinterpret_cast<f4 *>(&dst[roff[e]][koff[e]]) = f4{v[e][0], v[e][1], v[e][2], v[e][3]};
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if constexpr (KCONTIG)
            dst[roff[e]][koff[e] + i] = cvt<PREC>(v[e][i]);
          else
            dst[roff[e] + i][koff[e]] = cvt<PREC>(v[e][i]);
        }
      }
    }
  }
};

// acc += A[64 x (kb..ke)] B[(kb..ke) x 64], software-pipelined: the next
// stage's global loads are in flight while the current stage runs on MFMA
// from the other LDS buffer (one barrier per stage).
template <int PREC, class LA, class LB>
__device__ __forceinline__ void tile_mma(LA &la, LB &lb, int64_t kb, int64_t ke, Stage<PREC> (&st)[2], int wm,
                                         int wn, int lane, f32x16 &acc) {
  constexpr int KS = Prec<PREC>::KS;
  if (kb >= ke) return;
  la.load(kb, ke);
  lb.load(kb, ke);
  la.store(st[0].a);
  lb.store(st[0].b);
  __syncthreads();
  int buf = 0;
  for (int64_t k0 = kb; k0 < ke; k0 += KS) {
    const bool more = k0 + KS < ke;
    if (more) {
      la.load(k0 + KS, ke);
      lb.load(k0 + KS, ke);
    }
    mfma_stage<PREC>(st[buf], wm, wn, lane, acc);
    if (more) {
      la.store(st[buf ^ 1].a);
      lb.store(st[buf ^ 1].b);
    }
    __syncthreads();
    buf ^= 1;
  }
}

// ---------------------------------------------------------------------------
// Plain GEMM: C[M,N] (+)= A(m,k) B(k,n) (+ bias[n]), fp32 in and out.
//   A(m,k) = TA ? A[k*lda + m] : A[m*lda + k]
//   B(k,n) = TB ? B[n*ldb + k] : B[k*ldb + n]
// gridDim.z > 1 splits K: each split writes its partial tile to the
// workspace and splitk_reduce adds them in split order (deterministic).
// ---------------------------------------------------------------------------
struct GemmArgs {
  const void *A;  // float, or bf16 bits (uint16_t) for the 128 x 128 kernel's bf16 operands
  const void *B;
  const float *bias;  // [N] added in the epilogue, or null
  float *C;
  float *ws;          // [splits, M, N] when split
  int64_t M, N, K, lda, ldb, ldc, kchunk;
  int accumulate, splits;
  // bf16 operands on the 128 x 128 kernel only: C (+)= sum over p < parts of
  // op(A) op(B + p * b_part), each part's k range summed in turn (B points
  // at the first part summed; b_part may be negative)
  int parts = 1;
  int64_t b_part = 0;
  // an independent column sum cs_out[n] = sum_r cs_in[r, n] ([cs_rows,
  // cs_cols]) run by extra workgroups of the split-K reduce launch (from
  // red_blocks on), or after the GEMM when K is not split
  const float *cs_in = nullptr;
  float *cs_out = nullptr;
  int64_t cs_rows = 0, cs_cols = 0, red_blocks = 0;
};

// Writes one wave's 32 x 32 accumulator tile (rows row0 + acc_row(r, lane),
// column col): to plane `split` of the workspace when K is split, else
// C (+)= acc (+ bias[col]) with the adds in that order.  The branches are
// taken once per tile, and the bias and old C values are all loaded before
// the first store, so no store waits behind a load (the vector memory
// counter covers stores as well).
__device__ __forceinline__ void store_acc(const GemmArgs &g, const f32x16 &acc, int64_t row0, int64_t col, int lane,
                                          int64_t split) {
  if (col >= g.N) return;
  if (g.splits > 1) {
    float *ws = g.ws + split * g.M * g.N + col;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int64_t row = row0 + acc_row(r, lane);
      if (row < g.M) ws[row * g.N] = acc[r];
    }
    return;
  }
  float *c = g.C + col;
  if (!g.accumulate && g.bias == nullptr) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int64_t row = row0 + acc_row(r, lane);
      if (row < g.M) c[row * g.ldc] = acc[r];
    }
    return;
  }
  const float b = g.bias != nullptr ? g.bias[col] : 0.0f;
  float v[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int64_t row = row0 + acc_row(r, lane);
    v[r] = (g.accumulate && row < g.M) ? c[row * g.ldc] : 0.0f;
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int64_t row = row0 + acc_row(r, lane);
    float t = g.accumulate ? v[r] + acc[r] : acc[r];
    if (g.bias != nullptr) t = t + b;
    if (row < g.M) c[row * g.ldc] = t;
  }
}

// PA: A holds packed spike bits (lda in words), read by BitLoader.
template <int PREC, bool TA, bool TB, bool VA, bool VB, bool PA>
__global__ __launch_bounds__(256) void gemm_kernel(GemmArgs g) {
  __shared__ Stage<PREC> st[2];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, wm = w >> 1, wn = w & 1;
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * kTile, n0 = static_cast<int64_t>(blockIdx.x) * kTile;
  const int64_t kb = static_cast<int64_t>(blockIdx.z) * g.kchunk;
  const int64_t ke = (kb + g.kchunk < g.K) ? kb + g.kchunk : g.K;

  using SA = typename std::conditional<PA, int32_t, float>::type;
  typename std::conditional<PA, BitLoader<PREC, !TA>, TileLoader<PREC, !TA, VA>>::type la;
  if constexpr (TA) {
    la.map_rowcontig(tid, static_cast<const SA *>(g.A), m0, g.M, g.lda);
  } else {
    la.map_kcontig(tid);
#pragma unroll
    for (int e = 0; e < TileLoader<PREC, true, VA>::NV; ++e) {
      const int64_t m = m0 + la.roff[e];
      la.base[e] = m < g.M ? static_cast<const SA *>(g.A) + m * g.lda : nullptr;
    }
  }
  TileLoader<PREC, TB, VB> lb;
  if constexpr (TB) {
    lb.map_kcontig(tid);
#pragma unroll
    for (int e = 0; e < TileLoader<PREC, true, VB>::NV; ++e) {
      const int64_t n = n0 + lb.roff[e];
      lb.base[e] = n < g.N ? static_cast<const float *>(g.B) + n * g.ldb : nullptr;
    }
  } else {
    lb.map_rowcontig(tid, static_cast<const float *>(g.B), n0, g.N, g.ldb);
  }

  f32x16 acc;
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
  tile_mma<PREC>(la, lb, kb, ke, st, wm, wn, lane, acc);

  store_acc(g, acc, m0 + 32 * wm, n0 + 32 * wn + (lane & 31), lane, blockIdx.z);
}

// out[n] (+)= sum_r in[r, n], in a fixed order (deterministic).
// 8 columns per workgroup (a 2048-column sum spreads over 256 CUs): thread
// (column c = tid % 8, group q = tid / 8) sums rows q, q + 32, ... in order,
// then the 32 group sums are added in group order
__device__ __forceinline__ void col_sum_block(const float *__restrict__ in, float *__restrict__ out, int64_t rows,
                                              int64_t cols, int accumulate, int64_t block) {
  __shared__ float part[32][8];
  const int c = threadIdx.x & 7, q = threadIdx.x >> 3;
  const int64_t n = block * 8 + c;
  float s = 0.0f;
  if (n < cols)
    for (int64_t r = q; r < rows; r += 32) s = s + in[r * cols + n];
  part[q][c] = s;
  __syncthreads();
  if (q == 0 && n < cols) {
    float t = 0.0f;
    for (int i = 0; i < 32; ++i) t = t + part[i][c];
    out[n] = accumulate ? out[n] + t : t;
  }
}

// C (+)= sum over splits of the workspace planes (+ bias), four consecutive
// columns per thread (N, ldc, C and the workspace all allow 16-byte
// access): one 16-byte load per plane, adds in split order.  Workgroups
// from g.red_blocks on run the attached column sum instead.
__global__ __launch_bounds__(256) void splitk_reduce4(GemmArgs g) {
  if (static_cast<int64_t>(blockIdx.x) >= g.red_blocks) {
    col_sum_block(g.cs_in, g.cs_out, g.cs_rows, g.cs_cols, 0, blockIdx.x - g.red_blocks);
    return;
  }
  const int64_t i = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) * 4;
  if (i >= g.M * g.N) return;
  const int64_t row = i / g.N, col = i - row * g.N;
  float *dst = g.C + row * g.ldc + col;
  f4 v = {0.0f, 0.0f, 0.0f, 0.0f};
  if (g.accumulate) v = *reinterpret_cast<const f4 *>(dst);
  f4 part = {0.0f, 0.0f, 0.0f, 0.0f};
  const int64_t plane = g.M * g.N;
#pragma unroll 4
  for (int z = 0; z < g.splits; ++z) {
    const f4 w = *reinterpret_cast<const f4 *>(g.ws + z * plane + i);
#pragma unroll
    for (int e = 0; e < 4; ++e) part[e] = part[e] + w[e];
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    v[e] = v[e] + part[e];
    if (g.bias != nullptr) v[e] = v[e] + g.bias[col + e];
  }
  *reinterpret_cast<f4 *>(dst) = v;
}

__global__ __launch_bounds__(256) void splitk_reduce(GemmArgs g) {
  if (static_cast<int64_t>(blockIdx.x) >= g.red_blocks) {
    col_sum_block(g.cs_in, g.cs_out, g.cs_rows, g.cs_cols, 0, blockIdx.x - g.red_blocks);
    return;
  }
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= g.M * g.N) return;
  const int64_t row = i / g.N, col = i - row * g.N;
  float *dst = g.C + row * g.ldc + col;
  float v = g.accumulate ? *dst : 0.0f;
  // loads issued ahead, adds in split order
  float part = 0.0f;
  const int64_t plane = g.M * g.N;
#pragma unroll 8
  for (int z = 0; z < g.splits; ++z) part = part + g.ws[z * plane + i];
  v = v + part;
  if (g.bias != nullptr) v = v + g.bias[col];
  *dst = v;
}

// the split-K reduce: four columns per thread where rows and pointers allow,
// with the attached column sum's workgroups after the reduce's
void launch_reduce(GemmArgs g, hipStream_t s) {
  const bool v4 = g.N % 4 == 0 && g.ldc % 4 == 0 && myelin::aligned(g.C, 16) && myelin::aligned(g.ws, 16);
  const int64_t n = g.M * g.N;
  g.red_blocks = v4 ? (n / 4 + 255) / 256 : (n + 255) / 256;
  const int64_t blocks = g.red_blocks + (g.cs_in != nullptr ? (g.cs_cols + 7) / 8 : 0);
  if (v4)
    splitk_reduce4<<<dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s>>>(g);
  else
    splitk_reduce<<<dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s>>>(g);
}

// Three bf16 values whose float sum is exactly v: h = bf16(v) (nearest
// even), m = bf16(v - h), l = v - h - m.  v - h is exact and has at most 16
// significant bits, so after m at most 8 remain and l is exact as well (for
// |v| >= 2^-110; below that l would be subnormal in bf16).  Non-finite v:
// h carries it, m = l = 0.
__device__ __forceinline__ void split3(float v, uint16_t &h, uint16_t &m, uint16_t &l) {
  const __bf16 bh = static_cast<__bf16>(v);
  if (!__builtin_isfinite(v)) {
    h = __builtin_bit_cast(uint16_t, bh);
    m = l = 0;
    return;
  }
  const float r1 = v - static_cast<float>(bh);
  const __bf16 bm = static_cast<__bf16>(r1);
  const float r2 = r1 - static_cast<float>(bm);
  h = __builtin_bit_cast(uint16_t, bh);
  m = __builtin_bit_cast(uint16_t, bm);
  l = __builtin_bit_cast(uint16_t, static_cast<__bf16>(r2));
}

// ---------------------------------------------------------------------------
// Narrow GEMMs for the readout layers: outputs at most 32 columns wide
// (gemm_narrow: currents I = S W_o and dW_o = S^T G_o) or K at most 32
// (gemm_smallk: dS = G_o W_o^T, on the vector ALUs, below).  gemm_narrow
// streams the long operand A from global memory straight into MFMA
// fragments -- it is read once, so it skips LDS -- with the narrow operand
// in LDS.  Per-lane k layout of a group of 16 consecutive k:
//   lane l holds k = k0 + 8 * (l / 32) + [0, 8)
// and each group is one v_mfma_f32_32x32x16_bf16 (bf16 precision), or three
// to nine of them on exact bf16 planes of the operands (fp32 precision,
// gemm_narrow_x3 below).
// A(m, k) may be fp32 (TA: A[k*lda + m], else A[m*lda + k]) or packed spike
// bits (PA: bit m%32 of word A[k*lda + m/32] with TA, else bit k%32 of word
// A[m*lda + k/32]).
// ---------------------------------------------------------------------------
#ifndef MYELIN_NARROW_U
#define MYELIN_NARROW_U 8  // A groups loaded per batch by the narrow kernel
#endif
#ifndef MYELIN_NARROW_KCHUNK
#define MYELIN_NARROW_KCHUNK 512  // k per K split of the narrow kernel (before rounding to 64)
#endif
#ifndef MYELIN_NARROW_KSUB3
#define MYELIN_NARROW_KSUB3 256  // k per staged B sub-chunk, exact-split kernel
#endif

template <int PREC>
struct Narrow;
template <>
struct Narrow<1> {
  static constexpr int KG = 8, KSUB = 512, PAD = 8;
};

template <bool TA, bool PA>
__device__ __forceinline__ float a_elem(const GemmArgs &g, int64_t m, int64_t k) {
  if constexpr (PA) {
    const int32_t *A = static_cast<const int32_t *>(g.A);
    const uint32_t w = static_cast<uint32_t>(TA ? A[k * g.lda + (m >> 5)] : A[m * g.lda + (k >> 5)]);
    return ((w >> (TA ? (m & 31) : (k & 31))) & 1u) ? 1.0f : 0.0f;
  } else {
    const float *A = static_cast<const float *>(g.A);
    return TA ? A[k * g.lda + m] : A[m * g.lda + k];
  }
}

template <bool TB>
__device__ __forceinline__ float b_elem(const GemmArgs &g, int64_t k, int64_t n) {
  const float *B = static_cast<const float *>(g.B);
  return TB ? B[n * g.ldb + k] : B[k * g.ldb + n];
}

template <int PREC>
struct BFrag;  // a lane's B fragment for one group
template <>
struct BFrag<1> {
  using V = bf16x8;
};

// One group: acc += A-fragment (8 fp32 values, rounded to bf16) x B-fragment.
template <int PREC>
__device__ __forceinline__ void group_mfma(const float *a, typename BFrag<PREC>::V bv, f32x16 &acc) {
  bf16x8 av;
#pragma unroll
  for (int i = 0; i < 8; ++i) av[i] = static_cast<__bf16>(a[i]);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, bv, acc, 0, 0, 0);
}

// A lane's KG values of A for the group starting at k (row m).  FULL: the
// whole group lies below kend (no guards); VA: 16-byte loads (k-contiguous
// fp32 rows, aligned).
template <int PREC, bool TA, bool PA, bool VA, bool FULL>
__device__ __forceinline__ void load_group(const GemmArgs &g, int64_t m, int64_t k, int64_t kend, float *a) {
  constexpr int KG = Narrow<PREC>::KG;
  if constexpr (FULL && !TA && !PA && VA) {
    const f4 *q = reinterpret_cast<const f4 *>(static_cast<const float *>(g.A) + m * g.lda + k);
#pragma unroll
    for (int v = 0; v < KG / 4; ++v) {
      const f4 t = q[v];
      a[4 * v] = t.x;
      a[4 * v + 1] = t.y;
      a[4 * v + 2] = t.z;
      a[4 * v + 3] = t.w;
    }
  } else if constexpr (!TA && PA) {
    // KG bits of one word (k is a multiple of KG, so they never straddle
    // words); a group starting at or past kend reads nothing
    const uint32_t w =
        (FULL || k < kend) ? static_cast<uint32_t>(static_cast<const int32_t *>(g.A)[m * g.lda + (k >> 5)]) >> (k & 31)
                           : 0u;
#pragma unroll
    for (int i = 0; i < KG; ++i) a[i] = ((FULL || k + i < kend) && ((w >> i) & 1u)) ? 1.0f : 0.0f;
  } else {
#pragma unroll
    for (int i = 0; i < KG; ++i) a[i] = (FULL || k + i < kend) ? a_elem<TA, PA>(g, m, k + i) : 0.0f;
  }
}

template <int PREC>
struct NarrowB {
  static constexpr int LD = Narrow<PREC>::KSUB + Narrow<PREC>::PAD;
  alignas(16) typename Prec<PREC>::T b[32][LD];
};

// Stages B(k, n) for k in [ks, ks + kpad), n < N: put(n, k - ks, value),
// zero past klen; rows past N are never stored, so they stay unwritten.  The
// elements are walked flat in memory order -- contiguous when ldb equals the
// contiguous extent -- R loads issued before their LDS writes.
template <bool TB, typename Put, int R = 8>
__device__ __forceinline__ void stage_narrow(const GemmArgs &g, int64_t ks, int klen, int kpad, int N, int tid,
                                             int nt, Put put) {
  const float *B = static_cast<const float *>(g.B);
  const int total = N * klen;
  // e / d as a multiply-high by ceil(2^32 / d) (d >= 2; d = 1 is e
  // itself): exact for e * d < 2^32 (e < 32 * KSUB here), where a hardware
  // division would cost ~20 ops
  const uint32_t d = TB ? static_cast<uint32_t>(klen) : static_cast<uint32_t>(N);
  const uint32_t mag = d > 1 ? static_cast<uint32_t>((0x100000000ull + d - 1) / d) : 0u;
  auto split = [&](int e, int &n, int &kk) {
    const int q = d > 1 ? static_cast<int>(__umulhi(static_cast<uint32_t>(e), mag)) : e;
    if constexpr (TB) {
      n = q;
      kk = e - q * klen;
    } else {
      kk = q;
      n = e - q * N;
    }
  };
  for (int e0 = tid; e0 < total; e0 += nt * R) {
    float v[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      int e = e0 + nt * r;
      e = e < total ? e : total - 1;  // clamped: every load in range
      int n, kk;
      split(e, n, kk);
      v[r] = TB ? B[n * g.ldb + ks + kk] : B[(ks + kk) * g.ldb + n];
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int e = e0 + nt * r;
      if (e < total) {
        int n, kk;
        split(e, n, kk);
        put(n, kk, v[r]);
      }
    }
  }
  for (int e = tid; e < N * (kpad - klen); e += nt) {
    const int n = e / (kpad - klen);
    put(n, klen + (e - n * (kpad - klen)), 0.0f);
  }
}

template <int PREC, bool TB, int LD>
__device__ __forceinline__ void stage_narrow_b(const GemmArgs &g, int64_t ks, int klen, int kpad, int N,
                                               typename Prec<PREC>::T (*bs)[LD], int tid) {
  stage_narrow<TB>(g, ks, klen, kpad, N, tid, 256, [&](int n, int kk, float v) { bs[n][kk] = cvt<PREC>(v); });
}

// C[M, N] (+)= op(A) op(B) (+ bias) for N <= 32.  Workgroup: 4 waves x 32
// rows of the output; blockIdx.y selects a K split of kchunk (a multiple of
// 64).  The split is walked in sub-chunks of KSUB: B's N columns over the
// sub-chunk are staged to LDS, then each wave streams its rows of A, U
// groups of loads at a time (the first batch issued before B is staged).
template <int PREC, bool TA, bool TB, bool PA, bool VA>
__global__ __launch_bounds__(256) void gemm_narrow(GemmArgs g) {
  using T = typename Prec<PREC>::T;
  using BV = typename BFrag<PREC>::V;
  constexpr int KG = Narrow<PREC>::KG, KSUB = Narrow<PREC>::KSUB, LD = NarrowB<PREC>::LD;
  constexpr int GS = 2 * KG;            // k per group
  constexpr int U = MYELIN_NARROW_U;    // groups in flight per lane
  __shared__ NarrowB<PREC> sb;
  auto &bs = sb.b;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t kb = static_cast<int64_t>(blockIdx.y) * g.kchunk;
  const int64_t ke = (kb + g.kchunk < g.K) ? kb + g.kchunk : g.K;
  const int64_t m0 = static_cast<int64_t>(blockIdx.x) * 128 + 32 * w;
  const bool wave_on = m0 < g.M;  // uniform per wave
  const int64_t m = (m0 + (lane & 31) < g.M) ? m0 + (lane & 31) : g.M - 1;
  const int kh = (lane >> 5) * KG;
  const int N = static_cast<int>(g.N);

  f32x16 acc, acc_s;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    acc[r] = 0.0f;
    acc_s[r] = 0.0f;
  }

  for (int64_t ks = kb; ks < ke; ks += KSUB) {
    const int klen = static_cast<int>((ke - ks < KSUB) ? ke - ks : KSUB);
    const int kpad = (klen + GS - 1) / GS * GS;
    const int ng = kpad / GS;
    const int nfull = klen / (U * GS);  // batches of U groups wholly below ke
    float a[U][KG];
    if (wave_on && nfull > 0) {
#pragma unroll
      for (int u = 0; u < U; ++u) load_group<PREC, TA, PA, VA, true>(g, m, ks + u * GS + kh, ke, a[u]);
    }
    if (ks != kb) __syncthreads();  // the previous sub-chunk's fragments are read
    stage_narrow_b<PREC, TB, LD>(g, ks, klen, kpad, N, bs, tid);
    __syncthreads();
    if (!wave_on) continue;
    const T *brow = &bs[lane & 31][kh];
    for (int bi = 0; bi < nfull; ++bi) {
      if (bi > 0) {
#pragma unroll
        for (int u = 0; u < U; ++u)
          load_group<PREC, TA, PA, VA, true>(g, m, ks + (bi * U + u) * GS + kh, ke, a[u]);
      }
#pragma unroll
      for (int u = 0; u < U; ++u)
        group_mfma<PREC>(a[u], *reinterpret_cast<const BV *>(brow + (bi * U + u) * GS), acc);
    }
    for (int j = nfull * U; j < ng; ++j) {
      float t[KG];
      load_group<PREC, TA, PA, VA, false>(g, m, ks + j * GS + kh, ke, t);
      group_mfma<PREC>(t, *reinterpret_cast<const BV *>(brow + j * GS), acc);
    }
  }
  if (!wave_on) return;
  store_acc(g, acc, m0, lane & 31, lane, blockIdx.y);
}

// gemm_narrow at fp32 precision, on the bf16 MFMA with every product exact.
// B's staged sub-chunk is split into three bf16 planes (split3: hi + mid +
// lo == B), and A is packed spike bits (one plane of 0/1 values) or fp32
// values split the same way as they are loaded.  A product of two bf16
// values is exact in fp32, so only the fp32 accumulation rounds.  Two
// accumulators: one takes the products of the high planes of A and B, the
// other every smaller product (A planes 2 and 1 times B planes 2, 1, 0,
// then A plane 0 times B planes 2 and 1, each A plane skipped wave-uniformly
// when it is zero in every lane: a 0/1 matrix gives the same bits as words
// or as floats), and they are added once at the end.  Only the high-plane
// products then round against the full-size sum, as in a plain fp32 GEMM;
// in one accumulator every plane's products did (the 4096 -> 20 readout's
// currents and weight gradient lost up to 3x the accuracy of an fp32 GEMM).
// For a bit operand that is three bf16 MFMAs per 16 k where the fp32 MFMA
// takes eight 32x32x2 steps at a sixteenth of the bf16 rate; the 4096 -> 20
// readout's currents at T=2000, B=32 (64000 x 4096 bits x 20) and its dW_o
// measured 243 and 208 us on the fp32 MFMA.
struct NarrowB3 {
  static constexpr int KSUB = MYELIN_NARROW_KSUB3, LD = KSUB + 8;
  alignas(16) uint16_t b[3][32][LD];
};

__device__ __forceinline__ bf16x8 bf16_frag(const uint16_t *p) { return *reinterpret_cast<const bf16x8 *>(p); }

template <bool PA>
__device__ __forceinline__ void group_x3(const float (&a)[8], const uint16_t *b0, const uint16_t *b1,
                                         const uint16_t *b2, f32x16 &acc, f32x16 &acc_s) {
  const bf16x8 v0 = bf16_frag(b0), v1 = bf16_frag(b1), v2 = bf16_frag(b2);
  bf16x8 ap[3];
  bool nz1 = false, nz2 = false;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    if constexpr (PA) {
      ap[0][i] = static_cast<__bf16>(a[i]);  // 0 or 1
    } else {
      uint16_t h, m, l;
      split3(a[i], h, m, l);
      ap[0][i] = __builtin_bit_cast(__bf16, h);
      ap[1][i] = __builtin_bit_cast(__bf16, m);
      ap[2][i] = __builtin_bit_cast(__bf16, l);
      nz1 = nz1 || (m & 0x7fffu) != 0;
      nz2 = nz2 || (l & 0x7fffu) != 0;
    }
  }
  // the smaller products, smallest planes first, into acc_s
  if constexpr (!PA) {
    if (__ballot(nz2) != 0) {
      acc_s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ap[2], v2, acc_s, 0, 0, 0);
      acc_s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ap[2], v1, acc_s, 0, 0, 0);
      acc_s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ap[2], v0, acc_s, 0, 0, 0);
    }
    if (__ballot(nz1) != 0) {
      acc_s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ap[1], v2, acc_s, 0, 0, 0);
      acc_s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ap[1], v1, acc_s, 0, 0, 0);
      acc_s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ap[1], v0, acc_s, 0, 0, 0);
    }
  }
  acc_s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ap[0], v2, acc_s, 0, 0, 0);
  acc_s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ap[0], v1, acc_s, 0, 0, 0);
  // the largest (high planes of both operands) into acc
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ap[0], v0, acc, 0, 0, 0);
}

// Same workgroup shape, K split and A streaming as gemm_narrow<1>.
template <bool TA, bool TB, bool PA, bool VA>
__global__ __launch_bounds__(256) void gemm_narrow_x3(GemmArgs g) {
  constexpr int KG = 8, GS = 16, KSUB = NarrowB3::KSUB;
  constexpr int U = MYELIN_NARROW_U;  // groups in flight per lane
  __shared__ NarrowB3 sb;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t kb = static_cast<int64_t>(blockIdx.y) * g.kchunk;
  const int64_t ke = (kb + g.kchunk < g.K) ? kb + g.kchunk : g.K;
  const int64_t m0 = static_cast<int64_t>(blockIdx.x) * 128 + 32 * w;
  const bool wave_on = m0 < g.M;  // uniform per wave
  const int64_t m = (m0 + (lane & 31) < g.M) ? m0 + (lane & 31) : g.M - 1;
  const int kh = (lane >> 5) * KG;
  const int N = static_cast<int>(g.N);

  f32x16 acc, acc_s;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    acc[r] = 0.0f;
    acc_s[r] = 0.0f;
  }

  for (int64_t ks = kb; ks < ke; ks += KSUB) {
    const int klen = static_cast<int>((ke - ks < KSUB) ? ke - ks : KSUB);
    const int kpad = (klen + GS - 1) / GS * GS;
    const int ng = kpad / GS;
    const int nfull = klen / (U * GS);  // batches of U groups wholly below ke
    float a[U][KG];
    if (wave_on && nfull > 0) {
#pragma unroll
      for (int u = 0; u < U; ++u) load_group<1, TA, PA, VA, true>(g, m, ks + u * GS + kh, ke, a[u]);
    }
    if (ks != kb) __syncthreads();  // the previous sub-chunk's fragments are read
    stage_narrow<TB>(g, ks, klen, kpad, N, tid, 256, [&](int n, int kk, float v) {
      uint16_t h, mid, l;
      split3(v, h, mid, l);
      sb.b[0][n][kk] = h;
      sb.b[1][n][kk] = mid;
      sb.b[2][n][kk] = l;
    });
    __syncthreads();
    if (!wave_on) continue;
    const uint16_t *b0 = &sb.b[0][lane & 31][kh], *b1 = &sb.b[1][lane & 31][kh], *b2 = &sb.b[2][lane & 31][kh];
    for (int bi = 0; bi < nfull; ++bi) {
      if (bi > 0) {
#pragma unroll
        for (int u = 0; u < U; ++u) load_group<1, TA, PA, VA, true>(g, m, ks + (bi * U + u) * GS + kh, ke, a[u]);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int o = (bi * U + u) * GS;
        group_x3<PA>(a[u], b0 + o, b1 + o, b2 + o, acc, acc_s);
      }
    }
    for (int j = nfull * U; j < ng; ++j) {
      float t[KG];
      load_group<1, TA, PA, VA, false>(g, m, ks + j * GS + kh, ke, t);
      group_x3<PA>(t, b0 + j * GS, b1 + j * GS, b2 + j * GS, acc, acc_s);
    }
  }
  if (!wave_on) return;
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = acc[r] + acc_s[r];
  store_acc(g, acc, m0, lane & 31, lane, blockIdx.y);
}

// Narrow GEMM with row-major packed-bit A (the readout currents I = S W_o
// from the hidden spikes' packed twin): NP = 3 bf16 planes of B (fp32
// precision, exact, as gemm_narrow_x3) or NP = 1 (bf16 precision, B rounded,
// as gemm_narrow<1>), the same MFMAs on the same k in the same order as
// those kernels, so the bits equal theirs.  Eight waves of 32 rows share one
// staged sub-chunk of B (the staging and its split cost as much VALU as the
// MFMA feed at four waves), and a lane turns its 8 bits of a group into
// the bf16 fragment with integer operations (0/1 -> 0x0000/0x3F80) instead
// of going through floats.  64000 x 4096 x 20 at fp32: 150 -> 95 us.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t bf16_pair_of_bits(uint32_t t) {
  // bit 0 -> the low bf16, bit 1 -> the high one
  return ((t & 1u) | ((t & 2u) << 15)) * 0x3F80u;
}

template <int NP>
struct NarrowBits {
  static constexpr int KSUB = 256, LD = KSUB + 8, WAVES = 8;
  alignas(16) uint16_t b[NP][32][LD];
};

template <int NP>
__global__ __launch_bounds__(64 * NarrowBits<NP>::WAVES) void gemm_narrow_bits(GemmArgs g) {
  using L = NarrowBits<NP>;
  constexpr int KG = 8, GS = 16, KSUB = L::KSUB, WAVES = L::WAVES;
  __shared__ L sb;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t kb = static_cast<int64_t>(blockIdx.y) * g.kchunk;
  const int64_t ke = (kb + g.kchunk < g.K) ? kb + g.kchunk : g.K;
  const int64_t m0 = static_cast<int64_t>(blockIdx.x) * (32 * WAVES) + 32 * w;
  const bool wave_on = m0 < g.M;  // uniform per wave
  const int64_t m = (m0 + (lane & 31) < g.M) ? m0 + (lane & 31) : g.M - 1;
  const int kh = (lane >> 5) * KG;
  const int N = static_cast<int>(g.N);
  const int32_t *arow = static_cast<const int32_t *>(g.A) + m * g.lda;

  f32x16 acc, acc_s;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    acc[r] = 0.0f;
    acc_s[r] = 0.0f;
  }

  for (int64_t ks = kb; ks < ke; ks += KSUB) {
    const int klen = static_cast<int>((ke - ks < KSUB) ? ke - ks : KSUB);
    const int kpad = (klen + GS - 1) / GS * GS;
    if (ks != kb) __syncthreads();  // the previous sub-chunk's fragments are read
    stage_narrow<false>(g, ks, klen, kpad, N, tid, 64 * WAVES, [&](int n, int kk, float v) {
      if constexpr (NP == 3) {
        uint16_t h, mid, l;
        split3(v, h, mid, l);
        sb.b[0][n][kk] = h;
        sb.b[1][n][kk] = mid;
        sb.b[2][n][kk] = l;
      } else {
        sb.b[0][n][kk] = __builtin_bit_cast(uint16_t, static_cast<__bf16>(v));
      }
    });
    __syncthreads();
    if (!wave_on) continue;
    const int ng = kpad / GS, nfull = klen / GS;
    for (int j = 0; j < ng; ++j) {
      const int64_t k = ks + j * GS + kh;
      uint32_t wv = k < ke ? static_cast<uint32_t>(arow[k >> 5]) >> (k & 31) : 0u;
      if (j >= nfull && k + KG > ke) wv &= k < ke ? (1u << (ke - k)) - 1u : 0u;
      const u32x4 d = {bf16_pair_of_bits(wv), bf16_pair_of_bits(wv >> 2), bf16_pair_of_bits(wv >> 4),
                       bf16_pair_of_bits(wv >> 6)};
      const bf16x8 av = __builtin_bit_cast(bf16x8, d);
      const int o = j * GS + kh;
      // as gemm_narrow_x3: B planes 2 and 1 into acc_s, plane 0 into acc
#pragma unroll
      for (int p = NP - 1; p > 0; --p)
        acc_s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
            av, *reinterpret_cast<const bf16x8 *>(&sb.b[p][lane & 31][o]), acc_s, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, *reinterpret_cast<const bf16x8 *>(&sb.b[0][lane & 31][o]),
                                                    acc, 0, 0, 0);
    }
  }
  if (!wave_on) return;
  if constexpr (NP > 1) {
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = acc[r] + acc_s[r];
  }
  store_acc(g, acc, m0, lane & 31, lane, blockIdx.y);
}

// Narrow GEMM with transposed packed-bit A: dW_o = S^T G_o, A(m, k) = bit
// m%32 of word A[k*lda + m/32] (k a batch-step row, m a hidden neuron), the
// same MFMAs on the same k in the same order as gemm_narrow_x3 / gemm_narrow
// with that operand, so the bits equal theirs.  A lane of the MFMA needs 8
// k of one m: 8 rows' words, one bit each, which those kernels load and
// test one by one.  Here each lane of a wave loads one row's words of the
// wave's four 32-neuron word columns (one 16-byte load), 64 rows a wave;
// per column the two 32 x 32 bit blocks (lanes 0-31 and 32-63) are turned
// around with a 5-stage butterfly across lanes (stage D: lanes l and l ^ D
// swap the off-diagonal D x D blocks of their rows, a lane shuffle, a
// rotate and a bit-field insert), after which lane m holds one word of 32
// rows' bits of its neuron.  The rows are loaded in the order
// rho(j) = 16 (j%16 / 4) + 2 (j%4) + j/16 (+ 8 in lanes 32-63), so that
// bits b and b + 16 of that word are the rows of the lo and hi bf16 of
// fragment pair b%4 of group b/4: one mask and one 24-bit multiply by
// 0x3F80 make a pair of 0/1 bf16 values.  Four waves of four word columns
// each share one staged sub-chunk of B (NP planes, as gemm_narrow_bits);
// two workgroups per CU, so one stages while the other runs its MFMAs, and
// the 64000-row, 4096-neuron dW_o (8 workgroups per K split, 63 splits)
// fits the chip in one round.  A lane's words are loaded two 64-row blocks
// ahead of their MFMAs.  That dW_o (fp32, three planes) measured 168 -> 66
// us, with its split-K reduce 176 -> 75 us; bf16 precision 51 us.  Counters
// of the fp32 kernel: MFMA busy 31 %, VALU busy ~37 %, a third of each
// wave's cycles waiting (two waves a SIMD: the transposes' lane shuffles
// and the loads are latency the other wave only partly covers).
#ifndef MYELIN_BITS_T_MIN_WG
#define MYELIN_BITS_T_MIN_WG 256  // workgroups below which the four-wave kernels keep the shape
#endif
template <int NP>
struct NarrowBitsT {
  static constexpr int KSUB = 256, LD = KSUB + 8, WAVES = 4, TILES = 4, COLS = WAVES * TILES;
  alignas(16) uint16_t b[NP][32][LD];
};

// One butterfly stage of the transpose (the rotate amount and the mask are
// the lane's own: rows with bit D of the lane index clear keep their
// columns with bit D clear).
template <int D>
__device__ __forceinline__ uint32_t xpose_stage(uint32_t w, uint32_t rot, uint32_t keep) {
  uint32_t p;
  if constexpr (D == 1)
    p = static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(w), 0xB1, 0xF, 0xF, true));
  else if constexpr (D == 2)
    p = static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(w), 0x4E, 0xF, 0xF, true));
  else
    p = static_cast<uint32_t>(__builtin_amdgcn_ds_swizzle(static_cast<int>(w), 0x1F | (D << 10)));
  const uint32_t q = __builtin_amdgcn_alignbit(p, p, rot);
  return (w & keep) | (q & ~keep);
}

template <int NP>
__global__ __launch_bounds__(64 * NarrowBitsT<NP>::WAVES) __attribute__((amdgpu_waves_per_eu(2)))
void gemm_narrow_bits_t(GemmArgs g) {
  using L = NarrowBitsT<NP>;
  constexpr int GS = 16, KSUB = L::KSUB, WAVES = L::WAVES, TILES = L::TILES;
  __shared__ L sb;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t kb = static_cast<int64_t>(blockIdx.y) * g.kchunk;
  const int64_t ke = (kb + g.kchunk < g.K) ? kb + g.kchunk : g.K;
  const int64_t col0 = static_cast<int64_t>(blockIdx.x) * L::COLS + TILES * w;  // the wave's first word column
  const int N = static_cast<int>(g.N);
  const int kh = (lane >> 5) * 8;
  const int j = lane & 31;
  const int rho = 16 * ((j & 15) >> 2) + 2 * (j & 3) + (j >> 4) + kh;  // the lane's row of a 64-row block
  const int32_t *A = static_cast<const int32_t *>(g.A);
  bool on[TILES];
#pragma unroll
  for (int t = 0; t < TILES; ++t) on[t] = 32 * (col0 + t) < g.M;  // uniform per wave
  // the lane's rotate amounts and kept-column masks, stages 16, 8, 4, 2, 1
  uint32_t rot[5], keep[5];
#pragma unroll
  for (int i = 0; i < 5; ++i) {
    const int D = 16 >> i;
    const uint32_t m = i == 0 ? 0x0000FFFFu : i == 1 ? 0x00FF00FFu : i == 2 ? 0x0F0F0F0Fu : i == 3 ? 0x33333333u : 0x55555555u;
    const bool top = (lane & D) == 0;
    rot[i] = top ? 32 - D : D;
    keep[i] = top ? m : ~m;
  }
  // a 64-row block's words per lane (rows past ke read as 0): the wave's
  // four columns of a row in one 16-byte load where rows allow it
  const bool vec = on[TILES - 1] && g.lda % 4 == 0 && (reinterpret_cast<uintptr_t>(A) & 15) == 0;
  auto load_words = [&](int64_t row, uint32_t (&wd)[TILES]) {
    static_assert(TILES == 4, "one 16-byte load holds the four tiles' words");
    if (vec) {
      const u32x4 v = row < ke ? *reinterpret_cast<const u32x4 *>(A + row * g.lda + col0) : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
      for (int t = 0; t < TILES; ++t) wd[t] = v[t];
    } else {
#pragma unroll
      for (int t = 0; t < TILES; ++t)
        wd[t] = (on[t] && row < ke) ? static_cast<uint32_t>(A[row * g.lda + col0 + t]) : 0u;
    }
  };

  f32x16 acc[TILES], acc_s[TILES];
#pragma unroll
  for (int t = 0; t < TILES; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      acc[t][r] = 0.0f;
      acc_s[t][r] = 0.0f;
    }

  // the 32 x 32 bit blocks of a 64-row block turned around: x[t] the
  // lane's word of 32 rows of its neuron, x8[t] the same shifted down by 8
  auto transpose = [&](const uint32_t (&wd)[TILES], uint32_t (&x)[TILES], uint32_t (&x8)[TILES]) {
#pragma unroll
    for (int t = 0; t < TILES; ++t) {
      uint32_t v = wd[t];
      v = xpose_stage<16>(v, rot[0], keep[0]);
      v = xpose_stage<8>(v, rot[1], keep[1]);
      v = xpose_stage<4>(v, rot[2], keep[2]);
      v = xpose_stage<2>(v, rot[3], keep[3]);
      v = xpose_stage<1>(v, rot[4], keep[4]);
      x[t] = v;
      x8[t] = v >> 8;
    }
  };
  // group jg of the sub-chunk (16 k) for every tile: groups 0-1 of a block
  // take bits 0-7 (and 16-23) of the word, groups 2-3 bits 8-15 (24-31),
  // from the word shifted down by 8.  A tile past M runs on zero words and
  // is not stored.
  auto group = [&](int jg, int q, const uint32_t (&x)[TILES], const uint32_t (&x8)[TILES]) {
    const int o = jg * GS + kh;
    bf16x8 bv[NP];
#pragma unroll
    for (int p = 0; p < NP; ++p) bv[p] = *reinterpret_cast<const bf16x8 *>(&sb.b[p][lane & 31][o]);
    bf16x8 av[TILES];
#pragma unroll
    for (int t = 0; t < TILES; ++t) {
      const uint32_t xb = q >= 2 ? x8[t] : x[t];
      u32x4 d;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int bp = (4 * q + i) & 7;
        d[i] = __umul24(xb & (0x10001u << bp), 0x3F80u >> bp);
      }
      av[t] = __builtin_bit_cast(bf16x8, d);
    }
    // as gemm_narrow_x3: B planes 2 and 1 into acc_s, plane 0 into acc
#pragma unroll
    for (int p = NP - 1; p > 0; --p)
#pragma unroll
      for (int t = 0; t < TILES; ++t)
        acc_s[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[t], bv[p], acc_s[t], 0, 0, 0);
#pragma unroll
    for (int t = 0; t < TILES; ++t)
      acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[t], bv[0], acc[t], 0, 0, 0);
  };

  for (int64_t ks = kb; ks < ke; ks += KSUB) {
    const int klen = static_cast<int>((ke - ks < KSUB) ? ke - ks : KSUB);
    const int kpad = (klen + GS - 1) / GS * GS;
    const int ng = kpad / GS;
    // blocks 0-1's words, issued before B is staged; each later block's two
    // blocks ahead of its MFMAs
    uint32_t wa[TILES], wb[TILES];
    load_words(ks + rho, wa);
    load_words(ks + 64 + rho, wb);
    if (ks != kb) __syncthreads();  // the previous sub-chunk's fragments are read
    auto put = [&](int n, int kk, float v) {
      if constexpr (NP == 3) {
        uint16_t h, mid, l;
        split3(v, h, mid, l);
        sb.b[0][n][kk] = h;
        sb.b[1][n][kk] = mid;
        sb.b[2][n][kk] = l;
      } else {
        sb.b[0][n][kk] = __builtin_bit_cast(uint16_t, static_cast<__bf16>(v));
      }
    };
    // 10 loads in flight per thread: the 256 x 20 sub-chunk in two rounds
    stage_narrow<false, decltype(put), 10>(g, ks, klen, kpad, N, tid, 64 * WAVES, put);
    __syncthreads();
#pragma unroll 1
    for (int s = 0; 4 * s < ng; ++s) {
      uint32_t x[TILES], x8[TILES];
      transpose(wa, x, x8);
#pragma unroll
      for (int t = 0; t < TILES; ++t) wa[t] = wb[t];
      if (4 * s + 8 < ng) load_words(ks + 64 * (s + 2) + rho, wb);
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (4 * s + q < ng) group(4 * s + q, q, x, x8);
    }
  }
#pragma unroll
  for (int t = 0; t < TILES; ++t) {
    if (!on[t]) continue;
    if constexpr (NP > 1) {
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[t][r] = acc[t][r] + acc_s[t][r];
    }
    store_acc(g, acc[t], 32 * (col0 + t), lane & 31, lane, blockIdx.y);
  }
}

// Rounds an operand value to the MFMA input type of the precision (bf16:
// round to nearest even), kept in fp32.
template <int PREC>
__device__ __forceinline__ float round_in(float v) {
  if constexpr (PREC == 1)
    return static_cast<float>(static_cast<__bf16>(v));
  else
    return v;
}

// C[M, N] (+)= op(A) op(B) (+ bias) for K <= KMAX <= 32, on the vector ALUs
// (the arithmetic is a few FMAs per output; the cost is writing C).  Each
// lane owns 4 adjacent columns and holds B's K x 4 block in registers (B
// stored [N, K] is first staged k-major through LDS by the workgroup, whose
// 4 waves share the 256 columns, from one coalesced read); a wave owns RW
// rows.  The wave's RW x KMAX block of A is loaded up front,
// spread over the lanes (value q = row * KMAX + k in lane q % 64), and each
// value is broadcast to the wave with a lane read when its row is computed,
// so all loads are in flight at once.  Each row is one 16-byte store per
// lane, 1 KB contiguous per wave.  Products of the operands rounded to the
// precision's input type, summed in k order with fused multiply-adds (bf16
// products are exact in fp32).  VC: C rows allow 16-byte stores.
#ifndef MYELIN_SMALLK_RW
#define MYELIN_SMALLK_RW 16  // rows per wave of the small-K kernel
#endif

template <int PREC, bool TA, bool TB, bool PA, int KMAX, bool VC>
__global__ __launch_bounds__(256) void gemm_smallk(GemmArgs g) {
  constexpr int RW = MYELIN_SMALLK_RW;     // rows per wave
  constexpr int SLOTS = RW * KMAX / 64;    // A values per lane
  static_assert(RW * KMAX % 64 == 0, "the wave's A block fills whole slots");
  // TB (B stored [N, K]): the workgroup's 256 columns x K, k-major
  __shared__ __attribute__((aligned(16))) float bt[TB ? KMAX : 1][TB ? 256 : 4];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  // one-dimensional grid: column group fastest, then row group
  const int64_t cgroups = (g.N + 255) / 256;
  const int64_t cg = static_cast<int64_t>(blockIdx.x) % cgroups, rg = static_cast<int64_t>(blockIdx.x) / cgroups;
  const int64_t c0 = cg * 256 + 4 * lane;
  const int64_t r0 = (rg * 4 + w) * RW;
  const int K = static_cast<int>(g.K);
  // the wave's block of A first (rows clamped into range, so a wave past
  // the last row loads valid memory and discards it)
  float av[SLOTS];
#pragma unroll
  for (int q = 0; q < SLOTS; ++q) {
    const int idx = q * 64 + lane;
    const int k = idx % KMAX;
    const int64_t row = r0 + idx / KMAX;
    const int64_t rr = row < g.M ? row : g.M - 1;
    const float v = a_elem<TA, PA>(g, rr, k < K ? k : K - 1);
    av[q] = (k < K && row < g.M) ? round_in<PREC>(v) : 0.0f;
  }
  if constexpr (TB) {
    // B[n * ldb + k] for the 256 columns from n_begin, read in memory order
    // (contiguous when ldb == K), stored k-major; zero past N
    const int64_t n_begin = cg * 256;
    const float *B = static_cast<const float *>(g.B);
    constexpr int PER = KMAX;  // 256 * K <= 256 * KMAX elements, PER per thread at most
    float v[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int e = i * 256 + static_cast<int>(threadIdx.x);
      const int c = e / K, k = e - c * K;
      const int64_t n = n_begin + c;
      v[i] = (c < 256 && n < g.N) ? B[n * g.ldb + k] : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int e = i * 256 + static_cast<int>(threadIdx.x);
      const int c = e / K, k = e - c * K;
      if (c < 256) bt[k][c] = v[i];
    }
    __syncthreads();
  }
  if (r0 >= g.M) return;  // uniform per wave
  float b[KMAX][4];
  const bool vb = !TB && (c0 + 3 < g.N) && (g.ldb % 4 == 0) && ((reinterpret_cast<uintptr_t>(g.B) & 15) == 0);
#pragma unroll
  for (int k = 0; k < KMAX; ++k) {
    const int kk = k < K ? k : K - 1;
    f4 t;
    if constexpr (TB) {
      t = *reinterpret_cast<const f4 *>(&bt[kk][4 * lane]);
    } else if (vb) {
      t = *reinterpret_cast<const f4 *>(static_cast<const float *>(g.B) + kk * g.ldb + c0);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) t[j] = b_elem<TB>(g, kk, (c0 + j < g.N) ? c0 + j : g.N - 1);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) b[k][j] = k < K ? round_in<PREC>(t[j]) : 0.0f;
  }
  float bias[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (g.bias != nullptr) {
#pragma unroll
    for (int j = 0; j < 4; ++j) bias[j] = g.bias[(c0 + j < g.N) ? c0 + j : g.N - 1];
  }
  const bool full = c0 + 3 < g.N;
  // the row loop, compiled apart with and without reads of C: a read of C
  // inside the loop would make every row wait for all of the wave's stores
  auto rows = [&](auto acc_c) {
    constexpr bool ACC = decltype(acc_c)::value;
#pragma unroll
    for (int i = 0; i < RW; ++i) {
      const int64_t r = r0 + i;
      if (r >= g.M) break;  // uniform
      float o[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int k = 0; k < KMAX; ++k) {
        const int q = i * KMAX + k;
        const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(av[q / 64]), q % 64));
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] = __builtin_fmaf(a, b[k][j], o[j]);
      }
      float *dst = g.C + r * g.ldc + c0;
      if (VC && full) {
        f4 prev = {0.0f, 0.0f, 0.0f, 0.0f};
        if constexpr (ACC) prev = *reinterpret_cast<const f4 *>(dst);
        f4 v;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float t = ACC ? prev[j] + o[j] : o[j];
          if (g.bias != nullptr) t = t + bias[j];
          v[j] = t;
        }
        // streamed past the caches: the consumer (the next layer's reverse
        // pass) reads it once, and 105 MB written so at B = 256, T = 50
        // took 24.3 instead of 27.0 us, the pair 68.0 instead of 73.2 us
        __builtin_nontemporal_store(v, reinterpret_cast<f4 *>(dst));
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (c0 + j < g.N) {
            float t = o[j];
            if constexpr (ACC) t = dst[j] + t;
            if (g.bias != nullptr) t = t + bias[j];
            dst[j] = t;
          }
        }
      }
    }
  };
  if (g.accumulate)
    rows(std::true_type{});
  else
    rows(std::false_type{});
}

// ---------------------------------------------------------------------------
// Large-tile GEMM for long operands.  A workgroup of 4 waves computes a
// 128 x 128 output tile; each wave owns a 64 x 64 quarter as 2 x 2 MFMA
// blocks, so every LDS fragment read feeds two MFMAs and a stage carries
// twice the flops per loaded byte of the 64 x 64 tile.  Operands are read as
// fp32 in either layout and land in LDS k-contiguous in the MFMA input type,
// always as 16-byte writes: an mn-contiguous operand is transposed in
// registers (a thread loads a 4 (mn) x KQ (k) block as KQ float4 rows and
// writes four k-vectors).  The k order of the MFMA chain is that of the
// 64 x 64 kernel, so both produce identical sums.
// ---------------------------------------------------------------------------
constexpr int kBig = 128;

template <int PREC, int BM = kBig, int BN = kBig>
struct BigStage {
  using T = typename Prec<PREC>::T;
  static constexpr int KS = Prec<PREC>::KS;                         // 128 bytes of k per row
  static constexpr int LD = KS + 16 / static_cast<int>(sizeof(T));  // + 16-byte pad
  alignas(16) T a[BM][LD];
  alignas(16) T b[BN][LD];
};

template <int PREC>
__device__ __forceinline__ void store_kvec(typename Prec<PREC>::T *dst, const float *x) {
  if constexpr (PREC == 1) {
    bf16x8 t;
#pragma unroll
    for (int j = 0; j < 8; ++j) t[j] = static_cast<__bf16>(x[j]);
    *reinterpret_cast<bf16x8 *>(dst) = t;
  } else {
    *reinterpret_cast<f4 *>(dst) = f4{x[0], x[1], x[2], x[3]};
  }
}

// One operand's stage: 128 (mn) x KS (k), loaded from global memory into
// one of D register sets (so up to D stages can be in flight) and stored
// to LDS as [mn][k] in the MFMA input type, always as 16-byte writes.
//  KC: element (mn, k) at base[mn * ld + k];  MN: at base[k * ld + mn].
// Source S = float: KC pieces are KQ consecutive k (one LDS vector); an MN
// thread loads a 4 (mn) x KQ (k) block as KQ float4 rows and writes four
// k-vectors.  S = uint16_t (bf16 bits, bf16 MFMA only): KC pieces are one
// 16-byte load of 8 k copied as is; an MN thread loads a 4 x 8 block as
// eight 8-byte rows and regroups the 16-bit halves into four 8-k vectors.
// Alignment: fp32 rows 16 bytes (ld % 4 == 0); bf16 KC rows 16 bytes
// (ld % 8 == 0), bf16 MN rows 8 bytes (ld % 4 == 0).  The per-piece
// addresses are computed once.  fast() loads a whole KS-wide stage with no
// guards (rows / columns past the tile edge come from a clamped in-range
// address); slow() guards every element and zero-fills (the partial last
// stage).
typedef unsigned int u4 __attribute__((ext_vector_type(4)));
typedef unsigned int u2 __attribute__((ext_vector_type(2)));

template <int PREC, bool KC, typename S, int D, int ROWS = kBig, int NT = 256>
struct BigLoader {
  static constexpr bool H = sizeof(S) == 2;
  static_assert(!H || PREC == 1, "bf16 operands need the bf16 MFMA");
  static constexpr int KS = Prec<PREC>::KS;
  static constexpr int KQ = 16 / static_cast<int>(sizeof(typename Prec<PREC>::T));  // k per LDS vector
  static constexpr int NP = KC ? ROWS * KS / KQ / NT : 1;                            // pieces per thread
  // MN: ROWS/4 column blocks x 8 k-groups; with more threads than blocks the
  // extra threads load and store a duplicate of block tid % MNB (same data)
  static constexpr int MNB = ROWS / 4 * 8;
  static_assert(KC ? (ROWS * KS / KQ) % NT == 0 : NT % MNB == 0 || MNB % NT == 0, "thread mapping");
  static_assert(KC || MNB <= NT, "one MN block per thread at most");
  // register set: KC -> per piece one u4 (bf16 in memory) or KQ words (fp32
  // in memory); MN -> 8 x u2 (bf16) or 4*KQ floats (fp32)
  static constexpr int NW = KC ? NP * (H ? 4 : KQ) : (H ? 16 : 4 * KQ);
  unsigned int v[D][NW];
  const S *q[NP];      // KC: piece row + its k offset; MN: k row kk, column mn
  int kk[NP];          // k offset of the piece (KC) / of the thread's k rows (MN)
  bool ok[NP];         // KC: piece row exists; MN: all 4 columns exist
  int mn0_;            // MN: first column of the thread's block
  int64_t ld, mn_lim;

  __device__ __forceinline__ void init(int tid, const void *base_, int64_t mn0, int64_t mn_total, int64_t ld_) {
    const S *base = static_cast<const S *>(base_);
    ld = ld_;
    mn_lim = mn_total - mn0;
    // fast() reads rows / columns past the tile edge from a clamped, in-range
    // address: they only feed outputs the epilogue discards
    if constexpr (KC) {
#pragma unroll
      for (int e = 0; e < NP; ++e) {
        const int idx = e * NT + tid;
        const int mn = idx / (KS / KQ);
        kk[e] = (idx % (KS / KQ)) * KQ;
        ok[e] = mn < mn_lim;
        const int64_t mc = ok[e] ? mn : mn_lim - 1;
        q[e] = base + (mn0 + mc) * ld + kk[e];
      }
    } else {
      const int tt = tid % MNB;
      mn0_ = (tt % (ROWS / 4)) * 4;
      kk[0] = (tt / (ROWS / 4)) * (H ? 8 : KQ);
      ok[0] = mn0_ + 3 < mn_lim;
      const int64_t mc = ok[0] ? mn0_ : ((mn_lim - 4) & ~static_cast<int64_t>(3));
      q[0] = base + kk[0] * ld + mn0 + mc;
    }
  }

  template <int d>
  __device__ __forceinline__ void fast(int64_t k0) {
    if constexpr (KC) {
#pragma unroll
      for (int e = 0; e < NP; ++e) {
        const S *src = q[e] + k0;
        if constexpr (H) {
          const u4 t = *reinterpret_cast<const u4 *>(src);
          v[d][4 * e] = t.x;
          v[d][4 * e + 1] = t.y;
          v[d][4 * e + 2] = t.z;
          v[d][4 * e + 3] = t.w;
        } else {
#pragma unroll
          for (int h = 0; h < KQ; h += 4) {
            const u4 t = *reinterpret_cast<const u4 *>(src + h);
            v[d][e * KQ + h] = t.x;
            v[d][e * KQ + h + 1] = t.y;
            v[d][e * KQ + h + 2] = t.z;
            v[d][e * KQ + h + 3] = t.w;
          }
        }
      }
    } else {
      const S *src = q[0] + k0 * ld;
      if constexpr (H) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const u2 t = *reinterpret_cast<const u2 *>(src + j * ld);
          v[d][2 * j] = t.x;
          v[d][2 * j + 1] = t.y;
        }
      } else {
#pragma unroll
        for (int j = 0; j < KQ; ++j) {
          const u4 t = *reinterpret_cast<const u4 *>(src + j * ld);
          v[d][4 * j] = t.x;
          v[d][4 * j + 1] = t.y;
          v[d][4 * j + 2] = t.z;
          v[d][4 * j + 3] = t.w;
        }
      }
    }
  }

  // column the MN fast path reads from (clamped at the tile edge)
  __device__ __forceinline__ int64_t mcol() const {
    return ok[0] ? mn0_ : ((mn_lim - 4) & ~static_cast<int64_t>(3));
  }

  // one element (raw bits, zero when out of range)
  __device__ __forceinline__ unsigned int elem(const S *src, bool in) const {
    if (!in) return 0u;
    if constexpr (H)
      return *src;
    else
      return __builtin_bit_cast(unsigned int, *src);
  }

  template <int d>
  __device__ __forceinline__ void slow(int64_t k0, int64_t ke) {
    if constexpr (KC) {
#pragma unroll
      for (int e = 0; e < NP; ++e) {
        const S *src = q[e] + k0;
        const int64_t k = k0 + kk[e];
        if constexpr (H) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const unsigned int lo = elem(src + 2 * i, ok[e] && k + 2 * i < ke);
            const unsigned int hi = elem(src + 2 * i + 1, ok[e] && k + 2 * i + 1 < ke);
            v[d][4 * e + i] = lo | (hi << 16);
          }
        } else {
#pragma unroll
          for (int i = 0; i < KQ; ++i) v[d][e * KQ + i] = elem(src + i, ok[e] && k + i < ke);
        }
      }
    } else {
      // unclamped column base (q[0] may be clamped)
      const S *src = q[0] + k0 * ld + (mn0_ - mcol());
      const int64_t kbase = k0 + kk[0];
      if constexpr (H) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          unsigned int e4[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) e4[i] = elem(src + j * ld + i, kbase + j < ke && mn0_ + i < mn_lim);
          v[d][2 * j] = e4[0] | (e4[1] << 16);
          v[d][2 * j + 1] = e4[2] | (e4[3] << 16);
        }
      } else {
#pragma unroll
        for (int j = 0; j < KQ; ++j)
#pragma unroll
          for (int i = 0; i < 4; ++i) v[d][4 * j + i] = elem(src + j * ld + i, kbase + j < ke && mn0_ + i < mn_lim);
      }
    }
  }

  // fast() addresses are valid: the tile has a row (KC) / four columns (MN)
  __device__ __forceinline__ bool fast_ok() const { return KC ? mn_lim >= 1 : mn_lim >= 4; }

  // move to the same tile of another operand laid out like this one, d
  // elements further on
  __device__ __forceinline__ void shift(int64_t d) {
#pragma unroll
    for (int e = 0; e < NP; ++e) q[e] += d;
  }

  template <int d>
  __device__ __forceinline__ void store(typename Prec<PREC>::T (*dst)[BigStage<PREC>::LD]) const {
    if constexpr (KC) {
      const int tid = threadIdx.x;
#pragma unroll
      for (int e = 0; e < NP; ++e) {
        const int mn = (e * NT + tid) / (KS / KQ);
        if constexpr (H) {
          *reinterpret_cast<u4 *>(&dst[mn][kk[e]]) = u4{v[d][4 * e], v[d][4 * e + 1], v[d][4 * e + 2], v[d][4 * e + 3]};
        } else {
          float x[KQ];
#pragma unroll
          for (int i = 0; i < KQ; ++i) x[i] = __builtin_bit_cast(float, v[d][e * KQ + i]);
          store_kvec<PREC>(&dst[mn][kk[e]], x);
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if constexpr (H) {
          // v[2j] = {mn0 | mn1 << 16}, v[2j+1] = {mn2 | mn3 << 16} at k = j;
          // the vector for column i packs k = 2w, 2w + 1 into word w
          unsigned int w4[4];
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            const unsigned int a = v[d][2 * (2 * w) + (i >> 1)];
            const unsigned int b = v[d][2 * (2 * w + 1) + (i >> 1)];
            w4[w] = (i & 1) ? ((a >> 16) | (b & 0xffff0000u)) : ((a & 0xffffu) | (b << 16));
          }
          *reinterpret_cast<u4 *>(&dst[mn0_ + i][kk[0]]) = u4{w4[0], w4[1], w4[2], w4[3]};
        } else {
          float x[KQ];
#pragma unroll
          for (int j = 0; j < KQ; ++j) x[j] = __builtin_bit_cast(float, v[d][4 * j + i]);
          store_kvec<PREC>(&dst[mn0_ + i][kk[0]], x);
        }
      }
    }
  }
};

// One stage of a wave's WM x WN blocks of 32 x 32 (rows 32*WM*wm + 32*i,
// columns 32*WN*wn + 32*j): per k step, WM + WN fragment reads feed WM*WN
// MFMAs.
template <int PREC, class ST, int WM, int WN>
__device__ __forceinline__ void big_mfma(const ST &st, int wm, int wn, int lane, f32x16 (&acc)[WM][WN]) {
  constexpr int KS = Prec<PREC>::KS, KM = Prec<PREC>::KM, KV = Prec<PREC>::KV;
  const int r = 32 * WM * wm + (lane & 31), c = 32 * WN * wn + (lane & 31), kq = (lane >> 5) * KV;
#pragma unroll
  for (int kk = 0; kk < KS; kk += KM) {
    if constexpr (PREC == 1) {
      bf16x8 a[WM], b[WN];
#pragma unroll
      for (int i = 0; i < WM; ++i) a[i] = *reinterpret_cast<const bf16x8 *>(&st.a[r + 32 * i][kk + kq]);
#pragma unroll
      for (int j = 0; j < WN; ++j) b[j] = *reinterpret_cast<const bf16x8 *>(&st.b[c + 32 * j][kk + kq]);
#pragma unroll
      for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < WN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
    } else if (kk % 8 == 0) {
      // 16-byte fragment groups of 8 k, the k order of mfma_stage
      const int kg = (lane >> 5) * 4;
      f4 a[WM], b[WN];
#pragma unroll
      for (int i = 0; i < WM; ++i) a[i] = *reinterpret_cast<const f4 *>(&st.a[r + 32 * i][kk + kg]);
#pragma unroll
      for (int j = 0; j < WN; ++j) b[j] = *reinterpret_cast<const f4 *>(&st.b[c + 32 * j][kk + kg]);
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int i = 0; i < WM; ++i)
#pragma unroll
          for (int j = 0; j < WN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i][e], b[j][e], acc[i][j], 0, 0, 0);
    }
  }
}

template <int PREC, int DEPTH, class LA, class LB, class ST, int WM, int WN>
__device__ __forceinline__ void big_kloop(LA &la, LB &lb, int64_t kb, int64_t ke, ST (&st)[2], int wm, int wn,
                                          int lane, f32x16 (&acc)[WM][WN]) {
  constexpr int KS = Prec<PREC>::KS;
  if (kb >= ke) return;
  const int64_t nfull = (ke - kb) / KS;
  if (la.fast_ok() && lb.fast_ok() && nfull > 0) {
    const int64_t klast = kb + (nfull - 1) * KS;
    auto kof = [&](int64_t stage) { return stage < nfull ? kb + stage * KS : klast; };
    la.template fast<0>(kb);
    lb.template fast<0>(kb);
    la.template store<0>(st[0].a);
    lb.template store<0>(st[0].b);
    if constexpr (DEPTH == 1) {
      __syncthreads();
      for (int64_t sg = 0; sg < nfull; ++sg) {
        const int buf = sg & 1;
        la.template fast<0>(kof(sg + 1));
        lb.template fast<0>(kof(sg + 1));
        big_mfma<PREC, ST, WM, WN>(st[buf], wm, wn, lane, acc);
        if (sg + 1 < nfull) {
          la.template store<0>(st[buf ^ 1].a);
          lb.template store<0>(st[buf ^ 1].b);
        }
        __syncthreads();
      }
    } else {
      la.template fast<1>(kof(1));
      lb.template fast<1>(kof(1));
      __syncthreads();
      for (int64_t sg = 0; sg < nfull; sg += 2) {
        // stage sg in st[0]; set 1 holds stage sg + 1; fetch sg + 2 into set 0
        la.template fast<0>(kof(sg + 2));
        lb.template fast<0>(kof(sg + 2));
        big_mfma<PREC, ST, WM, WN>(st[0], wm, wn, lane, acc);
        if (sg + 1 < nfull) {
          la.template store<1>(st[1].a);
          lb.template store<1>(st[1].b);
        }
        __syncthreads();
        if (sg + 1 >= nfull) break;
        // stage sg + 1 in st[1]; set 0 holds stage sg + 2; fetch sg + 3 into set 1
        la.template fast<1>(kof(sg + 3));
        lb.template fast<1>(kof(sg + 3));
        big_mfma<PREC, ST, WM, WN>(st[1], wm, wn, lane, acc);
        if (sg + 2 < nfull) {
          la.template store<0>(st[0].a);
          lb.template store<0>(st[0].b);
        }
        __syncthreads();
      }
    }
    kb += nfull * KS;
    if (kb >= ke) return;
  }
  // guarded stages: the partial last stage, or every stage of a too-narrow operand
  for (int64_t k0 = kb; k0 < ke; k0 += KS) {
    la.template slow<0>(k0, ke);
    lb.template slow<0>(k0, ke);
    la.template store<0>(st[0].a);
    lb.template store<0>(st[0].b);
    __syncthreads();
    big_mfma<PREC, ST, WM, WN>(st[0], wm, wn, lane, acc);
    __syncthreads();
  }
}

// register sets per operand: 2, except fp32 operands feeding the bf16 MFMA
template <int PREC, typename S>
constexpr int big_depth() {
  return (PREC == 1 && sizeof(S) == 4) ? 1 : 2;
}

// Workgroup -> output tile.  Consecutive workgroup ids go round-robin to the
// 8 XCDs (each with its own L2), so when the grid is a multiple of 8 each
// XCD is handed a contiguous run of logical tiles; logical tiles walk groups
// of 8 tile rows column by column, so a run shares A rows and B columns.
__device__ __forceinline__ void big_tile(uint32_t bid, uint32_t nblk, uint32_t tiles_m, uint32_t tiles_n, int64_t &tm,
                                         int64_t &tn) {
  uint32_t t = bid;
  if (nblk % 8 == 0) t = (bid % 8) * (nblk / 8) + bid / 8;
  constexpr uint32_t G = 8;
  const uint32_t per_group = G * tiles_n;
  const uint32_t group = t / per_group, first = group * G;
  const uint32_t gs = (tiles_m - first < G) ? tiles_m - first : G;
  const uint32_t in = t - group * per_group;
  // wave-uniform by construction; pinned to scalar registers so the tile
  // bounds below branch on scalars
  tm = __builtin_amdgcn_readfirstlane(first + in % gs);
  tn = __builtin_amdgcn_readfirstlane(in / gs);
}

// Writes a wave's WM x WN blocks of 32 x 32 to C (or to the split-K
// workspace slice of blockIdx.y).  The per-element form measures faster
// here than store_acc's.
template <int WM, int WN>
__device__ __forceinline__ void big_epilogue(const GemmArgs &g, const f32x16 (&acc)[WM][WN], int64_t m0, int64_t n0,
                                             int wm, int wn, int lane) {
#pragma unroll
  for (int j = 0; j < WN; ++j) {
    const int64_t col = n0 + 32 * WN * wn + 32 * j + (lane & 31);
    if (col >= g.N) continue;
#pragma unroll
    for (int i = 0; i < WM; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = m0 + 32 * WM * wm + 32 * i + acc_row(r, lane);
        if (row >= g.M) continue;
        if (g.splits > 1) {
          g.ws[(static_cast<int64_t>(blockIdx.y) * g.M + row) * g.N + col] = acc[i][j][r];
        } else {
          float *dst = g.C + row * g.ldc + col;
          float v = g.accumulate ? *dst + acc[i][j][r] : acc[i][j][r];
          if (g.bias != nullptr) v = v + g.bias[col];
          *dst = v;
        }
      }
    }
  }
}

// BM x BN output tile; each wave owns WM x WN blocks of 32 x 32 (the
// launched kernels: 2 x 2, one wave per 64 x 64 quarter).  MP: bf16 operands
// summing g.parts B parts (a separate instantiation, so the one-part kernels
// keep their registers).  Wave tiles above 2 x 2 would run one wave per SIMD
// with up to 512 registers; a 256 x 128 tile of four 128 x 64 waves
// measured slower than this one (612 against 703 TFLOP/s at 8192 x 4096 x
// 3072 bf16), so none is launched.
template <int PREC, bool TA, bool TB, typename S, int BM, int BN, bool MP = false, int WM = 2, int WN = 2>
__global__ __launch_bounds__(64 * (BM / (32 * WM)) * (BN / (32 * WN)))
__attribute__((amdgpu_waves_per_eu(WM * WN > 4 ? 1 : 2))) void gemm_big(GemmArgs g) {
  constexpr int WGN = BN / (32 * WN);  // waves across the tile's columns
  constexpr int NT = 64 * (BM / (32 * WM)) * WGN;
  __shared__ BigStage<PREC, BM, BN> st[2];
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6), wm = w / WGN, wn = w % WGN;
  const uint32_t tiles_m = static_cast<uint32_t>((g.M + BM - 1) / BM);
  const uint32_t tiles_n = static_cast<uint32_t>((g.N + BN - 1) / BN);
  int64_t tm, tn;
  big_tile(blockIdx.x, gridDim.x, tiles_m, tiles_n, tm, tn);
  const int64_t m0 = tm * BM, n0 = tn * BN;
  const int64_t kb = static_cast<int64_t>(blockIdx.y) * g.kchunk;
  const int64_t ke = (kb + g.kchunk < g.K) ? kb + g.kchunk : g.K;

  constexpr int D = big_depth<PREC, S>();
  BigLoader<PREC, !TA, S, D, BM, NT> la;
  BigLoader<PREC, TB, S, D, BN, NT> lb;
  la.init(tid, g.A, m0, g.M, g.lda);
  lb.init(tid, g.B, n0, g.N, g.ldb);

  f32x16 acc[WM][WN];
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int j = 0; j < WN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
  if constexpr (MP) {
    static_assert(sizeof(S) == 2, "B parts are a bf16-operand feature");
    // the same k range of each B part in turn
    for (int p = 0; p < g.parts; ++p) {
      if (p > 0) lb.shift(g.b_part);
      big_kloop<PREC, D>(la, lb, kb, ke, st, wm, wn, lane, acc);
    }
  } else {
    big_kloop<PREC, D>(la, lb, kb, ke, st, wm, wn, lane, acc);
  }

  big_epilogue<WM, WN>(g, acc, m0, n0, wm, wn, lane);
}

// ---------------------------------------------------------------------------
// bf16 product with both operands k-contiguous (A [M, K], B [N, K], rows
// 16-byte aligned, K a multiple of 64), staged by direct global -> LDS loads.
//
// Each 16-byte piece of a stage (64 k of a row) goes from HBM / L2 straight
// into LDS (global_load_lds_dwordx4): no staging registers and no LDS write
// instructions, and the only wait on the loads is the vmcnt before each
// stage's barrier.  One wave's load fills 1 KB of LDS in lane order, so rows
// are unpadded (128 bytes); the chunk of logical k-group c (8 k) of tile row
// r sits at position c ^ dma_swz(r), which keeps the fragment reads
// (32 rows x one k-group per half-wave) on distinct banks.
//
// NS stages in LDS; per stage: wait for the stage's loads and barrier; read
// the fragments of the stage's first k step; issue the loads of stage
// s + NS - 1 into the buffer stage s - 1 used (whose readers all passed the
// barrier); run the MFMAs of each k step with the next k step's fragment
// reads in flight (two register sets of one k step: against reading the
// stage in halves, 8192 x 4096 x 3 x 1024 on 256 x 256 tiles 188 -> 178
// us, 218 -> 194 VGPRs, the same bits).  Against register staging at 8192 x 4096 x 3 x
// 1024 (256 x 128 tiles): 221 -> 208 us; on 128 x 128 tiles (two stages,
// two workgroups per CU) it measured mixed (12800 x 784 x 2048: 64 -> 69
// us), so those keep register staging.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int dma_swz(int r) { return (r ^ (r >> 3)) & 7; }

// Scheduling of one k step of the direct-load kernels: the next k step's
// NG fragment reads (RPG LDS reads each) are placed one group after each
// of the first NG of this step's NM MFMAs, the rest of the MFMAs after.
// Left to itself the scheduler issues all the reads after the last MFMA,
// so each k step starts by waiting for LDS (8192 x 4096 x 3 x 1024 on
// 256 x 256 tiles: 165 -> 156 us, the same bits).
template <int NM, int NG, int RPG>
__device__ __forceinline__ void interleave_reads() {
  static_assert(NG <= NM, "one read group per MFMA at most");
#pragma unroll
  for (int q = 0; q < NG; ++q) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);    // one MFMA
    __builtin_amdgcn_sched_group_barrier(0x100, RPG, 0);  // then RPG LDS reads
  }
  if constexpr (NM > NG) __builtin_amdgcn_sched_group_barrier(0x008, NM - NG, 0);
}

typedef __attribute__((address_space(3))) void lds_void;

// Loads of one operand tile: ROWS rows x 64 k, NP pieces per thread.
template <int ROWS, int NT>
struct DmaLoader {
  static constexpr int NP = ROWS * 8 / NT;
  static_assert(ROWS * 8 % NT == 0, "pieces per thread");
  // a wave-uniform base (scalar registers) and 32-bit byte offsets per
  // piece: the loads take the base + offset form, so a stage's addresses
  // cost no 64-bit vector arithmetic (8192 x 4096 x 3 x 1024 on 256 x 256
  // tiles: 4-8 % faster than 64-bit per-piece pointers; the host keeps
  // ROWS * ld * 2 bytes below 2^31)
  const uint16_t *base;
  uint32_t off[NP];
  int lds_off[NP];  // wave-uniform byte offset of the piece group in the tile

  __device__ __forceinline__ void init(int tid, int w, const uint16_t *b, int64_t mn0, int64_t mn_total,
                                       int64_t ld) {
    const int64_t lim = mn_total - mn0;
    base = b + mn0 * ld;
#pragma unroll
    for (int e = 0; e < NP; ++e) {
      const int idx = e * NT + tid;
      const int row = idx >> 3, pos = idx & 7;
      const int c = pos ^ dma_swz(row);
      // rows past the edge read the last row: they feed discarded outputs
      const int64_t rc = row < lim ? row : lim - 1;
      off[e] = static_cast<uint32_t>((rc * ld + 8 * c) * 2);
      lds_off[e] = (e * NT + w * 64) * 16;
    }
  }
  // The loads are issued from inline assembly, outside the compiler's
  // accounting of LDS writes in flight: the kernel waits for them itself
  // (vmcnt before each stage's barrier, and vmcnt(0) after the last stage,
  // before the epilogue's own loads).  M0 holds the wave's LDS base during
  // each load.
  __device__ __forceinline__ void issue(char *tile, int64_t k0) const {
    const uint16_t *p = base + k0;
#pragma unroll
    for (int e = 0; e < NP; ++e) {
      const uint32_t dst = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_void *)(tile + lds_off[e])));
      // M0 is the compiler's: saved and restored around the load (which
      // reads it at issue)
      uint32_t m0_saved;
      asm volatile(
          "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2\n\ts_mov_b32 m0, %0"
          : "=&s"(m0_saved)
          : "v"(off[e]), "s"(p), "s"(dst)
          : "memory");
    }
  }
  __device__ __forceinline__ void shift(int64_t d) { base += d; }
};

template <int BM, int BN, bool MP, int NS, int WM = 2, int WN = 2>
__global__ __launch_bounds__(64 * (BM / (32 * WM)) * (BN / (32 * WN))) __attribute__((amdgpu_waves_per_eu(2))) void gemm_dma(
    GemmArgs g) {
  constexpr int WGN = BN / (32 * WN);
  constexpr int NT = 64 * (BM / (32 * WM)) * WGN;
  constexpr int TILE = (BM + BN) * 128;  // bytes of one stage
  // loads per thread per stage; a stage's wait leaves the NS - 2 later
  // stages' loads in flight
  constexpr int NL = (BM + BN) * 8 / NT;
  static_assert(NS == 2 || NS == 3, "two or three stages");
  // one array per stage, so every access names its stage's array: the
  // compiler then sees that a stage's reads and the loads in flight into
  // the other stages do not alias, and leaves those loads in flight
  __shared__ __attribute__((aligned(1024))) char l0[TILE];
  __shared__ __attribute__((aligned(1024))) char l1[TILE];
  __shared__ __attribute__((aligned(1024))) char l2[NS > 2 ? TILE : 16];
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6), wm = w / WGN, wn = w % WGN;
  const uint32_t tiles_m = static_cast<uint32_t>((g.M + BM - 1) / BM);
  const uint32_t tiles_n = static_cast<uint32_t>((g.N + BN - 1) / BN);
  int64_t tm, tn;
  big_tile(blockIdx.x, gridDim.x, tiles_m, tiles_n, tm, tn);
  const int64_t m0 = tm * BM, n0 = tn * BN;
  const int64_t kb = static_cast<int64_t>(blockIdx.y) * g.kchunk;
  const int64_t ke = (kb + g.kchunk < g.K) ? kb + g.kchunk : g.K;

  DmaLoader<BM, NT> la;
  DmaLoader<BN, NT> lb;
  la.init(tid, w, static_cast<const uint16_t *>(g.A), m0, g.M, g.lda);
  lb.init(tid, w, static_cast<const uint16_t *>(g.B), n0, g.N, g.ldb);

  // fragment byte offsets in a stage: A rows, then B rows after BM rows
  int fa[WM][4], fb[WN][4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    const int c = 2 * ks + (lane >> 5);
#pragma unroll
    for (int i = 0; i < WM; ++i) {
      const int r = 32 * WM * wm + 32 * i + (lane & 31);
      fa[i][ks] = r * 128 + ((c ^ dma_swz(r)) << 4);
    }
#pragma unroll
    for (int j = 0; j < WN; ++j) {
      const int r = 32 * WN * wn + 32 * j + (lane & 31);
      fb[j][ks] = (BM + r) * 128 + ((c ^ dma_swz(r)) << 4);
    }
  }

  f32x16 acc[WM][WN];
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int j = 0; j < WN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int64_t per = (ke - kb) / 64;  // stages per part (the host checks 64 | K and 64 | kchunk)
  const int64_t total = MP ? per * g.parts : per;
  if (per > 0) {
    int64_t k_next = kb, left = per;  // next stage to load: k and stages left in its part
    auto issue = [&](char *tile) {
      la.issue(tile, k_next);
      lb.issue(tile + BM * 128, k_next);
      k_next += 64;
      if (MP && --left == 0) {
        // next part: the same k range of the following B plane
        left = per;
        k_next = kb;
        lb.shift(g.b_part);
      }
    };
    // stage s: wait for its loads, barrier, read its fragments from cur,
    // load stage s + NS - 1 into nxt (read in iteration s - 1, whose readers
    // have all passed the barrier with their fragments in registers),
    // multiply.  (Reading stage s + 1 during stage s's MFMAs needs a second
    // fragment set, which spills the load pointers at two waves per SIMD.)
    auto step = [&](const char *cur, char *nxt, int64_t s) {
      if (NS > 2 && s + 1 < total)
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(NL * (NS - 2)) : "memory");
      else
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      // the loads still in flight target other stages; lgkmcnt(0) retires
      // this wave's LDS reads of the previous stage, whose buffer the
      // direct loads issued after this barrier overwrite
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      // the fragments of k step ks + 1 are read while step ks multiplies
      // (two register sets of one k step each)
      bf16x8 a[2][WM], b[2][WN];
      auto rd = [&](int ks, int set) {
#pragma unroll
        for (int i = 0; i < WM; ++i) a[set][i] = *reinterpret_cast<const bf16x8 *>(cur + fa[i][ks]);
#pragma unroll
        for (int j = 0; j < WN; ++j) b[set][j] = *reinterpret_cast<const bf16x8 *>(cur + fb[j][ks]);
      };
      rd(0, 0);
      if (s + NS - 1 < total) issue(nxt);
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        if (ks + 1 < 4) rd(ks + 1, (ks + 1) & 1);
#pragma unroll
        for (int i = 0; i < WM; ++i)
#pragma unroll
          for (int j = 0; j < WN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[ks & 1][i], b[ks & 1][j], acc[i][j], 0, 0, 0);
        if (ks + 1 < 4) interleave_reads<WM * WN, WM + WN, 1>();
      }
    };
    issue(l0);
    if constexpr (NS > 2) {
      if (total > 1) issue(l1);
      for (int64_t s = 0; s < total; s += 3) {
        step(l0, l2, s);
        if (s + 1 < total) step(l1, l0, s + 1);
        if (s + 2 < total) step(l2, l1, s + 2);
      }
    } else {
      for (int64_t s = 0; s < total; s += 2) {
        step(l0, l1, s);
        if (s + 1 < total) step(l1, l0, s + 1);
      }
    }
  }
  big_epilogue<WM, WN>(g, acc, m0, n0, wm, wn, lane);
}

// ---------------------------------------------------------------------------
// bf16 product with both operands mn-contiguous (A stored [K, M], B stored
// [K, N]: the weight-gradient products x^T G), 128 x 128 tiles staged by
// direct global -> LDS loads.
//
// A stage holds 64 k rows of each operand as stored: [64][128] bf16, 256
// bytes a row.  The MFMA fragments (8 consecutive k of one column per lane)
// come out of LDS through the transposing read ds_read_b64_tr_b16: within
// each 16-lane group, lane r reads the 4 values at its own address and lane
// i receives value i % 4 of lanes i / 4, i / 4 + 4, i / 4 + 8, i / 4 + 12.
// So lane r of a group points at row kb + r / 4, columns n0 + 4 (r % 4) ..
// + 3, and lane i receives rows kb .. kb + 3 of column n0 + i; two reads
// (kb and kb + 4) make the fragment.  The 16-byte chunk of columns 8c ..
// 8c + 7 of row k sits at position c ^ (4 (k & 3)), which puts the 32
// lanes of two groups (4 rows x 2 chunk pairs) on distinct banks.
// A partial last stage (K, or a K split, not a multiple of 64) is loaded
// with guarded vector loads (zeros past the end) and written with LDS
// stores.
// ---------------------------------------------------------------------------
typedef short v4s __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4s lds_v4s;

__device__ __forceinline__ int mn_swz(int k) { return 4 * (k & 3); }

// Loads of one mn-contiguous operand tile: 64 k rows x COLS columns (COLS /
// 8 pieces of 16 bytes a row) over NT threads.
template <int COLS, int NT>
struct DmaLoaderMN {
  static constexpr int CPR = COLS / 8;  // pieces per row
  static constexpr int NP = 64 * CPR / NT;
  static_assert(64 * CPR % NT == 0, "pieces per thread");
  // wave-uniform base and 32-bit byte offsets of the pieces at k = 0 of
  // the stage (row kk[e]), as DmaLoader (the host keeps 64 * ld plus the
  // row length below 2^30 elements)
  const uint16_t *base;
  uint32_t off[NP];
  int kk[NP];
  int lds_off[NP];
  int64_t ld;

  __device__ __forceinline__ void init(int tid, int w, const uint16_t *b, int64_t mn0, int64_t mn_total,
                                       int64_t ld_) {
    ld = ld_;
    base = b;
#pragma unroll
    for (int e = 0; e < NP; ++e) {
      const int idx = e * NT + tid;
      const int k = idx / CPR, pos = idx % CPR;
      const int c = pos ^ mn_swz(k);
      // columns past the edge read the last whole piece (the host checks
      // that the column count is a multiple of 8): they feed discarded
      // outputs
      int64_t col = mn0 + 8 * c;
      if (col + 8 > mn_total) col = mn_total - 8;
      kk[e] = k;
      off[e] = static_cast<uint32_t>((k * ld + col) * 2);
      lds_off[e] = (e * NT + w * 64) * 16;
    }
  }
  // a whole stage: rows k0 .. k0 + 63
  __device__ __forceinline__ void issue(char *tile, int64_t k0) const {
    const uint16_t *p = base + k0 * ld;
#pragma unroll
    for (int e = 0; e < NP; ++e) {
      const uint32_t dst = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_void *)(tile + lds_off[e])));
      uint32_t m0_saved;
      asm volatile(
          "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2\n\ts_mov_b32 m0, %0"
          : "=&s"(m0_saved)
          : "v"(off[e]), "s"(p), "s"(dst)
          : "memory");
    }
  }
  // a partial stage: rows k0 .. ke - 1, zeros after
  __device__ __forceinline__ void tail(char *tile, int64_t k0, int64_t ke) const {
    const int lane = threadIdx.x & 63;
    const char *p = reinterpret_cast<const char *>(base + k0 * ld);
#pragma unroll
    for (int e = 0; e < NP; ++e) {
      u4 v = {0u, 0u, 0u, 0u};
      if (k0 + kk[e] < ke) v = *reinterpret_cast<const u4 *>(p + off[e]);
      *reinterpret_cast<u4 *>(tile + lds_off[e] + lane * 16) = v;
    }
  }
  __device__ __forceinline__ void shift(int64_t d) { base += d; }
};

template <bool MP, int NS, int BM = 128, int BN = 128, int WM = 2, int WN = 2>
__global__ __launch_bounds__(64 * (BM / (32 * WM)) * (BN / (32 * WN))) __attribute__((amdgpu_waves_per_eu(2))) void gemm_dma_mn(
    GemmArgs g) {
  constexpr int WGN = BN / (32 * WN);
  constexpr int NT = 64 * (BM / (32 * WM)) * WGN;
  constexpr int RA = 2 * BM, RB = 2 * BN;    // bytes of an A row and of a B row
  constexpr int TILE = 64 * (RA + RB);       // bytes of one stage: A rows, then B rows
  using LA = DmaLoaderMN<BM, NT>;
  using LB = DmaLoaderMN<BN, NT>;
  constexpr int NL = LA::NP + LB::NP;
  static_assert(NS == 2 || NS == 3, "two or three stages");
  __shared__ __attribute__((aligned(1024))) char l0[TILE];
  __shared__ __attribute__((aligned(1024))) char l1[TILE];
  __shared__ __attribute__((aligned(1024))) char l2[NS > 2 ? TILE : 16];
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6), wm = w / WGN, wn = w % WGN;
  const uint32_t tiles_m = static_cast<uint32_t>((g.M + BM - 1) / BM);
  const uint32_t tiles_n = static_cast<uint32_t>((g.N + BN - 1) / BN);
  int64_t tm, tn;
  big_tile(blockIdx.x, gridDim.x, tiles_m, tiles_n, tm, tn);
  const int64_t m0 = tm * BM, n0 = tn * BN;
  const int64_t kb = static_cast<int64_t>(blockIdx.y) * g.kchunk;
  const int64_t ke = (kb + g.kchunk < g.K) ? kb + g.kchunk : g.K;

  LA la;
  LB lb;
  la.init(tid, w, static_cast<const uint16_t *>(g.A), m0, g.M, g.lda);
  lb.init(tid, w, static_cast<const uint16_t *>(g.B), n0, g.N, g.ldb);

  // transposing-read byte offsets within a stage, per k-step (16 k) and
  // half (k offsets 0..3 / 4..7): lane r of 16-lane group gq points at row
  // 16 ks + 8 (gq >> 1) + 4 h + r / 4, columns c0 + 16 (gq & 1) + 4 (r % 4)
  const int gq = lane >> 4, r16 = lane & 15;
  int fa[WM][4][2], fb[WN][4][2];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int k = 16 * ks + 8 * (gq >> 1) + 4 * h + (r16 >> 2);
#pragma unroll
      for (int i = 0; i < WM; ++i) {
        const int col = 32 * (WM * wm + i) + 16 * (gq & 1) + 4 * (r16 & 3);
        fa[i][ks][h] = k * RA + (((col >> 3) ^ mn_swz(k)) << 4) + (col & 7) * 2;
      }
#pragma unroll
      for (int j = 0; j < WN; ++j) {
        const int col = 32 * (WN * wn + j) + 16 * (gq & 1) + 4 * (r16 & 3);
        fb[j][ks][h] = 64 * RA + k * RB + (((col >> 3) ^ mn_swz(k)) << 4) + (col & 7) * 2;
      }
    }

  f32x16 acc[WM][WN];
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int j = 0; j < WN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int64_t per = (ke - kb + 63) / 64;  // stages per part, the last maybe partial
  const int64_t total = MP ? per * g.parts : per;
  if (per > 0) {
    int64_t k_next = kb, left = per;
    auto issue = [&](char *tile) {
      if (k_next + 64 <= ke) {
        la.issue(tile, k_next);
        lb.issue(tile + 64 * RA, k_next);
      } else {
        la.tail(tile, k_next, ke);
        lb.tail(tile + 64 * RA, k_next, ke);
      }
      k_next += 64;
      if (MP && --left == 0) {
        left = per;
        k_next = kb;
        lb.shift(g.b_part);
      }
    };
    auto frag = [&](const char *cur, int off0, int off1) {
      const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s *)((lds_void *)(cur + off0)));
      const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s *)((lds_void *)(cur + off1)));
      typedef short v8s __attribute__((ext_vector_type(8)));
      const v8s v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      return __builtin_bit_cast(bf16x8, v);
    };
    // a partial stage (the last of a part) is loaded synchronously, so the
    // loads in flight after it are the earlier stages': no allowance then
    const bool ragged = (ke - kb) % 64 != 0;
    auto is_tail = [&](int64_t t) { return ragged && (t % per) == per - 1; };
    auto step = [&](const char *cur, char *nxt, int64_t s) {
      if (NS > 2 && s + 1 < total && !is_tail(s + 1))
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(NL * (NS - 2)) : "memory");
      else
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      // a tail stage was written with LDS stores: lgkmcnt(0) covers them
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      // k step ks + 1's fragments are read while step ks multiplies
      bf16x8 a[2][WM], b[2][WN];
      auto rd = [&](int ks, int set) {
#pragma unroll
        for (int i = 0; i < WM; ++i) a[set][i] = frag(cur, fa[i][ks][0], fa[i][ks][1]);
#pragma unroll
        for (int j = 0; j < WN; ++j) b[set][j] = frag(cur, fb[j][ks][0], fb[j][ks][1]);
      };
      rd(0, 0);
      if (s + NS - 1 < total) issue(nxt);
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        if (ks + 1 < 4) rd(ks + 1, (ks + 1) & 1);
#pragma unroll
        for (int i = 0; i < WM; ++i)
#pragma unroll
          for (int j = 0; j < WN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[ks & 1][i], b[ks & 1][j], acc[i][j], 0, 0, 0);
        if (ks + 1 < 4) interleave_reads<WM * WN, WM + WN, 2>();  // two transposing reads a fragment
      }
    };
    issue(l0);
    if constexpr (NS > 2) {
      if (total > 1) issue(l1);
      for (int64_t s = 0; s < total; s += 3) {
        step(l0, l2, s);
        if (s + 1 < total) step(l1, l0, s + 1);
        if (s + 2 < total) step(l2, l1, s + 2);
      }
    } else {
      for (int64_t s = 0; s < total; s += 2) {
        step(l0, l1, s);
        if (s + 1 < total) step(l1, l0, s + 1);
      }
    }
  }
  big_epilogue<WM, WN>(g, acc, m0, n0, wm, wn, lane);
}

// ---------------------------------------------------------------------------
// Fused current GEMM + LIF recurrence.
// ---------------------------------------------------------------------------
struct LinArgs {
  const float *x;     // [T, B, F]
  const float *w;     // [F, N]
  const uint16_t *xh; // bf16 operands instead of x / w: [T, B, F] and
  const uint16_t *wt; //   the transposed weight [N, F]
  const float *bias;  // [N] or null
  const float *m0;    // [B, N] or null (zeros)
  float *m_final;     // [B, N] or null
  float *spikes;      // [T, B, N] or null (absolute t)
  float *pre;         // [t_end - t_begin, B, N] or null (relative t)
  int32_t *packed;    // [T, B, ceil(N/32)] or null (absolute t)
  float *rates;       // [B, N] or null: spike count / T_total
  float *ckpt;        // [ceil((t_end - t_begin)/ckpt_every), B, N] or null
  int64_t T, B, F, N, t_begin, t_end, ckpt_every, W;
  float decay, thr, reset, slope, rate_denominator;
  int rule;
};

// the outputs a launch writes: bits 1 pre, 2 spikes, 4 packed, 8
// checkpoints, 16 rates
__host__ __device__ int lin_outputs(const LinArgs &p) {
  return (p.pre != nullptr ? 1 : 0) | (p.spikes != nullptr ? 2 : 0) | (p.packed != nullptr ? 4 : 0) |
         (p.ckpt != nullptr ? 8 : 0) | (p.rates != nullptr ? 16 : 0);
}

// BT batch rows x 64 neurons per workgroup, 64/BT timesteps per chunk
// (GEMM rows r = j*BT + bb).  Wave w owns batch rows bb = w*Q .. w*Q+Q-1
// (Q = BT/4) of the recurrence; lane = neuron.
template <int PREC, int BT, bool VEC>
__global__ __launch_bounds__(256) void linear_lif_fwd(LinArgs p) {
  constexpr int CH = kTile / BT;
  constexpr int Q = BT / 4;
  __shared__ Stage<PREC> st[2];
  __shared__ float cur[kTile][kTile + 1];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, wm = w >> 1, wn = w & 1;
  const int64_t b0 = static_cast<int64_t>(blockIdx.y) * BT, n0 = static_cast<int64_t>(blockIdx.x) * kTile;
  const int64_t BN = p.B * p.N;

  const int64_t n = n0 + lane;
  float m[Q], cnt[Q];
  bool act[Q];
  int64_t flat[Q];
#pragma unroll
  for (int q = 0; q < Q; ++q) {
    const int64_t b = b0 + Q * w + q;
    act[q] = (b < p.B) && (n < p.N);
    flat[q] = b * p.N + n;
    m[q] = (act[q] && p.m0 != nullptr) ? p.m0[flat[q]] : 0.0f;
    cnt[q] = 0.0f;
  }
  const float bias_n = (p.bias != nullptr && n < p.N) ? p.bias[n] : 0.0f;
  int64_t next_ck = p.t_begin, ck_row = 0;

  TileLoader<PREC, false, VEC> lb;  // W [F, N]: rows of the B tile are neurons, contiguous for a fixed k
  lb.map_rowcontig(tid, p.w, n0, p.N, p.N);
  TileLoader<PREC, true, VEC> la;
  la.map_kcontig(tid);

  for (int64_t t0 = p.t_begin; t0 < p.t_end; t0 += CH) {
#pragma unroll
    for (int e = 0; e < TileLoader<PREC, true, VEC>::NV; ++e) {
      const int r = la.roff[e];
      const int64_t t = t0 + r / BT, b = b0 + r % BT;
      la.base[e] = (t < p.t_end && b < p.B) ? p.x + (t * p.B + b) * p.F : nullptr;
    }
    f32x16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
    tile_mma<PREC>(la, lb, 0, p.F, st, wm, wn, lane, acc);
#pragma unroll
    for (int r = 0; r < 16; ++r) cur[32 * wm + acc_row(r, lane)][32 * wn + (lane & 31)] = acc[r];
    __syncthreads();

#pragma unroll
    for (int j = 0; j < CH; ++j) {
      const int64_t t = t0 + j;
      if (t >= p.t_end) break;  // uniform
      if (p.ckpt != nullptr && t == next_ck) {
#pragma unroll
        for (int q = 0; q < Q; ++q)
          if (act[q]) p.ckpt[ck_row * BN + flat[q]] = m[q];
        ++ck_row;
        next_ck += p.ckpt_every;
      }
      bool s[Q];
#pragma unroll
      for (int q = 0; q < Q; ++q) {
        // input_current = x_t @ W + bias ; m' = m*decay + input_current
        const float c_in = cur[j * BT + Q * w + q][lane] + bias_n;
        float mp = m[q] * p.decay;
        mp = mp + c_in;
        bool sp;
        if (p.rule == MYELIN_RULE_THRESHOLD) {
          sp = mp >= p.thr;
        } else {
          const float c = p.slope * (mp - p.thr);
          sp = c >= 0.0f;
        }
        s[q] = act[q] && sp;
        if (act[q]) {
          if (p.pre != nullptr) p.pre[(t - p.t_begin) * BN + flat[q]] = mp;
          if (p.spikes != nullptr) __builtin_nontemporal_store(sp ? 1.0f : 0.0f, p.spikes + t * BN + flat[q]);
          m[q] = sp ? p.reset : mp;
          cnt[q] = cnt[q] + (sp ? 1.0f : 0.0f);
        }
      }
      if (p.packed != nullptr) {
#pragma unroll
        for (int q = 0; q < Q; ++q) {
          const uint64_t bits = __ballot(s[q]);
          const int64_t b = b0 + Q * w + q;
          const int64_t word = n0 / 32 + (lane >> 5);
          // every lane of a half-wave stores its half's word (one value to
          // one address): no lane-selected branch a step
          if (b < p.B && word < p.W)
            p.packed[(t * p.B + b) * p.W + word] =
                static_cast<int32_t>((lane & 32) ? (bits >> 32) : (bits & 0xffffffffu));
        }
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int q = 0; q < Q; ++q) {
    if (!act[q]) continue;
    if (p.m_final != nullptr) p.m_final[flat[q]] = m[q];
    if (p.rates != nullptr) p.rates[flat[q]] = cnt[q] / p.rate_denominator;
  }
}

// ---------------------------------------------------------------------------
// Reverse recurrence over a chunk from its saved pre-reset trace, producing
// G = dL/dm' (the gradient of the synaptic current) for the backward GEMMs.
// Same closed form and op order as the reference's hand-written backward
// (autograd.py:540-556):  d  = slope * sigma'(slope * (pre - thr))
//                         gp = gm * ((1 - s) + (reset - pre) * d) + g_spike * d
//                         gm = gp * decay
// g_spike is grad_spikes[t] (spike outputs) or grad_rates / T (rate outputs).
// gbias_acc[b, n] += sum over the chunk of gp (reduced over b later).
// ---------------------------------------------------------------------------
template <int SID>
__device__ __forceinline__ float sg_deriv(float c) {
  if constexpr (SID == MYELIN_SG_SIGMOID) {
    const float e = expf(-fabsf(c));
    const float d = 1.0f + e;
    return e / (d * d);
  } else if constexpr (SID == MYELIN_SG_FAST_SIGMOID) {
    // 0.5 / d^2 = 0.5 * (1 / d^2), both rounded once (a power of two)
    float d = 1.0f + fabsf(c);
    return 0.5f * myelin::recip_rn_or_zero(d * d);
  } else if constexpr (SID == MYELIN_SG_ATAN) {
    float s = 1.5707963267948966f * c;
    return 0.5f * myelin::recip_rn_or_zero(1.0f + s * s);
  } else if constexpr (SID == MYELIN_SG_TRIANGULAR) {
    float sg = (c > 0.0f) ? 1.0f : ((c < 0.0f) ? -1.0f : 0.0f);
    return fabsf(c) < 1.0f ? -sg : 0.0f;
  } else if constexpr (SID == MYELIN_SG_SUPERSPIKE) {
    float d = 1.0f + fabsf(c);
    return myelin::recip_rn_or_zero(d * d);
  } else {
    float z = c / 0.5f, r = c - 1.0f, l = c + 1.0f;
    return 0.47873073648171924f * expf(-0.5f * z * z) + 0.07978845608028655f * expf(-0.5f * r * r) +
           0.07978845608028655f * expf(-0.5f * l * l);
  }
}

// Fused current GEMM + LIF on the 128 x 128 engine.  The workgroup owns BT
// batch rows x 128 neurons and walks time in chunks of CH = 128 / BT steps:
// the chunk's 128 x 128 current tile (GEMM rows j*BT + bb) is computed over
// the full input width, parked in LDS over the (then idle) staging buffers,
// and consumed by the recurrence, wave w taking neurons 64*(w & 1) + lane
// of batch rows (w >> 1)*Q .. +Q-1 (Q = BT / 2).  Same arithmetic per step
// as linear_lif_fwd: m' = m*decay + (x_t W + bias).
// A operand of the fused kernel: 128 rows given by pointer (null = zero
// row), k-contiguous, S = float or bf16 bits, D register sets.  The caller
// sets row[] and `full` (every row present, uniform) for each time chunk.
template <int PREC, typename S, int D>
struct BigRowLoader {
  static constexpr bool H = sizeof(S) == 2;
  static_assert(!H || PREC == 1, "bf16 operands need the bf16 MFMA");
  static constexpr int KS = Prec<PREC>::KS;
  static constexpr int KQ = 16 / static_cast<int>(sizeof(typename Prec<PREC>::T));
  static constexpr int NP = kBig * KS / KQ / 256;
  static constexpr int NW = H ? 4 : KQ;  // words per piece
  unsigned int v[D][NP * NW];
  const S *row[NP];
  int mn[NP], kk[NP];
  bool rok[NP];

  __device__ __forceinline__ void init(int tid) {
#pragma unroll
    for (int e = 0; e < NP; ++e) {
      const int idx = e * 256 + tid;
      mn[e] = idx / (KS / KQ);
      kk[e] = (idx % (KS / KQ)) * KQ;
    }
  }
  template <int d>
  __device__ __forceinline__ void fast(int64_t k0) {
#pragma unroll
    for (int e = 0; e < NP; ++e) {
#pragma unroll
      for (int h = 0; h < NW; h += 4) {
        const u4 t = *reinterpret_cast<const u4 *>(row[e] + k0 + kk[e] + (H ? 0 : h));
        v[d][e * NW + h] = t.x;
        v[d][e * NW + h + 1] = t.y;
        v[d][e * NW + h + 2] = t.z;
        v[d][e * NW + h + 3] = t.w;
      }
    }
  }
  template <int d>
  __device__ __forceinline__ void slow(int64_t k0, int64_t ke) {
#pragma unroll
    for (int e = 0; e < NP; ++e) {
      const int64_t k = k0 + kk[e];
      const bool ok = rok[e];
      if constexpr (H) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const unsigned int lo = (ok && k + 2 * i < ke) ? row[e][k + 2 * i] : 0u;
          const unsigned int hi = (ok && k + 2 * i + 1 < ke) ? row[e][k + 2 * i + 1] : 0u;
          v[d][e * NW + i] = lo | (hi << 16);
        }
      } else {
#pragma unroll
        for (int i = 0; i < KQ; ++i)
          v[d][e * NW + i] = (ok && k + i < ke) ? __builtin_bit_cast(unsigned int, row[e][k + i]) : 0u;
      }
    }
  }
  __device__ __forceinline__ bool fast_ok() const { return true; }
  template <int d>
  __device__ __forceinline__ void store(typename Prec<PREC>::T (*dst)[BigStage<PREC>::LD]) const {
#pragma unroll
    for (int e = 0; e < NP; ++e) {
      if constexpr (H) {
        *reinterpret_cast<u4 *>(&dst[mn[e]][kk[e]]) =
            u4{v[d][e * NW], v[d][e * NW + 1], v[d][e * NW + 2], v[d][e * NW + 3]};
      } else {
        float x[KQ];
#pragma unroll
        for (int i = 0; i < KQ; ++i) x[i] = __builtin_bit_cast(float, v[d][e * NW + i]);
        store_kvec<PREC>(&dst[mn[e]][kk[e]], x);
      }
    }
  }
};

template <int PREC>
union BigFusedSmem {
  BigStage<PREC> st[2];
  float cur[kBig][kBig + 1];
};

// H: bf16 operands in memory -- x rows bf16 [T, B, F] and the weight
// transposed to wt [N, F] bf16 (k-contiguous); otherwise fp32 x and w [F, N].
template <int PREC, int BT, bool H>
__global__ __launch_bounds__(256) void linear_lif_fwd_big(LinArgs p) {
  constexpr int CH = kBig / BT;
  constexpr int Q = BT / 2;
  __shared__ BigFusedSmem<PREC> sm;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6), wm = w >> 1, wn = w & 1;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * kBig, b0 = static_cast<int64_t>(blockIdx.y) * BT;
  const int64_t BN = p.B * p.N;
  const int h = w & 1, rg = w >> 1;
  const int64_t n = n0 + 64 * h + lane;
  const bool n_ok = n < p.N;
  // batch row of slot q: brow + q (wave-uniform); its flat index brow_n + q*N + n
  const int64_t brow = b0 + rg * Q, brow_n = brow * p.N;
  float m[Q], cnt[Q];
#pragma unroll
  for (int q = 0; q < Q; ++q) {
    const bool act = brow + q < p.B && n_ok;
    m[q] = (act && p.m0 != nullptr) ? p.m0[brow_n + q * p.N + n] : 0.0f;
    cnt[q] = 0.0f;
  }
  const float bias_n = (p.bias != nullptr && n_ok) ? p.bias[n] : 0.0f;
  int64_t next_ck = p.t_begin, ck_row = 0;

  using S = typename std::conditional<H, uint16_t, float>::type;
  // register sets of prefetched stages: a second fits in 256 VGPRs
  // (2 waves per SIMD, which the LDS allows anyway) only for 8-row bf16
  constexpr int D = (H && BT == 8) ? 2 : 1;
  // H: wt [N, F] rows are neurons (k-contiguous); else w [F, N], neurons
  // contiguous for a fixed k
  BigLoader<PREC, H, S, D> lb;
  lb.init(tid, H ? static_cast<const void *>(p.wt) : static_cast<const void *>(p.w), n0, p.N, H ? p.F : p.N);
  BigRowLoader<PREC, S, D> la;
  la.init(tid);

  for (int64_t t0 = p.t_begin; t0 < p.t_end; t0 += CH) {
#pragma unroll
    for (int e = 0; e < BigRowLoader<PREC, S, D>::NP; ++e) {
      const int r = la.mn[e];
      const int64_t t = t0 + r / BT, b = b0 + r % BT;
      const bool ok = t < p.t_end && b < p.B;
      // row (t0, b0) always exists
      const int64_t rix = ok ? t * p.B + b : t0 * p.B + b0;
      la.rok[e] = ok;
      if constexpr (H)
        la.row[e] = p.xh + rix * p.F;
      else
        la.row[e] = p.x + rix * p.F;
    }
    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
    big_kloop<PREC, D>(la, lb, 0, p.F, sm.st, wm, wn, lane, acc);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          sm.cur[64 * wm + 32 * i + acc_row(r, lane)][64 * wn + 32 * j + (lane & 31)] = acc[i][j][r];
    __syncthreads();

#pragma unroll 1
    for (int j = 0; j < CH; ++j) {
      const int64_t t = t0 + j;
      if (t >= p.t_end) break;  // uniform
      if (p.ckpt != nullptr && t == next_ck) {
#pragma unroll
        for (int q = 0; q < Q; ++q)
          if (brow + q < p.B && n_ok) p.ckpt[ck_row * BN + brow_n + q * p.N + n] = m[q];
        ++ck_row;
        next_ck += p.ckpt_every;
      }
      bool s[Q];
#pragma unroll
      for (int q = 0; q < Q; ++q) {
        const bool act = brow + q < p.B && n_ok;
        const int64_t flat = brow_n + q * p.N + n;
        const float c_in = sm.cur[j * BT + rg * Q + q][64 * h + lane] + bias_n;
        float mp = m[q] * p.decay;
        mp = mp + c_in;
        bool sp;
        if (p.rule == MYELIN_RULE_THRESHOLD) {
          sp = mp >= p.thr;
        } else {
          const float c = p.slope * (mp - p.thr);
          sp = c >= 0.0f;
        }
        s[q] = act && sp;
        if (act) {
          if (p.pre != nullptr) p.pre[(t - p.t_begin) * BN + flat] = mp;
          if (p.spikes != nullptr) __builtin_nontemporal_store(sp ? 1.0f : 0.0f, p.spikes + t * BN + flat);
          m[q] = sp ? p.reset : mp;
          cnt[q] = cnt[q] + (sp ? 1.0f : 0.0f);
        }
      }
      if (p.packed != nullptr) {
#pragma unroll
        for (int q = 0; q < Q; ++q) {
          const uint64_t bits = __ballot(s[q]);
          const int64_t b = brow + q;
          const int64_t word = (n0 + 64 * h) / 32 + (lane >> 5);
          // every lane of a half-wave stores its half's word (one value to
          // one address): no lane-selected branch a step
          if (b < p.B && word < p.W)
            p.packed[(t * p.B + b) * p.W + word] =
                static_cast<int32_t>((lane & 32) ? (bits >> 32) : (bits & 0xffffffffu));
        }
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int q = 0; q < Q; ++q) {
    if (!(brow + q < p.B && n_ok)) continue;
    const int64_t flat = brow_n + q * p.N + n;
    if (p.m_final != nullptr) p.m_final[flat] = m[q];
    if (p.rates != nullptr) p.rates[flat] = cnt[q] / p.rate_denominator;
  }
}

// ---------------------------------------------------------------------------
// Fused current GEMM + LIF, software-pipelined: the recurrence of time chunk
// c - 1 runs from the MFMA accumulators while the GEMM of chunk c runs.
// Operands are bf16 in memory: x [T, B, F] and wt [N, F], rows 16-byte
// aligned.
//
// Tile: 16 batch rows x 16 steps (256 GEMM rows) x 128 neurons, eight
// waves of 64 x 64, stages ("windows") of 64 k staged through three LDS
// buffers by direct global -> LDS loads (unpadded 128-byte rows, k-groups
// swizzled by swz), two
// windows ahead, continuously across chunks.  Element r of a lane's 32 x 32
// accumulator block is row 8 (r >> 2) + 4 (lane >> 5) + (r & 3) (acc_row);
// the A rows are gathered so that row R of a block is batch row
// ((R >> 2) & 1) of the block's pair at step 4 (R >> 3) + (R & 3), which
// makes element r step r of one (batch row, neuron) chain.  Each wave holds
// two accumulator sets: the GEMM of chunk c accumulates into one while the
// recurrence steps of chunk c - 1 are taken from the other, a few between
// consecutive windows, so the VALU work and the trace stores overlap the
// MFMAs and the operand loads of the next chunk.
//
// Vector memory operations retire in issue order (loads and stores share
// vmcnt), so a window waits for its loads with vmcnt(6): all but the six
// direct loads of the next window, issued last.  The recurrence steps of a
// window (and their stores) run between its barrier and that issue, so a
// window's stores need only retire by the next window's wait.  Lanes past B
// or N compute the chain of batch row B - 1 or neuron N - 1 (their operand
// rows, bias and start state are clamped to it) and store the same value to
// the same address as the lane that owns it, so the stores need no masks.
//
// In a partial last stage (F % 64 != 0) the pieces past F load a zero page
// and the 16-k steps entirely past F are skipped.  The k order -- stages of
// 64, four 16-k MFMAs each -- is the other bf16 engines', so the currents
// equal theirs bit for bit.  Workgroups go round-robin to the 8 XCDs; the
// logical tiles are batch-tile-major and each XCD is handed a contiguous run
// of them, so the workgroups sharing a batch tile's x rows share one L2.
// Offsets are 32-bit: B * N * 4 < 2^32 (a step's trace) and 32 B F < 2^32
// (16 steps of x).
// ---------------------------------------------------------------------------
namespace acc_fwd {
constexpr int BM = 256, BN = 128, NT = 512, WGN = 2;
constexpr int TILE = (BM + BN) * 128;  // bytes of one stage
constexpr int NPA = BM * 8 / NT, NPB = BN * 8 / NT;
constexpr int NL = NPA + NPB;  // direct loads per thread per stage

// batch row (0..15) and step (0..15) of tile row r
__device__ __forceinline__ int row_batch(int r) { return 2 * (r >> 5) + ((r >> 2) & 1); }
// the 16-byte k-group position swizzle of tile row r: a function of r & 31
// (so the row blocks of a wave share it), distinct over any 8 aligned rows
// and, with the row's bank half, over any 16 (the fragment reads are
// conflict-free whether the LDS serves 8 or 16 lanes a cycle)
__device__ __forceinline__ int swz(int r) { return (r ^ ((r >> 3) & 3)) & 7; }
__device__ __forceinline__ int row_step(int r) { return 4 * ((r >> 3) & 3) + (r & 3); }

// the source of the pieces of a partial last stage that lie past F
__device__ __align__(16) const uint16_t kZeroPiece[8] = {};

// one store at base + off (bytes; base uniform): the scalar-base form keeps
// the per-step address arithmetic on the scalar unit
__device__ __forceinline__ void store_at(const char *base, uint32_t off, float v) {
  asm volatile("global_store_dword %0, %1, %2" ::"v"(off), "v"(v), "s"(base) : "memory");
}
// the same, nontemporal (streamed past the caches' reuse)
__device__ __forceinline__ void store_nt_at(const char *base, uint32_t off, float v) {
  asm volatile("global_store_dword %0, %1, %2 nt" ::"v"(off), "v"(v), "s"(base) : "memory");
}
}  // namespace acc_fwd

// OUTS: the outputs written, as bits 1 pre, 2 spikes, 4 packed, 8
// checkpoints, 16 rates (the hot sets are compiled without the branches), or
// -1 for any set, read from p
template <int RULE, int OUTS>
__global__ __launch_bounds__(acc_fwd::NT) __attribute__((amdgpu_waves_per_eu(2))) void linear_lif_fwd_pipe(LinArgs p) {
  using namespace acc_fwd;
  __shared__ __attribute__((aligned(1024))) char lds[3 * TILE];
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6), wm = w / WGN, wn = w % WGN;
  const int64_t B = p.B, N = p.N, F = p.F, BNt = p.B * p.N;
  const uint32_t tiles_n = static_cast<uint32_t>((N + BN - 1) / BN), nblk = gridDim.x;
  uint32_t tile = blockIdx.x;
  if (nblk % 8 == 0) tile = (tile % 8) * (nblk / 8) + tile / 8;
  const int64_t n0 = __builtin_amdgcn_readfirstlane(tile % tiles_n) * static_cast<int64_t>(BN);
  const int64_t b0 = __builtin_amdgcn_readfirstlane(tile / tiles_n) * static_cast<int64_t>(16);
  const int64_t nchunks = (p.t_end - p.t_begin + 15) / 16;
  const int64_t nst = (F + 63) / 64;  // windows per chunk, the last possibly partial
  const int kq_last = F % 64 != 0 ? static_cast<int>((F % 64 + 15) / 16) : 4;

  // Operand pieces (16 bytes: 8 bf16 of k) as 32-bit byte offsets from a
  // uniform base: A piece e of thread tid is tile row (e * NT + tid) / 8 at
  // k-group position (idx & 7) ^ swz(row) of the stage, from the chunk's
  // first x row; B pieces likewise from row n0 of wt.  Rows past B read
  // batch row B - 1 at the same step (the chains the lanes past B
  // duplicate), rows past the end of time step t0 (accumulator rows the
  // recurrence skips), rows past N row N - 1.
  uint32_t oa[NPA], ob[NPB];
  const uint16_t *xa = nullptr;  // the current chunk's first x row
  auto point_a = [&](int64_t t0) {
    xa = p.xh + t0 * B * F;
#pragma unroll
    for (int e = 0; e < NPA; ++e) {
      const int idx = e * NT + tid, ra = idx >> 3;
      const int step = t0 + row_step(ra) < p.t_end ? row_step(ra) : 0;
      const int64_t b = b0 + row_batch(ra);
      oa[e] = static_cast<uint32_t>(((step * B + (b < B ? b : B - 1)) * F + 8 * ((idx & 7) ^ swz(ra))) * 2);
    }
  };
  const uint16_t *wb0 = p.wt + n0 * F;
#pragma unroll
  for (int e = 0; e < NPB; ++e) {
    const int idx = e * NT + tid, r = idx >> 3;
    const int64_t rr = n0 + r < N ? r : N - 1 - n0;
    ob[e] = static_cast<uint32_t>((rr * F + 8 * ((idx & 7) ^ swz(r))) * 2);
  }
  auto issue = [&](char *tile, int64_t k0) {
    const bool part = k0 + 64 > F;  // uniform: the partial last stage
    const char *xk = reinterpret_cast<const char *>(xa + k0), *wk = reinterpret_cast<const char *>(wb0 + k0);
#pragma unroll
    for (int e = 0; e < NL; ++e) {
      const int eo = e < NPA ? e : e - NPA, idx = eo * NT + tid;
      // the wave's 64 pieces fill 1 KB of the stage in lane order
      const uint32_t dst = static_cast<uint32_t>(
          reinterpret_cast<uintptr_t>((lds_void *)(tile + (e < NPA ? 0 : BM * 128) + (eo * NT + w * 64) * 16)));
      const char *base = e < NPA ? xk : wk;
      const uint32_t o = e < NPA ? oa[e] : ob[e - NPA];
      uint32_t m0_saved;
      if (part) {
        // pieces past F load the zero page
        const char *src = base + o;
        if (k0 + 8 * ((idx & 7) ^ swz(idx >> 3)) >= F) src = reinterpret_cast<const char *>(kZeroPiece);
        asm volatile(
            "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off\n\ts_mov_b32 m0, %0"
            : "=&s"(m0_saved)
            : "v"(src), "s"(dst)
            : "memory");
      } else {
        asm volatile(
            "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2\n\ts_mov_b32 m0, %0"
            : "=&s"(m0_saved)
            : "v"(o), "s"(base), "s"(dst)
            : "memory");
      }
    }
  };
  // fragment byte offsets in a stage (row blocks i, column blocks j sit
  // 4096 bytes apart: their rows have the same swizzle)
  int fa[4], fb[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    const int c = 2 * ks + (lane >> 5), r = lane & 31;
    fa[ks] = (64 * wm + r) * 128 + ((c ^ swz(r)) << 4);
    fb[ks] = (BM + 64 * wn + r) * 128 + ((c ^ swz(r)) << 4);
  }
  // kq: the stage's 16-k steps that hold data (4, or fewer in a partial last
  // stage: the rest multiply zeros)
  auto mfma_stage = [&](f32x16(&acc)[2][2], const char *cur, int kq) {
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      if (ks >= kq) break;  // uniform
      bf16x8 a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) a[i] = *reinterpret_cast<const bf16x8 *>(cur + fa[ks] + 4096 * i);
#pragma unroll
      for (int j = 0; j < 2; ++j) b[j] = *reinterpret_cast<const bf16x8 *>(cur + fb[ks] + 4096 * j);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
  };

  // chains: (row block i, column block j) -> batch row, neuron (clamped);
  // off: the chain's byte offset in a [B, N] slice; pk_off: the byte offset
  // of the packed word of column block 0 in a [B, W] slice
  const int64_t wpk = (n0 + 64 * wn) / 32;  // packed word of column block 0
  float m[2][2], cnt[2][2], bias[2];
  uint32_t off[2][2], pk_off[2];
  bool bok[2], nok[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int64_t n = n0 + 64 * wn + 32 * j + (lane & 31);
    nok[j] = n < N;
    bias[j] = p.bias != nullptr ? p.bias[nok[j] ? n : N - 1] : 0.0f;
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int64_t b = b0 + 4 * wm + 2 * i + (lane >> 5);
    bok[i] = b < B;
    const int64_t bc = bok[i] ? b : B - 1;
    pk_off[i] = static_cast<uint32_t>((bc * p.W + wpk) * 4);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int64_t n = n0 + 64 * wn + 32 * j + (lane & 31);
      const int64_t flat = bc * N + (nok[j] ? n : N - 1);
      off[i][j] = static_cast<uint32_t>(flat * 4);
      m[i][j] = p.m0 != nullptr ? p.m0[flat] : 0.0f;
      cnt[i][j] = 0.0f;
    }
  }
  // take the start state and bias before the loop: a first use inside it
  // would make the compiler wait for every vector memory operation
  // (vmcnt(0)) at each recurrence step, its scoreboard not seeing them retire
  asm volatile("" ::"v"(m[0][0]), "v"(m[0][1]), "v"(m[1][0]), "v"(m[1][1]), "v"(bias[0]), "v"(bias[1]));
  int next_ck = 0;  // the next checkpoint step, relative to t_begin

  // the next load batch: chunk ic, stage is, LDS buffer ib
  int ic = 0, is = 0, ib = 0, a_chunk = -1;
  const int nst32 = static_cast<int>(nst), nch32 = static_cast<int>(nchunks);
  auto issue_next = [&]() {
    if (ic >= nch32) return;  // uniform
    if (ic != a_chunk) {
      point_a(p.t_begin + 16 * static_cast<int64_t>(ic));
      a_chunk = ic;
    }
    issue(lds + ib * TILE, is * 64);
    ib = ib == 2 ? 0 : ib + 1;
    if (++is == nst32) {
      is = 0;
      ++ic;
    }
  };

  // recurrence step r (of its chunk: accumulator element r) at step t_cur,
  // from accumulator set acc; the trace pointers run with t_cur (advanced
  // per step rather than recomputed, which would let the compiler hoist
  // sixteen steps' addresses into scalar registers)
  int64_t t_cur = p.t_begin;
  const int outs = OUTS >= 0 ? OUTS : lin_outputs(p);
  const char *pre_c = reinterpret_cast<const char *>(p.pre);
  const char *spk_c = reinterpret_cast<const char *>(p.spikes + p.t_begin * BNt);
  const char *pk_c = reinterpret_cast<const char *>(p.packed + p.t_begin * B * p.W);
  const char *ck_c = reinterpret_cast<const char *>(p.ckpt);
  auto rec_step = [&](const f32x16(&acc)[2][2], int r) {
    const int64_t t = t_cur;
    if (t >= p.t_end) return;  // uniform
    if ((outs & 8) && t - p.t_begin == next_ck) {
      // every lane: the lanes past B or N write their owner's value
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) store_at(ck_c, off[i][j], m[i][j]);
      ck_c += BNt * 4;
      next_ck += static_cast<int>(p.ckpt_every);
    }
    const char *pre_t = pre_c, *spk_t = spk_c;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        // the empty asm pins the read (and the bias add) to this step: the
        // accumulator set is loop-invariant over the windows, and a hoisted
        // add would hold sixteen steps of currents in extra registers
        float a = acc[i][j][r];
        asm volatile("" : "+v"(a));
        const float c_in = a + bias[j];
        float mp = m[i][j] * p.decay;
        mp = mp + c_in;
        bool sp;
        if constexpr (RULE == MYELIN_RULE_THRESHOLD) {
          sp = mp >= p.thr;
        } else {
          const float c = p.slope * (mp - p.thr);
          sp = c >= 0.0f;
        }
        // both streamed past the caches: the trace is read once, by the
        // backward's reverse pass (T = 50, B = 256, N = 2048: forward 92.1
        // -> 90.5 us, forward + reverse pass 155-159 -> 144-145 us)
        if (outs & 1) store_nt_at(pre_t, off[i][j], mp);
        if (outs & 2) store_nt_at(spk_t, off[i][j], sp ? 1.0f : 0.0f);
        m[i][j] = sp ? p.reset : mp;
        if (outs & 16) cnt[i][j] = cnt[i][j] + (sp ? 1.0f : 0.0f);
        if (outs & 4) {
          // lanes 0-31: 32 neurons of the block's first batch row; 32-63: the next row
          // (every lane of a half stores its half's word: one value to one address)
          const uint64_t bits = __ballot(bok[i] && nok[j] && sp);
          if (bok[i] && wpk + j < p.W)
            store_at(pk_c + 4 * j, pk_off[i],
                     __builtin_bit_cast(float, static_cast<uint32_t>((lane & 32) ? (bits >> 32) : bits)));
        }
      }
    }
    ++t_cur;
    pre_c += BNt * 4;
    spk_c += BNt * 4;
    pk_c += B * p.W * 4;
  };
  auto rec_switch = [&](const f32x16(&acc)[2][2], int r) {
    switch (r) {
#define MYELIN_REC(k) \
  case k:             \
    rec_step(acc, k); \
    break;
      MYELIN_REC(0) MYELIN_REC(1) MYELIN_REC(2) MYELIN_REC(3) MYELIN_REC(4) MYELIN_REC(5) MYELIN_REC(6)
      MYELIN_REC(7) MYELIN_REC(8) MYELIN_REC(9) MYELIN_REC(10) MYELIN_REC(11) MYELIN_REC(12) MYELIN_REC(13)
      MYELIN_REC(14) MYELIN_REC(15)
#undef MYELIN_REC
      default: break;
    }
  };

  // Chunk c: its GEMM into cur (none past the last chunk) with the
  // recurrence of chunk c - 1 from prev (none for the first) spread over its
  // windows: step r runs in window ceil((r + 1) nst / 16) - 1, before the
  // window's load issue.  Waves 0-3 take their steps before their MFMAs,
  // waves 4-7 (the other wave on each SIMD) after theirs, so that one
  // wave's recurrence arithmetic runs while the other's MFMAs occupy the
  // SIMD's matrix pipe.  cur is copied to prev at the end of the chunk.
  const bool late = w >= 4;
  f32x16 cur[2][2], prev[2][2];
  int wb = 0;  // LDS buffer of the current window
  issue_next();
  issue_next();
  for (int c = 0; c <= nch32; ++c) {
    const int nw = c < nch32 ? nst32 : 0;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) cur[i][j][r] = 0.0f;
    int r = c > 0 ? 0 : 16;
    for (int s = 0; s < nw; ++s) {
      // this window's loads: every operation but the next window's batch
      // when that is issued (the last vector memory operations issued),
      // else all
      if (ic * nst32 + is > c * nst32 + s + 1)
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(NL) : "memory");
      else
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      const int kq = s + 1 < nst32 ? 4 : kq_last;
      if (late) mfma_stage(cur, lds + wb * TILE, kq);
      for (; r < 16 && ((r + 1) * nst32 + 15) / 16 <= s + 1; ++r) rec_switch(prev, r);
      issue_next();
      if (!late) mfma_stage(cur, lds + wb * TILE, kq);
      wb = wb == 2 ? 0 : wb + 1;
    }
    for (; r < 16; ++r) rec_switch(prev, r);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) prev[i][j] = cur[i][j];
  }
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      // every lane: the lanes past B or N write their owner's value
      if (p.m_final != nullptr) *reinterpret_cast<float *>(reinterpret_cast<char *>(p.m_final) + off[i][j]) = m[i][j];
      if (p.rates != nullptr)
        *reinterpret_cast<float *>(reinterpret_cast<char *>(p.rates) + off[i][j]) = cnt[i][j] / p.rate_denominator;
    }
}

// v is a bf16 value the MFMA multiplies exactly: its bf16 rounding returns
// it, and it is zero or normal (denormals may be flushed)
__device__ __forceinline__ bool bf16_exact(float v) {
  const float a = __builtin_fabsf(v);
  return static_cast<float>(static_cast<__bf16>(v)) == v && (a == 0.0f || a >= 1.17549435e-38f);
}

struct PreBwdArgs {
  const float *pre;     // [C, BN]
  const float *gs;      // [C, BN] or null
  const float *grate;   // [BN] or null
  float *gm;            // [BN] in/out
  void *G;              // [C, BN] float, or bf16 bits when the GEMMs read bf16, or three
                        // bf16 planes [3, C, BN] summing exactly to G
  float *gbias_acc;     // [BN] or null (accumulated)
  int64_t C, BN;
  float decay, thr, reset, slope, rate_denominator;
  int rule;
};

// Serial time loops over [L] steps stream their operands in blocks of kPipe
// steps, the next block's loads issued before the current block computes.
// Block 0 holds the first f = L - (nblk - 1) * kPipe steps (1..kPipe), the
// rest are full, so the steady state is straight-line code with a fixed
// number of loads in flight; every load address is clamped into range, so
// no load is predicated.
constexpr int kPipe = 16;

// One reverse step of one neuron: gp = dL/dI_j (reference op order), then
// the carried gm = gp * decay; gb accumulates gp.  RULE: the spike rule at
// compile time (MYELIN_RULE_*), or -1 to read p.rule.
template <int SID, bool GS, int RULE = -1>
__device__ __forceinline__ float pre_bwd_gp(const PreBwdArgs &p, float pre, float gsv, float gstep, float &gm,
                                            float &gb) {
  const float c = p.slope * (pre - p.thr);
  bool sp;
  if constexpr (RULE == MYELIN_RULE_THRESHOLD)
    sp = pre >= p.thr;
  else if constexpr (RULE == MYELIN_RULE_SURROGATE)
    sp = c >= 0.0f;
  else
    sp = (p.rule == MYELIN_RULE_THRESHOLD) ? (pre >= p.thr) : (c >= 0.0f);
  const float s = sp ? 1.0f : 0.0f;
  const float d = p.slope * sg_deriv<SID>(c);
  float gp = gm * ((1.0f - s) + (p.reset - pre) * d);
  if constexpr (GS) gp = gp + gsv * d;
  if (p.grate != nullptr) gp = gp + gstep * d;
  gb = gb + gp;
  gm = gp * p.decay;
  return gp;
}

template <int V>
struct PreVec;
template <>
struct PreVec<1> {
  using T = float;
  static __device__ __forceinline__ float at(float v, int) { return v; }
};
template <>
struct PreVec<2> {
  using T = float2;
  static __device__ __forceinline__ float at(float2 v, int e) { return e ? v.y : v.x; }
};

__device__ __forceinline__ uint16_t bf16_bits(float v) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(v));
}

// G[j, i .. i+V) = gp: fp32 (GM 0), bf16 (GM 1) or three bf16 planes (GM 2),
// one store per plane covering the lane's V neurons
template <int GM, int V>
__device__ __forceinline__ void store_g(const PreBwdArgs &p, int64_t i, int64_t j, const float (&gp)[V]) {
  const int64_t at = j * p.BN + i;
  if constexpr (GM == 0) {
    if constexpr (V == 2)
      *reinterpret_cast<float2 *>(static_cast<float *>(p.G) + at) = float2{gp[0], gp[1]};
    else
      static_cast<float *>(p.G)[at] = gp[0];
  } else if constexpr (GM == 1) {
    if constexpr (V == 2)
      *reinterpret_cast<uint32_t *>(static_cast<uint16_t *>(p.G) + at) =
          bf16_bits(gp[0]) | static_cast<uint32_t>(bf16_bits(gp[1])) << 16;
    else
      static_cast<uint16_t *>(p.G)[at] = bf16_bits(gp[0]);
  } else {
    uint16_t h[V], m[V], l[V];
#pragma unroll
    for (int e = 0; e < V; ++e) split3(gp[e], h[e], m[e], l[e]);
    uint16_t *g16 = static_cast<uint16_t *>(p.G) + at;
    const int64_t plane = p.C * p.BN;
    if constexpr (V == 2) {
      *reinterpret_cast<uint32_t *>(g16) = h[0] | static_cast<uint32_t>(h[1]) << 16;
      *reinterpret_cast<uint32_t *>(g16 + plane) = m[0] | static_cast<uint32_t>(m[1]) << 16;
      *reinterpret_cast<uint32_t *>(g16 + 2 * plane) = l[0] | static_cast<uint32_t>(l[1]) << 16;
    } else {
      g16[0] = h[0];
      g16[plane] = m[0];
      g16[2 * plane] = l[0];
    }
  }
}

template <int SID, bool GS, int GM, int V, int RULE = -1, typename VT>
__device__ __forceinline__ void pre_bwd_step(const PreBwdArgs &p, int64_t i, int64_t j, VT pre, VT gsv,
                                             const float (&gstep)[V], float (&gm)[V], float (&gb)[V]) {
  float gp[V];
#pragma unroll
  for (int e = 0; e < V; ++e)
    gp[e] = pre_bwd_gp<SID, GS, RULE>(p, PreVec<V>::at(pre, e), PreVec<V>::at(gsv, e), gstep[e], gm[e], gb[e]);
  store_g<GM, V>(p, i, j, gp);
}

// reverse time: relative index r = C - 1 - j.  GM: G is written as fp32
// (0), as bf16 rounded as the bf16 GEMMs would round it (1), or as three
// bf16 planes whose sum is G exactly (2).  V neurons per lane (V = 2: BN
// even and every operand 8-byte aligned, so each step is one 8-byte load
// per operand and one store per plane).  The loads run DEPTH steps ahead:
// 4 on the wide (V = 2) grids, where a 16-step block costs 150 registers
// and so occupancy (3 waves per SIMD instead of 8; 524288 neurons x 50
// steps: 54 -> 42 us, x 256 steps: 310 -> 293 us, 131072 x 225 with the
// three-plane G: 86 -> 78 us), and kPipe on the narrow ones, whose few
// waves need every load of a long serial walk in flight.  RULE: the spike
// rule at compile time on the narrow grids (a step of the 640-neuron,
// 2000-step readout walk is 28 instructions with it read at run time, 7 of
// them choosing the rule), -1 (read p.rule) on the wide ones.
template <int SID, bool GS, int GM, int V, int RULE = -1>
__global__ __launch_bounds__(256) void linear_pre_bwd(PreBwdArgs p) {
  using VT = typename PreVec<V>::T;
  constexpr int DEPTH = V == 2 ? 4 : kPipe;
  const int64_t i = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) * V;
  if (i >= p.BN) return;
  const int64_t C = p.C, row = p.BN / V;
  float gm[V], gstep[V], gb[V];
#pragma unroll
  for (int e = 0; e < V; ++e) {
    gm[e] = p.gm != nullptr ? p.gm[i + e] : 0.0f;
    gstep[e] = p.grate != nullptr ? p.grate[i + e] / p.rate_denominator : 0.0f;
    gb[e] = 0.0f;
  }
  const VT *pre = reinterpret_cast<const VT *>(p.pre + i);
  const VT *gs = GS ? reinterpret_cast<const VT *>(p.gs + i) : nullptr;
  const VT zero{};
  const int64_t nblk = (C + DEPTH - 1) / DEPTH;
  const int64_t f = C - (nblk - 1) * DEPTH;
  VT pv[DEPTH], gv[DEPTH];
#pragma unroll
  for (int u = 0; u < DEPTH; ++u) {
    const int64_t j = C - 1 - (u < f ? u : f - 1);
    pv[u] = pre[j * row];
    if constexpr (GS) gv[u] = gs[j * row];
  }
  // block 0 (f steps), prefetching block 1 (or re-reading block 0 when alone)
  {
    const int64_t r0 = nblk > 1 ? f : 0;
    VT np[DEPTH], ng[DEPTH];
#pragma unroll
    for (int u = 0; u < DEPTH; ++u) {
      const int64_t r = r0 + u < C ? r0 + u : C - 1;
      np[u] = pre[(C - 1 - r) * row];
      if constexpr (GS) ng[u] = gs[(C - 1 - r) * row];
    }
#pragma unroll
    for (int u = 0; u < DEPTH; ++u)
      if (u < f) pre_bwd_step<SID, GS, GM, V, RULE>(p, i, C - 1 - u, pv[u], GS ? gv[u] : zero, gstep, gm, gb);
#pragma unroll
    for (int u = 0; u < DEPTH; ++u) {
      pv[u] = np[u];
      if constexpr (GS) gv[u] = ng[u];
    }
  }
  for (int64_t r0 = f; r0 < C; r0 += DEPTH) {
    const int64_t rn = r0 + DEPTH < C ? r0 + DEPTH : r0;
    VT np[DEPTH], ng[DEPTH];
#pragma unroll
    for (int u = 0; u < DEPTH; ++u) {
      np[u] = pre[(C - 1 - rn - u) * row];
      if constexpr (GS) ng[u] = gs[(C - 1 - rn - u) * row];
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < DEPTH; ++u)
      pre_bwd_step<SID, GS, GM, V, RULE>(p, i, C - 1 - r0 - u, pv[u], GS ? gv[u] : zero, gstep, gm, gb);
#pragma unroll
    for (int u = 0; u < DEPTH; ++u) {
      pv[u] = np[u];
      if constexpr (GS) gv[u] = ng[u];
    }
  }
#pragma unroll
  for (int e = 0; e < V; ++e) {
    // no gm: the launch is the whole reverse pass (no carried adjoint in or
    // out), and the bias accumulator starts from zero here
    if (p.gm != nullptr) p.gm[i + e] = gm[e];
    if (p.gbias_acc != nullptr) p.gbias_acc[i + e] = (p.gm != nullptr ? p.gbias_acc[i + e] : 0.0f) + gb[e];
  }
}

// The hidden layer's reverse pass of a two-layer network with its spike
// gradient formed in the kernel: gs[j, b, n] = sum_o G_o[j, b, o] W_o[n, o]
// (dS = G_o W_o^T), summed in o order with fused multiply-adds from zero
// over KMAX terms (zero past O) -- the small-K GEMM's arithmetic, so G is
// the one dS written by that GEMM and read back gives, without dS's write
// and read ([C, B, N] floats each way).  A workgroup's 256 neurons lie in
// one batch row b (N a multiple of 256): it stages that row's G_o [C, O] in
// LDS, zero-padded to KMAX columns, and each step's row reaches every lane
// as broadcast 16-byte LDS reads.  A lane holds its neuron's row of W_o
// (KMAX registers).  The reverse walk is linear_pre_bwd's, with the
// pre-reset trace the one operand streamed from HBM, 8 steps ahead.  One
// neuron per lane: at 131072 neurons x 225 steps (config 4's hidden span)
// 79 us, against 100-108 us for two per lane (one wave per SIMD) with 4 or
// 8 steps ahead; 16 steps ahead 82 us.
template <int SID, int GM, int KMAX>
__global__ __launch_bounds__(256) void linear_pre_bwd_ds(PreBwdArgs p, const float *go, const float *wo, int O,
                                                         int64_t N) {
  extern __shared__ __attribute__((aligned(16))) float s_go[];  // [C][KMAX]
  constexpr int V = 1, DEPTH = 8;
  using VT = typename PreVec<V>::T;
  const int64_t C = p.C, row = p.BN / V;
  const int64_t base = static_cast<int64_t>(blockIdx.x) * (256 * V);
  const int64_t bi = base / N, Bn = p.BN / N;
  for (int64_t q = threadIdx.x; q < C * KMAX; q += 256) {
    const int64_t j = q / KMAX;
    const int o = static_cast<int>(q % KMAX);
    s_go[q] = o < O ? go[(j * Bn + bi) * O + o] : 0.0f;
  }
  __syncthreads();
  const int64_t i = base + static_cast<int64_t>(threadIdx.x) * V;  // < BN: the grid is BN / (256 V) exactly
  const int64_t n = i - bi * N;
  float w[V][KMAX];
#pragma unroll
  for (int e = 0; e < V; ++e)
#pragma unroll
    for (int o = 0; o < KMAX; ++o) w[e][o] = o < O ? wo[(n + e) * O + o] : 0.0f;
  float gm[V], gstep[V], gb[V];
#pragma unroll
  for (int e = 0; e < V; ++e) {
    gm[e] = p.gm != nullptr ? p.gm[i + e] : 0.0f;
    gstep[e] = p.grate != nullptr ? p.grate[i + e] / p.rate_denominator : 0.0f;
    gb[e] = 0.0f;
  }
  auto step = [&](int64_t j, VT pv) {
    const f4 *r = reinterpret_cast<const f4 *>(s_go + j * KMAX);
    float acc[V];
#pragma unroll
    for (int e = 0; e < V; ++e) acc[e] = 0.0f;
#pragma unroll
    for (int q = 0; q < KMAX / 4; ++q) {
      const f4 g4 = r[q];
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int e = 0; e < V; ++e) acc[e] = __builtin_fmaf(g4[u], w[e][4 * q + u], acc[e]);
    }
    pre_bwd_step<SID, true, GM, V>(p, i, j, pv, acc[0], gstep, gm, gb);
  };
  const VT *pre = reinterpret_cast<const VT *>(p.pre + i);
  const int64_t nblk = (C + DEPTH - 1) / DEPTH;
  const int64_t f = C - (nblk - 1) * DEPTH;
  VT pv[DEPTH];
#pragma unroll
  for (int u = 0; u < DEPTH; ++u) pv[u] = pre[(C - 1 - (u < f ? u : f - 1)) * row];
  // block 0 (f steps), prefetching block 1 (or re-reading block 0 when alone)
  {
    const int64_t r0 = nblk > 1 ? f : 0;
    VT np[DEPTH];
#pragma unroll
    for (int u = 0; u < DEPTH; ++u) np[u] = pre[(C - 1 - (r0 + u < C ? r0 + u : C - 1)) * row];
#pragma unroll
    for (int u = 0; u < DEPTH; ++u)
      if (u < f) step(C - 1 - u, pv[u]);
#pragma unroll
    for (int u = 0; u < DEPTH; ++u) pv[u] = np[u];
  }
  for (int64_t r0 = f; r0 < C; r0 += DEPTH) {
    const int64_t rn = r0 + DEPTH < C ? r0 + DEPTH : r0;
    VT np[DEPTH];
#pragma unroll
    for (int u = 0; u < DEPTH; ++u) np[u] = pre[(C - 1 - rn - u) * row];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < DEPTH; ++u) step(C - 1 - r0 - u, pv[u]);
#pragma unroll
    for (int u = 0; u < DEPTH; ++u) pv[u] = np[u];
  }
#pragma unroll
  for (int e = 0; e < V; ++e) {
    if (p.gm != nullptr) p.gm[i + e] = gm[e];
    if (p.gbias_acc != nullptr) p.gbias_acc[i + e] = (p.gm != nullptr ? p.gbias_acc[i + e] : 0.0f) + gb[e];
  }
}

// out[n] (+)= sum_r in[r, n] for the 8 columns of workgroup `block` (see
// col_sum_block)
__global__ __launch_bounds__(256) void col_sum(const float *__restrict__ in, float *__restrict__ out, int64_t rows,
                                               int64_t cols, int accumulate) {
  col_sum_block(in, out, rows, cols, accumulate, blockIdx.x);
}

// LIF recurrence over precomputed currents cur [t_end - t_begin, B, N]
// (bias already added by the GEMM epilogue), for outputs too narrow to
// fill the chip with the fused kernel.  Lanes map to (b, word, bit) so a
// half-wave owns one packed word.
struct CurArgs {
  const float *cur;
  const float *m0;
  float *m_final, *spikes, *pre, *rates, *ckpt, *counts;
  int32_t *packed;
  int64_t T, B, N, W, t_begin, t_end, ckpt_every, pre_origin, ck_origin;
  float decay, thr, reset, slope, rate_denominator;
  int rule;
};

// Output cursors of one lane of the currents recurrence: each points at the
// lane's element of the current step and advances one step at a time, so a
// step does no index arithmetic.
struct CurCursor {
  float *pre, *spk, *ck;
  int32_t *pk;
  int64_t next_ck;
};

// One step of the currents recurrence for lane (b, n); the outputs (PRE:
// pre-reset membrane, SPK: dense spikes, PK: ballot-packed words, CK:
// checkpoints) and the spike rule are chosen at compile time, so a step is
// its arithmetic and its stores.
template <bool PRE, bool SPK, bool PK, int RULE, bool CK>
__device__ __forceinline__ void cur_step(const CurArgs &p, int64_t t, float c, bool act, int64_t BN, int64_t gw,
                                         int lane, float &m, float &cnt, CurCursor &o) {
  // (stores from every lane: a lane past B or N repeats its owner's)
  if constexpr (CK) {
    if (t == o.next_ck) {
      *o.ck = m;
      o.ck += BN;
      o.next_ck += p.ckpt_every;
    }
  }
  float mp = m * p.decay;
  mp = mp + c;
  bool sp;
  if constexpr (RULE == MYELIN_RULE_THRESHOLD)
    sp = mp >= p.thr;
  else
    sp = p.slope * (mp - p.thr) >= 0.0f;
  if constexpr (PRE) *o.pre = mp;
  if constexpr (SPK) *o.spk = sp ? 1.0f : 0.0f;
  if constexpr (PRE) o.pre += BN;
  if constexpr (SPK) o.spk += BN;
  m = sp ? p.reset : mp;
  cnt = cnt + (sp ? 1.0f : 0.0f);
  if constexpr (PK) {
    const uint64_t bits = __ballot(act && sp);
    if (p.B * p.W % 2 == 0 && (reinterpret_cast<uintptr_t>(p.packed) & 7) == 0) {
      // the wave's two words as one 8-byte store, the same value from every
      // lane (gw is even and wave-uniform): no lane-selected branch a step
      if (gw < p.B * p.W) *reinterpret_cast<uint64_t *>(o.pk + gw) = bits;
    } else {
      if (lane == 0 && gw < p.B * p.W) o.pk[gw] = static_cast<int32_t>(bits & 0xffffffffu);
      if (lane == 32 && gw + 1 < p.B * p.W) o.pk[gw + 1] = static_cast<int32_t>(bits >> 32);
    }
    o.pk += p.B * p.W;
  }
}

template <bool PRE, bool SPK, bool PK, int RULE, bool CK>
__global__ __launch_bounds__(256) void lif_currents_fwd(CurArgs p) {
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t g = gid >> 5;
  const int bit = static_cast<int>(gid & 31);
  const int64_t b = g / p.W;
  const int64_t n = (g - b * p.W) * 32 + bit;
  const bool act = (b < p.B) && (n < p.N);
  // lanes past B or N run the chain of batch row B - 1 / neuron N - 1 and
  // store the same values to the same addresses as the lane that owns it,
  // so a step stores without a lane test
  const int64_t flat = (b < p.B ? b : p.B - 1) * p.N + (n < p.N ? n : p.N - 1), BN = p.B * p.N;
  const int lane = static_cast<int>(threadIdx.x & 63);
  // the wave's first packed word (wave-uniform: made a scalar)
  const int64_t gw_v = (gid - lane) >> 5;
  const int64_t gw = static_cast<int64_t>(static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(gw_v)))) |
                     (static_cast<int64_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(gw_v >> 32))) << 32);
  float m = p.m0 != nullptr ? p.m0[flat] : 0.0f;
  float cnt = p.counts != nullptr ? p.counts[flat] : 0.0f;
  // checkpoint rows are counted from ck_origin: row k holds the state before
  // step ck_origin + k*ckpt_every.
  CurCursor o{};
  if constexpr (PRE) o.pre = p.pre + (p.t_begin - p.pre_origin) * BN + flat;
  if constexpr (SPK) o.spk = p.spikes + p.t_begin * BN + flat;
  if constexpr (PK) o.pk = p.packed + p.t_begin * p.B * p.W;
  if constexpr (CK) {
    const int64_t ck_row = (p.t_begin - p.ck_origin + p.ckpt_every - 1) / p.ckpt_every;
    o.ck = p.ckpt + ck_row * BN + flat;
    o.next_ck = p.ck_origin + ck_row * p.ckpt_every;
  }
  const float *cur = p.cur + flat;
  const int64_t L = p.t_end - p.t_begin;
  const int64_t nblk = (L + kPipe - 1) / kPipe;
  const int64_t f = L - (nblk - 1) * kPipe;
  float cv[kPipe];
#pragma unroll
  for (int u = 0; u < kPipe; ++u) cv[u] = cur[(u < f ? u : f - 1) * BN];
  {
    const int64_t r0 = nblk > 1 ? f : 0;
    float nc[kPipe];
#pragma unroll
    for (int u = 0; u < kPipe; ++u) nc[u] = cur[(r0 + u < L ? r0 + u : L - 1) * BN];
#pragma unroll
    for (int u = 0; u < kPipe; ++u)
      if (u < f) cur_step<PRE, SPK, PK, RULE, CK>(p, p.t_begin + u, cv[u], act, BN, gw, lane, m, cnt, o);
#pragma unroll
    for (int u = 0; u < kPipe; ++u) cv[u] = nc[u];
  }
  for (int64_t r0 = f; r0 < L; r0 += kPipe) {
    const int64_t rn = r0 + kPipe < L ? r0 + kPipe : r0;
    float nc[kPipe];
#pragma unroll
    for (int u = 0; u < kPipe; ++u) nc[u] = cur[(rn + u) * BN];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < kPipe; ++u)
      cur_step<PRE, SPK, PK, RULE, CK>(p, p.t_begin + r0 + u, cv[u], act, BN, gw, lane, m, cnt, o);
#pragma unroll
    for (int u = 0; u < kPipe; ++u) cv[u] = nc[u];
  }
  if (act) {
    if (p.m_final != nullptr) p.m_final[flat] = m;
    if (p.counts != nullptr) p.counts[flat] = cnt;
    if (p.rates != nullptr) p.rates[flat] = cnt / p.rate_denominator;
  }
}

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

bool al16(const void *q) { return q == nullptr || myelin::aligned(q, 16); }

template <int PREC, bool VA, bool VB, bool PA = false>
void launch_gemm_v(const GemmArgs &g, int ta, int tb, dim3 grid, hipStream_t s) {
  if (!ta && !tb)
    gemm_kernel<PREC, false, false, VA, VB, PA><<<grid, dim3(256), 0, s>>>(g);
  else if (!ta && tb)
    gemm_kernel<PREC, false, true, VA, VB, PA><<<grid, dim3(256), 0, s>>>(g);
  else if (ta && !tb)
    gemm_kernel<PREC, true, false, VA, VB, PA><<<grid, dim3(256), 0, s>>>(g);
  else
    gemm_kernel<PREC, true, true, VA, VB, PA><<<grid, dim3(256), 0, s>>>(g);
}

#ifndef MYELIN_SPLIT_WANT
#define MYELIN_SPLIT_WANT 512  // tile GEMMs split K below this many output tiles
#endif

// K splits for an output of `tiles` workgroups: split when the output alone
// gives under `want` workgroups and K is long.
template <int PREC>
int64_t plan_splits(int64_t tiles, int64_t K, int64_t want) {
  constexpr int KS = Prec<PREC>::KS;
  if (tiles >= want || K < 8 * KS) return 1;
  int64_t splits = cdiv(want, tiles);
  const int64_t max_by_k = K / (4 * KS);
  if (splits > max_by_k) splits = max_by_k;
  if (splits > 64) splits = 64;
  return splits < 1 ? 1 : splits;
}

// fp32 operands: the 128 x 128 kernel takes outputs of at least one full
// tile per side whose operands allow 16-byte loads
bool use_big(const GemmArgs &g) {
  return g.M >= kBig && g.N >= kBig && al16(g.A) && al16(g.B) && g.lda % 4 == 0 && g.ldb % 4 == 0;
}

// bf16 operands (128 x 128 kernel only): k-contiguous rows 16-byte aligned,
// mn-contiguous rows 8-byte aligned
bool bf16_aligned(const void *q, int64_t ld, bool kcontig) {
  return kcontig ? (myelin::aligned(q, 16) && ld % 8 == 0) : (myelin::aligned(q, 8) && ld % 4 == 0);
}

#ifndef MYELIN_TALL_MIN_K
#define MYELIN_TALL_MIN_K 2048  // k (all parts) from which bf16 k-contiguous products take 256 x 128 tiles
#endif

// bf16 operands, both k-contiguous, long K: 256 x 128 tiles of eight 64 x 64
// waves (two per SIMD, one workgroup per CU, 110 KB of LDS).  A stage's
// operand bytes from L2 per flop are 3/4 of the 128 x 128 tiles', which
// pays on long K when the tiles fill whole rounds of 256 CUs: at 4096
// columns and K = 3 x 1024, 8192 rows (4 rounds) 274 -> 242 us and 7200
// rows (3.6) 251 -> 235 us, but 6400 rows (3.1: a last round 1/8 full)
// 209 -> 224 us.  So the register-staged ones run when the last round is
// at least half full; the direct-load ones from half a round (below).
// Short K (784, 12 stages) measured slower (137 vs 113 us).
// (mn-contiguous operands on these tiles, with a K split filling the
// rounds, measured slower on the split dW: 348 vs 325 us at 1024 x 4096 x
// 3*7200.)
bool use_dma(const GemmArgs &g, int ta, int tb, bool half);

bool use_tall(const GemmArgs &g, int ta, int tb, bool half) {
  if (!half || ta || !tb || g.M < 256 || g.K * g.parts < MYELIN_TALL_MIN_K) return false;
  const int64_t tiles = cdiv(g.M, 256) * cdiv(g.N, 128);
  // direct-load tiles (their fragment reads interleaved with the MFMAs)
  // pay from half a round: 1440 x 4096 x 3 x 1024 47-48 us against 60-65
  // on the 128 x 128 tiles
  if (use_dma(g, ta, tb, half)) return tiles >= 128;
  return tiles >= 256 && (tiles % 256 == 0 || tiles % 256 >= 128);
}

#ifndef MYELIN_GEMM_DMA
#define MYELIN_GEMM_DMA 1
#endif

// Direct global -> LDS staging (gemm_dma): bf16 operands, both k-contiguous,
// 16-byte aligned rows, whole 64-k stages in every part and K split.
// the direct loaders address a tile's pieces by 32-bit byte offsets from
// a scalar base: 256 rows of the leading dimension stay below 2^31 bytes
constexpr int64_t kDmaMaxLd = int64_t{1} << 22;

bool use_dma(const GemmArgs &g, int ta, int tb, bool half) {
  return MYELIN_GEMM_DMA && half && !ta && tb && g.K % 64 == 0 && al16(g.A) && al16(g.B) && g.lda % 8 == 0 &&
         g.ldb % 8 == 0 && (g.parts == 1 || g.b_part % 8 == 0) && g.lda < kDmaMaxLd && g.ldb < kDmaMaxLd;
}

// three 48 KB stages (144 KB of LDS, one workgroup per CU): each stage's
// loads are issued two stages ahead of its MFMAs
void launch_dma_tall(const GemmArgs &g, dim3 grid, hipStream_t s) {
  if (g.parts > 1)
    gemm_dma<256, 128, true, 3><<<grid, dim3(512), 0, s>>>(g);
  else
    gemm_dma<256, 128, false, 3><<<grid, dim3(512), 0, s>>>(g);
}

// The same for bf16 operands both mn-contiguous (the weight-gradient
// products) on 128 x 128 tiles (gemm_dma_mn): whole 16-byte column pieces
// and aligned rows.
bool use_dma_mn(const GemmArgs &g, int ta, int tb, bool half) {
  return MYELIN_GEMM_DMA && half && ta && !tb && g.M % 8 == 0 && g.N % 8 == 0 && al16(g.A) && al16(g.B) &&
         g.lda % 8 == 0 && g.ldb % 8 == 0 && (g.parts == 1 || g.b_part % 8 == 0) && g.lda < kDmaMaxLd &&
         g.ldb < kDmaMaxLd;
}

// two 32 KB stages (two workgroups per CU).  Against register staging,
// measured beside it: the split dW of 1024 x 4096 x 3 x 7200 288 -> 175 us
// (629 -> 1034 TF), 784 x 2048 x 12800 113 -> 82 us; three stages (one
// workgroup per CU) measured 276 and 99 us.
void launch_dma_mn(const GemmArgs &g, dim3 grid, hipStream_t s) {
  if (g.parts > 1)
    gemm_dma_mn<true, 2><<<grid, dim3(256), 0, s>>>(g);
  else
    gemm_dma_mn<false, 2><<<grid, dim3(256), 0, s>>>(g);
}

// 256 x 256 tiles of eight 128 x 64 waves (a quarter fewer fragment reads
// per MFMA than 64 x 64 waves, twice the MFMAs per barrier), two 64 KB
// stages, for long-K products with direct staging whose 256 x 256 tiles
// fill whole-ish rounds of 256 workgroups.  Against the 256 x 128 tiles,
// measured beside them: 8192 x 4096 x 3 x 1024 217 -> 179 us (1154 TF),
// 7200 rows 201 -> 168 us, 8192 x 4096 x 3072 207 -> 174 us.
// One workgroup per CU on either direct-load shape, so a product takes
// ceil(tiles / 256) rounds of the chip; a 256 x 256 tile costs 1.74 tiles of
// 256 x 128 (7200 x 4096 x 3 x 1024: 148 against 171 us), so the wide tiles
// run when their rounds cost no more than the tall tiles' (2880 rows: 76
// against 86 us; 1440 rows take the tall tiles, 48 against 76 us).
bool use_wide(const GemmArgs &g, int ta, int tb, bool half) {
  if (!use_dma(g, ta, tb, half) || g.M < 256 || g.N < 256 || g.K * g.parts < MYELIN_TALL_MIN_K) return false;
  const int64_t wide = cdiv(g.M, 256) * cdiv(g.N, 256), tall = cdiv(g.M, 256) * cdiv(g.N, 128);
  return 174 * cdiv(wide, 256) <= 100 * cdiv(tall, 256);
}

void launch_dma_wide(const GemmArgs &g, dim3 grid, hipStream_t s) {
  if (g.parts > 1)
    gemm_dma<256, 256, true, 2, 4, 2><<<grid, dim3(512), 0, s>>>(g);
  else
    gemm_dma<256, 256, false, 2, 4, 2><<<grid, dim3(512), 0, s>>>(g);
}

#ifndef MYELIN_MN_WIDE_WANT
#define MYELIN_MN_WIDE_WANT 256  // K splits bring 256 x 256 mn-contiguous products to this many workgroups
#endif

// mn-contiguous products on 256 x 256 tiles of eight 128 x 64 waves, the
// K split filling the CUs: when the 128 x 128 tiles alone would fill at
// most one round of 256 CUs (and a workspace allows the split).  Measured
// beside the 128 x 128 tiles: the 784 -> 2048 layer's dW at T=50, B=256,
// 784 x 2048 x 12800 (112 tiles of 128 x 128), 83 -> 63 us; at a full round
// (the split dW of the 1024 -> 4096 layer at T=2000, B=32, 1024 x 4096
// x 3 x 7200, 256 tiles) they first measured slower (174 against 182 us),
// and since the fragment reads run a k step ahead and the loads take
// offsets from a scalar base, faster: that network's training step
// 7.36-7.39 -> 7.18-7.24 ms on one box.  Without a K split they are far slower;
// splitting to 512 workgroups measured slower than to 256.
bool use_dma_mn_wide(const GemmArgs &g, int ta, int tb, bool half) {
  return use_dma_mn(g, ta, tb, half) && g.ws != nullptr && g.M >= 256 && g.N >= 256 &&
         cdiv(g.M, 128) * cdiv(g.N, 128) <= 256 && cdiv(g.M, 256) * cdiv(g.N, 256) >= 32;
}

void launch_dma_mn_wide(const GemmArgs &g, dim3 grid, hipStream_t s) {
  if (g.parts > 1)
    gemm_dma_mn<true, 2, 256, 256, 4, 2><<<grid, dim3(512), 0, s>>>(g);
  else
    gemm_dma_mn<false, 2, 256, 256, 4, 2><<<grid, dim3(512), 0, s>>>(g);
}

void launch_tall(const GemmArgs &g, dim3 grid, hipStream_t s) {
  if (use_dma(g, 0, 1, true)) {
    launch_dma_tall(g, grid, s);
    return;
  }
  if (g.parts > 1)
    gemm_big<1, false, true, uint16_t, 256, 128, true><<<grid, dim3(512), 0, s>>>(g);
  else
    gemm_big<1, false, true, uint16_t, 256, 128><<<grid, dim3(512), 0, s>>>(g);
}

template <int PREC, bool TA, bool TB, int BM, int BN>
void launch_big(const GemmArgs &g, bool half, dim3 grid, hipStream_t s) {
  constexpr int NT = BM * BN / 64;
  if constexpr (PREC == 1) {
    if (half) {
      if constexpr (TA && !TB && BM == 128 && BN == 128) {
        if (use_dma_mn(g, 1, 0, true)) {
          launch_dma_mn(g, grid, s);
          return;
        }
      }
      if (g.parts > 1)
        gemm_big<1, TA, TB, uint16_t, BM, BN, true><<<grid, dim3(NT), 0, s>>>(g);
      else
        gemm_big<1, TA, TB, uint16_t, BM, BN><<<grid, dim3(NT), 0, s>>>(g);
      return;
    }
  }
  gemm_big<PREC, TA, TB, float, BM, BN><<<grid, dim3(NT), 0, s>>>(g);
}

// Only 128 x 128 tiles are launched: 256 x 128 (8 waves, 110 KB of LDS, so
// one workgroup per CU) measured slower on the synapse shapes, every stage
// barrier stalling all 8 waves where two 4-wave workgroups overlap.
template <int PREC, int BM, int BN>
void launch_big_t(const GemmArgs &g, int ta, int tb, bool half, dim3 grid, hipStream_t s) {
  if (!ta && !tb)
    launch_big<PREC, false, false, BM, BN>(g, half, grid, s);
  else if (!ta && tb)
    launch_big<PREC, false, true, BM, BN>(g, half, grid, s);
  else if (ta && !tb)
    launch_big<PREC, true, false, BM, BN>(g, half, grid, s);
  else
    launch_big<PREC, true, true, BM, BN>(g, half, grid, s);
}

// K splits of the narrow kernel: chunks of about MYELIN_NARROW_KCHUNK k (at
// most 64 of them), a function of K alone.  Each output element then sums
// the same k ranges in the same order whatever M is, so a layer's currents
// come out the same bits however its caller divides the rows (all time
// steps at once, or a group of checkpoint chunks at a time) -- which keeps
// two routes through a network whose surrogate adjoint amplifies rounding
// over thousands of steps on the same trajectory.
int64_t narrow_splits(int64_t K) {
  int64_t s = cdiv(K, MYELIN_NARROW_KCHUNK);
  if (s > 64) s = 64;
  return s < 1 ? 1 : s;
}

template <int PREC, bool TA, bool TB, bool PA>
void launch_narrow_v(const GemmArgs &g, bool va, dim3 grid, hipStream_t s) {
  if constexpr (!TA && !PA) {
    if (va) {
      gemm_narrow<PREC, TA, TB, PA, true><<<grid, dim3(256), 0, s>>>(g);
      return;
    }
  }
  gemm_narrow<PREC, TA, TB, PA, false><<<grid, dim3(256), 0, s>>>(g);
}

template <bool TA, bool TB, bool PA>
void launch_narrow_x3_v(const GemmArgs &g, bool va, dim3 grid, hipStream_t s) {
  if constexpr (!TA && !PA) {
    if (va) {
      gemm_narrow_x3<TA, TB, PA, true><<<grid, dim3(256), 0, s>>>(g);
      return;
    }
  }
  gemm_narrow_x3<TA, TB, PA, false><<<grid, dim3(256), 0, s>>>(g);
}

template <bool PA>
void launch_narrow_x3(const GemmArgs &g, int ta, int tb, bool va, dim3 grid, hipStream_t s) {
  if (!ta && !tb)
    launch_narrow_x3_v<false, false, PA>(g, va, grid, s);
  else if (!ta)
    launch_narrow_x3_v<false, true, PA>(g, va, grid, s);
  else if (!tb)
    launch_narrow_x3_v<true, false, PA>(g, va, grid, s);
  else
    launch_narrow_x3_v<true, true, PA>(g, va, grid, s);
}

template <int PREC, bool PA>
void launch_narrow(const GemmArgs &g, int ta, int tb, bool va, dim3 grid, hipStream_t s) {
  if (!ta && !tb)
    launch_narrow_v<PREC, false, false, PA>(g, va, grid, s);
  else if (!ta)
    launch_narrow_v<PREC, false, true, PA>(g, va, grid, s);
  else if (!tb)
    launch_narrow_v<PREC, true, false, PA>(g, va, grid, s);
  else
    launch_narrow_v<PREC, true, true, PA>(g, va, grid, s);
}

template <int PREC, bool PA, int KMAX, bool VC>
void launch_smallk_k(const GemmArgs &g, int ta, int tb, dim3 grid, hipStream_t s) {
  if (!ta && !tb)
    gemm_smallk<PREC, false, false, PA, KMAX, VC><<<grid, dim3(256), 0, s>>>(g);
  else if (!ta)
    gemm_smallk<PREC, false, true, PA, KMAX, VC><<<grid, dim3(256), 0, s>>>(g);
  else if (!tb)
    gemm_smallk<PREC, true, false, PA, KMAX, VC><<<grid, dim3(256), 0, s>>>(g);
  else
    gemm_smallk<PREC, true, true, PA, KMAX, VC><<<grid, dim3(256), 0, s>>>(g);
}

template <int PREC, bool PA, int KMAX>
void launch_smallk_c(const GemmArgs &g, int ta, int tb, dim3 grid, hipStream_t s) {
  if (al16(g.C) && g.ldc % 4 == 0)
    launch_smallk_k<PREC, PA, KMAX, true>(g, ta, tb, grid, s);
  else
    launch_smallk_k<PREC, PA, KMAX, false>(g, ta, tb, grid, s);
}

// K <= 32, unrolled to the next multiple of 4 from 8 up to 24, else 32
// (the padded k cost full multiply-adds: the kernel is bound by them)
template <int PREC, bool PA>
void launch_smallk(const GemmArgs &g, int ta, int tb, dim3 grid, hipStream_t s) {
  if (g.K <= 8)
    launch_smallk_c<PREC, PA, 8>(g, ta, tb, grid, s);
  else if (g.K <= 12)
    launch_smallk_c<PREC, PA, 12>(g, ta, tb, grid, s);
  else if (g.K <= 16)
    launch_smallk_c<PREC, PA, 16>(g, ta, tb, grid, s);
  else if (g.K <= 20)
    launch_smallk_c<PREC, PA, 20>(g, ta, tb, grid, s);
  else if (g.K <= 24)
    launch_smallk_c<PREC, PA, 24>(g, ta, tb, grid, s);
  else
    launch_smallk_c<PREC, PA, 32>(g, ta, tb, grid, s);
}

template <int PREC>
int launch_gemm(GemmArgs g, int ta, int tb, bool half, int64_t ws_elems, hipStream_t s, bool bits = false,
                bool *reduced = nullptr) {
  constexpr int KS = Prec<PREC>::KS;
  if (!half && g.N <= 32) {
    // narrow output (readout currents, dW_o): stream A once
    int64_t splits = g.ws != nullptr ? narrow_splits(g.K) : 1;
    while (splits > 1 && splits * g.M * g.N > ws_elems) --splits;
    g.kchunk = cdiv(cdiv(g.K, splits), 64) * 64;
    splits = cdiv(g.K, g.kchunk);
    g.splits = static_cast<int>(splits);
    const dim3 grid(static_cast<unsigned>(cdiv(g.M, 128)), static_cast<unsigned>(splits));
    const bool va = !bits && al16(g.A) && g.lda % 4 == 0;
    if (bits && !ta && !tb && cdiv(g.M, 32 * NarrowBits<1>::WAVES) * splits >= 512) {
      // row-major bit rows with two rounds of eight-wave workgroups (fewer
      // measured slower: 12800 x 2048 x 10, 200 workgroups, 13 -> 16 us)
      const dim3 wide(static_cast<unsigned>(cdiv(g.M, 32 * NarrowBits<1>::WAVES)), static_cast<unsigned>(splits));
      if constexpr (PREC == 0)
        gemm_narrow_bits<3><<<wide, dim3(64 * NarrowBits<3>::WAVES), 0, s>>>(g);
      else
        gemm_narrow_bits<1><<<wide, dim3(64 * NarrowBits<1>::WAVES), 0, s>>>(g);
    } else if (bits && ta && !tb && cdiv(cdiv(g.M, 32), NarrowBitsT<1>::COLS) * splits >= MYELIN_BITS_T_MIN_WG) {
      // transposed bit rows (dW_o): word columns turned around in registers
      const dim3 cols(static_cast<unsigned>(cdiv(cdiv(g.M, 32), NarrowBitsT<1>::COLS)), static_cast<unsigned>(splits));
      if constexpr (PREC == 0)
        gemm_narrow_bits_t<3><<<cols, dim3(64 * NarrowBitsT<3>::WAVES), 0, s>>>(g);
      else
        gemm_narrow_bits_t<1><<<cols, dim3(64 * NarrowBitsT<1>::WAVES), 0, s>>>(g);
    } else if constexpr (PREC == 0) {
      // fp32: the exact three-plane split on the bf16 MFMA
      if (bits)
        launch_narrow_x3<true>(g, ta, tb, va, grid, s);
      else
        launch_narrow_x3<false>(g, ta, tb, va, grid, s);
    } else if (bits) {
      launch_narrow<PREC, true>(g, ta, tb, va, grid, s);
    } else {
      launch_narrow<PREC, false>(g, ta, tb, va, grid, s);
    }
    if (int rc = myelin::launched("gemm (narrow)")) return rc;
    if (splits > 1) {
      launch_reduce(g, s);
      if (reduced != nullptr) *reduced = true;
      return myelin::launched("gemm split-k reduce");
    }
    return MYELIN_OK;
  }
  if (!half && g.K <= 32) {
    // tiny K (dS = G_o W_o^T): one pass over the output
    const int64_t wgs = cdiv(g.N, 256) * cdiv(g.M, 4 * MYELIN_SMALLK_RW);
    if (wgs > 0x7fffffff) return myelin::invalid("gemm: output too large (%lld x %lld)", (long long)g.M, (long long)g.N);
    g.splits = 1;
    const dim3 grid(static_cast<unsigned>(wgs));
    if (bits)
      launch_smallk<PREC, true>(g, ta, tb, grid, s);
    else
      launch_smallk<PREC, false>(g, ta, tb, grid, s);
    return myelin::launched("gemm (small K)");
  }
  const bool big = !bits && (half || use_big(g));
  if constexpr (PREC == 1) {
    // the 256 x 256 mn-contiguous tiles pay only with a K split (their
    // grid is under one round of the chip): plan it first, and take the
    // 128 x 128 tiles below when K or the workspace allows no split
    if (!bits && use_dma_mn_wide(g, ta, tb, half)) {
      const int64_t tiles = cdiv(g.M, 256) * cdiv(g.N, 256);
      if (tiles > 0x7fffffff) return myelin::invalid("gemm: output too large");
      int64_t splits = plan_splits<1>(tiles, g.K, MYELIN_MN_WIDE_WANT);
      while (splits > 1 && splits * g.M * g.N > ws_elems) --splits;
      const int64_t kchunk = cdiv(cdiv(g.K, splits), KS) * KS;
      splits = cdiv(g.K, kchunk);
      if (splits > 1) {
        g.kchunk = kchunk;
        g.splits = static_cast<int>(splits);
        launch_dma_mn_wide(g, dim3(static_cast<unsigned>(tiles), static_cast<unsigned>(splits)), s);
        if (int rc = myelin::launched("gemm (mn-contiguous, 256 x 256 tiles)")) return rc;
        launch_reduce(g, s);
        if (reduced != nullptr) *reduced = true;
        return myelin::launched("gemm split-k reduce");
      }
    }
    if (!bits && use_wide(g, ta, tb, half)) {
      const int64_t tiles = cdiv(g.M, 256) * cdiv(g.N, 256);
      if (tiles > 0x7fffffff) return myelin::invalid("gemm: output too large");
      g.kchunk = cdiv(g.K, Prec<1>::KS) * Prec<1>::KS;  // no K split
      g.splits = 1;
      launch_dma_wide(g, dim3(static_cast<unsigned>(tiles)), s);
      return myelin::launched("gemm (256 x 256 tiles)");
    }
    if (!bits && use_tall(g, ta, tb, half)) {
      g.kchunk = cdiv(g.K, Prec<1>::KS) * Prec<1>::KS;  // no K split
      g.splits = 1;
      const int64_t tiles = cdiv(g.M, 256) * cdiv(g.N, 128);
      if (tiles > 0x7fffffff) return myelin::invalid("gemm: output too large");
      launch_tall(g, dim3(static_cast<unsigned>(tiles)), s);
      return myelin::launched("gemm (256 x 128 tiles)");
    }
  }
  const int64_t edge = big ? kBig : kTile;
  const int64_t tiles = cdiv(g.N, edge) * cdiv(g.M, edge);
  if (!big && cdiv(g.M, kTile) > 65535) return myelin::invalid("gemm: M too large (%lld)", (long long)g.M);
  int64_t splits = g.ws != nullptr ? plan_splits<PREC>(tiles, g.K, MYELIN_SPLIT_WANT) : 1;
  while (splits > 1 && splits * g.M * g.N > ws_elems) --splits;
  g.kchunk = cdiv(cdiv(g.K, splits), KS) * KS;
  splits = cdiv(g.K, g.kchunk);
  if (splits < 1) splits = 1;
  g.splits = static_cast<int>(splits);
  if (big) {
    const dim3 grid(static_cast<unsigned>(tiles), static_cast<unsigned>(splits));
    launch_big_t<PREC, kBig, kBig>(g, ta, tb, half, grid, s);
  } else {
    const dim3 grid(cdiv(g.N, kTile), cdiv(g.M, kTile), static_cast<unsigned>(splits));
    // 16-byte loads per operand where its base and leading dimension allow
    const bool va = al16(g.A) && g.lda % 4 == 0, vb = al16(g.B) && g.ldb % 4 == 0;
    if (bits) {
      if (vb)
        launch_gemm_v<PREC, false, true, true>(g, ta, tb, grid, s);
      else
        launch_gemm_v<PREC, false, false, true>(g, ta, tb, grid, s);
    } else if (va && vb)
      launch_gemm_v<PREC, true, true>(g, ta, tb, grid, s);
    else if (va)
      launch_gemm_v<PREC, true, false>(g, ta, tb, grid, s);
    else if (vb)
      launch_gemm_v<PREC, false, true>(g, ta, tb, grid, s);
    else
      launch_gemm_v<PREC, false, false>(g, ta, tb, grid, s);
  }
  if (int rc = myelin::launched("gemm")) return rc;
  if (splits > 1) {
    launch_reduce(g, s);
    if (reduced != nullptr) *reduced = true;
    return myelin::launched("gemm split-k reduce");
  }
  return MYELIN_OK;
}

template <int SID, int V, int RULE>
void launch_pre_bwd_r(const PreBwdArgs &a, bool gs, int gm, dim3 grid, hipStream_t s) {
  if (gs) {
    if (gm == 2)
      linear_pre_bwd<SID, true, 2, V, RULE><<<grid, dim3(256), 0, s>>>(a);
    else if (gm == 1)
      linear_pre_bwd<SID, true, 1, V, RULE><<<grid, dim3(256), 0, s>>>(a);
    else
      linear_pre_bwd<SID, true, 0, V, RULE><<<grid, dim3(256), 0, s>>>(a);
  } else {
    if (gm == 2)
      linear_pre_bwd<SID, false, 2, V, RULE><<<grid, dim3(256), 0, s>>>(a);
    else if (gm == 1)
      linear_pre_bwd<SID, false, 1, V, RULE><<<grid, dim3(256), 0, s>>>(a);
    else
      linear_pre_bwd<SID, false, 0, V, RULE><<<grid, dim3(256), 0, s>>>(a);
  }
}

template <int SID, int V>
void launch_pre_bwd_v(const PreBwdArgs &a, bool gs, int gm, dim3 grid, hipStream_t s) {
  if constexpr (V == 1) {
    if (a.rule == MYELIN_RULE_THRESHOLD)
      launch_pre_bwd_r<SID, V, MYELIN_RULE_THRESHOLD>(a, gs, gm, grid, s);
    else
      launch_pre_bwd_r<SID, V, MYELIN_RULE_SURROGATE>(a, gs, gm, grid, s);
  } else {
    launch_pre_bwd_r<SID, V, -1>(a, gs, gm, grid, s);
  }
}

// two neurons per lane where BN is even, every operand is 8-byte aligned and
// the grid stays wide (>= 512 waves): on a few waves the serial walk is the
// cost, and two neurons per lane double it (640 neurons x 2000 steps: 164
// -> 278 us), while wide grids gain from the 8-byte accesses (131072 x
// 225: 74 -> 68 us; 524288 x 256: 333 -> 315 us)
template <int SID>
void launch_pre_bwd(const PreBwdArgs &a, bool gs, int gm, hipStream_t s) {
  const bool v2 = a.BN >= 65536 && a.BN % 2 == 0 && myelin::aligned(a.pre, 8) && myelin::aligned(a.gs, 8) &&
                  myelin::aligned(a.gm, 8) && myelin::aligned(a.grate, 8) && myelin::aligned(a.gbias_acc, 8) &&
                  myelin::aligned(a.G, gm == 0 ? 8 : 4);
  if (v2)
    launch_pre_bwd_v<SID, 2>(a, gs, gm, dim3(cdiv(a.BN / 2, 256)), s);
  else
    launch_pre_bwd_v<SID, 1>(a, gs, gm, dim3(cdiv(a.BN, 256)), s);
}

// the spike-gradient-forming reverse pass: KMAX the small-K GEMM's
// unroll for K = O (8, 12, ..., 24, then 32), so the two sum alike
constexpr int64_t kPreBwdDsLds = 65536;  // bytes of staged G_o rows per workgroup

int pre_bwd_ds_kmax(int O) { return O <= 8 ? 8 : O <= 12 ? 12 : O <= 16 ? 16 : O <= 20 ? 20 : O <= 24 ? 24 : 32; }

template <int SID, int GM>
void launch_pre_bwd_ds_k(const PreBwdArgs &a, const float *go, const float *wo, int O, int64_t N, hipStream_t s) {
  const int kmax = pre_bwd_ds_kmax(O);
  const dim3 grid(static_cast<unsigned>(a.BN / 256));
  const size_t lds = static_cast<size_t>(a.C) * kmax * sizeof(float);
  switch (kmax) {
    case 8: linear_pre_bwd_ds<SID, GM, 8><<<grid, dim3(256), lds, s>>>(a, go, wo, O, N); break;
    case 12: linear_pre_bwd_ds<SID, GM, 12><<<grid, dim3(256), lds, s>>>(a, go, wo, O, N); break;
    case 16: linear_pre_bwd_ds<SID, GM, 16><<<grid, dim3(256), lds, s>>>(a, go, wo, O, N); break;
    case 20: linear_pre_bwd_ds<SID, GM, 20><<<grid, dim3(256), lds, s>>>(a, go, wo, O, N); break;
    case 24: linear_pre_bwd_ds<SID, GM, 24><<<grid, dim3(256), lds, s>>>(a, go, wo, O, N); break;
    default: linear_pre_bwd_ds<SID, GM, 32><<<grid, dim3(256), lds, s>>>(a, go, wo, O, N); break;
  }
}

template <int SID>
void launch_pre_bwd_ds(const PreBwdArgs &a, int gm, const float *go, const float *wo, int O, int64_t N,
                       hipStream_t s) {
  if (gm == 2)
    launch_pre_bwd_ds_k<SID, 2>(a, go, wo, O, N, s);
  else
    launch_pre_bwd_ds_k<SID, 0>(a, go, wo, O, N, s);
}

template <bool PRE, bool SPK, bool PK>
void launch_cur_rule(const CurArgs &a, dim3 grid, hipStream_t s) {
  const bool ck = a.ckpt != nullptr;
  if (a.rule == MYELIN_RULE_THRESHOLD) {
    if (ck)
      lif_currents_fwd<PRE, SPK, PK, MYELIN_RULE_THRESHOLD, true><<<grid, dim3(256), 0, s>>>(a);
    else
      lif_currents_fwd<PRE, SPK, PK, MYELIN_RULE_THRESHOLD, false><<<grid, dim3(256), 0, s>>>(a);
  } else {
    if (ck)
      lif_currents_fwd<PRE, SPK, PK, MYELIN_RULE_SURROGATE, true><<<grid, dim3(256), 0, s>>>(a);
    else
      lif_currents_fwd<PRE, SPK, PK, MYELIN_RULE_SURROGATE, false><<<grid, dim3(256), 0, s>>>(a);
  }
}

template <bool PRE, bool SPK>
void launch_cur_pk(const CurArgs &a, bool pk, dim3 grid, hipStream_t s) {
  if (pk)
    launch_cur_rule<PRE, SPK, true>(a, grid, s);
  else
    launch_cur_rule<PRE, SPK, false>(a, grid, s);
}

void launch_currents(const CurArgs &a, dim3 grid, hipStream_t s) {
  const bool pre = a.pre != nullptr, spk = a.spikes != nullptr, pk = a.packed != nullptr;
  if (pre && spk)
    launch_cur_pk<true, true>(a, pk, grid, s);
  else if (pre)
    launch_cur_pk<true, false>(a, pk, grid, s);
  else if (spk)
    launch_cur_pk<false, true>(a, pk, grid, s);
  else
    launch_cur_pk<false, false>(a, pk, grid, s);
}

}  // namespace

extern "C" int64_t myelin_gemm_workspace_elems(int64_t M, int64_t N, int64_t K, int precision) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  // the largest split any kernel for this output could use
  int64_t most = N <= 32 ? narrow_splits(K) : 1;
  for (int64_t edge : {static_cast<int64_t>(kTile), static_cast<int64_t>(kBig)}) {
    const int64_t tiles = cdiv(M, edge) * cdiv(N, edge);
    const int64_t s = precision == MYELIN_PREC_BF16 ? plan_splits<1>(tiles, K, MYELIN_SPLIT_WANT) : plan_splits<0>(tiles, K, MYELIN_SPLIT_WANT);
    if (s > most) most = s;
  }
  if (precision == MYELIN_PREC_BF16) {
    // the 256 x 256 mn-contiguous tiles
    const int64_t s = plan_splits<1>(cdiv(M, 256) * cdiv(N, 256), K, MYELIN_MN_WIDE_WANT);
    if (s > most) most = s;
  }
  return most > 1 ? most * M * N : 0;
}

namespace {
// the column sum attached to a GEMM, as a launch of its own when no split-K
// reduce launch has run it
int run_col_sum(const float *in, float *out, int64_t rows, int64_t cols, hipStream_t s) {
  if (cols == 0) return MYELIN_OK;
  col_sum<<<dim3(static_cast<unsigned>(cdiv(cols, 8))), dim3(256), 0, s>>>(in, out, rows, cols, 0);
  return myelin::launched("col_sum");
}

int col_sum_after(const GemmArgs &g, bool reduced, hipStream_t s) {
  if (g.cs_in == nullptr || reduced) return MYELIN_OK;
  return run_col_sum(g.cs_in, g.cs_out, g.cs_rows, g.cs_cols, s);
}

int check_col_sum(const float *cs_in, float *cs_out, int64_t cs_rows, int64_t cs_cols) {
  if (cs_rows < 0 || cs_cols < 0) return myelin::invalid("col_sum: negative size");
  if (cs_cols > 0 && (cs_out == nullptr || (cs_rows > 0 && cs_in == nullptr)))
    return myelin::invalid("col_sum: null pointer");
  if (cdiv(cs_cols, 8) > 0x3fffffff) return myelin::invalid("col_sum: too many columns");
  return MYELIN_OK;
}

int gemm_impl(const void *A, int a_dtype, const void *B, int b_dtype, const float *bias, float *C, int64_t M,
              int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t ldc, int trans_a, int trans_b, int accumulate,
              int precision, float *workspace, int64_t workspace_elems, const float *cs_in, float *cs_out,
              int64_t cs_rows, int64_t cs_cols, myelin_stream_t stream) {
  if (M < 0 || N < 0 || K < 0) return myelin::invalid("gemm: negative size");
  GemmArgs g{A, B, bias, C, workspace_elems > 0 ? workspace : nullptr, M, N, K, lda, ldb, ldc, 0, accumulate, 1};
  if (cs_cols > 0) {
    g.cs_in = cs_in;
    g.cs_out = cs_out;
    g.cs_rows = cs_rows;
    g.cs_cols = cs_cols;
  }
  if (M == 0 || N == 0) return col_sum_after(g, false, myelin::as_hip(stream));
  if (A == nullptr || B == nullptr || C == nullptr) return myelin::invalid("gemm: null pointer");
  if (ldc < N) return myelin::invalid("gemm: ldc < N");
  if ((a_dtype != MYELIN_DT_BITS && (trans_a ? lda < M : lda < K)) || (trans_b ? ldb < K : ldb < N))
    return myelin::invalid("gemm: bad leading dim");
  if (workspace_elems < 0) return myelin::invalid("gemm: negative workspace size");
  if (precision != MYELIN_PREC_BF16 && precision != MYELIN_PREC_F32)
    return myelin::invalid("gemm: unknown precision %d", precision);
  const bool bits = a_dtype == MYELIN_DT_BITS;
  if (bits) {
    if (b_dtype != MYELIN_DT_F32) return myelin::invalid("gemm: packed-bit A needs a float32 B");
    if (trans_a ? lda < (M + 31) / 32 : lda < (K + 31) / 32)
      return myelin::invalid("gemm: packed-bit A: lda (words per row) too small");
  } else if ((a_dtype != MYELIN_DT_F32 && a_dtype != MYELIN_DT_BF16) || b_dtype != a_dtype) {
    return myelin::invalid("gemm: operands must both be float32 or both bfloat16 (or packed-bit A, float32 B)");
  }
  const bool half = a_dtype == MYELIN_DT_BF16;
  if (half) {
    if (precision != MYELIN_PREC_BF16) return myelin::invalid("gemm: bfloat16 operands need bf16 precision");
    if (!bf16_aligned(A, lda, !trans_a) || !bf16_aligned(B, ldb, trans_b != 0))
      return myelin::invalid("gemm: bfloat16 operand rows must be 16-byte (k-contiguous) or 8-byte aligned");
  }
  if (K == 0) {  // C = (accumulate ? C : 0) + bias
    g.splits = 0;
    launch_reduce(g, myelin::as_hip(stream));
    return myelin::launched("gemm (K = 0)");
  }
  hipStream_t s = myelin::as_hip(stream);
  bool reduced = false;
  const int rc = precision == MYELIN_PREC_BF16
                     ? launch_gemm<1>(g, trans_a, trans_b, half, workspace_elems, s, bits, &reduced)
                     : launch_gemm<0>(g, trans_a, trans_b, false, workspace_elems, s, bits, &reduced);
  return rc != MYELIN_OK ? rc : col_sum_after(g, reduced, s);
}

int gemm_parts_impl(const uint16_t *A, const uint16_t *B, int parts, int64_t b_part, const float *bias, float *C,
                    int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t ldc, int trans_a, int trans_b,
                    int accumulate, float *workspace, int64_t workspace_elems, const float *cs_in, float *cs_out,
                    int64_t cs_rows, int64_t cs_cols, myelin_stream_t stream) {
  if (parts < 1 || parts > 8) return myelin::invalid("gemm_parts: parts must be in [1, 8]");
  if (parts > 1 && b_part < 0) return myelin::invalid("gemm_parts: negative part stride");
  if (M < 0 || N < 0 || K < 0) return myelin::invalid("gemm_parts: negative size");
  if (M == 0 || N == 0) return run_col_sum(cs_in, cs_out, cs_rows, cs_cols, myelin::as_hip(stream));
  if (A == nullptr || B == nullptr || C == nullptr) return myelin::invalid("gemm_parts: null pointer");
  if (ldc < N) return myelin::invalid("gemm_parts: ldc < N");
  if ((trans_a ? lda < M : lda < K) || (trans_b ? ldb < K : ldb < N)) return myelin::invalid("gemm_parts: bad leading dim");
  if (workspace_elems < 0) return myelin::invalid("gemm_parts: negative workspace size");
  // every part must satisfy the bf16 loaders' alignment, as B itself does
  if (!bf16_aligned(A, lda, !trans_a) || !bf16_aligned(B, ldb, trans_b != 0) ||
      (parts > 1 && !bf16_aligned(B + b_part, ldb, trans_b != 0)))
    return myelin::invalid("gemm_parts: bfloat16 operand rows must be 16-byte (k-contiguous) or 8-byte aligned");
  // The parts are summed from the last to the first: for the planes of an
  // exact split (largest first in memory) the smallest plane's products
  // then accumulate while the running sum is small, and only the largest
  // plane's products round against the full-size sum, as in a plain fp32
  // GEMM.  Summed largest first, each of the three planes' products rounds
  // against the full sum: the currents of a 1024 -> 4096 synapse over 8000
  // rows of spikes measured 5.3e-7 (max) / 2.9e-8 (rms) from float64 that
  // way, 6.8e-8 / 6.1e-9 this way (a CPU sgemm: 1.5e-7 / 1.3e-8).
  GemmArgs g{A, B + (parts - 1) * b_part, bias, C, workspace_elems > 0 ? workspace : nullptr,
             M, N, K, lda, ldb, ldc, 0, accumulate, 1};
  g.parts = parts;
  g.b_part = -b_part;
  if (cs_cols > 0) {
    g.cs_in = cs_in;
    g.cs_out = cs_out;
    g.cs_rows = cs_rows;
    g.cs_cols = cs_cols;
  }
  hipStream_t s = myelin::as_hip(stream);
  if (K == 0) {  // C = (accumulate ? C : 0) + bias
    g.splits = 0;
    launch_reduce(g, s);
    return myelin::launched("gemm_parts (K = 0)");
  }
  bool reduced = false;
  const int rc = launch_gemm<1>(g, trans_a, trans_b, true, workspace_elems, s, false, &reduced);
  return rc != MYELIN_OK ? rc : col_sum_after(g, reduced, s);
}
}  // namespace

extern "C" int myelin_gemm(const void *A, int a_dtype, const void *B, int b_dtype, const float *bias, float *C,
                           int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t ldc, int trans_a,
                           int trans_b, int accumulate, int precision, float *workspace, int64_t workspace_elems,
                           myelin_stream_t stream) {
  return gemm_impl(A, a_dtype, B, b_dtype, bias, C, M, N, K, lda, ldb, ldc, trans_a, trans_b, accumulate, precision,
                   workspace, workspace_elems, nullptr, nullptr, 0, 0, stream);
}

extern "C" int myelin_gemm_col_sum(const void *A, int a_dtype, const void *B, int b_dtype, const float *bias,
                                   float *C, int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t ldc,
                                   int trans_a, int trans_b, int accumulate, int precision, float *workspace,
                                   int64_t workspace_elems, const float *cs_in, float *cs_out, int64_t cs_rows,
                                   int64_t cs_cols, myelin_stream_t stream) {
  if (int rc = check_col_sum(cs_in, cs_out, cs_rows, cs_cols)) return rc;
  return gemm_impl(A, a_dtype, B, b_dtype, bias, C, M, N, K, lda, ldb, ldc, trans_a, trans_b, accumulate, precision,
                   workspace, workspace_elems, cs_in, cs_out, cs_rows, cs_cols, stream);
}

extern "C" int myelin_gemm_parts(const uint16_t *A, const uint16_t *B, int parts, int64_t b_part, const float *bias,
                                 float *C, int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t ldc,
                                 int trans_a, int trans_b, int accumulate, float *workspace, int64_t workspace_elems,
                                 myelin_stream_t stream) {
  return gemm_parts_impl(A, B, parts, b_part, bias, C, M, N, K, lda, ldb, ldc, trans_a, trans_b, accumulate,
                         workspace, workspace_elems, nullptr, nullptr, 0, 0, stream);
}

extern "C" int myelin_gemm_parts_col_sum(const uint16_t *A, const uint16_t *B, int parts, int64_t b_part,
                                         const float *bias, float *C, int64_t M, int64_t N, int64_t K, int64_t lda,
                                         int64_t ldb, int64_t ldc, int trans_a, int trans_b, int accumulate,
                                         float *workspace, int64_t workspace_elems, const float *cs_in, float *cs_out,
                                         int64_t cs_rows, int64_t cs_cols, myelin_stream_t stream) {
  if (int rc = check_col_sum(cs_in, cs_out, cs_rows, cs_cols)) return rc;
  return gemm_parts_impl(A, B, parts, b_part, bias, C, M, N, K, lda, ldb, ldc, trans_a, trans_b, accumulate,
                         workspace, workspace_elems, cs_in, cs_out, cs_rows, cs_cols, stream);
}

extern "C" int myelin_gemm_f32(const float *A, const float *B, const float *bias, float *C, int64_t M, int64_t N,
                               int64_t K, int64_t lda, int64_t ldb, int64_t ldc, int trans_a, int trans_b,
                               int accumulate, int precision, float *workspace, int64_t workspace_elems,
                               myelin_stream_t stream) {
  return myelin_gemm(A, MYELIN_DT_F32, B, MYELIN_DT_F32, bias, C, M, N, K, lda, ldb, ldc, trans_a, trans_b,
                     accumulate, precision, workspace, workspace_elems, stream);
}

namespace {
int fill_lin(LinArgs &a, const float *bias, const float *m0, float *m_final, float *spikes, float *pre,
             int32_t *packed, float *rates, float *ckpt, int64_t T, int64_t B, int64_t F, int64_t N, int64_t t_begin,
             int64_t t_end, int64_t ckpt_every, float decay, float threshold, float reset, float slope, int rule) {
  if (T < 1 || B < 1 || F < 1 || N < 1) return myelin::invalid("linear_lif_fwd: T, B, F, N must be positive");
  if (t_begin < 0 || t_end > T || t_begin >= t_end) return myelin::invalid("linear_lif_fwd: bad time range");
  if (ckpt != nullptr && ckpt_every < 1) return myelin::invalid("linear_lif_fwd: ckpt_every must be positive");
  if (rule != MYELIN_RULE_THRESHOLD && rule != MYELIN_RULE_SURROGATE)
    return myelin::invalid("linear_lif_fwd: unknown rule %d", rule);
  a.bias = bias;
  a.m0 = m0;
  a.m_final = m_final;
  a.spikes = spikes;
  a.pre = pre;
  a.packed = packed;
  a.rates = rates;
  a.ckpt = ckpt;
  a.T = T;
  a.B = B;
  a.F = F;
  a.N = N;
  a.t_begin = t_begin;
  a.t_end = t_end;
  a.ckpt_every = ckpt_every < 1 ? 1 : ckpt_every;
  a.W = (N + 31) / 32;
  a.decay = decay;
  a.thr = threshold;
  a.reset = reset;
  a.slope = slope;
  a.rate_denominator = static_cast<float>(T);
  a.rule = rule;
  return MYELIN_OK;
}
}  // namespace

extern "C" int myelin_linear_lif_fwd_bf16(const uint16_t *x, const uint16_t *wt, const float *bias, const float *m0,
                                          float *m_final, float *spikes, float *pre, int32_t *packed, float *rates,
                                          float *ckpt, int64_t T, int64_t B, int64_t F, int64_t N, int64_t t_begin,
                                          int64_t t_end, int64_t ckpt_every, float decay, float threshold,
                                          float reset, float slope, int rule, myelin_stream_t stream) {
  if (x == nullptr || wt == nullptr) return myelin::invalid("linear_lif_fwd_bf16: x and wt are required");
  LinArgs a{};
  if (int rc = fill_lin(a, bias, m0, m_final, spikes, pre, packed, rates, ckpt, T, B, F, N, t_begin, t_end,
                        ckpt_every, decay, threshold, reset, slope, rule))
    return rc;
  if (!myelin::aligned(x, 16) || !myelin::aligned(wt, 16) || F % 8 != 0)
    return myelin::invalid("linear_lif_fwd_bf16: x and wt need 16-byte aligned rows (F %% 8 == 0)");
  a.xh = x;
  a.wt = wt;
  hipStream_t s = myelin::as_hip(stream);
  // 16 batch rows x 128 neurons per workgroup (one per CU, 144 KB of LDS),
  // the recurrence run from the accumulators under the next chunk's GEMM,
  // when that fills at least three quarters of the chip and its 32-bit
  // offsets fit (a step's [B, N] trace, 16 steps of x); otherwise the 8- /
  // 16-row tiles below
  const int64_t acc_tiles = cdiv(N, acc_fwd::BN) * cdiv(B, 16);
  if (acc_tiles >= 192 && acc_tiles <= 0x7fffffff && B * N < (int64_t{1} << 30) && B * F < (int64_t{1} << 27)) {
    const dim3 grid(static_cast<unsigned>(acc_tiles)), block(acc_fwd::NT);
    const int outs = lin_outputs(a);
    const bool thr = a.rule == MYELIN_RULE_THRESHOLD;
    // a training forward (trace + spikes, with or without their packed
    // twin), an inference forward (spikes), anything else
    if (outs == 7)
      thr ? linear_lif_fwd_pipe<MYELIN_RULE_THRESHOLD, 7><<<grid, block, 0, s>>>(a)
          : linear_lif_fwd_pipe<MYELIN_RULE_SURROGATE, 7><<<grid, block, 0, s>>>(a);
    else if (outs == 3)
      thr ? linear_lif_fwd_pipe<MYELIN_RULE_THRESHOLD, 3><<<grid, block, 0, s>>>(a)
          : linear_lif_fwd_pipe<MYELIN_RULE_SURROGATE, 3><<<grid, block, 0, s>>>(a);
    else if (outs == 2)
      thr ? linear_lif_fwd_pipe<MYELIN_RULE_THRESHOLD, 2><<<grid, block, 0, s>>>(a)
          : linear_lif_fwd_pipe<MYELIN_RULE_SURROGATE, 2><<<grid, block, 0, s>>>(a);
    else
      thr ? linear_lif_fwd_pipe<MYELIN_RULE_THRESHOLD, -1><<<grid, block, 0, s>>>(a)
          : linear_lif_fwd_pipe<MYELIN_RULE_SURROGATE, -1><<<grid, block, 0, s>>>(a);
    return myelin::launched("linear_lif_fwd_bf16 (pipelined recurrence)");
  }
  const int bt = (cdiv(N, kBig) * cdiv(B, 16) >= 512) ? 16 : 8;
  const dim3 grid(cdiv(N, kBig), cdiv(B, bt));
  if (grid.y > 65535) return myelin::invalid("linear_lif_fwd_bf16: B too large");
  if (bt == 16)
    linear_lif_fwd_big<1, 16, true><<<grid, dim3(256), 0, s>>>(a);
  else
    linear_lif_fwd_big<1, 8, true><<<grid, dim3(256), 0, s>>>(a);
  return myelin::launched("linear_lif_fwd_bf16");
}

extern "C" int myelin_linear_lif_fwd(const float *x, const float *w, const float *bias, const float *m0,
                                     float *m_final, float *spikes, float *pre, int32_t *packed, float *rates,
                                     float *ckpt, int64_t T, int64_t B, int64_t F, int64_t N, int64_t t_begin,
                                     int64_t t_end, int64_t ckpt_every, float decay, float threshold, float reset,
                                     float slope, int rule, int precision, myelin_stream_t stream) {
  if (x == nullptr || w == nullptr) return myelin::invalid("linear_lif_fwd: x and w are required");
  LinArgs a{};
  if (int rc = fill_lin(a, bias, m0, m_final, spikes, pre, packed, rates, ckpt, T, B, F, N, t_begin, t_end,
                        ckpt_every, decay, threshold, reset, slope, rule))
    return rc;
  a.x = x;
  a.w = w;
  if (precision != MYELIN_PREC_BF16 && precision != MYELIN_PREC_F32)
    return myelin::invalid("linear_lif_fwd: unknown precision %d", precision);
  const bool vec = al16(x) && al16(w) && (F % 4 == 0) && (N % 4 == 0);
  hipStream_t s = myelin::as_hip(stream);
  if (vec && N >= kBig) {
    // 128 neurons x 16 batch rows x 8 steps per tile, or 8 x 16 when that
    // leaves the chip under ~2 workgroups per CU
    const int bt = (cdiv(N, kBig) * cdiv(B, 16) >= 512) ? 16 : 8;
    const dim3 grid(cdiv(N, kBig), cdiv(B, bt));
    if (grid.y > 65535) return myelin::invalid("linear_lif_fwd: B too large");
    if (precision == MYELIN_PREC_BF16) {
      if (bt == 16)
        linear_lif_fwd_big<1, 16, false><<<grid, dim3(256), 0, s>>>(a);
      else
        linear_lif_fwd_big<1, 8, false><<<grid, dim3(256), 0, s>>>(a);
    } else {
      if (bt == 16)
        linear_lif_fwd_big<0, 16, false><<<grid, dim3(256), 0, s>>>(a);
      else
        linear_lif_fwd_big<0, 8, false><<<grid, dim3(256), 0, s>>>(a);
    }
    return myelin::launched("linear_lif_fwd");
  }
  // 8 batch rows x 8 steps per 64 x 64 tile, or 4 x 16 when that leaves the
  // chip under ~2 workgroups per CU
  const int bt = (cdiv(N, kTile) * cdiv(B, 8) >= 512) ? 8 : 4;
  const dim3 grid(cdiv(N, kTile), cdiv(B, bt));
  if (grid.y > 65535) return myelin::invalid("linear_lif_fwd: B too large");
#define MYELIN_LAUNCH_FUSED(P, BT)                                                     \
  do {                                                                                 \
    if (vec)                                                                           \
      linear_lif_fwd<P, BT, true><<<grid, dim3(256), 0, s>>>(a);                       \
    else                                                                               \
      linear_lif_fwd<P, BT, false><<<grid, dim3(256), 0, s>>>(a);                      \
  } while (0)
  if (precision == MYELIN_PREC_BF16) {
    if (bt == 8)
      MYELIN_LAUNCH_FUSED(1, 8);
    else
      MYELIN_LAUNCH_FUSED(1, 4);
  } else {
    if (bt == 8)
      MYELIN_LAUNCH_FUSED(0, 8);
    else
      MYELIN_LAUNCH_FUSED(0, 4);
  }
#undef MYELIN_LAUNCH_FUSED
  return myelin::launched("linear_lif_fwd");
}

extern "C" int myelin_linear_pre_bwd(const float *pre, const float *grad_spikes, const float *grad_rates,
                                     float *grad_m, void *G, int g_dtype, float *gbias_acc, int64_t C, int64_t BN,
                                     int64_t T_total, float decay, float threshold, float reset, float slope,
                                     int surrogate_id, int rule, myelin_stream_t stream) {
  if (C < 1 || BN < 1) return myelin::invalid("linear_pre_bwd: C and BN must be positive");
  if (pre == nullptr || G == nullptr) return myelin::invalid("linear_pre_bwd: null pointer");
  if (g_dtype != MYELIN_DT_F32 && g_dtype != MYELIN_DT_BF16 && g_dtype != MYELIN_DT_BF16X3)
    return myelin::invalid("linear_pre_bwd: G must be float32, bfloat16 or three bfloat16 planes");
  PreBwdArgs a{pre, grad_spikes, grad_rates, grad_m, G, gbias_acc, C, BN, decay, threshold, reset, slope,
               static_cast<float>(T_total), rule};
  if (cdiv(BN, 256) > 0x7fffffff) return myelin::invalid("linear_pre_bwd: BN too large");
  hipStream_t s = myelin::as_hip(stream);
  const bool gs = grad_spikes != nullptr;
  const int gh = g_dtype == MYELIN_DT_BF16X3 ? 2 : g_dtype == MYELIN_DT_BF16 ? 1 : 0;
  switch (surrogate_id) {
    case MYELIN_SG_SIGMOID: launch_pre_bwd<MYELIN_SG_SIGMOID>(a, gs, gh, s); break;
    case MYELIN_SG_FAST_SIGMOID: launch_pre_bwd<MYELIN_SG_FAST_SIGMOID>(a, gs, gh, s); break;
    case MYELIN_SG_ATAN: launch_pre_bwd<MYELIN_SG_ATAN>(a, gs, gh, s); break;
    case MYELIN_SG_TRIANGULAR: launch_pre_bwd<MYELIN_SG_TRIANGULAR>(a, gs, gh, s); break;
    case MYELIN_SG_SUPERSPIKE: launch_pre_bwd<MYELIN_SG_SUPERSPIKE>(a, gs, gh, s); break;
    case MYELIN_SG_MULTI_GAUSSIAN: launch_pre_bwd<MYELIN_SG_MULTI_GAUSSIAN>(a, gs, gh, s); break;
    default: return myelin::invalid("linear_pre_bwd: unknown surrogate id %d", surrogate_id);
  }
  return myelin::launched("linear_pre_bwd");
}

extern "C" int myelin_linear_pre_bwd_readout(const float *pre, const float *grad_out, const float *w_out, int O,
                                             float *grad_m, void *G, int g_dtype, float *gbias_acc, int64_t C,
                                             int64_t B, int64_t N, float decay, float threshold, float reset,
                                             float slope, int surrogate_id, int rule, myelin_stream_t stream) {
  if (C < 1 || B < 1 || N < 1) return myelin::invalid("linear_pre_bwd_readout: C, B and N must be positive");
  if (pre == nullptr || grad_out == nullptr || w_out == nullptr || G == nullptr)
    return myelin::invalid("linear_pre_bwd_readout: null pointer");
  if (O < 1 || O > 32) return myelin::invalid("linear_pre_bwd_readout: O must be in [1, 32]; got %d", O);
  if (N % 256 != 0) return myelin::invalid("linear_pre_bwd_readout: N must be a multiple of 256; got %lld",
                                           static_cast<long long>(N));
  if (g_dtype != MYELIN_DT_F32 && g_dtype != MYELIN_DT_BF16X3)
    return myelin::invalid("linear_pre_bwd_readout: G must be float32 or three bfloat16 planes");
  if (C * pre_bwd_ds_kmax(O) * static_cast<int64_t>(sizeof(float)) > kPreBwdDsLds)
    return myelin::invalid("linear_pre_bwd_readout: C x O too large for the staged rows (C = %lld)",
                           static_cast<long long>(C));
  if (B * N / 256 > 0x7fffffff) return myelin::invalid("linear_pre_bwd_readout: B x N too large");
  PreBwdArgs a{pre, nullptr, nullptr, grad_m, G, gbias_acc, C, B * N, decay, threshold, reset, slope, 1.0f, rule};
  if (rule != MYELIN_RULE_THRESHOLD && rule != MYELIN_RULE_SURROGATE)
    return myelin::invalid("linear_pre_bwd_readout: unknown rule %d", rule);
  hipStream_t s = myelin::as_hip(stream);
  const int gh = g_dtype == MYELIN_DT_BF16X3 ? 2 : 0;
  switch (surrogate_id) {
    case MYELIN_SG_SIGMOID: launch_pre_bwd_ds<MYELIN_SG_SIGMOID>(a, gh, grad_out, w_out, O, N, s); break;
    case MYELIN_SG_FAST_SIGMOID: launch_pre_bwd_ds<MYELIN_SG_FAST_SIGMOID>(a, gh, grad_out, w_out, O, N, s); break;
    case MYELIN_SG_ATAN: launch_pre_bwd_ds<MYELIN_SG_ATAN>(a, gh, grad_out, w_out, O, N, s); break;
    case MYELIN_SG_TRIANGULAR: launch_pre_bwd_ds<MYELIN_SG_TRIANGULAR>(a, gh, grad_out, w_out, O, N, s); break;
    case MYELIN_SG_SUPERSPIKE: launch_pre_bwd_ds<MYELIN_SG_SUPERSPIKE>(a, gh, grad_out, w_out, O, N, s); break;
    case MYELIN_SG_MULTI_GAUSSIAN:
      launch_pre_bwd_ds<MYELIN_SG_MULTI_GAUSSIAN>(a, gh, grad_out, w_out, O, N, s);
      break;
    default: return myelin::invalid("linear_pre_bwd_readout: unknown surrogate id %d", surrogate_id);
  }
  return myelin::launched("linear_pre_bwd_readout");
}

extern "C" int myelin_col_sum_f32(const float *in, float *out, int64_t rows, int64_t cols, int accumulate,
                                  myelin_stream_t stream) {
  if (rows < 0 || cols < 0) return myelin::invalid("col_sum: negative size");
  if (cols == 0) return MYELIN_OK;
  if (out == nullptr || (rows > 0 && in == nullptr)) return myelin::invalid("col_sum: null pointer");
  if (cdiv(cols, 8) > 0x7fffffff) return myelin::invalid("col_sum: too many columns");
  col_sum<<<dim3(static_cast<unsigned>(cdiv(cols, 8))), dim3(256), 0, myelin::as_hip(stream)>>>(in, out, rows, cols,
                                                                                                 accumulate);
  return myelin::launched("col_sum");
}

namespace {
// ---------------------------------------------------------------------------
// Narrow layer (N <= 32 neurons) over a packed-spike input, currents and
// recurrence in one launch: one workgroup per batch row.  W^T is staged
// once into LDS as NP bf16 planes [p][n][k] (NP = 1: W rounded to bf16;
// NP = 3: the exact three-plane split of fp32 W); time is walked in chunks
// of 64 steps whose packed rows are staged into LDS, every load of a stage
// in flight at once.  The sums are those of the narrow GEMM and its
// split-K reduce, bit for bit: wave w takes K splits w, w + 4, ... (the
// same splits, a function of K alone), each split's 16-k MFMA steps in order
// into fresh accumulators on both 32-row blocks of the chunk (for NP = 3,
// planes 2 and 1 into a second accumulator, added at the split's end); N
// lanes of wave 0 then add the splits' sums in order from 0 and the bias
// and run the chunk's recurrence with the arithmetic of lif_currents_fwd.
// Replaces the GEMM, its split-K reduce and the recurrence launch when the
// batch alone fills the chip.  Dynamic LDS: narrow_lds_bytes.
// ---------------------------------------------------------------------------
struct NarrowLifArgs {
  const int32_t *words;  // [T, B, Wx] input spike bits, Wx = ceil(F / 32), bit k % 32 of word k / 32
  const float *w;        // [F, N]
  const float *bias;     // [N] or null
  const float *m0;       // [B, N] or null (zeros)
  float *m_final;        // [B, N] or null
  float *spikes;         // [T, B, N] or null (absolute t)
  float *pre;            // [t_end - t_begin, B, N] or null (relative t)
  float *rates;          // [B, N] or null: spike count over [t_begin, t_end) / T
  int64_t T, B, F, N, Wx, t_begin, t_end, kchunk, splits;
  int ldw, ldx;          // staged row lengths: W^T planes (bf16), bit rows (words)
  float decay, thr, reset, slope, rate_denominator;
};

namespace narrow_fwd {
constexpr int ROWS = 64;  // steps per chunk: two 32-row accumulator blocks
constexpr int LDP = 33;   // padded row (floats) of a split's partial currents
// staged k (bf16) per W^T row and words per bit row: 16 k of slack past F
// (the last MFMA step reads up to 16 k past a partial end), odd word rows
inline int narrow_ldw(int64_t F) { return static_cast<int>((F + 15) / 16 * 16 + 8); }
inline int narrow_ldx(int64_t Wx) { return static_cast<int>(Wx | 1); }
}  // namespace narrow_fwd

int64_t narrow_lds_bytes(int np, int64_t F, int64_t N, int64_t splits) {
  using namespace narrow_fwd;
  const int64_t Wx = (F + 31) / 32;
  return np * N * narrow_ldw(F) * 2 + ROWS * narrow_ldx(Wx) * 4 + splits * ROWS * LDP * 4;
}

template <int NP, int RULE>
__global__ __launch_bounds__(256) void narrow_bits_lif_fwd(NarrowLifArgs p) {
  using namespace narrow_fwd;
  extern __shared__ __attribute__((aligned(16))) char narrow_lds[];
  const int64_t B = p.B, F = p.F, N = p.N, Wx = p.Wx;
  const int nN = static_cast<int>(N), ldw = p.ldw, ldx = p.ldx, S = static_cast<int>(p.splits);
  uint16_t *ws = reinterpret_cast<uint16_t *>(narrow_lds);  // [NP][N][ldw]
  int32_t *xs = reinterpret_cast<int32_t *>(narrow_lds + NP * nN * ldw * 2);  // [ROWS][ldx]
  float *part = reinterpret_cast<float *>(narrow_lds + NP * nN * ldw * 2 + ROWS * ldx * 4);  // [S][ROWS][LDP]
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t b = blockIdx.x;
  const int n = lane & 31;         // the B fragment's column and the D column
  const int kh = 8 * (lane >> 5);  // the fragments' k offset in a 16-k step
  const bool n_on = n < nN;
  const int64_t BN = B * N;

  // W^T planes: W [F, N] read in flat order, 8 loads of 4 values in flight
  // per thread at a time (float4 where the layout allows), then zero past F
  auto put = [&](int flat, float v) {
    const int kk = flat / nN, nn = flat - kk * nN;
    if constexpr (NP == 3) {
      uint16_t h, mid, l;
      split3(v, h, mid, l);
      ws[(0 * nN + nn) * ldw + kk] = h;
      ws[(1 * nN + nn) * ldw + kk] = mid;
      ws[(2 * nN + nn) * ldw + kk] = l;
    } else {
      ws[nn * ldw + kk] = __builtin_bit_cast(uint16_t, static_cast<__bf16>(v));
    }
  };
  const int fn = static_cast<int>(F * N);
  if (fn % 4 == 0 && (reinterpret_cast<uintptr_t>(p.w) & 15) == 0) {
    const f4 *w4 = reinterpret_cast<const f4 *>(p.w);
    for (int e0 = 0; e0 < fn / 4; e0 += 256 * 8) {
      f4 v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int i = e0 + 256 * j + tid;
        v[j] = i < fn / 4 ? w4[i] : f4{0.0f, 0.0f, 0.0f, 0.0f};
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int i = e0 + 256 * j + tid;
        if (i < fn / 4) {
#pragma unroll
          for (int c = 0; c < 4; ++c) put(4 * i + c, v[j][c]);
        }
      }
    }
  } else {
    for (int e0 = 0; e0 < fn; e0 += 256 * 8) {
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int i = e0 + 256 * j + tid;
        v[j] = i < fn ? p.w[i] : 0.0f;
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int i = e0 + 256 * j + tid;
        if (i < fn) put(i, v[j]);
      }
    }
  }
  for (int e = tid; e < nN * (ldw - static_cast<int>(F)); e += 256) put(static_cast<int>(F) * nN + e, 0.0f);
  float m = 0.0f, cnt = 0.0f;
  if (tid < nN && p.m0 != nullptr) m = p.m0[b * N + tid];

  for (int64_t t0 = p.t_begin; t0 < p.t_end; t0 += ROWS) {
    const int rows = static_cast<int>(p.t_end - t0 < ROWS ? p.t_end - t0 : ROWS);
    __syncthreads();  // the previous chunk's bit rows and partials are read
    // the chunk's bit rows (rows past the chunk repeat its last), zero past
    // Wx, 8 loads in flight per thread at a time
    for (int e0 = 0; e0 < ROWS * ldx; e0 += 256 * 8) {
      int32_t v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int e = e0 + 256 * j + tid, r = e / ldx, c = e - r * ldx;
        const int64_t t = t0 + (r < rows ? r : rows - 1);
        v[j] = (e < ROWS * ldx && c < Wx) ? p.words[(t * B + b) * Wx + c] : 0;
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int e = e0 + 256 * j + tid;
        if (e < ROWS * ldx) xs[e] = v[j];
      }
    }
    __syncthreads();
    for (int sp = wv; sp < S; sp += 4) {
      const int64_t kb = sp * p.kchunk, ke = kb + p.kchunk < F ? kb + p.kchunk : F;
      f32x16 acc[2], acc_s[2];
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][r] = acc_s[i][r] = 0.0f;
      for (int64_t k = kb; k < ke; k += 16) {
        const int ka = static_cast<int>(k) + kh;
        bf16x8 bv[NP];
#pragma unroll
        for (int pl = 0; pl < NP; ++pl) {
          if (n_on) {
            bv[pl] = *reinterpret_cast<const bf16x8 *>(&ws[(pl * nN + n) * ldw + ka]);
          } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) bv[pl][e] = static_cast<__bf16>(0.0f);
          }
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          // 8 bits at ka (a multiple of 8, so inside one word)
          const uint32_t bits = (static_cast<uint32_t>(xs[(32 * i + (lane & 31)) * ldx + (ka >> 5)]) >> (ka & 31)) & 0xFFu;
          const u32x4 d = {bf16_pair_of_bits(bits), bf16_pair_of_bits(bits >> 2), bf16_pair_of_bits(bits >> 4),
                           bf16_pair_of_bits(bits >> 6)};
          const bf16x8 av = __builtin_bit_cast(bf16x8, d);
          // as gemm_narrow_x3: planes 2 and 1 into acc_s, plane 0 into acc
#pragma unroll
          for (int pl = NP - 1; pl > 0; --pl)
            acc_s[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, bv[pl], acc_s[i], 0, 0, 0);
          acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, bv[0], acc[i], 0, 0, 0);
        }
      }
      // this split's sums of the chunk's rows
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (n_on)
            part[(sp * ROWS + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)) * LDP + n] =
                NP > 1 ? acc[i][r] + acc_s[i][r] : acc[i][r];
    }
    __syncthreads();
    // the currents, into split 0's slots: the splits in order from 0 (the
    // split-K reduce), or the lone split's sum (the GEMM's own store), then
    // the bias
    for (int e = tid; e < rows * nN; e += 256) {
      const int r = e / nN, nn = e - r * nN;
      float c;
      if (S > 1) {
        float s_ = 0.0f;
        for (int q = 0; q < S; ++q) s_ = s_ + part[(q * ROWS + r) * LDP + nn];
        c = 0.0f + s_;
      } else {
        c = part[r * LDP + nn];
      }
      if (p.bias != nullptr) c = c + p.bias[nn];
      part[r * LDP + nn] = c;
    }
    __syncthreads();
    if (tid < nN) {
      const int64_t flat = b * N + tid;
      for (int r = 0; r < rows; ++r) {
        float mp = m * p.decay;
        mp = mp + part[r * LDP + tid];
        bool spk;
        if constexpr (RULE == MYELIN_RULE_THRESHOLD)
          spk = mp >= p.thr;
        else
          spk = p.slope * (mp - p.thr) >= 0.0f;
        const int64_t t = t0 + r;
        if (p.pre != nullptr) p.pre[(t - p.t_begin) * BN + flat] = mp;
        if (p.spikes != nullptr) p.spikes[t * BN + flat] = spk ? 1.0f : 0.0f;
        m = spk ? p.reset : mp;
        cnt = cnt + (spk ? 1.0f : 0.0f);
      }
    }
  }
  if (tid < nN) {
    const int64_t flat = b * N + tid;
    if (p.m_final != nullptr) p.m_final[flat] = m;
    if (p.rates != nullptr) p.rates[flat] = cnt / p.rate_denominator;
  }
}
}  // namespace

namespace {
// dynamic LDS of the one-launch narrow layer (of the 160 KB a CU holds)
constexpr int64_t kNarrowFusedLds = 150 * 1024;
}  // namespace

extern "C" int myelin_narrow_bits_fits(int64_t F, int64_t N, int precision) {
  if (F < 1 || N < 1 || N > 32 || (precision != 0 && precision != 1)) return 0;
  const int64_t splits = cdiv(F, cdiv(cdiv(F, narrow_splits(F)), 64) * 64);
  return narrow_lds_bytes(precision == 0 ? 3 : 1, F, N, splits) <= kNarrowFusedLds ? 1 : 0;
}

extern "C" int myelin_linear_lif_fwd_narrow_bits(const int32_t *words, const float *w, const float *bias,
                                                 const float *m0, float *m_final, float *spikes, float *pre,
                                                 float *rates, int64_t T, int64_t B, int64_t F, int64_t N,
                                                 int64_t t_begin, int64_t t_end, float decay, float threshold,
                                                 float reset, float slope, int rule, int precision,
                                                 myelin_stream_t stream) {
  if (T < 1 || B < 1 || F < 1 || N < 1) return myelin::invalid("linear_lif_fwd_narrow_bits: T, B, F, N must be positive");
  if (N > 32) return myelin::invalid("linear_lif_fwd_narrow_bits: at most 32 neurons (got %lld)", (long long)N);
  if (t_begin < 0 || t_end > T || t_begin >= t_end) return myelin::invalid("linear_lif_fwd_narrow_bits: bad time range");
  if (words == nullptr || w == nullptr) return myelin::invalid("linear_lif_fwd_narrow_bits: words and w are required");
  if (rates != nullptr && (t_begin != 0 || t_end != T))
    return myelin::invalid("linear_lif_fwd_narrow_bits: rates need the whole range [0, T)");
  if (rule != MYELIN_RULE_THRESHOLD && rule != MYELIN_RULE_SURROGATE)
    return myelin::invalid("linear_lif_fwd_narrow_bits: unknown rule %d", rule);
  if (precision != 0 && precision != 1) return myelin::invalid("linear_lif_fwd_narrow_bits: precision must be 0 or 1");
  if (B > 0x7fffffff) return myelin::invalid("linear_lif_fwd_narrow_bits: B too large");
  NarrowLifArgs a{};
  a.words = words;
  a.w = w;
  a.bias = bias;
  a.m0 = m0;
  a.m_final = m_final;
  a.spikes = spikes;
  a.pre = pre;
  a.rates = rates;
  a.T = T;
  a.B = B;
  a.F = F;
  a.N = N;
  a.Wx = (F + 31) / 32;
  a.t_begin = t_begin;
  a.t_end = t_end;
  // the narrow GEMM's K splits (its workspace always holds them)
  a.kchunk = cdiv(cdiv(F, narrow_splits(F)), 64) * 64;
  a.splits = cdiv(F, a.kchunk);
  a.ldw = narrow_fwd::narrow_ldw(F);
  a.ldx = narrow_fwd::narrow_ldx(a.Wx);
  const int64_t lds = narrow_lds_bytes(precision == 0 ? 3 : 1, F, N, a.splits);
  if (lds > kNarrowFusedLds)
    return myelin::invalid("linear_lif_fwd_narrow_bits: needs %lld bytes of LDS (at most %lld); see "
                           "myelin_narrow_bits_fits", (long long)lds, (long long)kNarrowFusedLds);
  a.decay = decay;
  a.thr = threshold;
  a.reset = reset;
  a.slope = slope;
  a.rate_denominator = static_cast<float>(T);
  hipStream_t s = myelin::as_hip(stream);
  const dim3 grid(static_cast<unsigned>(B)), block(256);
  const bool thr = rule == MYELIN_RULE_THRESHOLD;
  const size_t shm = static_cast<size_t>(lds);
  // dynamic LDS beyond the default 64 KB: raised once per instance
  static const hipError_t attr[4] = {
      hipFuncSetAttribute(reinterpret_cast<const void *>(&narrow_bits_lif_fwd<3, MYELIN_RULE_THRESHOLD>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kNarrowFusedLds)),
      hipFuncSetAttribute(reinterpret_cast<const void *>(&narrow_bits_lif_fwd<3, MYELIN_RULE_SURROGATE>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kNarrowFusedLds)),
      hipFuncSetAttribute(reinterpret_cast<const void *>(&narrow_bits_lif_fwd<1, MYELIN_RULE_THRESHOLD>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kNarrowFusedLds)),
      hipFuncSetAttribute(reinterpret_cast<const void *>(&narrow_bits_lif_fwd<1, MYELIN_RULE_SURROGATE>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kNarrowFusedLds))};
  for (hipError_t e : attr)
    if (e != hipSuccess) {
      myelin::set_error("linear_lif_fwd_narrow_bits: LDS attribute: %s", hipGetErrorString(e));
      return MYELIN_EHIP;
    }
  // fp32 (precision 0): the exact three-plane split; bf16: W rounded
  if (precision == 0)
    thr ? narrow_bits_lif_fwd<3, MYELIN_RULE_THRESHOLD><<<grid, block, shm, s>>>(a)
        : narrow_bits_lif_fwd<3, MYELIN_RULE_SURROGATE><<<grid, block, shm, s>>>(a);
  else
    thr ? narrow_bits_lif_fwd<1, MYELIN_RULE_THRESHOLD><<<grid, block, shm, s>>>(a)
        : narrow_bits_lif_fwd<1, MYELIN_RULE_SURROGATE><<<grid, block, shm, s>>>(a);
  return myelin::launched("linear_lif_fwd_narrow_bits");
}

extern "C" int myelin_lif_currents_fwd(const float *currents, const float *m0, float *m_final, float *spikes,
                                       float *pre, int32_t *packed, float *rates, float *counts, float *ckpt, int64_t T,
                                       int64_t B, int64_t N, int64_t t_begin, int64_t t_end, int64_t pre_origin,
                                       int64_t ck_origin, int64_t ckpt_every, float decay, float threshold,
                                       float reset, float slope, int rule, myelin_stream_t stream) {
  if (T < 1 || B < 1 || N < 1) return myelin::invalid("lif_currents_fwd: T, B, N must be positive");
  if (t_begin < 0 || t_end > T || t_begin >= t_end) return myelin::invalid("lif_currents_fwd: bad time range");
  if (pre_origin < 0 || pre_origin > t_begin || ck_origin < 0 || ck_origin > t_begin)
    return myelin::invalid("lif_currents_fwd: origins must lie in [0, t_begin]");
  if (currents == nullptr) return myelin::invalid("lif_currents_fwd: currents are required");
  if (ckpt != nullptr && ckpt_every < 1) return myelin::invalid("lif_currents_fwd: ckpt_every must be positive");
  if (rule != MYELIN_RULE_THRESHOLD && rule != MYELIN_RULE_SURROGATE)
    return myelin::invalid("lif_currents_fwd: unknown rule %d", rule);
  CurArgs a{};
  a.cur = currents;
  a.m0 = m0;
  a.m_final = m_final;
  a.spikes = spikes;
  a.pre = pre;
  a.rates = rates;
  a.ckpt = ckpt;
  a.counts = counts;
  a.packed = packed;
  a.T = T;
  a.B = B;
  a.N = N;
  a.W = (N + 31) / 32;
  a.t_begin = t_begin;
  a.t_end = t_end;
  a.pre_origin = pre_origin;
  a.ck_origin = ck_origin;
  a.ckpt_every = ckpt_every < 1 ? 1 : ckpt_every;
  a.decay = decay;
  a.thr = threshold;
  a.reset = reset;
  a.slope = slope;
  a.rate_denominator = static_cast<float>(T);
  a.rule = rule;
  const int64_t lanes = B * a.W * 32;
  launch_currents(a, dim3(cdiv(lanes, 256)), myelin::as_hip(stream));
  return myelin::launched("lif_currents_fwd");
}

// ---------------------------------------------------------------------------
// fp32 -> bf16 operand copies for the bf16 GEMMs (round to nearest even,
// exactly as the GEMM loaders round fp32 operands).
// ---------------------------------------------------------------------------
namespace {

__device__ __forceinline__ uint16_t to_bf16(float v) { return __builtin_bit_cast(uint16_t, static_cast<__bf16>(v)); }

// 8 elements per thread (from element i), one 32-byte read and one 16-byte write
__device__ __forceinline__ void cast8(const float *__restrict__ src, uint16_t *__restrict__ dst, int64_t n,
                                      int64_t i) {
  if (i + 8 <= n) {
    const f4 a = *reinterpret_cast<const f4 *>(src + i);
    const f4 b = *reinterpret_cast<const f4 *>(src + i + 4);
    const u4 o{to_bf16(a.x) | (unsigned)to_bf16(a.y) << 16, to_bf16(a.z) | (unsigned)to_bf16(a.w) << 16,
               to_bf16(b.x) | (unsigned)to_bf16(b.y) << 16, to_bf16(b.z) | (unsigned)to_bf16(b.w) << 16};
    *reinterpret_cast<u4 *>(dst + i) = o;
  } else {
    for (int64_t j = i; j < n; ++j) dst[j] = to_bf16(src[j]);
  }
}

__global__ __launch_bounds__(256) void cast_bf16(const float *__restrict__ src, uint16_t *__restrict__ dst,
                                                 int64_t n) {
  cast8(src, dst, n, (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) * 8);
}

// cast_bf16 that also reports whether every element was bf16-exact:
// inexact[0] is set to 1 by any wave holding an inexact element (and never
// cleared here)
__global__ __launch_bounds__(256) void cast_bf16_checked(const float *__restrict__ src, uint16_t *__restrict__ dst,
                                                         int64_t n, int *__restrict__ inexact) {
  const int64_t i = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) * 8;
  bool bad = false;
  if (i + 8 <= n) {
    const f4 a = *reinterpret_cast<const f4 *>(src + i);
    const f4 b = *reinterpret_cast<const f4 *>(src + i + 4);
    bad = !(bf16_exact(a.x) && bf16_exact(a.y) && bf16_exact(a.z) && bf16_exact(a.w) && bf16_exact(b.x) &&
            bf16_exact(b.y) && bf16_exact(b.z) && bf16_exact(b.w));
    const u4 o{to_bf16(a.x) | (unsigned)to_bf16(a.y) << 16, to_bf16(a.z) | (unsigned)to_bf16(a.w) << 16,
               to_bf16(b.x) | (unsigned)to_bf16(b.y) << 16, to_bf16(b.z) | (unsigned)to_bf16(b.w) << 16};
    *reinterpret_cast<u4 *>(dst + i) = o;
  } else {
    for (int64_t j = i; j < n; ++j) {
      bad = bad || !bf16_exact(src[j]);
      dst[j] = to_bf16(src[j]);
    }
  }
  if (__ballot(bad) != 0 && (threadIdx.x & 63) == 0) inexact[0] = 1;
}

// src [rows, cols] -> three bf16 planes (split3), plane p at dst + p*rows*cols,
// each [rows, cols] (row-major like src)
__global__ __launch_bounds__(256) void split_bf16x3(const float *__restrict__ src, uint16_t *__restrict__ dst,
                                                    int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  uint16_t h, m, l;
  split3(src[i], h, m, l);
  dst[i] = h;
  dst[n + i] = m;
  dst[2 * n + i] = l;
}

// src [rows, cols] -> three transposed bf16 planes [cols, rows] through a
// 64 x 64 LDS tile
__global__ __launch_bounds__(256) void split_bf16x3_t(const float *__restrict__ src, uint16_t *__restrict__ dst,
                                                      int64_t rows, int64_t cols) {
  __shared__ float tile[64][65];
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  const int64_t r0 = static_cast<int64_t>(blockIdx.y) * 64, c0 = static_cast<int64_t>(blockIdx.x) * 64;
  const int64_t plane = rows * cols;
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const int64_t r = r0 + ty + 4 * k, c = c0 + tx;
    tile[ty + 4 * k][tx] = (r < rows && c < cols) ? src[r * cols + c] : 0.0f;
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const int64_t c = c0 + ty + 4 * k, r = r0 + tx;
    if (c < cols && r < rows) {
      uint16_t h, m, l;
      split3(tile[tx][ty + 4 * k], h, m, l);
      dst[c * rows + r] = h;
      dst[plane + c * rows + r] = m;
      dst[2 * plane + c * rows + r] = l;
    }
  }
}

// dst[c, r] = bf16(src[r, c]) through a 32 x 32 LDS tile (4 elements per
// thread: a weight-sized matrix still spreads over the whole chip); this
// workgroup's tile is column block bx, row block by
__device__ __forceinline__ void transpose_tile(const float *__restrict__ src, uint16_t *__restrict__ dst,
                                               int64_t rows, int64_t cols, int64_t bx, int64_t by) {
  __shared__ float tile[32][33];
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
  const int64_t r0 = by * 32, c0 = bx * 32;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int64_t r = r0 + ty + 8 * k, c = c0 + tx;
    tile[ty + 8 * k][tx] = (r < rows && c < cols) ? src[r * cols + c] : 0.0f;
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int64_t c = c0 + ty + 8 * k, r = r0 + tx;
    if (c < cols && r < rows) dst[c * rows + r] = to_bf16(tile[tx][ty + 8 * k]);
  }
}

__global__ __launch_bounds__(256) void transpose_bf16(const float *__restrict__ src, uint16_t *__restrict__ dst,
                                                      int64_t rows, int64_t cols) {
  transpose_tile(src, dst, rows, cols, blockIdx.x, blockIdx.y);
}

// cast_bf16 of x and transpose_bf16 of w in one launch: the first
// cast_blocks workgroups cast, the rest each transpose one 32 x 32 tile
__global__ __launch_bounds__(256) void cast_transpose_bf16(const float *__restrict__ x, uint16_t *__restrict__ xb,
                                                           int64_t n, int64_t cast_blocks,
                                                           const float *__restrict__ w, uint16_t *__restrict__ wt,
                                                           int64_t rows, int64_t cols) {
  const int64_t b = blockIdx.x;
  if (b < cast_blocks) {
    cast8(x, xb, n, (b * blockDim.x + threadIdx.x) * 8);
    return;
  }
  const int64_t t = b - cast_blocks, tiles_x = (cols + 31) / 32;
  transpose_tile(w, wt, rows, cols, t % tiles_x, t / tiles_x);
}

}  // namespace

extern "C" int myelin_cast_bf16(const float *src, uint16_t *dst, int64_t n, myelin_stream_t stream) {
  if (n < 0) return myelin::invalid("cast_bf16: negative size");
  if (n == 0) return MYELIN_OK;
  if (src == nullptr || dst == nullptr) return myelin::invalid("cast_bf16: null pointer");
  if (!myelin::aligned(src, 16) || !myelin::aligned(dst, 16))
    return myelin::invalid("cast_bf16: src and dst must be 16-byte aligned");
  cast_bf16<<<dim3(cdiv(cdiv(n, 8), 256)), dim3(256), 0, myelin::as_hip(stream)>>>(src, dst, n);
  return myelin::launched("cast_bf16");
}

extern "C" int myelin_cast_bf16_checked(const float *src, uint16_t *dst, int64_t n, int *inexact,
                                        myelin_stream_t stream) {
  if (n < 0) return myelin::invalid("cast_bf16_checked: negative size");
  if (n == 0) return MYELIN_OK;
  if (src == nullptr || dst == nullptr || inexact == nullptr) return myelin::invalid("cast_bf16_checked: null pointer");
  if (!myelin::aligned(src, 16) || !myelin::aligned(dst, 16))
    return myelin::invalid("cast_bf16_checked: src and dst must be 16-byte aligned");
  cast_bf16_checked<<<dim3(cdiv(cdiv(n, 8), 256)), dim3(256), 0, myelin::as_hip(stream)>>>(src, dst, n, inexact);
  return myelin::launched("cast_bf16_checked");
}

extern "C" int myelin_split_bf16x3(const float *src, uint16_t *dst, int64_t rows, int64_t cols, int transpose,
                                   myelin_stream_t stream) {
  if (rows < 0 || cols < 0) return myelin::invalid("split_bf16x3: negative size");
  if (rows == 0 || cols == 0) return MYELIN_OK;
  if (src == nullptr || dst == nullptr) return myelin::invalid("split_bf16x3: null pointer");
  hipStream_t s = myelin::as_hip(stream);
  if (transpose) {
    if (cdiv(rows, 64) > 65535) return myelin::invalid("split_bf16x3: too many rows");
    split_bf16x3_t<<<dim3(cdiv(cols, 64), cdiv(rows, 64)), dim3(256), 0, s>>>(src, dst, rows, cols);
  } else {
    if (cdiv(rows * cols, 256) > 0x7fffffff) return myelin::invalid("split_bf16x3: too many elements");
    split_bf16x3<<<dim3(cdiv(rows * cols, 256)), dim3(256), 0, s>>>(src, dst, rows * cols);
  }
  return myelin::launched("split_bf16x3");
}

extern "C" int myelin_cast_transpose_bf16(const float *x, uint16_t *xb, int64_t n, const float *w, uint16_t *wt,
                                          int64_t rows, int64_t cols, myelin_stream_t stream) {
  if (n < 0 || rows < 0 || cols < 0) return myelin::invalid("cast_transpose_bf16: negative size");
  if (n > 0 && (x == nullptr || xb == nullptr)) return myelin::invalid("cast_transpose_bf16: null pointer");
  if (rows > 0 && cols > 0 && (w == nullptr || wt == nullptr))
    return myelin::invalid("cast_transpose_bf16: null pointer");
  if (n > 0 && (!myelin::aligned(x, 16) || !myelin::aligned(xb, 16)))
    return myelin::invalid("cast_transpose_bf16: x and xb must be 16-byte aligned");
  const int64_t cast_blocks = cdiv(cdiv(n, 8), 256);
  const int64_t tiles = rows > 0 && cols > 0 ? cdiv(rows, 32) * cdiv(cols, 32) : 0;
  if (cast_blocks + tiles == 0) return MYELIN_OK;
  if (cast_blocks + tiles > 0x7fffffff) return myelin::invalid("cast_transpose_bf16: too large");
  cast_transpose_bf16<<<dim3(static_cast<unsigned>(cast_blocks + tiles)), dim3(256), 0, myelin::as_hip(stream)>>>(
      x, xb, n, cast_blocks, w, wt, rows, cols);
  return myelin::launched("cast_transpose_bf16");
}

extern "C" int myelin_transpose_bf16(const float *src, uint16_t *dst, int64_t rows, int64_t cols,
                                     myelin_stream_t stream) {
  if (rows < 0 || cols < 0) return myelin::invalid("transpose_bf16: negative size");
  if (rows == 0 || cols == 0) return MYELIN_OK;
  if (src == nullptr || dst == nullptr) return myelin::invalid("transpose_bf16: null pointer");
  if (cdiv(rows, 32) > 65535 || cdiv(cols, 32) > 0x7fffffff) return myelin::invalid("transpose_bf16: too large");
  transpose_bf16<<<dim3(cdiv(cols, 32), cdiv(rows, 32)), dim3(256), 0, myelin::as_hip(stream)>>>(src, dst, rows, cols);
  return myelin::launched("transpose_bf16");
}

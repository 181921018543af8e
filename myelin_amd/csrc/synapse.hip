// Streamed synapse x_t @ W fused ahead of the LIF update, and the GEMMs of
// its backward, for gfx950.
//
// MFMA tiles: a workgroup of 4 waves computes a 64 x 64 output tile, each
// wave one 32 x 32 quarter with v_mfma_f32_32x32x16_bf16 (bf16 inputs,
// fp32 accumulate) or v_mfma_f32_32x32x2f32 (fp32).  Operand fragments, per
// lane l of a wave:
//   A (32 x K-step): row l % 32, k = (l / 32) * KV + [0, KV)   (KV = 8 bf16 | 1 f32)
//   B (K-step x 32): col l % 32, same k
//   D (32 x 32):     col l % 32, row 8*(r/4) + 4*(l/32) + r%4 for acc register r
// Tiles stage through LDS k-contiguous ([row][k] for A, [col][k] for B), so a
// bf16 fragment is one 16-byte LDS read.
//
// linear_lif_fwd: the workgroup owns 8 batch rows x 64 neurons and walks the
// time axis in chunks of 8 steps.  Per chunk it computes the 64 x 64 current
// tile (rows = 8 steps x 8 batch rows) over the full input width, parks it
// in LDS, and runs the 8 recurrence steps for its 512 neurons in registers;
// membrane (and spike counts) stay in registers across chunks, so currents
// never go to HBM.

#include "common.h"

namespace {

using myelin::kWave;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kTile = 64;  // output tile edge
constexpr int kChunk = 8;  // timesteps per fused chunk
constexpr int kBt = 8;     // batch rows per fused workgroup (kChunk * kBt == kTile)

template <int PREC>
struct Prec;
template <>
struct Prec<0> {  // fp32 MFMA
  using T = float;
  static constexpr int KS = 16;  // k per LDS stage
  static constexpr int KV = 1;   // k per lane per MFMA
  static constexpr int KM = 2;   // k per MFMA
};
template <>
struct Prec<1> {  // bf16 MFMA, fp32 accumulate
  using T = __bf16;
  static constexpr int KS = 32;
  static constexpr int KV = 8;
  static constexpr int KM = 16;
};

template <int PREC>
struct Stage {
  using T = typename Prec<PREC>::T;
  static constexpr int KS = Prec<PREC>::KS;
  static constexpr int LD = KS + (PREC == 1 ? 8 : 1);  // padded row length (elements)
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

// One wave's MFMA over one LDS stage: acc += A[wm rows] x B[wn cols].
template <int PREC>
__device__ __forceinline__ void mfma_stage(const Stage<PREC> &st, int wm, int wn, int lane, f32x16 &acc) {
  constexpr int KS = Prec<PREC>::KS, KM = Prec<PREC>::KM, KV = Prec<PREC>::KV;
  const int r = 32 * wm + (lane & 31), c = 32 * wn + (lane & 31), kq = (lane >> 5) * KV;
#pragma unroll
  for (int kk = 0; kk < KS; kk += KM) {
    if constexpr (PREC == 1) {
      const bf16x8 av = *reinterpret_cast<const bf16x8 *>(&st.a[r][kk + kq]);
      const bf16x8 bv = *reinterpret_cast<const bf16x8 *>(&st.b[c][kk + kq]);
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, bv, acc, 0, 0, 0);
    } else {
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(st.a[r][kk + kq], st.b[c][kk + kq], acc, 0, 0, 0);
    }
  }
}

// row index (within the wave's 32 x 32 quarter) of accumulator register r
__device__ __forceinline__ int acc_row(int r, int lane) { return 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3); }

// ---------------------------------------------------------------------------
// Plain GEMM: C[M,N] (+)= A(m,k) B(k,n), fp32 in and out.
//   A(m,k) = TA ? A[k*lda + m] : A[m*lda + k]
//   B(k,n) = TB ? B[n*ldb + k] : B[k*ldb + n]
// ---------------------------------------------------------------------------
struct GemmArgs {
  const float *A;
  const float *B;
  const float *bias;  // [N] added in the epilogue, or null
  float *C;
  int64_t M, N, K, lda, ldb, ldc;
  int accumulate;
};

template <int PREC, bool TA, bool TB>
__global__ __launch_bounds__(256) void gemm_kernel(GemmArgs g) {
  constexpr int KS = Prec<PREC>::KS;
  __shared__ Stage<PREC> st;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, wm = w >> 1, wn = w & 1;
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * kTile, n0 = static_cast<int64_t>(blockIdx.x) * kTile;
  f32x16 acc;
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = 0.0f;

  for (int64_t k0 = 0; k0 < g.K; k0 += KS) {
    // stage A and B (kTile * KS elements each, KS*kTile/256 per thread)
#pragma unroll
    for (int e = 0; e < kTile * KS / 256; ++e) {
      const int idx = e * 256 + tid;
      int row, kk;
      if constexpr (TA) {  // memory is k-major: consecutive threads take consecutive m
        kk = idx / kTile;
        row = idx % kTile;
      } else {
        row = idx / KS;
        kk = idx % KS;
      }
      const int64_t m = m0 + row, k = k0 + kk;
      float v = 0.0f;
      if (m < g.M && k < g.K) v = TA ? g.A[k * g.lda + m] : g.A[m * g.lda + k];
      st.a[row][kk] = cvt<PREC>(v);
    }
#pragma unroll
    for (int e = 0; e < kTile * KS / 256; ++e) {
      const int idx = e * 256 + tid;
      int col, kk;
      if constexpr (TB) {  // memory is n-major with k contiguous
        col = idx / KS;
        kk = idx % KS;
      } else {
        kk = idx / kTile;
        col = idx % kTile;
      }
      const int64_t n = n0 + col, k = k0 + kk;
      float v = 0.0f;
      if (n < g.N && k < g.K) v = TB ? g.B[n * g.ldb + k] : g.B[k * g.ldb + n];
      st.b[col][kk] = cvt<PREC>(v);
    }
    __syncthreads();
    mfma_stage<PREC>(st, wm, wn, lane, acc);
    __syncthreads();
  }
  const int64_t col = n0 + 32 * wn + (lane & 31);
  if (col >= g.N) return;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int64_t row = m0 + 32 * wm + acc_row(r, lane);
    if (row < g.M) {
      float *dst = g.C + row * g.ldc + col;
      float v = g.accumulate ? *dst + acc[r] : acc[r];
      if (g.bias != nullptr) v = v + g.bias[col];
      *dst = v;
    }
  }
}

// ---------------------------------------------------------------------------
// Fused current GEMM + LIF recurrence.
// ---------------------------------------------------------------------------
struct LinArgs {
  const float *x;     // [T, B, F]
  const float *w;     // [F, N]
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

template <int PREC>
struct FusedSmem {
  Stage<PREC> st;
  alignas(16) float cur[kTile][kTile + 1];  // currents [row = j*kBt + bb][col]
};

template <int PREC>
__global__ __launch_bounds__(256) void linear_lif_fwd(LinArgs p) {
  constexpr int KS = Prec<PREC>::KS;
  __shared__ FusedSmem<PREC> sm;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, wm = w >> 1, wn = w & 1;
  const int64_t b0 = static_cast<int64_t>(blockIdx.y) * kBt, n0 = static_cast<int64_t>(blockIdx.x) * kTile;
  const int64_t BN = p.B * p.N;

  // recurrence ownership: wave w owns batch rows bb = 2w, 2w+1; lane = neuron
  const int64_t n = n0 + lane;
  float m[2], cnt[2];
  bool act[2];
  int64_t flat[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int64_t b = b0 + 2 * w + q;
    act[q] = (b < p.B) && (n < p.N);
    flat[q] = b * p.N + n;
    m[q] = (act[q] && p.m0 != nullptr) ? p.m0[flat[q]] : 0.0f;
    cnt[q] = 0.0f;
  }
  const float bias_n = (p.bias != nullptr && n < p.N) ? p.bias[n] : 0.0f;
  int64_t next_ck = p.t_begin, ck_row = 0;

  for (int64_t t0 = p.t_begin; t0 < p.t_end; t0 += kChunk) {
    f32x16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
    for (int64_t k0 = 0; k0 < p.F; k0 += KS) {
      // A rows: r = j*kBt + bb  ->  x[t0 + j, b0 + bb, k]
#pragma unroll
      for (int e = 0; e < kTile * KS / 256; ++e) {
        const int idx = e * 256 + tid;
        const int row = idx / KS, kk = idx % KS;
        const int64_t t = t0 + row / kBt, b = b0 + row % kBt, k = k0 + kk;
        float v = 0.0f;
        if (t < p.t_end && b < p.B && k < p.F) v = p.x[(t * p.B + b) * p.F + k];
        sm.st.a[row][kk] = cvt<PREC>(v);
      }
#pragma unroll
      for (int e = 0; e < kTile * KS / 256; ++e) {
        const int idx = e * 256 + tid;
        const int kk = idx / kTile, col = idx % kTile;
        const int64_t k = k0 + kk, nn = n0 + col;
        float v = 0.0f;
        if (k < p.F && nn < p.N) v = p.w[k * p.N + nn];
        sm.st.b[col][kk] = cvt<PREC>(v);
      }
      __syncthreads();
      mfma_stage<PREC>(sm.st, wm, wn, lane, acc);
      __syncthreads();
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) sm.cur[32 * wm + acc_row(r, lane)][32 * wn + (lane & 31)] = acc[r];
    __syncthreads();

#pragma unroll
    for (int j = 0; j < kChunk; ++j) {
      const int64_t t = t0 + j;
      if (t >= p.t_end) break;  // uniform
      if (p.ckpt != nullptr && t == next_ck) {
#pragma unroll
        for (int q = 0; q < 2; ++q)
          if (act[q]) p.ckpt[ck_row * BN + flat[q]] = m[q];
        ++ck_row;
        next_ck += p.ckpt_every;
      }
      bool s[2];
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        // input_current = x_t @ W + bias ; m' = m*decay + input_current
        const float cur = sm.cur[j * kBt + 2 * w + q][lane] + bias_n;
        float mp = m[q] * p.decay;
        mp = mp + cur;
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
        for (int q = 0; q < 2; ++q) {
          const uint64_t bits = __ballot(s[q]);
          const int64_t b = b0 + 2 * w + q;
          const int64_t word = n0 / 32 + (lane >> 5);
          if ((lane & 31) == 0 && b < p.B && word < p.W)
            p.packed[(t * p.B + b) * p.W + word] = static_cast<int32_t>(lane ? (bits >> 32) : (bits & 0xffffffffu));
        }
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int q = 0; q < 2; ++q) {
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
    float d = 1.0f + fabsf(c);
    return 0.5f / (d * d);
  } else if constexpr (SID == MYELIN_SG_ATAN) {
    float s = 1.5707963267948966f * c;
    return 0.5f / (1.0f + s * s);
  } else if constexpr (SID == MYELIN_SG_TRIANGULAR) {
    float sg = (c > 0.0f) ? 1.0f : ((c < 0.0f) ? -1.0f : 0.0f);
    return fabsf(c) < 1.0f ? -sg : 0.0f;
  } else if constexpr (SID == MYELIN_SG_SUPERSPIKE) {
    float d = 1.0f + fabsf(c);
    return 1.0f / (d * d);
  } else {
    float z = c / 0.5f, r = c - 1.0f, l = c + 1.0f;
    return 0.47873073648171924f * expf(-0.5f * z * z) + 0.07978845608028655f * expf(-0.5f * r * r) +
           0.07978845608028655f * expf(-0.5f * l * l);
  }
}

struct PreBwdArgs {
  const float *pre;     // [C, BN]
  const float *gs;      // [C, BN] or null
  const float *grate;   // [BN] or null
  float *gm;            // [BN] in/out
  float *G;             // [C, BN]
  float *gbias_acc;     // [BN] or null (accumulated)
  int64_t C, BN;
  float decay, thr, reset, slope, rate_denominator;
  int rule;
};

template <int SID>
__global__ __launch_bounds__(256) void linear_pre_bwd(PreBwdArgs p) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= p.BN) return;
  float gm = p.gm[i];
  const float gstep = p.grate != nullptr ? p.grate[i] / p.rate_denominator : 0.0f;
  float gb = 0.0f;
  for (int64_t j = p.C - 1; j >= 0; --j) {
    const float pre = p.pre[j * p.BN + i];
    const float c = p.slope * (pre - p.thr);
    const bool sp = (p.rule == MYELIN_RULE_THRESHOLD) ? (pre >= p.thr) : (c >= 0.0f);
    const float s = sp ? 1.0f : 0.0f;
    const float d = p.slope * sg_deriv<SID>(c);
    float gp = gm * ((1.0f - s) + (p.reset - pre) * d);
    if (p.gs != nullptr) gp = gp + p.gs[j * p.BN + i] * d;
    if (p.grate != nullptr) gp = gp + gstep * d;
    p.G[j * p.BN + i] = gp;
    gb = gb + gp;
    gm = gp * p.decay;
  }
  p.gm[i] = gm;
  if (p.gbias_acc != nullptr) p.gbias_acc[i] = p.gbias_acc[i] + gb;
}

// out[n] (+)= sum_b in[b, n]  (fixed order per column: deterministic)
__global__ __launch_bounds__(256) void col_sum(const float *__restrict__ in, float *__restrict__ out, int64_t rows,
                                               int64_t cols, int accumulate) {
  const int64_t n = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (n >= cols) return;
  float s = 0.0f;
  for (int64_t r = 0; r < rows; ++r) s = s + in[r * cols + n];
  out[n] = accumulate ? out[n] + s : s;
}

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

template <int PREC>
int launch_gemm(const GemmArgs &g, int ta, int tb, hipStream_t s) {
  const dim3 grid(cdiv(g.N, kTile), cdiv(g.M, kTile));
  if (grid.y > 65535) return myelin::invalid("gemm: M too large (%lld)", (long long)g.M);
  if (!ta && !tb)
    gemm_kernel<PREC, false, false><<<grid, dim3(256), 0, s>>>(g);
  else if (!ta && tb)
    gemm_kernel<PREC, false, true><<<grid, dim3(256), 0, s>>>(g);
  else if (ta && !tb)
    gemm_kernel<PREC, true, false><<<grid, dim3(256), 0, s>>>(g);
  else
    gemm_kernel<PREC, true, true><<<grid, dim3(256), 0, s>>>(g);
  return myelin::launched("gemm");
}

}  // namespace

extern "C" int myelin_gemm_f32(const float *A, const float *B, const float *bias, float *C, int64_t M, int64_t N,
                               int64_t K, int64_t lda, int64_t ldb, int64_t ldc, int trans_a, int trans_b,
                               int accumulate, int precision, myelin_stream_t stream) {
  if (M < 0 || N < 0 || K < 0) return myelin::invalid("gemm: negative size");
  if (M == 0 || N == 0) return MYELIN_OK;
  if (A == nullptr || B == nullptr || C == nullptr) return myelin::invalid("gemm: null pointer");
  if (ldc < N) return myelin::invalid("gemm: ldc < N");
  if ((trans_a ? lda < M : lda < K) || (trans_b ? ldb < K : ldb < N)) return myelin::invalid("gemm: bad leading dim");
  GemmArgs g{A, B, bias, C, M, N, K, lda, ldb, ldc, accumulate};
  hipStream_t s = myelin::as_hip(stream);
  if (precision == MYELIN_PREC_BF16) return launch_gemm<1>(g, trans_a, trans_b, s);
  if (precision == MYELIN_PREC_F32) return launch_gemm<0>(g, trans_a, trans_b, s);
  return myelin::invalid("gemm: unknown precision %d", precision);
}

extern "C" int myelin_linear_lif_fwd(const float *x, const float *w, const float *bias, const float *m0,
                                     float *m_final, float *spikes, float *pre, int32_t *packed, float *rates,
                                     float *ckpt, int64_t T, int64_t B, int64_t F, int64_t N, int64_t t_begin,
                                     int64_t t_end, int64_t ckpt_every, float decay, float threshold, float reset,
                                     float slope, int rule, int precision, myelin_stream_t stream) {
  if (T < 1 || B < 1 || F < 1 || N < 1) return myelin::invalid("linear_lif_fwd: T, B, F, N must be positive");
  if (t_begin < 0 || t_end > T || t_begin >= t_end) return myelin::invalid("linear_lif_fwd: bad time range");
  if (x == nullptr || w == nullptr) return myelin::invalid("linear_lif_fwd: x and w are required");
  if (ckpt != nullptr && ckpt_every < 1) return myelin::invalid("linear_lif_fwd: ckpt_every must be positive");
  if (rule != MYELIN_RULE_THRESHOLD && rule != MYELIN_RULE_SURROGATE)
    return myelin::invalid("linear_lif_fwd: unknown rule %d", rule);
  LinArgs a{};
  a.x = x;
  a.w = w;
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
  const dim3 grid(cdiv(N, kTile), cdiv(B, kBt));
  if (grid.y > 65535) return myelin::invalid("linear_lif_fwd: B too large");
  hipStream_t s = myelin::as_hip(stream);
  if (precision == MYELIN_PREC_BF16)
    linear_lif_fwd<1><<<grid, dim3(256), 0, s>>>(a);
  else if (precision == MYELIN_PREC_F32)
    linear_lif_fwd<0><<<grid, dim3(256), 0, s>>>(a);
  else
    return myelin::invalid("linear_lif_fwd: unknown precision %d", precision);
  return myelin::launched("linear_lif_fwd");
}

extern "C" int myelin_linear_pre_bwd(const float *pre, const float *grad_spikes, const float *grad_rates,
                                     float *grad_m, float *G, float *gbias_acc, int64_t C, int64_t BN,
                                     int64_t T_total, float decay, float threshold, float reset, float slope,
                                     int surrogate_id, int rule, myelin_stream_t stream) {
  if (C < 1 || BN < 1) return myelin::invalid("linear_pre_bwd: C and BN must be positive");
  if (pre == nullptr || grad_m == nullptr || G == nullptr) return myelin::invalid("linear_pre_bwd: null pointer");
  PreBwdArgs a{pre, grad_spikes, grad_rates, grad_m, G, gbias_acc, C, BN, decay, threshold, reset, slope,
               static_cast<float>(T_total), rule};
  const dim3 grid(cdiv(BN, 256));
  hipStream_t s = myelin::as_hip(stream);
  switch (surrogate_id) {
    case MYELIN_SG_SIGMOID: linear_pre_bwd<MYELIN_SG_SIGMOID><<<grid, dim3(256), 0, s>>>(a); break;
    case MYELIN_SG_FAST_SIGMOID: linear_pre_bwd<MYELIN_SG_FAST_SIGMOID><<<grid, dim3(256), 0, s>>>(a); break;
    case MYELIN_SG_ATAN: linear_pre_bwd<MYELIN_SG_ATAN><<<grid, dim3(256), 0, s>>>(a); break;
    case MYELIN_SG_TRIANGULAR: linear_pre_bwd<MYELIN_SG_TRIANGULAR><<<grid, dim3(256), 0, s>>>(a); break;
    case MYELIN_SG_SUPERSPIKE: linear_pre_bwd<MYELIN_SG_SUPERSPIKE><<<grid, dim3(256), 0, s>>>(a); break;
    case MYELIN_SG_MULTI_GAUSSIAN: linear_pre_bwd<MYELIN_SG_MULTI_GAUSSIAN><<<grid, dim3(256), 0, s>>>(a); break;
    default: return myelin::invalid("linear_pre_bwd: unknown surrogate id %d", surrogate_id);
  }
  return myelin::launched("linear_pre_bwd");
}

extern "C" int myelin_col_sum_f32(const float *in, float *out, int64_t rows, int64_t cols, int accumulate,
                                  myelin_stream_t stream) {
  if (rows < 0 || cols < 0) return myelin::invalid("col_sum: negative size");
  if (cols == 0) return MYELIN_OK;
  if (out == nullptr || (rows > 0 && in == nullptr)) return myelin::invalid("col_sum: null pointer");
  col_sum<<<dim3(cdiv(cols, 256)), dim3(256), 0, myelin::as_hip(stream)>>>(in, out, rows, cols, accumulate);
  return myelin::launched("col_sum");
}
